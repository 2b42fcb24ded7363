"""Shared builders for the parity tests: seeded graphs, states and
attention, plus the oracle CSR tuple in both numpy and torch form."""
import numpy as np
import torch

from flashlog_amd import synth
from oracle import oracle as O


def small_graph(cfg_id=2, scale=0.05, seed=None):
    h, r, t, E, R = synth.make_graph(cfg_id, scale=scale, seed=seed)
    csr = O.build_csr_structure(h, t, r, E)
    return h, r, t, E, R, csr


def sparse_state(BL, E, nnz_per_row, rng, ties=False):
    A = np.zeros((BL, E), np.float32)
    for i in range(BL):
        k = min(E, nnz_per_row)
        idx = rng.choice(E, k, replace=False)
        if ties:
            vals = rng.integers(1, 4, size=k).astype(np.float32) / 8.0
        else:
            vals = rng.random(k).astype(np.float32) + np.float32(1e-3)
        A[i, idx] = vals
    return A


def attention(BL, n, rng):
    logits = rng.standard_normal((BL, n)).astype(np.float32)
    e = np.exp(logits - logits.max(-1, keepdims=True))
    return (e / e.sum(-1, keepdims=True)).astype(np.float32)


def masks_for(csr, M, rng, drop=0.1):
    m = (rng.random(M) >= drop)
    return m, (m[csr[3]].astype(np.float32), m[csr[7]].astype(np.float32))


def to_torch_csr(csr, device):
    return tuple(torch.from_numpy(np.ascontiguousarray(a)).to(device) for a in csr)


def bits(x):
    x = np.ascontiguousarray(x)
    return x.view(np.int32) if x.dtype == np.float32 else x.view(np.int64)


def sparse_coo_state(B, L, E, per_row, rng, ties=False):
    """Coalesced COO state: rows (b, l) ascending, entities ascending."""
    bs, ls, es, vs = [], [], [], []
    for b in range(B):
        for l in range(L):
            k = int(rng.integers(0, per_row + 1))
            e = np.sort(rng.choice(E, k, replace=False))
            v = (rng.integers(1, 4, k) / 8.0 if ties else rng.random(k) + 1e-3).astype(np.float32)
            bs.append(np.full(k, b)); ls.append(np.full(k, l)); es.append(e); vs.append(v)
    return (np.concatenate(bs).astype(np.int64), np.concatenate(ls).astype(np.int64),
            np.concatenate(es).astype(np.int64), np.concatenate(vs).astype(np.float32))


def assert_grad_close(got, ref, rtol=1e-5):
    """Gradient parity: within rtol relative, with the absolute slack scaled
    to the gradient's own magnitude (rtol/10 of its largest entry), so sums
    that cancel are compared against the size of their terms' totals."""
    got = np.asarray(got)
    ref = np.asarray(ref)
    scale = float(np.abs(ref).max()) if ref.size else 0.0
    np.testing.assert_allclose(got, ref, rtol=rtol, atol=0.1 * rtol * max(scale, 1e-30))
