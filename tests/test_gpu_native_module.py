"""The native-module names get_module() serves (flashlog.cpp:1935-1965,
signatures in flashlog.h:17-261), called with the reference's positional
arguments and checked against the oracle: the dense CPU pair on CPU
tensors, the dense sum and max CUDA forwards and backwards, the normalize
pair (also with the reference's (0, 0) marks for empty rows), the
fixed-relation step and the filtered ranks."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_grad_close, attention, bits, masks_for, small_graph, sparse_state

pytestmark = pytest.mark.gpu


def _mod():
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    return fk.get_module()


def _case(seed=5, K=3):
    rng = np.random.default_rng(seed)
    h, r, t, E, R, csr = small_graph(2, 0.03)
    BL, n = 6, 2 * R + 1
    A = sparse_state(BL, E, 25, rng)
    w = attention(BL, n, rng)
    _, masks = masks_for(csr, h.shape[0], rng)
    return rng, E, R, csr, A, w, masks, K


def _args(csr, masks, dev, full):
    c = [torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in csr]
    om, im = (torch.from_numpy(m).to(dev) for m in masks)
    if not full:  # the CPU signature: columns, mask, 4 group arrays per side
        return [c[1], om, c[8], c[9], c[10], c[11], c[5], im, c[12], c[13], c[14], c[15]]
    return [c[0], c[1], c[2], om, c[4], c[5], c[6], im, c[8], c[9], c[10], c[11], c[12], c[13], c[14], c[15]]


@pytest.mark.parametrize("K", [3, 1 << 60])
def test_dense_cpu_pair(K):
    rng, E, R, csr, A, w, masks, _ = _case(K=K)
    mod = _mod()
    At, wt = torch.from_numpy(A), torch.from_numpy(w)
    active = torch.from_numpy(O.active_nodes(A))
    outs = mod.flashlog_forward_cpu(At, wt, active, *_args(csr, masks, "cpu", False), R, False, K)
    ref = O.dense_forward(A, w, csr, masks, R, topk_edges=K)
    for o, rf in zip(outs, ref):
        assert o.device.type == "cpu" and np.array_equal(bits(o.numpy()), bits(rf))
    g = [rng.standard_normal(A.shape).astype(np.float32) for _ in range(3)]
    gA, gw = mod.flashlog_backward_cpu(*[torch.from_numpy(x) for x in g], At, wt, active,
                                       *_args(csr, masks, "cpu", False), R, False, K)
    gA_ref, gw_ref = O.dense_backward(*g, A, w, csr, masks, R, topk_edges=K)
    assert gA.device.type == "cpu" and np.array_equal(bits(gA.numpy()), bits(gA_ref))
    assert_grad_close(gw.numpy(), gw_ref)


@pytest.mark.parametrize("use_topk", [True, False])
def test_dense_cuda_sum_and_max(use_topk):
    rng, E, R, csr, A, w, masks, K = _case(9)
    mod = _mod()
    dev = torch.device("cuda")
    At, wt = torch.from_numpy(A).to(dev), torch.from_numpy(w).to(dev)
    active = torch.from_numpy(O.active_nodes(A)).to(dev)
    full = _args(csr, masks, dev, True)
    budget = K if use_topk else 1 << 60
    outs = mod.flashlog_forward_cuda(At, wt, active, *full, R, False, use_topk, K, 0)
    ref = O.dense_forward(A, w, csr, masks, R, topk_edges=budget)
    for o, rf in zip(outs, ref):
        assert np.array_equal(bits(o.cpu().numpy()), bits(rf))
    g = [rng.standard_normal(A.shape).astype(np.float32) for _ in range(3)]
    gt = [torch.from_numpy(x).to(dev) for x in g]
    gA, gw = mod.flashlog_backward_cuda(*gt, outs[1], outs[2], At, wt, active, *full, R, False, use_topk, K, 0)
    gA_ref, gw_ref = O.dense_backward(*g, A, w, csr, masks, R, topk_edges=budget)
    assert np.array_equal(bits(gA.cpu().numpy()), bits(gA_ref))
    assert_grad_close(gw.cpu().numpy(), gw_ref)
    mouts = mod.flashlog_forward_max_cuda(At, wt, active, *full, R, False, use_topk, K)
    mref = O.dense_max_forward(A, w, csr, masks, R, topk_edges=budget)
    for o, rf in zip(mouts, mref):
        got = o.cpu().numpy()
        assert np.array_equal(bits(got) if got.dtype == np.float32 else got, bits(rf) if rf.dtype == np.float32 else rf)
    gA, gw = mod.flashlog_backward_max_cuda(*gt, mouts[3], mouts[4], At, wt, active, *full, R, False, use_topk, K)
    gA_ref, gw_ref = O.dense_max_backward(*g, mref[3], mref[4], A, w, csr, masks, R, topk_edges=budget)
    assert np.array_equal(bits(gA.cpu().numpy()), bits(gA_ref))
    assert_grad_close(gw.cpu().numpy(), gw_ref)


def test_normalize_pair():
    mod = _mod()
    dev = torch.device("cuda")
    rng = np.random.default_rng(2)
    B, L = 3, 2
    rows = [(b, l) for b in range(B) for l in range(L) if (b, l) != (1, 0)]  # row (1, 0) empty
    b = np.concatenate([np.full(4, bb) for bb, _ in rows]).astype(np.int64)
    l = np.concatenate([np.full(4, ll) for _, ll in rows]).astype(np.int64)
    v = rng.random(b.size).astype(np.float32)
    out, denom, rs, re = mod.sparse3d_normalize_forward_cuda(torch.from_numpy(b).to(dev), torch.from_numpy(l).to(dev),
                                                             torch.from_numpy(v).to(dev), B, L, 1e-7)
    want, want_d = O.sparse_normalize(b, l, v, B, L)
    assert np.array_equal(bits(out.cpu().numpy()), bits(want))
    assert tuple(denom.shape) == (B, L) and np.array_equal(bits(denom.cpu().numpy().reshape(-1)), bits(want_d))
    g = rng.standard_normal(v.size).astype(np.float32)
    gt = torch.from_numpy(g).to(dev)
    vt = torch.from_numpy(v).to(dev)
    ga = mod.sparse3d_normalize_backward_cuda(gt, vt, denom, rs, re, 1e-7)
    # the reference marks the empty row (0, 0)
    rs2, re2 = rs.clone(), re.clone()
    rs2[2] = 0
    re2[2] = 0
    gb = mod.sparse3d_normalize_backward_cuda(gt, vt, denom, rs2, re2, 1e-7)
    assert torch.equal(ga, gb)
    row = b * L + l
    d = want_d[row].astype(np.float64)
    sgv = np.zeros(B * L)
    np.add.at(sgv, row, g.astype(np.float64) * v)
    np.testing.assert_allclose(ga.cpu().numpy(), g / d - sgv[row] / d ** 2, rtol=1e-5, atol=1e-6)


def test_fixed_relation_and_ranks():
    mod = _mod()
    dev = torch.device("cuda")
    rng = np.random.default_rng(4)
    h, r, t, E, R, csr = small_graph(3, 0.02)
    B, L = 2, 3
    b = np.repeat(np.arange(B), L * 4)
    l = np.tile(np.repeat(np.arange(L), 4), B)
    e = np.concatenate([np.sort(rng.choice(E, 4, replace=False)) for _ in range(B * L)])
    v = rng.integers(1, 4, b.size).astype(np.float32)
    ops = rng.integers(0, 2 * R + 1, (B, L))
    c = [torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in csr]
    ob, ol, oe, ov = mod.flashlog_forward_sparse3d_fixed_relation_cuda(
        *(torch.from_numpy(x).to(dev) for x in (b, l, e, v)), torch.from_numpy(ops).to(dev),
        c[1], c[8], c[9], c[10], c[11], c[5], c[12], c[13], c[14], c[15], B, L, E, R)
    got = {(int(x), int(y), int(z)): float(q) for x, y, z, q in zip(ob.cpu(), ol.cpu(), oe.cpu(), ov.cpu())}
    assert got == O.fixed_relation_step(b, l, e, v, ops, h, r, t, E, R)
    qb = np.repeat(np.arange(4), 30)
    qe = np.concatenate([np.sort(rng.choice(E, 30, replace=False)) for _ in range(4)])
    qv = rng.integers(0, 5, qb.size).astype(np.float32)
    tg = qe[::30].copy()
    keys = np.unique(qb[::7] * E + qe[::7])
    ranks = mod.sparse2d_filtered_ranks_cuda(*(torch.from_numpy(x).to(dev) for x in (qb, qe, qv, tg, keys)), 4, E,
                                             True)
    assert np.array_equal(ranks.cpu().numpy(), O.filtered_ranks(qb, qe, qv, tg, keys, 4, E, True))
