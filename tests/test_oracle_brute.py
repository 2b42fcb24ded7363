"""Pins of the C oracle that do not depend on the reference build: brute
force on tiny inputs and float64 closed forms, chosen so that a dropped term,
a wrong index or a transposed operand fails."""
import numpy as np
import pytest
from hypothesis import given, settings, strategies as st

from oracle import oracle as O
from tests.helpers import attention, masks_for, small_graph, sparse_state


@settings(max_examples=300, deadline=None)
@given(st.lists(st.integers(0, 6), min_size=1, max_size=12),
       st.lists(st.integers(1, 9), min_size=12, max_size=12),
       st.integers(1, 40))
def test_group_threshold_equals_expanded_sort(wq, sizes, budget):
    # weights drawn from a tiny set -> many exact ties; weight 0 is ineligible
    weights = np.array([0.0, 0.125, 0.25, 0.25, 0.5, 0.75, 1.0], np.float32)
    rel = np.array(wq, np.int16)
    cnt = np.array(sizes[: len(wq)], np.int32)
    got = O.group_threshold(weights, rel, cnt, budget)
    want = O.group_threshold_brute(weights, rel, cnt, budget)
    assert got == want


def _kept_brute(A, w, csr, masks, R, K):
    """Closed-form float64 dense hop with c2 by expanding every (source, row)
    into its edges: keep the K heaviest eligible edges, ties in CSR order."""
    BL, E = A.shape
    outs = []
    for side, (col, gptr, grel, gstart, gcount, off, m) in enumerate(
            [(csr[1], csr[8], csr[9], csr[10], csr[11], 0, masks[0]),
             (csr[5], csr[12], csr[13], csr[14], csr[15], R, masks[1])]):
        out = np.zeros((BL, E), np.float64)
        for bl in range(BL):
            for s in np.nonzero(A[bl])[0]:
                edges = []
                for g in range(gptr[s], gptr[s + 1]):
                    wv = w[bl, off + grel[g]]
                    if wv > 0:
                        edges += [(-float(wv), p, wv) for p in range(gstart[g], gstart[g] + gcount[g])]
                edges.sort()
                if K is not None:
                    edges = edges[:K]
                for _, p, wv in edges:
                    if m[p] != 0:
                        out[bl, col[p]] += float(A[bl, s]) * float(wv) * float(m[p])
        outs.append(out)
    return outs


@pytest.mark.parametrize("K", [None, 1, 2, 5])
def test_dense_forward_closed_form(K):
    rng = np.random.default_rng(5)
    h, r, t, E, R, csr = small_graph(2, 0.01, seed=11)
    n = 2 * R + 1
    A = sparse_state(6, E, 25, rng)
    w = attention(6, n, rng)
    w[1, :R] = w[1, 0]
    _, masks = masks_for(csr, h.shape[0], rng, drop=0.2)
    o = O.dense_forward(A, w, csr, masks, R, topk_edges=K if K else 1 << 60)
    ori, inv = _kept_brute(A, w, csr, masks, R, K)
    np.testing.assert_allclose(o[1], ori, rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(o[2], inv, rtol=2e-6, atol=1e-7)
    np.testing.assert_array_equal(o[0], A * w[:, -1:])


def test_dense_backward_is_adjoint_of_forward():
    """<g, F(A, w)> is bilinear in (A, w) per hop without pruning; its
    gradient must equal the oracle backward (float64 check)."""
    rng = np.random.default_rng(9)
    h, r, t, E, R, csr = small_graph(2, 0.01, seed=12)
    n = 2 * R + 1
    A = sparse_state(4, E, 20, rng)
    w = attention(4, n, rng)
    _, masks = masks_for(csr, h.shape[0], rng)
    g = [rng.standard_normal(A.shape) for _ in range(3)]
    gA, gw = O.dense_backward(*[x.astype(np.float32) for x in g], A, w, csr, masks, R)
    # closed form via float64 dense operators
    BL = A.shape[0]
    want_gA = g[0] * w[:, -1:].astype(np.float64)
    want_gw = np.zeros((BL, n))
    want_gw[:, -1] = (g[0] * A).sum(1)
    for (col, gptr, grel, gstart, gcount, off, m, gg) in [
            (csr[1], csr[8], csr[9], csr[10], csr[11], 0, masks[0], g[1]),
            (csr[5], csr[12], csr[13], csr[14], csr[15], R, masks[1], g[2])]:
        for s in range(E):
            for grp in range(gptr[s], gptr[s + 1]):
                rel = off + grel[grp]
                for p in range(gstart[grp], gstart[grp] + gcount[grp]):
                    act = A[:, s] != 0
                    want_gA[act, s] += gg[act, col[p]] * w[act, rel] * m[p]
                    want_gw[act, rel] += gg[act, col[p]] * A[act, s] * m[p]
    np.testing.assert_allclose(gA, want_gA, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(gw, want_gw, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("c", [0, 1, 3, 10, 40])
def test_dense_topc_matches_stable_sort(c):
    rng = np.random.default_rng(c)
    A = sparse_state(7, 200, 30, rng, ties=True)
    A[2, :] = 0
    A[3, 5:8] = -0.5  # negative nonzeros compete by value
    out, cutoff, last, changed = O.dense_topc(A, c)
    keep = O.dense_topc_brute(A, c)
    np.testing.assert_array_equal(out.view(np.int32), (A * keep.astype(np.float32)).view(np.int32))


def test_dense_max_forward_brute():
    rng = np.random.default_rng(3)
    h, r, t, E, R, csr = small_graph(2, 0.01, seed=13)
    n = 2 * R + 1
    A = sparse_state(5, E, 15, rng, ties=True)
    w = attention(5, n, rng)
    _, masks = masks_for(csr, h.shape[0], rng)
    oi, oo, ov, ao, av = O.dense_max_forward(A, w, csr, masks, R)
    for side, (col, gptr, grel, gstart, gcount, off, m, out, arg) in enumerate(
            [(csr[1], csr[8], csr[9], csr[10], csr[11], 0, masks[0], oo, ao),
             (csr[5], csr[12], csr[13], csr[14], csr[15], R, masks[1], ov, av)]):
        best = {}
        for bl in range(A.shape[0]):
            for s in np.nonzero(A[bl])[0]:
                for g in range(gptr[s], gptr[s + 1]):
                    wv = w[bl, off + grel[g]]
                    if wv <= 0:
                        continue
                    for p in range(gstart[g], gstart[g] + gcount[g]):
                        if m[p] == 0:
                            continue
                        v = np.float32(np.float32(A[bl, s] * wv) * m[p])
                        key = (bl, col[p])
                        if key not in best or v > best[key][0] or (v == best[key][0] and p < best[key][1]):
                            best[key] = (v, p)
        exp_v = np.zeros_like(out)
        exp_a = np.full(arg.shape, -1, np.int64)
        for (bl, d), (v, p) in best.items():
            exp_v[bl, d], exp_a[bl, d] = v, p
        np.testing.assert_array_equal(out, exp_v)
        np.testing.assert_array_equal(arg, exp_a)


@pytest.mark.parametrize("use_eql", [False, True])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("target_filtered", [True, False])
def test_filtered_ranks_brute(use_eql, dtype, target_filtered):
    rng = np.random.default_rng(1)
    B, E = 6, 50
    S = np.where(rng.random((B, E)) < 0.3, rng.integers(0, 4, (B, E)) / 4.0, 0.0).astype(dtype)
    targets = rng.integers(0, E, B)
    filt = rng.random((B, E)) < 0.1
    filt[np.arange(B), targets] = target_filtered
    b, e = np.nonzero(S)
    keys = np.nonzero(filt.reshape(-1))[0]
    got = O.filtered_ranks(b, e, S[b, e], targets, keys, B, E, use_eql)
    want = O.filtered_ranks_brute(S, targets, filt, use_eql)
    np.testing.assert_allclose(got, want)


@pytest.mark.parametrize("K", [1 << 60, 2])
@pytest.mark.parametrize("wot_i", [False, True])
def test_dense_max_backward_brute(K, wot_i):
    """Winner-only gradient, rebuilt in float64 from the per-position arrays
    (row_ptr / r_ind), not from the group walk the oracle uses."""
    rng = np.random.default_rng(4)
    h, r, t, E, R, csr = small_graph(2, 0.01, seed=17)
    n = 2 * R + 1
    BL = 5
    A = sparse_state(BL, E, 15, rng, ties=True)
    w = attention(BL, n, rng)
    _, masks = masks_for(csr, h.shape[0], rng)
    oi, oo, ov, ao, av = O.dense_max_forward(A, w, csr, masks, R, wot_i=wot_i, topk_edges=K)
    g = [rng.standard_normal((BL, E)).astype(np.float32) for _ in range(3)]
    g[1][rng.random((BL, E)) < 0.3] = 0.0
    gA, gw = O.dense_max_backward(*g, ao, av, A, w, csr, masks, R, wot_i=wot_i, topk_edges=K)
    eA = np.zeros((BL, E))
    ew = np.zeros((BL, n))
    if not wot_i:
        eA += g[0].astype(np.float64) * w[:, -1:].astype(np.float64)
        ew[:, -1] = (g[0].astype(np.float64) * A).sum(1)
    for side, (rp, ri, off, m, grad, arg) in enumerate([(csr[0], csr[2], 0, masks[0], g[1], ao),
                                                       (csr[4], csr[6], R, masks[1], g[2], av)]):
        for bl, d in zip(*np.nonzero(arg >= 0)):
            p = arg[bl, d]
            s = np.searchsorted(rp, p, side="right") - 1
            go = float(grad[bl, d])
            if go == 0.0:
                continue
            col = off + int(ri[p])
            eA[bl, s] += go * float(w[bl, col]) * float(m[p])
            ew[bl, col] += go * float(A[bl, s]) * float(m[p])
    np.testing.assert_allclose(gA, eA, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(gw, ew, rtol=1e-5, atol=1e-5)
