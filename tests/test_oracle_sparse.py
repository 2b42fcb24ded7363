"""Pins of the sparse (COO) oracle: bit-equality with the reference's own CPU
sparse path (oracle/_ref), float64 closed forms, an adjoint identity for the
backward, and a brute-force c1 rule."""
import os
import sys

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import attention, masks_for, small_graph, sparse_coo_state

REF_DIR = os.path.join(os.path.dirname(os.path.dirname(__file__)), "oracle", "_ref")


def _ref():
    sys.path.insert(0, REF_DIR)
    try:
        import torch  # noqa: F401
        import flashlog_ref_cpp
        return flashlog_ref_cpp
    except ImportError:
        pytest.skip("reference CPU module not built (oracle/Makefile.ref)")


def _expand64(mode, b, l, e, v, L, E, w, csr, masks, R, wot_i, K):
    """float64 closed form: dict key -> value, over the explicit edge list."""
    out = {}
    sides = [(csr[8], csr[9], csr[10], csr[11], csr[1], masks[0], 0),
             (csr[12], csr[13], csr[14], csr[15], csr[5], masks[1], R)]
    n = w.shape[-1]
    wf = w.reshape(-1, n)
    for i in range(v.shape[0]):
        row = b[i] * L + l[i]
        for gp, gr, gs, gc, col, m, off in sides:
            groups = range(gp[e[i]], gp[e[i] + 1])
            if mode == O.SPARSE_TOPK:
                # kept edges: the K heaviest eligible, ties in group order (brute force)
                edges = [(float(wf[row, off + gr[g]]), g, p) for g in groups
                         for p in range(gs[g], gs[g] + gc[g]) if wf[row, off + gr[g]] > 0]
                order = sorted(range(len(edges)), key=lambda j: (-edges[j][0], j))
                kept = sorted(order[:K]) if K < len(edges) else list(range(len(edges)))
                items = [(edges[j][2], edges[j][0]) for j in kept if m[edges[j][2]] != 0]
            else:
                items = [(p, float(wf[row, off + gr[g]])) for g in groups for p in range(gs[g], gs[g] + gc[g])]
            for p, wv in items:
                key = row * E + int(col[p])
                out[key] = out.get(key, 0.0) + float(v[i]) * wv * float(m[p])
        if not wot_i:
            key = row * E + int(e[i])
            out[key] = out.get(key, 0.0) + float(v[i]) * float(wf[row, n - 1])
    return out


@pytest.mark.parametrize("cfg,scale", [(1, 0.03), (2, 0.03), (3, 0.01)])
@pytest.mark.parametrize("K", [1 << 60, 2, 200])
@pytest.mark.parametrize("wot_i", [False, True])
def test_sparse_oracle_matches_reference_build(cfg, scale, K, wot_i):
    import torch
    ref = _ref()
    torch.set_num_threads(1)
    rng = np.random.default_rng(cfg * 7 + (K % 5) + wot_i)
    h, r, t, E, R, csr = small_graph(cfg, scale)
    B, L = 3, 2
    n = 2 * R + 1
    b, l, e, v = sparse_coo_state(B, L, E, 25, rng, ties=K == 2)
    w = attention(B * L, n, rng).reshape(B, L, n)
    if K == 2:
        w[..., : n // 2] = w[..., :1]
    _, masks = masks_for(csr, h.shape[0], rng)
    T = lambda x: torch.from_numpy(np.ascontiguousarray(x))
    args = (T(csr[1]), T(masks[0]), T(csr[8]), T(csr[9]), T(csr[10]), T(csr[11]), T(csr[5]), T(masks[1]),
            T(csr[12]), T(csr[13]), T(csr[14]), T(csr[15]))
    ro = ref.flashlog_forward_sparse3d_sum_cpu(T(b), T(l), T(e), T(v), T(w), *args, B, L, E, R, wot_i, K)
    keys, vals = O.sparse_forward(O.SPARSE_TOPK, b, l, e, v, B, L, E, w, csr, masks, R, wot_i, K)
    rkeys = (ro[0].numpy() * L + ro[1].numpy()) * E + ro[2].numpy()
    assert np.array_equal(keys, rkeys)
    assert np.array_equal(vals.view(np.int32), ro[3].numpy().view(np.int32))
    # the fused sum + normalize CPU path: the oracle's normalization of the oracle's sum
    rn = ref.flashlog_forward_sparse3d_sum_norm_cpu(T(b), T(l), T(e), T(v), T(w), *args, B, L, E, R, wot_i, K,
                                                     1e-7, False)
    ob, ol = keys // (L * E), (keys // E) % L
    nv, _ = O.sparse_normalize(ob, ol, vals, B, L, 1e-7)
    assert np.array_equal(nv.view(np.int32), rn[3].numpy().view(np.int32))


@pytest.mark.parametrize("cfg,scale", [(1, 0.03), (2, 0.03), (3, 0.01)])
@pytest.mark.parametrize("K", [1 << 60, 2, 200])
@pytest.mark.parametrize("wot_i", [False, True])
@pytest.mark.parametrize("soft", [False, True])
def test_sparse_backward_matches_reference_build(cfg, scale, K, wot_i, soft):
    """or_sparse_backward element by element against the reference's
    flashlog_backward_sparse3d_sum_cpu (oracle/_ref) on one thread, fed the
    raw metadata of its own forward: with 0/1 masks bit for bit (per entry
    the ORI items, the INV items, then the identity term, in raw order; per
    (row, column) the items in raw order); with fractional masks within
    1e-6 of the largest gradient (the GPU path's (g*m)*w against the CPU
    path's (g*w)*m)."""
    import torch
    ref = _ref()
    torch.set_num_threads(1)
    rng = np.random.default_rng(cfg * 11 + (K % 5) + 3 * wot_i + 7 * soft)
    h, r, t, E, R, csr = small_graph(cfg, scale)
    B, L = 3, 2
    n = 2 * R + 1
    b, l, e, v = sparse_coo_state(B, L, E, 25, rng, ties=K == 2)
    w = attention(B * L, n, rng).reshape(B, L, n)
    _, masks = masks_for(csr, h.shape[0], rng)
    if soft:
        masks = tuple((m * rng.uniform(0.25, 1.0, m.shape[0])).astype(np.float32) for m in masks)
    T = lambda x: torch.from_numpy(np.ascontiguousarray(x))
    args = (T(csr[1]), T(masks[0]), T(csr[8]), T(csr[9]), T(csr[10]), T(csr[11]), T(csr[5]), T(masks[1]),
            T(csr[12]), T(csr[13]), T(csr[14]), T(csr[15]))
    ro = ref.flashlog_forward_sparse3d_sum_cpu(T(b), T(l), T(e), T(v), T(w), *args, B, L, E, R, wot_i, K)
    keys, vals = O.sparse_forward(O.SPARSE_TOPK, b, l, e, v, B, L, E, w, csr, masks, R, wot_i, K)
    g = rng.standard_normal(keys.shape[0]).astype(np.float32)
    g[rng.random(g.shape[0]) < 0.2] = 0.0
    rgv, rgw = ref.flashlog_backward_sparse3d_sum_cpu(ro[0], ro[1], ro[2], T(g), T(b), T(l), T(e), T(v), T(w),
                                                      *ro[4:16], B, L, E, R, wot_i)
    gv, gw = O.sparse_backward(O.SPARSE_TOPK, b, l, e, v, B, L, E, w, csr, masks, R, keys, g, wot_i, K)
    rgv, rgw = rgv.numpy(), rgw.numpy().reshape(B * L, n)
    if soft:  # differently rounded terms: compare against the size of the sums
        np.testing.assert_allclose(gv, rgv, rtol=1e-6, atol=1e-6 * float(np.abs(rgv).max()))
        np.testing.assert_allclose(gw, rgw, rtol=1e-6, atol=1e-6 * float(np.abs(rgw).max()))
    else:
        assert np.array_equal(gv.view(np.int32), rgv.view(np.int32))
        assert np.array_equal(gw.view(np.int32), rgw.view(np.int32))


@pytest.mark.parametrize("mode", [O.SPARSE_TOPK, O.SPARSE_ALL])
@pytest.mark.parametrize("K", [1 << 60, 3])
def test_sparse_oracle_closed_form(mode, K):
    rng = np.random.default_rng(31 + mode + K % 7)
    h, r, t, E, R, csr = small_graph(2, 0.02, seed=5)
    B, L = 2, 3
    n = 2 * R + 1
    b, l, e, v = sparse_coo_state(B, L, E, 12, rng)
    w = attention(B * L, n, rng).reshape(B, L, n)
    w[0, 0, 1] = 0.0  # a zero weight: skipped by the top-k path, kept (0-valued) by all-edges
    _, masks = masks_for(csr, h.shape[0], rng, drop=0.3)
    kk = K if mode == O.SPARSE_TOPK else 1 << 60
    keys, vals = O.sparse_forward(mode, b, l, e, v, B, L, E, w, csr, masks, R, False, kk)
    want = _expand64(mode, b, l, e, v, L, E, w, csr, masks, R, False, kk)
    assert keys.tolist() == sorted(want)
    np.testing.assert_allclose(vals, [want[k] for k in keys.tolist()], rtol=2e-6, atol=1e-12)


def test_sparse_modes_agree_without_masks():
    rng = np.random.default_rng(8)
    h, r, t, E, R, csr = small_graph(3, 0.01)
    B, L = 2, 2
    n = 2 * R + 1
    b, l, e, v = sparse_coo_state(B, L, E, 30, rng)
    w = attention(B * L, n, rng).reshape(B, L, n)
    masks = (np.ones(h.shape[0], np.float32), np.ones(h.shape[0], np.float32))
    k0, v0 = O.sparse_forward(O.SPARSE_TOPK, b, l, e, v, B, L, E, w, csr, masks, R)
    k1, v1 = O.sparse_forward(O.SPARSE_ALL, b, l, e, v, B, L, E, w, csr, masks, R)
    assert np.array_equal(k0, k1) and np.array_equal(v0.view(np.int32), v1.view(np.int32))


@pytest.mark.parametrize("mode", [O.SPARSE_TOPK, O.SPARSE_ALL])
@pytest.mark.parametrize("wot_i", [False, True])
def test_sparse_backward_adjoint(mode, wot_i):
    """The hop is bilinear in (v, w): for any upstream g,
    <g, out> = <grad_v, v> = <grad_w, w> (float64 sums, tolerance)."""
    rng = np.random.default_rng(13 + mode + 2 * wot_i)
    h, r, t, E, R, csr = small_graph(2, 0.02, seed=9)
    B, L = 2, 3
    n = 2 * R + 1
    b, l, e, v = sparse_coo_state(B, L, E, 15, rng)
    w = attention(B * L, n, rng).reshape(B, L, n)
    _, masks = masks_for(csr, h.shape[0], rng)
    K = 4 if mode == O.SPARSE_TOPK else 1 << 60
    keys, vals = O.sparse_forward(mode, b, l, e, v, B, L, E, w, csr, masks, R, wot_i, K)
    g = rng.standard_normal(keys.shape[0]).astype(np.float32)
    gv, gw = O.sparse_backward(mode, b, l, e, v, B, L, E, w, csr, masks, R, keys, g, wot_i, K)
    lhs = float(np.dot(g.astype(np.float64), vals.astype(np.float64)))
    assert abs(lhs - float(np.dot(gv.astype(np.float64), v))) <= 1e-5 * (1 + abs(lhs))
    assert abs(lhs - float(np.sum(gw.astype(np.float64) * w.reshape(B * L, n)))) <= 1e-5 * (1 + abs(lhs))


@pytest.mark.parametrize("c", [0, 1, 3, 10])
def test_sparse_topc_brute(c):
    rng = np.random.default_rng(c)
    b, l, e, v = sparse_coo_state(3, 2, 60, 12, rng, ties=True)
    v[::7] = 0.0  # explicit zeros
    kept = set(O.sparse_topc(b, l, v, 2, c).tolist())
    rows = b * 2 + l
    for r in np.unique(rows):
        idx = [i for i in range(v.shape[0]) if rows[i] == r]
        nz = [i for i in idx if v[i] != 0]
        if len(nz) <= c:
            assert all(i in kept for i in idx)
        else:
            ranked = sorted(nz, key=lambda i: (-float(v[i]), i))[:c]
            assert sorted(i for i in idx if i in kept) == sorted(ranked)


def test_sparse_normalize_closed_form():
    rng = np.random.default_rng(2)
    b, l, e, v = sparse_coo_state(4, 3, 100, 20, rng)
    out, denom = O.sparse_normalize(b, l, v, 4, 3, 1e-7)
    row = b * 3 + l
    d = np.zeros(12)
    np.add.at(d, row, v.astype(np.float64))
    np.testing.assert_allclose(denom, d, rtol=1e-6)
    np.testing.assert_allclose(out, v / np.maximum(d[row], 1e-7), rtol=1e-6)


def _coalesced_state(rng, B, L, E, n):
    keys = np.unique(rng.choice(B * L * E, size=n, replace=False))
    return keys // (L * E), (keys // E) % L, keys % E


def test_sum_sp_3d_matches_brute_force_and_torch():
    import torch
    rng = np.random.default_rng(7)
    B, L, E = 6, 3, 50
    b, l, e = _coalesced_state(rng, B, L, E, 400)
    v = (rng.integers(1, 256, b.shape[0]) / 64.0).astype(np.float32)  # dyadic: sums exact in any order
    ob, oe, ov, slot = O.sum_sp_3d(b, l, e, v, B, L, E)
    acc = {}
    for bb, ee, vv in zip(b.tolist(), e.tolist(), v.tolist()):
        acc[(bb, ee)] = acc.get((bb, ee), 0.0) + vv
    ks = sorted(acc)
    assert [(int(x), int(y)) for x, y in zip(ob, oe)] == ks
    assert np.array_equal(ov, np.array([acc[k] for k in ks], np.float32))
    t = torch.sparse_coo_tensor(torch.from_numpy(np.stack([b, e])), torch.from_numpy(v), [B, E]).coalesce()
    assert np.array_equal(t.indices().numpy(), np.stack([ob, oe]))
    assert np.array_equal(t.values().numpy().view(np.int32), ov.view(np.int32))
    assert np.array_equal(ob[slot], b) and np.array_equal(oe[slot], e)


def test_sum_sp_3d_adds_in_channel_order():
    # 1e8 + 1 rounds back to 1e8 in float32, so the result depends on the order
    b = np.zeros(3, np.int64)
    l = np.arange(3, dtype=np.int64)
    e = np.full(3, 4, np.int64)
    _, _, ov, _ = O.sum_sp_3d(b, l, e, np.array([1e8, 1.0, -1e8], np.float32), 1, 3, 9)
    assert ov.tolist() == [0.0]
    _, _, ov, _ = O.sum_sp_3d(b, l, e, np.array([1e8, -1e8, 1.0], np.float32), 1, 3, 9)
    assert ov.tolist() == [1.0]
    _, _, ov, slot = O.sum_sp_3d(np.zeros(0), np.zeros(0), np.zeros(0), np.zeros(0, np.float32), 2, 3, 9)
    assert ov.shape == (0,) and slot.shape == (0,)
