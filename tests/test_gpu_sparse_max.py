"""GPU parity of the sparse max hop (FlashLogFunctionSparse3DTopKMax) and of
the training selections (quota c2, exponential-race c1,
sampled_sparse_propagation) against the oracle: coordinates, values and
winners bit for bit, gradients within 1e-5 relative."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_grad_close, attention, bits, masks_for, small_graph, sparse_coo_state, to_torch_csr

pytestmark = pytest.mark.gpu


def _fk():
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    return fk


def _case(cfg, scale, B, L, per_row, seed, ties=False, drop=0.1):
    rng = np.random.default_rng(seed)
    h, r, t, E, R, csr = small_graph(cfg, scale)
    n = 2 * R + 1
    b, l, e, v = sparse_coo_state(B, L, E, per_row, rng, ties=ties)
    w = attention(B * L, n, rng).reshape(B, L, n)
    if ties:
        w[..., : n // 2] = w[..., :1]
    mbool, masks = masks_for(csr, h.shape[0], rng, drop=drop)
    return rng, E, R, n, csr, mbool, masks, (b, l, e, v), w


def _keys(idx, L, E):
    idx = idx.cpu().numpy()
    return (idx[0] * L + idx[1]) * E + idx[2]


def _dev(*arrs):
    return [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in arrs]


def _hop(cls, state, w, csr, mbool, B, L, E, R, K, c1=None, wot_i=False, grad=False, sampling=False):
    b, l, e, v = _dev(*state)
    v.requires_grad_(grad)
    wt = torch.from_numpy(w).cuda().requires_grad_(grad)
    tc = to_torch_csr(csr, torch.device("cuda"))
    mk = torch.from_numpy(mbool).cuda()
    out = cls.apply(b, l, e, v, wt, *tc[:4], *tc[4:8], *tc[8:16], mk, None, B, L, E, R, wot_i, K, False, c1,
                    True, sampling)
    return out, v, wt


def _max(*a, **k):
    return _hop(_fk().FlashLogFunctionSparse3DTopKMax, *a, **k)


def _sum(*a, **k):
    return _hop(_fk().FlashLogFunctionSparse3DTopKSum, *a, **k)


def _check_max(out, v, wt, state, w, csr, masks, B, L, E, R, n, K, wot_i, rng, seed=-1, grad=True):
    keys, vals, went, wdir, wpos = O.sparse_max_forward(*state, B, L, E, w, csr, masks, R, wot_i, K, seed)
    assert np.array_equal(_keys(out.indices().detach(), L, E), keys)
    assert np.array_equal(bits(out.values().detach().cpu().numpy()), bits(vals))
    if not grad:
        return
    g = rng.standard_normal(keys.shape[0]).astype(np.float32)
    (out.values() * torch.from_numpy(g).cuda()).sum().backward()
    gv, gw = O.sparse_max_backward(state[0], state[1], state[3], B, L, w, csr, masks, R, g, went, wdir, wpos)
    assert_grad_close(v.grad.cpu().numpy(), gv)
    assert_grad_close(wt.grad.reshape(B * L, n).cpu().numpy(), gw)


@pytest.mark.parametrize("K", [2, 7, 200, 1 << 60])
@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("wot_i", [False, True])
def test_sparse_max_bitexact(K, ties, wot_i):
    B, L = 4, 3
    rng, E, R, n, csr, mbool, masks, state, w = _case(2, 1.0, B, L, 250, 140 + K % 13 + ties + 2 * wot_i,
                                                      ties=ties, drop=0.2)
    out, v, wt = _max(state, w, csr, mbool, B, L, E, R, K, wot_i=wot_i, grad=True)
    _check_max(out, v, wt, state, w, csr, masks, B, L, E, R, n, K, wot_i, rng)


@pytest.mark.parametrize("c1", [0, 5, 40])
def test_sparse_max_with_c1(c1):
    B, L = 3, 3
    rng, E, R, n, csr, mbool, masks, state, w = _case(2, 0.3, B, L, 80, 170 + c1, ties=True)
    kept = O.sparse_topc(state[0], state[1], state[3], L, c1)
    sel = tuple(a[kept] for a in state)
    keys, vals, *_ = O.sparse_max_forward(*sel, B, L, E, w, csr, masks, R, False, 3)
    out, v, wt = _max(state, w, csr, mbool, B, L, E, R, 3, c1=c1, grad=True)
    assert np.array_equal(_keys(out.indices().detach(), L, E), keys)
    assert np.array_equal(bits(out.values().detach().cpu().numpy()), bits(vals))
    g = torch.randn(out.values().shape, device="cuda")
    (out.values() * g).sum().backward()
    dropped = np.setdiff1d(np.arange(state[3].shape[0]), kept)
    assert np.all(v.grad.cpu().numpy()[dropped] == 0)


def test_sparse_max_hot_destination():
    """Most edges end at one destination: buckets far above one LDS chunk
    (the dense-LDS max path), E above one bucket, ties from repeated values."""
    rng = np.random.default_rng(31)
    E, R, M = 20000, 5, 60000
    h = rng.integers(0, E, M)
    t = np.where(rng.random(M) < 0.7, 12345, rng.integers(0, E, M))
    r = rng.integers(0, R, M)
    csr = O.build_csr_structure(h, t, r, E)
    n = 2 * R + 1
    B, L = 2, 2
    b, l, e, v = sparse_coo_state(B, L, E, 1500, rng, ties=True)
    w = attention(B * L, n, rng).reshape(B, L, n)
    w[..., :R] = w[..., :1]
    mbool, masks = masks_for(csr, M, rng, drop=0.05)
    state = (b, l, e, v)
    for K in (6, 1 << 60):
        out, vt, wt = _max(state, w, csr, mbool, B, L, E, R, K, grad=True)
        _check_max(out, vt, wt, state, w, csr, masks, B, L, E, R, n, K, False, rng)


def test_sparse_max_masked_edges_keep_coordinates():
    B, L = 2, 2
    rng, E, R, n, csr, mbool, masks, state, w = _case(2, 0.2, B, L, 60, 7, drop=0.5)
    out, _, _ = _max(state, w, csr, mbool, B, L, E, R, 1 << 60)
    s_out, _, _ = _sum(state, w, csr, mbool, B, L, E, R, 1 << 60)
    mk = set(_keys(out.indices(), L, E).tolist())
    sk = set(_keys(s_out.indices(), L, E).tolist())
    assert sk < mk
    zero = out.values().detach().cpu().numpy() == 0
    assert zero.sum() >= len(mk - sk)


@pytest.mark.parametrize("agg", ["sum", "max"])
@pytest.mark.parametrize("K", [1, 3, 40])
@pytest.mark.parametrize("seed", [0, 987654321])
@pytest.mark.parametrize("graph,weights", [("c2", "softmax"), ("c2", "wide"), ("many", "softmax"),
                                           ("many", "wide")])
def test_quota_hop_bitexact(agg, K, seed, graph, weights):
    """The training quotas (fixed seed) through the internal hop, against the
    oracle's sequential restatement; forward bits and gradients.  "many":
    sources with 150 groups per side (quota carries across group windows);
    "wide": a fifth of the weights scaled by 2^-70, so the weight sums round
    and the sequential sum order is taken."""
    fk = _fk()
    if graph == "c2":
        B, L = 4, 3
        rng, E, R, n, csr, mbool, masks, state, w = _case(2, 1.0, B, L, 200, 300 + K + seed % 7, drop=0.2)
    else:
        rng, E, R, n, csr, mbool, masks, state, w, B, L = _many_groups_case(400 + K + seed % 7, False)
    if weights == "wide":
        w = np.where(rng.random(w.shape) < 0.2, w * np.float32(2.0 ** -70), w).astype(np.float32)
    tc = to_torch_csr(csr, torch.device("cuda"))
    om, im = _dev(*masks)
    mx = agg == "max"
    sides = fk._SparseSides(tc[1], om, tc[8], tc[9], tc[10], tc[11], tc[5], im, tc[12], tc[13], tc[14], tc[15],
                            tc[3] if mx else None, tc[7] if mx else None)
    b, l, e, v = _dev(*state)
    wt = torch.from_numpy(w).cuda()
    idx, vals, st = fk._sparse_forward(b, l, e, v, wt, sides, B, L, E, R, False, fk._SPARSE_TOPK, K, True,
                                       aggregate=fk._SPARSE_MAX if mx else fk._SPARSE_SUM, seed=seed)
    keys = _keys(idx, L, E)
    g = rng.standard_normal(keys.shape[0]).astype(np.float32)
    gv, gw = fk._sparse_backward(st, torch.from_numpy(g).cuda())
    if mx:
        rk, rv, went, wdir, wpos = O.sparse_max_forward(*state, B, L, E, w, csr, masks, R, False, K, seed)
        gv_ref, gw_ref = O.sparse_max_backward(state[0], state[1], state[3], B, L, w, csr, masks, R, g, went, wdir,
                                               wpos)
    else:
        rk, rv = O.sparse_forward(O.SPARSE_TOPK, *state, B, L, E, w, csr, masks, R, False, K, seed)
        gv_ref, gw_ref = O.sparse_backward(O.SPARSE_TOPK, *state, B, L, E, w, csr, masks, R, rk, g, False, K, seed)
    assert np.array_equal(keys, rk)
    assert np.array_equal(bits(vals.cpu().numpy()), bits(rv))
    assert_grad_close(gv.cpu().numpy(), gv_ref)
    assert_grad_close(gw.cpu().numpy(), gw_ref)


@pytest.mark.parametrize("agg", ["sum", "max"])
def test_sampling_seed_drawn_like_reference(agg):
    """sampling=True draws the quota seed with one torch.randint on the CPU
    generator (flashlog_kernel.py:1201,1487); same torch seed, same bits."""
    B, L = 3, 2
    rng, E, R, n, csr, mbool, masks, state, w = _case(2, 1.0, B, L, 150, 77)
    torch.manual_seed(1234)
    out, _, _ = (_max if agg == "max" else _sum)(state, w, csr, mbool, B, L, E, R, 4, sampling=True)
    torch.manual_seed(1234)
    seed = int(torch.randint(0, 2 ** 63 - 1, ()).item())
    if agg == "max":
        keys, vals, *_ = O.sparse_max_forward(*state, B, L, E, w, csr, masks, R, False, 4, seed)
    else:
        keys, vals = O.sparse_forward(O.SPARSE_TOPK, *state, B, L, E, w, csr, masks, R, False, 4, seed)
    assert np.array_equal(_keys(out.indices().detach(), L, E), keys)
    assert np.array_equal(bits(out.values().detach().cpu().numpy()), bits(vals))


@pytest.mark.parametrize("c", [1, 6, 50])
def test_race_c1_matches_oracle(c):
    fk = _fk()
    rng = np.random.default_rng(c)
    B, L, E = 3, 2, 4000
    b, l, e, v = sparse_coo_state(B, L, E, 300, rng)
    v[rng.random(v.shape[0]) < 0.1] = 0.0  # explicit zeros: never candidates, dropped in over rows
    cand = O.sparse_topc_race_candidates(b, l, v, L, c)
    tb, tl, te, tv = _dev(b, l, e, v)
    torch.manual_seed(99)
    kept = fk._sparse_topc_entries(tb, tl, te, tv, c, L, sampling=True)
    torch.manual_seed(99)
    noise = torch.empty(cand.shape[0], dtype=torch.float64, device="cuda").exponential_()
    ref = O.sparse_topc_race(b, l, v, L, c, noise.cpu().numpy())
    assert kept is not None
    np.testing.assert_array_equal(kept.cpu().numpy(), ref)
    # the select's own compaction: the kept coordinates and values in entry order
    torch.manual_seed(99)
    ent, taken = fk._sparse_topc_select(tb, tl, te, tv, c, L, sampling=True)
    np.testing.assert_array_equal(ent.cpu().numpy(), ref)
    for got, full in zip(taken, (b, l, e, v)):
        np.testing.assert_array_equal(got.cpu().numpy(), full[ref])
    # validation: a negative candidate value is refused, as the reference does
    v2 = v.copy()
    v2[cand[0]] = -1.0
    with pytest.raises(ValueError):
        fk._sparse_topc_entries(tb, tl, te, torch.from_numpy(v2).cuda(), c, L, sampling=True)
    # no row over the budget: nothing pruned, no noise drawn
    assert fk._sparse_topc_entries(tb, tl, te, tv, 100000 if c > 1 else v.shape[0], L, sampling=True) is None


@pytest.mark.parametrize("nnz,E", [(1, 5), (5000, 7), (20000, 300000), (70000, 1000)])
def test_entry_order_groups_entities(nnz, E):
    """fl_sparse_entry_order: a permutation of the entries with ascending
    blocks of 64 entity ids (entries of one block in any order)."""
    fk = _fk()
    rng = np.random.default_rng(nnz)
    e = torch.from_numpy(rng.integers(0, E, nnz)).cuda()
    order = fk._entry_order(e, E).long().cpu().numpy()
    assert np.array_equal(np.sort(order), np.arange(nnz))
    assert np.all(np.diff(e.cpu().numpy()[order] >> 6) >= 0)


@pytest.mark.parametrize("mode", ["sum", "max"])
def test_sampled_sparse_propagation_two_hops(mode):
    """Two training hops with c1 and c2 through the public entry point:
    reproducible under torch's seed, budgets respected, gradients flow."""
    fk = _fk()
    rng = np.random.default_rng(5)
    h, r, t, E, R, csr = small_graph(2, 1.0)
    n = 2 * R + 1
    B, L = 4, 3
    tc = to_torch_csr(csr, torch.device("cuda"))
    mk = torch.from_numpy(masks_for(csr, h.shape[0], rng)[0]).cuda()
    w0 = torch.from_numpy(attention(B * L, n, rng).reshape(B, L, n)).cuda()
    src = torch.from_numpy(rng.integers(0, E, B)).cuda()

    def run(seed):
        torch.manual_seed(seed)
        w = w0.clone().requires_grad_(True)
        idx = torch.stack([torch.arange(B, device="cuda").repeat_interleave(L),
                           torch.arange(L, device="cuda").repeat(B), src.repeat_interleave(L)])
        s = torch.sparse_coo_tensor(idx, torch.ones(B * L, device="cuda"), (B, L, E)).coalesce()
        for _ in range(2):
            s = fk.sampled_sparse_propagation(s, w, tc, mk, R, None, False, 20, 5, mode)
            s = fk.normalize_sparse3d(s)
        loss = (s.values() ** 2).sum()
        loss.backward()
        return s.coalesce(), w.grad.clone()

    s1, g1 = run(3)
    s2, g2 = run(3)
    assert torch.equal(s1.indices(), s2.indices()) and torch.equal(s1.values(), s2.values())
    assert torch.equal(g1, g2)  # the backward adds in a fixed order: same bits on every run
    assert torch.isfinite(g1).all() and g1.abs().sum() > 0
    # c1 = 20 bounds each row's entries before the second hop: at most
    # 20 * (2 sides * 5 edges + identity) outputs per row
    rows = s1.indices()[0] * L + s1.indices()[1]
    assert int(torch.bincount(rows).max()) <= 20 * 11


@pytest.mark.parametrize("agg", ["sum", "max"])
def test_trainable_edge_weights(agg):
    """Soft edge weights (use_soft): masks mask*sigmoid(ew) and the edge-weight
    gradient of flashlog_kernel.py:1306-1336.  The forward bit for bit
    against the oracle fed the masks the GPU computed (their sigmoid within
    a few ulps of float64); the edge gradient, folded per position in a
    fixed order, within 1e-5 of a float64 brute force over the kept (sum)
    or winning (max) items, the same bits on a second backward, and a
    finite difference."""
    from tests.test_oracle_sparse_max import _kept_items
    B, L = 3, 2
    K = 4
    rng, E, R, n, csr, mbool, _, state, w = _case(2, 0.3, B, L, 60, 404 + (agg == "max"), drop=0.2)
    M = mbool.shape[0]
    ew = (rng.standard_normal(M) * 0.7).astype(np.float32)
    sig = (1.0 / (1.0 + np.exp(-ew.astype(np.float64))))
    masks = tuple((mbool[csr[o]] * sig[csr[o]]).astype(np.float32) for o in (3, 7))
    cls = _fk().FlashLogFunctionSparse3DTopKMax if agg == "max" else _fk().FlashLogFunctionSparse3DTopKSum
    b, l, e, v = _dev(*state)
    wt = torch.from_numpy(w).cuda()
    tc = to_torch_csr(csr, torch.device("cuda"))
    mk = torch.from_numpy(mbool).cuda()
    weight = torch.from_numpy(ew.reshape(M, 1)).cuda().requires_grad_(True)

    def fwd(wp):
        return cls.apply(b, l, e, v, wt, *tc[:4], *tc[4:8], *tc[8:16], mk, wp, B, L, E, R, False, K, False, None,
                         True, False)

    out = fwd(weight)
    keys = _keys(out.indices().detach(), L, E)
    gpu_masks = tuple(m.detach().cpu().numpy() for m in _fk().prepare_csr_masks(tc, mk, weight.detach()))
    for gm, m64 in zip(gpu_masks, masks):
        np.testing.assert_allclose(gm, m64, rtol=4e-7, atol=0)
    if agg == "max":
        rk, rv, went, wdir, wpos = O.sparse_max_forward(*state, B, L, E, w, csr, gpu_masks, R, False, K)
    else:
        rk, rv = O.sparse_forward(O.SPARSE_TOPK, *state, B, L, E, w, csr, gpu_masks, R, False, K)
    assert np.array_equal(keys, rk)
    assert np.array_equal(bits(out.values().detach().cpu().numpy()), bits(rv))
    g = rng.standard_normal(keys.shape[0]).astype(np.float32)
    (out.values() * torch.from_numpy(g).cuda()).sum().backward()
    ge = weight.grad.view(-1).cpu().numpy().astype(np.float64)
    first = weight.grad.clone()
    weight.grad = None
    (fwd(weight).values() * torch.from_numpy(g).cuda()).sum().backward()
    assert torch.equal(first, weight.grad)  # a fixed order: the same bits
    ref = np.zeros(M)
    pos = {int(k): o for o, k in enumerate(keys)}
    wf = w.reshape(-1, n).astype(np.float64)
    if agg == "max":
        for o in range(keys.shape[0]):
            if wdir[o] == 2:
                continue
            i, d, p = went[o], wdir[o], wpos[o]
            edge = int(csr[3 if d == 0 else 7][p])
            row = state[0][i] * L + state[1][i]
            col = (R if d else 0) + int(csr[6 if d else 2][p])
            m = float(masks[d][p])
            ref[edge] += g[o] * float(state[3][i]) * wf[row, col] * m * (1 - sig[edge])
    else:
        for key, val, d, edge, i, _, p in _kept_items(*state, L, w, csr, masks, R, K, False):
            if d == 2 or masks[d][p] == 0:
                continue
            row = state[0][i] * L + state[1][i]
            col = (R if d else 0) + int(csr[6 if d else 2][p])
            ref[edge] += g[pos[key]] * float(state[3][i]) * wf[row, col] * float(masks[d][p]) * (1 - sig[edge])
    assert_grad_close(ge, ref, rtol=1e-5)
    if agg == "max":
        return  # winners may switch under a perturbation: no finite difference
    # finite difference on the edges with the largest gradients
    gt = torch.from_numpy(g).cuda()
    for edge in np.argsort(-np.abs(ref))[:3]:
        d = torch.zeros(M, 1, device="cuda")
        d[edge] = 1e-2
        with torch.no_grad():
            fp = fwd(weight.detach() + d)
            fm = fwd(weight.detach() - d)
        lp = float((fp.values() * gt[:fp.values().numel()]).sum()) if fp._nnz() == keys.shape[0] else None
        lm = float((fm.values() * gt[:fm.values().numel()]).sum()) if fm._nnz() == keys.shape[0] else None
        if lp is None or lm is None:
            continue
        assert abs((lp - lm) / 2e-2 - ref[edge]) <= 2e-2 * abs(ref[edge]) + 1e-4


def _many_groups_case(seed, ties):
    """R = 150 relations; node 0 heads a group of every relation (1-4 edges
    each), node 7 receives every relation: sources with far more than 64
    groups per side, whose c2 threshold comes from the row's admission
    order.  Every row holds both hubs plus random entities."""
    rng = np.random.default_rng(seed)
    E, R = 3000, 150
    c0 = 1 + np.arange(R) % 4
    c7 = 1 + np.arange(R) % 3
    h = np.concatenate([np.zeros(c0.sum(), np.int64), rng.integers(0, E, c7.sum()), rng.integers(0, E, 20000)])
    t = np.concatenate([rng.integers(0, E, c0.sum()), np.full(c7.sum(), 7, np.int64), rng.integers(0, E, 20000)])
    r = np.concatenate([np.repeat(np.arange(R), c0), np.repeat(np.arange(R), c7), rng.integers(0, R, 20000)])
    csr = O.build_csr_structure(h, t, r, E)
    n = 2 * R + 1
    B, L = 2, 3
    b, l, e, v = sparse_coo_state(B, L, E, 60, rng)
    keep = (e != 0) & (e != 7)
    b, l, e, v = b[keep], l[keep], e[keep], v[keep]
    bl = np.concatenate([b * L + l, np.repeat(np.arange(B * L), 2)])
    e = np.concatenate([e, np.tile([0, 7], B * L)])
    v = np.concatenate([v, rng.random(2 * B * L).astype(np.float32) + 0.5])
    o = np.lexsort((e, bl))
    state = ((bl // L)[o], (bl % L)[o], e[o], v[o].astype(np.float32))
    w = attention(B * L, n, rng).reshape(B, L, n)
    w[rng.random(w.shape) < 0.15] = 0.0
    if ties:
        w[..., 10:R] = w[..., 10:11]
        w[..., R + 20:2 * R] = w[..., R + 20:R + 21]
    mbool, masks = masks_for(csr, h.shape[0], rng, drop=0.1)
    return rng, E, R, n, csr, mbool, masks, state, w, B, L


@pytest.mark.parametrize("K", [1, 30, 149, 250, 400, 1 << 60])
@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("agg", ["sum", "max"])
def test_topk_many_groups(K, ties, agg):
    rng, E, R, n, csr, mbool, masks, state, w, B, L = _many_groups_case(90 + K % 97 + ties, ties)
    if agg == "sum":
        keys, vals = O.sparse_forward(O.SPARSE_TOPK, *state, B, L, E, w, csr, masks, R, False, K)
        out, _, _ = _sum(state, w, csr, mbool, B, L, E, R, K)
        assert np.array_equal(_keys(out.indices().detach(), L, E), keys)
        assert np.array_equal(bits(out.values().detach().cpu().numpy()), bits(vals))
    else:
        out, v, wt = _max(state, w, csr, mbool, B, L, E, R, K, grad=True)
        _check_max(out, v, wt, state, w, csr, masks, B, L, E, R, n, K, False, rng)


@pytest.mark.parametrize("n", [1, 31, 64, 1000, 4097])
def test_mask_bits_match_packbits(n):
    """fl_mask_bits: bit j of word w = mask[32w + j] != 0 (little-endian bit
    order within each 32-bit word), the tail of the last word zero."""
    fk = _fk()
    rng = np.random.default_rng(n)
    mask = (rng.random(n) < 0.7).astype(np.float32)
    got = fk._mask_bits(torch.from_numpy(mask).cuda()).cpu().numpy().view(np.uint32)
    padded = np.zeros(((n + 31) // 32) * 32, np.uint8)
    padded[:n] = mask != 0
    want = np.packbits(padded, bitorder="little").view(np.uint32)
    np.testing.assert_array_equal(got[: want.size], want)


@pytest.mark.parametrize("n", [1, 31, 64, 1000, 4097, 100003])
def test_mask_order_bits_match_packbits(n):
    """fl_mask_order_bits: bit p of the side's bitmap = mask[order[p]] for a
    Boolean mask by edge id and a permutation order (a CSR side's), packed as
    numpy's little-endian packbits; the tail of the last word zero."""
    fk = _fk()
    rng = np.random.default_rng(n + 1)
    mask = rng.random(n) < 0.6
    order = rng.permutation(n).astype(np.int32)
    got = fk._mask_order_bits(torch.from_numpy(mask).cuda(), torch.from_numpy(order).cuda()).cpu().numpy()
    padded = np.zeros(((n + 31) // 32) * 32, np.uint8)
    padded[:n] = mask[order]
    want = np.packbits(padded, bitorder="little").view(np.uint32)
    np.testing.assert_array_equal(got.view(np.uint32)[: want.size], want)


def test_mask_updated_in_place_between_hops():
    """A training step hides its batch's triples in the mask in place and
    restores them afterwards (src/main.py:887-890,927-930): the top-k hop
    sees each version of the mask (its cached bitmap is rebuilt), checked
    bit for bit against the oracle with that version's masks."""
    B, L, K = 3, 2, 4
    rng, E, R, n, csr, mbool, _, state, w = _case(2, 0.3, B, L, 60, 515, drop=0.0)
    fk = _fk()
    b, l, e, v = _dev(*state)
    wt = torch.from_numpy(w).cuda()
    tc = to_torch_csr(csr, torch.device("cuda"))
    mk = torch.from_numpy(mbool).cuda()
    hidden = torch.from_numpy(rng.choice(mbool.shape[0], 500, replace=False)).cuda()
    for step in range(3):
        if step == 1:
            mk[hidden] = False
        if step == 2:
            mk[hidden] = True
        out = fk.FlashLogFunctionSparse3DTopKSum.apply(b, l, e, v, wt, *tc[:4], *tc[4:8], *tc[8:16], mk, None,
                                                       B, L, E, R, False, K, False, None, False, False)
        mnow = mk.cpu().numpy()
        masks = tuple(mnow[csr[o]].astype(np.float32) for o in (3, 7))
        keys, vals = O.sparse_forward(O.SPARSE_TOPK, *state, B, L, E, w, csr, masks, R, False, K)
        assert np.array_equal(_keys(out.indices(), L, E), keys), step
        assert np.array_equal(bits(out.values().cpu().numpy()), bits(vals)), step


@pytest.mark.parametrize("agg", ["sum", "max"])
def test_topk_hop_rejects_nonfinite_attention(agg):
    """flashlog.cu:2019-2021: a non-finite attention weight is rejected (the
    plan flags it; no item is expanded)."""
    B, L = 2, 2
    rng, E, R, n, csr, mbool, masks, state, w = _case(2, 0.2, B, L, 50, 3)
    w = w.copy()
    w[1, 0, 3] = np.nan
    with pytest.raises(RuntimeError, match="non-finite attention"):
        (_sum if agg == "sum" else _max)(state, w, csr, mbool, B, L, E, R, 5)


def test_entry_order_must_be_a_permutation(monkeypatch):
    """The plan checks the entry visiting order: an order that visits one
    entry twice (and another never) is reported before any item is expanded."""
    fk = _fk()
    B, L = 4, 3
    rng, E, R, n, csr, mbool, masks, state, w = _case(2, 1.0, B, L, 1500, 11)
    tc = to_torch_csr(csr, torch.device("cuda"))
    om, im = _dev(*masks)
    sides = fk._SparseSides(tc[1], om, tc[8], tc[9], tc[10], tc[11], tc[5], im, tc[12], tc[13], tc[14], tc[15])
    b, l, e, v = _dev(*state)
    assert v.numel() >= fk._ENTRY_ORDER_MIN
    wt = torch.from_numpy(w).cuda()
    good = fk._sparse_forward(b, l, e, v, wt, sides, B, L, E, R, False, fk._SPARSE_TOPK, 5, False)
    rk, rv = O.sparse_forward(O.SPARSE_TOPK, *state, B, L, E, w, csr, masks, R, False, 5)
    assert np.array_equal(_keys(good[0], L, E), rk)

    def bad(sp_e, E):
        order = torch.argsort(sp_e).to(torch.int32)
        order[1] = order[0]
        return order

    monkeypatch.setattr(fk, "_entry_order", bad)
    with pytest.raises(ValueError):
        fk._sparse_forward(b, l, e, v, wt, sides, B, L, E, R, False, fk._SPARSE_TOPK, 5, False)
