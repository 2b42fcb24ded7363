"""GPU parity of the sparse (COO) hop against the oracle: coordinates and
fp32 values bit for bit (the CPU path's addition order), normalization
bit for bit (the CPU path's sequential row sums), gradients within 1e-5
relative."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import assert_grad_close, attention, bits, masks_for, small_graph, sparse_coo_state, to_torch_csr

pytestmark = pytest.mark.gpu


def _fk():
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    return fk


def _case(cfg, scale, B, L, per_row, seed, ties=False, drop=0.1, graph_seed=None):
    rng = np.random.default_rng(seed)
    h, r, t, E, R, csr = small_graph(cfg, scale, seed=graph_seed)
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


def _all_edges(state, w, csr, masks, B, L, E, R, wot_i=False, grad=False):
    fk = _fk()
    b, l, e, v = _dev(*state)
    v.requires_grad_(grad)
    wt = torch.from_numpy(w).cuda().requires_grad_(grad)
    tc = to_torch_csr(csr, torch.device("cuda"))
    om, im = _dev(*masks)
    out = fk.FlashLogFunctionSparse3DAllEdgesSum.apply(b, l, e, v, wt, tc[1], om, tc[8], tc[9], tc[10], tc[11],
                                                       tc[5], im, tc[12], tc[13], tc[14], tc[15], B, L, E, R,
                                                       wot_i)
    return out, v, wt


def _topk(state, w, csr, mbool, B, L, E, R, K, c1=None, wot_i=False, grad=False):
    fk = _fk()
    b, l, e, v = _dev(*state)
    v.requires_grad_(grad)
    wt = torch.from_numpy(w).cuda().requires_grad_(grad)
    tc = to_torch_csr(csr, torch.device("cuda"))
    mk = torch.from_numpy(mbool).cuda()
    out = fk.FlashLogFunctionSparse3DTopKSum.apply(b, l, e, v, wt, *tc[:4], *tc[4:8], *tc[8:16], mk, None,
                                                   B, L, E, R, wot_i, K, False, c1, True)
    return out, v, wt


@pytest.mark.parametrize("cfg,scale,per_row", [(2, 0.05, 40), (2, 1.0, 300), (3, 0.05, 60)])
@pytest.mark.parametrize("wot_i", [False, True])
def test_sparse_all_edges_bitexact(cfg, scale, per_row, wot_i):
    B, L = 4, 3
    rng, E, R, n, csr, mbool, masks, state, w = _case(cfg, scale, B, L, per_row, 10 + cfg + wot_i)
    keys, vals = O.sparse_forward(O.SPARSE_ALL, *state, B, L, E, w, csr, masks, R, wot_i)
    out, _, _ = _all_edges(state, w, csr, masks, B, L, E, R, wot_i)
    torch.cuda.synchronize()
    assert out.is_coalesced()
    assert np.array_equal(_keys(out.indices().detach(), L, E), keys)
    assert np.array_equal(bits(out.values().detach().cpu().numpy()), bits(vals))


@pytest.mark.parametrize("K", [2, 7, 200, 1 << 60])
@pytest.mark.parametrize("ties", [False, True])
def test_sparse_topk_bitexact(K, ties):
    B, L = 4, 3
    rng, E, R, n, csr, mbool, masks, state, w = _case(2, 1.0, B, L, 250, 40 + K % 11 + ties, ties=ties)
    keys, vals = O.sparse_forward(O.SPARSE_TOPK, *state, B, L, E, w, csr, masks, R, False, K)
    out, _, _ = _topk(state, w, csr, mbool, B, L, E, R, K)
    torch.cuda.synchronize()
    assert np.array_equal(_keys(out.indices().detach(), L, E), keys)
    assert np.array_equal(bits(out.values().detach().cpu().numpy()), bits(vals))


@pytest.mark.parametrize("c1", [0, 5, 40])
def test_sparse_topk_with_c1(c1):
    B, L = 3, 3
    rng, E, R, n, csr, mbool, masks, state, w = _case(2, 0.3, B, L, 80, 70 + c1, ties=True)
    kept = O.sparse_topc(state[0], state[1], state[3], L, c1)
    sel = tuple(a[kept] for a in state)
    keys, vals = O.sparse_forward(O.SPARSE_TOPK, *sel, B, L, E, w, csr, masks, R, False, 3)
    out, v, wt = _topk(state, w, csr, mbool, B, L, E, R, 3, c1=c1, grad=True)
    torch.cuda.synchronize()
    assert np.array_equal(_keys(out.indices().detach(), L, E), keys)
    assert np.array_equal(bits(out.values().detach().cpu().numpy()), bits(vals))
    # gradient reaches only the kept entries
    g = torch.randn(out.values().shape, device="cuda")
    (out.values() * g).sum().backward()
    dropped = np.setdiff1d(np.arange(state[3].shape[0]), kept)
    assert np.all(v.grad.cpu().numpy()[dropped] == 0)


def test_sparse_unsorted_input_and_edges():
    fk = _fk()
    B, L = 3, 2
    rng, E, R, n, csr, mbool, masks, state, w = _case(2, 0.1, B, L, 30, 5)
    keys, vals = O.sparse_forward(O.SPARSE_ALL, *state, B, L, E, w, csr, masks, R)
    perm = rng.permutation(state[0].shape[0])
    shuffled = tuple(a[perm] for a in state)
    # the CPU path visits entries of a row in input order: compare with the oracle on the same order
    rows = shuffled[0] * L + shuffled[1]
    order = np.argsort(rows, kind="stable")
    k2, v2 = O.sparse_forward(O.SPARSE_ALL, *(a[order] for a in shuffled), B, L, E, w, csr, masks, R)
    out, _, _ = _all_edges(shuffled, w, csr, masks, B, L, E, R)
    assert np.array_equal(_keys(out.indices().detach(), L, E), k2)
    assert np.array_equal(bits(out.values().detach().cpu().numpy()), bits(v2))
    assert np.array_equal(k2, keys)
    # empty state
    empty = (np.zeros(0, np.int64),) * 3 + (np.zeros(0, np.float32),)
    out, _, _ = _all_edges(empty, w, csr, masks, B, L, E, R)
    assert out._nnz() == 0
    # top-k budget 0: only the identity terms
    out, _, _ = _topk(state, w, csr, mbool, B, L, E, R, 0)
    kk, vv = O.sparse_forward(O.SPARSE_TOPK, *state, B, L, E, w, csr, masks, R, False, 0)
    assert np.array_equal(_keys(out.indices().detach(), L, E), kk)
    # out-of-range entity
    bad = (state[0], state[1], state[2].copy(), state[3])
    bad[2][0] = E
    with pytest.raises(ValueError):
        _all_edges(bad, w, csr, masks, B, L, E, R)


@pytest.mark.parametrize("mode", ["all", "topk"])
@pytest.mark.parametrize("wot_i", [False, True])
def test_sparse_backward(mode, wot_i):
    B, L = 4, 3
    rng, E, R, n, csr, mbool, masks, state, w = _case(2, 1.0, B, L, 120, 90 + wot_i + (mode == "all"))
    if mode == "all":
        out, v, wt = _all_edges(state, w, csr, masks, B, L, E, R, wot_i, grad=True)
        m, K = O.SPARSE_ALL, 1 << 60
    else:
        out, v, wt = _topk(state, w, csr, mbool, B, L, E, R, 5, wot_i=wot_i, grad=True)
        m, K = O.SPARSE_TOPK, 5
    keys = _keys(out.indices().detach(), L, E)
    g = rng.standard_normal(keys.shape[0]).astype(np.float32)
    (out.values() * torch.from_numpy(g).cuda()).sum().backward()
    gv_ref, gw_ref = O.sparse_backward(m, *state, B, L, E, w, csr, masks, R, keys, g, wot_i, K)
    assert_grad_close(v.grad.cpu().numpy(), gv_ref)
    assert_grad_close(wt.grad.reshape(B * L, n).cpu().numpy(), gw_ref)


def test_normalize_sparse3d():
    """Values and denominators bit-identical to the CPU path (a left fold of
    each row in entry order, then IEEE division); gradients within 1e-5."""
    fk = _fk()
    rng = np.random.default_rng(3)
    B, L, E = 5, 3, 400
    b, l, e, v = sparse_coo_state(B, L, E, 90, rng)
    idx = torch.from_numpy(np.stack([b, l, e])).cuda()
    vt = torch.from_numpy(v).cuda().requires_grad_(True)
    s = torch.sparse_coo_tensor(idx, vt, (B, L, E), is_coalesced=True)
    out = fk.normalize_sparse3d(s)
    want, denom = O.sparse_normalize(b, l, v, B, L)
    assert np.array_equal(bits(out.values().detach().cpu().numpy()), bits(want))
    # the output takes the input's index tensor as it is (no copy)
    assert out._indices().data_ptr() == idx.data_ptr() and torch.equal(out._indices(), idx)
    # separate index rows are stacked
    rows = [idx[k].clone() for k in range(3)]
    o2 = fk.Sparse3DNormalizeFunction.apply(*rows, vt.detach(), B, L, E, 1e-7)
    assert torch.equal(o2._indices(), idx) and o2._indices().data_ptr() != idx.data_ptr()
    g = rng.standard_normal(v.shape[0]).astype(np.float32)
    (out.values() * torch.from_numpy(g).cuda()).sum().backward()
    row = b * L + l
    d = denom[row].astype(np.float64)
    sgx = np.zeros(B * L)
    np.add.at(sgx, row, g.astype(np.float64) * v)
    want_g = g / d - sgx[row] / (d * d)
    np.testing.assert_allclose(vt.grad.cpu().numpy(), want_g, rtol=1e-5, atol=1e-6)


def test_normalize_long_rows_bitexact():
    """Rows longer than one LDS chunk (2048 entries) and an empty row."""
    fk = _fk()
    rng = np.random.default_rng(31)
    B, L, E = 2, 2, 60000
    b, l, e, v = sparse_coo_state(B, L, E, 9000, rng)
    keep = ~((b == 1) & (l == 0))
    b, l, e, v = b[keep], l[keep], e[keep], v[keep]
    s = torch.sparse_coo_tensor(torch.from_numpy(np.stack([b, l, e])).cuda(), torch.from_numpy(v).cuda(),
                                (B, L, E), is_coalesced=True)
    out = fk.normalize_sparse3d(s)
    want, _ = O.sparse_normalize(b, l, v, B, L)
    assert np.array_equal(bits(out.values().cpu().numpy()), bits(want))


def test_normalize_nonfinite_rows():
    """A row holding NaN, a row holding inf and a row summing below eps
    against the GPU path's formula (flashlog.cu:2529-2591): d = row sum,
    dc = d if d >= eps else eps (so a NaN sum divides by eps), out = v / dc;
    backward g/dc - sum(g*v)/dc^2 where d >= eps, else g/dc."""
    fk = _fk()
    B, L, E, eps = 1, 4, 10, np.float32(1e-7)
    b = np.zeros(9, np.int64)
    l = np.array([0, 0, 1, 1, 2, 2, 3, 3, 3], np.int64)
    e = np.array([1, 4, 2, 3, 0, 9, 1, 2, 3], np.int64)
    v = np.array([0.5, np.nan, 0.25, np.inf, 1e-9, 2e-9, 0.125, -0.0, 0.375], np.float32)
    vt = torch.from_numpy(v).cuda().requires_grad_(True)
    s = torch.sparse_coo_tensor(torch.from_numpy(np.stack([b, l, e])).cuda(), vt, (B, L, E), is_coalesced=True)
    out = fk.normalize_sparse3d(s)
    row = l
    d = np.zeros(L, np.float32)
    for i in range(v.size):
        d[row[i]] = np.float32(d[row[i]] + v[i])
    dc = np.where(d >= eps, d, eps).astype(np.float32)
    want = (v / dc[row]).astype(np.float32)
    got = out.values().detach().cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(bits(got[fin]), bits(want[fin]))
    g = np.array([1, 2, 3, 4, 5, 6, 7, 8, 9], np.float32)
    (out.values() * torch.from_numpy(g).cuda()).sum().backward()
    gv = vt.grad.cpu().numpy()
    active = d >= eps
    sgx = np.zeros(L, np.float64)
    np.add.at(sgx, row, g.astype(np.float64) * v)
    want_g = np.where(active[row], g / dc[row] - sgx[row] / (dc[row].astype(np.float64) ** 2), g / dc[row])
    # row 0 (NaN sum) is inactive: g/eps; row 1 (inf sum) gives NaN corrections
    ok = row != 1
    np.testing.assert_allclose(gv[ok], want_g[ok], rtol=1e-5)
    assert np.array_equal(np.isnan(gv[row == 1]), np.isnan(want_g[row == 1]))


def test_three_hop_topk_pipeline():
    """Per hop: c1 + top-k hop + normalize, each hop checked bit for bit on
    the GPU's own input."""
    fk = _fk()
    B, L = 4, 3
    rng, E, R, n, csr, mbool, masks, _, _ = _case(2, 1.0, B, L, 1, 123)
    heads = rng.integers(0, E, B)
    b = np.repeat(np.arange(B), L).astype(np.int64)
    l = np.tile(np.arange(L), B).astype(np.int64)
    e = np.repeat(heads, L).astype(np.int64)
    v = np.ones(B * L, np.float32)
    idx = torch.from_numpy(np.stack([b, l, e])).cuda()
    state = torch.sparse_coo_tensor(idx, torch.from_numpy(v).cuda(), (B, L, E)).coalesce()
    tc = to_torch_csr(csr, torch.device("cuda"))
    mk = torch.from_numpy(mbool).cuda()
    for hop in range(3):
        w = attention(B * L, n, rng).reshape(B, L, n)
        si = state.indices().cpu().numpy()
        sv = state.values().cpu().numpy()
        kept = O.sparse_topc(si[0], si[1], sv, L, 100)
        keys, vals = O.sparse_forward(O.SPARSE_TOPK, si[0][kept], si[1][kept], si[2][kept], sv[kept], B, L, E, w,
                                      csr, masks, R, False, 200)
        s = fk.vectorized_operation_sparse3d_csr_sum(state, torch.from_numpy(w).cuda(), tc, mk, R, use_topk=True,
                                                     topk_edges=200, topk_nodes=100)
        assert np.array_equal(_keys(s.indices(), L, E), keys)
        assert np.array_equal(bits(s.values().cpu().numpy()), bits(vals))
        state = fk.normalize_sparse3d(s)


def test_cpu_sum_classes():
    """The CPU classes (FlashLogFunctionSparse3DCPUSum / CPUSumNorm) through
    their dispatchers: CPU tensors in and out, forward bit for bit, and the
    backward (grad_v, grad_w on the CPU) against the oracle's backward --
    for the fused normalization after the closed-form normalize backward --
    within 1e-5."""
    fk = _fk()
    B, L = 3, 2
    rng, E, R, n, csr, mbool, masks, state, w = _case(2, 0.1, B, L, 30, 17)
    tcsr = tuple(torch.from_numpy(np.ascontiguousarray(a)) for a in csr)

    def leaves():
        v_t = torch.from_numpy(state[3].copy()).requires_grad_(True)
        w_t = torch.from_numpy(w.copy()).requires_grad_(True)
        sp = torch.sparse_coo_tensor(torch.from_numpy(np.stack(state[:3])), v_t, (B, L, E)).coalesce()
        return v_t, w_t, sp

    v_t, w_t, sp = leaves()
    out = fk.vectorized_operation_sparse3d_csr_sum(sp, w_t, tcsr, torch.from_numpy(mbool), R,
                                                   use_topk=True, topk_edges=4)
    assert out.device.type == "cpu"
    keys, vals = O.sparse_forward(O.SPARSE_TOPK, *state, B, L, E, w, csr, masks, R, False, 4)
    assert np.array_equal(_keys(out.indices().detach(), L, E), keys)
    assert np.array_equal(bits(out.values().detach().numpy()), bits(vals))
    g = rng.standard_normal(keys.shape[0]).astype(np.float32)
    (out.values() * torch.from_numpy(g)).sum().backward()
    rgv, rgw = O.sparse_backward(O.SPARSE_TOPK, *state, B, L, E, w, csr, masks, R, keys, g, False, 4)
    assert v_t.grad.device.type == "cpu" and w_t.grad.device.type == "cpu"
    assert_grad_close(v_t.grad.numpy(), rgv)
    assert_grad_close(w_t.grad.numpy().reshape(B * L, n), rgw)

    v_t, w_t, sp = leaves()
    outn = fk.vectorized_operation_sparse3d_csr_sum_norm(sp, w_t, tcsr, torch.from_numpy(mbool),
                                                         R, use_topk=True, topk_edges=4)
    row = keys // E
    nv, denom = O.sparse_normalize(row // L, row % L, vals, B, L)
    assert np.array_equal(bits(outn.values().detach().numpy()), bits(nv))
    (outn.values() * torch.from_numpy(g)).sum().backward()
    d = np.maximum(denom.astype(np.float64), 1e-7)[row]
    sgv = np.zeros(B * L)
    np.add.at(sgv, row, g.astype(np.float64) * vals)
    g_sum = (g / d - sgv[row] / d ** 2).astype(np.float32)
    rgv, rgw = O.sparse_backward(O.SPARSE_TOPK, *state, B, L, E, w, csr, masks, R, keys, g_sum, False, 4)
    assert_grad_close(v_t.grad.numpy(), rgv)
    assert_grad_close(w_t.grad.numpy().reshape(B * L, n), rgw)


@pytest.mark.parametrize("mode", ["all", "topk"])
def test_sparse_hot_destination(mode):
    """A destination receiving most edges: buckets far above one LDS chunk
    (the chunked hot-bucket path), checked bit for bit, with gradients."""
    from oracle import oracle as Oc
    rng = np.random.default_rng(21)
    E, R, M = 20000, 5, 60000
    h = rng.integers(0, E, M)
    t = np.where(rng.random(M) < 0.7, 12345, rng.integers(0, E, M))
    r = rng.integers(0, R, M)
    csr = Oc.build_csr_structure(h, t, r, E)
    n = 2 * R + 1
    B, L = 2, 2
    b, l, e, v = sparse_coo_state(B, L, E, 1500, rng)
    w = attention(B * L, n, rng).reshape(B, L, n)
    mbool, masks = masks_for(csr, M, rng, drop=0.05)
    state = (b, l, e, v)
    if mode == "all":
        keys, vals = O.sparse_forward(O.SPARSE_ALL, *state, B, L, E, w, csr, masks, R)
        out, vt, wt = _all_edges(state, w, csr, masks, B, L, E, R, grad=True)
        m, K = O.SPARSE_ALL, 1 << 60
    else:
        keys, vals = O.sparse_forward(O.SPARSE_TOPK, *state, B, L, E, w, csr, masks, R, False, 6)
        out, vt, wt = _topk(state, w, csr, mbool, B, L, E, R, 6, grad=True)
        m, K = O.SPARSE_TOPK, 6
    assert np.array_equal(_keys(out.indices().detach(), L, E), keys)
    assert np.array_equal(bits(out.values().detach().cpu().numpy()), bits(vals))
    g = rng.standard_normal(keys.shape[0]).astype(np.float32)
    (out.values() * torch.from_numpy(g).cuda()).sum().backward()
    gv_ref, gw_ref = O.sparse_backward(m, *state, B, L, E, w, csr, masks, R, keys, g, False, K)
    assert_grad_close(vt.grad.cpu().numpy(), gv_ref)
    assert_grad_close(wt.grad.reshape(B * L, n).cpu().numpy(), gw_ref)


@pytest.mark.parametrize("mode", ["all", "topk"])
def test_sparse_backward_is_deterministic(mode):
    """The same backward twice gives the same bits (no atomics on grad_v or
    grad_w), on a hub graph where one destination receives 70% of the
    edges and rows span several backward chunks."""
    from oracle import oracle as Oc
    rng = np.random.default_rng(22)
    E, R, M = 20000, 5, 60000
    h = rng.integers(0, E, M)
    t = np.where(rng.random(M) < 0.7, 12345, rng.integers(0, E, M))
    r = rng.integers(0, R, M)
    csr = Oc.build_csr_structure(h, t, r, E)
    n = 2 * R + 1
    B, L = 2, 2
    state = sparse_coo_state(B, L, E, 1500, rng)
    w = attention(B * L, n, rng).reshape(B, L, n)
    mbool, masks = masks_for(csr, M, rng, drop=0.05)
    grads = []
    for _ in range(2):
        if mode == "all":
            out, vt, wt = _all_edges(state, w, csr, masks, B, L, E, R, grad=True)
        else:
            out, vt, wt = _topk(state, w, csr, mbool, B, L, E, R, 6, grad=True)
        g = torch.from_numpy(np.random.default_rng(3).standard_normal(out._nnz()).astype(np.float32)).cuda()
        (out.values() * g).sum().backward()
        grads.append((vt.grad.clone(), wt.grad.clone()))
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])


def test_backward_without_positions_matches(monkeypatch):
    """The top-k sum over several destination buckets with bitmap masks keeps
    no item CSR positions for its backward; its gradients are the same bits
    as those of the backward that reads them."""
    from oracle import oracle as Oc
    fk = _fk()
    rng = np.random.default_rng(23)
    E, R, M = 30000, 4, 80000
    h = rng.integers(0, E, M)
    t = np.where(rng.random(M) < 0.3, 777, rng.integers(0, E, M))
    r = rng.integers(0, R, M)
    csr = Oc.build_csr_structure(h, t, r, E)
    n = 2 * R + 1
    B, L = 3, 2
    state = sparse_coo_state(B, L, E, 900, rng)
    w = attention(B * L, n, rng).reshape(B, L, n)
    mbool, masks = masks_for(csr, M, rng, drop=0.2)
    seen = []
    orig = fk._SparseSides.positions_optional

    def spy(self, *a):
        seen.append(orig(self, *a))
        return seen[-1]

    grads = []
    for force in (False, True):
        monkeypatch.setattr(fk._SparseSides, "positions_optional",
                            spy if not force else (lambda self, *a: False))
        out, vt, wt = _topk(state, w, csr, mbool, B, L, E, R, 5, grad=True)
        g = torch.from_numpy(np.random.default_rng(4).standard_normal(out._nnz()).astype(np.float32)).cuda()
        (out.values() * g).sum().backward()
        grads.append((vt.grad.clone(), wt.grad.clone()))
    assert seen == [True]
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])
    keys = _keys(out.indices().detach(), L, E)
    gv_ref, gw_ref = O.sparse_backward(O.SPARSE_TOPK, *state, B, L, E, w, csr, masks, R, keys,
                                       g.cpu().numpy(), False, 5)
    assert_grad_close(grads[0][0].cpu().numpy(), gv_ref)
    assert_grad_close(grads[0][1].reshape(B * L, n).cpu().numpy(), gw_ref)


@pytest.mark.parametrize("E", [5000, 30000])
def test_few_destinations_with_holes(E):
    """Rows whose items (well above one wave's 512) go to a handful of
    destinations, with a quarter of the kept edges masked (holes of the
    top-k sum): the few-destination accumulation, with one bucket per row
    (holes among the row's raw items) and with several."""
    from oracle import oracle as Oc
    rng = np.random.default_rng(31)
    R = 40
    srcs = np.arange(6)
    tgts = np.array([7, 11, 12, 300, 2047, E - 1])
    h = np.repeat(srcs, R * tgts.size)
    t = np.tile(np.repeat(tgts, R), srcs.size)
    r = np.tile(np.arange(R), srcs.size * tgts.size)
    extra = 3000
    h = np.concatenate([h, rng.integers(0, E, extra)])
    t = np.concatenate([t, rng.integers(0, E, extra)])
    r = np.concatenate([r, rng.integers(0, R, extra)])
    csr = Oc.build_csr_structure(h, t, r, E)
    n = 2 * R + 1
    B, L = 2, 2
    b = np.repeat(np.arange(B), L * srcs.size)
    l = np.tile(np.repeat(np.arange(L), srcs.size), B)
    e = np.tile(srcs, B * L)
    v = (rng.random(b.size) + 0.1).astype(np.float32)
    state = (b.astype(np.int64), l.astype(np.int64), e.astype(np.int64), v)
    w = attention(B * L, n, rng).reshape(B, L, n)
    mbool, masks = masks_for(csr, h.shape[0], rng, drop=0.25)
    K = 1 << 20
    keys, vals = O.sparse_forward(O.SPARSE_TOPK, *state, B, L, E, w, csr, masks, R, False, K)
    out, vt, wt = _topk(state, w, csr, mbool, B, L, E, R, K, grad=True)
    assert np.array_equal(_keys(out.indices().detach(), L, E), keys)
    assert np.array_equal(bits(out.values().detach().cpu().numpy()), bits(vals))
    g = rng.standard_normal(keys.shape[0]).astype(np.float32)
    (out.values() * torch.from_numpy(g).cuda()).sum().backward()
    gv_ref, gw_ref = O.sparse_backward(O.SPARSE_TOPK, *state, B, L, E, w, csr, masks, R, keys, g, False, K)
    assert_grad_close(vt.grad.cpu().numpy(), gv_ref)
    assert_grad_close(wt.grad.reshape(B * L, n).cpu().numpy(), gw_ref)
