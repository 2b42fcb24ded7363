"""GPU parity of the dense max hop (dense_csr_max / FlashLogDenseMaxFunction)
against the oracle: values and winning positions bit for bit; the
winner-only grad_A bit for bit (fixed per-(source, row) walks in CSR
order) and grad_w within 1e-5 relative (per-pair partials in source
order)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import attention, bits, masks_for, small_graph, sparse_state, to_torch_csr

pytestmark = pytest.mark.gpu


def _fk():
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    return fk


def _setup(seed, K, ties, negative=False, cfg=2, scale=0.05, BL=12, per_row=60):
    rng = np.random.default_rng(seed)
    h, r, t, E, R, csr = small_graph(cfg, scale)
    n = 2 * R + 1
    A = sparse_state(BL, E, per_row, rng, ties=ties)
    if negative:
        idx = np.nonzero(A[0])[0][:10]
        A[0, idx] = -A[0, idx]  # negative products: larger float bits win, as in the packed compare
    w = attention(BL, n, rng)
    if ties:
        w[:, : n // 2] = w[:, :1]
    _, masks = masks_for(csr, h.shape[0], rng)
    return rng, h, E, R, n, csr, A, w, masks


def _run_forward(A, w, csr, masks, R, K, wot_i, B, L, grad=False):
    fk = _fk()
    dev = torch.device("cuda")
    E = A.shape[1]
    n = w.shape[1]
    tcsr = to_torch_csr(csr, dev)
    At = torch.from_numpy(A).to(dev).view(B, L, E).requires_grad_(grad)
    wt = torch.from_numpy(w).to(dev).view(B, L, n).requires_grad_(grad)
    mk = tuple(torch.from_numpy(m).to(dev) for m in masks)
    outs = fk.dense_csr_max(At, wt, tcsr, None, R, wot_i=wot_i, use_topk=K > 0, topk_nodes=E, topk_edges=K,
                            prepared_masks=mk)
    return At, wt, outs


@pytest.mark.parametrize("K", [0, 1, 3, 200])
@pytest.mark.parametrize("ties", [False, True])
@pytest.mark.parametrize("wot_i", [False, True])
def test_dense_max_forward_bitexact(K, ties, wot_i):
    rng, h, E, R, n, csr, A, w, masks = _setup(500 + K + 3 * ties + 7 * wot_i, K, ties, negative=ties)
    B, L = 4, 3
    BL = B * L
    kk = K if K > 0 else (1 << 60)
    oi, oo, ov, ao, av = O.dense_max_forward(A, w, csr, masks, R, wot_i=wot_i, topk_edges=kk)
    fk = _fk()
    _, _, outs = _run_forward(A, w, csr, masks, R, K, wot_i, B, L)
    torch.cuda.synchronize()
    for name, o, rr in zip(("ind", "ori", "inv"), outs, (oi, oo, ov)):
        got = o.reshape(BL, E).detach().cpu().numpy()
        assert np.array_equal(bits(got), bits(rr)), name
    # the winning positions come back through the saved tensors of the graph
    g = fk._graph_for(*[torch.from_numpy(np.ascontiguousarray(csr[i])).cuda() for i in (1, 8, 9, 10, 11,
                                                                                      5, 12, 13, 14, 15)])
    assert g.ori.nheavy + g.inv.nheavy > 0, "test graph must have heavy destinations"


def test_dense_max_args_bitexact():
    """The int64 winning positions (exposed by the forward helper)."""
    fk = _fk()
    rng, h, E, R, n, csr, A, w, masks = _setup(77, 3, True, negative=True)
    BL = A.shape[0]
    dev = torch.device("cuda")
    tc = to_torch_csr(csr, dev)
    graph = fk._graph_for(tc[1], tc[8], tc[9], tc[10], tc[11], tc[5], tc[12], tc[13], tc[14], tc[15])
    mk = tuple(torch.from_numpy(m).to(dev) for m in masks)
    out = fk._dense_max_forward(torch.from_numpy(A).to(dev), torch.from_numpy(w).to(dev), graph, mk[0], mk[1],
                                R, False, 3)
    ref = O.dense_max_forward(A, w, csr, masks, R, topk_edges=3)
    torch.cuda.synchronize()
    for o, rr in zip(out, ref):
        got = o.cpu().numpy()
        if got.dtype == np.float32:
            assert np.array_equal(bits(got), bits(rr))
        else:
            assert np.array_equal(got, rr)


@pytest.mark.parametrize("K", [0, 2, 200])
@pytest.mark.parametrize("wot_i", [False, True])
def test_dense_max_backward(K, wot_i):
    rng, h, E, R, n, csr, A, w, masks = _setup(900 + K + wot_i, K, True)
    B, L = 4, 3
    BL = B * L
    kk = K if K > 0 else (1 << 60)
    oi, oo, ov, ao, av = O.dense_max_forward(A, w, csr, masks, R, wot_i=wot_i, topk_edges=kk)
    g = [rng.standard_normal((BL, E)).astype(np.float32) for _ in range(3)]
    g[1][rng.random((BL, E)) < 0.3] = 0.0
    gA_ref, gw_ref = O.dense_max_backward(*g, ao, av, A, w, csr, masks, R, wot_i=wot_i, topk_edges=kk)
    At, wt, outs = _run_forward(A, w, csr, masks, R, K, wot_i, B, L, grad=True)
    dev = At.device
    loss = sum((o * torch.from_numpy(gg).to(dev).view(B, L, E)).sum() for o, gg in zip(outs, g))
    loss.backward()
    torch.cuda.synchronize()
    gA = At.grad.reshape(BL, E).cpu().numpy()
    gw = wt.grad.reshape(BL, n).cpu().numpy()
    assert np.array_equal(bits(gA), bits(gA_ref)), float(np.abs(gA - gA_ref).max())
    np.testing.assert_allclose(gw, gw_ref, rtol=1e-5, atol=1e-6 * float(np.abs(gw_ref).max()))


@pytest.mark.parametrize("K", [0, 5])
def test_dense_max_hub_destination(K):
    """A destination receiving 70% of 60k edges (~1300 segments, ~80
    supersegments: the per-supersegment pre-reduction and the unrolled
    heavy loop), values and winning positions bit for bit."""
    rng = np.random.default_rng(77 + K)
    E, R, M = 20000, 5, 60000
    h = rng.integers(0, E, M)
    t = np.where(rng.random(M) < 0.7, 12345, rng.integers(0, E, M))
    r = rng.integers(0, R, M)
    csr = O.build_csr_structure(h, t, r, E)
    n = 2 * R + 1
    B, L = 2, 3
    BL = B * L
    A = sparse_state(BL, E, 3000, rng, ties=True)
    w = attention(BL, n, rng)
    _, masks = masks_for(csr, M, rng, drop=0.1)
    kk = K if K > 0 else (1 << 60)
    oi, oo, ov, ao, av = O.dense_max_forward(A, w, csr, masks, R, topk_edges=kk)
    _, _, outs = _run_forward(A, w, csr, masks, R, K, False, B, L)
    for name, o, rr in zip(("ind", "ori", "inv"), outs, (oi, oo, ov)):
        assert np.array_equal(bits(o.reshape(BL, E).detach().cpu().numpy()), bits(rr)), name
    assert np.any(oo[:, 12345] != 0)
