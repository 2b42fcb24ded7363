"""GPU parity of the dense hop (c1 entity budget + sum propagation with the
c2 edge budget) against the CPU oracle, bit for bit."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import attention, bits, masks_for, small_graph, sparse_state, to_torch_csr

pytestmark = pytest.mark.gpu


def _fk():
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    return fk


@pytest.mark.parametrize("K", [0, 1, 2, 3, 7, 200])
@pytest.mark.parametrize("ties", [False, True])
def test_dense_sum_forward_bitexact(K, ties):
    fk = _fk()
    rng = np.random.default_rng(100 + K + 7 * ties)
    h, r, t, E, R, csr = small_graph(2, 0.05)
    n = 2 * R + 1
    B, L = 4, 3
    BL = B * L
    A = sparse_state(BL, E, 60, rng, ties=ties)
    w = attention(BL, n, rng)
    if ties:
        w[:, : n // 2] = w[:, :1]  # many equal relation weights -> tie quotas
    _, masks = masks_for(csr, h.shape[0], rng)
    kk = K if K > 0 else (1 << 60)
    ref = O.dense_forward(A, w, csr, masks, R, topk_edges=kk)
    dev = torch.device("cuda")
    tcsr = to_torch_csr(csr, dev)
    At = torch.from_numpy(A).to(dev).view(B, L, E)
    wt = torch.from_numpy(w).to(dev).view(B, L, n)
    mk = tuple(torch.from_numpy(m).to(dev) for m in masks)
    outs = fk.dense_csr_sum_cuda(At, wt, tcsr, None, R, use_topk=K > 0, topk_nodes=E,
                                 topk_edges=K, prepared_masks=mk)
    torch.cuda.synchronize()
    for name, o, rr in zip(("ind", "ori", "inv"), outs, ref):
        got = o.reshape(BL, E).cpu().numpy()
        assert np.array_equal(bits(got), bits(rr)), (name, np.abs(got - rr).max())


@pytest.mark.parametrize("c", [0, 1, 5, 50, 200])
@pytest.mark.parametrize("ties", [False, True])
def test_dense_topc_bitexact(c, ties):
    fk = _fk()
    rng = np.random.default_rng(7 + c)
    BL, E = 9, 3000
    A = sparse_state(BL, E, 120, rng, ties=ties)
    A[0] = 0.0
    A[1, :5] = np.float32(0.25)  # a row under budget for c >= 5
    ref, cutoff, last, changed = O.dense_topc(A, c)
    keep = O.dense_topc_brute(A, c)
    assert np.array_equal(ref != 0, (A != 0) & keep)
    At = torch.from_numpy(A).cuda()
    got = fk._dense_topc_state(At.view(3, 3, E), c).reshape(BL, E).cpu().numpy()
    assert np.array_equal(bits(got), bits(ref))


def test_dense_pipeline_three_hops_c2_shape():
    """Three DRUM hops at the C2 configuration (41k entities, B=32, N=3,
    c1=1000, c2=400), each hop fed the oracle's normalized state."""
    fk = _fk()
    from flashlog_amd import synth
    h, r, t, E, R = synth.make_graph(2)
    csr = O.build_csr_structure(h, t, r, E)
    n = 2 * R + 1
    B, L, T = 32, 3, 3
    rng = np.random.Generator(np.random.PCG64(1234 + 2))
    src, rel, tgt = synth.make_queries(h, r, t, R, B, rng)
    W = synth.make_attention(B, L, n, T, rng)
    dev = torch.device("cuda")
    tcsr = to_torch_csr(csr, dev)
    M = h.shape[0]
    masks = (np.ones(M, np.float32), np.ones(M, np.float32))
    mk = tuple(torch.from_numpy(m).to(dev) for m in masks)
    x = np.zeros((B * L, E), np.float32)
    x[np.arange(B * L), np.repeat(src, L)] = 1.0
    for hop in range(T):
        w = W[hop].reshape(B * L, n)
        xp, _, _, _ = O.dense_topc(x, 1000)
        ref = O.dense_forward(xp, w, csr, masks, R, topk_edges=200)
        outs = fk.dense_csr_sum_cuda(torch.from_numpy(x).to(dev).view(B, L, E),
                                     torch.from_numpy(w).to(dev).view(B, L, n), tcsr, None, R,
                                     use_topk=True, topk_nodes=1000, topk_edges=200, prepared_masks=mk)
        for o, rr in zip(outs, ref):
            assert np.array_equal(bits(o.reshape(B * L, E).cpu().numpy()), bits(rr))
        s = (ref[0] + ref[1]) + ref[2]
        x = (s / np.maximum(s.sum(-1, keepdims=True), np.float32(1e-7))).astype(np.float32)


@pytest.mark.parametrize("K", [0, 2, 7, 200])
@pytest.mark.parametrize("wot_i", [False, True])
def test_dense_sum_backward(K, wot_i):
    """grad_A bit-identical to the CPU path; grad_w (a different but fixed
    association of the same sums) within 1e-5 relative."""
    fk = _fk()
    rng = np.random.default_rng(300 + K + 11 * wot_i)
    h, r, t, E, R, csr = small_graph(2, 0.05)
    n = 2 * R + 1
    B, L = 4, 3
    BL = B * L
    A = sparse_state(BL, E, 60, rng, ties=True)
    w = attention(BL, n, rng)
    w[:, : n // 2] = w[:, :1]
    _, masks = masks_for(csr, h.shape[0], rng)
    g = [rng.standard_normal((BL, E)).astype(np.float32) for _ in range(3)]
    g[1][rng.random((BL, E)) < 0.3] = 0.0  # zero upstream grads are skipped, as in the reference
    kk = K if K > 0 else (1 << 60)
    gA_ref, gw_ref = O.dense_backward(*g, A, w, csr, masks, R, wot_i=wot_i, topk_edges=kk)
    dev = torch.device("cuda")
    tcsr = to_torch_csr(csr, dev)
    At = torch.from_numpy(A).to(dev).view(B, L, E).requires_grad_(True)
    wt = torch.from_numpy(w).to(dev).view(B, L, n).requires_grad_(True)
    mk = tuple(torch.from_numpy(m).to(dev) for m in masks)
    outs = fk.dense_csr_sum_cuda(At, wt, tcsr, None, R, wot_i=wot_i, use_topk=K > 0, topk_nodes=E,
                                 topk_edges=K, prepared_masks=mk)
    loss = sum((o * torch.from_numpy(gg).to(dev).view(B, L, E)).sum() for o, gg in zip(outs, g))
    loss.backward()
    gA = At.grad.reshape(BL, E).cpu().numpy()
    gw = wt.grad.reshape(BL, n).cpu().numpy()
    assert np.array_equal(bits(gA), bits(gA_ref)), np.abs(gA - gA_ref).max()
    np.testing.assert_allclose(gw, gw_ref, rtol=1e-5, atol=1e-6)


def test_dense_topc_backward_masks_gradient():
    fk = _fk()
    rng = np.random.default_rng(77)
    BL, E, c = 6, 500, 20
    A = sparse_state(BL, E, 60, rng, ties=True)
    keep = O.dense_topc_brute(A, c)
    At = torch.from_numpy(A).cuda().view(2, 3, E).requires_grad_(True)
    G = torch.from_numpy(rng.standard_normal((2, 3, E)).astype(np.float32)).cuda()
    (fk._dense_topc_state(At, c) * G).sum().backward()
    want = (G.cpu().numpy().reshape(BL, E) * keep.astype(np.float32))
    assert np.array_equal(bits(At.grad.reshape(BL, E).cpu().numpy()), bits(want))
