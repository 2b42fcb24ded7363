"""The dense models' CPU route (vectorized_operation_csr + FlashLogFunction,
flashlog_kernel.py:700-882), called as src/model_DRUM_kernel.py:133-140 and
src/model_NeuralLP_kernel.py:127-132 call it when CUDA is off: CPU state,
CPU attention, the CPU CSR tuple and mask, masks prepared once per forward
by prepare_csr_masks.  The tensors stay on the CPU; the kernels run on the
GPU.  Against the oracle (the CPU path's order, itself bit-equal to the
reference's flashlog_forward_cpu / flashlog_backward_cpu): outputs and
grad_A bit for bit, grad_w within 1e-5 relative.  Also _compute_active_nodes
and prepare_csr_masks on CPU tensors, and FlashLogFunction called directly."""
import numpy as np
import pytest
import torch

from flashlog_amd import synth
from oracle import oracle as O
from tests.helpers import bits

pytestmark = pytest.mark.gpu

_GRAPHS = {}


def _fk():
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    return fk


def _graph(cfg):
    if cfg not in _GRAPHS:
        h, r, t, E, R = synth.make_graph(cfg)
        csr = O.build_csr_structure(h, t, r, E)
        tcsr = tuple(torch.from_numpy(np.ascontiguousarray(a)) for a in csr)
        _GRAPHS[cfg] = (h, r, t, E, R, csr, tcsr)
    return _GRAPHS[cfg]


def _route_hops(cfg, B, L, use_topk, c1, c2, wot_i=False, width=None, hide=0.0, seed=0):
    """Three hops of the CPU route, each fed the oracle's normalized state."""
    fk = _fk()
    h, r, t, E, R, csr, tcsr = _graph(cfg)
    n = width if width is not None else 2 * R + 1
    BL = B * L
    K = c2 // 2
    rng = np.random.Generator(np.random.PCG64(4321 + cfg + seed))
    src, _, _ = synth.make_queries(h, r, t, R, B, rng)
    W = synth.make_attention(B, L, n, 3, rng)
    M = h.shape[0]
    mask = rng.random(M) >= hide  # the training loop hides a batch's triples (src/main.py:887-890)
    mask_t = torch.from_numpy(mask)
    prepared = fk.prepare_csr_masks(tcsr, mask_t, None)
    assert all(m.device.type == "cpu" for m in prepared)
    masks = (mask[csr[3]].astype(np.float32), mask[csr[7]].astype(np.float32))
    for m_got, m_ref in zip(prepared, masks):
        assert np.array_equal(m_got.numpy(), m_ref)
    x = np.zeros((BL, E), np.float32)
    x[np.arange(BL), np.repeat(src, L)] = 1.0
    budget = K if use_topk and K > 0 else 1 << 60
    for hop in range(3):
        w = W[hop].reshape(BL, n)
        xp = O.dense_topc(x, c1)[0] if use_topk else x
        ref = O.dense_forward(xp, w, csr, masks, R, wot_i=wot_i, topk_edges=budget)
        x_t = torch.from_numpy(x).view(B, L, E).requires_grad_(True)
        w_t = torch.from_numpy(w).view(B, L, n).requires_grad_(True)
        outs = fk.vectorized_operation_csr(x_t.float(), w_t, tcsr, mask_t, R, weight=None, wot_i=wot_i,
                                           use_topk=use_topk, topk_nodes=c1, topk_edges=K, prepared_masks=prepared)
        for name, o, rf in zip(("ind", "ori", "inv"), outs, ref):
            assert o.device.type == "cpu"
            got = o.detach().reshape(BL, E).numpy()
            assert np.array_equal(bits(got), bits(rf)), (cfg, hop, name)
        g = [rng.standard_normal((BL, E)).astype(np.float32) for _ in range(3)]
        g[2][rng.random((BL, E)) < 0.3] = 0.0
        sum((o * torch.from_numpy(gg).view(B, L, E)).sum() for o, gg in zip(outs, g)).backward()
        gA_ref, gw_ref = O.dense_backward(*g, xp, w, csr, masks, R, wot_i=wot_i, topk_edges=budget)
        if use_topk:
            over = (x != 0).sum(1) > c1
            gA_ref = gA_ref * np.where(over[:, None], xp != 0, True).astype(np.float32)
        assert x_t.grad.device.type == "cpu" and w_t.grad.device.type == "cpu"
        gx = x_t.grad.reshape(BL, E).numpy()
        assert np.array_equal(bits(gx), bits(gA_ref.astype(np.float32))), (cfg, hop)
        gw = w_t.grad.reshape(BL, n).numpy()
        scale = float(np.abs(gw_ref).max()) if gw_ref.size else 1.0
        np.testing.assert_allclose(gw, gw_ref, rtol=1e-5, atol=1e-6 * max(scale, 1e-30))
        s = ref[1] + ref[2] if wot_i else (ref[0] + ref[1]) + ref[2]
        x = (s / np.maximum(s.sum(-1, keepdims=True), np.float32(1e-7))).astype(np.float32)
    return x


def test_c1_drum_cpu_route_full_graph():
    """Config C1 exactly: DRUM, 3 hops, B = 32, N = 3, no top-k, on the CPU route."""
    x = _route_hops(1, 32, 3, False, 1000, 400)
    assert (x != 0).sum(1).min() > 0


def test_c1_drum_cpu_route_hidden_triples_and_budget():
    """C1 with a training-style mask (10% of triples hidden) and c1/c2 budgets
    small enough to bind on C1's rows."""
    _route_hops(1, 32, 3, True, 60, 8, hide=0.1, seed=1)


def test_c3_neurallp_cpu_route():
    """NeuralLP's call: one channel, wot_i, attention width 2R, c1 = 1000, c2 = 400."""
    R = synth.CONFIGS[3].relations
    _route_hops(3, 32, 1, True, 1000, 400, wot_i=True, width=2 * R)


def test_flashlog_function_direct_cpu_and_gpu():
    """FlashLogFunction as the reference's vectorized_operation_csr calls it,
    with the active nodes it computes, on CPU tensors and on GPU tensors:
    the same bits either way, equal to the oracle."""
    fk = _fk()
    h, r, t, E, R, csr, tcsr = _graph(1)
    rng = np.random.default_rng(7)
    B, L, n = 4, 3, 2 * R + 1
    x = np.zeros((B * L, E), np.float32)
    for i in range(B * L):
        x[i, rng.choice(E, 40, replace=False)] = rng.random(40).astype(np.float32) + np.float32(0.01)
    w = synth.make_attention(B, L, n, 1, rng)[0].reshape(B * L, n)
    masks = (np.ones(h.shape[0], np.float32), np.ones(h.shape[0], np.float32))
    ref = O.dense_forward(x, w, csr, masks, R, topk_edges=3)
    for dev in ("cpu", "cuda"):
        A = torch.from_numpy(x).view(B, L, E).to(dev)
        active = fk._compute_active_nodes(A)
        assert active.device.type == dev
        assert np.array_equal(active.cpu().numpy(), O.active_nodes(x))
        om, im = (torch.from_numpy(m).to(dev) for m in masks)
        c = [tc.to(dev) for tc in tcsr]
        outs = fk.FlashLogFunction.apply(A, torch.from_numpy(w).view(B, L, n).to(dev), active,
                                         c[1], om, c[8], c[9], c[10], c[11], c[5], im, c[12], c[13], c[14], c[15],
                                         R, False, 3)
        for o, rf in zip(outs, ref):
            assert o.device.type == dev
            assert np.array_equal(bits(o.reshape(B * L, E).cpu().numpy()), bits(rf))


def test_compute_active_nodes_edges():
    fk = _fk()
    A = torch.zeros(2, 3, 50)
    assert fk._compute_active_nodes(A).numel() == 0
    A[1, 2, 49] = -0.5
    A[0, 0, 0] = 1e-30
    A[1, 1, 17] = float("nan")
    got = fk._compute_active_nodes(A)
    assert got.dtype == torch.long and got.tolist() == O.active_nodes(A.reshape(-1, 50).numpy()).tolist() == [0, 17, 49]


def test_prepare_masks_cpu_with_trainable_edge_weight():
    """prepare_csr_masks on CPU tensors with a trainable edge weight (the
    models' use_soft parameter, [M, 1]): mask[order] * sigmoid(weight[order])
    and, as the reference's CPU expression, a gradient for the weight:
    g * mask * s * (1 - s) at each position's edge, over both sides."""
    fk = _fk()
    h, r, t, E, R, csr, tcsr = _graph(1)
    M = h.shape[0]
    rng = np.random.default_rng(3)
    mask = rng.random(M) >= 0.2
    wv = rng.standard_normal((M, 1)).astype(np.float32)
    weight = torch.from_numpy(wv).requires_grad_(True)
    om, im = fk.prepare_csr_masks(tcsr, torch.from_numpy(mask), weight)
    s = 1.0 / (1.0 + np.exp(-wv[:, 0].astype(np.float64)))
    for got, order in ((om, csr[3]), (im, csr[7])):
        assert got.device.type == "cpu"
        np.testing.assert_allclose(got.detach().numpy(), mask[order] * s[order], rtol=2e-6, atol=0)
    go = rng.standard_normal(M).astype(np.float32)
    gi = rng.standard_normal(M).astype(np.float32)
    ((om * torch.from_numpy(go)).sum() + (im * torch.from_numpy(gi)).sum()).backward()
    want = np.zeros(M)
    np.add.at(want, csr[3], go * mask[csr[3]] * s[csr[3]] * (1 - s[csr[3]]))
    np.add.at(want, csr[7], gi * mask[csr[7]] * s[csr[7]] * (1 - s[csr[7]]))
    np.testing.assert_allclose(weight.grad.numpy()[:, 0], want, rtol=1e-5, atol=1e-7)
