"""Dense hops on the full benchmark graphs (C1-C4), forward and backward,
against the CPU oracle: three hops each, every hop fed the oracle's state
so both sides see the same input.

- C1: DRUM without top-k (3k entities, 12 relations, 28k triples, B=32).
- C2: DRUM with c1=1000, c2=400 (41k entities, Zipf(1.1) degrees).
- C3: DRUM (n = 475 attention columns) and NeuralLP (wot_i, width 2R = 474,
  one channel) with c1=1000, c2=400 (14.5k entities, 237 relations).
- C4: mmDRUM dense max with c1=1000, c2=400 (123k entities, Zipf(1.2)
  degrees with hubs above 10k).

Outputs and winning positions are compared bit for bit; grad_A bit for bit
(the per-(source, row) walk adds in the CPU path's order); grad_w within
1e-5 relative (a fixed association of the same terms)."""
import numpy as np
import pytest
import torch

from flashlog_amd import synth
from oracle import oracle as O
from tests.helpers import bits, to_torch_csr

pytestmark = pytest.mark.gpu

_GRAPHS = {}


def _fk():
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    return fk


def _graph(cfg):
    if cfg not in _GRAPHS:
        h, r, t, E, R = synth.make_graph(cfg)
        csr = O.build_csr_structure(h, t, r, E)
        _GRAPHS[cfg] = (h, E, R, csr, to_torch_csr(csr, torch.device("cuda")))
    return _GRAPHS[cfg]


def _keep(x, c):
    """The c1 keep mask: rows over the budget keep their kept entries, the
    others everything (flashlog_kernel.py:814-842)."""
    if c is None:
        return np.ones(x.shape, bool)
    xp = O.dense_topc(x, c)[0]
    over = (x != 0).sum(1) > c
    return np.where(over[:, None], xp != 0, True)


def _upstream(rng, BL, E):
    g = [rng.standard_normal((BL, E)).astype(np.float32) for _ in range(3)]
    g[1][rng.random((BL, E)) < 0.3] = 0.0  # zero upstream grads are skipped, as in the reference
    return g


def _check_grads(x_t, w_t, gA_ref, gw_ref, keep, BL, E, n):
    gx = x_t.grad.reshape(BL, E).cpu().numpy()
    want = (gA_ref * keep.astype(np.float32)).astype(np.float32)
    assert np.array_equal(bits(gx), bits(want)), float(np.abs(gx - want).max())
    gw = w_t.grad.reshape(BL, n).cpu().numpy()
    scale = float(np.abs(gw_ref).max()) if gw_ref.size else 1.0
    np.testing.assert_allclose(gw, gw_ref, rtol=1e-5, atol=1e-6 * max(scale, 1e-30))


def _sum_hops(cfg, B, L, c1, K, wot_i=False, width=None, seed=0):
    fk = _fk()
    h, E, R, csr, tcsr = _graph(cfg)
    n = width if width is not None else 2 * R + 1
    BL = B * L
    dev = torch.device("cuda")
    rng = np.random.Generator(np.random.PCG64(1234 + cfg + seed))
    hh, rr, tt, _, _ = synth.make_graph(cfg)
    src, _, _ = synth.make_queries(hh, rr, tt, R, B, rng)
    W = synth.make_attention(B, L, n, 3, rng)
    M = h.shape[0]
    masks = (np.ones(M, np.float32), np.ones(M, np.float32))
    mk = tuple(torch.from_numpy(m).to(dev) for m in masks)
    x = np.zeros((BL, E), np.float32)
    x[np.arange(BL), np.repeat(src, L)] = 1.0
    kk = K if K else (1 << 60)
    for hop in range(3):
        w = W[hop].reshape(BL, n)
        xp = O.dense_topc(x, c1)[0] if c1 is not None else x
        ref = O.dense_forward(xp, w, csr, masks, R, wot_i=wot_i, topk_edges=kk)
        x_t = torch.from_numpy(x).to(dev).view(B, L, E).requires_grad_(True)
        w_t = torch.from_numpy(w).to(dev).view(B, L, n).requires_grad_(True)
        outs = fk.dense_csr_sum_cuda(x_t, w_t, tcsr, None, R, wot_i=wot_i, use_topk=K > 0,
                                     topk_nodes=c1 if c1 is not None else E, topk_edges=K, prepared_masks=mk)
        for name, o, rf in zip(("ind", "ori", "inv"), outs, ref):
            got = o.detach().reshape(BL, E).cpu().numpy()
            assert np.array_equal(bits(got), bits(rf)), (cfg, hop, name)
        g = _upstream(rng, BL, E)
        sum((o * torch.from_numpy(gg).to(dev).view(B, L, E)).sum() for o, gg in zip(outs, g)).backward()
        gA_ref, gw_ref = O.dense_backward(*g, xp, w, csr, masks, R, wot_i=wot_i, topk_edges=kk)
        _check_grads(x_t, w_t, gA_ref, gw_ref, _keep(x, c1), BL, E, n)
        s = ref[1] + ref[2] if wot_i else (ref[0] + ref[1]) + ref[2]
        x = (s / np.maximum(s.sum(-1, keepdims=True), np.float32(1e-7))).astype(np.float32)
        if wot_i:
            x = x + np.float32(0.5) * xp  # NeuralLP's memory attention keeps earlier states in play
    return x


def test_c1_drum_dense_no_topk():
    x = _sum_hops(1, 32, 3, None, 0)
    assert (x != 0).sum(1).min() > 0


def test_c2_drum_dense_forward_backward():
    _sum_hops(2, 32, 3, 1000, 200)


def test_c3_drum_dense_forward_backward():
    _sum_hops(3, 32, 3, 1000, 200)


def test_c3_neurallp_dense_forward_backward():
    R = synth.CONFIGS[3].relations
    _sum_hops(3, 32, 1, 1000, 200, wot_i=True, width=2 * R)


def test_c4_mmdrum_dense_max_forward_backward():
    fk = _fk()
    cfg, B, L, c1, K = 4, 32, 3, 1000, 200
    h, E, R, csr, tcsr = _graph(cfg)
    n = 2 * R + 1
    BL = B * L
    dev = torch.device("cuda")
    rng = np.random.Generator(np.random.PCG64(1234 + cfg))
    hh, rr, tt, _, _ = synth.make_graph(cfg)
    src, _, _ = synth.make_queries(hh, rr, tt, R, B, rng)
    W = synth.make_attention(B, L, n, 3, rng)
    M = h.shape[0]
    masks = (np.ones(M, np.float32), np.ones(M, np.float32))
    mk = tuple(torch.from_numpy(m).to(dev) for m in masks)
    graph = fk._graph_for(tcsr[1], tcsr[8], tcsr[9], tcsr[10], tcsr[11], tcsr[5], tcsr[12], tcsr[13], tcsr[14],
                          tcsr[15])
    assert graph.ori.nheavy + graph.inv.nheavy > 0
    x = np.zeros((BL, E), np.float32)
    x[np.arange(BL), np.repeat(src, L)] = 1.0
    for hop in range(3):
        w = W[hop].reshape(BL, n)
        xp = O.dense_topc(x, c1)[0]
        oi, oo, ov, ao, av = O.dense_max_forward(xp, w, csr, masks, R, topk_edges=K)
        x_t = torch.from_numpy(x).to(dev).view(B, L, E).requires_grad_(True)
        w_t = torch.from_numpy(w).to(dev).view(B, L, n).requires_grad_(True)
        outs = fk.dense_csr_max(x_t, w_t, tcsr, None, R, use_topk=True, topk_nodes=c1, topk_edges=K,
                                prepared_masks=mk)
        for name, o, rf in zip(("ind", "ori", "inv"), outs, (oi, oo, ov)):
            assert np.array_equal(bits(o.detach().reshape(BL, E).cpu().numpy()), bits(rf)), (hop, name)
        args = fk._dense_max_forward(torch.from_numpy(xp).to(dev), torch.from_numpy(w).to(dev), graph, mk[0],
                                     mk[1], R, False, K)[3:]
        assert np.array_equal(args[0].cpu().numpy(), ao) and np.array_equal(args[1].cpu().numpy(), av), hop
        g = _upstream(rng, BL, E)
        sum((o * torch.from_numpy(gg).to(dev).view(B, L, E)).sum() for o, gg in zip(outs, g)).backward()
        gA_ref, gw_ref = O.dense_max_backward(*g, ao, av, xp, w, csr, masks, R, topk_edges=K)
        _check_grads(x_t, w_t, gA_ref, gw_ref, _keep(x, c1), BL, E, n)
        s = np.maximum(np.maximum(oi, oo), ov)
        x = (s / np.maximum(s.sum(-1, keepdims=True), np.float32(1e-7))).astype(np.float32)
    assert (x != 0).sum(1).max() > 1000  # the last hops ran over-budget rows through c1
