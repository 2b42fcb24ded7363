"""GPU parity of the dense sum and max hops with many (query, channel) rows:
BL = 300 (ten 32-row words, the last partial; five 64-row blocks of the
heavy list phase, the last partial) and BL = 1000 (32 row words: the light
tiles shrink to fit LDS, the max tile holds 4 destinations).  On a graph
with a hub destination (heavy segments and supersegments on both sides)
and ordinary light destinations: values and winning positions bit for bit,
grad_A bit for bit, grad_w within 1e-5 relative, against the oracle."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import attention, bits, masks_for, sparse_state, to_torch_csr

pytestmark = pytest.mark.gpu


def _graph(seed):
    """3000 entities, 20k edges of 4 relations, 40% of them into entity 777
    and 20% out of entity 11 (a hub on each side)."""
    rng = np.random.default_rng(seed)
    E, R, M = 3000, 4, 20000
    h = np.where(rng.random(M) < 0.2, 11, rng.integers(0, E, M))
    t = np.where(rng.random(M) < 0.4, 777, rng.integers(0, E, M))
    r = rng.integers(0, R, M)
    return rng, E, R, M, O.build_csr_structure(h, t, r, E)


def _inputs(BL, seed):
    rng, E, R, M, csr = _graph(seed)
    n = 2 * R + 1
    A = sparse_state(BL, E, 40, rng, ties=True)
    A[:, 11] = 0.5  # the out-hub is active in every row
    w = attention(BL, n, rng)
    _, masks = masks_for(csr, M, rng)
    g = [rng.standard_normal((BL, E)).astype(np.float32) for _ in range(3)]
    g[1][rng.random((BL, E)) < 0.3] = 0.0
    return E, R, n, csr, A, w, masks, g


def _run(op, A, w, csr, masks, R, K, B, L, g):
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    dev = torch.device("cuda")
    E, n = A.shape[1], w.shape[1]
    At = torch.from_numpy(A).to(dev).view(B, L, E).requires_grad_(True)
    wt = torch.from_numpy(w).to(dev).view(B, L, n).requires_grad_(True)
    mk = tuple(torch.from_numpy(m).to(dev) for m in masks)
    fn = fk.dense_csr_sum_cuda if op == "sum" else fk.dense_csr_max
    outs = fn(At, wt, to_torch_csr(csr, dev), None, R, use_topk=K > 0, topk_nodes=E, topk_edges=K,
              prepared_masks=mk)
    loss = sum((o * torch.from_numpy(gg).to(dev).view(B, L, E)).sum() for o, gg in zip(outs, g))
    loss.backward()
    torch.cuda.synchronize()
    BL = B * L
    return ([o.reshape(BL, E).detach().cpu().numpy() for o in outs], At.grad.reshape(BL, E).cpu().numpy(),
            wt.grad.reshape(BL, n).cpu().numpy())


@pytest.mark.parametrize("B,L", [(60, 5), (200, 5)])
@pytest.mark.parametrize("K", [0, 3])
def test_dense_sum_wide(B, L, K):
    BL = B * L
    E, R, n, csr, A, w, masks, g = _inputs(BL, 40 + BL + K)
    kk = K if K > 0 else (1 << 60)
    ref = O.dense_forward(A, w, csr, masks, R, topk_edges=kk)
    gA_ref, gw_ref = O.dense_backward(*g, A, w, csr, masks, R, topk_edges=kk)
    outs, gA, gw = _run("sum", A, w, csr, masks, R, K, B, L, g)
    for name, o, rr in zip(("ind", "ori", "inv"), outs, ref):
        assert np.array_equal(bits(o), bits(rr)), (name, float(np.abs(o - rr).max()))
    assert np.any(ref[1][:, 777] != 0)
    assert np.array_equal(bits(gA), bits(gA_ref)), float(np.abs(gA - gA_ref).max())
    np.testing.assert_allclose(gw, gw_ref, rtol=1e-5, atol=1e-6 * float(np.abs(gw_ref).max()))


@pytest.mark.parametrize("B,L", [(60, 5), (200, 5)])
@pytest.mark.parametrize("K", [0, 3])
def test_dense_max_wide(B, L, K):
    BL = B * L
    E, R, n, csr, A, w, masks, g = _inputs(BL, 70 + BL + K)
    kk = K if K > 0 else (1 << 60)
    oi, oo, ov, ao, av = O.dense_max_forward(A, w, csr, masks, R, topk_edges=kk)
    gA_ref, gw_ref = O.dense_max_backward(*g, ao, av, A, w, csr, masks, R, topk_edges=kk)
    outs, gA, gw = _run("max", A, w, csr, masks, R, K, B, L, g)
    for name, o, rr in zip(("ind", "ori", "inv"), outs, (oi, oo, ov)):
        assert np.array_equal(bits(o), bits(rr)), (name, float(np.abs(o - rr).max()))
    assert np.any(oo[:, 777] != 0)
    assert np.array_equal(bits(gA), bits(gA_ref)), float(np.abs(gA - gA_ref).max())
    np.testing.assert_allclose(gw, gw_ref, rtol=1e-5, atol=1e-6 * float(np.abs(gw_ref).max()))
