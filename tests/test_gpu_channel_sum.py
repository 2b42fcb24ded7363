"""Channel sum of a coalesced [B, L, E] state (the models' sum_sp_3d,
src/model_DRUM_kernel_sp.py:22-28) through the C-ABI: indices, value bits
and gradients against torch's coalesce of the (b, e) re-index on the GPU
(what the reference runs) and against the oracle."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _fk():
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    return fk


def _state(seed, B, L, E, n, order_cases=False):
    rng = np.random.default_rng(seed)
    keys = np.unique(rng.choice(B * L * E, size=n, replace=False))
    b, l, e = keys // (L * E), (keys // E) % L, keys % E
    v = rng.random(b.shape[0]).astype(np.float32)
    if order_cases:  # large and small values on one (b, e): rounding depends on the channel order
        big = rng.random(b.shape[0]) < 0.3
        v[big] *= np.float32(1e7)
        v[(~big) & (rng.random(b.shape[0]) < 0.3)] *= np.float32(-1.0)
    return b, l, e, v


def _torch_sum(b, e, v, B, E, dev):
    t = torch.sparse_coo_tensor(torch.stack([b, e]), v, [B, E]).coalesce()
    return t


@pytest.mark.parametrize("B,L,E,n,seed", [
    (4, 3, 60, 300, 0),         # most (b, e) in several channels
    (16, 3, 5000, 20000, 1),
    (8, 1, 1000, 3000, 2),      # one channel: a copy
    (8, 5, 200, 6000, 3),       # dense: nearly every (b, e) in all channels
    (4, 8, 400, 9000, 5),       # many channels: every entry ranked in seven other rows
    (6, 10, 300, 12000, 6),
    (256, 3, 4_600_000, 3_000_000, 4),
])
def test_channel_sum_bitexact(B, L, E, n, seed):
    fk = _fk()
    dev = torch.device("cuda:0")
    b, l, e, v = _state(seed, B, L, E, n, order_cases=True)
    tb, tl, te = (torch.from_numpy(x).to(dev) for x in (b, l, e))
    vt = torch.from_numpy(v).to(dev).requires_grad_(True)
    s = torch.sparse_coo_tensor(torch.stack([tb, tl, te]), vt, [B, L, E], is_coalesced=True)
    got = fk.sum_sp_3d(s)
    vr = vt.detach().clone().requires_grad_(True)
    ref = _torch_sum(tb, te, vr, B, E, dev)
    assert got.is_coalesced() and tuple(got.shape) == (B, E)
    assert torch.equal(got.indices(), ref.indices())
    assert torch.equal(got.values().detach().view(torch.int32), ref.values().detach().view(torch.int32))
    if n <= 20000:
        ob, oe, ov, _ = O.sum_sp_3d(b, l, e, v, B, L, E)
        assert np.array_equal(got.indices().cpu().numpy(), np.stack([ob, oe]))
        assert np.array_equal(got.values().detach().cpu().numpy().view(np.int32), ov.view(np.int32))
    g = torch.randn(ref.values().shape[0], device=dev)
    (got.values() * g).sum().backward()
    (ref.values() * g).sum().backward()
    assert torch.equal(vt.grad, vr.grad)


def test_channel_sum_empty_and_errors():
    fk = _fk()
    dev = torch.device("cuda:0")
    z = torch.zeros((3, 0), dtype=torch.int64, device=dev)
    s = torch.sparse_coo_tensor(z, torch.zeros(0, device=dev), [2, 3, 10], is_coalesced=True)
    got = fk.sum_sp_3d(s)
    assert got.values().numel() == 0 and tuple(got.shape) == (2, 10)
    # marked coalesced, but the entities of row (0, 1) decrease: refused
    idx = torch.tensor([[0, 0, 0], [1, 1, 2], [5, 3, 1]], device=dev)
    bad = torch.sparse_coo_tensor(idx, torch.ones(3, device=dev), [1, 3, 10], is_coalesced=True)
    with pytest.raises(ValueError):
        fk.sum_sp_3d(bad)


def _reference_max_sp_3d(s):
    # the reference's steps (src/model_mmDRUM_kernel_sp.py:17-32) in torch
    s = s.coalesce()
    idx, val = s.indices(), s.values()
    B, _, E = s.shape
    flat_key = idx[0] * E + idx[2]
    order = torch.argsort(flat_key)
    flat_key, val = flat_key[order], val[order]
    uniq, inv = torch.unique_consecutive(flat_key, return_inverse=True)
    out_val = torch.zeros(uniq.shape[0], device=val.device, dtype=val.dtype)
    out_val = out_val.scatter_reduce(0, inv, val, reduce="amax", include_self=False)
    return torch.sparse_coo_tensor(torch.stack([uniq // E, uniq % E]), out_val, [B, E]).coalesce()


@pytest.mark.parametrize("B,L,E,n,seed", [(4, 3, 60, 300, 10), (16, 3, 5000, 20000, 11), (8, 5, 200, 6000, 12),
                                          (256, 3, 4_600_000, 2_000_000, 13)])
def test_channel_max_matches_reference_steps(B, L, E, n, seed):
    fk = _fk()
    dev = torch.device("cuda:0")
    b, l, e, _ = _state(seed, B, L, E, n)
    rng = np.random.default_rng(seed)
    v = (rng.integers(0, 6, b.shape[0]) / 8.0).astype(np.float32)  # ties and exact zeros
    tb, tl, te = (torch.from_numpy(x).to(dev) for x in (b, l, e))
    vt = torch.from_numpy(v).to(dev).requires_grad_(True)
    vr = vt.detach().clone().requires_grad_(True)
    got = fk.max_sp_3d(torch.sparse_coo_tensor(torch.stack([tb, tl, te]), vt, [B, L, E], is_coalesced=True))
    ref = _reference_max_sp_3d(torch.sparse_coo_tensor(torch.stack([tb, tl, te]), vr, [B, L, E]))
    assert torch.equal(got.indices(), ref.indices())
    assert torch.equal(got.values().detach().view(torch.int32), ref.values().detach().view(torch.int32))
    g = torch.randn(ref.values().shape[0], device=dev)
    (got.values() * g).sum().backward()
    (ref.values() * g).sum().backward()
    assert torch.equal(vt.grad.view(torch.int32), vr.grad.view(torch.int32))


@pytest.mark.parametrize("seed", [21, 22])
def test_channel_max_special_values(seed):
    """NaN and +-inf inside (b, e) groups: value bits and the amax gradient
    split as the reference's scatter_reduce steps give them.  (A group
    holding both -0.0 and +0.0 has no fixed reference: torch's atomic amax
    keeps whichever zero it stores first, so such ties are left out.)"""
    fk = _fk()
    dev = torch.device("cuda:0")
    B, L, E, n = 4, 3, 40, 240
    b, l, e, _ = _state(seed, B, L, E, n)
    rng = np.random.default_rng(seed)
    v = (rng.integers(-3, 4, b.shape[0]) / 4.0).astype(np.float32)
    specials = np.array([np.nan, np.inf, -np.inf], dtype=np.float32)
    pick = rng.choice(b.shape[0], size=min(40, b.shape[0]), replace=False)
    v[pick] = specials[rng.integers(0, specials.shape[0], pick.shape[0])]
    tb, tl, te = (torch.from_numpy(x).to(dev) for x in (b, l, e))
    vt = torch.from_numpy(v).to(dev).requires_grad_(True)
    vr = vt.detach().clone().requires_grad_(True)
    got = fk.max_sp_3d(torch.sparse_coo_tensor(torch.stack([tb, tl, te]), vt, [B, L, E], is_coalesced=True))
    ref = _reference_max_sp_3d(torch.sparse_coo_tensor(torch.stack([tb, tl, te]), vr, [B, L, E]))
    assert torch.equal(got.indices(), ref.indices())
    assert torch.equal(got.values().detach().view(torch.int32), ref.values().detach().view(torch.int32))
    g = torch.randn(ref.values().shape[0], device=dev)
    (got.values() * g).sum().backward()
    (ref.values() * g).sum().backward()
    assert torch.equal(vt.grad.view(torch.int32), vr.grad.view(torch.int32))
