"""Parity at full scale: the C5 workload (4.6M
entities, 822 relations, 20M triples with Zipf(1.3) hubs, batch 256, N = 3)
through two evaluation hops on the GPU, then the third hop (sum with the
c2 threshold, sum with the training quotas, max) checked bit for bit against
the oracle on sampled (query, channel) rows.  Rows are independent in the
hop (c1 per row, c2 per (source, row)), so a row's outputs depend only on
its own entries."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bits

pytestmark = pytest.mark.gpu

ROWS = (0, 383, 767)


@pytest.fixture(scope="module")
def c5():
    from flashlog_amd import synth
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    cfg = synth.CONFIGS[5]
    dev = torch.device("cuda")
    h, r, t, E, R = synth.make_graph(5)
    n = 2 * R + 1
    B, L, T = cfg.batch, cfg.channels, cfg.hops
    K = cfg.c2 // 2
    csr = fk.build_csr_structure(*(torch.from_numpy(a).to(dev) for a in (h, t, r)), E)
    mask = torch.ones(h.shape[0], dtype=torch.bool, device=dev)
    rng = np.random.Generator(np.random.PCG64(1234 + 5))
    src, _, _ = synth.make_queries(h, r, t, R, B, rng)
    W = torch.from_numpy(synth.make_attention(B, L, n, T, rng)).to(dev)
    b = torch.arange(B, device=dev).repeat_interleave(L)
    l = torch.arange(L, device=dev).repeat(B)
    e = torch.from_numpy(src).to(dev).repeat_interleave(L)
    v = torch.ones(B * L, device=dev)
    with torch.inference_mode():
        for hop in range(2):
            s = fk.FlashLogFunctionSparse3DTopKSum.apply(b, l, e, v, W[hop], *csr[:4], *csr[4:8], *csr[8:16], mask,
                                                         None, B, L, E, R, False, K, False, cfg.c1, False)
            s = fk.normalize_sparse3d(s)
            idx = s.indices()
            b, l, e, v = idx[0], idx[1], idx[2], s.values()
        keep = fk._sparse_topc_entries(b, l, e, v, cfg.c1, L)
    if keep is not None:
        b, l, e, v = b[keep], l[keep], e[keep], v[keep]
    csr_np = [c.cpu().numpy() for c in csr]
    ones = (np.ones(csr_np[1].shape[0], np.float32), np.ones(csr_np[5].shape[0], np.float32))
    return dict(fk=fk, csr=csr, csr_np=csr_np, masks=ones, mask=mask, W2=W[2], B=B, L=L, E=E, R=R, K=K,
                state=(b, l, e, v), dev=dev)


def _rows(c, keys):
    row = keys // c["E"]
    return np.isin(row, ROWS)


def _oracle_state(c):
    b, l, e, v = (x.cpu().numpy() for x in c["state"])
    sel = np.isin(b * c["L"] + l, ROWS)
    return b[sel], l[sel], e[sel], v[sel]


def _sides(c, mx):
    fk, tc, om = c["fk"], c["csr"], c["masks"]
    m0, m1 = (torch.from_numpy(x).to(c["dev"]) for x in om)
    return fk._SparseSides(tc[1], m0, tc[8], tc[9], tc[10], tc[11], tc[5], m1, tc[12], tc[13], tc[14], tc[15],
                           tc[3] if mx else None, tc[7] if mx else None)


@pytest.mark.parametrize("variant", ["sum", "sum_quota", "max"])
def test_c5_third_hop_rows_bitexact(c5, variant):
    c = c5
    fk = c["fk"]
    B, L, E, R, K = c["B"], c["L"], c["E"], c["R"], c["K"]
    b, l, e, v = c["state"]
    mx = variant == "max"
    seed = 8675309 if variant == "sum_quota" else -1
    with torch.inference_mode():
        idx, vals, _ = fk._sparse_forward(b, l, e, v, c["W2"], _sides(c, mx), B, L, E, R, False, fk._SPARSE_TOPK, K,
                                          False, aggregate=fk._SPARSE_MAX if mx else fk._SPARSE_SUM, seed=seed)
    idx = idx.cpu().numpy()
    keys = (idx[0] * L + idx[1]) * E + idx[2]
    vals = vals.cpu().numpy()
    sel = _rows(c, keys)
    ob, ol, oe, ov = _oracle_state(c)
    w = c["W2"].cpu().numpy()
    if mx:
        rk, rv, *_ = O.sparse_max_forward(ob, ol, oe, ov, B, L, E, w, c["csr_np"], c["masks"], R, False, K, seed)
    else:
        rk, rv = O.sparse_forward(O.SPARSE_TOPK, ob, ol, oe, ov, B, L, E, w, c["csr_np"], c["masks"], R, False, K,
                                  seed)
    assert rk.shape[0] > 10000  # hub rows: tens of thousands of outputs each
    assert np.array_equal(keys[sel], rk)
    assert np.array_equal(bits(vals[sel]), bits(rv))


@pytest.mark.parametrize("seed", [-1, 424242])
def test_c5_third_hop_backward_bilinear(c5, seed):
    """The hop is bilinear in (entry values, attention) once its selections
    are fixed: <g, out> = <grad_v, v> = <grad_w, w> for any output gradient
    g, at full scale (float64 sums of the fp32 terms; 1e-5 relative)."""
    c = c5
    fk = c["fk"]
    B, L, E, R, K = c["B"], c["L"], c["E"], c["R"], c["K"]
    b, l, e, v = c["state"]
    w2 = c["W2"]
    idx, vals, st = fk._sparse_forward(b, l, e, v, w2, _sides(c, False), B, L, E, R, False, fk._SPARSE_TOPK, K, True,
                                       seed=seed)
    gen = torch.Generator(device=c["dev"]).manual_seed(7)
    g = torch.randn(vals.shape[0], device=c["dev"], generator=gen)
    gv, gw = fk._sparse_backward(st, g)
    lhs = float((g.double() * vals.double()).sum())
    via_v = float((gv.double() * v.double()).sum())
    via_w = float((gw.double() * w2.reshape(B * L, -1).double()).sum())
    scale = float((g.double().abs() * vals.double().abs()).sum())
    assert abs(lhs - via_v) <= 1e-5 * scale
    assert abs(lhs - via_w) <= 1e-5 * scale


@pytest.mark.parametrize("seed", [-1, 424242])
def test_c5_third_hop_backward_rows_elementwise(c5, seed):
    """The third hop's backward at full scale, element by element on the
    sampled rows, against the oracle's backward (pinned element-wise to the
    reference's CPU backward): grad_v of their entries within 1e-5; their
    grad_w rows within 1e-5 of the magnitude of each element's terms.  A
    hub row's grad_w[r, c] adds ~10^5 fp32 terms of both signs, so two
    summation orders differ by about sqrt(N) ulps of the terms' 1-norm --
    as the reference's own CPU backward does between thread counts
    (flashlog.cpp:1068-1130) -- which can exceed 1e-5 of the cancelled
    result; the 1-norm S[r, c] = sum |g| * m * a comes from the same oracle
    with |g| (m >= 0, a > 0).  Rows are independent, so a row's gradients
    depend only on its own outputs' gradients."""
    from tests.helpers import assert_grad_close
    c = c5
    fk = c["fk"]
    B, L, E, R, K = c["B"], c["L"], c["E"], c["R"], c["K"]
    b, l, e, v = c["state"]
    w2 = c["W2"]
    idx, vals, st = fk._sparse_forward(b, l, e, v, w2, _sides(c, False), B, L, E, R, False, fk._SPARSE_TOPK, K, True,
                                       seed=seed)
    gen = torch.Generator(device=c["dev"]).manual_seed(11)
    g = torch.randn(vals.shape[0], device=c["dev"], generator=gen)
    gv, gw = fk._sparse_backward(st, g)
    idx = idx.cpu().numpy()
    keys = (idx[0] * L + idx[1]) * E + idx[2]
    sel = _rows(c, keys)
    ob, ol, oe, ov = _oracle_state(c)
    rgv, rgw = O.sparse_backward(O.SPARSE_TOPK, ob, ol, oe, ov, B, L, E, w2.cpu().numpy(), c["csr_np"], c["masks"], R,
                                 keys[sel], g.cpu().numpy()[sel], False, K, seed)
    rows = (b * L + l).cpu().numpy()
    assert_grad_close(gv.cpu().numpy()[np.isin(rows, ROWS)], rgv)
    _, norm1 = O.sparse_backward(O.SPARSE_TOPK, ob, ol, oe, ov, B, L, E, w2.cpu().numpy(), c["csr_np"], c["masks"],
                                 R, keys[sel], np.abs(g.cpu().numpy()[sel]), False, K, seed)
    gw = gw.cpu().numpy()
    for r in ROWS:
        err = np.abs(gw[r].astype(np.float64) - rgw[r])
        assert (err <= 1e-5 * norm1[r].astype(np.float64) + 1e-30).all(), (r, float((err / norm1[r]).max()))
        assert_grad_close(gw[r], rgw[r], rtol=1e-4)
