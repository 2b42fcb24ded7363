"""End-to-end evaluation pipeline of the sparse DRUM model against the
oracle: three hops (c1 entity budget, top-k sum hop, normalize_sparse3d),
the channel sum, then the filtered ranks -- the GPU and the oracle each
carry their own state from hop to hop, so nothing of one side feeds the
other.  Coordinates and value bits must agree after every hop and every
normalization, the channel sum must agree bit for bit, and the final ranks
must be equal (src/model_DRUM_kernel_sp.py:124-205, src/main.py:391-465).

C2 runs every query; C5 (4.6M entities, 20M triples) runs every query on
the GPU and checks a sample of queries (rows are independent through the
hops, the channel sum is per query, and a rank depends only on its query's
scores)."""
import numpy as np
import pytest
import torch

from flashlog_amd import synth
from oracle import oracle as O
from tests.helpers import bits

pytestmark = pytest.mark.gpu


def _run(cfg, check_queries, rank_filter_per_query=40):
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    c = synth.CONFIGS[cfg]
    dev = torch.device("cuda")
    h, r, t, E, R = synth.make_graph(cfg)
    n = 2 * R + 1
    B, L, T, K = c.batch, c.channels, c.hops, c.c2 // 2
    csr_t = fk.build_csr_structure(*(torch.from_numpy(a).to(dev) for a in (h, t, r)), E)
    csr = [x.cpu().numpy() for x in csr_t]
    mask = torch.ones(h.shape[0], dtype=torch.bool, device=dev)
    ones = (np.ones(csr[1].shape[0], np.float32), np.ones(csr[5].shape[0], np.float32))
    rng = np.random.Generator(np.random.PCG64(4321 + cfg))
    src, rel, tgt = synth.make_queries(h, r, t, R, B, rng)
    W = synth.make_attention(B, L, n, T, rng)
    Wt = torch.from_numpy(W).to(dev)
    qs = np.asarray(check_queries, np.int64)
    # GPU state: every query; oracle state: the checked queries only
    b = torch.arange(B, device=dev).repeat_interleave(L)
    l = torch.arange(L, device=dev).repeat(B)
    e = torch.from_numpy(src).to(dev).repeat_interleave(L)
    v = torch.ones(B * L, device=dev)
    ob = np.repeat(qs, L)
    ol = np.tile(np.arange(L), qs.size).astype(np.int64)
    oe = np.repeat(src[qs], L).astype(np.int64)
    ov = np.ones(ob.size, np.float32)

    def gpu_rows(idx, vals):
        sel = np.isin(idx[0], qs)
        return (idx[0][sel] * L + idx[1][sel]) * E + idx[2][sel], vals[sel]

    with torch.inference_mode():
        for hop in range(T):
            s = fk.FlashLogFunctionSparse3DTopKSum.apply(b, l, e, v, Wt[hop], *csr_t[:4], *csr_t[4:8],
                                                         *csr_t[8:16], mask, None, B, L, E, R, False, K, False,
                                                         c.c1, False)
            kept = O.sparse_topc(ob, ol, ov, L, c.c1)
            rk, rv = O.sparse_forward(O.SPARSE_TOPK, ob[kept], ol[kept], oe[kept], ov[kept], B, L, E, W[hop], csr,
                                      ones, R, False, K)
            gk, gv = gpu_rows(s.indices().cpu().numpy(), s.values().cpu().numpy())
            assert np.array_equal(gk, rk), (cfg, hop, "hop keys")
            assert np.array_equal(bits(gv), bits(rv)), (cfg, hop, "hop values")
            s = fk.normalize_sparse3d(s)
            ob, ol, oe = rk // (L * E), (rk // E) % L, rk % E
            ov, _ = O.sparse_normalize(ob, ol, rv, B, L)
            gk, gv = gpu_rows(s.indices().cpu().numpy(), s.values().cpu().numpy())
            assert np.array_equal(bits(gv), bits(ov)), (cfg, hop, "normalized values")
            idx = s.indices()
            b, l, e, v = idx[0], idx[1], idx[2], s.values()
        final = fk.sum_sp_3d(torch.sparse_coo_tensor(torch.stack((b, l, e)), v, (B, L, E), is_coalesced=True))
        fi = final.indices()
        fv = final.values()
        sb, se, sv, _ = O.sum_sp_3d(ob, ol, oe, ov, B, L, E)
        fb = fi[0].cpu().numpy()
        sel = np.isin(fb, qs)
        assert np.array_equal(fb[sel], sb) and np.array_equal(fi[1].cpu().numpy()[sel], se)
        assert np.array_equal(bits(fv.cpu().numpy()[sel]), bits(sv)), (cfg, "channel sum")
        # filter: some known answers per query plus the target
        fkeys = np.unique(np.concatenate([
            np.arange(B, dtype=np.int64).repeat(rank_filter_per_query) * E +
            rng.integers(0, E, B * rank_filter_per_query),
            np.arange(B, dtype=np.int64) * E + tgt]))
        for use_eql in (False, True):
            ranks = fk.sparse2d_filtered_ranks_cuda(fi[0], fi[1], fv, torch.from_numpy(tgt).to(dev),
                                                    torch.from_numpy(fkeys).to(dev), B, E, use_eql).cpu().numpy()
            # the oracle over the checked queries, renumbered 0..len(qs)-1
            pos = np.searchsorted(qs, sb)
            fsel = np.isin(fkeys // E, qs)
            fk_local = np.searchsorted(qs, fkeys[fsel] // E) * E + fkeys[fsel] % E
            want = O.filtered_ranks(pos, se, sv, tgt[qs], fk_local, qs.size, E, use_eql)
            assert np.array_equal(ranks[qs], want), (cfg, use_eql)
    return ranks


def test_c2_pipeline_end_to_end():
    ranks = _run(2, np.arange(synth.CONFIGS[2].batch))
    assert ranks.min() >= 1


def test_c5_pipeline_end_to_end():
    ranks = _run(5, [0, 101, 255])
    assert ranks.min() >= 1
