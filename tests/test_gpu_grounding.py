"""GPU parity of the soft-grounding kernels against the oracle (itself
bit-equal to the reference's soft_grounding.cpp): walk records, the capped
and united candidate rows, raw unique counts and the reservoir sampler, all
bit for bit."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import small_graph

pytestmark = pytest.mark.gpu


def _sg():
    from flashlog_amd.flashlog_kernel.soft_grounding_kernel import soft_grounding_kernel as sg
    return sg


def _hub_graph(seed=0):
    """R = 150 relations; node 0 has a group of every relation (150 ORI
    groups), node 7 receives every relation (150 INV groups); other edges
    random."""
    rng = np.random.default_rng(seed)
    E, R = 3000, 150
    h = [np.zeros(R, np.int64), rng.integers(0, E, R), rng.integers(0, E, 20000)]
    t = [rng.integers(0, E, R), np.full(R, 7, np.int64), rng.integers(0, E, 20000)]
    r = [np.arange(R), np.arange(R), rng.integers(0, R, 20000)]
    h, t, r = np.concatenate(h), np.concatenate(t), np.concatenate(r)
    return h, r, t, E, R, O.build_csr_structure(h, t, r, E)


def _att(rng, nheads, ranks, V, zero=0.3):
    a = rng.random((nheads, 3, ranks, V)).astype(np.float32)
    a[a < zero] = 0.0
    return a


@pytest.mark.parametrize("graph", ["small", "hub"])
@pytest.mark.parametrize("mask", [False, True])
@pytest.mark.parametrize("topk,temp", [(1, 1.0), (3, 1.0), (200, 1.0), (5, 2.0)])
def test_walk_records_bitexact(graph, mask, topk, temp):
    sg = _sg()
    rng = np.random.default_rng((graph == "hub") * 1000 + mask * 300 + topk)
    if graph == "small":
        h, r, t, E, R, csr = small_graph(2, 0.2)
        sources = rng.integers(0, E, 40)
    else:
        h, r, t, E, R, csr = _hub_graph()
        sources = np.concatenate([[0, 7, 0, 7], rng.integers(0, E, 30)])
    V = 2 * R + 1
    heads = [1, R + 2]
    att = _att(rng, len(heads), 3, V)
    seeds = [11, 2 ** 45 + 9]
    walks = 97
    dev = torch.device("cuda")
    g, keep = sg._graph(tuple(torch.from_numpy(np.asarray(a)) for a in csr), dev, R)
    n = sources.shape[0]
    th = torch.cat([torch.full((n,), i, dtype=torch.int32) for i in range(len(heads))])
    ts = torch.from_numpy(np.concatenate([sources] * len(heads)))
    ti = torch.cat([torch.arange(n, dtype=torch.int64)] * len(heads))
    keys, pos = sg._walks(g, torch.from_numpy(att), torch.tensor(heads, device=dev), seeds, th, ts, ti, walks, topk,
                          mask, temp, dev)
    keys = keys.cpu().numpy().view(np.uint64).reshape(-1, walks)
    pos = pos.cpu().numpy().reshape(-1, walks)
    for i, head in enumerate(heads):
        rk, rp = O.ground_walks(att[i], R, head, sources, np.arange(n), csr, walks, topk, mask, seeds[i], temp)
        np.testing.assert_array_equal(keys[i * n:(i + 1) * n], rk)
        np.testing.assert_array_equal(pos[i * n:(i + 1) * n], rp)
    assert (keys != 0).mean() > 0.3


@pytest.mark.parametrize("mask", [False, True])
def test_grounding_rows_match_oracle(mask):
    sg = _sg()
    rng = np.random.default_rng(4 + mask)
    h, r, t, E, R, csr = small_graph(2, 0.2)
    V = 2 * R + 1
    heads = [0, R + 1, 2 * R - 1, 3]
    att = _att(rng, len(heads), 2, V)
    folds = [[rng.integers(0, E, 9), rng.integers(0, E, 5)], [rng.integers(0, E, 12)],
             [rng.integers(0, E, 4), rng.integers(0, E, 4), rng.integers(0, E, 3)], [np.zeros(0, np.int64)]]
    seeds = [7, 2 ** 40 + 3, 99, 5]
    budgets = [4, 30, 100]
    walks = 128
    csr_t = tuple(torch.from_numpy(np.asarray(a)) for a in csr)
    cands, raw, secs = sg.ground_head_batch_source_folds_sampled_capped_counts(
        torch.from_numpy(att), heads, R, folds, csr_t, walks, 3, mask, seeds, 1000, 8, budgets)
    assert len(cands) == len(heads) and len(secs) == len(heads)
    for i, head in enumerate(heads):
        rows, rraw = O.ground(att[i], R, head, folds[i], csr, walks, 3, mask, seeds[i], budgets)
        assert cands[i].device.type == "cpu" and cands[i].dtype == torch.int64
        np.testing.assert_array_equal(cands[i].numpy(), rows.reshape(-1, 12))
        assert raw[i] == tuple(rraw)
    assert cands[3].shape == (0, 12)


def test_grounding_rows_wide_keys():
    """Relation ids near 2^15 (inverse operators need 16 bits) and 32769
    folds: the (fold, body) sort key needs 16 + 2 + 3*16 > 64 bits, so the
    counts take the per-fold segmented sort instead of the packed one."""
    sg = _sg()
    rng = np.random.default_rng(21)
    E, R, n_edges = 300, 20000, 4000
    h, t = rng.integers(0, E, n_edges), rng.integers(0, E, n_edges)
    r = rng.integers(19000, R, n_edges)
    csr = O.build_csr_structure(h, t, r, E)
    att = _att(rng, 1, 1, 2 * R + 1, zero=0.0)
    head = 19500
    nfolds = 32769
    folds = [[s] for s in rng.integers(0, E, nfolds)]
    budgets = [4, 30, 100]
    csr_t = tuple(torch.from_numpy(np.asarray(a)) for a in csr)
    cands, raw, _ = sg.ground_head_batch_source_folds_sampled_capped_counts(
        torch.from_numpy(att), [head], R, [[np.asarray(f) for f in folds]], csr_t, 1, 3, False, [5], 1000, 8,
        budgets)
    fold_src = [np.asarray(f, np.int64) for f in folds]
    rows, rraw = O.ground(att[0], R, head, fold_src, csr, 1, 3, False, 5, budgets)
    # the case is the wide one: 16-bit relation fields and 16 fold bits
    src = np.concatenate(fold_src)
    keys, _ = O.ground_walks(att[0], R, head, src, np.zeros(nfolds, np.int64), csr, 1, 3, False, 5)
    kor = int(np.bitwise_or.reduce(keys.reshape(-1)))
    fields = ((kor >> 40) | (kor >> 20) | kor) & ((1 << 20) - 1)
    assert fields.bit_length() == 16 and (nfolds - 1).bit_length() + 2 + 3 * 16 > 64
    np.testing.assert_array_equal(cands[0].numpy(), rows.reshape(-1, 12))
    assert raw[0] == tuple(rraw)


def test_grounding_api_checks():
    sg = _sg()
    h, r, t, E, R, csr = small_graph(2, 0.05)
    V = 2 * R + 1
    att = np.ones((1, 3, 1, V), np.float32)
    csr_t = tuple(torch.from_numpy(np.asarray(a)) for a in csr)
    args = dict(num_relations=R, csr=csr_t, walks_per_source=4, topk_edges=2, mask_query_head_from_source=False,
                transition_cache_size=10, num_threads=2)
    assert sg.ground_head_batch_source_folds_sampled_capped_counts(
        np.zeros((0, 3, 1, V), np.float32), [], source_folds=[], seeds=[], candidates_per_length=[1, 1, 1],
        **args) == ([], [], [])
    with pytest.raises(ValueError):
        sg.ground_head_batch_source_folds_sampled_capped_counts(att, [0], source_folds=[[[1]]], seeds=[1],
                                                                candidates_per_length=[1, 1], **args)
    with pytest.raises(ValueError):
        sg.ground_head_batch_source_folds_sampled_capped_counts(att, [0], source_folds=[[[1]]], seeds=[1],
                                                                candidates_per_length=[1, 1, 1],
                                                                sampling_temperature=0.0, **args)
    with pytest.raises(RuntimeError):
        sg.ground_head_batch_source_folds_sampled_capped_counts(att, [2 * R], source_folds=[[[1]]], seeds=[1],
                                                                candidates_per_length=[1, 1, 1], **args)


@pytest.mark.parametrize("max_sources", [1, 5, 64, 5000])
@pytest.mark.parametrize("seed", [0, 77, 2 ** 61 + 5])
def test_reservoir_bitexact(max_sources, seed):
    sg = _sg()
    h, r, t, E, R, csr = small_graph(2, 1.0)
    rels = np.array(sorted({0, 3, R - 1}), np.int64)
    out, avail = sg.sample_relation_sources_reservoir(torch.from_numpy(csr[8]), torch.from_numpy(csr[9]),
                                                      torch.from_numpy(rels), max_sources, seed)
    ro, ra = O.reservoir(csr[8], csr[9], rels, max_sources, seed)
    assert out.dtype == torch.int32 and avail.dtype == torch.int64
    np.testing.assert_array_equal(out.numpy(), ro)
    np.testing.assert_array_equal(avail.numpy(), ra)


def test_reservoir_checks_and_empty():
    sg = _sg()
    h, r, t, E, R, csr = small_graph(2, 0.05)
    gp, gr = torch.from_numpy(csr[8]), torch.from_numpy(csr[9])
    with pytest.raises(RuntimeError):
        sg.sample_relation_sources_reservoir(gp, gr, torch.tensor([1, 1]), 4, 0)
    with pytest.raises(RuntimeError):
        sg.sample_relation_sources_reservoir(gp, gr, torch.tensor([40000]), 4, 0)
    with pytest.raises(ValueError):
        sg.sample_relation_sources_reservoir(gp, gr, torch.tensor([1]), 0, 0)
    out, avail = sg.sample_relation_sources_reservoir(gp, gr, torch.zeros(0, dtype=torch.int64), 3, 0)
    assert out.shape == (0, 3) and avail.shape == (0,)
