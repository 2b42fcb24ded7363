"""Evaluation consumers on the GPU (src/main.py:117-512): the known-answer
indices of a query batch from a graph CSR, from triple-frame lookups and
from (head, relation) groupings, against the oracle and a scan of the
triples; the Hits@k / reciprocal-rank accumulations of the filtered and raw
rankings against the oracle's ranks."""
import types

import numpy as np
import pandas as pd
import pytest
import torch

from flashlog_amd import evaluation as ev
from flashlog_amd import synth
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _fk():
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    return fk


def _eq(got, want):
    assert got[0].dtype == torch.long and got[1].dtype == torch.long
    assert np.array_equal(got[0].cpu().numpy(), want[0]) and np.array_equal(got[1].cpu().numpy(), want[1])


def _tiny(seed, E=15, R=4, M=150):
    rng = np.random.default_rng(seed)
    h, r, t = rng.integers(0, E, M), rng.integers(0, R, M), rng.integers(0, E, M)
    h[:10], r[:10] = 3, 1
    t[5:10] = t[:5]
    return rng, h, r, t, E, R


@pytest.mark.parametrize("cfg", [1, 2, 4])
def test_filter_indices_from_graph_csr(cfg):
    h, r, t, E, R = synth.make_graph(cfg)
    rng = np.random.default_rng(cfg)
    csr = _fk().build_csr_structure(*(torch.from_numpy(a).cuda() for a in (h, t, r)), E)
    B = 5000 if cfg == 4 else 256
    i = rng.integers(0, h.size, B)
    inv = rng.random(B) < 0.5  # forward (h, r) and inverse (t, r + R) queries of real triples
    x = np.where(inv, t[i], h[i])
    q = np.where(inv, r[i] + R, r[i])
    x[:3] = E - 1  # and a few arbitrary ones
    xt, qt = torch.from_numpy(x).cuda(), torch.from_numpy(q).cuda()
    got = ev.build_filter_indices_csr(xt, qt, R, csr)
    host = [c.cpu().numpy() for c in csr]
    look = (O.filter_side_lookup(host[8], host[9], host[10], host[11], host[1], R),
            O.filter_side_lookup(host[12], host[13], host[14], host[15], host[5], R))
    want = O.filter_indices(x, q, R, look)
    assert got[0].is_cuda
    _eq(got, want)
    assert ev.build_filter_indices_csr(xt, qt, R, csr)[0].data_ptr() != got[0].data_ptr()  # cached lookup reused
    assert len([k for k in ev._FILTER_CSR_LOOKUP_CACHE if k[0] == R]) >= 1


def test_filter_indices_tiny_and_edge_cases():
    for seed in range(4):
        rng, h, r, t, E, R = _tiny(seed)
        csr = _fk().build_csr_structure(*(torch.from_numpy(a).cuda() for a in (h, t, r)), E)
        x = rng.integers(0, E, 60)
        q = rng.integers(0, 2 * R, 60)
        _eq(ev.build_filter_indices_csr(torch.from_numpy(x).cuda(), torch.from_numpy(q).cuda(), R, csr),
            O.filter_indices_brute(h, r, t, R, x, q))
    # CPU inputs: results come back on the CPU
    got = ev.build_filter_indices_csr(torch.from_numpy(x), torch.from_numpy(q), R, csr)
    assert got[0].device.type == "cpu"
    _eq(got, O.filter_indices_brute(h, r, t, R, x, q))
    # empty batch, no known answers, only inverse queries, a source past the last entity
    e = np.zeros(0, np.int64)
    for x, q in [(e, e), (np.array([E - 1]), np.array([0])), (np.array([0, 3, 5]), np.array([R, R + 1, 2 * R - 1])),
                 (np.array([E + 3, 2]), np.array([1, 0]))]:
        got = ev.build_filter_indices_csr(torch.from_numpy(x).cuda(), torch.from_numpy(q).cuda(), R, csr)
        _eq(got, O.filter_indices_brute(h, r, t, R, x, q))
    # a graph without edges
    z = torch.zeros(0, dtype=torch.long, device="cuda")
    empty_csr = _fk().build_csr_structure(z, z, z, 4)
    got = ev.build_filter_indices_csr(torch.tensor([1], device="cuda"), torch.tensor([0], device="cuda"), 2, empty_csr)
    assert got[0].numel() == 0 and got[1].numel() == 0


def _dataset(h, r, t, R, rng):
    M = h.size
    split = rng.permutation(M)
    frame = pd.DataFrame({0: h, 1: r, 2: t})
    a, b = int(M * 0.8), int(M * 0.9)
    return types.SimpleNamespace(kg=frame.iloc[split[:a]].reset_index(drop=True),
                                 valid_data=frame.iloc[split[a:b]].reset_index(drop=True),
                                 test_data=frame.iloc[split[b:]].reset_index(drop=True), relation_size=R)


@pytest.mark.parametrize("seed", [0, 1])
def test_filter_indices_from_frame_lookups(seed):
    rng, h, r, t, E, R = _tiny(seed, E=40, R=5, M=600)
    ds = _dataset(h, r, t, R, rng)
    lookups, a, b = ev.create_eval_filter_csr(ds, E, "cuda")
    assert a is None and b is None and len(lookups["filter_lookups"]) == 2
    x = rng.integers(0, E, 80)
    q = rng.integers(0, 2 * R, 80)
    got = ev.build_filter_indices_csr(torch.from_numpy(x).cuda(), torch.from_numpy(q).cuda(), R, lookups)
    held = pd.concat([ds.valid_data, ds.test_data], ignore_index=True)
    parts = []
    for fr in (ds.kg, held):
        fh, fr_, ft = (fr[i].values for i in range(3))
        parts.append(O.filter_indices(x, q, R, (O.filter_edge_lookup(fh, fr_, ft, R),
                                                 O.filter_edge_lookup(ft, fr_, fh, R))))
        brute = O.filter_indices_brute(fh, fr_, ft, R, x, q)
        assert np.array_equal(parts[-1][0], brute[0]) and np.array_equal(parts[-1][1], brute[1])
    _eq(got, (np.concatenate([p[0] for p in parts]), np.concatenate([p[1] for p in parts])))
    # the single-side builder agrees with the frame lookup
    side = ev._build_filter_edge_lookup(torch.from_numpy(h).cuda(), torch.from_numpy(r).cuda(),
                                        torch.from_numpy(t).cuda(), R)
    gk, st, ct, cols = O.filter_edge_lookup(h, r, t, R)
    assert np.array_equal(side.group_start.cpu().numpy(), st)
    assert np.array_equal(side.group_count.cpu().numpy(), ct)
    assert np.array_equal(side.columns.cpu().numpy(), cols)


def test_filter_indices_from_groupings():
    rng, h, r, t, E, R = _tiny(5, E=30, R=4, M=300)
    frame = pd.DataFrame({0: h, 1: r, 2: t})
    graph, graph_inv = frame.groupby([0, 1]), frame.groupby([2, 1])
    batches = [{"h": int(a), "r": int(b), "t": 0} for a, b in zip(rng.integers(0, E, 50), rng.integers(0, 2 * R, 50))]
    ds = types.SimpleNamespace(relation_size=R)
    got = ev.build_filter_indices_graph(batches, graph, graph_inv, ds, "cuda")
    bids, ents = [], []  # the reference's per-item order: items in batch order
    for j, it in enumerate(batches):
        if it["r"] < R:
            key, col, g = (it["h"], it["r"]), 2, graph
        else:
            key, col, g = (it["h"], it["r"] - R), 0, graph_inv
        if key in g.indices:
            vals = g.get_group(key)[col].values
            bids += [j] * len(vals)
            ents += list(vals)
    _eq(got, (np.array(bids, np.int64), np.array(ents, np.int64)))


def _sparse_state(rng, B, E, density=0.05, dtype=torch.float32):
    dense = torch.from_numpy(np.where(rng.random((B, E)) < density,
                                      rng.choice([0.25, 0.5, 1.0, 2.0], (B, E)), 0.0)).to(dtype)
    return dense, dense.to_sparse().coalesce().cuda()


@pytest.mark.parametrize("use_eql", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_hits_full_sparse(use_eql, dtype):
    rng = np.random.default_rng(7)
    B, E = 64, 500
    dense, state = _sparse_state(rng, B, E, dtype=dtype)
    targets = rng.integers(0, E, B)
    batches = [{"h": 0, "r": 0, "t": int(x)} for x in targets]
    fb = rng.integers(0, B, 300)
    fe = rng.integers(0, E, 300)
    hits = np.zeros(10)
    mrr = ev.calculate_hits_full_sparse(state, batches, (torch.from_numpy(fb).cuda(), torch.from_numpy(fe).cuda()),
                                        hits, use_eql=use_eql)
    keys = np.unique(np.concatenate([fb * E + fe, np.arange(B) * E + targets]))
    ix = state.indices().cpu().numpy()
    ranks = O.filtered_ranks(ix[0], ix[1], state.values().cpu().numpy(), targets, keys, B, E, use_eql)
    want_hits = np.zeros(10)
    for rv in ranks:
        want_hits += (float(rv) <= np.arange(1, 11))
    assert mrr == float((1.0 / ranks).sum())
    assert np.array_equal(hits, want_hits)
    # no filter: only the targets
    hits2 = np.zeros(10)
    mrr2 = ev.calculate_hits_full_sparse(state, batches, None, hits2, use_eql=use_eql)
    ranks2 = O.filtered_ranks(ix[0], ix[1], state.values().cpu().numpy(), targets, np.arange(B) * E + targets, B, E,
                              use_eql)
    assert mrr2 == float((1.0 / ranks2).sum())


@pytest.mark.parametrize("use_eql", [False, True])
def test_hits_full_dense(use_eql):
    rng = np.random.default_rng(8)
    B, E = 48, 700
    state = torch.from_numpy(rng.choice([0.0, 0.1, 0.5, 1.0], (B, E)).astype(np.float32)).cuda()
    targets = rng.integers(0, E, B)
    batches = [{"h": 0, "r": 0, "t": int(x)} for x in targets]
    fb, fe = rng.integers(0, B, 500), rng.integers(0, E, 500)
    hits = np.zeros(10)
    mrr = ev.calculate_hits_full_with_filter_indices(state, batches, (torch.from_numpy(fb).cuda(),
                                                                      torch.from_numpy(fe).cuda()), hits, use_eql)
    ranks = O.dense_filtered_ranks(state.cpu().numpy(), targets, fb, fe, use_eql)
    want_mrr = 0
    want_hits = np.zeros(10)
    for rv in ranks.tolist():
        want_hits += (rv <= np.arange(1, 11))
        want_mrr += 1 / rv
    assert mrr == want_mrr and np.array_equal(hits, want_hits)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_raw_hits_sparse(dtype):
    rng = np.random.default_rng(9)
    B, E = 40, 300
    dense, state = _sparse_state(rng, B, E, density=0.1, dtype=dtype)
    targets = rng.integers(0, E, B)
    batches = [{"h": 0, "r": 0, "t": int(x)} for x in targets]
    hits = np.zeros(10)
    mrr = ev.calculate_raw_hits_sparse(state, batches, hits)
    ix = state.indices().cpu().numpy()
    ranks = O.raw_sparse_ranks(ix[0], ix[1], state.values().cpu().numpy(), B, E, targets)
    want_hits = np.zeros(10)
    want_mrr = 0.0
    for rv in ranks.tolist():
        rv = int(rv)
        want_hits[rv - 1:] += 1
        want_mrr += 1.0 / rv
    assert mrr == want_mrr and np.array_equal(hits, want_hits)
    truth = ev._sparse_truth_scores(state, torch.from_numpy(targets).cuda())
    assert torch.equal(truth.cpu(), dense[np.arange(B), targets])
