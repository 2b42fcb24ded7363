"""GPU parity of the rule-bank evaluation module (flashlog_amd.rules.evaluate,
the reference's rules/evaluate.py:94-119,188-734,746-854): the ev
primitives bit for bit against the torch steps the reference performs
(coalesce, scatter_reduce amax) on the same grounded states, the
normalizers within 1e-6 of the float64 closed form, score_rule_batch's six
aggregations within 1e-5 of the float64 oracle (and bit-identical on a
second call), the filter keys and the metrics."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bits, small_graph, to_torch_csr

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def graph():
    h, r, t, E, R, csr = small_graph(3, 0.05)
    return h, r, t, E, R, to_torch_csr(csr, torch.device("cuda"))


def _rules(rng, R, n, ranks=3, groups=4):
    out = []
    for i in range(n):
        body = tuple(int(x) for x in rng.integers(0, 2 * R, rng.integers(1, 4)))
        out.append({"rule_id": i, "head": 0, "body": body,
                    "weight": float(rng.choice([0.0, 0.125, 0.5, 1.0, 2.0])),
                    "rank_weights": tuple(float(x) for x in rng.choice([0.0, 0.25, 0.5, 0.75], ranks)),
                    "group_id": int(rng.integers(0, groups))})
    return out


def _sources(h, rng, n):
    return torch.from_numpy(h[rng.integers(0, h.shape[0], n)]).cuda()


def _state(graph, rng, nb=8, nr=40):
    from flashlog_amd.rules import evaluate as ev
    h, r, t, E, R, tc = graph
    rules = _rules(rng, R, nr)
    src = _sources(h, rng, nb)
    return ev._ground_shared_rules(src, rules, tc, R, E), rules, src


def _coalesced(idx, vals, shape):
    return torch.sparse_coo_tensor(idx, vals, shape).coalesce()


def _same(a, b):
    a, b = a.coalesce(), b.coalesce()
    assert tuple(a.shape) == tuple(b.shape)
    assert torch.equal(a.indices(), b.indices())
    assert np.array_equal(bits(a.values().cpu().numpy()), bits(b.values().cpu().numpy()))


def test_grounding_matches_path_counts(graph):
    h, r, t, E, R, tc = graph
    rng = np.random.default_rng(1)
    state, rules, src = _state(graph, rng)
    counts = O.rule_path_counts(h, r, t, E, R, src.cpu().tolist(), [list(x["body"]) for x in rules])
    dense = state.to_dense().cpu().numpy()
    for l, x in enumerate(counts):
        want = np.zeros((src.numel(), E))
        np.add.at(want, (x.col, x.row), x.data)
        assert np.array_equal(dense[:, l, :], want), l
    assert state._nnz() > 30


@pytest.mark.parametrize("boolean", [False, True])
def test_reductions_match_torch_steps(graph, boolean):
    from flashlog_amd.rules import evaluate as ev
    rng = np.random.default_rng(2 + boolean)
    state, rules, _ = _state(graph, rng)
    B, C, E = state.shape
    b, l, e = state.indices()
    v = state.values()
    vb = (v > 0).float() if boolean else v
    w = torch.tensor([x["weight"] for x in rules], device="cuda")
    _same(ev.reduce_rule_state(state, w, boolean=boolean), _coalesced(torch.stack((b, e)), vb * w[l], (B, E)))
    rw = torch.tensor([x["rank_weights"] for x in rules], device="cuda")
    K = rw.shape[1]
    ov = (vb.unsqueeze(1) * rw[l]).reshape(-1)
    oi = torch.stack((b.repeat_interleave(K), torch.arange(K, device="cuda").repeat(b.numel()),
                      e.repeat_interleave(K)))
    pos = ov > 0
    _same(ev.reduce_rule_state_by_rank(state, rw, boolean=boolean), _coalesced(oi[:, pos], ov[pos], (B, K, E)))
    if not boolean:
        g = torch.tensor([x["group_id"] for x in rules], device="cuda")
        gv = v * w[l]
        pos = gv > 0
        _same(ev.reduce_rule_state_by_group(state, w, g, 4),
              _coalesced(torch.stack((b, g[l], e))[:, pos], gv[pos], (B, 4, E)))
        mv = (v > 0).float() * w[l]
        keys = b * E + e
        uk, inv = torch.unique(keys, sorted=True, return_inverse=True)
        amax = torch.full((uk.numel(),), -torch.inf, device="cuda").scatter_reduce_(0, inv, mv, reduce="amax",
                                                                                       include_self=True)
        got = ev.max_reduce_rule_state(state, w)
        assert torch.equal(got.indices(), torch.stack((uk // E, uk % E)))
        assert torch.equal(got.values(), amax)


def test_merges_and_normalizers(graph):
    from flashlog_amd.rules import evaluate as ev
    rng = np.random.default_rng(7)
    s1, rules, _ = _state(graph, rng, nb=3)
    s2, _, _ = _state(graph, np.random.default_rng(8), nb=3)
    w = torch.rand(len(rules), device="cuda") + 0.1
    a = ev.reduce_rule_state(s1, w)
    c = ev.reduce_rule_state(s2, w)
    _same(ev.add_sparse(a, c), _coalesced(torch.cat((a.indices(), c.indices()), 1),
                                         torch.cat((a.values(), c.values())), a.shape))
    assert ev.add_sparse(None, c) is c
    mx = ev.max_sparse(a, c).to_dense()
    assert torch.equal(mx, torch.maximum(a.to_dense(), c.to_dense()))
    # packed [B, K, E] operands merge per (b, k) row
    rw = torch.rand(len(rules), 2, device="cuda")
    p1, p2 = ev.reduce_rule_state_by_rank(s1, rw), ev.reduce_rule_state_by_rank(s2, rw)
    _same(ev.add_sparse(p1, p2), _coalesced(torch.cat((p1.indices(), p2.indices()), 1),
                                           torch.cat((p1.values(), p2.values())), p1.shape))
    # normalizers against float64
    n = ev.normalize_sparse_rows(a)
    d = a.to_dense().double()
    want = d / d.sum(1, keepdim=True).clamp_min(1e-30)
    np.testing.assert_allclose(n.to_dense().cpu().numpy(), want.cpu().numpy(), rtol=1e-6, atol=1e-12)
    ns = ev.normalize_and_sum_rank_scores(p1)
    d = p1.to_dense().double()
    want = (d / d.sum(2, keepdim=True).clamp_min(1e-30)).sum(1)
    np.testing.assert_allclose(ns.to_dense().cpu().numpy(), want.cpu().numpy(), rtol=1e-6, atol=1e-12)


def test_memory_bounded_advance_equals_the_step(graph):
    from flashlog_amd.rules import evaluate as ev
    h, r, t, E, R, tc = graph
    rng = np.random.default_rng(11)
    src = _sources(h, rng, 1)
    st = ev.vectorized_operation_sparse3d_fixed_relation(ev.initial_rule_state(src, 1, E),
                                                          torch.tensor([[3]], device="cuda"), tc, R)
    ops = torch.tensor([[R + 5]], device="cuda")
    whole = ev.vectorized_operation_sparse3d_fixed_relation(st, ops, tc, R)
    for chunk in (1, 2, 64):
        _same(ev.advance_single_rule_state_memory_bounded(st, ops, tc, R, input_chunk_size=chunk), whole)


AGGS = ("weighted_path_count", "weighted_boolean", "max_confidence", "rank_normalized", "rank_boolean_normalized",
        "routed_normalized")


@pytest.mark.parametrize("chunk", [1, 7, 32])
def test_score_rule_batch_all_aggregations(graph, chunk):
    from flashlog_amd.rules import evaluate as ev
    h, r, t, E, R, tc = graph
    rng = np.random.default_rng(100 + chunk)
    rules = _rules(rng, R, 60)
    src = _sources(h, rng, 6)
    outs = [ev.score_rule_batch(src, rules, tc, R, E, chunk, AGGS) for _ in range(2)]
    for name in AGGS:
        _same(outs[0][name], outs[1][name])
        want, reached = O.rule_batch_scores(h, r, t, E, R, src.cpu().tolist(), rules, name)
        got = outs[0][name]
        gi = got.indices().cpu().numpy()
        present = np.zeros_like(reached)
        present[gi[0], gi[1]] = True
        assert np.array_equal(present, reached), name
        np.testing.assert_allclose(got.to_dense().cpu().numpy(), want, rtol=1e-5, atol=1e-7, err_msg=name)


def test_score_rule_batch_routed_only_and_streamed(graph, monkeypatch):
    from flashlog_amd.rules import evaluate as ev
    h, r, t, E, R, tc = graph
    rng = np.random.default_rng(5)
    rules = _rules(rng, R, 40)
    src = _sources(h, rng, 4)
    # routed_normalized alone: compaction by (head, body), then rank_normalized over the groups
    got = ev.score_rule_batch(src, rules, tc, R, E, 8, ("routed_normalized",))["routed_normalized"]
    want, _ = O.rule_batch_scores(h, r, t, E, R, src.cpu().tolist(), rules, "routed_normalized")
    np.testing.assert_allclose(got.to_dense().cpu().numpy(), want, rtol=1e-5, atol=1e-7)
    # more rules than the streaming threshold: the rank modes go through shared_inference.score
    monkeypatch.setattr(ev, "RANK_STREAMING_RULE_THRESHOLD", 10)
    ev._SERIAL_RANK_HEADS.clear()
    out = ev.score_rule_batch(src, rules, tc, R, E, 8, ("rank_normalized", "weighted_path_count"))
    for name in ("rank_normalized", "weighted_path_count"):
        want, _ = O.rule_batch_scores(h, r, t, E, R, src.cpu().tolist(), rules, name)
        np.testing.assert_allclose(out[name].to_dense().cpu().numpy(), want, rtol=1e-5, atol=1e-7, err_msg=name)
    empty = ev.score_rule_batch(src, [], tc, R, E, 8, AGGS)
    assert all(v._nnz() == 0 and tuple(v.shape) == (4, E) for v in empty.values())


def test_filter_keys_and_metrics(graph):
    from flashlog_amd.rules import evaluate as ev
    h, r, t, E, R, tc = graph
    rng = np.random.default_rng(9)
    idx = rng.integers(0, h.shape[0], 6)
    batch = [(int(h[i]), int(r[i]), int(t[i])) for i in idx[:3]] + \
            [(int(t[i]), int(r[i]) + R, int(h[i])) for i in idx[3:]]
    known = ev.build_split_known([(int(h[0]), int(r[0]), 7)], [], R)
    src = torch.tensor([q[0] for q in batch], device="cuda")
    keys = ev.filter_keys_for_batch_flashlog(tc, batch, src, known, R, E).cpu().numpy()
    want = set()
    for b, (s, rel, tg) in enumerate(batch):
        if rel < R:
            ends = t[(h == s) & (r == rel)]
        else:
            ends = h[(t == s) & (r == rel - R)]
        want.update(b * E + int(x) for x in ends)
        want.update(b * E + x for x in known.get((s, rel), ()))
        want.add(b * E + tg)
    assert keys.tolist() == sorted(want)
    # metrics: ranks of the rule scores through the rank kernel, against the oracle
    rules = _rules(rng, R, 30)
    scores = ev.score_rule_batch(src, rules, tc, R, E, 8, ("rank_normalized",))["rank_normalized"]
    targets = torch.tensor([q[2] for q in batch], device="cuda")
    acc = {"ranks": [], "covered_targets": 0}
    ev.update_metrics(acc, scores, targets, torch.from_numpy(keys).cuda())
    si = scores.indices().cpu().numpy()
    want_r = O.filtered_ranks(si[0], si[1], scores.values().cpu().numpy(), targets.cpu().numpy(), keys, len(batch), E,
                              True)
    assert acc["ranks"] == want_r.astype(np.float64).tolist()
    dense = scores.to_dense().cpu().numpy()
    assert acc["covered_targets"] == int(sum(dense[b, q[2]] != 0 for b, q in enumerate(batch)))
    row = ev.select_sparse_score_row(scores, 2)
    assert np.array_equal(row.to_dense().cpu().numpy()[0], dense[2])
