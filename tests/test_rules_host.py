"""Host-side logic of the rule scorers on the CPU: the out-of-memory
ladders of shared_inference.score and score_rule_batch, forced from the host
with a stand-in ``ev`` module whose grounding raises
torch.cuda.OutOfMemoryError for large chunks (the accumulation is replaced
by a recorder, so no device call is made), the routed-rule compaction and
the metric helpers."""
import types

import numpy as np
import pytest
import torch

from flashlog_amd.rules import evaluate as ev_mod
from flashlog_amd.rules import shared_inference as si

R, E = 3, 12


def _csr():
    """A tiny CSR 16-tuple (CPU) whose first hops from every source exist."""
    from oracle import oracle as O
    rng = np.random.default_rng(0)
    h = np.repeat(np.arange(E), R)  # every entity has an edge of every relation
    t = rng.integers(0, E, h.size)
    r = np.tile(np.arange(R), E)
    return tuple(torch.from_numpy(np.ascontiguousarray(a)) for a in O.build_csr_structure(h, t, r, E))


def _rules(n):
    return [{"body": (i % R,), "rank_weights": (0.5, 0.25)} for i in range(n)]


def _fake_ev(max_rules, calls):
    def initial_rule_state(sources, num_rules, num_entities):
        return ev_mod.initial_rule_state(sources, num_rules, num_entities)

    def step(state, ops, csr, relations):
        calls.append(("step", state.shape[0], state.shape[1]))
        if state.shape[1] > max_rules:
            raise torch.cuda.OutOfMemoryError("forced")
        return state  # the identity suffices for the control flow

    def bounded(state, ops, csr, relations):
        calls.append(("bounded", state.shape[0], state.shape[1]))
        return state

    return types.SimpleNamespace(initial_rule_state=initial_rule_state,
                                 vectorized_operation_sparse3d_fixed_relation=step,
                                 advance_single_rule_state_memory_bounded=bounded)


@pytest.fixture
def recorder(monkeypatch):
    seen = []
    monkeypatch.setattr(si, "_accumulate_chunk", lambda state, W, dense, is_max, nb, E_: seen.append(W.shape[0]))
    monkeypatch.setattr(si, "_finalize", lambda dense, nb, E_, fm: (torch.zeros(0, dtype=torch.long),
                                                                     torch.zeros(0)))
    return seen


def test_chunk_halving_ladder(recorder):
    """8-rule chunks run out of memory, 4-rule ones too, 2-rule ones fit: two
    retries, then every rule is accumulated in 2-rule chunks."""
    calls = []
    stats = {}
    si.score(_fake_ev(2, calls), torch.tensor([1, 4]), _rules(8), _csr(), R, E, 8, stats=stats)
    assert stats["oom_retries"] == 2 and stats["rules_after"] == 8
    assert recorder == [2, 2, 2, 2]
    assert stats["chunks"] == 4
    assert [c[2] for c in calls if c[0] == "step"][:2] == [8, 4]


def test_ladder_gives_up_at_one_rule(recorder):
    calls = []
    with pytest.raises(torch.cuda.OutOfMemoryError, match="smaller query batch"):
        si.score(_fake_ev(0, calls), torch.tensor([1, 4]), _rules(3), _csr(), R, E, 4)


def test_single_source_single_rule_takes_the_bounded_advance(recorder):
    calls = []
    stats = {}
    si.score(_fake_ev(0, calls), torch.tensor([2]), _rules(2), _csr(), R, E, 1, stats=stats)
    assert ("bounded", 1, 1) in calls
    assert stats["oom_retries"] == 0 and recorder == [1, 1]


def test_score_rule_batch_streaming_falls_back_to_serial(monkeypatch):
    """More rules than the streaming threshold: the shared scorer's
    out-of-memory error sends the head to the rank-serial scorer, which is
    then remembered for it."""
    seen = []

    def shared(*a, **k):
        seen.append("shared")
        raise torch.cuda.OutOfMemoryError("forced")

    def serial(sources, rules, csr, nr, ne, chunk, modes):
        seen.append("serial")
        return {name: ev_mod._empty((sources.numel(), ne), sources.device) for name in modes}

    monkeypatch.setattr(ev_mod, "_score_rank_batch_shared", shared)
    monkeypatch.setattr(ev_mod, "_score_rank_batch_serial", serial)
    monkeypatch.setattr(ev_mod, "RANK_STREAMING_RULE_THRESHOLD", 2)
    ev_mod._SERIAL_RANK_HEADS.clear()
    rules = [{"head": 7, "body": (0,), "weight": 1.0, "rank_weights": (1.0,), "group_id": 0} for _ in range(3)]
    csr = _csr()
    for _ in range(2):
        out = ev_mod.score_rule_batch(torch.tensor([1]), rules, csr, R, E, 2, ("rank_normalized",))
        assert out["rank_normalized"]._nnz() == 0
    assert seen == ["shared", "serial", "serial"]


def test_ground_shared_rules_bounded_fallback(monkeypatch):
    calls = []
    fake = _fake_ev(0, calls)
    monkeypatch.setattr(ev_mod, "vectorized_operation_sparse3d_fixed_relation",
                        fake.vectorized_operation_sparse3d_fixed_relation)
    monkeypatch.setattr(ev_mod, "advance_single_rule_state_memory_bounded",
                        fake.advance_single_rule_state_memory_bounded)
    ev_mod._ground_shared_rules(torch.tensor([3]), [{"body": (1, 2)}], _csr(), R, E)
    assert [c[0] for c in calls] == ["step", "bounded", "step", "bounded"]
    with pytest.raises(torch.cuda.OutOfMemoryError):
        ev_mod._ground_shared_rules(torch.tensor([3, 4]), [{"body": (1,)}], _csr(), R, E)


def test_compact_routed_rules():
    rules = [{"head": 1, "body": (0, 2), "weight": 0.5, "group_id": 1, "rule_id": 0, "rank_weights": None},
             {"head": 1, "body": (0, 2), "weight": 0.25, "group_id": 0, "rule_id": 1, "rank_weights": None},
             {"head": 1, "body": (3,), "weight": 2.0, "group_id": 2, "rule_id": 2, "rank_weights": None}]
    out = ev_mod.compact_routed_rules(rules)
    assert [(r["body"], r["rank_weights"], r["weight"], r["group_id"], r["rule_id"]) for r in out] == \
        [((0, 2), (0.25, 0.5, 0.0), 1.0, None, 0), ((3,), (0.0, 0.0, 2.0), 1.0, None, 2)]
    with pytest.raises(ValueError, match="duplicate"):
        ev_mod.compact_routed_rules(rules + [dict(rules[0])])
    with pytest.raises(ValueError, match="group_id"):
        ev_mod.compact_routed_rules([{**rules[0], "group_id": None}])


def test_metrics_and_evaluation_inputs():
    m = ev_mod.finalize_metrics({"ranks": [1.0, 2.0, 4.0, 11.0], "covered_targets": 3})
    assert m["count"] == 4 and m["hit_1"] == 0.25 and m["hit_3"] == 0.5 and m["hit_10"] == 0.75
    assert abs(m["mrr"] - np.mean([1, 0.5, 0.25, 1 / 11])) < 1e-15 and m["target_coverage"] == 0.75
    assert ev_mod.finalize_metrics({"ranks": [], "covered_targets": 0})["count"] == 0
    assert ev_mod.build_evaluation([(1, 0, 2), (3, 1, 4)], 5) == [(1, 0, 2), (2, 5, 1), (3, 1, 4), (4, 6, 3)]
    known = ev_mod.build_split_known([(1, 0, 2)], [(1, 0, 3)], 5)
    assert known[(1, 0)] == {2, 3} and known[(2, 5)] == {1} and known[(3, 5)] == {1}


def test_load_rules_and_compact_csr_cache(tmp_path):
    p = tmp_path / "rules.tsv"
    p.write_text("head_id\tbody_ids\tweight\trank_weights\tgroup_id\n3\t1 4\t0.5\t0.1 0.2\t0\n3\t\t1.25\t\t\n")
    rules = ev_mod.load_rules(str(p))
    assert rules[0] == {"rule_id": 0, "head": 3, "body": (1, 4), "weight": 0.5, "rank_weights": (0.1, 0.2),
                        "group_id": 0}
    assert rules[1]["body"] == () and rules[1]["rank_weights"] is None and rules[1]["group_id"] is None
    with pytest.raises(ValueError, match="weight field"):
        ev_mod.load_rules(str(p), weight_field="confidence")
    # the CSR cache format: {"num_entities", "csr"}, read with weights_only=True
    csr = _csr()
    cache = tmp_path / "csr.pt"
    torch.save({"num_entities": E, "csr": csr}, cache)
    got = ev_mod.build_compact_rule_csr(None, E, torch.device("cpu"), str(cache))
    for i, (a, b) in enumerate(zip(got, csr)):
        assert torch.equal(a, b) if i in ev_mod.CSR_RULE_FIELDS else a.numel() == 0
    with pytest.raises(ValueError, match="entity count"):
        ev_mod.build_compact_rule_csr(None, E + 1, torch.device("cpu"), str(cache))


def test_foreign_evaluation_module_grounds_on_this_build():
    """score()'s ev: a module other than this package's evaluation module
    (e.g. the reference's rules.evaluate passed without install()) is
    replaced by this package's; None likewise; a caller's own hook object
    (not a module) is used as given."""
    foreign = types.ModuleType("rules.evaluate")
    foreign.vectorized_operation_sparse3d_fixed_relation = lambda *a: pytest.fail("foreign grounding called")
    assert si._grounding_hooks(foreign) is ev_mod
    assert si._grounding_hooks(None) is ev_mod
    assert si._grounding_hooks(ev_mod) is ev_mod
    own = types.SimpleNamespace()
    assert si._grounding_hooks(own) is own


def test_foreign_module_score_uses_this_builds_hooks(monkeypatch, recorder):
    """Through score(): the grounding calls reach this package's hooks, not
    the foreign module's."""
    calls = []
    monkeypatch.setattr(ev_mod, "vectorized_operation_sparse3d_fixed_relation",
                        lambda state, ops, csr, rel: calls.append(state.shape) or state)
    foreign = types.ModuleType("rules.evaluate")
    foreign.initial_rule_state = lambda *a: pytest.fail("foreign initial state called")
    foreign.vectorized_operation_sparse3d_fixed_relation = lambda *a: pytest.fail("foreign grounding called")
    si.score(foreign, torch.tensor([1, 4]), _rules(4), _csr(), R, E, 4)
    assert calls and recorder == [4]
