"""GPU parity of the fixed-relation rule step and of the rule-bank scores
against the float64 oracle (tests/test_oracle_rules.py pins it)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import small_graph, to_torch_csr

pytestmark = pytest.mark.gpu


def _fk():
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    return fk


def test_fixed_relation_step_exact():
    fk = _fk()
    rng = np.random.default_rng(4)
    h, r, t, E, R, csr = small_graph(3, 0.02)
    B, L = 3, 5
    rows = []
    for b in range(B):
        for l in range(L):
            for e in np.sort(rng.choice(E, 6, replace=False)):
                rows.append((b, l, e, float(rng.integers(1, 4))))
    b, l, e, v = (np.array(x) for x in zip(*rows))
    ops = rng.integers(0, 2 * R + 1, (B, L))
    ops[0, 0] = 2 * R       # identity
    ops[1, 1] = 2 * R + 5   # no such operator: no output
    tc = to_torch_csr(csr, torch.device("cuda"))
    st = torch.sparse_coo_tensor(torch.from_numpy(np.stack([b, l, e])).cuda(),
                                 torch.from_numpy(v.astype(np.float32)).cuda(), (B, L, E)).coalesce()
    out = fk.vectorized_operation_sparse3d_fixed_relation(st, torch.from_numpy(ops).cuda(), tc, R)
    want = O.fixed_relation_step(b, l, e, v, ops, h, r, t, E, R)
    idx = out.indices().cpu().numpy()
    got = {(int(a), int(c), int(d)): float(x) for a, c, d, x in zip(*idx, out.values().cpu().numpy())}
    assert got == want
    assert out.is_coalesced()


@pytest.mark.parametrize("reduction,boolean,final_max", [("sum", False, False), ("sum", True, False),
                                                         ("max", True, False), ("max", True, True)])
@pytest.mark.parametrize("chunk", [1, 7, 64])
def test_rule_scores(reduction, boolean, final_max, chunk):
    from flashlog_amd.rules import shared_inference
    rng = np.random.default_rng(10 + chunk)
    h, r, t, E, R, csr = small_graph(3, 0.02)
    bodies = [list(map(int, rng.integers(0, 2 * R + 1, rng.integers(1, 4)))) for _ in range(40)]
    bodies.append([])  # empty body: the source itself
    W = rng.random((len(bodies), 3)).astype(np.float32)
    rules = [{"body": bd, "rank_weights": list(map(float, w))} for bd, w in zip(bodies, W)]
    sources = rng.integers(0, E, 5)
    tc = to_torch_csr(csr, torch.device("cuda"))
    stats = {}
    out = shared_inference.score(None, torch.from_numpy(sources).cuda(), rules, tc, R, E, chunk,
                                 final_max=final_max, reduction=reduction, boolean_paths=boolean,
                                 dense_budget_bytes=2 * 3 * E * 4, stats=stats)
    want = O.rule_scores(h, r, t, E, R, list(sources), bodies, W.astype(np.float64), reduction, boolean,
                         final_max)
    got = out.to_dense().cpu().numpy()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-7)
    assert stats["chunks"] >= 1 and stats["rules_after"] <= stats["rules_before"]


def test_rule_scores_edges():
    from flashlog_amd.rules import max_inference, shared_inference
    h, r, t, E, R, csr = small_graph(3, 0.02)
    tc = to_torch_csr(csr, torch.device("cuda"))
    src = torch.tensor([1, 2], device="cuda")
    assert shared_inference.score(None, src, [], tc, R, E, 4)._nnz() == 0
    with pytest.raises(ValueError):
        shared_inference.score(None, src, [{"body": [2 * R], "rank_weights": [-1.0]}], tc, R, E, 4)
    with pytest.raises(ValueError):
        shared_inference.score(None, src, [{"body": [0], "rank_weights": [1.0]}], tc, R, E, 4, reduction="mean")
    rules = [{"body": [2 * R], "rank_weights": [0.5]}]
    out = max_inference.score(None, src, rules, tc, R, E, 4)
    assert out.to_dense()[0, 1].item() == 1.0 and out.to_dense()[1, 2].item() == 1.0


@pytest.mark.parametrize("reduction,boolean,final_max", [("sum", False, False), ("sum", True, False),
                                                         ("max", True, False), ("max", True, True)])
def test_rule_bank_c3_full_graph(reduction, boolean, final_max):
    """1000 random rules (bodies of 1-3 operators, uniform rank weights) for
    100 query sources on the full C3 graph (14.5k entities, 237 relations,
    272k triples), chunk 16 as the reference's evaluation uses
    (rules/evaluate.py:890), against the float64 oracle; a second call gives
    the same bits (no atomics in the sums)."""
    from flashlog_amd import synth
    from flashlog_amd.rules import shared_inference
    h, r, t, E, R = synth.make_graph(3)
    csr = O.build_csr_structure(h, t, r, E)
    rng = np.random.default_rng(2024)
    bodies = [list(map(int, rng.integers(0, 2 * R, rng.integers(1, 4)))) for _ in range(1000)]
    W = rng.random((len(bodies), 3)).astype(np.float32)
    rules = [{"body": bd, "rank_weights": list(map(float, w))} for bd, w in zip(bodies, W)]
    # sources drawn from the triples' heads, so most rules ground to something
    sources = h[rng.integers(0, h.shape[0], 100)]
    tc = to_torch_csr(csr, torch.device("cuda"))
    outs = []
    for _ in range(2):
        out = shared_inference.score(None, torch.from_numpy(sources).cuda(), rules, tc, R, E, 16,
                                     final_max=final_max, reduction=reduction, boolean_paths=boolean)
        outs.append(out.coalesce())
    assert torch.equal(outs[0].indices(), outs[1].indices()) and torch.equal(outs[0].values(), outs[1].values())
    want = O.rule_scores(h, r, t, E, R, list(sources), bodies, W.astype(np.float64), reduction, boolean, final_max)
    got = outs[0].to_dense().cpu().numpy()
    assert (want > 0).sum() > 10000
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-9)


@pytest.mark.parametrize("reduction,final_max,sample", [("sum", False, None), ("max", True, 60)])
def test_rule_bank_c3_scale(reduction, final_max, sample):
    """C3's rule-bank scale: 5000 random rules (bodies of 1-3 operators, 3
    uniform rank weights) for 500 query sources on the full C3 graph, chunk
    16 (rules/evaluate.py:890), one call of shared_inference.score.  The sum
    is checked on every source against the float64 oracle; the Boolean max
    with final_max on a sample of 60 sources (each source's scores depend
    only on its own paths, so the oracle runs on the sample)."""
    from flashlog_amd import synth
    from flashlog_amd.rules import shared_inference
    h, r, t, E, R = synth.make_graph(3)
    csr = O.build_csr_structure(h, t, r, E)
    rng = np.random.default_rng(77)
    bodies = [list(map(int, rng.integers(0, 2 * R, rng.integers(1, 4)))) for _ in range(5000)]
    W = rng.random((len(bodies), 3)).astype(np.float32)
    rules = [{"body": bd, "rank_weights": list(map(float, w))} for bd, w in zip(bodies, W)]
    sources = h[rng.integers(0, h.shape[0], 500)]
    tc = to_torch_csr(csr, torch.device("cuda"))
    out = shared_inference.score(None, torch.from_numpy(sources).cuda(), rules, tc, R, E, 16,
                                 final_max=final_max, reduction=reduction).coalesce()
    got = out.to_dense().cpu().numpy()
    rows = np.arange(len(sources)) if sample is None else np.sort(rng.choice(len(sources), sample, replace=False))
    want = O.rule_scores(h, r, t, E, R, list(sources[rows]), bodies, W.astype(np.float64), reduction, False,
                         final_max)
    assert (want > 0).sum() > 100000
    np.testing.assert_allclose(got[rows], want, rtol=1e-5, atol=1e-9)
