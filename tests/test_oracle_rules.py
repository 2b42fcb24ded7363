"""Pins of the rule-scoring oracle: matrix path counts against explicit path
enumeration, and the score combination against a direct loop."""
import numpy as np

from oracle import oracle as O


def _tiny(seed):
    rng = np.random.default_rng(seed)
    E, R, M = 12, 3, 40
    return rng, E, R, rng.integers(0, E, M), rng.integers(0, R, M), rng.integers(0, E, M)


def test_path_counts_match_enumeration():
    rng, E, R, h, r, t = _tiny(0)
    for _ in range(30):
        body = list(rng.integers(0, 2 * R + 1, rng.integers(0, 4)))
        s = int(rng.integers(0, E))
        x = O.rule_scores(h, r, t, E, R, [s], [body], np.ones((1, 1)), "sum", False, False)
        brute = O.rule_paths_brute(h, r, t, R, s, body)
        tot = sum(brute.values())
        want = np.zeros(E)
        for k, c in brute.items():
            want[k] = c / tot if tot else 0.0
        np.testing.assert_allclose(x[0], want, rtol=1e-12, atol=1e-15)


def test_fixed_step_matches_paths():
    rng, E, R, h, r, t = _tiny(1)
    ops = rng.integers(0, 2 * R + 1, (2, 3))
    b = np.array([0, 0, 1, 1, 1]); l = np.array([0, 2, 0, 1, 2]); e = rng.integers(0, E, 5)
    v = np.array([1.0, 2.0, 1.0, 3.0, 1.0])
    out = O.fixed_relation_step(b, l, e, v, ops, h, r, t, E, R)
    for (bi, li, d), val in out.items():
        want = 0.0
        for j in range(5):
            if b[j] == bi and l[j] == li:
                want += v[j] * O.rule_paths_brute(h, r, t, R, int(e[j]), [int(ops[bi][li])]).get(d, 0)
        assert val == want


def test_score_modes_direct_loop():
    rng, E, R, h, r, t = _tiny(2)
    bodies = [list(rng.integers(0, 2 * R + 1, rng.integers(1, 4))) for _ in range(7)]
    W = rng.random((7, 3))
    sources = [1, 5]
    for reduction, boolean, fmax in [("sum", False, False), ("sum", True, False), ("max", True, True)]:
        got = O.rule_scores(h, r, t, E, R, sources, bodies, W, reduction, boolean, fmax)
        want = np.zeros((2, E))
        for bi, s in enumerate(sources):
            per_rank = []
            for k in range(3):
                row = np.zeros(E)
                for ri, body in enumerate(bodies):
                    c = O.rule_paths_brute(h, r, t, R, s, body)
                    for node, cnt in c.items():
                        val = (1.0 if cnt > 0 else 0.0) if boolean else float(cnt)
                        if reduction == "max":
                            row[node] = max(row[node], W[ri, k] * val)
                        else:
                            row[node] += W[ri, k] * val
                per_rank.append(row / max(row.sum(), 1e-30))
            want[bi] = np.max(per_rank, 0) if fmax else np.sum(per_rank, 0)
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-15)


def test_rule_batch_scores_direct_loop():
    """The DRUM scorer's aggregations against explicit path enumeration."""
    rng, E, R, h, r, t = _tiny(3)
    rules = []
    for i in range(9):
        body = tuple(int(x) for x in rng.integers(0, 2 * R + 1, rng.integers(1, 4)))
        rules.append({"body": body, "weight": float(rng.choice([0.0, 0.25, 0.5, 1.5])),
                      "rank_weights": tuple(float(x) for x in rng.choice([0.0, 0.3, 0.7], 3)),
                      "group_id": int(rng.integers(0, 3))})
    sources = [1, 5, 7]
    for agg in ("weighted_path_count", "weighted_boolean", "max_confidence", "rank_normalized",
                "rank_boolean_normalized", "routed_normalized"):
        got, reached = O.rule_batch_scores(h, r, t, E, R, sources, rules, agg)
        boolean = agg in ("weighted_boolean", "rank_boolean_normalized", "max_confidence")
        want = np.zeros((len(sources), E))
        want_reached = np.zeros((len(sources), E), bool)
        for bi, s in enumerate(sources):
            paths = [O.rule_paths_brute(h, r, t, R, s, list(rule["body"])) for rule in rules]
            for c in paths:
                for node, cnt in c.items():
                    if cnt > 0:
                        want_reached[bi, node] = True
            if agg in ("weighted_path_count", "weighted_boolean", "max_confidence"):
                best = {}
                for rule, c in zip(rules, paths):
                    for node, cnt in c.items():
                        if cnt <= 0:
                            continue
                        val = rule["weight"] * (1.0 if boolean else cnt)
                        best[node] = max(best.get(node, -np.inf), val) if agg == "max_confidence" \
                            else best.get(node, 0.0) + val
                for node, val in best.items():
                    want[bi, node] = val
            else:
                for k in range(3):  # 3 ranks, or the 3 routed groups
                    row = np.zeros(E)
                    for rule, c in zip(rules, paths):
                        if agg == "routed_normalized":
                            wk = max(rule["weight"], 0.0) if rule["group_id"] == k else 0.0
                        else:
                            wk = max(rule["rank_weights"][k], 0.0)
                        for node, cnt in c.items():
                            if cnt > 0:
                                row[node] += wk * (1.0 if boolean else cnt)
                    want[bi] += row / max(row.sum(), 1e-30)
        np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-15, err_msg=agg)
        if agg in ("weighted_path_count", "weighted_boolean", "max_confidence"):
            assert np.array_equal(reached, want_reached), agg
