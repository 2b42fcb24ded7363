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
