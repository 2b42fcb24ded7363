"""Pin of the dense filtered-rank oracle (src/main.py:468-512) by a direct
loop over each query's entities: greater / equal counted over the entities
outside the filter (the filter plus the target; none without a filter)."""
import numpy as np
import pytest

from oracle import oracle as O


def _brute(state, targets, fb, fe, use_eql):
    B, E = state.shape
    out = []
    for b in range(B):
        truth = state[b, targets[b]]
        filt = set() if fb is None else {int(e) for bb, e in zip(fb, fe) if bb == b} | {int(targets[b])}
        greater = sum(1 for e in range(E) if e not in filt and state[b, e] > truth)
        equal = sum(1 for e in range(E) if e not in filt and state[b, e] == truth)
        out.append(greater + (equal + 2) / 2 if use_eql else greater + 1)
    return np.array(out, np.float64)


@pytest.mark.parametrize("use_eql", [False, True])
@pytest.mark.parametrize("filtered", [False, True])
@pytest.mark.parametrize("seed", range(4))
def test_dense_ranks_oracle_brute_force(use_eql, filtered, seed):
    rng = np.random.default_rng(seed)
    B, E = 7, 60
    state = (rng.integers(0, 6, (B, E)) / 4.0).astype(np.float32)  # many ties
    targets = rng.integers(0, E, B)
    fb = fe = None
    if filtered:
        n = 40
        fb = rng.integers(0, B, n)
        fe = rng.integers(0, E, n)  # duplicates and targets among them
    got = O.dense_filtered_ranks(state, targets, fb, fe, use_eql)
    np.testing.assert_array_equal(got.astype(np.float64), _brute(state, targets, fb, fe, use_eql))


def test_dense_ranks_distinct_scores_are_positions():
    rng = np.random.default_rng(9)
    state = rng.permutation(500).reshape(5, 100).astype(np.float32)
    targets = rng.integers(0, 100, 5)
    r = O.dense_filtered_ranks(state, targets)
    for b in range(5):
        order = np.argsort(-state[b], kind="stable")
        assert r[b] == 1 + int(np.nonzero(order == targets[b])[0][0])
