"""Pins of the extraction oracle (rules/extract.py:65-201): rank weights
against an enumeration of the identity placements (closed form and the
dynamic program with sums; maxima exactly), the two evaluations against
each other, and the selection order against Python's sort."""
import numpy as np
import pytest

from oracle import oracle as O


def _case(seed, T, L=3, R=5, N=60, dtype=np.float32):
    rng = np.random.default_rng(seed)
    n = 2 * R + 1
    att = rng.random((T, L, n)).astype(dtype)
    att /= att.sum(axis=2, keepdims=True)
    rows = np.zeros((N, 1 + T + 8), np.int64)
    rows[:, 0] = rng.integers(0, T + 2, N)  # includes empty and too-long bodies
    rows[:, 1:1 + T] = rng.integers(0, n - 1, (N, T))
    rows[:, 1 + T:] = rng.integers(0, 6, (N, 8))
    return rng, att, rows, n - 1


@pytest.mark.parametrize("seed", range(3))
def test_closed_form_matches_enumeration(seed):
    _, att, rows, ident = _case(seed, 3)
    got = O.rank_weights_closed_form(att, rows, ident)
    np.testing.assert_allclose(got, O.rank_weights_brute(att, rows, ident), rtol=1e-13, atol=0)
    np.testing.assert_allclose(got, O.rank_weights_dp(att, rows, ident), rtol=1e-13, atol=0)
    assert np.all(got[(rows[:, 0] == 0) | (rows[:, 0] > 3)] == 0)


@pytest.mark.parametrize("T", [1, 2, 3, 4, 5])
def test_dp_matches_enumeration(T):
    _, att, rows, ident = _case(T, T, dtype=np.float64)
    np.testing.assert_allclose(O.rank_weights_dp(att, rows, ident), O.rank_weights_brute(att, rows, ident),
                               rtol=1e-13, atol=0)
    # maxima: monotone rounding makes the dynamic program exact
    assert np.array_equal(O.rank_weights_dp(att, rows, ident, maximum=True),
                          O.rank_weights_brute(att, rows, ident, maximum=True))


def test_select_order_and_fallback():
    rng, att, rows, ident = _case(7, 3, N=200)
    rows[:, -5] = rng.integers(0, 3, rows.shape[0])  # many ties on the first key
    sel, prec, rw, used = O.select_and_annotate(rows, att, ident, 2)
    keep = rows[rows[:, -6] >= 2]
    assert not used and sel.shape == keep.shape
    order = O.select_order_brute(sel, rw, 3)
    assert order == list(range(len(order)))
    trials, pos = sel[:, -8], sel[:, -6]
    assert np.array_equal(prec, np.where(trials != 0, pos / np.where(trials == 0, 1, trials), 0.0))
    # no candidate reaches the minimum: the single best by (weight sum, body)
    sel, prec, rw, used = O.select_and_annotate(rows, att, ident, 100)
    allw = O.rank_weights_closed_form(att, rows, ident)
    best = max(range(rows.shape[0]), key=lambda j: (allw[j].sum(), tuple(rows[j, 1:1 + rows[j, 0]])))
    assert used and sel.shape[0] == 1 and np.array_equal(sel[0], rows[best])
    assert O.select_and_annotate(rows[:0], att, ident, 1)[0].shape == (0, rows.shape[1])
