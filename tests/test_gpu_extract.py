"""Extraction post-processing on the GPU (rules/extract.py:65-299): rank
weights bit for bit against the oracle's numpy evaluation (closed form,
dynamic program with sums and maxima, float32 and float64 attention), the
selection and order, the fallback, the batched entry point and the TSV
lines."""
import numpy as np
import pytest

from flashlog_amd.rules import extract as X
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _case(seed, T, L=3, R=40, N=5000, dtype=np.float32):
    rng = np.random.default_rng(seed)
    n = 2 * R + 1
    att = rng.random((T, L, n)).astype(dtype) ** 3
    att /= att.sum(axis=2, keepdims=True)
    rows = np.zeros((N, 1 + T + 8), np.int64)
    rows[:, 0] = rng.integers(0, T + 2, N)
    rows[:, 1:1 + T] = rng.integers(0, n - 1, (N, T))
    rows[:, 1 + T:] = rng.integers(0, 9, (N, 8))
    return rng, att, rows, n - 1


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_rank_weights_bit_exact(dtype):
    _, att, rows, ident = _case(0, 3, dtype=dtype)
    assert np.array_equal(X._three_step_weights(att, rows, ident), O.rank_weights_closed_form(att, rows, ident))
    assert np.array_equal(X.attention_rank_weights(att, rows, ident), O.rank_weights_closed_form(att, rows, ident))
    for maximum in (False, True):
        assert np.array_equal(X.collapsed_rule_weights(att, rows, ident, maximum),
                              O.rank_weights_dp(att, rows, ident, maximum))


@pytest.mark.parametrize("T", [1, 2, 4, 6])
def test_rank_weights_other_depths(T):
    _, att, rows, ident = _case(T, T, L=5)
    assert np.array_equal(X.attention_rank_weights(att, rows, ident), O.rank_weights_dp(att, rows, ident))
    assert np.array_equal(X.collapsed_rule_weights(att, rows, ident, True), O.rank_weights_dp(att, rows, ident, True))


def test_operator_indexing():
    _, att, rows, ident = _case(3, 3, N=50)
    rows[:5, 0] = 1
    rows[:5, 1] = -1  # numpy reads negative operators from the end
    assert np.array_equal(X._three_step_weights(att, rows, ident), O.rank_weights_closed_form(att, rows, ident))
    assert np.array_equal(X._three_step_weights(att, rows, -1), O.rank_weights_closed_form(att, rows, -1))
    rows[7, 0], rows[7, 2] = 2, att.shape[2]
    with pytest.raises(IndexError):
        X._three_step_weights(att, rows, ident)


@pytest.mark.parametrize("L", [3, 9, 20])
def test_fallback_scores(L, monkeypatch):
    rng = np.random.default_rng(L)
    rw = rng.random((300, L)) * rng.choice([1e-9, 1.0, 1e9], (300, L))
    assert np.array_equal(X.fallback_rule_scores(rw), rw.sum(axis=1))
    monkeypatch.setattr(X, "FALLBACK_CHANNEL_AGGREGATION", "max")
    assert np.array_equal(X.fallback_rule_scores(rw), rw.max(axis=1))


def _same(got, want):
    assert got[3] == want[3]
    for a, b in zip(got[:3], want[:3]):
        assert a.dtype == b.dtype and a.shape == b.shape and np.array_equal(a, b)


@pytest.mark.parametrize("T", [3, 4])
def test_select_and_annotate(T):
    rng, att, rows, ident = _case(11 + T, T, N=3000)
    rows[:, -5] = rng.integers(0, 3, rows.shape[0])
    rows[::7, -8] = 0  # zero trials: precision 0
    for minimum in (0, 3, 8):
        _same(X.select_and_annotate_array(rows, att, ident, minimum), O.select_and_annotate(rows, att, ident, minimum))
    # fallback: nothing reaches the minimum
    _same(X.select_and_annotate_array(rows, att, ident, 100), O.select_and_annotate(rows, att, ident, 100))
    # duplicate best scores: the first of equal (score, body) keys
    dup = np.concatenate([rows[:10], rows[:10]])
    _same(X.select_and_annotate_array(dup, att, ident, 100), O.select_and_annotate(dup, att, ident, 100))
    _same(X.select_and_annotate_array(rows[:0], att, ident, 1), O.select_and_annotate(rows[:0], att, ident, 1))


def test_select_batch_matches_per_head():
    rng = np.random.default_rng(5)
    H, T, L, n = 6, 3, 3, 81
    att = rng.random((H, T, L, n)).astype(np.float32)
    cands = []
    for h in range(H):
        N = [0, 1, 40, 700, 3, 2000][h]
        rows = np.zeros((N, 12), np.int64)
        rows[:, 0] = rng.integers(1, 4, N)
        rows[:, 1:4] = rng.integers(0, n - 1, (N, 3))
        rows[:, 4:] = rng.integers(0, 5 if h != 4 else 1, (N, 8))
        cands.append(rows)
    got = X.select_and_annotate_batch(cands, att, n - 1, 2)
    assert len(got) == H
    for h in range(H):
        _same(got[h], O.select_and_annotate(cands[h], att[h], n - 1, 2))


def test_output_lines():
    sel = np.array([[2, 4, 7, 0, 10, 9, 3, 2, 1, 1, 1, 1]], np.int64)
    prec = np.array([0.3])
    rw = np.array([[0.25, 0.0, 1.0 / 3.0]])
    line = X.output_lines(5, sel, prec, rw)[0]
    want = "\t".join(["5", "4 7", "2", f"{0.25 + 0.0 + 1.0 / 3.0:.17g}", "10", "9", "3", "2", "1", "1", "1", "1",
                      "flashlog-graph-guided-rule", f"{0.25:.17g} {0.0:.17g} {1.0 / 3.0:.17g}", f"{0.3:.17g}"]) + "\r\n"
    assert line == want
    detailed, scalar = X.output_rule_lines(5, sel, prec, rw, {4: "r4", 7: "r7_inv"})
    assert detailed[0] == want.replace("\t4 7\t", "\tr4 r7_inv\t")
    assert scalar == [f"5\tr4 r7_inv\t2\t{0.25:.17g}\t0\tflashlog-rank-weighted-rule\r\n",
                      f"5\tr4 r7_inv\t2\t{1.0 / 3.0:.17g}\t2\tflashlog-rank-weighted-rule\r\n"]
