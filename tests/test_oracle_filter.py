"""Pins of the evaluation oracle: the known-answer expansion
(src/main.py:147-317) against a scan of every triple, over both the
triple-frame lookup and the CSR-side lookup; the raw sparse ranks
(src/main.py:365-388) against a per-entity count."""
import numpy as np
import pytest

from oracle import oracle as O


def _graph(seed, E=15, R=4, M=120):
    rng = np.random.default_rng(seed)
    h, r, t = rng.integers(0, E, M), rng.integers(0, R, M), rng.integers(0, E, M)
    # duplicate triples and a hub
    h[:10] = 3
    r[:10] = 1
    t[5:10] = t[:5]
    return rng, h, r, t, E, R


def _queries(rng, E, R, B):
    x = rng.integers(0, E + 2, B)  # some sources without any edge
    q = rng.integers(0, 2 * R, B)
    return x, q


@pytest.mark.parametrize("seed", range(6))
def test_filter_indices_match_triple_scan(seed):
    rng, h, r, t, E, R = _graph(seed)
    x, q = _queries(rng, E, R, 40)
    look = (O.filter_edge_lookup(h, r, t, R), O.filter_edge_lookup(t, r, h, R))
    got = O.filter_indices(x, q, R, look)
    want = O.filter_indices_brute(h, r, t, R, x, q)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])


@pytest.mark.parametrize("seed", range(4))
def test_csr_side_lookup_matches_triple_lookup(seed):
    rng, h, r, t, E, R = _graph(seed + 10)
    x, q = _queries(rng, E, R, 50)
    csr = O.build_csr_structure(h, t, r, E)
    side = (O.filter_side_lookup(csr[8], csr[9], csr[10], csr[11], csr[1], R),
            O.filter_side_lookup(csr[12], csr[13], csr[14], csr[15], csr[5], R))
    frame = (O.filter_edge_lookup(h, r, t, R), O.filter_edge_lookup(t, r, h, R))
    for a, b in zip(side, frame):  # the same groups, keys and columns
        for u, v in zip(a, b):
            assert np.array_equal(u, v)
    got = O.filter_indices(x, q, R, side)
    want = O.filter_indices_brute(h, r, t, R, x, q)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])


def test_filter_indices_edge_cases():
    rng, h, r, t, E, R = _graph(99)
    look = (O.filter_edge_lookup(h, r, t, R), O.filter_edge_lookup(t, r, h, R))
    e = np.zeros(0, np.int64)
    for x, q in [(e, e), (np.array([E + 5]), np.array([0])), (np.array([0, 1]), np.array([R, R + 1]))]:
        got = O.filter_indices(x, q, R, look)
        want = O.filter_indices_brute(h, r, t, R, x, q)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
    empty = (O.filter_edge_lookup(e, e, e, R),) * 2
    assert O.filter_indices(np.array([1]), np.array([0]), R, empty)[0].size == 0


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_raw_sparse_ranks_count(dtype):
    rng = np.random.default_rng(3)
    B, E = 9, 30
    dense = np.where(rng.random((B, E)) < 0.3, rng.choice([0.0, 0.5, 1.0, 2.0, -1.0], (B, E)), 0.0).astype(dtype)
    dense[0, :] = 0
    dense[1, 4] = 0.0  # explicit zero entry below
    b, e = np.nonzero(dense)
    b = np.concatenate([b, [1]])
    e = np.concatenate([e, [4]])
    order = np.argsort(b * E + e)
    b, e = b[order], e[order]
    v = dense[b, e]
    targets = rng.integers(0, E, B)
    targets[1] = 4
    got = O.raw_sparse_ranks(b, e, v, B, E, targets)
    for i in range(B):
        tv = dense[i, targets[i]]
        entries = [(int(ee), dense[i, ee]) for bb, ee in zip(b, e) if bb == i]
        ge = sum(1 for _, val in entries if val >= tv)
        missing = E - len(entries)
        want = ge + (missing if tv <= 0 else 0)
        assert got[i] == want and got.dtype == dtype
