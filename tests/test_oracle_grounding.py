"""Pins of the soft-grounding oracle: the C++ standard's mt19937_64 check,
and bit equality with the reference's own soft_grounding.cpp compiled into
oracle/_ref (Makefile.ref) for the reservoir sampler and whole grounding
runs (walk records aggregated, capped and united over folds)."""
import os
import sys

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import small_graph

REF_DIR = os.path.join(os.path.dirname(os.path.dirname(__file__)), "oracle", "_ref")


def _ref():
    sys.path.insert(0, REF_DIR)
    try:
        import torch  # noqa: F401
        import flashlog_grounding_ref
        return flashlog_grounding_ref
    except ImportError:
        pytest.skip("reference soft-grounding module not built (oracle/Makefile.ref)")


def test_mt19937_64_standard_check():
    # [rand.predef]: the 10000th consecutive invocation of a default-constructed
    # mt19937_64 (seed 5489) produces 9981545732273789042.
    assert O.mt64_nth(5489, 10000) == 9981545732273789042


@pytest.mark.parametrize("max_sources", [1, 7, 50, 100000])
@pytest.mark.parametrize("seed", [0, 12345, 2 ** 62 + 17])
def test_reservoir_matches_reference(max_sources, seed):
    import torch
    ref = _ref()
    h, r, t, E, R, csr = small_graph(2, 0.5)
    rels = np.array(sorted({0, 1, R - 1, R // 2}), np.int64)
    out, avail = O.reservoir(csr[8], csr[9], rels, max_sources, seed)
    rs, ra = ref.sample_relation_sources_reservoir(torch.from_numpy(csr[8].astype(np.int32)),
                                                   torch.from_numpy(csr[9].astype(np.int16)),
                                                   torch.from_numpy(rels), max_sources, seed)
    np.testing.assert_array_equal(out, rs.numpy())
    np.testing.assert_array_equal(avail, ra.numpy())
    # available counts are the per-relation group counts
    for i, rel in enumerate(rels):
        assert avail[i] == int((csr[9] == rel).sum())


def _ref_ground(ref, att, heads, folds, csr, R, walks, topk, mask, seeds, budgets):
    import torch
    tens = [torch.from_numpy(np.ascontiguousarray(csr[i])) for i in (1, 5, 8, 9, 10, 11, 12, 13, 14, 15)]
    tf = [[torch.from_numpy(np.asarray(f, np.int64)) for f in hf] for hf in folds]
    cands, raw, _ = ref.ground_head_batch_source_folds_sampled_capped_counts(
        torch.from_numpy(att), heads, R, tf, *tens, walks, topk, mask, seeds, 100000, 4, budgets)
    return [c.numpy() for c in cands], [r.numpy() for r in raw]


@pytest.mark.parametrize("cfg,scale", [(1, 0.05), (2, 0.2)])
@pytest.mark.parametrize("mask", [False, True])
@pytest.mark.parametrize("topk", [1, 3, 200])
def test_grounding_matches_reference(cfg, scale, mask, topk):
    ref = _ref()
    rng = np.random.default_rng(cfg * 10 + mask + topk)
    h, r, t, E, R, csr = small_graph(cfg, scale)
    V = 2 * R + 1
    heads = [0, R + 1, 2 * R - 1]
    ranks = 3
    att = rng.random((len(heads), 3, ranks, V)).astype(np.float32)
    att[att < 0.3] = 0.0  # some operators unavailable
    att[:, :, :, -1] = np.where(rng.random((len(heads), 3, ranks)) < 0.5, 0.0, att[:, :, :, -1])
    folds = [[rng.integers(0, E, 9), rng.integers(0, E, 5)], [rng.integers(0, E, 12)], [rng.integers(0, E, 4),
             rng.integers(0, E, 4), rng.integers(0, E, 3)]]
    seeds = [7, 2 ** 40 + 3, 99]
    budgets = [4, 30, 100]
    walks = 64
    rc, rr = _ref_ground(ref, att, heads, folds, csr, R, walks, topk, mask, seeds, budgets)
    for i, head in enumerate(heads):
        rows, raw = O.ground(att[i], R, head, folds[i], csr, walks, topk, mask, seeds[i], budgets)
        np.testing.assert_array_equal(rows, rc[i])
        np.testing.assert_array_equal(raw, rr[i])
