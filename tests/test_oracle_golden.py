"""The C oracle against golden vectors produced by the reference's own CPU
code (flashlog.cpp / csr.cpp built in place, tests/golden/make_golden.py)."""
import os

import numpy as np
import pytest

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden", "dense_golden.npz")


def _cases():
    z = np.load(GOLD, allow_pickle=False)
    for spec in z["specs"]:
        seed, E, R, M, B, L = (int(x) for x in spec)
        yield seed, E, R, z


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_build_side_matches_reference(seed):
    z = np.load(GOLD, allow_pickle=False)
    spec = [s for s in z["specs"] if s[0] == seed][0]
    E = int(spec[1])
    b = "s%d" % seed
    mine = O.build_csr_structure(z[b + "_h"], z[b + "_t"], z[b + "_r"], E)
    for k, a in enumerate(mine):
        assert np.array_equal(a, z["%s_csr%d" % (b, k)]), k


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_dense_forward_backward_match_reference_bits(seed):
    z = np.load(GOLD, allow_pickle=False)
    spec = [s for s in z["specs"] if s[0] == seed][0]
    E, R = int(spec[1]), int(spec[2])
    b = "s%d" % seed
    csr = tuple(z["%s_csr%d" % (b, k)] for k in range(16))
    mask = z[b + "_mask"]
    masks = (mask[csr[3]].astype(np.float32), mask[csr[7]].astype(np.float32))
    A, w = z[b + "_A"], z[b + "_w"]
    g = (z[b + "_gind"], z[b + "_gori"], z[b + "_ginv"])
    keys = sorted({k.rsplit("_", 1)[0] for k in z.files if k.startswith(b + "_K")})
    assert keys
    for key in keys:
        K = int(key.split("_K")[1].split("_")[0])
        K = 1 << 60 if K == 10 ** 9 else K
        wot_i = key.endswith("_w1")
        fo = O.dense_forward(A, w, csr, masks, R, wot_i=wot_i, topk_edges=K)
        for nm, x in zip(("ind", "ori", "inv"), fo):
            assert np.array_equal(x.view(np.int32), z[key + "_" + nm].view(np.int32)), (key, nm)
        gA, gw = O.dense_backward(*g, A, w, csr, masks, R, wot_i=wot_i, topk_edges=K)
        assert np.array_equal(gA.view(np.int32), z[key + "_gA"].view(np.int32)), key
        assert np.array_equal(gw.view(np.int32), z[key + "_gw"].view(np.int32)), key
