"""The C oracle against the reference's own CPU module built from its
sources (oracle/_ref, present where /root/reference is mounted)."""
import os
import sys

import numpy as np
import pytest

from oracle import oracle as O
from tests.helpers import attention, masks_for, small_graph, sparse_state

REF_DIR = os.path.join(os.path.dirname(os.path.dirname(__file__)), "oracle", "_ref")


def _ref():
    sys.path.insert(0, REF_DIR)
    try:
        import torch  # noqa: F401
        import flashlog_ref_cpp
        import flashlog_csr_ref
        return flashlog_ref_cpp, flashlog_csr_ref
    except ImportError:
        pytest.skip("reference CPU module not built (oracle/Makefile.ref)")


@pytest.mark.parametrize("cfg,scale", [(1, 0.05), (2, 0.03), (3, 0.01), (4, 0.003)])
@pytest.mark.parametrize("K", [1 << 60, 2, 200])
def test_oracle_matches_reference_build(cfg, scale, K):
    import torch
    ref, cref = _ref()
    rng = np.random.default_rng(cfg * 10 + (K % 7))
    h, r, t, E, R, csr = small_graph(cfg, scale)
    o = cref.build_side(h, t, r, E)
    i = cref.build_side(t, h, r, E)
    for k, (a, b) in enumerate(zip((*o[:4], *i[:4], *o[4:], *i[4:]), csr)):
        assert np.array_equal(np.asarray(a), b), k
    n = 2 * R + 1
    A = sparse_state(6, E, max(3, E // 20), rng)
    w = attention(6, n, rng)
    _, masks = masks_for(csr, h.shape[0], rng)
    T = lambda x: torch.from_numpy(np.ascontiguousarray(x))
    act = O.active_nodes(A)
    args = (T(csr[1]), T(masks[0]), T(csr[8]), T(csr[9]), T(csr[10]), T(csr[11]), T(csr[5]), T(masks[1]),
            T(csr[12]), T(csr[13]), T(csr[14]), T(csr[15]))
    ro = ref.flashlog_forward_cpu(T(A), T(w), T(act), *args, R, False, K)
    mo = O.dense_forward(A, w, csr, masks, R, topk_edges=K)
    for a, b in zip(mo, ro):
        assert np.array_equal(a.view(np.int32), b.numpy().view(np.int32))
    g = [rng.standard_normal(A.shape).astype(np.float32) for _ in range(3)]
    rb = ref.flashlog_backward_cpu(*[T(x) for x in g], T(A), T(w), T(act), *args, R, False, K)
    mb = O.dense_backward(*g, A, w, csr, masks, R, topk_edges=K)
    for a, b in zip(mb, rb):
        assert np.array_equal(a.view(np.int32), b.numpy().view(np.int32))
