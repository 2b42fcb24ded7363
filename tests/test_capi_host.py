"""The C-ABI library on the CPU: it loads, exports every symbol the header
declares, and its host-side graph preparation matches the oracle and the
pull-index invariants.  (No device call is made here.)"""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import small_graph

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _lib():
    from flashlog_amd import _lib
    return _lib


def test_library_exports_every_declared_symbol():
    header = open(os.path.join(ROOT, "include", "flashlog_hip.h")).read()
    declared = set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(fl_[a-z_0-9]+)\s*\(", header, re.M))
    assert declared, "no declarations parsed"
    lib = ctypes.CDLL(_lib().LIB_PATH)
    for name in sorted(declared):
        assert hasattr(lib, name), name
    assert declared == set(_lib().exported_symbols())
    assert _lib().lib().fl_abi_version() == _lib().ABI_VERSION


def test_struct_layouts_match_the_library():
    """The ctypes mirrors of fl_side, fl_sparse_hop and fl_ground_graph have
    the sizes the library was compiled with."""
    L = _lib()
    lib = L.lib()
    for struct, size_fn in L.STRUCT_SIZES:
        assert ctypes.sizeof(struct) == getattr(lib, size_fn)(), struct.__name__
    assert ctypes.sizeof(L.FlSide) == 8 * len(L.FlSide._fields_)


@pytest.mark.parametrize("cfg,scale", [(1, 0.05), (2, 0.05), (3, 0.02)])
def test_build_csr_structure_matches_oracle(cfg, scale):
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    h, r, t, E, R, ref = small_graph(cfg, scale)
    got = fk.build_csr_structure(torch.from_numpy(h), torch.from_numpy(t), torch.from_numpy(r), E)
    for k, (a, b) in enumerate(zip(got, ref)):
        assert np.array_equal(a.numpy(), b), k


def test_build_csr_rejects_out_of_range():
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    with pytest.raises(ValueError):
        fk.build_csr_structure(torch.tensor([0, 5]), torch.tensor([1, 1]), torch.tensor([0, 0]), 3)


def test_pull_index_is_destination_major_in_position_order():
    h, r, t, E, R, csr = small_graph(2, 0.05)
    lib = _lib().lib()
    for col, gptr, grel, gst, gcnt in ((csr[1], csr[8], csr[9], csr[10], csr[11]),
                                       (csr[5], csr[12], csr[13], csr[14], csr[15])):
        M = col.shape[0]
        arrs = [np.ascontiguousarray(a) for a in (col, gptr, grel, gst, gcnt)]
        pp = np.empty(E + 1, np.int32)
        pos = np.empty(M, np.int32)
        src = np.empty(M, np.int32)
        rel = np.empty(M, np.int16)
        p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
        assert lib.fl_pull_index_build(E, M, grel.shape[0], *[p(a) for a in arrs], p(pp), p(pos), p(src), p(rel)) == 0
        # slots of destination d list every position with col == d, ascending
        assert pp[0] == 0 and pp[-1] == M
        for d in range(0, E, max(1, E // 50)):
            want = np.nonzero(col == d)[0]
            assert np.array_equal(pos[pp[d]:pp[d + 1]], want)
        # source and relation of each slot agree with the group arrays
        row_of_pos = np.repeat(np.arange(E), np.diff(csr[0] if col is csr[1] else csr[4]))
        assert np.array_equal(src, row_of_pos[pos])
        rel_of_pos = (csr[2] if col is csr[1] else csr[6])
        assert np.array_equal(rel, rel_of_pos[pos])
        # heavy-destination segments cover exactly the heavy slots
        cnt = [ctypes.c_int64(0) for _ in range(3)]
        assert lib.fl_pull_segments(E, p(pp), *[ctypes.byref(c) for c in cnt], *([None] * 8)) == 0
        nseg, nheavy, nsup = (c.value for c in cnt)
        a = [np.empty(k, np.int32) for k in (nseg, nseg, nseg, nheavy, nheavy + 1, nheavy + 1, nsup, nsup)]
        assert lib.fl_pull_segments(E, p(pp), *[ctypes.byref(c) for c in cnt], *[p(x) for x in a]) == 0
        seg_dst, seg_start, seg_h, heavy_dst, hsp, hup, sup_h, sup_seg0 = a
        deg = np.diff(pp)
        assert np.array_equal(heavy_dst, np.nonzero(deg > _lib().FL_SEG)[0])
        for k, d in enumerate(heavy_dst):
            segs = np.arange(hsp[k], hsp[k + 1])
            assert np.all(seg_dst[segs] == d) and np.all(seg_h[segs] == k)
            assert np.array_equal(seg_start[segs], pp[d] + _lib().FL_SEG * np.arange(segs.size))
            sups = np.arange(hup[k], hup[k + 1])
            assert np.array_equal(sup_seg0[sups], hsp[k] + _lib().FL_SUP * np.arange(sups.size))
