"""The allocation-free filtered ranks (fl_filtered_ranks_noalloc) against
the workspace entry point fl_filtered_ranks, through the C-ABI: two calls
in a row on one GPU, the second with fewer queries (the shared device
scratch keeps the first call's contents, so the second must clear what it
uses), float and double scores, both tie rules, and the size limit."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _case(rng, B, E, per_row, f64):
    b = np.repeat(np.arange(B), per_row)
    e = np.concatenate([np.sort(rng.choice(E, per_row, replace=False)) for _ in range(B)])
    v = rng.integers(0, 6, b.size).astype(np.float64 if f64 else np.float32) / 4.0  # many ties, some zeros
    tgt = rng.integers(0, E, B)
    fkeys = np.unique(np.concatenate([np.arange(B) * E + tgt, rng.integers(0, B * E, 3 * B)]))
    return [torch.from_numpy(np.ascontiguousarray(x)).cuda() for x in (b, e, v, tgt, fkeys)]


def _ranks(lib, noalloc, b, e, v, tgt, fkeys, B, E, use_eql):
    from flashlog_amd._lib import check, ptr
    f64 = 1 if v.dtype == torch.float64 else 0
    out = torch.full((B,), -1.0, dtype=torch.float32, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = (ptr(b), ptr(e), ptr(v), f64, ptr(tgt), ptr(fkeys), b.numel(), fkeys.numel(), B, E, int(use_eql))
    if noalloc:
        check(lib.fl_filtered_ranks_noalloc(st, *args, ptr(out)), "filtered_ranks_noalloc")
    else:
        nbytes = lib.fl_filtered_ranks_workspace_bytes(B, f64)
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        check(lib.fl_filtered_ranks(st, *args, ptr(out), ptr(ws), nbytes), "filtered_ranks")
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("f64", [False, True])
@pytest.mark.parametrize("use_eql", [False, True])
def test_noalloc_ranks_match_workspace_entry_point(f64, use_eql):
    from flashlog_amd import _lib
    lib = _lib.lib()
    rng = np.random.default_rng(5 + 2 * f64 + use_eql)
    E = 5000
    for B, per_row in ((4000, 50), (700, 30)):  # the second call is smaller
        args = _case(rng, B, E, per_row, f64)
        want = _ranks(lib, False, *args, B, E, use_eql)
        got = _ranks(lib, True, *args, B, E, use_eql)
        assert (want >= 1).all()
        assert np.array_equal(got.view(np.int32), want.view(np.int32)), B


def test_noalloc_ranks_refuse_too_many_queries():
    from flashlog_amd import _lib
    lib = _lib.lib()
    B = 65536 + 1
    z = torch.zeros(1, dtype=torch.int64, device="cuda")
    v = torch.zeros(1, dtype=torch.float32, device="cuda")
    out = torch.empty(B, dtype=torch.float32, device="cuda")
    from flashlog_amd._lib import ptr
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.fl_filtered_ranks_noalloc(st, ptr(z), ptr(z), ptr(v), 0, ptr(z), ptr(z), 1, 1, B, 10, 0, ptr(out))
    assert rc != 0
    assert b"at most 65536" in lib.fl_last_error()
