"""Public C-ABI entry points that read no device data back on the host
handle malformed states on the device: fl_rule_accumulate writes nothing for
a state that is not coalesced or holds an index outside [B, L, E] (the
accumulator is checked together with a guard region after it), and
fl_sparse_normalize_forward writes every output entry whatever the row keys
hold (the output is pre-filled with a sentinel)."""
import ctypes

import numpy as np
import pytest
import torch

from flashlog_amd import _lib
from flashlog_amd._lib import check, ptr

pytestmark = pytest.mark.gpu


def _stream():
    return _lib.stream_handle(torch.device("cuda"))


def _accumulate(b, l, e, v, W, B, L, E, is_max):
    dev = torch.device("cuda")
    K = W.shape[1]
    guard = 1024
    buf = torch.full((K * B * E + guard,), 0.5, dtype=torch.float32, device=dev)
    ix = [torch.tensor(x, dtype=torch.int64, device=dev) for x in (b, l, e)]
    vv = torch.tensor(v, dtype=torch.float32, device=dev)
    Wt = torch.tensor(W, dtype=torch.float32, device=dev)
    lib = _lib.lib()
    nbytes = lib.fl_rule_accumulate_bytes(len(v), B, L)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    check(lib.fl_rule_accumulate(_stream(), ptr(ix[0]), ptr(ix[1]), ptr(ix[2]), ptr(vv), len(v), ptr(Wt), K, B, L, E,
                                 1 if is_max else 0, ptr(buf), ptr(ws), nbytes), "rule_accumulate")
    torch.cuda.synchronize()
    return buf.cpu().numpy(), K * B * E


@pytest.mark.parametrize("E", [10, 20000])
@pytest.mark.parametrize("is_max", [0, 1])
def test_rule_accumulate_well_formed(is_max, E):
    """Both sum paths: entities in LDS (E <= 16384) and the merge over the
    channels (larger E)."""
    B, L = 2, 3
    b, l, e = [0, 0, 1, 1], [0, 2, 1, 2], [3, 3, 9, 9]
    v = [1.0, 2.0, 3.0, 1.0]
    W = np.array([[0.5, 1.0], [0.25, 2.0], [1.0, 0.125]], np.float32)
    got, n = _accumulate(b, l, e, v, W, B, L, E, is_max)
    want = np.full(n, 0.5, np.float32)
    for k in range(2):
        for q in range(4):
            slot = k * B * E + b[q] * E + e[q]
            x = np.float32(v[q]) * W[l[q], k]
            want[slot] = max(want[slot], x) if is_max else want[slot] + x
    if not is_max:  # one writer per slot: the chunk's sum from 0, then added
        want = np.full(n, 0.5, np.float32)
        for k in range(2):
            for bb, ee, qs in ((0, 3, (0, 1)), (1, 9, (2, 3))):
                acc = np.float32(0.0)
                for q in qs:
                    acc = np.float32(acc + np.float32(v[q]) * W[l[q], k])
                want[k * B * E + bb * E + ee] = np.float32(want[k * B * E + bb * E + ee] + acc)
    assert np.array_equal(got[:n], want)
    assert (got[n:] == 0.5).all()


@pytest.mark.parametrize("E", [8, 20000])
@pytest.mark.parametrize("is_max", [0, 1])
@pytest.mark.parametrize("case", ["entity_high", "entity_negative", "batch_high", "unsorted", "duplicate"])
def test_rule_accumulate_malformed_writes_nothing_out_of_shape(case, is_max, E):
    B, L = 2, 2
    b, l, e, v = [0, 0, 1], [0, 1, 1], [1, 2, 7], [1.0, 1.0, 1.0]
    if case == "entity_high":
        e = [1, 2, E]
    elif case == "entity_negative":
        e = [-1, 2, 7]
    elif case == "batch_high":
        b = [0, 0, 2]
    elif case == "unsorted":
        b, l, e = [0, 0, 0], [1, 1, 0], [5, 2, 1]
    else:  # an entity twice in one row (not coalesced)
        b, l, e = [0, 0, 1], [1, 1, 1], [2, 2, 7]
    W = np.ones((L, 1), np.float32)
    got, n = _accumulate(b, l, e, v, W, B, L, E, is_max)
    assert (got[n:] == 0.5).all()
    if not is_max:
        assert (got[:n] == 0.5).all()  # a flagged state adds nothing
    else:  # entries outside the shape are skipped, the others kept
        ok = [q for q in range(3) if 0 <= b[q] < B and 0 <= e[q] < E]
        for q in ok:
            assert got[b[q] * E + e[q]] == 1.0


@pytest.mark.parametrize("keys", [[-1, 0, 0, 1], [0, 1, 1, 5], [1, 0, 0, 1], [3, 3, 3, 3]])
def test_normalize_writes_every_output(keys):
    dev = torch.device("cuda")
    B, L = 2, 2
    kb = np.array(keys, np.int64)
    sb = torch.tensor(np.floor_divide(kb, L), device=dev)
    sl = torch.tensor(np.mod(kb, L), device=dev)
    v = torch.tensor([1.0, 2.0, 3.0, 4.0], device=dev)
    out = torch.full((4,), float("nan"), device=dev)
    denom = torch.empty(B * L, device=dev)
    row_ptr = torch.empty(B * L + 1, dtype=torch.int64, device=dev)
    err = torch.empty(2, dtype=torch.int64, device=dev)
    check(_lib.lib().fl_sparse_normalize_forward(_stream(), ptr(sb), ptr(sl), ptr(v), 4, B, L, ctypes.c_float(1e-7),
                                                 ptr(out), ptr(denom), ptr(row_ptr), ptr(err)), "normalize")
    rp = row_ptr.cpu().numpy()
    assert rp[0] == 0 and rp[-1] == 4 and (np.diff(rp) >= 0).all()
    assert torch.isfinite(out).all()
