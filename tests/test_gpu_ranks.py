"""sparse2d_filtered_ranks_cuda on the GPU against the oracle restatement of
flashlog.cu:2754-2910 (bit-exact fp32 ranks)."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _fk():
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    return fk


def _case(rng, B, E, per_row, dtype, target_rate=0.7, filter_rate=0.02, dup_filter=True):
    rows, cols, vals = [], [], []
    targets = rng.integers(0, E, B)
    for b in range(B):
        k = int(rng.integers(0, per_row + 1))
        e = np.sort(rng.choice(E, k, replace=False))
        if rng.random() < target_rate and targets[b] not in e:
            e = np.sort(np.append(e, targets[b]))
        v = (rng.integers(0, 5, e.shape[0]) / 4.0).astype(dtype)  # many ties, explicit zeros
        v[rng.random(e.shape[0]) < 0.05] = -0.0
        rows.append(np.full(e.shape[0], b, np.int64))
        cols.append(e.astype(np.int64))
        vals.append(v)
    idx_b = np.concatenate(rows) if rows else np.zeros(0, np.int64)
    idx_e = np.concatenate(cols) if cols else np.zeros(0, np.int64)
    values = np.concatenate(vals).astype(dtype) if vals else np.zeros(0, dtype)
    fb = np.nonzero(rng.random(B * E) < filter_rate)[0]
    tk = np.arange(B, dtype=np.int64) * E + targets
    keys = np.concatenate([fb, tk[rng.random(B) < 0.8]]).astype(np.int64)
    if dup_filter and keys.size:
        keys = np.concatenate([keys, keys[: max(1, keys.size // 10)]])
    return idx_b, idx_e, values, targets, np.sort(keys)


def _run(idx_b, idx_e, values, targets, keys, B, E, use_eql, perm=None):
    dev = torch.device("cuda")
    if perm is not None:
        idx_b, idx_e, values = idx_b[perm], idx_e[perm], values[perm]
    t = [torch.from_numpy(np.ascontiguousarray(a)).to(dev) for a in (idx_b, idx_e, values, targets, keys)]
    out = _fk().sparse2d_filtered_ranks_cuda(*t, B, E, use_eql=use_eql)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("use_eql", [False, True])
@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("shuffle", [False, True])
def test_filtered_ranks_bitexact(use_eql, dtype, shuffle):
    rng = np.random.default_rng(11 + 2 * use_eql + shuffle)
    B, E = 97, 700
    idx_b, idx_e, values, targets, keys = _case(rng, B, E, 120, dtype)
    want = O.filtered_ranks(idx_b, idx_e, values, targets, keys, B, E, use_eql)
    perm = rng.permutation(idx_b.shape[0]) if shuffle else None
    got = _run(idx_b, idx_e, values, targets, keys, B, E, use_eql, perm)
    assert got.dtype == np.float32
    assert np.array_equal(got.view(np.int32), want.view(np.int32))


@pytest.mark.parametrize("use_eql", [False, True])
def test_filtered_ranks_edges(use_eql):
    rng = np.random.default_rng(5)
    B, E = 9, 40
    empty = np.zeros(0, np.int64)
    targets = rng.integers(0, E, B)
    # no entries and no filter: every query's truth is 0
    got = _run(empty, empty, np.zeros(0, np.float32), targets, empty, B, E, use_eql)
    want = O.filtered_ranks(empty, empty, np.zeros(0, np.float32), targets, empty, B, E, use_eql)
    assert np.array_equal(got, want)
    # entries but an empty filter
    idx_b, idx_e, values, targets, _ = _case(rng, B, E, 30, np.float32)
    got = _run(idx_b, idx_e, values, targets, empty, B, E, use_eql)
    want = O.filtered_ranks(idx_b, idx_e, values, targets, empty, B, E, use_eql)
    assert np.array_equal(got, want)


def test_filtered_ranks_c4_shape():
    """C4 evaluation shape: 5k queries over 123k entities, ~1k scored entities
    per query; checked against the oracle and, through the dense brute-force
    count, on a sample of rows."""
    rng = np.random.default_rng(2024)
    B, E = 5000, 123000
    idx_b, idx_e, values, targets, keys = _case(rng, B, E, 1000, np.float32, filter_rate=2e-5, dup_filter=False)
    for use_eql in (False, True):
        want = O.filtered_ranks(idx_b, idx_e, values, targets, keys, B, E, use_eql)
        got = _run(idx_b, idx_e, values, targets, keys, B, E, use_eql)
        assert np.array_equal(got.view(np.int32), want.view(np.int32))
    sample = np.arange(0, B, 997)
    S = np.zeros((sample.size, E), np.float32)
    filt = np.zeros((sample.size, E), bool)
    for j, b in enumerate(sample):
        m = idx_b == b
        S[j, idx_e[m]] = values[m]
        kb = keys[(keys >= b * E) & (keys < (b + 1) * E)] - b * E
        filt[j, kb] = True
    brute = O.filtered_ranks_brute(S, targets[sample], filt, True)
    np.testing.assert_array_equal(got[sample].astype(np.float64), brute)


def test_filtered_ranks_rejects_cpu_and_half():
    fk = _fk()
    z = torch.zeros(1, dtype=torch.long)
    with pytest.raises(RuntimeError):
        fk.sparse2d_filtered_ranks_cuda(z, z, torch.zeros(1), z, z, 1, 4)
    d = torch.device("cuda")
    with pytest.raises(RuntimeError):
        fk.sparse2d_filtered_ranks_cuda(z.to(d), z.to(d), torch.zeros(1, dtype=torch.float16, device=d), z.to(d),
                                        z.to(d), 1, 4)


@pytest.mark.parametrize("use_eql", [False, True])
@pytest.mark.parametrize("filtered", [False, True])
@pytest.mark.parametrize("E", [777, 5000])
def test_dense_filtered_ranks_bitexact(use_eql, filtered, E):
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    rng = np.random.default_rng(E + 2 * use_eql + filtered)
    B = 64
    state = (rng.integers(0, 9, (B, E)) / 8.0).astype(np.float32)  # heavy ties
    state[3] = 0.0  # a row of zeros: everything ties with the target
    targets = rng.integers(0, E, B)
    fb = fe = None
    fidx = None
    if filtered:
        n = 3000
        fb = rng.integers(0, B, n)
        fe = rng.integers(0, E, n)
        fidx = (torch.from_numpy(fb).cuda(), torch.from_numpy(fe).cuda())
    got = fk.dense_filtered_ranks_cuda(torch.from_numpy(state).cuda(), torch.from_numpy(targets).cuda(), fidx,
                                       use_eql)
    want = O.dense_filtered_ranks(state, targets, fb, fe, use_eql)
    assert got.dtype == torch.float32
    np.testing.assert_array_equal(got.cpu().numpy(), want)


def test_dense_filtered_ranks_checks():
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    s = torch.zeros(2, 10, device="cuda")
    with pytest.raises(ValueError):
        fk.dense_filtered_ranks_cuda(s, torch.tensor([0, 10], device="cuda"))
    with pytest.raises(ValueError):
        fk.dense_filtered_ranks_cuda(s, torch.tensor([0, 1], device="cuda"),
                                     (torch.tensor([2], device="cuda"), torch.tensor([0], device="cuda")))
    out = fk.dense_filtered_ranks_cuda(torch.zeros(0, 10, device="cuda"), torch.zeros(0, dtype=torch.long,
                                                                                      device="cuda"))
    assert out.shape == (0,)
