"""The measurement tooling of bench.py on synthetic inputs (CPU only): the
sparse hop's byte formula against its terms counted by hand, the per-item
kernel bytes, the dense pull's byte count against a brute force over the
admitted edges, the counter summary's copy calibration and per-step MB, and
the kernel-statistics table with its default-batch means from a trace."""
import csv
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_sparse_hop_bytes_terms():
    plan = {"nnz": 10, "rows": 4, "n": 7, "nout": 30, "groups": 50, "items": 110, "wot_i": False,
            "backward": False}
    kept = 110 - 10
    fwd = 28 * 10 + 4 * 4 * 7 + (2 * 8 * 10 + 10 * 50 + 9 * kept) + 28 * 30
    assert bench.sparse_hop_bytes(plan) == fwd
    plan["backward"] = True
    bwd = 28 * 10 + 4 * 30 + 8 * 4 * 7 + (2 * 8 * 10 + 10 * 50 + 13 * kept) + 4 * 10
    assert bench.sparse_hop_bytes(plan) == fwd + bwd
    plan["wot_i"] = True  # no identity items: every raw item is a kept edge
    assert bench.sparse_hop_bytes(plan) - bench.sparse_hop_bytes(dict(plan, items=100)) == (9 + 13) * 10


def test_item_kernel_bytes():
    plan = {"nnz": 10, "rows": 4, "n": 7, "nout": 30, "groups": 50, "items": 110, "wot_i": False,
            "backward": True, "chunks": 3}
    b = bench.item_kernel_bytes([plan, plan])
    assert b["k_sp_hist"] == 2 * 4 * 110
    assert b["k_sp_partition"] == 2 * 20 * 110
    assert b["k_sp_local_to_out"] == 2 * 12 * 110
    assert b["k_sp_select"] == 2 * ((24 + 16 + 24) * 10 + 10 * 50)
    assert b["k_sp_expand_fused"] == 2 * ((36 + 32) * 10 + 10 * 50 + 4 * 100 + 10 * 110)
    nb = bench.item_kernel_bytes([dict(plan, backward=False)])
    assert nb["k_sp_local_to_out"] == 0 and nb["k_sp_bwd"] == 0


def _admitted_brute(wts, cnts, K):
    """Edges kept per group under the c2 budget, edge by edge: the eligible
    edges (w > 0) in (weight desc, position asc) order, the first K kept --
    the rule of flashlog.cpp:12-89 (ties admitted in group order)."""
    edges = [(-wt, j, q) for j, (wt, c) in enumerate(zip(wts, cnts)) if wt > 0 for q in range(c)]
    if K > 0:
        edges = sorted(edges)[:K]
    keep = [0] * len(wts)
    for _, j, _ in edges:
        keep[j] += 1
    return keep


def test_c2_admitted_brute():
    rng = np.random.default_rng(9)
    for _ in range(300):
        g = int(rng.integers(1, 8))
        wts = rng.choice([0.0, 0.25, 0.5, 0.75], g).astype(np.float32)
        cnts = rng.integers(1, 6, g)
        K = int(rng.integers(0, 20))
        assert list(bench.c2_admitted(wts, cnts, K)) == _admitted_brute(wts.tolist(), cnts.tolist(), K)


def test_hop_pull_bytes_brute():
    """Output bytes + per active source its row pointers and group records +
    8 B per edge admitted for at least one row, counted edge by edge."""
    from oracle import oracle as O
    rng = np.random.default_rng(5)
    E, R, M = 40, 3, 300
    h, t, r = rng.integers(0, E, M), rng.integers(0, E, M), rng.integers(0, R, M)
    csr = O.build_csr_structure(h, t, r, E)
    BL = 5
    A = np.zeros((BL, E), np.float32)
    A[rng.integers(0, BL, 30), rng.integers(0, E, 30)] = 1.0
    w = rng.random((BL, 2 * R + 1)).astype(np.float32)
    for K in (0, 2):
        got = bench.hop_pull_bytes(A, w, csr, R, K)
        want = 8 * BL * E
        act = np.nonzero((A != 0).any(0))[0]
        for gp, grel, gst, gcnt, off in ((csr[8], csr[9], csr[10], csr[11], 0), (csr[12], csr[13], csr[14], csr[15], R)):
            want += 8 * act.size + 10 * int(sum(gp[s + 1] - gp[s] for s in act))
            for s in act:
                rows = np.nonzero(A[:, s])[0]
                edges = set()
                for bl in rows:
                    # the kept edges of (s, row): c2 admission when over the budget
                    g = range(gp[s], gp[s + 1])
                    wts = [float(w[bl, off + grel[j]]) for j in g]
                    cnts = [int(gcnt[j]) for j in g]
                    keep = _admitted_brute(wts, cnts, K)
                    for j, k in zip(g, keep):
                        edges.update(range(int(gst[j]), int(gst[j]) + int(k)))
                want += 8 * len(edges)
        assert got == want, K


def _write_csv(path, rows):
    with open(path, "w", newline="") as f:
        wr = csv.DictWriter(f, fieldnames=list(rows[0]))
        wr.writeheader()
        wr.writerows(rows)


def test_pmc_summary(tmp_path):
    def rows(counter, copy_kib, per):
        out = [{"Dispatch_Id": "1", "Kernel_Name": "__amd_rocclr_copyBuffer", "Counter_Name": counter,
                "Counter_Value": str(copy_kib)}]
        d = 2
        for name, vals in per.items():
            for v in vals:
                out.append({"Dispatch_Id": str(d), "Kernel_Name": "void fl::%s(int*)" % name, "Counter_Name": counter,
                            "Counter_Value": str(v)})
                d += 1
        return out
    steps = 2
    # the copy reads half its bytes through FETCH_SIZE and writes all of them
    fetch = rows("FETCH_SIZE", 131072.0, {"k_pull": [1000.0, 1000.0], "k_csr_fill": [50.0]})
    write = rows("WRITE_SIZE", 262144.0, {"k_pull": [500.0, 500.0], "k_csr_fill": [10.0]})
    _write_csv(tmp_path / "f.csv", fetch)
    _write_csv(tmp_path / "w.csv", write)
    out = tmp_path / "s.txt"
    bench.pmc_summary(str(tmp_path / "f.csv"), str(tmp_path / "w.csv"), steps, str(out), config=2)
    text = out.read_text()
    assert "C2 dense sum step" in text and "--config 2 --copy-mb 256 --counter-steps 2" in text
    # k_pull: fetch 2 x 1000 KiB x 2.0, write 2 x 500 KiB x 1.0, per step
    f_mb, w_mb = 2 * 1000 * 2.0 * 1024 / 1e6 / steps, 2 * 500 * 1.0 * 1024 / 1e6 / steps
    line = [ln for ln in text.splitlines() if ln.startswith("k_pull ")][0]
    assert line == "k_pull %.1f (fetch %.1f, write %.1f)" % (f_mb + w_mb, f_mb, w_mb)
    assert "k_csr_fill:" in text  # dispatched once: listed apart
    bench.TRAFFIC_FILE, old = str(out), bench.TRAFFIC_FILE
    try:
        assert bench.measured_traffic(["k_pull"]) == pytest.approx(float(line.split()[1]) * 1e6)
    finally:
        bench.TRAFFIC_FILE = old


def test_stats_table_default_batch_means(tmp_path):
    stats = [{"Name": "void fl::k_sp_partition(long)", "Calls": "9", "TotalDurationNs": "900", "AverageNs": "100",
              "Percentage": "60", "MinNs": "10", "MaxNs": "200"},
             {"Name": "fl::k_fill(int*)", "Calls": "2", "TotalDurationNs": "20", "AverageNs": "10",
              "Percentage": "40", "MinNs": "10", "MaxNs": "10"}]
    _write_csv(tmp_path / "stats.csv", stats)
    # 3 launches per step: the first 2 steps (6 launches) at 10 ns, then 3 of another batch at 100 ns
    trace, t = [], 0
    for d in [10] * 6 + [100] * 3:
        trace.append({"Kernel_Name": "void fl::k_sp_partition(long)", "Start_Timestamp": str(t),
                      "End_Timestamp": str(t + d)})
        t += 1000
    _write_csv(tmp_path / "trace.csv", trace)
    out = tmp_path / "t.md"
    bench.stats_table(str(out), str(tmp_path / "stats.csv"), "T", "python3 <repo>/bench.py",
                      trace_csv=str(tmp_path / "trace.csv"), first_steps=2)
    text = out.read_text()
    assert "| fl::k_sp_partition | 9 | 0.1 |" in text
    assert "| fl::k_sp_partition | 0.0 |" in text  # 10 ns = 0.01 us over the first 6 launches
    assert "<the run's kernel_trace.csv> 2" in text
    bench.stats_table(str(out), str(tmp_path / "stats.csv"), "T", "cmd")
    assert "default batch" not in out.read_text()


def test_counter_table_dense(tmp_path):
    # two dispatches of k_seg_max, one of k_pull_max, a torch kernel left out;
    # the derived columns are means of per-dispatch sums
    def rows(per):
        out, d = [], 1
        for name, vals in per.items():
            for counter, v in vals:
                out.append({"Dispatch_Id": str(d), "Kernel_Name": name, "Counter_Name": counter,
                            "Counter_Value": str(v)})
                d += 1
        return out
    p0 = rows({"void fl::k_seg_max<true>(int*)": [("SQ_LDS_BANK_CONFLICT", 10.0), ("SQ_LDS_IDX_ACTIVE", 40.0)],
               "void fl::k_seg_max<true>(long*)": [("SQ_LDS_BANK_CONFLICT", 30.0), ("SQ_LDS_IDX_ACTIVE", 40.0)],
               "void at::native::reduce_kernel(int)": [("SQ_LDS_BANK_CONFLICT", 5.0), ("SQ_LDS_IDX_ACTIVE", 5.0)]})
    p1 = rows({"void fl::k_pull_max(int*)": [("SQ_INSTS_VALU", 640.0), ("SQ_WAVES", 4.0)]})
    _write_csv(tmp_path / "p0.csv", p0)
    _write_csv(tmp_path / "p1.csv", p1)
    out = tmp_path / "c.md"
    bench.counter_table(str(out), [str(tmp_path / "p0.csv"), str(tmp_path / "p1.csv")], config=4)
    text = out.read_text()
    assert "dense hop kernels, C4 dense max step" in text
    assert "bench.py --config 4 --counter-steps 3" in text
    assert "reduce_kernel" not in text
    rows_ = {ln.split("|")[1].strip(): [c.strip() for c in ln.split("|")[2:-1]]
             for ln in text.splitlines() if ln.startswith("| k_")}
    assert set(rows_) == {"k_seg_max", "k_pull_max"}
    head = [c.strip() for c in [ln for ln in text.splitlines() if ln.startswith("| kernel")][0].split("|")[1:-1]]
    seg = dict(zip(head[1:], rows_["k_seg_max"]))
    assert seg["dispatches"] == "2" and seg["SQ_LDS_BANK_CONFLICT"] == "20"
    assert seg["LDS conflict / SQ_LDS_IDX_ACTIVE"] == "0.500"
    pull = dict(zip(head[1:], rows_["k_pull_max"]))
    assert pull["VALU insts / wave"] == "160.000"
