"""Benchmark of the FlashLog propagation hot path on one MI355X.

Default workload: BASELINE.json configs[4] (C5), the largest configuration
and the one the throughput target is stated on -- DRUM --sparse on one GPU,
4.6M entities, 822 base relations, 20M triples (Zipf(1.0) relations,
Zipf(1.3) degrees), batch 256, N=3 channels, T=3 hops, c1=1000, c2=400,
forward and backward.  A step is one training step of that model
(src/model_DRUM_kernel_sp.py:92-205): three hops of sampled_sparse_propagation
(exponential-race c1, quota c2), each followed by normalize_sparse3d, the sum
over the channels, the model's log loss on each query's target entity
(src/utils.py:37-47) and the backward pass to the per-hop attention.  The
attention is random (softmax of N(0,1) logits) in place of the model's LSTM;
graph and queries are synthetic and seeded (flashlog_amd/synth.py).
--mode eval: the evaluation pass (c1/c2 thresholds, no gradients).
--config 2: configs[1] (C2), the dense DRUM hop (dense_csr_sum_cuda,
flashlog_kernel.py:1629-1663) with c1=1000, c2=400 and the model's
normalization.  --config 4: configs[3] (C4), the mmDRUM dense max hop with
its backward and the 5k-query filtered ranking.  --grounding: the soft
grounding sampler on the C3 graph.  --rules: C3's rule-bank scoring.

Prints one JSON line.  ``value`` = queries/sec (batch / step time) with all
inputs resident in HBM.  ``roofline`` is for the propagation kernel (k_sp_items
for C5, k_pull for C2), timed with HIP events the library records around its
launches on its own stream; ``cpu_baseline`` is the reference's CPU path (its
flashlog.cpp built into oracle/_ref) on a bounded sample of the same workload.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="bound on the CPU baseline sample (0 disables it)")
    ap.add_argument("--profile-steps", type=int, default=10)
    ap.add_argument("--sparse", action="store_true",
                    help="the DRUM --sparse GPU path (default for --config 5)")
    ap.add_argument("--grounding", action="store_true",
                    help="soft grounding (rule extraction's walk sampler) on the C3 graph")
    ap.add_argument("--rules", action="store_true",
                    help="rule-bank scoring (rules/shared_inference.score) on the C3 graph")
    ap.add_argument("--mode", choices=["train", "eval"], default="train",
                    help="--sparse step: a training step (sampled hops, loss, backward; the default, as "
                         "configs[4] is quoted forward and backward) or an evaluation pass")
    ap.add_argument("--copy-mb", type=int, default=0,
                    help="first run 3 plain device copies of this many MiB (a known-size reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--counter-steps", type=int, default=0,
                    help="run exactly this many steps of the configuration's step and stop (a rocprofv3 "
                         "counter pass; no timing, no CPU baseline)")
    ap.add_argument("--pmc-summary", nargs=4, metavar=("FETCH_CSV", "WRITE_CSV", "STEPS", "OUT"),
                    help="write the per-step HBM traffic summary of two rocprofv3 counter passes "
                         "(FETCH_SIZE, then WRITE_SIZE, each over --copy-mb 256 --counter-steps STEPS); "
                         "with --config, of that configuration's runs")
    ap.add_argument("--stats-table", nargs="+", metavar="ARG",
                    help="OUT STATS_CSV TITLE RUN_COMMAND [TRACE_CSV FIRST_STEPS]: write the kernel-time table "
                         "of a rocprofv3 --kernel-trace --stats run (its kernel_stats.csv) as markdown, naming "
                         "the run's command; with its kernel_trace.csv, also each per-hop kernel's mean over "
                         "the run's first FIRST_STEPS steps")
    ap.add_argument("--counter-table", nargs="+", metavar="ARG",
                    help="OUT CSV [CSV ...]: write the per-dispatch means of every counter in these "
                         "rocprofv3 counter_collection.csv files (one per pass over --counter-steps) for "
                         "the sparse hop kernels, as a markdown table")
    return ap.parse_args()


def stats_table(out_path, stats_csv, title, run_command, top=30, trace_csv=None, first_steps=0, per_step=3):
    """The rocprofv3 kernel statistics (per kernel: calls, average, min and
    max duration, share of GPU time) as a markdown table.  With a kernel
    trace and first_steps: for the kernels launched per_step times a step,
    also the mean duration over their first first_steps * per_step launches
    (the default workload's steps, which the C5 bench runs before its
    reference-batch steps) -- the figure the bench's own per-launch timing
    is comparable with."""
    import csv
    rows = list(csv.DictReader(open(stats_csv)))
    rows.sort(key=lambda r: -float(r["Percentage"]))
    first = {}
    if trace_csv and first_steps > 0:
        launches = {}
        for r in sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"])):
            launches.setdefault(r["Kernel_Name"], []).append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
        n = first_steps * per_step
        for name, d in launches.items():
            if len(d) >= n and len(d) % per_step == 0:
                first[name] = sum(d[:n]) / n / 1e3
    lines = ["# %s" % title, "", "Commands (from the repo root, on one MI355X):", "", "```",
             "cd /tmp && rocprofv3 --kernel-trace --stats --output-format csv -d /tmp/prof -o run -- " + run_command,
             "python3 <repo>/bench.py --stats-table <this file> <the run's kernel_stats.csv> <title> <run command>"
             + (" <the run's kernel_trace.csv> %d" % first_steps if first else ""),
             "```", "",
             "Names: fl:: are this library's kernels, at:: and rocprim:: torch's.", "",
             "| kernel | calls | avg us | min us | max us | % of GPU time |", "|---|---|---|---|---|---|"]
    for r in rows[:top]:
        name = r["Name"].replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "")[:72]
        lines.append("| %s | %s | %.1f | %.1f | %.1f | %.2f |" % (
            name, r["Calls"], float(r["AverageNs"]) / 1e3, float(r["MinNs"]) / 1e3, float(r["MaxNs"]) / 1e3,
            float(r["Percentage"])))
    if first:
        lines += ["", "The default batch's steps alone (the first %d steps of the run, %d launches per step of "
                  "each kernel below; the reference batch's %s-query steps follow them): mean us per launch, "
                  "from the run's kernel trace." % (first_steps, per_step, "512"), "",
                  "| kernel | mean us per launch, default batch |", "|---|---|"]
        for name, us in sorted(first.items(), key=lambda x: -x[1])[:20]:
            short = name.replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "")[:72]
            lines.append("| %s | %.1f |" % (short, us))
    with open(out_path, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("wrote", out_path)


def _pmc_counters(path):
    """Names of the counters in a rocprofv3 counter_collection.csv."""
    import csv
    with open(path) as f:
        return sorted({row.get("Counter_Name") or row.get("Counter-Name") for row in csv.DictReader(f)})


def counter_table(out_path, csvs, config=5):
    """Per hop kernel of the workload (C5: the sparse hop's; C2 / C4: every
    kernel of this library in the run): dispatches and the mean over its
    dispatches of every counter of the passes (a dispatch's value summed
    over its rows), with two derived columns where their counters were
    collected: LDS bank-conflict cycles per LDS-active cycle and VALU
    instructions per wave."""
    cols = {}
    for path in csvs:
        for c in _pmc_counters(path):
            cols[c] = _pmc_per_kernel(path, c)
    if config == 5:
        names = [k for k in SPARSE_KERNELS if any(k in per for per in cols.values())]
    else:
        names = sorted({k for per in cols.values() for k in per if k.startswith("k_")})
    title, run = PMC_WORKLOADS[config]
    counters = sorted(cols)
    head = ["kernel", "dispatches"] + counters
    derived = []
    for active in ("SQ_LDS_IDX_ACTIVE", "SQ_ACTIVE_INST_LDS"):
        if "SQ_LDS_BANK_CONFLICT" in cols and active in cols:
            derived.append(("LDS conflict / %s" % active, "SQ_LDS_BANK_CONFLICT", active))
            break
    if "SQ_INSTS_VALU" in cols and "SQ_WAVES" in cols:
        derived.append(("VALU insts / wave", "SQ_INSTS_VALU", "SQ_WAVES"))
    head += [d[0] for d in derived]
    lines = ["# Counters per dispatch of the %s kernels, %s"
             % ("sparse hop" if config == 5 else "dense hop", title), "",
             "One rocprofv3 pass per counter set over `--counter-steps` (from the repo root, on one MI355X), "
             "then this table:", ""]
    for i, path in enumerate(csvs):
        lines.append("    cd /tmp && rocprofv3 --pmc %s --output-format csv -d /tmp/p_%d -o run -- "
                     "python3 <repo>/bench.py %s--counter-steps 3" % (" ".join(_pmc_counters(path)), i, run))
    lines += ["    python3 <repo>/bench.py %s--counter-table <this file> " % run
              + " ".join("<pass %d counter_collection.csv>" % i for i in range(len(csvs))), "",
              "Means over each kernel's dispatches (all hops of the run); a dispatch's value is summed "
              "over the counter's instances.", ""]
    lines += ["| " + " | ".join(head) + " |", "|" + "---|" * len(head)]

    def mean(c, k):
        v = cols[c].get(k)
        return sum(v) / len(v) if v else None

    for k in names:
        disp = max(len(cols[c].get(k, [])) for c in counters)
        row = [k, str(disp)]
        for c in counters:
            m = mean(c, k)
            row.append("-" if m is None else ("%.4g" % m))
        for _, a, b in derived:
            x, y = mean(a, k), mean(b, k)
            row.append("%.3f" % (x / y) if x is not None and y else "-")
        lines.append("| " + " | ".join(row) + " |")
    with open(out_path, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("wrote", out_path)


def _pmc_per_kernel(path, counter):
    """{kernel: (dispatches, [values])} of one counter in a rocprofv3
    counter_collection.csv (a dispatch's value summed over its rows)."""
    import collections
    import csv
    per = collections.defaultdict(dict)
    with open(path) as f:
        for row in csv.DictReader(f):
            if (row.get("Counter_Name") or row.get("Counter-Name")) != counter:
                continue
            name = (row.get("Kernel_Name") or row.get("Kernel-Name") or "").replace("(anonymous namespace)::", "")
            name = name.split("(")[0]
            name = name.replace("void ", "").split("<")[0].split("::")[-1]
            disp = row.get("Dispatch_Id") or row.get("Dispatch-Id")
            per[name][disp] = per[name].get(disp, 0.0) + float(row.get("Counter_Value") or 0.0)
    return {k: list(v.values()) for k, v in per.items()}


PMC_WORKLOADS = {5: ("C5 sparse training step", ""),
                 2: ("C2 dense sum step (evaluation)", "--config 2 "),
                 4: ("C4 dense max step (forward + backward)", "--config 4 ")}


def pmc_summary(fetch_csv, write_csv, steps, out_path, config=5):
    """Per kernel: HBM MB per step = (FETCH_SIZE, WRITE_SIZE in KiB per
    dispatch, each scaled by the ratio of the bytes a plain 256 MiB device
    copy moves to what the counter reads for it) summed over the kernel's
    dispatches / steps.  Kernels dispatched fewer times than there are steps
    (once per run) are listed apart."""
    fe = _pmc_per_kernel(fetch_csv, "FETCH_SIZE")
    wr = _pmc_per_kernel(write_csv, "WRITE_SIZE")
    copy = [k for k in fe if "copyBuffer" in k]
    cf = max(max(fe[k]) for k in copy)
    cw = max(max(wr[k]) for k in copy if k in wr)
    ff, fw = 262144.0 / cf, 262144.0 / cw
    rows = []
    for k in fe:
        if "copyBuffer" in k or not k.startswith("k_"):
            continue
        f_mb = sum(fe[k]) * ff * 1024 / 1e6
        w_mb = sum(wr.get(k, [])) * fw * 1024 / 1e6
        rows.append(((f_mb + w_mb) / steps, k, len(fe[k]), f_mb / steps, w_mb / steps))
    rows.sort(reverse=True)
    title, run = PMC_WORKLOADS[config]
    lines = ["# HBM traffic per step of this library's kernels, %s" % title,
             "",
             "Two rocprofv3 counter passes over `--counter-steps %d` (from the repo root, on one MI355X):" % steps,
             "",
             "    cd /tmp && rocprofv3 --pmc FETCH_SIZE --output-format csv -d /tmp/p_fetch -o run -- "
             "python3 <repo>/bench.py %s--copy-mb 256 --counter-steps %d" % (run, steps),
             "    cd /tmp && rocprofv3 --pmc WRITE_SIZE --output-format csv -d /tmp/p_write -o run -- "
             "python3 <repo>/bench.py %s--copy-mb 256 --counter-steps %d" % (run, steps),
             "    python3 <repo>/bench.py %s--pmc-summary <fetch counter_collection.csv> "
             "<write counter_collection.csv> %d <this file>" % (run, steps),
             "",
             "Copy calibration: a 256 MiB device copy reads FETCH_SIZE %.1f KiB and WRITE_SIZE %.1f KiB; "
             "scale factors to bytes %.3f (fetch) and %.3f (write)." % (cf, cw, ff, fw),
             "",
             "Per-step kernels (name, MB per step, then its fetched and written MB):", ""]
    once = []
    for mb, k, d, f_mb, w_mb in rows:
        if d < steps:
            once.append((mb * steps, k, d))
            continue
        # "<kernel> <MB per step> ..." lines are read by bench.py
        lines.append("%s %.1f (fetch %.1f, write %.1f)" % (k, mb, f_mb, w_mb))
    lines += ["", "Once-per-run kernels (MB in the run, dispatches):", ""]
    lines += ["    %s: %.1f MB, %d" % (k, mb, d) for mb, k, d in once]
    with open(out_path, "w") as f:
        f.write("\n".join(lines) + "\n")
    print("wrote", out_path)


def copy_calibration(mb):
    import torch
    x = torch.ones(mb * (1 << 20) // 4, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    print("copy calibration: 3 copies of %d MiB" % mb, file=sys.stderr, flush=True)


FLUSH_MIB = 512


def cache_flusher(mib=FLUSH_MIB):
    """A callable that writes a `mib` MiB device buffer.  Run before each hop
    of a timed pass it evicts the L2s and the 256 MB Infinity Cache: the
    cold-cache condition of the roofline measurement (the hop then reads its
    graph and state from HBM)."""
    import torch
    buf = torch.empty(mib * (1 << 20) // 4, dtype=torch.float32, device="cuda")
    return lambda: buf.fill_(0.0)


def profile_pass(lib, kernels, steps, run):
    """Per-launch ms of `kernels` over `steps` calls of run() (HIP events
    around each launch inside the library)."""
    import torch
    lib.prof_enable(True)
    for _ in range(steps):
        run()
    torch.cuda.synchronize()
    prof = {k: lib.prof_read(k) for k in kernels}
    lib.prof_enable(False)
    return {k: (v[0] / v[1] if v[1] else 0.0) for k, v in prof.items()}


def host_cpu():
    """CPU model and core counts of the host the baseline runs on."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    return {"cpu_model": model, "nproc": os.cpu_count() or 1, "usable_cpus": usable}


def c2_admitted(wv, cnt, K):
    """Edges admitted per group for one (source, row, direction) under the c2
    budget K (flashlog.cpp:12-89): groups with w > theta in full, ties at
    theta by a shared quota in group order."""
    import numpy as np
    elig = wv > 0
    take = np.where(elig, cnt, 0)
    if K <= 0 or take.sum() <= K:
        return take
    order = np.argsort(-wv, kind="stable")
    cum = np.cumsum(take[order])
    k = int(np.searchsorted(cum, K))
    theta = wv[order[k]]
    left = K - int(take[wv > theta].sum())
    out = np.where(wv > theta, cnt, 0)
    for g in np.nonzero(wv == theta)[0]:
        t = min(int(cnt[g]), max(left, 0))
        out[g] = t
        left -= t
    return out


def hop_pull_bytes(Ap, w, csr, R, K, out_bytes=8):
    """Algorithmic HBM bytes of one k_pull launch (the propagation kernel):
    the two graph outputs (8 B per state cell) plus, per direction and active
    source, its row pointers (8 B), group records (10 B each) and the column
    and mask of every edge admitted for at least one row (8 B each) -- the
    graph term of the dense hop's byte count.  The identity output and the
    read of A (8 B per cell) belong to k_col_count."""
    import numpy as np
    BL, E = Ap.shape
    nz = Ap != 0
    act = np.nonzero(nz.any(0))[0]
    total = out_bytes * BL * E
    for (gptr, grel, gcount, off) in ((csr[8], csr[9], csr[11], 0), (csr[12], csr[13], csr[15], R)):
        g0 = gptr[act].astype(np.int64)
        g1 = gptr[act + 1].astype(np.int64)
        total += 8 * act.size + 10 * int((g1 - g0).sum())
        for s, a, b in zip(act, g0, g1):
            if b == a:
                continue
            rows = np.nonzero(nz[:, s])[0]
            rel = grel[a:b].astype(np.int64) + off
            cnt = gcount[a:b].astype(np.int64)
            W = w[rows][:, rel]
            if K <= 0 or cnt.sum() <= K:
                e_hat = int(cnt[(W > 0).any(0)].sum())
            else:
                take = np.stack([c2_admitted(W[i], cnt, K) for i in range(W.shape[0])])
                e_hat = int(take.max(0).sum())
            total += 8 * e_hat
    return total


def main():
    args = parse()
    if args.pmc_summary:
        fetch_csv, write_csv, steps, out = args.pmc_summary
        return pmc_summary(fetch_csv, write_csv, int(steps), out, args.config)
    if args.stats_table:
        if len(args.stats_table) not in (4, 6):
            sys.exit("--stats-table takes OUT STATS_CSV TITLE RUN_COMMAND [TRACE_CSV FIRST_STEPS]")
        out, csv_path, title, run_command = args.stats_table[:4]
        trace, first_steps = (args.stats_table[4], int(args.stats_table[5])) if len(args.stats_table) == 6 else (None, 0)
        return stats_table(out, csv_path, title, run_command, trace_csv=trace, first_steps=first_steps)
    if args.counter_table:
        if len(args.counter_table) < 2:
            sys.exit("--counter-table needs OUT and at least one CSV")
        return counter_table(args.counter_table[0], args.counter_table[1:], args.config)
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(every (query, channel) row is independent, so batches would shard by query)",
              file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch
    from flashlog_amd import _lib, synth
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk

    if args.copy_mb > 0:
        copy_calibration(args.copy_mb)
    if args.grounding:
        return main_grounding(args)
    if args.rules:
        return main_rules(args)
    if args.sparse or args.config == 5:
        return main_sparse(args)
    if args.config == 4:
        return main_c4(args)
    cfg = synth.CONFIGS[args.config]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    h, r, t, E, R = synth.make_graph(args.config)
    n = 2 * R + 1
    B, L, T = cfg.batch, cfg.channels, cfg.hops
    K = cfg.c2 // 2 if cfg.use_topk else 0
    c1 = cfg.c1
    M = h.shape[0]
    th, tr, tt = (torch.from_numpy(a) for a in (h, r, t))
    csr = fk.build_csr_structure(th.to(dev), tt.to(dev), tr.to(dev), E)
    masks = fk.prepare_csr_masks(csr, torch.ones(M, dtype=torch.bool, device=dev))
    rng = np.random.Generator(np.random.PCG64(1234 + args.config))
    src, qrel, tgt = synth.make_queries(h, r, t, R, B, rng)
    W = torch.from_numpy(synth.make_attention(B, L, n, T, rng)).to(dev)
    x0 = torch.zeros(B, L, E, dtype=torch.float32, device=dev)
    x0[torch.arange(B, device=dev), :, torch.from_numpy(src).to(dev)] = 1.0

    def step(capture=None, flush=None):
        x = x0
        for hop in range(T):
            if flush is not None:
                flush()
            if capture is not None:
                capture.append((fk._dense_topc_state(x, c1 if cfg.use_topk else None), W[hop]))
            s_i, s_h, s_t = fk.dense_csr_sum_cuda(x, W[hop], csr, None, R, use_topk=cfg.use_topk,
                                                  topk_nodes=c1, topk_edges=K, prepared_masks=masks)
            s = s_i + s_h + s_t
            x = s / s.sum(dim=-1, keepdim=True).clamp(1e-7)
        return x.sum(dim=1)

    with torch.inference_mode():
        if args.counter_steps > 0:
            for _ in range(args.counter_steps):
                step()
            torch.cuda.synchronize()
            print("counter run: %d steps" % args.counter_steps, file=sys.stderr, flush=True)
            return
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(args.steps):
            out = step()
        e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms_step = e0.elapsed_time(e1) / args.steps
        print("timed %d steps: %.3f ms/step (host wall %.3f ms/step)" % (args.steps, ms_step, 1e3 * wall / args.steps),
              file=sys.stderr, flush=True)

        # per-kernel HIP-event timing inside the library
        kernels = ["k_topc_rows", "k_col_count", "k_frontier", "k_c2_hard", "k_pull", "k_heavy_offsets",
                   "k_heavy_copy", "k_fold_heavy"]
        per_launch = profile_pass(_lib, kernels, args.profile_steps, step)
        print("per-launch ms: " + json.dumps({k: round(v, 5) for k, v in per_launch.items()}),
              file=sys.stderr, flush=True)
        flush = cache_flusher()
        cold = profile_pass(_lib, kernels, args.profile_steps, lambda: step(flush=flush))
        print("per-launch ms, cold cache: " + json.dumps({k: round(v, 5) for k, v in cold.items()}),
              file=sys.stderr, flush=True)

        # algorithmic bytes of k_pull per hop, from the hop inputs of one step
        cap = []
        step(capture=cap)
        csr_np = [c.cpu().numpy() for c in csr]
        hop_bytes = [hop_pull_bytes(a.reshape(B * L, E).cpu().numpy(), w.reshape(B * L, n).cpu().numpy(),
                                    csr_np, R, K) for a, w in cap]
    bytes_per_launch = float(np.mean(hop_bytes))
    traffic = measured_traffic(["k_pull"], DENSE_TRAFFIC_FILES[2])
    traffic = traffic / T if traffic is not None else None  # per launch: T launches per step
    pull_ms = cold["k_pull"]
    achieved = bytes_per_launch / (pull_ms * 1e-3) / 1e9 if pull_ms > 0 else 0.0
    warm_ms = per_launch["k_pull"]
    warm = bytes_per_launch / (warm_ms * 1e-3) / 1e9 if warm_ms > 0 else 0.0

    cpu = cpu_baseline(args, cfg, h, r, t, E, R, src, W.cpu().numpy()) if args.cpu_seconds > 0 else None

    result = {
        "metric": "queries/sec for L=3 propagation + % of HBM roofline; top-k select ms",
        "value": B / (ms_step * 1e-3),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded %s graph, flashlog_amd/synth.py)" % cfg.name,
        "config": {"workload": "%s DRUM dense eval: E=%d, R=%d, M=%d, B=%d, N=%d, T=%d, c1=%d, c2=%d"
                   % (cfg.name, E, R, M, B, L, T, c1, cfg.c2),
                   "batch": B, "channels": L, "hops": T, "c1": c1, "c2": cfg.c2},
        "topk_select_ms": {"c1_per_hop": per_launch["k_topc_rows"], "c2_per_hop": per_launch["k_c2_hard"]},
        "kernel_ms_per_launch": per_launch,
        "kernel_ms_per_launch_cold": cold,
        "roofline": {"kernel": "k_pull", "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "algorithmic_bytes_per_launch": bytes_per_launch, "traffic": traffic, "ms": pull_ms,
                     "traffic_source": os.path.relpath(DENSE_TRAFFIC_FILES[2], ROOT) if traffic is not None else None,
                     "cache": "cold: %d MiB written before each hop" % FLUSH_MIB,
                     "warm": {"achieved": warm, "frac": warm / HBM_PEAK_GBS, "ms": warm_ms}},
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


def main_c4(args):
    """C4: mmDRUM on the dense GPU path, 123k
    entities, 37 relations, 1.08M triples with Zipf(1.2) hubs, batch 32,
    N = 3, T = 3, c1 = 1000, c2 = 400, forward and backward: per hop
    dense_csr_max, the elementwise max of its three outputs and the row
    normalization, then the max over channels (src/model_mmDRUM_kernel.py:
    101-126), the model's log loss (src/utils.py:28-34) and the backward
    pass to the attention.  Plus the evaluation's filtered ranking of 5,000
    queries over all entities (src/main.py:468-512) by
    dense_filtered_ranks_cuda, reported in "ranking"."""
    import numpy as np
    import torch
    from flashlog_amd import _lib, synth
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk

    cfg = synth.CONFIGS[4]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    h, r, t, E, R = synth.make_graph(4)
    n = 2 * R + 1
    B, L, T = cfg.batch, cfg.channels, cfg.hops
    K, c1 = cfg.c2 // 2, cfg.c1
    M = h.shape[0]
    csr = fk.build_csr_structure(*(torch.from_numpy(a).to(dev) for a in (h, t, r)), E)
    masks = fk.prepare_csr_masks(csr, torch.ones(M, dtype=torch.bool, device=dev))
    rng = np.random.Generator(np.random.PCG64(1234 + 4))
    src, qrel, tgt = synth.make_queries(h, r, t, R, B, rng)
    W = torch.from_numpy(synth.make_attention(B, L, n, T, rng)).to(dev).requires_grad_(True)
    x0 = torch.zeros(B, L, E, dtype=torch.float32, device=dev)
    x0[torch.arange(B, device=dev), :, torch.from_numpy(src).to(dev)] = 1.0
    tgt_t = torch.from_numpy(tgt).to(dev)

    def step(capture=None, flush=None):
        x = x0
        for hop in range(T):
            if flush is not None:
                flush()
            if capture is not None:
                capture.append((fk._dense_topc_state(x.detach(), c1), W[hop].detach()))
            s_i, s_h, s_t = fk.dense_csr_max(x, W[hop], csr, None, R, use_topk=True, topk_nodes=c1,
                                             topk_edges=K, prepared_masks=masks)
            s = torch.max(torch.stack([s_i, s_h, s_t], dim=0), dim=0).values
            x = s / s.sum(dim=-1, keepdim=True).clamp(1e-7)
        p = x.max(dim=1)[0]
        loss = -torch.log(torch.clamp(p[torch.arange(B, device=dev), tgt_t], min=1e-7)).mean()
        W.grad = None
        loss.backward()
        return loss

    kernels = ["k_topc_rows", "k_col_count", "k_frontier", "k_c2_hard", "k_pull_max", "k_seg_max", "k_sup_max",
               "k_heavy_max", "k_bwd_pairs_max", "k_bwd_identity", "k_row_count", "k_row_fill"]
    if args.counter_steps > 0:
        for _ in range(args.counter_steps):
            step()
        torch.cuda.synchronize()
        print("counter run: %d mmDRUM steps" % args.counter_steps, file=sys.stderr, flush=True)
        return
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps
    print("timed %d mmDRUM steps: %.3f ms/step" % (args.steps, ms_step), file=sys.stderr, flush=True)
    per_launch = profile_pass(_lib, kernels, max(args.profile_steps, 1), step)
    print("per-launch ms: " + json.dumps({k: round(v, 5) for k, v in per_launch.items()}), file=sys.stderr,
          flush=True)
    flush = cache_flusher()
    cold = profile_pass(_lib, kernels, max(args.profile_steps, 1), lambda: step(flush=flush))
    print("per-launch ms, cold cache: " + json.dumps({k: round(v, 5) for k, v in cold.items()}), file=sys.stderr,
          flush=True)
    cap = []
    step(capture=cap)
    csr_np = [c.cpu().numpy() for c in csr]
    # the max gather: k_pull_max (light destinations) + k_seg_max / k_sup_max / k_heavy_max (hubs);
    # outputs 24 B per (row, destination): two fp32 values and two int64 winning positions
    hop_bytes = [hop_pull_bytes(a.reshape(B * L, E).cpu().numpy(), w.reshape(B * L, n).cpu().numpy(), csr_np, R, K,
                                out_bytes=24) for a, w in cap]
    gather = ("k_pull_max", "k_seg_max", "k_sup_max", "k_heavy_max")
    gather_ms = sum(cold[k] for k in gather)
    warm_ms = sum(per_launch[k] for k in gather)
    bytes_per_hop = float(np.mean(hop_bytes))
    traffic = measured_traffic(list(gather), DENSE_TRAFFIC_FILES[4])
    traffic = traffic / T if traffic is not None else None  # per hop: T hops per step
    achieved = bytes_per_hop / (gather_ms * 1e-3) / 1e9 if gather_ms > 0 else 0.0
    warm = bytes_per_hop / (warm_ms * 1e-3) / 1e9 if warm_ms > 0 else 0.0

    # filtered ranking: 5,000 queries over all entities; filter = each query's known answers + target
    QN = 5000
    qrng = np.random.Generator(np.random.PCG64(4321))
    scores = (qrng.integers(0, 1 << 12, (QN, E)) / float(1 << 12)).astype(np.float32)  # ties on purpose
    qt = qrng.integers(0, E, QN)
    nf = 20 * QN
    fb, fe = qrng.integers(0, QN, nf), qrng.integers(0, E, nf)
    st_d = torch.from_numpy(scores).to(dev)
    qt_d = torch.from_numpy(qt).to(dev)
    fidx = (torch.from_numpy(fb).to(dev), torch.from_numpy(fe).to(dev))
    for _ in range(2):
        fk.dense_filtered_ranks_cuda(st_d, qt_d, fidx, True)
    torch.cuda.synchronize()
    _lib.prof_enable(True)
    r0, r1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    r0.record()
    for _ in range(10):
        fk.dense_filtered_ranks_cuda(st_d, qt_d, fidx, True)
    r1.record()
    torch.cuda.synchronize()
    rk = _lib.prof_read("k_dense_rank")
    _lib.prof_enable(False)
    rank_ms = r0.elapsed_time(r1) / 10
    rank_kernel_ms = rk[0] / rk[1] if rk[1] else 0.0
    rank_bytes = 4.0 * QN * E + 8.0 * QN + 16.0 * (nf + QN)
    cpu_rank = None
    if args.cpu_seconds > 0:
        from oracle import oracle as O
        Qs = 500
        t0 = time.perf_counter()
        reps = 0
        while True:
            O.dense_filtered_ranks(scores[:Qs], qt[:Qs], fb[fb < Qs], fe[fb < Qs], True)
            reps += 1
            if time.perf_counter() - t0 >= min(args.cpu_seconds, 5.0):
                break
        el = time.perf_counter() - t0
        cpu_rank = {**host_cpu(), "value": reps * Qs / el, "unit": "queries/s", "cores": 1, "kind": "port",
                    "sample": "%d rankings of %d queries over %d entities (numpy restatement of src/main.py:468-512)"
                              % (reps, Qs, E)}
    cpu = cpu_baseline_c4(args, cap, csr_np, B, L, E, R, K) if args.cpu_seconds > 0 else None
    result = {
        "metric": "queries/sec for L=3 propagation + % of HBM roofline; top-k select ms",
        "value": B / (ms_step * 1e-3),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded C4 graph, flashlog_amd/synth.py; random attention in place of the model's LSTM)",
        "config": {"workload": "C4 mmDRUM dense max step (forward + backward): E=%d, R=%d, M=%d, B=%d, N=%d, T=%d, "
                               "c1=%d, c2=%d" % (E, R, M, B, L, T, c1, cfg.c2),
                   "batch": B, "channels": L, "hops": T, "c1": c1, "c2": cfg.c2},
        "topk_select_ms": {"c1_per_hop": per_launch["k_topc_rows"], "c2_per_hop": per_launch["k_c2_hard"]},
        "kernel_ms_per_launch": per_launch,
        "kernel_ms_per_launch_cold": cold,
        "roofline": {"kernel": "k_pull_max+k_seg_max+k_sup_max+k_heavy_max", "bound": "hbm", "achieved": achieved,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "algorithmic_bytes_per_launch": bytes_per_hop, "traffic": traffic, "ms": gather_ms,
                     "traffic_source": os.path.relpath(DENSE_TRAFFIC_FILES[4], ROOT) if traffic is not None else None,
                     "cache": "cold: %d MiB written before each hop" % FLUSH_MIB,
                     "warm": {"achieved": warm, "frac": warm / HBM_PEAK_GBS, "ms": warm_ms}},
        "cpu_baseline": cpu,
        "ranking": {"queries": QN, "entities": E, "filter_entries": nf, "ms": rank_ms,
                    "queries_per_s": QN / (rank_ms * 1e-3),
                    "roofline": {"kernel": "k_dense_rank", "bound": "hbm",
                                 "achieved": rank_bytes / (rank_kernel_ms * 1e-3) / 1e9 if rank_kernel_ms else 0.0,
                                 "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                 "frac": rank_bytes / (rank_kernel_ms * 1e-3) / 1e9 / HBM_PEAK_GBS
                                 if rank_kernel_ms else 0.0,
                                 "algorithmic_bytes_per_launch": rank_bytes},
                    "cpu_baseline": cpu_rank},
    }
    print(json.dumps(result), flush=True)


def cpu_baseline_c4(args, cap, csr_np, B, L, E, R, K):
    """mmDRUM's dense max has no CPU path in the reference (GPU only,
    flashlog_kernel.py:1666-1688), so the CPU figure is the C restatement of
    the op (oracle: or_dense_max_forward / or_dense_max_backward, one thread)
    forward and backward on each hop's pruned input for the first Bs queries
    (rows are independent); the model's elementwise ops are not included."""
    import numpy as np
    from oracle import oracle as O
    n = 2 * R + 1
    Bs = min(4, B)
    ones = (np.ones(csr_np[1].shape[0], np.float32), np.ones(csr_np[5].shape[0], np.float32))
    hops = [(a.reshape(B * L, E)[:Bs * L].cpu().numpy(), w.reshape(B * L, n)[:Bs * L].cpu().numpy())
            for a, w in cap]
    g = np.ones((Bs * L, E), np.float32)
    t0 = time.perf_counter()
    reps = 0
    while True:
        for A, w in hops:
            o = O.dense_max_forward(A, w, csr_np, ones, R, False, K)
            O.dense_max_backward(g, g, g, o[3], o[4], A, w, csr_np, ones, R, False, K)
        reps += 1
        if time.perf_counter() - t0 >= args.cpu_seconds:
            break
    el = time.perf_counter() - t0
    return {**host_cpu(), "value": reps * Bs / el, "unit": "queries/s", "cores": 1, "kind": "port",
            "sample": "%d x %d hops forward + backward of the dense max op for %d queries (oracle C restatement; "
                      "the reference has no CPU max path) in %.1f s, 1 thread" % (reps, len(hops), Bs, el)}


def main_grounding(args):
    """Soft grounding (ground_head_batch_source_folds_sampled_capped_counts,
    soft_grounding.cpp:898-1027) with the reference extraction's defaults
    (rules/extract.py:385-427): a batch of 16 head relations, one fold of up
    to 512 sources per head from sample_relation_sources_reservoir, 4096
    walks per source, top-k 200 edges (c2 = 400), temperature 1, length caps
    [64, 4096, 16384], seeds seed ^ (head * 0x9E3779B1); on the C3 graph
    (14.5k entities, 237 relations, 272k triples) with random attention.
    value = walks per second over the whole call (walks, counting and the
    candidate rows returned on the host, as the reference returns them)."""
    import numpy as np
    import torch
    from flashlog_amd import _lib, synth
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    from flashlog_amd.flashlog_kernel.soft_grounding_kernel import soft_grounding_kernel as sg

    cfg = synth.CONFIGS[3]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    h, r, t, E, R = synth.make_graph(3)
    V = 2 * R + 1
    csr = fk.build_csr_structure(*(torch.from_numpy(a) for a in (h, t, r)), E)
    csr = tuple(c.cpu() for c in csr)
    rng = np.random.Generator(np.random.PCG64(1234 + 3))
    NH, SPF, WALKS, TOPK, CAPS, SEED = 16, 512, 4096, 200, [64, 4096, 16384], 1234
    heads = [int(x) for x in rng.choice(2 * R, NH, replace=False)]
    rels = np.array(sorted(set(hd % R for hd in heads)), np.int64)
    # sources of a head: the reservoir of rows holding a group of its relation (inverse heads use the INV side)
    picked = {}
    for side, (gptr, grel) in enumerate(((csr[8], csr[9]), (csr[12], csr[13]))):
        out, _ = sg.sample_relation_sources_reservoir(gptr, grel, torch.from_numpy(rels), SPF, SEED)
        for i, rel in enumerate(rels):
            picked[(side, int(rel))] = [int(x) for x in out[i].tolist() if x >= 0]
    folds = [[np.array(picked[(hd // R, hd % R)] or [0], np.int64)] for hd in heads]
    logits = rng.standard_normal((NH, 3, 3, V)).astype(np.float32)
    att = np.exp(logits - logits.max(-1, keepdims=True))
    att = (att / att.sum(-1, keepdims=True)).astype(np.float32)
    seeds = [SEED ^ (hd * 0x9E3779B1) for hd in heads]
    walks_total = sum(len(f[0]) for f in folds) * WALKS
    att_t = torch.from_numpy(att)

    def call():
        return sg.ground_head_batch_source_folds_sampled_capped_counts(att_t, heads, R, folds, csr, WALKS, TOPK, False,
                                                                       seeds, 500000, 16, CAPS)

    for _ in range(max(args.warmup, 1)):
        call()
    torch.cuda.synchronize()
    reps = max(1, min(args.steps, 10))
    _lib.prof_enable(True)
    t0 = time.perf_counter()
    for _ in range(reps):
        cands, raw, _ = call()
    torch.cuda.synchronize()
    el = (time.perf_counter() - t0) / reps
    kn = ["k_gr_hubs", "k_gr_walk", "k_ct_flags", "k_ct_accum", "k_ct_capkey", "k_ct_keep", "k_ct_gather", "k_ct_emit"]
    prof = {k: _lib.prof_read(k) for k in kn}
    _lib.prof_enable(False)
    per_call = {k: v[0] / reps for k, v in prof.items()}
    print("grounding: %.1f ms per call, %d walks; kernel ms per call %s"
          % (el * 1e3, walks_total, json.dumps({k: round(v, 3) for k, v in per_call.items()})),
          file=sys.stderr, flush=True)
    cpu = None
    if args.cpu_seconds > 0:
        sys.path.insert(0, os.path.join(ROOT, "oracle", "_ref"))
        try:
            import flashlog_grounding_ref as ref
        except ImportError:
            ref = None
        if ref is not None:
            threads = min(16, os.cpu_count() or 1)
            nh = 2  # bounded sample: the first heads of the batch
            tens = [csr[i] for i in (1, 5, 8, 9, 10, 11, 12, 13, 14, 15)]
            tf = [[torch.from_numpy(f[0])] for f in folds[:nh]]
            t1 = time.perf_counter()
            n = 0
            while True:
                ref.ground_head_batch_source_folds_sampled_capped_counts(
                    att_t[:nh].contiguous(), heads[:nh], R, tf, *tens, WALKS, TOPK, False, seeds[:nh], 500000,
                    threads, CAPS)
                n += 1
                if time.perf_counter() - t1 >= args.cpu_seconds:
                    break
            cel = time.perf_counter() - t1
            cwalks = sum(len(f[0]) for f in folds[:nh]) * WALKS
            cpu = {**host_cpu(), "value": n * cwalks / cel, "unit": "walks/s", "cores": threads, "kind": "reference",
                   "sample": "%d calls of %d heads x %d walks (soft_grounding.cpp built in oracle/_ref, OpenMP) in "
                             "%.1f s, %d threads" % (n, nh, cwalks, cel, threads)}
    result = {
        "metric": "soft grounding walks/sec (rule extraction sampler)",
        "value": walks_total / el,
        "unit": "walks/s",
        "n_gpus": 1,
        "steps": reps,
        "warmup": max(args.warmup, 1),
        "ms_per_step": el * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64/f64 (mt19937_64, double masses)",
        "data": "synthetic (seeded C3 graph, flashlog_amd/synth.py; random attention)",
        "config": {"workload": "soft grounding, C3 graph: %d heads x <=%d sources x %d walks, top-k %d, caps %s"
                               % (NH, SPF, WALKS, TOPK, CAPS)},
        "kernel_ms_per_call": per_call,
        "roofline": None,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


def main_rules(args):
    """Rule-bank scoring (rules/shared_inference.py:12-245, called once per head
    relation by rules/evaluate.py:521-527) on BASELINE configs[2] (C3: 14.5k
    entities, 237 relations, 272k triples): 20k random rules with bodies of
    1-3 directed relations and uniform(0, 1) weights for 3 ranks, spread over
    the directed head relations; 5k (source, head) queries, each head's
    sources scored against its rules (sum reduction, paths counted, chunks of
    64 rules).  value = queries/s over the whole pass."""
    import numpy as np
    import torch
    from flashlog_amd import _lib, synth
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk
    from flashlog_amd.rules import shared_inference
    sys.path.insert(0, ROOT)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    h, r, t, E, R = synth.make_graph(3)
    csr = fk.build_csr_structure(*(torch.from_numpy(a).to(dev) for a in (h, t, r)), E)
    rng = np.random.Generator(np.random.PCG64(1234 + 33))
    NR, NQ, RANKS, CHUNK = 20000, 5000, 3, 64
    rule_head = rng.integers(0, 2 * R, NR)
    bodies = [[int(x) for x in rng.integers(0, 2 * R, int(rng.integers(1, 4)))] for _ in range(NR)]
    weights = rng.random((NR, RANKS)).astype(np.float32)
    by_head = {}
    for k in range(NR):
        by_head.setdefault(int(rule_head[k]), []).append(k)
    heads = np.array(sorted(by_head), np.int64)
    q_head = rng.choice(heads, NQ)
    q_src = h[rng.integers(0, h.shape[0], NQ)]
    groups = []
    for hd in np.unique(q_head):
        ks = by_head[int(hd)]
        rules = [{"body": bodies[k], "rank_weights": [float(x) for x in weights[k]]} for k in ks]
        srcs = torch.from_numpy(q_src[q_head == hd].astype(np.int64)).to(dev)
        groups.append((int(hd), srcs, rules, ks))

    def run():
        return [shared_inference.score(None, srcs, rules, csr, R, E, CHUNK) for _, srcs, rules, _ in groups]

    for _ in range(max(args.warmup, 1)):
        run()
    torch.cuda.synchronize()
    reps = max(1, min(args.steps, 5))
    t0 = time.perf_counter()
    for _ in range(reps):
        run()
    torch.cuda.synchronize()
    el = (time.perf_counter() - t0) / reps
    # kernel times (HIP events around each launch) and the steps' sizes, one more pass
    _lib.prof_enable(True)
    fk.plan_log = []
    run()
    torch.cuda.synchronize()
    plans = fk.plan_log
    fk.plan_log = None
    prof = {k: _lib.prof_read(k) for k in RULE_STEP_KERNELS + RULE_ACC_KERNELS}
    _lib.prof_enable(False)
    per_pass = {k: v[0] for k, v in prof.items()}
    step_ms = sum(per_pass[k] for k in RULE_STEP_KERNELS)
    step_bytes = float(sum(rule_step_bytes(p) for p in plans))
    achieved = step_bytes / (step_ms * 1e-3) / 1e9 if step_ms > 0 else 0.0
    dominant = max(per_pass, key=lambda k: per_pass[k])
    print("rules: %.1f ms per pass of %d queries x %d rules (%d heads), %d grounding steps; kernel ms per pass %s"
          % (el * 1e3, NQ, NR, len(groups), len(plans), json.dumps({k: round(v, 3) for k, v in per_pass.items()})),
          file=sys.stderr, flush=True)
    cpu = None
    if args.cpu_seconds > 0:
        from oracle import oracle as O
        t1 = time.perf_counter()
        nq = 0
        for hd, srcs, rules, ks in groups:
            O.rule_scores(h, r, t, E, R, [int(x) for x in srcs.cpu().tolist()], [bodies[k] for k in ks],
                          weights[ks].astype(np.float64), "sum", False, False)
            nq += srcs.numel()
            if time.perf_counter() - t1 > args.cpu_seconds:
                break
        dt = time.perf_counter() - t1
        cpu = {**host_cpu(), "value": nq / dt, "unit": "queries/s", "cores": 1, "kind": "port",
               "sample": "%d queries of the first heads (the oracle's float64 path enumeration, numpy, "
                         "1 thread; the reference's scorer is GPU-only Python) in %.1f s" % (nq, dt)}
    result = {
        "metric": "rule-bank scoring queries/sec (rules/shared_inference.score)",
        "value": NQ / el, "unit": "queries/s", "n_gpus": 1, "steps": reps, "warmup": max(args.warmup, 1),
        "ms_per_step": el * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic (seeded C3 graph, flashlog_amd/synth.py; random rules and queries)",
        "config": {"workload": "C3 rule-bank scoring: %d rules (1-3 relations, %d ranks) over %d (source, head) "
                               "queries, %d heads, chunks of %d rules" % (NR, RANKS, NQ, len(groups), CHUNK)},
        "kernel_ms_per_pass": per_pass,
        "kernel_ms_total": sum(per_pass.values()),
        "roofline": {"kernel": "fixed-relation rule steps (their kernels, per pass)", "bound": "hbm",
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "algorithmic_bytes_per_launch": step_bytes, "ms_per_launch": step_ms, "traffic": None,
                     "steps_per_pass": len(plans)},
        "dominant_kernel": {"name": dominant, "ms_per_pass": per_pass[dominant]},
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


# The fixed-relation rule step's kernels (the sparse pipeline's mode 2) and the
# rule bank's accumulation kernels.
RULE_STEP_KERNELS = ["k_fx_count", "k_fx_fill", "k_sp_rowptr", "k_sp_rowinfo", "k_sp_hist", "k_sp_vscan",
                     "k_sp_partition", "k_sp_accum_small", "k_sp_accum_few", "k_sp_accum_mid", "k_sp_accum_hot",
                     "k_sp_emit", "k_scan_tiles", "k_scan_totals", "k_scan_apply", "k_scan_one", "k_fill_i32",
                     "k_fill_i64", "k_sp_plan_out"]
RULE_ACC_KERNELS = ["k_ra_rows", "k_ra_sum", "k_cs_rank", "k_cs_weighted_add", "k_rule_accum_max", "k_rule_rowsum",
                    "k_rule_combine"]


def rule_step_bytes(plan):
    """Algorithmic bytes of one fixed-relation rule step by the measurement
    plan's formula: 28 nnz_in (entries) + 8 per row (its operator) + per
    entry 8 B of row group pointers, 2 ceil(log2 g) B of group relations
    searched and 8 B of group start and count + 4 B per item (its column) +
    28 nnz_out; g is taken as the entries' mean groups per side."""
    import math
    nnz, items, nout, rows = plan["nnz"], plan["items"], plan["nout"], plan["rows"]
    g = plan["groups"] / max(2 * nnz, 1)
    lg = math.ceil(math.log2(g)) if g > 1 else 0
    return 28 * nnz + 8 * rows + nnz * (16 + 2 * lg) + 4 * items + 28 * nout


SPARSE_KERNELS = ["k_sp_topc", "k_race_flags", "k_race_keys", "k_race_rows", "k_race_select", "k_fill_from",
                  "k_sp_rowptr", "k_sp_relorder", "k_sp_select", "k_sp_rowinfo", "k_sp_runs", "k_sp_items",
                  "k_sp_expand_fused",
                  "k_sp_hist",
                  "k_sp_partition", "k_sp_accum_small", "k_sp_accum_few", "k_sp_accum_mid", "k_sp_accum_hot", "k_sp_emit", "k_sp_local_to_out",
                  "k_norm_fwd", "k_norm_bwd", "k_sp_bwd", "k_fill_f32", "k_scan_tiles", "k_scan_totals",
                  "k_scan_apply", "k_scan_one", "k_sp_vscan", "k_fill_i32", "k_fill_i64", "k_sp_plan_out", "k_apply_mask",
                  "k_sp_ord_count", "k_sp_ord_place", "k_sp_rowptr_search", "k_sp_order_count", "k_sp_order_check", "k_sp_gather_nch",
                  "k_sp_finite", "k_sp_bw_chunks", "k_sp_gw_fin",
                  "k_cs_rank", "k_cs_emit", "k_pack_bool_bits", "k_order_bits"]


# The sparse hop's own kernels (forward and backward), without the c1 entity
# selection, the normalizer and the channel sums that surround it in a step.
HOP_EXCLUDE = ("k_sp_topc", "k_race_flags", "k_race_keys", "k_race_rows", "k_race_select", "k_fill_from",
               "k_norm_fwd", "k_norm_bwd", "k_cs_rank", "k_cs_emit")
HOP_KERNELS = [k for k in SPARSE_KERNELS if k not in HOP_EXCLUDE]


def sparse_hop_bytes(plan):
    """Algorithmic bytes of one sparse sum hop, forward and (with a backward)
    backward, by the sparse formulas of the measurement plan:
      forward  28 nnz_in + 4 BL n + sum over sides and entries (8 + 10 g(src)
               + 9 kept) + 28 nnz_out
      backward 28 nnz_in + 4 nnz_out + 8 BL n + sum (8 + 10 g + 13 kept)
               + 4 nnz_in
    with nnz_in the entries after c1, g the source's groups on a side and
    kept its kept edges (the raw items less the identity items)."""
    nnz, rows, n, nout, groups = plan["nnz"], plan["rows"], plan["n"], plan["nout"], plan["groups"]
    kept = plan["items"] - (0 if plan["wot_i"] else nnz)
    fwd = 28 * nnz + 4 * rows * n + 16 * nnz + 10 * groups + 9 * kept + 28 * nout
    if not plan["backward"]:
        return fwd
    bwd = 28 * nnz + 4 * nout + 8 * rows * n + 16 * nnz + 10 * groups + 13 * kept + 4 * nnz
    return fwd + bwd


def item_kernel_bytes(plans):
    """Algorithmic bytes per step of the kernels whose work is linear in the
    entries' group records and raw items, summed over the step's hops
    (k_sp_select reads each entry's coordinates, 24 B, and per side its
    group range, 8 B, and every group record once, 10 B, and writes the
    entry's counts, thresholds and cuts, 24 B; k_sp_expand_fused reads each
    entry's coordinates, value and item range, 36 B, per side the group
    range and the threshold and cut, 16 B, every group record, 10 B, and per
    kept item its CSR column, 4 B, and writes every raw item's destination
    and value, 8 B, + 2 B of attention column with a backward; per raw item: k_sp_items reads
    the column and mask and writes the destination and value, 16 B, + 6 B of
    CSR position and attention column with a backward; k_sp_hist reads the
    destination, 4 B; k_sp_partition reads destination and value and writes
    them in bucket order, 16 B, + 4 B of the item's bucket position with a
    backward; k_sp_local_to_out reads that position (which carries the
    item's bucket) and the bucket-order output index and writes the
    raw-order one, 12 B;
    k_sp_bwd reads CSR position, column and output index and the output's
    gradient, 14 B)."""
    out = {"k_sp_select": 0, "k_sp_expand_fused": 0, "k_sp_items": 0, "k_sp_hist": 0, "k_sp_partition": 0,
           "k_sp_local_to_out": 0, "k_sp_bwd": 0}
    for p in plans:
        it, bw = p["items"], p["backward"]
        kept = it - (0 if p["wot_i"] else p["nnz"])
        out["k_sp_select"] += (24 + 2 * 8 + 24) * p["nnz"] + 10 * p["groups"]
        out["k_sp_expand_fused"] += (36 + 2 * 16) * p["nnz"] + 10 * p["groups"] + 4 * kept + (8 + (2 if bw else 0)) * it
        out["k_sp_items"] += (16 + (6 if bw else 0)) * it
        out["k_sp_hist"] += 4 * it
        out["k_sp_partition"] += (16 + (4 if bw else 0)) * it
        if bw:
            out["k_sp_local_to_out"] += 12 * it
            out["k_sp_bwd"] += 14 * it
    return out


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "sparse_hop_c5_train_traffic_per_step.txt")
DENSE_TRAFFIC_FILES = {2: os.path.join(ROOT, "profiles", "dense_hop_c2_traffic_per_step.txt"),
                       4: os.path.join(ROOT, "profiles", "dense_max_c4_traffic_per_step.txt")}


def measured_traffic(kernels, path=None):
    """HBM bytes per step of the given kernels from a committed counter
    summary (lines "<kernel> <MB per step> ..."; by default the C5 one), or
    None when it is absent."""
    path = path or TRAFFIC_FILE
    if not os.path.exists(path):
        return None
    mb = {}
    for line in open(path):
        parts = line.split()
        if len(parts) >= 2 and parts[0].startswith("k_"):
            try:
                mb[parts[0]] = float(parts[1])
            except ValueError:
                pass
    if not mb:
        return None
    return sum(mb.get(k, 0.0) for k in kernels) * 1e6


def main_sparse(args):
    """C5: DRUM --sparse on one GPU, T = 3 hops of
    the sparse sum hop (c1 = 1000 entities, c2 = 400 edges), each followed by
    normalize_sparse3d, from one-hot query states, then the sum over the
    channels (src/model_DRUM_kernel_sp.py:124-205).
      train (default): the training step of that model -- each hop is
      sampled_sparse_propagation (exponential-race c1, quota c2), then the
      model's log loss on the target entity (src/utils.py:37-47) and the
      backward pass to the per-hop attention;
      eval: FlashLogFunctionSparse3DTopKSum with the c1/c2 thresholds, no
      gradients."""
    import numpy as np
    import torch
    from flashlog_amd import _lib, synth
    from flashlog_amd.flashlog_kernel import flashlog_kernel as fk

    cfg = synth.CONFIGS[args.config]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    train = args.mode == "train"
    t_gen = time.perf_counter()
    h, r, t, E, R = synth.make_graph(args.config)
    n = 2 * R + 1
    B, L, T = cfg.batch, cfg.channels, cfg.hops
    K = cfg.c2 // 2
    c1 = cfg.c1
    M = h.shape[0]
    th, tr, tt = (torch.from_numpy(a) for a in (h, r, t))
    csr = fk.build_csr_structure(th.to(dev), tt.to(dev), tr.to(dev), E)
    mask_values = torch.ones(M, dtype=torch.bool, device=dev)
    rng = np.random.Generator(np.random.PCG64(1234 + args.config))
    src, qrel, tgt, qidx = synth.make_queries(h, r, t, R, B, rng, return_index=True)
    W = torch.from_numpy(synth.make_attention(B, L, n, T, rng)).to(dev)
    print("graph %s: E=%d M=%d (%.1f s to generate)" % (cfg.name, E, M, time.perf_counter() - t_gen),
          file=sys.stderr, flush=True)
    # the reference's own training batch: --batch_size 256 propagates each
    # triple forward and inverse (src/dataloader.py:114-122), 2B queries
    src2, _, tgt2 = synth.training_queries(h, r, t, R, qidx)
    W2 = torch.from_numpy(synth.make_attention(2 * B, L, n, T, np.random.Generator(np.random.PCG64(4321 + args.config)))).to(dev)

    def workload(q_src, q_tgt, Wq):
        nb = q_src.shape[0]
        b0 = torch.arange(nb, device=dev).repeat_interleave(L)
        l0 = torch.arange(L, device=dev).repeat(nb)
        e0 = torch.from_numpy(q_src).to(dev).repeat_interleave(L)
        v0 = torch.ones(nb * L, device=dev)
        state0 = torch.sparse_coo_tensor(torch.stack([b0, l0, e0]), v0, [nb, L, E]).coalesce()
        return nb, state0, Wq.clone().requires_grad_(train), torch.from_numpy(q_tgt).to(dev)

    work = [workload(src, tgt, W)]
    batch_edges = torch.from_numpy(qidx).to(dev)

    def hop(s, w):
        if train:
            return fk.sampled_sparse_propagation(s, w, csr, mask_values, R, None, False, c1, K, "sum")
        idx = s.indices()
        nb = s.shape[0]
        return fk.FlashLogFunctionSparse3DTopKSum.apply(
            idx[0], idx[1], idx[2], s.values(), w, *csr[:4], *csr[4:8], *csr[8:16], mask_values, None,
            nb, L, E, R, False, K, False, c1, False)

    def model_sum_sp_3d(s):
        # the model file's own channel sum (src/model_DRUM_kernel_sp.py:22-28): torch's coalesce
        s = s.coalesce()
        idx = s.indices()
        return torch.sparse_coo_tensor(torch.stack([idx[0], idx[2]], dim=0), s.values(),
                                       [s.shape[0], s.shape[2]]).coalesce()

    def log_loss_common_sp(p_score, label):
        # src/utils.py:37-47 (tau_2 = 1): the target's score through a sparse one-hot product
        i = torch.stack([torch.arange(label.shape[0], device=dev), label])
        one_hot = torch.sparse_coo_tensor(i, torch.ones(label.shape[0], device=dev), [label.shape[0], E])
        logits = torch.sparse.sum(p_score * one_hot, dim=-1).to_dense()
        return -torch.mean(torch.log(torch.maximum(logits, torch.ones_like(logits) * 1e-7)), dim=-1)

    native_sum = [False]

    def step(flush=None):
        # src/main.py:887-890: the batch's triples are hidden from the graph
        # for the step (the mask is updated in place), restored after it (:927-930);
        # src/model_DRUM_kernel_sp.py:132-205 per hop: the hop, normalize_sparse3d, dropout
        _, state0, Wl, tgt_t = work[0]
        if train:
            mask_values[batch_edges] = False
        s = state0
        for t_ in range(T):
            if flush is not None:
                flush()
            s = fk.normalize_sparse3d(hop(s, Wl[t_]))
            if train:
                s = torch.sparse_coo_tensor(s.indices(), torch.nn.functional.dropout(s.values(), 0.1, True),
                                            s.shape, is_coalesced=True)
        final = fk.sum_sp_3d(s) if native_sum[0] else model_sum_sp_3d(s)
        if not train:
            return final
        loss = log_loss_common_sp(final, tgt_t)
        Wl.grad = None
        loss.backward()
        mask_values[batch_edges] = True
        return loss

    ctx = torch.enable_grad() if train else torch.inference_mode()
    if args.counter_steps > 0:
        with ctx:
            for _ in range(args.counter_steps):
                step()
            torch.cuda.synchronize()
        print("counter run: %d %s steps" % (args.counter_steps, args.mode), file=sys.stderr, flush=True)
        return
    with ctx:
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        e_0 = torch.cuda.Event(enable_timing=True)
        e_1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e_0.record()
        for _ in range(args.steps):
            step()
        e_1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms_step = e_0.elapsed_time(e_1) / args.steps
        print("timed %d %s steps: %.3f ms/step (host wall %.3f ms/step)"
              % (args.steps, args.mode, ms_step, 1e3 * wall / args.steps), file=sys.stderr, flush=True)
        # the same steps with this library's channel sum (flashlog_kernel.sum_sp_3d) in place of
        # the model file's torch coalesce: what a model that imports it would run
        native_sum[0] = True
        for _ in range(2):
            step()
        torch.cuda.synchronize()
        e_0.record()
        for _ in range(args.steps):
            step()
        e_1.record()
        torch.cuda.synchronize()
        ms_step_native = e_0.elapsed_time(e_1) / args.steps
        native_sum[0] = False
        print("with flashlog_kernel.sum_sp_3d: %.3f ms/step" % ms_step_native, file=sys.stderr, flush=True)
        _lib.prof_enable(True)
        for _ in range(args.profile_steps):
            step()
        torch.cuda.synchronize()
        prof = {k: _lib.prof_read(k) for k in SPARSE_KERNELS}
        _lib.prof_enable(False)
        per_launch = {k: (v[0] / v[1] if v[1] else 0.0) for k, v in prof.items()}
        per_step = {k: (v[0] / max(args.profile_steps, 1)) for k, v in prof.items()}
        # the same steps with the caches flushed before each hop
        flush = cache_flusher()
        _lib.prof_enable(True)
        for _ in range(args.profile_steps):
            step(flush=flush)
        torch.cuda.synchronize()
        prof_cold = {k: _lib.prof_read(k) for k in SPARSE_KERNELS}
        _lib.prof_enable(False)
        del flush
        cold_step = {k: (v[0] / max(args.profile_steps, 1)) for k, v in prof_cold.items()}
        print("per-launch ms: " + json.dumps({k: round(v, 4) for k, v in per_launch.items()}),
              file=sys.stderr, flush=True)
        print("per-step ms: " + json.dumps({k: round(v, 4) for k, v in per_step.items()}),
              file=sys.stderr, flush=True)
        # plan sizes of one step's hops, for the algorithmic bytes of k_sp_items
        fk.plan_log = []
        step()
        torch.cuda.synchronize()
        plans = fk.plan_log
        fk.plan_log = None
        # the reference's training batch for --batch_size 256: 2B queries (each
        # triple forward and inverse), the same step otherwise; run last, so
        # that in a kernel trace the default batch's launches come first
        ref_batch = None
        if train:
            work.insert(0, workload(src2, tgt2, W2))
            for _ in range(2):
                step()
            torch.cuda.synchronize()
            e_0.record()
            for _ in range(args.steps):
                step()
            e_1.record()
            torch.cuda.synchronize()
            ms_step_2b = e_0.elapsed_time(e_1) / args.steps
            work.pop(0)
            ref_batch = {"queries_per_step": 2 * B, "ms_per_step": ms_step_2b,
                         "value": 2 * B / (ms_step_2b * 1e-3), "unit": "queries/s",
                         "what": "the same training step on the %d queries the reference propagates for "
                                 "--batch_size %d (each batch triple forward and inverse, "
                                 "src/dataloader.py:114-122)" % (2 * B, B)}
            print("reference batch (%d queries): %.3f ms/step" % (2 * B, ms_step_2b), file=sys.stderr, flush=True)
    csr_np = [c.cpu().numpy() for c in csr]
    cpu = (cpu_baseline_sparse(args, csr_np, L, E, R, K, c1, src, tgt, W.cpu(), T, train)
           if args.cpu_seconds > 0 else None)
    # roofline of the whole hop: the hop formula's bytes of the step's hops over
    # the live time of the hop's kernels (HIP events around each launch)
    step_bytes = float(sum(sparse_hop_bytes(p) for p in plans))
    hop_ms = sum(cold_step[k] for k in HOP_KERNELS)
    achieved = step_bytes / (hop_ms * 1e-3) / 1e9 if hop_ms > 0 else 0.0
    warm_ms = sum(per_step[k] for k in HOP_KERNELS)
    warm = step_bytes / (warm_ms * 1e-3) / 1e9 if warm_ms > 0 else 0.0
    # the committed counter summary is of the training step: no figure for eval
    traffic = measured_traffic(HOP_KERNELS) if train else None
    kernel_rooflines = {}
    for k, b in item_kernel_bytes(plans).items():
        if cold_step.get(k, 0.0) > 0 and per_step.get(k, 0.0) > 0 and b > 0:
            a = b / (cold_step[k] * 1e-3) / 1e9
            aw = b / (per_step[k] * 1e-3) / 1e9
            kernel_rooflines[k] = {"achieved": a, "frac": a / HBM_PEAK_GBS, "algorithmic_bytes_per_step": b,
                                   "ms_per_step": cold_step[k], "traffic": measured_traffic([k]) if train else None,
                                   "warm": {"achieved": aw, "frac": aw / HBM_PEAK_GBS, "ms_per_step": per_step[k]}}
    dominant = max(per_step, key=lambda k: per_step[k])
    result = {
        "metric": "queries/sec for L=3 propagation + % of HBM roofline; top-k select ms",
        "value": B / (ms_step * 1e-3),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded %s graph, flashlog_amd/synth.py; random attention in place of the "
                "model's LSTM)" % cfg.name,
        "config": {"workload": "%s DRUM --sparse %s step (%s): E=%d, R=%d, M=%d, B=%d, N=%d, T=%d, c1=%d, c2=%d"
                   % (cfg.name, args.mode, "forward + backward" if train else "forward", E, R, M, B, L, T,
                      c1, cfg.c2),
                   "batch": B, "channels": L, "hops": T, "c1": c1, "c2": cfg.c2, "mode": args.mode},
        "channel_sum": "the model file's torch sum_sp_3d (src/model_DRUM_kernel_sp.py:22-28)",
        "ms_per_step_native_channel_sum": ms_step_native,
        "mask": ("the batch's %d triples hidden in the edge mask in place before each step and restored after "
                 "it (src/main.py:887-890,927-930), so each step rebuilds the CSR-ordered mask bitmaps" % B
                 if train else "all edges visible"),
        "reference_batch": ref_batch,
        "topk_select_ms": {"c1_per_hop": per_launch["k_race_select"] if train else per_launch["k_sp_topc"],
                           "c2_per_hop": per_launch["k_sp_select"]},
        "kernel_ms_per_launch": per_launch,
        "kernel_ms_per_step": per_step,
        "kernel_ms_per_step_cold": cold_step,
        "roofline": {"kernel": "sparse hop (its forward and backward kernels, per step)", "bound": "hbm",
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                     "algorithmic_bytes_per_launch": step_bytes, "ms_per_launch": hop_ms,
                     "cache": "cold: %d MiB written before each hop" % FLUSH_MIB,
                     "warm": {"achieved": warm, "frac": warm / HBM_PEAK_GBS, "ms_per_launch": warm_ms},
                     "traffic": traffic,
                     "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT) if traffic is not None else None},
        "dominant_kernel": {"name": dominant, "ms_per_step": per_step[dominant]},
        "kernel_rooflines": kernel_rooflines,
        "hop_plans": plans,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


def cpu_baseline_sparse(args, csr_np, L, E, R, K, c1, src, tgt, W, T, train):
    """The reference's CPU --sparse path on a sample of the batch: per hop the
    c1 entity selection of flashlog_kernel.py:1093-1140 (torch ops, restated
    here) and flashlog_forward_sparse3d_sum_norm_cpu from the reference's
    flashlog.cpp (oracle/_ref; at::parallel_for over the entries,
    flashlog_kernel.py:1902-1913 dispatch), then the sum over channels.
    train: also the log-loss gradient on the target entities and
    flashlog_backward_sparse3d_sum_norm_cpu back through the hops
    (flashlog_kernel.py:1790-1811).  The reference's sampled selections on
    the CPU are Python code (flashlog_kernel.py:1955-2100), so the CPU
    training step uses the deterministic c1/c2 budgets.  Query rows are
    independent: the sample is the first Bs queries of the same batch, run
    as whole steps until ~cpu_seconds."""
    import torch
    sys.path.insert(0, os.path.join(ROOT, "oracle", "_ref"))
    try:
        import flashlog_ref_cpp as ref
    except ImportError:
        print("cpu baseline skipped: oracle/_ref not built", file=sys.stderr, flush=True)
        return None
    threads = min(16, os.cpu_count() or 1)
    tc = [torch.from_numpy(a) for a in csr_np]
    om = torch.ones(tc[1].shape[0], dtype=torch.float32)
    im = torch.ones(tc[5].shape[0], dtype=torch.float32)
    n = 2 * R + 1

    def topc(b, l, e, v):
        if e.numel() <= c1:
            return None
        groups, inv = torch.unique_consecutive(b * L + l, return_inverse=True)
        nz = v != 0
        cnt = torch.zeros(groups.numel(), dtype=torch.long).scatter_add_(0, inv, nz.long())
        over = cnt > c1
        if not bool(over.any()):
            return None
        keep = ~over[inv]
        cand = torch.nonzero(over[inv] & nz, as_tuple=True)[0]
        ranked = cand[torch.argsort(v[cand], descending=True, stable=True)]
        ranked = ranked[torch.argsort(inv[ranked], stable=True)]
        g = inv[ranked]
        first = torch.searchsorted(g, g, right=False)
        keep[ranked[(torch.arange(g.numel()) - first) < c1]] = True
        return torch.nonzero(keep, as_tuple=True)[0]

    def step(Bs):
        Wt = W[:, :Bs].contiguous()
        tg = torch.from_numpy(tgt[:Bs]).long()
        b = torch.arange(Bs).repeat_interleave(L)
        l = torch.arange(L).repeat(Bs)
        e = torch.from_numpy(src[:Bs]).repeat_interleave(L)
        v = torch.ones(Bs * L)
        tape = []
        for hop in range(T):
            keep = topc(b, l, e, v)
            if keep is not None:
                b, l, e, v = b[keep], l[keep], e[keep], v[keep]
            w = Wt[hop].reshape(Bs, L, n)
            o = ref.flashlog_forward_sparse3d_sum_norm_cpu(
                b, l, e, v, w, tc[1], om, tc[8], tc[9], tc[10], tc[11],
                tc[5], im, tc[12], tc[13], tc[14], tc[15], Bs, L, E, R, False, K, 1e-7, train)
            tape.append((keep, b, l, e, v, w, o))
            b, l, e, v = o[0], o[1], o[2], o[3]
        # sum over the channels: per (query, entity)
        key = b * E + e
        fk_, inv = torch.unique(key, return_inverse=True)
        final = torch.zeros(fk_.numel()).index_add_(0, inv, v)
        if not train:
            return
        tk = torch.arange(Bs) * E + tg
        pos = torch.searchsorted(fk_, tk).clamp(max=max(fk_.numel() - 1, 0))
        hit = fk_[pos] == tk
        logit = torch.where(hit, final[pos], torch.zeros(()))
        dlogit = torch.where(hit & (logit > 1e-7), -1.0 / (Bs * logit), torch.zeros(()))
        grad = torch.where(e == tg[b], dlogit[b], torch.zeros(()))  # d loss / d output values
        for hop in reversed(range(T)):
            keep, hb, hl, he, hv, w, o = tape[hop]
            gsp, gw = ref.flashlog_backward_sparse3d_sum_norm_cpu(
                o[0], o[1], o[2], grad.float(), o[4], o[5], o[6], hb, hl, he, hv, w,
                *o[7:14], *o[14:21], o[21], Bs, L, E, R, False, 1e-7)
            if hop > 0:
                prev = tape[hop - 1][6]
                grad = torch.zeros(prev[3].numel())
                if keep is None:
                    grad = gsp
                else:
                    grad[keep] = gsp

    def timed(nthreads, Bs, seconds):
        torch.set_num_threads(nthreads)
        t0 = time.perf_counter()
        steps = 0
        while True:
            step(Bs)
            steps += 1
            if time.perf_counter() - t0 >= seconds:
                break
        return steps, time.perf_counter() - t0

    what = "forward + backward" if train else "forward"
    Bs = min(16, W.shape[1])
    steps, el = timed(threads, Bs, args.cpu_seconds)
    # the reference's sum_norm CPU path at one thread (its at::parallel_for
    # over the rows, flashlog.cpp:1454, serial), on a smaller sample
    Bs1 = min(4, W.shape[1])
    steps1, el1 = timed(1, Bs1, args.cpu_seconds / 2)
    torch.set_num_threads(threads)
    return {**host_cpu(), "value": steps * Bs / el, "unit": "queries/s", "cores": threads, "kind": "reference",
            "sample": "%d full %s steps of %d queries x %d hops (first %d queries of the batch; deterministic "
                      "c1/c2 selections) in %.1f s, %d threads" % (steps, what, Bs, T, Bs, el, threads),
            "one_thread": {"value": steps1 * Bs1 / el1, "unit": "queries/s", "cores": 1,
                           "sample": "%d full %s steps of %d queries x %d hops in %.1f s, 1 thread"
                                     % (steps1, what, Bs1, T, el1)}}


def cpu_baseline(args, cfg, h, r, t, E, R, src, W):
    """The reference's CPU dense path on the same inputs: c1 by torch top-k as
    in flashlog_kernel.py:814-842, active nodes, then flashlog_forward_cpu from
    the reference's flashlog.cpp (oracle/_ref; serial in the reference), then
    the model's normalization.  Falls back to the C restatement if the
    reference build is absent.  Runs whole steps until ~cpu_seconds."""
    import numpy as np
    import torch
    torch.set_num_threads(1)
    sys.path.insert(0, os.path.join(ROOT, "oracle", "_ref"))
    kind = "reference"
    try:
        import flashlog_ref_cpp as ref
    except ImportError:
        ref = None
        kind = "port"
    from oracle import oracle as O
    csr = O.build_csr_structure(h, t, r, E)
    tc = [torch.from_numpy(np.ascontiguousarray(a)) for a in csr]
    M = h.shape[0]
    ones = torch.ones(M, dtype=torch.float32)
    B, L, T = cfg.batch, cfg.channels, cfg.hops
    n = 2 * R + 1
    K = cfg.c2 // 2 if cfg.use_topk else (1 << 60)
    Wt = torch.from_numpy(W)

    def topc(A, c):
        nonzero = A != 0
        over = nonzero.sum(-1, keepdim=True) > c
        if not bool(over.any()):
            return A
        scores = A.masked_fill(~nonzero, -float("inf"))
        cutoff = scores.topk(c, dim=-1).values.min(-1, keepdim=True).values
        above = nonzero & (A > cutoff)
        tied = nonzero & (A == cutoff)
        remaining = c - above.sum(-1, keepdim=True)
        keep = ~over | above | (tied & (tied.cumsum(-1) <= remaining))
        return A * keep

    def step():
        x = torch.zeros(B * L, E)
        x[torch.arange(B * L), torch.from_numpy(np.repeat(src, L))] = 1.0
        for hop in range(T):
            A = topc(x, cfg.c1) if cfg.use_topk else x
            w = Wt[hop].reshape(B * L, n).contiguous()
            act = torch.nonzero(A.sum(0)).reshape(-1)
            if ref is not None:
                o = ref.flashlog_forward_cpu(A.contiguous(), w, act, tc[1], ones, tc[8], tc[9], tc[10], tc[11],
                                             tc[5], ones, tc[12], tc[13], tc[14], tc[15], R, False, K)
            else:
                o = [torch.from_numpy(a) for a in
                     O.dense_forward(A.numpy(), w.numpy(), csr, (ones.numpy(), ones.numpy()), R, topk_edges=K)]
            s = o[0] + o[1] + o[2]
            x = s / s.sum(-1, keepdim=True).clamp(1e-7)
        return x.view(B, L, E).sum(1)

    t0 = time.perf_counter()
    steps = 0
    while True:
        step()
        steps += 1
        if time.perf_counter() - t0 >= args.cpu_seconds:
            break
    el = time.perf_counter() - t0
    return {**host_cpu(), "value": steps * B / el, "unit": "queries/s", "cores": 1, "kind": kind,
            "sample": "%d full steps (%d queries x %d hops) in %.1f s, 1 thread" % (steps, B, T, el)}


if __name__ == "__main__":
    main()
