"""Soft-guided grounding on gfx950.

Mirrors flashlog_kernel/soft_grounding_kernel/soft_grounding_kernel.py
(same functions, arguments, argument checks and CPU return values) over the
kernels of libflashlog_hip.so (fl_grounding.hip), which replace the
reference's OpenMP module source/soft_grounding.cpp.  Inputs may live on the
CPU or the GPU; the work runs on the current GPU and the results come back
as CPU tensors, as the reference returns them.  There is no CPU path.
"""
import ctypes
import math
import time

import torch

from ... import _lib
from ..._lib import FlGroundGraph, check, ptr

RULE_STEPS = 3  # the reference's default build (FLASHLOG_RULE_STEPS)
HUB_MIN_GROUPS = 8  # sides with more groups make a node a hub of the walk's option cache
HUB_CACHE_MAX_BYTES = 2 << 30  # the cache is skipped above this size


def _device():
    if not torch.cuda.is_available():
        raise RuntimeError("flashlog_amd needs a ROCm GPU: the soft-grounding sampler has no CPU path")
    return torch.device("cuda", torch.cuda.current_device())


def _stream(dev):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _temperature(value):
    """soft_grounding_kernel.py:16-21."""
    value = float(value)
    if not math.isfinite(value) or value <= 0:
        raise ValueError("sampling temperature must be finite and positive")
    return value


def _graph(csr, dev, num_relations):
    """Device copies of the CSR arrays the walks read (entries 1, 5, 8-15)."""
    t = {i: torch.as_tensor(csr[i]).to(dev) for i in (1, 5, 8, 9, 10, 11, 12, 13, 14, 15)}
    for i in (1, 5, 8, 10, 11, 12, 14, 15):
        t[i] = t[i].to(torch.int32).contiguous()
    for i in (9, 13):
        t[i] = t[i].to(torch.int16).contiguous()
    g = FlGroundGraph()
    g.ori_col, g.inv_col = ptr(t[1]).value, ptr(t[5]).value
    g.ori_ptr, g.ori_rel, g.ori_start, g.ori_count = (ptr(t[i]).value for i in (8, 9, 10, 11))
    g.inv_ptr, g.inv_rel, g.inv_start, g.inv_count = (ptr(t[i]).value for i in (12, 13, 14, 15))
    g.nodes = t[8].numel() - 1
    g.num_relations = int(num_relations)
    widths = [int((p[1:] - p[:-1]).max()) if p.numel() > 1 else 0 for p in (t[8], t[12])]
    g.max_groups = max(widths + [1])
    # hub cache: nodes with more than 64 groups on a side (their options are
    # ranked once per call for every head, step and rank)
    fw = (t[8][1:] - t[8][:-1]).long()
    iv = (t[12][1:] - t[12][:-1]).long()
    hub = (fw > HUB_MIN_GROUPS) | (iv > HUB_MIN_GROUPS)
    hub_node = torch.nonzero(hub).view(-1)
    nhub = hub_node.numel()
    g.nhub, g.hub_options = 0, 0
    if nhub:
        hub_id = torch.full((g.nodes,), -1, dtype=torch.int32, device=dev)
        hub_id[hub_node] = torch.arange(nhub, dtype=torch.int32, device=dev)
        cap = (fw + iv)[hub_node]
        hub_off = torch.zeros(nhub + 1, dtype=torch.int64, device=dev)
        hub_off[1:] = torch.cumsum(cap, 0)
        t["hub_id"], t["hub_node"], t["hub_off"] = hub_id, hub_node.to(torch.int32).contiguous(), hub_off
        g.nhub, g.hub_options = nhub, int(hub_off[-1])
        g.hub_id, g.hub_node, g.hub_off = ptr(hub_id).value, ptr(t["hub_node"]).value, ptr(hub_off).value
    return g, t


def _walks(g, attentions, heads_d, seeds, task_head, task_source, task_index, walks, topk_edges, mask, temperature,
           dev):
    """Walk records (body keys as int64, positive flags) of every task."""
    lib = _lib.lib()
    ntasks = task_source.numel()
    att = attentions.to(dev).contiguous()
    seeds_d = torch.tensor(seeds, dtype=torch.int64, device=dev)
    th = task_head.to(device=dev, dtype=torch.int32).contiguous()
    ts = task_source.to(device=dev, dtype=torch.int64).contiguous()
    ti = task_index.to(device=dev, dtype=torch.int64).contiguous()
    keys = torch.empty(max(ntasks * walks, 1), dtype=torch.int64, device=dev)
    positive = torch.empty(max(ntasks * walks, 1), dtype=torch.uint8, device=dev)
    nheads, ranks = attentions.shape[0], attentions.shape[2]
    if g.nhub and 3 * nheads * ranks * (20 * g.hub_options + 16 * g.nhub) > HUB_CACHE_MAX_BYTES:
        g.nhub = 0  # too large a cache: every step ranks its options
    ws = torch.empty(max(lib.fl_ground_walk_bytes(ctypes.byref(g), ntasks, nheads, ranks), 1), dtype=torch.uint8,
                     device=dev)
    check(lib.fl_ground_walks(_stream(dev), ctypes.byref(g), ptr(att), att.shape[0], att.shape[2], ptr(heads_d),
                              ptr(seeds_d), ntasks, ptr(th), ptr(ts), ptr(ti), walks, int(topk_edges),
                              1 if mask else 0, temperature, ptr(ws), ws.numel(), ptr(keys), ptr(positive)),
          "ground_walks")
    return keys, positive


def ground_head_batch_source_folds_sampled_capped_counts(
    attentions,
    heads,
    num_relations,
    source_folds,
    csr,
    walks_per_source,
    topk_edges,
    mask_query_head_from_source,
    seeds,
    transition_cache_size,
    num_threads,
    candidates_per_length,
    sampling_temperature=1.0,
):
    """Return ordered candidates, counts, and attributed wall times
    (soft_grounding_kernel.py:36-84; soft_grounding.cpp:898-1027).

    Per head: attention-guided walks from every source of every fold, body
    counts per fold capped per length, folds united by body with totals and
    minimums.  transition_cache_size and num_threads only size the
    reference's CPU caches and thread team; they are checked, not used.
    The wall time of the batch is attributed to its heads by source count.
    """
    budgets = tuple(map(int, candidates_per_length))
    attentions = torch.as_tensor(attentions, dtype=torch.float32).contiguous()
    heads = list(map(int, heads))
    seeds = list(map(int, seeds))
    folds = [[torch.as_tensor(sources, dtype=torch.int64, device="cpu").contiguous() for sources in head_folds]
             for head_folds in source_folds]
    if attentions.ndim != 4 or attentions.shape[1] <= 0:
        raise ValueError("attentions must have shape [heads, steps, rank, operators+1]")
    if len(budgets) != attentions.shape[1] or any(b < 0 for b in budgets):
        raise ValueError("candidates_per_length requires one nonnegative budget per step")
    if not (len(heads) == len(seeds) == len(folds) == len(attentions)):
        raise ValueError("attentions, heads, source_folds and seeds must have equal lengths")
    if any(not head_folds or any(sources.ndim != 1 for sources in head_folds) for head_folds in folds):
        raise ValueError("each head must have nonempty folds of one-dimensional vectors")
    temperature = _temperature(sampling_temperature)
    if attentions.shape[1] != RULE_STEPS:
        raise NotImplementedError("flashlog_amd grounds rule bodies of %d steps" % RULE_STEPS)
    # the checks of soft_grounding.cpp:973-997
    count = attentions.shape[0]
    R = int(num_relations)
    if attentions.shape[2] <= 0 or attentions.shape[3] != 2 * R + 1:
        raise RuntimeError("attentions must have shape [heads, 3, ranks > 0, 2*num_relations + 1]")
    if count > 0:
        if not (R > 0 and 2 * R < (1 << 20)):
            raise RuntimeError("num_relations must be positive with 2*num_relations < 2^20")
        if not (int(walks_per_source) > 0 and int(topk_edges) > 0):
            raise RuntimeError("walks_per_source and topk_edges must be positive")
        if not (int(transition_cache_size) >= 0 and int(num_threads) > 0):
            raise RuntimeError("transition_cache_size must be nonnegative and num_threads positive")
    for h in heads:
        if not 0 <= h < 2 * R:
            raise RuntimeError("head %d is not a directed relation in [0, %d)" % (h, 2 * R))
    if count == 0:
        return [], [], []
    dev = _device()
    started = time.perf_counter()
    g, keep = _graph(csr, dev, R)
    walks = int(walks_per_source)
    task_head, task_source, task_index, seg_task_off, seg_head = [], [], [], [0], []
    for h, head_folds in enumerate(folds):
        for sources in head_folds:
            n = sources.numel()
            if n and (int(sources.min()) < 0 or int(sources.max()) >= g.nodes):
                raise RuntimeError("source ids must lie in [0, %d)" % g.nodes)
            task_head.append(torch.full((n,), h, dtype=torch.int32))
            task_source.append(sources)
            task_index.append(torch.arange(n, dtype=torch.int64))
            seg_task_off.append(seg_task_off[-1] + n)
            seg_head.append(h)
    ntasks = seg_task_off[-1]
    if ntasks * walks >= (1 << 32):
        raise RuntimeError("more than 2^32 walks in one batch")
    nseg = len(seg_head)
    lib = _lib.lib()
    st = _stream(dev)
    heads_d = torch.tensor(heads, dtype=torch.int64, device=dev)
    keys, positive = _walks(g, attentions, heads_d, seeds, torch.cat(task_head), torch.cat(task_source),
                            torch.cat(task_index), walks, topk_edges, mask_query_head_from_source, temperature, dev)
    n = ntasks * walks
    cap = max(min(n, nseg * sum(budgets)), 1)
    rows = torch.empty((cap, 12), dtype=torch.int64, device=dev)
    info = torch.empty(nseg + count + 1, dtype=torch.int64, device=dev)
    off_d = torch.tensor(seg_task_off, dtype=torch.int64, device=dev)
    seg_head_d = torch.tensor(seg_head, dtype=torch.int64, device=dev)
    folds_d = torch.tensor([len(f) for f in folds], dtype=torch.int64, device=dev)
    budgets_h = (ctypes.c_int64 * 3)(*budgets)
    cws = torch.empty(max(lib.fl_ground_count_bytes(n, nseg, count), 1), dtype=torch.uint8, device=dev)
    check(lib.fl_ground_count(st, ptr(keys), ptr(positive), walks, nseg, ptr(off_d), ptr(seg_head_d), count,
                              ptr(heads_d), ptr(folds_d), budgets_h, ptr(cws), cws.numel(), ptr(rows), cap,
                              ptr(info)), "ground_count")
    info_h = info.cpu()
    rows_h = rows.cpu()
    elapsed = time.perf_counter() - started
    del keep
    raw = info_h[:nseg].tolist()
    offsets = info_h[nseg:].tolist()
    candidates, raw_counts, seconds = [], [], []
    total_sources = max(ntasks, 1)
    s = 0
    for h in range(count):
        candidates.append(rows_h[offsets[h]:offsets[h + 1]].clone())
        raw_counts.append(tuple(int(x) for x in raw[s:s + len(folds[h])]))
        s += len(folds[h])
        seconds.append(elapsed * sum(f.numel() for f in folds[h]) / total_sources)
    return candidates, raw_counts, seconds


def sample_relation_sources_reservoir(row_group_ptr, group_relations, relations, max_sources, seed):
    """Uniformly sample source rows per relation in one linear CSR pass
    (soft_grounding_kernel.py:87-112; soft_grounding.cpp:1029-1124).
    Returns [sampled int32 [len(relations), max_sources] (-1 padded),
    available int64 [len(relations)]] as CPU tensors."""
    row_group_ptr = torch.as_tensor(row_group_ptr, dtype=torch.int32).contiguous()
    group_relations = torch.as_tensor(group_relations, dtype=torch.int16).contiguous()
    relations = torch.as_tensor(relations, dtype=torch.int64, device="cpu").contiguous()
    if row_group_ptr.ndim != 1 or group_relations.ndim != 1:
        raise ValueError("CSR group metadata must be one-dimensional")
    if relations.ndim != 1:
        raise ValueError("relations must be a vector")
    if max_sources <= 0:
        raise ValueError("max_sources must be positive")
    max_sources = int(max_sources)
    # the checks of soft_grounding.cpp:1036-1077
    if row_group_ptr.numel() == 0:
        raise RuntimeError("row_group_ptr must be a nonempty vector")
    if int(row_group_ptr[-1]) != group_relations.numel():
        raise RuntimeError("row_group_ptr does not cover group_relations")
    nreq = relations.numel()
    sampled = torch.full((nreq, max_sources), -1, dtype=torch.int32)
    available = torch.zeros(nreq, dtype=torch.int64)
    if nreq == 0 or group_relations.numel() == 0:
        return [sampled, available]
    if int(relations.min()) < 0 or int(relations.max()) > 32767:
        raise RuntimeError("relation ID is outside int16 range")
    if torch.unique(relations).numel() != nreq:
        raise RuntimeError("relations contains duplicates")
    dev = _device()
    lib = _lib.lib()
    gp = row_group_ptr.to(dev)
    gr = group_relations.to(dev)
    rel = relations.to(dev)
    rows, groups = gp.numel() - 1, gr.numel()
    out = torch.empty((nreq, max_sources), dtype=torch.int32, device=dev)
    avail = torch.empty(nreq, dtype=torch.int64, device=dev)
    ws = torch.empty(max(lib.fl_reservoir_bytes(groups, rows, nreq, max_sources), 1), dtype=torch.uint8, device=dev)
    check(lib.fl_reservoir(_stream(dev), ptr(gp), rows, ptr(gr), groups, ptr(rel), nreq, max_sources,
                           ctypes.c_int64(int(seed)).value, ptr(ws), ws.numel(), ptr(out), ptr(avail)), "reservoir")
    return [out.cpu(), avail.cpu()]
