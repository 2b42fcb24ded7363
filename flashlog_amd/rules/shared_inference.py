"""Shared grounding for SUM and MAX rule inference (rules/shared_inference.py:
12-245): every rule body (at most a few operators) is grounded from every
source with the fixed-relation step, and the grounded endpoints are scored
per rank.

For sources s_b, rules r with operator bodies and rank weights W[r, k] >= 0:
  reduction='sum':  S_k[b, e] = sum_r W[r, k] * C_r(b, e)
  reduction='max':  S_k[b, e] = max_r W[r, k] * [C_r(b, e) > 0]
where C_r is the number of graph paths from s_b to e along r's body, or
[paths > 0] with Boolean paths (then every intermediate state is Boolean
too, as the reference's advance does).  Each (k, b) row of S_k is divided by
its sum (clamped to 1e-30) and the ranks are summed (or maxed with
final_max) into one score per (b, e); the result is a coalesced sparse
[B, entities] tensor of the positive scores.

Execution: the grounding calls go through ``ev`` (the evaluate module: the
reference's, or this package's flashlog_amd.rules.evaluate when ``ev`` is
None): ev.initial_rule_state and ev.vectorized_operation_sparse3d_fixed_relation,
with ev.advance_single_rule_state_memory_bounded after an out-of-memory
step of one source and one rule.  A chunk whose grounding runs out of
memory is retried with half as many rules (stats["oom_retries"]), down to
one rule.  Grounded chunks are added into a dense [ranks, sources x
entities] accumulator by fl_rule_accumulate (sums: per (source, entity) the
chunk's rules in rule order, chunks in order; maxima: exact) and finalized
by fl_rule_finalize.  Sources are taken in blocks sized so that the
accumulator fits ``dense_budget_bytes``; as in the reference, a batch whose
first hop would expand a frontier beyond ``source_frontier_budget_bytes`` is
scored one source at a time.  The reference's prefix cache, source splits
and sparse accumulators change only how the exact integer path counts are
produced or the order of floating-point additions of the normalizers, not
the values of the channel sums.
"""
import types
import weakref

import numpy as np
import torch

from .. import _lib
from .._lib import check, ptr
from ..flashlog_kernel import flashlog_kernel as fk


def _empty(shape, device):
    return torch.sparse_coo_tensor(torch.empty((2, 0), dtype=torch.long, device=device),
                                   torch.empty(0, device=device), shape, is_coalesced=True)


# Host copies of a CSR tuple's group arrays (row group pointers, group
# relations and counts of both sides), kept while the tensors live
# unmodified: the first-hop degrees of every call read them on the host
# instead of slicing device tensors source by source.
_HOST_GROUPS = {}


def _host_groups(csr):
    keyed = tuple(csr[i] for i in (8, 9, 11, 12, 13, 15))
    key = tuple((id(t), t._version) for t in keyed)
    hit = _HOST_GROUPS.get(key)
    if hit is not None and all(r() is t for r, t in zip(hit[0], keyed)):
        return hit[1]
    for k in [k for k, v in _HOST_GROUPS.items() if any(r() is None for r in v[0])]:
        del _HOST_GROUPS[k]
    arrays = tuple(t.detach().cpu().numpy().astype(np.int64) for t in keyed)
    _HOST_GROUPS[key] = (tuple(weakref.ref(t) for t in keyed), arrays)
    return arrays


def _first_degrees(sources, csr, relations):
    """(operators, group sizes) of every first-hop group of the sources, as
    int64 arrays: forward groups as their relation, inverse ones offset by
    relations (rules/shared_inference.py:34-47; one read of the sources)."""
    gp_o, rel_o, cnt_o, gp_i, rel_i, cnt_i = _host_groups(csr)
    src = sources.detach().cpu().numpy().astype(np.int64)
    ops, cnts = [], []
    for side, (gp, rel, cnt) in enumerate(((gp_o, rel_o, cnt_o), (gp_i, rel_i, cnt_i))):
        lo, hi = gp[src], gp[src + 1]
        n = hi - lo
        if n.sum() == 0:
            continue
        # every group index of every source, sources in order
        idx = np.repeat(lo - np.concatenate(([0], np.cumsum(n)[:-1])), n) + np.arange(int(n.sum()))
        ops.append(rel[idx] + side * relations)
        cnts.append(cnt[idx])
    if not ops:
        return np.zeros(0, np.int64), np.zeros(0, np.int64)
    return np.concatenate(ops), np.concatenate(cnts)


def _default_ev():
    from . import evaluate
    return evaluate


def _grounding_hooks(ev):
    """The ``ev`` whose grounding hooks score() calls: this package's
    evaluation module for None or for any module other than it (a caller
    passing the reference's own rules.evaluate module, without install(),
    still grounds on this build's kernels); an object that is not a module
    (a caller's own hook set) is used as given."""
    own = _default_ev()
    if ev is None or (isinstance(ev, types.ModuleType) and ev is not own):
        return own
    return ev


def _accumulate_chunk(state, W, dense, is_max, nb, E):
    """dense [ranks, nb*E] += (max=) the chunk state's weighted rule sums."""
    if state._nnz() == 0:
        return
    ix = state.indices()
    vals = state.values().float().contiguous()
    C = state.shape[1]
    lib = _lib.lib()
    ws_bytes = lib.fl_rule_accumulate_bytes(vals.numel(), nb, C)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=vals.device)
    check(lib.fl_rule_accumulate(fk._stream(vals), ptr(ix[0].contiguous()), ptr(ix[1].contiguous()),
                                 ptr(ix[2].contiguous()), ptr(vals), vals.numel(), ptr(W.contiguous()), W.shape[1],
                                 nb, C, E, 1 if is_max else 0, ptr(dense), ptr(ws), ws_bytes),
          "rule_accumulate")


def _finalize(dense, nb, E, final_max):
    """(flat keys, scores) of the block: rows normalized, ranks combined."""
    ranks = dense.shape[0]
    rowsum = torch.empty(ranks * nb, dtype=torch.float32, device=dense.device)
    total = torch.empty(nb * E, dtype=torch.float32, device=dense.device)
    check(_lib.lib().fl_rule_finalize(fk._stream(dense), ptr(dense), ranks, nb, E, 1 if final_max else 0,
                                      ptr(rowsum), ptr(total)), "rule_finalize")
    keys = total.nonzero().flatten()
    return keys, total[keys]


@torch.inference_mode()
def score(ev, sources, rules, csr, relations, entities, chunk_size,
          final_max=False, reduction="sum", boolean_paths=False, dense_budget_bytes=None,
          prefix_budget_bytes=512 * 1024**2, stats=None,
          source_frontier_budget_bytes=64 * 1024**2):
    """Signature of rules/shared_inference.py:12-15."""
    if reduction not in ("sum", "max"):
        raise ValueError("Unknown reduction")
    boolean_paths = boolean_paths or reduction == "max"
    if chunk_size < 1:
        raise ValueError("chunk_size must be positive")
    ev = _grounding_hooks(ev)
    stats = {} if stats is None else stats
    for name in ("ground_calls", "prefix_hits", "chunks", "oom_retries"):
        stats.setdefault(name, 0)
    sources = sources.reshape(-1).long()
    device = sources.device
    batch = sources.numel()
    E = int(entities)
    shape = (batch, E)
    if not rules:
        return _empty(shape, device)
    all_rules = rules
    stats["rules_before"] = len(rules)
    if len(csr) >= 16 and batch > 0:
        deg_ops, deg_cnt = _first_degrees(sources, csr, relations)
        available = set(np.unique(deg_ops[deg_cnt > 0]).tolist()) | {2 * relations}
        rules = [r for r in rules if not r["body"] or r["body"][0] in available]
    else:
        deg_ops, deg_cnt = np.zeros(0, np.int64), np.zeros(0, np.int64)
    stats["rules_after"] = len(rules)
    if not rules or batch == 0:
        return _empty(shape, device)
    # the first hop's frontier per rule chunk (28 B per COO entry)
    first_ops = {}
    for r in rules:
        if r["body"]:
            first_ops[r["body"][0]] = first_ops.get(r["body"][0], 0) + 1
    # per first-hop group: the rules starting with its operator (0 for none)
    table = np.zeros(2 * relations + 2, np.int64)
    for op, k in first_ops.items():
        if 0 <= op < table.size:
            table[op] = k
    uses = table[np.clip(deg_ops, 0, table.size - 1)] if deg_ops.size else deg_ops
    max_first = int(deg_cnt[uses > 0].max()) if (uses > 0).any() else 0
    stats["first_frontier_bytes"] = int((deg_cnt * np.minimum(chunk_size, uses) * 28).max()) if deg_ops.size else 0
    if batch > 1 and max_first * 28 > source_frontier_budget_bytes:
        stats["source_splits"] = stats.get("source_splits", 0) + 1
        rows_out, cols_out, vals_out = [], [], []
        for b in range(batch):
            part = score(ev, sources[b:b + 1], all_rules, csr, relations, entities, chunk_size,
                         final_max=final_max, reduction=reduction, boolean_paths=boolean_paths,
                         dense_budget_bytes=dense_budget_bytes, prefix_budget_bytes=prefix_budget_bytes,
                         stats=stats, source_frontier_budget_bytes=source_frontier_budget_bytes).coalesce()
            rows_out.append(part.indices()[0] + b)
            cols_out.append(part.indices()[1])
            vals_out.append(part.values())
        return torch.sparse_coo_tensor(torch.stack((torch.cat(rows_out), torch.cat(cols_out))), torch.cat(vals_out),
                                       shape, is_coalesced=True)
    widths = {len(r["rank_weights"]) for r in rules}
    if len(widths) != 1 or next(iter(widths)) < 1:
        raise ValueError("nonempty rank_weights must have matching widths")
    ranks = next(iter(widths))
    host_w = np.asarray([r["rank_weights"] for r in rules], dtype=np.float32)
    if not np.isfinite(host_w).all() or (host_w < 0).any():
        raise ValueError("MAX rule weights must be finite and nonnegative")
    weights = torch.from_numpy(host_w).to(device)
    identity = 2 * relations
    steps = max(len(r["body"]) for r in rules)
    operators = torch.tensor([tuple(r["body"]) + (identity,) * (steps - len(r["body"])) for r in rules],
                             dtype=torch.long, device=device).reshape(len(rules), max(steps, 1))
    lengths = [len(r["body"]) for r in rules]
    if dense_budget_bytes is None:
        free = torch.cuda.mem_get_info(device)[0] if device.type == "cuda" else 256 * 1024**2
        dense_budget_bytes = max(free // 3, ranks * E * 4)
    block = max(1, min(batch, int(dense_budget_bytes) // max(1, ranks * E * 4)))
    stats["dense_accumulation"] = True
    stats["prefix_enabled"] = False
    is_max = reduction == "max"

    def advance(state, ops, nb):
        stats["ground_calls"] += 1
        try:
            out = ev.vectorized_operation_sparse3d_fixed_relation(state, ops, csr, relations)
        except torch.cuda.OutOfMemoryError:
            if nb != 1 or state.shape[1] != 1:
                raise
            torch.cuda.empty_cache()
            out = ev.advance_single_rule_state_memory_bounded(state, ops, csr, relations)
        out = out.coalesce()
        if boolean_paths:
            # several paths are one piece of Boolean evidence, not a multiplicity
            out = torch.sparse_coo_tensor(out.indices(), (out.values() > 0).to(out.dtype), out.shape,
                                          is_coalesced=True)
        return out

    def ground(src, lo, hi):
        nb = src.numel()
        state = ev.initial_rule_state(src, hi - lo, E)
        ops = operators[lo:hi]
        for step in range(max(lengths[lo:hi])):
            if state._nnz() == 0:
                break
            state = advance(state, ops[:, step].unsqueeze(0).expand(nb, -1), nb)
        return state

    keys_out, vals_out = [], []
    for s0 in range(0, batch, block):
        src = sources[s0:s0 + block]
        nb = src.numel()
        dense = torch.zeros((ranks, nb * E), dtype=torch.float32, device=device)
        off, size = 0, chunk_size
        while off < len(rules):
            hi = min(off + size, len(rules))
            try:
                state = ground(src, off, hi)
            except torch.cuda.OutOfMemoryError:
                state = None
                torch.cuda.empty_cache()
                stats["oom_retries"] += 1
                if size == 1:
                    raise torch.cuda.OutOfMemoryError("MAX grounding needs a smaller query batch")
                size = max(1, size // 2)
                continue
            _accumulate_chunk(state, weights[off:hi], dense, is_max, nb, E)
            off = hi
            stats["chunks"] += 1
        keys, vals = _finalize(dense, nb, E, final_max)
        keys_out.append(keys + s0 * E)
        vals_out.append(vals)
        del dense
    keys = torch.cat(keys_out)
    return torch.sparse_coo_tensor(torch.stack((keys // E, keys % E)), torch.cat(vals_out), shape,
                                   is_coalesced=True)
