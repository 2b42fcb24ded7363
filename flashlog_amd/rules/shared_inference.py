"""Shared grounding for SUM and MAX rule inference (rules/shared_inference.py:
12-245): every rule body (at most a few operators) is grounded from every
source with the fixed-relation step of flashlog_kernel, and the grounded
endpoints are scored per rank.

For sources s_b, rules r with operator bodies and rank weights W[r, k] >= 0:
  reduction='sum':  S_k[b, e] = sum_r W[r, k] * C_r(b, e)
  reduction='max':  S_k[b, e] = max_r W[r, k] * [C_r(b, e) > 0]
where C_r is the number of graph paths from s_b to e along r's body, or
[paths > 0] with Boolean paths (then every intermediate state is Boolean
too, as the reference's advance does).  Each (k, b) row of S_k is divided by
its sum (clamped to 1e-30) and the ranks are summed (or maxed with
final_max) into one score per (b, e); the result is a coalesced sparse
[B, entities] tensor of the positive scores.

Execution: chunks of ``chunk_size`` rules are grounded for a block of sources
at once (one fixed-relation launch sequence per body step); the grounded
states are added into a dense [ranks, sources x entities] accumulator by
fl_rule_accumulate and finalized by fl_rule_finalize.  Sources are taken in
blocks sized so that the accumulator fits ``dense_budget_bytes``.  The
reference's prefix cache, source splits and sparse accumulators change only
the order of floating-point additions, not what is computed.
"""
import ctypes  # noqa: F401  (ctypes types are used through _lib)

import torch

from .. import _lib
from .._lib import check, ptr
from ..flashlog_kernel import flashlog_kernel as fk


def _empty(shape, device):
    return torch.sparse_coo_tensor(torch.empty((2, 0), dtype=torch.long, device=device),
                                   torch.empty(0, device=device), shape, is_coalesced=True)


def _available_first_ops(sources, csr, relations):
    """Operators that leave at least one source through an edge (plus the
    identity): rules starting elsewhere ground to nothing
    (shared_inference.py:34-47)."""
    positions = torch.stack((sources, sources + 1), dim=1).reshape(-1)
    bounds = torch.stack((csr[8][positions], csr[12][positions])).cpu().tolist()
    available = {2 * relations}
    for direction, (ri, ci) in enumerate(((9, 11), (13, 15))):
        for i in range(sources.numel()):
            start, end = bounds[direction][2 * i:2 * i + 2]
            if end > start:
                rels = (csr[ri][start:end].long() + direction * relations).tolist()
                cnts = csr[ci][start:end].tolist()
                available.update(rel for rel, c in zip(rels, cnts) if c > 0)
    return available


@torch.inference_mode()
def score(ev, sources, rules, csr, relations, entities, chunk_size,
          final_max=False, reduction="sum", boolean_paths=False, dense_budget_bytes=None,
          prefix_budget_bytes=512 * 1024**2, stats=None,
          source_frontier_budget_bytes=64 * 1024**2):
    """Signature of rules/shared_inference.py:12-15.  ``ev`` (the reference's
    evaluate module) is accepted for compatibility; grounding and reduction
    run on this build's kernels."""
    if reduction not in ("sum", "max"):
        raise ValueError("Unknown reduction")
    boolean_paths = boolean_paths or reduction == "max"
    if chunk_size < 1:
        raise ValueError("chunk_size must be positive")
    stats = {} if stats is None else stats
    for name in ("ground_calls", "prefix_hits", "chunks", "oom_retries"):
        stats.setdefault(name, 0)
    sources = sources.reshape(-1).long()
    device = sources.device
    batch = sources.numel()
    shape = (batch, int(entities))
    if not rules:
        return _empty(shape, device)
    stats["rules_before"] = len(rules)
    if len(csr) >= 16 and batch > 0:
        available = _available_first_ops(sources, csr, relations)
        rules = [r for r in rules if not r["body"] or r["body"][0] in available]
    stats["rules_after"] = len(rules)
    if not rules or batch == 0:
        return _empty(shape, device)
    widths = {len(r["rank_weights"]) for r in rules}
    if len(widths) != 1 or next(iter(widths)) < 1:
        raise ValueError("nonempty rank_weights must have matching widths")
    ranks = next(iter(widths))
    weights = torch.tensor([r["rank_weights"] for r in rules], dtype=torch.float32, device=device)
    if not bool(torch.isfinite(weights).all()) or bool((weights < 0).any()):
        raise ValueError("MAX rule weights must be finite and nonnegative")
    identity = 2 * relations
    lengths = [len(r["body"]) for r in rules]
    max_steps = max(lengths)
    operators = torch.tensor([list(r["body"]) + [identity] * (max_steps - len(r["body"])) for r in rules],
                             dtype=torch.long, device=device).reshape(len(rules), max(max_steps, 1))
    E = int(entities)
    if dense_budget_bytes is None:
        free = torch.cuda.mem_get_info(device)[0] if device.type == "cuda" else 256 * 1024**2
        dense_budget_bytes = max(free // 3, ranks * E * 4)
    block = max(1, min(batch, int(dense_budget_bytes) // max(1, ranks * E * 4)))
    stats["dense_accumulation"] = True
    lib = _lib.lib()
    st = fk._stream(sources)
    is_max = 1 if reduction == "max" else 0
    rows_out, cols_out, vals_out = [], [], []
    for s0 in range(0, batch, block):
        src = sources[s0:s0 + block]
        nb = src.numel()
        dense = torch.zeros((ranks, nb * E), dtype=torch.float32, device=device)
        for off in range(0, len(rules), chunk_size):
            C = min(chunk_size, len(rules) - off)
            b = torch.arange(nb, device=device).repeat_interleave(C)
            l = torch.arange(C, device=device).repeat(nb)
            e = src.repeat_interleave(C)
            state = torch.sparse_coo_tensor(torch.stack((b, l, e)), torch.ones(nb * C, device=device),
                                            (nb, C, E), is_coalesced=True)
            steps = max(lengths[off:off + C])
            ops = operators[off:off + C]
            for step in range(steps):
                if state._nnz() == 0:
                    break
                stats["ground_calls"] += 1
                state = fk.vectorized_operation_sparse3d_fixed_relation(
                    state, ops[:, step].unsqueeze(0).expand(nb, -1), csr, relations)
                if boolean_paths:
                    state = torch.sparse_coo_tensor(state.indices(), (state.values() > 0).float(), state.shape,
                                                    is_coalesced=True)
            if state._nnz():
                ix = state.indices()
                vals = state.values().float().contiguous()
                w = weights[off:off + C].contiguous()
                ws_bytes = lib.fl_rule_accumulate_bytes(vals.numel(), nb, C)
                ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
                check(lib.fl_rule_accumulate(st, ptr(ix[0].contiguous()), ptr(ix[1].contiguous()),
                                             ptr(ix[2].contiguous()), ptr(vals), vals.numel(), ptr(w), ranks, nb,
                                             C, E, is_max, ptr(dense), ptr(ws), ws_bytes), "rule_accumulate")
            stats["chunks"] += 1
        rowsum = torch.empty(ranks * nb, dtype=torch.float32, device=device)
        total = torch.empty(nb * E, dtype=torch.float32, device=device)
        check(lib.fl_rule_finalize(st, ptr(dense), ranks, nb, E, 1 if final_max else 0, ptr(rowsum), ptr(total)),
              "rule_finalize")
        keys = total.nonzero().flatten()
        rows_out.append(keys // E + s0)
        cols_out.append(keys % E)
        vals_out.append(total[keys])
    indices = torch.stack((torch.cat(rows_out), torch.cat(cols_out)))
    return torch.sparse_coo_tensor(indices, torch.cat(vals_out), shape, is_coalesced=True)
