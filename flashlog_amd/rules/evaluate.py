"""Rule-bank evaluation primitives and DRUM rule scoring
(rules/evaluate.py:94-119,188-734,746-854 of the reference), on this
library's kernels.

This module plays the role of the reference's ``evaluate`` module, which
rules/shared_inference.py receives as ``ev``: the grounding step, the
memory-bounded single-rule advance, the per-chunk reductions, the sparse
merges and normalizers, and the DRUM scorer ``score_rule_batch`` with its
routed-rule compaction, rank streaming and out-of-memory fallbacks.

Grounding is the fixed-relation step (fl_sparse_* mode 2).  Sparse
reductions that the reference performs as torch coalesces of a re-indexed
state -- a sum (or maximum) over rules per (query, entity) in rule order --
run on the channel-merge kernels (fl_sparse_channel_sum_plan/emit: the
entries of every (query, entity) are ranked across the rule channels and
added from 0 in channel order, the order torch's coalesce adds them in), and
row normalizations on fl_sparse_normalize_forward.  score_rule_batch
accumulates every requested aggregation of a rule chunk into dense
[channels, sources x entities] buffers with fl_rule_accumulate (one writer
per slot: chunk sums in rule order, chunks in order, as the reference's
per-chunk coalesce followed by add_sparse) and finalizes the normalized
ones with fl_rule_finalize.
"""
import csv
import os

import numpy as np
import torch

from .. import _lib
from .._lib import check, ptr
from ..flashlog_kernel import flashlog_kernel as fk
from ..flashlog_kernel.flashlog_kernel import (  # noqa: F401  (re-exported names)
    build_csr_structure,
    sparse2d_filtered_ranks_cuda,
    vectorized_operation_sparse3d_fixed_relation,
)

CSR_RULE_FIELDS = frozenset((1, 5, 8, 9, 10, 11, 12, 13, 14, 15))
RANK_STREAMING_RULE_THRESHOLD = int(os.environ.get("FLASHLOG_RANK_STREAMING_RULE_THRESHOLD", "1024"))
_NORM_EPS = 1e-30  # the rank and row normalizers' clamp (rules/evaluate.py:355,374)


# ---------------------------------------------------------------------------
# sparse helpers

def _sparse(indices, values, shape):
    return torch.sparse_coo_tensor(indices, values, tuple(int(s) for s in shape), is_coalesced=True)


def _empty(shape, device):
    return _sparse(torch.empty((len(shape), 0), dtype=torch.long, device=device),
                   torch.empty(0, device=device), shape)


def _rows_and_cols(s):
    """(row ids over all leading dimensions, last-dimension ids, number of
    rows, width) of a coalesced sparse tensor."""
    idx = s.indices()
    rows = idx[0]
    nrows = s.shape[0]
    for d in range(1, s.dim() - 1):
        rows = rows * s.shape[d] + idx[d]
        nrows *= s.shape[d]
    return rows, idx[-1], int(nrows), int(s.shape[-1])


def _unflatten_rows(rows, cols, shape):
    """Indices of a coalesced tensor from its row ids (over the leading
    dimensions of `shape`) and last-dimension ids."""
    parts = []
    for d in reversed(range(1, len(shape) - 1)):
        parts.append(rows % shape[d])
        rows = rows // shape[d]
    parts.append(rows)
    return torch.stack(list(reversed(parts)) + [cols])


def _channel_reduce(b, l, e, v, B, L, E, op):
    """Per (b, e) of a coalesced [B, L, E] state the sum from 0 (op 0) or the
    maximum (op 1) over its channels in channel order; returns a coalesced
    [B, E] tensor."""
    if v.numel() == 0:
        return _empty((B, E), v.device)
    idx, out, _, _ = fk._channel_reduce(b, l, e, v, int(B), int(L), int(E), op)
    return _sparse(idx, out, (B, E))


def _merge_two(left, right, op):
    """The entry-wise sum (op 0: left + right, as left's then right's value
    added from 0) or maximum (op 1) of two coalesced tensors of one shape,
    through the channel merge: left is channel 0 and right channel 1 of each
    row."""
    left = left.coalesce()
    right = right.coalesce()
    if left.shape != right.shape:
        raise ValueError("sparse operands must have the same shape")
    shape = tuple(left.shape)
    dev = left.device
    lr, lc, nrows, width = _rows_and_cols(left)
    rr, rc, _, _ = _rows_and_cols(right)
    nl, nr = lr.numel(), rr.numel()
    if nl + nr == 0:
        return _empty(shape, dev)
    bounds = torch.arange(nrows + 1, device=dev)
    lptr = torch.searchsorted(lr, bounds)
    rptr = torch.searchsorted(rr, bounds)
    # merged position: the row's left entries, then its right entries
    lpos = torch.arange(nl, device=dev) + rptr[lr]
    rpos = torch.arange(nr, device=dev) + lptr[rr + 1]
    mb = torch.empty(nl + nr, dtype=torch.long, device=dev)
    ml = torch.empty_like(mb)
    me = torch.empty_like(mb)
    mv = torch.empty(nl + nr, dtype=torch.float32, device=dev)
    for pos, rows, cols, vals, ch in ((lpos, lr, lc, left.values(), 0), (rpos, rr, rc, right.values(), 1)):
        mb[pos] = rows
        ml[pos] = ch
        me[pos] = cols
        mv[pos] = vals.float()
    red = _channel_reduce(mb, ml, me, mv, nrows, 2, width, op)
    ri = red.indices()
    return _sparse(_unflatten_rows(ri[0], ri[1], shape), red.values().to(left.dtype), shape)


def _normalize_rows(rows, vals, nrows):
    """vals / max(row sum, 1e-30) per row (entries sorted by row)."""
    out, _, _ = fk._normalize_forward(rows, torch.zeros_like(rows), vals, int(nrows), 1, _NORM_EPS)
    return out


# ---------------------------------------------------------------------------
# ev primitives (rules/evaluate.py:188-447)

def initial_rule_state(sources, num_rules, num_entities):
    """(source b, rule l, s_b) with value 1 for every source and rule, a
    coalesced [B, num_rules, num_entities] state (rules/evaluate.py:188-197)."""
    B = sources.numel()
    dev = sources.device
    b = torch.arange(B, device=dev).repeat_interleave(num_rules)
    l = torch.arange(num_rules, device=dev).repeat(B)
    e = sources.reshape(-1).long().repeat_interleave(num_rules)
    return _sparse(torch.stack((b, l, e)), torch.ones(B * num_rules, device=dev), (B, num_rules, num_entities))


def advance_single_rule_state_memory_bounded(state, operators, csr, num_relations, input_chunk_size=64):
    """One step of one query and one rule with a bounded expansion
    (rules/evaluate.py:200-273): slices of at most input_chunk_size frontier
    entries are advanced one after the other (halved after an out-of-memory
    error, down to one entry) and their path counts added into one dense
    [entities] vector; path counts are integers, exact in any order."""
    state = state.coalesce()
    if state.shape[0] != 1 or state.shape[1] != 1:
        raise ValueError("memory-bounded advance requires one query and one rule")
    if tuple(operators.shape) != (1, 1):
        raise ValueError("memory-bounded operators must have shape [1, 1]")
    n = state._nnz()
    if n == 0:
        return state
    E = state.shape[2]
    dev = state.device
    acc = torch.zeros(E, device=dev, dtype=state.dtype)
    idx, vals = state.indices(), state.values()
    lo, size = 0, min(input_chunk_size, n)
    while lo < n:
        hi = min(lo + size, n)
        try:
            part = vectorized_operation_sparse3d_fixed_relation(
                _sparse(idx[:, lo:hi], vals[lo:hi], state.shape), operators, csr, num_relations)
            acc.index_add_(0, part.indices()[2], part.values())
        except torch.cuda.OutOfMemoryError:
            part = None
            torch.cuda.empty_cache()
            if size == 1:
                raise
            size = max(1, size // 2)
            continue
        lo = hi
    ent = torch.nonzero(acc, as_tuple=True)[0]
    zero = torch.zeros_like(ent)
    return _sparse(torch.stack((zero, zero, ent)), acc[ent], state.shape)


def reduce_rule_state(state, weights, boolean=False):
    """[B, rules, E] -> [B, E]: per (source, entity) the sum over rules, in
    rule order, of value * weights[rule] (value > 0 as 1 when boolean)
    (rules/evaluate.py:276-288)."""
    state = state.coalesce()
    b, l, e = state.indices()
    v = state.values()
    if boolean:
        v = (v > 0).to(v.dtype)
    return _channel_reduce(b, l, e, v * weights[l], state.shape[0], state.shape[1], state.shape[2], 0)


def reduce_rule_state_by_rank(state, rank_weights, boolean=False):
    """[B, rules, E] -> [B, ranks, E]: per rank k the rule-order sum of the
    positive terms value * rank_weights[rule, k] (rules/evaluate.py:291-323)."""
    state = state.coalesce()
    B, C, E = state.shape
    b, l, e = state.indices()
    v = state.values()
    if boolean:
        v = (v > 0).to(v.dtype)
    K = rank_weights.shape[1]
    keys, vals = [], []
    for k in range(K):
        x = v * rank_weights[l, k]
        pos = x > 0
        part = _channel_reduce(b[pos], l[pos], e[pos], x[pos], B, C, E, 0)
        pi = part.indices()
        keys.append((pi[0] * K + k) * E + pi[1])
        vals.append(part.values())
    keys = torch.cat(keys)
    order = torch.argsort(keys)
    keys = keys[order]
    return _sparse(torch.stack((keys // (K * E), (keys // E) % K, keys % E)), torch.cat(vals)[order], (B, K, E))


def reduce_rule_state_by_group(state, weights, groups, num_groups):
    """[B, rules, E] -> [B, groups, E]: per routed group the rule-order sum of
    the positive terms value * weights[rule] of its rules
    (rules/evaluate.py:326-343)."""
    state = state.coalesce()
    if groups.shape != weights.shape:
        raise ValueError("groups and weights must have the same shape")
    if num_groups <= 0 or bool((groups < 0).any()) or bool((groups >= num_groups).any()):
        raise ValueError("group IDs must be within the routed group count")
    B, C, E = state.shape
    b, l, e = state.indices()
    x = state.values() * weights[l]
    pos = x > 0
    b, l, e, x = b[pos], l[pos], e[pos], x[pos]
    # rows (b, group): a stable sort keeps each row's rules in rule order
    row = b * num_groups + groups[l]
    order = torch.sort(row, stable=True).indices
    red = _channel_reduce(row[order], l[order], e[order], x[order], B * num_groups, C, E, 0)
    ri = red.indices()
    return _sparse(torch.stack((ri[0] // num_groups, ri[0] % num_groups, ri[1])), red.values(),
                   (B, num_groups, E))


def normalize_and_sum_rank_scores(scores):
    """[B, ranks, E] -> [B, E]: each (source, rank) row divided by
    max(its sum, 1e-30), then the ranks added in rank order
    (rules/evaluate.py:346-363)."""
    scores = scores.coalesce()
    B, K, E = scores.shape
    b, k, e = scores.indices()
    if e.numel() == 0:
        return _empty((B, E), scores.device)
    normed, _, _ = fk._normalize_forward(b, k, scores.values(), int(B), int(K), _NORM_EPS)
    return _channel_reduce(b, k, e, normed, B, K, E, 0)


def normalize_sparse_rows(scores):
    """Each row of a [B, E] tensor divided by max(its sum, 1e-30)
    (rules/evaluate.py:366-378)."""
    scores = scores.coalesce()
    idx = scores.indices()
    if scores._nnz() == 0:
        return scores
    return _sparse(idx, _normalize_rows(idx[0], scores.values(), scores.shape[0]).to(scores.dtype),
                   scores.shape)


def add_sparse(left, right):
    """left + right (rules/evaluate.py:381-390); None is the empty operand."""
    if left is None:
        return right
    return _merge_two(left, right, 0)


def max_sparse(left, right):
    """Entry-wise maximum (rules/evaluate.py:393-419); None is the empty
    operand."""
    if left is None:
        return right
    return _merge_two(left, right, 1)


def max_reduce_rule_state(state, weights):
    """[B, rules, E] -> [B, E]: per (source, entity) the largest weight of a
    rule with a path there (rules/evaluate.py:422-446)."""
    state = state.coalesce()
    b, l, e = state.indices()
    v = (state.values() > 0).to(state.values().dtype) * weights[l]
    return _channel_reduce(b, l, e, v, state.shape[0], state.shape[1], state.shape[2], 1)


# ---------------------------------------------------------------------------
# routed rules, rule files

def compact_routed_rules(rules):
    """One rule per distinct (head, body), its rank_weights holding the
    weight of each routed group (rules/evaluate.py:94-119); an indexed head
    (IndexedHeadRules) compacts itself."""
    if hasattr(rules, "compact"):
        return rules.compact()
    if any(r["group_id"] is None for r in rules):
        raise ValueError("routed_normalized requires a group_id column")
    width = 1 + max(r["group_id"] for r in rules)
    merged = {}
    for r in rules:
        slot = merged.setdefault((r["head"], tuple(r["body"])),
                                 ({**r, "weight": 1.0, "group_id": None}, [0.0] * width))
        if slot[1][r["group_id"]] != 0:
            raise ValueError("duplicate Horn rule/group instance")
        slot[1][r["group_id"]] = r["weight"]
    return [{**rule, "rank_weights": tuple(w)} for rule, w in merged.values()]


def load_rules(path, weight_field="weight"):
    """The rule bank TSV (columns head_id, body_ids, the weight field and
    optionally rank_weights and group_id; rules/evaluate.py:64-91)."""
    out = []
    with open(path, newline="") as f:
        for rid, row in enumerate(csv.DictReader(f, delimiter="\t")):
            if weight_field not in row:
                raise ValueError("rule weight field %r is not present in %s" % (weight_field, path))
            group = row.get("group_id")
            out.append({
                "rule_id": rid,
                "head": int(row["head_id"]),
                "body": tuple(int(x) for x in row["body_ids"].split()) if row["body_ids"] else (),
                "weight": float(row[weight_field]),
                "rank_weights": tuple(float(x) for x in row["rank_weights"].split()) if row.get("rank_weights")
                else None,
                "group_id": int(group) if group not in (None, "") else None,
            })
    return out


def build_compact_rule_csr(train_path, num_entities, device, cache_path=None):
    """The rule-serving CSR (rules/evaluate.py:131-185): the 16-tuple with
    only the fields rule grounding reads (CSR_RULE_FIELDS), the rest empty;
    read from / written to a torch cache file {"num_entities", "csr"} (loaded
    with weights_only=True).  The CSR is built on the device."""
    if cache_path is not None and os.path.exists(cache_path):
        payload = torch.load(cache_path, map_location="cpu", weights_only=True)
        if payload["num_entities"] != num_entities:
            raise ValueError("CSR cache entity count does not match the dataset")
        return tuple(t.to(device) if i in CSR_RULE_FIELDS else torch.empty(0, device=device)
                     for i, t in enumerate(payload["csr"]))
    cols = np.loadtxt(train_path, dtype=np.int64, ndmin=2)
    h, r, t = (torch.from_numpy(np.ascontiguousarray(cols[:, i])).to(device) for i in range(3))
    csr = build_csr_structure(h, t, r, num_entities)
    compact = tuple(x if i in CSR_RULE_FIELDS else torch.empty(0, device=x.device) for i, x in enumerate(csr))
    if cache_path is not None:
        os.makedirs(os.path.dirname(os.path.abspath(cache_path)), exist_ok=True)
        torch.save({"num_entities": num_entities, "csr": tuple(x.cpu() for x in compact)}, cache_path)
    return compact


# ---------------------------------------------------------------------------
# DRUM rule scoring (rules/evaluate.py:449-734)

def _score_rank_batch_serial(sources, rules, csr, num_relations, num_entities, rule_chunk_size, modes):
    """One scoring pass per rank over the rules with a positive weight in
    it, each rank normalized per query row and the ranks added in order
    (rules/evaluate.py:449-497)."""
    if any(r["rank_weights"] is None for r in rules):
        raise ValueError("rank aggregation requires a rank_weights column")
    widths = {len(r["rank_weights"]) for r in rules}
    if len(widths) != 1:
        raise ValueError("rank_weights widths must match")
    wanted = tuple(dict.fromkeys("weighted_boolean" if bl else "weighted_path_count" for bl in modes.values()))
    out = {name: None for name in modes}
    for k in range(next(iter(widths))):
        ranked = [{**r, "weight": r["rank_weights"][k]} for r in rules if r["rank_weights"][k] > 0]
        part = score_rule_batch(sources, ranked, csr, num_relations, num_entities, rule_chunk_size, wanted)
        for name, bl in modes.items():
            out[name] = add_sparse(out[name],
                                   normalize_sparse_rows(part["weighted_boolean" if bl else "weighted_path_count"]))
    return out


def _ground_shared_rules(sources, chunk, csr, relations, entities):
    """Unweighted path counts of a rule chunk for every source
    (rules/evaluate.py:500-518); an out-of-memory step of one source and one
    rule takes the memory-bounded advance."""
    identity = 2 * relations
    steps = max(len(r["body"]) for r in chunk)
    ops = torch.tensor([tuple(r["body"]) + (identity,) * (steps - len(r["body"])) for r in chunk],
                       device=sources.device, dtype=torch.long)
    state = initial_rule_state(sources, len(chunk), entities)
    for step in range(steps):
        if state._nnz() == 0:
            break
        step_ops = ops[:, step].unsqueeze(0).expand(sources.numel(), -1)
        try:
            state = vectorized_operation_sparse3d_fixed_relation(state, step_ops, csr, relations)
        except torch.cuda.OutOfMemoryError:
            if len(chunk) != 1 or sources.numel() != 1:
                raise
            torch.cuda.empty_cache()
            state = advance_single_rule_state_memory_bounded(state, step_ops, csr, relations)
    return state


@torch.inference_mode()
def _score_rank_batch_shared(sources, rules, csr, num_relations, num_entities, rule_chunk_size, modes):
    """The shared-grounding scorer for every requested rank mode
    (rules/evaluate.py:521-527)."""
    import sys
    from . import shared_inference
    return {name: shared_inference.score(sys.modules[__name__], sources, rules, csr, num_relations, num_entities,
                                         rule_chunk_size, reduction="sum", boolean_paths=bl)
            for name, bl in modes.items()}


_SERIAL_RANK_HEADS = set()


@torch.inference_mode()
def score_rank_batch_streamed_modes(sources, rules, csr, num_relations, num_entities, rule_chunk_size, modes):
    """Shared grounding first; after an out-of-memory error the rank-serial
    scorer, remembered per (CSR, device, batch size, head)
    (rules/evaluate.py:533-550)."""
    key = (id(csr), str(sources.device), int(sources.numel()), rules[0].get("head"))
    if key not in _SERIAL_RANK_HEADS:
        try:
            return _score_rank_batch_shared(sources, rules, csr, num_relations, num_entities, rule_chunk_size,
                                            modes)
        except torch.cuda.OutOfMemoryError:
            pass
        torch.cuda.empty_cache()
        _SERIAL_RANK_HEADS.add(key)
    return _score_rank_batch_serial(sources, rules, csr, num_relations, num_entities, rule_chunk_size, modes)


# aggregation -> (boolean paths, accumulation: "sum" / "max", channel source)
_AGGREGATIONS = {
    "weighted_path_count": (False, "sum", "weight"),
    "weighted_boolean": (True, "sum", "weight"),
    "max_confidence": (True, "max", "weight"),
    "rank_normalized": (False, "sum", "rank"),
    "rank_boolean_normalized": (True, "sum", "rank"),
    "routed_normalized": (False, "sum", "group"),
}


def _accumulate(state, W, dense, is_max, nb, E, boolean):
    """dense [channels, nb*E] += (or max=) the chunk state's per (source,
    entity) rule-order sums of value * W[rule, channel]."""
    if state._nnz() == 0:
        return
    ix = state.indices()
    v = state.values().float()
    if boolean:
        v = (v > 0).float()
    v = v.contiguous()
    C = state.shape[1]
    lib = _lib.lib()
    ws_bytes = lib.fl_rule_accumulate_bytes(v.numel(), nb, C)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=v.device)
    check(lib.fl_rule_accumulate(fk._stream(v), ptr(ix[0].contiguous()), ptr(ix[1].contiguous()),
                                 ptr(ix[2].contiguous()), ptr(v), v.numel(), ptr(W.contiguous()), W.shape[1], nb, C,
                                 E, 1 if is_max else 0, ptr(dense), ptr(ws), ws_bytes), "rule_accumulate")


def _finalize_normalized(dense, nb, E, s0, device):
    K = dense.shape[0]
    rowsum = torch.empty(K * nb, dtype=torch.float32, device=device)
    total = torch.empty(nb * E, dtype=torch.float32, device=device)
    check(_lib.lib().fl_rule_finalize(fk._stream(dense), ptr(dense), K, nb, E, 0, ptr(rowsum), ptr(total)),
          "rule_finalize")
    keys = total.nonzero().flatten()
    return keys // E + s0, keys % E, total[keys]


@torch.inference_mode()
def score_rule_batch(sources, rules, csr, num_relations, num_entities, rule_chunk_size, aggregations):
    """DRUM rule scoring (rules/evaluate.py:554-734): for query sources s_b
    and rules r (weight w_r, rank_weights rw_r, group g_r), per aggregation
      weighted_path_count      sum_r w_r C_r(b, e)
      weighted_boolean         sum_r w_r [C_r(b, e) > 0]
      max_confidence           max_r w_r over rules with C_r(b, e) > 0
      rank_normalized          sum_k normalize_b(sum_r rw_r[k] C_r(b, e))
      rank_boolean_normalized  the same with [C_r > 0]
      routed_normalized        sum_g normalize_b(sum_{r in g} w_r C_r(b, e))
    where C_r is the path count of r's body from s_b to e and normalize_b
    divides a (source, channel) row by max(its sum, 1e-30); the terms of the
    channel sums are the positive ones.  Returns {aggregation: coalesced
    sparse [sources, entities]}; an entity a rule reaches with a zero weight
    is kept as an explicit 0 in the unnormalized aggregations.

    Only routed_normalized: the rules are compacted by (head, body) and
    scored as rank_normalized.  More than RANK_STREAMING_RULE_THRESHOLD
    rules: the rank modes go through score_rank_batch_streamed_modes.
    Otherwise chunks of rule_chunk_size rules are grounded once each
    (one out-of-memory step of one source and one rule takes the
    memory-bounded advance) and every aggregation is accumulated into a
    dense [channels, sources x entities] buffer."""
    requested = tuple(aggregations)
    dev = sources.device
    sources = sources.reshape(-1).long()
    B, E = sources.numel(), int(num_entities)
    if not rules:
        return {name: _empty((B, E), dev) for name in requested}
    for name in requested:
        if name not in _AGGREGATIONS:
            raise ValueError("unknown aggregation %r" % (name,))
    if requested == ("routed_normalized",):
        compact = compact_routed_rules(rules)
        part = score_rule_batch(sources, compact, csr, num_relations, num_entities, rule_chunk_size,
                                ("rank_normalized",))
        return {"routed_normalized": part["rank_normalized"]}
    streamed = {}
    pending = requested
    if len(rules) > RANK_STREAMING_RULE_THRESHOLD:
        modes = {name: bl for name, bl in (("rank_normalized", False), ("rank_boolean_normalized", True))
                 if name in requested}
        if modes:
            streamed = score_rank_batch_streamed_modes(sources, rules, csr, num_relations, num_entities,
                                                       rule_chunk_size, modes)
        pending = tuple(name for name in requested if name not in streamed)
        if not pending:
            return {name: streamed[name].coalesce() for name in requested}
    # per-rule channel weights of every pending aggregation
    weights = torch.tensor([float(r["weight"]) for r in rules], dtype=torch.float32, device=dev)
    chans = {}
    for name in pending:
        kind = _AGGREGATIONS[name][2]
        if kind == "weight":
            chans[name] = weights.unsqueeze(1)
        elif kind == "rank":
            if any(r["rank_weights"] is None for r in rules):
                raise ValueError("rank aggregation requires a rank_weights column")
            if len({len(r["rank_weights"]) for r in rules}) != 1:
                raise ValueError("rank_weights widths must match")
            rw = torch.tensor([r["rank_weights"] for r in rules], dtype=torch.float32, device=dev)
            chans[name] = torch.where(rw > 0, rw, torch.zeros_like(rw))
        else:
            if any(r["group_id"] is None for r in rules):
                raise ValueError("routed_normalized requires a group_id column")
            G = 1 + max(r["group_id"] for r in rules)
            W = torch.zeros((len(rules), G), dtype=torch.float32, device=dev)
            W[torch.arange(len(rules), device=dev), torch.tensor([r["group_id"] for r in rules], device=dev)] = \
                torch.where(weights > 0, weights, torch.zeros_like(weights))
            chans[name] = W
    if "max_confidence" in pending and bool((weights < 0).any()):
        raise ValueError("max_confidence needs nonnegative rule weights")
    ones = torch.ones((len(rules), 1), dtype=torch.float32, device=dev)
    needs_presence = any(_AGGREGATIONS[n][2] == "weight" for n in pending)
    dense = {name: torch.zeros((chans[name].shape[1], B * E), dtype=torch.float32, device=dev) for name in pending}
    presence = torch.zeros((1, B * E), dtype=torch.float32, device=dev) if needs_presence else None
    for off in range(0, len(rules), rule_chunk_size):
        chunk = rules[off:off + rule_chunk_size]
        state = _ground_shared_rules(sources, chunk, csr, num_relations, E)
        for name in pending:
            bl, red, _ = _AGGREGATIONS[name]
            _accumulate(state, chans[name][off:off + len(chunk)], dense[name], red == "max", B, E, bl)
        if presence is not None:
            _accumulate(state, ones[off:off + len(chunk)], presence, True, B, E, True)
    out = dict(streamed)
    for name in pending:
        if _AGGREGATIONS[name][2] == "weight":
            keys = presence[0].nonzero().flatten()
            out[name] = _sparse(torch.stack((keys // E, keys % E)), dense[name][0][keys], (B, E))
        else:
            rows, cols, vals = _finalize_normalized(dense[name], B, E, 0, dev)
            out[name] = _sparse(torch.stack((rows, cols)), vals, (B, E))
    return {name: out[name].coalesce() for name in requested}


# ---------------------------------------------------------------------------
# evaluation inputs and metrics (rules/evaluate.py:122-128,737-854)

def build_evaluation(triples, num_relations, max_triples=None):
    """Each (h, r, t) as the query (h, r) -> t and (t, r + R) -> h."""
    rows = triples if max_triples is None else triples[:max_triples]
    out = []
    for h, r, t in rows:
        out.extend(((h, r, t), (t, r + num_relations, h)))
    return out


def build_split_known(valid, test, num_relations):
    """(source, query relation) -> the set of answers in valid and test."""
    from collections import defaultdict
    known = defaultdict(set)
    for h, r, t in list(valid) + list(test):
        known[(h, r)].add(t)
        known[(t, r + num_relations)].add(h)
    return known


@torch.inference_mode()
def filter_keys_for_batch_flashlog(csr, batch, sources, split_known, num_relations, num_entities,
                                   include_targets=True):
    """Sorted unique keys b*E + e of the filtered answers of every query b
    of the batch (rules/evaluate.py:746-780): its (source, relation)
    neighbours in the CSR -- one fixed-relation step of all queries at once
    -- plus its known valid/test answers and, with include_targets, its
    target."""
    E = int(num_entities)
    B = len(batch)
    dev = sources.device
    if B == 0:
        return torch.empty(0, dtype=torch.long, device=dev)
    rels = torch.tensor([[q[1]] for q in batch], dtype=torch.long, device=dev)
    step = vectorized_operation_sparse3d_fixed_relation(
        initial_rule_state(sources.reshape(-1)[:B], 1, E), rels, csr, num_relations)
    si = step.indices()
    parts = [si[0] * E + si[2]]
    extra = []
    for b, (source, relation, target) in enumerate(batch):
        answers = set(split_known.get((source, relation), ()))
        if include_targets:
            answers.add(target)
        extra.extend(b * E + int(x) for x in answers)
    if extra:
        parts.append(torch.tensor(extra, dtype=torch.long, device=dev))
    return torch.unique(torch.cat(parts), sorted=True)


def target_coverage(scores, targets):
    """Number of queries whose target has an explicit score."""
    scores = scores.coalesce()
    if scores._nnz() == 0:
        return 0
    idx = scores.indices()
    keys = idx[0] * scores.shape[1] + idx[1]  # coalesced: ascending
    want = torch.arange(scores.shape[0], device=targets.device) * scores.shape[1] + targets.long()
    pos = torch.searchsorted(keys, want).clamp(max=keys.numel() - 1)
    return int((keys[pos] == want).sum())


def select_sparse_score_row(scores, row):
    """Row `row` of a [B, E] tensor as a [1, E] tensor."""
    scores = scores.coalesce()
    idx = scores.indices()
    sel = idx[0] == row
    cols = idx[1][sel]
    return _sparse(torch.stack((torch.zeros_like(cols), cols)), scores.values()[sel], (1, scores.shape[1]))


def update_metrics(accumulator, scores, targets, filter_keys):
    """Adds the batch's filtered, tie-aware ranks (use_eql) and target
    coverage to the accumulator {"ranks": list, "covered_targets": int}."""
    scores = scores.coalesce()
    idx = scores.indices()
    ranks = sparse2d_filtered_ranks_cuda(idx[0], idx[1], scores.values(), targets, filter_keys, scores.shape[0],
                                         scores.shape[1], use_eql=True)
    accumulator["ranks"].extend(ranks.cpu().double().tolist())
    accumulator["covered_targets"] += target_coverage(scores, targets)


def finalize_metrics(accumulator):
    """MRR, Hits@1/3/10 and target coverage of the accumulated ranks."""
    r = np.asarray(accumulator["ranks"], dtype=np.float64)
    covered = int(accumulator["covered_targets"])
    if r.size == 0:
        return {"count": 0, "mrr": 0.0, "hit_1": 0.0, "hit_3": 0.0, "hit_10": 0.0,
                "covered_targets": covered, "target_coverage": 0.0}
    return {"count": int(r.size), "mrr": float(np.mean(1.0 / r)), "hit_1": float(np.mean(r <= 1)),
            "hit_3": float(np.mean(r <= 3)), "hit_10": float(np.mean(r <= 10)),
            "covered_targets": accumulator["covered_targets"], "target_coverage": covered / int(r.size)}
