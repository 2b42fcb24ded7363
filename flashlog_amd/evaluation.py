"""Evaluation consumers of the propagation (src/main.py:117-512): the
known-answer ("filter") indices of a query batch and the filtered ranking
metrics, with the reference driver's names, arguments and return values.

Known answers.  A lookup side holds, per (source, relation) group of a graph
direction, the group's targets in edge order: the group pointers, relations,
starts, counts and columns of one CSR side (the same arrays the propagation
uses).  A query (x, r) with r < R is looked up on the forward side under
(x, r), one with r >= R on the inverse side under (x, r - R); the reference
keys groups as source * R + relation (src/main.py:147-161,192-207) and a
query key is found by binary search (src/main.py:212-250).  On the GPU the
key is split back into (source, relation) and the relation is searched
among the source's groups (fl_filter_expand_count), then every (query,
known entity) pair is written by one thread (fl_filter_expand_fill).  The
pairs come out as the reference's: forward queries in batch order, then
inverse queries, each query's entities in the group's order (for a lookup
over a graph CSR, its CSR order; for lookups built from triple frames,
their edge order -- the reference sorts those keys with an unstable argsort,
so its order within one query is not fixed; every consumer uniques the keys).

Ranks.  calculate_hits_full_sparse and calculate_hits_full_with_filter_indices
compute the filtered tie-aware ranks on the GPU (sparse2d_filtered_ranks_cuda,
dense_filtered_ranks_cuda) and accumulate Hits@k and the reciprocal-rank sum
as the reference does (src/main.py:391-512).  Everything here runs on the GPU;
CPU inputs are moved to the lookup's GPU and results returned on the input's
device, as the reference returns them.
"""
import collections

import numpy as np
import torch

from . import _lib
from ._lib import check, ptr
from .flashlog_kernel import flashlog_kernel as fk

# One lookup side: a CSR side's group arrays and columns on the GPU, and the
# relation count R that query keys (source * R + relation) are formed with.
FilterSide = collections.namedtuple("FilterSide",
                                    "group_ptr group_rel group_start group_count columns relation_size")

_FILTER_CSR_LOOKUP_CACHE = {}


def _gpu_device(*tensors):
    for t in tensors:
        if torch.is_tensor(t) and t.is_cuda:
            return t.device
    if not torch.cuda.is_available():
        raise RuntimeError("flashlog_amd evaluation needs a ROCm GPU")
    return torch.device("cuda", torch.cuda.current_device())


def _empty(device):
    e = torch.empty(0, device=device, dtype=torch.long)
    return e, e


def _build_filter_edge_lookup(source, relation, target, relation_size):
    """Lookup side of the triples (source, relation, target)
    (src/main.py:147-161): targets grouped by (source, relation), in edge
    order within a group.  Built on the GPU by the CSR side builder."""
    dev = _gpu_device(source, relation, target)
    source, relation, target = (torch.as_tensor(x).to(device=dev, dtype=torch.long) for x in
                                (source, relation, target))
    if relation.numel() and (int(relation.min()) < 0 or int(relation.max()) >= int(relation_size)):
        raise ValueError("filter lookup: relation ids must lie in [0, relation_size)")
    nodes = int(torch.maximum(source.max(), target.max())) + 1 if source.numel() else 0
    (side,) = fk._gpu_csr_sides(source, target, relation, int(nodes), sides=((0, 1),))
    return FilterSide(side[4], side[5], side[6], side[7], side[1], int(relation_size))


def _frame_columns(frame):
    return tuple(torch.from_numpy(np.ascontiguousarray(frame[i].values)) for i in range(3))


def create_eval_filter_csr(dataset, entity_size, device):
    """Known-answer lookups of the training triples and of the held-out
    (valid + test) triples, each as a (forward, inverse) pair of sides
    (src/main.py:133-144); returns ({"filter_lookups": [...]}, None, None)."""
    import pandas as pd
    dev = torch.device(device) if device is not None else _gpu_device()
    if dev.type != "cuda":
        dev = _gpu_device()
    lookups = []
    for frame in (dataset.kg, pd.concat([dataset.valid_data, dataset.test_data], ignore_index=True)):
        h, r, t = (x.to(dev) for x in _frame_columns(frame))
        if r.numel() and (int(r.min()) < 0 or int(r.max()) >= int(dataset.relation_size)):
            raise ValueError("filter lookup: relation ids must lie in [0, relation_size)")
        ori, inv = fk._gpu_csr_sides(h, t, r, int(entity_size))
        R = int(dataset.relation_size)
        lookups.append((FilterSide(ori[4], ori[5], ori[6], ori[7], ori[1], R),
                        FilterSide(inv[4], inv[5], inv[6], inv[7], inv[1], R)))
    return {"filter_lookups": lookups}, None, None


def _filter_csr_cache_key(csr_struct, relation_size):
    """The reference's cache key (src/main.py:169-178): the relation count
    and the device, address, shape and dtype of the group and column fields."""
    fields = (1, 5, 8, 9, 10, 11, 12, 13, 14, 15)
    return (int(relation_size),
            tuple((str(csr_struct[i].device), int(csr_struct[i].data_ptr()), tuple(csr_struct[i].shape),
                   str(csr_struct[i].dtype)) for i in fields))


def _build_filter_side_lookup(row_group_ptr, group_rel, group_edge_start, group_edge_count, col_ind,
                              relation_size):
    """Lookup side over one CSR side's group arrays (src/main.py:181-200);
    the arrays are used in place (on the GPU; CPU arrays are copied there)."""
    dev = _gpu_device(row_group_ptr, group_rel, group_edge_start, group_edge_count, col_ind)
    return FilterSide(*(x.detach().to(device=dev).contiguous() for x in
                        (row_group_ptr, group_rel, group_edge_start, group_edge_count, col_ind)),
                      int(relation_size))


def _get_filter_csr_lookup(csr_struct, relation_size):
    """(forward, inverse) lookup of a 16-tuple CSR, cached by its arrays
    (src/main.py:203-224)."""
    key = _filter_csr_cache_key(csr_struct, relation_size)
    cached = _FILTER_CSR_LOOKUP_CACHE.get(key)
    if cached is None:
        cached = (_build_filter_side_lookup(csr_struct[8], csr_struct[9], csr_struct[10], csr_struct[11],
                                            csr_struct[1], relation_size),
                  _build_filter_side_lookup(csr_struct[12], csr_struct[13], csr_struct[14], csr_struct[15],
                                            csr_struct[5], relation_size))
        _FILTER_CSR_LOOKUP_CACHE[key] = cached
    return cached


def _expand_filter_side(batch_pos, query_key, lookup):
    """(batch positions, entities) of every known answer of the queries
    (src/main.py:227-267): per query key = source * R + relation the targets
    of that group of the side, queries in order."""
    side = lookup
    dev = side.group_ptr.device
    batch_pos = batch_pos.to(device=dev, dtype=torch.long).contiguous()
    query_key = query_key.to(device=dev, dtype=torch.long).contiguous()
    Q = query_key.numel()
    if Q == 0 or side.group_rel.numel() == 0:
        return _empty(dev)
    if batch_pos.numel() != Q:
        raise ValueError("_expand_filter_side: one batch position per query key")
    lib = _lib.lib()
    nodes = side.group_ptr.numel() - 1
    gptr = side.group_ptr.to(torch.int32).contiguous()
    grel = side.group_rel.to(torch.int16).contiguous()
    gstart = side.group_start.to(torch.int32).contiguous()
    gcount = side.group_count.to(torch.int32).contiguous()
    cols = side.columns.to(torch.int32).contiguous()
    ws_bytes = lib.fl_filter_expand_bytes(Q)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    off = torch.empty(Q + 1, dtype=torch.long, device=dev)
    st = fk._stream(off)
    check(lib.fl_filter_expand_count(st, ptr(gptr), ptr(grel), ptr(gcount), nodes, ptr(query_key),
                                     side.relation_size, Q, ptr(off), ptr(ws), ws_bytes), "filter_expand_count")
    total = int(off[Q])
    if total == 0:
        return _empty(dev)
    out_b = torch.empty(total, dtype=torch.long, device=dev)
    out_e = torch.empty(total, dtype=torch.long, device=dev)
    check(lib.fl_filter_expand_fill(st, ptr(gstart), ptr(cols), Q, ptr(off), ptr(batch_pos), total, ptr(ws),
                                    ptr(out_b), ptr(out_e)), "filter_expand_fill")
    return out_b, out_e


def _filter_indices_from_lookup(input_x, input_r, relation_size, lookup):
    """Known answers of a query batch (src/main.py:291-317): forward queries
    (r < R) on the forward side, then inverse queries on the inverse side,
    returned on the input's device."""
    ori_lookup, inv_lookup = lookup
    out_device = input_x.device
    dev = ori_lookup.group_ptr.device
    R = int(relation_size)
    x = input_x.detach().to(device=dev).long().reshape(-1)
    r = input_r.detach().to(device=dev).long().reshape(-1)
    batch_pos = torch.arange(x.numel(), dtype=torch.long, device=dev)
    ori_mask = r < R
    if ori_lookup.relation_size != R or inv_lookup.relation_size != R:
        raise ValueError("filter lookup was built for another relation_size")
    ori_b, ori_e = _expand_filter_side(batch_pos[ori_mask], x[ori_mask] * R + r[ori_mask], ori_lookup)
    inv_mask = ~ori_mask
    inv_b, inv_e = _expand_filter_side(batch_pos[inv_mask], x[inv_mask] * R + (r[inv_mask] - R), inv_lookup)
    if ori_b.numel() == 0 and inv_b.numel() == 0:
        return _empty(out_device)
    return (torch.cat([ori_b, inv_b]).to(out_device, non_blocking=True),
            torch.cat([ori_e, inv_e]).to(out_device, dtype=torch.long, non_blocking=True))


def build_filter_indices_csr(input_x, input_r, relation_size, csr_struct):
    """Known answers of a query batch from a graph CSR (the 16-tuple) or from
    create_eval_filter_csr's lookups (src/main.py:281-288)."""
    if isinstance(csr_struct, dict) and "filter_lookups" in csr_struct:
        results = [_filter_indices_from_lookup(input_x, input_r, relation_size, lookup)
                   for lookup in csr_struct["filter_lookups"]]
        return tuple(torch.cat([res[i] for res in results]) for i in range(2))
    return _filter_indices_from_lookup(input_x, input_r, relation_size,
                                       _get_filter_csr_lookup(csr_struct, relation_size))


_GRAPH_LOOKUP_CACHE = {}


def build_filter_indices_graph(batches, graph, graph_inv, dataset, device):
    """Known answers from the (head, relation) and (tail, relation) groupings
    of the triples (src/main.py:320-340): per batch item j in order, the
    tails of (h, r) or, for r >= R, the heads of (h, r - R), in frame order.
    The groupings' triples are looked up on the GPU as lookup sides."""
    R = int(dataset.relation_size)
    key = (id(graph), id(graph_inv), R)
    sides = _GRAPH_LOOKUP_CACHE.get(key)
    if sides is None:
        dev = torch.device(device) if device is not None else _gpu_device()
        dev = dev if dev.type == "cuda" else _gpu_device()
        h, r, t = _frame_columns(graph.obj)
        ori = _build_filter_edge_lookup(h.to(dev), r.to(dev), t.to(dev), R)
        h, r, t = _frame_columns(graph_inv.obj)
        inv = _build_filter_edge_lookup(t.to(dev), r.to(dev), h.to(dev), R)
        sides = _GRAPH_LOOKUP_CACHE[key] = (ori, inv, graph, graph_inv)
    ori, inv = sides[0], sides[1]
    dev = ori.group_ptr.device
    x = torch.tensor([int(it["h"]) for it in batches], dtype=torch.long, device=dev)
    r = torch.tensor([int(it["r"]) for it in batches], dtype=torch.long, device=dev)
    pos = torch.arange(x.numel(), dtype=torch.long, device=dev)
    fwd = r < R
    ob, oe = _expand_filter_side(pos[fwd], x[fwd] * R + r[fwd], ori)
    ib, ie = _expand_filter_side(pos[~fwd], x[~fwd] * R + (r[~fwd] - R), inv)
    b = torch.cat([ob, ib])
    if b.numel() == 0:
        return _empty(torch.device(device))
    order = torch.sort(b, stable=True).indices  # batch order; each item is on one side
    return b[order].to(device), torch.cat([oe, ie])[order].to(device)


def _targets(batches, device):
    return torch.tensor([int(it["t"]) for it in batches], dtype=torch.long, device=device)


def _hits_and_mrr(ranks, hits, float32_sum):
    """Adds Hits@k of the ranks into ``hits``; returns the reciprocal-rank sum
    as the reference forms it: a float32 numpy sum after the GPU rank kernel
    (src/main.py:416-420), a Python float loop after the dense ranks
    (src/main.py:507-511)."""
    ranks_cpu = ranks.detach().cpu().numpy()
    for rank_value in ranks_cpu:
        hits += (float(rank_value) <= np.arange(1, len(hits) + 1))
    if float32_sum:
        return float((1.0 / ranks_cpu).sum())
    mrr = 0
    for rank_value in ranks_cpu.tolist():
        mrr += 1 / rank_value
    return mrr


def _sparse_truth_scores(state, targets):
    """Each query's score at its target in a [B, E] sparse state
    (src/main.py:343-362), 0 where the target holds no entry."""
    fk._require_cuda(state)
    state = state.coalesce()
    idx = state.indices()
    values = state.values()
    B, E = state.shape
    truth = torch.zeros(B, device=values.device, dtype=values.dtype)
    if values.numel() == 0:
        return truth
    keys = idx[0] * E + idx[1]  # coalesced: ascending
    target_keys = torch.arange(B, device=values.device) * E + targets.to(values.device).long()
    pos = torch.searchsorted(keys, target_keys)
    safe = pos.clamp(max=keys.numel() - 1)
    hit = (pos < keys.numel()) & (keys[safe] == target_keys)
    truth[hit] = values[safe[hit]]
    return truth


def calculate_raw_hits_sparse(state, batches, hits):
    """Unfiltered ranks counting every tie (src/main.py:365-388): rank =
    #entries >= the target's score, plus the implicit zeros when the target
    scores <= 0.  Adds Hits@k into ``hits`` and returns the reciprocal-rank
    sum."""
    fk._require_cuda(state)
    state = state.coalesce()
    idx = state.indices()
    values = state.values()
    B, E = state.shape
    truth = _sparse_truth_scores(state, _targets(batches, values.device))
    explicit = torch.zeros(B, device=values.device, dtype=values.dtype)
    ge = torch.zeros(B, device=values.device, dtype=values.dtype)
    if values.numel():
        explicit.scatter_add_(0, idx[0], torch.ones_like(values))
        ge.scatter_add_(0, idx[0], (values >= truth[idx[0]]).to(values.dtype))
    ranks = ge + torch.where(truth <= 0, E - explicit, torch.zeros_like(explicit))
    mrr = 0.0
    for rank in ranks.detach().cpu().tolist():
        rank = int(rank)
        hits[rank - 1:] += 1
        mrr += 1.0 / rank
    return mrr


def calculate_hits_full_sparse(state, batches, filter_indices, hits, use_eql=False):
    """Filtered tie-aware ranks over a [B, E] sparse score state
    (src/main.py:391-465) on the GPU rank kernel; the targets join the known
    answers and duplicate keys count once."""
    fk._require_cuda(state)
    if not state.is_coalesced():
        state = state.coalesce()
    idx = state.indices()
    values = state.values()
    B, E = state.shape
    dev = values.device
    targets = _targets(batches, dev)
    target_keys = torch.arange(B, device=dev, dtype=torch.long) * E + targets
    if filter_indices is None:
        keys = target_keys
    else:
        fb, fe = filter_indices
        keys = torch.cat([fb.to(dev).long() * E + fe.to(dev).long(), target_keys])
    keys = torch.unique(keys, sorted=True)
    ranks = fk.sparse2d_filtered_ranks_cuda(idx[0], idx[1], values, targets, keys, B, E, use_eql=use_eql)
    return _hits_and_mrr(ranks, hits, True)


def calculate_hits_full_with_filter_indices(state, batches, filter_indices, hits, use_eql=False):
    """Filtered tie-aware ranks over a dense [B, E] score matrix
    (src/main.py:468-512) on the GPU rank kernel."""
    ranks = fk.dense_filtered_ranks_cuda(state, _targets(batches, state.device), filter_indices, use_eql=use_eql)
    return _hits_and_mrr(ranks, hits, False)
