"""Drop-in mirror of the reference operator API ``flashlog_kernel.flashlog_kernel``
(flashlog_kernel/flashlog_kernel.py in qikunxun/FlashLog), running on the
gfx950 HIP library ``libflashlog_hip.so`` through its C-ABI.

Every public name, positional order, default and return type follows the
reference; each definition cites the reference lines it mirrors.  The
internals are this library's: the dense hop is a destination-major pull with
a per-source frontier (no atomics on outputs, bit-identical to the
reference's CPU accumulation order).

This module has no CPU compute path: CPU tensors raise, and a missing or
stale HIP library raises.  (The reference's CPU kernels are the oracle this
library is tested against, not part of it.)
"""
import ctypes
import os
import weakref

import numpy as np
import torch
from torch import autograd

from .. import _lib
from .._lib import FlSide, check, ptr, stream_handle

_FLASHLOG_CPU_THREADS_CONFIGURED = False


# ---------------------------------------------------------------------------
# CPU thread configuration (flashlog_kernel.py:13-102).  Kept for callers of
# the reference API; it only adjusts torch's intra-op thread count.

def _flashlog_available_logical_cpus():
    try:
        return len(os.sched_getaffinity(0))
    except Exception:
        return os.cpu_count() or 1


def _flashlog_physical_cores():
    try:
        cores = set()
        phys = core = None
        with open("/proc/cpuinfo") as f:
            for line in f:
                line = line.strip()
                if not line:
                    if phys is not None and core is not None:
                        cores.add((phys, core))
                    phys = core = None
                elif line.startswith("physical id"):
                    phys = line.split(":", 1)[1].strip()
                elif line.startswith("core id"):
                    core = line.split(":", 1)[1].strip()
        if phys is not None and core is not None:
            cores.add((phys, core))
        return len(cores) or None
    except Exception:
        return None


def _choose_flashlog_cpu_threads():
    logical = max(1, _flashlog_available_logical_cpus())
    physical = _flashlog_physical_cores() or max(1, logical // 2 if logical >= 8 else logical)
    usable = min(physical, logical)
    if logical >= 96:
        return min(32, max(16, usable // 2))
    if logical >= 48:
        return min(24, max(12, usable // 2))
    if logical >= 24:
        return min(16, max(8, usable))
    return max(1, logical)


def configure_flashlog_cpu_threads(force=False):
    """FLASHLOG_CPU_THREADS: unset/off/0/false leaves torch alone, ``auto``
    picks a bandwidth-friendly count, an integer forces it
    (flashlog_kernel.py:60-102)."""
    global _FLASHLOG_CPU_THREADS_CONFIGURED
    if _FLASHLOG_CPU_THREADS_CONFIGURED and not force:
        return torch.get_num_threads()
    setting = os.environ.get("FLASHLOG_CPU_THREADS", "off").strip().lower()
    if setting in ("", "auto"):
        target = _choose_flashlog_cpu_threads()
    elif setting in ("off", "none", "false", "0"):
        _FLASHLOG_CPU_THREADS_CONFIGURED = True
        return torch.get_num_threads()
    else:
        try:
            target = int(setting)
        except ValueError:
            target = _choose_flashlog_cpu_threads()
    target = max(1, min(target, _flashlog_available_logical_cpus()))
    if torch.get_num_threads() != target:
        torch.set_num_threads(target)
    interop = os.environ.get("FLASHLOG_CPU_INTEROP_THREADS")
    if interop is not None:
        try:
            n = max(1, int(interop))
            if torch.get_num_interop_threads() != n:
                torch.set_num_interop_threads(n)
        except (ValueError, RuntimeError):
            pass
    _FLASHLOG_CPU_THREADS_CONFIGURED = True
    return torch.get_num_threads()


def _require_cuda(*tensors):
    for t in tensors:
        if torch.is_tensor(t) and not t.is_cuda:
            raise RuntimeError("flashlog_amd runs on the GPU only; got a CPU tensor")


def _stream(t):
    return stream_handle(t.device)


# ---------------------------------------------------------------------------
# Graph preparation

def _ind2ptr_cpu(index, size):
    """int32 CSR offsets of a sorted index (flashlog_kernel.py:626-634)."""
    counts = torch.bincount(index, minlength=size)
    np.cumsum(counts.numpy(), out=counts.numpy())
    out = torch.empty(size + 1, dtype=torch.int32)
    out[0] = 0
    out[1:].copy_(counts)
    return out


def _group_starts_and_counts(sorted_values, sorted_relations=None):
    """Starts and lengths of runs of equal (value[, relation])
    (flashlog_kernel.py:637-661)."""
    n = sorted_values.numel()
    if not n:
        return torch.empty(0, dtype=torch.int32), torch.empty(0, dtype=torch.int32)
    v = sorted_values.numpy() if sorted_values.device.type == "cpu" else sorted_values.cpu().numpy()
    fresh = np.empty(n, bool)
    fresh[0] = True
    np.not_equal(v[1:], v[:-1], out=fresh[1:])
    if sorted_relations is not None:
        r = sorted_relations.cpu().numpy()
        fresh[1:] |= r[1:] != r[:-1]
    starts = np.nonzero(fresh)[0].astype(np.int32)
    counts = np.empty_like(starts)
    counts[:-1] = starts[1:] - starts[:-1]
    counts[-1] = n - starts[-1]
    return torch.from_numpy(starts), torch.from_numpy(counts)


def _build_group_metadata(sorted_rows, sorted_rels, num_nodes, row_ptr=None):
    """(group_ptr, relations, starts, counts) of a CSR side sorted by
    (row, relation) (flashlog_kernel.py:664-673)."""
    starts, counts = _group_starts_and_counts(sorted_rows, sorted_rels)
    relations = sorted_rels[starts.long()].to(torch.int16) if starts.numel() else \
        torch.empty(0, dtype=torch.int16)
    if row_ptr is None:
        row_ptr = _ind2ptr_cpu(sorted_rows, num_nodes)
    group_ptr = torch.searchsorted(starts, row_ptr, out_int32=True)
    return group_ptr, relations, starts, counts


def build_csr_structure(row_indices, col_indices, r_indices, num_nodes):
    """The reference's 16-tuple (flashlog_kernel.py:678-697; csr.cpp:12-69):
    (ori_row_ptr, ori_col_ind, ori_r_ind, order_ori, inv_..., ori_row_group_ptr,
    ori_group_rel, ori_group_edge_start, ori_group_edge_count, inv_...),
    built by the library's host CSR builder and moved to the input's device."""
    device = row_indices.device
    row, col, rel = [x.detach().to(device="cpu", dtype=torch.int64).contiguous()
                     for x in (row_indices, col_indices, r_indices)]
    if not (row.dim() == col.dim() == rel.dim() == 1) or not (row.numel() == col.numel() == rel.numel()):
        raise ValueError("CSR requires equal 1D arrays and int32-sized graph")
    nodes = int(num_nodes)

    def side(source, target):
        m = source.numel()
        row_ptr = torch.empty(nodes + 1, dtype=torch.int32)
        cols = torch.empty(m, dtype=torch.int32)
        erel = torch.empty(m, dtype=torch.int16)
        order = torch.empty(m, dtype=torch.int32)
        gptr = torch.empty(nodes + 1, dtype=torch.int32)
        grel = torch.empty(max(m, 1), dtype=torch.int16)
        gstart = torch.empty(max(m, 1), dtype=torch.int32)
        gcount = torch.empty(max(m, 1), dtype=torch.int32)
        ng = ctypes.c_int64(0)
        rc = _lib.lib().fl_csr_build_side(m, nodes, ptr(source), ptr(target), ptr(rel), ptr(row_ptr),
                                          ptr(cols), ptr(erel), ptr(order), ptr(gptr), ptr(grel),
                                          ptr(gstart), ptr(gcount), ctypes.byref(ng))
        if rc != 0:
            raise ValueError(_lib.lib().fl_last_error().decode())
        g = ng.value
        arrays = (row_ptr, cols, erel, order, gptr, grel[:g].clone(), gstart[:g].clone(), gcount[:g].clone())
        return tuple(a.to(device) for a in arrays)

    ori = side(row, col)
    inv = side(col, row)
    return (*ori[:4], *inv[:4], *ori[4:], *inv[4:])


class _PullSide:
    """Destination-major index of one CSR side, resident on the device."""

    def __init__(self, col_ind, row_group_ptr, group_rel, group_start, group_count):
        device = col_ind.device
        nodes = row_group_ptr.numel() - 1
        m = col_ind.numel()
        g = group_rel.numel()
        host = [t.detach().to("cpu").contiguous() for t in
                (col_ind.int(), row_group_ptr.int(), group_rel.short(), group_start.int(), group_count.int())]
        pull_ptr = torch.empty(nodes + 1, dtype=torch.int32)
        pull_pos = torch.empty(m, dtype=torch.int32)
        pull_src = torch.empty(m, dtype=torch.int32)
        pull_rel = torch.empty(m, dtype=torch.int16)
        check(_lib.lib().fl_pull_index_build(nodes, m, g, *[ptr(t) for t in host], ptr(pull_ptr),
                                             ptr(pull_pos), ptr(pull_src), ptr(pull_rel)), "pull_index_build")
        counts = [ctypes.c_int64(0) for _ in range(3)]
        check(_lib.lib().fl_pull_segments(nodes, ptr(pull_ptr), *[ctypes.byref(c) for c in counts],
                                          *([None] * 8)), "pull_segments")
        nseg, nheavy, nsup = (c.value for c in counts)
        arrays = [torch.empty(k, dtype=torch.int32) for k in
                  (nseg, nseg, nseg, nheavy, nheavy + 1, nheavy + 1, nsup, nsup)]
        check(_lib.lib().fl_pull_segments(nodes, ptr(pull_ptr), *[ctypes.byref(c) for c in counts],
                                          *[ptr(a) for a in arrays]), "pull_segments")
        self.nseg, self.nheavy, self.nsup = nseg, nheavy, nsup
        (self.seg_dst, self.seg_start, self.seg_h, self.heavy_dst, self.heavy_seg_ptr, self.heavy_sup_ptr,
         self.sup_h, self.sup_seg0) = [a.to(device) for a in arrays]
        self.edges, self.groups, self.nodes = m, g, nodes
        self.max_rel = int(host[2].max()) if g else -1
        self.col_ind = col_ind.int().contiguous()
        self.row_group_ptr = row_group_ptr.int().contiguous()
        self.group_rel = group_rel.short().contiguous()
        self.group_start = group_start.int().contiguous()
        self.group_count = group_count.int().contiguous()
        self.pull_ptr = pull_ptr.to(device)
        self.pull_pos = pull_pos.to(device)
        self.pull_src = pull_src.to(device)
        self.pull_rel = pull_rel.to(device)
        pos_src = torch.empty(m, dtype=torch.int32)
        pos_rel = torch.empty(m, dtype=torch.int16)
        pidx = pull_pos.long()
        pos_src[pidx] = pull_src
        pos_rel[pidx] = pull_rel
        self.pos_src = pos_src.to(device)
        self.pos_rel = pos_rel.to(device)

    def struct(self, mask):
        return FlSide(self.edges, self.groups, self.col_ind.data_ptr(), mask.data_ptr() if mask.numel() else 0,
                      self.row_group_ptr.data_ptr(), self.group_rel.data_ptr() if self.groups else 0,
                      self.group_start.data_ptr() if self.groups else 0,
                      self.group_count.data_ptr() if self.groups else 0,
                      self.pull_ptr.data_ptr(), self.pull_pos.data_ptr() if self.edges else 0,
                      self.pull_src.data_ptr() if self.edges else 0,
                      self.pull_rel.data_ptr() if self.edges else 0,
                      self.nseg, self.nheavy, self.nsup, *[t.data_ptr() if t.numel() else 0 for t in (
                          self.seg_dst, self.seg_start, self.seg_h, self.heavy_dst, self.heavy_seg_ptr,
                          self.heavy_sup_ptr, self.sup_h, self.sup_seg0, self.pos_src, self.pos_rel)])


class _Graph:
    def __init__(self, ori_args, inv_args):
        self.ori = _PullSide(*ori_args)
        self.inv = _PullSide(*inv_args)


_GRAPHS = {}


def _graph_for(ori_col, ori_gptr, ori_grel, ori_gstart, ori_gcount,
               inv_col, inv_gptr, inv_grel, inv_gstart, inv_gcount):
    keyed = (ori_col, ori_gptr, ori_gstart, inv_col, inv_gptr, inv_gstart)
    key = tuple((t.data_ptr(), t.numel(), t._version) for t in keyed) + (str(ori_col.device),)
    hit = _GRAPHS.get(key)
    if hit is not None:
        refs, graph = hit
        if all(r() is t for r, t in zip(refs, keyed)):
            return graph
    for k in [k for k, (refs, _) in _GRAPHS.items() if any(r() is None for r in refs)]:
        del _GRAPHS[k]
    graph = _Graph((ori_col, ori_gptr, ori_grel, ori_gstart, ori_gcount),
                   (inv_col, inv_gptr, inv_grel, inv_gstart, inv_gcount))
    _GRAPHS[key] = (tuple(weakref.ref(t) for t in keyed), graph)
    return graph


# ---------------------------------------------------------------------------
# Masks (flashlog_kernel.py:221-255)

def score_function(x):
    return torch.sigmoid(x)


def _prepared_mask_pair(mask_values):
    if (isinstance(mask_values, (tuple, list)) and len(mask_values) == 2 and
            torch.is_tensor(mask_values[0]) and torch.is_tensor(mask_values[1])):
        return mask_values[0].contiguous().float(), mask_values[1].contiguous().float()
    return None


def _apply_mask_order(mask_values, order, weight=None):
    mask_f = (mask_values if mask_values.dtype == torch.bool else mask_values.float()).contiguous().view(-1)
    _require_cuda(mask_f)
    return _HipModule.apply_mask_cuda(
        mask_f, order.to(device=mask_f.device, dtype=torch.int32).contiguous(),
        torch.empty(0, device=mask_f.device) if weight is None else
        weight.to(device=mask_f.device, dtype=torch.float).squeeze(-1).contiguous())


def prepare_csr_masks(csr_struct, mask_values, weight=None):
    """CSR-ordered ORI/INV masks, prepared once per model forward."""
    return (_apply_mask_order(mask_values, csr_struct[3], weight),
            _apply_mask_order(mask_values, csr_struct[7], weight))


def _compute_active_nodes(A):
    """Sorted unique entities with a nonzero in any row of A [B, L, E]
    (flashlog_kernel.py:617-623)."""
    _require_cuda(A)
    flat = A.reshape(-1, A.shape[-1]).contiguous().float()
    return _HipModule.compute_active_nodes_cuda(flat)


# ---------------------------------------------------------------------------
# c1 entity budget on dense states (flashlog_kernel.py:814-842)

class _DenseTopC(autograd.Function):
    """A * keep, keep = the c largest nonzeros of each over-budget (item,
    rule) row, ties at the cutoff to the smaller entity; rows within budget
    keep everything.  Backward: grad * keep."""

    @staticmethod
    def forward(ctx, A, c):
        if A.dtype != torch.float32:
            raise TypeError("flashlog_amd dense states are float32")
        shape = A.shape
        E = shape[-1]
        flat = A.reshape(-1, E).contiguous()
        BL = flat.shape[0]
        out = torch.empty_like(flat)
        state = torch.empty(BL * 4, dtype=torch.int32, device=A.device)
        check(_lib.lib().fl_dense_topc(_stream(A), ptr(flat), ptr(out), BL, E, int(c), ptr(state)),
              "dense_topc")
        ctx.save_for_backward(flat, state)
        ctx.shape = shape
        return out.view(shape)

    @staticmethod
    def backward(ctx, grad):
        flat, state = ctx.saved_tensors
        BL, E = flat.shape
        g = grad.reshape(BL, E).contiguous().float()
        gA = torch.empty_like(flat)
        check(_lib.lib().fl_dense_topc_backward(_stream(g), ptr(g), ptr(flat), ptr(state), ptr(gA), BL, E),
              "dense_topc_backward")
        return gA.view(ctx.shape), None


def _dense_topc_state(A, topk_nodes):
    """Prune graph sources per (item, rule) row to the c1 budget.  The
    selection is detached; gradients flow only through admitted sources."""
    if topk_nodes is None:
        return A
    if topk_nodes < 0:
        raise ValueError("topk_nodes/c must be nonnegative")
    if topk_nodes >= A.shape[-1]:
        return A
    _require_cuda(A)
    return _DenseTopC.apply(A, int(topk_nodes))


# ---------------------------------------------------------------------------
# The native-module surface (get_module(), flashlog_kernel.py:212-218)

class _HipModule:
    """Reference pybind names (flashlog.cpp:1935-1965) backed by the C-ABI."""

    @staticmethod
    def apply_mask_cuda(mask_values, order, weight):
        _require_cuda(mask_values, order)
        order = order.to(torch.int32).contiguous()
        nnz = order.numel()
        out = torch.empty(nnz, dtype=torch.float32, device=mask_values.device)
        if nnz == 0:
            return out
        if mask_values.dtype not in (torch.bool, torch.float32):
            raise RuntimeError("edge visibility mask must be bool or float32")
        has_w = weight is not None and weight.numel() > 0
        check(_lib.lib().fl_apply_mask(_stream(out), ptr(mask_values.contiguous()),
                                       1 if mask_values.dtype == torch.bool else 0, ptr(order),
                                       ptr(weight.float().contiguous()) if has_w else None, ptr(out), nnz),
              "apply_mask")
        return out

    @staticmethod
    def compute_active_nodes_cuda(A_flat):
        _require_cuda(A_flat)
        BL, E = A_flat.shape
        flags = torch.empty(E, dtype=torch.int32, device=A_flat.device)
        check(_lib.lib().fl_mark_active(_stream(A_flat), ptr(A_flat.contiguous().float()), BL, E, ptr(flags)),
              "mark_active")
        return flags.nonzero().reshape(-1).to(torch.long)

    @staticmethod
    def flashlog_forward_cuda(A, w, active_nodes,
                              ori_row_ptr, ori_col_ind, ori_r_ind, ori_mask,
                              inv_row_ptr, inv_col_ind, inv_r_ind, inv_mask,
                              ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
                              inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
                              r_size, wot_i, use_topk, topk_edges, agg_mode):
        """flashlog.cu:898-995 (agg_mode 0).  ``active_nodes`` is accepted
        for signature compatibility; the frontier is derived from A."""
        if int(agg_mode) != 0:
            raise NotImplementedError("agg_mode=max on the sum entry point: use dense_csr_max")
        graph = _graph_for(ori_col_ind, ori_row_group_ptr, ori_group_rel, ori_group_edge_start,
                           ori_group_edge_count, inv_col_ind, inv_row_group_ptr, inv_group_rel,
                           inv_group_edge_start, inv_group_edge_count)
        K = int(topk_edges) if use_topk else 0
        return _dense_sum_forward(A, w, graph, ori_mask.float().contiguous(), inv_mask.float().contiguous(),
                                  int(r_size), bool(wot_i), K)


_module = _HipModule()


def get_module():
    """The native module: this library's C-ABI behind the reference names."""
    _lib.lib()
    return _module


def _dense_check(A_flat, w_flat, graph, ori_mask, inv_mask, r_size):
    _require_cuda(A_flat, w_flat, ori_mask, inv_mask)
    if A_flat.dtype != torch.float32 or w_flat.dtype != torch.float32:
        raise TypeError("flashlog_amd dense propagation computes in float32")
    BL, E = A_flat.shape
    n = w_flat.shape[1]
    if w_flat.shape[0] != BL:
        raise ValueError("w must have one row per state row")
    if graph.ori.nodes != E or graph.inv.nodes != E:
        raise ValueError("CSR has %d nodes, state has %d entities" % (graph.ori.nodes, E))
    if ori_mask.numel() != graph.ori.edges or inv_mask.numel() != graph.inv.edges:
        raise ValueError("mask length must equal the number of CSR positions")
    if max(graph.ori.max_rel, graph.inv.max_rel) >= r_size or 2 * r_size > n:
        raise ValueError("relation ids must be < r_size and w must hold 2*r_size (+1) columns")
    return BL, E, n


def _dense_sum_forward(A_flat, w_flat, graph, ori_mask, inv_mask, r_size, wot_i, K):
    A_flat = A_flat.contiguous()
    w_flat = w_flat.contiguous()
    BL, E, n = _dense_check(A_flat, w_flat, graph, ori_mask, inv_mask, r_size)
    out_ind = torch.empty_like(A_flat)
    out_ori = torch.empty_like(A_flat)
    out_inv = torch.empty_like(A_flat)
    so = graph.ori.struct(ori_mask)
    si = graph.inv.struct(inv_mask)
    ws_bytes = _lib.lib().fl_dense_workspace_bytes(ctypes.byref(so), ctypes.byref(si), BL, E)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=A_flat.device)
    check(_lib.lib().fl_dense_sum_forward(_stream(A_flat), ctypes.byref(so), ctypes.byref(si), ptr(A_flat),
                                          ptr(w_flat), BL, E, n, r_size, 1 if wot_i else 0, int(K),
                                          ptr(out_ind), ptr(out_ori), ptr(out_inv), ptr(ws), ws_bytes),
          "dense_sum_forward")
    return out_ind, out_ori, out_inv


def _dense_max_forward(A_flat, w_flat, graph, ori_mask, inv_mask, r_size, wot_i, K):
    """flashlog_forward_max_cuda (flashlog.cu:997-1072): values and int64
    winning CSR positions (-1 where nothing arrives)."""
    A_flat = A_flat.contiguous()
    w_flat = w_flat.contiguous()
    BL, E, n = _dense_check(A_flat, w_flat, graph, ori_mask, inv_mask, r_size)
    out_ind = torch.empty_like(A_flat)
    out_ori = torch.empty_like(A_flat)
    out_inv = torch.empty_like(A_flat)
    arg_ori = torch.empty((BL, E), dtype=torch.int64, device=A_flat.device)
    arg_inv = torch.empty((BL, E), dtype=torch.int64, device=A_flat.device)
    so = graph.ori.struct(ori_mask)
    si = graph.inv.struct(inv_mask)
    ws_bytes = _lib.lib().fl_dense_workspace_bytes(ctypes.byref(so), ctypes.byref(si), BL, E)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=A_flat.device)
    check(_lib.lib().fl_dense_max_forward(_stream(A_flat), ctypes.byref(so), ctypes.byref(si), ptr(A_flat),
                                          ptr(w_flat), BL, E, n, r_size, 1 if wot_i else 0, int(K),
                                          ptr(out_ind), ptr(out_ori), ptr(out_inv), ptr(arg_ori), ptr(arg_inv),
                                          ptr(ws), ws_bytes),
          "dense_max_forward")
    return out_ind, out_ori, out_inv, arg_ori, arg_inv


def _dense_max_backward(grad_ind, grad_ori, grad_inv, arg_ori, arg_inv, A_f, w_f, graph, om, im, r_size, wot_i):
    """flashlog_backward_max_cuda (flashlog.cu:1187-1255)."""
    BL, E = A_f.shape
    n = w_f.shape[1]

    def g(x):
        if x is None:
            return torch.zeros_like(A_f)
        return x.reshape(BL, E).contiguous().float()

    gi, go, gv = g(grad_ind), g(grad_ori), g(grad_inv)
    so = graph.ori.struct(om)
    si = graph.inv.struct(im)
    gA = torch.empty_like(A_f)
    gw = torch.empty_like(w_f)
    check(_lib.lib().fl_dense_max_backward(_stream(A_f), ctypes.byref(so), ctypes.byref(si), ptr(A_f), ptr(w_f),
                                           ptr(gi), ptr(go), ptr(gv), ptr(arg_ori), ptr(arg_inv), BL, E, n,
                                           r_size, 1 if wot_i else 0, ptr(gA), ptr(gw)),
          "dense_max_backward")
    return gA, gw


# ---------------------------------------------------------------------------
# Dense autograd functions

class FlashLogFunction(autograd.Function):
    """Dense propagation with precomputed active nodes and CSR-ordered masks
    (flashlog_kernel.py:700-811)."""

    @staticmethod
    def forward(ctx, A, w, active_nodes,
                ori_col_ind, ori_mask,
                ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
                inv_col_ind, inv_mask,
                inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
                r_size, wot_i, topk_edges):
        _require_cuda(A, w)
        B, L, E = A.shape
        graph = _graph_for(ori_col_ind, ori_row_group_ptr, ori_group_rel, ori_group_edge_start,
                           ori_group_edge_count, inv_col_ind, inv_row_group_ptr, inv_group_rel,
                           inv_group_edge_start, inv_group_edge_count)
        A_f = A.reshape(B * L, E).contiguous().float()
        w_f = w.reshape(B * L, -1).contiguous().float()
        om, im = ori_mask.float().contiguous(), inv_mask.float().contiguous()
        K = int(topk_edges) if 0 < int(topk_edges) < (1 << 60) else 0
        out_ind, out_ori, out_inv = _dense_sum_forward(A_f, w_f, graph, om, im, int(r_size), bool(wot_i), K)
        ctx.save_for_backward(A_f, w_f, om, im)
        ctx.graph, ctx.r_size, ctx.wot_i, ctx.K, ctx.shape = graph, int(r_size), bool(wot_i), K, (B, L, E)
        return out_ind.view(B, L, E), out_ori.view(B, L, E), out_inv.view(B, L, E)

    @staticmethod
    def backward(ctx, grad_ind, grad_ori, grad_inv):
        A_f, w_f, om, im = ctx.saved_tensors
        gA, gw = _dense_sum_backward(grad_ind, grad_ori, grad_inv, A_f, w_f, ctx.graph, om, im,
                                     ctx.r_size, ctx.wot_i, ctx.K)
        B, L, E = ctx.shape
        return (gA.view(B, L, E), gw.view(B, L, -1)) + (None,) * 16


_DENSE_BACKWARD_ENABLED = False


def _dense_sum_backward(grad_ind, grad_ori, grad_inv, A_f, w_f, graph, om, im, r_size, wot_i, K):
    """flashlog_backward_cuda (flashlog.cu:1077-1185) with the CPU path's
    order (flashlog.cpp:216-278): grad_A bit-identical, grad_w in a fixed
    order (within float rounding of the CPU sum).

    Disabled: an earlier build of this path faulted the GPU (k_col_count
    wrote the identity output through the null pointer the backward passes);
    the store is now guarded, and the path stays off until a GPU run has
    verified it."""
    if not _DENSE_BACKWARD_ENABLED:
        raise RuntimeError("dense sum backward is disabled: its GPU kernels are awaiting verification "
                           "after a memory fault (null identity-output store, now fixed)")
    BL, E = A_f.shape
    n = w_f.shape[1]

    def g(x):
        if x is None:
            return torch.zeros_like(A_f)
        return x.reshape(BL, E).contiguous().float()

    gi, go, gv = g(grad_ind), g(grad_ori), g(grad_inv)
    so = graph.ori.struct(om)
    si = graph.inv.struct(im)
    ws_bytes = _lib.lib().fl_dense_backward_workspace_bytes(ctypes.byref(so), ctypes.byref(si), BL, E)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=A_f.device)
    gA = torch.empty_like(A_f)
    gw = torch.empty_like(w_f)
    pairs = int(torch.count_nonzero(A_f))  # nonzero (row, source) pairs: rows of the partial buffer
    pg = torch.empty(max(pairs, 1) * n, dtype=torch.float32, device=A_f.device)
    check(_lib.lib().fl_dense_sum_backward(_stream(A_f), ctypes.byref(so), ctypes.byref(si), ptr(A_f), ptr(w_f),
                                           ptr(gi), ptr(go), ptr(gv), BL, E, n, r_size, 1 if wot_i else 0, int(K),
                                           ptr(gA), ptr(gw), ptr(pg), pairs, ptr(ws), ws_bytes),
          "dense_sum_backward")
    return gA, gw


def vectorized_operation_csr(A, w, csr_struct, mask_values, r_size,
                             weight=None, wot_i=False,
                             use_topk=False, topk_nodes=100000, topk_edges=0,
                             prepared_masks=None):
    """Dense entry point of the reference's CPU path (flashlog_kernel.py:845-882);
    here it runs the same arithmetic on the GPU."""
    (ori_row_ptr, ori_col_ind, ori_r_ind, order_ori,
     inv_row_ptr, inv_col_ind, inv_r_ind, order_inv,
     ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
     inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count) = csr_struct
    prepared = _prepared_mask_pair(prepared_masks) if prepared_masks is not None else _prepared_mask_pair(mask_values)
    if prepared is not None:
        ori_mask, inv_mask = prepared
    else:
        ori_mask, inv_mask = prepare_csr_masks(csr_struct, mask_values, weight)
    A = _dense_topc_state(A, topk_nodes if use_topk else None)
    effective_topk = topk_edges if (use_topk and topk_edges > 0) else (1 << 60)
    return FlashLogFunction.apply(
        A, w, None,
        ori_col_ind, ori_mask,
        ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
        inv_col_ind, inv_mask,
        inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
        r_size, wot_i, effective_topk)


class FlashLogDenseSumFunction(autograd.Function):
    """GPU dense sum hop (flashlog_kernel.py:885-989)."""

    @staticmethod
    def forward(ctx, A, w, ori_row_ptr, ori_col_ind, ori_r_ind, ori_order,
                inv_row_ptr, inv_col_ind, inv_r_ind, inv_order,
                ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
                inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
                mask_values, weight, r_size, wot_i,
                use_topk, topk_nodes, topk_edges, agg_mode):
        _require_cuda(A, w)
        if int(agg_mode) != 0:
            raise NotImplementedError("agg_mode=max on the sum entry point: use dense_csr_max")
        B, L, E = A.shape
        BL = B * L
        A_flat = A.reshape(BL, E).contiguous().float()
        w_flat = w.reshape(BL, -1).contiguous().float()
        prepared = _prepared_mask_pair(mask_values)
        if prepared is not None:
            ori_mask, inv_mask = prepared
        else:
            mask_f = (mask_values if mask_values.dtype == torch.bool else mask_values.float()).contiguous()
            w_tensor = weight.to(device=A.device, dtype=torch.float).squeeze(-1) if weight is not None \
                else torch.empty(0, device=A.device)
            ori_mask = _HipModule.apply_mask_cuda(mask_f, ori_order, w_tensor)
            inv_mask = _HipModule.apply_mask_cuda(mask_f, inv_order, w_tensor)
        graph = _graph_for(ori_col_ind, ori_row_group_ptr, ori_group_rel, ori_group_edge_start,
                           ori_group_edge_count, inv_col_ind, inv_row_group_ptr, inv_group_rel,
                           inv_group_edge_start, inv_group_edge_count)
        K = int(topk_edges) if (use_topk and 0 < int(topk_edges) < (1 << 60)) else 0
        out_ind, out_ori, out_inv = _dense_sum_forward(A_flat, w_flat, graph, ori_mask, inv_mask,
                                                       int(r_size), bool(wot_i), K)
        ctx.save_for_backward(A_flat, w_flat, ori_mask, inv_mask)
        ctx.graph, ctx.r_size, ctx.wot_i, ctx.K, ctx.shape = graph, int(r_size), bool(wot_i), K, (B, L, E)
        return out_ind.view(B, L, E), out_ori.view(B, L, E), out_inv.view(B, L, E)

    @staticmethod
    def backward(ctx, grad_ind, grad_ori, grad_inv):
        A_f, w_f, om, im = ctx.saved_tensors
        gA, gw = _dense_sum_backward(grad_ind, grad_ori, grad_inv, A_f, w_f, ctx.graph, om, im,
                                     ctx.r_size, ctx.wot_i, ctx.K)
        B, L, E = ctx.shape
        return (gA.view(B, L, E), gw.view(B, L, -1)) + (None,) * 24


def dense_csr_sum_cuda(A, w, csr_struct, mask_values, r_size,
                       weight=None, wot_i=False,
                       use_topk=False, topk_nodes=100000, topk_edges=0,
                       agg_mode="sum", prepared_masks=None):
    """GPU dense sum entry point (flashlog_kernel.py:1629-1663): c1 pruning,
    then the sum hop with c2 = topk_edges when use_topk."""
    (ori_row_ptr, ori_col_ind, ori_r_ind, order_ori,
     inv_row_ptr, inv_col_ind, inv_r_ind, order_inv,
     ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
     inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count) = csr_struct
    agg_id = 1 if agg_mode == "max" else 0
    A = _dense_topc_state(A, topk_nodes if use_topk else None)
    mask_input = prepared_masks if prepared_masks is not None else mask_values
    weight_input = None if prepared_masks is not None else weight
    return FlashLogDenseSumFunction.apply(
        A, w,
        ori_row_ptr, ori_col_ind, ori_r_ind, order_ori,
        inv_row_ptr, inv_col_ind, inv_r_ind, order_inv,
        ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
        inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
        mask_input, weight_input,
        r_size, wot_i,
        use_topk, topk_nodes, topk_edges, agg_id)


# ---------------------------------------------------------------------------
# Entry points not yet carried by this build.  Signatures follow the
# reference so callers fail with a clear message instead of a NameError.

def _not_yet(name):
    raise NotImplementedError("%s is not available in this flashlog_amd build yet" % name)


def sparse2d_filtered_ranks_cuda(idx_b, idx_e, values, targets, filter_keys, B, E, use_eql=False):
    """Filtered tie-aware ranks of each query's target over a COO [B, E] score
    matrix (flashlog_kernel.py:168-179 -> flashlog.cu:2839-2910).  Returns
    float32 ranks [B].  filter_keys (b*E + e) must be sorted ascending."""
    tensors = (idx_b, idx_e, values, targets, filter_keys)
    _require_cuda(*tensors)
    if values.dtype not in (torch.float32, torch.float64):
        raise RuntimeError("sparse2d_filtered_ranks_cuda: values must be float32 or float64")
    idx_b = idx_b.long().contiguous()
    idx_e = idx_e.long().contiguous()
    values = values.contiguous()
    targets = targets.long().contiguous()
    filter_keys = filter_keys.long().contiguous()
    B, E = int(B), int(E)
    f64 = 1 if values.dtype == torch.float64 else 0
    ranks = torch.empty(B, dtype=torch.float32, device=values.device)
    ws_bytes = _lib.lib().fl_filtered_ranks_workspace_bytes(B, f64)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=values.device)
    check(_lib.lib().fl_filtered_ranks(_stream(values), ptr(idx_b), ptr(idx_e), ptr(values), f64, ptr(targets),
                                       ptr(filter_keys), values.shape[0], filter_keys.shape[0], B, E,
                                       1 if use_eql else 0, ptr(ranks), ptr(ws), ws_bytes),
          "sparse2d_filtered_ranks_cuda")
    return ranks


def vectorized_operation_sparse3d_fixed_relation(sp_state, operators, csr_struct, r_size):
    _not_yet("vectorized_operation_sparse3d_fixed_relation")


def normalize_sparse3d(s, eps=1e-7):
    _not_yet("normalize_sparse3d")


class FlashLogDenseMaxFunction(autograd.Function):
    """GPU dense max hop (flashlog_kernel.py:992-1089): per destination the
    largest kept (a*w)*m, ties to the smaller CSR position; the backward
    routes the gradient to the winning edge only."""

    @staticmethod
    def forward(ctx, A, w, ori_row_ptr, ori_col_ind, ori_r_ind, ori_order,
                inv_row_ptr, inv_col_ind, inv_r_ind, inv_order,
                ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
                inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
                mask_values, weight, r_size, wot_i,
                use_topk, topk_nodes, topk_edges):
        _require_cuda(A, w)
        B, L, E = A.shape
        BL = B * L
        A_flat = A.reshape(BL, E).contiguous().float()
        w_flat = w.reshape(BL, -1).contiguous().float()
        prepared = _prepared_mask_pair(mask_values)
        if prepared is not None:
            ori_mask, inv_mask = prepared
        else:
            mask_f = (mask_values if mask_values.dtype == torch.bool else mask_values.float()).contiguous()
            w_tensor = weight.to(device=A.device, dtype=torch.float).squeeze(-1) if weight is not None \
                else torch.empty(0, device=A.device)
            ori_mask = _HipModule.apply_mask_cuda(mask_f, ori_order, w_tensor)
            inv_mask = _HipModule.apply_mask_cuda(mask_f, inv_order, w_tensor)
        graph = _graph_for(ori_col_ind, ori_row_group_ptr, ori_group_rel, ori_group_edge_start,
                           ori_group_edge_count, inv_col_ind, inv_row_group_ptr, inv_group_rel,
                           inv_group_edge_start, inv_group_edge_count)
        K = int(topk_edges) if (use_topk and 0 < int(topk_edges) < (1 << 60)) else 0
        out_ind, out_ori, out_inv, arg_ori, arg_inv = _dense_max_forward(
            A_flat, w_flat, graph, ori_mask, inv_mask, int(r_size), bool(wot_i), K)
        ctx.save_for_backward(A_flat, w_flat, ori_mask, inv_mask, arg_ori, arg_inv)
        ctx.graph, ctx.r_size, ctx.wot_i, ctx.shape = graph, int(r_size), bool(wot_i), (B, L, E)
        return out_ind.view(B, L, E), out_ori.view(B, L, E), out_inv.view(B, L, E)

    @staticmethod
    def backward(ctx, grad_ind, grad_ori, grad_inv):
        A_f, w_f, om, im, arg_ori, arg_inv = ctx.saved_tensors
        gA, gw = _dense_max_backward(grad_ind, grad_ori, grad_inv, arg_ori, arg_inv, A_f, w_f, ctx.graph, om, im,
                                     ctx.r_size, ctx.wot_i)
        B, L, E = ctx.shape
        return (gA.view(B, L, E), gw.view(B, L, -1)) + (None,) * 23


def dense_csr_max(A, w, csr_struct, mask_values, r_size, weight=None, wot_i=False,
                  use_topk=False, topk_nodes=100000, topk_edges=0, prepared_masks=None):
    """GPU dense max entry point (flashlog_kernel.py:1666-1688): c1 pruning,
    then the max hop with c2 = topk_edges when use_topk."""
    (ori_row_ptr, ori_col_ind, ori_r_ind, order_ori,
     inv_row_ptr, inv_col_ind, inv_r_ind, order_inv,
     ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
     inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count) = csr_struct
    A = _dense_topc_state(A, topk_nodes if use_topk else None)
    mask_input = prepared_masks if prepared_masks is not None else mask_values
    weight_input = None if prepared_masks is not None else weight
    return FlashLogDenseMaxFunction.apply(
        A, w,
        ori_row_ptr, ori_col_ind, ori_r_ind, order_ori,
        inv_row_ptr, inv_col_ind, inv_r_ind, order_inv,
        ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
        inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
        mask_input, weight_input,
        r_size, wot_i,
        use_topk, topk_nodes, topk_edges)


def vectorized_operation_sparse3d_csr_sum(sp_state, w, csr_struct, mask_values, r_size, weight=None,
                                          wot_i=False, use_topk=False, topk_edges=0, prepared_masks=None,
                                          topk_nodes=None, sampling=False):
    _not_yet("vectorized_operation_sparse3d_csr_sum")


def vectorized_operation_sparse3d_csr_sum_norm(sp_state, w, csr_struct, mask_values, r_size, weight=None,
                                               wot_i=False, use_topk=False, topk_edges=0, prepared_masks=None,
                                               eps=1e-7, topk_nodes=None, sampling=False):
    _not_yet("vectorized_operation_sparse3d_csr_sum_norm")


def sampled_sparse_propagation(state, w, csr_struct, mask_values, r_size, weight=None, wot_i=False,
                               topk_nodes=None, topk_edges=0, mode="sum"):
    _not_yet("sampled_sparse_propagation")
