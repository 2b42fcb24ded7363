"""Drop-in mirror of the reference operator API ``flashlog_kernel.flashlog_kernel``
(flashlog_kernel/flashlog_kernel.py in qikunxun/FlashLog), running on the
gfx950 HIP library ``libflashlog_hip.so`` through its C-ABI.

Every public name, positional order, default and return type follows the
reference; each definition cites the reference lines it mirrors.  The
internals are this library's: the dense hop is a destination-major pull with
a per-source frontier (no atomics on outputs, bit-identical to the
reference's CPU accumulation order).

This module has no CPU compute path.  The reference's CPU routes
(vectorized_operation_csr / FlashLogFunction, the CPU sparse classes and
their dispatch, prepare_csr_masks and _compute_active_nodes on CPU tensors)
take CPU tensors and return CPU tensors, but the arithmetic runs in this
library's GPU kernels; with no GPU visible they raise, and a missing or stale
HIP library raises.  (The reference's CPU kernels are the oracle this library
is tested against, not part of it.)
"""
import ctypes
import os
import weakref

import numpy as np
import torch
from torch import autograd

from .. import _lib
from .._lib import FlSide, FlSparseHop, check, ptr, stream_handle

_FLASHLOG_CPU_THREADS_CONFIGURED = False


# ---------------------------------------------------------------------------
# CPU thread configuration (flashlog_kernel.py:13-102: the FLASHLOG_CPU_THREADS
# and FLASHLOG_CPU_INTEROP_THREADS switches).  This module computes nothing on
# the CPU, so the setting only reaches torch's own CPU ops; the rule for
# "auto" is the reference's, so a process configures torch the same way.

def _logical_cpus():
    """CPUs this process may run on."""
    try:
        return len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        return os.cpu_count() or 1


def _machine_cores():
    """Physical cores of the machine: distinct (package, core) pairs over
    every online CPU, from the kernel's topology files (the count of
    distinct (physical id, core id) pairs the reference reads from
    /proc/cpuinfo), or None when they cannot be read."""
    root = "/sys/devices/system/cpu"
    try:
        names = [d for d in os.listdir(root) if d.startswith("cpu") and d[3:].isdigit()]
    except OSError:
        return None
    pairs = set()
    for d in names:
        topo = os.path.join(root, d, "topology")
        try:
            with open(os.path.join(topo, "physical_package_id")) as f:
                pkg = f.read().strip()
            with open(os.path.join(topo, "core_id")) as f:
                core = f.read().strip()
        except OSError:
            continue  # offline CPUs have no topology
        pairs.add((pkg, core))
    return len(pairs) or None


_PROBE = object()


def _auto_cpu_threads(logical=None, physical=_PROBE):
    """The "auto" thread count (flashlog_kernel.py:45-57): the whole usable
    count on small machines, then capped tiers chosen by the logical CPU
    count -- 24+ CPUs: the physical cores within [8, 16]; 48+: half of them
    within [12, 24]; 96+: half within [16, 32].  Without a core count the
    physical cores are taken as half the logical CPUs (8 or more) or all of
    them.  ``logical`` and ``physical`` default to this machine's (a
    physical of None stands for an unreadable core count)."""
    logical = max(1, _logical_cpus() if logical is None else logical)
    if physical is _PROBE:
        physical = _machine_cores()
    if physical is None:
        physical = max(1, logical // 2 if logical >= 8 else logical)
    usable = min(physical, logical)
    for floor_cpus, lo, hi, halve in ((96, 16, 32, True), (48, 12, 24, True), (24, 8, 16, False)):
        if logical >= floor_cpus:
            want = usable // 2 if halve else usable
            return min(hi, max(lo, want))
    return logical


def configure_flashlog_cpu_threads(force=False):
    """Apply FLASHLOG_CPU_THREADS to torch's intra-op pool, once (again with
    force=True): unset, "off", "none", "false" or "0" leave it alone; "" or
    "auto" take _auto_cpu_threads(); an integer is used as given and an
    unparsable value counts as "auto"; the count is kept within [1, CPUs
    this process may use].  FLASHLOG_CPU_INTEROP_THREADS, when set, is tried
    for the inter-op pool (at least 1; an unparsable value, or a pool that
    has already started, leaves it as is).  Returns torch's intra-op thread
    count."""
    global _FLASHLOG_CPU_THREADS_CONFIGURED
    if _FLASHLOG_CPU_THREADS_CONFIGURED and not force:
        return torch.get_num_threads()
    _FLASHLOG_CPU_THREADS_CONFIGURED = True
    raw = os.environ.get("FLASHLOG_CPU_THREADS", "off").strip().lower()
    if raw in ("off", "none", "false", "0"):
        return torch.get_num_threads()
    try:
        wanted = _auto_cpu_threads() if raw in ("", "auto") else int(raw)
    except ValueError:
        wanted = _auto_cpu_threads()
    wanted = min(max(wanted, 1), _logical_cpus())
    if wanted != torch.get_num_threads():
        torch.set_num_threads(wanted)
    interop = os.environ.get("FLASHLOG_CPU_INTEROP_THREADS")
    if interop is not None:
        try:
            pool = max(1, int(interop))
            if pool != torch.get_num_interop_threads():
                torch.set_num_interop_threads(pool)
        except (ValueError, RuntimeError):
            pass  # unparsable, or the inter-op pool is already running
    return torch.get_num_threads()


def _require_cuda(*tensors):
    for t in tensors:
        if torch.is_tensor(t) and not t.is_cuda:
            raise RuntimeError("flashlog_amd runs on the GPU only; got a CPU tensor")


def _work_device():
    """The GPU that computes for CPU inputs (the reference's CPU routes run
    this library's kernels there; inputs go over, results come back)."""
    if not torch.cuda.is_available():
        raise RuntimeError("flashlog_amd computes on a ROCm GPU; none is visible for these CPU tensors")
    return torch.device("cuda", torch.cuda.current_device())


# Device copies of CPU graph arrays (CSR tuples are built once per graph and
# passed on every call): kept while the CPU tensor lives unmodified.
_RESIDENT = {}


def _resident(t, dev):
    if not torch.is_tensor(t) or t.device == dev:
        return t
    key = (id(t), t._version, str(dev))
    hit = _RESIDENT.get(key)
    if hit is not None and hit[0]() is t:
        return hit[1]
    for k in [k for k, v in _RESIDENT.items() if v[0]() is None]:
        del _RESIDENT[k]
    copy = t.to(dev)
    _RESIDENT[key] = (weakref.ref(t), copy)
    return copy


def _stream(t):
    return stream_handle(t.device)


# ---------------------------------------------------------------------------
# Graph preparation

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
        # first position of every row (and the end), by binary search in the sorted rows
        row_ptr = torch.searchsorted(sorted_rows.to("cpu", torch.int64),
                                     torch.arange(num_nodes + 1, dtype=torch.int64), out_int32=True)
    group_ptr = torch.searchsorted(starts, row_ptr, out_int32=True)
    return group_ptr, relations, starts, counts


def _gpu_csr_sides(row, col, rel, nodes, sides=((0, 1), (1, 0))):
    """CSR sides built on the GPU: for each (s, t) in ``sides`` the side whose
    sources are (row, col)[s] and targets (row, col)[t], as (row_ptr, columns,
    edge_rel, order, group_ptr, group_rel, group_start, group_count)."""
    if not (row.dim() == col.dim() == rel.dim() == 1) or not (row.numel() == col.numel() == rel.numel()):
        raise ValueError("CSR requires equal 1D arrays and int32-sized graph")
    dev = row.device
    row, col, rel = (x.to(torch.int64).contiguous() for x in (row, col, rel))
    ends = (row, col)
    m = row.numel()
    lib = _lib.lib()
    ws_bytes = lib.fl_csr_build_side_gpu_bytes(m, nodes)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    st = _stream(row)
    info = torch.empty(2, dtype=torch.int64, device=dev)
    out = []
    for s, t in sides:
        row_ptr = torch.empty(nodes + 1, dtype=torch.int32, device=dev)
        cols = torch.empty(m, dtype=torch.int32, device=dev)
        erel = torch.empty(m, dtype=torch.int16, device=dev)
        order = torch.empty(m, dtype=torch.int32, device=dev)
        gptr = torch.empty(nodes + 1, dtype=torch.int32, device=dev)
        grel = torch.empty(max(m, 1), dtype=torch.int16, device=dev)
        gstart = torch.empty(max(m, 1), dtype=torch.int32, device=dev)
        gcount = torch.empty(max(m, 1), dtype=torch.int32, device=dev)
        check(lib.fl_csr_build_side_gpu(st, m, nodes, ptr(ends[s]), ptr(ends[t]), ptr(rel), ptr(row_ptr), ptr(cols),
                                        ptr(erel), ptr(order), ptr(gptr), ptr(grel), ptr(gstart), ptr(gcount),
                                        ptr(info), ptr(ws), ws_bytes), "csr_build_side_gpu")
        g, err = info.tolist()
        if err:
            raise ValueError("CSR entity or relation ID outside supported range")
        out.append((row_ptr, cols, erel, order, gptr, grel[:g].clone(), gstart[:g].clone(), gcount[:g].clone()))
    return out


def _build_csr_structure_gpu(row, col, rel, nodes):
    ori, inv = _gpu_csr_sides(row, col, rel, nodes)
    return (*ori[:4], *inv[:4], *ori[4:], *inv[4:])


def build_csr_structure(row_indices, col_indices, r_indices, num_nodes):
    """The reference's 16-tuple (flashlog_kernel.py:678-697; csr.cpp:12-69):
    (ori_row_ptr, ori_col_ind, ori_r_ind, order_ori, inv_..., ori_row_group_ptr,
    ori_group_rel, ori_group_edge_start, ori_group_edge_count, inv_...).
    Inputs on a GPU are built there (fl_csr_build_side_gpu, one radix sort
    per side); CPU inputs by the library's host builder.  Both give the
    reference's arrays bit for bit, on the input's device."""
    device = row_indices.device
    if device.type == "cuda":
        return _build_csr_structure_gpu(row_indices, col_indices, r_indices, int(num_nodes))
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


class _HostMaskOrder(autograd.Function):
    """mask[order] * sigmoid(weight[order]) for CPU inputs, computed by the
    GPU kernel and returned on the CPU.  As the reference's CPU expression
    (flashlog_kernel.py:250-254, torch ops) it is differentiable in the edge
    weight: d/dweight[order[i]] = g[i] * mask * s * (1 - s), one position
    per edge and side (order is a permutation), so the scatter has no
    collisions."""

    @staticmethod
    def forward(ctx, mask_f, order, weight):
        dev = _work_device()
        m, o = mask_f.to(dev), _resident(order, dev).to(torch.int32).contiguous()
        wt = weight.detach().to(device=dev, dtype=torch.float).squeeze(-1).contiguous() if weight is not None \
            else torch.empty(0, device=dev)
        out = _HipModule.apply_mask_cuda(m, o, wt)
        ctx.keep = (m, o, wt, weight is not None)
        ctx.weight_meta = (weight.shape, weight.dtype) if weight is not None else None
        return out.to(mask_f.device)

    @staticmethod
    def backward(ctx, grad):
        m, o, wt, has_w = ctx.keep
        if not has_w or not ctx.needs_input_grad[2]:
            return None, None, None
        pos = o.long()
        s = torch.sigmoid(wt[pos])
        g = grad.to(m.device).float() * m[pos].float() * s * (1.0 - s)
        gw = torch.zeros(wt.numel(), dtype=torch.float32, device=m.device).index_put_((pos,), g)
        shape, dtype = ctx.weight_meta
        return None, None, gw.view(shape).to(device=grad.device, dtype=dtype)


def _apply_mask_order(mask_values, order, weight=None):
    mask_f = (mask_values if mask_values.dtype == torch.bool else mask_values.float()).contiguous().view(-1)
    if not mask_f.is_cuda:
        return _HostMaskOrder.apply(mask_f, order, weight)
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
    (flashlog_kernel.py:617-623), on the input's device.  The reference
    takes the nonzeros of A.sum(1); the two differ only where a (b, e)'s
    channel values cancel to exactly 0, which no propagation state (sums of
    nonnegative products) produces."""
    dev = A.device if A.is_cuda else _work_device()
    flat = A.detach().reshape(-1, A.shape[-1]).to(dev).contiguous().float()
    return _HipModule.compute_active_nodes_cuda(flat).to(A.device)


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
    if not A.is_cuda:  # the CPU route: selected on the GPU, returned to the CPU (differentiably)
        return _DenseTopC.apply(A.to(_work_device()), int(topk_nodes)).to(A.device)
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
        return _dense_sum_forward(A, w, graph, ori_mask.float().contiguous(), inv_mask.float().contiguous(),
                                  int(r_size), bool(wot_i), _edge_budget(use_topk, topk_edges))

    @staticmethod
    def flashlog_forward_max_cuda(A, w, active_nodes,
                                  ori_row_ptr, ori_col_ind, ori_r_ind, ori_mask,
                                  inv_row_ptr, inv_col_ind, inv_r_ind, inv_mask,
                                  ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
                                  inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
                                  r_size, wot_i, use_topk, topk_edges):
        """flashlog.cu:997-1072: (out_ind, out_ori, out_inv, ori_arg, inv_arg),
        the args int64 winning CSR positions (-1 where nothing arrives)."""
        graph = _graph_for(ori_col_ind, ori_row_group_ptr, ori_group_rel, ori_group_edge_start,
                           ori_group_edge_count, inv_col_ind, inv_row_group_ptr, inv_group_rel,
                           inv_group_edge_start, inv_group_edge_count)
        return _dense_max_forward(A.float(), w.float(), graph, ori_mask.float().contiguous(),
                                  inv_mask.float().contiguous(), int(r_size), bool(wot_i),
                                  _edge_budget(use_topk, topk_edges))

    @staticmethod
    def flashlog_backward_cuda(grad_ind, grad_ori, grad_inv, out_ori, out_inv, A, w, active_nodes,
                               ori_row_ptr, ori_col_ind, ori_r_ind, ori_mask,
                               inv_row_ptr, inv_col_ind, inv_r_ind, inv_mask,
                               ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
                               inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
                               r_size, wot_i, use_topk, topk_edges, agg_mode):
        """flashlog.cu:1077-1185 (agg_mode 0): (grad_A [BL, E], grad_w [BL, n]).
        out_ori / out_inv served the reference's legacy max tolerance only."""
        if int(agg_mode) != 0:
            raise NotImplementedError("agg_mode=max on the sum entry point: use flashlog_backward_max_cuda")
        graph = _graph_for(ori_col_ind, ori_row_group_ptr, ori_group_rel, ori_group_edge_start,
                           ori_group_edge_count, inv_col_ind, inv_row_group_ptr, inv_group_rel,
                           inv_group_edge_start, inv_group_edge_count)
        return _dense_sum_backward(grad_ind, grad_ori, grad_inv, A.contiguous().float(), w.contiguous().float(),
                                   graph, ori_mask.float().contiguous(), inv_mask.float().contiguous(), int(r_size),
                                   bool(wot_i), _edge_budget(use_topk, topk_edges))

    @staticmethod
    def flashlog_backward_max_cuda(grad_ind, grad_ori, grad_inv, ori_arg, inv_arg, A, w, active_nodes,
                                   ori_row_ptr, ori_col_ind, ori_r_ind, ori_mask,
                                   inv_row_ptr, inv_col_ind, inv_r_ind, inv_mask,
                                   ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
                                   inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
                                   r_size, wot_i, use_topk, topk_edges):
        """flashlog.cu:1187-1255: the gradient reaches only each destination's
        winning position."""
        graph = _graph_for(ori_col_ind, ori_row_group_ptr, ori_group_rel, ori_group_edge_start,
                           ori_group_edge_count, inv_col_ind, inv_row_group_ptr, inv_group_rel,
                           inv_group_edge_start, inv_group_edge_count)
        return _dense_max_backward(grad_ind, grad_ori, grad_inv, ori_arg.long().contiguous(),
                                   inv_arg.long().contiguous(), A.contiguous().float(), w.contiguous().float(), graph,
                                   ori_mask.float().contiguous(), inv_mask.float().contiguous(), int(r_size),
                                   bool(wot_i), _edge_budget(use_topk, topk_edges))

    @staticmethod
    def flashlog_forward_cpu(A, w, active_nodes,
                             ori_col_ind, ori_mask,
                             ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
                             inv_col_ind, inv_mask,
                             inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
                             r_size, wot_i, topk_edges):
        """flashlog.cpp:284-337 for CPU tensors [BL, E]: computed by the GPU
        kernels (the same order and bits), returned on the CPU."""
        dev = _work_device()
        BL, E = A.shape
        graph = _graph_for(*(_resident(t, dev) for t in (
            ori_col_ind, ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
            inv_col_ind, inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count)))
        K = int(topk_edges) if 0 < int(topk_edges) < (1 << 60) else 0
        outs = _dense_sum_forward(A.to(dev).contiguous().float(), w.to(dev).contiguous().float(), graph,
                                  ori_mask.to(dev).float().contiguous(), inv_mask.to(dev).float().contiguous(),
                                  int(r_size), bool(wot_i), K)
        return tuple(o.to(A.device) for o in outs)

    @staticmethod
    def flashlog_backward_cpu(grad_ind, grad_ori, grad_inv, A, w, active_nodes,
                              ori_col_ind, ori_mask,
                              ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
                              inv_col_ind, inv_mask,
                              inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
                              r_size, wot_i, topk_edges):
        """flashlog.cpp:339-393 for CPU tensors: (grad_A, grad_w) on the CPU,
        grad_A bit-equal to the CPU path's, grad_w its terms in a fixed
        association."""
        dev = _work_device()
        graph = _graph_for(*(_resident(t, dev) for t in (
            ori_col_ind, ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
            inv_col_ind, inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count)))
        K = int(topk_edges) if 0 < int(topk_edges) < (1 << 60) else 0
        grads = [g.to(dev) if g is not None else None for g in (grad_ind, grad_ori, grad_inv)]
        gA, gw = _dense_sum_backward(*grads, A.to(dev).contiguous().float(), w.to(dev).contiguous().float(), graph,
                                     ori_mask.to(dev).float().contiguous(), inv_mask.to(dev).float().contiguous(),
                                     int(r_size), bool(wot_i), K)
        return gA.to(A.device), gw.to(A.device)

    @staticmethod
    def sparse3d_normalize_forward_cuda(sp_batch, sp_level, values, B, L, eps):
        """flashlog.cu:2593-2649: (out_values, denom [B, L], row_start [B*L],
        row_end [B*L]) of a state sorted by row."""
        out, denom, row_ptr = _normalize_forward(sp_batch, sp_level, values, int(B), int(L), float(eps))
        R = int(B) * int(L)
        return out.to(values.dtype), denom.view(int(B), int(L)), row_ptr[:R].clone(), row_ptr[1:R + 1].clone()

    @staticmethod
    def sparse3d_normalize_backward_cuda(grad_out_values, values, denom, row_start, row_end, eps):
        """flashlog.cu:2651-2691.  Rows are [row_start, row_end) of a state
        sorted by row; an empty row may hold any equal pair (the reference
        marks it (0, 0)): the row pointer is rebuilt from the nonempty rows."""
        _require_cuda(grad_out_values, values, denom, row_start, row_end)
        nnz = values.numel()
        starts = row_start.long()
        nonempty = row_end.long() > starts
        nxt = torch.where(nonempty, starts, torch.full_like(starts, nnz))
        nxt = torch.flip(torch.cummin(torch.flip(nxt, (0,)), 0).values, (0,))
        row_ptr = torch.cat([nxt, nxt.new_full((1,), nnz)]).contiguous()
        return _normalize_backward(row_ptr, grad_out_values, values.contiguous().float(),
                                   denom.contiguous().view(-1).float(), float(eps)).to(values.dtype)

    @staticmethod
    def flashlog_forward_sparse3d_fixed_relation_cuda(sp_batch, sp_level, sp_entity, sp_value, operators,
                                                      ori_col_ind, ori_row_group_ptr, ori_group_rel,
                                                      ori_group_edge_start, ori_group_edge_count,
                                                      inv_col_ind, inv_row_group_ptr, inv_group_rel,
                                                      inv_group_edge_start, inv_group_edge_count,
                                                      B, L, E, r_size):
        """flashlog.cu:1677-1741: the (b, l, e, v) of one fixed-relation step,
        here already coalesced (path counts are exact integers, so the
        caller's coalesce of them gives the same state)."""
        csr = [None] * 16
        for slot, t in zip((1, 8, 9, 10, 11, 5, 12, 13, 14, 15),
                           (ori_col_ind, ori_row_group_ptr, ori_group_rel, ori_group_edge_start,
                            ori_group_edge_count, inv_col_ind, inv_row_group_ptr, inv_group_rel,
                            inv_group_edge_start, inv_group_edge_count)):
            csr[slot] = t
        st = torch.sparse_coo_tensor(torch.stack([sp_batch.long(), sp_level.long(), sp_entity.long()]),
                                     sp_value.float(), (int(B), int(L), int(E)))
        out = vectorized_operation_sparse3d_fixed_relation(st, operators, tuple(csr), int(r_size))
        b, l, e = out.indices()
        return b, l, e, out.values()

    @staticmethod
    def sparse2d_filtered_ranks_cuda(idx_b, idx_e, values, targets, filter_keys, B, E, use_eql):
        """flashlog.cu:2839-2910."""
        return sparse2d_filtered_ranks_cuda(idx_b, idx_e, values, targets, filter_keys, B, E, use_eql)


def _edge_budget(use_topk, topk_edges):
    """The c2 budget the dense kernels take (0: none), as the reference's host
    wrappers decide it (flashlog.cu:958,1142: use_topk and 0 < K < 2^60)."""
    K = int(topk_edges)
    return K if use_topk and 0 < K < (1 << 60) else 0


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


def _dense_max_backward(grad_ind, grad_ori, grad_inv, arg_ori, arg_inv, A_f, w_f, graph, om, im, r_size, wot_i,
                        K):
    """flashlog_backward_max_cuda (flashlog.cu:1187-1255) as fixed-order
    walks of the kept positions of every (source, row): only the winning
    position of a destination passes its gradient on."""
    return _dense_backward(grad_ind, grad_ori, grad_inv, A_f, w_f, graph, om, im, r_size, wot_i, K,
                           arg_ori, arg_inv)


def _dense_backward(grad_ind, grad_ori, grad_inv, A_f, w_f, graph, om, im, r_size, wot_i, K,
                    arg_ori=None, arg_inv=None):
    """Both dense backwards: the sum's (arg_ori None) and the max's."""
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
    common = (ctypes.byref(so), ctypes.byref(si), ptr(A_f), ptr(w_f), ptr(gi), ptr(go), ptr(gv))
    tail = (BL, E, n, r_size, 1 if wot_i else 0, int(K), ptr(gA), ptr(gw), ptr(pg), pairs, ptr(ws), ws_bytes)
    if arg_ori is None:
        check(_lib.lib().fl_dense_sum_backward(_stream(A_f), *common, *tail), "dense_sum_backward")
    else:
        check(_lib.lib().fl_dense_max_backward(_stream(A_f), *common, ptr(arg_ori), ptr(arg_inv), *tail),
              "dense_max_backward")
    return gA, gw


# ---------------------------------------------------------------------------
# Dense autograd functions

class FlashLogFunction(autograd.Function):
    """Dense propagation with precomputed active nodes and CSR-ordered masks
    (flashlog_kernel.py:700-811).  GPU tensors run in place; CPU tensors (the
    reference's flashlog_forward_cpu / flashlog_backward_cpu route) run the
    same kernels on the GPU, with the graph arrays' device copies kept per
    CSR tensor, and get CPU outputs and gradients back.  ``active_nodes`` is
    accepted for the signature: the kernels derive the frontier from A."""

    @staticmethod
    def forward(ctx, A, w, active_nodes,
                ori_col_ind, ori_mask,
                ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
                inv_col_ind, inv_mask,
                inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
                r_size, wot_i, topk_edges):
        home = A.device
        dev = home if A.is_cuda else _work_device()
        B, L, E = A.shape
        graph = _graph_for(*(_resident(t, dev) for t in (
            ori_col_ind, ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
            inv_col_ind, inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count)))
        A_f = A.reshape(B * L, E).to(dev).contiguous().float()
        w_f = w.reshape(B * L, -1).to(dev).contiguous().float()
        om, im = (m.to(dev).float().contiguous() for m in (ori_mask, inv_mask))
        K = int(topk_edges) if 0 < int(topk_edges) < (1 << 60) else 0
        outs = _dense_sum_forward(A_f, w_f, graph, om, im, int(r_size), bool(wot_i), K)
        ctx.save_for_backward(A_f, w_f, om, im)
        ctx.graph, ctx.r_size, ctx.wot_i, ctx.K, ctx.shape = graph, int(r_size), bool(wot_i), K, (B, L, E)
        ctx.home = home
        return tuple(o.view(B, L, E).to(home) for o in outs)

    @staticmethod
    def backward(ctx, grad_ind, grad_ori, grad_inv):
        A_f, w_f, om, im = ctx.saved_tensors
        dev = A_f.device
        grads = [g.to(dev) if g is not None else None for g in (grad_ind, grad_ori, grad_inv)]
        gA, gw = _dense_sum_backward(*grads, A_f, w_f, ctx.graph, om, im, ctx.r_size, ctx.wot_i, ctx.K)
        B, L, E = ctx.shape
        return (gA.view(B, L, E).to(ctx.home), gw.view(B, L, -1).to(ctx.home)) + (None,) * 16


def _dense_sum_backward(grad_ind, grad_ori, grad_inv, A_f, w_f, graph, om, im, r_size, wot_i, K):
    """flashlog_backward_cuda (flashlog.cu:1077-1185) with the CPU path's
    order (flashlog.cpp:216-278): grad_A bit-identical, grad_w from
    per-(source, row) partials added in ascending source order (within
    float rounding of the CPU's single sequential sum)."""
    return _dense_backward(grad_ind, grad_ori, grad_inv, A_f, w_f, graph, om, im, r_size, wot_i, K)


def vectorized_operation_csr(A, w, csr_struct, mask_values, r_size,
                             weight=None, wot_i=False,
                             use_topk=False, topk_nodes=100000, topk_edges=0,
                             prepared_masks=None):
    """Dense entry point of the reference's CPU route (flashlog_kernel.py:
    845-882), used by the dense models when CUDA is off
    (src/model_DRUM_kernel.py:133-140, src/model_NeuralLP_kernel.py:127-132):
    masks, c1, then FlashLogFunction with topk_edges or, without a budget,
    1 << 60.  CPU tensors in, CPU tensors out; the arithmetic runs on the GPU
    in the CPU path's order (bit-equal to flashlog.cpp:151-278)."""
    masks = _prepared_mask_pair(mask_values if prepared_masks is None else prepared_masks)
    if masks is None:
        masks = prepare_csr_masks(csr_struct, mask_values, weight)
    # FlashLogFunction takes per side: columns, mask, then the 4 group arrays
    sides = [(csr_struct[col], m, *csr_struct[g0:g0 + 4]) for col, m, g0 in ((1, masks[0], 8), (5, masks[1], 12))]
    budget = topk_edges if use_topk and topk_edges > 0 else 1 << 60
    return FlashLogFunction.apply(_dense_topc_state(A, topk_nodes if use_topk else None), w, None,
                                  *sides[0], *sides[1], r_size, wot_i, budget)


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


def _dense_gpu_args(A, w, csr_struct, mask_values, weight, use_topk, topk_nodes, prepared_masks):
    """Leading positional arguments of the dense GPU autograd functions: the
    c1-pruned state, w, the 16 CSR arrays in tuple order (the order of their
    parameters), then the masks and edge weights (prepared masks, when
    given, replace both)."""
    pruned = _dense_topc_state(A, topk_nodes if use_topk else None)
    if prepared_masks is not None:
        mask_values, weight = prepared_masks, None
    return (pruned, w, *csr_struct, mask_values, weight)


def dense_csr_sum_cuda(A, w, csr_struct, mask_values, r_size,
                       weight=None, wot_i=False,
                       use_topk=False, topk_nodes=100000, topk_edges=0,
                       agg_mode="sum", prepared_masks=None):
    """GPU dense sum entry point (flashlog_kernel.py:1629-1663): c1 pruning,
    then the sum hop with c2 = topk_edges when use_topk."""
    lead = _dense_gpu_args(A, w, csr_struct, mask_values, weight, use_topk, topk_nodes, prepared_masks)
    return FlashLogDenseSumFunction.apply(*lead, r_size, wot_i, use_topk, topk_nodes, topk_edges,
                                          int(agg_mode == "max"))


# ---------------------------------------------------------------------------
# Filtered ranks of the evaluation (flashlog_kernel.py:168-179, src/main.py:468-512).

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


def dense_filtered_ranks_cuda(state, targets, filter_indices=None, use_eql=False):
    """Filtered tie-aware ranks of each query's target over a dense [B, E]
    score matrix: the rank computation of the evaluation driver's
    calculate_hits_full_with_filter_indices (src/main.py:468-512), where it
    is a chain of torch ops.  filter_indices: (batch, entity) index tensors
    of the known answers, or None for no filtering; as in the reference, the
    targets join the filter and duplicate keys count once.  Returns float32
    ranks [B] (greater + 1, or greater + (equal + 1) / 2 with use_eql,
    equal already counting the target once)."""
    _require_cuda(state, targets)
    if state.dim() != 2:
        raise ValueError("dense_filtered_ranks_cuda: state must be [B, E]")
    B, E = state.shape
    state = state.float().contiguous()
    targets = targets.long().contiguous()
    if targets.numel() != B:
        raise ValueError("dense_filtered_ranks_cuda: one target per query")
    if B and (int(targets.min()) < 0 or int(targets.max()) >= E):
        raise ValueError("dense_filtered_ranks_cuda: target out of range")
    keys = None
    if filter_indices is not None:
        fb, fe = filter_indices
        batch_idx = torch.arange(B, device=state.device, dtype=torch.long)
        fb = torch.cat([fb.to(state.device).long(), batch_idx])
        fe = torch.cat([fe.to(state.device).long(), targets])
        if fb.numel() and (int(fb.min()) < 0 or int(fb.max()) >= B or int(fe.min()) < 0 or int(fe.max()) >= E):
            raise ValueError("dense_filtered_ranks_cuda: filter index out of range")
        keys = torch.unique(fb * E + fe)
    ranks = torch.empty(B, dtype=torch.float32, device=state.device)
    check(_lib.lib().fl_dense_filtered_ranks(_stream(state), ptr(state), ptr(targets),
                                             ptr(keys) if keys is not None else None,
                                             keys.numel() if keys is not None else 0, B, E,
                                             1 if use_eql else 0, ptr(ranks)), "dense_filtered_ranks_cuda")
    return ranks


def vectorized_operation_sparse3d_fixed_relation(sp_state, operators, csr_struct, r_size):
    """Advance sparse rule levels through one fixed relation per level
    (flashlog_kernel.py:182-210).  ``operators`` is shaped ``[B, L]`` with the
    FlashLog operator ids: forward relations, inverse relations offset by
    ``r_size`` and the identity at ``2 * r_size``.  Values are carried
    unchanged and summed per endpoint (path counts)."""
    if not sp_state.is_cuda:
        raise ValueError("fixed-relation rule inference currently requires CUDA")
    sp_state = sp_state.coalesce()
    indices = sp_state.indices()
    values = sp_state.values()
    B, L, E = sp_state.shape
    if tuple(operators.shape) != (B, L):
        raise ValueError("operators must have shape [{}, {}], got {}".format(B, L, tuple(operators.shape)))
    sides = _fixed_sides(csr_struct)
    idx, vals, _ = _sparse_forward(indices[0], indices[1], indices[2], values.float(), None, sides, B, L, E,
                                   int(r_size), False, _SPARSE_FIXED, 0, False,
                                   operators=operators.to(device=values.device, dtype=torch.int64).contiguous())
    return _coo(idx, vals.to(values.dtype), int(B), int(L), int(E))


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
        ctx.graph, ctx.r_size, ctx.wot_i, ctx.K, ctx.shape = graph, int(r_size), bool(wot_i), K, (B, L, E)
        return out_ind.view(B, L, E), out_ori.view(B, L, E), out_inv.view(B, L, E)

    @staticmethod
    def backward(ctx, grad_ind, grad_ori, grad_inv):
        A_f, w_f, om, im, arg_ori, arg_inv = ctx.saved_tensors
        gA, gw = _dense_max_backward(grad_ind, grad_ori, grad_inv, arg_ori, arg_inv, A_f, w_f, ctx.graph, om, im,
                                     ctx.r_size, ctx.wot_i, ctx.K)
        B, L, E = ctx.shape
        return (gA.view(B, L, E), gw.view(B, L, -1)) + (None,) * 23


def dense_csr_max(A, w, csr_struct, mask_values, r_size, weight=None, wot_i=False,
                  use_topk=False, topk_nodes=100000, topk_edges=0, prepared_masks=None):
    """GPU dense max entry point (flashlog_kernel.py:1666-1688): c1 pruning,
    then the max hop with c2 = topk_edges when use_topk."""
    lead = _dense_gpu_args(A, w, csr_struct, mask_values, weight, use_topk, topk_nodes, prepared_masks)
    return FlashLogDenseMaxFunction.apply(*lead, r_size, wot_i, use_topk, topk_nodes, topk_edges)


def sampled_sparse_propagation(state, w, csr_struct, mask_values, r_size, weight=None, wot_i=False,
                               topk_nodes=None, topk_edges=0, mode="sum"):
    """Training-time hop (flashlog_kernel.py:1955-1969): the top-k sum or max
    hop with sampling=True (exponential-race c1, quota c2), topk_edges <= 0
    meaning no edge budget.  A CPU state runs the same GPU hop (inputs moved
    to the GPU, output moved back), so its random selections follow the GPU
    path's draws."""
    state = state.coalesce()
    on_cpu = not state.is_cuda
    if on_cpu:
        dev = torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() else None
        if dev is None:
            raise RuntimeError("flashlog_amd needs a ROCm GPU: sampled_sparse_propagation has no CPU path")
        state = state.to(dev)
        w = w.to(dev)
        csr_struct = tuple(t.to(dev) for t in csr_struct)
        mask_values = mask_values.to(dev)
        weight = weight.to(dev) if weight is not None else None
    idx, val = state.indices(), state.values()
    B, L, E = state.shape
    function = FlashLogFunctionSparse3DTopKMax if mode == "max" else FlashLogFunctionSparse3DTopKSum
    out = function.apply(idx[0], idx[1], idx[2], val, w, *csr_struct,
                         mask_values, weight, B, L, E, r_size, wot_i,
                         topk_edges if topk_edges > 0 else (1 << 60),
                         False, topk_nodes, torch.is_grad_enabled(), True)
    return out.cpu() if on_cpu else out


# ---------------------------------------------------------------------------
# Sparse (COO) propagation (flashlog_kernel.py:1092-1954): one hop expands
# every entry of the state through its kept edges and coalesces per
# (b, l, entity) in the CPU path's addition order (fl_sparse_* in
# libflashlog_hip.so).

_SPARSE_TOPK, _SPARSE_ALL, _SPARSE_FIXED = 0, 1, 2
_SPARSE_SUM, _SPARSE_MAX = 0, 1


class _SparseSides:
    """FlSide views of the CSR arrays the sparse kernels read (no pull index)."""

    def __init__(self, ori_col, ori_mask, ori_gptr, ori_grel, ori_gstart, ori_gcount,
                 inv_col, inv_mask, inv_gptr, inv_grel, inv_gstart, inv_gcount, ori_order=None, inv_order=None,
                 ori_dscore=None, inv_dscore=None, ori_bits=None, inv_bits=None):
        self.keep = []
        self.ori = self._side(ori_col, ori_mask, ori_gptr, ori_grel, ori_gstart, ori_gcount, ori_order, ori_dscore,
                              ori_bits)
        self.inv = self._side(inv_col, inv_mask, inv_gptr, inv_grel, inv_gstart, inv_gcount, inv_order, inv_dscore,
                              inv_bits)

    def set_grad_edge(self, grad_edge):
        """Points both sides' edge-weight gradient at grad_edge (or None)."""
        p = ptr(grad_edge).value if grad_edge is not None else None
        self.ori.grad_edge = p
        self.inv.grad_edge = p

    def positions_optional(self, mode, aggregate, buckets):
        """True when the backward reads no item's CSR position: the top-k
        sum over several destination buckets (masked items are dropped and
        carry no output index), every mask a bitmap (kept items have mask 1)
        and no edge-weight factors."""
        def ok(s):
            return (not s.mask or s.mask_bits) and not s.dscore
        return mode == _SPARSE_TOPK and aggregate == _SPARSE_SUM and buckets > 1 and ok(self.ori) and ok(self.inv)

    def _side(self, col, mask, gptr, grel, gstart, gcount, order=None, dscore=None, bits=None):
        _require_cuda(col, gptr, grel, gstart, gcount)
        col = col.int().contiguous()
        gptr = gptr.int().contiguous()
        grel = grel.short().contiguous()
        gstart = gstart.int().contiguous()
        gcount = gcount.int().contiguous()
        if mask is not None:
            _require_cuda(mask)
            mask = mask.float().contiguous()
            if mask.numel() != col.numel():
                raise ValueError("mask length must equal the number of CSR positions")
        if order is not None:
            _require_cuda(order)
            order = order.int().contiguous()
            if order.numel() != col.numel():
                raise ValueError("order length must equal the number of CSR positions")
        if bits is not None and bits.numel() < (col.numel() + 31) // 32:
            raise ValueError("mask bits must cover every CSR position of a masked side")
        self.keep += [col, mask, gptr, grel, gstart, gcount, order, dscore, bits]
        side = FlSide()
        side.mask_bits = ptr(bits).value if bits is not None else None
        side.edges, side.groups = col.numel(), grel.numel()
        side.order = ptr(order).value if order is not None else None
        side.dscore = ptr(dscore).value if dscore is not None else None
        side.col_ind, side.mask = ptr(col).value, (ptr(mask).value if mask is not None else None)
        side.row_group_ptr, side.group_rel = ptr(gptr).value, ptr(grel).value
        side.group_start, side.group_count = ptr(gstart).value, ptr(gcount).value
        side.min_rel, side.max_rel = _relation_range(grel)
        return side


# Smallest and largest relation id of a group-relation array, kept per
# tensor object and version (the CSR arrays of a graph serve every hop; a
# read of the range costs reductions and a device synchronization).
_REL_RANGE = {}


def _relation_range(grel):
    if grel.numel() == 0:
        return 0, -1
    hit = _REL_RANGE.get(id(grel))
    if hit is not None and hit[0]() is grel and hit[1] == grel._version:
        return hit[2]
    for k in [k for k, v in _REL_RANGE.items() if v[0]() is None]:
        del _REL_RANGE[k]
    lo, hi = (int(x) for x in torch.stack([grel.min(), grel.max()]).tolist())
    _REL_RANGE[id(grel)] = (weakref.ref(grel), grel._version, (lo, hi))
    return lo, hi


# Hops with at least this many entries visit them by source entity.
_ENTRY_ORDER_MIN = 4096

def _entry_order(sp_e, E):
    """Entries by source entity: a source's rows then share cached group
    records in the plan and the run writer (fl_sparse_entry_order's counting
    sort over blocks of 64 entity ids; any order within a block)."""
    nnz = sp_e.numel()
    lib = _lib.lib()
    ws = torch.empty(max(int(lib.fl_sparse_entry_order_bytes(nnz, int(E))), 1), dtype=torch.uint8,
                     device=sp_e.device)
    order = torch.empty(max(nnz, 1), dtype=torch.int32, device=sp_e.device)
    check(lib.fl_sparse_entry_order(_stream(sp_e), ptr(sp_e), nnz, int(E), ptr(ws), ws.numel(), ptr(order)),
          "sparse_entry_order")
    return order[:nnz]


# When a list, every sparse hop appends its sizes to it as {"nnz" (entries
# after c1), "items" (raw items), "chunks", "backward", "nout" (output
# entries), "groups" (the entries' sources' groups over both sides), "rows"
# (B*L), "n" (attention width), "wot_i"} (for byte counts in measurements).
plan_log = None


class _SparseState:
    """A forward hop's saved pieces for the backward."""


def _sparse_forward(sp_b, sp_l, sp_e, sp_v, w, sides, B, L, E, r_size, wot_i, mode, topk_edges,
                    need_backward, operators=None, aggregate=_SPARSE_SUM, seed=-1, check_finite=False):
    """Runs plan -> expand -> emit.  Returns (indices [3, nout], values, state).
    aggregate: sum or max; seed >= 0: training quotas instead of the c2
    threshold."""
    _require_cuda(sp_b, sp_l, sp_e, sp_v)
    dev = sp_v.device
    B, L, E, r_size = int(B), int(L), int(E), int(r_size)
    R = B * L
    sp_b = sp_b.long().contiguous()
    sp_l = sp_l.long().contiguous()
    sp_e = sp_e.long().contiguous()
    sp_v = sp_v.contiguous()
    if sp_v.dtype != torch.float32:
        raise TypeError("flashlog_amd sparse propagation computes in float32")
    if mode == _SPARSE_FIXED:
        w_flat = torch.zeros(1, dtype=torch.float32, device=dev)
        n = 1
    else:
        _require_cuda(w)
        w_flat = w.reshape(R, -1).contiguous().float()
        n = w_flat.shape[1]
        if (max(sides.ori.max_rel, sides.inv.max_rel) >= r_size or min(sides.ori.min_rel, sides.inv.min_rel) < 0
                or 2 * r_size > n):
            raise ValueError("relation ids must be in [0, r_size) and w must hold 2*r_size (+1) columns")
    nnz = sp_v.numel()
    lib = _lib.lib()
    st = _stream(sp_v)
    perm = None
    order = None
    for attempt in range(2):
        if mode != _SPARSE_FIXED and nnz >= _ENTRY_ORDER_MIN:
            order = _entry_order(sp_e, E)
        h = FlSparseHop()
        h.entry_order = ptr(order).value if order is not None else None
        h.sp_b, h.sp_l, h.sp_e, h.sp_v = (ptr(t).value for t in (sp_b, sp_l, sp_e, sp_v))
        h.nnz, h.w = nnz, ptr(w_flat).value
        h.B, h.L, h.E, h.n, h.r_size = B, L, E, n, r_size
        h.wot_i, h.mode, h.topk_edges = 1 if wot_i else 0, int(mode), int(topk_edges)
        h.operators = ptr(operators).value if operators is not None else None
        h.aggregate, h.sampling_seed = int(aggregate), int(seed)
        ws1 = torch.empty(max(lib.fl_sparse_plan_bytes(nnz, R, 0 if mode == _SPARSE_FIXED else r_size), 1),
                          dtype=torch.uint8, device=dev)
        h.ws1, h.ws1_bytes = ptr(ws1).value, ws1.numel()
        plan = torch.empty(6, dtype=torch.int64, device=dev)
        check(lib.fl_sparse_plan(st, ctypes.byref(sides.ori), ctypes.byref(sides.inv), ctypes.byref(h), ptr(plan)),
              "sparse_plan")
        items, tiles, err, nb, chunks, nonfinite = plan.tolist()
        if check_finite and nonfinite:
            # flashlog.cu:2019-2021, checked by the plan after c1
            raise RuntimeError("FlashLog sparse top-k received non-finite attention weights; "
                               "aborting before edge count/fill to prevent uninitialized indices")
        if err == 2 and attempt == 0:
            # rows out of order: process them in row order, entries of a row in input order
            perm = torch.argsort(sp_b * L + sp_l, stable=True)
            # (operators are per row, unaffected by the entry order)
            sp_b, sp_l, sp_e, sp_v = sp_b[perm], sp_l[perm], sp_e[perm], sp_v[perm].contiguous()
            continue
        if err:
            raise ValueError("sparse state index out of range for shape (%d, %d, %d)" % (B, L, E))
        break
    h.items, h.tiles, h.chunks = items, tiles, chunks
    ws2_bytes = lib.fl_sparse_expand_bytes(items, tiles, chunks, R, E, 1 if need_backward else 0, int(aggregate))
    ws2 = torch.empty(max(ws2_bytes, 1), dtype=torch.uint8, device=dev)
    h.ws2, h.ws2_bytes = ptr(ws2).value, ws2.numel()
    out_base = torch.empty(R * nb + 1, dtype=torch.int64, device=dev)
    raw_local = torch.empty(max(items, 1), dtype=torch.int32, device=dev) if need_backward else None
    raw_pos = raw_col = None
    if need_backward:
        if not sides.positions_optional(mode, aggregate, nb):
            raw_pos = torch.empty(max(items, 1), dtype=torch.int32, device=dev)
        raw_col = torch.empty(max(items, 1), dtype=torch.int16, device=dev)
        h.raw_pos = ptr(raw_pos).value if raw_pos is not None else None
        h.raw_col = ptr(raw_col).value
    check(lib.fl_sparse_expand(st, ctypes.byref(sides.ori), ctypes.byref(sides.inv), ctypes.byref(h),
                               ptr(out_base), ptr(raw_local) if need_backward else None), "sparse_expand")
    nout = int(out_base[-1])
    if plan_log is not None:
        # sizes for byte counts: the groups the entries' sources hold on both sides
        go, gi = sides.keep[2].long(), sides.keep[11].long()
        groups = int((go[sp_e + 1] - go[sp_e] + gi[sp_e + 1] - gi[sp_e]).sum()) if nnz else 0
        plan_log.append({"nnz": nnz, "items": items, "chunks": chunks, "backward": bool(need_backward),
                         "nout": nout, "groups": groups, "rows": R, "n": n, "wot_i": bool(wot_i)})
    idx = torch.empty((3, nout), dtype=torch.int64, device=dev)
    vals = torch.empty(nout, dtype=torch.float32, device=dev)
    check(lib.fl_sparse_emit(st, ctypes.byref(h), ptr(out_base), ptr(idx[0]), ptr(idx[1]), ptr(idx[2]),
                             ptr(vals)), "sparse_emit")
    state = None
    if need_backward:
        state = _SparseState()
        state.h, state.sides, state.perm = h, sides, perm
        state.keep = (sp_b, sp_l, sp_e, sp_v, w_flat, ws1, out_base, raw_local, raw_pos, raw_col, order)
        state.out_base, state.raw_local, state.nout, state.n = out_base, raw_local, nout, n
    del ws2
    return idx, vals, state


def _fixed_sides(csr_struct):
    """Sides for the fixed-relation step (no masks): cached per CSR tuple."""
    keyed = (csr_struct[1], csr_struct[8], csr_struct[10], csr_struct[5], csr_struct[12], csr_struct[14])
    key = tuple((t.data_ptr(), t.numel(), t._version) for t in keyed)
    hit = _FIXED_SIDES.get(key)
    if hit is not None and all(r() is t for r, t in zip(hit[0], keyed)):
        return hit[1]
    for k in [k for k, v in _FIXED_SIDES.items() if any(r() is None for r in v[0])]:
        del _FIXED_SIDES[k]
    sides = _SparseSides(csr_struct[1], None, csr_struct[8], csr_struct[9], csr_struct[10], csr_struct[11],
                         csr_struct[5], None, csr_struct[12], csr_struct[13], csr_struct[14], csr_struct[15])
    _FIXED_SIDES[key] = (tuple(weakref.ref(t) for t in keyed), sides)
    return sides


_FIXED_SIDES = {}


def _sparse_backward(state, grad_values, grad_edge=None):
    """grad_values: gradient of every output entry.  Returns (grad_v, grad_w [R, n]);
    grad_edge (zeroed, by original edge id) receives the edge-weight gradient
    when the forward's sides carry the dscore factors."""
    h = state.h
    dev = grad_values.device
    grad_values = grad_values.contiguous().float()
    gv = torch.empty(max(h.nnz, 1), dtype=torch.float32, device=dev)
    gw = torch.empty((h.B * h.L, state.n), dtype=torch.float32, device=dev)
    lib = _lib.lib()
    ws_bytes = lib.fl_sparse_backward_bytes(h.nnz, h.B * h.L, state.n)
    if grad_edge is not None:  # the edge terms' sort and fold scratch
        ws_bytes += lib.fl_sparse_backward_edge_bytes(h.items, state.sides.ori.edges, state.sides.inv.edges)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    state.sides.set_grad_edge(grad_edge)
    try:
        check(lib.fl_sparse_backward(_stream(grad_values), ctypes.byref(state.sides.ori),
                                     ctypes.byref(state.sides.inv), ctypes.byref(h), ptr(state.out_base),
                                     ptr(state.raw_local), ptr(grad_values), ptr(gv), ptr(gw), ptr(ws), ws_bytes),
              "sparse_backward")
    finally:
        state.sides.set_grad_edge(None)
    gv = gv[:h.nnz]
    if state.perm is not None:
        restored = torch.empty_like(gv)
        restored[state.perm] = gv
        gv = restored
    return gv, gw


def _same_index_rows(gi, rows):
    """True when the rows of gi are the very tensors in rows (same storage),
    so the values already follow those coordinates (no device round trip)."""
    if gi.dim() != 2 or gi.shape[0] != len(rows) or gi.device != rows[0].device:
        return False
    return all(gi[k].numel() == r.numel() and gi[k].data_ptr() == r.data_ptr() and gi[k].stride() == r.stride()
               for k, r in enumerate(rows))


def _grad_at_outputs(grad, out_indices, L, E):
    """The upstream gradient's values at the hop's output coordinates
    [3, n] (the role of flashlog_kernel.py:360-376): a dense gradient is
    indexed; a sparse one with the very index rows of the output is taken
    as is; any other sparse one is coalesced and looked up by fl_sparse_gather
    (0 where it holds no entry)."""
    if not grad.is_sparse:
        return grad[tuple(out_indices)].contiguous()
    rows = [out_indices[k] for k in range(out_indices.shape[0])]
    if _same_index_rows(grad._indices(), rows):
        return grad._values().contiguous()
    g = grad.coalesce()
    gi = g.indices()
    gv = g.values().float().contiguous()
    q = out_indices.long()
    out = torch.empty(q.shape[1], dtype=torch.float32, device=q.device)
    check(_lib.lib().fl_sparse_gather(_stream(q), ptr(gi[0].contiguous()), ptr(gi[1].contiguous()),
                                      ptr(gi[2].contiguous()), ptr(gv), gv.numel(), ptr(q[0].contiguous()),
                                      ptr(q[1].contiguous()), ptr(q[2].contiguous()), q.shape[1], int(L), int(E),
                                      ptr(out)), "sparse_gather")
    return out.to(grad.dtype)


def _sparse_rows_scratch(R, device):
    return (torch.empty(R + 1, dtype=torch.int64, device=device),
            torch.empty(1, dtype=torch.int64, device=device))


@torch.no_grad()
def _sparse_topc_entries(sp_batch, sp_level, sp_entity, sp_value, topk_nodes, num_rules, sampling=False, B=None):
    """Kept entries of the c1 budget per (item, rule) row of a coalesced state
    (flashlog_kernel.py:1092-1140), or None when nothing is pruned.  B: the
    batch size when the caller knows it (else 1 + the largest batch index)."""
    picked = _sparse_topc_select(sp_batch, sp_level, sp_entity, sp_value, topk_nodes, num_rules, sampling, B)
    return None if picked is None else picked[0]


def _sparse_topc_select(sp_batch, sp_level, sp_entity, sp_value, topk_nodes, num_rules, sampling=False, B=None):
    """(kept entries, their (b, l, e, v) or None) of the c1 budget, or None
    when nothing is pruned.  The sampled race compacts the kept entries in
    its select kernel, with their count known from its plan."""
    if topk_nodes is None:
        return None
    if topk_nodes < 0:
        raise ValueError("topk_nodes/c must be nonnegative")
    if sp_entity.numel() <= topk_nodes:
        return None
    _require_cuda(sp_batch, sp_level, sp_value)
    L = int(num_rules)
    if B is None:
        B = int(sp_batch.max()) + 1 if sp_batch.numel() else 0
    sp_batch = sp_batch.long().contiguous()
    sp_level = sp_level.long().contiguous()
    sp_value = sp_value.contiguous().float()
    keep = torch.empty(sp_value.numel(), dtype=torch.int32, device=sp_value.device)
    if sampling and topk_nodes > 0:
        return _sparse_race_entries(sp_batch, sp_level, sp_entity.long().contiguous(), sp_value, B, L,
                                    int(topk_nodes), keep)
    row_ptr, err = _sparse_rows_scratch(B * L, sp_value.device)
    check(_lib.lib().fl_sparse_topc(_stream(sp_value), ptr(sp_batch), ptr(sp_level), ptr(sp_value),
                                    sp_value.numel(), B, L, int(topk_nodes), ptr(keep), ptr(row_ptr), ptr(err)),
          "sparse_topc")
    if int(err) != 0:
        raise ValueError("sparse c1 needs a state coalesced by (batch, rule, entity)")
    if bool(keep.all()):
        return None
    return torch.nonzero(keep, as_tuple=True)[0], None


def _sparse_race_entries(sp_batch, sp_level, sp_entity, sp_value, B, L, c, keep):
    """Sampled c1 (flashlog_kernel.py:1121-1132): the exponential race over
    the nonzero entries of over-limit rows.  The Exp(1) noise is drawn as the
    reference draws it (one float64 per candidate, entry order, torch's
    generator of the state's device).  Returns (kept entries, their
    (b, l, e, v)), both written by the select; the kept count comes with the
    candidate count."""
    lib = _lib.lib()
    dev = sp_value.device
    nnz = sp_value.numel()
    ws = torch.empty(max(lib.fl_sparse_race_bytes(nnz, B * L), 1), dtype=torch.uint8, device=dev)
    info = torch.empty(3, dtype=torch.int64, device=dev)
    st = _stream(sp_value)
    check(lib.fl_sparse_race_plan(st, ptr(sp_batch), ptr(sp_level), ptr(sp_value), nnz, B, L, c, ptr(ws),
                                  ws.numel(), ptr(info)), "sparse_race_plan")
    ncand, err, kept = info.tolist()
    if err in (1, 2):
        raise ValueError("sparse c1 needs a state coalesced by (batch, rule, entity)")
    if ncand == 0:
        return None
    if err == 3:
        raise ValueError("Entity sampling requires finite nonnegative state scores")
    noise = torch.empty(ncand, dtype=torch.float64, device=dev).exponential_()
    entries = torch.empty(kept, dtype=torch.int64, device=dev)
    out = torch.empty((3, kept), dtype=torch.int64, device=dev)
    out_v = torch.empty(kept, dtype=torch.float32, device=dev)
    check(lib.fl_sparse_race_select_compact(st, ptr(sp_batch), ptr(sp_level), ptr(sp_entity), ptr(sp_value), nnz,
                                            B, L, c, ptr(noise), ptr(ws), ws.numel(), ptr(keep), ptr(entries),
                                            ptr(out[0]), ptr(out[1]), ptr(out[2]), ptr(out_v)),
          "sparse_race_select")
    return entries, (out[0], out[1], out[2], out_v)


class _C1Pick:
    """The entries a hop keeps under the c1 budget (all when `entries` is
    None), applied to the state's arrays and undone on the gradient (the
    role of flashlog_kernel.py:1140-1155)."""

    def __init__(self, picked, size):
        self.entries, self.taken = picked if picked is not None else (None, None)
        self.size = size

    def take(self, *arrays):
        if self.entries is None:
            return arrays
        if self.taken is not None:
            # the selection wrote the kept (b, l, e, v) itself
            return tuple(t.to(x.dtype) for t, x in zip(self.taken, arrays))
        return tuple(x.index_select(0, self.entries) for x in arrays)

    def untake(self, grad):
        if self.entries is None:
            return grad
        return grad.new_zeros(self.size).index_copy_(0, self.entries, grad)


def _c1_pick(ctx, batch, level, entity, value, topk_nodes, num_rules, sampling=False, B=None):
    pick = _C1Pick(_sparse_topc_select(batch, level, entity, value, topk_nodes, num_rules, sampling, B),
                   value.numel())
    ctx.c1_pick = pick
    return pick.take(batch, level, entity, value)


def _coo(idx, vals, B, L, E):
    return torch.sparse_coo_tensor(idx, vals, [B, L, E], is_coalesced=True)


_MASK_CACHE = {}


def _mask_bits(mask_f):
    """One bit per CSR position (mask != 0), for masks of 0s and 1s."""
    n = mask_f.numel()
    bits = torch.empty(max((n + 31) // 32, 1), dtype=torch.int32, device=mask_f.device)
    check(_lib.lib().fl_mask_bits(_stream(mask_f), ptr(mask_f), n, ptr(bits)), "mask_bits")
    return bits


def _mask_order_bits(mask_values, order):
    """The side's bitmap (bit p = mask[order[p]]) straight from a Boolean
    mask by edge id (fl_mask_order_bits: no float mask is gathered)."""
    n = order.numel()
    words = max((n + 31) // 32, 1)
    edge_bits = torch.empty(words, dtype=torch.int32, device=mask_values.device)
    bits = torch.empty(words, dtype=torch.int32, device=mask_values.device)
    check(_lib.lib().fl_mask_order_bits(_stream(mask_values), ptr(mask_values), ptr(order), n, ptr(edge_bits),
                                        ptr(bits)), "mask_order_bits")
    return bits


def _cached_mask_order(mask_values, order):
    """(mask[order] as float, or None; its bitmap, or None) for a side of the
    top-k hop without edge weights: a Boolean mask gives only the bitmap
    (every value 0 or 1, read as bits by the kernels), another mask only the
    float gather.  Reused while the same (unmodified) mask and order tensors
    are passed again (the hop gets the raw per-edge mask on every call; a
    training step that hides its batch's triples in place changes the
    mask's version, so the first hop of the step rebuilds it)."""
    key = (mask_values.data_ptr(), mask_values._version, mask_values.numel(), order.data_ptr(), order._version,
           order.numel())
    hit = _MASK_CACHE.get(key)
    if hit is not None and hit[0]() is mask_values and hit[1]() is order:
        return hit[2]
    for k in [k for k, v in _MASK_CACHE.items() if v[0]() is None or v[1]() is None]:
        del _MASK_CACHE[k]
    flat = mask_values.contiguous().view(-1)
    _require_cuda(flat, order)
    if flat.dtype == torch.bool:
        if order.numel() != flat.numel():
            raise ValueError("mask length must equal the number of CSR positions")
        out = (None, _mask_order_bits(flat, order.to(torch.int32).contiguous()))
    else:
        out = (_apply_mask_order(flat, order, None), None)
    _MASK_CACHE[key] = (weakref.ref(mask_values), weakref.ref(order), out)
    return out


class FlashLogFunctionSparse3DAllEdgesSum(autograd.Function):
    """Sparse sum hop over every edge, masked ones included as 0-valued
    coordinates (flashlog_kernel.py:1351-1447)."""

    @staticmethod
    def forward(ctx, sp_batch, sp_level, sp_entity, sp_value, w,
                ori_col_ind, ori_mask,
                ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
                inv_col_ind, inv_mask,
                inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
                B, L, E, r_size, wot_i, cache_backward=True):
        sides = _SparseSides(ori_col_ind, ori_mask, ori_row_group_ptr, ori_group_rel, ori_group_edge_start,
                             ori_group_edge_count, inv_col_ind, inv_mask, inv_row_group_ptr, inv_group_rel,
                             inv_group_edge_start, inv_group_edge_count)
        need = bool(any(ctx.needs_input_grad))
        idx, vals, state = _sparse_forward(sp_batch, sp_level, sp_entity, sp_value, w, sides, B, L, E, r_size,
                                           wot_i, _SPARSE_ALL, 0, need)
        ctx.state, ctx.out_indices, ctx.dims = state, idx, (int(B), int(L), int(E), tuple(w.shape))
        return _coo(idx, vals, int(B), int(L), int(E))

    @staticmethod
    def backward(ctx, grad_out):
        B, L, E, wshape = ctx.dims
        aligned = _grad_at_outputs(grad_out, ctx.out_indices, L, E)
        gv, gw = _sparse_backward(ctx.state, aligned)
        grads = (None, None, None, gv, gw.view(wshape)) + (None,) * 17
        return (grads + (None,))[:len(ctx.needs_input_grad)]


def _topk_hop_forward(ctx, aggregate, sp_batch, sp_level, sp_entity, sp_value, w, ori_col_ind, ori_order,
                      inv_col_ind, inv_order, ori_row_group_ptr, ori_group_rel, ori_group_edge_start,
                      ori_group_edge_count, inv_row_group_ptr, inv_group_rel, inv_group_edge_start,
                      inv_group_edge_count, mask_values, weight, B, L, E, r_size, wot_i, topk_edges,
                      edge_weight_is_score, topk_nodes, sampling):
    """Forward of the top-k sum / max hops (flashlog_kernel.py:1158-1348,
    1450-1626): c1 (sampled with the exponential race when training), then
    the hop with the c2 threshold or, when sampling, the training quotas
    seeded by one draw of torch's CPU generator, as the reference draws it."""
    trainable = weight is not None and bool(getattr(weight, "requires_grad", False))
    _require_cuda(sp_value, w)
    sp_batch, sp_level, sp_entity, sp_value = _c1_pick(
        ctx, sp_batch, sp_level, sp_entity, sp_value, topk_nodes, w.size(1), sampling, B=int(B))
    mask_f = mask_values.contiguous().view(-1)
    ori_bits = inv_bits = None
    if weight is not None and edge_weight_is_score:
        m = mask_f.float() * weight.to(device=mask_f.device, dtype=torch.float).view(-1)
        ori_mask = m[ori_order.long()].contiguous()
        inv_mask = m[inv_order.long()].contiguous()
    elif weight is None:
        ori_mask, ori_bits = _cached_mask_order(mask_values, ori_order)
        inv_mask, inv_bits = _cached_mask_order(mask_values, inv_order)
    else:
        ori_mask = _apply_mask_order(mask_f, ori_order, weight)
        inv_mask = _apply_mask_order(mask_f, inv_order, weight)
    max_hop = aggregate == _SPARSE_MAX
    dscore = (None, None)
    if trainable:
        ew = weight.detach().to(device=mask_f.device, dtype=torch.float).contiguous().view(-1)
        dscore = tuple(_edge_dscore(ew, order) for order in (ori_order, inv_order))
    with_order = max_hop or trainable
    sides = _SparseSides(ori_col_ind, ori_mask, ori_row_group_ptr, ori_group_rel, ori_group_edge_start,
                         ori_group_edge_count, inv_col_ind, inv_mask, inv_row_group_ptr, inv_group_rel,
                         inv_group_edge_start, inv_group_edge_count,
                         ori_order if with_order else None, inv_order if with_order else None, *dscore,
                         ori_bits=ori_bits, inv_bits=inv_bits)
    seed = int(torch.randint(0, 2 ** 63 - 1, ()).item()) if sampling else -1
    need = bool(any(ctx.needs_input_grad))
    idx, vals, state = _sparse_forward(sp_batch, sp_level, sp_entity, sp_value, w, sides, B, L, E, r_size,
                                       wot_i, _SPARSE_TOPK, int(topk_edges), need, aggregate=aggregate, seed=seed,
                                       check_finite=True)
    ctx.state, ctx.out_indices, ctx.dims = state, idx, (int(B), int(L), int(E), tuple(w.shape))
    ctx.edge_weight = (tuple(weight.shape), weight.dtype, weight.device) if trainable else None
    return _coo(idx, vals, int(B), int(L), int(E))


def _edge_dscore(ew, order):
    order = order.to(device=ew.device, dtype=torch.int32).contiguous()
    out = torch.empty(order.numel(), dtype=torch.float32, device=ew.device)
    check(_lib.lib().fl_edge_dscore(_stream(ew), ptr(ew), ptr(order), ptr(out), order.numel()), "edge_dscore")
    return out


def _topk_hop_backward(ctx, grad_out):
    B, L, E, wshape = ctx.dims
    aligned = _grad_at_outputs(grad_out, ctx.out_indices, L, E)
    grad_edge = None
    if ctx.edge_weight is not None:
        shape, dtype, device = ctx.edge_weight
        grad_edge = torch.zeros(int(np.prod(shape)), dtype=torch.float32, device=aligned.device)
    gv, gw = _sparse_backward(ctx.state, aligned, grad_edge)
    gv = ctx.c1_pick.untake(gv)
    ge = grad_edge.view(shape).to(device=device, dtype=dtype) if grad_edge is not None else None
    grads = (None, None, None, gv, gw.view(wshape)) + (None,) * 17 + (ge,) + (None,) * 10
    return grads[:len(ctx.needs_input_grad)]


class FlashLogFunctionSparse3DTopKSum(autograd.Function):
    """Sparse sum hop with the c1 entity budget and the c2 edge budget
    (flashlog_kernel.py:1158-1348): hard-masked edges take part in the c2
    selection but produce no coordinate.  sampling=True: the training
    selections (exponential-race c1, quota c2)."""

    @staticmethod
    def forward(ctx, sp_batch, sp_level, sp_entity, sp_value, w,
                ori_row_ptr, ori_col_ind, ori_r_ind, ori_order,
                inv_row_ptr, inv_col_ind, inv_r_ind, inv_order,
                ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
                inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
                mask_values, weight, B, L, E, r_size, wot_i, topk_edges,
                edge_weight_is_score=False, topk_nodes=None, cache_backward=True, sampling=False):
        return _topk_hop_forward(ctx, _SPARSE_SUM, sp_batch, sp_level, sp_entity, sp_value, w, ori_col_ind,
                                 ori_order, inv_col_ind, inv_order, ori_row_group_ptr, ori_group_rel,
                                 ori_group_edge_start, ori_group_edge_count, inv_row_group_ptr, inv_group_rel,
                                 inv_group_edge_start, inv_group_edge_count, mask_values, weight, B, L, E, r_size,
                                 wot_i, topk_edges, edge_weight_is_score, topk_nodes, sampling)

    @staticmethod
    def backward(ctx, grad_out):
        return _topk_hop_backward(ctx, grad_out)


class FlashLogFunctionSparse3DTopKMax(autograd.Function):
    """Sparse max hop (flashlog_kernel.py:1450-1626): per output the largest
    item, ties to ORI before INV before the identity term, then the smaller
    original edge id, then the earlier item; masked kept edges are 0-valued
    items (their coordinates exist).  The backward routes each output's
    gradient to its winner only."""

    @staticmethod
    def forward(ctx, sp_batch, sp_level, sp_entity, sp_value, w,
                ori_row_ptr, ori_col_ind, ori_r_ind, ori_order,
                inv_row_ptr, inv_col_ind, inv_r_ind, inv_order,
                ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
                inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
                mask_values, weight, B, L, E, r_size, wot_i, topk_edges,
                edge_weight_is_score=False, topk_nodes=None, cache_backward=True, sampling=False):
        return _topk_hop_forward(ctx, _SPARSE_MAX, sp_batch, sp_level, sp_entity, sp_value, w, ori_col_ind,
                                 ori_order, inv_col_ind, inv_order, ori_row_group_ptr, ori_group_rel,
                                 ori_group_edge_start, ori_group_edge_count, inv_row_group_ptr, inv_group_rel,
                                 inv_group_edge_start, inv_group_edge_count, mask_values, weight, B, L, E, r_size,
                                 wot_i, topk_edges, edge_weight_is_score, topk_nodes, sampling)

    @staticmethod
    def backward(ctx, grad_out):
        return _topk_hop_backward(ctx, grad_out)


class _SparseCpuPath:
    """The reference's CPU sparse classes, run on the GPU: inputs and outputs
    stay CPU tensors, the hop is the same fl_sparse_* pipeline (mode 0 with
    the given c2 budget, i.e. the CPU path's kept-edge semantics)."""

    @staticmethod
    def run(ctx, sp_batch, sp_level, sp_entity, sp_value, w, side_args, B, L, E, r_size, wot_i, topk_edges):
        if not torch.cuda.is_available():
            raise RuntimeError("flashlog_amd runs its sparse kernels on the GPU; no GPU is visible")
        dev = torch.device("cuda")
        g = [t.to(dev) for t in side_args]
        sides = _SparseSides(*g)
        K = int(topk_edges)
        need = bool(any(ctx.needs_input_grad))
        idx, vals, state = _sparse_forward(sp_batch.to(dev), sp_level.to(dev), sp_entity.to(dev),
                                           sp_value.to(dev).float(), w.to(dev), sides, B, L, E, r_size, wot_i,
                                           _SPARSE_TOPK, K, need)
        ctx.state, ctx.out_indices, ctx.dims = state, idx, (int(B), int(L), int(E), tuple(w.shape))
        return idx, vals


class FlashLogFunctionSparse3DCPUSum(autograd.Function):
    """flashlog_kernel.py:1691-1744 with CPU tensors in and out."""

    @staticmethod
    def forward(ctx, sp_batch, sp_level, sp_entity, sp_value, w,
                ori_col_ind, ori_mask,
                ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
                inv_col_ind, inv_mask,
                inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
                B, L, E, r_size, wot_i, topk_edges):
        idx, vals = _SparseCpuPath.run(
            ctx, sp_batch, sp_level, sp_entity, sp_value, w,
            (ori_col_ind, ori_mask, ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
             inv_col_ind, inv_mask, inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count),
            B, L, E, r_size, wot_i, topk_edges)
        ctx.home = sp_value.device
        return _coo(idx.to(ctx.home), vals.to(ctx.home, sp_value.dtype), int(B), int(L), int(E))

    @staticmethod
    def backward(ctx, grad_out):
        B, L, E, wshape = ctx.dims
        dev = ctx.out_indices.device
        aligned = _grad_at_outputs(grad_out.to(dev), ctx.out_indices, L, E)
        gv, gw = _sparse_backward(ctx.state, aligned)
        return (None, None, None, gv.to(ctx.home), gw.view(wshape).to(ctx.home)) + (None,) * 18


class FlashLogFunctionSparse3DCPUSumNorm(autograd.Function):
    """flashlog_kernel.py:1747-1811 with CPU tensors in and out: the sum hop,
    then the per-row normalization."""

    @staticmethod
    def forward(ctx, sp_batch, sp_level, sp_entity, sp_value, w,
                ori_col_ind, ori_mask,
                ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
                inv_col_ind, inv_mask,
                inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count,
                B, L, E, r_size, wot_i, topk_edges, eps):
        idx, vals = _SparseCpuPath.run(
            ctx, sp_batch, sp_level, sp_entity, sp_value, w,
            (ori_col_ind, ori_mask, ori_row_group_ptr, ori_group_rel, ori_group_edge_start, ori_group_edge_count,
             inv_col_ind, inv_mask, inv_row_group_ptr, inv_group_rel, inv_group_edge_start, inv_group_edge_count),
            B, L, E, r_size, wot_i, topk_edges)
        out, denom, row_ptr = _normalize_forward(idx[0], idx[1], vals, int(B), int(L), float(eps))
        ctx.norm = (vals, denom, row_ptr, float(eps))
        ctx.home = sp_value.device
        return _coo(idx.to(ctx.home), out.to(ctx.home, sp_value.dtype), int(B), int(L), int(E))

    @staticmethod
    def backward(ctx, grad_out):
        B, L, E, wshape = ctx.dims
        dev = ctx.out_indices.device
        vals, denom, row_ptr, eps = ctx.norm
        aligned = _grad_at_outputs(grad_out.to(dev), ctx.out_indices, L, E)
        g_sum = _normalize_backward(row_ptr, aligned, vals, denom, eps)
        gv, gw = _sparse_backward(ctx.state, g_sum)
        return (None, None, None, gv.to(ctx.home), gw.view(wshape).to(ctx.home)) + (None,) * 19


def _normalize_forward(sp_b, sp_l, values, B, L, eps):
    """As the reference's GPU path (flashlog.cu:2594-2649) the entry order
    is not checked on the host (no device read): the state comes from
    coalesce(), and rows out of order give unspecified values without any
    access out of bounds."""
    _require_cuda(sp_b, sp_l, values)
    values = values.contiguous().float()
    R = B * L
    out = torch.empty_like(values)
    denom = torch.empty(max(R, 1), dtype=torch.float32, device=values.device)
    row_ptr, err = _sparse_rows_scratch(R, values.device)
    check(_lib.lib().fl_sparse_normalize_forward(_stream(values), ptr(sp_b.long().contiguous()),
                                                 ptr(sp_l.long().contiguous()), ptr(values), values.numel(),
                                                 B, L, ctypes.c_float(eps), ptr(out), ptr(denom), ptr(row_ptr),
                                                 ptr(err)), "sparse_normalize")
    return out, denom[:R], row_ptr


def _normalize_backward(row_ptr, grad, values, denom, eps):
    grad = grad.contiguous().float()
    gv = torch.empty_like(values)
    check(_lib.lib().fl_sparse_normalize_backward(_stream(values), ptr(row_ptr), ptr(grad), ptr(values),
                                                  ptr(denom), denom.numel(), ctypes.c_float(eps), ptr(gv)),
          "sparse_normalize_backward")
    return gv


def _stacked_rows(*rows):
    """torch.stack(rows): a view when the rows already are the consecutive
    rows of one contiguous [k, n] tensor (a state's own index tensor), else
    a copy."""
    r0 = rows[0]
    n = r0.numel()
    if all(r.dim() == 1 and r.dtype == r0.dtype and r.device == r0.device and r.stride(0) == 1 and r.numel() == n
           and r.untyped_storage().data_ptr() == r0.untyped_storage().data_ptr()
           and r.storage_offset() == r0.storage_offset() + k * n for k, r in enumerate(rows)):
        return r0.as_strided((len(rows), n), (n, 1), r0.storage_offset())
    return torch.stack(rows, dim=0)


class Sparse3DNormalizeFunction(autograd.Function):
    """Per (b, l) row: v / max(sum of the row, eps) (flashlog_kernel.py:536-606).
    The entries must be sorted by row with b*L + l in [0, B*L) (a coalesced
    state); as in the reference's GPU path this is not checked, and other
    input gives unspecified (but written) values."""

    @staticmethod
    def forward(ctx, sp_batch, sp_level, sp_entity, sp_value, B, L, E, eps):
        sp_batch = sp_batch.contiguous().long()
        sp_level = sp_level.contiguous().long()
        sp_entity = sp_entity.contiguous().long()
        values = sp_value.contiguous()
        out, denom, row_ptr = _normalize_forward(sp_batch, sp_level, values, int(B), int(L), float(eps))
        idx = _stacked_rows(sp_batch, sp_level, sp_entity)
        ctx.save_for_backward(idx, values.float(), denom, row_ptr)
        ctx.B, ctx.L, ctx.E, ctx.eps = int(B), int(L), int(E), float(eps)
        return torch.sparse_coo_tensor(idx, out.to(sp_value.dtype), [int(B), int(L), int(E)], is_coalesced=True)

    @staticmethod
    def backward(ctx, grad_out):
        idx, values, denom, row_ptr = ctx.saved_tensors
        # the output's own index tensor: a gradient built on it needs no lookup
        g = _grad_at_outputs(grad_out, idx, ctx.L, ctx.E)
        gv = _normalize_backward(row_ptr, g, values, denom, ctx.eps)
        return None, None, None, gv, None, None, None, None


def normalize_sparse3d(s, eps=1e-7):
    """Per-(b, l) normalization of a [B, L, E] COO state
    (flashlog_kernel.py:610-614), through Sparse3DNormalizeFunction."""
    c = s.coalesce()  # returns s itself when it is already coalesced
    b, l, e = c.indices()
    return Sparse3DNormalizeFunction.apply(b, l, e, c.values(), *c.shape, eps)


def _channel_reduce(sp_batch, sp_level, sp_entity, sp_value, B, L, E, op):
    _require_cuda(sp_batch, sp_level, sp_entity, sp_value)
    dev = sp_value.device
    sb, sl, se = (x.long().contiguous() for x in (sp_batch, sp_level, sp_entity))
    v = sp_value.detach().contiguous().float()
    nnz = v.numel()
    lib = _lib.lib()
    st = _stream(v)
    ws = torch.empty(max(int(lib.fl_sparse_channel_sum_bytes(nnz, B, L)), 1), dtype=torch.uint8, device=dev)
    plan = torch.empty(2, dtype=torch.int64, device=dev)
    check(lib.fl_sparse_channel_sum_plan(st, ptr(sb), ptr(sl), ptr(se), nnz, B, L, E, ptr(ws), ws.numel(),
                                         ptr(plan)), "sparse_channel_sum_plan")
    nout, err = (int(x) for x in plan.cpu())
    if err != 0:
        raise ValueError("the channel reduction needs a state coalesced by (batch, rule, entity) within its shape")
    idx = torch.empty((2, nout), dtype=torch.int64, device=dev)
    out = torch.empty(nout, dtype=torch.float32, device=dev)
    slot = torch.empty(nnz, dtype=torch.int32, device=dev)
    check(lib.fl_sparse_channel_sum_emit(st, ptr(sb), ptr(se), ptr(v), nnz, B, L, op, ptr(ws), nout,
                                         ptr(idx[0]), ptr(idx[1]), ptr(out), ptr(slot)),
          "sparse_channel_sum_emit")
    return idx, out, slot.long(), v


class Sparse3DChannelSumFunction(autograd.Function):
    """Values of the channel sum of a coalesced [B, L, E] state: per (b, e)
    the entries of every channel added from 0 in channel order, as torch's
    coalesce of the (b, e) re-index adds them (src/model_DRUM_kernel_sp.py:
    22-28); the gradient of an entry is its output's."""

    @staticmethod
    def forward(ctx, sp_batch, sp_level, sp_entity, sp_value, B, L, E):
        idx, out, slot, _ = _channel_reduce(sp_batch, sp_level, sp_entity, sp_value, B, L, E, 0)
        ctx.slot = slot
        ctx.mark_non_differentiable(idx)
        return idx, out

    @staticmethod
    def backward(ctx, grad_idx, grad_out):
        if grad_out is None:
            return (None,) * 7
        return None, None, None, grad_out.contiguous().float()[ctx.slot], None, None, None


class Sparse3DChannelMaxFunction(autograd.Function):
    """Values of the channel maximum of a coalesced [B, L, E] state
    (src/model_mmDRUM_kernel_sp.py:17-32, scatter_reduce amax with
    include_self=False).  Backward as torch's for amax: an output's gradient
    is divided evenly among the entries equal to it and, where the maximum
    is 0, the zero the reference reduces into (torch counts that initial
    value among the ties)."""

    @staticmethod
    def forward(ctx, sp_batch, sp_level, sp_entity, sp_value, B, L, E):
        idx, out, slot, v = _channel_reduce(sp_batch, sp_level, sp_entity, sp_value, B, L, E, 1)
        ctx.save_for_backward(v, out, slot)
        ctx.mark_non_differentiable(idx)
        return idx, out

    @staticmethod
    def backward(ctx, grad_idx, grad_out):
        if grad_out is None:
            return (None,) * 7
        v, out, slot = ctx.saved_tensors
        value = out[slot]
        is_max = (v == value).to(v.dtype)
        count = (out == 0).to(out.dtype).scatter_add_(0, slot, is_max)
        share = grad_out.contiguous().float() / count
        return None, None, None, is_max * share[slot], None, None, None


def _channel_state(s, fn):
    s = s if s.is_coalesced() else s.coalesce()
    B, L, E = s.shape
    idx = s.indices()
    out_idx, out_val = fn.apply(idx[0], idx[1], idx[2], s.values(), B, L, E)
    return torch.sparse_coo_tensor(out_idx, out_val, [B, E], is_coalesced=True)


def sum_sp_3d(s):
    """[B, L, E] -> [B, E]: the sum over channels (src/model_DRUM_kernel_sp.py:
    22-28), a coalesced COO tensor whose values carry the gradient."""
    return _channel_state(s, Sparse3DChannelSumFunction)


def max_sp_3d(s):
    """[B, L, E] -> [B, E]: the maximum over channels
    (src/model_mmDRUM_kernel_sp.py:17-32), a coalesced COO tensor."""
    return _channel_state(s, Sparse3DChannelMaxFunction)


# ---------------------------------------------------------------------------
# Sparse dispatch (the two entry points of flashlog_kernel.py:1814-1954).
# One routine serves both: it decides a route from where the state lives and
# what the call budgets, and builds the chosen class's positional arguments
# from slices of the CSR tuple.  Routes:
#   "sampled" -- training selections (sampling with use_topk);
#   "all"     -- GPU state, no budget and no trainable edge weight: every edge;
#   "topk"    -- GPU state with a c1/c2 budget or a trainable edge weight;
#   "host"    -- CPU state: the CPU classes (computed on the GPU, CPU tensors
#                out), after c1 when a node budget is given.

# Per side, the CSR tuple slots of (columns, group pointer, group relations,
# group starts, group counts).
_SIDE_SLOTS = ((1, 8, 9, 10, 11), (5, 12, 13, 14, 15))


def _side_parameters(csr_struct, masks):
    """(columns, mask, 4 group arrays) of ORI then INV: the side parameters
    of the all-edges and CPU hop classes."""
    params = []
    for (col, *groups), mask in zip(_SIDE_SLOTS, masks):
        params.append(csr_struct[col])
        params.append(mask)
        params.extend(csr_struct[g] for g in groups)
    return params


def _ordered_masks(csr_struct, mask_values, weight, prepared_masks, accept_raw_pair):
    """CSR-ordered masks: the prepared pair when one is given (or, where the
    reference accepts it, a pair passed as the raw mask), else prepared here."""
    candidates = [prepared_masks] if prepared_masks is not None else []
    if accept_raw_pair and prepared_masks is None:
        candidates.append(mask_values)
    for c in candidates:
        pair = _prepared_mask_pair(c)
        if pair is not None:
            return pair
    return prepare_csr_masks(csr_struct, mask_values, weight)


def _sparse_route(state, use_topk, topk_edges, topk_nodes, weight, sampling):
    if sampling and use_topk:
        return "sampled"
    if not state.is_cuda:
        return "host"
    budgeted = use_topk and (topk_edges > 0 or topk_nodes is not None)
    trained = weight is not None and bool(getattr(weight, "requires_grad", False))
    return "topk" if (budgeted or trained) else "all"


def _normalized(out, eps):
    return out if eps is None else normalize_sparse3d(out, eps=eps)


def _host_c1_subset(state, topk_nodes):
    """The CPU state restricted to its c1 entries (selected on the GPU), or
    None when the budget prunes nothing."""
    idx, val = state.indices(), state.values()
    if not torch.cuda.is_available():
        raise RuntimeError("flashlog_amd runs its sparse kernels on the GPU; no GPU is visible")
    dev = torch.device("cuda")
    kept = _sparse_topc_entries(*(x.to(dev) for x in (idx[0], idx[1], idx[2], val)), topk_nodes, state.shape[1])
    if kept is None:
        return None
    kept = kept.cpu()
    return torch.sparse_coo_tensor(idx.index_select(1, kept), val.index_select(0, kept), state.shape,
                                   is_coalesced=True)


def _sparse_hop(sp_state, w, csr_struct, mask_values, r_size, weight, wot_i, use_topk, topk_edges,
                prepared_masks, topk_nodes, sampling, eps):
    """The sum hop (eps None) or the sum followed by the per-row
    normalization with eps, on the route _sparse_route picks."""
    route = _sparse_route(sp_state, use_topk, topk_edges, topk_nodes, weight, sampling)
    if route == "sampled":
        out = sampled_sparse_propagation(sp_state, w, csr_struct, mask_values, r_size, weight, wot_i, topk_nodes,
                                         topk_edges, "sum")
        return _normalized(out, eps)
    state = sp_state.coalesce()
    B, L, E = state.shape
    coords = (*state.indices(), state.values(), w)
    budget = topk_edges if (use_topk and topk_edges > 0) else (1 << 60)
    grad_on = torch.is_grad_enabled()
    if route == "topk":
        out = FlashLogFunctionSparse3DTopKSum.apply(
            *coords, *csr_struct[:16], mask_values, weight, B, L, E, r_size, wot_i, budget, False,
            topk_nodes if use_topk else None, grad_on)
        return _normalized(out, eps)
    if route == "all":
        masks = _ordered_masks(csr_struct, mask_values, weight, prepared_masks, True)
        out = FlashLogFunctionSparse3DAllEdgesSum.apply(*coords, *_side_parameters(csr_struct, masks),
                                                        B, L, E, r_size, wot_i, grad_on)
        return _normalized(out, eps)
    # route "host": c1 first; a pruned state takes the (unfused) sum, then the normalization
    if use_topk and topk_nodes is not None:
        subset = _host_c1_subset(state, topk_nodes)
        if subset is not None:
            out = _sparse_hop(subset, w, csr_struct, mask_values, r_size, weight, wot_i, True, topk_edges,
                              prepared_masks, None, False, None)
            return _normalized(out, eps)
    masks = _ordered_masks(csr_struct, mask_values, weight, prepared_masks, False)
    sides = _side_parameters(csr_struct, masks)
    if eps is None:
        return FlashLogFunctionSparse3DCPUSum.apply(*coords, *sides, B, L, E, r_size, wot_i, budget)
    return FlashLogFunctionSparse3DCPUSumNorm.apply(*coords, *sides, B, L, E, r_size, wot_i, budget, eps)


def vectorized_operation_sparse3d_csr_sum(sp_state, w, csr_struct, mask_values,
                                          r_size, weight=None, wot_i=False,
                                          use_topk=False, topk_edges=0,
                                          prepared_masks=None, topk_nodes=None, sampling=False):
    """Sparse sum entry point (flashlog_kernel.py:1814-1888)."""
    return _sparse_hop(sp_state, w, csr_struct, mask_values, r_size, weight, wot_i, use_topk, topk_edges,
                       prepared_masks, topk_nodes, sampling, None)


def vectorized_operation_sparse3d_csr_sum_norm(sp_state, w, csr_struct, mask_values,
                                               r_size, weight=None, wot_i=False,
                                               use_topk=False, topk_edges=0,
                                               prepared_masks=None, eps=1e-7, topk_nodes=None, sampling=False):
    """Sparse sum + per-row normalization entry point
    (flashlog_kernel.py:1901-1954)."""
    return _sparse_hop(sp_state, w, csr_struct, mask_values, r_size, weight, wot_i, use_topk, topk_edges,
                       prepared_masks, topk_nodes, sampling, eps)
