"""numpy/ctypes front end of the C oracle (oracle/flashlog_oracle.c).

TEST INFRASTRUCTURE ONLY.  Every function mirrors a reference function
(citations in flashlog_oracle.c and below) in the reference's own float
evaluation order, so its outputs are the bit-exact targets for the HIP path.

Parity pinning of each function is listed in the C file's header; functions
restated here in numpy (``dense_topc_brute``, ``group_threshold_brute``,
``filtered_ranks_brute``) are the independent brute-force checks used to pin
the C restatement, not restatements of the reference.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SRC = os.path.join(_HERE, "flashlog_oracle.c")
_SRCS = [_SRC, os.path.join(_HERE, "grounding_oracle.c")]
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_i64p = ctypes.POINTER(ctypes.c_int64)


def build(force=False):
    """Compile the C oracle with gcc (no FMA contraction, IEEE semantics)."""
    if force or not os.path.exists(_LIB_PATH) or \
            os.path.getmtime(_LIB_PATH) < max(os.path.getmtime(f) for f in _SRCS):
        tmp = _LIB_PATH + ".tmp"
        subprocess.check_call(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math",
                               "-fPIC", "-shared", "-o", tmp] + _SRCS + ["-lm"])
        os.replace(tmp, _LIB_PATH)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# --------------------------------------------------------------------------
# CSR build: csr.cpp:12-69 (via flashlog_kernel.py:678-697 for the 16-tuple)

def build_side(source, target, relation, nodes):
    source = _c(source, np.int64)
    target = _c(target, np.int64)
    relation = _c(relation, np.int64)
    m = source.shape[0]
    row_ptr = np.empty(nodes + 1, np.int32)
    cols = np.empty(m, np.int32)
    erel = np.empty(m, np.int16)
    order = np.empty(m, np.int32)
    gptr = np.empty(nodes + 1, np.int32)
    grel = np.empty(max(m, 1), np.int16)
    gstart = np.empty(max(m, 1), np.int32)
    gcount = np.empty(max(m, 1), np.int32)
    ng = ctypes.c_int64(0)
    rc = lib().or_build_side(ctypes.c_int64(m), ctypes.c_int64(nodes), _p(source), _p(target),
                             _p(relation), _p(row_ptr), _p(cols), _p(erel), _p(order), _p(gptr),
                             _p(grel), _p(gstart), _p(gcount), ctypes.byref(ng))
    if rc != 0:
        raise ValueError("CSR entity or relation ID outside supported range")
    g = ng.value
    return row_ptr, cols, erel, order, gptr, grel[:g].copy(), gstart[:g].copy(), gcount[:g].copy()


def build_csr_structure(h, t, r, nodes):
    """The reference's 16-tuple (flashlog_kernel.py:678-697) as numpy arrays."""
    ori = build_side(h, t, r, nodes)
    inv = build_side(t, h, r, nodes)
    return (*ori[:4], *inv[:4], *ori[4:], *inv[4:])


# --------------------------------------------------------------------------
# c2 threshold: flashlog.cpp:12-35

def group_threshold(weights, relations, sizes, budget):
    weights = _c(weights, np.float32)
    relations = _c(relations, np.int16)
    sizes = _c(sizes, np.int32)
    rem = ctypes.c_int64(0)
    f = lib().or_group_threshold_f32
    f.restype = ctypes.c_float
    th = f(_p(weights), _p(relations), _p(sizes), ctypes.c_int64(0),
           ctypes.c_int64(relations.shape[0]), ctypes.c_int64(budget), ctypes.byref(rem))
    return float(th), int(rem.value)


def group_threshold_brute(weights, relations, sizes, budget):
    """Independent check: expand every eligible group into its edges, sort by
    weight descending, read the budget-th edge."""
    ws = []
    for g in range(len(relations)):
        wv = np.float32(weights[relations[g]])
        if wv > 0:
            ws.extend([wv] * int(sizes[g]))
    if len(ws) <= budget:
        return -1.0, 0
    ws = sorted(ws, reverse=True)
    th = ws[budget - 1]
    higher = sum(1 for x in ws if x > th)
    return float(th), int(budget - higher)


# --------------------------------------------------------------------------
# Dense forward / backward: flashlog.cpp:151-211, :216-278

def _csr_args(csr, masks):
    (ori_rp, ori_col, ori_ri, ori_ord, inv_rp, inv_col, inv_ri, inv_ord,
     ori_gp, ori_gr, ori_gs, ori_gc, inv_gp, inv_gr, inv_gs, inv_gc) = csr
    ori_mask, inv_mask = masks
    return [_c(ori_col, np.int32), ori_mask, _c(ori_gp, np.int32), _c(ori_gr, np.int16),
            _c(ori_gs, np.int32), _c(ori_gc, np.int32),
            _c(inv_col, np.int32), inv_mask, _c(inv_gp, np.int32), _c(inv_gr, np.int16),
            _c(inv_gs, np.int32), _c(inv_gc, np.int32)]


def active_nodes(A):
    """Sorted entities with a nonzero in any row (flashlog_kernel.py:617-623)."""
    A = np.asarray(A)
    return np.nonzero((A != 0).any(axis=0))[0].astype(np.int64)


def dense_forward(A, w, csr, masks, r_size, wot_i=False, topk_edges=1 << 60, active=None):
    A = np.asarray(A)
    dt = np.float64 if A.dtype == np.float64 else np.float32
    suf = "f64" if dt == np.float64 else "f32"
    A = _c(A, dt)
    BL, E = A.shape
    w = _c(w, dt).reshape(BL, -1)
    n = w.shape[1]
    if active is None:
        active = active_nodes(A)
    active = _c(active, np.int64)
    masks = tuple(_c(m, dt) for m in masks)
    args = _csr_args(csr, masks)
    out = [np.empty((BL, E), dt) for _ in range(3)]
    getattr(lib(), "or_dense_forward_" + suf)(
        ctypes.c_int64(BL), ctypes.c_int64(E), ctypes.c_int64(n), _p(A), _p(w), _p(active),
        ctypes.c_int64(active.shape[0]), *[_p(a) for a in args], ctypes.c_int64(r_size),
        ctypes.c_int(int(bool(wot_i))), ctypes.c_int64(int(topk_edges)), *[_p(o) for o in out])
    return tuple(out)


def dense_backward(grad_ind, grad_ori, grad_inv, A, w, csr, masks, r_size, wot_i=False,
                   topk_edges=1 << 60, active=None):
    A = np.asarray(A)
    dt = np.float64 if A.dtype == np.float64 else np.float32
    suf = "f64" if dt == np.float64 else "f32"
    A = _c(A, dt)
    BL, E = A.shape
    w = _c(w, dt).reshape(BL, -1)
    n = w.shape[1]
    if active is None:
        active = active_nodes(A)
    active = _c(active, np.int64)
    grads = [_c(g, dt).reshape(BL, E) for g in (grad_ind, grad_ori, grad_inv)]
    masks = tuple(_c(m, dt) for m in masks)
    args = _csr_args(csr, masks)
    gA = np.empty((BL, E), dt)
    gw = np.empty((BL, n), dt)
    getattr(lib(), "or_dense_backward_" + suf)(
        ctypes.c_int64(BL), ctypes.c_int64(E), ctypes.c_int64(n), *[_p(g) for g in grads],
        _p(A), _p(w), _p(active), ctypes.c_int64(active.shape[0]), *[_p(a) for a in args],
        ctypes.c_int64(r_size), ctypes.c_int(int(bool(wot_i))), ctypes.c_int64(int(topk_edges)),
        _p(gA), _p(gw))
    return gA, gw


def dense_max_forward(A, w, csr, masks, r_size, wot_i=False, topk_edges=1 << 60, active=None):
    A = _c(A, np.float32)
    BL, E = A.shape
    w = _c(w, np.float32).reshape(BL, -1)
    n = w.shape[1]
    if active is None:
        active = active_nodes(A)
    active = _c(active, np.int64)
    masks = tuple(_c(m, np.float32) for m in masks)
    args = _csr_args(csr, masks)
    out = [np.empty((BL, E), np.float32) for _ in range(3)]
    args_out = [np.empty((BL, E), np.int64) for _ in range(2)]
    lib().or_dense_max_forward(
        ctypes.c_int64(BL), ctypes.c_int64(E), ctypes.c_int64(n), _p(A), _p(w), _p(active),
        ctypes.c_int64(active.shape[0]), *[_p(a) for a in args], ctypes.c_int64(r_size),
        ctypes.c_int(int(bool(wot_i))), ctypes.c_int64(int(topk_edges)),
        *[_p(o) for o in out], *[_p(o) for o in args_out])
    return (*out, *args_out)


def dense_max_backward(grad_ind, grad_ori, grad_inv, arg_ori, arg_inv, A, w, csr, masks, r_size, wot_i=False,
                       topk_edges=1 << 60, active=None):
    A = _c(A, np.float32)
    BL, E = A.shape
    w = _c(w, np.float32).reshape(BL, -1)
    n = w.shape[1]
    if active is None:
        active = active_nodes(A)
    active = _c(active, np.int64)
    masks = tuple(_c(m, np.float32) for m in masks)
    args = _csr_args(csr, masks)
    g = [_c(x, np.float32).reshape(BL, E) for x in (grad_ind, grad_ori, grad_inv)]
    arg = [_c(x, np.int64).reshape(BL, E) for x in (arg_ori, arg_inv)]
    gA = np.empty((BL, E), np.float32)
    gw = np.empty((BL, n), np.float32)
    lib().or_dense_max_backward(
        ctypes.c_int64(BL), ctypes.c_int64(E), ctypes.c_int64(n), _p(A), _p(w), *[_p(x) for x in g],
        *[_p(x) for x in arg], _p(active), ctypes.c_int64(active.shape[0]), *[_p(a) for a in args],
        ctypes.c_int64(r_size), ctypes.c_int(int(bool(wot_i))), ctypes.c_int64(int(topk_edges)), _p(gA), _p(gw))
    return gA, gw


# --------------------------------------------------------------------------
# c1 entity budget: flashlog_kernel.py:814-842

def dense_topc(A, c):
    """Returns (A_pruned, cutoff[BL], last_tie[BL], changed)."""
    A = _c(A, np.float32)
    BL, E = A.shape
    out = np.empty_like(A)
    cutoff = np.zeros(BL, np.float32)
    last = np.zeros(BL, np.int32)
    changed = ctypes.c_int(0)
    rc = lib().or_dense_topc(ctypes.c_int64(BL), ctypes.c_int64(E), ctypes.c_int64(c), _p(A),
                             _p(out), _p(cutoff), _p(last), ctypes.byref(changed))
    if rc != 0:
        raise ValueError("topk_nodes/c must be nonnegative")
    return out, cutoff, last, bool(changed.value)


def dense_topc_brute(A, c):
    """Independent check of the c1 keep set: stable sort of the nonzeros of
    each over-budget row by (value desc, entity asc), keep the first c."""
    A = np.asarray(A, np.float32)
    keep = np.ones(A.shape, bool)
    for r in range(A.shape[0]):
        nz = np.nonzero(A[r] != 0)[0]
        if nz.size <= c:
            continue
        order = sorted(nz.tolist(), key=lambda e: (-float(A[r, e]), e))
        keep[r] = False
        keep[r, order[:c]] = True
    return keep


# --------------------------------------------------------------------------
# Filtered ranks: flashlog.cu:2754-2910

def filtered_ranks(idx_b, idx_e, values, targets, filter_keys, B, E, use_eql=False):
    idx_b = _c(idx_b, np.int64)
    idx_e = _c(idx_e, np.int64)
    f64 = np.asarray(values).dtype == np.float64
    values = _c(values, np.float64 if f64 else np.float32)
    targets = _c(targets, np.int64)
    filter_keys = np.sort(_c(filter_keys, np.int64))
    ranks = np.empty(B, np.float32)
    fn = lib().or_filtered_ranks_f64 if f64 else lib().or_filtered_ranks
    fn(ctypes.c_int64(values.shape[0]), _p(idx_b), _p(idx_e), _p(values),
                            ctypes.c_int64(B), ctypes.c_int64(E), _p(targets),
                            ctypes.c_int64(filter_keys.shape[0]), _p(filter_keys),
                            ctypes.c_int(int(bool(use_eql))), _p(ranks))
    return ranks


def filtered_ranks_brute(dense_scores, targets, filter_mask, use_eql=False):
    """Independent check on a dense [B, E] score matrix: count unfiltered
    entities scoring above / equal to the target (the target itself is not
    counted unless it is unfiltered, in which case it is one of the ties)."""
    S = np.asarray(dense_scores)
    if S.dtype != np.float64:
        S = S.astype(np.float32)
    B, E = S.shape
    ranks = np.empty(B, np.float64)
    for b in range(B):
        t = S[b, targets[b]]
        unf = ~filter_mask[b]
        greater = int(np.sum(S[b][unf] > t))
        eq = int(np.sum(S[b][unf] == t)) + 1
        ranks[b] = greater + (eq + 1) / 2.0 if use_eql else greater + 1
    return ranks


# --------------------------------------------------------------------------
# Sparse (COO) hop: flashlog.cpp:1388-1486 (mode 0, top-k / CPU order) and the
# all-edges coordinates of flashlog.cu:1743-1854 (mode 1)

SPARSE_TOPK, SPARSE_ALL = 0, 1


def _sparse_args(b, l, e, v):
    return (_c(b, np.int64), _c(l, np.int64), _c(e, np.int64), _c(v, np.float32))


def _sparse_cap(e, csr, nnz):
    gc = [np.asarray(csr[11]), np.asarray(csr[15])]
    gp = [np.asarray(csr[8]), np.asarray(csr[12])]
    e = np.asarray(e, np.int64)
    cap = nnz
    for side in range(2):
        deg = np.zeros(gp[side].shape[0] - 1, np.int64)
        csum = np.concatenate([[0], np.cumsum(gc[side].astype(np.int64))])
        deg = csum[gp[side][1:]] - csum[gp[side][:-1]]
        cap += int(deg[e].sum()) if e.size else 0
    return max(cap, 1)


def sparse_forward(mode, b, l, e, v, B, L, E, w, csr, masks, r_size, wot_i=False, topk_edges=1 << 60, seed=-1):
    """Returns (keys, values): keys = (b*L + l)*E + e ascending.  seed >= 0:
    the training quotas (flashlog.cu:1433-1528) instead of the threshold."""
    b, l, e, v = _sparse_args(b, l, e, v)
    w = _c(w, np.float32).reshape(B * L, -1)
    n = w.shape[1]
    masks = tuple(_c(m, np.float32) for m in masks)
    args = _csr_args(csr, masks)
    cap = _sparse_cap(e, csr, v.shape[0])
    keys = np.empty(cap, np.int64)
    vals = np.empty(cap, np.float32)
    fn = lib().or_sparse_forward
    fn.restype = ctypes.c_int64
    cnt = fn(ctypes.c_int(mode), ctypes.c_int64(v.shape[0]), _p(b), _p(l), _p(e), _p(v), ctypes.c_int64(B),
             ctypes.c_int64(L), ctypes.c_int64(E), _p(w), ctypes.c_int64(n), *[_p(a) for a in args],
             ctypes.c_int64(r_size), ctypes.c_int(int(bool(wot_i))), ctypes.c_int64(int(topk_edges)),
             ctypes.c_int64(int(seed)), ctypes.c_int64(cap), _p(keys), _p(vals))
    assert cnt >= 0
    return keys[:cnt].copy(), vals[:cnt].copy()


def sparse_backward(mode, b, l, e, v, B, L, E, w, csr, masks, r_size, out_keys, grad_out, wot_i=False,
                    topk_edges=1 << 60, seed=-1):
    b, l, e, v = _sparse_args(b, l, e, v)
    w = _c(w, np.float32).reshape(B * L, -1)
    n = w.shape[1]
    masks = tuple(_c(m, np.float32) for m in masks)
    args = _csr_args(csr, masks)
    out_keys = _c(out_keys, np.int64)
    grad_out = _c(grad_out, np.float32)
    gv = np.empty(v.shape[0], np.float32)
    gw = np.empty((B * L, n), np.float32)
    lib().or_sparse_backward(ctypes.c_int(mode), ctypes.c_int64(v.shape[0]), _p(b), _p(l), _p(e), _p(v),
                             ctypes.c_int64(B), ctypes.c_int64(L), ctypes.c_int64(E), _p(w), ctypes.c_int64(n),
                             *[_p(a) for a in args], ctypes.c_int64(r_size), ctypes.c_int(int(bool(wot_i))),
                             ctypes.c_int64(int(topk_edges)), ctypes.c_int64(int(seed)), _p(out_keys),
                             ctypes.c_int64(out_keys.shape[0]), _p(grad_out), _p(gv), _p(gw))
    return gv, gw


def sparse_max_forward(b, l, e, v, B, L, E, w, csr, masks, r_size, wot_i=False, topk_edges=1 << 60, seed=-1):
    """Sparse max hop (flashlog_kernel.py:399-478,1450-1626).  Returns
    (keys, values, win_entry, win_dir, win_pos): the winner of every output
    (entry index, 0 ORI / 1 INV / 2 identity, CSR position or -1)."""
    b, l, e, v = _sparse_args(b, l, e, v)
    w = _c(w, np.float32).reshape(B * L, -1)
    n = w.shape[1]
    masks = tuple(_c(m, np.float32) for m in masks)
    args = _csr_args(csr, masks)
    orders = [_c(csr[3], np.int32), _c(csr[7], np.int32)]
    cap = _sparse_cap(e, csr, v.shape[0])
    keys = np.empty(cap, np.int64)
    vals = np.empty(cap, np.float32)
    went = np.empty(cap, np.int64)
    wdir = np.empty(cap, np.int32)
    wpos = np.empty(cap, np.int64)
    fn = lib().or_sparse_max_forward
    fn.restype = ctypes.c_int64
    cnt = fn(ctypes.c_int64(v.shape[0]), _p(b), _p(l), _p(e), _p(v), ctypes.c_int64(B), ctypes.c_int64(L),
             ctypes.c_int64(E), _p(w), ctypes.c_int64(n), *[_p(a) for a in args], *[_p(a) for a in orders],
             ctypes.c_int64(r_size), ctypes.c_int(int(bool(wot_i))), ctypes.c_int64(int(topk_edges)),
             ctypes.c_int64(int(seed)), ctypes.c_int64(cap), _p(keys), _p(vals), _p(went), _p(wdir), _p(wpos))
    assert cnt >= 0
    return keys[:cnt].copy(), vals[:cnt].copy(), went[:cnt].copy(), wdir[:cnt].copy(), wpos[:cnt].copy()


def sparse_max_backward(b, l, v, B, L, w, csr, masks, r_size, grad_out, win_entry, win_dir, win_pos):
    """Gradient of the sparse max through the forward's winners
    (flashlog.cu:2364-2410).  Returns (grad_v, grad_w [B*L, n])."""
    b, l, _, v = _sparse_args(b, l, b, v)
    w = _c(w, np.float32).reshape(B * L, -1)
    n = w.shape[1]
    om, im = (_c(m, np.float32) for m in masks)
    orel = _c(np.asarray(csr[2]), np.int16)
    irel = _c(np.asarray(csr[6]), np.int16)
    grad_out = _c(grad_out, np.float32)
    went, wdir, wpos = _c(win_entry, np.int64), _c(win_dir, np.int32), _c(win_pos, np.int64)
    gv = np.empty(max(v.shape[0], 1), np.float32)
    gw = np.empty((B * L, n), np.float32)
    lib().or_sparse_max_backward(ctypes.c_int64(v.shape[0]), _p(b), _p(l), _p(v), ctypes.c_int64(B),
                                 ctypes.c_int64(L), _p(w), ctypes.c_int64(n), _p(om), _p(orel), _p(im), _p(irel),
                                 ctypes.c_int64(r_size), ctypes.c_int64(grad_out.shape[0]), _p(grad_out), _p(went),
                                 _p(wdir), _p(wpos), _p(gv), _p(gw))
    return gv[:v.shape[0]], gw


def splitmix64(state):
    """One SplitMix64 output from state (uint64)."""
    fn = lib().or_splitmix64
    fn.restype = ctypes.c_uint64
    return int(fn(ctypes.c_uint64(state & 0xFFFFFFFFFFFFFFFF)))


def quota_takes(weights, counts, topk_edges, b, l, src, is_inv, seed):
    """Training quotas of one (entry, side) (flashlog.cu:1433-1528)."""
    weights = _c(weights, np.float32)
    counts = _c(counts, np.int32)
    takes = np.empty(max(weights.shape[0], 1), np.int32)
    lib().or_quota_takes(ctypes.c_int64(weights.shape[0]), _p(weights), _p(counts), ctypes.c_int64(int(topk_edges)),
                         ctypes.c_int64(int(b)), ctypes.c_int64(int(l)), ctypes.c_int64(int(src)),
                         ctypes.c_int(int(is_inv)), ctypes.c_int64(int(seed)), _p(takes))
    return takes[:weights.shape[0]]


def quota_phase(b, l, src, is_inv, seed):
    """The SplitMix64 rounding phase in [0, 1) of one (b, l, source, side)."""
    m = 0xFFFFFFFFFFFFFFFF
    z = (int(seed) & m) ^ ((int(b) * 0x9e3779b97f4a7c15) & m) ^ ((int(l) * 0xbf58476d1ce4e5b9) & m) ^ \
        ((int(src) * 0x94d049bb133111eb) & m) ^ (0xd1b54a32d192ed03 if is_inv else 0x8cb92baa3f3d8dd7)
    return (splitmix64(z) >> 11) * 2.0 ** -53


def quota_closed_form(weights, counts, topk_edges, phase):
    """Independent check of quota_takes: the reference's own CPU quota rule
    (flashlog_kernel.py:1978-2003: weighted floors, then differences of the
    rounded residual-capacity prefix, the last one pinned to the residual)
    with the same phase.  Agrees with the sequential rule except at
    floating-point boundaries."""
    w = np.asarray(weights, np.float32).astype(np.float64)
    c = np.asarray(counts, np.int64) * (w > 0)
    cap = int(c.sum())
    target = min(cap, int(topk_edges))
    if target == cap:
        return c
    wsum = 0.0
    for x in w[c > 0]:
        wsum += float(x)
    base = np.where(c > 0, np.minimum(c, np.floor(target * w / wsum)), 0).astype(np.int64)
    spare = c - base
    residual = target - int(base.sum())
    cumulative = np.floor(residual * np.cumsum(spare).astype(np.float64) / int(spare.sum()) + phase).astype(np.int64)
    cumulative[-1] = residual
    return base + np.diff(cumulative, prepend=0)


def sparse_normalize(b, l, v, B, L, eps=1e-7):
    b, l, _, v = _sparse_args(b, l, b, v)
    out = np.empty(v.shape[0], np.float32)
    denom = np.empty(B * L, np.float32)
    lib().or_sparse_normalize(ctypes.c_int64(v.shape[0]), _p(b), _p(l), _p(v), ctypes.c_int64(B),
                              ctypes.c_int64(L), ctypes.c_float(eps), _p(out), _p(denom))
    return out, denom


def sum_sp_3d(b, l, e, v, B, L, E):
    """Channel sum of a coalesced [B, L, E] state (src/model_DRUM_kernel_sp.py:
    22-28): torch's coalesce of the (b, e) re-index, whose stable sort keeps
    each key's entries in channel order, adds them from 0 in that order.
    Returns (out_b, out_e, out_v, slot), slot[i] the output of entry i.
    Pinned in tests/test_oracle_sparse.py by brute-force sums and torch's CPU
    coalesce on dyadic values (exact in any order) and by a case whose
    rounding depends on the channel order."""
    b, l, e = (np.asarray(x, np.int64) for x in (b, l, e))
    v = np.asarray(v, np.float32)
    n = v.shape[0]
    key = b * E + e
    order = np.argsort(key, kind="stable")
    ks, vs = key[order], v[order]
    head = np.ones(n, bool)
    head[1:] = ks[1:] != ks[:-1]
    gid = np.cumsum(head) - 1
    start = np.flatnonzero(head)
    out = np.zeros(start.shape[0], np.float32)
    rank = np.arange(n) - start[gid] if n else np.zeros(0, np.int64)
    for k in range(int(rank.max()) + 1 if n else 0):
        sel = rank == k
        out[gid[sel]] = out[gid[sel]] + vs[sel]
    slot = np.empty(n, np.int64)
    slot[order] = gid
    return ks[start] // E, ks[start] % E, out, slot


def sparse_topc(b, l, v, L, c):
    """Kept entry indices of the c1 budget on a coalesced COO state
    (flashlog_kernel.py:1092-1140): per (b, l) row with more than c nonzeros,
    its c largest nonzeros (ties to the earlier entry); other rows keep all."""
    b = np.asarray(b, np.int64)
    l = np.asarray(l, np.int64)
    v = np.asarray(v, np.float32)
    row = b * L + l
    keep = np.ones(v.shape[0], bool)
    for r in np.unique(row):
        idx = np.nonzero(row == r)[0]
        nz = idx[v[idx] != 0]
        if nz.size <= c:
            continue
        keep[idx] = False
        if c == 0:
            continue
        order = nz[np.lexsort((np.arange(nz.size), -v[nz].astype(np.float64)))]
        keep[order[:c]] = True
    return np.nonzero(keep)[0]


def sparse_topc_race_candidates(b, l, v, L, c):
    """Entry indices of the sampled c1's candidates (nonzero entries of rows
    with more than c nonzeros), in entry order: one noise draw each."""
    row = np.asarray(b, np.int64) * L + np.asarray(l, np.int64)
    v = np.asarray(v, np.float32)
    cand = []
    for r in np.unique(row):
        idx = np.nonzero(row == r)[0]
        nz = idx[v[idx] != 0]
        if nz.size > c:
            cand.append(nz)
    return np.sort(np.concatenate(cand)) if cand else np.zeros(0, np.int64)


def sparse_topc_race(b, l, v, L, c, noise):
    """Sampled c1 (flashlog_kernel.py:1121-1132, sampling=True): in rows with
    more than c nonzeros keep the c candidates with the largest
    log(v) - log(noise) (float64; ties to the earlier entry), noise[k] for
    the k-th candidate in entry order; other rows keep every entry."""
    row = np.asarray(b, np.int64) * L + np.asarray(l, np.int64)
    v = np.asarray(v, np.float32)
    cand = sparse_topc_race_candidates(b, l, v, L, c)
    noise = np.asarray(noise, np.float64)
    assert noise.shape[0] == cand.shape[0]
    keep = np.ones(v.shape[0], bool)
    score = np.full(v.shape[0], -np.inf)
    score[cand] = np.log(v[cand].astype(np.float64)) - np.log(noise)
    is_cand = np.zeros(v.shape[0], bool)
    is_cand[cand] = True
    for r in np.unique(row[cand]):
        idx = np.nonzero(row == r)[0]
        keep[idx] = False
        ci = idx[is_cand[idx]]
        order = ci[np.lexsort((np.arange(ci.size), -score[ci]))]
        keep[order[:c]] = True
    return np.nonzero(keep)[0]


# --------------------------------------------------------------------------
# Rule-bank scoring: rules/shared_inference.py:12-245 and the fixed-relation
# step flashlog.cu:1561-1741 (float64, from the raw triples)

def _op_matrix(h, r, t, E, R, op):
    """Operator op as an E x E path-count matrix: op < R the relation,
    R <= op < 2R its inverse, op == 2R the identity."""
    import scipy.sparse as sp
    if op == 2 * R:
        return sp.identity(E, format="csr", dtype=np.float64)
    rel = op if op < R else op - R
    sel = np.asarray(r) == rel
    src, dst = (np.asarray(h)[sel], np.asarray(t)[sel]) if op < R else (np.asarray(t)[sel], np.asarray(h)[sel])
    return sp.csr_matrix((np.ones(src.shape[0]), (src, dst)), shape=(E, E))


def fixed_relation_step(b, l, e, v, ops, h, r, t, E, R):
    """{(b, l, e'): value}: every entry follows its row's operator through
    every matching triple, values summed per endpoint."""
    out = {}
    h, r, t = (np.asarray(x) for x in (h, r, t))
    for bi, li, ei, vi in zip(np.asarray(b), np.asarray(l), np.asarray(e), np.asarray(v, np.float64)):
        op = int(ops[bi][li])
        if op == 2 * R:
            dsts = [ei]
        elif 0 <= op < R:
            dsts = t[(h == ei) & (r == op)]
        elif R <= op < 2 * R:
            dsts = h[(t == ei) & (r == op - R)]
        else:
            dsts = []
        for d in dsts:
            key = (int(bi), int(li), int(d))
            out[key] = out.get(key, 0.0) + float(vi)
    return out


def rule_path_counts(h, r, t, E, R, sources, bodies, boolean_paths=False):
    """Per rule body, the path counts of every source as a sparse [E, B]
    float64 matrix (column b: e_{s_b}^T M_op1 M_op2 ...; Boolean after every
    step when boolean_paths)."""
    import scipy.sparse as sp
    mats = {}
    B = len(sources)
    start = sp.csc_matrix((np.ones(B), (np.asarray(sources, np.int64), np.arange(B))), shape=(E, B))
    out = []
    for body in bodies:
        x = start
        for op in body:
            if op not in mats:
                mats[op] = _op_matrix(h, r, t, E, R, op).T.tocsr()
            x = (mats[op] @ x).tocsc()
            if boolean_paths:
                x.data = (x.data > 0).astype(np.float64)
                x.eliminate_zeros()
        out.append(x.tocoo())
    return out


def rule_scores(h, r, t, E, R, sources, bodies, W, reduction="sum", boolean_paths=False, final_max=False):
    """Dense [B, E] float64 scores: per rule the path-count vectors of every
    source (rule_path_counts; Boolean when boolean_paths or max), per rank the
    weighted sum (or max) over rules, each (rank, source) row divided by
    max(its sum, 1e-30), ranks summed (or maxed)."""
    boolean_paths = boolean_paths or reduction == "max"
    W = np.asarray(W, np.float64)
    B, K = len(sources), W.shape[1]
    S = np.zeros((K, E, B))
    for ri, x in enumerate(rule_path_counts(h, r, t, E, R, sources, bodies, boolean_paths)):
        for k in range(K):
            if reduction == "max":
                np.maximum.at(S[k], (x.row, x.col), W[ri, k] * (x.data > 0))
            else:
                np.add.at(S[k], (x.row, x.col), W[ri, k] * x.data)
    total = np.zeros((B, E))
    for k in range(K):
        Sk = S[k].T
        d = np.maximum(Sk.sum(1, keepdims=True), 1e-30)
        part = Sk / d
        total = np.maximum(total, part) if final_max else total + part
    return total


def rule_batch_scores(h, r, t, E, R, sources, rules, aggregation):
    """The DRUM scorer's aggregations (rules/evaluate.py:554-734) as dense
    [B, E] float64 arrays plus the Boolean set of reached (source, entity)
    pairs: weighted_path_count / weighted_boolean (sum_r w_r C_r or
    [C_r > 0]), max_confidence (max_r w_r over C_r > 0), rank_normalized /
    rank_boolean_normalized (per rank the positive terms rw_r[k] C_r, rows
    normalized, ranks summed), routed_normalized (the same over the routed
    groups with w_r)."""
    boolean = aggregation in ("weighted_boolean", "rank_boolean_normalized", "max_confidence")
    B = len(sources)
    counts = rule_path_counts(h, r, t, E, R, sources, [list(x["body"]) for x in rules], boolean)
    reached = np.zeros((B, E), bool)
    for x in counts:
        reached[x.col, x.row] = True
    if aggregation in ("weighted_path_count", "weighted_boolean", "max_confidence"):
        S = np.full((B, E), -np.inf) if aggregation == "max_confidence" else np.zeros((B, E))
        for rule, x in zip(rules, counts):
            w = float(rule["weight"])
            if aggregation == "max_confidence":
                np.maximum.at(S, (x.col, x.row), w * (x.data > 0))
            else:
                np.add.at(S, (x.col, x.row), w * x.data)
        return np.where(reached, S, 0.0), reached
    if aggregation == "routed_normalized":
        G = 1 + max(x["group_id"] for x in rules)
        chan = np.zeros((len(rules), G))
        for i, rule in enumerate(rules):
            chan[i, rule["group_id"]] = max(float(rule["weight"]), 0.0)
    else:
        chan = np.maximum(np.asarray([x["rank_weights"] for x in rules], np.float64), 0.0)
    S = np.zeros((chan.shape[1], B, E))
    for i, x in enumerate(counts):
        for k in range(chan.shape[1]):
            np.add.at(S[k], (x.col, x.row), chan[i, k] * x.data)
    total = np.zeros((B, E))
    for k in range(chan.shape[1]):
        total += S[k] / np.maximum(S[k].sum(1, keepdims=True), 1e-30)
    return total, total > 0


def rule_paths_brute(h, r, t, R, source, body):
    """Path counts by explicit enumeration of the edge sequences (tiny graphs)."""
    h, r, t = (list(map(int, x)) for x in (h, r, t))
    ends = {source: 1}
    for op in body:
        nxt = {}
        for node, cnt in ends.items():
            if op == 2 * R:
                nxt[node] = nxt.get(node, 0) + cnt
                continue
            for hh, rr, tt in zip(h, r, t):
                if op < R and rr == op and hh == node:
                    nxt[tt] = nxt.get(tt, 0) + cnt
                elif R <= op < 2 * R and rr == op - R and tt == node:
                    nxt[hh] = nxt.get(hh, 0) + cnt
        ends = nxt
    return ends


# --------------------------------------------------------------------------
# Soft grounding (flashlog_kernel/soft_grounding_kernel/source/
# soft_grounding.cpp): reservoir, walks (C, grounding_oracle.c), and the
# count merge / cap / fold union (numpy, :454-614)

def mt64_nth(seed, k):
    """k-th output of std::mt19937_64 seeded with seed."""
    fn = lib().or_mt64_nth
    fn.restype = ctypes.c_uint64
    return int(fn(ctypes.c_uint64(seed), ctypes.c_int64(k)))


def reservoir(row_group_ptr, group_rel, relations, max_sources, seed):
    """sample_relation_sources_reservoir (soft_grounding.cpp:1029-1124)."""
    gp = _c(row_group_ptr, np.int32)
    gr = _c(group_rel, np.int16)
    rel = _c(relations, np.int64)
    out = np.empty((rel.shape[0], max_sources), np.int32)
    avail = np.empty(rel.shape[0], np.int64)
    rc = lib().or_reservoir(ctypes.c_int64(gp.shape[0] - 1), _p(gp), _p(gr), ctypes.c_int64(rel.shape[0]), _p(rel),
                            ctypes.c_int64(max_sources), ctypes.c_int64(seed), _p(out), _p(avail))
    if rc != 0:
        raise ValueError("relation ids must be unique and in [0, 32767]")
    return out, avail


def ground_walks(att, R, head, task_source, task_index, csr, walks, topk_edges, mask_query_head, seed,
                 temperature=1.0):
    """Walk records of every source task: (keys [tasks, walks] uint64,
    positive [tasks, walks] uint8); att [3, ranks, 2R+1]."""
    att = _c(att, np.float32)
    steps, ranks, vocab = att.shape
    assert steps == 3 and vocab == 2 * R + 1
    ts = _c(task_source, np.int64)
    ti = _c(task_index, np.int64)
    arrs = [_c(csr[1], np.int32), _c(csr[5], np.int32), _c(csr[8], np.int32), _c(csr[9], np.int16),
            _c(csr[10], np.int32), _c(csr[11], np.int32), _c(csr[12], np.int32), _c(csr[13], np.int16),
            _c(csr[14], np.int32), _c(csr[15], np.int32)]
    gp = [np.asarray(csr[8]), np.asarray(csr[12])]
    max_groups = max(int(np.max(np.diff(g))) if g.shape[0] > 1 else 0 for g in gp) + 1
    keys = np.empty((ts.shape[0], walks), np.uint64)
    pos = np.empty((ts.shape[0], walks), np.uint8)
    lib().or_ground_walks(_p(att), ctypes.c_int64(ranks), ctypes.c_int64(vocab), ctypes.c_int64(R),
                          ctypes.c_int32(head), ctypes.c_int64(ts.shape[0]), _p(ts), _p(ti), *[_p(a) for a in arrs],
                          ctypes.c_int64(walks), ctypes.c_int64(topk_edges), ctypes.c_int(int(bool(mask_query_head))),
                          ctypes.c_int64(seed), ctypes.c_double(temperature), ctypes.c_int64(max_groups), _p(keys),
                          _p(pos))
    return keys, pos


def _encode(length, body):
    m = (1 << 20) - 1
    return (length << 60) | ((body[0] & m) << 40) | ((body[1] & m) << 20) | (body[2] & m)


def ground_aggregate(keys, pos, task_fold, nfolds, head, budgets):
    """Per fold the body counts (walk hits, source hits, positive walk hits,
    positive source hits; soft_grounding.cpp:427-449), capped per length by
    (walk hits desc, key asc) (:454-531), then united over folds with totals
    and per-fold minimums, the trivial body (head) dropped, ascending key
    (:533-614).  Returns (rows int64 [n, 12], raw unique counts per fold)."""
    capped, raw = [], []
    for f in range(nfolds):
        stats = {}
        for t in np.nonzero(np.asarray(task_fold) == f)[0]:
            local = {}
            for k, p in zip(keys[t].tolist(), pos[t].tolist()):
                if k == 0:
                    continue
                c = local.setdefault(k, [0, 0])
                c[0] += 1
                c[1] += p
            for k, (wh, pw) in local.items():
                s = stats.setdefault(k, [0, 0, 0, 0])
                s[0] += wh
                s[1] += 1
                s[2] += pw
                s[3] += 1 if pw > 0 else 0
        raw.append(len(stats))
        rows = []
        for length in (1, 2, 3):
            b = budgets[length - 1]
            if b <= 0:
                continue
            cand = sorted(((k, v) for k, v in stats.items() if k >> 60 == length), key=lambda kv: (-kv[1][0], kv[0]))
            rows += cand[:b]
        capped.append(rows)
    trivial = _encode(1, (head, 0, 0))
    agg = {}
    for rows in capped:
        for k, v in rows:
            if k == trivial:
                continue
            if k not in agg:
                agg[k] = [list(v), list(v), 1]
            else:
                a = agg[k]
                a[0] = [x + y for x, y in zip(a[0], v)]
                a[1] = [min(x, y) for x, y in zip(a[1], v)]
                a[2] += 1
    out = np.zeros((len(agg), 12), np.int64)
    m = (1 << 20) - 1
    for i, k in enumerate(sorted(agg)):
        tot, mn, seen = agg[k]
        if seen != nfolds:
            mn = [0, 0, 0, 0]
        out[i, :4] = [k >> 60, (k >> 40) & m, (k >> 20) & m, k & m]
        out[i, 4:8] = tot
        out[i, 8:12] = mn
    return out, raw


def ground(att, R, head, folds, csr, walks, topk_edges, mask_query_head, seed, budgets, temperature=1.0):
    """One head of ground_head_batch_source_folds_sampled_capped_counts:
    folds = list of source arrays.  Returns (rows, raw counts per fold)."""
    src = np.concatenate([np.asarray(f, np.int64) for f in folds]) if folds else np.zeros(0, np.int64)
    idx = np.concatenate([np.arange(len(f), dtype=np.int64) for f in folds]) if folds else src
    fold = np.concatenate([np.full(len(f), i, np.int64) for i, f in enumerate(folds)]) if folds else src
    keys, pos = ground_walks(att, R, head, src, idx, csr, walks, topk_edges, mask_query_head, seed, temperature)
    return ground_aggregate(keys, pos, fold, len(folds), head, budgets)


def dense_filtered_ranks(state, targets, filter_b=None, filter_e=None, use_eql=False):
    """Ranks of calculate_hits_full_with_filter_indices (src/main.py:468-512)
    in its float32 arithmetic: greater / equal over the row, minus the
    filtered entities' (the filter with the targets appended, unique keys)."""
    state = np.asarray(state, np.float32)
    B, E = state.shape
    targets = np.asarray(targets, np.int64)
    truth = state[np.arange(B), targets]
    greater = (state > truth[:, None]).sum(1).astype(np.float32)
    equal = (state == truth[:, None]).sum(1).astype(np.float32)
    if filter_b is not None:
        keys = np.unique(np.concatenate([np.asarray(filter_b, np.int64) * E + np.asarray(filter_e, np.int64),
                                         np.arange(B) * E + targets]))
        fb, fe = keys // E, keys % E
        fs = state[fb, fe]
        fg = np.zeros(B, np.float32)
        fq = np.zeros(B, np.float32)
        np.add.at(fg, fb, (fs > truth[fb]).astype(np.float32))
        np.add.at(fq, fb, (fs == truth[fb]).astype(np.float32))
        greater = (greater - fg).astype(np.float32)
        equal = (equal - fq).astype(np.float32)
    if use_eql:
        equal = (equal + np.float32(1)).astype(np.float32)
        return (greater + (equal + np.float32(1)) / np.float32(2)).astype(np.float32)
    return (greater + np.float32(1)).astype(np.float32)


# --------------------------------------------------------------------------
# Known-answer ("filter") indices of the evaluation (src/main.py:147-317)

def filter_edge_lookup(source, relation, target, R):
    """_build_filter_edge_lookup (src/main.py:147-161): (group keys ascending,
    starts, counts, columns) with key = source * R + relation; equal keys
    keep edge order (a stable sort; the reference's argsort leaves that
    order open)."""
    keys = np.asarray(source, np.int64) * R + np.asarray(relation, np.int64)
    order = np.argsort(keys, kind="stable")
    sk = keys[order]
    cols = np.asarray(target, np.int64)[order]
    if sk.size == 0:
        e = np.zeros(0, np.int64)
        return e, e, e, cols
    starts = np.flatnonzero(np.r_[True, sk[1:] != sk[:-1]])
    counts = np.diff(np.r_[starts, sk.size])
    return sk[starts], starts, counts, cols


def filter_side_lookup(row_group_ptr, group_rel, group_start, group_count, col_ind, R):
    """_build_filter_side_lookup (src/main.py:181-200): a CSR side's groups
    keyed by source * R + relation (the source of group g is the row whose
    group range holds g)."""
    gp = np.asarray(row_group_ptr, np.int64)
    G = np.asarray(group_rel).size
    if G == 0:
        e = np.zeros(0, np.int64)
        return e, e, e, np.asarray(col_ind, np.int64)
    src = np.searchsorted(gp, np.arange(G), side="right") - 1
    return (src * R + np.asarray(group_rel, np.int64), np.asarray(group_start, np.int64),
            np.asarray(group_count, np.int64), np.asarray(col_ind, np.int64))


def expand_filter_side(batch_pos, query_key, lookup):
    """_expand_filter_side (src/main.py:227-267): every known answer of each
    query key, queries in order, a group's columns in order."""
    gk, starts, counts, cols = lookup
    qk = np.asarray(query_key, np.int64)
    bp = np.asarray(batch_pos, np.int64)
    if qk.size == 0 or gk.size == 0:
        e = np.zeros(0, np.int64)
        return e, e
    pos = np.searchsorted(gk, qk)
    safe = np.minimum(pos, gk.size - 1)
    ok = (pos < gk.size) & (gk[safe] == qk)
    st, ct, b = starts[safe[ok]], counts[safe[ok]], bp[ok]
    out_b = np.repeat(b, ct)
    local = np.arange(out_b.size) - np.repeat(np.cumsum(ct) - ct, ct)
    return out_b, cols[np.repeat(st, ct) + local]


def filter_indices(input_x, input_r, R, lookup):
    """_filter_indices_from_lookup (src/main.py:291-317): forward queries
    (r < R) on the forward lookup, then inverse queries (key with r - R) on
    the inverse lookup."""
    x = np.asarray(input_x, np.int64).reshape(-1)
    r = np.asarray(input_r, np.int64).reshape(-1)
    pos = np.arange(x.size)
    fwd = r < R
    ob, oe = expand_filter_side(pos[fwd], x[fwd] * R + r[fwd], lookup[0])
    ib, ie = expand_filter_side(pos[~fwd], x[~fwd] * R + (r[~fwd] - R), lookup[1])
    return np.concatenate([ob, ib]), np.concatenate([oe, ie])


def filter_indices_brute(h, r, t, R, input_x, input_r):
    """Independent check: per query in batch order, a scan of every triple
    (forward: tails of (x, r); inverse: heads of tail x under r - R); the
    forward queries' pairs first, then the inverse queries'."""
    h, r, t = (np.asarray(a, np.int64) for a in (h, r, t))
    fwd_pairs, inv_pairs = [], []
    for j, (x, q) in enumerate(zip(np.asarray(input_x).tolist(), np.asarray(input_r).tolist())):
        if q < R:
            fwd_pairs += [(j, int(t[i])) for i in range(h.size) if h[i] == x and r[i] == q]
        else:
            inv_pairs += [(j, int(h[i])) for i in range(h.size) if t[i] == x and r[i] == q - R]
    pairs = fwd_pairs + inv_pairs
    return (np.array([p[0] for p in pairs], np.int64), np.array([p[1] for p in pairs], np.int64))


def raw_sparse_ranks(b, e, v, B, E, targets):
    """Ranks of calculate_raw_hits_sparse (src/main.py:365-388) over a
    coalesced [B, E] COO state: #entries >= the target's score, plus the
    implicit zeros when that score is <= 0, in the values' dtype."""
    b = np.asarray(b, np.int64)
    e = np.asarray(e, np.int64)
    v = np.asarray(v)
    dt = v.dtype
    truth = np.zeros(B, dt)
    keys = b * E + e
    tk = np.arange(B) * E + np.asarray(targets, np.int64)
    pos = np.searchsorted(keys, tk)
    safe = np.minimum(pos, max(keys.size - 1, 0))
    ok = (pos < keys.size) & (keys[safe] == tk) if keys.size else np.zeros(B, bool)
    truth[ok] = v[safe[ok]]
    explicit = np.zeros(B, dt)
    ge = np.zeros(B, dt)
    np.add.at(explicit, b, np.ones_like(v))
    np.add.at(ge, b, (v >= truth[b]).astype(dt))
    missing = (dt.type(E) - explicit).astype(dt)
    return (ge + np.where(truth <= 0, missing, np.zeros_like(missing))).astype(dt)


# --------------------------------------------------------------------------
# Extraction post-processing (rules/extract.py:65-201)

def rank_weights_closed_form(attention, rows, identity):
    """_three_step_weights (rules/extract.py:65-105): per body length 1..3
    the sum over identity placements, each term's products left to right,
    terms added left to right, in float64."""
    a = np.asarray(attention)
    rows = np.asarray(rows, np.int64)
    out = np.zeros((rows.shape[0], a.shape[1]))
    idw = a[:, :, identity].astype(np.float64)
    v = lambda s, ops: a[s, :, ops].astype(np.float64)  # noqa: E731  [k, L]
    i = np.flatnonzero(rows[:, 0] == 1)
    if i.size:
        o = rows[i, 1]
        out[i] = v(0, o) * idw[1] * idw[2] + idw[0] * v(1, o) * idw[2] + idw[0] * idw[1] * v(2, o)
    i = np.flatnonzero(rows[:, 0] == 2)
    if i.size:
        f, s = rows[i, 1], rows[i, 2]
        out[i] = v(0, f) * v(1, s) * idw[2] + v(0, f) * idw[1] * v(2, s) + idw[0] * v(1, f) * v(2, s)
    i = np.flatnonzero(rows[:, 0] == 3)
    if i.size:
        out[i] = v(0, rows[i, 1]) * v(1, rows[i, 2]) * v(2, rows[i, 3])
    return out


def rank_weights_dp(attention, rows, identity, maximum=False):
    """collapsed_rule_weights (rules/extract.py:108-129): dp over (step,
    operators placed), float64, sums or numpy maxima."""
    a = np.asarray(attention, np.float64)
    T, L, _ = a.shape
    rows = np.asarray(rows, np.int64)
    out = np.zeros((rows.shape[0], L))
    for length in range(1, T + 1):
        i = np.flatnonzero(rows[:, 0] == length)
        if not i.size:
            continue
        ops = rows[i, 1:1 + length]
        dp = np.zeros((i.size, length + 1, L))
        dp[:, 0] = 1.0
        for s in range(T):
            nx = dp * a[s, :, identity]
            for p in range(1, min(length, s + 1) + 1):
                c = dp[:, p - 1] * a[s, :, ops[:, p - 1]]
                nx[:, p] = np.maximum(nx[:, p], c) if maximum else nx[:, p] + c
            dp = nx
        out[i] = dp[:, length]
    return out


def rank_weights_brute(attention, rows, identity, maximum=False):
    """Independent check: enumerate the step sets that hold the body's
    operators (in order; the identity elsewhere), each product formed in
    step order from 1.0; sum (in float64, no fixed order) or max."""
    import itertools
    a = np.asarray(attention, np.float64)
    T, L, _ = a.shape
    rows = np.asarray(rows, np.int64)
    out = np.zeros((rows.shape[0], L))
    for r, row in enumerate(rows):
        length = int(row[0])
        if not 1 <= length <= T:
            continue
        for c in range(L):
            terms = []
            for places in itertools.combinations(range(T), length):
                prod, k = 1.0, 0
                for s in range(T):
                    if k < length and places[k] == s:
                        prod *= a[s, c, row[1 + k]]
                        k += 1
                    else:
                        prod *= a[s, c, identity]
                terms.append(prod)
            out[r, c] = max(terms) if maximum else float(np.sum(terms))
    return out


def select_and_annotate(candidates, attention, identity, minimum_positive_walks, fallback="sum"):
    """select_and_annotate_array (rules/extract.py:148-201): selection,
    fallback, precision and the lexicographic order, in numpy."""
    cand = np.asarray(candidates, np.int64)
    a = np.asarray(attention)
    T = a.shape[0]
    weights = (lambda rows: rank_weights_closed_form(a, rows, identity)) if T == 3 else \
        (lambda rows: rank_weights_dp(a, rows, identity))
    idx = np.flatnonzero(cand[:, -6] >= minimum_positive_walks)
    used = False
    allw = None
    if idx.size == 0 and cand.shape[0]:
        used = True
        allw = weights(cand)
        tot = allw.max(axis=1) if fallback == "max" else allw.sum(axis=1)
        idx = np.asarray([max(range(cand.shape[0]),
                              key=lambda j: (float(tot[j]), tuple(cand[j, 1:1 + cand[j, 0]])))])
    sel = cand[idx]
    rw = weights(sel) if allw is None else allw[idx]
    trials = sel[:, -8].astype(np.float64)
    pos = sel[:, -6].astype(np.float64)
    prec = np.divide(pos, trials, out=np.zeros_like(pos), where=trials != 0)
    cols = [np.where(sel[:, 0] >= p, sel[:, p], -1) for p in range(1, T + 1)]
    order = np.lexsort(tuple(reversed(cols)) + (-rw.sum(axis=1), -sel[:, -5]))
    return sel[order], prec[order], rw[order], used


def select_order_brute(selected, rank_weights, T):
    """Independent check of the output order: Python's stable sort by
    (-positive source hits, -weight sum, body padded with -1)."""
    keys = []
    for j, row in enumerate(selected):
        body = [int(row[p]) if row[0] >= p else -1 for p in range(1, T + 1)]
        keys.append((-int(row[-5]), -float(np.sum(rank_weights[j])), tuple(body)))
    return sorted(range(len(keys)), key=lambda j: keys[j])
