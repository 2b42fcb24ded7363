"""ctypes binding of libflashlog_hip.so (the C-ABI declared in
include/flashlog_hip.h).

The library is loaded from this package directory only.  There is no
fallback: if the library is missing or fails to load, every GPU entry point
raises, so a run can never silently use another implementation.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libflashlog_hip.so")
ABI_VERSION = 24
FL_SEG = 32
FL_SUP = 16

_lib = None


class FlSide(ctypes.Structure):
    """Mirror of ``fl_side`` (include/flashlog_hip.h)."""
    _fields_ = [
        ("edges", ctypes.c_int64),
        ("groups", ctypes.c_int64),
        ("col_ind", ctypes.c_void_p),
        ("mask", ctypes.c_void_p),
        ("row_group_ptr", ctypes.c_void_p),
        ("group_rel", ctypes.c_void_p),
        ("group_start", ctypes.c_void_p),
        ("group_count", ctypes.c_void_p),
        ("pull_ptr", ctypes.c_void_p),
        ("pull_pos", ctypes.c_void_p),
        ("pull_src", ctypes.c_void_p),
        ("pull_rel", ctypes.c_void_p),
        ("nseg", ctypes.c_int64),
        ("nheavy", ctypes.c_int64),
        ("nsup", ctypes.c_int64),
        ("seg_dst", ctypes.c_void_p),
        ("seg_start", ctypes.c_void_p),
        ("seg_h", ctypes.c_void_p),
        ("heavy_dst", ctypes.c_void_p),
        ("heavy_seg_ptr", ctypes.c_void_p),
        ("heavy_sup_ptr", ctypes.c_void_p),
        ("sup_h", ctypes.c_void_p),
        ("sup_seg0", ctypes.c_void_p),
        ("pos_src", ctypes.c_void_p),
        ("pos_rel", ctypes.c_void_p),
        ("order", ctypes.c_void_p),
        ("dscore", ctypes.c_void_p),
        ("grad_edge", ctypes.c_void_p),
        ("mask_bits", ctypes.c_void_p),
    ]


class FlSparseHop(ctypes.Structure):
    """Mirror of ``fl_sparse_hop`` (include/flashlog_hip.h)."""
    _fields_ = [
        ("sp_b", ctypes.c_void_p), ("sp_l", ctypes.c_void_p), ("sp_e", ctypes.c_void_p),
        ("sp_v", ctypes.c_void_p), ("nnz", ctypes.c_int64), ("w", ctypes.c_void_p),
        ("B", ctypes.c_int64), ("L", ctypes.c_int64), ("E", ctypes.c_int64), ("n", ctypes.c_int64),
        ("r_size", ctypes.c_int64), ("wot_i", ctypes.c_int), ("mode", ctypes.c_int),
        ("topk_edges", ctypes.c_int64), ("ws1", ctypes.c_void_p), ("ws1_bytes", ctypes.c_size_t),
        ("ws2", ctypes.c_void_p), ("ws2_bytes", ctypes.c_size_t), ("items", ctypes.c_int64),
        ("tiles", ctypes.c_int64), ("operators", ctypes.c_void_p), ("aggregate", ctypes.c_int),
        ("sampling_seed", ctypes.c_int64), ("raw_pos", ctypes.c_void_p), ("raw_col", ctypes.c_void_p),
        ("chunks", ctypes.c_int64), ("entry_order", ctypes.c_void_p),
    ]


class FlGroundGraph(ctypes.Structure):
    """Mirror of ``fl_ground_graph`` (include/flashlog_hip.h)."""
    _fields_ = [
        ("ori_col", ctypes.c_void_p), ("inv_col", ctypes.c_void_p),
        ("ori_ptr", ctypes.c_void_p), ("ori_start", ctypes.c_void_p), ("ori_count", ctypes.c_void_p),
        ("ori_rel", ctypes.c_void_p),
        ("inv_ptr", ctypes.c_void_p), ("inv_start", ctypes.c_void_p), ("inv_count", ctypes.c_void_p),
        ("inv_rel", ctypes.c_void_p),
        ("nodes", ctypes.c_int64), ("num_relations", ctypes.c_int64), ("max_groups", ctypes.c_int64),
        ("nhub", ctypes.c_int64), ("hub_options", ctypes.c_int64), ("hub_id", ctypes.c_void_p),
        ("hub_node", ctypes.c_void_p), ("hub_off", ctypes.c_void_p),
    ]


_SIGS = {
    "fl_last_error": (ctypes.c_char_p, []),
    "fl_abi_version": (ctypes.c_int, []),
    "fl_side_bytes": (ctypes.c_size_t, []),
    "fl_sparse_hop_bytes": (ctypes.c_size_t, []),
    "fl_ground_graph_bytes": (ctypes.c_size_t, []),
    "fl_csr_build_side": (ctypes.c_int, [ctypes.c_int64, ctypes.c_int64] + [ctypes.c_void_p] * 11 +
                          [ctypes.POINTER(ctypes.c_int64)]),
    "fl_csr_build_side_gpu_bytes": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int64]),
    "fl_csr_build_side_gpu": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64] + [ctypes.c_void_p] * 13 +
                              [ctypes.c_size_t]),
    "fl_pull_index_build": (ctypes.c_int, [ctypes.c_int64] * 3 + [ctypes.c_void_p] * 9),
    "fl_pull_segments": (ctypes.c_int, [ctypes.c_int64, ctypes.c_void_p] + [ctypes.POINTER(ctypes.c_int64)] * 3 +
                         [ctypes.c_void_p] * 8),
    "fl_apply_mask": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]),
    "fl_edge_dscore": (ctypes.c_int, [ctypes.c_void_p] * 4 + [ctypes.c_int64]),
    "fl_mark_active": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                      ctypes.c_int64, ctypes.c_void_p]),
    "fl_dense_topc": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p]),
    "fl_dense_topc_backward": (ctypes.c_int, [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 2),
    "fl_dense_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(FlSide), ctypes.POINTER(FlSide),
                                                   ctypes.c_int64, ctypes.c_int64]),
    "fl_dense_sum_forward": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(FlSide), ctypes.POINTER(FlSide),
                                            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                            ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int64,
                                            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                            ctypes.c_void_p, ctypes.c_size_t]),
    "fl_dense_backward_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(FlSide), ctypes.POINTER(FlSide),
                                                            ctypes.c_int64, ctypes.c_int64]),
    "fl_dense_sum_backward": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(FlSide), ctypes.POINTER(FlSide)] +
                              [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 4 + [ctypes.c_int, ctypes.c_int64] +
                              [ctypes.c_void_p] * 3 + [ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t]),
    "fl_dense_max_forward": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(FlSide), ctypes.POINTER(FlSide),
                                            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                            ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int64] +
                             [ctypes.c_void_p] * 6 + [ctypes.c_size_t]),
    "fl_dense_max_backward": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(FlSide), ctypes.POINTER(FlSide)] +
                              [ctypes.c_void_p] * 7 + [ctypes.c_int64] * 4 + [ctypes.c_int, ctypes.c_int64] +
                              [ctypes.c_void_p] * 3 + [ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t]),
    "fl_sparse_buckets": (ctypes.c_int64, [ctypes.c_int64]),
    "fl_sparse_plan_bytes": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]),
    "fl_sparse_plan": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(FlSide), ctypes.POINTER(FlSide),
                                      ctypes.POINTER(FlSparseHop), ctypes.c_void_p]),
    "fl_mask_bits": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]),
    "fl_mask_order_bits": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                          ctypes.c_void_p, ctypes.c_void_p]),
    "fl_sparse_expand_bytes": (ctypes.c_size_t, [ctypes.c_int64] * 5 + [ctypes.c_int] * 2),
    "fl_sparse_expand": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(FlSide), ctypes.POINTER(FlSide),
                                        ctypes.POINTER(FlSparseHop), ctypes.c_void_p, ctypes.c_void_p]),
    "fl_sparse_emit": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(FlSparseHop)] + [ctypes.c_void_p] * 5),
    "fl_sparse_backward_bytes": (ctypes.c_size_t, [ctypes.c_int64] * 3),
    "fl_sparse_backward_edge_bytes": (ctypes.c_size_t, [ctypes.c_int64] * 3),
    "fl_sparse_backward": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(FlSide), ctypes.POINTER(FlSide),
                                          ctypes.POINTER(FlSparseHop)] + [ctypes.c_void_p] * 6 +
                           [ctypes.c_size_t]),
    "fl_sparse_topc": (ctypes.c_int, [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 4 + [ctypes.c_void_p] * 3),
    "fl_sparse_rowptr_bytes": (ctypes.c_size_t, [ctypes.c_int64]),
    "fl_sparse_channel_sum_bytes": (ctypes.c_size_t, [ctypes.c_int64] * 3),
    "fl_sparse_channel_sum_plan": (ctypes.c_int, [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 4 +
                                   [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "fl_sparse_channel_sum_emit": (ctypes.c_int, [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 3 +
                                   [ctypes.c_int, ctypes.c_void_p, ctypes.c_int64] + [ctypes.c_void_p] * 4),
    "fl_reservoir_bytes": (ctypes.c_size_t, [ctypes.c_int64] * 4),
    "fl_reservoir": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                                    ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p,
                                    ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]),
    "fl_ground_walk_bytes": (ctypes.c_size_t, [ctypes.POINTER(FlGroundGraph)] + [ctypes.c_int64] * 3),
    "fl_ground_walks": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(FlGroundGraph), ctypes.c_void_p,
                                       ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_int64] + [ctypes.c_void_p] * 3 +
                        [ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_double, ctypes.c_void_p,
                         ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]),
    "fl_ground_count_bytes": (ctypes.c_size_t, [ctypes.c_int64] * 3),
    "fl_ground_count": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                       ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                                       ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]),
    "fl_sparse_race_bytes": (ctypes.c_size_t, [ctypes.c_int64] * 2),
    "fl_sparse_race_plan": (ctypes.c_int, [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 4 +
                            [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "fl_sparse_race_select": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 4 +
                              [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "fl_sparse_race_select_compact": (ctypes.c_int, [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 4 +
                                      [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t] + [ctypes.c_void_p] * 6),
    "fl_sparse_entry_order_bytes": (ctypes.c_size_t, [ctypes.c_int64] * 2),
    "fl_sparse_entry_order": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                             ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "fl_sparse_normalize_forward": (ctypes.c_int, [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 3 +
                                    [ctypes.c_float] + [ctypes.c_void_p] * 4),
    "fl_sparse_gather": (ctypes.c_int, [ctypes.c_void_p] * 5 + [ctypes.c_int64] + [ctypes.c_void_p] * 3 +
                         [ctypes.c_int64] * 3 + [ctypes.c_void_p]),
    "fl_sparse_normalize_backward": (ctypes.c_int, [ctypes.c_void_p] * 5 + [ctypes.c_int64, ctypes.c_float,
                                                                            ctypes.c_void_p]),
    "fl_sparse_channel_weighted_add": (ctypes.c_int, [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 4 +
                                       [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p]),
    "fl_rule_accumulate_bytes": (ctypes.c_size_t, [ctypes.c_int64] * 3),
    "fl_rule_accumulate": (ctypes.c_int, [ctypes.c_void_p] * 5 + [ctypes.c_int64, ctypes.c_void_p] +
                           [ctypes.c_int64] * 4 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t]),
    "fl_rule_finalize": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 3 +
                         [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]),
    "fl_filtered_ranks_workspace_bytes": (ctypes.c_size_t, [ctypes.c_int64, ctypes.c_int]),
    "fl_dense_filtered_ranks": (ctypes.c_int, [ctypes.c_void_p] * 4 + [ctypes.c_int64] * 3 + [ctypes.c_int,
                                                                                            ctypes.c_void_p]),
    "fl_filtered_ranks": (ctypes.c_int, [ctypes.c_void_p] * 4 + [ctypes.c_int] + [ctypes.c_void_p] * 2 +
                          [ctypes.c_int64] * 4 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                                  ctypes.c_size_t]),
    "fl_filtered_ranks_noalloc": (ctypes.c_int, [ctypes.c_void_p] * 4 + [ctypes.c_int] + [ctypes.c_void_p] * 2 +
                                  [ctypes.c_int64] * 4 + [ctypes.c_int, ctypes.c_void_p]),
    "fl_rule_rank_weights": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int] + [ctypes.c_int64] * 4 +
                             [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                              ctypes.c_int] + [ctypes.c_void_p] * 4),
    "fl_row_pairwise_sums": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                            ctypes.c_void_p]),
    "fl_filter_expand_bytes": (ctypes.c_size_t, [ctypes.c_int64]),
    "fl_filter_expand_count": (ctypes.c_int, [ctypes.c_void_p] * 4 + [ctypes.c_int64, ctypes.c_void_p,
                                                                     ctypes.c_int64, ctypes.c_int64,
                                                                     ctypes.c_void_p, ctypes.c_void_p,
                                                                     ctypes.c_size_t]),
    "fl_filter_expand_fill": (ctypes.c_int, [ctypes.c_void_p] * 3 + [ctypes.c_int64, ctypes.c_void_p,
                                                                    ctypes.c_void_p, ctypes.c_int64] +
                              [ctypes.c_void_p] * 3),
    "fl_prof_enable": (ctypes.c_int, [ctypes.c_int]),
    "fl_prof_read": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                    ctypes.POINTER(ctypes.c_int64)]),
}


def prof_enable(on=True):
    check(lib().fl_prof_enable(1 if on else 0), "prof_enable")


def prof_read(kernel):
    """(total_ms, launches) of `kernel` since prof_enable (waits on its events)."""
    tot = ctypes.c_double(0.0)
    cnt = ctypes.c_int64(0)
    check(lib().fl_prof_read(kernel.encode(), ctypes.byref(tot), ctypes.byref(cnt)), "prof_read")
    return tot.value, cnt.value


def exported_symbols():
    """Names the C-ABI header declares (the ctypes signature table)."""
    return sorted(_SIGS)


# each argument struct and the entry point returning the library's sizeof
STRUCT_SIZES = ((FlSide, "fl_side_bytes"), (FlSparseHop, "fl_sparse_hop_bytes"),
                (FlGroundGraph, "fl_ground_graph_bytes"))


def lib():
    """Load libflashlog_hip.so once; raise if it is missing or stale."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                "libflashlog_hip.so is not built (expected at %s); run "
                "`python flashlog_amd/build.py` or __graft_entry__.build()" % LIB_PATH)
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.fl_abi_version() != ABI_VERSION:
            raise RuntimeError("libflashlog_hip.so ABI version mismatch; rebuild it")
        for struct, size_fn in STRUCT_SIZES:
            if ctypes.sizeof(struct) != getattr(handle, size_fn)():
                raise RuntimeError("ctypes layout of %s differs from the library's (%d vs %d bytes)"
                                   % (struct.__name__, ctypes.sizeof(struct), getattr(handle, size_fn)()))
        _lib = handle
    return _lib


def check(rc, what):
    if rc != 0:
        msg = lib().fl_last_error().decode(errors="replace")
        if "nonnegative" in msg or "shape" in msg or "range" in msg:
            raise ValueError("%s: %s" % (what, msg))
        raise RuntimeError("%s failed (%d): %s" % (what, rc, msg))


def stream_handle(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None and t.numel() > 0 else ctypes.c_void_p(0)
