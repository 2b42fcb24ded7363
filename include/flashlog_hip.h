/*
 * flashlog_hip.h -- C-ABI of the MI355X (gfx950) FlashLog propagation library
 * (libflashlog_hip.so).  Plain pointers and sizes only; every device pointer
 * is a device (HBM) address, every stream is a hipStream_t passed as void*.
 *
 * Each entry point names the reference interface it replaces
 * (paths relative to the qikunxun/FlashLog tree).
 *
 * Conventions
 *   - Return value: FL_OK (0) or an FL_ERR_* code; fl_last_error() gives the
 *     message of the last failure on the calling thread.
 *   - No entry point allocates device memory.  Outputs and workspaces are
 *     allocated by the caller (so allocation failures surface in the caller's
 *     allocator, e.g. torch.cuda.OutOfMemoryError).  Workspace sizes come from
 *     the matching *_workspace_bytes query.
 *   - All device work is enqueued on the given stream; nothing synchronizes
 *     the host unless stated.
 */
#ifndef FLASHLOG_HIP_H
#define FLASHLOG_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FL_OK 0
#define FL_ERR_ARG 1
#define FL_ERR_HIP 2

/* Destinations with more than FL_SEG incoming positions on a side are
 * "heavy": their slots are processed in segments of FL_SEG. */
#define FL_SEG 32
/* Segments are grouped FL_SUP at a time into supersegments. */
#define FL_SUP 16

/* One side (ORI or INV) of the graph in device memory.  col_ind and the
 * group arrays are the reference's CSR tuple entries for that side
 * (flashlog_kernel.py:697), mask the prepared CSR-ordered mask
 * (flashlog_kernel.py:232-255).  The pull_* and heavy-destination fields are
 * this library's destination-major index of the same positions, built once
 * per graph by fl_pull_index_build and fl_pull_segments. */
typedef struct fl_side {
    int64_t edges;                 /* M: CSR positions on this side        */
    int64_t groups;                /* G: (source, relation) groups         */
    const int32_t *col_ind;        /* [M] destination of each position     */
    const float *mask;             /* [M] prepared mask, CSR order         */
    const int32_t *row_group_ptr;  /* [E+1]                                */
    const int16_t *group_rel;      /* [G]                                  */
    const int32_t *group_start;    /* [G]                                  */
    const int32_t *group_count;    /* [G]                                  */
    const int32_t *pull_ptr;       /* [E+1] slots of each destination      */
    const int32_t *pull_pos;       /* [M] CSR position of each slot        */
    const int32_t *pull_src;       /* [M] source entity of each slot       */
    const int16_t *pull_rel;       /* [M] relation of each slot            */
    int64_t nseg;                  /* segments of heavy destinations       */
    int64_t nheavy;                /* heavy destinations                   */
    int64_t nsup;                  /* supersegments                        */
    const int32_t *seg_dst;        /* [nseg] destination of each segment   */
    const int32_t *seg_start;      /* [nseg] first slot of each segment    */
    const int32_t *seg_h;          /* [nseg] heavy index of each segment   */
    const int32_t *heavy_dst;      /* [nheavy] heavy destinations          */
    const int32_t *heavy_seg_ptr;  /* [nheavy+1] segments of each          */
    const int32_t *heavy_sup_ptr;  /* [nheavy+1] supersegments of each     */
    const int32_t *sup_h;          /* [nsup] heavy index of each           */
    const int32_t *sup_seg0;       /* [nsup] first segment of each         */
    const int32_t *pos_src;        /* [M] source entity of each position   */
    const int16_t *pos_rel;        /* [M] relation of each position        */
    const int32_t *order;          /* [M] original edge id of each position
                                      (sparse max tie order, edge-weight
                                      gradients; else unused)              */
    const float *dscore;           /* [M] optional: 1 - sigmoid(edge weight)
                                      of each position (trainable edge
                                      weights, sparse backward)            */
    float *grad_edge;              /* optional: [edges] gradient of the edge
                                      weights by original edge id (both
                                      sides may share it)                  */
    const uint32_t *mask_bits;     /* optional: [ceil(M/32)] bit p = mask[p]
                                      != 0, set only when every mask value
                                      is 0 or 1 (fl_mask_bits, or
                                      fl_mask_order_bits from a bool mask);
                                      the sparse hop then tests bits and
                                      never reads mask, which may be null  */
} fl_side;

const char *fl_last_error(void);
int fl_abi_version(void);
/* sizeof of the argument structs, so that a binding can check its own
 * layout against the library's (no counterpart in the reference: its
 * pybind11 bindings take tensors, not structs). */
size_t fl_side_bytes(void);
size_t fl_sparse_hop_bytes(void);
size_t fl_ground_graph_bytes(void);

/* ---- host-side graph preparation ------------------------------------- */

/* Replaces csr.cpp:12-69 (build_side) on the GPU: the same arrays as
 * fl_csr_build_side (positions ordered by (source, relation, edge id),
 * groups the runs of equal (source, relation)) from device arrays, by one
 * stable radix sort of (source << 15 | relation) carrying the edge ids.
 * Group arrays need capacity >= edges; info (device int64[2]) receives
 * {number of groups, error} (error 1: an entity outside [0, nodes) or a
 * relation outside [0, 32767]); workspace of fl_csr_build_side_gpu_bytes. */
size_t fl_csr_build_side_gpu_bytes(int64_t edges, int64_t nodes);
int fl_csr_build_side_gpu(void *stream, int64_t edges, int64_t nodes,
                          const int64_t *source, const int64_t *target,
                          const int64_t *relation, int32_t *row_ptr,
                          int32_t *columns, int16_t *edge_rel, int32_t *order,
                          int32_t *group_ptr, int16_t *group_rel,
                          int32_t *group_start, int32_t *group_count,
                          int64_t *info, void *workspace,
                          size_t workspace_bytes);

/* Replaces csr.cpp:12-69 (build_side), called by build_csr_structure
 * (flashlog_kernel.py:678-697).  Host arrays.  Positions are ordered by
 * (source, relation, edge id); group arrays need capacity >= edges. */
int fl_csr_build_side(int64_t edges, int64_t nodes, const int64_t *source,
                      const int64_t *target, const int64_t *relation,
                      int32_t *row_ptr, int32_t *columns, int16_t *edge_rel,
                      int32_t *order, int32_t *group_ptr, int16_t *group_rel,
                      int32_t *group_start, int32_t *group_count,
                      int64_t *num_groups);

/* No reference counterpart (the reference pushes with atomics): the
 * destination-major pull index of one CSR side, host arrays.  Slots of a
 * destination are in ascending CSR position, the order in which the
 * reference's CPU path accumulates (flashlog.cpp:194-210). */
int fl_pull_index_build(int64_t nodes, int64_t edges, int64_t groups,
                        const int32_t *columns, const int32_t *row_group_ptr,
                        const int16_t *group_rel, const int32_t *group_start,
                        const int32_t *group_count, int32_t *pull_ptr,
                        int32_t *pull_pos, int32_t *pull_src, int16_t *pull_rel);

/* Heavy-destination segments of one side from its pull_ptr (host arrays):
 * first call with null outputs to get the counts, then with arrays of those
 * sizes (the *_ptr arrays have nheavy+1 entries). */
int fl_pull_segments(int64_t nodes, const int32_t *pull_ptr, int64_t *nseg,
                     int64_t *nheavy, int64_t *nsup, int32_t *seg_dst,
                     int32_t *seg_start, int32_t *seg_h, int32_t *heavy_dst,
                     int32_t *heavy_seg_ptr, int32_t *heavy_sup_ptr,
                     int32_t *sup_h, int32_t *sup_seg0);

/* ---- device entry points --------------------------------------------- */

/* Replaces apply_mask_cuda (flashlog.cu:1291-1340):
 * out[i] = mask[order[i]] * (weight ? sigmoid(weight[order[i]]) : 1). */
int fl_apply_mask(void *stream, const void *mask_values, int mask_is_bool,
                  const int32_t *order, const float *weight, float *out,
                  int64_t nnz);

/* bits[w] bit j = (mask[32w + j] != 0) for the n positions of a CSR-ordered
 * mask (bits: ceil(n/32) words): a side's mask_bits, for masks whose values
 * are all 0 or 1 (a bool visibility mask without edge weights).  No
 * counterpart in the reference: a compact copy of the mask the sparse
 * kernels gather from. */
int fl_mask_bits(void *stream, const float *mask, int64_t n, uint32_t *bits);

/* A side's mask_bits straight from the Boolean visibility mask by original
 * edge id (bool [n], one byte each) and the side's order (CSR position ->
 * edge id): bits[w] bit j = mask[order[32w + j]], for the n positions.
 * edge_bits is caller scratch of ceil(n/32) words (the mask packed by edge
 * id).  Replaces apply_mask_cuda (flashlog.cu:1291-1340) followed by
 * fl_mask_bits for a bool mask without edge weights, without the float
 * gather (a bit gather from an M/8-byte table instead). */
int fl_mask_order_bits(void *stream, const uint8_t *mask, const int32_t *order, int64_t n,
                       uint32_t *edge_bits, uint32_t *bits);

/* out[i] = 1 - sigmoid(weight[order[i]]) for i < nnz: the per-position edge
 * score derivative factor of the sparse backward with trainable edge
 * weights (flashlog_kernel.py:1306-1336, score_function :221). */
int fl_edge_dscore(void *stream, const float *weight, const int32_t *order,
                   float *out, int64_t nnz);

/* Replaces compute_active_nodes_cuda's flag pass (flashlog.cu:1257-1284):
 * flags[e] = 1 if any A[:, e] != 0 else 0. */
int fl_mark_active(void *stream, const float *A, int64_t BL, int64_t E,
                   int32_t *flags);

/* Replaces _dense_topc_state (flashlog_kernel.py:814-842), the c1 entity
 * budget: per row of A[BL, E], rows with more than c nonzeros keep their c
 * largest nonzeros (ties at the cutoff go to the smaller entity id);
 * out = A * keep.  row_state[BL*4] receives, per row, {over, cutoff key,
 * last kept tied entity, nonzero count} for fl_dense_topc_backward. */
int fl_dense_topc(void *stream, const float *A, float *out, int64_t BL,
                  int64_t E, int64_t c, int32_t *row_state);

/* Backward of the product A * keep: grad_A = grad * keep. */
int fl_dense_topc_backward(void *stream, const float *grad, const float *A,
                           const int32_t *row_state, float *grad_A, int64_t BL,
                           int64_t E);

/* Workspace for fl_dense_sum_forward on this graph and state shape. */
size_t fl_dense_workspace_bytes(const fl_side *ori, const fl_side *inv,
                                int64_t BL, int64_t E);

/* Replaces flashlog_forward_cuda with agg_mode = sum (flashlog.cu:898-995),
 * with the CPU path's bit-exact semantics (flashlog.cpp:151-211):
 *   out_ind = A * w[:, n-1] (0 if wot_i);
 *   out_ori[bl, d] = sum over kept ORI positions p (ascending) with
 *       col[p] == d of (A[bl, src(p)] * w[bl, rel(p)]) * mask[p];
 *   out_inv likewise with INV positions and w[bl, r_size + rel].
 * topk_edges <= 0 or >= 2^60 disables c2 pruning (flashlog.cu:958).
 * Requires BL <= 1024 and BL*E < 2^31. */
int fl_dense_sum_forward(void *stream, const fl_side *ori, const fl_side *inv,
                         const float *A, const float *w, int64_t BL, int64_t E,
                         int64_t n, int64_t r_size, int wot_i,
                         int64_t topk_edges, float *out_ind, float *out_ori,
                         float *out_inv, void *workspace,
                         size_t workspace_bytes);

/* Workspace for fl_dense_sum_backward. */
size_t fl_dense_backward_workspace_bytes(const fl_side *ori, const fl_side *inv,
                                         int64_t BL, int64_t E);

/* Replaces flashlog_backward_cuda with agg_mode = sum (flashlog.cu:1077-1185),
 * with the CPU path's semantics (flashlog.cpp:91-146,216-278): grad_A is the
 * identity term 0 + g_ind*w[n-1] plus the ORI then INV terms added in CSR
 * order (bit-identical to the CPU path); grad_w's identity column is a fixed
 * tree sum over entities and its relation columns add per-group partial
 * sums in ascending source order (a fixed order, equal to the CPU path
 * within float rounding).  pg holds pg_pairs * n floats of scratch, where
 * pg_pairs must be the number of nonzero entries of A (rows beyond
 * pg_pairs are skipped, never written).  The edge admission is rebuilt from
 * A and w, so A must be the state the forward saw (after c1). */
int fl_dense_sum_backward(void *stream, const fl_side *ori, const fl_side *inv,
                          const float *A, const float *w,
                          const float *grad_ind, const float *grad_ori,
                          const float *grad_inv, int64_t BL, int64_t E,
                          int64_t n, int64_t r_size, int wot_i,
                          int64_t topk_edges, float *grad_A, float *grad_w,
                          float *pg, int64_t pg_pairs, void *workspace,
                          size_t workspace_bytes);

/* Replaces flashlog_forward_max_cuda (flashlog.cu:997-1072; kernels
 * :523-637, packing :104-135), called by FlashLogDenseMaxFunction
 * (flashlog_kernel.py:992-1055).  Same kept edges as fl_dense_sum_forward;
 * out_ori[bl, d] is the product (A*w)*mask of the winning kept ORI position
 * p, where the winner maximizes the 64-bit key (float bits of the product
 * << 32 | 0xFFFFFFFF - p): larger value bits win, ties go to the smaller
 * position.  arg_ori[bl, d] = p, or -1 (and 0.0) when no kept edge enters d.
 * INV likewise.  out_ind = A * w[:, n-1] (0 if wot_i).  Uses the workspace
 * size of fl_dense_workspace_bytes. */
int fl_dense_max_forward(void *stream, const fl_side *ori, const fl_side *inv,
                         const float *A, const float *w, int64_t BL, int64_t E,
                         int64_t n, int64_t r_size, int wot_i,
                         int64_t topk_edges, float *out_ind, float *out_ori,
                         float *out_inv, int64_t *arg_ori, int64_t *arg_inv,
                         void *workspace, size_t workspace_bytes);

/* Replaces flashlog_backward_max_cuda (flashlog.cu:1187-1255; kernel
 * :639-726) without its atomics: grad_A[bl, src] = g_ind*w[n-1] (0 if
 * wot_i) plus, over the kept ORI then INV positions p of src in CSR order
 * that won their destination d (arg[bl, d] == p) with mask and grad
 * nonzero, (grad*w[rel(p)])*mask[p] -- a fixed order, so every run gives
 * the same bits; grad_w[bl, n-1] = sum_e g_ind*A (fixed tree order) and the
 * relation columns add per-(source, row) partials of (grad*A)*mask in
 * ascending source order.  topk_edges must be the forward's (the kept
 * positions are rebuilt from A and w as in fl_dense_sum_backward); pg,
 * pg_pairs and the workspace (fl_dense_backward_workspace_bytes) as there. */
int fl_dense_max_backward(void *stream, const fl_side *ori, const fl_side *inv,
                          const float *A, const float *w,
                          const float *grad_ind, const float *grad_ori,
                          const float *grad_inv, const int64_t *arg_ori,
                          const int64_t *arg_inv, int64_t BL, int64_t E,
                          int64_t n, int64_t r_size, int wot_i,
                          int64_t topk_edges, float *grad_A, float *grad_w,
                          float *pg, int64_t pg_pairs, void *workspace,
                          size_t workspace_bytes);

/* ---- sparse (COO) hop ------------------------------------------------- */

/* One sparse hop: the COO state (entries sorted by row r = b*L + l, as a
 * coalesced state is), attention w [B*L, n], and the caller's workspaces.
 * mode 0 = top-k sum (kept edges with a nonzero mask; FlashLogFunction-
 * Sparse3DTopKSum, flashlog.cu:1368-1559), mode 1 = all edges
 * (FlashLogFunctionSparse3DAllEdgesSum, flashlog.cu:1743-1829), mode 2 =
 * fixed-relation rule step (flashlog_forward_sparse3d_fixed_relation_cuda,
 * flashlog.cu:1561-1741: row (b, l) follows operators[b*L + l], values
 * unchanged, no masks; w, n and wot_i unused, r_size = base relations).
 * items / tiles / chunks come from fl_sparse_plan's plan[0] / plan[1] /
 * plan[4]. */
typedef struct fl_sparse_hop {
    const int64_t *sp_b, *sp_l, *sp_e;  /* [nnz] */
    const float *sp_v;                 /* [nnz] */
    int64_t nnz;
    const float *w;                    /* [B*L, n] */
    int64_t B, L, E, n, r_size;
    int wot_i;
    int mode;
    int64_t topk_edges;                /* c2 budget K (mode 0): K >= 2^60 keeps
                                          every eligible edge, 0 < K selects,
                                          K <= 0 keeps none (the reference's
                                          min(eligible, K) count)            */
    void *ws1;                         /* plan workspace */
    size_t ws1_bytes;
    void *ws2;                         /* expansion workspace */
    size_t ws2_bytes;
    int64_t items, tiles;
    const int64_t *operators;          /* mode 2: [B*L] operator per row     */
    int aggregate;                     /* 0 sum (masked kept edges produce no
                                          coordinate), 1 max (masked kept
                                          edges are 0-valued items; ties go to
                                          ORI < INV < identity, then the
                                          smaller original edge id, then raw
                                          order: flashlog_kernel.py:399-478) */
    int64_t sampling_seed;             /* mode 0: < 0 the c2 threshold;
                                          >= 0 the training quotas of
                                          flashlog.cu:1433-1528 (weighted
                                          floors + SplitMix64-phased
                                          systematic residuals)             */
    int32_t *raw_pos;                  /* with raw_local (fl_sparse_expand):
                                          [items] receives every raw item's
                                          CSR position in its side (-1 for
                                          the identity item).  May be null
                                          when the backward reads no mask
                                          value or edge factor: the top-k
                                          sum (masked items are dropped)
                                          with E > 8192, each side's mask
                                          absent or given as mask_bits, and
                                          no side carrying dscore.          */
    int16_t *raw_col;                  /* with raw_local: [items] receives its
                                          attention column (ORI relation,
                                          r_size + INV relation, n - 1 for the
                                          identity); needs n <= 32767.  The
                                          backward reads both instead of
                                          walking the groups again.          */
    int64_t chunks;                    /* the plan's 64-item chunks (each
                                          entry's items cut into chunks of
                                          64), sizing the expansion's chunk
                                          table                              */
    const int32_t *entry_order;        /* optional: [nnz] a permutation of
                                          the entries (e.g. by source
                                          entity) in which the plan and the
                                          expansion visit them, so that
                                          entries of one source run close
                                          together; results do not depend on
                                          it.  The same array for plan and
                                          expand; a non-permutation is
                                          error 1                            */
} fl_sparse_hop;

/* Destination buckets per row (8192 entities each).  The sparse hop
 * supports E <= 2^27 entities. */
int64_t fl_sparse_buckets(int64_t E);

/* Plan workspace bytes for nnz entries, R = B*L rows and r_size relations
 * per side (0 for the fixed-relation step).  With 0 < r_size <= 4096 the
 * plan holds each row's c2 admission order (relations by weight desc, id
 * asc), which the top-k threshold of sources with many groups reads. */
size_t fl_sparse_plan_bytes(int64_t nnz, int64_t R, int64_t r_size);

/* Replaces the count kernels and the host .item() syncs of
 * flashlog_forward_sparse3d_topk_cuda / _alledges_cuda (flashlog.cu:
 * 1999-2241): per entry and side the c2 threshold (flashlog.cpp:12-35) and
 * item counts; plan (device int64[6]) receives {items, tiles, error,
 * buckets, chunks, nonfinite} (chunks: the sum over entries of ceil(items
 * / 64); nonfinite: 1 when an attention weight of w is not finite, the
 * condition the top-k hops reject, flashlog.cu:2019-2021).  error: 0 ok, 1 index out of range, 2 entries not sorted by row.
 * The caller reads plan after the stream completes. */
int fl_sparse_plan(void *stream, const fl_side *ori, const fl_side *inv,
                   const fl_sparse_hop *h, int64_t *plan);

/* Expansion workspace bytes (backward = 1 when raw_local will be kept;
 * aggregate as in fl_sparse_hop). */
size_t fl_sparse_expand_bytes(int64_t items, int64_t tiles, int64_t chunks,
                              int64_t R, int64_t E, int backward,
                              int aggregate);

/* Replaces the fill kernels (flashlog.cu:1402-1559,1759-1854) and the
 * coalesce (flashlog_kernel.py:258-357 sum, :399-478 max): raw items in the
 * CPU path's order (flashlog.cpp:1388-1486), grouped per (row, destination)
 * and added to 0 in that order (sum) or reduced to the winning item (max).
 * out_base [B*L*buckets + 1] receives the output offsets of every (row,
 * bucket) (out_base[last] = output count); raw_local (optional, [items],
 * needs items < 2^31) the output index of every raw item (-1 for the losing
 * items of the max; unspecified for the holes of the sum, which the backward
 * recognises by their mask), for fl_sparse_backward. */
int fl_sparse_expand(void *stream, const fl_side *ori, const fl_side *inv,
                     const fl_sparse_hop *h, int64_t *out_base,
                     int32_t *raw_local);

/* Writes the coalesced output (ascending (b, l, e)); arrays hold
 * out_base[last] entries. */
int fl_sparse_emit(void *stream, const fl_sparse_hop *h,
                   const int64_t *out_base, int64_t *out_b, int64_t *out_l,
                   int64_t *out_e, float *out_v);

/* Workspace bytes of fl_sparse_backward (nnz entries, R = B*L rows, n
 * attention columns). */
size_t fl_sparse_backward_bytes(int64_t nnz, int64_t R, int64_t n);

/* Replaces flashlog_backward_sparse3d_cached_cuda and, for max,
 * flashlog_backward_sparse3d_max_cached_cuda (flashlog.cu:2243-2478,
 * kernels :1856-1997) without their atomics: grad_v[i] = sum over entry
 * i's items (max: its winning items) of (g*m)*w (+ g*w[n-1] for the
 * identity item), added by one wave in a fixed order; grad_w [B*L, n] =
 * per row the sum of (g*m)*a (+ g*a at n-1) over its items, in a fixed
 * order (per entry and column the run of the column, entries in fixed
 * chunks, chunks in order), so every run gives the same bits.  grad_out
 * holds the gradient of every output entry.  With a side's grad_edge set
 * (trainable edge weights, flashlog_kernel.py:1306-1336),
 * grad_edge[order[p]] also receives (((g*a)*w)*m)*dscore[p] of the side's
 * items without atomics (the reference adds them with index_add_): per
 * position the terms are folded from 0 in raw item order, then added to
 * the edge's value, the ORI side before the INV side (the caller zeroes
 * grad_edge; the same bits on every run).  Needs the plan workspace of the
 * forward, the raw_pos / raw_col arrays that its expand filled
 * (h->raw_pos, h->raw_col) and a workspace of fl_sparse_backward_bytes,
 * plus fl_sparse_backward_edge_bytes when a side has grad_edge. */
int fl_sparse_backward(void *stream, const fl_side *ori, const fl_side *inv,
                       const fl_sparse_hop *h, const int64_t *out_base,
                       const int32_t *raw_local, const float *grad_out,
                       float *grad_v, float *grad_w, void *workspace,
                       size_t workspace_bytes);

/* Extra workspace bytes fl_sparse_backward needs, after its own, when a
 * side carries grad_edge: per raw item a key and a term, their sorted
 * copies and the radix sort's scratch (no counterpart in the reference,
 * whose edge gradient is an atomic index_add_). */
size_t fl_sparse_backward_edge_bytes(int64_t items, int64_t ori_edges,
                                     int64_t inv_edges);

/* Replaces _sparse_topc_entries (flashlog_kernel.py:1092-1140), the c1
 * budget on a COO state sorted by row: keep[i] = 1 for the entries to keep.
 * Rows with more than c nonzeros keep their c largest nonzeros (ties to the
 * earlier entry); other rows keep every entry.  row_ptr [B*L+1] and err [1]
 * are caller scratch as for fl_sparse_normalize_forward. */
int fl_sparse_topc(void *stream, const int64_t *sp_b, const int64_t *sp_l,
                   const float *v, int64_t nnz, int64_t B, int64_t L,
                   int64_t c, int32_t *keep, int64_t *row_ptr, int64_t *err);

/* Sampled c1 (_sparse_topc_entries with sampling=True, flashlog_kernel.py:
 * 1092-1140): the exponential race.  Two phases around the caller's noise
 * draw.  fl_sparse_race_plan (c >= 1; c = 0 is fl_sparse_topc): per row r =
 * b*L + l of a COO state sorted by row, rows with more than c nonzeros make
 * their nonzero entries candidates; info (device int64[3]) receives
 * {candidates, error, kept} (error 1 index out of range, 2 not sorted by
 * row, 3 a candidate value not finite and positive; kept = the entries the
 * select will keep: c per over-limit row, every entry of the others).  The
 * caller then draws one Exp(1) double per candidate (entry order) into noise
 * and calls fl_sparse_race_select: in those rows keep[i] = 1 for the c
 * candidates with the largest log(v) - log(noise) (ties to the earlier
 * entry), 0 for the rest; other rows keep every entry.  ws is the same
 * workspace in both calls.  fl_sparse_race_select_compact does the same and
 * also writes the kept entries in entry order (the reference's
 * torch.nonzero(keep) and the gathers of _prune_sparse_sources,
 * flashlog_kernel.py:1137-1147): entries [kept] their indices, out_b, out_l,
 * out_e, out_v [kept] their coordinates and values (kept from info[2], so
 * the caller sizes them without another read of the device). */
size_t fl_sparse_race_bytes(int64_t nnz, int64_t R);
int fl_sparse_race_plan(void *stream, const int64_t *sp_b, const int64_t *sp_l,
                        const float *v, int64_t nnz, int64_t B, int64_t L,
                        int64_t c, void *ws, size_t ws_bytes, int64_t *info);
int fl_sparse_race_select(void *stream, const float *v, int64_t nnz,
                          int64_t B, int64_t L, int64_t c,
                          const double *noise, void *ws, size_t ws_bytes,
                          int32_t *keep);
int fl_sparse_race_select_compact(void *stream, const int64_t *sp_b,
                                  const int64_t *sp_l, const int64_t *sp_e,
                                  const float *v, int64_t nnz, int64_t B,
                                  int64_t L, int64_t c, const double *noise,
                                  void *ws, size_t ws_bytes, int32_t *keep,
                                  int64_t *entries, int64_t *out_b,
                                  int64_t *out_l, int64_t *out_e,
                                  float *out_v);

/* The entry visiting order a sparse hop may take (fl_sparse_hop.entry_order).
 * No counterpart in the reference: a locality order for this library's plan
 * and run writer (the entries of one source entity read the same group
 * records); the hop's results do not depend on it.  order [nnz] (int32)
 * lists the entries grouped by ascending blocks of 64 entity ids (sp_e >> 6;
 * a counting sort over the blocks, the entries of one block in any order).
 * nnz < 2^31; ws of fl_sparse_entry_order_bytes(nnz, E). */
size_t fl_sparse_entry_order_bytes(int64_t nnz, int64_t E);
int fl_sparse_entry_order(void *stream, const int64_t *sp_e, int64_t nnz,
                          int64_t E, void *ws, size_t ws_bytes,
                          int32_t *order);

/* Bytes of the row pointer + error slots used by the normalize calls. */
size_t fl_sparse_rowptr_bytes(int64_t R);

/* Replaces sparse3d_normalize_forward_cuda (flashlog.cu:2480-2640):
 * per row r = b*L + l, denom[r] = the left fold from 0 of its values in
 * entry order (the CPU path's order, flashlog.cpp:1561-1565, so the bits
 * equal the CPU path's) and out = v / dc with dc = denom >= eps ? denom :
 * eps (the GPU path's clamp, flashlog.cu:2540: a NaN sum divides by eps),
 * IEEE division.  Precondition: entries sorted by row with every row key in
 * [0, R) (not checked, as the reference's GPU path does not: rows found by
 * binary search).  Other input gives unspecified values, but every entry of
 * out is written (row 0 starts at entry 0 and row R-1 ends at nnz) and
 * nothing is accessed out of range; row_ptr [R+1] and err [1] are caller
 * scratch (err is cleared). */
int fl_sparse_normalize_forward(void *stream, const int64_t *sp_b,
                                const int64_t *sp_l, const float *v,
                                int64_t nnz, int64_t B, int64_t L, float eps,
                                float *out, float *denom, int64_t *row_ptr,
                                int64_t *err);

/* Replaces _align_sparse_grad_to_output (flashlog_kernel.py:360-376):
 * out[i] = the value of the coalesced COO tensor (gb, gl, ge, gv; ng
 * entries, keys (b*L + l)*E + e strictly increasing) at query coordinate
 * (qb[i], ql[i], qe[i]), or 0 where it has no entry. */
int fl_sparse_gather(void *stream, const int64_t *gb, const int64_t *gl,
                     const int64_t *ge, const float *gv, int64_t ng,
                     const int64_t *qb, const int64_t *ql, const int64_t *qe,
                     int64_t nq, int64_t L, int64_t E, float *out);

/* Replaces sparse3d_normalize_backward_cuda (flashlog.cu:2642-2691):
 * grad_v = g/dc - sum_row(g*v)/dc^2 where denom >= eps (dc = denom), else
 * g/eps (dc = eps, NaN denominators included); sum_row in a fixed tree
 * order. */
int fl_sparse_normalize_backward(void *stream, const int64_t *row_ptr,
                                 const float *grad, const float *v,
                                 const float *denom, int64_t R, float eps,
                                 float *grad_v);

/* Replaces the models' channel sum sum_sp_3d (src/model_DRUM_kernel_sp.py:
 * 22-28, also the sum of src/model_smDRUM_kernel_sp.py and
 * src/model_NeuralLP_kernel_sp.py): of a coalesced [B, L, E] state (entries
 * sorted by (b, l), entities strictly increasing within a row), the [B, E]
 * state out[b, e] = sum over l of v[b, l, e], added from 0 in channel order
 * (torch's coalesce of the (b, e) re-index sorts stably, so duplicates add
 * in l order).  fl_sparse_channel_sum_plan ranks the entries into the
 * caller's workspace (fl_sparse_channel_sum_bytes) and writes plan[2] =
 * {outputs, error} on the device (error != 0: entries out of range or not
 * coalesced); after the host has read it, fl_sparse_channel_sum_emit (same
 * workspace) writes out_b, out_e, out_v [outputs], in (b, e) order, and
 * slot[nnz], the output slot of every entry (for the backward).  op 1
 * instead takes the maximum over the channels (max_sp_3d,
 * src/model_mmDRUM_kernel_sp.py:17-32: scatter_reduce amax, NaN propagated;
 * of equal values the first channel's is kept); op 0 is the sum. */
size_t fl_sparse_channel_sum_bytes(int64_t nnz, int64_t B, int64_t L);
int fl_sparse_channel_sum_plan(void *stream, const int64_t *sp_b,
                               const int64_t *sp_l, const int64_t *sp_e,
                               int64_t nnz, int64_t B, int64_t L, int64_t E,
                               void *ws, size_t ws_bytes, int64_t *plan);
int fl_sparse_channel_sum_emit(void *stream, const int64_t *sp_b,
                               const int64_t *sp_e, const float *v,
                               int64_t nnz, int64_t B, int64_t L, int op,
                               void *ws, int64_t nout, int64_t *out_b,
                               int64_t *out_e, float *out_v, int32_t *slot);

/* ---- rule-bank scoring ------------------------------------------------- */

/* Adds weighted channel sums of a coalesced [B, L, E] state into a dense
 * accumulator: for every (b, e) and rank k, dense[k, b*E + e] += the sum
 * from 0, in channel order, of v[b, l, e] * W[l, k].  Uses the workspace
 * that fl_sparse_channel_sum_plan filled (the host need not read its plan
 * first: a state the plan flagged adds nothing, the kernel reads the error
 * word itself); one writer per accumulator slot, so no atomics. */
int fl_sparse_channel_weighted_add(void *stream, const int64_t *sp_b,
                                   const int64_t *sp_l, const int64_t *sp_e,
                                   const float *v, int64_t nnz, int64_t B,
                                   int64_t L, int64_t E, const float *W,
                                   int64_t K, void *ws, float *dense);

/* ---- rule-bank scoring ------------------------------------------------- */

/* Workspace bytes of fl_rule_accumulate (sum) for a chunk state of nnz
 * entries, B sources and L rules. */
size_t fl_rule_accumulate_bytes(int64_t nnz, int64_t B, int64_t L);

/* Replaces the dense accumulation of rules/shared_inference.py:200-206
 * (index_add_ / scatter_reduce_ amax): the grounded, coalesced COO state of
 * a chunk of L rules (b, rule l, entity e, v) is added into dense [K, B*E]
 * as, per (b, e), the sum over the chunk's rules in rule order of
 * v * W[l, k] (is_max = 0; one writer per slot, so the bits are the same on
 * every run), or maxed into it (is_max = 1; values >= 0: exact in any order,
 * no workspace needed).  Malformed states write nothing out of bounds: with
 * is_max = 0 a state that is not coalesced or holds an index outside
 * [B, L, E] adds nothing (the plan's error word, read on the device); with
 * is_max = 1 such entries are skipped.  No error is returned for them (that
 * would need a host read of device data). */
int fl_rule_accumulate(void *stream, const int64_t *sb, const int64_t *sl,
                       const int64_t *se, const float *sv, int64_t nnz,
                       const float *W, int64_t K, int64_t B, int64_t L,
                       int64_t E, int is_max, float *dense, void *ws,
                       size_t ws_bytes);

/* Replaces the finalization of rules/shared_inference.py:224-237: rowsum
 * [K*B] = per (rank, source) row sums (fixed order); total [B*E] = over ranks
 * in order, the sum (or max with final_max) of dense / max(rowsum, 1e-30)
 * at the nonzero entries. */
int fl_rule_finalize(void *stream, const float *dense, int64_t K, int64_t B,
                     int64_t E, int final_max, float *rowsum, float *total);

/* ---- evaluation --------------------------------------------------------- */

/* Replaces the rank computation of calculate_hits_full_with_filter_indices
 * (src/main.py:468-512, torch ops in the reference): state [B, E] fp32
 * dense scores, targets [B]; filter_keys (n_filter >= 0) the sorted unique
 * keys b*E + e of the filter with every (b, targets[b]) included, or none
 * (n_filter = 0: no filtering, as filter_indices=None).  ranks[b] =
 * greater + 1, or with use_eql greater + ((equal + 1) + 1) / 2, where
 * greater / equal count the unfiltered entities scoring above / exactly at
 * state[b, targets[b]] (fp32, exact below 2^24). */
int fl_dense_filtered_ranks(void *stream, const float *state, const int64_t *targets,
                            const int64_t *filter_keys, int64_t n_filter, int64_t B,
                            int64_t E, int use_eql, float *ranks);

/* Replaces the known-answer expansion of the filtered evaluation
 * (src/main.py:212-276, _expand_filter_side): per query q with key
 * keys[q] = source * R + relation, the columns (in CSR order) of that
 * (source, relation) group of one CSR side (its group pointers, relations,
 * starts, counts and columns), as (qpos[q], entity) pairs, queries in the
 * given order; a key with no group gives none.
 * fl_filter_expand_count writes off [Q+1] (exclusive offsets; off[Q] = the
 * number of pairs) using the workspace (fl_filter_expand_bytes); after the
 * host has read off[Q], fl_filter_expand_fill (same workspace) writes the
 * pairs. */
size_t fl_filter_expand_bytes(int64_t Q);
int fl_filter_expand_count(void *stream, const int32_t *gptr, const int16_t *grel,
                           const int32_t *gcount, int64_t nodes, const int64_t *keys,
                           int64_t R, int64_t Q, int64_t *off, void *ws,
                           size_t ws_bytes);
int fl_filter_expand_fill(void *stream, const int32_t *gstart, const int32_t *col,
                          int64_t Q, const int64_t *off, const int64_t *qpos,
                          int64_t total, const void *ws, int64_t *out_b,
                          int64_t *out_e);

/* Replaces the attention rank weights of extracted rule candidates
 * (rules/extract.py:65-135, _three_step_weights / collapsed_rule_weights)
 * and the row statistics of select_and_annotate_array (:148-201).
 * attention: [H, T, L, n] float (att_f64 = 0) or double; rows: int64
 * [N, W] = [length, op_1..op_T, ...] with trials at column W-8 and
 * positives at W-6; row_head: int64 [N] head of each row in [0, H) (NULL:
 * head 0).  mode 0: the 3-step closed form; 1: the dynamic program with
 * sums; 2: with maxima.  Writes rank_weights double [N, L]; rank_sums
 * (double [N], numpy's pairwise row sums; may be NULL) and precision
 * (double [N], positives / trials or 0; may be NULL).  *err (device int64)
 * is 1 when an operator lies outside [-n, n) (numpy's indexing) and 2 when
 * a row head lies outside [0, H); the weights of such rows are 0. */
int fl_rule_rank_weights(void *stream, const void *attention, int att_f64, int64_t H,
                         int64_t T, int64_t L, int64_t n, const int64_t *rows, int64_t N,
                         int64_t W, const int64_t *row_head, int64_t identity, int mode,
                         double *rank_weights, double *rank_sums, double *precision,
                         int64_t *err);
/* Row sums of a double [N, L] matrix (L <= 128) in numpy's pairwise order
 * (x.sum(axis=1) of fallback_rule_scores, rules/extract.py:141-145). */
int fl_row_pairwise_sums(void *stream, const double *x, int64_t N, int64_t L, double *out);

/* Workspace for fl_filtered_ranks (values_f64: 1 for double scores). */
size_t fl_filtered_ranks_workspace_bytes(int64_t B, int values_f64);

/* Replaces sparse2d_filtered_ranks_cuda (flashlog.cu:2754-2910; wrapper
 * flashlog_kernel.py:168-179).  Scores are a COO [B, E] matrix (idx_b,
 * idx_e, values of float or double); filter_keys are b*E + e, sorted
 * ascending.  truth[b] = the score of (b, targets[b]) or 0; over unfiltered
 * explicit entries: greater / equal / explicit counts; ranks[b] =
 * greater + (eq + 1) * 0.5 with eq = equal + (truth == 0 ? E - filtered -
 * explicit : 0) + 1 when use_eql, else greater + 1 (fp32, exact for counts
 * below 2^24).  Entries with idx_b outside [0, B) are ignored. */
int fl_filtered_ranks(void *stream, const int64_t *idx_b, const int64_t *idx_e,
                      const void *values, int values_f64,
                      const int64_t *targets, const int64_t *filter_keys,
                      int64_t nnz, int64_t n_filter, int64_t B, int64_t E,
                      int use_eql, float *ranks, void *workspace,
                      size_t workspace_bytes);

/* No counterpart in the reference.  fl_filtered_ranks without a workspace
 * argument, for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): its
 * scratch is a file-scope device array of fixed size (about 1.5 MiB, held by
 * every GPU the library runs on until the process ends), so at most
 * FL_RANKS_NOALLOC_MAX_B queries per call (larger B is refused with
 * FL_ERR_ARG).  It calls no allocator.  Every call on one GPU shares that
 * GPU's array (each call clears what it uses, with kernels), so calls that
 * overlap on one GPU -- on different streams or threads -- race. */
#define FL_RANKS_NOALLOC_MAX_B 65536
int fl_filtered_ranks_noalloc(void *stream, const int64_t *idx_b,
                              const int64_t *idx_e, const void *values,
                              int values_f64, const int64_t *targets,
                              const int64_t *filter_keys, int64_t nnz,
                              int64_t n_filter, int64_t B, int64_t E,
                              int use_eql, float *ranks);

/* ---- measurement ------------------------------------------------------ */

/* No reference counterpart (the reference's FLASHLOG_STAGE_TIMING,
 * flashlog_kernel.py:145-165, times whole stages with host syncs): per-kernel
 * HIP-event timing on the stream each kernel runs on.  fl_prof_enable(1)
 * starts recording and discards earlier records; fl_prof_read waits for the
 * recorded events of `kernel` and returns their summed duration (ms) and
 * launch count.  Single-threaded use only. */
int fl_prof_enable(int on);
int fl_prof_read(const char *kernel, double *total_ms, int64_t *launches);

/* ---- soft grounding (flashlog_kernel/soft_grounding_kernel) ---------- */

/* Replaces sample_relation_sources_reservoir (soft_grounding.cpp:1029-1124,
 * soft_grounding_kernel.py:87-112): per requested relation (relations
 * [nreq], unique, in [0, 32767]) a uniform reservoir of at most max_sources
 * rows holding a group of that relation, in CSR group order with SplitMix64
 * positions, then a SplitMix64 Fisher-Yates shuffle.  sampled
 * [nreq, max_sources] (-1 padded), available [nreq] = groups per relation.
 * All pointers are device memory. */
size_t fl_reservoir_bytes(int64_t groups, int64_t rows, int64_t nreq,
                          int64_t max_sources);
int fl_reservoir(void *stream, const int32_t *row_group_ptr, int64_t rows,
                 const int16_t *group_rel, int64_t groups,
                 const int64_t *relations, int64_t nreq, int64_t max_sources,
                 int64_t seed, void *ws, size_t ws_bytes, int32_t *sampled,
                 int64_t *available);

/* The CSR arrays the grounding walks read (the 16-tuple's entries 1, 5,
 * 8-15, soft_grounding_kernel.py:79). */
typedef struct fl_ground_graph {
    const int32_t *ori_col, *inv_col;
    const int32_t *ori_ptr, *ori_start, *ori_count;
    const int16_t *ori_rel;
    const int32_t *inv_ptr, *inv_start, *inv_count;
    const int16_t *inv_rel;
    int64_t nodes;          /* entities (ptr arrays hold nodes + 1)       */
    int64_t num_relations;  /* R: operators 0..2R-1, identity 2R          */
    int64_t max_groups;     /* most groups of one node on one side        */
    /* optional hub cache (nhub = 0 disables it): nodes with more than 64
       groups on a side get their transition options precomputed once per
       call for every (head, step, rank) instead of ranked at every visit */
    int64_t nhub;           /* hub nodes                                  */
    int64_t hub_options;    /* hub_off[nhub]                              */
    const int32_t *hub_id;  /* [nodes] hub index of a node, -1 for others */
    const int32_t *hub_node;/* [nhub] node of each hub                    */
    const int64_t *hub_off; /* [nhub+1] option slots of each hub (its
                               groups on both sides)                      */
} fl_ground_graph;

/* Replaces the walk part of ground_head_batch_source_folds_sampled_capped_
 * counts (soft_grounding.cpp:112-449, 898-1027) for rule_steps = 3: for
 * task t (head slot task_head[t], source task_source[t], position
 * task_index[t] within its fold) walks attention-guided walks with the
 * engine std::mt19937_64(splitmix64(seeds[h] ^ index << 32 ^ source)),
 * option masses proposal(w) = w^(1/temperature), the c2 edge prefix
 * topk_edges per side, the query head excluded from the source when
 * mask_query_head.  Record t*walks + j receives the body key (length << 60 |
 * three 20-bit operators; 0 when the walk stops or stays) and whether it
 * ends at a positive target of (source, head).  att: [nheads, 3, ranks,
 * 2R+1].  The draws are those of libstdc++ 11 (generate_canonical<double,
 * 64>, uniform_int_distribution by Lemire's method). */
size_t fl_ground_walk_bytes(const fl_ground_graph *g, int64_t ntasks,
                            int64_t nheads, int64_t ranks);
int fl_ground_walks(void *stream, const fl_ground_graph *g, const float *att,
                    int64_t nheads, int64_t ranks, const int64_t *heads,
                    const int64_t *seeds, int64_t ntasks,
                    const int32_t *task_head, const int64_t *task_source,
                    const int64_t *task_index, int64_t walks,
                    int64_t topk_edges, int mask_query_head,
                    double temperature, void *ws, size_t ws_bytes,
                    uint64_t *keys, uint8_t *positive);

/* Replaces merge_and_cap_source_stats and union_encoded_source_folds
 * (soft_grounding.cpp:454-614): records of segment s = (head, fold) are
 * tasks [seg_task_off[s], seg_task_off[s+1]) (segments head-major);
 * seg_head [nsegments] head slot; heads [nheads] head operators;
 * head_folds [nheads] folds per head; budgets (host int64[3]) per body
 * length.  rows [row_cap, 12] receives per head (in head order) the united
 * rows (length, 3 operators, totals of walk / source / positive walk /
 * positive source hits, their minimums over folds or 0 when a fold lacks
 * the body), ascending body key, trivial body (head) dropped; info (device
 * int64[nsegments + nheads + 1]) the unique bodies per fold, then the row
 * offsets of every head.  Synchronises the stream (sizes). */
size_t fl_ground_count_bytes(int64_t nrecords, int64_t nsegments,
                             int64_t nheads);
int fl_ground_count(void *stream, const uint64_t *keys,
                    const uint8_t *positive, int64_t walks,
                    int64_t nsegments, const int64_t *seg_task_off,
                    const int64_t *seg_head, int64_t nheads,
                    const int64_t *heads, const int64_t *head_folds,
                    const int64_t *budgets, void *ws, size_t ws_bytes,
                    int64_t *rows, int64_t row_cap, int64_t *info);

#ifdef __cplusplus
}
#endif

#endif /* FLASHLOG_HIP_H */
