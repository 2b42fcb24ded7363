/*
 * flashlog_oracle.c -- CPU restatement of FlashLog's propagation arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (flashlog_amd/) links,
 * loads or calls this file.  It is the checker that tests/, the smoke entry
 * point and bench.py's cpu_baseline leg compare the HIP path against.
 *
 * Every function restates the reference's algorithm in plain C, in the same
 * floating-point evaluation order, and cites the reference file:line it
 * follows (paths relative to the qikunxun/FlashLog tree):
 *
 *   or_build_side            flashlog_kernel/source/csr.cpp:12-69
 *   or_group_threshold       flashlog_kernel/source/flashlog.cpp:12-35
 *   or_dense_forward         flashlog_kernel/source/flashlog.cpp:38-89,151-211
 *   or_dense_backward        flashlog_kernel/source/flashlog.cpp:91-146,216-278
 *   or_dense_topc            flashlog_kernel/flashlog_kernel.py:814-842
 *   or_dense_max_forward     flashlog_kernel/source/flashlog.cu:104-121,523-637
 *   or_dense_max_backward    flashlog_kernel/source/flashlog.cu:639-726,1187-1255
 *   or_filtered_ranks        flashlog_kernel/source/flashlog.cu:2754-2910
 *   or_sparse_forward        flashlog_kernel/source/flashlog.cpp:1388-1486 (mode 0),
 *                            flashlog.cu:1743-1854 coordinates (mode 1)
 *   or_sparse_backward       flashlog_kernel/source/flashlog.cu:1856-1959
 *   or_quota_takes           flashlog_kernel/source/flashlog.cu:1433-1528 (training quotas)
 *   or_sparse_max_forward    flashlog_kernel/flashlog_kernel.py:399-478,1450-1626
 *   or_sparse_max_backward   flashlog_kernel/source/flashlog.cu:1918-1997,2364-2410
 *   or_sparse_normalize      flashlog_kernel/flashlog_kernel.py:551-555
 *
 * Pinning (how each function is checked, see tests/test_oracle_*.py):
 *   or_build_side, or_dense_forward, or_dense_backward: bit-compared against
 *     the reference's own CPU sources compiled into oracle/_ref/ (Makefile.ref),
 *     and against committed golden vectors produced from that build.
 *   or_group_threshold: brute force (expand groups to edges, sort) on tiny inputs.
 *   or_dense_topc: brute-force stable sort (value desc, entity asc) per row.
 *   or_dense_max_forward: brute-force max over edges with explicit tie rule.
 *   or_dense_max_backward: float64 brute force over the expanded edge list
 *     (each winner edge's partial derivatives), and finite differences.
 *   or_filtered_ranks: brute-force count over a dense score row.
 *   or_sparse_forward: bit-compared with the reference's flashlog_forward_sparse3d_sum_cpu
 *     (oracle/_ref) in mode 0 and, where the modes coincide, in mode 1; float64
 *     closed form over the expanded edge list.
 *   or_sparse_backward: element by element against the reference's
 *     flashlog_backward_sparse3d_sum_cpu (oracle/_ref, one thread): bit for bit
 *     with 0/1 masks, within 1e-6 with fractional ones; float64 adjoint of the
 *     closed form.
 *   or_quota_takes: the published SplitMix64 output sequence (seed 0); the
 *     closed form of the reference's own CPU quota rule (flashlog_kernel.py:
 *     1978-2003: floors + differences of the rounded capacity prefix) with
 *     the same phase; budget and capacity invariants.
 *   or_sparse_max_forward/backward: numpy brute force over the expanded item
 *     list (lexicographic sort by value, source, edge id, item order), the
 *     plain maximum where values are distinct, and constructed ties.
 *   or_sparse_normalize: closed form.
 *
 * Compile with -O2 -ffp-contract=off (no FMA contraction: the reference's
 * CPU build is ISO C++17 on x86-64 without -march, so it never fuses a*b+c).
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <math.h>

static int64_t or_lower_bound(const int64_t *a, int64_t n, int64_t key)
{
    int64_t lo = 0, hi = n;
    while (lo < hi) { int64_t mid = lo + (hi - lo) / 2; if (a[mid] < key) lo = mid + 1; else hi = mid; }
    return lo;
}

/* ------------------------------------------------------------------------ */
/* CSR side builder: csr.cpp:12-69.  Positions are ordered by (source,
 * relation, original edge id); groups are maximal runs of equal
 * (source, relation).  Group arrays must have capacity >= edges.          */
int or_build_side(int64_t edges, int64_t nodes,
                  const int64_t *source, const int64_t *target, const int64_t *relation,
                  int32_t *row_ptr, int32_t *columns, int16_t *edge_rel, int32_t *order,
                  int32_t *group_ptr, int16_t *group_rel, int32_t *group_start,
                  int32_t *group_count, int64_t *num_groups)
{
    int64_t relations = 0;
    for (int64_t i = 0; i < edges; ++i) {
        if (source[i] < 0 || source[i] >= nodes || target[i] < 0 || target[i] >= nodes ||
            relation[i] < 0 || relation[i] > 32767)
            return -1;
        if (relation[i] + 1 > relations) relations = relation[i] + 1;
    }
    /* stable bucket by relation, then stable bucket by source */
    int64_t nb = relations > nodes ? relations : nodes;
    int64_t *cur = (int64_t *)calloc((size_t)(nb + 1), sizeof(int64_t));
    int32_t *by_rel = (int32_t *)malloc((size_t)(edges > 0 ? edges : 1) * sizeof(int32_t));
    for (int64_t i = 0; i < edges; ++i) cur[relation[i]]++;
    int64_t acc = 0;
    for (int64_t r = 0; r < relations; ++r) { int64_t c = cur[r]; cur[r] = acc; acc += c; }
    for (int64_t i = 0; i < edges; ++i) by_rel[cur[relation[i]]++] = (int32_t)i;
    memset(cur, 0, (size_t)(nb + 1) * sizeof(int64_t));
    for (int64_t i = 0; i < edges; ++i) cur[source[i]]++;
    acc = 0;
    for (int64_t v = 0; v < nodes; ++v) { int64_t c = cur[v]; row_ptr[v] = (int32_t)acc; cur[v] = acc; acc += c; }
    row_ptr[nodes] = (int32_t)edges;
    for (int64_t k = 0; k < edges; ++k) { int32_t i = by_rel[k]; order[cur[source[i]]++] = i; }
    for (int64_t v = 0; v <= nodes; ++v) group_ptr[v] = 0;
    int64_t g = -1;
    for (int64_t j = 0; j < edges; ++j) {
        int32_t i = order[j];
        columns[j] = (int32_t)target[i];
        edge_rel[j] = (int16_t)relation[i];
        int fresh = (j == 0) || source[i] != source[order[j - 1]] || relation[i] != relation[order[j - 1]];
        if (fresh) {
            if (g >= 0) group_count[g] = (int32_t)(j - group_start[g]);
            ++g;
            group_start[g] = (int32_t)j;
            group_rel[g] = (int16_t)relation[i];
            group_ptr[source[i] + 1]++;
        }
    }
    if (g >= 0) group_count[g] = (int32_t)(edges - group_start[g]);
    for (int64_t v = 0; v < nodes; ++v) group_ptr[v + 1] += group_ptr[v];
    *num_groups = g + 1;
    free(cur);
    free(by_rel);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* c2 threshold: flashlog.cpp:12-35.  Groups [begin,end) of one source row;
 * weight of group g is weights[relations[g]].  Returns -1 when every
 * eligible (w > 0) edge fits in the budget; otherwise the weight theta of
 * the group holding the budget-th edge in weight-descending order, with
 * *remaining = budget - #edges of weight > theta.                          */
typedef struct { float w; int32_t c; } or_wc_f32;
typedef struct { double w; int32_t c; } or_wc_f64;

static int or_cmp_desc_f32(const void *a, const void *b)
{
    float x = ((const or_wc_f32 *)a)->w, y = ((const or_wc_f32 *)b)->w;
    return (x < y) - (x > y);
}
static int or_cmp_desc_f64(const void *a, const void *b)
{
    double x = ((const or_wc_f64 *)a)->w, y = ((const or_wc_f64 *)b)->w;
    return (x < y) - (x > y);
}

#define OR_DEFINE_THRESHOLD(T, SUF)                                                   \
T or_group_threshold_##SUF(const T *weights, const int16_t *relations,               \
                           const int32_t *sizes, int64_t begin, int64_t end,         \
                           int64_t budget, int64_t *remaining)                       \
{                                                                                     \
    int64_t cnt = 0, total = 0;                                                       \
    or_wc_##SUF *buf = (or_wc_##SUF *)malloc((size_t)((end - begin) > 0 ? (end - begin) : 1) * sizeof(or_wc_##SUF)); \
    for (int64_t g = begin; g < end; ++g) {                                           \
        T s = weights[relations[g]];                                                  \
        if (s > (T)0) { buf[cnt].w = s; buf[cnt].c = sizes[g]; ++cnt; total += sizes[g]; } \
    }                                                                                 \
    *remaining = 0;                                                                   \
    if (total <= budget) { free(buf); return (T)-1; }                                 \
    qsort(buf, (size_t)cnt, sizeof(or_wc_##SUF), or_cmp_desc_##SUF);                  \
    int64_t consumed = 0, higher = 0;                                                 \
    T previous = (T)-1;                                                               \
    for (int64_t k = 0; k < cnt; ++k) {                                               \
        if (buf[k].w != previous) { higher = consumed; previous = buf[k].w; }         \
        if (consumed + buf[k].c >= budget) {                                          \
            *remaining = budget - higher; T th = buf[k].w; free(buf); return th;      \
        }                                                                             \
        consumed += buf[k].c;                                                         \
    }                                                                                 \
    free(buf);                                                                        \
    return (T)-1;                                                                     \
}
OR_DEFINE_THRESHOLD(float, f32)
OR_DEFINE_THRESHOLD(double, f64)

/* Per-group take under the threshold: flashlog.cpp:61-77 (forward) and
 * :117-133 (backward).  Groups of weight == theta consume a shared quota in
 * group order; masked edges still consume it (mask is applied per edge).   */
#define OR_TAKE(T)                                                                    \
    int32_t take = w_val > (T)0 ? group_edge_count[g] : 0;                            \
    if (take > 0 && threshold_weight >= 0) {                                          \
        if (w_val < threshold_weight) take = 0;                                       \
        else if (w_val == threshold_weight) {                                         \
            int64_t left = keep_in_threshold - threshold_seen;                        \
            take = left > 0 ? (int32_t)(left < group_edge_count[g] ? left : group_edge_count[g]) : 0; \
            threshold_seen += take;                                                   \
        }                                                                             \
    }

#define OR_DEFINE_DENSE(T, SUF)                                                       \
static void or_forward_row_##SUF(int64_t src, int64_t bl, T a_val, const T *w,        \
    const int32_t *row_group_ptr, const int16_t *group_rel,                           \
    const int32_t *group_edge_start, const int32_t *group_edge_count,                 \
    const int32_t *col_ind, const T *mask, T *out, int64_t topk_edges,                \
    int64_t E, int64_t n, int64_t rel_offset)                                         \
{                                                                                     \
    int64_t g0 = row_group_ptr[src], g1 = row_group_ptr[src + 1];                     \
    int64_t keep_in_threshold = 0;                                                    \
    T threshold_weight = or_group_threshold_##SUF(w + bl * n + rel_offset, group_rel, \
        group_edge_count, g0, g1, topk_edges, &keep_in_threshold);                    \
    int64_t threshold_seen = 0;                                                       \
    for (int64_t g = g0; g < g1; ++g) {                                               \
        int64_t rel = group_rel[g];                                                   \
        T w_val = w[bl * n + rel_offset + rel];                                       \
        OR_TAKE(T)                                                                    \
        if (take <= 0) continue;                                                      \
        int64_t s = group_edge_start[g];                                              \
        for (int64_t p = s; p < s + take; ++p) {                                      \
            T m = mask[p];                                                            \
            if (m == 0) continue;                                                     \
            T prod = a_val * w_val;                                                   \
            prod = prod * m;                                                          \
            out[bl * E + col_ind[p]] += prod;                                         \
        }                                                                             \
    }                                                                                 \
}                                                                                     \
                                                                                      \
static void or_backward_row_##SUF(int64_t src, int64_t bl, const T *grad_out,         \
    const T *A, const T *w, const int32_t *row_group_ptr, const int16_t *group_rel,   \
    const int32_t *group_edge_start, const int32_t *group_edge_count,                 \
    const int32_t *col_ind, const T *mask, T *gA, T *gw, int64_t topk_edges,          \
    int64_t E, int64_t n, int64_t rel_offset)                                         \
{                                                                                     \
    int64_t g0 = row_group_ptr[src], g1 = row_group_ptr[src + 1];                     \
    int64_t keep_in_threshold = 0;                                                    \
    T threshold_weight = or_group_threshold_##SUF(w + bl * n + rel_offset, group_rel, \
        group_edge_count, g0, g1, topk_edges, &keep_in_threshold);                    \
    T a_val = A[bl * E + src];                                                        \
    int64_t threshold_seen = 0;                                                       \
    for (int64_t g = g0; g < g1; ++g) {                                               \
        int64_t rel = group_rel[g];                                                   \
        T w_val = w[bl * n + rel_offset + rel];                                       \
        OR_TAKE(T)                                                                    \
        if (take <= 0) continue;                                                      \
        int64_t s = group_edge_start[g];                                              \
        for (int64_t p = s; p < s + take; ++p) {                                      \
            T m = mask[p];                                                            \
            if (m == 0) continue;                                                     \
            T go = grad_out[bl * E + col_ind[p]];                                     \
            if (go == 0) continue;                                                    \
            T t1 = go * w_val; t1 = t1 * m;                                           \
            gA[bl * E + src] += t1;                                                   \
            T t2 = go * a_val; t2 = t2 * m;                                           \
            gw[bl * n + rel_offset + rel] += t2;                                      \
        }                                                                             \
    }                                                                                 \
}                                                                                     \
                                                                                      \
void or_dense_forward_##SUF(int64_t BL, int64_t E, int64_t n, const T *A, const T *w, \
    const int64_t *active, int64_t num_active,                                        \
    const int32_t *ori_col, const T *ori_mask, const int32_t *ori_gptr,               \
    const int16_t *ori_grel, const int32_t *ori_gstart, const int32_t *ori_gcount,    \
    const int32_t *inv_col, const T *inv_mask, const int32_t *inv_gptr,               \
    const int16_t *inv_grel, const int32_t *inv_gstart, const int32_t *inv_gcount,    \
    int64_t r_size, int wot_i, int64_t topk_edges, T *out_ind, T *out_ori, T *out_inv) \
{                                                                                     \
    for (int64_t i = 0; i < BL * E; ++i) { out_ori[i] = 0; out_inv[i] = 0; }          \
    for (int64_t bl = 0; bl < BL; ++bl) {                                             \
        T wid = w[bl * n + (n - 1)];                                                  \
        for (int64_t e = 0; e < E; ++e)                                               \
            out_ind[bl * E + e] = wot_i ? (T)0 : A[bl * E + e] * wid;                 \
    }                                                                                 \
    for (int64_t ai = 0; ai < num_active; ++ai) {                                     \
        int64_t src = active[ai];                                                     \
        for (int64_t bl = 0; bl < BL; ++bl) {                                         \
            T a_val = A[bl * E + src];                                                \
            if (a_val == 0) continue;                                                 \
            or_forward_row_##SUF(src, bl, a_val, w, ori_gptr, ori_grel, ori_gstart,   \
                ori_gcount, ori_col, ori_mask, out_ori, topk_edges, E, n, 0);         \
            or_forward_row_##SUF(src, bl, a_val, w, inv_gptr, inv_grel, inv_gstart,   \
                inv_gcount, inv_col, inv_mask, out_inv, topk_edges, E, n, r_size);    \
        }                                                                             \
    }                                                                                 \
}                                                                                     \
                                                                                      \
void or_dense_backward_##SUF(int64_t BL, int64_t E, int64_t n,                        \
    const T *grad_ind, const T *grad_ori, const T *grad_inv, const T *A, const T *w,  \
    const int64_t *active, int64_t num_active,                                        \
    const int32_t *ori_col, const T *ori_mask, const int32_t *ori_gptr,               \
    const int16_t *ori_grel, const int32_t *ori_gstart, const int32_t *ori_gcount,    \
    const int32_t *inv_col, const T *inv_mask, const int32_t *inv_gptr,               \
    const int16_t *inv_grel, const int32_t *inv_gstart, const int32_t *inv_gcount,    \
    int64_t r_size, int wot_i, int64_t topk_edges, T *gA, T *gw)                      \
{                                                                                     \
    for (int64_t i = 0; i < BL * E; ++i) gA[i] = 0;                                   \
    for (int64_t i = 0; i < BL * n; ++i) gw[i] = 0;                                   \
    if (!wot_i) {                                                                     \
        for (int64_t bl = 0; bl < BL; ++bl) {                                         \
            T wid = w[bl * n + (n - 1)];                                              \
            T acc = 0;                                                                \
            for (int64_t e = 0; e < E; ++e) {                                         \
                T gi = grad_ind[bl * E + e];                                          \
                gA[bl * E + e] += gi * wid;                                           \
                acc += gi * A[bl * E + e];                                            \
            }                                                                         \
            gw[bl * n + (n - 1)] += acc;                                              \
        }                                                                             \
    }                                                                                 \
    for (int64_t ai = 0; ai < num_active; ++ai) {                                     \
        int64_t src = active[ai];                                                     \
        for (int64_t bl = 0; bl < BL; ++bl) {                                         \
            if (A[bl * E + src] == 0) continue;                                       \
            or_backward_row_##SUF(src, bl, grad_ori, A, w, ori_gptr, ori_grel,        \
                ori_gstart, ori_gcount, ori_col, ori_mask, gA, gw, topk_edges, E, n, 0); \
            or_backward_row_##SUF(src, bl, grad_inv, A, w, inv_gptr, inv_grel,        \
                inv_gstart, inv_gcount, inv_col, inv_mask, gA, gw, topk_edges, E, n, r_size); \
        }                                                                             \
    }                                                                                 \
}
OR_DEFINE_DENSE(float, f32)
OR_DEFINE_DENSE(double, f64)

/* ------------------------------------------------------------------------ */
/* c1 entity budget on a dense state: flashlog_kernel.py:814-842.
 * Per row: when #nonzero > c, keep the c largest nonzeros; at the cutoff
 * value keep the earliest entities (cumsum rule, :835-840); the result is
 * A * keep (so a dropped entry becomes A*0.0f).  Rows at or under the
 * budget are untouched.  When no row is over budget the input is returned
 * unchanged, which *changed == 0 reports.  Also returns per-row cutoff
 * value and the last kept tied entity (E when every tie is kept; -1 for a
 * row under budget) so the GPU's selection can be compared directly.     */
typedef struct { float v; int32_t e; } or_ve;
static int or_cmp_ve(const void *a, const void *b)
{
    const or_ve *x = (const or_ve *)a, *y = (const or_ve *)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return (x->e > y->e) - (x->e < y->e);
}

int or_dense_topc(int64_t BL, int64_t E, int64_t c, const float *A, float *out,
                  float *cutoff, int32_t *last_tie, int *changed)
{
    *changed = 0;
    memcpy(out, A, (size_t)(BL * E) * sizeof(float));
    if (c < 0) return -1;
    if (c >= E) { for (int64_t r = 0; r < BL; ++r) { cutoff[r] = 0.f; last_tie[r] = -1; } return 0; }
    or_ve *buf = (or_ve *)malloc((size_t)(E > 0 ? E : 1) * sizeof(or_ve));
    unsigned char *over = (unsigned char *)calloc((size_t)(BL > 0 ? BL : 1), 1);
    unsigned char *keep = (unsigned char *)malloc((size_t)(E > 0 ? E : 1));
    int any = 0;
    for (int64_t r = 0; r < BL; ++r) {
        int64_t nz = 0;
        for (int64_t e = 0; e < E; ++e) if (A[r * E + e] != 0) ++nz;
        over[r] = nz > c;
        any |= over[r];
        cutoff[r] = 0.f;
        last_tie[r] = -1;
    }
    if (!any) { free(buf); free(over); free(keep); return 0; }
    *changed = 1;
    for (int64_t r = 0; r < BL; ++r) {
        const float *row = A + r * E;
        if (!over[r]) {
            for (int64_t e = 0; e < E; ++e) out[r * E + e] = row[e] * 1.0f;
            continue;
        }
        if (c == 0) {
            for (int64_t e = 0; e < E; ++e) out[r * E + e] = row[e] * 0.0f;
            continue;
        }
        int64_t k = 0;
        for (int64_t e = 0; e < E; ++e) if (row[e] != 0) { buf[k].v = row[e]; buf[k].e = (int32_t)e; ++k; }
        qsort(buf, (size_t)k, sizeof(or_ve), or_cmp_ve);
        float cut = buf[c - 1].v;
        int64_t above = 0, tied_total = 0;
        for (int64_t e = 0; e < E; ++e) {
            if (row[e] == 0) continue;
            if (row[e] > cut) ++above; else if (row[e] == cut) ++tied_total;
        }
        int64_t remaining = c - above, seen = 0;
        int32_t last = -1;
        for (int64_t e = 0; e < E; ++e) {
            int kp = 0;
            if (row[e] != 0) {
                if (row[e] > cut) kp = 1;
                else if (row[e] == cut) { ++seen; if (seen <= remaining) { kp = 1; last = (int32_t)e; } }
            }
            keep[e] = (unsigned char)kp;
        }
        cutoff[r] = cut;
        last_tie[r] = (remaining >= tied_total) ? (int32_t)E : last;
        for (int64_t e = 0; e < E; ++e) out[r * E + e] = row[e] * (keep[e] ? 1.0f : 0.0f);
    }
    free(buf); free(over); free(keep);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Dense max aggregation forward: flashlog.cu:104-121 (packed (value, -p)
 * CAS max: larger value wins, ties go to the smaller CSR position p) with
 * the same source admission and c2 quota as the sum path (flashlog.cu:523-637).
 * Untouched outputs are 0 with arg -1 (flashlog.cu:123-135: packed 0 means
 * no contribution).  The comparison is on the raw float bits, as the
 * reference packs __float_as_uint(value) in the high word.                  */
static void or_max_row(int64_t src, int64_t bl, float a_val, const float *w,
    const int32_t *gptr, const int16_t *grel, const int32_t *gstart, const int32_t *gcount,
    const int32_t *col, const float *mask, uint64_t *packed, int64_t topk_edges,
    int64_t E, int64_t n, int64_t off)
{
    int64_t g0 = gptr[src], g1 = gptr[src + 1];
    int64_t keep_in_threshold = 0;
    float threshold_weight = or_group_threshold_f32(w + bl * n + off, grel, gcount, g0, g1,
                                                    topk_edges, &keep_in_threshold);
    int64_t threshold_seen = 0;
    for (int64_t g = g0; g < g1; ++g) {
        int32_t *group_edge_count = (int32_t *)gcount;
        float w_val = w[bl * n + off + grel[g]];
        OR_TAKE(float)
        if (take <= 0) continue;
        float prod = a_val * w_val;
        for (int64_t p = gstart[g]; p < gstart[g] + take; ++p) {
            float m = mask[p];
            if (m == 0) continue;
            float v = prod * m;
            uint32_t bits; memcpy(&bits, &v, 4);
            uint64_t cand = ((uint64_t)bits << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)p);
            uint64_t *slot = &packed[bl * E + col[p]];
            if (cand > *slot) *slot = cand;
        }
    }
}

void or_dense_max_forward(int64_t BL, int64_t E, int64_t n, const float *A, const float *w,
    const int64_t *active, int64_t num_active,
    const int32_t *ori_col, const float *ori_mask, const int32_t *ori_gptr,
    const int16_t *ori_grel, const int32_t *ori_gstart, const int32_t *ori_gcount,
    const int32_t *inv_col, const float *inv_mask, const int32_t *inv_gptr,
    const int16_t *inv_grel, const int32_t *inv_gstart, const int32_t *inv_gcount,
    int64_t r_size, int wot_i, int64_t topk_edges,
    float *out_ind, float *out_ori, float *out_inv, int64_t *ori_arg, int64_t *inv_arg)
{
    uint64_t *po = (uint64_t *)calloc((size_t)(BL * E > 0 ? BL * E : 1), 8);
    uint64_t *pi = (uint64_t *)calloc((size_t)(BL * E > 0 ? BL * E : 1), 8);
    for (int64_t bl = 0; bl < BL; ++bl) {
        float wid = w[bl * n + (n - 1)];
        for (int64_t e = 0; e < E; ++e) out_ind[bl * E + e] = wot_i ? 0.f : A[bl * E + e] * wid;
    }
    for (int64_t ai = 0; ai < num_active; ++ai) {
        int64_t src = active[ai];
        for (int64_t bl = 0; bl < BL; ++bl) {
            float a = A[bl * E + src];
            if (a == 0) continue;
            or_max_row(src, bl, a, w, ori_gptr, ori_grel, ori_gstart, ori_gcount, ori_col,
                       ori_mask, po, topk_edges, E, n, 0);
            or_max_row(src, bl, a, w, inv_gptr, inv_grel, inv_gstart, inv_gcount, inv_col,
                       inv_mask, pi, topk_edges, E, n, r_size);
        }
    }
    for (int64_t i = 0; i < BL * E; ++i) {
        uint32_t hb = (uint32_t)(po[i] >> 32); memcpy(&out_ori[i], &hb, 4);
        ori_arg[i] = po[i] == 0 ? -1 : (int64_t)(int32_t)(0xFFFFFFFFu - (uint32_t)(po[i] & 0xFFFFFFFFu));
        hb = (uint32_t)(pi[i] >> 32); memcpy(&out_inv[i], &hb, 4);
        inv_arg[i] = pi[i] == 0 ? -1 : (int64_t)(int32_t)(0xFFFFFFFFu - (uint32_t)(pi[i] & 0xFFFFFFFFu));
    }
    free(po); free(pi);
}

/* Winner-only max backward: flashlog.cu:639-726 (kernel) and 1187-1255
 * (host), in a sequential order: identity gA = g_ind * w[n-1] and gw[n-1] =
 * sum over entities (ascending) of g_ind * A, then for active sources
 * (ascending), rows, ORI then INV kept edges in CSR order: an edge p whose
 * destination's arg is p adds (go*w)*m to gA[bl, src] and (go*a)*m to
 * gw[bl, off + rel].  (The reference adds the winner terms with atomics.)  */
static void or_max_bwd_row(int64_t src, int64_t bl, float a_val, const float *w,
    const int32_t *gptr, const int16_t *grel, const int32_t *gstart, const int32_t *gcount,
    const int32_t *col, const float *mask, const float *grad, const int64_t *arg,
    float *gA, float *gw, int64_t topk_edges, int64_t E, int64_t n, int64_t off)
{
    int64_t g0 = gptr[src], g1 = gptr[src + 1];
    int64_t keep_in_threshold = 0;
    float threshold_weight = or_group_threshold_f32(w + bl * n + off, grel, gcount, g0, g1,
                                                    topk_edges, &keep_in_threshold);
    int64_t threshold_seen = 0;
    for (int64_t g = g0; g < g1; ++g) {
        int32_t *group_edge_count = (int32_t *)gcount;
        float w_val = w[bl * n + off + grel[g]];
        OR_TAKE(float)
        if (take <= 0) continue;
        for (int64_t p = gstart[g]; p < gstart[g] + take; ++p) {
            float m = mask[p];
            if (m == 0) continue;
            int64_t dst = col[p];
            if (arg[bl * E + dst] != p) continue;
            float go = grad[bl * E + dst];
            if (go == 0) continue;
            gA[bl * E + src] += (go * w_val) * m;
            gw[bl * n + off + grel[g]] += (go * a_val) * m;
        }
    }
}

void or_dense_max_backward(int64_t BL, int64_t E, int64_t n, const float *A, const float *w,
    const float *grad_ind, const float *grad_ori, const float *grad_inv,
    const int64_t *ori_arg, const int64_t *inv_arg,
    const int64_t *active, int64_t num_active,
    const int32_t *ori_col, const float *ori_mask, const int32_t *ori_gptr,
    const int16_t *ori_grel, const int32_t *ori_gstart, const int32_t *ori_gcount,
    const int32_t *inv_col, const float *inv_mask, const int32_t *inv_gptr,
    const int16_t *inv_grel, const int32_t *inv_gstart, const int32_t *inv_gcount,
    int64_t r_size, int wot_i, int64_t topk_edges, float *gA, float *gw)
{
    memset(gA, 0, sizeof(float) * (size_t)(BL * E));
    memset(gw, 0, sizeof(float) * (size_t)(BL * n));
    if (!wot_i) {
        for (int64_t bl = 0; bl < BL; ++bl) {
            float wid = w[bl * n + (n - 1)], acc = 0.0f;
            for (int64_t e = 0; e < E; ++e) {
                gA[bl * E + e] = grad_ind[bl * E + e] * wid;
                acc += grad_ind[bl * E + e] * A[bl * E + e];
            }
            gw[bl * n + (n - 1)] = acc;
        }
    }
    for (int64_t ai = 0; ai < num_active; ++ai) {
        int64_t src = active[ai];
        for (int64_t bl = 0; bl < BL; ++bl) {
            float a = A[bl * E + src];
            if (a == 0) continue;
            or_max_bwd_row(src, bl, a, w, ori_gptr, ori_grel, ori_gstart, ori_gcount, ori_col, ori_mask,
                           grad_ori, ori_arg, gA, gw, topk_edges, E, n, 0);
            or_max_bwd_row(src, bl, a, w, inv_gptr, inv_grel, inv_gstart, inv_gcount, inv_col, inv_mask,
                           grad_inv, inv_arg, gA, gw, topk_edges, E, n, r_size);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Sparse (COO) sum hop.
 * mode 0 (top-k): flashlog.cpp:1388-1486 (rowwise branch of the CPU sum and
 *   sum+norm paths): rows in order; per row its entries in input order; per
 *   entry ORI kept edges with a nonzero mask (CSR order), then INV, then the
 *   identity term (unless wot_i); a destination's first contribution is
 *   added to 0.  value = (v * w) * m; identity = v * w[n-1].
 * mode 1 (all edges): flashlog.cu:1743-1854 coordinates (every edge of every
 *   group, masked or not, any weight, plus identity) added in the same order.
 * Output: keys row*E + e ascending with their values; returns the count, or
 * -1 when cap is too small.                                                 */
typedef struct {
    const int32_t *col; const float *mask; const int32_t *gptr; const int16_t *grel;
    const int32_t *gstart; const int32_t *gcount; const int32_t *order;
} or_side_t;

/* SplitMix64 output function (Steele, Lea and Flood 2014; public-domain
 * splitmix64.c): one step from state z. */
uint64_t or_splitmix64(uint64_t z)
{
    z += 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

/* Training quotas of one (entry, side): flashlog.cu:1433-1528, sequentially
 * in group order.  weights[k] / counts[k] are group k's attention weight and
 * edge count; takes[k] receives its kept edge count.                        */
void or_quota_takes(int64_t ngroups, const float *weights, const int32_t *counts, int64_t topk_edges,
                    int64_t b, int64_t l, int64_t src, int is_inv, int64_t seed, int32_t *takes)
{
    int64_t capacity = 0;
    double weight_sum = 0.0;
    for (int64_t g = 0; g < ngroups; ++g) {
        double weight = weights[g];
        if (weight > 0 && counts[g] > 0) { capacity += counts[g]; weight_sum += weight; }
    }
    int64_t target = topk_edges < capacity ? topk_edges : capacity;
    int64_t allocated = capacity;
    if (target < capacity) {
        allocated = 0;
        for (int64_t g = 0; g < ngroups; ++g) {
            double weight = weights[g];
            int64_t count = counts[g];
            if (weight > 0 && count > 0)
                allocated += (int64_t)fmin((double)count, floor((double)target * weight / weight_sum));
        }
    }
    int64_t residual = target - allocated, spare_total = capacity - allocated;
    int64_t left = residual, capacity_left = spare_total, prefix = 0;
    uint64_t z = (uint64_t)seed ^ ((uint64_t)b * 0x9e3779b97f4a7c15ULL) ^ ((uint64_t)l * 0xbf58476d1ce4e5b9ULL) ^
                 ((uint64_t)src * 0x94d049bb133111ebULL) ^ (is_inv ? 0xd1b54a32d192ed03ULL : 0x8cb92baa3f3d8dd7ULL);
    double phase = (double)(or_splitmix64(z) >> 11) * 0x1.0p-53;
    for (int64_t g = 0; g < ngroups; ++g) {
        float score = weights[g];
        int32_t cnt = counts[g];
        int32_t take = score > 0.0f ? cnt : 0;
        if (take > 0 && spare_total > 0) {
            int64_t base = (int64_t)fmin((double)cnt, floor((double)target * (double)score / weight_sum));
            int64_t spare = (int64_t)cnt - base;
            prefix += spare;
            capacity_left -= spare;
            int64_t cumulative = prefix == spare_total ? residual
                : (int64_t)floor((double)residual * (double)prefix / (double)spare_total + phase);
            int64_t extra = cumulative - (residual - left);
            if (extra > left) extra = left;
            if (extra > spare) extra = spare;
            if (extra < 0) extra = 0;
            if (extra < left - capacity_left) extra = left - capacity_left;
            left -= extra;
            take = (int32_t)(base + extra);
        }
        takes[g] = take;
    }
}

/* Item callback: dir 0 ORI, 1 INV, 2 identity (p = edge = -1, rel = -1);
 * edge = the original edge id (order[p]) when the side has an order array. */
typedef void (*or_item_fn)(void *ctx, int64_t entry, int dir, int64_t p, int64_t edge, int64_t dst, int rel, float m,
                           float value);

/* Walks the items of one entry in raw order.  mode 0 (top-k): kept edges by
 * the c2 threshold (seed < 0) or the training quotas (seed >= 0); masked kept
 * edges are skipped unless keep_masked (the max keeps them as 0-valued
 * items).  mode 1: every edge of every group. */
static void or_sparse_walk(int mode, int keep_masked, int64_t seed, int64_t i, const int64_t *sb, const int64_t *sl,
                           const int64_t *se, const float *sv, int64_t L, const float *w, int64_t n,
                           const or_side_t *sides, int64_t r_size, int wot_i, int64_t topk_edges, or_item_fn fn,
                           void *ctx)
{
    int64_t row = sb[i] * L + sl[i], src = se[i];
    const float *w_bl = w + row * n;
    for (int dir = 0; dir < 2; ++dir) {
        const or_side_t *sd = &sides[dir];
        int64_t off = dir ? r_size : 0;
        int64_t g0 = sd->gptr[src], g1 = sd->gptr[src + 1];
        if (g0 == g1) continue;
        int64_t keep_in_threshold = 0;
        float threshold_weight = -1.0f;
        int32_t *quota = NULL;
        if (mode == 0 && seed >= 0 && topk_edges > 0) {
            float *wg = (float *)malloc(sizeof(float) * (size_t)(g1 - g0));
            quota = (int32_t *)malloc(sizeof(int32_t) * (size_t)(g1 - g0));
            for (int64_t g = g0; g < g1; ++g) wg[g - g0] = w_bl[off + sd->grel[g]];
            or_quota_takes(g1 - g0, wg, sd->gcount + g0, topk_edges, sb[i], sl[i], src, dir, seed, quota);
            free(wg);
        } else if (mode == 0) {
            threshold_weight = or_group_threshold_f32(w_bl + off, sd->grel, sd->gcount, g0, g1, topk_edges,
                                                      &keep_in_threshold);
        }
        int64_t threshold_seen = 0;
        for (int64_t g = g0; g < g1; ++g) {
            int32_t *group_edge_count = (int32_t *)sd->gcount;
            float w_val = w_bl[off + sd->grel[g]];
            int32_t kept;
            if (mode == 0) {
                if (quota) {
                    kept = quota[g - g0];
                } else {
                    OR_TAKE(float)
                    kept = take;
                }
                if (kept <= 0) continue;
                for (int64_t p = sd->gstart[g]; p < sd->gstart[g] + kept; ++p) {
                    float m = sd->mask[p];
                    if (m == 0 && !keep_masked) continue;
                    fn(ctx, i, dir, p, sd->order ? sd->order[p] : -1, sd->col[p], sd->grel[g], m,
                       sv[i] * w_val * m);
                }
            } else {
                kept = group_edge_count[g];
                float gp = sv[i] * w_val;
                for (int64_t p = sd->gstart[g]; p < sd->gstart[g] + kept; ++p) {
                    float m = sd->mask[p];
                    fn(ctx, i, dir, p, sd->order ? sd->order[p] : -1, sd->col[p], sd->grel[g], m, gp * m);
                }
            }
        }
        free(quota);
    }
    if (!wot_i) fn(ctx, i, 2, -1, -1, src, -1, 1.0f, sv[i] * w_bl[n - 1]);
}

typedef struct { float *acc; int64_t *mark; int64_t *touched; int64_t ntouched; int64_t stamp; } or_acc_t;

static void or_acc_item(void *ctx, int64_t entry, int dir, int64_t p, int64_t edge, int64_t dst, int rel, float m,
                        float value)
{
    or_acc_t *a = (or_acc_t *)ctx;
    (void)entry; (void)dir; (void)p; (void)edge; (void)rel; (void)m;
    if (a->mark[dst] != a->stamp) {
        a->mark[dst] = a->stamp;
        a->acc[dst] = 0.0f;
        a->touched[a->ntouched++] = dst;
    }
    a->acc[dst] += value;
}

static int or_cmp_i64(const void *x, const void *y)
{
    int64_t a = *(const int64_t *)x, b = *(const int64_t *)y;
    return a < b ? -1 : a > b;
}

#define OR_SIDES                                                                                    \
    or_side_t sides[2] = {{ori_col, ori_mask, ori_gptr, ori_grel, ori_gstart, ori_gcount, ori_order}, \
                          {inv_col, inv_mask, inv_gptr, inv_grel, inv_gstart, inv_gcount, inv_order}}

int64_t or_sparse_forward(int mode, int64_t nnz, const int64_t *sb, const int64_t *sl, const int64_t *se,
    const float *sv, int64_t B, int64_t L, int64_t E, const float *w, int64_t n,
    const int32_t *ori_col, const float *ori_mask, const int32_t *ori_gptr, const int16_t *ori_grel,
    const int32_t *ori_gstart, const int32_t *ori_gcount,
    const int32_t *inv_col, const float *inv_mask, const int32_t *inv_gptr, const int16_t *inv_grel,
    const int32_t *inv_gstart, const int32_t *inv_gcount,
    int64_t r_size, int wot_i, int64_t topk_edges, int64_t seed, int64_t cap, int64_t *out_key, float *out_v)
{
    const int32_t *ori_order = NULL, *inv_order = NULL;
    OR_SIDES;
    or_acc_t a;
    a.acc = (float *)calloc((size_t)(E > 0 ? E : 1), sizeof(float));
    a.mark = (int64_t *)malloc((size_t)(E > 0 ? E : 1) * sizeof(int64_t));
    a.touched = (int64_t *)malloc((size_t)(E > 0 ? E : 1) * sizeof(int64_t));
    for (int64_t e = 0; e < E; ++e) a.mark[e] = -1;
    int64_t total = 0;
    for (int64_t row = 0; row < B * L; ++row) {
        a.ntouched = 0;
        a.stamp = row;
        for (int64_t i = 0; i < nnz; ++i)
            if (sb[i] * L + sl[i] == row)
                or_sparse_walk(mode, 0, seed, i, sb, sl, se, sv, L, w, n, sides, r_size, wot_i, topk_edges,
                               or_acc_item, &a);
        qsort(a.touched, (size_t)a.ntouched, sizeof(int64_t), or_cmp_i64);
        if (total + a.ntouched > cap) { total = -1; break; }
        for (int64_t k = 0; k < a.ntouched; ++k) {
            out_key[total + k] = row * E + a.touched[k];
            out_v[total + k] = a.acc[a.touched[k]];
        }
        total += a.ntouched;
    }
    free(a.acc); free(a.mark); free(a.touched);
    return total;
}

/* Backward of the sparse hop (flashlog.cu:1856-1959 semantics, sequential
 * order): grad_v[i] = sum over entry i's items of (g*m)*w, then + g*w[n-1]
 * for the identity item; grad_w[row, off+rel] += (g*m)*v and
 * grad_w[row, n-1] += g*v.  g is grad_out at the item's output key.        */
typedef struct {
    const int64_t *out_key; int64_t nout; const float *grad; const float *w; const float *sv;
    const int64_t *sb, *sl; int64_t L, E, n, r_size; float *grad_v; float *grad_w; float gsp;
} or_bwd_t;

static void or_bwd_item(void *ctx, int64_t entry, int dir, int64_t p, int64_t edge, int64_t dst, int rel, float m,
                        float value)
{
    or_bwd_t *c = (or_bwd_t *)ctx;
    (void)p; (void)edge; (void)value;
    int64_t row = c->sb[entry] * c->L + c->sl[entry];
    int64_t key = row * c->E + dst;
    int64_t pos = or_lower_bound(c->out_key, c->nout, key);
    float gv = (pos < c->nout && c->out_key[pos] == key) ? c->grad[pos] : 0.0f;
    if (dir == 2) {
        c->gsp += gv * c->w[row * c->n + c->n - 1];
        c->grad_w[row * c->n + c->n - 1] += gv * c->sv[entry];
        return;
    }
    int64_t col = (dir ? c->r_size : 0) + rel;
    c->gsp += gv * m * c->w[row * c->n + col];
    c->grad_w[row * c->n + col] += gv * m * c->sv[entry];
}

void or_sparse_backward(int mode, int64_t nnz, const int64_t *sb, const int64_t *sl, const int64_t *se,
    const float *sv, int64_t B, int64_t L, int64_t E, const float *w, int64_t n,
    const int32_t *ori_col, const float *ori_mask, const int32_t *ori_gptr, const int16_t *ori_grel,
    const int32_t *ori_gstart, const int32_t *ori_gcount,
    const int32_t *inv_col, const float *inv_mask, const int32_t *inv_gptr, const int16_t *inv_grel,
    const int32_t *inv_gstart, const int32_t *inv_gcount,
    int64_t r_size, int wot_i, int64_t topk_edges, int64_t seed, const int64_t *out_key, int64_t nout,
    const float *grad_out, float *grad_v, float *grad_w)
{
    const int32_t *ori_order = NULL, *inv_order = NULL;
    OR_SIDES;
    or_bwd_t c = {out_key, nout, grad_out, w, sv, sb, sl, L, E, n, r_size, grad_v, grad_w, 0.0f};
    memset(grad_w, 0, sizeof(float) * (size_t)(B * L * n));
    for (int64_t i = 0; i < nnz; ++i) {
        c.gsp = 0.0f;
        or_sparse_walk(mode, 0, seed, i, sb, sl, se, sv, L, w, n, sides, r_size, wot_i, topk_edges, or_bwd_item, &c);
        grad_v[i] = c.gsp;
    }
}

/* Sparse max hop: FlashLogFunctionSparse3DTopKMax (flashlog_kernel.py:
 * 1450-1626) with the coalesce of :399-478.  Items as the top-k walk, masked
 * kept edges included as (v*w)*0 items; per (row, destination) the winner is
 * the largest value (== comparison, so zeros of either sign tie), then the
 * smallest source (ORI 0, INV 1, identity 2), then the smallest original edge
 * id (0 for the identity item), then the earliest item (raw order within a
 * source).  Outputs: keys ascending, the winner's value (+0 for a zero), and
 * the winner's entry, dir (0/1/2) and CSR position (-1 for the identity).  */
typedef struct {
    float *best; int32_t *src_rank; int64_t *edge; int64_t *entry; int32_t *dir; int64_t *pos;
    int64_t *mark; int64_t *touched; int64_t ntouched; int64_t stamp;
} or_max_t;

static void or_max_item(void *ctx, int64_t entry, int dir, int64_t p, int64_t edge, int64_t dst, int rel, float m,
                        float value)
{
    or_max_t *a = (or_max_t *)ctx;
    (void)rel; (void)m;
    int64_t tie_edge = dir == 2 ? 0 : edge;
    if (a->mark[dst] != a->stamp) {
        a->mark[dst] = a->stamp;
        a->touched[a->ntouched++] = dst;
    } else {
        float b = a->best[dst];
        int better = value > b || (value == b && (dir < a->src_rank[dst] ||
                                                  (dir == a->src_rank[dst] && tie_edge < a->edge[dst])));
        if (!better) return;
    }
    a->best[dst] = value;
    a->src_rank[dst] = dir;
    a->edge[dst] = tie_edge;
    a->entry[dst] = entry;
    a->dir[dst] = dir;
    a->pos[dst] = p;
}

int64_t or_sparse_max_forward(int64_t nnz, const int64_t *sb, const int64_t *sl, const int64_t *se,
    const float *sv, int64_t B, int64_t L, int64_t E, const float *w, int64_t n,
    const int32_t *ori_col, const float *ori_mask, const int32_t *ori_gptr, const int16_t *ori_grel,
    const int32_t *ori_gstart, const int32_t *ori_gcount,
    const int32_t *inv_col, const float *inv_mask, const int32_t *inv_gptr, const int16_t *inv_grel,
    const int32_t *inv_gstart, const int32_t *inv_gcount, const int32_t *ori_order, const int32_t *inv_order,
    int64_t r_size, int wot_i, int64_t topk_edges, int64_t seed, int64_t cap, int64_t *out_key, float *out_v,
    int64_t *win_entry, int32_t *win_dir, int64_t *win_pos)
{
    OR_SIDES;
    size_t e1 = (size_t)(E > 0 ? E : 1);
    or_max_t a;
    a.best = (float *)calloc(e1, sizeof(float));
    a.src_rank = (int32_t *)calloc(e1, sizeof(int32_t));
    a.edge = (int64_t *)calloc(e1, sizeof(int64_t));
    a.entry = (int64_t *)calloc(e1, sizeof(int64_t));
    a.dir = (int32_t *)calloc(e1, sizeof(int32_t));
    a.pos = (int64_t *)calloc(e1, sizeof(int64_t));
    a.mark = (int64_t *)malloc(e1 * sizeof(int64_t));
    a.touched = (int64_t *)malloc(e1 * sizeof(int64_t));
    for (int64_t e = 0; e < E; ++e) a.mark[e] = -1;
    int64_t total = 0;
    for (int64_t row = 0; row < B * L; ++row) {
        a.ntouched = 0;
        a.stamp = row;
        for (int64_t i = 0; i < nnz; ++i)
            if (sb[i] * L + sl[i] == row)
                or_sparse_walk(0, 1, seed, i, sb, sl, se, sv, L, w, n, sides, r_size, wot_i, topk_edges,
                               or_max_item, &a);
        qsort(a.touched, (size_t)a.ntouched, sizeof(int64_t), or_cmp_i64);
        if (total + a.ntouched > cap) { total = -1; break; }
        for (int64_t k = 0; k < a.ntouched; ++k) {
            int64_t d = a.touched[k];
            out_key[total + k] = row * E + d;
            out_v[total + k] = a.best[d] == 0.0f ? 0.0f : a.best[d];
            win_entry[total + k] = a.entry[d];
            win_dir[total + k] = a.dir[d];
            win_pos[total + k] = a.pos[d];
        }
        total += a.ntouched;
    }
    free(a.best); free(a.src_rank); free(a.edge); free(a.entry); free(a.dir); free(a.pos);
    free(a.mark); free(a.touched);
    return total;
}

/* Backward of the sparse max (flashlog.cu:2364-2410): the gradient of every
 * output goes to its winner only: edge winner (entry i, side, position p):
 * grad_v[i] += (g*m)*w[off+rel], grad_w[row, off+rel] += (g*m)*v; identity
 * winner: grad_v[i] += g*w[n-1], grad_w[row, n-1] += g*v (outputs in order). */
void or_sparse_max_backward(int64_t nnz, const int64_t *sb, const int64_t *sl, const float *sv, int64_t B,
    int64_t L, const float *w, int64_t n, const float *ori_mask, const int16_t *ori_prel, const float *inv_mask,
    const int16_t *inv_prel, int64_t r_size, int64_t nout, const float *grad_out, const int64_t *win_entry,
    const int32_t *win_dir, const int64_t *win_pos, float *grad_v, float *grad_w)
{
    memset(grad_v, 0, sizeof(float) * (size_t)nnz);
    memset(grad_w, 0, sizeof(float) * (size_t)(B * L * n));
    for (int64_t o = 0; o < nout; ++o) {
        int64_t i = win_entry[o];
        int64_t row = sb[i] * L + sl[i];
        float g = grad_out[o];
        if (win_dir[o] == 2) {
            grad_v[i] += g * w[row * n + n - 1];
            grad_w[row * n + n - 1] += g * sv[i];
            continue;
        }
        int64_t p = win_pos[o];
        float m = win_dir[o] ? inv_mask[p] : ori_mask[p];
        int64_t col = (win_dir[o] ? r_size + inv_prel[p] : ori_prel[p]);
        grad_v[i] += g * m * w[row * n + col];
        grad_w[row * n + col] += g * m * sv[i];
    }
}

/* normalize_sparse3d on the CPU (flashlog_kernel.py:551-555): per row the
 * sum of its values in entry order (index_add_), out = v / max(d, eps).     */
void or_sparse_normalize(int64_t nnz, const int64_t *sb, const int64_t *sl, const float *v, int64_t B, int64_t L,
                         float eps, float *out, float *denom)
{
    for (int64_t r = 0; r < B * L; ++r) denom[r] = 0.0f;
    for (int64_t i = 0; i < nnz; ++i) denom[sb[i] * L + sl[i]] += v[i];
    for (int64_t i = 0; i < nnz; ++i) {
        float d = denom[sb[i] * L + sl[i]];
        out[i] = v[i] / (d < eps ? eps : d);
    }
}

/* ------------------------------------------------------------------------ */
/* Filtered, tie-aware rank of the target per query: flashlog.cu:2754-2910.
 * Scores are a sparse [B, E] matrix given as (b, e, v) entries sorted by
 * (b, e), at most one entry per coordinate; absent coordinates score 0.
 * filter_keys holds b*E + e for the filtered answers (sorted ascending).
 * truth = score of (b, target_b).  Over unfiltered explicit entries:
 * greater = #(v > truth), eq_explicit = #(v == truth).  With use_eql:
 *   eq = eq_explicit + (truth == 0 ? E - |filter_b| - explicit_unfiltered : 0) + 1
 *   rank = greater + (eq + 1) / 2
 * otherwise rank = greater + 1.  The target itself counts as filtered when
 * its key is in filter_keys (the reference keeps it out of both counts).    */

#define OR_DEFINE_FILTERED_RANKS(NAME, T)                                                    \
void NAME(int64_t nnz, const int64_t *idx_b, const int64_t *idx_e, const T *values,             \
          int64_t B, int64_t E, const int64_t *targets,                                          \
          int64_t nfilter, const int64_t *filter_keys, int use_eql, float *ranks)                \
{                                                                                                \
    T *truth = (T *)calloc((size_t)(B > 0 ? B : 1), sizeof(T));                                  \
    float *greater = (float *)calloc((size_t)(B > 0 ? B : 1), sizeof(float));                    \
    float *equal = (float *)calloc((size_t)(B > 0 ? B : 1), sizeof(float));                      \
    float *explicit_unf = (float *)calloc((size_t)(B > 0 ? B : 1), sizeof(float));               \
    float *fcount = (float *)calloc((size_t)(B > 0 ? B : 1), sizeof(float));                     \
    for (int64_t i = 0; i < nnz; ++i)                                                            \
        if (idx_e[i] == targets[idx_b[i]]) truth[idx_b[i]] = values[i];                          \
    for (int64_t k = 0; k < nfilter; ++k) {                                                      \
        int64_t b = filter_keys[k] / E;                                                          \
        if (b >= 0 && b < B) fcount[b] += 1.0f;                                                  \
    }                                                                                            \
    for (int64_t i = 0; i < nnz; ++i) {                                                          \
        int64_t b = idx_b[i], key = b * E + idx_e[i];                                            \
        int64_t pos = or_lower_bound(filter_keys, nfilter, key);                                 \
        if (pos < nfilter && filter_keys[pos] == key) continue;                                  \
        explicit_unf[b] += 1.0f;                                                                 \
        if (values[i] > truth[b]) greater[b] += 1.0f;                                            \
        else if (values[i] == truth[b]) equal[b] += 1.0f;                                        \
    }                                                                                            \
    for (int64_t b = 0; b < B; ++b) {                                                            \
        if (use_eql) {                                                                           \
            float missing = (float)E - fcount[b] - explicit_unf[b];                              \
            float eq = equal[b] + (truth[b] == (T)0 ? missing : 0.0f);                           \
            eq += 1.0f;                                                                          \
            ranks[b] = greater[b] + (eq + 1.0f) * 0.5f;                                          \
        } else {                                                                                 \
            ranks[b] = greater[b] + 1.0f;                                                        \
        }                                                                                        \
    }                                                                                            \
    free(truth); free(greater); free(equal); free(explicit_unf); free(fcount);                   \
}

/* flashlog.cu:2754-2910 for float and double scores (AT_DISPATCH_FLOATING_TYPES). */
OR_DEFINE_FILTERED_RANKS(or_filtered_ranks, float)
OR_DEFINE_FILTERED_RANKS(or_filtered_ranks_f64, double)
