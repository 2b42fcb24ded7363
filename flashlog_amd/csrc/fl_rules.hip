// Rule-bank scoring accumulators (rules/shared_inference.py:12-245, the
// dense-accumulator branch :87-96,200-206,224-237).
//
// A chunk of rules has been grounded for every source b: a COO state
// (b, rule l, entity e, v) with v the path count (or 0/1 with Boolean paths).
// Per rank k the scores are
//   sum:  S_k[b, e] += sum over the chunk's rules, in rule order, of v * W[rule, k]
//   max:  S_k[b, e]  = max(S_k[b, e], v * W[rule, k])      (W >= 0)
// accumulated over chunks in a dense [K, B*E] buffer; then every (k, b) row
// is normalized by its sum (clamped to 1e-30) and the ranks are summed (or
// maxed with final_max) into one [B*E] score.
#include "fl_abi.h"
#include "fl_common.h"

namespace fl {

constexpr int RB_NT = 256;

// Maxima: thread per state entry; the maximum of nonnegative values is
// exact in any order (the integer order of their bits), so atomics give the
// same bits on every run.  (Sums go through fl_sparse_channel_weighted_add,
// one writer per accumulator slot.)
__global__ __launch_bounds__(RB_NT) void k_rule_accum_max(const int64_t *__restrict__ sb,
                                                         const int64_t *__restrict__ sl,
                                                         const int64_t *__restrict__ se,
                                                         const float *__restrict__ sv, int64_t nnz,
                                                         const float *__restrict__ W, int64_t K, int64_t B,
                                                         int64_t L, int64_t E, float *__restrict__ dense) {
    const int64_t i = (int64_t)blockIdx.x * RB_NT + threadIdx.x;
    if (i >= nnz) return;
    if (sb[i] < 0 || sb[i] >= B || se[i] < 0 || se[i] >= E || sl[i] < 0 || sl[i] >= L) return;  // outside the shape
    const int64_t key = sb[i] * E + se[i];
    const float v = sv[i];
    const float *wr = W + sl[i] * K;
    for (int64_t k = 0; k < K; ++k) {
        const float x = fl_mul(v, wr[k]);
        if (x > 0.0f) atomicMax((unsigned int *)(dense + k * B * E + key), __float_as_uint(x));
    }
}

// Sums through LDS (entities of a source fit a workgroup's LDS): row
// pointers of the coalesced chunk state first (thread per entry; err 1: an
// index outside [B, L, E], 2: rows out of order, 3: entities not strictly
// increasing within a row), then a workgroup per (source b, rank k) holds
// acc[e] for every entity in LDS and walks the chunk's rules in order: rule
// l's entries (distinct entities: no two lanes add into one slot) add
// v * W[l, k] to acc, a barrier between rules.  Per entity the terms are
// thus added from 0 in rule order, then the chunk's sum is added to the
// dense accumulator: the order of k_cs_weighted_add, without the merge.
constexpr int RA_NT = 256;

__global__ void k_ra_zero(unsigned long long *err) {
    if (threadIdx.x == 0) *err = 0;
}
constexpr int64_t RA_LDS_MAX_E = 16384;  // 64 KB of LDS per workgroup

__global__ __launch_bounds__(RA_NT) void k_ra_rows(const int64_t *__restrict__ sb, const int64_t *__restrict__ sl,
                                                  const int64_t *__restrict__ se, int64_t nnz, int64_t B, int64_t L,
                                                  int64_t E, int64_t *__restrict__ row_ptr,
                                                  unsigned long long *__restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * RA_NT + threadIdx.x;
    if (i >= nnz) return;
    const int64_t b = sb[i], l = sl[i], e = se[i];
    if (b < 0 || b >= B || l < 0 || l >= L || e < 0 || e >= E) {
        atomicMax(err, 1ull);
        return;
    }
    const int64_t r = b * L + l;
    int64_t rp = -1;
    if (i > 0) {
        const int64_t pb = sb[i - 1], pl = sl[i - 1];
        rp = (pb >= 0 && pb < B && pl >= 0 && pl < L) ? pb * L + pl : r;
        if (rp > r) {
            atomicMax(err, 2ull);
            return;
        }
        if (rp == r && se[i - 1] >= e) {
            atomicMax(err, 3ull);
            return;
        }
    }
    for (int64_t q = rp + 1; q <= r; ++q) row_ptr[q] = i;
    if (i == nnz - 1)
        for (int64_t q = r + 1; q <= B * L; ++q) row_ptr[q] = nnz;
}

__global__ __launch_bounds__(RA_NT) void k_ra_sum(const int64_t *__restrict__ se, const float *__restrict__ sv,
                                                 const int64_t *__restrict__ row_ptr,
                                                 const unsigned long long *__restrict__ err,
                                                 const float *__restrict__ W, int64_t K, int64_t B, int64_t L,
                                                 int64_t E, float *__restrict__ dense) {
    extern __shared__ float acc[];  // [E]
    if (*err != 0) return;          // a malformed state adds nothing
    const int64_t b = blockIdx.x, k = blockIdx.y;
    const int t = threadIdx.x;
    for (int64_t e = t; e < E; e += RA_NT) acc[e] = 0.0f;
    __syncthreads();
    for (int64_t l = 0; l < L; ++l) {
        const int64_t a = row_ptr[b * L + l], z = row_ptr[b * L + l + 1];
        const float wk = W[l * K + k];
        for (int64_t i = a + t; i < z; i += RA_NT) {
            const int64_t e = se[i];
            acc[e] = fl_add(acc[e], fl_mul(sv[i], wk));
        }
        __syncthreads();
    }
    float *drow = dense + k * B * E + b * E;
    for (int64_t e = t; e < E; e += RA_NT) {
        const float x = acc[e];
        if (x != 0.0f) drow[e] = fl_add(drow[e], x);
    }
}

// Workgroup per (k, b): the row's sum in a fixed order.
__global__ __launch_bounds__(RB_NT) void k_rule_rowsum(const float *__restrict__ dense, int64_t E,
                                                      float *__restrict__ rowsum) {
    __shared__ float red[RB_NT];
    const float *row = dense + (int64_t)blockIdx.x * E;
    float s = 0.0f;
    for (int64_t e = threadIdx.x; e < E; e += RB_NT) s = fl_add(s, row[e]);
    red[threadIdx.x] = s;
    __syncthreads();
    for (int st = RB_NT / 2; st > 0; st >>= 1) {
        if ((int)threadIdx.x < st) red[threadIdx.x] = fl_add(red[threadIdx.x], red[threadIdx.x + st]);
        __syncthreads();
    }
    if (threadIdx.x == 0) rowsum[blockIdx.x] = red[0];
}

// Thread per (b, e): the normalized ranks combined in rank order.
__global__ __launch_bounds__(RB_NT) void k_rule_combine(const float *__restrict__ dense,
                                                       const float *__restrict__ rowsum, int64_t K, int64_t B,
                                                       int64_t E, int final_max, float *__restrict__ total) {
    const int64_t q = (int64_t)blockIdx.x * RB_NT + threadIdx.x;
    if (q >= B * E) return;
    const int64_t b = q / E;
    float t = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
        const float x = dense[k * B * E + q];
        if (x == 0.0f) continue;
        const float d = rowsum[k * B + b];
        const float p = __fdiv_rn(x, d < 1e-30f ? 1e-30f : d);
        t = final_max ? (p > t ? p : t) : fl_add(t, p);
    }
    total[q] = t;
}

}  // namespace fl

extern "C" {

size_t fl_rule_accumulate_bytes(int64_t nnz, int64_t B, int64_t L) {
    if (nnz < 0 || B < 0 || L < 0) return 0;
    const size_t merge = ((fl_sparse_channel_sum_bytes(nnz, B, L) + 255) & ~(size_t)255) + 256;
    const size_t lds = ((sizeof(int64_t) * (size_t)(B * L + 1) + 255) & ~(size_t)255) + 256;
    return merge > lds ? merge : lds;
}

int fl_rule_accumulate(void *stream, const int64_t *sb, const int64_t *sl, const int64_t *se, const float *sv,
                       int64_t nnz, const float *W, int64_t K, int64_t B, int64_t L, int64_t E, int is_max,
                       float *dense, void *ws, size_t ws_bytes) {
    if (nnz < 0 || K < 1 || B < 0 || L < 0 || E < 0) return fl::fl_fail(FL_ERR_ARG, "rule_accumulate: bad shape");
    if (nnz == 0) return FL_OK;
    if (!sb || !sl || !se || !sv || !W || !dense) return fl::fl_fail(FL_ERR_ARG, "rule_accumulate: null pointer");
    hipStream_t st = (hipStream_t)stream;
    if (is_max) {
        FL_LAUNCH("k_rule_accum_max", fl::k_rule_accum_max, dim3((unsigned)((nnz + fl::RB_NT - 1) / fl::RB_NT)),
                  dim3(fl::RB_NT), 0, st, sb, sl, se, sv, nnz, W, K, B, L, E, dense);
        return fl::fl_check_launch("rule_accumulate");
    }
    if (!ws || ws_bytes < fl_rule_accumulate_bytes(nnz, B, L))
        return fl::fl_fail(FL_ERR_ARG, "rule_accumulate: workspace too small");
    if (E <= fl::RA_LDS_MAX_E && B * K <= 0x7fffffff && K <= 65535) {
        // rules in order through an LDS accumulator per (source, rank)
        int64_t *row_ptr = (int64_t *)ws;
        unsigned long long *err =
            (unsigned long long *)((char *)ws + ((sizeof(int64_t) * (size_t)(B * L + 1) + 255) & ~(size_t)255));
        FL_LAUNCH("k_fill_u64", fl::k_ra_zero, dim3(1), dim3(64), 0, st, err);
        FL_LAUNCH("k_ra_rows", fl::k_ra_rows, dim3((unsigned)((nnz + fl::RA_NT - 1) / fl::RA_NT)), dim3(fl::RA_NT), 0,
                  st, sb, sl, se, nnz, B, L, E, row_ptr, err);
        FL_LAUNCH("k_ra_sum", fl::k_ra_sum, dim3((unsigned)B, (unsigned)K), dim3(fl::RA_NT),
                  sizeof(float) * (size_t)E, st, se, sv, row_ptr, err, W, K, B, L, E, dense);
        return fl::fl_check_launch("rule_accumulate");
    }
    // rank the entries of every (b, e) in rule order, then one writer per slot
    const size_t cs = (fl_sparse_channel_sum_bytes(nnz, B, L) + 255) & ~(size_t)255;
    int64_t *plan = (int64_t *)((char *)ws + cs);
    int rc = fl_sparse_channel_sum_plan(stream, sb, sl, se, nnz, B, L, E, ws, cs, plan);
    if (rc != FL_OK) return rc;
    return fl_sparse_channel_weighted_add(stream, sb, sl, se, sv, nnz, B, L, E, W, K, ws, dense);
}

int fl_rule_finalize(void *stream, const float *dense, int64_t K, int64_t B, int64_t E, int final_max,
                     float *rowsum, float *total) {
    if (K < 1 || B < 0 || E < 0) return fl::fl_fail(FL_ERR_ARG, "rule_finalize: bad shape");
    if (B * E == 0) return FL_OK;
    if (!dense || !rowsum || !total) return fl::fl_fail(FL_ERR_ARG, "rule_finalize: null pointer");
    hipStream_t st = (hipStream_t)stream;
    FL_LAUNCH("k_rule_rowsum", fl::k_rule_rowsum, dim3((unsigned)(K * B)), dim3(fl::RB_NT), 0, st, dense, E, rowsum);
    FL_LAUNCH("k_rule_combine", fl::k_rule_combine, dim3((unsigned)((B * E + fl::RB_NT - 1) / fl::RB_NT)),
              dim3(fl::RB_NT), 0, st, dense, rowsum, K, B, E, final_max, total);
    return fl::fl_check_launch("rule_finalize");
}

}  // extern "C"
