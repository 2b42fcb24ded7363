// Filtered tie-aware entity ranks over a sparse [B, E] score matrix
// (flashlog.cu:2754-2910, wrapper flashlog_kernel.py:168-179).
//
// For query b with target t_b and truth score s = score(b, t_b) (0 when the
// target has no explicit entry):
//   greater  = unfiltered explicit entries scoring above s
//   equal    = unfiltered explicit entries scoring exactly s
//   explicit = unfiltered explicit entries
//   filtered = filter keys of row b (keys are b*E + e, sorted ascending)
//   use_eql:  eq = equal + (s == 0 ? E - filtered - explicit : 0) + 1
//             rank = greater + (eq + 1) * 0.5
//   else:     rank = greater + 1
// Counts are kept as u32 and converted once (exact, as the reference's fp32
// counters are, for counts below 2^24).  The per-row filter count is two
// binary searches over the sorted keys instead of one atomic per key.
// Entries whose query index lies outside [0, B) are ignored.
#include <mutex>

#include "fl_common.h"
#include "fl_abi.h"
#include "fl_scan.h"

namespace fl {

constexpr int RK_NT = 256;

__device__ __forceinline__ int64_t rk_lower_bound(const int64_t *__restrict__ keys, int64_t n, int64_t key) {
    int64_t lo = 0, hi = n;
    while (lo < hi) {
        const int64_t mid = lo + ((hi - lo) >> 1);
        if (keys[mid] < key) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// Per query: zero the truth score and counters; the filter count of the row.
template <typename T>
__global__ __launch_bounds__(RK_NT) void k_rank_init(const int64_t *__restrict__ filter_keys, int64_t n_filter,
                                                     int64_t B, int64_t E, T *__restrict__ truth,
                                                     uint32_t *__restrict__ cnt, uint32_t *__restrict__ fcount) {
    const int64_t b = (int64_t)blockIdx.x * RK_NT + threadIdx.x;
    if (b >= B) return;
    truth[b] = (T)0;
    cnt[b] = 0;
    cnt[B + b] = 0;
    cnt[2 * B + b] = 0;
    const int64_t lo = rk_lower_bound(filter_keys, n_filter, b * E);
    const int64_t hi = rk_lower_bound(filter_keys, n_filter, (b + 1) * E);
    fcount[b] = (uint32_t)(hi - lo);
}

template <typename T>
__global__ __launch_bounds__(RK_NT) void k_rank_truth(const int64_t *__restrict__ idx_b,
                                                      const int64_t *__restrict__ idx_e, const T *__restrict__ values,
                                                      const int64_t *__restrict__ targets, int64_t nnz, int64_t B,
                                                      T *__restrict__ truth) {
    const int64_t i = (int64_t)blockIdx.x * RK_NT + threadIdx.x;
    if (i >= nnz) return;
    const int64_t b = idx_b[i];
    if (b < 0 || b >= B) return;
    if (idx_e[i] == targets[b]) truth[b] = values[i];
}

// Per entry: skip filtered keys, then count explicit / greater / equal.
// COO rows are usually contiguous, so a wave whose live lanes share one
// query reduces its three counts and adds them with one atomic each.
template <typename T>
__global__ __launch_bounds__(RK_NT) void k_rank_count(const int64_t *__restrict__ idx_b,
                                                      const int64_t *__restrict__ idx_e, const T *__restrict__ values,
                                                      const T *__restrict__ truth,
                                                      const int64_t *__restrict__ filter_keys, int64_t n_filter,
                                                      int64_t nnz, int64_t B, int64_t E, uint32_t *__restrict__ cnt) {
    const int64_t i = (int64_t)blockIdx.x * RK_NT + threadIdx.x;
    int64_t b = -1;
    int gt = 0, eq = 0, ex = 0;
    if (i < nnz) {
        b = idx_b[i];
        if (b >= 0 && b < B) {
            const int64_t key = b * E + idx_e[i];
            const int64_t pos = rk_lower_bound(filter_keys, n_filter, key);
            if (!(pos < n_filter && filter_keys[pos] == key)) {
                const T v = values[i];
                const T t = truth[b];
                ex = 1;
                if (v > t) gt = 1;
                else if (v == t) eq = 1;
            }
        } else {
            b = -1;
        }
    }
    const int live = ex;
    const unsigned long long lanes = __ballot(live);
    if (!lanes) return;
    const int first = __ffsll((long long)lanes) - 1;
    const int64_t b0 = __shfl(b, first, FL_WAVE);
    const bool uniform = __ballot(live && b != b0) == 0ull;
    if (uniform) {
        const int sg = fl_wave_sum_i32(gt), se = fl_wave_sum_i32(eq), sx = fl_wave_sum_i32(ex);
        if (fl_lane() == first) {
            if (sx) atomicAdd(&cnt[2 * B + b0], (uint32_t)sx);
            if (sg) atomicAdd(&cnt[b0], (uint32_t)sg);
            if (se) atomicAdd(&cnt[B + b0], (uint32_t)se);
        }
    } else if (live) {
        atomicAdd(&cnt[2 * B + b], 1u);
        if (gt) atomicAdd(&cnt[b], 1u);
        if (eq) atomicAdd(&cnt[B + b], 1u);
    }
}

template <typename T>
__global__ __launch_bounds__(RK_NT) void k_rank_final(const T *__restrict__ truth, const uint32_t *__restrict__ cnt,
                                                      const uint32_t *__restrict__ fcount, int64_t B, int64_t E,
                                                      int use_eql, float *__restrict__ ranks) {
    const int64_t b = (int64_t)blockIdx.x * RK_NT + threadIdx.x;
    if (b >= B) return;
    const float greater = (float)cnt[b];
    if (use_eql) {
        const float equal = (float)cnt[B + b];
        const float explicit_unf = (float)cnt[2 * B + b];
        const float missing = __fsub_rn(__fsub_rn((float)E, (float)fcount[b]), explicit_unf);
        float eq = fl_add(equal, truth[b] == (T)0 ? missing : 0.0f);
        eq = fl_add(eq, 1.0f);
        ranks[b] = fl_add(greater, fl_mul(fl_add(eq, 1.0f), 0.5f));
    } else {
        ranks[b] = fl_add(greater, 1.0f);
    }
}

template <typename T>
int launch_ranks(hipStream_t st, const int64_t *idx_b, const int64_t *idx_e, const T *values,
                 const int64_t *targets, const int64_t *filter_keys, int64_t nnz, int64_t n_filter, int64_t B,
                 int64_t E, int use_eql, float *ranks, char *ws) {
    T *truth = (T *)ws;
    uint32_t *cnt = (uint32_t *)(ws + ((sizeof(T) * (size_t)B + 255) & ~(size_t)255));
    uint32_t *fcount = cnt + 3 * B;
    const unsigned gb = (unsigned)((B + RK_NT - 1) / RK_NT);
    FL_LAUNCH("k_rank_init", k_rank_init<T>, dim3(gb), dim3(RK_NT), 0, st, filter_keys, n_filter, B, E, truth, cnt,
              fcount);
    if (nnz > 0) {
        const unsigned gn = (unsigned)((nnz + RK_NT - 1) / RK_NT);
        FL_LAUNCH("k_rank_truth", k_rank_truth<T>, dim3(gn), dim3(RK_NT), 0, st, idx_b, idx_e, values, targets, nnz,
                  B, truth);
        FL_LAUNCH("k_rank_count", k_rank_count<T>, dim3(gn), dim3(RK_NT), 0, st, idx_b, idx_e, values, truth,
                  filter_keys, n_filter, nnz, B, E, cnt);
    }
    FL_LAUNCH("k_rank_final", k_rank_final<T>, dim3(gb), dim3(RK_NT), 0, st, truth, cnt, fcount, B, E, use_eql,
              ranks);
    return fl_check_launch("filtered_ranks");
}

}  // namespace fl

extern "C" {

size_t fl_filtered_ranks_workspace_bytes(int64_t B, int values_f64) {
    if (B <= 0) return 256;
    const size_t tb = (values_f64 ? 8 : 4) * (size_t)B;
    return ((tb + 255) & ~(size_t)255) + ((sizeof(uint32_t) * 4 * (size_t)B + 255) & ~(size_t)255);
}

int fl_filtered_ranks(void *stream, const int64_t *idx_b, const int64_t *idx_e, const void *values, int values_f64,
                      const int64_t *targets, const int64_t *filter_keys, int64_t nnz, int64_t n_filter, int64_t B,
                      int64_t E, int use_eql, float *ranks, void *workspace, size_t workspace_bytes) {
    if (nnz < 0 || n_filter < 0 || B < 0 || E < 0) return fl::fl_fail(FL_ERR_ARG, "filtered_ranks: negative size");
    if (B == 0) return FL_OK;
    if (B > INT64_MAX / (E + 1)) return fl::fl_fail(FL_ERR_ARG, "filtered_ranks: B*E overflows int64");
    if (!ranks || !targets || (nnz > 0 && (!idx_b || !idx_e || !values)) || (n_filter > 0 && !filter_keys))
        return fl::fl_fail(FL_ERR_ARG, "filtered_ranks: null pointer");
    if (!workspace || workspace_bytes < fl_filtered_ranks_workspace_bytes(B, values_f64))
        return fl::fl_fail(FL_ERR_ARG, "filtered_ranks: workspace too small");
    hipStream_t st = (hipStream_t)stream;
    if (values_f64)
        return fl::launch_ranks<double>(st, idx_b, idx_e, (const double *)values, targets, filter_keys, nnz,
                                        n_filter, B, E, use_eql, ranks, (char *)workspace);
    return fl::launch_ranks<float>(st, idx_b, idx_e, (const float *)values, targets, filter_keys, nnz, n_filter, B,
                                   E, use_eql, ranks, (char *)workspace);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free variant of fl_filtered_ranks: its scratch (truth scores and
// counters, at most FL_RANKS_NOALLOC_MAX_B queries) lives in a file-scope
// device array.  Each GPU holds its own copy; the host looks up that copy's
// address once per device (hipGetSymbolAddress, with the device current) and
// passes that address to the kernels -- the array's name in host code is not
// a device address.

namespace fl {
namespace {

constexpr size_t NOALLOC_BYTES =
    ((sizeof(double) * (size_t)FL_RANKS_NOALLOC_MAX_B + 255) & ~(size_t)255) +
    ((sizeof(uint32_t) * 4 * (size_t)FL_RANKS_NOALLOC_MAX_B + 255) & ~(size_t)255);

__device__ __align__(256) unsigned char scratch[NOALLOC_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[NOALLOC_MAX_DEVICES];

// This device's copy of `scratch` (looked up on the first call per device).
int scratch_for_current_device(void **out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0)
        return fl_fail(FL_ERR_HIP, "filtered_ranks_noalloc: no current device");
    if (dev >= NOALLOC_MAX_DEVICES)
        return fl_fail(FL_ERR_ARG, "filtered_ranks_noalloc: device %d beyond %d", dev, NOALLOC_MAX_DEVICES);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void *p = nullptr;
        const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (rc != hipSuccess || !p)
            return fl_fail(FL_ERR_HIP, "filtered_ranks_noalloc: hipGetSymbolAddress failed: %s",
                           hipGetErrorString(rc));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return FL_OK;
}

}  // namespace
}  // namespace fl

extern "C" {

int fl_filtered_ranks_noalloc(void *stream, const int64_t *idx_b, const int64_t *idx_e, const void *values,
                              int values_f64, const int64_t *targets, const int64_t *filter_keys, int64_t nnz,
                              int64_t n_filter, int64_t B, int64_t E, int use_eql, float *ranks) {
    if (nnz < 0 || n_filter < 0 || B < 0 || E < 0)
        return fl::fl_fail(FL_ERR_ARG, "filtered_ranks_noalloc: negative size");
    if (B > FL_RANKS_NOALLOC_MAX_B)
        return fl::fl_fail(FL_ERR_ARG, "filtered_ranks_noalloc: %lld queries, at most %d without a workspace",
                           (long long)B, FL_RANKS_NOALLOC_MAX_B);
    if (B == 0) return FL_OK;
    void *ws = nullptr;
    const int rc = fl::scratch_for_current_device(&ws);
    if (rc != FL_OK) return rc;
    return fl_filtered_ranks(stream, idx_b, idx_e, values, values_f64, targets, filter_keys, nnz, n_filter, B, E,
                             use_eql, ranks, ws, fl::NOALLOC_BYTES);
}

}  // extern "C"

namespace fl {

// Dense filtered ranks (src/main.py:468-512, the ranks of
// calculate_hits_full_with_filter_indices): one workgroup per query row b
// of a dense score matrix [B, E]; truth = state[b, target_b];
//   greater = #{e : s > truth} - #{e in filter_b : s > truth}
//   equal   = #{e : s == truth} - #{e in filter_b : s == truth}
//   use_eql: rank = greater + ((equal + 1) + 1) / 2;  else greater + 1
// with the reference's fp32 arithmetic on exact integer counts.  The row is
// read once (coalesced, HBM-bound); filter_b is the row's range of the
// sorted unique keys b*E + e.
constexpr int DR_NT = 256;

__global__ __launch_bounds__(DR_NT) void k_dense_rank(const float *__restrict__ state, int64_t E,
                                                      const int64_t *__restrict__ targets,
                                                      const int64_t *__restrict__ filter_keys, int64_t n_filter,
                                                      int use_eql, float *__restrict__ ranks) {
    __shared__ uint32_t red[4][DR_NT / FL_WAVE];
    const int64_t b = blockIdx.x;
    const int t = threadIdx.x;
    const float *row = state + b * E;
    const float truth = row[targets[b]];
    uint32_t gt = 0, eq = 0;
    // 16-byte loads over the aligned middle of the row, scalars at its ends
    const int64_t pre = ((4 - ((b * E) & 3)) & 3) < E ? ((4 - ((b * E) & 3)) & 3) : E;
    const int64_t nvec = (E - pre) >> 2;
    if (t < pre) {
        const float x = row[t];
        gt += x > truth;
        eq += x == truth;
    }
    const float4 *v4 = reinterpret_cast<const float4 *>(row + pre);
    for (int64_t k = t; k < nvec; k += DR_NT) {
        const float4 x = v4[k];
        gt += (x.x > truth) + (x.y > truth) + (x.z > truth) + (x.w > truth);
        eq += (x.x == truth) + (x.y == truth) + (x.z == truth) + (x.w == truth);
    }
    for (int64_t e = pre + 4 * nvec + t; e < E; e += DR_NT) {
        const float x = row[e];
        gt += x > truth;
        eq += x == truth;
    }
    uint32_t fgt = 0, feq = 0;
    if (n_filter > 0) {
        const int64_t lo = rk_lower_bound(filter_keys, n_filter, b * E);
        const int64_t hi = rk_lower_bound(filter_keys, n_filter, (b + 1) * E);
        for (int64_t k = lo + t; k < hi; k += DR_NT) {
            const float x = row[filter_keys[k] - b * E];
            fgt += x > truth;
            feq += x == truth;
        }
    }
    gt = (uint32_t)fl_wave_sum_i32((int)gt);
    eq = (uint32_t)fl_wave_sum_i32((int)eq);
    fgt = (uint32_t)fl_wave_sum_i32((int)fgt);
    feq = (uint32_t)fl_wave_sum_i32((int)feq);
    const int w = t / FL_WAVE;
    if (fl_lane() == 0) {
        red[0][w] = gt;
        red[1][w] = eq;
        red[2][w] = fgt;
        red[3][w] = feq;
    }
    __syncthreads();
    if (t == 0) {
        uint32_t a[4] = {0, 0, 0, 0};
        for (int q = 0; q < 4; ++q)
            for (int i = 0; i < DR_NT / FL_WAVE; ++i) a[q] += red[q][i];
        // the reference's float counters: sum().float(), then scatter_add of 1.0f
        float greater = (float)a[0];
        if (n_filter > 0) greater = greater - (float)a[2];
        if (use_eql) {
            float equal = (float)a[1];
            if (n_filter > 0) equal = equal - (float)a[3];
            equal = equal + 1.0f;
            ranks[b] = greater + (equal + 1.0f) / 2.0f;
        } else {
            ranks[b] = greater + 1.0f;
        }
    }
}

}  // namespace fl

extern "C" {

int fl_dense_filtered_ranks(void *stream, const float *state, const int64_t *targets, const int64_t *filter_keys,
                            int64_t n_filter, int64_t B, int64_t E, int use_eql, float *ranks) {
    if (B < 0 || E <= 0 || n_filter < 0) return fl::fl_fail(FL_ERR_ARG, "dense_filtered_ranks: bad sizes");
    if (B == 0) return FL_OK;
    if (B > INT64_MAX / E) return fl::fl_fail(FL_ERR_ARG, "dense_filtered_ranks: B*E overflows int64");
    if (!state || !targets || !ranks || (n_filter > 0 && !filter_keys))
        return fl::fl_fail(FL_ERR_ARG, "dense_filtered_ranks: null pointer");
    FL_LAUNCH("k_dense_rank", fl::k_dense_rank, dim3((unsigned)B), dim3(fl::DR_NT), 0, (hipStream_t)stream, state, E,
              targets, filter_keys, n_filter, use_eql, ranks);
    return fl::fl_check_launch("dense_filtered_ranks");
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Known-answer expansion of the filtered evaluation (src/main.py:212-276,
// _expand_filter_side / _filter_indices_from_lookup).  The reference keys
// the (source, relation) groups of one side as source * R + relation and
// looks every query key up by binary search; here the key is split back into
// (key floor-div R, key mod R) and the relation is searched among that
// source's groups (ascending relation), which finds the same group for every
// key.  The group's columns in CSR order are the query's known answers.
// Outputs (query position, entity) pairs, queries in the given order.

namespace fl {

__global__ void k_flt_count(const int32_t *__restrict__ gptr, const int16_t *__restrict__ grel,
                            const int32_t *__restrict__ gcount, int64_t nodes, const int64_t *__restrict__ keys,
                            int64_t R, int64_t Q, int32_t *__restrict__ cnt, int64_t *__restrict__ gsel) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q >= Q) return;
    const int64_t k = keys[q];
    int64_t s = k / R, r = k % R;
    if (r < 0) { r += R; s -= 1; }  // floor division
    int64_t g = -1;
    if (s >= 0 && s < nodes) {
        int64_t lo = gptr[s], hi = gptr[s + 1];
        while (lo < hi) {
            const int64_t mid = lo + ((hi - lo) >> 1);
            if (grel[mid] < r) lo = mid + 1; else hi = mid;
        }
        if (lo < gptr[s + 1] && grel[lo] == r) g = lo;
    }
    gsel[q] = g;
    cnt[q] = g >= 0 ? gcount[g] : 0;
}

// Thread per output pair: its query by binary search over the offsets.
__global__ void k_flt_fill(const int32_t *__restrict__ gstart, const int32_t *__restrict__ col,
                           const int64_t *__restrict__ gsel, const int64_t *__restrict__ off, int64_t Q,
                           const int64_t *__restrict__ qpos, int64_t total, int64_t *__restrict__ out_b,
                           int64_t *__restrict__ out_e) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    int64_t lo = 0, hi = Q;  // last q with off[q] <= i
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (off[mid] <= i) lo = mid; else hi = mid;
    }
    const int64_t g = gsel[lo];
    out_b[i] = qpos[lo];
    out_e[i] = col[(int64_t)gstart[g] + (i - off[lo])];
}

size_t flt_al(size_t x) { return (x + 255) & ~(size_t)255; }

}  // namespace fl

extern "C" {

size_t fl_filter_expand_bytes(int64_t Q) {
    if (Q < 0) return 0;
    const size_t q1 = (size_t)(Q > 0 ? Q : 1);
    return fl::flt_al(sizeof(int32_t) * q1) + fl::flt_al(sizeof(int64_t) * q1) + fl::flt_al(fl::scan_tmp_bytes(Q + 1));
}

int fl_filter_expand_count(void *stream, const int32_t *gptr, const int16_t *grel, const int32_t *gcount,
                           int64_t nodes, const int64_t *keys, int64_t R, int64_t Q, int64_t *off, void *ws,
                           size_t ws_bytes) {
    if (Q < 0 || nodes < 0 || R < 1) return fl::fl_fail(FL_ERR_ARG, "filter_expand: bad size");
    if (!off || !ws || ws_bytes < fl_filter_expand_bytes(Q) || (Q > 0 && (!gptr || !grel || !gcount || !keys)))
        return fl::fl_fail(FL_ERR_ARG, "filter_expand: null argument or workspace too small");
    const size_t q1 = (size_t)(Q > 0 ? Q : 1);
    int32_t *cnt = (int32_t *)ws;
    int64_t *gsel = (int64_t *)((char *)ws + fl::flt_al(sizeof(int32_t) * q1));
    int64_t *tmp = (int64_t *)((char *)gsel + fl::flt_al(sizeof(int64_t) * q1));
    hipStream_t st = (hipStream_t)stream;
    if (Q > 0)
        FL_LAUNCH("k_flt_count", fl::k_flt_count, dim3((unsigned)((Q + 255) / 256)), dim3(256), 0, st, gptr, grel,
                  gcount, nodes, keys, R, Q, cnt, gsel);
    const int rc = fl::exclusive_scan(st, cnt, off, Q, tmp);
    if (rc != FL_OK) return rc;
    return fl::fl_check_launch("filter_expand_count");
}

int fl_filter_expand_fill(void *stream, const int32_t *gstart, const int32_t *col, int64_t Q, const int64_t *off,
                          const int64_t *qpos, int64_t total, const void *ws, int64_t *out_b, int64_t *out_e) {
    if (Q < 0 || total < 0) return fl::fl_fail(FL_ERR_ARG, "filter_expand: negative size");
    if (total == 0) return FL_OK;
    if (Q == 0 || !gstart || !col || !off || !qpos || !ws || !out_b || !out_e)
        return fl::fl_fail(FL_ERR_ARG, "filter_expand: null argument");
    const size_t q1 = (size_t)Q;
    const int64_t *gsel = (const int64_t *)((const char *)ws + fl::flt_al(sizeof(int32_t) * q1));
    FL_LAUNCH("k_flt_fill", fl::k_flt_fill, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
              (hipStream_t)stream, gstart, col, gsel, off, Q, qpos, total, out_b, out_e);
    return fl::fl_check_launch("filter_expand_fill");
}

}  // extern "C"
