// Device-wide exclusive prefix sum (int32 or int64 input, int64 output) in
// three launches: per-tile totals, a scan of the tile totals by one
// workgroup, and the per-tile scan with its offset.  Used for the count ->
// offset steps of the sparse hop (entry item offsets, bucket bases, output
// offsets).  out may alias in for int64 input.
#include "fl_common.h"
#include "fl_abi.h"
#include "fl_scan.h"

namespace fl {

constexpr int SC_NT = 256;
constexpr int SC_IPT = 16;
constexpr int SC_TILE = SC_NT * SC_IPT;

template <typename T>
__global__ __launch_bounds__(SC_NT) void k_scan_tiles(const T *__restrict__ in, int64_t n,
                                                     int64_t *__restrict__ tile_sum) {
    __shared__ long long red[SC_NT / FL_WAVE];
    const int64_t base = (int64_t)blockIdx.x * SC_TILE;
    long long s = 0;
#pragma unroll
    for (int j = 0; j < SC_IPT; ++j) {
        const int64_t i = base + (int64_t)j * SC_NT + threadIdx.x;
        if (i < n) s += (long long)in[i];
    }
    s = fl_wave_sum_i64(s);
    if (fl_lane() == 0) red[threadIdx.x / FL_WAVE] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        long long t = 0;
        for (int k = 0; k < SC_NT / FL_WAVE; ++k) t += red[k];
        tile_sum[blockIdx.x] = t;
    }
}

// One workgroup: exclusive scan of the tile totals in place; total at [ntiles].
__global__ __launch_bounds__(SC_NT) void k_scan_totals(int64_t *__restrict__ tile_sum, int64_t ntiles) {
    __shared__ long long wsum[SC_NT / FL_WAVE];
    __shared__ long long carry;
    if (threadIdx.x == 0) carry = 0;
    __syncthreads();
    for (int64_t b0 = 0; b0 < ntiles; b0 += SC_NT) {
        const int64_t i = b0 + threadIdx.x;
        const long long v = i < ntiles ? tile_sum[i] : 0;
        const long long incl = fl_wave_incl_scan_i64(v);
        if (fl_lane() == FL_WAVE - 1) wsum[threadIdx.x / FL_WAVE] = incl;
        __syncthreads();
        long long wpre = 0, tot = 0;
        for (int k = 0; k < SC_NT / FL_WAVE; ++k) {
            if (k < (int)(threadIdx.x / FL_WAVE)) wpre += wsum[k];
            tot += wsum[k];
        }
        const long long c = carry;
        if (i < ntiles) tile_sum[i] = c + wpre + incl - v;
        __syncthreads();
        if (threadIdx.x == 0) carry = c + tot;
        __syncthreads();
    }
    if (threadIdx.x == 0) tile_sum[ntiles] = carry;
}

template <typename T>
__global__ __launch_bounds__(SC_NT) void k_scan_apply(const T *in, int64_t n, const int64_t *__restrict__ tile_sum,
                                                     int64_t *out) {
    __shared__ long long wsum[SC_NT / FL_WAVE];
    const int64_t base = (int64_t)blockIdx.x * SC_TILE;
    // blocked: thread t owns elements [base + t*IPT, +IPT)
    long long v[SC_IPT];
    long long s = 0;
#pragma unroll
    for (int j = 0; j < SC_IPT; ++j) {
        const int64_t i = base + (int64_t)threadIdx.x * SC_IPT + j;
        v[j] = i < n ? (long long)in[i] : 0;
        s += v[j];
    }
    const long long incl = fl_wave_incl_scan_i64(s);
    if (fl_lane() == FL_WAVE - 1) wsum[threadIdx.x / FL_WAVE] = incl;
    __syncthreads();
    long long run = tile_sum[blockIdx.x];
    for (int k = 0; k < (int)(threadIdx.x / FL_WAVE); ++k) run += wsum[k];
    run += incl - s;
#pragma unroll
    for (int j = 0; j < SC_IPT; ++j) {
        const int64_t i = base + (int64_t)threadIdx.x * SC_IPT + j;
        if (i < n) out[i] = run;
        run += v[j];
    }
    if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) out[n] = tile_sum[gridDim.x];
}

// One workgroup for at most one tile (n <= SC_TILE): every element read
// before any is written (out may alias in), one launch instead of three.
template <typename T>
__global__ __launch_bounds__(SC_NT) void k_scan_one(const T *in, int64_t n, int64_t *out) {
    __shared__ long long wsum[SC_NT / FL_WAVE];
    long long v[SC_IPT];
    long long s = 0;
#pragma unroll
    for (int j = 0; j < SC_IPT; ++j) {
        const int64_t i = (int64_t)threadIdx.x * SC_IPT + j;
        v[j] = i < n ? (long long)in[i] : 0;
        s += v[j];
    }
    const long long incl = fl_wave_incl_scan_i64(s);
    if (fl_lane() == FL_WAVE - 1) wsum[threadIdx.x / FL_WAVE] = incl;
    __syncthreads();
    long long run = 0, tot = 0;
    for (int k = 0; k < SC_NT / FL_WAVE; ++k) {
        if (k < (int)(threadIdx.x / FL_WAVE)) run += wsum[k];
        tot += wsum[k];
    }
    run += incl - s;
#pragma unroll
    for (int j = 0; j < SC_IPT; ++j) {
        const int64_t i = (int64_t)threadIdx.x * SC_IPT + j;
        if (i < n) out[i] = run;
        run += v[j];
    }
    if (threadIdx.x == 0) out[n] = tot;
}

size_t scan_tmp_bytes(int64_t n) {
    const int64_t nt = (n + SC_TILE - 1) / SC_TILE;
    return sizeof(int64_t) * (size_t)(nt + 1);
}

template <typename T>
static int scan_impl(hipStream_t st, const T *in, int64_t *out, int64_t n, int64_t *tmp) {
    if (n <= 0) {
        hipLaunchKernelGGL(k_scan_totals, dim3(1), dim3(SC_NT), 0, st, out, (int64_t)0);
        return fl_check_launch("exclusive_scan");
    }
    if (n <= SC_TILE) {
        FL_LAUNCH("k_scan_one", k_scan_one<T>, dim3(1), dim3(SC_NT), 0, st, in, n, out);
        return fl_check_launch("exclusive_scan");
    }
    const int64_t nt = (n + SC_TILE - 1) / SC_TILE;
    FL_LAUNCH("k_scan_tiles", k_scan_tiles<T>, dim3((unsigned)nt), dim3(SC_NT), 0, st, in, n, tmp);
    FL_LAUNCH("k_scan_totals", k_scan_totals, dim3(1), dim3(SC_NT), 0, st, tmp, nt);
    FL_LAUNCH("k_scan_apply", k_scan_apply<T>, dim3((unsigned)nt), dim3(SC_NT), 0, st, in, n, tmp, out);
    return fl_check_launch("exclusive_scan");
}

int exclusive_scan(hipStream_t st, const int32_t *in, int64_t *out, int64_t n, int64_t *tmp) {
    return scan_impl<int32_t>(st, in, out, n, tmp);
}

int exclusive_scan(hipStream_t st, const int64_t *in, int64_t *out, int64_t n, int64_t *tmp) {
    return scan_impl<int64_t>(st, in, out, n, tmp);
}

}  // namespace fl
