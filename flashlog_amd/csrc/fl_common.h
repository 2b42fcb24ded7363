// Shared device helpers for the gfx950 FlashLog kernels (wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define FL_WAVE 64

// Explicitly rounded float ops: the bit-exact paths must never be contracted
// into FMAs (the reference CPU path evaluates (a*w)*m then adds).
__device__ __forceinline__ float fl_mul(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float fl_add(float a, float b) { return __fadd_rn(a, b); }

__device__ __forceinline__ int fl_lane() { return threadIdx.x & (FL_WAVE - 1); }

__device__ __forceinline__ int fl_wave_sum_i32(int v) {
#pragma unroll
    for (int o = FL_WAVE / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, FL_WAVE);
    return v;
}

__device__ __forceinline__ long long fl_wave_sum_i64(long long v) {
#pragma unroll
    for (int o = FL_WAVE / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, FL_WAVE);
    return v;
}

// Butterfly sum of one float per lane (a fixed association, so the result
// is the same on every run); every lane receives the total.
__device__ __forceinline__ float fl_wave_sum_f32(float v) {
#pragma unroll
    for (int o = FL_WAVE / 2; o > 0; o >>= 1) v = fl_add(v, __shfl_xor(v, o, FL_WAVE));
    return v;
}

// Inclusive prefix sum across the 64 lanes of a wave.
__device__ __forceinline__ int fl_wave_incl_scan_i32(int v) {
    const int lane = fl_lane();
#pragma unroll
    for (int o = 1; o < FL_WAVE; o <<= 1) {
        int t = __shfl_up(v, o, FL_WAVE);
        if (lane >= o) v += t;
    }
    return v;
}

__device__ __forceinline__ long long fl_wave_incl_scan_i64(long long v) {
    const int lane = fl_lane();
#pragma unroll
    for (int o = 1; o < FL_WAVE; o <<= 1) {
        long long t = __shfl_up(v, o, FL_WAVE);
        if (lane >= o) v += t;
    }
    return v;
}

// Block-wide exclusive scan of one int per thread (NT threads, NT % 64 == 0,
// NT <= 1024).  lds must hold NT/64 + 1 ints.  Returns the exclusive prefix;
// *total receives the block sum.  Contains __syncthreads.
template <int NT>
__device__ __forceinline__ int fl_block_excl_scan(int v, int *lds, int *total) {
    constexpr int NW = NT / FL_WAVE;
    const int lane = fl_lane();
    const int wid = threadIdx.x / FL_WAVE;
    int incl = fl_wave_incl_scan_i32(v);
    if (lane == FL_WAVE - 1) lds[wid] = incl;
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0;
        for (int i = 0; i < NW; ++i) { int t = lds[i]; lds[i] = run; run += t; }
        lds[NW] = run;
    }
    __syncthreads();
    int res = lds[wid] + incl - v;
    *total = lds[NW];
    __syncthreads();
    return res;
}

// A wave-uniform value moved to scalar registers (the value of the first
// active lane; every lane must hold the same value).
__device__ __forceinline__ long long fl_uniform_i64(long long x) {
    const int lo = __builtin_amdgcn_readfirstlane((int)(unsigned long long)x);
    const int hi = __builtin_amdgcn_readfirstlane((int)((unsigned long long)x >> 32));
    return (long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo);
}
__device__ __forceinline__ double fl_uniform_f64(double x) {
    return __longlong_as_double(fl_uniform_i64(__double_as_longlong(x)));
}

// Float key that orders like the value (ascending) for every non-NaN float.
__device__ __forceinline__ uint32_t fl_order_key(float v) {
    uint32_t u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// SplitMix64 output function (Steele, Lea and Flood 2014; the public-domain
// splitmix64.c of Vigna): one step from state z.
__device__ __forceinline__ uint64_t fl_splitmix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
