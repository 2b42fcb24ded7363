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

// Workgroups of a launch go to the 8 XCDs round robin (workgroup g on XCD
// g % 8).  This maps workgroup g of a grid of G to an index such that every
// XCD takes one contiguous range of indices (work items that share cache
// lines at their edges then meet in one L2); a bijection on [0, G).
#define FL_XCDS 8
__device__ __forceinline__ int64_t fl_xcd_contig(int64_t g, int64_t G) {
    const int64_t q = G / FL_XCDS, rem = G % FL_XCDS, x = g % FL_XCDS, k = g / FL_XCDS;
    return x * q + (x < rem ? x : rem) + k;
}

__device__ __forceinline__ int fl_wave_incl_scan_i32(int v);
__device__ __forceinline__ long long fl_wave_incl_scan_i64(long long v);
__device__ __forceinline__ long long fl_readlane_i64(long long x, int l);

// Integer wave sums (any order gives the same total): the inclusive scan's
// last lane, uniform in scalar registers.
__device__ __forceinline__ int fl_wave_sum_i32(int v) {
    return __builtin_amdgcn_readlane(fl_wave_incl_scan_i32(v), FL_WAVE - 1);
}

__device__ __forceinline__ long long fl_wave_sum_i64(long long v) {
    return fl_readlane_i64(fl_wave_incl_scan_i64(v), FL_WAVE - 1);
}

// Butterfly sum of one float per lane (a fixed association, so the result
// is the same on every run); every lane receives the total.
__device__ __forceinline__ float fl_wave_sum_f32(float v) {
#pragma unroll
    for (int o = FL_WAVE / 2; o > 0; o >>= 1) v = fl_add(v, __shfl_xor(v, o, FL_WAVE));
    return v;
}

// A lane's value moved by a DPP control (gfx9 encodings: row_shr:n =
// 0x110 + n, row_bcast:15 = 0x142, row_bcast:31 = 0x143); lanes without a
// source, or outside row_mask / bank_mask, receive 0.
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ int fl_dpp(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, BANK_MASK, false);
}
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ long long fl_dpp64(long long v) {
    const unsigned long long u = (unsigned long long)v;
    const unsigned lo = (unsigned)fl_dpp<CTRL, ROW_MASK, BANK_MASK>((int)(unsigned)u);
    const unsigned hi = (unsigned)fl_dpp<CTRL, ROW_MASK, BANK_MASK>((int)(unsigned)(u >> 32));
    return (long long)(((unsigned long long)hi << 32) | lo);
}

// Inclusive prefix sum across the 64 lanes of a wave with DPP moves: the
// Hillis-Steele steps 1, 2, 4, 8 inside each row of 16 lanes, then row 0's
// total into row 1 and row 2's into row 3 (row_bcast:15), then the total of
// rows 0-1 into rows 2-3 (row_bcast:31).
__device__ __forceinline__ int fl_wave_incl_scan_i32(int v) {
    v += fl_dpp<0x111>(v);
    v += fl_dpp<0x112>(v);
    v += fl_dpp<0x114>(v);
    v += fl_dpp<0x118>(v);
    v += fl_dpp<0x142, 0xa>(v);
    v += fl_dpp<0x143, 0xc>(v);
    return v;
}

__device__ __forceinline__ long long fl_wave_incl_scan_i64(long long v) {
    v += fl_dpp64<0x111>(v);
    v += fl_dpp64<0x112>(v);
    v += fl_dpp64<0x114>(v);
    v += fl_dpp64<0x118>(v);
    v += fl_dpp64<0x142, 0xa>(v);
    v += fl_dpp64<0x143, 0xc>(v);
    return v;
}

// The previous lane's value (wave_shr:1); lane 0 receives 0.
__device__ __forceinline__ long long fl_wave_shr1_i64(long long v) { return fl_dpp64<0x138>(v); }

// Lane l's 64-bit value, in scalar registers.
__device__ __forceinline__ long long fl_readlane_i64(long long x, int l) {
    const unsigned long long u = (unsigned long long)x;
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)u, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(u >> 32), l);
    return (long long)(((unsigned long long)hi << 32) | lo);
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

// base[idx] with the byte offset computed in 32 bits (a scalar base plus a
// 32-bit vector offset is one load with no 64-bit address arithmetic); the
// caller guarantees idx * sizeof(T) < 2^32.
template <typename T>
__device__ __forceinline__ T fl_ld32(const T *base, uint32_t idx) {
    return *reinterpret_cast<const T *>(reinterpret_cast<const char *>(base) + (uint32_t)(idx * (uint32_t)sizeof(T)));
}

// base[idx] = v with the byte offset computed in 32 bits (as fl_ld32).
template <typename T>
__device__ __forceinline__ void fl_st32(T *base, uint32_t idx, T v) {
    *reinterpret_cast<T *>(reinterpret_cast<char *>(base) + (uint32_t)(idx * (uint32_t)sizeof(T))) = v;
}

// The wave's index within its workgroup, in a scalar register (so that
// per-wave indices, and loads at them, stay scalar).
__device__ __forceinline__ int fl_wave_id() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x / FL_WAVE)); }

// LDS ordering between the lanes of one wave (program order + fence).
__device__ __forceinline__ void fl_wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
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
