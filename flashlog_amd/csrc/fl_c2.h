// c2 edge budget shared by the dense and sparse kernels
// (flashlog.cpp:12-89, flashlog.cu:16-63,210-233,1342-1366).
#pragma once
#include "fl_common.h"
#include "../../include/flashlog_hip.h"

namespace fl {

// Wave-level c2 threshold for one (source, row, direction): the weighted
// order statistic of flashlog.cpp:12-35 by MSB-first radix select over the
// float bits of the group weights (4 passes of 8 bits, group sizes as
// multiplicities), then the tie-quota cut: ties are admitted in group order,
// so the admitted tied edges are exactly the positions below `cut`.
// Returns false when every eligible edge fits (no pruning).
static __device__ bool c2_select(const fl_side &s, int64_t g0, int64_t g1, const float *wrow,
                          int64_t K, int *hist, uint32_t *th_key, int32_t *cut) {
    const int lane = fl_lane();
    long long tot = 0;
    for (int64_t g = g0 + lane; g < g1; g += FL_WAVE) {
        float wv = wrow[s.group_rel[g]];
        if (wv > 0.0f) tot += s.group_count[g];
    }
    tot = fl_wave_sum_i64(tot);
    if (tot <= K) return false;
    int need = (int)K;
    uint32_t prefix = 0, pmask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        hist[lane * 4 + 0] = 0; hist[lane * 4 + 1] = 0;
        hist[lane * 4 + 2] = 0; hist[lane * 4 + 3] = 0;
        __builtin_amdgcn_wave_barrier();
        for (int64_t g = g0 + lane; g < g1; g += FL_WAVE) {
            float wv = wrow[s.group_rel[g]];
            uint32_t k = __float_as_uint(wv);
            if (wv > 0.0f && (k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & 255], s.group_count[g]);
        }
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const int owner = FL_WAVE - 1 - lane;
        int h[4];
        int v = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) { h[k] = hist[owner * 4 + k]; v += h[k]; }
        int incl = fl_wave_incl_scan_i32(v);
        int above = incl - v;
        int found = 0, digit = 0, nneed = 0;
#pragma unroll
        for (int k = 3; k >= 0; --k) {
            if (!found && above < need && need <= above + h[k]) { found = 1; digit = owner * 4 + k; nneed = need - above; }
            above += h[k];
        }
        unsigned long long bal = __ballot(found);
        int src_lane = __ffsll((long long)bal) - 1;
        digit = __shfl(digit, src_lane, FL_WAVE);
        nneed = __shfl(nneed, src_lane, FL_WAVE);
        prefix |= (uint32_t)digit << shift;
        pmask |= 0xFFu << shift;
        need = nneed;
        __builtin_amdgcn_wave_barrier();
    }
    // cut: first tied group whose cumulative tie count passes `need`
    int run = 0;
    int32_t c = 0x7FFFFFFF;
    for (int64_t base = g0; base < g1; base += FL_WAVE) {
        const int64_t g = base + lane;
        int cnt = 0;
        int st = 0;
        if (g < g1) {
            float wv = wrow[s.group_rel[g]];
            if (wv > 0.0f && __float_as_uint(wv) == prefix) { cnt = s.group_count[g]; st = s.group_start[g]; }
        }
        int incl = fl_wave_incl_scan_i32(cnt);
        int before = run + incl - cnt;
        int hit = (cnt > 0) && (before + cnt > need);
        unsigned long long bal = __ballot(hit);
        if (bal) {
            int hl = __ffsll((long long)bal) - 1;
            c = __shfl(st + (need - before), hl, FL_WAVE);
            break;
        }
        run += __shfl(incl, FL_WAVE - 1, FL_WAVE);
    }
    *th_key = prefix;
    *cut = c;
    return true;
}

// c2_select for a side of at most one window of groups: lane j reads group
// g0 + j once and every pass (the total, the four radix passes and the cut)
// works from registers.  Same threshold and cut as the general form.  (The
// dense hard-case kernel takes it; in the sparse selection, whose sides
// mostly stop at the total, it measured slower.)
static __device__ bool c2_select_window(const fl_side &s, int64_t g0, int64_t g1, const float *wrow, int64_t K,
                                        int *hist, uint32_t *th_key, int32_t *cut) {
    const int lane = fl_lane();
    const int64_t g = g0 + lane;
    float wv = 0.0f;
    int cnt = 0, st = 0;
    if (g < g1) {
        wv = wrow[s.group_rel[g]];
        cnt = s.group_count[g];
        st = s.group_start[g];
    }
    const bool el = wv > 0.0f;  // (groups past the end have wv 0)
    const uint32_t k = __float_as_uint(wv);
    const long long tot = fl_wave_sum_i64(el ? cnt : 0);
    if (tot <= K) return false;
    int need = (int)K;
    uint32_t prefix = 0, pmask = 0;
    for (int shift = 24; shift >= 0; shift -= 8) {
        hist[lane * 4 + 0] = 0; hist[lane * 4 + 1] = 0;
        hist[lane * 4 + 2] = 0; hist[lane * 4 + 3] = 0;
        __builtin_amdgcn_wave_barrier();
        if (el && (k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & 255], cnt);
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        const int owner = FL_WAVE - 1 - lane;
        int h[4];
        int v = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) { h[q] = hist[owner * 4 + q]; v += h[q]; }
        int incl = fl_wave_incl_scan_i32(v);
        int above = incl - v;
        int found = 0, digit = 0, nneed = 0;
#pragma unroll
        for (int q = 3; q >= 0; --q) {
            if (!found && above < need && need <= above + h[q]) { found = 1; digit = owner * 4 + q; nneed = need - above; }
            above += h[q];
        }
        unsigned long long bal = __ballot(found);
        int src_lane = __ffsll((long long)bal) - 1;
        digit = __shfl(digit, src_lane, FL_WAVE);
        nneed = __shfl(nneed, src_lane, FL_WAVE);
        prefix |= (uint32_t)digit << shift;
        pmask |= 0xFFu << shift;
        need = nneed;
        __builtin_amdgcn_wave_barrier();
    }
    // cut: first tied group whose cumulative tie count passes `need`
    const int tc = (el && k == prefix) ? cnt : 0;
    const int incl = fl_wave_incl_scan_i32(tc);
    const int before = incl - tc;
    const unsigned long long bal = __ballot(tc > 0 && before + tc > need);
    int32_t c = 0x7FFFFFFF;
    if (bal) {
        const int hl = __ffsll((long long)bal) - 1;
        c = __shfl(st + (need - before), hl, FL_WAVE);
    }
    *th_key = prefix;
    *cut = c;
    return true;
}

// c2_select, with sides of at most one window from registers.
static __device__ __forceinline__ bool c2_select_fast(const fl_side &s, int64_t g0, int64_t g1, const float *wrow,
                                                      int64_t K, int *hist, uint32_t *th_key, int32_t *cut) {
    if (g1 - g0 <= FL_WAVE) return c2_select_window(s, g0, g1, wrow, K, hist, th_key, cut);
    return c2_select(s, g0, g1, wrow, K, hist, th_key, cut);
}

// group_take in 32 bits (CSR positions and group sizes are int32, so the
// tie difference cut - start cannot overflow).
__device__ __forceinline__ int32_t group_take32(float wv, float th, int32_t cut, int32_t start, int32_t count) {
    if (!(wv > 0.0f)) return 0;
    if (wv > th) return count;
    if (wv == th) {
        const int32_t t = cut - start;
        return t <= 0 ? 0 : (t < count ? t : count);
    }
    return 0;
}

// Kept range of group g for (source, row): [start, start + take).
__device__ __forceinline__ int64_t group_take(float wv, float th, int32_t cut, int64_t start, int64_t count) {
    if (!(wv > 0.0f)) return 0;
    if (wv > th) return count;
    if (wv == th) {
        const int64_t t = (int64_t)cut - start;
        return t <= 0 ? 0 : (t < count ? t : count);
    }
    return 0;
}

}  // namespace fl
