// c1 entity budget helpers shared by the dense and sparse kernels
// (flashlog_kernel.py:814-842, 1092-1140): block radix select over the
// order-preserving float keys.
#pragma once
#include "fl_common.h"

namespace fl {

constexpr int TOPC_NT = 1024;

template <int NBINS>
__device__ __forceinline__ void topc_select(const int *hist, int need, int *lds_scan,
                                            int *sel_bin, int *sel_need) {
    constexpr int PER = NBINS / TOPC_NT;  // bins per thread (1 or 2)
    const int t = threadIdx.x;
    const int owner = TOPC_NT - 1 - t;    // reversed ownership: scan gives suffix sums
    int v = 0;
#pragma unroll
    for (int k = 0; k < PER; ++k) v += hist[owner * PER + k];
    int total;
    int above = fl_block_excl_scan<TOPC_NT>(v, lds_scan, &total);
#pragma unroll
    for (int k = PER - 1; k >= 0; --k) {
        int b = owner * PER + k;
        int h = hist[b];
        if (above < need && need <= above + h) { *sel_bin = b; *sel_need = need - above; }
        above += h;
    }
    __syncthreads();
}

// Loads of TOPC_U elements per thread are issued together before their use.
constexpr int TOPC_U = 16;

#define TOPC_FOR_ROW(BODY)                                                        \
    for (int64_t base_ = 0; base_ < E; base_ += (int64_t)TOPC_NT * TOPC_U) {      \
        float v_[TOPC_U];                                                         \
        _Pragma("unroll") for (int u_ = 0; u_ < TOPC_U; ++u_) {                   \
            const int64_t e_ = base_ + (int64_t)u_ * TOPC_NT + t;                 \
            v_[u_] = e_ < E ? a[e_] : 0.0f;                                       \
        }                                                                         \
        _Pragma("unroll") for (int u_ = 0; u_ < TOPC_U; ++u_) {                   \
            const int64_t e = base_ + (int64_t)u_ * TOPC_NT + t;                  \
            const float v = v_[u_];                                               \
            if (e < E) { BODY }                                                   \
        }                                                                         \
    }

}  // namespace fl
