// Dense-state propagation kernels for gfx950 (MI355X) and their C-ABI.
//
// One hop of the reference's dense sum path (flashlog.cu:898-995, with the
// CPU path's accumulation order, flashlog.cpp:151-211):
//
//   k_col_count      identity output and the row bitmask BM[word][source]
//                    (thread per (source, 32-row word), coalesced over sources).
//   k_frontier       per active source: the record PK[dir][source][row] =
//                    {a, theta, cut} of each nonzero (source, row), and the
//                    list of pairs whose source exceeds the c2 budget.
//   k_c2_hard        one wave per listed pair: the c2 threshold and tie cut
//                    from a wave-level radix select over the source's
//                    relation groups.
//   k_pull           the propagation: one thread per (light destination,
//                    row) walks the destination's incoming slots (staged in
//                    LDS) in ascending CSR position and adds (a*w)*m in a
//                    register -- the order in which the reference's CPU loop
//                    adds into out[row, dst] -- with tiles of destinations
//                    written coalesced from LDS; destinations with more than FL_SEG
//                    incoming slots are cut into FL_SEG-slot segments whose
//                    kept products are listed, in slot order, per row.
//   k_heavy_offsets  per heavy destination and row, where each segment's list
//   k_heavy_copy     goes in one contiguous run per row, and the copy there.
//   k_fold_heavy     the runs added in order, staged through LDS: the same
//                    sequence of additions as a single walk.
//
// No atomics touch output values, so results are deterministic and equal to
// the reference CPU bits.
#include "fl_common.h"
#include "fl_abi.h"
#include "fl_c2.h"
#include "fl_topc.h"

namespace fl {

// ---------------------------------------------------------------------------
// Masks and active flags

template <typename MT>
__global__ void k_apply_mask(const MT *__restrict__ mask, const int32_t *__restrict__ order,
                             const float *__restrict__ weight, float *__restrict__ out,
                             int64_t nnz) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nnz) return;
    int64_t idx = order[i];
    float m = (float)mask[idx];
    if (weight != nullptr) {
        float wv = weight[idx];
        m = m * (1.0f / (1.0f + expf(-wv)));
    }
    out[i] = m;
}

// out[i] = 1 - sigmoid(weight[order[i]]): the edge-score derivative factor
// of the sparse backward (flashlog_kernel.py:1306-1336), the sigmoid of
// k_apply_mask.
__global__ void k_edge_dscore(const float *__restrict__ weight, const int32_t *__restrict__ order,
                              float *__restrict__ out, int64_t nnz) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nnz) return;
    out[i] = 1.0f - 1.0f / (1.0f + expf(-weight[order[i]]));
}

__global__ void k_mark_active(const float *__restrict__ A, int32_t *__restrict__ flags,
                              int64_t BL, int64_t E) {
    int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    int f = 0;
    for (int64_t bl = 0; bl < BL; ++bl)
        if (A[bl * E + e] != 0.0f) { f = 1; break; }
    flags[e] = f;
}

// ---------------------------------------------------------------------------
// c1 entity budget (flashlog_kernel.py:814-842): one 1024-thread workgroup per
// row; exact radix select (11/11/10 bits) of the c-th largest nonzero, then an
// ordered scan for the last kept tie.

__global__ __launch_bounds__(TOPC_NT) void k_topc_rows(const float *__restrict__ A,
                                                        float *__restrict__ out, int64_t E,
                                                        int64_t c, int32_t *__restrict__ row_state) {
    __shared__ int hist[2048];
    __shared__ int lds_scan[TOPC_NT / FL_WAVE + 1];
    __shared__ int sel_bin, sel_need, s_last, s_done;
    const int64_t row = blockIdx.x;
    const float *a = A + row * E;
    float *o = out + row * E;
    const int t = threadIdx.x;

    for (int i = t; i < 2048; i += TOPC_NT) hist[i] = 0;
    __syncthreads();
    int nz_local = 0;
    TOPC_FOR_ROW(if (v != 0.0f) { ++nz_local; atomicAdd(&hist[fl_order_key(v) >> 21], 1); })
    int nz;
    (void)fl_block_excl_scan<TOPC_NT>(nz_local, lds_scan, &nz);
    const bool over = (int64_t)nz > c;
    uint32_t cutkey = 0;
    int64_t last = -1;
    if (over && c > 0) {
        // pass 1: bits [31:21]
        topc_select<2048>(hist, (int)c, lds_scan, &sel_bin, &sel_need);
        uint32_t prefix = (uint32_t)sel_bin << 21;
        int need = sel_need;
        // pass 2: bits [20:10]
        for (int i = t; i < 2048; i += TOPC_NT) hist[i] = 0;
        __syncthreads();
        TOPC_FOR_ROW(const uint32_t k = fl_order_key(v);
                     if (v != 0.0f && (k >> 21) == (prefix >> 21)) atomicAdd(&hist[(k >> 10) & 2047], 1);)
        __syncthreads();
        topc_select<2048>(hist, need, lds_scan, &sel_bin, &sel_need);
        prefix |= (uint32_t)sel_bin << 10;
        need = sel_need;
        // pass 3: bits [9:0]
        for (int i = t; i < 2048; i += TOPC_NT) hist[i] = 0;
        __syncthreads();
        TOPC_FOR_ROW(const uint32_t k = fl_order_key(v);
                     if (v != 0.0f && (k >> 10) == (prefix >> 10)) atomicAdd(&hist[k & 1023], 1);)
        __syncthreads();
        topc_select<1024>(hist, need, lds_scan, &sel_bin, &sel_need);
        prefix |= (uint32_t)sel_bin;
        need = sel_need;               // ties (key == cutkey) to keep, >= 1
        const int tied_total = hist[sel_bin];
        cutkey = prefix;
        if (need >= tied_total) {
            last = E;
        } else {
            // ordered scan for the need-th tie in ascending entity order
            if (t == 0) { s_last = -1; s_done = 0; }
            __syncthreads();
            int run = 0;
            for (int64_t base = 0; base < E; base += TOPC_NT) {
                int64_t e = base + t;
                int flag = 0;
                if (e < E) {
                    float v = a[e];
                    flag = (v != 0.0f && fl_order_key(v) == cutkey) ? 1 : 0;
                }
                int tot;
                int ex = fl_block_excl_scan<TOPC_NT>(flag, lds_scan, &tot);
                if (flag && run + ex + 1 == need) { s_last = (int)e; s_done = 1; }
                run += tot;
                __syncthreads();
                if (s_done) break;
            }
            last = s_last;
        }
    }
    // apply: out = A * keep  (keep as 1.0f / 0.0f, like the reference's A * keep)
    TOPC_FOR_ROW(bool keep = true;
                 if (over) {
                     keep = false;
                     if (c > 0 && v != 0.0f) {
                         const uint32_t k = fl_order_key(v);
                         keep = (k > cutkey) || (k == cutkey && e <= last);
                     }
                 }
                 o[e] = v * (keep ? 1.0f : 0.0f);)
    if (t == 0) {
        row_state[row * 4 + 0] = over ? 1 : 0;
        row_state[row * 4 + 1] = (int32_t)cutkey;
        row_state[row * 4 + 2] = (int32_t)last;
        row_state[row * 4 + 3] = nz;
    }
}

__global__ void k_topc_backward(const float *__restrict__ grad, const float *__restrict__ A,
                                const int32_t *__restrict__ row_state, float *__restrict__ gA,
                                int64_t E) {
    const int64_t row = blockIdx.y;
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const int over = row_state[row * 4 + 0];
    const uint32_t cutkey = (uint32_t)row_state[row * 4 + 1];
    const int64_t last = row_state[row * 4 + 2];
    const int64_t i = row * E + e;
    bool keep = true;
    if (over) {
        float v = A[i];
        keep = false;
        if (last >= 0 && v != 0.0f) {  // last < 0 only when c == 0
            uint32_t k = fl_order_key(v);
            keep = (k > cutkey) || (k == cutkey && e <= last);
        }
    }
    gA[i] = grad[i] * (keep ? 1.0f : 0.0f);
}

// ---------------------------------------------------------------------------
// Dense sum forward
//
// Per-(source, row) record PK[dir][src][row] = {a, theta}: the state value
// and the c2 threshold of that source in that row and direction; the tie cut
// CUT[dir][src][row] is written only where theta > 0.  An edge at position p
// of relation weight w is kept iff w > theta, or w == theta > 0 and p < cut
// (theta = 0 admits every w > 0 edge).  Records exist only for nonzero
// (source, row) pairs; the row bitmask BM[word][src] says which.

constexpr int COL_NT = 256;

// One thread per (source, 32-row word): identity output (skipped when
// out_ind is null) and the bitmask word.
// Threads of a wave cover consecutive sources of the same rows (coalesced);
// the 32 loads of a word are issued before use.
__global__ __launch_bounds__(COL_NT) void k_col_count(
    const float *__restrict__ A, const float *__restrict__ w, int64_t BL, int64_t E, int64_t n,
    int wot_i, float *__restrict__ out_ind, uint32_t *__restrict__ BM, int32_t *__restrict__ hard_count) {
    const int64_t q = (int64_t)blockIdx.x * COL_NT + threadIdx.x;
    if (q == 0) *hard_count = 0;
    const int64_t nw = (BL + 31) / 32;
    if (q >= nw * E) return;
    const int64_t wi = q / E, e = q - wi * E;
    const int64_t b0 = wi * 32;
    const int nb = (int)((b0 + 32 < BL) ? 32 : BL - b0);
    float v[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) v[k] = (k < nb) ? A[(b0 + k) * E + e] : 0.0f;
    uint32_t bits = 0;
#pragma unroll
    for (int k = 0; k < 32; ++k) {
        if (k < nb) {
            if (out_ind) {
                const float wid = w[(b0 + k) * n + (n - 1)];
                out_ind[(b0 + k) * E + e] = wot_i ? 0.0f : fl_mul(v[k], wid);
            }
            if (v[k] != 0.0f) bits |= 1u << k;
        }
    }
    BM[wi * E + e] = bits;
}

__device__ __forceinline__ void row_positions(const fl_side &s, int64_t src, int64_t *p0, int64_t *p1) {
    const int64_t g0 = s.row_group_ptr[src], g1 = s.row_group_ptr[src + 1];
    if (g1 > g0) {
        *p0 = s.group_start[g0];
        *p1 = (int64_t)s.group_start[g1 - 1] + s.group_count[g1 - 1];
    } else {
        *p0 = 0; *p1 = 0;
    }
}

// One thread per source: records of every nonzero (source, row).  Rows of a
// source whose out-degree on a side exceeds the c2 budget go to the hard list
// (entry = src * 4 + dirmask, row) for the wave-level selection.
__global__ __launch_bounds__(COL_NT) void k_frontier(
    fl_side ori, fl_side inv, const float *__restrict__ A, int64_t BL, int64_t E, int64_t K, int do_topk,
    const uint32_t *__restrict__ BM, float2 *__restrict__ PK, int32_t *__restrict__ hard_count,
    int2 *__restrict__ hard) {
    const int64_t e = (int64_t)blockIdx.x * COL_NT + threadIdx.x;
    if (e >= E) return;
    const int64_t nw = (BL + 31) / 32;
    int cnt = 0;
    for (int64_t wi = 0; wi < nw; ++wi) cnt += __popc(BM[wi * E + e]);
    if (cnt == 0) return;
    int dirmask = 0;
    if (do_topk) {
        int64_t p0, p1;
        row_positions(ori, e, &p0, &p1);
        if (p1 - p0 > K) dirmask |= 1;
        row_positions(inv, e, &p0, &p1);
        if (p1 - p0 > K) dirmask |= 2;
    }
    int slot = 0;
    if (dirmask) slot = atomicAdd(hard_count, cnt);
    float2 *pk0 = PK + e * BL;
    float2 *pk1 = PK + (E + e) * BL;
    for (int64_t wi = 0; wi < nw; ++wi) {
        uint32_t bits = BM[wi * E + e];
        while (bits) {
            int bb[8];
            float av[8];
            int m = 0;
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (bits) {
                    bb[u] = __ffs(bits) - 1;
                    bits &= bits - 1;
                    m = u + 1;
                    av[u] = A[(wi * 32 + bb[u]) * E + e];
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (u < m) {
                    const int64_t bl = wi * 32 + bb[u];
                    const float2 r = make_float2(av[u], 0.0f);
                    pk0[bl] = r;
                    pk1[bl] = r;
                    if (dirmask) hard[slot++] = make_int2((int)(e * 4 + dirmask), (int)bl);
                }
            }
        }
    }
}

constexpr int C2_NT = 256;

// One wave per hard (source, row): the c2 selection for each flagged side.
__global__ __launch_bounds__(C2_NT) void k_c2_hard(fl_side ori, fl_side inv, const float *__restrict__ w,
                                                   int64_t BL, int64_t E, int64_t n, int64_t r_size, int64_t K,
                                                   const int32_t *__restrict__ hard_count,
                                                   const int2 *__restrict__ hard, float2 *__restrict__ PK,
                                                   int32_t *__restrict__ CUT) {
    __shared__ int hist_all[C2_NT / FL_WAVE][256];
    const int lane = fl_lane();
    const int wid = fl_wave_id();
    int *hist = hist_all[wid];
    const int64_t nwaves = (int64_t)gridDim.x * (C2_NT / FL_WAVE);
    const int64_t total = *hard_count;
    for (int64_t j = (int64_t)blockIdx.x * (C2_NT / FL_WAVE) + wid; j < total; j += nwaves) {
        const int2 hj = hard[j];
        const int64_t src = hj.x >> 2;
        const int dm = hj.x & 3;
        const int64_t bl = hj.y;
        for (int dir = 0; dir < 2; ++dir) {
            if (!(dm & (1 << dir))) continue;
            const fl_side &s = dir ? inv : ori;
            const int64_t g0 = s.row_group_ptr[src], g1 = s.row_group_ptr[src + 1];
            uint32_t k2; int32_t c2;
            if (c2_select_fast(s, g0, g1, w + bl * n + (dir ? r_size : 0), K, hist, &k2, &c2) && lane == 0) {
                const int64_t at = ((int64_t)dir * E + src) * BL + bl;
                PK[at].y = __uint_as_float(k2);
                CUT[at] = c2;
            }
        }
    }
}

// Slots whose weight and record loads are requested together in a walk.
constexpr int WALK_U = 8;

// Max: the largest packed key (value bits << 32 | ~position) of the kept
// products, 0 when none (flashlog.cu:104-121): larger value bits win, equal
// bits go to the smaller position.
__device__ __forceinline__ uint64_t max_key(float v, int pos) {
    return ((uint64_t)__float_as_uint(v) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)pos);
}

constexpr int PULL_NT = 256;
constexpr int MAX_TD = 16;  // destinations per light tile, at most
constexpr int SUM_TD = 8;   // the sum's tiles: smaller LDS, more workgroups per CU (C2: k_pull 0.117 -> 0.081 ms)
constexpr int HEAVY_BL = 64;

// Dynamic LDS of a light k_pull tile: the output tile (2 x BL x TD floats)
// and the staged slots of both sides.
inline size_t pull_lds_bytes(int64_t BL, int TD) {
    const int64_t nw = (BL + 31) / 32;
    return sizeof(float) * 2 * (size_t)BL * (size_t)TD + (size_t)2 * TD * FL_SEG * (16 + 4 * (size_t)nw);
}
constexpr int HEAVY_TASKS = FL_SUP * HEAVY_BL;  // (segment, row) tasks of one heavy block

// The propagation kernel.  Workgroups [nheavy_wg, +nlight) take tiles of TD
// destinations: the light ones' slots (in-degree <= FL_SEG) are staged in
// LDS, one thread per (destination, row) walks the destination's slots in
// ascending CSR position and adds in a register -- the reference CPU loop's
// order -- then the tile is written from LDS, coalesced.  Light tiles are dealt to XCDs in contiguous ranges
// (workgroup b runs on XCD b % 8), so each output line is written from one
// L2.  Workgroups [0, nheavy_wg) -- the longer ones, dispatched first --
// take (supersegment, block of 64 rows) of heavy
// destinations: thread (segment, row) records its kept products in slot order
// (list, cnt), the offset of its run inside the supersegment (loff) and the
// supersegment's per-row total (stot); the fold finishes those rows.
__global__ __launch_bounds__(PULL_NT) void k_pull(
    fl_side ori, fl_side inv, const float *__restrict__ w, int64_t BL, int64_t E, int64_t n, int64_t r_size,
    int TD, int64_t ntiles, int64_t nlight, int64_t nheavy_wg, const uint32_t *__restrict__ BM,
    const float2 *__restrict__ PK,
    const int32_t *__restrict__ CUT, float *__restrict__ out_ori, float *__restrict__ out_inv,
    float *__restrict__ list_ori, float *__restrict__ list_inv, int32_t *__restrict__ cnt_ori,
    int32_t *__restrict__ cnt_inv, int32_t *__restrict__ loff_ori, int32_t *__restrict__ loff_inv,
    int32_t *__restrict__ stot_ori, int32_t *__restrict__ stot_inv) {
    extern __shared__ __align__(16) unsigned char pull_lds[];
    __shared__ int cnt_lds[FL_SUP][HEAVY_BL];
    __shared__ int32_t lfirst[2][MAX_TD], lpre[2][MAX_TD + 1];
    if ((int64_t)blockIdx.x >= nheavy_wg) {
        // light tile: the tile's light slots (destinations of in-degree <=
        // FL_SEG, listed through an LDS prefix of their counts) staged in
        // LDS -- source, position, relation, mask and the source's row words
        // -- then thread per (destination, row) walks its destination's
        // slots from LDS in CSR position order, reading a slot's weight and
        // record only where the source is active in the row
        const int64_t lb = (int64_t)blockIdx.x - nheavy_wg;  // nheavy_wg is a multiple of 8
        const int64_t per = nlight / 8;
        const int64_t tid = (lb % 8) * per + lb / 8;
        if (tid >= ntiles) return;
        const int64_t d0 = tid * TD;
        const int nd = (int)(E - d0 < TD ? E - d0 : TD);
        const int64_t nw = (BL + 31) / 32;
        const int S = TD * FL_SEG;  // light slots of a side in one tile, at most
        float *tile = reinterpret_cast<float *>(pull_lds);  // [2][BL][TD]
        int32_t *st_src = reinterpret_cast<int32_t *>(tile + 2 * BL * TD);  // [2][S]
        int32_t *st_pos = st_src + 2 * S;
        int32_t *st_rel = st_pos + 2 * S;
        float *st_m = reinterpret_cast<float *>(st_rel + 2 * S);
        uint32_t *st_w = reinterpret_cast<uint32_t *>(st_m + 2 * S);  // [2][S][nw]
        if (threadIdx.x < 2 * FL_WAVE) {
            const int dir = threadIdx.x / FL_WAVE, j = fl_lane();
            const fl_side &s = dir ? inv : ori;
            int32_t c = 0;
            if (j < nd) {
                const int64_t p0 = s.pull_ptr[d0 + j], p1 = s.pull_ptr[d0 + j + 1];
                lfirst[dir][j] = (int32_t)p0;
                c = p1 - p0 <= FL_SEG ? (int32_t)(p1 - p0) : 0;
            }
            const int32_t incl = fl_wave_incl_scan_i32(c);
            if (j < nd) lpre[dir][j + 1] = incl;
            if (j == 0) lpre[dir][0] = 0;
        }
        __syncthreads();
#pragma unroll
        for (int dir = 0; dir < 2; ++dir) {
            const fl_side &s = dir ? inv : ori;
            const int32_t *pp = lpre[dir], *fs = lfirst[dir];
            for (int k = threadIdx.x; k < pp[nd]; k += PULL_NT) {
                int lo = 0, hi = nd;  // the destination: pp[lo] <= k < pp[lo + 1]
                while (hi - lo > 1) {
                    const int mid = (lo + hi) >> 1;
                    if (pp[mid] <= k) lo = mid;
                    else hi = mid;
                }
                const int64_t sl = fs[lo] + (k - pp[lo]);
                const int32_t src = s.pull_src[sl], pos = s.pull_pos[sl];
                const int at = dir * S + k;
                st_src[at] = src;
                st_pos[at] = pos;
                st_rel[at] = s.pull_rel[sl];
                st_m[at] = s.mask[pos];
                for (int64_t wi = 0; wi < nw; ++wi) st_w[(int64_t)at * nw + wi] = BM[wi * E + src];
            }
        }
        __syncthreads();
        const int64_t ntask = (int64_t)nd * BL;
        for (int64_t q = threadIdx.x; q < ntask; q += PULL_NT) {
            const int64_t dl = q / BL, bl = q - dl * BL;
            const int64_t wi = bl >> 5;
            const uint32_t bit = 1u << (bl & 31);
#pragma unroll
            for (int dir = 0; dir < 2; ++dir) {
                const int k0 = lpre[dir][dl], k1 = lpre[dir][dl + 1];
                const float *wr = w + bl * n + (dir ? r_size : 0);
                const int64_t plane = (int64_t)dir * E * BL + bl;
                float acc = 0.0f;
                for (int kb = k0; kb < k1; kb += WALK_U) {
                    bool act[WALK_U];
                    float wv[WALK_U];
                    float2 rc[WALK_U];
#pragma unroll
                    for (int u = 0; u < WALK_U; ++u) {
                        const int at = dir * S + kb + u;
                        act[u] = kb + u < k1 && (st_w[(int64_t)at * nw + wi] & bit) && st_m[at] != 0.0f;
                        wv[u] = 0.0f;
                        rc[u] = make_float2(0.0f, 0.0f);
                        if (act[u]) {
                            wv[u] = wr[st_rel[at]];
                            rc[u] = PK[plane + (int64_t)st_src[at] * BL];
                        }
                    }
#pragma unroll
                    for (int u = 0; u < WALK_U; ++u) {
                        if (!act[u] || !(wv[u] > 0.0f)) continue;
                        const int at = dir * S + kb + u;
                        bool kept = wv[u] > rc[u].y;
                        if (!kept && wv[u] == rc[u].y) kept = st_pos[at] < CUT[plane + (int64_t)st_src[at] * BL];
                        if (kept) acc = fl_add(acc, fl_mul(fl_mul(rc[u].x, wv[u]), st_m[at]));
                    }
                }
                tile[(dir * BL + bl) * TD + dl] = acc;
            }
        }
        __syncthreads();
        for (int64_t i = threadIdx.x; i < (int64_t)TD * BL; i += PULL_NT) {
            const int64_t bl = i / TD, dl = i - bl * TD;
            if (dl < nd) {
                out_ori[bl * E + d0 + dl] = tile[(0 * BL + bl) * TD + dl];
                out_inv[bl * E + d0 + dl] = tile[(1 * BL + bl) * TD + dl];
            }
        }
        return;
    }
    // heavy block
    const int64_t nblc = (BL + HEAVY_BL - 1) / HEAVY_BL;
    const int64_t hb = blockIdx.x;
    const int64_t supg = hb / nblc;
    const int64_t blc = hb - supg * nblc;
    if (supg >= ori.nsup + inv.nsup) return;  // padding of the heavy range
    const int dir = supg >= ori.nsup;
    const int64_t sup = dir ? supg - ori.nsup : supg;
    const fl_side &s = dir ? inv : ori;
    const int64_t h = s.sup_h[sup];
    const int64_t seg0 = s.sup_seg0[sup];
    const int64_t segend = s.heavy_seg_ptr[h + 1];
    const int64_t dst = s.heavy_dst[h];
    const int64_t end = s.pull_ptr[dst + 1];
    // the supersegment's slots (its segments tile [first, last) in order),
    // staged in LDS with the row words of this block's 64 rows
    const int64_t first = s.seg_start[seg0];
    const int64_t last = first + (int64_t)FL_SUP * FL_SEG < end ? first + (int64_t)FL_SUP * FL_SEG : end;
    const int nst = (int)(last - first);
    const int64_t nw = (BL + 31) / 32;
    const int64_t wi0 = blc * (HEAVY_BL / 32);
    int32_t *st_src = reinterpret_cast<int32_t *>(pull_lds);  // [FL_SUP * FL_SEG]
    int32_t *st_pos = st_src + FL_SUP * FL_SEG;
    int32_t *st_rel = st_pos + FL_SUP * FL_SEG;
    float *st_m = reinterpret_cast<float *>(st_rel + FL_SUP * FL_SEG);
    uint32_t *st_w = reinterpret_cast<uint32_t *>(st_m + FL_SUP * FL_SEG);  // [slot][HEAVY_BL / 32]
    for (int k = threadIdx.x; k < nst; k += PULL_NT) {
        const int64_t sl = first + k;
        const int32_t src = s.pull_src[sl], pos = s.pull_pos[sl];
        st_src[k] = src;
        st_pos[k] = pos;
        st_rel[k] = s.pull_rel[sl];
        st_m[k] = s.mask[pos];
#pragma unroll
        for (int j = 0; j < HEAVY_BL / 32; ++j)
            st_w[k * (HEAVY_BL / 32) + j] = wi0 + j < nw ? BM[(wi0 + j) * E + src] : 0u;
    }
    __syncthreads();
    const int64_t off = dir ? r_size : 0;
    for (int task = threadIdx.x; task < HEAVY_TASKS; task += PULL_NT) {
        const int sl = task / HEAVY_BL, bll = task % HEAVY_BL;
        const int64_t bl = blc * HEAVY_BL + bll;
        const int64_t seg = seg0 + sl;
        int k = 0;
        if (seg < segend && bl < BL) {
            // the segment's slots [k0, k1) of the staged range, in order;
            // a slot's weight and record are read only where its source is
            // active in the row
            const int k0 = sl * FL_SEG, k1 = k0 + FL_SEG < nst ? k0 + FL_SEG : nst;
            float *list = (dir ? list_inv : list_ori) + (seg * BL + bl) * FL_SEG;
            const int wj = bll >> 5;
            const uint32_t bit = 1u << (bll & 31);
            const float *wr = w + bl * n + off;
            const int64_t plane = (int64_t)dir * E * BL + bl;
            for (int kb = k0; kb < k1; kb += WALK_U) {
                bool act[WALK_U];
                float wv[WALK_U];
                float2 rc[WALK_U];
#pragma unroll
                for (int u = 0; u < WALK_U; ++u) {
                    const int q = kb + u;
                    act[u] = q < k1 && (st_w[q * (HEAVY_BL / 32) + wj] & bit) && st_m[q] != 0.0f;
                    wv[u] = 0.0f;
                    rc[u] = make_float2(0.0f, 0.0f);
                    if (act[u]) {
                        wv[u] = wr[st_rel[q]];
                        rc[u] = PK[plane + (int64_t)st_src[q] * BL];
                    }
                }
#pragma unroll
                for (int u = 0; u < WALK_U; ++u) {
                    if (!act[u] || !(wv[u] > 0.0f)) continue;
                    const int q = kb + u;
                    bool kept = wv[u] > rc[u].y;
                    if (!kept && wv[u] == rc[u].y) kept = st_pos[q] < CUT[plane + (int64_t)st_src[q] * BL];
                    if (kept) list[k++] = fl_mul(fl_mul(rc[u].x, wv[u]), st_m[q]);
                }
            }
            (dir ? cnt_inv : cnt_ori)[seg * BL + bl] = k;
        }
        cnt_lds[sl][bll] = k;
    }
    __syncthreads();
    for (int task = threadIdx.x; task < HEAVY_TASKS; task += PULL_NT) {
        const int sl = task / HEAVY_BL, bll = task % HEAVY_BL;
        const int64_t bl = blc * HEAVY_BL + bll;
        const int64_t seg = seg0 + sl;
        if (seg < segend && bl < BL) {
            int run = 0;
            for (int q = 0; q < sl; ++q) run += cnt_lds[q][bll];
            (dir ? loff_inv : loff_ori)[seg * BL + bl] = run;
            if (seg == segend - 1 || sl == FL_SUP - 1)
                (dir ? stot_inv : stot_ori)[sup * BL + bl] = run + cnt_lds[sl][bll];
        }
    }
}

// One workgroup per heavy (destination, side): exclusive prefix over the
// destination's supersegments of their per-row totals (sup_base), and the
// per-row totals of the destination (tot).  P groups of BL threads scan
// contiguous supersegment ranges.
constexpr int HSCAN_NT = 1024;

__global__ __launch_bounds__(HSCAN_NT) void k_heavy_offsets(fl_side ori, fl_side inv, int64_t BL,
                                                           const int32_t *__restrict__ stot_ori,
                                                           const int32_t *__restrict__ stot_inv,
                                                           int32_t *__restrict__ sbase_ori,
                                                           int32_t *__restrict__ sbase_inv,
                                                           int32_t *__restrict__ tot_ori,
                                                           int32_t *__restrict__ tot_inv) {
    extern __shared__ int part[];  // [P][BL]
    const int dir = blockIdx.x >= ori.nheavy;
    const int64_t h = dir ? blockIdx.x - ori.nheavy : blockIdx.x;
    const fl_side &s = dir ? inv : ori;
    const int32_t *stot = dir ? stot_inv : stot_ori;
    int32_t *sbase = dir ? sbase_inv : sbase_ori;
    const int64_t u0 = s.heavy_sup_ptr[h], u1 = s.heavy_sup_ptr[h + 1];
    const int P = (int)(HSCAN_NT / BL);
    const int64_t per = (u1 - u0 + P - 1) / P;
    const int t = threadIdx.x;
    const int64_t bl = t % BL;
    const int grp = t / (int)BL;
    const bool active = grp < P;
    int64_t a0 = 0, a1 = 0;
    if (active) {
        a0 = u0 + grp * per;
        a1 = (a0 + per < u1) ? a0 + per : u1;
        int local = 0;
        for (int64_t u = a0; u < a1; ++u) local += stot[u * BL + bl];
        part[grp * BL + bl] = local;
    }
    __syncthreads();
    if (active) {
        int run = 0;
        for (int q = 0; q < grp; ++q) run += part[q * BL + bl];
        for (int64_t u = a0; u < a1; ++u) { sbase[u * BL + bl] = run; run += stot[u * BL + bl]; }
        if (grp == P - 1) (dir ? tot_inv : tot_ori)[h * BL + bl] = run;
    }
}

// One thread per (heavy segment, row): copy the segment's list into the
// row's contiguous run of the destination's region (the whole 32-value list
// is read at once; only its first cnt values are written).
__global__ __launch_bounds__(PULL_NT) void k_heavy_copy(
    fl_side ori, fl_side inv, int64_t BL, const float *__restrict__ list_ori, const float *__restrict__ list_inv,
    const int32_t *__restrict__ cnt_ori, const int32_t *__restrict__ cnt_inv, const int32_t *__restrict__ loff_ori,
    const int32_t *__restrict__ loff_inv, const int32_t *__restrict__ sbase_ori,
    const int32_t *__restrict__ sbase_inv, float *__restrict__ region_ori, float *__restrict__ region_inv) {
    const int64_t q = (int64_t)blockIdx.x * PULL_NT + threadIdx.x;
    const int64_t nq_ori = ori.nseg * BL;
    if (q >= nq_ori + inv.nseg * BL) return;
    const int dir = q >= nq_ori;
    const int64_t qq = dir ? q - nq_ori : q;
    const int64_t seg = qq / BL, bl = qq - seg * BL;
    const fl_side &s = dir ? inv : ori;
    const int c = (dir ? cnt_inv : cnt_ori)[qq];
    if (c == 0) return;
    const int64_t h = s.seg_h[seg];
    const int64_t g0 = s.heavy_seg_ptr[h], g1 = s.heavy_seg_ptr[h + 1];
    const int64_t sup = s.heavy_sup_ptr[h] + (seg - g0) / FL_SUP;
    const int64_t off = (int64_t)(dir ? sbase_inv : sbase_ori)[sup * BL + bl] + (dir ? loff_inv : loff_ori)[qq];
    const int64_t cap = (g1 - g0) * FL_SEG;
    const float4 *src = (const float4 *)((dir ? list_inv : list_ori) + qq * FL_SEG);
    float v[FL_SEG];
#pragma unroll
    for (int k = 0; k < FL_SEG / 4; ++k) {
        const float4 x = src[k];
        v[4 * k] = x.x; v[4 * k + 1] = x.y; v[4 * k + 2] = x.z; v[4 * k + 3] = x.w;
    }
    float *dstp = (dir ? region_inv : region_ori) + g0 * FL_SEG * BL + bl * cap + off;
#pragma unroll
    for (int k = 0; k < FL_SEG; ++k)
        if (k < c) dstp[k] = v[k];
}

// One workgroup per (heavy destination, side, block of FOLD_ROWS rows):
// each row's run is staged through LDS in chunks (one float4 per thread per
// row, all issued before the LDS stores) and added in order by one thread --
// the additions of a single walk over all the slots.
constexpr int FOLD_NT = 256;
constexpr int FOLD_ROWS = 16;
constexpr int FOLD_CHUNK = 4 * FOLD_NT;

// a + v[0] + v[1] + ... + v[lim-1], left to right, from a 16-byte aligned
// LDS row: the values are read 32 at a time with 16-byte loads, so the
// chain of additions waits on one LDS round trip per 32 of them.
__device__ __forceinline__ float fold_lds(float a, const float *v, int lim) {
    const float4 *v4 = reinterpret_cast<const float4 *>(v);
    int q = 0;
    for (; q + 32 <= lim; q += 32) {
        float4 x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = v4[(q >> 2) + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            a = fl_add(a, x[u].x);
            a = fl_add(a, x[u].y);
            a = fl_add(a, x[u].z);
            a = fl_add(a, x[u].w);
        }
    }
    for (; q + 4 <= lim; q += 4) {
        const float4 x = v4[q >> 2];
        a = fl_add(a, x.x);
        a = fl_add(a, x.y);
        a = fl_add(a, x.z);
        a = fl_add(a, x.w);
    }
    for (; q < lim; ++q) a = fl_add(a, v[q]);
    return a;
}

__global__ __launch_bounds__(FOLD_NT) void k_fold_heavy(
    fl_side ori, fl_side inv, int64_t BL, int64_t E, const float *__restrict__ region_ori,
    const float *__restrict__ region_inv, const int32_t *__restrict__ tot_ori, const int32_t *__restrict__ tot_inv,
    float *__restrict__ out_ori, float *__restrict__ out_inv) {
    __shared__ float4 stage[FOLD_ROWS][FOLD_NT];
    __shared__ int s_tot[FOLD_ROWS];
    const int dir = blockIdx.x >= ori.nheavy;
    const int64_t h = dir ? blockIdx.x - ori.nheavy : blockIdx.x;
    const fl_side &s = dir ? inv : ori;
    const float *region = dir ? region_inv : region_ori;
    const int64_t g0 = s.heavy_seg_ptr[h], g1 = s.heavy_seg_ptr[h + 1];
    const int64_t cap = (g1 - g0) * FL_SEG;
    const int64_t rb = (int64_t)blockIdx.y * FOLD_ROWS;
    const int t = threadIdx.x;
    if (t < FOLD_ROWS) s_tot[t] = (rb + t < BL) ? (dir ? tot_inv : tot_ori)[h * BL + rb + t] : 0;
    __syncthreads();
    int maxtot = 0;
    for (int r = 0; r < FOLD_ROWS; ++r) maxtot = s_tot[r] > maxtot ? s_tot[r] : maxtot;
    float acc = 0.0f;
    for (int64_t c0 = 0; c0 < maxtot; c0 += FOLD_CHUNK) {
        float4 x[FOLD_ROWS];
#pragma unroll
        for (int r = 0; r < FOLD_ROWS; ++r) {
            const int64_t k = c0 + 4 * t;  // cap is a multiple of FL_SEG: a float4 is all in or all out
            x[r] = (k < s_tot[r]) ? *(const float4 *)(region + g0 * FL_SEG * BL + (rb + r) * cap + k)
                                  : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int r = 0; r < FOLD_ROWS; ++r) stage[r][t] = x[r];
        __syncthreads();
        if (t < FOLD_ROWS && rb + t < BL) {
            const int lim = (int)((s_tot[t] - c0 < FOLD_CHUNK) ? s_tot[t] - c0 : FOLD_CHUNK);
            acc = fold_lds(acc, (const float *)stage[t], lim);
        }
        __syncthreads();
    }
    if (t < FOLD_ROWS && rb + t < BL) (dir ? out_inv : out_ori)[(rb + t) * E + s.heavy_dst[h]] = acc;
}

// ---------------------------------------------------------------------------
// Dense max forward (flashlog.cu:523-637, 997-1072) and backward (:639-726,
// 1187-1255).  The kept edges are the sum path's (same frontier and c2
// selection); per (row, destination) the result is the largest packed key
// over the kept products, which is order-free, so heavy destinations take
// the maximum of their segments' maxima.

__device__ __forceinline__ void max_unpack(uint64_t best, float *out, int64_t *arg) {
    *out = __uint_as_float((uint32_t)(best >> 32));
    *arg = best == 0 ? (int64_t)-1 : (int64_t)(int32_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFu));
}

// The kept products of nslot slots of one side, reduced into LDS cells:
// slot_of(k, &sl, &c) names the k-th slot and its cell row (its destination
// within the tile, or its segment within the chunk).  Task (slot, 32-row
// word): the slot's source and row word, its position and mask, then one
// key per row of the word where the source is active, folded into cell[row]
// with a 64-bit LDS max (the max is order-free, so every order gives the
// same cells).
template <typename SlotOf>
__device__ __forceinline__ void max_slots(const fl_side &s, int64_t nslot, int dir, int64_t BL, int64_t E,
                                          int64_t n, int64_t off, const float *__restrict__ w,
                                          const uint32_t *__restrict__ BM, const float2 *__restrict__ PK,
                                          const int32_t *__restrict__ CUT, uint64_t *cells, SlotOf &&slot_of) {
    const int64_t nw = (BL + 31) / 32;
    const int64_t plane = (int64_t)dir * E * BL;
    const int64_t ntask = nslot * nw;
    for (int64_t t = threadIdx.x; t < ntask; t += PULL_NT) {
        const int64_t k = t / nw, wi = t - k * nw;
        int32_t sl;
        int c;
        slot_of(k, &sl, &c);
        const int32_t src = s.pull_src[sl];
        uint32_t bits = BM[wi * E + src];
        if (!bits) continue;
        const int32_t pos = s.pull_pos[sl];
        const float m = s.mask[pos];
        if (m == 0.0f) continue;
        const int rel = s.pull_rel[sl];
        uint64_t *crow = cells + (int64_t)c * BL;
        const float *wc = w + off + rel;
        const int64_t at0 = plane + (int64_t)src * BL;
        // the word's active rows 8 at a time: their weights and records
        // requested together, then the tests
        while (bits) {
            int64_t bl[8];
            float wv[8];
            float2 rc[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                bl[j] = -1;
                wv[j] = 0.0f;
                rc[j] = make_float2(0.0f, 0.0f);
                if (bits) {
                    bl[j] = wi * 32 + __ffs(bits) - 1;
                    bits &= bits - 1;
                    wv[j] = wc[bl[j] * n];
                    rc[j] = PK[at0 + bl[j]];
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (bl[j] < 0 || !(wv[j] > 0.0f)) continue;
                bool kept = wv[j] > rc[j].y;
                if (!kept && wv[j] == rc[j].y) kept = pos < CUT[at0 + bl[j]];
                if (kept)
                    atomicMax((unsigned long long *)&crow[bl[j]],
                              (unsigned long long)max_key(fl_mul(fl_mul(rc[j].x, wv[j]), m), pos));
            }
        }
    }
}

// Light tiles of the max: workgroup per tile of td <= MAX_TD destinations (dealt
// to XCDs in contiguous ranges), the kept products of the tile's light
// slots (destinations of in-degree <= FL_SEG; the slots of each listed
// through an LDS prefix of their counts) reduced per (destination, row) in
// LDS (max_slots), then the tile written coalesced.  Heavy destinations get
// 0 / -1 here and their values from k_heavy_max.
__global__ __launch_bounds__(PULL_NT) void k_pull_max(
    fl_side ori, fl_side inv, const float *__restrict__ w, int64_t BL, int64_t E, int64_t n, int64_t r_size,
    int td, int64_t ntiles, const uint32_t *__restrict__ BM, const float2 *__restrict__ PK,
    const int32_t *__restrict__ CUT, float *__restrict__ out_ori, float *__restrict__ out_inv,
    int64_t *__restrict__ arg_ori, int64_t *__restrict__ arg_inv) {
    extern __shared__ uint64_t ktile[];  // [2][td][BL]
    __shared__ int32_t first[2][MAX_TD], pre[2][MAX_TD + 1];
    const int64_t tid = fl_xcd_contig(blockIdx.x, gridDim.x);
    if (tid >= ntiles) return;
    const int64_t d0 = tid * td;
    const int nd = (int)(E - d0 < td ? E - d0 : td);
    for (int64_t i = threadIdx.x; i < 2 * td * BL; i += PULL_NT) ktile[i] = 0;
    if (threadIdx.x < 2 * FL_WAVE) {
        // wave 0: ORI, wave 1: INV; lane j < nd: destination j's light slots
        const int dir = threadIdx.x / FL_WAVE, j = fl_lane();
        const fl_side &s = dir ? inv : ori;
        int32_t c = 0;
        if (j < nd) {
            const int64_t p0 = s.pull_ptr[d0 + j], p1 = s.pull_ptr[d0 + j + 1];
            first[dir][j] = (int32_t)p0;
            c = p1 - p0 <= FL_SEG ? (int32_t)(p1 - p0) : 0;
        }
        const int32_t incl = fl_wave_incl_scan_i32(c);
        if (j < nd) pre[dir][j + 1] = incl;
        if (j == 0) pre[dir][0] = 0;
    }
    __syncthreads();
#pragma unroll
    for (int dir = 0; dir < 2; ++dir) {
        const fl_side &s = dir ? inv : ori;
        const int32_t *pp = pre[dir], *fs = first[dir];
        max_slots(s, pp[nd], dir, BL, E, n, dir ? r_size : 0, w, BM, PK, CUT, ktile + dir * td * BL,
                  [&](int64_t k, int32_t *sl, int *c) {
                      int lo = 0, hi = nd;  // the destination: pp[lo] <= k < pp[lo + 1]
                      while (hi - lo > 1) {
                          const int mid = (lo + hi) >> 1;
                          if (pp[mid] <= k) lo = mid;
                          else hi = mid;
                      }
                      *sl = fs[lo] + (int32_t)(k - pp[lo]);
                      *c = lo;
                  });
    }
    __syncthreads();
    for (int64_t i = threadIdx.x; i < (int64_t)td * BL; i += PULL_NT) {
        const int64_t bl = i / td, dl = i - bl * td;
        if (dl < nd) {
            const int64_t at = bl * E + d0 + dl;
            max_unpack(ktile[dl * BL + bl], &out_ori[at], &arg_ori[at]);
            max_unpack(ktile[(td + dl) * BL + bl], &out_inv[at], &arg_inv[at]);
        }
    }
}

// Heavy destinations, step 1: workgroup per chunk of SEGS_PER_WG segments
// of one side, each segment's best key per row (max_slots over the
// segments' slots -- segment j holds [seg_start, seg_start + FL_SEG) clipped
// to its destination's end -- cell = segment within the chunk), stored to
// sb[segment][row].  STAGED: the chunk's slots -- source, position,
// relation, mask, cell and the source's row words -- are first read into LDS
// (one slot per thread, the loads of every slot in flight together), so a
// task (slot, row word) reads only its rows' weights and records from
// global memory.
constexpr int SEGS_PER_WG = 8;
constexpr int SEG_SLOTS = SEGS_PER_WG * FL_SEG;  // slots of one chunk, at most

// Dynamic LDS of the staged k_seg_max: the cells and the slots' row words.
inline size_t seg_max_lds_bytes(int64_t BL, bool staged) {
    return sizeof(uint64_t) * SEGS_PER_WG * (size_t)BL +
           (staged ? sizeof(uint32_t) * SEG_SLOTS * (size_t)((BL + 31) / 32) : 0);
}

template <bool STAGED>
__global__ __launch_bounds__(PULL_NT) void k_seg_max(fl_side ori, fl_side inv, const float *__restrict__ w,
                                                     int64_t BL, int64_t E, int64_t n, int64_t r_size,
                                                     const uint32_t *__restrict__ BM, const float2 *__restrict__ PK,
                                                     const int32_t *__restrict__ CUT, uint64_t *__restrict__ sb_ori,
                                                     uint64_t *__restrict__ sb_inv) {
    extern __shared__ uint64_t cells[];  // [SEGS_PER_WG][BL], then (STAGED) [SEG_SLOTS][nw] row words
    __shared__ int32_t first[SEGS_PER_WG], pre[SEGS_PER_WG + 1];
    __shared__ int32_t st_src[STAGED ? SEG_SLOTS : 1], st_pos[STAGED ? SEG_SLOTS : 1];
    __shared__ int16_t st_rel[STAGED ? SEG_SLOTS : 1];
    __shared__ uint8_t st_c[STAGED ? SEG_SLOTS : 1];
    __shared__ float st_m[STAGED ? SEG_SLOTS : 1];
    const int64_t nwg_ori = (ori.nseg + SEGS_PER_WG - 1) / SEGS_PER_WG;
    const int dir = (int64_t)blockIdx.x >= nwg_ori;
    const fl_side &s = dir ? inv : ori;
    const int64_t seg0 = ((int64_t)blockIdx.x - (dir ? nwg_ori : 0)) * SEGS_PER_WG;
    if (seg0 >= s.nseg) return;
    const int ns = (int)(s.nseg - seg0 < SEGS_PER_WG ? s.nseg - seg0 : SEGS_PER_WG);
    for (int64_t i = threadIdx.x; i < (int64_t)SEGS_PER_WG * BL; i += PULL_NT) cells[i] = 0;
    if (threadIdx.x < FL_WAVE) {
        const int j = fl_lane();
        int32_t c = 0;
        if (j < ns) {
            const int64_t a = s.seg_start[seg0 + j];
            const int64_t end = s.pull_ptr[(int64_t)s.seg_dst[seg0 + j] + 1];
            first[j] = (int32_t)a;
            c = (int32_t)(a + FL_SEG < end ? FL_SEG : end - a);
        }
        const int32_t incl = fl_wave_incl_scan_i32(c);
        if (j < ns) pre[j + 1] = incl;
        if (j == 0) pre[0] = 0;
    }
    __syncthreads();
    auto slot_of = [&](int64_t k, int32_t *sl, int *c) {
        int lo = 0, hi = ns;  // the segment: pre[lo] <= k < pre[lo + 1]
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (pre[mid] <= k) lo = mid;
            else hi = mid;
        }
        *sl = first[lo] + (int32_t)(k - pre[lo]);
        *c = lo;
    };
    if constexpr (!STAGED) {
        max_slots(s, pre[ns], dir, BL, E, n, dir ? r_size : 0, w, BM, PK, CUT, cells, slot_of);
    } else {
        const int64_t nw = (BL + 31) / 32;
        uint32_t *st_w = reinterpret_cast<uint32_t *>(cells + SEGS_PER_WG * BL);  // [SEG_SLOTS][nw]
        const int nslot = pre[ns];  // at most SEG_SLOTS
        for (int k = threadIdx.x; k < nslot; k += PULL_NT) {
            int32_t sl;
            int c;
            slot_of(k, &sl, &c);
            const int32_t src = s.pull_src[sl], pos = s.pull_pos[sl];
            st_src[k] = src;
            st_pos[k] = pos;
            st_rel[k] = s.pull_rel[sl];
            st_c[k] = (uint8_t)c;
            st_m[k] = s.mask[pos];
            for (int64_t wi = 0; wi < nw; ++wi) st_w[k * nw + wi] = BM[wi * E + src];
        }
        __syncthreads();
        const int64_t plane = (int64_t)dir * E * BL;
        const float *wb = w + (dir ? r_size : 0);
        for (int64_t t = threadIdx.x; t < (int64_t)nslot * nw; t += PULL_NT) {
            const int64_t k = t / nw, wi = t - k * nw;
            uint32_t bits = st_w[t];  // = st_w[k * nw + wi]
            if (!bits) continue;
            const float m = st_m[k];
            if (m == 0.0f) continue;
            const int32_t src = st_src[k], pos = st_pos[k];
            uint64_t *crow = cells + (int64_t)st_c[k] * BL;
            const float *wc = wb + st_rel[k];
            const int64_t at0 = plane + (int64_t)src * BL;
            // the word's active rows 8 at a time (as max_slots)
            while (bits) {
                int64_t bl[8];
                float wv[8];
                float2 rc[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    bl[j] = -1;
                    wv[j] = 0.0f;
                    rc[j] = make_float2(0.0f, 0.0f);
                    if (bits) {
                        bl[j] = wi * 32 + __ffs(bits) - 1;
                        bits &= bits - 1;
                        wv[j] = wc[bl[j] * n];
                        rc[j] = PK[at0 + bl[j]];
                    }
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if (bl[j] < 0 || !(wv[j] > 0.0f)) continue;
                    bool kept = wv[j] > rc[j].y;
                    if (!kept && wv[j] == rc[j].y) kept = pos < CUT[at0 + bl[j]];
                    if (kept)
                        atomicMax((unsigned long long *)&crow[bl[j]],
                                  (unsigned long long)max_key(fl_mul(fl_mul(rc[j].x, wv[j]), m), pos));
                }
            }
        }
    }
    __syncthreads();
    uint64_t *sb = (dir ? sb_inv : sb_ori) + seg0 * BL;
    for (int64_t i = threadIdx.x; i < (int64_t)ns * BL; i += PULL_NT) sb[i] = cells[i];
}

// Heavy destinations, step 2: thread per (supersegment, row): the maximum of
// its (at most FL_SUP) segments' maxima, stored in place of its first
// segment's (every segment belongs to one supersegment).
__global__ __launch_bounds__(PULL_NT) void k_sup_max(fl_side ori, fl_side inv, int64_t BL,
                                                     uint64_t *__restrict__ sb_ori, uint64_t *__restrict__ sb_inv) {
    const int64_t q = (int64_t)blockIdx.x * PULL_NT + threadIdx.x;
    const int64_t nq_ori = ori.nsup * BL;
    if (q >= nq_ori + inv.nsup * BL) return;
    const int dir = q >= nq_ori;
    const int64_t qq = dir ? q - nq_ori : q;
    const int64_t sup = qq / BL, bl = qq - sup * BL;
    const fl_side &s = dir ? inv : ori;
    uint64_t *sb = dir ? sb_inv : sb_ori;
    const int64_t seg0 = s.sup_seg0[sup];
    const int64_t end = s.heavy_seg_ptr[(int64_t)s.sup_h[sup] + 1];
    const int64_t seg1 = seg0 + FL_SUP < end ? seg0 + FL_SUP : end;
    uint64_t best = 0;
    for (int64_t g = seg0; g < seg1; ++g) {
        const uint64_t k = sb[g * BL + bl];
        best = k > best ? k : best;
    }
    sb[seg0 * BL + bl] = best;
}

// Heavy destinations, step 3: thread per (heavy destination, row): the
// maximum over its supersegments (8 loads in flight).
__global__ __launch_bounds__(PULL_NT) void k_heavy_max(fl_side ori, fl_side inv, int64_t BL, int64_t E,
                                                       const uint64_t *__restrict__ sb_ori,
                                                       const uint64_t *__restrict__ sb_inv,
                                                       float *__restrict__ out_ori, float *__restrict__ out_inv,
                                                       int64_t *__restrict__ arg_ori, int64_t *__restrict__ arg_inv) {
    const int64_t q = (int64_t)blockIdx.x * PULL_NT + threadIdx.x;
    const int64_t nq_ori = ori.nheavy * BL;
    if (q >= nq_ori + inv.nheavy * BL) return;
    const int dir = q >= nq_ori;
    const int64_t qq = dir ? q - nq_ori : q;
    const int64_t h = qq / BL, bl = qq - h * BL;
    const fl_side &s = dir ? inv : ori;
    const uint64_t *sb = dir ? sb_inv : sb_ori;
    const int64_t u0 = s.heavy_sup_ptr[h], u1 = s.heavy_sup_ptr[h + 1];
    uint64_t b8[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t u = u0;
    for (; u + 8 <= u1; u += 8) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint64_t k = sb[(int64_t)s.sup_seg0[u + j] * BL + bl];
            b8[j] = k > b8[j] ? k : b8[j];
        }
    }
    for (; u < u1; ++u) {
        const uint64_t k = sb[(int64_t)s.sup_seg0[u] * BL + bl];
        b8[0] = k > b8[0] ? k : b8[0];
    }
    uint64_t best = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) best = b8[j] > best ? b8[j] : best;
    const int64_t at = bl * E + s.heavy_dst[h];
    max_unpack(best, dir ? &out_inv[at] : &out_ori[at], dir ? &arg_inv[at] : &arg_ori[at]);
}

// ---------------------------------------------------------------------------
// Dense sum backward (flashlog.cpp:91-146,216-278)
//
//   k_bwd_identity  per row: gA = 0 + g_ind * w[n-1] for every entity, and
//                   gw[row, n-1] = sum_e g_ind * A (fixed tree order).
//   (frontier)      the forward's k_col_count / k_frontier / k_c2_hard on the
//                   same A and w give the same admitted edges.
//   k_row_count, k_row_fill  per row, its active sources in ascending order
//                   (per chunk of sources and 32-row word: counts, then ranks).
//   k_bwd_pairs     one wave per active (source, row): the ORI then INV row
//                   walk of the reference, adding (go*w)*m onto the identity
//                   term in CSR order (bit-exact gA), and per relation group
//                   the partial sum of (go*a)*m into the pair's row of PG.
//   k_bwd_gw        per row: gw[row, rel] = the pair partials of rel added in
//                   ascending source order, staged through LDS.

constexpr int BWD_NT = 256;

// Block (row, slice): gA for the slice's entities, and the slice's sum of
// g_ind * A (tree order) -- with one slice written to gw[row, n-1] (the rest
// of the row zeroed), else stored in gw[row, slice] for k_bwd_identity_fin,
// which adds the slices in order.
constexpr int BWD_SLICES_MAX = 32;

__global__ __launch_bounds__(BWD_NT) void k_bwd_identity(const float *__restrict__ g_ind, const float *__restrict__ A,
                                                        const float *__restrict__ w, int64_t E, int64_t n, int wot_i,
                                                        int add_zero, int nsl, float *__restrict__ gA,
                                                        float *__restrict__ gw) {
    __shared__ float part[BWD_NT];
    const int64_t bl = blockIdx.x;
    const int64_t span = (E + nsl - 1) / nsl;
    const int64_t e0 = (int64_t)blockIdx.y * span, e1 = e0 + span < E ? e0 + span : E;
    const int t = threadIdx.x;
    const float wid = w[bl * n + (n - 1)];
    float acc = 0.0f;
    for (int64_t e = e0 + t; e < e1; e += BWD_NT) {
        const int64_t i = bl * E + e;
        if (wot_i) {
            gA[i] = 0.0f;
        } else {
            const float gi = g_ind[i];
            const float t0 = fl_mul(gi, wid);
            gA[i] = add_zero ? fl_add(0.0f, t0) : t0;
            acc = fl_add(acc, fl_mul(gi, A[i]));
        }
    }
    part[t] = acc;
    __syncthreads();
    for (int st = BWD_NT / 2; st > 0; st >>= 1) {
        if (t < st) part[t] = fl_add(part[t], part[t + st]);
        __syncthreads();
    }
    if (nsl > 1) {
        if (t == 0) gw[bl * n + blockIdx.y] = wot_i ? 0.0f : part[0];
        return;
    }
    for (int64_t r = t; r < n; r += BWD_NT) gw[bl * n + r] = 0.0f;
    __syncthreads();
    if (t == 0 && !wot_i) gw[bl * n + (n - 1)] = part[0];
}

__global__ __launch_bounds__(BWD_NT) void k_bwd_identity_fin(int64_t n, int nsl, int wot_i,
                                                            float *__restrict__ gw) {
    __shared__ float total;
    const int64_t bl = blockIdx.x;
    const int t = threadIdx.x;
    if (t == 0) {
        float sum = 0.0f;
        for (int c = 0; c < nsl; ++c) sum = fl_add(sum, gw[bl * n + c]);
        total = sum;
    }
    __syncthreads();
    for (int64_t r = t; r < n; r += BWD_NT) gw[bl * n + r] = 0.0f;
    __syncthreads();
    if (t == 0 && !wot_i) gw[bl * n + (n - 1)] = total;
}

// The identity term of a dense backward: gA (every entity) and gw[:, n-1],
// rows split into slices so that the launch fills the chip.
static void bwd_identity(hipStream_t st, const float *g_ind, const float *A, const float *w, int64_t BL, int64_t E,
                         int64_t n, int wot_i, int add_zero, float *gA, float *gw) {
    int64_t nsl = (E + 4 * BWD_NT - 1) / (4 * BWD_NT);
    if (nsl > BWD_SLICES_MAX) nsl = BWD_SLICES_MAX;
    if (nsl > n - 1) nsl = n - 1;  // the partials live in gw[row, 0 .. n-2]
    if (nsl < 1) nsl = 1;
    FL_LAUNCH("k_bwd_identity", k_bwd_identity, dim3((unsigned)BL, (unsigned)nsl), dim3(BWD_NT), 0, st, g_ind,
                   A, w, E, n, wot_i, add_zero, (int)nsl, gA, gw);
    if (nsl > 1)
        FL_LAUNCH("k_bwd_identity_fin", k_bwd_identity_fin, dim3((unsigned)BL), dim3(BWD_NT), 0, st, n,
                       (int)nsl, wot_i, gw);
}

constexpr int RL_NT = 1024;  // sources per row-list chunk, one per thread

__device__ __forceinline__ uint32_t sp_lanes_below_u64(unsigned long long m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Row lists (each row's active sources in ascending order) in two passes
// over (chunk of RL_NT sources, 32-row word) workgroups.  k_row_count: per
// row of the word, the chunk's active sources (a ballot per row and wave).
__global__ __launch_bounds__(RL_NT) void k_row_count(const uint32_t *__restrict__ BM, int64_t BL, int64_t E,
                                                     int64_t nch, int32_t *__restrict__ ccnt) {
    __shared__ int wc[RL_NT / FL_WAVE][32];
    const int64_t c = blockIdx.x, wi = blockIdx.y;
    const int64_t src = c * RL_NT + threadIdx.x;
    const uint32_t bits = src < E ? BM[wi * E + src] : 0u;
    const int lane = fl_lane(), w = fl_wave_id();
#pragma unroll
    for (int r = 0; r < 32; ++r) {
        const unsigned long long m = __ballot((bits >> r) & 1u);
        if (lane == 0) wc[w][r] = __popcll(m);
    }
    __syncthreads();
    if (threadIdx.x < 32) {
        const int64_t bl = wi * 32 + threadIdx.x;
        int tot = 0;
        for (int q = 0; q < RL_NT / FL_WAVE; ++q) tot += wc[q][threadIdx.x];
        if (bl < BL) ccnt[bl * nch + c] = tot;
    }
}

// k_row_fill: each active source's rank in its row = the row's active
// sources in earlier chunks + in earlier waves of this chunk + in lower
// lanes; the last chunk also stores the row's count.
__global__ __launch_bounds__(RL_NT) void k_row_fill(const uint32_t *__restrict__ BM, int64_t BL, int64_t E,
                                                    int64_t nch, const int32_t *__restrict__ ccnt,
                                                    int32_t *__restrict__ rowlist, int32_t *__restrict__ rowcnt) {
    __shared__ int wc[RL_NT / FL_WAVE][32];
    const int64_t c = blockIdx.x, wi = blockIdx.y;
    const int64_t src = c * RL_NT + threadIdx.x;
    const uint32_t bits = src < E ? BM[wi * E + src] : 0u;
    const int lane = fl_lane(), w = fl_wave_id();
#pragma unroll
    for (int r = 0; r < 32; ++r) {
        const unsigned long long m = __ballot((bits >> r) & 1u);
        if (lane == 0) wc[w][r] = __popcll(m);
    }
    // the chunk's offset in each row of the word: thread (j, r) adds the
    // counts of chunks j, j + 32, ... before this one for row r
    __shared__ int part[32][33];
    {
        const int r = threadIdx.x & 31, j = threadIdx.x >> 5;
        const int64_t bl = wi * 32 + r;
        int x = 0;
        if (bl < BL)
            for (int64_t q = j; q < c; q += RL_NT / 32) x += ccnt[bl * nch + q];
        part[j][r] = x;
    }
    __syncthreads();
    if (threadIdx.x < 32) {
        // wave prefixes in place, the chunk's offset in the row added
        const int64_t bl = wi * 32 + threadIdx.x;
        int run = 0;
        for (int j = 0; j < RL_NT / 32; ++j) run += part[j][threadIdx.x];
        for (int q = 0; q < RL_NT / FL_WAVE; ++q) {
            const int x = wc[q][threadIdx.x];
            wc[q][threadIdx.x] = run;
            run += x;
        }
        if (bl < BL && c == nch - 1) rowcnt[bl] = run;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 32; ++r) {
        const unsigned long long m = __ballot((bits >> r) & 1u);
        if ((bits >> r) & 1u) {
            const int64_t bl = wi * 32 + r;  // set bits are rows < BL
            rowlist[bl * E + wc[w][r] + (int)sp_lanes_below_u64(m)] = (int32_t)src;
        }
    }
}

// One side of an active (source, row) pair, by one wave: the kept positions
// in CSR order (groups in order, each group's first `take` edges), 64 at a
// time.  Lane j of a window holds group j; item k of the window belongs to
// the first group whose inclusive take prefix exceeds k.  Each item's terms
// (go*w)*m and (go*a)*m are formed in parallel; the contributing items are
// then added one after another in position order -- the first term onto
// acc, the second onto its group's partial, held by the group's lane -- so
// the additions are those of a sequential walk.  MAX: only positions that
// won their destination (arg[row, dst] == p) contribute, as in the
// winner-only backward (flashlog.cu:699-710); a winning position is always a
// kept one.  Group partials go to the pair's row of relation columns in LDS
// (pgl, written where take > 0).
template <bool MAX>
__device__ __forceinline__ float bwd_side(const fl_side &s, int64_t src, int64_t bl, int64_t BL, int64_t E,
                                          int64_t n, int64_t off, int dir, float a, const float *__restrict__ w,
                                          const float *__restrict__ grad, const int64_t *__restrict__ arg,
                                          const float2 *__restrict__ PK, const int32_t *__restrict__ CUT,
                                          float acc, float *pgl) {
    const int lane = fl_lane();
    const int64_t at = ((int64_t)dir * E + src) * BL + bl;
    const float th = PK[at].y;
    const int32_t cut = th > 0.0f ? CUT[at] : 0;
    const float *wr = w + bl * n + off;
    const float *gr = grad + bl * E;
    const int64_t *ar = MAX ? arg + bl * E : nullptr;
    const int64_t g0 = s.row_group_ptr[src], g1 = s.row_group_ptr[src + 1];
    for (int64_t gb = g0; gb < g1; gb += FL_WAVE) {
        const int64_t g = gb + lane;
        int rel = 0;
        int32_t start = 0, take = 0;
        float wv = 0.0f;
        if (g < g1) {
            rel = s.group_rel[g];
            wv = wr[rel];
            start = s.group_start[g];
            take = (int32_t)group_take(wv, th, cut, start, s.group_count[g]);
        }
        // a source's kept edges on a side fit int32 (CSR positions are int32)
        const int32_t incl = fl_wave_incl_scan_i32(take);
        const int32_t total = __builtin_amdgcn_readlane(incl, FL_WAVE - 1);
        const int32_t first = start - (incl - take);  // item k of group j sits at first_j + k
        float gs = 0.0f;
        for (int32_t q0 = 0; q0 < total; q0 += FL_WAVE) {
            const int32_t k = q0 + lane;
            int j = 0;  // lanes whose inclusive prefix is <= k
#pragma unroll
            for (int step = FL_WAVE / 2; step > 0; step >>= 1)
                if (__shfl(incl, j + step - 1, FL_WAVE) <= k) j += step;
            const bool valid = k < total;
            const int32_t p = __shfl(first, j, FL_WAVE) + k;
            const float wj = __shfl(wv, j, FL_WAVE);
            float m = 0.0f, go = 0.0f;
            bool win = false;
            if (valid) {
                m = s.mask[p];
                const int32_t dst = s.col_ind[p];
                if (m != 0.0f) {
                    go = gr[dst];
                    win = MAX ? ar[dst] == (int64_t)p : true;
                }
            }
            const bool contrib = valid && win && m != 0.0f && go != 0.0f;
            const float t1 = fl_mul(fl_mul(go, wj), m);
            const float t2 = fl_mul(fl_mul(go, a), m);
            for (uint64_t bal = __ballot(contrib); bal; bal &= bal - 1) {
                const int i = __ffsll((long long)bal) - 1;
                acc = fl_add(acc, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t1), i)));
                const int gi = __builtin_amdgcn_readlane(j, i);
                const float t2i = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t2), i));
                if (lane == gi) gs = fl_add(gs, t2i);
            }
        }
        if (take > 0) pgl[off + rel] = gs;
    }
    return acc;
}

// One wave per active (source, row) pair, pairs in row-major order (the
// row's sources ascending, from k_row_fill): gA[row, src] = the identity
// term written by k_bwd_identity plus the ORI then INV walks, and the pair's
// row of PG (relation partials, 0 where no edge of the relation is kept).
constexpr int BWDP_WAVES = BWD_NT / FL_WAVE;

template <bool MAX>
__global__ __launch_bounds__(BWD_NT) void k_bwd_pairs(
    fl_side ori, fl_side inv, const float *__restrict__ A, const float *__restrict__ w,
    const float *__restrict__ g_ori, const float *__restrict__ g_inv, const int64_t *__restrict__ arg_ori,
    const int64_t *__restrict__ arg_inv, int64_t BL, int64_t E, int64_t n,
    int64_t r_size, const float2 *__restrict__ PK, const int32_t *__restrict__ CUT,
    const int32_t *__restrict__ rowlist, const int32_t *__restrict__ rowcnt, const int64_t *__restrict__ rowoff,
    int64_t pairs, float *__restrict__ gA, float *__restrict__ PG) {
    extern __shared__ float pg_lds[];  // [BWDP_WAVES][n]
    const int lane = fl_lane();
    const int wid = fl_wave_id();
    const int64_t q = (int64_t)blockIdx.x * BWDP_WAVES + wid;
    if (q >= pairs || q >= rowoff[BL]) return;  // no block barrier follows
    int64_t lo = 0, hi = BL;  // the row: rowoff[lo] <= q < rowoff[lo + 1]
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (rowoff[mid] <= q) lo = mid;
        else hi = mid;
    }
    const int64_t bl = lo, k = q - rowoff[bl];
    if (k >= rowcnt[bl]) return;
    const int64_t src = rowlist[bl * E + k];
    const float a = A[bl * E + src];
    float *pgl = pg_lds + (int64_t)wid * n;
    for (int64_t r = lane; r < n; r += FL_WAVE) pgl[r] = 0.0f;
    fl_wave_sync();
    float acc = gA[bl * E + src];  // identity term written by k_bwd_identity
    acc = bwd_side<MAX>(ori, src, bl, BL, E, n, 0, 0, a, w, g_ori, arg_ori, PK, CUT, acc, pgl);
    acc = bwd_side<MAX>(inv, src, bl, BL, E, n, r_size, 1, a, w, g_inv, arg_inv, PK, CUT, acc, pgl);
    fl_wave_sync();
    float *pg = PG + q * n;
    for (int64_t r = lane; r < n; r += FL_WAVE) pg[r] = pgl[r];
    if (lane == 0) gA[bl * E + src] = acc;
}

// gw[row, r] for the relation columns r < 2*r_size: the pairs' partials in
// ascending source order, GW_C pairs at a time through LDS.
constexpr int GW_C = 32;

__global__ __launch_bounds__(BWD_NT) void k_bwd_gw(const float *__restrict__ PG, const int32_t *__restrict__ rowcnt,
                                                  const int64_t *__restrict__ rowoff, int64_t pairs, int64_t n,
                                                  int64_t nrel, float *__restrict__ gw) {
    extern __shared__ float stage[];  // [GW_C][n]
    const int64_t bl = blockIdx.x;
    int64_t cnt = rowcnt[bl];
    if (rowoff[bl] + cnt > pairs) cnt = pairs - rowoff[bl] > 0 ? pairs - rowoff[bl] : 0;
    const float *pg = PG + rowoff[bl] * n;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};  // columns t, t+256, t+512, t+768
    for (int64_t k0 = 0; k0 < cnt; k0 += GW_C) {
        const int64_t kc = (cnt - k0 < GW_C) ? cnt - k0 : GW_C;
        for (int64_t i = threadIdx.x; i < kc * n; i += BWD_NT) stage[i] = pg[k0 * n + i];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t r = threadIdx.x + j * BWD_NT;
            if (r < nrel)
                for (int64_t k = 0; k < kc; ++k) acc[j] = fl_add(acc[j], stage[k * n + r]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t r = threadIdx.x + j * BWD_NT;
        if (r < nrel) gw[bl * n + r] = acc[j];
    }
}

__global__ void k_row_offsets(const int32_t *__restrict__ rowcnt, int64_t BL, int64_t *__restrict__ rowoff) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        int64_t run = 0;
        for (int64_t b = 0; b < BL; ++b) { rowoff[b] = run; run += rowcnt[b]; }
        rowoff[BL] = run;
    }
}

}  // namespace fl

// ---------------------------------------------------------------------------
// C-ABI

using namespace fl;

namespace {

struct DenseWs {
    uint32_t *bm;
    float2 *pk;
    int32_t *cut;
    int2 *hard;
    int32_t *hard_count, *cnt_ori, *cnt_inv, *loff_ori, *loff_inv, *stot_ori, *stot_inv, *sbase_ori, *sbase_inv,
        *tot_ori, *tot_inv;
    float *list_ori, *list_inv, *region_ori, *region_inv;
    size_t bytes;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

DenseWs dense_ws_layout(int64_t BL, int64_t E, const fl_side *ori, const fl_side *inv, char *base) {
    DenseWs ws{};
    const int64_t nw = (BL + 31) / 32;
    const int64_t cap = BL * E;
    size_t off = 0;
    auto take = [&](size_t bytes) { char *p = base ? base + off : nullptr; off += align256(bytes); return p; };
    ws.bm = (uint32_t *)take(sizeof(uint32_t) * (size_t)(nw * E));
    ws.pk = (float2 *)take(sizeof(float2) * (size_t)(2 * cap));
    ws.cut = (int32_t *)take(sizeof(int32_t) * (size_t)(2 * cap));
    ws.hard = (int2 *)take(sizeof(int2) * (size_t)cap);
    ws.hard_count = (int32_t *)take(sizeof(int32_t));
    ws.cnt_ori = (int32_t *)take(sizeof(int32_t) * (size_t)(ori->nseg * BL));
    ws.cnt_inv = (int32_t *)take(sizeof(int32_t) * (size_t)(inv->nseg * BL));
    ws.loff_ori = (int32_t *)take(sizeof(int32_t) * (size_t)(ori->nseg * BL));
    ws.loff_inv = (int32_t *)take(sizeof(int32_t) * (size_t)(inv->nseg * BL));
    ws.stot_ori = (int32_t *)take(sizeof(int32_t) * (size_t)(ori->nsup * BL));
    ws.stot_inv = (int32_t *)take(sizeof(int32_t) * (size_t)(inv->nsup * BL));
    ws.sbase_ori = (int32_t *)take(sizeof(int32_t) * (size_t)(ori->nsup * BL));
    ws.sbase_inv = (int32_t *)take(sizeof(int32_t) * (size_t)(inv->nsup * BL));
    ws.tot_ori = (int32_t *)take(sizeof(int32_t) * (size_t)(ori->nheavy * BL));
    ws.tot_inv = (int32_t *)take(sizeof(int32_t) * (size_t)(inv->nheavy * BL));
    ws.list_ori = (float *)take(sizeof(float) * (size_t)(ori->nseg * BL * FL_SEG));
    ws.list_inv = (float *)take(sizeof(float) * (size_t)(inv->nseg * BL * FL_SEG));
    ws.region_ori = (float *)take(sizeof(float) * (size_t)(ori->nseg * BL * FL_SEG));
    ws.region_inv = (float *)take(sizeof(float) * (size_t)(inv->nseg * BL * FL_SEG));
    ws.bytes = off;
    return ws;
}

int check_side(const fl_side *s, const char *name) {
    if (!s) return fl_fail(FL_ERR_ARG, "%s side is null", name);
    if (s->edges > 0 && (!s->col_ind || !s->mask || !s->group_rel || !s->group_start ||
                         !s->group_count || !s->pull_pos || !s->pull_src || !s->pull_rel))
        return fl_fail(FL_ERR_ARG, "%s side has a null array", name);
    if (!s->row_group_ptr || !s->pull_ptr) return fl_fail(FL_ERR_ARG, "%s side has null row pointers", name);
    if (s->nseg < 0 || s->nheavy < 0 || s->nsup < 0 ||
        (s->nseg > 0 && (!s->seg_dst || !s->seg_start || !s->seg_h)) ||
        (s->nsup > 0 && (!s->sup_h || !s->sup_seg0)) ||
        (s->nheavy > 0 && (!s->heavy_dst || !s->heavy_seg_ptr || !s->heavy_sup_ptr)))
        return fl_fail(FL_ERR_ARG, "%s side has inconsistent heavy-destination segments", name);
    return FL_OK;
}

}  // namespace

extern "C" {

int fl_abi_version(void) { return 24; }

int fl_apply_mask(void *stream, const void *mask_values, int mask_is_bool, const int32_t *order,
                  const float *weight, float *out, int64_t nnz) {
    if (nnz < 0) return fl_fail(FL_ERR_ARG, "apply_mask: negative nnz");
    if (nnz == 0) return FL_OK;
    if (!mask_values || !order || !out) return fl_fail(FL_ERR_ARG, "apply_mask: null pointer");
    const int nt = 256;
    const int64_t nb = (nnz + nt - 1) / nt;
    hipStream_t st = (hipStream_t)stream;
    if (mask_is_bool)
        FL_LAUNCH("k_apply_mask", k_apply_mask<uint8_t>, dim3((unsigned)nb), dim3(nt), 0, st,
                           (const uint8_t *)mask_values, order, weight, out, nnz);
    else
        FL_LAUNCH("k_apply_mask", k_apply_mask<float>, dim3((unsigned)nb), dim3(nt), 0, st,
                           (const float *)mask_values, order, weight, out, nnz);
    return fl_check_launch("apply_mask");
}

int fl_edge_dscore(void *stream, const float *weight, const int32_t *order, float *out, int64_t nnz) {
    if (nnz < 0) return fl_fail(FL_ERR_ARG, "edge_dscore: negative nnz");
    if (nnz == 0) return FL_OK;
    if (!weight || !order || !out) return fl_fail(FL_ERR_ARG, "edge_dscore: null pointer");
    FL_LAUNCH("k_edge_dscore", k_edge_dscore, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
              weight, order, out, nnz);
    return fl_check_launch("edge_dscore");
}

int fl_mark_active(void *stream, const float *A, int64_t BL, int64_t E, int32_t *flags) {
    if (BL < 0 || E < 0) return fl_fail(FL_ERR_ARG, "mark_active: negative size");
    if (E == 0) return FL_OK;
    const int nt = 256;
    FL_LAUNCH("k_mark_active", k_mark_active, dim3((unsigned)((E + nt - 1) / nt)), dim3(nt), 0,
                       (hipStream_t)stream, A, flags, BL, E);
    return fl_check_launch("mark_active");
}

int fl_dense_topc(void *stream, const float *A, float *out, int64_t BL, int64_t E, int64_t c,
                  int32_t *row_state) {
    if (c < 0) return fl_fail(FL_ERR_ARG, "topk_nodes/c must be nonnegative");
    if (BL < 0 || E < 0 || E > INT32_MAX - 1) return fl_fail(FL_ERR_ARG, "dense_topc: bad shape");
    if (BL == 0) return FL_OK;
    FL_LAUNCH("k_topc_rows", k_topc_rows, dim3((unsigned)BL), dim3(TOPC_NT), 0, (hipStream_t)stream,
                       A, out, E, c, row_state);
    return fl_check_launch("dense_topc");
}

int fl_dense_topc_backward(void *stream, const float *grad, const float *A,
                           const int32_t *row_state, float *grad_A, int64_t BL, int64_t E) {
    if (BL <= 0 || E <= 0) return FL_OK;
    const int nt = 256;
    FL_LAUNCH("k_topc_backward", k_topc_backward, dim3((unsigned)((E + nt - 1) / nt), (unsigned)BL), dim3(nt), 0,
                       (hipStream_t)stream, grad, A, row_state, grad_A, E);
    return fl_check_launch("dense_topc_backward");
}

size_t fl_dense_workspace_bytes(const fl_side *ori, const fl_side *inv, int64_t BL, int64_t E) {
    if (BL <= 0 || E <= 0 || !ori || !inv) return 256;
    return dense_ws_layout(BL, E, ori, inv, nullptr).bytes;
}

int fl_dense_sum_forward(void *stream, const fl_side *ori, const fl_side *inv, const float *A,
                         const float *w, int64_t BL, int64_t E, int64_t n, int64_t r_size, int wot_i,
                         int64_t topk_edges, float *out_ind, float *out_ori, float *out_inv,
                         void *workspace, size_t workspace_bytes) {
    int rc;
    if ((rc = check_side(ori, "ori")) != FL_OK) return rc;
    if ((rc = check_side(inv, "inv")) != FL_OK) return rc;
    if (BL < 0 || E < 0 || n < 1) return fl_fail(FL_ERR_ARG, "dense_sum_forward: bad shape");
    if (BL * E >= (int64_t)INT32_MAX) return fl_fail(FL_ERR_ARG, "dense_sum_forward: BL*E must be < 2^31");
    if (BL > HSCAN_NT) return fl_fail(FL_ERR_ARG, "dense_sum_forward: BL=%lld above %d", (long long)BL, HSCAN_NT);
    if (r_size < 0 || 2 * r_size + 1 > n + (wot_i ? 1 : 0))
        return fl_fail(FL_ERR_ARG, "dense_sum_forward: w width %lld too small for r_size %lld",
                       (long long)n, (long long)r_size);
    if (BL == 0 || E == 0) return FL_OK;
    DenseWs ws = dense_ws_layout(BL, E, ori, inv, (char *)workspace);
    if (!workspace || workspace_bytes < ws.bytes)
        return fl_fail(FL_ERR_ARG, "dense_sum_forward: workspace of %zu bytes, need %zu", workspace_bytes, ws.bytes);
    hipStream_t st = (hipStream_t)stream;
    const int64_t nw = (BL + 31) / 32;
    const int do_topk = (topk_edges > 0 && topk_edges < ((int64_t)1 << 60)) ? 1 : 0;
    const int64_t K = do_topk ? topk_edges : 0;
    FL_LAUNCH("k_col_count", k_col_count, dim3((unsigned)((nw * E + COL_NT - 1) / COL_NT)), dim3(COL_NT), 0, st, A,
              w, BL, E, n, wot_i, out_ind, ws.bm, ws.hard_count);
    FL_LAUNCH("k_frontier", k_frontier, dim3((unsigned)((E + COL_NT - 1) / COL_NT)), dim3(COL_NT), 0, st, *ori,
              *inv, A, BL, E, K, do_topk, ws.bm, ws.pk, ws.hard_count, ws.hard);
    if (do_topk)
        FL_LAUNCH("k_c2_hard", k_c2_hard, dim3(1024), dim3(C2_NT), 0, st, *ori, *inv, w, BL, E, n, r_size, K,
                  ws.hard_count, ws.hard, ws.pk, ws.cut);
    // light destinations: TD <= SUM_TD destinations per workgroup, with the
    // output tile and the staged slots (two sides of TD*FL_SEG slots, 16
    // bytes and nw row words each) in at most 64 KiB of LDS
    int TD = SUM_TD;
    while (TD > 1 && pull_lds_bytes(BL, TD) > 65536) --TD;
    const int64_t ntiles = (E + TD - 1) / TD;
    const int64_t nlight = ((ntiles + 7) / 8) * 8;
    const int64_t nblc = (BL + HEAVY_BL - 1) / HEAVY_BL;
    const int64_t nheavy_wg = (((ori->nsup + inv->nsup) * nblc + 7) / 8) * 8;
    // the heavy blocks stage FL_SUP * FL_SEG slots (16 bytes and two row
    // words each) in the same area
    size_t lds = pull_lds_bytes(BL, TD);
    const size_t heavy_lds = (size_t)FL_SUP * FL_SEG * (16 + 4 * (HEAVY_BL / 32));
    if (lds < heavy_lds) lds = heavy_lds;
    FL_LAUNCH("k_pull", k_pull, dim3((unsigned)(nlight + nheavy_wg)), dim3(PULL_NT), lds, st, *ori, *inv, w, BL,
              E, n, r_size, TD, ntiles, nlight, nheavy_wg, ws.bm, ws.pk, ws.cut, out_ori, out_inv, ws.list_ori,
              ws.list_inv,
              ws.cnt_ori, ws.cnt_inv, ws.loff_ori, ws.loff_inv, ws.stot_ori, ws.stot_inv);
    const int64_t nq_seg = (ori->nseg + inv->nseg) * BL;
    if (nq_seg > 0) {
        const size_t slds = sizeof(int) * (size_t)((HSCAN_NT / BL) * BL);
        FL_LAUNCH("k_heavy_offsets", k_heavy_offsets, dim3((unsigned)(ori->nheavy + inv->nheavy)), dim3(HSCAN_NT),
                  slds, st, *ori, *inv, BL, ws.stot_ori, ws.stot_inv, ws.sbase_ori, ws.sbase_inv, ws.tot_ori,
                  ws.tot_inv);
        FL_LAUNCH("k_heavy_copy", k_heavy_copy, dim3((unsigned)((nq_seg + PULL_NT - 1) / PULL_NT)), dim3(PULL_NT), 0,
                  st, *ori, *inv, BL, ws.list_ori, ws.list_inv, ws.cnt_ori, ws.cnt_inv, ws.loff_ori, ws.loff_inv,
                  ws.sbase_ori, ws.sbase_inv, ws.region_ori, ws.region_inv);
        FL_LAUNCH("k_fold_heavy", k_fold_heavy,
                  dim3((unsigned)(ori->nheavy + inv->nheavy), (unsigned)((BL + FOLD_ROWS - 1) / FOLD_ROWS)),
                  dim3(FOLD_NT), 0, st, *ori, *inv, BL, E, ws.region_ori, ws.region_inv, ws.tot_ori, ws.tot_inv,
                  out_ori, out_inv);
    }
    return fl_check_launch("dense_sum_forward");
}

size_t fl_dense_backward_workspace_bytes(const fl_side *ori, const fl_side *inv, int64_t BL, int64_t E) {
    if (BL <= 0 || E <= 0 || !ori || !inv) return 256;
    // the forward's frontier arrays plus the row lists and their chunk counts
    const int64_t nch = (E + RL_NT - 1) / RL_NT;
    return dense_ws_layout(BL, E, ori, inv, nullptr).bytes + align256(sizeof(int32_t) * (size_t)(BL * E)) +
           align256(sizeof(int32_t) * (size_t)BL) + align256(sizeof(int64_t) * (size_t)(BL + 1)) +
           align256(sizeof(int32_t) * (size_t)(BL * nch));
}

}  // extern "C"

namespace {

// The dense backward of both aggregations (arg_ori/arg_inv null: sum; else
// the winner-only max backward): identity term, the forward's frontier and
// c2 records, per-row source lists, the per-(source, row) walks, then grad_w.
int dense_backward_impl(const char *name, void *stream, const fl_side *ori, const fl_side *inv, const float *A,
                        const float *w, const float *grad_ind, const float *grad_ori, const float *grad_inv,
                        const int64_t *arg_ori, const int64_t *arg_inv, int64_t BL, int64_t E, int64_t n,
                        int64_t r_size, int wot_i, int64_t topk_edges, float *grad_A, float *grad_w, float *pg,
                        int64_t pg_pairs, void *workspace, size_t workspace_bytes) {
    int rc;
    if ((rc = check_side(ori, "ori")) != FL_OK) return rc;
    if ((rc = check_side(inv, "inv")) != FL_OK) return rc;
    if (BL <= 0 || E <= 0 || n < 1) return fl_fail(FL_ERR_ARG, "%s: bad shape", name);
    if (BL * E >= (int64_t)INT32_MAX) return fl_fail(FL_ERR_ARG, "%s: BL*E must be < 2^31", name);
    if (r_size < 0 || 2 * r_size + 1 > n + (wot_i ? 1 : 0))
        return fl_fail(FL_ERR_ARG, "%s: w width too small for r_size", name);
    const int64_t nrel = 2 * r_size;
    if (nrel > 4 * BWD_NT) return fl_fail(FL_ERR_ARG, "%s: more than %d relation columns", name, 4 * BWD_NT);
    if ((size_t)GW_C * n * sizeof(float) > 65536) return fl_fail(FL_ERR_ARG, "%s: w width too large", name);
    if (pg_pairs < 0 || (pg_pairs > 0 && !pg)) return fl_fail(FL_ERR_ARG, "%s: bad partial buffer", name);
    if (!workspace || workspace_bytes < fl_dense_backward_workspace_bytes(ori, inv, BL, E))
        return fl_fail(FL_ERR_ARG, "%s: workspace too small", name);
    const bool is_max = arg_ori != nullptr;
    DenseWs ws = dense_ws_layout(BL, E, ori, inv, (char *)workspace);
    int32_t *rowlist = (int32_t *)((char *)workspace + ws.bytes);
    int32_t *rowcnt = (int32_t *)((char *)rowlist + align256(sizeof(int32_t) * (size_t)(BL * E)));
    int64_t *rowoff = (int64_t *)((char *)rowcnt + align256(sizeof(int32_t) * (size_t)BL));
    hipStream_t st = (hipStream_t)stream;
    const int64_t nw = (BL + 31) / 32;
    const int do_topk = (topk_edges > 0 && topk_edges < ((int64_t)1 << 60)) ? 1 : 0;
    const int64_t K = do_topk ? topk_edges : 0;
    // the sum's identity term is added to 0 first (flashlog.cpp:242); the
    // max's is stored as is (flashlog.cu:173-207)
    bwd_identity(st, grad_ind, A, w, BL, E, n, wot_i, is_max ? 0 : 1, grad_A, grad_w);
    // the forward's frontier (same A and w: same admitted edges); no identity output
    FL_LAUNCH("k_col_count", k_col_count, dim3((unsigned)((nw * E + COL_NT - 1) / COL_NT)), dim3(COL_NT), 0, st, A,
              w, BL, E, n, wot_i, (float *)nullptr, ws.bm, ws.hard_count);
    FL_LAUNCH("k_frontier", k_frontier, dim3((unsigned)((E + COL_NT - 1) / COL_NT)), dim3(COL_NT), 0, st, *ori,
              *inv, A, BL, E, K, do_topk, ws.bm, ws.pk, ws.hard_count, ws.hard);
    if (do_topk)
        FL_LAUNCH("k_c2_hard", k_c2_hard, dim3(1024), dim3(C2_NT), 0, st, *ori, *inv, w, BL, E, n, r_size, K,
                  ws.hard_count, ws.hard, ws.pk, ws.cut);
    const int64_t nch = (E + RL_NT - 1) / RL_NT;
    int32_t *ccnt = (int32_t *)((char *)rowoff + align256(sizeof(int64_t) * (size_t)(BL + 1)));
    FL_LAUNCH("k_row_count", k_row_count, dim3((unsigned)nch, (unsigned)nw), dim3(RL_NT), 0, st, ws.bm, BL, E, nch,
              ccnt);
    FL_LAUNCH("k_row_fill", k_row_fill, dim3((unsigned)nch, (unsigned)nw), dim3(RL_NT), 0, st, ws.bm, BL, E, nch, ccnt,
              rowlist, rowcnt);
    FL_LAUNCH("k_row_offsets", k_row_offsets, dim3(1), dim3(64), 0, st, rowcnt, BL, rowoff);
    if (pg_pairs > 0) {
        // a wave per pair: the host's pair count bounds the grid (pairs past
        // the row lists' total leave at once)
        const unsigned nb = (unsigned)((pg_pairs + BWDP_WAVES - 1) / BWDP_WAVES);
        const size_t plds = sizeof(float) * (size_t)(BWDP_WAVES * n);
        if (is_max)
            FL_LAUNCH("k_bwd_pairs_max", k_bwd_pairs<true>, dim3(nb), dim3(BWD_NT), plds, st, *ori, *inv, A, w,
                      grad_ori, grad_inv, arg_ori, arg_inv, BL, E, n, r_size, ws.pk, ws.cut, rowlist, rowcnt,
                      rowoff, pg_pairs, grad_A, pg);
        else
            FL_LAUNCH("k_bwd_pairs", k_bwd_pairs<false>, dim3(nb), dim3(BWD_NT), plds, st, *ori, *inv, A, w,
                      grad_ori, grad_inv, (const int64_t *)nullptr, (const int64_t *)nullptr, BL, E, n, r_size,
                      ws.pk, ws.cut, rowlist, rowcnt, rowoff, pg_pairs, grad_A, pg);
        const size_t lds = sizeof(float) * (size_t)(GW_C * n);
        FL_LAUNCH("k_bwd_gw", k_bwd_gw, dim3((unsigned)BL), dim3(BWD_NT), lds, st, pg, rowcnt, rowoff, pg_pairs, n,
                  nrel, grad_w);
    }
    return fl_check_launch(name);
}

}  // namespace

extern "C" {

int fl_dense_sum_backward(void *stream, const fl_side *ori, const fl_side *inv, const float *A, const float *w,
                          const float *grad_ind, const float *grad_ori, const float *grad_inv, int64_t BL, int64_t E,
                          int64_t n, int64_t r_size, int wot_i, int64_t topk_edges, float *grad_A, float *grad_w,
                          float *pg, int64_t pg_pairs, void *workspace, size_t workspace_bytes) {
    return dense_backward_impl("dense_sum_backward", stream, ori, inv, A, w, grad_ind, grad_ori, grad_inv, nullptr,
                               nullptr, BL, E, n, r_size, wot_i, topk_edges, grad_A, grad_w, pg, pg_pairs, workspace,
                               workspace_bytes);
}

int fl_dense_max_forward(void *stream, const fl_side *ori, const fl_side *inv, const float *A, const float *w,
                         int64_t BL, int64_t E, int64_t n, int64_t r_size, int wot_i, int64_t topk_edges,
                         float *out_ind, float *out_ori, float *out_inv, int64_t *arg_ori, int64_t *arg_inv,
                         void *workspace, size_t workspace_bytes) {
    int rc;
    if ((rc = check_side(ori, "ori")) != FL_OK) return rc;
    if ((rc = check_side(inv, "inv")) != FL_OK) return rc;
    if (BL < 0 || E < 0 || n < 1) return fl_fail(FL_ERR_ARG, "dense_max_forward: bad shape");
    if (BL * E >= (int64_t)INT32_MAX) return fl_fail(FL_ERR_ARG, "dense_max_forward: BL*E must be < 2^31");
    if (BL > HSCAN_NT) return fl_fail(FL_ERR_ARG, "dense_max_forward: BL=%lld above %d", (long long)BL, HSCAN_NT);
    if (r_size < 0 || 2 * r_size + 1 > n + (wot_i ? 1 : 0))
        return fl_fail(FL_ERR_ARG, "dense_max_forward: w width %lld too small for r_size %lld", (long long)n,
                       (long long)r_size);
    if (BL == 0 || E == 0) return FL_OK;
    DenseWs ws = dense_ws_layout(BL, E, ori, inv, (char *)workspace);
    if (!workspace || workspace_bytes < ws.bytes)
        return fl_fail(FL_ERR_ARG, "dense_max_forward: workspace of %zu bytes, need %zu", workspace_bytes, ws.bytes);
    hipStream_t st = (hipStream_t)stream;
    const int64_t nw = (BL + 31) / 32;
    const int do_topk = (topk_edges > 0 && topk_edges < ((int64_t)1 << 60)) ? 1 : 0;
    const int64_t K = do_topk ? topk_edges : 0;
    FL_LAUNCH("k_col_count", k_col_count, dim3((unsigned)((nw * E + COL_NT - 1) / COL_NT)), dim3(COL_NT), 0, st, A,
              w, BL, E, n, wot_i, out_ind, ws.bm, ws.hard_count);
    FL_LAUNCH("k_frontier", k_frontier, dim3((unsigned)((E + COL_NT - 1) / COL_NT)), dim3(COL_NT), 0, st, *ori,
              *inv, A, BL, E, K, do_topk, ws.bm, ws.pk, ws.hard_count, ws.hard);
    if (do_topk)
        FL_LAUNCH("k_c2_hard", k_c2_hard, dim3(1024), dim3(C2_NT), 0, st, *ori, *inv, w, BL, E, n, r_size, K,
                  ws.hard_count, ws.hard, ws.pk, ws.cut);
    // key cells of a tile: 2 * td * BL, at most 64 KiB of LDS (BL <= 1024)
    int td = (int)(4096 / BL);
    if (td < 1) td = 1;
    if (td > MAX_TD) td = MAX_TD;
    const int64_t ntiles = (E + td - 1) / td;
    const size_t lds = sizeof(uint64_t) * 2 * (size_t)BL * (size_t)td;
    FL_LAUNCH("k_pull_max", k_pull_max, dim3((unsigned)ntiles), dim3(PULL_NT), lds, st, *ori, *inv, w, BL, E, n,
              r_size, td, ntiles, ws.bm, ws.pk, ws.cut, out_ori, out_inv, arg_ori, arg_inv);
    // segment maxima reuse the heavy-list area (nseg*BL*FL_SEG floats >= nseg*BL keys)
    uint64_t *sb_ori = (uint64_t *)ws.list_ori, *sb_inv = (uint64_t *)ws.list_inv;
    const int64_t nq_seg = (ori->nseg + inv->nseg) * BL;
    if (nq_seg > 0) {
        const int64_t nwg = (ori->nseg + SEGS_PER_WG - 1) / SEGS_PER_WG + (inv->nseg + SEGS_PER_WG - 1) / SEGS_PER_WG;
        // the staged form while its LDS stays within 64 KiB (BL up to 640)
        const bool staged = seg_max_lds_bytes(BL, true) + 4096 <= 65536;
        FL_LAUNCH("k_seg_max", staged ? k_seg_max<true> : k_seg_max<false>, dim3((unsigned)nwg), dim3(PULL_NT),
                  seg_max_lds_bytes(BL, staged), st, *ori, *inv, w, BL, E, n, r_size, ws.bm, ws.pk, ws.cut, sb_ori,
                  sb_inv);
        const int64_t nq_sup = (ori->nsup + inv->nsup) * BL;
        if (nq_sup > 0)
            FL_LAUNCH("k_sup_max", k_sup_max, dim3((unsigned)((nq_sup + PULL_NT - 1) / PULL_NT)), dim3(PULL_NT), 0,
                      st, *ori, *inv, BL, sb_ori, sb_inv);
        const int64_t nq_h = (ori->nheavy + inv->nheavy) * BL;
        FL_LAUNCH("k_heavy_max", k_heavy_max, dim3((unsigned)((nq_h + PULL_NT - 1) / PULL_NT)), dim3(PULL_NT), 0,
                  st, *ori, *inv, BL, E, sb_ori, sb_inv, out_ori, out_inv, arg_ori, arg_inv);
    }
    return fl_check_launch("dense_max_forward");
}

int fl_dense_max_backward(void *stream, const fl_side *ori, const fl_side *inv, const float *A, const float *w,
                          const float *grad_ind, const float *grad_ori, const float *grad_inv,
                          const int64_t *arg_ori, const int64_t *arg_inv, int64_t BL, int64_t E, int64_t n,
                          int64_t r_size, int wot_i, int64_t topk_edges, float *grad_A, float *grad_w, float *pg,
                          int64_t pg_pairs, void *workspace, size_t workspace_bytes) {
    if (!arg_ori || !arg_inv) return fl_fail(FL_ERR_ARG, "dense_max_backward: null winner arrays");
    return dense_backward_impl("dense_max_backward", stream, ori, inv, A, w, grad_ind, grad_ori, grad_inv, arg_ori,
                               arg_inv, BL, E, n, r_size, wot_i, topk_edges, grad_A, grad_w, pg, pg_pairs,
                               workspace, workspace_bytes);
}

}  // extern "C"
