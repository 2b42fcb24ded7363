// Dense-state propagation kernels for gfx950 (MI355X) and their C-ABI.
//
// One hop of the reference's dense sum path (flashlog.cu:898-995, with the
// CPU path's accumulation order, flashlog.cpp:151-211) runs as five kernels:
//
//   k_col_count  column walk of A[BL, E] (thread per entity, coalesced over
//                entities): identity output, per-entity nonzero count and a
//                bitmask of the nonzero rows, per-block totals.
//   k_block_scan exclusive scan of the per-block totals (one workgroup).
//   k_col_fill   the frontier: per active source, its nonzero (row, value)
//                entries in row order (the transpose of A's sparsity).
//   k_c2         per frontier entry and direction, the c2 edge budget as a
//                (threshold, cut position) pair from a wave-level radix
//                select over the source's relation groups; marks the pull
//                slots of every position leaving an active source.
//   k_pull       per tile of 64 destinations: walk the marked incoming slots
//                in ascending CSR position and add (a*w)*m into LDS
//                accumulators -- exactly the order in which the reference's
//                CPU loop adds into out[bl, dst] -- then write the tile.
//
// No atomics touch output values, so results are deterministic and equal to
// the reference CPU bits.
#include "fl_common.h"
#include "fl_abi.h"

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
    for (int64_t e = t; e < E; e += TOPC_NT) {
        float v = a[e];
        if (v != 0.0f) { ++nz_local; atomicAdd(&hist[fl_order_key(v) >> 21], 1); }
    }
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
        for (int64_t e = t; e < E; e += TOPC_NT) {
            float v = a[e];
            uint32_t k = fl_order_key(v);
            if (v != 0.0f && (k >> 21) == (prefix >> 21)) atomicAdd(&hist[(k >> 10) & 2047], 1);
        }
        __syncthreads();
        topc_select<2048>(hist, need, lds_scan, &sel_bin, &sel_need);
        prefix |= (uint32_t)sel_bin << 10;
        need = sel_need;
        // pass 3: bits [9:0]
        for (int i = t; i < 2048; i += TOPC_NT) hist[i] = 0;
        __syncthreads();
        for (int64_t e = t; e < E; e += TOPC_NT) {
            float v = a[e];
            uint32_t k = fl_order_key(v);
            if (v != 0.0f && (k >> 10) == (prefix >> 10)) atomicAdd(&hist[k & 1023], 1);
        }
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
    for (int64_t e = t; e < E; e += TOPC_NT) {
        float v = a[e];
        bool keep = true;
        if (over) {
            keep = false;
            if (c > 0 && v != 0.0f) {
                uint32_t k = fl_order_key(v);
                keep = (k > cutkey) || (k == cutkey && e <= last);
            }
        }
        o[e] = v * (keep ? 1.0f : 0.0f);
    }
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

constexpr int COL_NT = 256;

__global__ __launch_bounds__(COL_NT) void k_col_count(
    const float *__restrict__ A, const float *__restrict__ w, int64_t BL, int64_t E, int64_t n,
    int wot_i, float *__restrict__ out_ind, int32_t *__restrict__ colcnt,
    uint32_t *__restrict__ bitmask, int32_t *__restrict__ blocksum) {
    __shared__ int lds_scan[COL_NT / FL_WAVE + 1];
    const int64_t e = (int64_t)blockIdx.x * COL_NT + threadIdx.x;
    int cnt = 0;
    if (e < E) {
        const int64_t nw = (BL + 31) / 32;
        for (int64_t wi = 0; wi < nw; ++wi) {
            const int64_t b0 = wi * 32;
            const int64_t b1 = (b0 + 32 < BL) ? b0 + 32 : BL;
            uint32_t bits = 0;
#pragma unroll 8
            for (int64_t bl = b0; bl < b1; ++bl) {
                const float a = A[bl * E + e];
                const float wid = w[bl * n + (n - 1)];
                out_ind[bl * E + e] = wot_i ? 0.0f : fl_mul(a, wid);
                if (a != 0.0f) bits |= 1u << (bl - b0);
            }
            bitmask[wi * E + e] = bits;
            cnt += __popc(bits);
        }
        colcnt[e] = cnt;
    }
    int tot;
    (void)fl_block_excl_scan<COL_NT>(cnt, lds_scan, &tot);
    if (threadIdx.x == 0) blocksum[blockIdx.x] = tot;
}

constexpr int SCAN_NT = 1024;

__global__ __launch_bounds__(SCAN_NT) void k_block_scan(const int32_t *__restrict__ in,
                                                         int32_t *__restrict__ out, int64_t nblk) {
    __shared__ int lds_scan[SCAN_NT / FL_WAVE + 1];
    const int64_t per = (nblk + SCAN_NT - 1) / SCAN_NT;
    const int64_t b0 = threadIdx.x * per;
    const int64_t b1 = (b0 + per < nblk) ? b0 + per : nblk;
    int local = 0;
    for (int64_t i = b0; i < b1; ++i) local += in[i];
    int tot;
    int run = fl_block_excl_scan<SCAN_NT>(local, lds_scan, &tot);
    for (int64_t i = b0; i < b1; ++i) { int v = in[i]; out[i] = run; run += v; }
    if (threadIdx.x == 0) out[nblk] = tot;
}

__global__ __launch_bounds__(COL_NT) void k_col_fill(
    const float *__restrict__ A, int64_t BL, int64_t E, const int32_t *__restrict__ colcnt,
    const uint32_t *__restrict__ bitmask, const int32_t *__restrict__ blockoff,
    int32_t *__restrict__ colptr, int32_t *__restrict__ fr_src, int4 *__restrict__ fr_ori) {
    __shared__ int lds_scan[COL_NT / FL_WAVE + 1];
    const int64_t e = (int64_t)blockIdx.x * COL_NT + threadIdx.x;
    const int cnt = (e < E) ? colcnt[e] : 0;
    int tot;
    const int ex = fl_block_excl_scan<COL_NT>(cnt, lds_scan, &tot);
    if (e >= E) return;
    int slot = blockoff[blockIdx.x] + ex;
    colptr[e] = slot;
    if (e == E - 1) colptr[E] = slot + cnt;
    if (cnt == 0) return;
    const int64_t nw = (BL + 31) / 32;
    for (int64_t wi = 0; wi < nw; ++wi) {
        uint32_t bits = bitmask[wi * E + e];
        while (bits) {
            const int b = __ffs(bits) - 1;
            bits &= bits - 1;
            const int64_t bl = wi * 32 + b;
            const float a = A[bl * E + e];
            fr_src[slot] = (int32_t)e;
            fr_ori[slot] = make_int4((int)bl, __float_as_int(a), 0, 0);
            ++slot;
        }
    }
}

// Wave-level c2 threshold for one (source, row, direction): the weighted
// order statistic of flashlog.cpp:12-35 by MSB-first radix select over the
// float bits of the group weights (4 passes of 8 bits, group sizes as
// multiplicities), then the tie-quota cut: ties are admitted in group order,
// so the admitted tied edges are exactly the positions below `cut`.
// Returns false when every eligible edge fits (no pruning).
__device__ bool c2_select(const fl_side &s, int64_t g0, int64_t g1, const float *wrow,
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

__device__ __forceinline__ void row_positions(const fl_side &s, int64_t src, int64_t *p0, int64_t *p1) {
    const int64_t g0 = s.row_group_ptr[src], g1 = s.row_group_ptr[src + 1];
    if (g1 > g0) {
        *p0 = s.group_start[g0];
        *p1 = (int64_t)s.group_start[g1 - 1] + s.group_count[g1 - 1];
    } else {
        *p0 = 0; *p1 = 0;
    }
}

constexpr int C2_NT = 256;

__global__ __launch_bounds__(C2_NT) void k_c2(fl_side ori, fl_side inv, const float *__restrict__ w,
                                              int64_t n, int64_t r_size, int64_t K, int do_topk,
                                              int64_t E, const int32_t *__restrict__ colptr,
                                              const int32_t *__restrict__ fr_src,
                                              int4 *__restrict__ fr_ori, int4 *__restrict__ fr_inv,
                                              uint8_t epoch) {
    __shared__ int hist_all[C2_NT / FL_WAVE][256];
    const int lane = fl_lane();
    const int wid = threadIdx.x / FL_WAVE;
    int *hist = hist_all[wid];
    const int64_t nwaves = (int64_t)gridDim.x * (C2_NT / FL_WAVE);
    const int64_t total = colptr[E];
    for (int64_t j = (int64_t)blockIdx.x * (C2_NT / FL_WAVE) + wid; j < total; j += nwaves) {
        const int64_t src = fr_src[j];
        const int4 f = fr_ori[j];
        const int64_t bl = f.x;
        for (int dir = 0; dir < 2; ++dir) {
            const fl_side &s = dir ? inv : ori;
            const int64_t off = dir ? r_size : 0;
            uint32_t thk = 0;
            int32_t cut = 0;
            if (do_topk) {
                const int64_t g0 = s.row_group_ptr[src], g1 = s.row_group_ptr[src + 1];
                int64_t p0, p1;
                row_positions(s, src, &p0, &p1);
                if (p1 - p0 > K) {
                    uint32_t k2; int32_t c2;
                    if (c2_select(s, g0, g1, w + bl * n + off, K, hist, &k2, &c2)) { thk = k2; cut = c2; }
                }
            }
            if (lane == 0) {
                int4 r = make_int4(f.x, f.y, (int)thk, cut);
                if (dir) fr_inv[j] = r; else fr_ori[j] = r;
            }
        }
        if (j == colptr[src]) {
            for (int dir = 0; dir < 2; ++dir) {
                const fl_side &s = dir ? inv : ori;
                int64_t p0, p1;
                row_positions(s, src, &p0, &p1);
                for (int64_t p = p0 + lane; p < p1; p += FL_WAVE) s.marks[s.slot_of_pos[p]] = epoch;
            }
        }
    }
}

// Pull: one workgroup per (64-destination tile, chunk of <= 128 rows).
constexpr int PULL_NT = 256;
constexpr int PULL_TILE = 64;

__global__ __launch_bounds__(PULL_NT) void k_pull(fl_side ori, fl_side inv, const float *__restrict__ w,
                                                  int64_t BL, int64_t E, int64_t n, int64_t r_size,
                                                  int blc, const int32_t *__restrict__ colptr,
                                                  const int4 *__restrict__ fr_ori,
                                                  const int4 *__restrict__ fr_inv, uint8_t epoch,
                                                  float *__restrict__ out_ori, float *__restrict__ out_inv) {
    extern __shared__ float acc[];  // [2][blc][PULL_TILE]
    const int lane = fl_lane();
    const int wid = threadIdx.x / FL_WAVE;
    const int64_t d0 = (int64_t)blockIdx.x * PULL_TILE;
    const int64_t bl0 = (int64_t)blockIdx.y * blc;
    const int64_t nbl = (bl0 + blc < BL) ? blc : BL - bl0;
    for (int i = threadIdx.x; i < 2 * blc * PULL_TILE; i += PULL_NT) acc[i] = 0.0f;
    __syncthreads();

    for (int dl = wid; dl < PULL_TILE; dl += PULL_NT / FL_WAVE) {
        const int64_t dst = d0 + dl;
        if (dst >= E) break;
        for (int dir = 0; dir < 2; ++dir) {
            const fl_side &s = dir ? inv : ori;
            const int4 *fr = dir ? fr_inv : fr_ori;
            const int64_t off = dir ? r_size : 0;
            float *accd = acc + (int64_t)dir * blc * PULL_TILE;
            const int64_t s0 = s.pull_ptr[dst], s1 = s.pull_ptr[dst + 1];
            for (int64_t base = s0; base < s1; base += FL_WAVE) {
                const int64_t slot = base + lane;
                int live = 0, pos = 0, rel = 0, j0 = 0, j1 = 0;
                float m = 0.0f;
                if (slot < s1 && s.marks[slot] == epoch) {
                    pos = s.pull_pos[slot];
                    const int src = s.pull_src[slot];
                    rel = s.pull_rel[slot];
                    m = s.mask[pos];
                    if (m != 0.0f) {
                        j0 = colptr[src];
                        j1 = colptr[src + 1];
                        live = j1 > j0;
                    }
                }
                unsigned long long bal = __ballot(live);
                while (bal) {
                    const int i = __ffsll((long long)bal) - 1;
                    bal &= bal - 1;
                    const int ipos = __shfl(pos, i, FL_WAVE);
                    const int irel = __shfl(rel, i, FL_WAVE);
                    const float im = __shfl(m, i, FL_WAVE);
                    const int ij0 = __shfl(j0, i, FL_WAVE);
                    const int ij1 = __shfl(j1, i, FL_WAVE);
                    for (int j = ij0 + lane; j < ij1; j += FL_WAVE) {
                        const int4 f = fr[j];
                        const int64_t bl = f.x;
                        if (bl < bl0 || bl >= bl0 + nbl) continue;
                        const float wv = w[bl * n + off + irel];
                        const float th = __int_as_float(f.z);
                        if (wv > th || (wv == th && ipos < f.w)) {
                            const float prod = fl_mul(fl_mul(__int_as_float(f.y), wv), im);
                            float *cell = accd + (bl - bl0) * PULL_TILE + dl;
                            *cell = fl_add(*cell, prod);
                        }
                    }
                }
            }
        }
    }
    __syncthreads();
    const int64_t ncol = (d0 + PULL_TILE <= E) ? PULL_TILE : E - d0;
    for (int dir = 0; dir < 2; ++dir) {
        float *out = dir ? out_inv : out_ori;
        const float *accd = acc + (int64_t)dir * blc * PULL_TILE;
        for (int64_t i = threadIdx.x; i < nbl * PULL_TILE; i += PULL_NT) {
            const int64_t r = i / PULL_TILE, cidx = i % PULL_TILE;
            if (cidx < ncol) out[(bl0 + r) * E + d0 + cidx] = accd[i];
        }
    }
}

}  // namespace fl

// ---------------------------------------------------------------------------
// C-ABI

using namespace fl;

namespace {

struct DenseWs {
    int32_t *colcnt, *colptr, *blocksum, *blockoff, *fr_src;
    uint32_t *bitmask;
    int4 *fr_ori, *fr_inv;
    size_t bytes;
};

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

DenseWs dense_ws_layout(int64_t BL, int64_t E, char *base) {
    DenseWs ws{};
    const int64_t nblk = (E + COL_NT - 1) / COL_NT;
    const int64_t nw = (BL + 31) / 32;
    const int64_t cap = BL * E;
    size_t off = 0;
    auto take = [&](size_t bytes) { char *p = base ? base + off : nullptr; off += align256(bytes); return p; };
    ws.colcnt = (int32_t *)take(sizeof(int32_t) * (size_t)(E + 1));
    ws.colptr = (int32_t *)take(sizeof(int32_t) * (size_t)(E + 1));
    ws.blocksum = (int32_t *)take(sizeof(int32_t) * (size_t)(nblk + 1));
    ws.blockoff = (int32_t *)take(sizeof(int32_t) * (size_t)(nblk + 1));
    ws.bitmask = (uint32_t *)take(sizeof(uint32_t) * (size_t)(nw * E));
    ws.fr_src = (int32_t *)take(sizeof(int32_t) * (size_t)cap);
    ws.fr_ori = (int4 *)take(sizeof(int4) * (size_t)cap);
    ws.fr_inv = (int4 *)take(sizeof(int4) * (size_t)cap);
    ws.bytes = off;
    return ws;
}

int check_side(const fl_side *s, const char *name) {
    if (!s) return fl_fail(FL_ERR_ARG, "%s side is null", name);
    if (s->edges > 0 && (!s->col_ind || !s->mask || !s->group_rel || !s->group_start ||
                         !s->group_count || !s->pull_pos || !s->pull_src || !s->pull_rel ||
                         !s->slot_of_pos || !s->marks))
        return fl_fail(FL_ERR_ARG, "%s side has a null array", name);
    if (!s->row_group_ptr || !s->pull_ptr) return fl_fail(FL_ERR_ARG, "%s side has null row pointers", name);
    return FL_OK;
}

}  // namespace

extern "C" {

int fl_abi_version(void) { return 1; }

int fl_apply_mask(void *stream, const void *mask_values, int mask_is_bool, const int32_t *order,
                  const float *weight, float *out, int64_t nnz) {
    if (nnz < 0) return fl_fail(FL_ERR_ARG, "apply_mask: negative nnz");
    if (nnz == 0) return FL_OK;
    if (!mask_values || !order || !out) return fl_fail(FL_ERR_ARG, "apply_mask: null pointer");
    const int nt = 256;
    const int64_t nb = (nnz + nt - 1) / nt;
    hipStream_t st = (hipStream_t)stream;
    if (mask_is_bool)
        hipLaunchKernelGGL(k_apply_mask<uint8_t>, dim3((unsigned)nb), dim3(nt), 0, st,
                           (const uint8_t *)mask_values, order, weight, out, nnz);
    else
        hipLaunchKernelGGL(k_apply_mask<float>, dim3((unsigned)nb), dim3(nt), 0, st,
                           (const float *)mask_values, order, weight, out, nnz);
    return fl_check_launch("apply_mask");
}

int fl_mark_active(void *stream, const float *A, int64_t BL, int64_t E, int32_t *flags) {
    if (BL < 0 || E < 0) return fl_fail(FL_ERR_ARG, "mark_active: negative size");
    if (E == 0) return FL_OK;
    const int nt = 256;
    hipLaunchKernelGGL(k_mark_active, dim3((unsigned)((E + nt - 1) / nt)), dim3(nt), 0,
                       (hipStream_t)stream, A, flags, BL, E);
    return fl_check_launch("mark_active");
}

int fl_dense_topc(void *stream, const float *A, float *out, int64_t BL, int64_t E, int64_t c,
                  int32_t *row_state) {
    if (c < 0) return fl_fail(FL_ERR_ARG, "topk_nodes/c must be nonnegative");
    if (BL < 0 || E < 0 || E > INT32_MAX - 1) return fl_fail(FL_ERR_ARG, "dense_topc: bad shape");
    if (BL == 0) return FL_OK;
    hipLaunchKernelGGL(k_topc_rows, dim3((unsigned)BL), dim3(TOPC_NT), 0, (hipStream_t)stream,
                       A, out, E, c, row_state);
    return fl_check_launch("dense_topc");
}

int fl_dense_topc_backward(void *stream, const float *grad, const float *A,
                           const int32_t *row_state, float *grad_A, int64_t BL, int64_t E) {
    if (BL <= 0 || E <= 0) return FL_OK;
    const int nt = 256;
    hipLaunchKernelGGL(k_topc_backward, dim3((unsigned)((E + nt - 1) / nt), (unsigned)BL), dim3(nt), 0,
                       (hipStream_t)stream, grad, A, row_state, grad_A, E);
    return fl_check_launch("dense_topc_backward");
}

size_t fl_dense_workspace_bytes(int64_t BL, int64_t E) {
    if (BL <= 0 || E <= 0) return 256;
    return dense_ws_layout(BL, E, nullptr).bytes;
}

int fl_dense_sum_forward(void *stream, const fl_side *ori, const fl_side *inv, const float *A,
                         const float *w, int64_t BL, int64_t E, int64_t n, int64_t r_size, int wot_i,
                         int64_t topk_edges, int epoch, float *out_ind, float *out_ori,
                         float *out_inv, void *workspace, size_t workspace_bytes) {
    int rc;
    if ((rc = check_side(ori, "ori")) != FL_OK) return rc;
    if ((rc = check_side(inv, "inv")) != FL_OK) return rc;
    if (BL < 0 || E < 0 || n < 1) return fl_fail(FL_ERR_ARG, "dense_sum_forward: bad shape");
    if (BL * E >= (int64_t)INT32_MAX) return fl_fail(FL_ERR_ARG, "dense_sum_forward: BL*E must be < 2^31");
    if (r_size < 0 || 2 * r_size + 1 > n + (wot_i ? 1 : 0))
        return fl_fail(FL_ERR_ARG, "dense_sum_forward: w width %lld too small for r_size %lld",
                       (long long)n, (long long)r_size);
    if (epoch < 1 || epoch > 255) return fl_fail(FL_ERR_ARG, "dense_sum_forward: epoch out of range");
    if (BL == 0 || E == 0) return FL_OK;
    DenseWs ws = dense_ws_layout(BL, E, (char *)workspace);
    if (!workspace || workspace_bytes < ws.bytes)
        return fl_fail(FL_ERR_ARG, "dense_sum_forward: workspace of %zu bytes, need %zu", workspace_bytes, ws.bytes);
    hipStream_t st = (hipStream_t)stream;
    const int64_t nblk = (E + COL_NT - 1) / COL_NT;
    hipLaunchKernelGGL(k_col_count, dim3((unsigned)nblk), dim3(COL_NT), 0, st, A, w, BL, E, n, wot_i,
                       out_ind, ws.colcnt, ws.bitmask, ws.blocksum);
    hipLaunchKernelGGL(k_block_scan, dim3(1), dim3(SCAN_NT), 0, st, ws.blocksum, ws.blockoff, nblk);
    hipLaunchKernelGGL(k_col_fill, dim3((unsigned)nblk), dim3(COL_NT), 0, st, A, BL, E, ws.colcnt,
                       ws.bitmask, ws.blockoff, ws.colptr, ws.fr_src, ws.fr_ori);
    const int do_topk = (topk_edges > 0 && topk_edges < ((int64_t)1 << 60)) ? 1 : 0;
    const int64_t K = do_topk ? topk_edges : 0;
    hipLaunchKernelGGL(k_c2, dim3(2048), dim3(C2_NT), 0, st, *ori, *inv, w, n, r_size, K, do_topk, E,
                       ws.colptr, ws.fr_src, ws.fr_ori, ws.fr_inv, (uint8_t)epoch);
    const int blc = (int)(BL < 128 ? BL : 128);
    const size_t lds = sizeof(float) * 2 * (size_t)blc * PULL_TILE;
    dim3 grid((unsigned)((E + PULL_TILE - 1) / PULL_TILE), (unsigned)((BL + blc - 1) / blc));
    hipLaunchKernelGGL(k_pull, grid, dim3(PULL_NT), lds, st, *ori, *inv, w, BL, E, n, r_size, blc,
                       ws.colptr, ws.fr_ori, ws.fr_inv, (uint8_t)epoch, out_ori, out_inv);
    return fl_check_launch("dense_sum_forward");
}

}  // extern "C"
