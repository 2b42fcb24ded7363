// Sparse (COO) hop on gfx950, sum and max aggregation.
//
// Replaces the expansion kernels of flashlog.cu (count/fill top-k
// :1368-1559, all edges :1743-1829, identity :1831-1854) and the coalesce
// of flashlog_kernel.py:258-357 (sum) and :399-478 (max).  Sum keeps the
// addition order of the reference's CPU path (flashlog.cpp:1388-1486): per
// (row, destination) the contributions are added to 0 in input-entry order,
// and per entry ORI kept edges (CSR position order), then INV kept edges,
// then the identity term.  Max keeps, per (row, destination), the item with
// the largest value; ties go to ORI before INV before the identity term,
// then to the smaller original edge id, then to the earlier raw item.
//
// Pipeline (rows r = b*L + l; entries must be sorted by row):
//   plan    k_sp_rowptr   entry range of every row, input validation
//           k_sp_select   per (entry, side): c2 threshold and cut (training:
//                         quota parameters), item counts and 64-item chunks
//           scan          item and chunk offsets of every entry (raw order)
//           k_sp_rowinfo  item range and tile count of every row; scan
//   expand  k_sp_runs     wave per entry: one descriptor per run (the kept
//                         edges of one group) and the entry's chunk records
//           k_sp_items    wave per 64 raw items: destination and value of
//                         each, from the runs that cover the chunk
//           k_sp_hist     workgroup per tile: the tile's bucket histogram
//           k_sp_vscan    per (row, bucket): prefixes over the row's tiles
//           scan          the buckets' first positions
//           k_sp_partition workgroup per tile of a row: stable scatter of the
//                         tile's items into destination buckets (block radix
//                         rank over the bucket id)
//           k_sp_accum_small  wave per (row, bucket) of at most 512 items
//                         and 64 destinations: each destination's values added
//                         in raw order; other buckets are listed for
//                         k_sp_accum_few (at most 64 destinations), then
//                         k_sp_accum_mid (workgroup sort, persistent) and
//                         k_sp_accum_hot (chunks into a dense LDS accumulator,
//                         persistent); max: k_sp_max / k_sp_max_hot
//           scan          output offsets
//           k_sp_local_to_out  (with a backward) every raw item's output index
//   emit    k_sp_emit     coalesced COO (b, l, e, v), ascending key
//   backward k_sp_bwd     wave per entry over its raw items (CSR position,
//                         column and output index saved by the forward)
// The plan and the run writer may visit entries in a given order (by source
// entity: a source's rows then share cached group records); a Boolean
// visibility mask may be read as a bitmap (k_mask_bits).
#include <limits.h>

#include "fl_abi.h"
#include "fl_c2.h"
#include "fl_common.h"
#include "fl_scan.h"
#include "fl_topc.h"

namespace fl {

constexpr int SP_S = 13;               // destinations per bucket = 2^SP_S
constexpr int SP_W = 1 << SP_S;
constexpr int SP_NT = 256;
constexpr int NM_NT0 = 256;  // row-reduction workgroup size
constexpr int SP_IPT = 16;
constexpr int SP_TILE = SP_NT * SP_IPT;  // items per partition tile

enum { SP_TOPK = 0, SP_ALL = 1, SP_FIXED = 2 };
enum { SP_SUM = 0, SP_MAX = 1 };
// raw item tie keys of the max (ascending = preferred on equal values)
constexpr uint32_t SP_TIE_INV = 0x80000000u;  // | original edge id
constexpr uint32_t SP_TIE_IDENTITY = 0xFFFFFFFFu;


// ---------------------------------------------------------------------------
// plan

// row_ptr[r] = first entry of row r (entries sorted by row); err[0] gets a
// nonzero code for a malformed input (1: index out of range, 2: rows not
// sorted).
__global__ void k_sp_rowptr(const int64_t *__restrict__ sb, const int64_t *__restrict__ sl,
                            const int64_t *__restrict__ se, int64_t nnz, int64_t B, int64_t L, int64_t E,
                            int64_t *__restrict__ row_ptr, int64_t *__restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t R = B * L;
    if (nnz == 0) {
        for (int64_t r = i; r <= R; r += (int64_t)gridDim.x * blockDim.x) row_ptr[r] = 0;
        return;
    }
    if (i >= nnz) return;
    const int64_t b = sb[i], l = sl[i], e = se[i];
    if (b < 0 || b >= B || l < 0 || l >= L || e < 0 || e >= E) {
        atomicMax((unsigned long long *)err, 1ull);
        return;
    }
    const int64_t r = b * L + l;
    int64_t rp = -1;
    if (i > 0) {
        const int64_t pb = sb[i - 1], pl = sl[i - 1];
        rp = (pb >= 0 && pb < B && pl >= 0 && pl < L) ? pb * L + pl : r;
        if (rp > r) { atomicMax((unsigned long long *)err, 2ull); return; }
    }
    for (int64_t q = rp + 1; q <= r; ++q) row_ptr[q] = i;
    if (i == nnz - 1)
        for (int64_t q = r + 1; q <= R; ++q) row_ptr[q] = nnz;
}

// Take rule of one (entry, side).  TAKE_ALL: every edge (all-edges mode);
// TAKE_TH: the c2 threshold th and tie cut (group_take); TAKE_QUOTA: the
// training quotas of flashlog.cu:1433-1528 (sampling seed >= 0, more eligible
// edges than K): every eligible group (w > 0, count > 0) first gets
// base = min(count, floor(K*w/wsum)); the residual K - sum(base) is spread
// over the groups' spare capacities by systematic rounding of the spare
// prefix with a SplitMix64 phase per (b, l, source, side).
//
// The reference runs the residual loop sequentially with clamps on each
// group's extra; with cum(p) = floor(residual * p / spare + phase) (residual
// at p == spare) none of those clamps can bind (cum is monotone, below the
// residual, grows by at most a group's spare and stays above
// residual - spare + p, each with a margin of at least 1/spare, far above
// the double rounding error for any budget and graph that fit in int32), so
// a group's extra is exactly cum(p_g) - cum(p_{g-1}), p_g the inclusive
// spare prefix in group order: one wave scan per 64 groups.
//   The reference adds wsum sequentially in group order.  When every
// partial sum is exact in double (all eligible weights are multiples of
// 2^emin and the total stays below 2^(emin+53)) any order gives the same
// bits, and the wave sums in parallel; otherwise the groups are added one by
// one in order.
enum { TAKE_ALL = 0, TAKE_TH = 1, TAKE_QUOTA = 2 };

// Counts in 32 bits: a side's capacity, and with it the target, residual,
// spare and prefixes, is at most the source's edges on that side (CSR
// positions are int32); the double arithmetic is the reference's.
struct SpTake {
    int kind;
    float th;
    int32_t cut;
    double wsum, phase;
    double wsum_r, spare_r;  // RN(1 / wsum), RN(1 / spare)
    int32_t target, residual, spare, prefix, cum;
};

// x / y rounded to nearest, from yr = RN(1 / y) computed once per divisor
// (Markstein's theorem: q0 = RN(x * yr) is within an ulp of x / y, the
// remainder x - q0 * y is exact with an FMA, and RN(q0 + r * yr) is the
// correctly rounded quotient; the operands here stay far from overflow and
// underflow).  Three instructions instead of a full division per group.
__device__ __forceinline__ double sp_div_r(double x, double y, double yr) {
    const double q0 = __dmul_rn(x, yr);
    const double r = __fma_rn(-q0, y, x);
    return __fma_rn(r, yr, q0);
}

__device__ __forceinline__ int32_t sp_quota_base(const SpTake &tk, float wv, int32_t cnt) {
    return (int32_t)fmin((double)cnt,
                         floor(sp_div_r(__dmul_rn((double)tk.target, (double)wv), tk.wsum, tk.wsum_r)));
}

__device__ __forceinline__ int32_t sp_quota_cum(const SpTake &tk, int32_t p) {
    return p == tk.spare ? tk.residual
                         : (int32_t)floor(__dadd_rn(
                               sp_div_r(__dmul_rn((double)tk.residual, (double)p), (double)tk.spare, tk.spare_r),
                               tk.phase));
}

// exponent of the lowest set bit's place value of a positive finite float
__device__ __forceinline__ int sp_lsb_exp(float w) {
    const uint32_t u = __float_as_uint(w);
    const int e = (int)((u >> 23) & 0xFF);
    return (e == 0 ? 1 : e) - 150;
}

// Quota parameters of one (entry, side), computed once by k_sp_select and
// read by the fill: wsum, target = min(K, capacity), residual, spare.
struct SpQuota {
    double wsum;
    long long cap, target, residual, spare;
};

// A side's groups, U windows of 64 at a time (the loads of a batch in
// flight together; one window for sides that have no more groups, so that
// they issue no work for empty windows), each lane visiting its groups in
// order: fn(w, count) for every eligible group (w > 0, count > 0).  Loads at
// clamped indices (every one issued, none behind a branch); groups past the
// side's end are zeroed.
template <int U, typename F>
__device__ __forceinline__ void sp_quota_windows(const int16_t *__restrict__ grel, const int32_t *__restrict__ gcnt,
                                                 uint32_t ng, const float *wr, F &&fn) {
    const int lane = fl_lane();
    for (uint32_t gb = 0; gb < ng; gb += U * FL_WAVE) {
        int rl[U];
        int32_t cl[U];
        float wl[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t g = gb + u * FL_WAVE + (uint32_t)lane;
            const uint32_t gc = g < ng ? g : ng - 1;
            rl[u] = fl_ld32(grel, gc);
            cl[u] = fl_ld32(gcnt, gc);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool in = gb + u * FL_WAVE + (uint32_t)lane < ng;
            const float wraw = fl_ld32(wr, (uint32_t)rl[u]);
            wl[u] = in ? wraw : 0.0f;
            cl[u] = in ? cl[u] : 0;
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (wl[u] > 0.0f && cl[u] > 0) fn(wl[u], cl[u]);
    }
}

template <typename F>
__device__ __forceinline__ void sp_quota_groups(const int16_t *__restrict__ grel, const int32_t *__restrict__ gcnt,
                                                uint32_t ng, const float *wr, F &&fn) {
    if (ng <= FL_WAVE) sp_quota_windows<1>(grel, gcnt, ng, wr, fn);
    else sp_quota_windows<4>(grel, gcnt, ng, wr, fn);
}

__device__ SpQuota sp_quota_setup(const fl_side &s, int64_t g0, int64_t g1, const float *wr, int64_t K) {
    const int lane = fl_lane();
    // 32-bit offsets from the side's first group (a wave-uniform base)
    const uint32_t ng = (uint32_t)(g1 - g0);  // at most 32767: one group per relation
    const int16_t *__restrict__ grel = s.group_rel + g0;
    const int32_t *__restrict__ gcnt = s.group_count + g0;
    // per lane: capacity and eligible groups in 32 bits (at most the
    // source's edges on the side), and the smallest and largest eligible
    // weight as bit patterns (positive floats order as their bits); the
    // place value of the lowest mantissa bit and the exponent are both
    // nondecreasing in the weight, so their extremes come from these two
    double ws = 0.0;
    int32_t cap32 = 0, nel32 = 0;
    uint32_t umin = 0xFFFFFFFFu, umax = 0u;
    sp_quota_groups(grel, gcnt, ng, wr, [&](float wv, int32_t c) {
        cap32 += c;
        ++nel32;
        ws = __dadd_rn(ws, (double)wv);
        const uint32_t u = __float_as_uint(wv);
        umin = min(umin, u);
        umax = max(umax, u);
    });
    // wave totals in 32 bits: at most the source's edges on the side
    const long long cap = fl_wave_sum_i32(cap32);
    const long long nel = fl_wave_sum_i32(nel32);
#pragma unroll
    for (int o = FL_WAVE / 2; o > 0; o >>= 1) {
        ws = __dadd_rn(ws, __shfl_xor(ws, o, FL_WAVE));
        umin = min(umin, (uint32_t)__shfl_xor((int)umin, o, FL_WAVE));
        umax = max(umax, (uint32_t)__shfl_xor((int)umax, o, FL_WAVE));
    }
    int emin = 1 << 20, emax = -(1 << 20);
    if (nel > 0) {
        emin = sp_lsb_exp(__uint_as_float(umin));
        emax = (int)((umax >> 23) & 0xFF) - 127;
    }
    int lg = 0;
    while ((1ll << lg) < nel) ++lg;
    if (emax + 1 + lg - emin > 53) {
        // partial sums may round: the reference's sequential order
        ws = 0.0;
        for (uint32_t gb = 0; gb < ng; gb += FL_WAVE) {
            const uint32_t g = gb + (uint32_t)lane;
            float wv = 0.0f;
            if (g < ng && fl_ld32(gcnt, g) > 0) wv = fl_ld32(wr, (uint32_t)fl_ld32(grel, g));
            const int nl = (int)((ng - gb) < FL_WAVE ? (ng - gb) : FL_WAVE);
            for (int j = 0; j < nl; ++j) {  // group order
                const float wj = __shfl(wv, j, FL_WAVE);
                if (wj > 0.0f) ws = __dadd_rn(ws, (double)wj);
            }
        }
    }
    SpQuota q;
    q.wsum = ws;
    q.cap = cap;
    q.target = K < cap ? K : cap;
    if (cap <= K) {
        // every eligible edge is kept: no quotas, no residual to spread
        q.residual = 0;
        q.spare = 0;
        return q;
    }
    SpTake tk{};
    tk.wsum = fl_uniform_f64(ws);
    tk.wsum_r = __ddiv_rn(1.0, tk.wsum);
    tk.target = (int32_t)q.target;
    int32_t alloc32 = 0;  // at most the lane's capacity
    sp_quota_groups(grel, gcnt, ng, wr, [&](float wv, int32_t c) { alloc32 += sp_quota_base(tk, wv, c); });
    const long long alloc = fl_wave_sum_i32(alloc32);
    q.residual = q.target - alloc;
    q.spare = cap - alloc;
    return q;
}

template <bool Q>
__device__ __forceinline__ SpTake sp_take(int mode, float thv, int32_t ct, const SpQuota *qp, int64_t seed,
                                          int64_t b, int64_t l, int64_t src, int dir) {
    SpTake tk{};
    tk.th = thv;
    tk.cut = ct;
    if (mode == SP_ALL) { tk.kind = TAKE_ALL; return tk; }
    if (!Q || !__builtin_isnan(thv)) { tk.kind = TAKE_TH; return tk; }
    tk.kind = TAKE_QUOTA;
    tk.wsum = qp->wsum;
    tk.wsum_r = __ddiv_rn(1.0, tk.wsum);
    tk.target = (int32_t)qp->target;
    tk.residual = (int32_t)qp->residual;
    tk.spare = (int32_t)qp->spare;
    tk.spare_r = __ddiv_rn(1.0, (double)tk.spare);
    tk.prefix = 0;
    tk.cum = 0;  // cum(0) = floor(phase) = 0
    const uint64_t z = (uint64_t)seed ^ ((uint64_t)b * 0x9e3779b97f4a7c15ull) ^ ((uint64_t)l * 0xbf58476d1ce4e5b9ull) ^
                       ((uint64_t)src * 0x94d049bb133111ebull) ^ (dir ? 0xd1b54a32d192ed03ull : 0x8cb92baa3f3d8dd7ull);
    tk.phase = (double)(fl_splitmix64(z) >> 11) * 0x1.0p-53;
    return tk;
}

// Quota takes of the window's groups (lane j: one group, valid = it exists):
// base + cum(p_g) - cum(p_{g-1}) for eligible groups, carried across windows.
__device__ __forceinline__ int32_t sp_quota_window(SpTake &tk, float wv, int32_t cnt, bool valid) {
    const int lane = fl_lane();
    const bool el = valid && wv > 0.0f && cnt > 0;
    const int32_t base = el ? sp_quota_base(tk, wv, cnt) : 0;
    // a window's spares add up to at most the source's edges on the side
    // and cum stays within the residual
    const int32_t spare = el ? cnt - base : 0;
    const int32_t incl = fl_wave_incl_scan_i32(spare);
    const int32_t cum = sp_quota_cum(tk, tk.prefix + incl);
    const int32_t prev = fl_dpp<0x138>(cum);  // wave_shr:1
    const int32_t extra = cum - (lane == 0 ? tk.cum : prev);
    tk.prefix += __builtin_amdgcn_readlane(incl, FL_WAVE - 1);
    tk.cum = __builtin_amdgcn_readlane(cum, FL_WAVE - 1);
    return el ? base + extra : 0;
}

// Kept runs of one (entry, side) in raw order (group order; a run = the
// first take edges of a group, from CSR position start).  Groups are read
// 64 at a time, lane j holding one group and its kept count (threshold,
// every edge, or the quota window); fn(take, start, rel, wv, ex) is called
// by every lane for each window that keeps an item, with ex = the lane's
// first item index within the side (a wave prefix sum of the takes).
// Returns the side's item count.  KIND: the side's take rule.
template <int KIND, typename F>
__device__ __forceinline__ int64_t sp_side_runs_k(const fl_side &s, int64_t g0, int64_t g1, const float *wr,
                                                  SpTake &tk, F &&fn) {
    const int lane = fl_lane();
    int64_t base = 0;
    // software pipeline over the windows: the records two windows ahead and
    // the weights one window ahead are requested before this window's takes
    // are computed; records at clamped indices, groups past the end zeroed.
    // The windows' registers rotate through three sets (the loop body holds
    // three windows), so that no register copy waits on a load in flight.
    // 32-bit offsets from the side's first group (a wave-uniform base; a side
    // has at most 32767 groups, one per relation).
    const uint32_t ng = (uint32_t)(g1 - g0);
    if (ng == 0) return 0;
    const int16_t *__restrict__ grel = s.group_rel + g0;
    const int32_t *__restrict__ gsta = s.group_start + g0;
    const int32_t *__restrict__ gcnt = s.group_count + g0;
    const uint32_t glast = ng - 1;
    const uint32_t ul = (uint32_t)lane;
    struct Win {
        int rel;
        int32_t start, cnt;
        float w;
    };
    auto load_rec = [&](Win &x, uint32_t gb) {
        const uint32_t gn = gb + ul;
        const uint32_t gc = min(gn, glast);
        x.rel = fl_ld32(grel, gc);
        x.start = fl_ld32(gsta, gc);
        x.cnt = fl_ld32(gcnt, gc);
    };
    // Every load is issued, past the side's end at the clamped index, so
    // that each window waits only for its own loads (a skipped load would
    // make the wait count depend on the path and the waits cover every load).
    Win A, B, C;
    load_rec(A, 0);
    load_rec(B, FL_WAVE);
    A.w = fl_ld32(wr, (uint32_t)A.rel);
    // window gb from cur; nxt holds window gb + 64 (its weights requested
    // here), nx2 receives window gb + 128
    auto step = [&](Win &cur, Win &nxt, Win &nx2, uint32_t gb) {
        load_rec(nx2, gb + 2 * FL_WAVE);
        nxt.w = fl_ld32(wr, (uint32_t)nxt.rel);
        __builtin_amdgcn_sched_barrier(0);  // the loads issued before this window's work
        const bool in = gb + ul < ng;
        const float wv = in ? cur.w : 0.0f;
        const int32_t cnt = in ? cur.cnt : 0;
        int32_t take;
        if (KIND == TAKE_ALL) take = cnt;
        else if (KIND == TAKE_TH) take = group_take32(wv, tk.th, tk.cut, cur.start, cnt);
        else take = sp_quota_window(tk, wv, cnt, in);
        if (__ballot(take > 0) != 0) {
            // a window's takes add up to at most the source's edges (int32)
            const int32_t incl = fl_wave_incl_scan_i32(take);
            fn((long long)take, (int64_t)cur.start, cur.rel, wv, (long long)(base + incl - take));
            base += __builtin_amdgcn_readlane(incl, FL_WAVE - 1);
        }
    };
    for (uint32_t gb = 0;;) {
        step(A, B, C, gb);
        if ((gb += FL_WAVE) >= ng) break;
        step(B, C, A, gb);
        if ((gb += FL_WAVE) >= ng) break;
        step(C, A, B, gb);
        if ((gb += FL_WAVE) >= ng) break;
    }
    return base;
}

// The walk above for the side's take rule (one code path per rule: no
// per-window test of the rule).
template <bool Q, typename F>
__device__ __forceinline__ int64_t sp_side_runs(const fl_side &s, int64_t g0, int64_t g1, const float *wr,
                                                SpTake &tk, F &&fn) {
    if (Q && tk.kind == TAKE_QUOTA) return sp_side_runs_k<TAKE_QUOTA>(s, g0, g1, wr, tk, fn);
    if (tk.kind == TAKE_ALL) return sp_side_runs_k<TAKE_ALL>(s, g0, g1, wr, tk, fn);
    return sp_side_runs_k<TAKE_TH>(s, g0, g1, wr, tk, fn);
}

// Admission order of c2 per (row, side): the relations with a positive
// weight sorted by (weight desc, relation asc), ties in relation order =
// group order (flashlog.cpp:12-89).  Workgroup per (row, side), bitonic sort
// in LDS; sides of more than RO_MAX relations are not ordered (their
// entries use c2_select).
constexpr int RO_MAX = 4096;
constexpr int RO_NT = 256;

__global__ __launch_bounds__(RO_NT) void k_sp_relorder(const float *__restrict__ w, int64_t n, int64_t r_size,
                                                      int16_t *__restrict__ order, int32_t *__restrict__ nelig) {
    __shared__ unsigned long long key[RO_MAX];
    const int64_t row = blockIdx.x >> 1;
    const int side = blockIdx.x & 1;
    const float *wr = w + row * n + (side ? r_size : 0);
    const int t = threadIdx.x;
    int P = 64;
    while (P < r_size) P <<= 1;
    for (int i = t; i < P; i += RO_NT) {
        unsigned long long k = ~0ull;
        if (i < r_size) {
            const float wv = wr[i];
            if (wv > 0.0f) k = ((unsigned long long)(~fl_order_key(wv)) << 32) | (unsigned)i;
        }
        key[i] = k;
    }
    __syncthreads();
    for (int k = 2; k <= P; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = t; i < P; i += RO_NT) {
                const int l = i ^ j;
                if (l > i) {
                    const unsigned long long a = key[i], b = key[l];
                    if (((i & k) == 0) ? (a > b) : (a < b)) {
                        key[i] = b;
                        key[l] = a;
                    }
                }
            }
            __syncthreads();
        }
    int16_t *o = order + (row * 2 + side) * r_size;
    for (int i = t; i < r_size; i += RO_NT) o[i] = key[i] != ~0ull ? (int16_t)(key[i] & 0xFFFFull) : (int16_t)-1;
    if (t == 0) {
        int lo = 0, hi = P;  // first ineligible slot
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (key[mid] != ~0ull) lo = mid + 1;
            else hi = mid;
        }
        nelig[row * 2 + side] = lo < r_size ? lo : (int)r_size;
    }
}

// c2 of one (entry, side) whose source has more than K edges, from the
// row's admission order: the source's group counts are found in that order
// (64 relations at a time) until the cumulative edge count reaches K.  The
// group holding the K-th edge gives the threshold weight and the tie cut
// (its CSR start plus the edges still admitted), the same (threshold, cut)
// as c2_select.  cmap (wave-private LDS, r_size ints, all zero on entry and
// on return) maps relation -> group count; without it each relation is
// found by binary search over the source's group relations.  Returns the
// kept items (lane partial sums).
__device__ __forceinline__ int64_t sp_find_group(const fl_side &s, int64_t g0, int64_t g1, int rel) {
    int64_t lo = g0, hi = g1;
    while (lo < hi) {
        const int64_t mid = lo + ((hi - lo) >> 1);
        if ((int)s.group_rel[mid] < rel) lo = mid + 1;
        else hi = mid;
    }
    return (lo < g1 && (int)s.group_rel[lo] == rel) ? lo : -1;
}

__device__ long long sp_select_lookup(const fl_side &s, int64_t g0, int64_t g1, const float *wr, int64_t K,
                                      const int16_t *__restrict__ ord, int ne, int *cmap, int64_t r_size,
                                      float *thv_out, int32_t *ct_out) {
    const int lane = fl_lane();
    if (cmap) {
        // four windows of group records in flight per round
#pragma unroll 4
        for (int64_t g = g0 + lane; g < g1; g += FL_WAVE) cmap[s.group_rel[g]] = s.group_count[g];
        fl_wave_sync();
    }
    // counts in 32 bits: the source's edges on the side (more than K here)
    // are CSR positions; the next window of the order is requested before
    // this one is counted (two alternating registers, every load issued at
    // an index clamped to the order's end)
    int32_t carry = 0;
    int hit_rel = -1;
    int32_t hit_before = 0;
    const int32_t K32 = (int32_t)K;
    auto ord_at = [&](int k0) { return ne > 0 ? (int)ord[min(k0 + lane, ne - 1)] : -1; };
    auto window = [&](int k0, int rel_raw) {  // true: the K-th edge is in this window
        const int rel = k0 + lane < ne ? rel_raw : -1;
        int32_t cnt = 0;
        if (rel >= 0) {
            if (cmap) {
                cnt = cmap[rel];
            } else {
                const int64_t g = sp_find_group(s, g0, g1, rel);
                cnt = g >= 0 ? s.group_count[g] : 0;
            }
        }
        const int32_t incl = fl_wave_incl_scan_i32(cnt);
        const int32_t before = carry + incl - cnt;
        const bool hit = cnt > 0 && before < K32 && before + cnt >= K32;
        const unsigned long long bal = __ballot(hit);
        if (bal) {
            const int hl = __ffsll((long long)bal) - 1;
            hit_rel = __shfl(rel, hl, FL_WAVE);
            hit_before = __shfl(before, hl, FL_WAVE);
            return true;
        }
        carry += __builtin_amdgcn_readlane(incl, FL_WAVE - 1);
        return false;
    };
    int ra = ord_at(0), rb = 0;
    for (int k0 = 0; k0 < ne;) {
        rb = ord_at(k0 + FL_WAVE);
        if (window(k0, ra)) break;
        if ((k0 += FL_WAVE) >= ne) break;
        ra = ord_at(k0 + FL_WAVE);
        if (window(k0, rb)) break;
        k0 += FL_WAVE;
    }
    if (cmap) {
        // the whole map cleared from LDS alone (no second read of the records)
        fl_wave_sync();
        for (int64_t q = lane; q < r_size; q += FL_WAVE) cmap[q] = 0;
        fl_wave_sync();
    }
    if (hit_rel >= 0) {
        const int64_t gj = sp_find_group(s, g0, g1, hit_rel);
        *thv_out = wr[hit_rel];
        *ct_out = (int32_t)(s.group_start[gj] + (K - hit_before));
        return lane == 0 ? K : 0;
    }
    *thv_out = 0.0f;  // fewer than K eligible edges: every one is kept
    *ct_out = 0;
    return lane == 0 ? carry : 0;
}

// One wave per entry: per side the c2 threshold (bits of the threshold
// weight, 0 = no pruning, NaN = training quotas) and tie cut, and the number
// of raw items: kept edges (top-k mode; for the sum a kept edge with a zero
// mask becomes a hole, raw destination -1, skipped downstream) or every edge
// (all-edges mode), plus the identity item.  With quotas the side keeps
// exactly min(eligible, K) edges, as the threshold does.
constexpr int SEL_NT = 256;
constexpr int SP_ICHUNK = FL_WAVE;  // raw items per chunk of the item pass
constexpr int SEL_MAP_MAX = 2048;  // relations per side of the LDS count maps

template <bool QS>
__global__ __launch_bounds__(SEL_NT) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_sp_select(fl_side ori, fl_side inv, const int64_t *__restrict__ sb,
                                                     const int64_t *__restrict__ sl, const int64_t *__restrict__ se,
                                                     int64_t nnz, const float *__restrict__ w, int64_t B, int64_t L,
                                                     int64_t E, int64_t n, int64_t r_size, int wot_i, int mode, int64_t K,
                                                     int64_t seed, float *__restrict__ th, int32_t *__restrict__ cut,
                                                     int32_t *__restrict__ cnt, const int16_t *__restrict__ rel_order,
                                                     const int32_t *__restrict__ rel_nelig, int use_map,
                                                     SpQuota *__restrict__ qout, int32_t *__restrict__ nch,
                                                     const int32_t *__restrict__ order) {
    __shared__ int hist_all[SEL_NT / FL_WAVE][256];
    extern __shared__ int cmap_all[];  // [SEL_NT / FL_WAVE][r_size] when the map is used
    const int lane = fl_lane();
    const int wid = fl_wave_id();
    const int64_t wv_i = (int64_t)blockIdx.x * (SEL_NT / FL_WAVE) + wid;
    // entries visited in the given order (by source entity: neighbouring
    // waves read the same group records), results stored by entry
    const int64_t i = (order && wv_i < nnz) ? (int64_t)order[wv_i] : wv_i;
    int *cmap = use_map ? cmap_all + wid * r_size : nullptr;
    if (cmap) {
        for (int64_t q = lane; q < r_size; q += FL_WAVE) cmap[q] = 0;
        fl_wave_sync();
    }
    if (i < 0 || i >= nnz) return;  // (an order outside [0, nnz) is reported by the plan)
    const int64_t src = se[i];
    if (sb[i] < 0 || sb[i] >= B || sl[i] < 0 || sl[i] >= L || src < 0 || src >= E) {
        if (lane == 0) {
            cnt[i] = 0;
            nch[i] = 0;
            th[2 * i] = th[2 * i + 1] = 0.0f;
            cut[2 * i] = cut[2 * i + 1] = 0;
        }
        return;  // reported by k_sp_rowptr; the plan is not used
    }
    const float *wrow = w + (sb[i] * L + sl[i]) * n;
    int total = wot_i ? 0 : 1;
    for (int dir = 0; dir < 2; ++dir) {
        const fl_side &s = dir ? inv : ori;
        const float *wr = wrow + (dir ? r_size : 0);
        const int64_t g0 = s.row_group_ptr[src], g1 = s.row_group_ptr[src + 1];
        float thv = 0.0f;
        int32_t ct = 0;
        long long c = 0;
        if (mode == SP_ALL) {
            for (int64_t g = g0 + lane; g < g1; g += FL_WAVE) c += s.group_count[g];
        } else if (K > 0 && seed < 0 && rel_order && g1 - g0 > FL_WAVE) {
            // more than one window of groups: every edge kept when the source
            // has at most K, else the admission-order lookup
            const int64_t deg = (int64_t)s.group_start[g1 - 1] + s.group_count[g1 - 1] - s.group_start[g0];
            if (deg <= K) {
#pragma unroll 4
                for (int64_t g = g0 + lane; g < g1; g += FL_WAVE)
                    c += wr[s.group_rel[g]] > 0.0f ? s.group_count[g] : 0;
            } else {
                const int64_t ro = (sb[i] * L + sl[i]) * 2 + dir;
                c = sp_select_lookup(s, g0, g1, wr, K, rel_order + ro * r_size, rel_nelig[ro], cmap, r_size, &thv,
                                     &ct);
            }
        } else {
            uint32_t key;
            int32_t cc;
            bool quota = false;
            long long eligible = -1;
            if (K < 0) {
                thv = __int_as_float(0x7f800000);  // budget <= 0: no edge is kept
            } else if (QS && K > 0 && seed >= 0) {
                const SpQuota q = sp_quota_setup(s, g0, g1, wr, K);
                quota = q.cap > K;  // more eligible edges than the budget
                if (quota) {
                    thv = __int_as_float(0x7fc00000);
                    if (lane == 0) qout[2 * i + dir] = q;
                }
                eligible = q.cap;  // without quotas every eligible edge is kept
            } else if (K > 0 && c2_select(s, g0, g1, wr, K, hist_all[wid], &key, &cc)) {
                thv = __uint_as_float(key);
                ct = cc;
            }
            if (quota) {
                c = lane == 0 ? K : 0;
            } else if (eligible >= 0) {
                c = lane == 0 ? eligible : 0;
            } else {
                // kept edges, masked ones included
                for (int64_t g = g0 + lane; g < g1; g += FL_WAVE)
                    c += group_take32(wr[s.group_rel[g]], thv, ct, s.group_start[g], s.group_count[g]);
            }
        }
        c = fl_wave_sum_i64(c);
        total += (int)c;
        if (lane == 0) {
            th[2 * i + dir] = thv;
            cut[2 * i + dir] = ct;
        }
    }
    if (lane == 0) {
        cnt[i] = total;
        nch[i] = (total + SP_ICHUNK - 1) / SP_ICHUNK;  // 64-item chunks of the entry's items
    }
}

// Fixed-relation rule step (flashlog.cu:1561-1741): entry (b, l, e, v) with
// operator op = operators[b*L + l] goes to every edge of its (e, op) group
// with the value unchanged (op < R: ORI relation op; R <= op < 2R: INV
// relation op - R; op == 2R: the identity, one item at e).  No masks and no
// budgets.  k_fx_count: thread per entry, the group by binary search over
// the source's group relations (stored in cut[2i], side in cut[2i+1]).
__device__ __forceinline__ int64_t fx_find_group(const fl_side &s, int64_t src, int rel) {
    int64_t lo = s.row_group_ptr[src], hi = s.row_group_ptr[src + 1];
    const int64_t end = hi;
    while (lo < hi) {
        const int64_t mid = lo + ((hi - lo) >> 1);
        if ((int)s.group_rel[mid] < rel) lo = mid + 1;
        else hi = mid;
    }
    return (lo < end && (int)s.group_rel[lo] == rel) ? lo : -1;
}

__global__ void k_fx_count(fl_side ori, fl_side inv, const int64_t *__restrict__ sb, const int64_t *__restrict__ sl,
                           const int64_t *__restrict__ se, const int64_t *__restrict__ ops, int64_t nnz, int64_t B,
                           int64_t L, int64_t E, int64_t R, int32_t *__restrict__ cut, int32_t *__restrict__ cnt) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nnz) return;
    const int64_t b = sb[i], l = sl[i], src = se[i];
    int32_t c = 0, g = -1, side = 0;
    if (b >= 0 && b < B && l >= 0 && l < L && src >= 0 && src < E) {
        const int64_t op = ops[b * L + l];
        if (op == 2 * R) {
            c = 1;
            side = 2;
        } else if (op >= 0 && op < 2 * R) {
            side = op >= R ? 1 : 0;
            const fl_side &s = side ? inv : ori;
            const int64_t gg = fx_find_group(s, src, (int)(side ? op - R : op));
            if (gg >= 0) {
                g = (int32_t)gg;
                c = s.group_count[gg];
            }
        }
    }
    cut[2 * i] = g;
    cut[2 * i + 1] = side;
    cnt[i] = c;
}

// Wave per entry: the entry's items (group columns, or itself) at item_off[i].
__global__ __launch_bounds__(SEL_NT) void k_fx_fill(fl_side ori, fl_side inv, const int64_t *__restrict__ se,
                                                   const float *__restrict__ sv, int64_t nnz,
                                                   const int32_t *__restrict__ cut,
                                                   const int64_t *__restrict__ item_off,
                                                   int32_t *__restrict__ raw_dst, float *__restrict__ raw_val) {
    const int lane = fl_lane();
    const int64_t i = (int64_t)blockIdx.x * (SEL_NT / FL_WAVE) + fl_wave_id();
    if (i >= nnz) return;
    const int64_t pos = item_off[i];
    const int64_t c = item_off[i + 1] - pos;
    if (c == 0) return;
    const float v = sv[i];
    const int32_t side = cut[2 * i + 1];
    if (side == 2) {
        if (lane == 0) {
            raw_dst[pos] = (int32_t)se[i];
            raw_val[pos] = v;
        }
        return;
    }
    const fl_side &s = side ? inv : ori;
    const int64_t start = s.group_start[cut[2 * i]];
    for (int64_t k = lane; k < c; k += FL_WAVE) {
        raw_dst[pos + k] = s.col_ind[start + k];
        raw_val[pos + k] = v;
    }
}

// Per row r (and r = R): first item and tile count.
__global__ void k_sp_rowinfo(const int64_t *__restrict__ row_ptr, const int64_t *__restrict__ item_off, int64_t R,
                             int64_t *__restrict__ row_item0, int32_t *__restrict__ ntiles) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r > R) return;
    const int64_t a = item_off[row_ptr[r]];
    row_item0[r] = a;
    if (r < R) {
        const int64_t b = item_off[row_ptr[r + 1]];
        ntiles[r] = (int32_t)((b - a + SP_TILE - 1) / SP_TILE);
    }
}

// ---------------------------------------------------------------------------
// expand

struct SpRows {
    const int64_t *row_item0;  // [R+1]
    const int64_t *tile_base;  // [R+1]
    int64_t NB;                // buckets per row
};

// Mask of position p on a side: its bit when the side has a bitmap (every
// mask value 0 or 1), else the mask value.
__device__ __forceinline__ float sp_mask_at(const uint32_t *bits, const float *mask, int64_t p) {
    return bits ? (((bits[p >> 5] >> (p & 31)) & 1u) ? 1.0f : 0.0f) : mask[p];
}

// Raw items are written in two passes.  k_sp_runs (wave per entry) walks
// the entry's groups as the plan did and writes one descriptor per kept
// group (a run: the group's first take edges, at consecutive item slots)
// plus one for the identity item, at run slot item_off[i] + (its index in
// the entry) (an entry has at most as many runs as items): its first item
// (within the entry), CSR position (the source for the identity), a * w of
// its relation, and its attention column | side flags.  An entry's items
// are cut into chunks of 64 (chunk_off from the plan); for each chunk the
// walk records its first item, item count, the run holding that item and
// the entry's run-slot limit.  k_sp_items (wave per chunk) then writes the
// chunk's items from the at most 64 runs that touch it, all lanes loading
// and storing consecutive slots.
constexpr uint32_t SP_RUN_INV = 0x80000000u;  // run of the INV side
constexpr uint32_t SP_RUN_ID = 0x40000000u;   // the identity item
constexpr uint32_t SP_RUN_COL = 0x3FFFFFFFu;  // attention column

struct SpRuns {
    int32_t *first;    // [items] first item of the run within its entry
    int32_t *p;        // [items] CSR position of the first item (identity: the source)
    float *aw;         // [items] a * w[column]
    uint32_t *meta;    // [items] column | SP_RUN_INV | SP_RUN_ID
    int64_t *c_base;   // [chunks] first item slot of the chunk's entry
    int64_t *c_run;    // [chunks] run slot holding the chunk's first item
    int64_t *c_rlim;   // [chunks] end of the entry's run slots
    int32_t *c_off;    // [chunks] first item of the chunk within the entry
    int32_t *c_n;      // [chunks] items in the chunk
};

template <bool Q>
__global__ __launch_bounds__(SEL_NT) void k_sp_runs(fl_side ori, fl_side inv, const int64_t *__restrict__ sb,
                                                   const int64_t *__restrict__ sl, const int64_t *__restrict__ se,
                                                   const float *__restrict__ sv, int64_t nnz,
                                                   const float *__restrict__ w, int64_t L, int64_t n,
                                                   int64_t r_size, int wot_i, int mode, int64_t seed,
                                                   const float *__restrict__ th, const int32_t *__restrict__ cut,
                                                   const SpQuota *__restrict__ quota,
                                                   const int64_t *__restrict__ item_off,
                                                   const int64_t *__restrict__ chunk_off,
                                                   const int32_t *__restrict__ order, SpRuns ru) {
    const int lane = fl_lane();
    const int64_t wv_i = (int64_t)blockIdx.x * (SEL_NT / FL_WAVE) + fl_wave_id();
    if (wv_i >= nnz) return;
    // entry visited in the plan's order; its chunks follow that order
    const int64_t i = order ? (int64_t)order[wv_i] : wv_i;
    if (i < 0 || i >= nnz) return;
    const int64_t src = se[i];
    const int64_t r = sb[i] * L + sl[i];
    const float a = sv[i];
    const float *wrow = w + r * n;
    const int64_t base = item_off[i];
    const int64_t nitems = item_off[i + 1] - base;
    const int64_t u0 = chunk_off[wv_i];
    // the plan's item count bounds every write (the walk reproduces it)
    const int64_t lim = nitems - (wot_i ? 0 : 1);
    int64_t pos = 0, rix = 0;  // within the entry
    const uint64_t below = (1ull << lane) - 1;
    for (int dir = 0; dir < 2; ++dir) {
        const fl_side &s = dir ? inv : ori;
        const float *wr = wrow + (dir ? r_size : 0);
        const int64_t g0 = s.row_group_ptr[src], g1 = s.row_group_ptr[src + 1];
        SpTake tk = sp_take<Q>(mode, th[2 * i + dir], cut[2 * i + dir], quota + 2 * i + dir, seed, sb[i], sl[i], src,
                               dir);
        const uint32_t side = dir ? SP_RUN_INV : 0u;
        const uint32_t col0 = dir ? (uint32_t)r_size : 0u;
        pos += sp_side_runs<Q>(s, g0, g1, wr, tk, [&](long long take, int64_t start, int rel, float wv, long long ex) {
            const uint64_t m = __ballot(take > 0);
            const int64_t ri = rix + __popcll(m & below);
            const int64_t o = pos + ex;
            if (take > 0 && o + take <= lim) {  // then ri < o + 1 <= nitems
                ru.first[base + ri] = (int32_t)o;
                ru.p[base + ri] = (int32_t)start;
                ru.aw[base + ri] = fl_mul(a, wv);
                ru.meta[base + ri] = side | (col0 + (uint32_t)rel);
                for (int64_t q = (o + SP_ICHUNK - 1) / SP_ICHUNK; q * SP_ICHUNK < o + take; ++q)
                    ru.c_run[u0 + q] = base + ri;
            }
            rix += __popcll(m);
        });
    }
    if (!wot_i && lane == 0 && pos == lim && rix <= lim) {
        ru.first[base + rix] = (int32_t)lim;
        ru.p[base + rix] = (int32_t)src;
        ru.aw[base + rix] = fl_mul(a, wrow[n - 1]);
        ru.meta[base + rix] = SP_RUN_ID | (uint32_t)(n - 1);
        if (lim % SP_ICHUNK == 0) ru.c_run[u0 + lim / SP_ICHUNK] = base + rix;
    }
    const int64_t nr = rix + (wot_i ? 0 : 1);
    const int64_t nq = chunk_off[wv_i + 1] - u0;
    for (int64_t q = lane; q < nq; q += FL_WAVE) {
        const int64_t c0 = q * SP_ICHUNK;
        ru.c_base[u0 + q] = base;
        ru.c_rlim[u0 + q] = base + (nr < nitems ? nr : nitems);
        ru.c_off[u0 + q] = (int32_t)c0;
        ru.c_n[u0 + q] = (int32_t)(nitems - c0 < SP_ICHUNK ? nitems - c0 : SP_ICHUNK);
    }
}

// Wave per chunk (grid-stride): lane j loads run slot r0 + j (r0 holds the
// chunk's first item); the runs starting inside the chunk mark their first
// slot in LDS, and the owner of slot k is the number of marks at slots
// 1..k (an entry's runs tile its items in order).  The items are the
// reference's raw items: destination (-1 for a masked edge of the top-k
// sum), value (a * w) * m, and for the max the tie key, for the backward
// the CSR position and attention column.
constexpr int SP_ITEMS_NT = 256;
constexpr int64_t SP_ITEMS_GRID = 8192;  // workgroups of the grid-stride item pass

template <bool MAXT, bool BWD>
__global__ __launch_bounds__(SP_ITEMS_NT) void k_sp_items(fl_side ori, fl_side inv, int64_t nchunks, SpRuns ru,
                                                         int holes, int32_t *__restrict__ raw_dst,
                                                         float *__restrict__ raw_val, uint32_t *__restrict__ raw_tie,
                                                         int32_t *__restrict__ raw_pos,
                                                         int16_t *__restrict__ raw_col) {
    __shared__ uint8_t mark_all[SP_ITEMS_NT / FL_WAVE][SP_ICHUNK];
    const int lane = fl_lane();
    uint8_t *mark = mark_all[fl_wave_id()];
    const int64_t waves = (int64_t)gridDim.x * (SP_ITEMS_NT / FL_WAVE);
    const uint64_t upto = lane == FL_WAVE - 1 ? ~0ull : ((2ull << lane) - 1);
    for (int64_t c = (int64_t)blockIdx.x * (SP_ITEMS_NT / FL_WAVE) + fl_wave_id(); c < nchunks; c += waves) {
        const int64_t base = fl_uniform_i64(ru.c_base[c]);
        const int64_t r0 = fl_uniform_i64(ru.c_run[c]);
        const int64_t rlim = fl_uniform_i64(ru.c_rlim[c]);
        const int off = __builtin_amdgcn_readfirstlane(ru.c_off[c]);
        const int cn = __builtin_amdgcn_readfirstlane(ru.c_n[c]);
        const int64_t rj = r0 + lane;
        int32_t d = SP_ICHUNK, rp = 0;
        float aw = 0.0f;
        uint32_t rm = 0;
        if (rj >= base && rj < rlim) {
            // first item of the run relative to the chunk's (both within the entry)
            const int32_t f = ru.first[rj] - off;
            d = f < SP_ICHUNK ? f : SP_ICHUNK;
            rp = ru.p[rj];
            aw = ru.aw[rj];
            rm = ru.meta[rj];
        }
        mark[lane] = 0;
        fl_wave_sync();
        if (lane > 0 && d > 0 && d < SP_ICHUNK) mark[d] = 1;
        fl_wave_sync();
        const uint64_t starts = __ballot(mark[lane] != 0);
        const int j = __popcll(starts & upto);
        const int32_t dj = __shfl(d, j, FL_WAVE);
        const int32_t pj = __shfl(rp, j, FL_WAVE) + (lane - dj);
        const float awj = __shfl(aw, j, FL_WAVE);
        const uint32_t mj = (uint32_t)__shfl((int)rm, j, FL_WAVE);
        fl_wave_sync();  // marks read before the next chunk clears them
        if (lane >= cn) continue;
        const int64_t k = base + off + lane;
        int32_t dst = -1, pos = -1;
        float val = 0.0f;
        uint32_t tie = SP_TIE_IDENTITY;
        if (mj & SP_RUN_ID) {
            dst = pj;
            val = awj;
        } else {
            const bool inv_side = (mj & SP_RUN_INV) != 0;
            const int64_t edges = inv_side ? inv.edges : ori.edges;
            const float *mk = inv_side ? inv.mask : ori.mask;
            const uint32_t *mb = inv_side ? inv.mask_bits : ori.mask_bits;
            const int32_t *ci = inv_side ? inv.col_ind : ori.col_ind;
            if (pj >= 0 && pj < edges) {
                const float m = sp_mask_at(mb, mk, pj);
                const int32_t e = ci[pj];
                dst = (!holes || m != 0.0f) ? e : -1;
                val = fl_mul(awj, m);
                if (MAXT) tie = (inv_side ? SP_TIE_INV : 0u) | (uint32_t)(inv_side ? inv.order : ori.order)[pj];
                pos = pj;
            }
        }
        raw_dst[k] = dst;
        raw_val[k] = val;
        if (MAXT) raw_tie[k] = tie;
        if (BWD) {
            if (raw_pos) raw_pos[k] = pos;
            raw_col[k] = (int16_t)(mj & SP_RUN_COL);
        }
    }
}

// Fused run writer and item pass for budgeted (top-k) hops, whose entries
// have at most 2K+1 items: wave per entry, the entry's runs (as k_sp_runs
// writes them) kept in the wave's LDS instead of a global run table, then
// the entry's items written 64 at a time as k_sp_items writes a chunk (the
// runs starting inside the round marked in LDS, the owner of slot k the
// number of marks at 1..k).  rcap: runs per wave the dynamic LDS holds.
constexpr int64_t SP_FUSE_KMAX = 256;  // budgets whose runs fit the fused kernel's LDS
constexpr int64_t SP_OFF32_EDGES = (int64_t)1 << 30;  // positions addressed with 32-bit byte offsets

// A run in LDS, one 8-byte record (one LDS store and one load per run):
// x = first item << 20 | side and identity flags (bits 19, 18) | column,
// y = CSR position.  The item pass takes a*w as a * w[column], the product
// the walk formed (the same float load and multiply).
struct SpLdsRuns {
    int2 *rec;
};
constexpr int SP_LR_FIRST = 20;
constexpr uint32_t SP_LR_INV = 1u << 19, SP_LR_ID = 1u << 18, SP_LR_COL = (1u << 18) - 1;
__device__ __forceinline__ int32_t sp_lr_pack(int32_t first, uint32_t meta) {
    const uint32_t fl = ((meta & SP_RUN_INV) ? SP_LR_INV : 0u) | ((meta & SP_RUN_ID) ? SP_LR_ID : 0u);
    return (int32_t)(((uint32_t)first << SP_LR_FIRST) | fl | (meta & SP_LR_COL));
}
__device__ __forceinline__ uint32_t sp_lr_meta(int32_t x) {
    const uint32_t u = (uint32_t)x;
    return ((u & SP_LR_INV) ? SP_RUN_INV : 0u) | ((u & SP_LR_ID) ? SP_RUN_ID : 0u) | (u & SP_LR_COL);
}

template <bool Q, bool MAXT, bool BWD>
__global__ __launch_bounds__(SEL_NT) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_sp_expand_fused(
    fl_side ori, fl_side inv, const int64_t *__restrict__ sb, const int64_t *__restrict__ sl,
    const int64_t *__restrict__ se, const float *__restrict__ sv, int64_t nnz, const float *__restrict__ w, int64_t L,
    int64_t n, int64_t r_size, int wot_i, int mode, int64_t seed, const float *__restrict__ th,
    const int32_t *__restrict__ cut, const SpQuota *__restrict__ quota, const int64_t *__restrict__ item_off,
    const int32_t *__restrict__ order, int rcap, int holes, int32_t *__restrict__ raw_dst, float *__restrict__ raw_val,
    uint32_t *__restrict__ raw_tie, int32_t *__restrict__ raw_pos, int16_t *__restrict__ raw_col) {
    extern __shared__ __align__(16) unsigned char fused_lds[];
    __shared__ uint8_t mark_all[SEL_NT / FL_WAVE][SP_ICHUNK];
    const int lane = fl_lane();
    const int wid = fl_wave_id();
    uint8_t *mark = mark_all[wid];
    SpLdsRuns ru;
    {
        ru.rec = reinterpret_cast<int2 *>(fused_lds + (size_t)wid * rcap * 8);
    }
    const int64_t wv_i = (int64_t)blockIdx.x * (SEL_NT / FL_WAVE) + wid;
    if (wv_i >= nnz) return;  // no block barrier follows
    const int64_t i = order ? (int64_t)order[wv_i] : wv_i;
    if (i < 0 || i >= nnz) return;
    const int64_t src = se[i];
    const int64_t r = sb[i] * L + sl[i];
    const float a = sv[i];
    const float *wrow = w + r * n;
    const int64_t base = item_off[i];
    const int64_t nitems = item_off[i + 1] - base;
    // the plan's item count bounds every run (the walk reproduces it)
    // per-entry counts in 32 bits (at most 2K+1 items)
    const int32_t lim = (int32_t)nitems - (wot_i ? 0 : 1);
    int32_t pos = 0, rix = 0;  // within the entry
    const uint64_t below = (1ull << lane) - 1;
    for (int dir = 0; dir < 2; ++dir) {
        const fl_side &s = dir ? inv : ori;
        const float *wr = wrow + (dir ? r_size : 0);
        const int64_t g0 = s.row_group_ptr[src], g1 = s.row_group_ptr[src + 1];
        SpTake tk = sp_take<Q>(mode, th[2 * i + dir], cut[2 * i + dir], quota + 2 * i + dir, seed, sb[i], sl[i], src,
                               dir);
        const uint32_t side = dir ? SP_RUN_INV : 0u;
        const uint32_t col0 = dir ? (uint32_t)r_size : 0u;
        pos += (int32_t)sp_side_runs<Q>(s, g0, g1, wr, tk, [&](long long take, int64_t start, int rel, float wv,
                                                               long long ex) {
            const uint64_t m = __ballot(take > 0);
            const int32_t ri = rix + __popcll(m & below);
            const int32_t o = pos + (int32_t)ex;
            if (take > 0 && o + (int32_t)take <= lim && ri < rcap)
                ru.rec[ri] = make_int2(sp_lr_pack(o, side | (col0 + (uint32_t)rel)), (int32_t)start);
            rix += __popcll(m);
        });
    }
    if (!wot_i && lane == 0 && pos == lim && rix < rcap)
        ru.rec[rix] = make_int2(sp_lr_pack(lim, SP_RUN_ID | (uint32_t)(n - 1)), (int32_t)src);
    int32_t nr = rix + (wot_i ? 0 : 1);
    if (nr > rcap) nr = rcap;
    fl_wave_sync();
    const uint64_t upto = lane == FL_WAVE - 1 ? ~0ull : ((2ull << lane) - 1);
    int32_t r0 = 0;  // the run holding the round's first item
    for (int32_t q0 = 0; q0 < (int32_t)nitems; q0 += SP_ICHUNK) {
        const int32_t rj = r0 + lane;
        int32_t d = SP_ICHUNK, rp = 0;
        uint32_t rm = 0;
        if (rj < nr) {
            const int2 x = ru.rec[rj];
            const int32_t f = (int32_t)((uint32_t)x.x >> SP_LR_FIRST) - q0;
            d = f < SP_ICHUNK ? f : SP_ICHUNK;
            rp = x.y;
            rm = sp_lr_meta(x.x);
        }
        mark[lane] = 0;
        fl_wave_sync();
        if (lane > 0 && d > 0 && d < SP_ICHUNK) mark[d] = 1;
        fl_wave_sync();
        const uint64_t starts = __ballot(mark[lane] != 0);
        const int j = __popcll(starts & upto);
        const int32_t dj = __shfl(d, j, FL_WAVE);
        const int32_t pj = __shfl(rp, j, FL_WAVE) + (lane - dj);
        const uint32_t mj = (uint32_t)__shfl((int)rm, j, FL_WAVE);
        // the next round's first item: in the last run that started here, or
        // in the run starting right at it
        r0 += __popcll(starts);
        if (r0 + 1 < nr && (int32_t)((uint32_t)ru.rec[r0 + 1].x >> SP_LR_FIRST) <= q0 + SP_ICHUNK) ++r0;
        fl_wave_sync();  // marks read before the next round clears them
        const int32_t it = q0 + lane;
        const bool live = it < (int32_t)nitems;
        // the sides of the round's edge items: one side but for the round
        // that crosses from the ORI runs to the INV runs
        const bool edge_it = live && !(mj & SP_RUN_ID);
        const uint64_t inv_items = __ballot(edge_it && (mj & SP_RUN_INV));
        const uint64_t ori_items = __ballot(edge_it && !(mj & SP_RUN_INV));
        if (!live) continue;
        const float wc = fl_ld32(wrow, mj & SP_RUN_COL);  // a * wc formed where it is used
        int32_t dst = -1, pp = -1;
        float val = 0.0f;
        uint32_t tie = SP_TIE_IDENTITY;
        // an edge item of side s (wave-uniform: its arrays from scalar bases
        // and 32-bit byte offsets, for sides of fewer than 2^30 positions)
        auto side_item = [&](const fl_side &s, bool inv_side) {
            if ((uint32_t)pj < (uint32_t)s.edges) {
                const int32_t e = fl_ld32(s.col_ind, (uint32_t)pj);  // requested before the mask
                const float m = s.mask_bits ? (((fl_ld32(s.mask_bits, (uint32_t)pj >> 5) >> (pj & 31)) & 1u) ? 1.0f : 0.0f)
                                            : fl_ld32(s.mask, (uint32_t)pj);
                dst = (!holes || m != 0.0f) ? e : -1;
                val = fl_mul(fl_mul(a, wc), m);
                if (MAXT) tie = (inv_side ? SP_TIE_INV : 0u) | (uint32_t)fl_ld32(s.order, (uint32_t)pj);
                pp = pj;
            }
        };
        if (mj & SP_RUN_ID) {
            dst = pj;
            val = fl_mul(a, wc);
        } else if (inv_items == 0 && ori.edges < SP_OFF32_EDGES) {
            side_item(ori, false);
        } else if (ori_items == 0 && inv.edges < SP_OFF32_EDGES) {
            side_item(inv, true);
        } else {
            const bool inv_side = (mj & SP_RUN_INV) != 0;
            const uint32_t edges = (uint32_t)(inv_side ? inv.edges : ori.edges);
            const float *mk = inv_side ? inv.mask : ori.mask;
            const uint32_t *mb = inv_side ? inv.mask_bits : ori.mask_bits;
            const int32_t *ci = inv_side ? inv.col_ind : ori.col_ind;
            if ((uint32_t)pj < edges) {
                const float m = sp_mask_at(mb, mk, pj);
                const int32_t e = ci[pj];
                dst = (!holes || m != 0.0f) ? e : -1;
                val = fl_mul(fl_mul(a, wc), m);
                if (MAXT) tie = (inv_side ? SP_TIE_INV : 0u) | (uint32_t)(inv_side ? inv.order : ori.order)[pj];
                pp = pj;
            }
        }
        // the entry's items from wave-uniform bases, 32-bit offsets
        fl_st32(raw_dst + base, (uint32_t)it, dst);
        fl_st32(raw_val + base, (uint32_t)it, val);
        if (MAXT) fl_st32(raw_tie + base, (uint32_t)it, tie);
        if (BWD) {
            if (raw_pos) fl_st32(raw_pos + base, (uint32_t)it, pp);
            fl_st32(raw_col + base, (uint32_t)it, (int16_t)(mj & SP_RUN_COL));
        }
    }
}

// Row of a tile: the r with tile_base[r] <= tile < tile_base[r+1].
__device__ __forceinline__ int64_t sp_tile_row(const int64_t *tile_base, int64_t R, int64_t tile) {
    int64_t lo = 0, hi = R;  // invariant: tile_base[lo] <= tile < tile_base[hi]
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (tile_base[mid] <= tile) lo = mid;
        else hi = mid;
    }
    return lo;
}

// Workgroup per tile of a row: the tile's destination-bucket histogram
// (LDS atomics), written as hist[tile * NB + bucket] (coalesced) for
// k_sp_vscan.  Holes (destination -1) are not counted.
__global__ __launch_bounds__(SP_NT) void k_sp_hist(int64_t R, SpRows rows, const int32_t *__restrict__ raw_dst,
                                                  int32_t *__restrict__ hist) {
    extern __shared__ int hb[];  // [NB]
    const int64_t tile = fl_xcd_contig(blockIdx.x, gridDim.x);
    const int64_t r = sp_tile_row(rows.tile_base, R, tile);
    const int64_t tl = tile - rows.tile_base[r];
    const int64_t i0 = rows.row_item0[r] + tl * SP_TILE;
    const int64_t i1e = rows.row_item0[r + 1];
    const int c = (int)((i1e - i0) < SP_TILE ? (i1e - i0) : SP_TILE);
    for (int64_t q = threadIdx.x; q < rows.NB; q += SP_NT) hb[q] = 0;
    __syncthreads();
    const int32_t *__restrict__ tdst = raw_dst + i0;
    if (c == SP_TILE) {
        // a full tile: every load in flight before the LDS atomics
        constexpr int Q = SP_TILE / SP_NT;
        int32_t dd[Q];
#pragma unroll
        for (int j = 0; j < Q; ++j) dd[j] = fl_ld32(tdst, (uint32_t)(j * SP_NT) + threadIdx.x);
#pragma unroll
        for (int j = 0; j < Q; ++j)
            if (dd[j] >= 0) atomicAdd(&hb[dd[j] >> SP_S], 1);
    } else {
        for (uint32_t idx = threadIdx.x; idx < (uint32_t)c; idx += SP_NT) {
            const int32_t d = fl_ld32(tdst, idx);
            if (d >= 0) atomicAdd(&hb[d >> SP_S], 1);
        }
    }
    __syncthreads();
    int32_t *hrow = hist + tile * rows.NB;
    for (int64_t q = threadIdx.x; q < rows.NB; q += SP_NT) hrow[q] = hb[q];
}

// Thread per (row, bucket): the bucket's count in each of the row's tiles
// replaced by the exclusive prefix over the row's earlier tiles (in place),
// the bucket's total to tot[row * NB + bucket] (then scanned into the
// buckets' first positions).  Neighbouring threads read neighbouring
// buckets of one tile: every access is coalesced.
__global__ void k_sp_vscan(int64_t R, SpRows rows, int32_t *__restrict__ hist, int32_t *__restrict__ tot) {
    const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= R * rows.NB) return;
    const int64_t r = s / rows.NB, bk = s - r * rows.NB;
    int32_t run = 0;
    for (int64_t t = rows.tile_base[r]; t < rows.tile_base[r + 1]; ++t) {
        const int32_t c = hist[t * rows.NB + bk];
        hist[t * rows.NB + bk] = run;
        run += c;
    }
    tot[s] = run;
}

// Stable LSD block sort of SP_NT * IPT keys held in LDS (kin, in positions
// 0 .. SP_NT*IPT-1) by bits [lo, lo + nbits), SP_RB bits per pass; kout is
// the second LDS buffer.  Returns the buffer with the result.
//   A pass reads the keys striped (round j, thread t: position j*SP_NT + t,
// so the current order is round-major, then wave, then lane) and ranks each
// key among the equal digits of its wave and round with SP_RB ballots (the
// lanes whose digit bits all agree, counted below the lane).  The lowest
// such lane writes the group's size into the count table at
// (digit, round, wave); an exclusive scan of the table in that order gives
// every (digit, round, wave) its first output position, and each key goes
// to that position plus its rank.  Equal digits keep their current order:
// the sort is stable.  The table (two buffers: one is cleared while the
// other is scanned) pads one entry per digit to spread the LDS banks.
constexpr int SP_RB = 5;                     // radix bits per pass
constexpr int SP_ND = 1 << SP_RB;            // digits
constexpr int SP_NWV = SP_NT / FL_WAVE;      // waves per workgroup
constexpr int SP_SORT_IPT_MAX = 16;
constexpr int SP_SORT_TAB = 2 * SP_ND * (SP_SORT_IPT_MAX * SP_NWV + 1);  // uint16 entries

// This lane's peers among the lanes set in m0: the lanes whose v agrees with
// this lane's in bits [0, NBITS), as two 32-bit halves.  Per bit, sb = 0 or
// -1 (the bit moved to the sign and shifted back) and the peers keep
// ~(ballot ^ sb): five VALU operations per bit.
template <int NBITS>
__device__ __forceinline__ void sp_peers(uint32_t v, unsigned long long m0, uint32_t &mlo, uint32_t &mhi) {
    static_assert(NBITS >= 1 && NBITS <= 32, "peer bits");
    mlo = (uint32_t)m0;
    mhi = (uint32_t)(m0 >> 32);
#pragma unroll
    for (int b = 0; b < NBITS; ++b) {
        const int32_t sb = (int32_t)(v << (31 - b)) >> 31;
        const unsigned long long bal = __builtin_amdgcn_ballot_w64(sb < 0);
        mlo &= ~((uint32_t)bal ^ (uint32_t)sb);
        mhi &= ~((uint32_t)(bal >> 32) ^ (uint32_t)sb);
    }
}

template <int IPT, int NT = SP_NT, bool TWO_TABLES = true>
__device__ uint32_t *sp_block_sort(uint32_t *kin, uint32_t *kout, int lo_bit, int nbits, uint16_t *cnt,
                                   int *scan_lds) {
    constexpr int NWV = NT / FL_WAVE;
    static_assert(IPT % 2 == 0 && IPT * NWV <= SP_SORT_IPT_MAX * SP_NWV, "sort table sized for 64 (round, wave)s");
    constexpr int SPAN = IPT * NWV;                   // entries of one digit
    constexpr int TAB = SP_ND * (SPAN + 1);           // one buffer, padded
    constexpr int PER = SP_ND * SPAN / NT;            // scanned entries per thread
    const int t = threadIdx.x;
    const int w = fl_wave_id();
    uint16_t *tab = cnt, *nxt = TWO_TABLES ? cnt + TAB : cnt;
    for (int q = t; q < TAB; q += NT) tab[q] = 0;
    __syncthreads();
    for (int shift = lo_bit; shift < lo_bit + nbits; shift += SP_RB) {
        if (!TWO_TABLES && shift != lo_bit) {
            // one table: cleared after the previous pass's scatter
            for (int q = t; q < TAB; q += NT) tab[q] = 0;
            __syncthreads();
        }
        uint32_t key[IPT];
        uint16_t dg[IPT], rk[IPT];
#pragma unroll
        for (int j = 0; j < IPT; ++j) {
            key[j] = kin[j * NT + t];
            const uint32_t ks = key[j] >> shift;
            uint32_t mlo, mhi;  // the lanes whose digit equals this lane's
            sp_peers<SP_RB>(ks, ~0ull, mlo, mhi);
            const int d = (int)(ks & (SP_ND - 1));
            const uint32_t below = __builtin_amdgcn_mbcnt_hi(mhi, __builtin_amdgcn_mbcnt_lo(mlo, 0u));
            dg[j] = (uint16_t)d;
            rk[j] = (uint16_t)below;
            if (below == 0) tab[d * (SPAN + 1) + j * NWV + w] = (uint16_t)(__popc(mlo) + __popc(mhi));
        }
        __syncthreads();
        // exclusive scan in (digit, round, wave) order; the other buffer is cleared
        int v[PER];
        int sum = 0;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int f = t * PER + q;
            v[q] = tab[f + f / SPAN];
            sum += v[q];
        }
        int tot;
        int run = fl_block_excl_scan<NT>(sum, scan_lds, &tot);
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int f = t * PER + q;
            tab[f + f / SPAN] = (uint16_t)run;
            run += v[q];
        }
        if (TWO_TABLES)
            for (int q = t; q < TAB; q += NT) nxt[q] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < IPT; ++j) kout[tab[dg[j] * (SPAN + 1) + j * NWV + w] + rk[j]] = key[j];
        __syncthreads();
        uint32_t *x = kin; kin = kout; kout = x;
        uint16_t *y = tab; tab = nxt; nxt = y;
    }
    return kin;
}

// Workgroup per tile: stable scatter of the tile's items into the row's
// destination buckets (bases from the scanned histogram).  With part_inv
// (a backward), every item's partition position is recorded at its raw
// position (written within the tile's range, not scattered over the row).
// the partition's workgroup: one 4096-item tile over 512 threads (8 items
// each: twice the waves per CU of 256 threads at the same LDS)
// The inverse map of a row (raw index -> partition position) is encoded as
// bucket << pos_bits | position within the row's partitioned items when the
// row has fewer than 2^pos_bits items (pos_bits = 31 - the bucket bits, so
// the value stays nonnegative; holes are -1) and the row's buckets fit the
// partition's LDS table; else it holds the global partition position.  Both
// the partition and the output map decide it per row from the same sizes.
__device__ __forceinline__ bool sp_inv_encoded(const SpRows &rows, int64_t r, int pos_bits) {
    return pos_bits > 0 && rows.NB <= SP_TILE / 2 &&
           rows.row_item0[r + 1] - rows.row_item0[r] < ((int64_t)1 << pos_bits);
}

constexpr int SP_PT_NT = 512;
constexpr int SP_PT_IPT = SP_TILE / SP_PT_NT;

__global__ __launch_bounds__(SP_PT_NT) void k_sp_partition(int64_t R, SpRows rows, int nbits, int pos_bits,
                                                       const int64_t *__restrict__ base,
                                                       const int32_t *__restrict__ colpre,
                                                       const int32_t *__restrict__ raw_dst,
                                                       const float *__restrict__ raw_val,
                                                       int32_t *__restrict__ part_dst, float *__restrict__ part_val,
                                                       int32_t *__restrict__ part_inv,
                                                       const uint32_t *__restrict__ raw_tie,
                                                       uint32_t *__restrict__ part_tie) {
    __shared__ __align__(16) uint32_t kb[2][SP_TILE];
    __shared__ uint16_t cnt[SP_SORT_TAB / 2];  // one count table: four workgroups per CU
    __shared__ int scan_lds[SP_PT_NT / FL_WAVE + 1];
    const int64_t tile = fl_xcd_contig(blockIdx.x, gridDim.x);
    const int64_t r = sp_tile_row(rows.tile_base, R, tile);
    const int64_t tl = tile - rows.tile_base[r];
    const int64_t i0 = rows.row_item0[r] + tl * SP_TILE;
    const int64_t i1e = rows.row_item0[r + 1];
    const int c = (int)((i1e - i0) < SP_TILE ? (i1e - i0) : SP_TILE);
    const int t = threadIdx.x;
    // a tile holds at least one item (a row has ceil(items / SP_TILE) tiles),
    // so every destination is requested at once at an index clamped to c - 1
    int32_t dk[SP_PT_IPT];
#pragma unroll
    for (int j = 0; j < SP_PT_IPT; ++j) {
        const int idx = j * SP_PT_NT + t;
        dk[j] = fl_ld32(raw_dst + i0, (uint32_t)(idx < c ? idx : c - 1));
    }
#pragma unroll
    for (int j = 0; j < SP_PT_IPT; ++j) {
        const int idx = j * SP_PT_NT + t;
        uint32_t key = 0xFFFFF000u | (uint32_t)idx;  // padding and holes sort last
        if (idx < c && dk[j] >= 0) key = ((uint32_t)(dk[j] >> SP_S) << 12) | (uint32_t)idx;
        kb[0][idx] = key;
    }
    __syncthreads();
    const uint32_t *sorted = sp_block_sort<SP_PT_IPT, SP_PT_NT, false>(kb[0], kb[1], 12, nbits, cnt, scan_lds);
    // bucket bk's first position in this tile: the bucket's first position
    // in the row plus the row's earlier tiles' items of the bucket
    const int64_t *bb = base + r * rows.NB;
    const int32_t *cp = colpre + tile * rows.NB;
    // per bucket present: its output base minus its first sorted position
    // (one base load per bucket and tile), in the sort's idle buffer when the
    // buckets fit (else a binary search per item)
    int64_t *boff = reinterpret_cast<int64_t *>(sorted == kb[0] ? kb[1] : kb[0]);
    const bool table = rows.NB <= SP_TILE / 2;
    if (table) {
        // every bucket start of the thread's slots found first, then all
        // their base loads issued together (index 0 where no bucket starts;
        // the positions from c on hold hole or padding keys: the at most c
        // items with a bucket sort first)
        uint32_t key[SP_PT_IPT];
        bool first[SP_PT_IPT];
#pragma unroll
        for (int j = 0; j < SP_PT_IPT; ++j) {
            const int p = j * SP_PT_NT + t;
            key[j] = sorted[p];
            const uint32_t bk = key[j] >> 12;
            first[j] = bk != 0xFFFFFu && (p == 0 || (sorted[p - 1] >> 12) != bk);
        }
        int64_t b0[SP_PT_IPT];
        int32_t c0[SP_PT_IPT];
#pragma unroll
        for (int j = 0; j < SP_PT_IPT; ++j) {
            const uint32_t bq = first[j] ? key[j] >> 12 : 0u;
            b0[j] = bb[bq];
            c0[j] = fl_ld32(cp, bq);
        }
#pragma unroll
        for (int j = 0; j < SP_PT_IPT; ++j)
            if (first[j]) boff[key[j] >> 12] = b0[j] + c0[j] - (j * SP_PT_NT + t);
        __syncthreads();
        // every item's destination and value requested before the stores
        // (raw index 0 for holes and padding)
        int32_t dv[SP_PT_IPT];
        float vv[SP_PT_IPT];
#pragma unroll
        for (int j = 0; j < SP_PT_IPT; ++j) {
            const bool ok = j * SP_PT_NT + t < c && (key[j] >> 12) != 0xFFFFFu;
            const uint32_t idx = ok ? key[j] & 4095u : 0u;
            dv[j] = fl_ld32(raw_dst + i0, idx);
            vv[j] = fl_ld32(raw_val + i0, idx);
        }
        if (!part_inv) {
#pragma unroll
            for (int j = 0; j < SP_PT_IPT; ++j) {
                const int p = j * SP_PT_NT + t;  // striped: consecutive threads write consecutive slots
                const uint32_t bk = key[j] >> 12;
                if (p >= c || bk == 0xFFFFFu) continue;
                const int64_t q = boff[bk] + p;
                part_dst[q] = dv[j];
                part_val[q] = vv[j];
                if (part_tie) part_tie[q] = fl_ld32(raw_tie + i0, key[j] & 4095u);
            }
            return;
        }
        // the key buffer (every read of it precedes the barrier above) takes
        // the inverse map (raw index -> partition position), stored to
        // part_inv coalesced instead of one scattered store per item
        int32_t *inv_lds = reinterpret_cast<int32_t *>(const_cast<uint32_t *>(sorted));
        // rows of fewer than 2^pos_bits items store bucket << pos_bits | the
        // position within the row's partitioned items, so that the output
        // map needs no destination (sp_inv_encoded)
        const bool enc = sp_inv_encoded(rows, r, pos_bits);
        const int64_t rowpos0 = bb[0];
#pragma unroll
        for (int j = 0; j < SP_PT_IPT; ++j) {
            const int p = j * SP_PT_NT + t;
            if (p >= c) continue;
            const uint32_t bk = key[j] >> 12;
            const uint32_t idx = key[j] & 4095u;
            if (bk == 0xFFFFFu) {  // hole: no partition position
                inv_lds[idx] = -1;
                continue;
            }
            const int64_t q = boff[bk] + p;
            part_dst[q] = dv[j];
            part_val[q] = vv[j];
            inv_lds[idx] = enc ? (int32_t)((bk << pos_bits) | (uint32_t)(q - rowpos0)) : (int32_t)q;
            if (part_tie) part_tie[q] = fl_ld32(raw_tie + i0, idx);
        }
        __syncthreads();
        for (uint32_t idx = (uint32_t)t; idx < (uint32_t)c; idx += SP_PT_NT) fl_st32(part_inv + i0, idx, inv_lds[idx]);
        return;
    }
    // buckets beyond the table: each item's bucket start by binary search
#pragma unroll 4
    for (int j = 0; j < SP_PT_IPT; ++j) {
        const int p = j * SP_PT_NT + t;  // striped: consecutive threads write consecutive slots
        if (p >= c) continue;
        const uint32_t key = sorted[p];
        const uint32_t bk = key >> 12;
        if (bk == 0xFFFFFu) continue;  // hole
        int lo = 0, hi = p;
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if ((sorted[mid] >> 12) < bk) lo = mid + 1;
            else hi = mid;
        }
        const int64_t q = bb[bk] + cp[bk] + (p - lo);
        const uint32_t idx = key & 4095u;
        part_dst[q] = fl_ld32(raw_dst + i0, idx);
        part_val[q] = fl_ld32(raw_val + i0, idx);
        if (part_inv) fl_st32(part_inv + i0, idx, (int32_t)q);
        if (part_tie) part_tie[q] = fl_ld32(raw_tie + i0, idx);
    }
}

// Workgroup per (row, bucket): the bucket's items (raw order) grouped by
// destination with each destination's values added to 0 in raw order; the
// outputs are compacted in destination order into the first slots of the
// bucket's item range, and raw_local[the item's position in the bucket's
// items] = its output index within the bucket (for the backward).  Items are stably sorted by
// destination in LDS (keys destination << 11 | index, LSD radix) and the
// first thread of every run adds the run's values in order.
//   sp_accum_one    buckets of at most SP_CHUNK items, one sort (the
//                   workgroup path of k_sp_accum_mid);
//   k_sp_accum_hot  larger buckets: chunks of SP_CHUNK items in raw order,
//                   each sorted and folded into a dense LDS accumulator of
//                   the bucket's 8192 destinations that carries the partial
//                   sums from chunk to chunk.
constexpr int SP_CHUNK_IPT = 8;
constexpr int SP_CHUNK = SP_NT * SP_CHUNK_IPT;
constexpr int SP_HOT_GRID = 1024;  // workgroups of the persistent hot-bucket kernels

__device__ __forceinline__ void sp_bucket_range(const SpRows &rows, const int64_t *base, int64_t r, int64_t bk,
                                                int64_t *start, int64_t *end) {
    if (rows.NB == 1) {
        *start = rows.row_item0[r];
        *end = rows.row_item0[r + 1];
    } else {
        *start = base[r * rows.NB + bk];
        *end = base[r * rows.NB + bk + 1];
    }
}

// Loads items [c0, c0 + SP_NT*IPT) of the bucket (blocked) as sort keys and
// LDS values, sorts them, and returns the sorted keys.
template <int IPT>
__device__ __forceinline__ const uint32_t *sp_load_sort(const int32_t *__restrict__ dst_arr,
                                                        const float *__restrict__ val_arr, int64_t start, int64_t c0,
                                                        int64_t n, uint32_t (*kb)[SP_CHUNK], float *val,
                                                        uint16_t *cnt, int *scan_lds) {
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
        const int k = t * IPT + j;
        uint32_t dl = SP_W;  // no item / hole: sorts last
        if (c0 + k < n) {
            const int32_t d = dst_arr[start + c0 + k];
            if (d >= 0) {
                dl = (uint32_t)d & (SP_W - 1);
                val[k] = val_arr[start + c0 + k];
            }
        }
        kb[0][k] = (dl << 11) | (uint32_t)k;
    }
    __syncthreads();
    return sp_block_sort<IPT>(kb[0], kb[1], 11, 14, cnt, scan_lds);
}

// The chunk's items [c0, c0 + SP_NT*IPT) of a bucket in registers (blocked:
// thread t holds items t*IPT ..), destination -2 past the end; and those
// registers turned into sort keys and LDS values as sp_load_sort does.
template <int IPT>
__device__ __forceinline__ void sp_chunk_regs(const int32_t *__restrict__ dst_arr, const float *__restrict__ val_arr,
                                              int64_t start, int64_t c0, int64_t n, int32_t *pd, float *pv) {
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
        const int64_t k = c0 + t * IPT + j;
        pd[j] = -2;
        pv[j] = 0.0f;
        if (k < n) {
            pd[j] = dst_arr[start + k];
            pv[j] = val_arr[start + k];
        }
    }
}

template <int IPT>
__device__ __forceinline__ void sp_regs_to_lds(const int32_t *pd, const float *pv, uint32_t (*kb)[SP_CHUNK],
                                               float *val) {
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
        const int k = t * IPT + j;
        uint32_t dl = SP_W;  // no item / hole: sorts last
        if (pd[j] >= 0) {
            dl = (uint32_t)pd[j] & (SP_W - 1);
            val[k] = pv[j];
        }
        kb[0][k] = (dl << 11) | (uint32_t)k;
    }
}

// Values in sorted order: sv[p] = val[index of key p], for this thread's
// blocked positions (sv is the sort's idle ping-pong buffer).
template <int IPT>
__device__ __forceinline__ float *sp_sorted_values(const uint32_t *key, uint32_t (*kb)[SP_CHUNK], const float *val) {
    float *sv = reinterpret_cast<float *>(key == kb[0] ? kb[1] : kb[0]);
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
        const int p = t * IPT + j;
        sv[p] = val[key[p] & 2047u];
    }
    __syncthreads();
    return sv;
}

// a + sv[p] + sv[p+1] + ... + sv[e-1], left to right.  Long runs (hub
// destinations) are a sequential chain of adds: their values are read 32 at
// a time with 16-byte LDS loads (sv is 16-byte aligned) so the chain waits
// on one LDS round trip per 32 adds.
__device__ __forceinline__ float sp_fold(float a, const float *sv, int p, int e) {
    int q = p;
    while (q < e && (q & 3)) a = fl_add(a, sv[q++]);
    const float4 *v4 = reinterpret_cast<const float4 *>(sv);
    for (; q + 32 <= e; q += 32) {
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
    for (; q + 4 <= e; q += 4) {
        const float4 x = v4[q >> 2];
        a = fl_add(a, x.x);
        a = fl_add(a, x.y);
        a = fl_add(a, x.z);
        a = fl_add(a, x.w);
    }
    for (; q < e; ++q) a = fl_add(a, sv[q]);
    return a;
}

__device__ __forceinline__ bool sp_is_head(const uint32_t *key, int p) {
    const uint32_t d = key[p] >> 11;
    return d < SP_W && (p == 0 || (key[p - 1] >> 11) != d);
}

__device__ __forceinline__ int sp_run_end(const uint32_t *key, int p, int size) {
    // the run holds positions [p, lo); probes at p + 1, 2, 4, .. find a key
    // above the run (or the end), then a binary search between
    const uint32_t d = key[p] >> 11;
    int lo = p + 1, hi, step = 1;
    for (;;) {
        hi = p + step;
        if (hi >= size) { hi = size; break; }
        if ((key[hi] >> 11) > d) break;
        lo = hi + 1;
        step <<= 1;
    }
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if ((key[mid] >> 11) <= d) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

// raw_local of the items at sorted positions [p0, p0 + IPT): the output rank
// of each one's run.  rank0 = the runs that start before p0, so a position
// before this thread's first head belongs to run rank0 - 1.
template <int IPT>
__device__ __forceinline__ void sp_raw_ranks(const uint32_t *key, int p0, int rank0, int64_t start,
                                             int32_t *__restrict__ raw_local) {
    int r = rank0 - 1;
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
        const int p = p0 + j;
        const uint32_t k = key[p];
        if ((k >> 11) >= SP_W) continue;  // hole or padding (sorted last)
        if (sp_is_head(key, p)) ++r;
        const int idx = (int)(k & 2047u);
        raw_local[start + idx] = r;
    }
}

template <int IPT>
__device__ __forceinline__ void sp_accum_one(int64_t start, int64_t n, int32_t dbase, int32_t *__restrict__ dst_arr,
                             float *__restrict__ val_arr, int32_t *__restrict__ raw_local, int32_t *out_count, uint32_t (*kb)[SP_CHUNK],
                             float *val, uint16_t *cnt, int *scan_lds) {
    constexpr int SIZE = SP_NT * IPT;
    const int t = threadIdx.x;
    const uint32_t *key = sp_load_sort<IPT>(dst_arr, val_arr, start, 0, n, kb, val, cnt, scan_lds);
    const float *sv = sp_sorted_values<IPT>(key, kb, val);
    int heads = 0;
#pragma unroll
    for (int j = 0; j < IPT; ++j) heads += sp_is_head(key, t * IPT + j) ? 1 : 0;
    int total;
    int rank = fl_block_excl_scan<SP_NT>(heads, scan_lds, &total);
    if (raw_local) sp_raw_ranks<IPT>(key, t * IPT, rank, start, raw_local);
    // all items were read before the first barrier: outputs may overwrite them
    for (int j = 0; j < IPT; ++j) {
        const int p = t * IPT + j;
        if (!sp_is_head(key, p)) continue;
        const int e = sp_run_end(key, p, SIZE);
        const float a = sp_fold(0.0f, sv, p, e);
        dst_arr[start + rank] = dbase + (int32_t)(key[p] >> 11);
        val_arr[start + rank] = a;
        ++rank;
    }
    if (t == 0) *out_count = total;
}

// ---- Small buckets (at most SP_WB items): one wave per bucket with
// wave-private LDS and no block barriers; four buckets per workgroup.  A
// small bucket of more than SP_WFEW destinations goes to the workgroup sort
// of k_sp_accum_mid.
constexpr int SP_WIPT = 8;
constexpr int SP_WB = FL_WAVE * SP_WIPT;  // 512 items
constexpr int SP_SMALL_WAVES = SP_NT / FL_WAVE;
constexpr int SP_MID_GRID = 2048;  // workgroups of the persistent mid-size kernel

// A bucket of at most 64 * IPT items with at most SP_WFEW distinct
// destinations, by one wave without a sort: the destinations are marked in
// a bitmap, destination j (in destination order) is slot j and the bucket's
// output j; each item's slot is ranked among the equal slots of its round
// (64 items in raw order) with SP_WFEW_RB ballots, the values are scattered
// slot-major in raw order within each slot, and lane j adds slot j's run to
// 0 in order.  Holes are skipped.  Returns false, having written nothing,
// when the bucket has more destinations.  LDS: bits (SP_W / 32 words), wpre
// (their prefix counts), tab ((SP_WFEW) x (IPT + 1) counts), dl (slot
// destinations), sv (64 * IPT values, 16-byte aligned).
constexpr int SP_WFEW = 64;
constexpr int SP_WFEW_RB = 6;
template <int IPT>
__device__ __forceinline__ bool sp_wave_few(int64_t start, int64_t n, int32_t dbase, int32_t *__restrict__ dst_arr,
                                            float *__restrict__ val_arr, int32_t *__restrict__ raw_local,
                                            int32_t *out_count, uint32_t *bits, uint16_t *wpre, uint16_t *tab,
                                            int16_t *dl_of, float *sv) {
    constexpr int WPL = SP_W / 32 / FL_WAVE;  // bitmap words per lane
    const int lane = fl_lane();
    int32_t d[IPT];
    float v[IPT];
#pragma unroll
    for (int j = 0; j < IPT; ++j) {  // striped: round j, lane t holds item j*64 + t
        const int64_t k = (int64_t)j * FL_WAVE + lane;
        d[j] = k < n ? dst_arr[start + k] : -1;
        v[j] = k < n ? val_arr[start + k] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < WPL; ++q) bits[lane * WPL + q] = 0;
    fl_wave_sync();
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
        if (d[j] < 0) continue;
        const int x = d[j] & (SP_W - 1);
        const uint32_t b = 1u << (x & 31);
        if (!(bits[x >> 5] & b)) atomicOr(&bits[x >> 5], b);
    }
    fl_wave_sync();
    uint32_t wd[WPL];
    int c = 0;
#pragma unroll
    for (int q = 0; q < WPL; ++q) {
        wd[q] = bits[lane * WPL + q];
        c += __popc(wd[q]);
    }
    const int incl = fl_wave_incl_scan_i32(c);
    const int total = __builtin_amdgcn_readlane(incl, FL_WAVE - 1);
    if (total > SP_WFEW) return false;
    int pre = incl - c;
#pragma unroll
    for (int q = 0; q < WPL; ++q) {
        wpre[lane * WPL + q] = (uint16_t)pre;
        uint32_t m = wd[q];
        for (int o = pre; m; ++o) {
            dl_of[o] = (int16_t)((lane * WPL + q) * 32 + __ffs(m) - 1);
            m &= m - 1;
        }
        pre += __popc(wd[q]);
    }
#pragma unroll
    for (int j = 0; j < IPT; ++j) tab[lane * (IPT + 1) + j] = 0;
    fl_wave_sync();
    uint8_t sl[IPT], rk[IPT];
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
        const bool valid = d[j] >= 0;
        int sj = 0;
        if (valid) {
            const int x = d[j] & (SP_W - 1);
            sj = wpre[x >> 5] + __popc(bits[x >> 5] & ((1u << (x & 31)) - 1u));
        }
        uint32_t mlo, mhi;
        sp_peers<SP_WFEW_RB>((uint32_t)sj, __builtin_amdgcn_ballot_w64(valid), mlo, mhi);
        const uint32_t below = __builtin_amdgcn_mbcnt_hi(mhi, __builtin_amdgcn_mbcnt_lo(mlo, 0u));
        if (valid && below == 0) tab[sj * (IPT + 1) + j] = (uint16_t)(__popc(mlo) + __popc(mhi));
        if (valid && raw_local) raw_local[start + (int64_t)j * FL_WAVE + lane] = sj;
        sl[j] = (uint8_t)sj;
        rk[j] = (uint8_t)below;
    }
    fl_wave_sync();
    // lane s: slot s's rounds in order; the slots' runs are consecutive
    int cs = 0;
#pragma unroll
    for (int j = 0; j < IPT; ++j) cs += tab[lane * (IPT + 1) + j];
    const int sincl = fl_wave_incl_scan_i32(cs);
    const int lo = sincl - cs;
    {
        int run = lo;
#pragma unroll
        for (int j = 0; j < IPT; ++j) {
            const int x = tab[lane * (IPT + 1) + j];
            tab[lane * (IPT + 1) + j] = (uint16_t)run;
            run += x;
        }
    }
    fl_wave_sync();
#pragma unroll
    for (int j = 0; j < IPT; ++j)
        if (d[j] >= 0) sv[tab[sl[j] * (IPT + 1) + j] + rk[j]] = v[j];
    fl_wave_sync();
    // every item was read before: outputs may overwrite them
    if (lane < total) {
        const float a = sp_fold(0.0f, sv, lo, lo + cs);
        dst_arr[start + lane] = dbase + dl_of[lane];
        val_arr[start + lane] = a;
    }
    if (lane == 0) *out_count = total;
    return true;
}

// One wave per (row, bucket) slot: small buckets are accumulated here,
// larger ones listed for the persistent kernels (lists[0] hot, lists[2]
// mid-size; lists[1], lists[3] their claim counters).
__global__ __launch_bounds__(SP_NT) void k_sp_accum_small(SpRows rows, const int64_t *__restrict__ base,
                                                         int32_t *__restrict__ dst_arr, float *__restrict__ val_arr,
                                                         int32_t *__restrict__ raw_local,
                                                         int32_t *__restrict__ out_count, int64_t nslots,
                                                         int32_t *__restrict__ hot_list,
                                                         int32_t *__restrict__ mid_list,
                                                         int32_t *__restrict__ mid_fb,
                                                         int32_t *__restrict__ lists) {
    // per wave: the destination bitmap, its word prefixes, the slots'
    // destinations, the count table and the values in slot order (4.8 KB:
    // eight workgroups per CU)
    constexpr int FB_WORDS = SP_W / 32, FP_WORDS = SP_W / 64, FD_WORDS = SP_WFEW / 2,
                  FT_WORDS = (SP_WFEW * (SP_WIPT + 1) + 1) / 2;
    __shared__ __align__(16) uint32_t fw[SP_SMALL_WAVES][FB_WORDS + FP_WORDS + FD_WORDS + FT_WORDS];
    __shared__ __align__(16) float val[SP_SMALL_WAVES][SP_WB];
    const int w = fl_wave_id();
    const int64_t slot = fl_xcd_contig(blockIdx.x, gridDim.x) * SP_SMALL_WAVES + w;
    if (slot >= nslots) return;  // no block barrier follows
    const int64_t r = slot / rows.NB, bk = slot - r * rows.NB;
    int64_t start, end;
    sp_bucket_range(rows, base, r, bk, &start, &end);
    const int64_t n = end - start;
    const int lane = fl_lane();
    if (n > SP_CHUNK) {
        if (lane == 0) hot_list[atomicAdd(&lists[0], 1)] = (int32_t)slot;
        return;
    }
    if (n > SP_WB) {
        if (lane == 0) mid_list[atomicAdd(&lists[2], 1)] = (int32_t)slot;
        return;
    }
    int32_t *oc = &out_count[slot];
    if (n == 0) {
        if (lane == 0) *oc = 0;
        return;
    }
    const int32_t dbase = (int32_t)(bk << SP_S);
    // buckets of few destinations without a sort; the others go to the
    // workgroup sort of k_sp_accum_mid
    uint32_t *fbits = fw[w];
    uint16_t *fwpre = reinterpret_cast<uint16_t *>(fw[w] + FB_WORDS);
    int16_t *fdl = reinterpret_cast<int16_t *>(fw[w] + FB_WORDS + FP_WORDS);
    uint16_t *ftab = reinterpret_cast<uint16_t *>(fw[w] + FB_WORDS + FP_WORDS + FD_WORDS);
    bool done;
    if (n <= FL_WAVE)
        done = sp_wave_few<1>(start, n, dbase, dst_arr, val_arr, raw_local, oc, fbits, fwpre, ftab, fdl, val[w]);
    else if (n <= 2 * FL_WAVE)
        done = sp_wave_few<2>(start, n, dbase, dst_arr, val_arr, raw_local, oc, fbits, fwpre, ftab, fdl, val[w]);
    else if (n <= 4 * FL_WAVE)
        done = sp_wave_few<4>(start, n, dbase, dst_arr, val_arr, raw_local, oc, fbits, fwpre, ftab, fdl, val[w]);
    else
        done = sp_wave_few<8>(start, n, dbase, dst_arr, val_arr, raw_local, oc, fbits, fwpre, ftab, fdl, val[w]);
    if (!done && lane == 0) mid_fb[atomicAdd(&lists[6], 1)] = (int32_t)slot;
}

// Persistent grid over a list of buckets of at most SP_CHUNK items and more
// destinations than the few-destination paths take; ctr[0] = listed
// buckets, ctr[1] = next one to claim.
__global__ __launch_bounds__(SP_NT) void k_sp_accum_mid(SpRows rows, const int64_t *__restrict__ base,
                                                       int32_t *__restrict__ dst_arr, float *__restrict__ val_arr,
                                                       int32_t *__restrict__ raw_local,
                                                       int32_t *__restrict__ out_count,
                                                       const int32_t *__restrict__ mid_list,
                                                       int32_t *__restrict__ ctr) {
    __shared__ __align__(16) uint32_t kb[2][SP_CHUNK];
    __shared__ float val[SP_CHUNK];
    __shared__ uint16_t cnt[SP_SORT_TAB];
    __shared__ int scan_lds[SP_NT / FL_WAVE + 1];
    __shared__ int claim;
    const int nmid = ctr[0];
    if ((int)blockIdx.x >= nmid) return;  // no bucket left for this workgroup (see k_sp_accum_few)
    for (;;) {
        __syncthreads();  // the previous bucket is done with the LDS arrays
        if (threadIdx.x == 0) claim = atomicAdd(&ctr[1], 1);
        __syncthreads();
        const int mi = __builtin_amdgcn_readfirstlane(claim);  // uniform: scalar registers
        if (mi >= nmid) break;
        const int64_t slot = mid_list[mi];
        const int64_t r = slot / rows.NB, bk = slot - r * rows.NB;
        int64_t start, end;
        sp_bucket_range(rows, base, r, bk, &start, &end);
        const int64_t n = end - start;
        const int32_t dbase = (int32_t)(bk << SP_S);
        int32_t *oc = &out_count[slot];
        if (n <= SP_NT * 4)
            sp_accum_one<4>(start, n, dbase, dst_arr, val_arr, raw_local, oc, kb, val, cnt, scan_lds);
        else
            sp_accum_one<8>(start, n, dbase, dst_arr, val_arr, raw_local, oc, kb, val, cnt, scan_lds);
    }
}

// ---- Buckets with few distinct destinations (at most SP_FEW): mid-size and
// hot buckets are taken here first (persistent grid, hot list then mid
// list).  One pass over the bucket marks its destinations; with more than
// SP_FEW the bucket goes to a fallback list (k_sp_accum_mid / k_sp_accum_hot).
// Otherwise destination j (in destination order) is slot j, the bucket's
// output j, and thread j owns its sum in a register.  Chunks of SP_FEW_CHUNK
// items in raw order: each item's slot is ranked among the equal slots of its
// wave and round with ballots (as sp_block_sort does, one 6-bit pass), the
// values are scattered slot-major into LDS in raw order within each slot, and
// thread j adds its slot's run to its sum, in order.  raw_local (partition
// order) gets each item's slot, written in place.  Holes (destination -1:
// with one bucket per row the bucket is the row's raw items) are skipped.
constexpr int SP_FEW = 64;
constexpr int SP_FEW_RB = 6;
constexpr int SP_FEW_CHUNK = 1024;  // items per ranked chunk
constexpr int SP_FEW_IPT = SP_FEW_CHUNK / SP_NT;
constexpr int SP_FEW_SPAN = SP_FEW_IPT * SP_NWV;           // (round, wave) entries of one slot
constexpr int SP_FEW_TAB = SP_FEW * (SP_FEW_SPAN + 1);     // one count table, padded per slot
constexpr int SP_FEW_PER = SP_FEW * SP_FEW_SPAN / SP_NT;   // scanned entries per thread
static_assert(SP_FEW == (1 << SP_FEW_RB) && SP_FEW <= SP_NT, "one slot per thread");

__device__ __forceinline__ void sp_few_one(int64_t start, int64_t n, int32_t dbase, int32_t *__restrict__ dst_arr,
                                           float *__restrict__ val_arr, int32_t *__restrict__ raw_local,
                                           int32_t *out_count, int total, const uint32_t *bits, const int *wpre,
                                           const int32_t *slot_dl, uint16_t (*tab)[SP_FEW_TAB], float *sv,
                                           int *scan_lds) {
    const int t = threadIdx.x;
    const int w = fl_wave_id();
    for (int q = t; q < SP_FEW_TAB; q += SP_NT) tab[0][q] = 0;
    float acc = 0.0f;  // thread t < total: the sum of slot t
    // the bucket's items from wave-uniform bases, 32-bit offsets (a bucket
    // holds fewer than 2^31 items)
    const int32_t *__restrict__ bd = dst_arr + start;
    const float *__restrict__ bv = val_arr + start;
    const uint32_t un = (uint32_t)n;
    int32_t pd[SP_FEW_IPT];
    float pv[SP_FEW_IPT];
#pragma unroll
    for (int j = 0; j < SP_FEW_IPT; ++j) {  // striped: round j, thread t holds item j*SP_NT + t
        const uint32_t k = (uint32_t)(j * SP_NT + t);
        pd[j] = k < un ? fl_ld32(bd, k) : 0;
        pv[j] = k < un ? fl_ld32(bv, k) : 0.0f;
    }
    __syncthreads();  // table cleared
    int cur = 0;
    for (uint32_t c0 = 0; c0 < un; c0 += SP_FEW_CHUNK) {
        uint8_t sl[SP_FEW_IPT], rk[SP_FEW_IPT];
        float vv[SP_FEW_IPT];
        uint32_t okm = 0;  // bit j: item j exists and is no hole
#pragma unroll
        for (int j = 0; j < SP_FEW_IPT; ++j) {
            const uint32_t k = c0 + (uint32_t)(j * SP_NT + t);
            const bool valid = k < un && pd[j] >= 0;
            okm |= valid ? 1u << j : 0u;
            int sj = 0;
            if (valid) {
                const int dl = pd[j] & (SP_W - 1);
                sj = wpre[dl >> 5] + __popc(bits[dl >> 5] & ((1u << (dl & 31)) - 1u));
            }
            uint32_t mlo, mhi;
            sp_peers<SP_FEW_RB>((uint32_t)sj, __builtin_amdgcn_ballot_w64(valid), mlo, mhi);
            const uint32_t below = __builtin_amdgcn_mbcnt_hi(mhi, __builtin_amdgcn_mbcnt_lo(mlo, 0u));
            if (valid && below == 0)
                tab[cur][sj * (SP_FEW_SPAN + 1) + j * SP_NWV + w] = (uint16_t)(__popc(mlo) + __popc(mhi));
            if (valid && raw_local) fl_st32(raw_local + start, k, (int32_t)sj);
            sl[j] = (uint8_t)sj;
            rk[j] = (uint8_t)below;
            vv[j] = pv[j];
        }
        // the next chunk's items are requested while this one is scanned and added
        if (c0 + SP_FEW_CHUNK < un) {
#pragma unroll
            for (int j = 0; j < SP_FEW_IPT; ++j) {
                const uint32_t k = c0 + SP_FEW_CHUNK + (uint32_t)(j * SP_NT + t);
                pd[j] = k < un ? fl_ld32(bd, k) : 0;
                pv[j] = k < un ? fl_ld32(bv, k) : 0.0f;
            }
        }
        __syncthreads();  // counts written; every thread is past its previous sum
        // exclusive scan in (slot, round, wave) order; the other table is cleared
        int v[SP_FEW_PER];
        int sum = 0;
#pragma unroll
        for (int q = 0; q < SP_FEW_PER; ++q) {
            const int f = t * SP_FEW_PER + q;
            v[q] = tab[cur][f + f / SP_FEW_SPAN];
            sum += v[q];
        }
        int tot;
        int run = fl_block_excl_scan<SP_NT>(sum, scan_lds, &tot);
#pragma unroll
        for (int q = 0; q < SP_FEW_PER; ++q) {
            const int f = t * SP_FEW_PER + q;
            tab[cur][f + f / SP_FEW_SPAN] = (uint16_t)run;
            run += v[q];
        }
        for (int q = t; q < SP_FEW_TAB; q += SP_NT) tab[cur ^ 1][q] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < SP_FEW_IPT; ++j) {
            if (okm & (1u << j)) sv[tab[cur][sl[j] * (SP_FEW_SPAN + 1) + j * SP_NWV + w] + rk[j]] = vv[j];
        }
        __syncthreads();
        if (t < total) {
            const int lo = tab[cur][t * (SP_FEW_SPAN + 1)];
            const int hi = t + 1 < SP_FEW ? tab[cur][(t + 1) * (SP_FEW_SPAN + 1)] : tot;
            acc = sp_fold(acc, sv, lo, hi);
        }
        cur ^= 1;
    }
    __syncthreads();  // every item was read: outputs may overwrite them
    if (t < total) {
        dst_arr[start + t] = dbase + slot_dl[t];
        val_arr[start + t] = acc;
    }
    if (t == 0) *out_count = total;
}

// lists: hot_list (ctr[0] listed, ctr[1] claim), then mid_list (ctr[2],
// ctr[3]); fallbacks to hot_fb (ctr[4]) and mid_fb (ctr[6]).
__global__ __launch_bounds__(SP_NT) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_sp_accum_few(SpRows rows, const int64_t *__restrict__ base,
                                                       int32_t *__restrict__ dst_arr, float *__restrict__ val_arr,
                                                       int32_t *__restrict__ raw_local,
                                                       int32_t *__restrict__ out_count,
                                                       const int32_t *__restrict__ hot_list,
                                                       const int32_t *__restrict__ mid_list,
                                                       int32_t *__restrict__ hot_fb, int32_t *__restrict__ mid_fb,
                                                       int32_t *__restrict__ ctr) {
    __shared__ uint32_t bits[SP_W / 32];
    __shared__ int wpre[SP_W / 32];
    __shared__ int32_t slot_dl[SP_FEW];
    __shared__ __align__(16) float sv[SP_FEW_CHUNK];
    __shared__ uint16_t tab[2][SP_FEW_TAB];
    __shared__ int scan_lds[SP_NT / FL_WAVE + 1];
    __shared__ int claim;
    static_assert(SP_W / 32 == SP_NT, "one bitmap word per thread");
    const int t = threadIdx.x;
    const int nhot = ctr[0], nmid = ctr[2];
    // workgroups past the listed buckets take none: the others claim every
    // one (a participant stops only after a claim past the lists); the whole
    // workgroup leaves at once, before any barrier
    if ((int)blockIdx.x >= nhot + nmid) return;
    for (;;) {
        __syncthreads();  // the previous bucket is done with the LDS arrays
        if (t == 0) {
            int c = atomicAdd(&ctr[1], 1);
            if (c >= nhot) c = nhot + atomicAdd(&ctr[3], 1);
            claim = c;
        }
        __syncthreads();
        const int ci = __builtin_amdgcn_readfirstlane(claim);  // uniform: scalar registers
        if (ci >= nhot + nmid) break;
        const bool hot = ci < nhot;
        const int64_t slot = hot ? hot_list[ci] : mid_list[ci - nhot];
        const int64_t r = slot / rows.NB, bk = slot - r * rows.NB;
        int64_t start, end;
        sp_bucket_range(rows, base, r, bk, &start, &end);
        const int64_t n = end - start;
        bits[t] = 0;
        __syncthreads();
        // 8 loads in flight per thread, then the marks; a bit already set
        // (the common case: few destinations) is read, not written again
        const int32_t *__restrict__ bd = dst_arr + start;
        for (uint32_t k0 = (uint32_t)t; k0 < (uint32_t)n; k0 += 8 * SP_NT) {
            int32_t dv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t k = k0 + (uint32_t)(u * SP_NT);
                dv[u] = k < (uint32_t)n ? fl_ld32(bd, k) : -1;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (dv[u] < 0) continue;
                const int dl = dv[u] & (SP_W - 1);
                const uint32_t b = 1u << (dl & 31);
                if (!(bits[dl >> 5] & b)) atomicOr(&bits[dl >> 5], b);
            }
        }
        __syncthreads();
        const uint32_t word = bits[t];
        int total;
        const int pre = fl_block_excl_scan<SP_NT>(__popc(word), scan_lds, &total);
        if (total > SP_FEW) {
            if (t == 0) {
                if (hot) hot_fb[atomicAdd(&ctr[4], 1)] = (int32_t)slot;
                else mid_fb[atomicAdd(&ctr[6], 1)] = (int32_t)slot;
            }
            continue;
        }
        wpre[t] = pre;
        uint32_t wd = word;
        for (int q = pre; wd; ++q) {
            const int bit = __ffs(wd) - 1;
            wd &= wd - 1;
            slot_dl[q] = t * 32 + bit;
        }
        __syncthreads();
        sp_few_one(start, n, (int32_t)(bk << SP_S), dst_arr, val_arr, raw_local, &out_count[slot], total, bits, wpre,
                   slot_dl, tab, sv, scan_lds);
    }
}

__device__ __forceinline__ void sp_accum_hot_one(SpRows rows, const int64_t *__restrict__ base, int64_t r, int64_t bk,
                                 int32_t *__restrict__ dst_arr, float *__restrict__ val_arr,
                                 int32_t *__restrict__ raw_local,
                                 int32_t *__restrict__ out_count, uint32_t (*kb)[SP_CHUNK], float *val,
                                 uint16_t *cnt, float *acc, uint32_t *bits, int *wpre, int *scan_lds);

// Persistent grid over a list of hot buckets (hot_count[0] listed,
// hot_count[1] next to claim).
__global__ __launch_bounds__(SP_NT) void k_sp_accum_hot(SpRows rows, const int64_t *__restrict__ base,
                                                       int32_t *__restrict__ dst_arr, float *__restrict__ val_arr,
                                                       int32_t *__restrict__ raw_local,
                                                       int32_t *__restrict__ out_count,
                                                       const int32_t *__restrict__ hot_list,
                                                       int32_t *__restrict__ hot_count) {
    __shared__ __align__(16) uint32_t kb[2][SP_CHUNK];
    __shared__ float val[SP_CHUNK];
    __shared__ uint16_t cnt[SP_SORT_TAB];
    __shared__ float acc[SP_W];
    __shared__ uint32_t bits[SP_W / 32];
    __shared__ int wpre[SP_W / 32];
    __shared__ int scan_lds[SP_NT / FL_WAVE + 1];
    __shared__ int claim;
    const int nhot = hot_count[0];
    if ((int)blockIdx.x >= nhot) return;  // no bucket left for this workgroup (see k_sp_accum_few)
    for (;;) {
        __syncthreads();  // the previous bucket is done with the LDS arrays
        if (threadIdx.x == 0) claim = atomicAdd(&hot_count[1], 1);
        __syncthreads();
        const int hi = __builtin_amdgcn_readfirstlane(claim);  // uniform: scalar registers
        if (hi >= nhot) break;
        const int64_t slot = hot_list[hi];
        sp_accum_hot_one(rows, base, slot / rows.NB, slot % rows.NB, dst_arr, val_arr, raw_local,
                         out_count, kb, val, cnt, acc, bits, wpre, scan_lds);
    }
}

__device__ __forceinline__ void sp_accum_hot_one(SpRows rows, const int64_t *__restrict__ base, int64_t r, int64_t bk,
                                 int32_t *__restrict__ dst_arr, float *__restrict__ val_arr,
                                 int32_t *__restrict__ raw_local,
                                 int32_t *__restrict__ out_count, uint32_t (*kb)[SP_CHUNK], float *val,
                                 uint16_t *cnt, float *acc, uint32_t *bits, int *wpre, int *scan_lds) {
    int64_t start, end;
    sp_bucket_range(rows, base, r, bk, &start, &end);
    const int64_t n = end - start;
    const int t = threadIdx.x;
    for (int q = t; q < SP_W / 32; q += SP_NT) bits[q] = 0;
    // the next chunk's items are requested while this chunk is sorted and folded
    int32_t pd[SP_CHUNK_IPT];
    float pv[SP_CHUNK_IPT];
    sp_chunk_regs<SP_CHUNK_IPT>(dst_arr, val_arr, start, 0, n, pd, pv);
    for (int64_t c0 = 0; c0 < n; c0 += SP_CHUNK) {
        __syncthreads();  // previous chunk's folds done with kb / val
        sp_regs_to_lds<SP_CHUNK_IPT>(pd, pv, kb, val);
        if (c0 + SP_CHUNK < n) sp_chunk_regs<SP_CHUNK_IPT>(dst_arr, val_arr, start, c0 + SP_CHUNK, n, pd, pv);
        __syncthreads();
        const uint32_t *key = sp_block_sort<SP_CHUNK_IPT>(kb[0], kb[1], 11, 14, cnt, scan_lds);
        const float *sv = sp_sorted_values<SP_CHUNK_IPT>(key, kb, val);
        for (int j = 0; j < SP_CHUNK_IPT; ++j) {
            const int p = t * SP_CHUNK_IPT + j;
            if (!sp_is_head(key, p)) continue;
            const int e = sp_run_end(key, p, SP_CHUNK);
            const uint32_t d = key[p] >> 11;
            const uint32_t m = 1u << (d & 31);
            const uint32_t old = atomicOr(&bits[d >> 5], m);
            acc[d] = sp_fold((old & m) ? acc[d] : 0.0f, sv, p, e);
        }
    }
    __syncthreads();
    const uint32_t word = bits[t];
    int total;
    const int pre = fl_block_excl_scan<SP_NT>(__popc(word), scan_lds, &total);
    wpre[t] = pre;
    __syncthreads();
    if (raw_local) {
#pragma unroll 4
        for (int64_t k = t; k < n; k += SP_NT) {
            const int32_t d = dst_arr[start + k];
            if (d < 0) continue;  // hole
            const int dl = d & (SP_W - 1);
            raw_local[start + k] =
                wpre[dl >> 5] + __popc(bits[dl >> 5] & ((1u << (dl & 31)) - 1u));
        }
        __syncthreads();
    }
    const int32_t dbase = (int32_t)(bk << SP_S);
    uint32_t wd = word;
    int64_t o = start + pre;
    while (wd) {
        const int bit = __ffs(wd) - 1;
        wd &= wd - 1;
        const int dl = t * 32 + bit;
        dst_arr[o] = dbase + dl;
        val_arr[o] = acc[dl];
        ++o;
    }
    if (t == 0) out_count[r * rows.NB + bk] = total;
}

// Max per (row, bucket) (flashlog_kernel.py:399-478): per destination the
// winning item is the largest value (zeros of either sign equal), then the
// smallest tie key (ORI < INV < identity, then the original edge id), then
// the earliest raw item; outputs are compacted in destination order as for
// the sum, with the winning value (+0 for a zero), and raw_local[the item's
// position] = the output index of winners, -1 for the other items.
//   k_sp_max      buckets of at most SP_CHUNK items: stable LDS sort by
//                 destination, the first thread of every run scans it;
//   k_sp_max_hot  larger buckets: dense LDS arrays over the bucket's 8192
//                 destinations, a max of the value keys, then a min of
//                 (tie key, position) among the items holding the max.
__device__ __forceinline__ float sp_canon(float v) { return v == 0.0f ? 0.0f : v; }

__device__ __forceinline__ float fl_order_key_inv(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

template <int IPT>
__device__ __forceinline__ void sp_max_one(int64_t start, int64_t n, int32_t dbase, int32_t *__restrict__ dst_arr,
                           float *__restrict__ val_arr, const uint32_t *__restrict__ tie_arr,
                           int32_t *__restrict__ raw_local, int32_t *out_count,
                           uint32_t (*kb)[SP_CHUNK], float *val, uint32_t *tie, uint16_t *cnt,
                           int *scan_lds) {
    constexpr int SIZE = SP_NT * IPT;
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < IPT; ++j) {
        const int k = t * IPT + j;
        if (k < n) tie[k] = tie_arr[start + k];
    }
    const uint32_t *key = sp_load_sort<IPT>(dst_arr, val_arr, start, 0, n, kb, val, cnt, scan_lds);
    int heads = 0;
#pragma unroll
    for (int j = 0; j < IPT; ++j) heads += sp_is_head(key, t * IPT + j) ? 1 : 0;
    int total;
    int rank = fl_block_excl_scan<SP_NT>(heads, scan_lds, &total);
    // all items were read before the first barrier: outputs may overwrite them
    for (int j = 0; j < IPT; ++j) {
        const int p = t * IPT + j;
        if (!sp_is_head(key, p)) continue;
        const int e = sp_run_end(key, p, SIZE);
        int bi = (int)(key[p] & 2047u);
        float bv = sp_canon(val[bi]);
        uint32_t bt = tie[bi];
        for (int q = p + 1; q < e; ++q) {
            const int idx = (int)(key[q] & 2047u);
            const float v = sp_canon(val[idx]);
            const uint32_t tq = tie[idx];
            if (v > bv || (v == bv && tq < bt)) { bi = idx; bv = v; bt = tq; }
        }
        if (raw_local)
            for (int q = p; q < e; ++q) {
                const int idx = (int)(key[q] & 2047u);
                raw_local[start + idx] = idx == bi ? rank : -1;
            }
        dst_arr[start + rank] = dbase + (int32_t)(key[p] >> 11);
        val_arr[start + rank] = bv;
        ++rank;
    }
    if (t == 0) *out_count = total;
}

__global__ __launch_bounds__(SP_NT) void k_sp_max(SpRows rows, const int64_t *__restrict__ base,
                                                 int32_t *__restrict__ dst_arr, float *__restrict__ val_arr,
                                                 const uint32_t *__restrict__ tie_arr,
                                                 int32_t *__restrict__ raw_local, int32_t *__restrict__ out_count,
                                                 int32_t *__restrict__ hot_list, int32_t *__restrict__ hot_count) {
    __shared__ __align__(16) uint32_t kb[2][SP_CHUNK];
    __shared__ float val[SP_CHUNK];
    __shared__ uint32_t tie[SP_CHUNK];
    __shared__ uint16_t cnt[SP_SORT_TAB];
    __shared__ int scan_lds[SP_NT / FL_WAVE + 1];
    const int64_t r = blockIdx.x / rows.NB, bk = blockIdx.x - (blockIdx.x / rows.NB) * rows.NB;
    int64_t start, end;
    sp_bucket_range(rows, base, r, bk, &start, &end);
    const int64_t n = end - start;
    if (n > SP_CHUNK) {  // for k_sp_max_hot
        if (threadIdx.x == 0) hot_list[atomicAdd(hot_count, 1)] = (int32_t)blockIdx.x;
        return;
    }
    int32_t *oc = &out_count[r * rows.NB + bk];
    if (n == 0) {
        if (threadIdx.x == 0) *oc = 0;
        return;
    }
    const int32_t dbase = (int32_t)(bk << SP_S);
    if (n <= SP_NT * 2)
        sp_max_one<2>(start, n, dbase, dst_arr, val_arr, tie_arr, raw_local, oc, kb, val, tie, cnt, scan_lds);
    else if (n <= SP_NT * 4)
        sp_max_one<4>(start, n, dbase, dst_arr, val_arr, tie_arr, raw_local, oc, kb, val, tie, cnt, scan_lds);
    else
        sp_max_one<8>(start, n, dbase, dst_arr, val_arr, tie_arr, raw_local, oc, kb, val, tie, cnt, scan_lds);
}

__device__ __forceinline__ void sp_max_hot_one(SpRows rows, const int64_t *__restrict__ base, int64_t r, int64_t bk,
                               int32_t *__restrict__ dst_arr, float *__restrict__ val_arr,
                               const uint32_t *__restrict__ tie_arr, int32_t *__restrict__ raw_local, int32_t *__restrict__ out_count, uint32_t *vbest,
                               unsigned long long *tbest, uint32_t *bits, int *wpre, int *scan_lds);

// Persistent grid over the list of hot buckets collected by k_sp_max.
__global__ __launch_bounds__(SP_NT) void k_sp_max_hot(SpRows rows, const int64_t *__restrict__ base,
                                                     int32_t *__restrict__ dst_arr, float *__restrict__ val_arr,
                                                     const uint32_t *__restrict__ tie_arr,
                                                     int32_t *__restrict__ raw_local,
                                                     int32_t *__restrict__ out_count,
                                                     const int32_t *__restrict__ hot_list,
                                                     int32_t *__restrict__ hot_count) {
    __shared__ uint32_t vbest[SP_W];
    __shared__ unsigned long long tbest[SP_W];
    __shared__ uint32_t bits[SP_W / 32];
    __shared__ int wpre[SP_W / 32];
    __shared__ int scan_lds[SP_NT / FL_WAVE + 1];
    __shared__ int claim;
    const int nhot = hot_count[0];
    if ((int)blockIdx.x >= nhot) return;  // no bucket left for this workgroup (see k_sp_accum_few)
    for (;;) {
        __syncthreads();  // the previous bucket is done with the LDS arrays
        if (threadIdx.x == 0) claim = atomicAdd(&hot_count[1], 1);
        __syncthreads();
        const int hi = __builtin_amdgcn_readfirstlane(claim);  // uniform: scalar registers
        if (hi >= nhot) break;
        const int64_t slot = hot_list[hi];
        sp_max_hot_one(rows, base, slot / rows.NB, slot % rows.NB, dst_arr, val_arr, tie_arr, raw_local,
                       out_count, vbest, tbest, bits, wpre, scan_lds);
    }
}

__device__ __forceinline__ void sp_max_hot_one(SpRows rows, const int64_t *__restrict__ base, int64_t r, int64_t bk,
                               int32_t *__restrict__ dst_arr, float *__restrict__ val_arr,
                               const uint32_t *__restrict__ tie_arr, int32_t *__restrict__ raw_local, int32_t *__restrict__ out_count, uint32_t *vbest,
                               unsigned long long *tbest, uint32_t *bits, int *wpre, int *scan_lds) {
    int64_t start, end;
    sp_bucket_range(rows, base, r, bk, &start, &end);
    const int64_t n = end - start;
    const int t = threadIdx.x;
    for (int q = t; q < SP_W; q += SP_NT) {
        vbest[q] = 0u;  // below the key of every non-NaN value
        tbest[q] = ~0ull;
    }
    for (int q = t; q < SP_W / 32; q += SP_NT) bits[q] = 0;
    __syncthreads();
    for (int64_t k = t; k < n; k += SP_NT) {
        const int32_t d = dst_arr[start + k];
        if (d < 0) continue;
        const int dl = d & (SP_W - 1);
        atomicMax(&vbest[dl], fl_order_key(sp_canon(val_arr[start + k])));
        atomicOr(&bits[dl >> 5], 1u << (dl & 31));
    }
    __syncthreads();
    for (int64_t k = t; k < n; k += SP_NT) {
        const int32_t d = dst_arr[start + k];
        if (d < 0) continue;
        const int dl = d & (SP_W - 1);
        if (fl_order_key(sp_canon(val_arr[start + k])) == vbest[dl])
            atomicMin(&tbest[dl], ((unsigned long long)tie_arr[start + k] << 32) | (unsigned long long)k);
    }
    __syncthreads();
    const uint32_t word = bits[t];
    int total;
    const int pre = fl_block_excl_scan<SP_NT>(__popc(word), scan_lds, &total);
    wpre[t] = pre;
    __syncthreads();
    if (raw_local) {
#pragma unroll 4
        for (int64_t k = t; k < n; k += SP_NT) {
            const int32_t d = dst_arr[start + k];
            if (d < 0) continue;
            const int dl = d & (SP_W - 1);
            const int o = wpre[dl >> 5] + __popc(bits[dl >> 5] & ((1u << (dl & 31)) - 1u));
            raw_local[start + k] = (uint32_t)tbest[dl] == (uint32_t)k ? o : -1;
        }
        __syncthreads();
    }
    const int32_t dbase = (int32_t)(bk << SP_S);
    uint32_t wd = word;
    int64_t o = start + pre;
    while (wd) {
        const int bit = __ffs(wd) - 1;
        wd &= wd - 1;
        const int dl = t * 32 + bit;
        dst_arr[o] = dbase + dl;
        val_arr[o] = fl_order_key_inv(vbest[dl]);
        ++o;
    }
    if (t == 0) out_count[r * rows.NB + bk] = total;
}

// Wave per (row, bucket), four per workgroup: staged outputs -> COO at
// out_base.
constexpr int SP_EMIT_WAVES = 4;
constexpr int SP_EMIT_SLOTS = 4 * SP_EMIT_WAVES;  // slots per workgroup of k_sp_emit

__global__ __launch_bounds__(SP_EMIT_WAVES * FL_WAVE) void k_sp_emit(SpRows rows, int64_t L, int64_t nslot,
                                                  const int64_t *__restrict__ base,
                                                  const int32_t *__restrict__ dst_arr,
                                                  const float *__restrict__ val_arr,
                                                  const int64_t *__restrict__ out_base, int64_t *__restrict__ ob,
                                                  int64_t *__restrict__ ol, int64_t *__restrict__ oe,
                                                  float *__restrict__ ov) {
    // a workgroup takes SP_EMIT_SLOTS consecutive slots, its waves every
    // SP_EMIT_WAVES-th of them (most slots of an early hop are empty or small)
    const int64_t g = fl_xcd_contig(blockIdx.x, gridDim.x);
    for (int s_ = 0; s_ < SP_EMIT_SLOTS / SP_EMIT_WAVES; ++s_) {
    const int64_t slot = g * SP_EMIT_SLOTS + (int64_t)s_ * SP_EMIT_WAVES + fl_wave_id();
    if (slot >= nslot) return;
    const int64_t r = slot / rows.NB;
    const int64_t o0 = out_base[slot];
    const int64_t cnt = out_base[slot + 1] - o0;
    if (cnt == 0) continue;
    int64_t start;
    if (rows.NB == 1) {
        start = rows.row_item0[r];
    } else {
        start = base[slot];
    }
    const int64_t b = r / L, l = r - (r / L) * L;
    // a bucket's outputs (at most 8192) from wave-uniform bases, 32-bit offsets
    int64_t *__restrict__ pb = ob + o0;
    int64_t *__restrict__ pl = ol + o0;
    int64_t *__restrict__ pe = oe + o0;
    float *__restrict__ pv = ov + o0;
    const int32_t *__restrict__ sd = dst_arr + start;
    const float *__restrict__ svl = val_arr + start;
    for (uint32_t k = fl_lane(); k < (uint32_t)cnt; k += FL_WAVE) {
        fl_st32(pb, k, b);
        fl_st32(pl, k, l);
        fl_st32(pe, k, (int64_t)fl_ld32(sd, k));
        fl_st32(pv, k, fl_ld32(svl, k));
    }
    }
}

// ---------------------------------------------------------------------------
// backward

// After the accumulation: every raw item's output index, the index within
// its (row, bucket) that the accumulation recorded plus the bucket's output
// base (the losing items of the max stay -1).  With one bucket per row the
// accumulation has compacted its outputs into raw_dst, so the destinations
// are read only with several buckets (then holes of the sum become -1);
// with one, holes keep an unspecified index and the backward skips them by
// their mask.  Workgroup per tile of a row, as k_sp_hist.

constexpr int SP_LTO_NB = 2048;  // buckets per row kept in LDS by k_sp_local_to_out

__global__ __launch_bounds__(SP_NT) void k_sp_local_to_out(int64_t R, SpRows rows, const int32_t *__restrict__ raw_dst,
                                                          const int64_t *__restrict__ out_base,
                                                          const int64_t *__restrict__ base, int pos_bits,
                                                          const int32_t *__restrict__ part_inv,
                                                          const int32_t *__restrict__ part_local,
                                                          int32_t *__restrict__ raw_local) {
    const int64_t tile = fl_xcd_contig(blockIdx.x, gridDim.x);
    const int64_t r = sp_tile_row(rows.tile_base, R, tile);
    const int64_t tl = tile - rows.tile_base[r];
    const int64_t i0 = rows.row_item0[r] + tl * SP_TILE;
    const int64_t i1e = rows.row_item0[r + 1];
    const int c = (int)((i1e - i0) < SP_TILE ? (i1e - i0) : SP_TILE);
    const int64_t *orow = out_base + r * rows.NB;
    // the row's bucket bases in LDS when they fit (one load each per tile)
    // (32-bit: output indices are below the item count, which the expand
    // holds below 2^31 when a map is made)
    __shared__ int32_t obase[SP_LTO_NB];
    const bool lds = rows.NB <= SP_LTO_NB;
    if (lds) {
        for (int64_t q = threadIdx.x; q < rows.NB; q += SP_NT) obase[q] = (int32_t)orow[q];
        __syncthreads();
    }
    // the tile's items from wave-uniform bases, 32-bit offsets
    const int32_t *__restrict__ tdst = raw_dst + i0;
    int32_t *__restrict__ tloc = raw_local + i0;
    const int32_t *__restrict__ tinv = part_inv ? part_inv + i0 : nullptr;
    if (tinv && lds && sp_inv_encoded(rows, r, pos_bits)) {
        // the map carries each item's bucket: no destination is read; every
        // entry of the map first, then every gather, then every store
        constexpr int Q = SP_TILE / SP_NT;
        const int32_t *__restrict__ rloc = part_local + base[r * rows.NB];
        const uint32_t pmask = (1u << pos_bits) - 1u;
        int32_t qq[Q];
#pragma unroll
        for (int j = 0; j < Q; ++j) {
            const uint32_t idx = (uint32_t)(j * SP_NT) + threadIdx.x;
            qq[j] = idx < (uint32_t)c ? fl_ld32(tinv, idx) : -1;
        }
        int32_t ll[Q];
#pragma unroll
        for (int j = 0; j < Q; ++j) ll[j] = qq[j] >= 0 ? fl_ld32(rloc, (uint32_t)qq[j] & pmask) : -1;
#pragma unroll
        for (int j = 0; j < Q; ++j) {
            const uint32_t idx = (uint32_t)(j * SP_NT) + threadIdx.x;
            if (idx < (uint32_t)c)
                fl_st32(tloc, idx, ll[j] >= 0 ? obase[(uint32_t)qq[j] >> pos_bits] + ll[j] : -1);
        }
        return;
    }
    if (tinv && lds && c == SP_TILE) {
        // a full tile: every position and destination first, then every
        // gather, then every store (16 independent chains per thread)
        constexpr int Q = SP_TILE / SP_NT;
        int32_t dd[Q], qq[Q];
#pragma unroll
        for (int j = 0; j < Q; ++j) {
            const uint32_t idx = (uint32_t)(j * SP_NT) + threadIdx.x;
            dd[j] = fl_ld32(tdst, idx);
            qq[j] = fl_ld32(tinv, idx);
        }
#pragma unroll
        for (int j = 0; j < Q; ++j) qq[j] = dd[j] >= 0 ? part_local[qq[j]] : -1;
#pragma unroll
        for (int j = 0; j < Q; ++j) {
            const uint32_t idx = (uint32_t)(j * SP_NT) + threadIdx.x;
            fl_st32(tloc, idx, qq[j] >= 0 ? obase[dd[j] >> SP_S] + qq[j] : -1);
        }
        return;
    }
#pragma unroll 4
    for (uint32_t idx = threadIdx.x; idx < (uint32_t)c; idx += SP_NT) {
        if (tinv) {
            // partitioned: the local index sits at the item's partition position
            // (holes were not partitioned)
            const int32_t d = fl_ld32(tdst, idx);
            int32_t o = -1;
            if (d >= 0) {
                const int32_t loc = part_local[fl_ld32(tinv, idx)];
                if (loc >= 0) o = (int32_t)((lds ? (int64_t)obase[d >> SP_S] : orow[d >> SP_S]) + loc);
            }
            fl_st32(tloc, idx, o);
        } else {
            const int32_t loc = fl_ld32(tloc, idx);
            fl_st32(tloc, idx, loc >= 0 ? (int32_t)(orow[0] + loc) : -1);
        }
    }
}

// Segmented inclusive sum of x over runs of equal key across the wave (runs
// are contiguous), with DPP moves; lanes whose source is outside the wave
// see key -1 + 1 = 0, which matches only the unused key -1 (x = 0 there).
__device__ __forceinline__ float sp_dpp_add_if(float x, int key1, float y, int ky) {
    return ky == key1 ? fl_add(x, y) : x;
}
template <int CTRL, int RM = 0xf>
__device__ __forceinline__ float sp_seg_step(float x, int key1) {
    const float y = __int_as_float(fl_dpp<CTRL, RM>(__float_as_int(x)));
    const int ky = fl_dpp<CTRL, RM>(key1);
    return sp_dpp_add_if(x, key1, y, ky);
}
__device__ __forceinline__ float sp_seg_scan(float x, int key) {
    const int key1 = key + 1;
    x = sp_seg_step<0x111>(x, key1);
    x = sp_seg_step<0x112>(x, key1);
    x = sp_seg_step<0x114>(x, key1);
    x = sp_seg_step<0x118>(x, key1);
    x = sp_seg_step<0x142, 0xa>(x, key1);
    x = sp_seg_step<0x143, 0xc>(x, key1);
    return x;
}

// Backward, wave per entry over the entry's raw items (raw order; the
// forward recorded each one's CSR position, attention column and output
// index): grad_v[i] = sum over items of (g*m)*w, the identity item taken
// with m = 1 (flashlog.cu:1856-1959); grad_w[r, col] = sum of (g*m)*a over
// the row's items of that column (flashlog.cu:1910-1914,1957-1958, where
// atomics add them).  Holes (sum: masked kept edges, m == 0) and, for max,
// the losing items (output index -1) take no part (flashlog.cu:2364-2410).
// The next chunk's records are requested before the current chunk's
// gathers.
//
// grad_w without atomics, in a fixed order.  Within an entry every column
// belongs to one run of consecutive items (one relation group, or the
// identity item).  A workgroup takes BW_CH consecutive entries of one row;
// wave w of it takes entries w, w+4, ... of those and adds, in that order,
// each run's per-chunk segmented sums into a row of n floats of its own
// (LDS, or global memory when n > BW_LDS_MAX_N); the workgroup writes the
// sum ((row0 + row1) + row2) + row3 to its partial row, and k_sp_gw_fin adds
// a row's partial rows in chunk order.
constexpr int BW_CH = 128;
constexpr int BW_WAVES = SEL_NT / FL_WAVE;
constexpr int64_t BW_LDS_MAX_N = 4096;  // columns of the LDS rows (4 * 4 * n bytes)

__device__ __forceinline__ void sp_bwd_entry(fl_side ori, fl_side inv, const int64_t *__restrict__ sb,
                                             const int64_t *__restrict__ sl, const float *__restrict__ sv,
                                             const float *__restrict__ w, int64_t L, int64_t n, int64_t r_size,
                                             int holes, const int64_t *__restrict__ item_off,
                                             const int32_t *__restrict__ raw_out,
                                             const int32_t *__restrict__ raw_pos,
                                             const int16_t *__restrict__ raw_col, const float *__restrict__ grad,
                                             float *__restrict__ grad_v, int64_t i, float *gdst,
                                             uint32_t *__restrict__ ekey, float *__restrict__ eval);

// Thread per row: its number of BW_CH-entry chunks.
__global__ void k_sp_bw_chunks(const int64_t *__restrict__ row_ptr, int64_t R, int64_t *__restrict__ nchunk) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= R) return;
    nchunk[r] = (row_ptr[r + 1] - row_ptr[r] + BW_CH - 1) / BW_CH;
}

template <bool USE_LDS>
__global__ __launch_bounds__(SEL_NT) void k_sp_bwd(fl_side ori, fl_side inv, const int64_t *__restrict__ sb,
                                                  const int64_t *__restrict__ sl, const float *__restrict__ sv,
                                                  const int64_t *__restrict__ row_ptr,
                                                  const int64_t *__restrict__ chunk_ptr, int64_t R,
                                                  const float *__restrict__ w, int64_t L, int64_t n, int64_t r_size,
                                                  int holes, const int64_t *__restrict__ item_off,
                                                  const int32_t *__restrict__ raw_out,
                                                  const int32_t *__restrict__ raw_pos,
                                                  const int16_t *__restrict__ raw_col,
                                                  const float *__restrict__ grad, float *__restrict__ grad_v,
                                                  float *__restrict__ wave_rows, float *__restrict__ part,
                                                  uint32_t *__restrict__ ekey, float *__restrict__ eval) {
    extern __shared__ float bw_rows[];  // [BW_WAVES][n] when USE_LDS
    const int64_t nblk = chunk_ptr[R];
    if ((int64_t)blockIdx.x >= nblk) return;  // the grid is an upper bound of the chunk count
    // chunks in contiguous ranges per XCD: the gradient rows a range reads
    // stay in that XCD's L2
    const int64_t blk = fl_xcd_contig(blockIdx.x, nblk);
    // the block's row: chunk_ptr[r] <= blk < chunk_ptr[r + 1]
    int64_t lo = 0, hi = R;
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (chunk_ptr[mid] <= blk) lo = mid; else hi = mid;
    }
    const int64_t r = lo;
    const int64_t e0 = row_ptr[r] + (blk - chunk_ptr[r]) * BW_CH;
    const int64_t e1 = e0 + BW_CH < row_ptr[r + 1] ? e0 + BW_CH : row_ptr[r + 1];
    const int wid = fl_wave_id();
    float *rows = USE_LDS ? bw_rows : wave_rows + blk * BW_WAVES * n;
    for (int64_t q = threadIdx.x; q < BW_WAVES * n; q += SEL_NT) rows[q] = 0.0f;
    __syncthreads();
    for (int64_t i = e0 + wid; i < e1; i += BW_WAVES)
        sp_bwd_entry(ori, inv, sb, sl, sv, w, L, n, r_size, holes, item_off, raw_out, raw_pos, raw_col, grad, grad_v,
                     i, rows + wid * n, ekey, eval);
    __syncthreads();
    for (int64_t c = threadIdx.x; c < n; c += SEL_NT) {
        float x = rows[c];
#pragma unroll
        for (int k = 1; k < BW_WAVES; ++k) x = fl_add(x, rows[k * n + c]);
        part[blk * n + c] = x;
    }
}

// Edge-weight gradients: the items' terms sorted stably by key (side offset +
// CSR position), so each position's terms form a run in raw item order.  A
// thread per run head of one side folds its run from 0 and adds the sum to
// the position's edge: the ORI side's launch first, then the INV side's (an
// edge id has one position per side, so within a launch every edge has one
// writer).  grad_edge[e] = (g + ORI fold) + INV fold, the same bits each run.
constexpr uint32_t SP_EDGE_NONE = 0xFFFFFFFFu;

__global__ void k_sp_edge_fold(const uint32_t *__restrict__ key, const float *__restrict__ val, int64_t items,
                               uint32_t lo, uint32_t hi, const int32_t *__restrict__ order,
                               float *__restrict__ grad_edge) {
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= items) return;
    const uint32_t k = key[j];
    if (k < lo || k >= hi || (j > 0 && key[j - 1] == k)) return;
    float x = 0.0f;
    for (int64_t q = j; q < items && key[q] == k; ++q) x = fl_add(x, val[q]);
    float *dst = grad_edge + order[k - lo];
    *dst = fl_add(*dst, x);
}

// grad_w[r, c] = the row's partial rows added in chunk order.
__global__ void k_sp_gw_fin(const int64_t *__restrict__ chunk_ptr, const float *__restrict__ part, int64_t n,
                            float *__restrict__ grad_w) {
    const int64_t r = blockIdx.y;
    const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= n) return;
    float x = 0.0f;
    for (int64_t b = chunk_ptr[r]; b < chunk_ptr[r + 1]; ++b) x = fl_add(x, part[b * n + c]);
    grad_w[r * n + c] = x;
}

__device__ __forceinline__ void sp_bwd_entry(fl_side ori, fl_side inv, const int64_t *__restrict__ sb,
                                             const int64_t *__restrict__ sl, const float *__restrict__ sv,
                                             const float *__restrict__ w, int64_t L, int64_t n, int64_t r_size,
                                             int holes, const int64_t *__restrict__ item_off,
                                             const int32_t *__restrict__ raw_out,
                                             const int32_t *__restrict__ raw_pos,
                                             const int16_t *__restrict__ raw_col, const float *__restrict__ grad,
                                             float *__restrict__ grad_v, int64_t i, float *gdst,
                                             uint32_t *__restrict__ ekey, float *__restrict__ eval) {
    const int lane = fl_lane();
    const int64_t r = sb[i] * L + sl[i];
    const float a = sv[i];
    const float *wrow = w + r * n;
    const int64_t k0 = item_off[i], k1 = item_off[i + 1];
    const bool edge_grads = ori.grad_edge || inv.grad_edge;
    float gsp = 0.0f;
    // without positions every kept item has mask 1 (the holes, the masked
    // items, carry output index -1) and there are no edge factors.
    //   The next round's records are requested before this round's gathers;
    // the two rounds' registers alternate between two sets (the loop body
    // holds two rounds) and every load is issued, past the entry's end at
    // its last item, so that a round waits only for the loads issued a round
    // earlier (lanes past the end take no part: -1 where the round uses them)
    struct Rec {
        int32_t p, loc;
        int col;
    };
    // has_pos: raw_pos given (a compile-time branch, so that no load is
    // conditional inside the loop)
    auto load = [&](Rec &x, int64_t kb, auto has_pos) {
        const int64_t k = kb + lane;
        const int64_t kc = k < k1 ? k : k1 - 1;
        if constexpr (decltype(has_pos)::value) x.p = raw_pos[kc];
        else x.p = -1;
        x.col = raw_col[kc];
        x.loc = raw_out[kc];
    };
    auto do_round = [&](const Rec &cur, Rec &nxt, int64_t kb, auto has_pos) {
        load(nxt, kb + FL_WAVE, has_pos);
        __builtin_amdgcn_sched_barrier(0);  // the next round's loads issued first
        const bool in = kb + lane < k1;
        const int32_t p = in ? cur.p : -1, loc = in ? cur.loc : -1;
        const int col = in ? cur.col : -1;
        float gwv = 0.0f;
        const bool iv = p >= 0 && col >= r_size;
        const float m =
            (loc >= 0 && p >= 0) ? sp_mask_at(iv ? inv.mask_bits : ori.mask_bits, iv ? inv.mask : ori.mask, p) : 1.0f;
        uint32_t key = SP_EDGE_NONE;
        float ge = 0.0f;
        if (loc >= 0 && !(holes && p >= 0 && m == 0.0f)) {
            const float gv = grad[loc];
            const float wv = wrow[col];
            const float gm = fl_mul(gv, m);
            gsp = fl_add(gsp, fl_mul(gm, wv));
            gwv = fl_mul(gm, a);
            if (edge_grads && p >= 0) {
                const fl_side &s = iv ? inv : ori;
                if (s.grad_edge) {
                    // trainable edge weights: the item's term, keyed by its
                    // side and CSR position, is folded per position in raw
                    // order after a stable sort (no atomics)
                    ge = fl_mul(fl_mul(fl_mul(fl_mul(gv, a), wv), m), s.dscore[p]);
                    key = (uint32_t)(iv ? ori.edges + p : p);
                }
            }
        }
        if (ekey && kb + lane < k1) {
            ekey[kb + lane] = key;
            eval[kb + lane] = ge;
        }
        // per-column sums of this chunk (segmented scan keyed by the column);
        // the tail lane of each segment adds it to the wave's row -- each
        // column has one tail per chunk, and the chunks go in order
        const float x = sp_seg_scan(gwv, col);
        const int next1 = fl_dpp<0x130>(col + 1);  // wave_shl:1, lane 63 receives 0
        const bool tail = next1 != col + 1;
        if (col >= 0 && tail) gdst[col] = fl_add(gdst[col], x);
    };
    auto walk = [&](auto has_pos) {
        Rec A, B;
        load(A, k0, has_pos);
        for (int64_t kb = k0;;) {
            do_round(A, B, kb, has_pos);
            if ((kb += FL_WAVE) >= k1) break;
            do_round(B, A, kb, has_pos);
            if ((kb += FL_WAVE) >= k1) break;
        }
    };
    if (k0 < k1) {
        if (raw_pos) walk(std::true_type{});
        else walk(std::false_type{});
    }
    gsp = fl_wave_sum_f32(gsp);
    if (lane == 0) grad_v[i] = gsp;
}

// Mask bitmap: thread per position, one ballot per 64 positions.
__global__ void k_mask_bits(const float *__restrict__ mask, int64_t n, uint32_t *__restrict__ bits) {
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t b = __ballot(p < n && mask[p] != 0.0f);
    const int lane = fl_lane();
    const int64_t w0 = (p - lane) >> 5;  // first word of this wave's 64 positions
    const int64_t nw = (n + 31) >> 5;
    if (lane == 0 && w0 < nw) bits[w0] = (uint32_t)b;
    if (lane == 32 && w0 + 1 < nw) bits[w0 + 1] = (uint32_t)(b >> 32);
}

// A Boolean visibility mask straight to a side's bitmap, without the float
// gather of fl_apply_mask: the mask (by original edge id, one byte each) is
// packed into bits by edge id (coalesced, one ballot per 64 edges), then each
// CSR position reads its edge's bit through order (a 4-byte gather from a
// bitmap of M/8 bytes, which stays in L2) and the bits are packed again by
// position.  An order value outside [0, n) reads as 0.
__global__ void k_pack_bool_bits(const uint8_t *__restrict__ mask, int64_t n, uint32_t *__restrict__ bits) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t b = __ballot(e < n && mask[e] != 0);
    const int lane = fl_lane();
    const int64_t w0 = (e - lane) >> 5;
    const int64_t nw = (n + 31) >> 5;
    if (lane == 0 && w0 < nw) bits[w0] = (uint32_t)b;
    if (lane == 32 && w0 + 1 < nw) bits[w0 + 1] = (uint32_t)(b >> 32);
}

// Wave per OB_U consecutive 64-position rounds: every round's order entry,
// then every bitmap word, requested before the first is used.
constexpr int OB_U = 4;

__global__ void k_order_bits(const uint32_t *__restrict__ edge_bits, const int32_t *__restrict__ order, int64_t n,
                             uint32_t *__restrict__ bits) {
    const int lane = fl_lane();
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / FL_WAVE;
    const int64_t p0 = wave * (OB_U * FL_WAVE) + lane;
    int32_t e[OB_U];
#pragma unroll
    for (int u = 0; u < OB_U; ++u) {
        const int64_t p = p0 + u * FL_WAVE;
        e[u] = p < n ? order[p] : -1;
    }
    uint32_t wd[OB_U];
#pragma unroll
    for (int u = 0; u < OB_U; ++u) wd[u] = e[u] >= 0 && e[u] < n ? edge_bits[e[u] >> 5] : 0u;
    const int64_t nw = (n + 31) >> 5;
#pragma unroll
    for (int u = 0; u < OB_U; ++u) {
        const bool on = e[u] >= 0 && e[u] < n && ((wd[u] >> (e[u] & 31)) & 1u);
        const uint64_t b = __ballot(on);
        const int64_t w0 = (p0 + u * FL_WAVE - lane) >> 5;
        if (lane == 0 && w0 < nw) bits[w0] = (uint32_t)b;
        if (lane == 32 && w0 + 1 < nw) bits[w0 + 1] = (uint32_t)(b >> 32);
    }
}

// Entry order validation: every entry visited exactly once (else error 1).
__global__ void k_sp_order_count(const int32_t *__restrict__ order, int64_t nnz, int32_t *__restrict__ seen,
                                 int64_t *__restrict__ err) {
    const int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= nnz) return;
    const int32_t o = order[w];
    if (o < 0 || o >= nnz) atomicMax((unsigned long long *)err, 1ull);
    else atomicAdd(&seen[o], 1);
}

__global__ void k_sp_order_check(const int32_t *__restrict__ seen, int64_t nnz, int64_t *__restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < nnz && seen[i] != 1) atomicMax((unsigned long long *)err, 1ull);
}

// Entry visiting order by source entity, in blocks of SP_ORD_BLK entity ids
// (a counting sort over the blocks; the entries of one block in any order):
// rank[i] = the entry's slot among its block's entries, then
// order[start of block + rank] = i.  Entity ids outside [0, E) share the
// last bin (the plan reports them).
constexpr int SP_ORD_SHIFT = 6;  // 64 entity ids per block
__device__ __forceinline__ int64_t sp_ord_bin(int64_t e, int64_t E) {
    return (e >= 0 && e < E) ? (e >> SP_ORD_SHIFT) : (E >> SP_ORD_SHIFT) + 1;
}

__global__ void k_sp_ord_count(const int64_t *__restrict__ se, int64_t nnz, int64_t E, int32_t *__restrict__ cnt,
                               int32_t *__restrict__ rank) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nnz) return;
    rank[i] = atomicAdd(&cnt[sp_ord_bin(se[i], E)], 1);
}

__global__ void k_sp_ord_place(const int64_t *__restrict__ se, int64_t nnz, int64_t E,
                               const int64_t *__restrict__ start, const int32_t *__restrict__ rank,
                               int32_t *__restrict__ order) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nnz) return;
    order[start[sp_ord_bin(se[i], E)] + rank[i]] = (int32_t)i;
}

// Chunk counts in visiting order.
__global__ void k_sp_gather_nch(const int32_t *__restrict__ nch, const int32_t *__restrict__ order, int64_t nnz,
                                int32_t *__restrict__ out) {
    const int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (w < nnz) {
        const int32_t o = order[w];
        out[w] = (o >= 0 && o < nnz) ? nch[o] : 0;
    }
}

__global__ void k_fill_i32(int32_t *__restrict__ p, int64_t n, int32_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void k_fill_i64(int64_t *__restrict__ p, int64_t n, int64_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// plan[5] = 1 when an attention weight is not finite (any lane of a wave
// that sees one sets it).
__global__ void k_sp_finite(const float *__restrict__ w, int64_t count, unsigned long long *__restrict__ flag) {
    bool bad = false;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        bad |= !isfinite(w[i]);
    if (__ballot(bad) != 0 && fl_lane() == 0) atomicOr(flag, 1ull);
}

__global__ void k_sp_plan_out(const int64_t *__restrict__ items, const int64_t *__restrict__ tiles, int64_t NB,
                              const int64_t *__restrict__ chunks, int64_t *__restrict__ plan) {
    plan[0] = *items;
    plan[1] = *tiles;
    plan[3] = NB;
    plan[4] = chunks ? *chunks : 0;
}

__global__ void k_fill_from(const int64_t *__restrict__ src, int64_t *__restrict__ dst) { *dst = *src; }

__global__ void k_fill_f32(float *__restrict__ p, int64_t n, float v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// ---------------------------------------------------------------------------
// c1 on a coalesced COO state (_sparse_topc_entries, flashlog_kernel.py:
// 1092-1140): one 1024-thread workgroup per row; rows with more than c
// nonzeros keep their c largest nonzeros (ties to the earlier entry, i.e. the
// smaller entity), other rows keep every entry, explicit zeros included.
__global__ __launch_bounds__(TOPC_NT) void k_sp_topc(const int64_t *__restrict__ row_ptr,
                                                    const float *__restrict__ vals, int64_t c,
                                                    int32_t *__restrict__ keep) {
    __shared__ int hist[2048];
    __shared__ int lds_scan[TOPC_NT / FL_WAVE + 1];
    __shared__ int sel_bin, sel_need, s_last, s_done;
    const int64_t row = blockIdx.x;
    const int64_t start = row_ptr[row];
    const int64_t E = row_ptr[row + 1] - start;
    if (E == 0) return;
    const float *a = vals + start;
    int32_t *kp = keep + start;
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
        topc_select<2048>(hist, (int)c, lds_scan, &sel_bin, &sel_need);
        uint32_t prefix = (uint32_t)sel_bin << 21;
        int need = sel_need;
        for (int i = t; i < 2048; i += TOPC_NT) hist[i] = 0;
        __syncthreads();
        TOPC_FOR_ROW(const uint32_t k = fl_order_key(v);
                     if (v != 0.0f && (k >> 21) == (prefix >> 21)) atomicAdd(&hist[(k >> 10) & 2047], 1);)
        __syncthreads();
        topc_select<2048>(hist, need, lds_scan, &sel_bin, &sel_need);
        prefix |= (uint32_t)sel_bin << 10;
        need = sel_need;
        for (int i = t; i < 2048; i += TOPC_NT) hist[i] = 0;
        __syncthreads();
        TOPC_FOR_ROW(const uint32_t k = fl_order_key(v);
                     if (v != 0.0f && (k >> 10) == (prefix >> 10)) atomicAdd(&hist[k & 1023], 1);)
        __syncthreads();
        topc_select<1024>(hist, need, lds_scan, &sel_bin, &sel_need);
        prefix |= (uint32_t)sel_bin;
        need = sel_need;
        const int tied_total = hist[sel_bin];
        cutkey = prefix;
        if (need >= tied_total) {
            last = E;
        } else {
            if (t == 0) { s_last = -1; s_done = 0; }
            __syncthreads();
            int run = 0;
            for (int64_t base = 0; base < E; base += TOPC_NT) {
                const int64_t e = base + t;
                int flag = 0;
                if (e < E) {
                    const float v = a[e];
                    flag = (v != 0.0f && fl_order_key(v) == cutkey) ? 1 : 0;
                }
                int tot;
                const int ex = fl_block_excl_scan<TOPC_NT>(flag, lds_scan, &tot);
                if (flag && run + ex + 1 == need) { s_last = (int)e; s_done = 1; }
                run += tot;
                __syncthreads();
                if (s_done) break;
            }
            last = s_last;
        }
    }
    TOPC_FOR_ROW(int k = 1;
                 if (over) {
                     k = 0;
                     if (c > 0 && v != 0.0f) {
                         const uint32_t q = fl_order_key(v);
                         k = (q > cutkey) || (q == cutkey && e <= last);
                     }
                 }
                 kp[e] = k;)
}

// ---------------------------------------------------------------------------
// Sampled c1 (flashlog_kernel.py:1121-1132, sampling=True): in rows with
// more than c nonzeros the candidates (nonzero entries, which must be finite
// and positive) are ranked by the exponential race score
// log(v) - log(noise), noise ~ Exp(1) one per candidate in entry order, and
// the c best are kept (ties to the earlier entry); zero entries of those rows
// are dropped and other rows keep every entry.
//   k_race_rows   workgroup per row: over[r] = (nonzeros > c)
//   k_race_flags  thread per entry: candidate flag, score validation
//   (scan)        candidate offsets; the caller draws the noise
//   k_race_keys   thread per entry: 64-bit order key of the score
//   k_race_select 1024-thread workgroup per row: radix select (11/11/11/11/
//                 10/10 bits) of the c-th largest key, ordered tie scan

__device__ __forceinline__ unsigned long long fl_order_key64(double d) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(d);
    return (u >> 63) ? ~u : (u | 0x8000000000000000ull);
}

__global__ __launch_bounds__(NM_NT0) void k_race_rows(const int64_t *__restrict__ row_ptr,
                                                      const float *__restrict__ v, int64_t c,
                                                      int32_t *__restrict__ over, int64_t *__restrict__ kept) {
    __shared__ int red[NM_NT0 / FL_WAVE];
    const int64_t r = blockIdx.x;
    const int64_t a = row_ptr[r], b = row_ptr[r + 1];
    int nz = 0;
    for (int64_t k = a + threadIdx.x; k < b; k += NM_NT0) nz += v[k] != 0.0f ? 1 : 0;
    nz = fl_wave_sum_i32(nz);
    if (fl_lane() == 0) red[threadIdx.x / FL_WAVE] = nz;
    __syncthreads();
    if (threadIdx.x == 0) {
        long long t = 0;
        for (int q = 0; q < NM_NT0 / FL_WAVE; ++q) t += red[q];
        over[r] = t > c ? 1 : 0;
        kept[r] = t > c ? c : b - a;  // an over-limit row keeps exactly c of its nonzeros
    }
}

__global__ void k_race_flags(const int64_t *__restrict__ sb, const int64_t *__restrict__ sl,
                             const float *__restrict__ v, int64_t nnz, int64_t L, const int32_t *__restrict__ over,
                             int32_t *__restrict__ cand, int64_t *__restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nnz) return;
    const float x = v[i];
    const int f = (over[sb[i] * L + sl[i]] && x != 0.0f) ? 1 : 0;
    cand[i] = f;
    if (f && !(x > 0.0f && x <= 3.402823466e38f)) atomicMax((unsigned long long *)err, 3ull);
}

__global__ void k_race_keys(const float *__restrict__ v, int64_t nnz, const int32_t *__restrict__ cand,
                            const int64_t *__restrict__ cand_off, const double *__restrict__ noise,
                            unsigned long long *__restrict__ keys) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nnz) return;
    keys[i] = cand[i] ? fl_order_key64(__dsub_rn(log((double)v[i]), log(noise[cand_off[i]]))) : 0ull;
}

// With a compaction (entries non-null): the kept entries of row r also go,
// in entry order, to positions kept_off[r] .. of entries (their indices) and
// of ob, ol, oe, ov (their coordinates and values).
struct SpCompact {
    const int64_t *sb, *sl, *se;
    const float *v;
    const int64_t *kept_off;
    int64_t *entries, *ob, *ol, *oe;
    float *ov;
};

__device__ __forceinline__ void sp_compact_put(const SpCompact &cp, int64_t i, int64_t q) {
    cp.entries[q] = i;
    cp.ob[q] = cp.sb[i];
    cp.ol[q] = cp.sl[i];
    cp.oe[q] = cp.se[i];
    cp.ov[q] = cp.v[i];
}

__global__ __launch_bounds__(TOPC_NT) void k_race_select(const int64_t *__restrict__ row_ptr,
                                                        const int32_t *__restrict__ over,
                                                        const int32_t *__restrict__ cand,
                                                        const unsigned long long *__restrict__ keys, int64_t c,
                                                        int32_t *__restrict__ keep, SpCompact cp) {
    __shared__ int hist[2048];
    __shared__ int lds_scan[TOPC_NT / FL_WAVE + 1];
    __shared__ int sel_bin, sel_need, s_last, s_done;
    const int64_t row = blockIdx.x;
    const int64_t a = row_ptr[row], n = row_ptr[row + 1] - a;
    const int t = threadIdx.x;
    if (n == 0) return;
    if (!over[row]) {
        const int64_t q0 = cp.entries ? cp.kept_off[row] : 0;
        for (int64_t k = t; k < n; k += TOPC_NT) {
            keep[a + k] = 1;
            if (cp.entries) sp_compact_put(cp, a + k, q0 + k);
        }
        return;
    }
    // radix select of the c-th largest candidate key, most significant first
    const int shifts[6] = {53, 42, 31, 20, 10, 0};
    const int widths[6] = {11, 11, 11, 11, 10, 10};
    unsigned long long prefix = 0, pmask = 0;
    int need = (int)c;
    int tied_total = 0;
    for (int ps = 0; ps < 6; ++ps) {
        const int sh = shifts[ps], wd = widths[ps];
        const int nb = 1 << wd;
        for (int q = t; q < 2048; q += TOPC_NT) hist[q] = 0;
        __syncthreads();
        for (int64_t k = t; k < n; k += TOPC_NT) {
            if (!cand[a + k]) continue;
            const unsigned long long key = keys[a + k];
            if ((key & pmask) == prefix) atomicAdd(&hist[(key >> sh) & (nb - 1)], 1);
        }
        __syncthreads();
        if (nb == 2048) topc_select<2048>(hist, need, lds_scan, &sel_bin, &sel_need);
        else topc_select<1024>(hist, need, lds_scan, &sel_bin, &sel_need);
        prefix |= (unsigned long long)sel_bin << sh;
        pmask |= (unsigned long long)(nb - 1) << sh;
        need = sel_need;
        tied_total = hist[sel_bin];
        __syncthreads();
    }
    const unsigned long long cutkey = prefix;
    int64_t last = n;
    if (need < tied_total) {
        if (t == 0) { s_last = -1; s_done = 0; }
        __syncthreads();
        int run = 0;
        for (int64_t base = 0; base < n; base += TOPC_NT) {
            const int64_t k = base + t;
            const int flag = (k < n && cand[a + k] && keys[a + k] == cutkey) ? 1 : 0;
            int tot;
            const int ex = fl_block_excl_scan<TOPC_NT>(flag, lds_scan, &tot);
            if (flag && run + ex + 1 == need) { s_last = (int)k; s_done = 1; }
            run += tot;
            __syncthreads();
            if (s_done) break;
        }
        last = s_last;
    }
    const int64_t q0 = cp.entries ? cp.kept_off[row] : 0;
    int64_t run = 0;
    for (int64_t base = 0; base < n; base += TOPC_NT) {
        const int64_t k = base + t;
        int kp = 0;
        if (k < n && cand[a + k]) {
            const unsigned long long key = keys[a + k];
            kp = key > cutkey || (key == cutkey && k <= last);
        }
        if (k < n) keep[a + k] = kp;
        if (cp.entries) {
            // the row keeps exactly c entries: ranks beyond c are never written
            int tot;
            const int ex = fl_block_excl_scan<TOPC_NT>(kp, lds_scan, &tot);
            if (kp && run + ex < c) sp_compact_put(cp, a + k, q0 + run + ex);
            run += tot;
        }
    }
}

// ---------------------------------------------------------------------------
// normalize_sparse3d (flashlog.cu:2480-2691; flashlog_kernel.py:536-614):
// per row the sum of its values (fixed order: 256 strided partial sums, then
// a tree), out = v / max(d, eps); backward g/dc - sum(g*v)/dc^2 where d >= eps.

constexpr int NM_NT = 256;

__device__ __forceinline__ float block_tree_sum(float v, float *red) {
    red[threadIdx.x] = v;
    __syncthreads();
    for (int st = NM_NT / 2; st > 0; st >>= 1) {
        if ((int)threadIdx.x < st) red[threadIdx.x] = fl_add(red[threadIdx.x], red[threadIdx.x + st]);
        __syncthreads();
    }
    const float s = red[0];
    __syncthreads();
    return s;
}

// row_ptr[r] for r in [0, R] by binary search over the row keys b*L + l of
// entries sorted by row (the first entry of row r or later), without
// checking the order: every value stays in [0, nnz], so kernels bounded by
// it stay in range on any input.
__global__ void k_sp_rowptr_search(const int64_t *__restrict__ sb, const int64_t *__restrict__ sl, int64_t nnz,
                                   int64_t L, int64_t R, int64_t *__restrict__ row_ptr) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r > R) return;
    int64_t lo = 0, hi = nnz;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (sb[mid] * L + sl[mid] < r) lo = mid + 1;
        else hi = mid;
    }
    // The first row starts at entry 0 and the last ends at nnz whatever the
    // keys hold: the search result is monotone in r even over unsorted keys,
    // so every entry then lies in exactly one row's range and every output
    // is written (keys outside [0, R) or out of order give unspecified
    // values, never unwritten ones).
    row_ptr[r] = r == 0 ? 0 : (r == R ? nnz : lo);
}

// Per row (workgroup): the denominator is a left fold from 0 over the row's
// values in entry (= output key) order, as the CPU path adds them
// (flashlog.cpp:1561-1565); the workgroup stages chunks of the row in LDS
// (double-buffered) while its first thread folds the previous chunk.  The
// clamp is the GPU path's (flashlog.cu:2540): d >= eps ? d : eps, so a NaN
// sum divides by eps.
constexpr int NF_CHUNK = 2048;

__global__ __launch_bounds__(NM_NT) void k_norm_fwd(const int64_t *__restrict__ row_ptr,
                                                   const float *__restrict__ v, float eps, float *__restrict__ out,
                                                   float *__restrict__ denom) {
    __shared__ float4 buf[2][NF_CHUNK / 4];
    __shared__ float dsh;
    const int64_t r = blockIdx.x;
    const int64_t a = row_ptr[r], b = row_ptr[r + 1];
    const int t = threadIdx.x;
    float acc = 0.0f;
    int c = 0;
    for (int64_t base = a; base < b; base += NF_CHUNK, ++c) {
        const int len = (int)((b - base) < NF_CHUNK ? (b - base) : NF_CHUNK);
        float *cb = (float *)buf[c & 1];
        for (int i = t; i < len; i += NM_NT) cb[i] = v[base + i];
        __syncthreads();
        if (t == 0) acc = sp_fold(acc, cb, 0, len);  // 32 values per LDS round trip
    }
    if (t == 0) {
        dsh = acc;
        denom[r] = acc;
    }
    __syncthreads();
    const float d = dsh;
    const float dc = d >= eps ? d : eps;
    for (int64_t k = a + t; k < b; k += NM_NT) out[k] = __fdiv_rn(v[k], dc);
}

// Backward (flashlog.cu:2553-2591): g/d - sum(g*v)/d^2 where d >= eps, else
// g/eps; sum(g*v) in a fixed tree order.
__global__ __launch_bounds__(NM_NT) void k_norm_bwd(const int64_t *__restrict__ row_ptr,
                                                   const float *__restrict__ g, const float *__restrict__ v,
                                                   const float *__restrict__ denom, float eps,
                                                   float *__restrict__ gv) {
    __shared__ float red[NM_NT];
    const int64_t r = blockIdx.x;
    const int64_t a = row_ptr[r], b = row_ptr[r + 1];
    const float d = denom[r];
    const bool active = d >= eps;
    const float dc = active ? d : eps;
    float s = 0.0f;
    for (int64_t k = a + threadIdx.x; k < b; k += NM_NT) s = fl_add(s, fl_mul(g[k], v[k]));
    const float sgx = block_tree_sum(s, red);
    const float corr = active ? __fdiv_rn(sgx, fl_mul(dc, dc)) : 0.0f;
    for (int64_t k = a + threadIdx.x; k < b; k += NM_NT) gv[k] = __fsub_rn(__fdiv_rn(g[k], dc), corr);
}

// Thread per query coordinate: the value stored at the same (b, l, e) of a
// coalesced COO tensor (keys (b*L + l)*E + e strictly increasing), found by
// binary search, or 0 when the tensor has no entry there.
__global__ void k_sp_gather(const int64_t *__restrict__ gb, const int64_t *__restrict__ gl,
                            const int64_t *__restrict__ ge, const float *__restrict__ gv, int64_t ng,
                            const int64_t *__restrict__ qb, const int64_t *__restrict__ ql,
                            const int64_t *__restrict__ qe, int64_t nq, int64_t L, int64_t E,
                            float *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nq) return;
    const int64_t key = (qb[i] * L + ql[i]) * E + qe[i];
    // the usual case: the same coordinates in the same order
    if (i < ng && (gb[i] * L + gl[i]) * E + ge[i] == key) {
        out[i] = gv[i];
        return;
    }
    int64_t lo = 0, hi = ng;
    while (lo < hi) {
        const int64_t mid = lo + ((hi - lo) >> 1);
        const int64_t mk = (gb[mid] * L + gl[mid]) * E + ge[mid];
        if (mk < key) lo = mid + 1; else hi = mid;
    }
    float val = 0.0f;
    if (lo < ng && (gb[lo] * L + gl[lo]) * E + ge[lo] == key) val = gv[lo];
    out[i] = val;
}

}  // namespace fl

// ---------------------------------------------------------------------------
// C-ABI

using namespace fl;

namespace {

size_t al(size_t x) { return (x + 255) & ~(size_t)255; }

int64_t sp_buckets(int64_t E) { return E <= 0 ? 1 : (E + SP_W - 1) / SP_W; }

int sp_bucket_bits(int64_t NB) {
    int b = 0;
    while (((int64_t)1 << b) < NB) ++b;
    return b;
}

// plan workspace layout
struct SpPlan {
    float *th;
    int32_t *cut, *cnt, *ntiles, *nch, *nch_ord;
    int64_t *item_off, *row_ptr, *row_item0, *tile_base, *tmp, *chunk_off;
    SpQuota *quota;       // [nnz][2] training quota parameters (quota sides only)
    int16_t *rel_order;   // [R][2][r_size] c2 admission order (r_size <= RO_MAX)
    int32_t *rel_nelig;   // [R][2] relations with a positive weight
    size_t bytes;
};

SpPlan sp_plan_layout(int64_t nnz, int64_t R, int64_t r_size, char *base) {
    SpPlan p{};
    size_t off = 0;
    auto take = [&](size_t b) { char *q = base ? base + off : nullptr; off += al(b); return q; };
    p.th = (float *)take(sizeof(float) * 2 * (size_t)nnz);
    p.cut = (int32_t *)take(sizeof(int32_t) * 2 * (size_t)nnz);
    p.cnt = (int32_t *)take(sizeof(int32_t) * (size_t)nnz);
    p.item_off = (int64_t *)take(sizeof(int64_t) * (size_t)(nnz + 1));
    p.nch = (int32_t *)take(sizeof(int32_t) * (size_t)nnz);
    p.nch_ord = (int32_t *)take(sizeof(int32_t) * (size_t)nnz);
    p.chunk_off = (int64_t *)take(sizeof(int64_t) * (size_t)(nnz + 1));
    p.row_ptr = (int64_t *)take(sizeof(int64_t) * (size_t)(R + 1));
    p.row_item0 = (int64_t *)take(sizeof(int64_t) * (size_t)(R + 1));
    p.ntiles = (int32_t *)take(sizeof(int32_t) * (size_t)R);
    p.tile_base = (int64_t *)take(sizeof(int64_t) * (size_t)(R + 1));
    const int64_t mx = nnz > R ? nnz : R;
    p.tmp = (int64_t *)take(scan_tmp_bytes(mx + 1));
    p.quota = (SpQuota *)take(sizeof(SpQuota) * 2 * (size_t)(nnz > 0 ? nnz : 1));
    if (r_size > 0 && r_size <= RO_MAX) {
        p.rel_order = (int16_t *)take(sizeof(int16_t) * 2 * (size_t)R * (size_t)r_size);
        p.rel_nelig = (int32_t *)take(sizeof(int32_t) * 2 * (size_t)(R > 0 ? R : 1));
    }
    p.bytes = off;
    return p;
}

// expansion workspace layout
struct SpExp {
    int32_t *raw_dst, *part_dst, *part_inv, *hist, *tot, *out_count;
    float *raw_val, *part_val;
    uint32_t *raw_tie, *part_tie;
    int32_t *hot_list, *mid_list, *hot_fb, *mid_fb, *hot_count;
    int64_t *base, *tmp;
    SpRuns runs;
    size_t bytes;
};

SpExp sp_exp_layout(int64_t T, int64_t tiles, int64_t chunks, int64_t R, int64_t NB, int backward, int agg,
                    char *base) {
    SpExp x{};
    size_t off = 0;
    auto take = [&](size_t b) { char *q = base ? base + off : nullptr; off += al(b); return q; };
    const int64_t T1 = T > 0 ? T : 1;
    const int64_t U1 = chunks > 0 ? chunks : 1;
    // run table (at most one run per item) and chunk table
    x.runs.first = (int32_t *)take(sizeof(int32_t) * (size_t)T1);
    x.runs.p = (int32_t *)take(sizeof(int32_t) * (size_t)T1);
    x.runs.aw = (float *)take(sizeof(float) * (size_t)T1);
    x.runs.meta = (uint32_t *)take(sizeof(uint32_t) * (size_t)T1);
    x.runs.c_base = (int64_t *)take(sizeof(int64_t) * (size_t)U1);
    x.runs.c_run = (int64_t *)take(sizeof(int64_t) * (size_t)U1);
    x.runs.c_rlim = (int64_t *)take(sizeof(int64_t) * (size_t)U1);
    x.runs.c_off = (int32_t *)take(sizeof(int32_t) * (size_t)U1);
    x.runs.c_n = (int32_t *)take(sizeof(int32_t) * (size_t)U1);
    x.raw_dst = (int32_t *)take(sizeof(int32_t) * (size_t)T1);
    x.raw_val = (float *)take(sizeof(float) * (size_t)T1);
    if (agg == SP_MAX) x.raw_tie = (uint32_t *)take(sizeof(uint32_t) * (size_t)T1);
    if (NB > 1) {
        x.part_dst = (int32_t *)take(sizeof(int32_t) * (size_t)T1);
        x.part_val = (float *)take(sizeof(float) * (size_t)T1);
        if (agg == SP_MAX) x.part_tie = (uint32_t *)take(sizeof(uint32_t) * (size_t)T1);
        x.hist = (int32_t *)take(sizeof(int32_t) * (size_t)(tiles * NB > 0 ? tiles * NB : 1));
        x.tot = (int32_t *)take(sizeof(int32_t) * (size_t)(R * NB > 0 ? R * NB : 1));
        x.base = (int64_t *)take(sizeof(int64_t) * (size_t)(R * NB + 1));
    }
    x.out_count = (int32_t *)take(sizeof(int32_t) * (size_t)(R * NB > 0 ? R * NB : 1));
    int64_t mx = tiles * NB;
    if (R * NB > mx) mx = R * NB;
    x.tmp = (int64_t *)take(scan_tmp_bytes(mx + 1));
    x.hot_list = (int32_t *)take(sizeof(int32_t) * (size_t)(R * NB > 0 ? R * NB : 1));
    x.mid_list = (int32_t *)take(sizeof(int32_t) * (size_t)(R * NB > 0 ? R * NB : 1));
    x.hot_fb = (int32_t *)take(sizeof(int32_t) * (size_t)(R * NB > 0 ? R * NB : 1));
    x.mid_fb = (int32_t *)take(sizeof(int32_t) * (size_t)(R * NB > 0 ? R * NB : 1));
    x.hot_count = (int32_t *)take(8 * sizeof(int32_t));
    // last, so that every other offset is the same with and without it
    if (NB > 1 && backward) x.part_inv = (int32_t *)take(sizeof(int32_t) * (size_t)T1);
    x.bytes = off;
    return x;
}

int sp_check(const fl_side *ori, const fl_side *inv, const fl_sparse_hop *h, const char *what) {
    if (!ori || !inv || !h) return fl_fail(FL_ERR_ARG, "%s: null argument", what);
    if (h->nnz < 0 || h->B < 0 || h->L < 0 || h->E < 0 || h->n < 1)
        return fl_fail(FL_ERR_ARG, "%s: bad shape", what);
    if (h->E > ((int64_t)SP_W << 14)) return fl_fail(FL_ERR_ARG, "%s: E must be <= 2^27", what);
    if (h->mode != SP_TOPK && h->mode != SP_ALL && h->mode != SP_FIXED)
        return fl_fail(FL_ERR_ARG, "%s: unknown mode", what);
    if (h->aggregate != SP_SUM && h->aggregate != SP_MAX) return fl_fail(FL_ERR_ARG, "%s: unknown aggregate", what);
    if (h->aggregate == SP_MAX && h->mode != SP_TOPK)
        return fl_fail(FL_ERR_ARG, "%s: the max aggregate needs the top-k mode", what);
    if (h->sampling_seed >= 0 && h->mode != SP_TOPK)
        return fl_fail(FL_ERR_ARG, "%s: training quotas need the top-k mode", what);
    if (h->mode != SP_FIXED && (h->r_size < 0 || 2 * h->r_size + 1 > h->n + (h->wot_i ? 1 : 0)))
        return fl_fail(FL_ERR_ARG, "%s: w width %lld too small for r_size %lld", what, (long long)h->n,
                       (long long)h->r_size);
    if (h->nnz > 0 && (!h->sp_b || !h->sp_l || !h->sp_e || !h->sp_v))
        return fl_fail(FL_ERR_ARG, "%s: null input", what);
    if (h->nnz > 0 && h->mode != SP_FIXED && !h->w) return fl_fail(FL_ERR_ARG, "%s: null attention", what);
    if (h->nnz > 0 && h->mode == SP_FIXED && !h->operators) return fl_fail(FL_ERR_ARG, "%s: null operators", what);
    for (const fl_side *s : {ori, inv})
        if (s->edges > 0 && (!s->col_ind || (!s->mask && !s->mask_bits && h->mode != SP_FIXED) || !s->group_rel ||
                             !s->group_start || !s->group_count))
            return fl_fail(FL_ERR_ARG, "%s: side without CSR arrays", what);
    if (h->aggregate == SP_MAX)
        for (const fl_side *s : {ori, inv})
            if (s->edges > 0 && !s->order) return fl_fail(FL_ERR_ARG, "%s: max needs the sides' edge order", what);
    for (const fl_side *s : {ori, inv})
        if (s->edges > 0 && s->grad_edge && (!s->order || !s->dscore))
            return fl_fail(FL_ERR_ARG, "%s: edge-weight gradients need the order and dscore arrays", what);
    return FL_OK;
}

}  // namespace

// ---- channel sum of a coalesced [B, L, E] state (the models' sum_sp_3d) ----
// Within one query b the L channel rows are each sorted by entity, so the
// (b, e) order of the re-indexed entries is a merge of L sorted lists: an
// entry's merged position is its index in its own row plus, in every other
// row of b, the entries before it (entity < e, or <= e in an earlier channel,
// so ties keep channel order as a stable sort does).  An entry is a head when
// no earlier channel holds its entity; heads are scanned into output slots and
// each head adds its run of the merged order from 0 in that order.
__device__ __forceinline__ int64_t cs_lower_bound(const int64_t *__restrict__ se, int64_t lo, int64_t hi, int64_t e) {
    while (lo < hi) {
        const int64_t mid = lo + ((hi - lo) >> 1);
        if (se[mid] < e) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

__global__ void k_cs_rank(const int64_t *__restrict__ sb, const int64_t *__restrict__ sl,
                          const int64_t *__restrict__ se, int64_t nnz, int64_t L, int64_t R, int64_t E,
                          const int64_t *__restrict__ row_ptr, int32_t *__restrict__ perm,
                          int32_t *__restrict__ head, int64_t *__restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nnz) return;
    const int64_t b = sb[i], l = sl[i], e = se[i];
    if (b < 0 || l < 0 || l >= L || b * L + l >= R) return;  // flagged by k_sp_rowptr
    if (e < 0 || e >= E) {  // flagged by k_sp_rowptr as well; never placed
        atomicMax((unsigned long long *)err, 1ull);
        return;
    }
    const int64_t r = b * L + l;
    const int64_t rs = row_ptr[r];
    if (i > rs && se[i - 1] >= e) {  // entities not strictly increasing within the row
        atomicMax((unsigned long long *)err, 3ull);
        return;
    }
    int64_t pos = i - rs;
    int h = 1;
    for (int64_t q = 0; q < L; ++q) {
        if (q == l) continue;
        const int64_t a = row_ptr[b * L + q], z = row_ptr[b * L + q + 1];
        const int64_t lb = cs_lower_bound(se, a, z, e);
        if (q < l && lb < z && se[lb] == e) {
            ++pos;
            h = 0;
        }
        pos += lb - a;
    }
    const int64_t m = row_ptr[b * L] + pos;
    if (m < row_ptr[b * L] || m >= row_ptr[b * L + L]) {
        atomicMax((unsigned long long *)err, 4ull);
        return;
    }
    perm[m] = (int32_t)i;
    head[m] = h;
}

__global__ void k_cs_plan_out(const int64_t *__restrict__ hoff, int64_t nnz, const int64_t *__restrict__ err,
                              int64_t *__restrict__ plan) {
    if (threadIdx.x == 0) {
        plan[0] = hoff[nnz];
        plan[1] = err[0];
    }
}

// op 0: the sum from 0 in channel order; op 1: the maximum (first of equal
// values kept, NaN propagated, as torch's amax).
template <int OP>
__global__ void k_cs_emit(const int64_t *__restrict__ sb, const int64_t *__restrict__ se,
                          const float *__restrict__ v, int64_t nnz, const int32_t *__restrict__ perm,
                          const int32_t *__restrict__ head, const int64_t *__restrict__ hoff, int64_t nout,
                          int64_t *__restrict__ out_b, int64_t *__restrict__ out_e, float *__restrict__ out_v,
                          int32_t *__restrict__ slot) {
    const int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (m >= nnz || !head[m]) return;
    const int64_t o = hoff[m];
    const int32_t i = perm[m];
    if (o < 0 || o >= nout || i < 0 || i >= nnz) return;
    float acc = 0.0f;
    for (int64_t k = m; k < nnz && (k == m || !head[k]); ++k) {
        const int32_t j = perm[k];
        if (j < 0 || j >= nnz) break;
        const float x = v[j];
        if (OP == 0) acc = acc + x;
        else acc = (k == m || x > acc || x != x) ? x : acc;
        slot[j] = (int32_t)o;
    }
    out_b[o] = sb[i];
    out_e[o] = se[i];
    out_v[o] = acc;
}

// Weighted channel sums into a dense accumulator (rule-bank scoring): for
// the run of entries sharing (b, e), in channel order, and every rank k,
// acc = sum from 0 of v * W[l, k]; then dense[k, b*E + e] += acc.  One thread
// per run: each accumulator slot has one writer per call, so the dense sums
// are added in a fixed order (calls in order, channels in order).  A state
// the plan flagged (not coalesced, or an index outside [B, L, E]) adds
// nothing: the plan's error word is read here, on the device.
__global__ void k_cs_weighted_add(const int64_t *__restrict__ sb, const int64_t *__restrict__ sl,
                                  const int64_t *__restrict__ se, const float *__restrict__ v, int64_t nnz,
                                  const int32_t *__restrict__ perm, const int32_t *__restrict__ head,
                                  const float *__restrict__ W, int64_t K, int64_t B, int64_t E,
                                  const int64_t *__restrict__ err, float *__restrict__ dense) {
    const int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (m >= nnz || *err != 0 || !head[m]) return;
    const int32_t i = perm[m];
    if (i < 0 || i >= nnz) return;
    const int64_t key = sb[i] * E + se[i];
    for (int64_t k = 0; k < K; ++k) {
        float acc = 0.0f;
        for (int64_t q = m; q < nnz && (q == m || !head[q]); ++q) {
            const int32_t j = perm[q];
            if (j < 0 || j >= nnz) break;
            acc = fl_add(acc, fl_mul(v[j], W[sl[j] * K + k]));
        }
        float *slot = dense + k * B * E + key;
        *slot = fl_add(*slot, acc);
    }
}

extern "C" {

int64_t fl_sparse_buckets(int64_t E) { return sp_buckets(E); }

size_t fl_sparse_plan_bytes(int64_t nnz, int64_t R, int64_t r_size) {
    if (nnz < 0 || R < 0 || r_size < 0) return 0;
    return sp_plan_layout(nnz, R, r_size, nullptr).bytes;
}

static int64_t sp_budget(const fl_sparse_hop *h);
// relations per side of the hop's attention (0 for the fixed-relation step)
static int64_t sp_rsize(const fl_sparse_hop *h) { return h->mode == SP_FIXED ? 0 : h->r_size; }
// Training quotas can apply (sampling seed, top-k mode, a positive budget).
static bool sp_quotas(const fl_sparse_hop *h) { return h->sampling_seed >= 0 && sp_budget(h) > 0; }
// The backward reads an item's CSR position only for its mask value and edge
// factor.  It does without them for the top-k sum over several buckets per
// row (masked items are holes with output index -1, kept items have mask 1
// when every mask is a bitmap) with no edge factors.
static bool sp_pos_optional(const fl_side *ori, const fl_side *inv, const fl_sparse_hop *h) {
    const auto side_ok = [](const fl_side *s) { return (!s->mask || s->mask_bits) && !s->dscore; };
    return h->mode == SP_TOPK && h->aggregate == SP_SUM && sp_buckets(h->E) > 1 && side_ok(ori) && side_ok(inv);
}

int fl_sparse_plan(void *stream, const fl_side *ori, const fl_side *inv, const fl_sparse_hop *h, int64_t *plan) {
    int rc;
    if ((rc = sp_check(ori, inv, h, "sparse_plan")) != FL_OK) return rc;
    if (!plan || !h->ws1) return fl_fail(FL_ERR_ARG, "sparse_plan: null plan or workspace");
    const int64_t R = h->B * h->L;
    if (h->ws1_bytes < fl_sparse_plan_bytes(h->nnz, R, sp_rsize(h)))
        return fl_fail(FL_ERR_ARG, "sparse_plan: workspace too small");
    SpPlan p = sp_plan_layout(h->nnz, R, sp_rsize(h), (char *)h->ws1);
    hipStream_t st = (hipStream_t)stream;
    const int64_t nnz = h->nnz;
    const int64_t K = sp_budget(h);
    // plan[0] items, plan[1] tiles, plan[2] error, plan[3] buckets per row, plan[4] item chunks,
    // plan[5] non-finite attention
    FL_LAUNCH("k_fill_i32", k_fill_i32, dim3(1), dim3(64), 0, st, (int32_t *)plan, (int64_t)12, 0);
    if (h->mode != SP_FIXED && h->w && R * h->n > 0) {
        const int64_t cnt = R * h->n;
        const int64_t blocks = (cnt + 255) / 256 < 1024 ? (cnt + 255) / 256 : 1024;
        FL_LAUNCH("k_sp_finite", k_sp_finite, dim3((unsigned)blocks), dim3(256), 0, st, h->w, cnt,
                  (unsigned long long *)(plan + 5));
    }
    FL_LAUNCH("k_fill_i64", k_fill_i64, dim3((unsigned)((R + 1 + 255) / 256)), dim3(256), 0, st, p.row_ptr, R + 1,
              (int64_t)0);
    const int64_t g1 = (nnz > R + 1 ? nnz : R + 1);
    FL_LAUNCH("k_sp_rowptr", k_sp_rowptr, dim3((unsigned)((g1 + 255) / 256)), dim3(256), 0, st, h->sp_b, h->sp_l,
              h->sp_e, nnz, h->B, h->L, h->E, p.row_ptr, plan + 2);
    if (h->entry_order && nnz > 0 && h->mode != SP_FIXED) {
        // the order must visit every entry once (nch_ord is the count scratch here)
        FL_LAUNCH("k_fill_i32", k_fill_i32, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0, st, p.nch_ord, nnz, 0);
        FL_LAUNCH("k_sp_order_count", k_sp_order_count, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0, st,
                  h->entry_order, nnz, p.nch_ord, plan + 2);
        FL_LAUNCH("k_sp_order_check", k_sp_order_check, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0, st,
                  p.nch_ord, nnz, plan + 2);
    }
    if (nnz > 0 && h->mode == SP_FIXED)
        FL_LAUNCH("k_fx_count", k_fx_count, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0, st, *ori, *inv,
                  h->sp_b, h->sp_l, h->sp_e, h->operators, nnz, h->B, h->L, h->E, h->r_size, p.cut, p.cnt);
    else if (nnz > 0) {
        if (p.rel_order && h->mode == SP_TOPK && K > 0 && h->sampling_seed < 0 && R > 0)
            FL_LAUNCH("k_sp_relorder", k_sp_relorder, dim3((unsigned)(2 * R)), dim3(RO_NT), 0, st, h->w, h->n,
                      h->r_size, p.rel_order, p.rel_nelig);
        const bool lookup = p.rel_order && h->mode == SP_TOPK && K > 0 && h->sampling_seed < 0;
        // relation -> count maps in LDS for up to SEL_MAP_MAX relations
        const int use_map = lookup && h->r_size <= SEL_MAP_MAX;
        const size_t lds = use_map ? sizeof(int) * (SEL_NT / FL_WAVE) * (size_t)h->r_size : 0;
        FL_LAUNCH("k_sp_select", sp_quotas(h) ? k_sp_select<true> : k_sp_select<false>, dim3((unsigned)((nnz + SEL_NT / FL_WAVE - 1) / (SEL_NT / FL_WAVE))),
                  dim3(SEL_NT), lds, st, *ori, *inv, h->sp_b, h->sp_l, h->sp_e, nnz, h->w, h->B, h->L, h->E, h->n,
                  h->r_size, h->wot_i, h->mode, K, h->sampling_seed, p.th, p.cut, p.cnt,
                  lookup ? p.rel_order : (const int16_t *)nullptr, lookup ? p.rel_nelig : (const int32_t *)nullptr,
                  use_map, p.quota, p.nch, h->entry_order);
    }
    if ((rc = exclusive_scan(st, p.cnt, p.item_off, nnz, p.tmp)) != FL_OK) return rc;
    const bool fixed = h->mode == SP_FIXED;
    if (!fixed && h->entry_order && nnz > 0) {
        FL_LAUNCH("k_sp_gather_nch", k_sp_gather_nch, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0, st, p.nch,
                  h->entry_order, nnz, p.nch_ord);
        if ((rc = exclusive_scan(st, p.nch_ord, p.chunk_off, nnz, p.tmp)) != FL_OK) return rc;
    } else if (!fixed && (rc = exclusive_scan(st, p.nch, p.chunk_off, nnz, p.tmp)) != FL_OK) {
        return rc;
    }
    FL_LAUNCH("k_sp_rowinfo", k_sp_rowinfo, dim3((unsigned)((R + 1 + 255) / 256)), dim3(256), 0, st, p.row_ptr,
              p.item_off, R, p.row_item0, p.ntiles);
    if ((rc = exclusive_scan(st, p.ntiles, p.tile_base, R, p.tmp)) != FL_OK) return rc;
    FL_LAUNCH("k_sp_plan_out", k_sp_plan_out, dim3(1), dim3(1), 0, st, p.item_off + nnz, p.tile_base + R,
              sp_buckets(h->E), fixed ? (const int64_t *)nullptr : p.chunk_off + nnz, plan);
    return fl_check_launch("sparse_plan");
}

size_t fl_sparse_expand_bytes(int64_t items, int64_t tiles, int64_t chunks, int64_t R, int64_t E, int backward,
                              int aggregate) {
    if (items < 0 || tiles < 0 || chunks < 0 || R < 0) return 0;
    return sp_exp_layout(items, tiles, chunks, R, sp_buckets(E), backward, aggregate, nullptr).bytes;
}

// c2 budget of the plan and walk kernels: K > 0 selects, 0 keeps every
// eligible edge, < 0 keeps none.
static int64_t sp_budget(const fl_sparse_hop *h) {
    if (h->mode != SP_TOPK || h->topk_edges >= ((int64_t)1 << 60)) return 0;
    return h->topk_edges > 0 ? h->topk_edges : -1;
}

int fl_sparse_expand(void *stream, const fl_side *ori, const fl_side *inv, const fl_sparse_hop *h,
                     int64_t *out_base, int32_t *raw_local) {
    int rc;
    if ((rc = sp_check(ori, inv, h, "sparse_expand")) != FL_OK) return rc;
    const int64_t R = h->B * h->L, NB = sp_buckets(h->E);
    if (!h->ws1 || !h->ws2 || !out_base) return fl_fail(FL_ERR_ARG, "sparse_expand: null workspace or out_base");
    if (h->items < 0 || h->tiles < 0 || h->chunks < 0)
        return fl_fail(FL_ERR_ARG, "sparse_expand: negative plan sizes");
    if (h->mode != SP_FIXED && h->chunks > h->items + h->nnz)
        return fl_fail(FL_ERR_ARG, "sparse_expand: more item chunks than the plan allows");
    if (h->ws2_bytes <
        fl_sparse_expand_bytes(h->items, h->tiles, h->chunks, R, h->E, raw_local != nullptr, h->aggregate))
        return fl_fail(FL_ERR_ARG, "sparse_expand: workspace too small");
    if (raw_local && h->mode != SP_FIXED && h->items > 0) {
        if (!h->raw_col || (!h->raw_pos && !sp_pos_optional(ori, inv, h)))
            return fl_fail(FL_ERR_ARG, "sparse_expand: raw_local needs raw_pos and raw_col");
        if (h->n > 32767) return fl_fail(FL_ERR_ARG, "sparse_expand: backward columns need n <= 32767");
        if (h->items > INT32_MAX) return fl_fail(FL_ERR_ARG, "sparse_expand: backward output indices need items < 2^31");
    }
    SpPlan p = sp_plan_layout(h->nnz, R, sp_rsize(h), (char *)h->ws1);
    SpExp x = sp_exp_layout(h->items, h->tiles, h->chunks, R, NB, raw_local != nullptr, h->aggregate,
                            (char *)h->ws2);
    const bool mx = h->aggregate == SP_MAX;
    hipStream_t st = (hipStream_t)stream;
    const int64_t nnz = h->nnz;
    SpRows rows{p.row_item0, p.tile_base, NB};
    if (nnz > 0 && h->mode == SP_FIXED)
        FL_LAUNCH("k_fx_fill", k_fx_fill, dim3((unsigned)((nnz + SEL_NT / FL_WAVE - 1) / (SEL_NT / FL_WAVE))),
                  dim3(SEL_NT), 0, st, *ori, *inv, h->sp_e, h->sp_v, nnz, p.cut, p.item_off, x.raw_dst, x.raw_val);
    else if (nnz > 0 && h->items > 0 && sp_budget(h) > 0 && sp_budget(h) <= SP_FUSE_KMAX &&
             h->n <= (int64_t)SP_LR_COL + 1) {
        // budgeted hop: at most 2K+1 items (and runs) per entry, kept in LDS
        const int holes = h->mode == SP_TOPK && h->aggregate == SP_SUM;
        const int rcap = (int)(2 * sp_budget(h) + 2);
        const size_t lds = (size_t)(SEL_NT / FL_WAVE) * (size_t)rcap * 8;
        const dim3 grid((unsigned)((nnz + SEL_NT / FL_WAVE - 1) / (SEL_NT / FL_WAVE)));
        int32_t *rp = raw_local ? h->raw_pos : (int32_t *)nullptr;
        int16_t *rc16 = raw_local ? h->raw_col : (int16_t *)nullptr;
        auto kern = sp_quotas(h) ? (mx ? (raw_local ? k_sp_expand_fused<true, true, true> : k_sp_expand_fused<true, true, false>)
                                       : (raw_local ? k_sp_expand_fused<true, false, true> : k_sp_expand_fused<true, false, false>))
                                 : (mx ? (raw_local ? k_sp_expand_fused<false, true, true> : k_sp_expand_fused<false, true, false>)
                                       : (raw_local ? k_sp_expand_fused<false, false, true> : k_sp_expand_fused<false, false, false>));
        FL_LAUNCH("k_sp_expand_fused", kern, grid, dim3(SEL_NT), lds, st, *ori, *inv, h->sp_b, h->sp_l, h->sp_e,
                  h->sp_v, nnz, h->w, h->L, h->n, h->r_size, h->wot_i, h->mode, h->sampling_seed, p.th, p.cut,
                  p.quota, p.item_off, h->entry_order, rcap, holes, x.raw_dst, x.raw_val, x.raw_tie, rp, rc16);
    } else if (nnz > 0 && h->items > 0 && h->chunks > 0) {
        FL_LAUNCH("k_sp_runs", sp_quotas(h) ? k_sp_runs<true> : k_sp_runs<false>,
                  dim3((unsigned)((nnz + SEL_NT / FL_WAVE - 1) / (SEL_NT / FL_WAVE))), dim3(SEL_NT), 0, st, *ori,
                  *inv, h->sp_b, h->sp_l, h->sp_e, h->sp_v, nnz, h->w, h->L, h->n, h->r_size, h->wot_i, h->mode,
                  h->sampling_seed, p.th, p.cut, p.quota, p.item_off, p.chunk_off, h->entry_order, x.runs);
        const int64_t wpb = SP_ITEMS_NT / FL_WAVE;
        const int64_t blocks = (h->chunks + wpb - 1) / wpb;
        const unsigned grid = (unsigned)(blocks < SP_ITEMS_GRID ? blocks : SP_ITEMS_GRID);
        const int holes = h->mode == SP_TOPK && h->aggregate == SP_SUM;
        int32_t *rp = raw_local ? h->raw_pos : (int32_t *)nullptr;
        int16_t *rc16 = raw_local ? h->raw_col : (int16_t *)nullptr;
        if (mx && raw_local)
            FL_LAUNCH("k_sp_items", (k_sp_items<true, true>), dim3(grid), dim3(SP_ITEMS_NT), 0, st, *ori, *inv,
                      h->chunks, x.runs, holes, x.raw_dst, x.raw_val, x.raw_tie, rp, rc16);
        else if (mx)
            FL_LAUNCH("k_sp_items", (k_sp_items<true, false>), dim3(grid), dim3(SP_ITEMS_NT), 0, st, *ori, *inv,
                      h->chunks, x.runs, holes, x.raw_dst, x.raw_val, x.raw_tie, rp, rc16);
        else if (raw_local)
            FL_LAUNCH("k_sp_items", (k_sp_items<false, true>), dim3(grid), dim3(SP_ITEMS_NT), 0, st, *ori, *inv,
                      h->chunks, x.runs, holes, x.raw_dst, x.raw_val, x.raw_tie, rp, rc16);
        else
            FL_LAUNCH("k_sp_items", (k_sp_items<false, false>), dim3(grid), dim3(SP_ITEMS_NT), 0, st, *ori, *inv,
                      h->chunks, x.runs, holes, x.raw_dst, x.raw_val, x.raw_tie, rp, rc16);
    }
    int32_t *dst_arr = x.raw_dst;
    float *val_arr = x.raw_val;
    uint32_t *tie_arr = x.raw_tie;
    if (NB > 1) {
        if (h->tiles > 0)
            FL_LAUNCH("k_sp_hist", k_sp_hist, dim3((unsigned)h->tiles), dim3(SP_NT), sizeof(int) * (size_t)NB, st, R,
                      rows, x.raw_dst, x.hist);
        if (R * NB > 0)
            FL_LAUNCH("k_sp_vscan", k_sp_vscan, dim3((unsigned)((R * NB + 255) / 256)), dim3(256), 0, st, R, rows,
                      x.hist, x.tot);
        if ((rc = exclusive_scan(st, x.tot, x.base, R * NB, x.tmp)) != FL_OK) return rc;
        if (h->tiles > 0)
            FL_LAUNCH("k_sp_partition", k_sp_partition, dim3((unsigned)h->tiles), dim3(SP_PT_NT), 0, st, R, rows,
                      sp_bucket_bits(NB + 1), 31 - sp_bucket_bits(NB), x.base, x.hist, x.raw_dst, x.raw_val,
                      x.part_dst, x.part_val,
                      raw_local ? x.part_inv : (int32_t *)nullptr, x.raw_tie, x.part_tie);
        dst_arr = x.part_dst;
        val_arr = x.part_val;
        tie_arr = x.part_tie;
    }
    // with a backward the accumulation kernels write each item's output index
    // within its bucket at the item's position: the raw map itself when the
    // items were not partitioned, else a partition-order array in the raw
    // value array (dead after the partition), mapped back by k_sp_local_to_out
    int32_t *acc_local = raw_local && NB > 1 ? reinterpret_cast<int32_t *>(x.raw_val) : raw_local;
    // hot buckets (more than one LDS chunk) are listed by the first kernel
    // and taken by a persistent grid of the second.  The persistent grids
    // are no larger than their lists can be (a bucket holds at most the
    // hop's items: at most items / (SP_CHUNK + 1) hot buckets and items /
    // (SP_WB + 1) hot and mid ones), so that a small hop launches a few
    // workgroups, not thousands that find nothing to claim
    const int64_t hot_cap = h->items / (SP_CHUNK + 1) + 1, mid_cap = h->items / (SP_WB + 1) + 1;
    int64_t hot_g = R * NB < SP_HOT_GRID ? R * NB : SP_HOT_GRID;
    if (hot_g > hot_cap) hot_g = hot_cap;
    int64_t mid_g = R * NB < SP_MID_GRID ? R * NB : SP_MID_GRID;
    if (mid_g > mid_cap) mid_g = mid_cap;
    const unsigned hot_grid = (unsigned)hot_g;
    if (R * NB > 0)
        FL_LAUNCH("k_fill_i32", k_fill_i32, dim3(1), dim3(64), 0, st, x.hot_count, (int64_t)8, 0);
    if (R * NB > 0 && mx) {
        FL_LAUNCH("k_sp_max", k_sp_max, dim3((unsigned)(R * NB)), dim3(SP_NT), 0, st, rows, x.base, dst_arr,
                  val_arr, tie_arr, acc_local, x.out_count, x.hot_list, x.hot_count);
        FL_LAUNCH("k_sp_max_hot", k_sp_max_hot, dim3(hot_grid), dim3(SP_NT), 0, st, rows, x.base, dst_arr, val_arr,
                  tie_arr, acc_local, x.out_count, x.hot_list, x.hot_count);
    } else if (R * NB > 0) {
        const int64_t nslot = R * NB;
        FL_LAUNCH("k_sp_accum_small", k_sp_accum_small,
                  dim3((unsigned)((nslot + SP_SMALL_WAVES - 1) / SP_SMALL_WAVES)), dim3(SP_NT), 0, st, rows, x.base,
                  dst_arr, val_arr, acc_local, x.out_count, nslot, x.hot_list, x.mid_list, x.mid_fb, x.hot_count);
        // buckets of more than SP_WB items: few destinations here, the rest
        // on the fallback lists
        FL_LAUNCH("k_sp_accum_few", k_sp_accum_few, dim3((unsigned)mid_g),
                  dim3(SP_NT), 0, st, rows, x.base, dst_arr, val_arr, acc_local, x.out_count, x.hot_list,
                  x.mid_list, x.hot_fb, x.mid_fb, x.hot_count);
        FL_LAUNCH("k_sp_accum_mid", k_sp_accum_mid, dim3((unsigned)mid_g),
                  dim3(SP_NT), 0, st, rows, x.base, dst_arr, val_arr, acc_local, x.out_count, x.mid_fb,
                  x.hot_count + 6);
        FL_LAUNCH("k_sp_accum_hot", k_sp_accum_hot, dim3(hot_grid), dim3(SP_NT), 0, st, rows, x.base, dst_arr,
                  val_arr, acc_local, x.out_count, x.hot_fb, x.hot_count + 4);
    }
    if ((rc = exclusive_scan(st, x.out_count, out_base, R * NB, x.tmp)) != FL_OK) return rc;
    // the backward's map: each raw item's output index
    if (raw_local && h->tiles > 0)
        FL_LAUNCH("k_sp_local_to_out", k_sp_local_to_out, dim3((unsigned)h->tiles), dim3(SP_NT), 0, st, R, rows,
                  x.raw_dst, out_base, x.base, 31 - sp_bucket_bits(NB),
                  NB > 1 ? x.part_inv : (const int32_t *)nullptr, acc_local, raw_local);
    return fl_check_launch("sparse_expand");
}

int fl_sparse_emit(void *stream, const fl_sparse_hop *h, const int64_t *out_base, int64_t *out_b, int64_t *out_l,
                   int64_t *out_e, float *out_v) {
    if (!h || !out_base) return fl_fail(FL_ERR_ARG, "sparse_emit: null argument");
    const int64_t R = h->B * h->L, NB = sp_buckets(h->E);
    if (R * NB == 0) return FL_OK;
    SpPlan p = sp_plan_layout(h->nnz, R, sp_rsize(h), (char *)h->ws1);
    SpExp x = sp_exp_layout(h->items, h->tiles, h->chunks, R, NB, 0, h->aggregate, (char *)h->ws2);
    SpRows rows{p.row_item0, p.tile_base, NB};
    FL_LAUNCH("k_sp_emit", k_sp_emit, dim3((unsigned)((R * NB + SP_EMIT_SLOTS - 1) / SP_EMIT_SLOTS)),
              dim3(SP_EMIT_WAVES * FL_WAVE), 0, (hipStream_t)stream, rows, h->L, R * NB, x.base,
              NB > 1 ? x.part_dst : x.raw_dst, NB > 1 ? x.part_val : x.raw_val, out_base, out_b, out_l, out_e,
              out_v);
    return fl_check_launch("sparse_emit");
}

}  // extern "C"

namespace {

// fl_sparse_backward's workspace: chunk counts / pointers, scan scratch, the
// partial rows and (n > BW_LDS_MAX_N) the waves' rows.
struct SpBwd {
    int64_t *chunk_ptr, *tmp;
    float *part, *wave_rows;
    int64_t blocks;
    size_t bytes;
};

SpBwd sp_bwd_layout(int64_t nnz, int64_t R, int64_t n, char *base) {
    SpBwd x{};
    size_t off = 0;
    auto take = [&](size_t b) { char *q = base ? base + off : nullptr; off += al(b); return q; };
    x.blocks = (nnz + BW_CH - 1) / BW_CH + R;  // at least the number of chunks
    x.chunk_ptr = (int64_t *)take(sizeof(int64_t) * (size_t)(R + 1));
    x.tmp = (int64_t *)take(scan_tmp_bytes(R + 1));
    x.part = (float *)take(sizeof(float) * (size_t)(x.blocks * n));
    x.wave_rows = n > BW_LDS_MAX_N ? (float *)take(sizeof(float) * (size_t)(x.blocks * BW_WAVES * n)) : nullptr;
    x.bytes = off;
    return x;
}

}  // namespace

extern "C" {

size_t fl_sparse_backward_bytes(int64_t nnz, int64_t R, int64_t n) {
    if (nnz < 0 || R < 0 || n < 1) return 0;
    return sp_bwd_layout(nnz, R, n, nullptr).bytes;
}

// The edge-gradient scratch after fl_sparse_backward's own workspace: the
// items' keys and terms, their sorted copies and the sort's scratch.
struct SpEdge {
    uint32_t *key, *skey;
    float *val, *sval;
    void *sort_tmp;
    size_t sort_bytes, bytes;
    int bits;
};

static int sp_key_bits(int64_t keys) {
    int b = 1;
    while (b < 32 && ((int64_t)1 << b) <= keys) ++b;
    return b;
}

static SpEdge sp_edge_layout(int64_t items, int64_t ori_edges, int64_t inv_edges, char *base) {
    SpEdge x{};
    size_t off = 0;
    auto take = [&](size_t b) { char *q = base ? base + off : nullptr; off += al(b); return q; };
    const int64_t n1 = items > 0 ? items : 1;
    x.key = (uint32_t *)take(sizeof(uint32_t) * (size_t)n1);
    x.skey = (uint32_t *)take(sizeof(uint32_t) * (size_t)n1);
    x.val = (float *)take(sizeof(float) * (size_t)n1);
    x.sval = (float *)take(sizeof(float) * (size_t)n1);
    // keys below N = ori_edges + inv_edges < 2^bits: the no-edge key (all
    // ones) has low bits 2^bits - 1 > N - 1, so it sorts last on these bits
    x.bits = sp_key_bits(ori_edges + inv_edges);
    size_t sb = 0;
    if (radix_sort_u32_f32(nullptr, nullptr, &sb, nullptr, nullptr, nullptr, nullptr, n1, x.bits) != FL_OK) sb = 0;
    x.sort_bytes = sb;
    x.sort_tmp = take(sb);
    x.bytes = off;
    return x;
}

size_t fl_sparse_backward_edge_bytes(int64_t items, int64_t ori_edges, int64_t inv_edges) {
    if (items < 0 || ori_edges < 0 || inv_edges < 0) return 0;
    return sp_edge_layout(items, ori_edges, inv_edges, nullptr).bytes;
}

int fl_sparse_backward(void *stream, const fl_side *ori, const fl_side *inv, const fl_sparse_hop *h,
                       const int64_t *out_base, const int32_t *raw_local, const float *grad_out, float *grad_v,
                       float *grad_w, void *workspace, size_t workspace_bytes) {
    int rc;
    if ((rc = sp_check(ori, inv, h, "sparse_backward")) != FL_OK) return rc;
    if (!h->ws1 || !out_base || !grad_v || !grad_w) return fl_fail(FL_ERR_ARG, "sparse_backward: null argument");
    if (h->items > 0 && (!raw_local || !grad_out || !h->raw_col || (!h->raw_pos && !sp_pos_optional(ori, inv, h))))
        return fl_fail(FL_ERR_ARG, "sparse_backward: null raw map (raw_local, raw_pos, raw_col)");
    if (h->items > 0 && !h->raw_pos && (ori->grad_edge || inv->grad_edge))
        return fl_fail(FL_ERR_ARG, "sparse_backward: edge-weight gradients need raw_pos");
    if (h->mode == SP_FIXED) return fl_fail(FL_ERR_ARG, "sparse_backward: the fixed-relation step has no backward");
    const int64_t R = h->B * h->L;
    const bool edge_grads = (ori->grad_edge || inv->grad_edge) && h->items > 0;
    if (edge_grads && ori->edges + inv->edges >= (int64_t)SP_EDGE_NONE)
        return fl_fail(FL_ERR_ARG, "sparse_backward: edge-weight gradients need fewer than 2^32 - 1 positions");
    const size_t own = fl_sparse_backward_bytes(h->nnz, R, h->n);
    const size_t extra = edge_grads ? fl_sparse_backward_edge_bytes(h->items, ori->edges, inv->edges) : 0;
    if (!workspace || workspace_bytes < own + extra)
        return fl_fail(FL_ERR_ARG, "sparse_backward: workspace too small");
    SpPlan p = sp_plan_layout(h->nnz, R, sp_rsize(h), (char *)h->ws1);
    SpBwd x = sp_bwd_layout(h->nnz, R, h->n, (char *)workspace);
    SpEdge eg = sp_edge_layout(h->items, ori->edges, inv->edges, edge_grads ? (char *)workspace + own : nullptr);
    hipStream_t st = (hipStream_t)stream;
    if (R * h->n > 0)
        FL_LAUNCH("k_fill_f32", k_fill_f32, dim3((unsigned)((R * h->n + 255) / 256)), dim3(256), 0, st, grad_w,
                  R * h->n, 0.0f);
    if (h->nnz == 0 || R == 0) return fl_check_launch("sparse_backward");
    FL_LAUNCH("k_sp_bw_chunks", k_sp_bw_chunks, dim3((unsigned)((R + 255) / 256)), dim3(256), 0, st, p.row_ptr, R,
              x.chunk_ptr);
    if ((rc = exclusive_scan(st, x.chunk_ptr, x.chunk_ptr, R, x.tmp)) != FL_OK) return rc;
    const int holes = (h->mode == SP_TOPK && h->aggregate == SP_SUM) ? 1 : 0;
    if (h->n <= BW_LDS_MAX_N)
        FL_LAUNCH("k_sp_bwd", k_sp_bwd<true>, dim3((unsigned)x.blocks), dim3(SEL_NT),
                  sizeof(float) * BW_WAVES * (size_t)h->n, st, *ori, *inv, h->sp_b, h->sp_l, h->sp_v, p.row_ptr,
                  x.chunk_ptr, R, h->w, h->L, h->n, h->r_size, holes, p.item_off, raw_local, h->raw_pos, h->raw_col,
                  grad_out, grad_v, x.wave_rows, x.part, eg.key, eg.val);
    else
        FL_LAUNCH("k_sp_bwd", k_sp_bwd<false>, dim3((unsigned)x.blocks), dim3(SEL_NT), 0, st, *ori, *inv, h->sp_b,
                  h->sp_l, h->sp_v, p.row_ptr, x.chunk_ptr, R, h->w, h->L, h->n, h->r_size, holes, p.item_off,
                  raw_local, h->raw_pos, h->raw_col, grad_out, grad_v, x.wave_rows, x.part, eg.key, eg.val);
    FL_LAUNCH("k_sp_gw_fin", k_sp_gw_fin, dim3((unsigned)((h->n + 255) / 256), (unsigned)R), dim3(256), 0, st,
              x.chunk_ptr, x.part, h->n, grad_w);
    if (edge_grads) {
        size_t sb = eg.sort_bytes;
        if ((rc = radix_sort_u32_f32(st, eg.sort_tmp, &sb, eg.key, eg.skey, eg.val, eg.sval, h->items, eg.bits)) !=
            FL_OK)
            return rc;
        const unsigned g = (unsigned)((h->items + 255) / 256);
        const uint32_t split = (uint32_t)ori->edges, end = (uint32_t)(ori->edges + inv->edges);
        if (ori->grad_edge)
            FL_LAUNCH("k_sp_edge_fold", k_sp_edge_fold, dim3(g), dim3(256), 0, st, eg.skey, eg.sval, h->items,
                      (uint32_t)0, split, ori->order, ori->grad_edge);
        if (inv->grad_edge)
            FL_LAUNCH("k_sp_edge_fold", k_sp_edge_fold, dim3(g), dim3(256), 0, st, eg.skey, eg.sval, h->items, split,
                      end, inv->order, inv->grad_edge);
    }
    return fl_check_launch("sparse_backward");
}

int fl_mask_order_bits(void *stream, const uint8_t *mask, const int32_t *order, int64_t n, uint32_t *edge_bits,
                       uint32_t *bits) {
    if (n < 0 || n > INT32_MAX) return fl_fail(FL_ERR_ARG, "mask_order_bits: bad length");
    if (n == 0) return FL_OK;
    if (!mask || !order || !edge_bits || !bits) return fl_fail(FL_ERR_ARG, "mask_order_bits: null pointer");
    hipStream_t st = (hipStream_t)stream;
    const unsigned g = (unsigned)((n + 255) / 256);
    FL_LAUNCH("k_pack_bool_bits", k_pack_bool_bits, dim3(g), dim3(256), 0, st, mask, n, edge_bits);
    FL_LAUNCH("k_order_bits", k_order_bits, dim3((unsigned)((n + 256 * OB_U - 1) / (256 * OB_U))), dim3(256), 0, st,
              edge_bits, order, n, bits);
    return fl_check_launch("mask_order_bits");
}

int fl_mask_bits(void *stream, const float *mask, int64_t n, uint32_t *bits) {
    if (n < 0) return fl_fail(FL_ERR_ARG, "mask_bits: negative length");
    if (n == 0) return FL_OK;
    if (!mask || !bits) return fl_fail(FL_ERR_ARG, "mask_bits: null pointer");
    FL_LAUNCH("k_mask_bits", k_mask_bits, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, mask,
              n, bits);
    return fl_check_launch("mask_bits");
}

int fl_sparse_topc(void *stream, const int64_t *sp_b, const int64_t *sp_l, const float *v, int64_t nnz, int64_t B,
                   int64_t L, int64_t c, int32_t *keep, int64_t *row_ptr, int64_t *err) {
    if (c < 0) return fl_fail(FL_ERR_ARG, "topk_nodes/c must be nonnegative");
    if (nnz < 0 || B < 0 || L < 0) return fl_fail(FL_ERR_ARG, "sparse_topc: negative size");
    if (!row_ptr || !err || (nnz > 0 && (!sp_b || !sp_l || !v || !keep)))
        return fl_fail(FL_ERR_ARG, "sparse_topc: null argument");
    const int64_t R = B * L;
    hipStream_t st = (hipStream_t)stream;
    FL_LAUNCH("k_fill_i64", k_fill_i64, dim3((unsigned)((R + 1 + 255) / 256)), dim3(256), 0, st, row_ptr, R + 1,
              (int64_t)0);
    FL_LAUNCH("k_fill_i64", k_fill_i64, dim3(1), dim3(64), 0, st, err, (int64_t)1, (int64_t)0);
    const int64_t g1 = (nnz > R + 1 ? nnz : R + 1);
    FL_LAUNCH("k_sp_rowptr", k_sp_rowptr, dim3((unsigned)((g1 + 255) / 256)), dim3(256), 0, st, sp_b, sp_l, sp_b,
              nnz, B, L, INT64_MAX, row_ptr, err);
    if (R > 0 && nnz > 0)
        FL_LAUNCH("k_sp_topc", k_sp_topc, dim3((unsigned)R), dim3(TOPC_NT), 0, st, row_ptr, v, c, keep);
    return fl_check_launch("sparse_topc");
}

// Sampled c1 workspace: row pointer, over flags, candidate flags and
// offsets, order keys, scan scratch.
struct SpRace {
    int64_t *row_ptr, *cand_off, *tmp, *kept, *kept_off;
    int32_t *over, *cand;
    unsigned long long *keys;
    size_t bytes;
};

static SpRace sp_race_layout(int64_t nnz, int64_t R, char *base) {
    SpRace x{};
    size_t off = 0;
    auto take = [&](size_t b) { char *q = base ? base + off : nullptr; off += al(b); return q; };
    const int64_t n1 = nnz > 0 ? nnz : 1;
    x.row_ptr = (int64_t *)take(sizeof(int64_t) * (size_t)(R + 1));
    x.over = (int32_t *)take(sizeof(int32_t) * (size_t)(R > 0 ? R : 1));
    x.kept = (int64_t *)take(sizeof(int64_t) * (size_t)(R > 0 ? R : 1));
    x.kept_off = (int64_t *)take(sizeof(int64_t) * (size_t)(R + 1));
    x.cand = (int32_t *)take(sizeof(int32_t) * (size_t)n1);
    x.cand_off = (int64_t *)take(sizeof(int64_t) * (size_t)(nnz + 1));
    x.keys = (unsigned long long *)take(sizeof(unsigned long long) * (size_t)n1);
    x.tmp = (int64_t *)take(scan_tmp_bytes((nnz > R ? nnz : R) + 1));
    x.bytes = off;
    return x;
}

size_t fl_sparse_race_bytes(int64_t nnz, int64_t R) {
    if (nnz < 0 || R < 0) return 0;
    return sp_race_layout(nnz, R, nullptr).bytes;
}

int fl_sparse_race_plan(void *stream, const int64_t *sp_b, const int64_t *sp_l, const float *v, int64_t nnz,
                        int64_t B, int64_t L, int64_t c, void *ws, size_t ws_bytes, int64_t *info) {
    if (c < 1) return fl_fail(FL_ERR_ARG, "sparse_race: c must be positive (c = 0 needs no ranking)");
    if (nnz < 0 || B < 0 || L < 0) return fl_fail(FL_ERR_ARG, "sparse_race: negative size");
    if (!ws || !info || (nnz > 0 && (!sp_b || !sp_l || !v))) return fl_fail(FL_ERR_ARG, "sparse_race: null argument");
    const int64_t R = B * L;
    if (ws_bytes < fl_sparse_race_bytes(nnz, R)) return fl_fail(FL_ERR_ARG, "sparse_race: workspace too small");
    SpRace x = sp_race_layout(nnz, R, (char *)ws);
    hipStream_t st = (hipStream_t)stream;
    FL_LAUNCH("k_fill_i64", k_fill_i64, dim3(1), dim3(64), 0, st, info, (int64_t)3, (int64_t)0);
    FL_LAUNCH("k_fill_i64", k_fill_i64, dim3((unsigned)((R + 1 + 255) / 256)), dim3(256), 0, st, x.row_ptr, R + 1,
              (int64_t)0);
    const int64_t g1 = (nnz > R + 1 ? nnz : R + 1);
    FL_LAUNCH("k_sp_rowptr", k_sp_rowptr, dim3((unsigned)((g1 + 255) / 256)), dim3(256), 0, st, sp_b, sp_l, sp_b, nnz,
              B, L, INT64_MAX, x.row_ptr, info + 1);
    if (R > 0)
        FL_LAUNCH("k_race_rows", k_race_rows, dim3((unsigned)R), dim3(NM_NT0), 0, st, x.row_ptr, v, c, x.over,
                  x.kept);
    if (nnz > 0)
        FL_LAUNCH("k_race_flags", k_race_flags, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0, st, sp_b, sp_l, v,
                  nnz, L, x.over, x.cand, info + 1);
    int rc;
    if ((rc = exclusive_scan(st, x.cand, x.cand_off, nnz, x.tmp)) != FL_OK) return rc;
    FL_LAUNCH("k_fill_from", k_fill_from, dim3(1), dim3(1), 0, st, x.cand_off + nnz, info);
    if (R > 0) {
        if ((rc = exclusive_scan(st, x.kept, x.kept_off, R, x.tmp)) != FL_OK) return rc;
        FL_LAUNCH("k_fill_from", k_fill_from, dim3(1), dim3(1), 0, st, x.kept_off + R, info + 2);
    }
    return fl_check_launch("sparse_race_plan");
}

int fl_sparse_race_select(void *stream, const float *v, int64_t nnz, int64_t B, int64_t L, int64_t c,
                          const double *noise, void *ws, size_t ws_bytes, int32_t *keep) {
    if (c < 1 || nnz < 0 || B < 0 || L < 0) return fl_fail(FL_ERR_ARG, "sparse_race_select: bad arguments");
    const int64_t R = B * L;
    if (!ws || ws_bytes < fl_sparse_race_bytes(nnz, R)) return fl_fail(FL_ERR_ARG, "sparse_race_select: workspace");
    if (nnz == 0 || R == 0) return FL_OK;
    if (!v || !noise || !keep) return fl_fail(FL_ERR_ARG, "sparse_race_select: null argument");
    SpRace x = sp_race_layout(nnz, R, (char *)ws);
    hipStream_t st = (hipStream_t)stream;
    FL_LAUNCH("k_race_keys", k_race_keys, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0, st, v, nnz, x.cand,
              x.cand_off, noise, x.keys);
    FL_LAUNCH("k_race_select", k_race_select, dim3((unsigned)R), dim3(TOPC_NT), 0, st, x.row_ptr, x.over, x.cand,
              x.keys, c, keep, SpCompact{});
    return fl_check_launch("sparse_race_select");
}

int fl_sparse_race_select_compact(void *stream, const int64_t *sp_b, const int64_t *sp_l, const int64_t *sp_e,
                                  const float *v, int64_t nnz, int64_t B, int64_t L, int64_t c, const double *noise,
                                  void *ws, size_t ws_bytes, int32_t *keep, int64_t *entries, int64_t *out_b,
                                  int64_t *out_l, int64_t *out_e, float *out_v) {
    if (c < 1 || nnz < 0 || B < 0 || L < 0) return fl_fail(FL_ERR_ARG, "sparse_race_select: bad arguments");
    const int64_t R = B * L;
    if (!ws || ws_bytes < fl_sparse_race_bytes(nnz, R)) return fl_fail(FL_ERR_ARG, "sparse_race_select: workspace");
    if (nnz == 0 || R == 0) return FL_OK;
    if (!sp_b || !sp_l || !sp_e || !v || !noise || !keep || !entries || !out_b || !out_l || !out_e || !out_v)
        return fl_fail(FL_ERR_ARG, "sparse_race_select: null argument");
    SpRace x = sp_race_layout(nnz, R, (char *)ws);
    hipStream_t st = (hipStream_t)stream;
    FL_LAUNCH("k_race_keys", k_race_keys, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0, st, v, nnz, x.cand,
              x.cand_off, noise, x.keys);
    const SpCompact cp{sp_b, sp_l, sp_e, v, x.kept_off, entries, out_b, out_l, out_e, out_v};
    FL_LAUNCH("k_race_select", k_race_select, dim3((unsigned)R), dim3(TOPC_NT), 0, st, x.row_ptr, x.over, x.cand,
              x.keys, c, keep, cp);
    return fl_check_launch("sparse_race_select");
}

// the count bins of the entry order: (E >> SP_ORD_SHIFT) + 1 blocks and one
// for out-of-range ids
static int64_t sp_ord_bins(int64_t E) { return (E >> SP_ORD_SHIFT) + 2; }

static size_t sp_order_layout(int64_t nnz, int64_t E, char *base, int32_t **cnt, int32_t **rank, int64_t **start,
                              int64_t **tmp) {
    size_t off = 0;
    auto take = [&](size_t b) { char *q = base ? base + off : nullptr; off += al(b); return q; };
    const int64_t nb = sp_ord_bins(E);
    *cnt = (int32_t *)take(sizeof(int32_t) * (size_t)nb);
    *rank = (int32_t *)take(sizeof(int32_t) * (size_t)(nnz > 0 ? nnz : 1));
    *start = (int64_t *)take(sizeof(int64_t) * (size_t)(nb + 1));
    *tmp = (int64_t *)take(scan_tmp_bytes(nb + 1));
    return off;
}

size_t fl_sparse_entry_order_bytes(int64_t nnz, int64_t E) {
    if (nnz < 0 || E < 0) return 0;
    int32_t *a, *b;
    int64_t *c, *d;
    return sp_order_layout(nnz, E, nullptr, &a, &b, &c, &d);
}

int fl_sparse_entry_order(void *stream, const int64_t *sp_e, int64_t nnz, int64_t E, void *ws, size_t ws_bytes,
                          int32_t *order) {
    if (nnz < 0 || E < 0 || nnz > INT32_MAX) return fl_fail(FL_ERR_ARG, "sparse_entry_order: bad size");
    if (nnz == 0) return FL_OK;
    if (!sp_e || !ws || !order) return fl_fail(FL_ERR_ARG, "sparse_entry_order: null argument");
    if (ws_bytes < fl_sparse_entry_order_bytes(nnz, E)) return fl_fail(FL_ERR_ARG, "sparse_entry_order: workspace");
    int32_t *cnt, *rank;
    int64_t *start, *tmp;
    sp_order_layout(nnz, E, (char *)ws, &cnt, &rank, &start, &tmp);
    hipStream_t st = (hipStream_t)stream;
    const int64_t nb = sp_ord_bins(E);
    FL_LAUNCH("k_fill_i32", k_fill_i32, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, st, cnt, nb, 0);
    FL_LAUNCH("k_sp_ord_count", k_sp_ord_count, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0, st, sp_e, nnz, E,
              cnt, rank);
    int rc;
    if ((rc = exclusive_scan(st, cnt, start, nb, tmp)) != FL_OK) return rc;
    FL_LAUNCH("k_sp_ord_place", k_sp_ord_place, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0, st, sp_e, nnz, E,
              start, rank, order);
    return fl_check_launch("sparse_entry_order");
}

size_t fl_sparse_rowptr_bytes(int64_t R) { return al(sizeof(int64_t) * (size_t)(R + 1)) + al(sizeof(int64_t) * 2); }

int fl_sparse_normalize_forward(void *stream, const int64_t *sp_b, const int64_t *sp_l, const float *v, int64_t nnz,
                                int64_t B, int64_t L, float eps, float *out, float *denom, int64_t *row_ptr,
                                int64_t *err) {
    if (nnz < 0 || B < 0 || L < 0) return fl_fail(FL_ERR_ARG, "sparse_normalize: negative size");
    if (!row_ptr || !err || (nnz > 0 && (!sp_b || !sp_l || !v || !out)) || (B * L > 0 && !denom))
        return fl_fail(FL_ERR_ARG, "sparse_normalize: null argument");
    const int64_t R = B * L;
    hipStream_t st = (hipStream_t)stream;
    // the reference's GPU path checks no order either (flashlog.cu:2594-2649):
    // row starts by binary search, err cleared
    FL_LAUNCH("k_fill_i64", k_fill_i64, dim3(1), dim3(64), 0, st, err, (int64_t)1, (int64_t)0);
    FL_LAUNCH("k_sp_rowptr_search", k_sp_rowptr_search, dim3((unsigned)((R + 1 + 255) / 256)), dim3(256), 0, st,
              sp_b, sp_l, nnz, L, R, row_ptr);
    if (R > 0)
        FL_LAUNCH("k_norm_fwd", k_norm_fwd, dim3((unsigned)R), dim3(NM_NT), 0, st, row_ptr, v, eps, out, denom);
    return fl_check_launch("sparse_normalize");
}

int fl_sparse_gather(void *stream, const int64_t *gb, const int64_t *gl, const int64_t *ge, const float *gv,
                     int64_t ng, const int64_t *qb, const int64_t *ql, const int64_t *qe, int64_t nq, int64_t L,
                     int64_t E, float *out) {
    if (ng < 0 || nq < 0 || L < 1 || E < 0) return fl_fail(FL_ERR_ARG, "sparse_gather: bad shape");
    if (nq == 0) return FL_OK;
    if ((ng > 0 && (!gb || !gl || !ge || !gv)) || !qb || !ql || !qe || !out)
        return fl_fail(FL_ERR_ARG, "sparse_gather: null argument");
    FL_LAUNCH("k_sp_gather", k_sp_gather, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, (hipStream_t)stream, gb,
              gl, ge, gv, ng, qb, ql, qe, nq, L, E, out);
    return fl_check_launch("sparse_gather");
}

int fl_sparse_normalize_backward(void *stream, const int64_t *row_ptr, const float *grad, const float *v,
                                 const float *denom, int64_t R, float eps, float *grad_v) {
    if (R < 0 || !row_ptr) return fl_fail(FL_ERR_ARG, "sparse_normalize_backward: bad arguments");
    if (R > 0)
        FL_LAUNCH("k_norm_bwd", k_norm_bwd, dim3((unsigned)R), dim3(NM_NT), 0, (hipStream_t)stream, row_ptr, grad,
                  v, denom, eps, grad_v);
    return fl_check_launch("sparse_normalize_backward");
}

struct CsLayout {
    int64_t *row_ptr, *err, *hoff, *tmp;
    int32_t *perm, *head;
    size_t bytes;
};

static CsLayout cs_layout(int64_t nnz, int64_t R, char *base) {
    CsLayout x{};
    size_t off = 0;
    auto take = [&](size_t b) { char *q = base ? base + off : nullptr; off += al(b); return q; };
    const int64_t n1 = nnz > 0 ? nnz : 1;
    x.row_ptr = (int64_t *)take(sizeof(int64_t) * (size_t)(R + 1));
    x.err = (int64_t *)take(sizeof(int64_t) * 2);
    x.hoff = (int64_t *)take(sizeof(int64_t) * (size_t)(n1 + 1));
    x.tmp = (int64_t *)take(scan_tmp_bytes(n1 + 1));
    x.perm = (int32_t *)take(sizeof(int32_t) * (size_t)n1);
    x.head = (int32_t *)take(sizeof(int32_t) * (size_t)n1);
    x.bytes = off;
    return x;
}

size_t fl_sparse_channel_sum_bytes(int64_t nnz, int64_t B, int64_t L) {
    if (nnz < 0 || B < 0 || L < 0) return 0;
    return cs_layout(nnz, B * L, nullptr).bytes;
}

int fl_sparse_channel_sum_plan(void *stream, const int64_t *sp_b, const int64_t *sp_l, const int64_t *sp_e,
                               int64_t nnz, int64_t B, int64_t L, int64_t E, void *ws, size_t ws_bytes,
                               int64_t *plan) {
    if (nnz < 0 || B < 0 || L < 0 || E < 0) return fl_fail(FL_ERR_ARG, "sparse_channel_sum: negative size");
    if (nnz > INT32_MAX) return fl_fail(FL_ERR_ARG, "sparse_channel_sum: more than 2^31 - 1 entries");
    if (!ws || !plan || (nnz > 0 && (!sp_b || !sp_l || !sp_e)))
        return fl_fail(FL_ERR_ARG, "sparse_channel_sum: null argument");
    const int64_t R = B * L;
    if (ws_bytes < fl_sparse_channel_sum_bytes(nnz, B, L))
        return fl_fail(FL_ERR_ARG, "sparse_channel_sum: workspace too small");
    CsLayout x = cs_layout(nnz, R, (char *)ws);
    hipStream_t st = (hipStream_t)stream;
    FL_LAUNCH("k_fill_i64", k_fill_i64, dim3((unsigned)((R + 1 + 255) / 256)), dim3(256), 0, st, x.row_ptr, R + 1,
              (int64_t)0);
    FL_LAUNCH("k_fill_i64", k_fill_i64, dim3(1), dim3(64), 0, st, x.err, (int64_t)2, (int64_t)0);
    const int64_t g1 = (nnz > R + 1 ? nnz : R + 1);
    FL_LAUNCH("k_sp_rowptr", k_sp_rowptr, dim3((unsigned)((g1 + 255) / 256)), dim3(256), 0, st, sp_b, sp_l, sp_e,
              nnz, B, L, E, x.row_ptr, x.err);
    if (nnz > 0) {
        FL_LAUNCH("k_fill_i32", k_fill_i32, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0, st, x.head, nnz, 0);
        FL_LAUNCH("k_cs_rank", k_cs_rank, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0, st, sp_b, sp_l, sp_e,
                  nnz, L, R, E, x.row_ptr, x.perm, x.head, x.err);
    }
    int rc = exclusive_scan(st, x.head, x.hoff, nnz, x.tmp);
    if (rc != FL_OK) return rc;
    FL_LAUNCH("k_cs_plan_out", k_cs_plan_out, dim3(1), dim3(64), 0, st, x.hoff, nnz, x.err, plan);
    return fl_check_launch("sparse_channel_sum_plan");
}

int fl_sparse_channel_weighted_add(void *stream, const int64_t *sp_b, const int64_t *sp_l, const int64_t *sp_e,
                                   const float *v, int64_t nnz, int64_t B, int64_t L, int64_t E, const float *W,
                                   int64_t K, void *ws, float *dense) {
    if (nnz < 0 || B < 0 || L < 0 || E < 0 || K < 1)
        return fl_fail(FL_ERR_ARG, "sparse_channel_weighted_add: bad sizes");
    if (nnz == 0) return FL_OK;
    if (!ws || !sp_b || !sp_l || !sp_e || !v || !W || !dense)
        return fl_fail(FL_ERR_ARG, "sparse_channel_weighted_add: null argument");
    CsLayout x = cs_layout(nnz, B * L, (char *)ws);
    FL_LAUNCH("k_cs_weighted_add", k_cs_weighted_add, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0,
              (hipStream_t)stream, sp_b, sp_l, sp_e, v, nnz, x.perm, x.head, W, K, B, E, x.err, dense);
    return fl_check_launch("sparse_channel_weighted_add");
}

int fl_sparse_channel_sum_emit(void *stream, const int64_t *sp_b, const int64_t *sp_e, const float *v, int64_t nnz,
                               int64_t B, int64_t L, int op, void *ws, int64_t nout, int64_t *out_b,
                               int64_t *out_e, float *out_v, int32_t *slot) {
    if (op != 0 && op != 1) return fl_fail(FL_ERR_ARG, "sparse_channel_sum_emit: op must be 0 (sum) or 1 (max)");
    if (nnz < 0 || B < 0 || L < 0 || nout < 0 || nout > nnz)
        return fl_fail(FL_ERR_ARG, "sparse_channel_sum_emit: bad sizes");
    if (!ws || (nnz > 0 && (!sp_b || !sp_e || !v || !slot)) || (nout > 0 && (!out_b || !out_e || !out_v)))
        return fl_fail(FL_ERR_ARG, "sparse_channel_sum_emit: null argument");
    CsLayout x = cs_layout(nnz, B * L, (char *)ws);
    if (nnz > 0)
        FL_LAUNCH("k_cs_emit", op ? k_cs_emit<1> : k_cs_emit<0>, dim3((unsigned)((nnz + 255) / 256)), dim3(256), 0,
                  (hipStream_t)stream, sp_b, sp_e, v, nnz, x.perm, x.head, x.hoff, nout, out_b, out_e, out_v, slot);
    return fl_check_launch("sparse_channel_sum_emit");
}

}  // extern "C"
