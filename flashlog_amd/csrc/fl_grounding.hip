// Soft grounding on gfx950: replaces the CPU module of
// flashlog_kernel/soft_grounding_kernel/source/soft_grounding.cpp.
//
//   reservoir  sample_relation_sources_reservoir (:1029-1124): per requested
//              relation a uniform reservoir of the rows holding a group of
//              that relation, in one pass of CSR group order, then a
//              Fisher-Yates shuffle; all randomness is SplitMix64 of
//              counters, so the pass becomes a stable sort of the groups by
//              relation, a per-position max of occurrence numbers and a
//              per-relation shuffle.
//   walks      ground_head_batch_source_folds_sampled_capped_counts
//              (:112-449, 898-1027): attention-guided walks of rule_steps
//              = 3 steps from every source, one wave per source task with
//              the source's std::mt19937_64 in LDS (the walks of a source
//              share one engine, so they run in order); a walk becomes a
//              record (body key, ends at a positive target).
//   count      per (head, fold) the records are sorted by body key (stable
//              radix sort), runs give walk hits / source hits / positive
//              walk and source hits; per length the rows are ranked by
//              (walk hits desc, key asc) and capped (:454-531); the folds of
//              a head are united by key with totals and minimums (:533-614).
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_segmented_radix_sort.hpp>

#include "fl_abi.h"
#include "fl_common.h"
#include "fl_scan.h"

namespace fl {

// ---------------------------------------------------------------------------
// Random draws: std::mt19937_64 (the C++ standard's [rand.predef]
// parameters) with its state in LDS, one engine per wave, every lane at the
// same position (uniform control flow), and the two library algorithms the
// reference's build uses (libstdc++ 11).

constexpr int MT_N = 312, MT_M = 156;

__device__ void mt_seed(uint64_t *mt, uint64_t seed) {
    const int lane = fl_lane();
    uint64_t x = seed;
    if (lane == 0) mt[0] = x;
    for (int i = 1; i < MT_N; ++i) {
        x = 6364136223846793005ull * (x ^ (x >> 62)) + (uint64_t)i;
        if ((i & (FL_WAVE - 1)) == lane) mt[i] = x;
    }
    __syncthreads();
}

// next word i from mt[i] (a), mt[i+1] (b) and mt[i+m] (c)
__device__ __forceinline__ uint64_t mt_mix(uint64_t a, uint64_t b, uint64_t c) {
    const uint64_t y = (a & 0xFFFFFFFF80000000ull) | (b & 0x7FFFFFFFull);
    return c ^ (y >> 1) ^ ((y & 1ull) ? 0xB5026F5AA96619E9ull : 0ull);
}

// Regeneration in two data-parallel phases: words [0, 156) read only old
// words; words [156, 312) read old words and new words of the first phase.
__device__ void mt_twist(uint64_t *mt) {
    const int lane = fl_lane();
    uint64_t v[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int i = lane + FL_WAVE * k;
        if (i < MT_M) v[k] = mt_mix(mt[i], mt[i + 1], mt[i + MT_M]);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int i = lane + FL_WAVE * k;
        if (i < MT_M) mt[i] = v[k];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int i = MT_M + lane + FL_WAVE * k;
        if (i < MT_N) v[k] = mt_mix(mt[i], mt[i + 1 < MT_N ? i + 1 : 0], mt[i - MT_M]);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int i = MT_M + lane + FL_WAVE * k;
        if (i < MT_N) mt[i] = v[k];
    }
    __syncthreads();
}

__device__ __forceinline__ uint64_t mt_next(uint64_t *mt, int &idx) {
    if (idx >= MT_N) {
        mt_twist(mt);
        idx = 0;
    }
    uint64_t z = mt[idx++];
    z ^= (z >> 29) & 0x5555555555555555ull;
    z ^= (z << 17) & 0x71D67FFFEDA60000ull;
    z ^= (z << 37) & 0xFFF7EEE000000000ull;
    z ^= z >> 43;
    return z;
}

// std::generate_canonical<double, 64> with a 64-bit engine: one draw x,
// (double)x / 2^64 rounded to nearest, values >= 1 clamped below 1.
__device__ __forceinline__ double gr_canonical(uint64_t *mt, int &idx) {
    const double r = __dmul_rn(__ull2double_rn(mt_next(mt, idx)), 0x1.0p-64);
    return r >= 1.0 ? 0x1.fffffffffffffp-1 : r;
}

// std::uniform_int_distribution over [0, range) with a 64-bit engine:
// Lemire's nearly divisionless method with the 128-bit product.
__device__ __forceinline__ uint64_t gr_below(uint64_t *mt, int &idx, uint64_t range) {
    uint64_t x = mt_next(mt, idx);
    uint64_t hi = __umul64hi(x, range), lo = x * range;
    if (lo < range) {
        const uint64_t threshold = (0ull - range) % range;
        while (lo < threshold) {
            x = mt_next(mt, idx);
            hi = __umul64hi(x, range);
            lo = x * range;
        }
    }
    return hi;
}

// ---------------------------------------------------------------------------
// Transition options of a node (soft_grounding.cpp:146-250): per side the
// eligible groups (operator != excluded, weight > 0, edges > 0) by (weight
// desc, operator asc), prefixes of at most topk edges in total, each with
// mass proposal(weight) * take; then the identity operator when its weight
// is positive (mass proposal(weight)).  A node side with at most 64 groups
// is ranked by a bitonic network across the lanes (options stay in
// registers); larger sides are sorted in the wave's scratch.

struct GrSide {
    const int32_t *col, *ptr, *start, *count;
    const int16_t *rel;
};

struct GrGraph {
    GrSide fw, inv;
    int32_t R;
};

__device__ __forceinline__ double gr_proposal(float v, double temperature) {
    if (temperature == 1.0) return (double)v;
    if (temperature == 2.0) return __dsqrt_rn((double)v);
    return pow((double)v, __ddiv_rn(1.0, temperature));
}

// ascending = weight desc, operator asc
__device__ __forceinline__ uint64_t gr_key(float w, int32_t op) {
    return ((uint64_t)(~fl_order_key(w)) << 32) | (uint32_t)op;
}

struct GrOpts {
    int n;          // options (lanes 0..n-1 in register mode)
    int mem;        // options in scratch
    int32_t op, start, take;
    double mass;    // register mode; cumulative mass after gr_cumulate
};

__device__ __forceinline__ GrOpts gr_side_reg(const GrSide &s, int32_t off, int64_t g0, int G, const float *w, int32_t excluded,
                              int64_t topk, double temp) {
    const int lane = fl_lane();
    uint64_t key = ~0ull;
    int32_t g = -1;
    if (lane < G) {
        g = (int32_t)(g0 + lane);
        const int32_t op = (int32_t)s.rel[g] + off;
        const float wv = w[op];
        if (op != excluded && wv > 0.0f && s.count[g] > 0) key = gr_key(wv, op);
    }
#pragma unroll
    for (int k = 2; k <= FL_WAVE; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const uint64_t ok = __shfl_xor(key, j, FL_WAVE);
            const int32_t og = __shfl_xor(g, j, FL_WAVE);
            const bool up = (lane & k) == 0, lower = (lane & j) == 0;
            if ((lower == up) ? (ok < key) : (ok > key)) {
                key = ok;
                g = og;
            }
        }
    const bool el = key != ~0ull;
    const long long cnt = el ? s.count[g] : 0;
    const long long incl = fl_wave_incl_scan_i64(cnt);
    long long take = topk - (incl - cnt);
    take = take < cnt ? take : cnt;
    take = take > 0 ? take : 0;
    GrOpts o;
    o.mem = 0;
    o.op = el ? (int32_t)(key & 0xFFFFFFFFull) : -1;
    o.start = el ? s.start[g] : 0;
    o.take = (int32_t)take;
    o.mass = take > 0 ? __dmul_rn(gr_proposal(w[o.op], temp), (double)take) : 0.0;
    o.n = __popcll(__ballot(take > 0));
    return o;
}

struct GrScratch {
    uint64_t *skey;
    int32_t *sgrp;
    int32_t *oop, *ostart, *otake;
    double *omass;
};

// Hub cache: per (head slot, step, rank) combination c and hub h, the
// node's option lists (fw options, then inv options) with cumulative masses
// at c * nopt + hub_off[h], and the header {fw count, inv count, total}.
struct GrHubHdr {
    int32_t nf, ni;
    double total;
    int64_t off;  // first option slot in the pool
};

struct GrHubPool {
    GrHubHdr *hdr;                // [combos][nhub]
    int32_t *op, *start, *take;   // [combos][nopt]
    double *cum;                  // [combos][nopt]
    const int32_t *hub_id, *hub_node;
    const int64_t *hub_off;
    int64_t nhub, nopt;
};

// Options of a side of up to 64*RR groups (RR keys per lane, element
// i = r*64 + lane): the same bitonic network as the scratch sort, with
// compare-exchanges inside a lane for strides >= 64 and across lanes
// below; keys are distinct (the operator is in the low bits), so the order
// is the same.  Options are written to the scratch lists at o; returns n.
template <int RR>
__device__ __forceinline__ int gr_side_regsort(const GrSide &s, int32_t off, int64_t g0, int64_t G, const float *w,
                                               int32_t excluded, int64_t topk, double temp, const GrScratch &sc,
                                               int o) {
    const int lane = fl_lane();
    uint64_t key[RR];
    int32_t grp[RR];
#pragma unroll
    for (int r = 0; r < RR; ++r) {
        const int64_t i = (int64_t)r * FL_WAVE + lane;
        key[r] = ~0ull;
        grp[r] = -1;
        if (i < G) {
            const int32_t g = (int32_t)(g0 + i);
            const int32_t op = (int32_t)s.rel[g] + off;
            const float wv = w[op];
            if (op != excluded && wv > 0.0f && s.count[g] > 0) key[r] = gr_key(wv, op);
            grp[r] = g;
        }
    }
    constexpr int LOGP = RR == 2 ? 7 : RR == 4 ? 8 : 9;
    static_assert((1 << LOGP) == RR * FL_WAVE, "RR is 2, 4 or 8");
#pragma unroll
    for (int lk = 1; lk <= LOGP; ++lk) {
        const int k = 1 << lk;
#pragma unroll
        for (int lj = lk - 1; lj >= 0; --lj) {
            const int j = 1 << lj;
            if (j >= FL_WAVE) {
                const int jr = j / FL_WAVE;
#pragma unroll
                for (int r = 0; r < RR; ++r) {
                    const int pr = r ^ jr;
                    if (pr > r) {
                        const bool up = (((r * FL_WAVE + lane) & k) == 0);
                        if (up ? (key[r] > key[pr]) : (key[r] < key[pr])) {
                            const uint64_t tk = key[r];
                            key[r] = key[pr];
                            key[pr] = tk;
                            const int32_t tg = grp[r];
                            grp[r] = grp[pr];
                            grp[pr] = tg;
                        }
                    }
                }
            } else {
#pragma unroll
                for (int r = 0; r < RR; ++r) {
                    const uint64_t ok = __shfl_xor(key[r], j, FL_WAVE);
                    const int32_t og = __shfl_xor(grp[r], j, FL_WAVE);
                    const bool up = (((r * FL_WAVE + lane) & k) == 0), lower = (lane & j) == 0;
                    if ((lower == up) ? (ok < key[r]) : (ok > key[r])) {
                        key[r] = ok;
                        grp[r] = og;
                    }
                }
            }
        }
    }
    long long carry = 0;
    int n = 0;
#pragma unroll
    for (int r = 0; r < RR; ++r) {
        if (carry >= topk) break;
        const bool el = key[r] != ~0ull;
        const int32_t g = grp[r];
        const long long cnt = el ? s.count[g] : 0;
        const long long incl = fl_wave_incl_scan_i64(cnt);
        long long take = topk - (carry + incl - cnt);
        take = take < cnt ? take : cnt;
        take = take > 0 ? take : 0;
        if (take > 0) {
            const int32_t op = (int32_t)(key[r] & 0xFFFFFFFFull);
            sc.oop[o + n + lane] = op;
            sc.ostart[o + n + lane] = s.start[g];
            sc.otake[o + n + lane] = (int32_t)take;
            sc.omass[o + n + lane] = __dmul_rn(gr_proposal(w[op], temp), (double)take);
        }
        n += __popcll(__ballot(take > 0));
        carry += __shfl(incl, FL_WAVE - 1, FL_WAVE);
        if (__ballot(el) != ~0ull) break;
    }
    __syncthreads();  // the option lists are visible to every lane
    return n;
}

// Options of a large side written at o (options [o, o + n) of the scratch
// lists).  Returns n.
__device__ __forceinline__ int gr_side_mem(const GrSide &s, int32_t off, int64_t g0, int64_t G, const float *w,
                                           int32_t excluded,
                           int64_t topk, double temp, const GrScratch &sc, int o) {
    const int lane = fl_lane();
    int64_t P = 128;
    while (P < G) P <<= 1;
    __syncthreads();  // earlier reads of the scratch are done
    for (int64_t i = lane; i < P; i += FL_WAVE) {
        uint64_t key = ~0ull;
        int32_t g = -1;
        if (i < G) {
            g = (int32_t)(g0 + i);
            const int32_t op = (int32_t)s.rel[g] + off;
            const float wv = w[op];
            if (op != excluded && wv > 0.0f && s.count[g] > 0) key = gr_key(wv, op);
        }
        sc.skey[i] = key;
        sc.sgrp[i] = g;
    }
    __syncthreads();
    for (int64_t k = 2; k <= P; k <<= 1)
        for (int64_t j = k >> 1; j > 0; j >>= 1) {
            for (int64_t i = lane; i < P; i += FL_WAVE) {
                const int64_t l = i ^ j;
                if (l > i) {
                    const uint64_t a = sc.skey[i], b = sc.skey[l];
                    const bool up = (i & k) == 0;
                    if (up ? (a > b) : (a < b)) {
                        const int32_t ga = sc.sgrp[i], gb = sc.sgrp[l];
                        sc.skey[i] = b;
                        sc.skey[l] = a;
                        sc.sgrp[i] = gb;
                        sc.sgrp[l] = ga;
                    }
                }
            }
            __syncthreads();
        }
    long long carry = 0;
    int n = 0;
    for (int64_t base = 0; base < P && carry < topk; base += FL_WAVE) {
        const uint64_t key = sc.skey[base + lane];
        const bool el = key != ~0ull;
        const int32_t g = sc.sgrp[base + lane];
        const long long cnt = el ? s.count[g] : 0;
        const long long incl = fl_wave_incl_scan_i64(cnt);
        long long take = topk - (carry + incl - cnt);
        take = take < cnt ? take : cnt;
        take = take > 0 ? take : 0;
        if (take > 0) {
            const int32_t op = (int32_t)(key & 0xFFFFFFFFull);
            sc.oop[o + n + lane] = op;
            sc.ostart[o + n + lane] = s.start[g];
            sc.otake[o + n + lane] = (int32_t)take;
            sc.omass[o + n + lane] = __dmul_rn(gr_proposal(w[op], temp), (double)take);
        }
        n += __popcll(__ballot(take > 0));
        carry += __shfl(incl, FL_WAVE - 1, FL_WAVE);
        if (__ballot(el) != ~0ull) break;
    }
    return n;
}

// A side of more than 64 groups: register sort up to 256 groups, else the
// scratch (or LDS) sort.
__device__ __forceinline__ int gr_side_large(const GrSide &s, int32_t off, int64_t g0, int64_t G, const float *w,
                                             int32_t excluded, int64_t topk, double temp, const GrScratch &sc,
                                             int o) {
    if (G <= 2 * FL_WAVE) return gr_side_regsort<2>(s, off, g0, G, w, excluded, topk, temp, sc, o);
    if (G <= 4 * FL_WAVE) return gr_side_regsort<4>(s, off, g0, G, w, excluded, topk, temp, sc, o);
    return gr_side_mem(s, off, g0, G, w, excluded, topk, temp, sc, o);
}

// Cumulative masses in option order (one sequential sum, as the reference):
// register options get their cumulative mass in .mass, scratch options in
// omass.  Returns the running total.
__device__ __forceinline__ double gr_cumulate(GrOpts &o, const GrScratch &sc, int obase, double run, double *mb) {
    // mb: wave-private LDS [64].  Lane j adds the broadcast masses 0..j in
    // order, so its value is the sequential sum up to its option.
    const int lane = fl_lane();
    if (!o.mem) {
        mb[lane] = lane < o.n ? o.mass : 0.0;
        __syncthreads();
        double acc = run;
        for (int i = 0; i < o.n; ++i) {
            const double m = mb[i];
            if (i <= lane) acc = __dadd_rn(acc, m);
        }
        __syncthreads();
        o.mass = lane < o.n ? acc : 0.0;
        return o.n > 0 ? __shfl(acc, o.n - 1, FL_WAVE) : run;
    }
    for (int base = 0; base < o.n; base += FL_WAVE) {
        const int cnt = o.n - base < FL_WAVE ? o.n - base : FL_WAVE;
        mb[lane] = lane < cnt ? sc.omass[obase + base + lane] : 0.0;
        __syncthreads();
        double acc = run;
        for (int i = 0; i < cnt; ++i) {
            const double m = mb[i];
            if (i <= lane) acc = __dadd_rn(acc, m);
        }
        __syncthreads();
        if (lane < cnt) sc.omass[obase + base + lane] = acc;
        run = __shfl(acc, cnt - 1, FL_WAVE);
    }
    __syncthreads();
    return run;
}

// First option of the side with draw < cumulative mass: its index, or -1.
__device__ __forceinline__ int gr_pick(const GrOpts &o, const GrScratch &sc, int obase, double draw) {
    const int lane = fl_lane();
    if (!o.mem) {
        const unsigned long long b = __ballot(lane < o.n && draw < o.mass);
        return b ? __ffsll((long long)b) - 1 : -1;
    }
    // the first four windows of 64 options requested together
    double m[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = u * FL_WAVE + lane;
        m[u] = i < o.n ? sc.omass[obase + i] : 0.0;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = u * FL_WAVE + lane;
        const unsigned long long b = __ballot(i < o.n && draw < m[u]);
        if (b) return u * FL_WAVE + __ffsll((long long)b) - 1;
    }
    for (int base = 4 * FL_WAVE; base < o.n; base += FL_WAVE) {
        const int i = base + lane;
        const unsigned long long b = __ballot(i < o.n && draw < sc.omass[obase + i]);
        if (b) return base + __ffsll((long long)b) - 1;
    }
    return -1;
}

// (op, start, take) of option i of a side
__device__ __forceinline__ void gr_option(const GrOpts &o, const GrScratch &sc, int obase, int i, int32_t *op,
                                          int32_t *start, int32_t *take) {
    if (!o.mem) {
        *op = __shfl(o.op, i, FL_WAVE);
        *start = __shfl(o.start, i, FL_WAVE);
        *take = __shfl(o.take, i, FL_WAVE);
    } else {
        *op = sc.oop[obase + i];
        *start = sc.ostart[obase + i];
        *take = sc.otake[obase + i];
    }
}

constexpr int GR_NT = 64;
constexpr int64_t GR_LDS_SORT_MAX = 4096;  // groups per side sorted in LDS (48 KB)

// Hub cache fill, wave per (combination, hub) (grid-stride): the hub's
// options ranked and their masses accumulated exactly as a walk step does
// (no excluded operator), written to the pool; the sort scratch of large
// sides is the block's walk scratch.
__global__ __launch_bounds__(GR_NT) void k_gr_hubs(GrGraph gg, GrHubPool hp, const float *__restrict__ att,
                                                  int64_t ranks, int64_t vocab, int64_t ncombo, int64_t topk,
                                                  double temp, int64_t pmax, int64_t ocap, char *__restrict__ scratch,
                                                  size_t stride) {
    __shared__ double gr_mb[FL_WAVE];
    const int lane = fl_lane();
    char *ws = scratch + (size_t)blockIdx.x * stride;
    const int32_t R = gg.R;
    for (int64_t u = blockIdx.x; u < ncombo * hp.nhub; u += gridDim.x) {
        const int64_t combo = u / hp.nhub, hid = u - combo * hp.nhub;
        const int32_t node = hp.hub_node[hid];
        const int64_t hslot = combo / (3 * ranks), step = (combo / ranks) % 3, rank = combo % ranks;
        const float *w = att + hslot * 3 * ranks * vocab + (step * ranks + rank) * vocab;
        const int64_t ob = combo * hp.nopt + hp.hub_off[hid];
        GrScratch sc;
        sc.skey = (uint64_t *)ws;
        sc.sgrp = (int32_t *)(sc.skey + pmax);
        sc.oop = hp.op + ob;
        sc.ostart = hp.start + ob;
        sc.otake = hp.take + ob;
        sc.omass = hp.cum + ob;
        (void)ocap;
        const int64_t fg0 = gg.fw.ptr[node], fG = gg.fw.ptr[node + 1] - fg0;
        const int64_t ig0 = gg.inv.ptr[node], iG = gg.inv.ptr[node + 1] - ig0;
        GrOpts fo, io;
        if (fG <= FL_WAVE) {
            fo = gr_side_reg(gg.fw, 0, fg0, (int)fG, w, -1, topk, temp);
            if (lane < fo.n) {
                sc.oop[lane] = fo.op;
                sc.ostart[lane] = fo.start;
                sc.otake[lane] = fo.take;
                sc.omass[lane] = fo.mass;
            }
            fo.mem = 1;
        } else {
            fo.mem = 1;
            fo.n = gr_side_large(gg.fw, 0, fg0, fG, w, -1, topk, temp, sc, 0);
        }
        const int ibase = fo.n;
        if (iG <= FL_WAVE) {
            io = gr_side_reg(gg.inv, R, ig0, (int)iG, w, -1, topk, temp);
            if (lane < io.n) {
                sc.oop[ibase + lane] = io.op;
                sc.ostart[ibase + lane] = io.start;
                sc.otake[ibase + lane] = io.take;
                sc.omass[ibase + lane] = io.mass;
            }
            io.mem = 1;
        } else {
            io.mem = 1;
            io.n = gr_side_large(gg.inv, R, ig0, iG, w, -1, topk, temp, sc, ibase);
        }
        __syncthreads();  // the lists are visible to every lane
        double total = gr_cumulate(fo, sc, 0, 0.0, gr_mb);
        total = gr_cumulate(io, sc, ibase, total, gr_mb);
        const float wid = w[2 * R];
        if (wid > 0.0f) total = __dadd_rn(total, gr_proposal(wid, temp));
        if (lane == 0) {
            GrHubHdr hd;
            hd.nf = fo.n;
            hd.ni = io.n;
            hd.total = total;
            hd.off = ob;
            hp.hdr[combo * hp.nhub + hid] = hd;
        }
        __syncthreads();  // scratch reused by the next hub
    }
}

// One wave per source task (grid-stride over tasks): the task's walks in
// order with the task's engine; record j of task t = (body key, positive).
template <bool LS>
__global__ __launch_bounds__(GR_NT) void k_gr_walk(GrGraph gg, const float *__restrict__ att, int64_t ranks,
                                                  int64_t vocab, const int64_t *__restrict__ heads,
                                                  const int64_t *__restrict__ seeds, int64_t ntasks,
                                                  const int32_t *__restrict__ task_head,
                                                  const int64_t *__restrict__ task_source,
                                                  const int64_t *__restrict__ task_index, int64_t walks,
                                                  int64_t topk, int mask_head, double temp, int64_t pmax,
                                                  int64_t ocap, char *__restrict__ scratch, size_t stride,
                                                  GrHubPool hp, uint64_t *__restrict__ out_key,
                                                  uint8_t *__restrict__ out_pos) {
    __shared__ uint64_t mt[MT_N];
    __shared__ double gr_mb[FL_WAVE];
    extern __shared__ __align__(8) char gr_lds[];  // [pmax] keys + [pmax] groups when lds_sort
    const int lane = fl_lane();
    char *ws = scratch + (size_t)blockIdx.x * stride;
    GrScratch sc;
    sc.skey = (uint64_t *)ws;
    sc.omass = (double *)(sc.skey + pmax);
    sc.sgrp = (int32_t *)(sc.omass + ocap);
    sc.oop = sc.sgrp + pmax;
    sc.ostart = sc.oop + ocap;
    sc.otake = sc.ostart + ocap;
    if (LS) {  // the large-side sort runs in LDS (the option lists stay in the scratch)
        sc.skey = (uint64_t *)gr_lds;
        sc.sgrp = (int32_t *)(sc.skey + pmax);
    }
    const int32_t R = gg.R, identity = 2 * R;
    for (int64_t t = blockIdx.x; t < ntasks; t += gridDim.x) {
        const int32_t hslot = task_head[t];
        const int32_t head = (int32_t)heads[hslot];
        const float *hatt = att + (int64_t)hslot * 3 * ranks * vocab;
        const int32_t source = (int32_t)task_source[t];
        mt_seed(mt, fl_splitmix64((uint64_t)seeds[hslot] ^ ((uint64_t)task_index[t] << 32) ^
                                  (uint64_t)(uint32_t)source));
        int idx = MT_N;
        // positive targets: the (source, head) group of the head's side
        const GrSide &hs = head >= R ? gg.inv : gg.fw;
        const int32_t hrel = head >= R ? head - R : head;
        int32_t plo = hs.ptr[source], phi = hs.ptr[source + 1];
        const int32_t pend = phi;
        while (plo < phi) {
            const int32_t mid = plo + (phi - plo) / 2;
            if ((int32_t)hs.rel[mid] < hrel) plo = mid + 1;
            else phi = mid;
        }
        int64_t pstart = 0, pcount = 0;
        if (plo < pend && (int32_t)hs.rel[plo] == hrel) {
            pstart = hs.start[plo];
            pcount = hs.count[plo];
        }
        const int32_t preg = lane < pcount ? hs.col[pstart + lane] : -1;
        for (int64_t j = 0; j < walks; ++j) {
            const int64_t rank = j % ranks;
            int32_t node = source;
            int32_t body[3] = {0, 0, 0};
            int len = 0;
            bool viable = true;
            for (int step = 0; step < 3; ++step) {
                const int32_t excl = (mask_head && node == source) ? head : -1;
                const float *w = hatt + (step * ranks + rank) * vocab;
                const int32_t hid = (hp.nhub > 0 && excl < 0) ? hp.hub_id[node] : -1;
                const float wid = w[identity];
                GrOpts fo, io;
                GrScratch scs = sc;
                int ibase;
                double total;
                if (hid >= 0) {
                    // a hub: the options this (head, step, rank) gives it, ranked once per call
                    const int64_t combo = ((int64_t)hslot * 3 + step) * ranks + rank;
                    const GrHubHdr hd = hp.hdr[combo * hp.nhub + hid];
                    const int64_t ob = hd.off;
                    scs.oop = hp.op + ob;
                    scs.ostart = hp.start + ob;
                    scs.otake = hp.take + ob;
                    scs.omass = hp.cum + ob;
                    fo.n = hd.nf;
                    fo.mem = 1;
                    io.n = hd.ni;
                    io.mem = 1;
                    ibase = hd.nf;
                    total = hd.total;
                } else {
                    const int64_t fg0 = gg.fw.ptr[node], fG = gg.fw.ptr[node + 1] - fg0;
                    const int64_t ig0 = gg.inv.ptr[node], iG = gg.inv.ptr[node + 1] - ig0;
                    if (fG <= FL_WAVE) {
                        fo = gr_side_reg(gg.fw, 0, fg0, (int)fG, w, excl, topk, temp);
                    } else {
                        fo.mem = 1;
                        fo.n = gr_side_large(gg.fw, 0, fg0, fG, w, excl, topk, temp, sc, 0);
                    }
                    ibase = fo.mem ? fo.n : 0;
                    if (iG <= FL_WAVE) {
                        io = gr_side_reg(gg.inv, R, ig0, (int)iG, w, excl, topk, temp);
                    } else {
                        io.mem = 1;
                        io.n = gr_side_large(gg.inv, R, ig0, iG, w, excl, topk, temp, sc, ibase);
                    }
                    if (fo.mem || io.mem) __syncthreads();
                    total = gr_cumulate(fo, sc, 0, 0.0, gr_mb);
                    total = gr_cumulate(io, sc, ibase, total, gr_mb);
                    if (wid > 0.0f) total = __dadd_rn(total, gr_proposal(wid, temp));
                }
                if (!(total > 0.0)) {
                    viable = false;
                    break;
                }
                const double draw = __dmul_rn(gr_canonical(mt, idx), total);
                int32_t op = identity, start = 0, take = 1;
                int k = gr_pick(fo, scs, 0, draw);
                if (k >= 0) {
                    gr_option(fo, scs, 0, k, &op, &start, &take);
                } else {
                    k = gr_pick(io, scs, ibase, draw);
                    if (k >= 0) gr_option(io, scs, ibase, k, &op, &start, &take);
                    else if (!(wid > 0.0f)) {
                        // none below the draw: the last option
                        if (io.n > 0) gr_option(io, scs, ibase, io.n - 1, &op, &start, &take);
                        else gr_option(fo, scs, 0, fo.n - 1, &op, &start, &take);
                    }
                }
                if (op != identity) {
                    const uint64_t pick = gr_below(mt, idx, (uint64_t)take);
                    node = (op >= R ? gg.inv.col : gg.fw.col)[start + (int64_t)pick];
                    body[len++] = op;
                }
                if (fo.mem || io.mem) __syncthreads();  // scratch reused next step
            }
            uint64_t key = 0;
            bool pos = false;
            if (viable && len > 0) {
                const uint64_t m = (1ull << 20) - 1;
                key = ((uint64_t)len << 60) | (((uint64_t)body[0] & m) << 40) | (((uint64_t)body[1] & m) << 20) |
                      ((uint64_t)body[2] & m);
                if (pcount <= FL_WAVE) {
                    pos = __ballot(preg == node && lane < pcount) != 0;
                } else {
                    for (int64_t q = 0; q < pcount && !pos; q += FL_WAVE)
                        pos = __ballot(q + lane < pcount && hs.col[pstart + q + lane] == node) != 0;
                }
            }
            if (lane == 0) {
                out_key[t * walks + j] = key;
                out_pos[t * walks + j] = pos ? 1 : 0;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Counting (soft_grounding.cpp:427-614).  Records of (head, fold) segment s
// are [seg_off[s], seg_off[s+1]) x walks; after the stable sort by key the
// runs of equal nonzero keys are the fold's bodies.

constexpr int CT_NT = 256;

__device__ __forceinline__ int64_t ct_segment(const int64_t *off, int64_t nseg, int64_t rec) {
    int64_t lo = 0, hi = nseg;  // off[lo] <= rec < off[hi]
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (off[mid] <= rec) lo = mid;
        else hi = mid;
    }
    return lo;
}

// flags of sorted record i: run head (a new nonzero key within its segment)
// and source head (a new task within its run)
__global__ void k_ct_flags(const uint64_t *__restrict__ key, const uint32_t *__restrict__ rec, int64_t n,
                           const int64_t *__restrict__ rec_off, int64_t nseg, int64_t walks,
                           int32_t *__restrict__ run_head, int32_t *__restrict__ src_head) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t k = key[i];
    int rh = 0, sh = 0;
    if (k != 0) {
        const int64_t s = ct_segment(rec_off, nseg, i);
        const bool first = i == rec_off[s] || key[i - 1] != k;
        rh = first ? 1 : 0;
        sh = (first || rec[i - 1] / walks != rec[i] / walks) ? 1 : 0;
    }
    run_head[i] = rh;
    src_head[i] = sh;
}

// per run: key, segment, walk hits, positive walk hits, source hits; per
// source run: any positive
__global__ void k_ct_accum(const uint64_t *__restrict__ key, const uint32_t *__restrict__ rec,
                           const uint8_t *__restrict__ pos, int64_t n, const int64_t *__restrict__ rec_off,
                           int64_t nseg, const int32_t *__restrict__ run_head, const int64_t *__restrict__ run_id,
                           const int32_t *__restrict__ src_head, const int64_t *__restrict__ src_id,
                           uint64_t *__restrict__ rkey, int32_t *__restrict__ rseg,
                           unsigned long long *__restrict__ rcnt, int32_t *__restrict__ src_run,
                           int32_t *__restrict__ src_pos) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n || key[i] == 0) return;
    const int64_t r = run_id[i] + run_head[i] - 1;  // inclusive
    const int64_t q = src_id[i] + src_head[i] - 1;
    const int p = pos[rec[i]];
    if (run_head[i]) {
        rkey[r] = key[i];
        rseg[r] = (int32_t)ct_segment(rec_off, nseg, i);
    }
    if (src_head[i]) {
        src_run[q] = (int32_t)r;
        atomicAdd(&rcnt[4 * r + 1], 1ull);
    }
    atomicAdd(&rcnt[4 * r + 0], 1ull);
    if (p) {
        atomicAdd(&rcnt[4 * r + 2], 1ull);
        atomicMax(&src_pos[q], 1);
    }
}

__global__ void k_ct_srcpos(const int32_t *__restrict__ src_run, const int32_t *__restrict__ src_pos, int64_t nsrc,
                            unsigned long long *__restrict__ rcnt) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (q < nsrc && src_pos[q]) atomicAdd(&rcnt[4 * (int64_t)src_run[q] + 3], 1ull);
}

// cap sort key of run r: segment, length, walk hits descending
__global__ void k_ct_capkey(const uint64_t *__restrict__ rkey, const int32_t *__restrict__ rseg,
                            const unsigned long long *__restrict__ rcnt, int64_t nrun, uint64_t *__restrict__ ckey,
                            uint32_t *__restrict__ cval) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= nrun) return;
    const uint64_t len = rkey[r] >> 60;
    const uint64_t hits = rcnt[4 * r];
    ckey[r] = ((uint64_t)rseg[r] << 34) | (len << 32) | (uint64_t)(0xFFFFFFFFull - hits);
    cval[r] = (uint32_t)r;
}

// kept rows: position within its (segment, length) group below the budget
__global__ void k_ct_keep(const uint64_t *__restrict__ ckey, int64_t nrun, int64_t b1, int64_t b2, int64_t b3,
                          int32_t *__restrict__ keep) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nrun) return;
    const uint64_t grp = ckey[i] >> 32;
    int64_t lo = 0, hi = i;  // first position of the group
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if ((ckey[mid] >> 32) < grp) lo = mid + 1;
        else hi = mid;
    }
    const int len = (int)(grp & 3u);
    const int64_t b = len == 1 ? b1 : (len == 2 ? b2 : b3);
    keep[i] = (i - lo) < b ? 1 : 0;
}

// kept rows in (segment, length, rank) order -> union list (head-major)
__global__ void k_ct_gather(const uint32_t *__restrict__ cval, const int32_t *__restrict__ keep,
                            const int64_t *__restrict__ kept_off, int64_t nrun, const uint64_t *__restrict__ rkey,
                            const int32_t *__restrict__ rseg, const int64_t *__restrict__ seg_head,
                            uint64_t *__restrict__ ukey, uint32_t *__restrict__ urow, int32_t *__restrict__ uhead) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nrun || !keep[i]) return;
    const int64_t o = kept_off[i];
    const uint32_t r = cval[i];
    ukey[o] = rkey[r];
    urow[o] = r;
    uhead[o] = (int32_t)seg_head[rseg[r]];
}

// united rows: per (head, key) run of the key-sorted union list
__global__ void k_ct_uflags(const uint64_t *__restrict__ ukey, const int64_t *__restrict__ uoff, int64_t nheads,
                            int64_t nu, const int64_t *__restrict__ heads, int32_t *__restrict__ uhead_flag) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nu) return;
    const int64_t h = ct_segment(uoff, nheads, i);
    const uint64_t trivial = (1ull << 60) | (((uint64_t)heads[h] & ((1ull << 20) - 1)) << 40);
    const uint64_t k = ukey[i];
    uhead_flag[i] = (k != trivial && (i == uoff[h] || ukey[i - 1] != k)) ? 1 : 0;
}

__global__ void k_ct_emit(const uint64_t *__restrict__ ukey, const uint32_t *__restrict__ urow,
                          const int64_t *__restrict__ uoff, int64_t nheads, int64_t nu,
                          const int64_t *__restrict__ nfolds, const int32_t *__restrict__ uhead_flag,
                          const int64_t *__restrict__ out_id, const unsigned long long *__restrict__ rcnt,
                          int64_t *__restrict__ rows) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nu || !uhead_flag[i]) return;
    const int64_t h = ct_segment(uoff, nheads, i);
    const uint64_t k = ukey[i];
    long long tot[4] = {0, 0, 0, 0}, mn[4];
    int64_t seen = 0;
    for (int64_t q = i; q < uoff[h + 1] && ukey[q] == k; ++q, ++seen) {
        const unsigned long long *c = rcnt + 4 * (int64_t)urow[q];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            tot[m] += (long long)c[m];
            mn[m] = seen == 0 ? (long long)c[m] : ((long long)c[m] < mn[m] ? (long long)c[m] : mn[m]);
        }
    }
    int64_t *row = rows + 12 * out_id[i];
    const uint64_t msk = (1ull << 20) - 1;
    row[0] = (int64_t)(k >> 60);
    row[1] = (int64_t)((k >> 40) & msk);
    row[2] = (int64_t)((k >> 20) & msk);
    row[3] = (int64_t)(k & msk);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        row[4 + m] = tot[m];
        row[8 + m] = seen == nfolds[h] ? mn[m] : 0;
    }
}

// Histogram of a nondecreasing array of bins (entries with flag 0 skipped):
// each wave takes CT_SPAN consecutive entries, counts them per distinct bin
// with ballots and keeps a running (bin, count) pair, so an atomic is issued
// only where the bin changes (instead of one per entry on a few addresses).
constexpr int CT_SPAN = 16 * FL_WAVE;

__global__ void k_ct_sorted_hist(const int32_t *__restrict__ bin, const int32_t *__restrict__ flag, int64_t n,
                                 int64_t *__restrict__ count) {
    const int lane = fl_lane();
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / FL_WAVE;
    const int64_t base = wave * CT_SPAN;
    if (base >= n) return;  // whole wave
    int32_t cur = -1;
    unsigned long long cnt = 0;
    for (int r = 0; r < CT_SPAN / FL_WAVE; ++r) {
        const int64_t i = base + (int64_t)r * FL_WAVE + lane;
        const bool valid = i < n && (!flag || flag[i]);
        const int32_t b = valid ? bin[i] : -1;
        uint64_t left = __ballot(valid);
        while (left) {
            const int32_t k = __shfl(b, __ffsll((long long)left) - 1, FL_WAVE);
            const uint64_t m = __ballot(valid && b == k);
            left &= ~m;
            if (k != cur) {
                if (lane == 0 && cnt) atomicAdd((unsigned long long *)&count[cur], cnt);
                cur = k;
                cnt = 0;
            }
            cnt += (unsigned long long)__popcll(m);
        }
    }
    if (lane == 0 && cnt) atomicAdd((unsigned long long *)&count[cur], cnt);
}

// OR of every body key (the widest relation field sets the packed width)
__global__ void k_ct_or(const uint64_t *__restrict__ keys, int64_t n, unsigned long long *__restrict__ acc) {
    uint64_t v = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        v |= keys[i];
#pragma unroll
    for (int o = FL_WAVE / 2; o > 0; o >>= 1) v |= __shfl_xor(v, o, FL_WAVE);
    if (fl_lane() == 0 && v) atomicOr(acc, (unsigned long long)v);
}

// Sort key of record i: (fold segment, len, body[0..2]) with rb bits per
// relation field, ordered as (segment, body key), so one stable sort of the
// whole batch is the per-segment stable sort by body key.
__global__ void k_ct_pack(const uint64_t *__restrict__ keys, int64_t n, const int64_t *__restrict__ rec_off,
                          int64_t nseg, int rb, uint64_t *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t lo = 0, hi = nseg;  // last s with rec_off[s] <= i
    while (hi - lo > 1) {
        const int64_t mid = (lo + hi) >> 1;
        if (rec_off[mid] <= i) lo = mid;
        else hi = mid;
    }
    const uint64_t k = keys[i], m = (1ull << 20) - 1;
    const uint64_t body = ((k >> 60) << (3 * rb)) | (((k >> 40) & m) << (2 * rb)) | (((k >> 20) & m) << rb) | (k & m);
    out[i] = ((uint64_t)lo << (2 + 3 * rb)) | body;
}

// back to body keys, in place
__global__ void k_ct_unpack(uint64_t *__restrict__ keys, int64_t n, int rb) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t p = keys[i], m = (1ull << rb) - 1;
    keys[i] = (((p >> (3 * rb)) & 3ull) << 60) | (((p >> (2 * rb)) & m) << 40) | (((p >> rb) & m) << 20) | (p & m);
}

// ---------------------------------------------------------------------------
// Reservoir (soft_grounding.cpp:1029-1124).

// row of every group
__global__ void k_rs_rows(const int32_t *__restrict__ ptr, int64_t rows, int32_t *__restrict__ grow) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    for (int32_t g = ptr[r]; g < ptr[r + 1]; ++g) grow[g] = (int32_t)r;
}

// sort key of every group: its requested slot (nreq for the others)
__global__ void k_rs_keys(const int16_t *__restrict__ grel, int64_t G, const int32_t *__restrict__ slot_of,
                          int64_t nreq, uint32_t *__restrict__ key, uint32_t *__restrict__ val) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= G) return;
    const int32_t rel = grel[g];
    const int32_t slot = rel < 0 ? -1 : slot_of[rel];
    key[g] = slot < 0 ? (uint32_t)nreq : (uint32_t)slot;
    val[g] = (uint32_t)g;
}

__global__ void k_rs_slots(const int64_t *__restrict__ rel, int64_t nreq, int32_t *__restrict__ slot_of) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < nreq) slot_of[rel[i]] = (int32_t)i;
}

// sorted position i (slot s, k-th occurrence, 1-based): reservoir position;
// the occurrence with the largest k per position wins
__global__ void k_rs_place(const uint32_t *__restrict__ key, int64_t G, const int64_t *__restrict__ slot_off,
                           const int64_t *__restrict__ rel, int64_t nreq, int64_t max_sources, uint64_t seed,
                           unsigned int *__restrict__ win) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= G) return;
    const uint32_t s = key[i];
    if (s >= (uint32_t)nreq) return;
    const uint64_t seen = (uint64_t)(i - slot_off[s] + 1);
    int64_t p = (int64_t)seen - 1;
    if (seen > (uint64_t)max_sources) {
        const uint64_t rnd = fl_splitmix64(seed ^ ((uint64_t)rel[s] << 32) ^ seen);
        p = (int64_t)__umul64hi(rnd, seen);
        if (p >= max_sources) return;
    }
    atomicMax(&win[s * max_sources + p], (unsigned int)seen);
}

__global__ void k_rs_fill(const unsigned int *__restrict__ win, const uint32_t *__restrict__ val,
                          const int64_t *__restrict__ slot_off, const int32_t *__restrict__ grow, int64_t nreq,
                          int64_t max_sources, int32_t *__restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nreq * max_sources) return;
    const int64_t s = i / max_sources;
    const unsigned int k = win[i];
    out[i] = k ? grow[val[slot_off[s] + k - 1]] : -1;
}

// Fisher-Yates of one slot's kept prefix (sequential; one thread per slot)
__global__ void k_rs_shuffle(const int64_t *__restrict__ slot_off, const int64_t *__restrict__ rel, int64_t nreq,
                             int64_t max_sources, uint64_t seed, int32_t *__restrict__ out,
                             int64_t *__restrict__ available) {
    const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= nreq) return;
    const int64_t n = slot_off[s + 1] - slot_off[s];
    available[s] = n;
    const int64_t kept = n < max_sources ? n : max_sources;
    int32_t *o = out + s * max_sources;
    const uint64_t r = (uint64_t)rel[s];
    for (int64_t i = kept - 1; i > 0; --i) {
        const uint64_t rnd = fl_splitmix64(seed ^ (r << 32) ^ 0xd1b54a32d192ed03ull ^ (uint64_t)i);
        const int64_t other = (int64_t)__umul64hi(rnd, (uint64_t)(i + 1));
        const int32_t t = o[i];
        o[i] = o[other];
        o[other] = t;
    }
}

// slot_off[s] = first sorted position of slot s (lower bound over the sorted keys)
__global__ void k_rs_bounds(const uint32_t *__restrict__ key, int64_t G, int64_t nreq, int64_t *__restrict__ off) {
    const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s > nreq) return;
    int64_t lo = 0, hi = G;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (key[mid] < (uint32_t)s) lo = mid + 1;
        else hi = mid;
    }
    off[s] = lo;
}

__global__ void k_i32_fill(int32_t *__restrict__ p, int64_t n, int32_t v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void k_u32_fill(unsigned int *__restrict__ p, int64_t n, unsigned int v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

__global__ void k_u64_fill(unsigned long long *__restrict__ p, int64_t n, unsigned long long v) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

}  // namespace fl

// ---------------------------------------------------------------------------
// C-ABI

using namespace fl;

namespace {

size_t gal(size_t x) { return (x + 255) & ~(size_t)255; }

unsigned nblk(int64_t n, int nt = CT_NT) { return (unsigned)((n + nt - 1) / nt); }

int gr_rc(hipError_t e, const char *what) {
    return e == hipSuccess ? FL_OK : fl_fail(FL_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

GrGraph gr_graph(const fl_ground_graph *g) {
    GrGraph gg;
    gg.fw = {g->ori_col, g->ori_ptr, g->ori_start, g->ori_count, g->ori_rel};
    gg.inv = {g->inv_col, g->inv_ptr, g->inv_start, g->inv_count, g->inv_rel};
    gg.R = (int32_t)g->num_relations;
    return gg;
}

struct GrWalkLayout {
    int64_t pmax, ocap, waves, ncombo;
    size_t stride, bytes;
    size_t hub_hdr, hub_cum, hub_op, hub_start, hub_take;  // byte offsets of the hub cache (ncombo > 0)
};

GrWalkLayout gr_walk_layout(const fl_ground_graph *g, int64_t ntasks, int64_t nheads, int64_t ranks) {
    GrWalkLayout L{};
    L.pmax = 128;
    while (L.pmax < g->max_groups) L.pmax <<= 1;
    L.ocap = 2 * (g->max_groups > 1 ? g->max_groups : 1);
    L.waves = ntasks < 8192 ? ntasks : 8192;
    L.stride = gal(sizeof(uint64_t) * (size_t)L.pmax + sizeof(double) * (size_t)L.ocap +
                   sizeof(int32_t) * (size_t)L.pmax + 3 * sizeof(int32_t) * (size_t)L.ocap);
    L.bytes = L.stride * (size_t)(L.waves > 0 ? L.waves : 1);
    if (g->nhub > 0 && g->hub_options > 0 && nheads > 0 && ranks > 0) {
        L.ncombo = nheads * 3 * ranks;
        const size_t slots = (size_t)L.ncombo * (size_t)g->hub_options;
        L.hub_hdr = L.bytes;
        L.bytes += gal(sizeof(GrHubHdr) * (size_t)L.ncombo * (size_t)g->nhub);
        L.hub_cum = L.bytes;
        L.bytes += gal(sizeof(double) * slots);
        L.hub_op = L.bytes;
        L.bytes += gal(sizeof(int32_t) * slots);
        L.hub_start = L.bytes;
        L.bytes += gal(sizeof(int32_t) * slots);
        L.hub_take = L.bytes;
        L.bytes += gal(sizeof(int32_t) * slots);
    }
    return L;
}

// count workspace
struct GrCount {
    uint64_t *skey, *rkey, *ckey, *ukey, *ukey2;
    uint32_t *rec_in, *rec, *cval_in, *cval, *urow, *urow2;
    int32_t *run_head, *src_head, *rseg, *src_run, *src_pos, *keep, *uhead, *uflag;
    int64_t *run_id, *src_id, *kept_off, *out_id, *rec_off, *uoff, *head_rows, *tmp;
    unsigned long long *rcnt;
    void *sort_tmp;
    size_t sort_bytes, bytes;
};

size_t gr_sort_tmp(int64_t n, int64_t nseg) {
    size_t a = 0, b = 0, c = 0;
    const unsigned un = (unsigned)(n > 0 ? n : 1);
    (void)rocprim::segmented_radix_sort_pairs(nullptr, a, (const uint64_t *)nullptr, (uint64_t *)nullptr,
                                        (const uint32_t *)nullptr, (uint32_t *)nullptr, un, (unsigned)nseg,
                                        (const int64_t *)nullptr, (const int64_t *)nullptr, 0, 63);
    (void)rocprim::radix_sort_pairs(nullptr, b, (const uint64_t *)nullptr, (uint64_t *)nullptr, (const uint32_t *)nullptr,
                              (uint32_t *)nullptr, un, 0, 64);
    (void)rocprim::radix_sort_pairs(nullptr, c, (const uint32_t *)nullptr, (uint32_t *)nullptr, (const uint32_t *)nullptr,
                              (uint32_t *)nullptr, un, 0, 32);
    size_t m = a > b ? a : b;
    return m > c ? m : c;
}

GrCount gr_count_layout(int64_t n, int64_t nseg, int64_t nheads, char *base) {
    GrCount x{};
    size_t off = 0;
    auto take = [&](size_t b) { char *q = base ? base + off : nullptr; off += gal(b); return q; };
    const size_t n1 = (size_t)(n > 0 ? n : 1);
    x.skey = (uint64_t *)take(8 * n1);
    x.rkey = (uint64_t *)take(8 * n1);
    x.ckey = (uint64_t *)take(8 * n1);
    x.ukey = (uint64_t *)take(8 * n1);
    x.ukey2 = (uint64_t *)take(8 * n1);
    x.rec_in = (uint32_t *)take(4 * n1);
    x.rec = (uint32_t *)take(4 * n1);
    x.cval_in = (uint32_t *)take(4 * n1);
    x.cval = (uint32_t *)take(4 * n1);
    x.urow = (uint32_t *)take(4 * n1);
    x.urow2 = (uint32_t *)take(4 * n1);
    x.run_head = (int32_t *)take(4 * n1);
    x.src_head = (int32_t *)take(4 * n1);
    x.rseg = (int32_t *)take(4 * n1);
    x.src_run = (int32_t *)take(4 * n1);
    x.src_pos = (int32_t *)take(4 * n1);
    x.keep = (int32_t *)take(4 * n1);
    x.uhead = (int32_t *)take(4 * n1);
    x.uflag = (int32_t *)take(4 * n1);
    x.run_id = (int64_t *)take(8 * (n1 + 1));
    x.src_id = (int64_t *)take(8 * (n1 + 1));
    x.kept_off = (int64_t *)take(8 * (n1 + 1));
    x.out_id = (int64_t *)take(8 * (n1 + 1));
    x.rec_off = (int64_t *)take(8 * (size_t)(nseg + 1));
    x.uoff = (int64_t *)take(8 * (size_t)(nheads + 1));
    x.head_rows = (int64_t *)take(8 * (size_t)(nheads + 1));
    x.tmp = (int64_t *)take(scan_tmp_bytes(n + 1));
    x.rcnt = (unsigned long long *)take(32 * n1);
    x.sort_bytes = gr_sort_tmp(n, nseg > nheads ? nseg : nheads);
    x.sort_tmp = take(x.sort_bytes);
    x.bytes = off;
    return x;
}

__global__ void k_iota_u32(uint32_t *p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = (uint32_t)i;
}

__global__ void k_scale_off(const int64_t *__restrict__ task_off, int64_t nseg, int64_t walks,
                            int64_t *__restrict__ rec_off) {
    const int64_t s = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (s <= nseg) rec_off[s] = task_off[s] * walks;
}

__global__ void k_head_bounds(const int32_t *__restrict__ uhead, int64_t nu, int64_t nheads,
                              int64_t *__restrict__ uoff) {
    const int64_t h = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (h > nheads) return;
    int64_t lo = 0, hi = nu;
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (uhead[mid] < (int32_t)h) lo = mid + 1;
        else hi = mid;
    }
    uoff[h] = lo;
}

__global__ void k_copy_i64(const int64_t *__restrict__ src, int64_t *__restrict__ dst) { *dst = *src; }

}  // namespace

extern "C" {

size_t fl_ground_walk_bytes(const fl_ground_graph *g, int64_t ntasks, int64_t nheads, int64_t ranks) {
    if (!g || ntasks < 0 || nheads < 0 || ranks < 0) return 0;
    return gr_walk_layout(g, ntasks, nheads, ranks).bytes;
}

int fl_ground_walks(void *stream, const fl_ground_graph *g, const float *att, int64_t nheads, int64_t ranks,
                    const int64_t *heads, const int64_t *seeds, int64_t ntasks, const int32_t *task_head,
                    const int64_t *task_source, const int64_t *task_index, int64_t walks, int64_t topk_edges,
                    int mask_query_head, double temperature, void *ws, size_t ws_bytes, uint64_t *keys,
                    uint8_t *positive) {
    if (!g || nheads < 0 || ranks < 1 || ntasks < 0 || walks < 1 || topk_edges < 1 || !(temperature > 0.0))
        return fl_fail(FL_ERR_ARG, "ground_walks: bad arguments");
    if (g->num_relations < 1 || 2 * g->num_relations >= (1 << 20))
        return fl_fail(FL_ERR_ARG, "ground_walks: num_relations out of range");
    if (ntasks == 0) return FL_OK;
    if (!att || !heads || !seeds || !task_head || !task_source || !task_index || !keys || !positive || !ws)
        return fl_fail(FL_ERR_ARG, "ground_walks: null argument");
    if (g->nhub > 0 && (!g->hub_id || !g->hub_node || !g->hub_off))
        return fl_fail(FL_ERR_ARG, "ground_walks: hub cache without its arrays");
    const GrWalkLayout L = gr_walk_layout(g, ntasks, nheads, ranks);
    if (ws_bytes < L.bytes) return fl_fail(FL_ERR_ARG, "ground_walks: workspace too small");
    GrHubPool hp{};
    char *wsb = (char *)ws;
    if (L.ncombo > 0) {
        hp.hdr = (GrHubHdr *)(wsb + L.hub_hdr);
        hp.cum = (double *)(wsb + L.hub_cum);
        hp.op = (int32_t *)(wsb + L.hub_op);
        hp.start = (int32_t *)(wsb + L.hub_start);
        hp.take = (int32_t *)(wsb + L.hub_take);
        hp.hub_id = g->hub_id;
        hp.hub_node = g->hub_node;
        hp.hub_off = g->hub_off;
        hp.nhub = g->nhub;
        hp.nopt = g->hub_options;
        const int64_t units = L.ncombo * g->nhub;
        FL_LAUNCH("k_gr_hubs", k_gr_hubs, dim3((unsigned)(units < L.waves ? units : L.waves)), dim3(GR_NT), 0,
                  (hipStream_t)stream, gr_graph(g), hp, att, ranks, 2 * g->num_relations + 1, L.ncombo, topk_edges,
                  temperature, L.pmax, L.ocap, wsb, L.stride);
    }
    // sides of up to GR_LDS_SORT_MAX groups are sorted in LDS, larger ones in the scratch
    const int lds_sort = L.pmax <= GR_LDS_SORT_MAX ? 1 : 0;
    const size_t lds = lds_sort ? (sizeof(uint64_t) + sizeof(int32_t)) * (size_t)L.pmax : 0;
    FL_LAUNCH("k_gr_walk", lds_sort ? k_gr_walk<true> : k_gr_walk<false>, dim3((unsigned)L.waves), dim3(GR_NT), lds,
              (hipStream_t)stream, gr_graph(g), att, ranks, 2 * g->num_relations + 1, heads, seeds, ntasks, task_head,
              task_source, task_index, walks, topk_edges, mask_query_head, temperature, L.pmax, L.ocap, wsb,
              L.stride, hp, keys, positive);
    return fl_check_launch("ground_walks");
}

size_t fl_ground_count_bytes(int64_t nrecords, int64_t nsegments, int64_t nheads) {
    if (nrecords < 0 || nsegments < 0 || nheads < 0) return 0;
    return gr_count_layout(nrecords, nsegments, nheads, nullptr).bytes;
}

int fl_ground_count(void *stream, const uint64_t *keys, const uint8_t *positive, int64_t walks, int64_t nsegments,
                    const int64_t *seg_task_off, const int64_t *seg_head, int64_t nheads, const int64_t *heads,
                    const int64_t *head_folds, const int64_t *budgets, void *ws, size_t ws_bytes, int64_t *rows,
                    int64_t row_cap, int64_t *info) {
    if (walks < 1 || nsegments < 1 || nheads < 1 || !budgets || row_cap < 0)
        return fl_fail(FL_ERR_ARG, "ground_count: bad arguments");
    if (!keys || !positive || !seg_task_off || !seg_head || !heads || !head_folds || !ws || !info)
        return fl_fail(FL_ERR_ARG, "ground_count: null argument");
    if (nsegments >= ((int64_t)1 << 30)) return fl_fail(FL_ERR_ARG, "ground_count: too many folds");
    // the task count was written on the caller's stream: read it there
    int64_t ntasks = 0;
    if (hipMemcpyAsync(&ntasks, seg_task_off + nsegments, sizeof(int64_t), hipMemcpyDeviceToHost,
                       (hipStream_t)stream) != hipSuccess ||
        hipStreamSynchronize((hipStream_t)stream) != hipSuccess)
        return fl_fail(FL_ERR_HIP, "ground_count: reading the task count");
    const int64_t n = ntasks * walks;
    if (n >= ((int64_t)1 << 32)) return fl_fail(FL_ERR_ARG, "ground_count: more than 2^32 walk records");
    GrCount x = gr_count_layout(n, nsegments, nheads, (char *)ws);
    if (ws_bytes < x.bytes) return fl_fail(FL_ERR_ARG, "ground_count: workspace too small");
    hipStream_t st = (hipStream_t)stream;
    int rc;
    // info: [nsegments] raw unique bodies per fold, [nheads + 1] row offsets per head
    FL_LAUNCH("k_u64_fill", k_u64_fill, dim3(nblk(nsegments + nheads + 1)), dim3(CT_NT), 0, st,
              (unsigned long long *)info, nsegments + nheads + 1, 0ull);
    if (n == 0) return fl_check_launch("ground_count");
    FL_LAUNCH("k_scale_off", k_scale_off, dim3(nblk(nsegments + 1)), dim3(CT_NT), 0, st, seg_task_off, nsegments,
              walks, x.rec_off);
    FL_LAUNCH("k_iota_u32", k_iota_u32, dim3(nblk(n)), dim3(CT_NT), 0, st, x.rec_in, n);
    size_t sb = x.sort_bytes;
    // width of the relation fields from the OR of all keys
    unsigned long long kor = 0;
    FL_LAUNCH("k_u64_fill", k_u64_fill, dim3(1), dim3(CT_NT), 0, st, x.rcnt, (int64_t)1, 0ull);
    FL_LAUNCH("k_ct_or", k_ct_or, dim3((unsigned)std::min<int64_t>(nblk(n), 2048)), dim3(CT_NT), 0, st, keys, n,
              x.rcnt);
    if (hipMemcpyAsync(&kor, x.rcnt, sizeof(kor), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return fl_fail(FL_ERR_HIP, "ground_count: reading the key width");
    const uint64_t fields = ((kor >> 40) | (kor >> 20) | kor) & ((1ull << 20) - 1);
    const int rb = fields ? 64 - __builtin_clzll(fields) : 1;
    const int segbits = nsegments > 1 ? 64 - __builtin_clzll((unsigned long long)(nsegments - 1)) : 0;
    const int tb = segbits + 2 + 3 * rb;
    if (tb <= 64) {
        FL_LAUNCH("k_ct_pack", k_ct_pack, dim3(nblk(n)), dim3(CT_NT), 0, st, keys, n, x.rec_off, nsegments, rb,
                  x.rkey);
        if ((rc = gr_rc(rocprim::radix_sort_pairs(x.sort_tmp, sb, x.rkey, x.skey, x.rec_in, x.rec, (unsigned)n, 0,
                                                  (unsigned)tb, st),
                        "ground_count: record sort")) != FL_OK)
            return rc;
        FL_LAUNCH("k_ct_unpack", k_ct_unpack, dim3(nblk(n)), dim3(CT_NT), 0, st, x.skey, n, rb);
    } else if ((rc = gr_rc(rocprim::segmented_radix_sort_pairs(x.sort_tmp, sb, keys, x.skey, x.rec_in, x.rec,
                                                               (unsigned)n, (unsigned)nsegments, x.rec_off,
                                                               x.rec_off + 1, 0, 63, st),
                           "ground_count: record sort")) != FL_OK) {
        return rc;
    }
    FL_LAUNCH("k_ct_flags", k_ct_flags, dim3(nblk(n)), dim3(CT_NT), 0, st, x.skey, x.rec, n, x.rec_off, nsegments,
              walks, x.run_head, x.src_head);
    if ((rc = exclusive_scan(st, x.run_head, x.run_id, n, x.tmp)) != FL_OK) return rc;
    if ((rc = exclusive_scan(st, x.src_head, x.src_id, n, x.tmp)) != FL_OK) return rc;
    int64_t nrun = 0, nsrc = 0;
    if (hipMemcpyAsync(&nrun, x.run_id + n, sizeof(int64_t), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipMemcpyAsync(&nsrc, x.src_id + n, sizeof(int64_t), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return fl_fail(FL_ERR_HIP, "ground_count: reading run counts");
    if (nrun == 0) return fl_check_launch("ground_count");
    FL_LAUNCH("k_u64_fill", k_u64_fill, dim3(nblk(4 * nrun)), dim3(CT_NT), 0, st, x.rcnt, 4 * nrun, 0ull);
    FL_LAUNCH("k_i32_fill", k_i32_fill, dim3(nblk(nsrc)), dim3(CT_NT), 0, st, x.src_pos, nsrc, 0);
    FL_LAUNCH("k_ct_accum", k_ct_accum, dim3(nblk(n)), dim3(CT_NT), 0, st, x.skey, x.rec, positive, n, x.rec_off,
              nsegments, x.run_head, x.run_id, x.src_head, x.src_id, x.rkey, x.rseg, x.rcnt, x.src_run, x.src_pos);
    FL_LAUNCH("k_ct_srcpos", k_ct_srcpos, dim3(nblk(nsrc)), dim3(CT_NT), 0, st, x.src_run, x.src_pos, nsrc, x.rcnt);
    // cap: stable sort of the runs by (segment, length, walk hits desc)
    FL_LAUNCH("k_ct_capkey", k_ct_capkey, dim3(nblk(nrun)), dim3(CT_NT), 0, st, x.rkey, x.rseg, x.rcnt, nrun, x.ckey,
              x.cval_in);
    uint64_t *ckey_sorted = x.ukey2;
    sb = x.sort_bytes;
    if ((rc = gr_rc(rocprim::radix_sort_pairs(x.sort_tmp, sb, x.ckey, ckey_sorted, x.cval_in, x.cval, (unsigned)nrun,
                                              0, 64, st),
                    "ground_count: cap sort")) != FL_OK)
        return rc;
    FL_LAUNCH("k_ct_keep", k_ct_keep, dim3(nblk(nrun)), dim3(CT_NT), 0, st, ckey_sorted, nrun, budgets[0], budgets[1],
              budgets[2], x.keep);
    if ((rc = exclusive_scan(st, x.keep, x.kept_off, nrun, x.tmp)) != FL_OK) return rc;
    int64_t nu = 0;
    if (hipMemcpyAsync(&nu, x.kept_off + nrun, sizeof(int64_t), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return fl_fail(FL_ERR_HIP, "ground_count: reading kept rows");
    FL_LAUNCH("k_ct_gather", k_ct_gather, dim3(nblk(nrun)), dim3(CT_NT), 0, st, x.cval, x.keep, x.kept_off, nrun,
              x.rkey, x.rseg, seg_head, x.ukey, x.urow, x.uhead);
    FL_LAUNCH("k_head_bounds", k_head_bounds, dim3(nblk(nheads + 1)), dim3(CT_NT), 0, st, x.uhead, nu, nheads,
              x.uoff);
    if (nu > 0) {
        sb = x.sort_bytes;
        if ((rc = gr_rc(rocprim::segmented_radix_sort_pairs(x.sort_tmp, sb, x.ukey, x.ukey2, x.urow, x.urow2,
                                                            (unsigned)nu, (unsigned)nheads, x.uoff, x.uoff + 1, 0,
                                                            63, st),
                        "ground_count: union sort")) != FL_OK)
            return rc;
        FL_LAUNCH("k_ct_uflags", k_ct_uflags, dim3(nblk(nu)), dim3(CT_NT), 0, st, x.ukey2, x.uoff, nheads, nu, heads,
                  x.uflag);
        if ((rc = exclusive_scan(st, x.uflag, x.out_id, nu, x.tmp)) != FL_OK) return rc;
        int64_t nrows = 0;
        if (hipMemcpyAsync(&nrows, x.out_id + nu, sizeof(int64_t), hipMemcpyDeviceToHost, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess)
            return fl_fail(FL_ERR_HIP, "ground_count: reading row count");
        if (nrows > row_cap) return fl_fail(FL_ERR_ARG, "ground_count: row buffer too small (%lld rows)",
                                            (long long)nrows);
        if (!rows && nrows > 0) return fl_fail(FL_ERR_ARG, "ground_count: null rows");
        FL_LAUNCH("k_ct_emit", k_ct_emit, dim3(nblk(nu)), dim3(CT_NT), 0, st, x.ukey2, x.urow2, x.uoff, nheads, nu,
                  head_folds, x.uflag, x.out_id, x.rcnt, rows);
    }
    FL_LAUNCH("k_u64_fill", k_u64_fill, dim3(nblk(nheads + 1)), dim3(CT_NT), 0, st,
              (unsigned long long *)x.head_rows, nheads + 1, 0ull);
    const auto hist_blocks = [](int64_t m) { return dim3((unsigned)((m + CT_SPAN * (CT_NT / FL_WAVE) - 1) /
                                                                    (CT_SPAN * (CT_NT / FL_WAVE)))); };
    if (nrun > 0)
        FL_LAUNCH("k_ct_sorted_hist", k_ct_sorted_hist, hist_blocks(nrun), dim3(CT_NT), 0, st, x.rseg,
                  (const int32_t *)nullptr, nrun, info);
    if (nu > 0)
        FL_LAUNCH("k_ct_sorted_hist", k_ct_sorted_hist, hist_blocks(nu), dim3(CT_NT), 0, st, x.uhead, x.uflag, nu,
                  x.head_rows);
    // row offsets per head: exclusive scan of the per-head row counts
    if ((rc = exclusive_scan(st, x.head_rows, info + nsegments, nheads, x.tmp)) != FL_OK) return rc;
    return fl_check_launch("ground_count");
}

size_t fl_reservoir_bytes(int64_t groups, int64_t rows, int64_t nreq, int64_t max_sources) {
    if (groups < 0 || rows < 0 || nreq < 0 || max_sources < 1) return 0;
    const size_t g1 = (size_t)(groups > 0 ? groups : 1);
    size_t sb = 0;
    (void)rocprim::radix_sort_pairs(nullptr, sb, (const uint32_t *)nullptr, (uint32_t *)nullptr, (const uint32_t *)nullptr,
                              (uint32_t *)nullptr, (unsigned)g1, 0, 32);
    return gal(4 * 32768) + 4 * gal(4 * g1) + gal(4 * g1) + gal(8 * (size_t)(nreq + 1)) +
           gal(4 * (size_t)(nreq > 0 ? nreq : 1) * (size_t)max_sources) + gal(sb);
}

int fl_reservoir(void *stream, const int32_t *row_group_ptr, int64_t rows, const int16_t *group_rel, int64_t groups,
                 const int64_t *relations, int64_t nreq, int64_t max_sources, int64_t seed, void *ws,
                 size_t ws_bytes, int32_t *sampled, int64_t *available) {
    if (rows < 0 || groups < 0 || nreq < 0 || max_sources < 1) return fl_fail(FL_ERR_ARG, "reservoir: bad arguments");
    if (nreq == 0) return FL_OK;
    if (!sampled || !available || !ws || (groups > 0 && (!row_group_ptr || !group_rel)) || !relations)
        return fl_fail(FL_ERR_ARG, "reservoir: null argument");
    if (ws_bytes < fl_reservoir_bytes(groups, rows, nreq, max_sources))
        return fl_fail(FL_ERR_ARG, "reservoir: workspace too small");
    if (groups >= ((int64_t)1 << 31)) return fl_fail(FL_ERR_ARG, "reservoir: too many groups");
    hipStream_t st = (hipStream_t)stream;
    const size_t g1 = (size_t)(groups > 0 ? groups : 1);
    char *p = (char *)ws;
    int32_t *slot_of = (int32_t *)p; p += gal(4 * 32768);
    uint32_t *kin = (uint32_t *)p; p += gal(4 * g1);
    uint32_t *kout = (uint32_t *)p; p += gal(4 * g1);
    uint32_t *vin = (uint32_t *)p; p += gal(4 * g1);
    uint32_t *vout = (uint32_t *)p; p += gal(4 * g1);
    int32_t *grow = (int32_t *)p; p += gal(4 * g1);
    int64_t *slot_off = (int64_t *)p; p += gal(8 * (size_t)(nreq + 1));
    unsigned int *win = (unsigned int *)p; p += gal(4 * (size_t)nreq * (size_t)max_sources);
    void *sort_tmp = p;
    size_t sb = 0;
    (void)rocprim::radix_sort_pairs(nullptr, sb, (const uint32_t *)nullptr, (uint32_t *)nullptr, (const uint32_t *)nullptr,
                              (uint32_t *)nullptr, (unsigned)g1, 0, 32);
    FL_LAUNCH("k_u32_fill", k_u32_fill, dim3(nblk(nreq * max_sources)), dim3(CT_NT), 0, st, win, nreq * max_sources,
              0u);
    if (groups == 0) {
        FL_LAUNCH("k_i32_fill", k_i32_fill, dim3(nblk(nreq * max_sources)), dim3(CT_NT), 0, st, sampled,
                  nreq * max_sources, -1);
        FL_LAUNCH("k_u64_fill", k_u64_fill, dim3(nblk(nreq)), dim3(CT_NT), 0, st, (unsigned long long *)available,
                  nreq, 0ull);
        return fl_check_launch("reservoir");
    }
    FL_LAUNCH("k_i32_fill", k_i32_fill, dim3(nblk(32768)), dim3(CT_NT), 0, st, slot_of, (int64_t)32768, -1);
    FL_LAUNCH("k_rs_slots", k_rs_slots, dim3(nblk(nreq)), dim3(CT_NT), 0, st, relations, nreq, slot_of);
    FL_LAUNCH("k_rs_rows", k_rs_rows, dim3(nblk(rows)), dim3(CT_NT), 0, st, row_group_ptr, rows, grow);
    FL_LAUNCH("k_rs_keys", k_rs_keys, dim3(nblk(groups)), dim3(CT_NT), 0, st, group_rel, groups, slot_of, nreq, kin,
              vin);
    int bits = 1;
    while (((int64_t)1 << bits) <= nreq) ++bits;
    int rc;
    if ((rc = gr_rc(rocprim::radix_sort_pairs(sort_tmp, sb, kin, kout, vin, vout, (unsigned)groups, 0, bits, st),
                    "reservoir: sort")) != FL_OK)
        return rc;
    FL_LAUNCH("k_rs_bounds", k_rs_bounds, dim3(nblk(nreq + 1)), dim3(CT_NT), 0, st, kout, groups, nreq, slot_off);
    FL_LAUNCH("k_rs_place", k_rs_place, dim3(nblk(groups)), dim3(CT_NT), 0, st, kout, groups, slot_off, relations,
              nreq, max_sources, (uint64_t)seed, win);
    FL_LAUNCH("k_rs_fill", k_rs_fill, dim3(nblk(nreq * max_sources)), dim3(CT_NT), 0, st, win, vout, slot_off, grow,
              nreq, max_sources, sampled);
    FL_LAUNCH("k_rs_shuffle", k_rs_shuffle, dim3(nblk(nreq, 64)), dim3(64), 0, st, slot_off, relations, nreq,
              max_sources, (uint64_t)seed, sampled, available);
    return fl_check_launch("reservoir");
}

}  // extern "C"
