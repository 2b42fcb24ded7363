/*
 * grounding_oracle.c -- CPU restatement of FlashLog's soft-grounding sampler.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (flashlog_amd/) links,
 * loads or calls this file; it is compiled into oracle/liboracle.so next to
 * flashlog_oracle.c and used by tests/ as the checker.
 *
 *   or_mt64_*            std::mt19937_64 (the C++ standard's [rand.predef]
 *                        parameters; Matsumoto and Nishimura's MT19937-64)
 *   or_canonical         std::generate_canonical<double, 64> with a 64-bit
 *                        engine as libstdc++ 11 computes it (one draw,
 *                        (double)x / 2^64, values >= 1 clamped below 1)
 *   or_uniform_below     std::uniform_int_distribution with a 64-bit engine
 *                        as libstdc++ 11 computes it (Lemire's nearly
 *                        divisionless method with a 128-bit product)
 *   or_reservoir         soft_grounding.cpp:1029-1124
 *   or_ground_walks      soft_grounding.cpp:57-62,112-250,264-449: the walks
 *                        of every source task as records (body key, positive)
 *
 * The reference draws from the C++ library of its build; the two library
 * algorithms above are the ones of GCC 11's libstdc++ (this image's g++
 * 11.4), whose build of the reference (oracle/_ref) pins them.
 *
 * Pinning: the standard's 10000th-output check of mt19937_64, and bit
 * equality with the reference's own soft_grounding.cpp compiled into
 * oracle/_ref (Makefile.ref) for the reservoir and for whole grounding runs
 * (walk records aggregated by oracle.py's ground_aggregate).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

uint64_t or_splitmix64(uint64_t z);

typedef struct { uint64_t mt[312]; int idx; } or_mt64;

void or_mt64_seed(or_mt64 *g, uint64_t seed)
{
    g->mt[0] = seed;
    for (int i = 1; i < 312; ++i)
        g->mt[i] = 6364136223846793005ULL * (g->mt[i - 1] ^ (g->mt[i - 1] >> 62)) + (uint64_t)i;
    g->idx = 312;
}

static void or_mt64_twist(or_mt64 *g)
{
    const uint64_t upper = 0xFFFFFFFF80000000ULL, lower = 0x7FFFFFFFULL;
    for (int i = 0; i < 312; ++i) {
        uint64_t y = (g->mt[i] & upper) | (g->mt[(i + 1) % 312] & lower);
        uint64_t v = g->mt[(i + 156) % 312] ^ (y >> 1);
        if (y & 1) v ^= 0xB5026F5AA96619E9ULL;
        g->mt[i] = v;
    }
    g->idx = 0;
}

uint64_t or_mt64_next(or_mt64 *g)
{
    if (g->idx >= 312) or_mt64_twist(g);
    uint64_t z = g->mt[g->idx++];
    z ^= (z >> 29) & 0x5555555555555555ULL;
    z ^= (z << 17) & 0x71D67FFFEDA60000ULL;
    z ^= (z << 37) & 0xFFF7EEE000000000ULL;
    z ^= z >> 43;
    return z;
}

/* k-th output (1-based) of an engine seeded with seed. */
uint64_t or_mt64_nth(uint64_t seed, int64_t k)
{
    or_mt64 g;
    or_mt64_seed(&g, seed);
    uint64_t x = 0;
    for (int64_t i = 0; i < k; ++i) x = or_mt64_next(&g);
    return x;
}

double or_canonical(or_mt64 *g)
{
    double r = (double)or_mt64_next(g) * 0x1.0p-64;
    return r >= 1.0 ? nextafter(1.0, 0.0) : r;
}

uint64_t or_uniform_below(or_mt64 *g, uint64_t range)
{
    unsigned __int128 product = (unsigned __int128)or_mt64_next(g) * range;
    uint64_t low = (uint64_t)product;
    if (low < range) {
        uint64_t threshold = (0 - range) % range;
        while (low < threshold) {
            product = (unsigned __int128)or_mt64_next(g) * range;
            low = (uint64_t)product;
        }
    }
    return (uint64_t)(product >> 64);
}

/* ------------------------------------------------------------------------ */
/* Per-relation reservoir of source rows in one pass over the CSR groups
 * (soft_grounding.cpp:1029-1124): sampled [nreq, max_sources] (-1 padded),
 * available[nreq] = groups seen per requested relation.  Returns 0, or -1
 * for a relation outside [0, 32767] or a duplicate.                         */
int or_reservoir(int64_t rows, const int32_t *row_group_ptr, const int16_t *group_rel, int64_t nreq,
                 const int64_t *relations, int64_t max_sources, int64_t seed, int32_t *sampled, int64_t *available)
{
    int32_t *slot_of = (int32_t *)malloc(sizeof(int32_t) * 32768);
    for (int r = 0; r < 32768; ++r) slot_of[r] = -1;
    for (int64_t s = 0; s < nreq; ++s) {
        if (relations[s] < 0 || relations[s] > 32767 || slot_of[relations[s]] != -1) { free(slot_of); return -1; }
        slot_of[relations[s]] = (int32_t)s;
    }
    for (int64_t i = 0; i < nreq * max_sources; ++i) sampled[i] = -1;
    for (int64_t s = 0; s < nreq; ++s) available[s] = 0;
    for (int64_t row = 0; row < rows; ++row) {
        for (int32_t g = row_group_ptr[row]; g < row_group_ptr[row + 1]; ++g) {
            int32_t rel = group_rel[g];
            if (rel < 0) continue;
            int32_t slot = slot_of[rel];
            if (slot < 0) continue;
            uint64_t seen = (uint64_t)(++available[slot]);
            int64_t pos = (int64_t)(seen - 1);
            if (seen > (uint64_t)max_sources) {
                uint64_t rnd = or_splitmix64((uint64_t)seed ^ ((uint64_t)rel << 32) ^ seen);
                pos = (int64_t)(((unsigned __int128)rnd * seen) >> 64);
                if (pos >= max_sources) continue;
            }
            sampled[(int64_t)slot * max_sources + pos] = (int32_t)row;
        }
    }
    for (int64_t s = 0; s < nreq; ++s) {
        int64_t kept = available[s] < max_sources ? available[s] : max_sources;
        uint64_t rel = (uint64_t)relations[s];
        int32_t *o = sampled + s * max_sources;
        for (int64_t i = kept - 1; i > 0; --i) {
            uint64_t rnd = or_splitmix64((uint64_t)seed ^ (rel << 32) ^ 0xd1b54a32d192ed03ULL ^ (uint64_t)i);
            int64_t other = (int64_t)(((unsigned __int128)rnd * (uint64_t)(i + 1)) >> 64);
            int32_t t = o[i]; o[i] = o[other]; o[other] = t;
        }
    }
    free(slot_of);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Attention-guided walks (soft_grounding.cpp:112-250, 264-449).            */
typedef struct {
    const int32_t *col, *ptr, *start, *count;
    const int16_t *rel;
} or_gside;

typedef struct { int32_t op; const int32_t *cols; int32_t take; double mass, cum; } or_gopt;

static double or_proposal(float v, double temperature)
{
    if (temperature == 1.0) return (double)v;
    if (temperature == 2.0) return sqrt((double)v);
    return pow((double)v, 1.0 / temperature);
}

typedef struct { int32_t g; int32_t op; float w; } or_gcand;

static int or_gcand_cmp(const void *a, const void *b)
{
    const or_gcand *x = (const or_gcand *)a, *y = (const or_gcand *)b;
    if (x->w != y->w) return x->w > y->w ? -1 : 1;
    return (x->op > y->op) - (x->op < y->op);
}

/* Options of one side: eligible groups (op != excluded, w > 0, count > 0)
 * by (w desc, op asc), prefixes of up to topk edges in total. */
static int or_side_options(const or_gside *s, int32_t offset, int32_t node, const float *w, int32_t excluded,
                           int64_t topk, double temperature, or_gopt *out, or_gcand *tmp)
{
    int n = 0, k = 0;
    for (int32_t g = s->ptr[node]; g < s->ptr[node + 1]; ++g) {
        int32_t op = (int32_t)s->rel[g] + offset;
        if (op != excluded && w[op] > 0.0f && s->count[g] > 0) { tmp[n].g = g; tmp[n].op = op; tmp[n].w = w[op]; ++n; }
    }
    qsort(tmp, (size_t)n, sizeof(or_gcand), or_gcand_cmp);
    int64_t remaining = topk;
    for (int i = 0; i < n; ++i) {
        if (remaining <= 0) break;
        int32_t g = tmp[i].g;
        int32_t take = (int32_t)(s->count[g] < remaining ? s->count[g] : remaining);
        if (take > 0) {
            out[k].op = tmp[i].op;
            out[k].cols = s->col + s->start[g];
            out[k].take = take;
            out[k].mass = or_proposal(tmp[i].w, temperature) * take;
            ++k;
            remaining -= take;
        }
    }
    return k;
}

/* Walk records of every task: out_key[t * walks + j] = encoded body (0 when
 * the walk is not viable or has no non-identity step), out_pos = 1 when the
 * walk ends at a positive target of (source, head).  rule steps = 3.
 * The task's seed index is task_index[t] (its position within its fold). */
void or_ground_walks(const float *att, int64_t ranks, int64_t vocab, int64_t num_relations, int32_t head,
                     int64_t ntasks, const int64_t *task_source, const int64_t *task_index,
                     const int32_t *ori_col, const int32_t *inv_col, const int32_t *ori_ptr, const int16_t *ori_rel,
                     const int32_t *ori_start, const int32_t *ori_count, const int32_t *inv_ptr,
                     const int16_t *inv_rel, const int32_t *inv_start, const int32_t *inv_count, int64_t walks,
                     int64_t topk_edges, int mask_query_head, int64_t seed, double temperature, int64_t max_groups,
                     uint64_t *out_key, uint8_t *out_pos)
{
    const int steps = 3;
    or_gside fw = {ori_col, ori_ptr, ori_start, ori_count, ori_rel};
    or_gside bw = {inv_col, inv_ptr, inv_start, inv_count, inv_rel};
    const int32_t R = (int32_t)num_relations, identity = 2 * R;
    or_gopt *opts = (or_gopt *)malloc(sizeof(or_gopt) * (size_t)(2 * max_groups + 1));
    or_gcand *tmp = (or_gcand *)malloc(sizeof(or_gcand) * (size_t)(max_groups + 1));
    for (int64_t t = 0; t < ntasks; ++t) {
        int32_t source = (int32_t)task_source[t];
        uint64_t ss = or_splitmix64((uint64_t)seed ^ ((uint64_t)task_index[t] << 32) ^ (uint64_t)(uint32_t)source);
        or_mt64 g;
        or_mt64_seed(&g, ss);
        /* positive targets: the (source, head) group of the head's side */
        const or_gside *hs = head >= R ? &bw : &fw;
        int32_t hrel = head >= R ? head - R : head;
        const int32_t *pcols = NULL;
        int32_t pcount = 0;
        {
            int32_t lo = hs->ptr[source], hi = hs->ptr[source + 1];
            while (lo < hi) { int32_t mid = lo + (hi - lo) / 2; if ((int32_t)hs->rel[mid] < hrel) lo = mid + 1; else hi = mid; }
            if (lo < hs->ptr[source + 1] && (int32_t)hs->rel[lo] == hrel) { pcols = hs->col + hs->start[lo]; pcount = hs->count[lo]; }
        }
        for (int64_t j = 0; j < walks; ++j) {
            int64_t rank = j % ranks;
            int32_t node = source;
            int32_t body[3] = {0, 0, 0};
            int len = 0, viable = 1;
            for (int step = 0; step < steps; ++step) {
                int exclude = mask_query_head && node == source;
                const float *w = att + (step * ranks + rank) * vocab;
                int k = or_side_options(&fw, 0, node, w, exclude ? head : -1, topk_edges, temperature, opts, tmp);
                k += or_side_options(&bw, R, node, w, exclude ? head : -1, topk_edges, temperature, opts + k, tmp);
                if (w[identity] > 0.0f) {
                    opts[k].op = identity; opts[k].cols = NULL; opts[k].take = 1;
                    opts[k].mass = or_proposal(w[identity], temperature);
                    ++k;
                }
                double total = 0.0;
                for (int o = 0; o < k; ++o) { total += opts[o].mass; opts[o].cum = total; }
                if (total <= 0.0) { viable = 0; break; }
                double draw = or_canonical(&g) * total;
                int sel = k - 1;
                for (int o = 0; o < k; ++o) if (draw < opts[o].cum) { sel = o; break; }
                if (opts[sel].op != identity) {
                    uint64_t idx = or_uniform_below(&g, (uint64_t)opts[sel].take);
                    node = opts[sel].cols[idx];
                    body[len++] = opts[sel].op;
                }
            }
            uint64_t key = 0;
            uint8_t pos = 0;
            if (viable && len > 0) {
                const uint64_t m = (1ULL << 20) - 1;
                key = ((uint64_t)len << 60) | (((uint64_t)body[0] & m) << 40) | (((uint64_t)body[1] & m) << 20) |
                      ((uint64_t)body[2] & m);
                for (int32_t q = 0; q < pcount; ++q) pos |= pcols[q] == node;
            }
            out_key[t * walks + j] = key;
            out_pos[t * walks + j] = pos;
        }
    }
    free(opts);
    free(tmp);
}
