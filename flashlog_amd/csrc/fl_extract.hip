// Rank weights of extracted rule candidates (rules/extract.py:65-135) and
// their selection statistics (rules/extract.py:148-201).
//
// A candidate row is [length, op_1 .. op_T, ..., trials (col W-8), ...,
// positives (col W-6), ...] (int64).  For attention a[h, s, c, o] of the
// row's head h (steps s < T, channels c < L, operators o < n; float or
// double, taken as double), the weight of channel c is the sum (or max)
// over the placements of the body's operators into the T steps, in order,
// of the product of the attention of each step: the operator placed there
// or the identity.  The reference evaluates it two ways, reproduced here
// operation for operation in double precision (no contraction):
//   mode 0 (T == 3): the closed form per length (extract.py:65-105),
//   mode 1 / 2: the dynamic program over (step, placed operators) with sums
//               or maxima (extract.py:108-129).
// Then per row: the sum of its L weights in numpy's pairwise order (the
// row sums rank_weights.sum(axis=1) of extract.py:130,189) and the
// precision positives / trials (0 when trials == 0, extract.py:181-187).
#include "fl_abi.h"
#include "fl_common.h"

namespace fl {
namespace {

constexpr int EX_NT = 256;
constexpr int EX_MAX_T = 16;
constexpr int EX_MAX_L = 128;

__device__ __forceinline__ double dmul(double a, double b) { return __dmul_rn(a, b); }
__device__ __forceinline__ double dadd(double a, double b) { return __dadd_rn(a, b); }

template <typename T>
__device__ __forceinline__ double att_at(const T *att, int64_t base, int64_t s, int64_t c, int64_t o, int64_t L,
                                         int64_t n) {
    return (double)att[base + (s * L + c) * n + o];
}

// numpy's np.maximum: the first argument when it is >= the second or NaN.
__device__ __forceinline__ double np_max(double a, double b) { return (a >= b || a != a) ? a : b; }

// Operator index as numpy reads it: -n <= o < n, negatives from the end.
__device__ __forceinline__ bool wrap_op(int64_t &o, int64_t n) {
    if (o < -n || o >= n) return false;
    if (o < 0) o += n;
    return true;
}

template <typename T>
__global__ __launch_bounds__(EX_NT) void k_rank_weights(const T *__restrict__ att, const int64_t *__restrict__ rows,
                                                        const int64_t *__restrict__ row_head, int64_t N, int64_t W,
                                                        int64_t H, int64_t Ts, int64_t L, int64_t n, int64_t ident,
                                                        int mode, double *__restrict__ rw, int64_t *__restrict__ err) {
    const int64_t q = (int64_t)blockIdx.x * EX_NT + threadIdx.x;
    if (q >= N * L) return;
    const int64_t r = q / L, c = q - r * L;
    const int64_t *row = rows + r * W;
    const int64_t len = row[0];
    const int64_t h = row_head ? row_head[r] : 0;
    double out = 0.0;
    if (h < 0 || h >= H) {
        atomicMax((unsigned long long *)err, 2ull);
        rw[q] = 0.0;
        return;
    }
    const int64_t base = h * Ts * L * n;
    if (len >= 1 && len <= Ts) {
        int64_t ops[EX_MAX_T];
        for (int64_t p = 0; p < len; ++p) {
            int64_t o = row[1 + p];
            if (!wrap_op(o, n)) {
                atomicMax((unsigned long long *)err, 1ull);
                rw[q] = 0.0;
                return;
            }
            ops[p] = o;
        }
        if (mode == 0) {
            const double i0 = att_at(att, base, 0, c, ident, L, n), i1 = att_at(att, base, 1, c, ident, L, n),
                         i2 = att_at(att, base, 2, c, ident, L, n);
            if (len == 1) {
                const double v0 = att_at(att, base, 0, c, ops[0], L, n), v1 = att_at(att, base, 1, c, ops[0], L, n),
                             v2 = att_at(att, base, 2, c, ops[0], L, n);
                out = dadd(dadd(dmul(dmul(v0, i1), i2), dmul(dmul(i0, v1), i2)), dmul(dmul(i0, i1), v2));
            } else if (len == 2) {
                const double f0 = att_at(att, base, 0, c, ops[0], L, n), f1 = att_at(att, base, 1, c, ops[0], L, n);
                const double s1 = att_at(att, base, 1, c, ops[1], L, n), s2 = att_at(att, base, 2, c, ops[1], L, n);
                out = dadd(dadd(dmul(dmul(f0, s1), i2), dmul(dmul(f0, i1), s2)), dmul(dmul(i0, f1), s2));
            } else {
                out = dmul(dmul(att_at(att, base, 0, c, ops[0], L, n), att_at(att, base, 1, c, ops[1], L, n)),
                           att_at(att, base, 2, c, ops[2], L, n));
            }
        } else {
            // dp[p]: weight of having placed the first p operators
            double dp[EX_MAX_T + 1], nx[EX_MAX_T + 1];
            dp[0] = 1.0;
            for (int64_t p = 1; p <= len; ++p) dp[p] = 0.0;
            for (int64_t s = 0; s < Ts; ++s) {
                const double id = att_at(att, base, s, c, ident, L, n);
                for (int64_t p = 0; p <= len; ++p) nx[p] = dmul(dp[p], id);
                const int64_t top = len < s + 1 ? len : s + 1;
                for (int64_t p = 1; p <= top; ++p) {
                    const double contrib = dmul(dp[p - 1], att_at(att, base, s, c, ops[p - 1], L, n));
                    nx[p] = mode == 2 ? np_max(nx[p], contrib) : dadd(nx[p], contrib);
                }
                for (int64_t p = 0; p <= len; ++p) dp[p] = nx[p];
            }
            out = dp[len];
        }
    }
    rw[q] = out;
}

// numpy's row sum of n contiguous doubles (n <= 128: one block of its
// pairwise summation), added to the reduction's initial 0.0 (so that a row of
// negative zeros sums to +0.0 as in numpy).
__device__ double np_pairwise_sum(const double *a, int64_t n) {
    if (n < 8) {
        double res = 0.0;
        for (int64_t i = 0; i < n; ++i) res = dadd(res, a[i]);
        return res;
    }
    double r[8];
    for (int j = 0; j < 8; ++j) r[j] = a[j];
    int64_t i = 8;
    for (; i < n - (n % 8); i += 8)
        for (int j = 0; j < 8; ++j) r[j] = dadd(r[j], a[i + j]);
    double res = dadd(dadd(dadd(r[0], r[1]), dadd(r[2], r[3])), dadd(dadd(r[4], r[5]), dadd(r[6], r[7])));
    for (; i < n; ++i) res = dadd(res, a[i]);
    return dadd(0.0, res);
}

__global__ __launch_bounds__(EX_NT) void k_rank_stats(const double *__restrict__ rw, const int64_t *__restrict__ rows,
                                                      int64_t N, int64_t W, int64_t L, double *__restrict__ rwsum,
                                                      double *__restrict__ precision) {
    const int64_t r = (int64_t)blockIdx.x * EX_NT + threadIdx.x;
    if (r >= N) return;
    if (rwsum) rwsum[r] = np_pairwise_sum(rw + r * L, L);
    if (precision) {
        const double trials = __ll2double_rn(rows[r * W + W - 8]);
        const double pos = __ll2double_rn(rows[r * W + W - 6]);
        precision[r] = trials != 0.0 ? __ddiv_rn(pos, trials) : 0.0;
    }
}

__global__ void k_ex_zero(int64_t *p) {
    if (threadIdx.x == 0) *p = 0;
}

}  // namespace
}  // namespace fl

extern "C" {

int fl_rule_rank_weights(void *stream, const void *attention, int att_f64, int64_t H, int64_t T, int64_t L, int64_t n,
                         const int64_t *rows, int64_t N, int64_t W, const int64_t *row_head, int64_t identity,
                         int mode, double *rank_weights, double *rank_sums, double *precision, int64_t *err) {
    if (N < 0 || H < 1 || T < 1 || L < 1 || n < 1 || W < 1 || mode < 0 || mode > 2)
        return fl::fl_fail(FL_ERR_ARG, "rule_rank_weights: bad shape or mode");
    if (T > fl::EX_MAX_T) return fl::fl_fail(FL_ERR_ARG, "rule_rank_weights: at most %d steps", fl::EX_MAX_T);
    if (mode == 0 && T != 3) return fl::fl_fail(FL_ERR_ARG, "rule_rank_weights: the closed form needs 3 steps");
    if (rank_sums && L > fl::EX_MAX_L)
        return fl::fl_fail(FL_ERR_ARG, "rule_rank_weights: row sums of at most %d channels", fl::EX_MAX_L);
    if (W < 1 + T && N > 0) return fl::fl_fail(FL_ERR_ARG, "rule_rank_weights: rows narrower than 1 + steps");
    if (precision && W < 8) return fl::fl_fail(FL_ERR_ARG, "rule_rank_weights: precision needs 8 columns");
    if (identity < -n || identity >= n) return fl::fl_fail(FL_ERR_ARG, "rule_rank_weights: identity out of range");
    if (!err || (N > 0 && (!attention || !rows || !rank_weights)))
        return fl::fl_fail(FL_ERR_ARG, "rule_rank_weights: null pointer");
    const int64_t ident = identity < 0 ? identity + n : identity;
    hipStream_t st = (hipStream_t)stream;
    FL_LAUNCH("k_ex_zero", fl::k_ex_zero, dim3(1), dim3(64), 0, st, err);
    if (N == 0) return fl::fl_check_launch("rule_rank_weights");
    const unsigned g1 = (unsigned)((N * L + fl::EX_NT - 1) / fl::EX_NT);
    if (att_f64)
        FL_LAUNCH("k_rank_weights", fl::k_rank_weights<double>, dim3(g1), dim3(fl::EX_NT), 0, st,
                  (const double *)attention, rows, row_head, N, W, H, T, L, n, ident, mode, rank_weights, err);
    else
        FL_LAUNCH("k_rank_weights", fl::k_rank_weights<float>, dim3(g1), dim3(fl::EX_NT), 0, st,
                  (const float *)attention, rows, row_head, N, W, H, T, L, n, ident, mode, rank_weights, err);
    if (rank_sums || precision)
        FL_LAUNCH("k_rank_stats", fl::k_rank_stats, dim3((unsigned)((N + fl::EX_NT - 1) / fl::EX_NT)),
                  dim3(fl::EX_NT), 0, st, rank_weights, rows, N, W, L, rank_sums, precision);
    return fl::fl_check_launch("rule_rank_weights");
}

int fl_row_pairwise_sums(void *stream, const double *x, int64_t N, int64_t L, double *out) {
    if (N < 0 || L < 0 || L > fl::EX_MAX_L)
        return fl::fl_fail(FL_ERR_ARG, "row_pairwise_sums: at most %d columns", fl::EX_MAX_L);
    if (N == 0) return FL_OK;
    if (!out || (L > 0 && !x)) return fl::fl_fail(FL_ERR_ARG, "row_pairwise_sums: null pointer");
    FL_LAUNCH("k_rank_stats", fl::k_rank_stats, dim3((unsigned)((N + fl::EX_NT - 1) / fl::EX_NT)), dim3(fl::EX_NT), 0,
              (hipStream_t)stream, x, nullptr, N, 0, L, out, nullptr);
    return fl::fl_check_launch("row_pairwise_sums");
}

}  // extern "C"
