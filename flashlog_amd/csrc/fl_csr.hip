// CSR side construction on the GPU (csr.cpp:12-69, build_side, called by
// build_csr_structure, flashlog_kernel.py:678-697).
//
// The reference orders the positions of a side by two stable counting sorts
// (by relation, then by source), i.e. by (source, relation, edge id), and
// takes the groups as the maximal runs of equal (source, relation).  Here
// one stable LSD radix sort of the keys (source << 15 | relation), carrying
// the edge ids, gives that order: equal keys keep ascending edge ids.  Then,
// thread per position: the column, the relation, the row pointers and the
// group-start flags; a scan numbers the groups; thread per group start: the
// group's start, relation and the group pointers; thread per group: its
// size.  The arrays are bit-identical to the host builder's.
#include <rocprim/device/device_radix_sort.hpp>

#include "fl_abi.h"
#include "fl_common.h"
#include "fl_scan.h"

namespace fl {
namespace {

constexpr int CSR_NT = 256;
constexpr int CSR_REL_BITS = 15;  // relation ids <= INT16_MAX

__global__ void k_csr_keys(const int64_t *__restrict__ src, const int64_t *__restrict__ tgt,
                           const int64_t *__restrict__ rel, int64_t M, int64_t nodes, uint64_t *__restrict__ keys,
                           uint32_t *__restrict__ ids, int64_t *__restrict__ err) {
    const int64_t i = (int64_t)blockIdx.x * CSR_NT + threadIdx.x;
    if (i >= M) return;
    const int64_t s = src[i], t = tgt[i], r = rel[i];
    ids[i] = (uint32_t)i;
    if (s < 0 || s >= nodes || t < 0 || t >= nodes || r < 0 || r > INT16_MAX) {
        atomicMax((unsigned long long *)err, 1ull);
        keys[i] = 0;
        return;
    }
    keys[i] = ((uint64_t)s << CSR_REL_BITS) | (uint64_t)r;
}

// Position j of the sorted side: column, relation, group-start flag, and the
// row pointers of the sources from the previous position's (exclusive) to
// its own (inclusive); the last position also ends the remaining rows.
__global__ void k_csr_fill(const uint64_t *__restrict__ skeys, const uint32_t *__restrict__ order,
                           const int64_t *__restrict__ tgt, int64_t M, int64_t nodes, int32_t *__restrict__ columns,
                           int16_t *__restrict__ edge_rel, int32_t *__restrict__ row_ptr,
                           int32_t *__restrict__ flags) {
    const int64_t j = (int64_t)blockIdx.x * CSR_NT + threadIdx.x;
    if (j >= M) return;
    const uint64_t key = skeys[j];
    const int64_t s = (int64_t)(key >> CSR_REL_BITS);
    columns[j] = (int32_t)tgt[order[j]];
    edge_rel[j] = (int16_t)(key & ((1u << CSR_REL_BITS) - 1));
    const int64_t ps = j > 0 ? (int64_t)(skeys[j - 1] >> CSR_REL_BITS) : -1;
    for (int64_t v = ps + 1; v <= s; ++v) row_ptr[v] = (int32_t)j;
    if (j == M - 1)
        for (int64_t v = s + 1; v <= nodes; ++v) row_ptr[v] = (int32_t)M;
    flags[j] = (j == 0 || skeys[j - 1] != key) ? 1 : 0;
}

// Group start j (group g = gid[j]): start, relation and the group pointers
// of the sources from the previous position's to its own.
__global__ void k_csr_groups(const uint64_t *__restrict__ skeys, const int32_t *__restrict__ flags,
                             const int64_t *__restrict__ gid, int64_t M, int64_t nodes,
                             int32_t *__restrict__ group_start, int16_t *__restrict__ group_rel,
                             int32_t *__restrict__ group_ptr, int64_t *__restrict__ num_groups) {
    const int64_t j = (int64_t)blockIdx.x * CSR_NT + threadIdx.x;
    if (j >= M || !flags[j]) return;
    const int64_t g = gid[j], G = gid[M];
    const uint64_t key = skeys[j];
    const int64_t s = (int64_t)(key >> CSR_REL_BITS);
    group_start[g] = (int32_t)j;
    group_rel[g] = (int16_t)(key & ((1u << CSR_REL_BITS) - 1));
    const int64_t ps = j > 0 ? (int64_t)(skeys[j - 1] >> CSR_REL_BITS) : -1;
    for (int64_t v = ps + 1; v <= s; ++v) group_ptr[v] = (int32_t)g;
    if (g == G - 1) {
        for (int64_t v = s + 1; v <= nodes; ++v) group_ptr[v] = (int32_t)G;
        *num_groups = G;
    }
}

__global__ void k_csr_counts(const int32_t *__restrict__ group_start, const int64_t *__restrict__ gid, int64_t M,
                             int32_t *__restrict__ group_count) {
    const int64_t g = (int64_t)blockIdx.x * CSR_NT + threadIdx.x;
    const int64_t G = gid[M];
    if (g >= G) return;
    group_count[g] = (int32_t)((g + 1 < G ? (int64_t)group_start[g + 1] : M) - group_start[g]);
}

// Empty side: zero row and group pointers.
__global__ void k_csr_empty(int64_t nodes, int32_t *__restrict__ row_ptr, int32_t *__restrict__ group_ptr,
                            int64_t *__restrict__ num_groups) {
    const int64_t v = (int64_t)blockIdx.x * CSR_NT + threadIdx.x;
    if (v == 0) *num_groups = 0;
    if (v > nodes) return;
    row_ptr[v] = 0;
    group_ptr[v] = 0;
}

__global__ void k_csr_zero(int64_t *__restrict__ p, int n) {
    if ((int)threadIdx.x < n) p[threadIdx.x] = 0;
}

size_t csr_al(size_t x) { return (x + 255) & ~(size_t)255; }

struct CsrWs {
    uint64_t *keys, *skeys;
    uint32_t *ids;
    int32_t *flags;
    int64_t *gid, *tmp;
    void *sort_tmp;
    size_t sort_bytes, bytes;
};

int key_bits(int64_t nodes) {
    int b = 0;
    while (((int64_t)1 << b) < nodes) ++b;
    return b + CSR_REL_BITS;
}

CsrWs csr_ws(int64_t M, int64_t nodes, char *base) {
    CsrWs w{};
    size_t off = 0;
    auto take = [&](size_t b) { char *q = base ? base + off : nullptr; off += csr_al(b); return q; };
    const int64_t m1 = M > 0 ? M : 1;
    w.keys = (uint64_t *)take(sizeof(uint64_t) * (size_t)m1);
    w.skeys = (uint64_t *)take(sizeof(uint64_t) * (size_t)m1);
    w.ids = (uint32_t *)take(sizeof(uint32_t) * (size_t)m1);
    w.flags = (int32_t *)take(sizeof(int32_t) * (size_t)m1);
    w.gid = (int64_t *)take(sizeof(int64_t) * (size_t)(m1 + 1));
    w.tmp = (int64_t *)take(scan_tmp_bytes(m1 + 1));
    size_t sb = 0;
    (void)rocprim::radix_sort_pairs(nullptr, sb, (const uint64_t *)nullptr, (uint64_t *)nullptr,
                                    (const uint32_t *)nullptr, (uint32_t *)nullptr, (unsigned)m1, 0,
                                    (unsigned)key_bits(nodes));
    w.sort_bytes = sb;
    w.sort_tmp = take(sb);
    w.bytes = off;
    return w;
}

}  // namespace

int radix_sort_u32_f32(hipStream_t st, void *tmp, size_t *tmp_bytes, const uint32_t *keys_in, uint32_t *keys_out,
                       const float *vals_in, float *vals_out, int64_t n, int bits) {
    if (n < 0 || n > UINT32_MAX || bits < 1 || bits > 32 || !tmp_bytes)
        return fl_fail(FL_ERR_ARG, "radix_sort_u32_f32: bad arguments");
    size_t sb = *tmp_bytes;
    const hipError_t e = rocprim::radix_sort_pairs(tmp, sb, keys_in, keys_out, vals_in, vals_out, (unsigned)n, 0,
                                                   (unsigned)bits, st);
    if (!tmp) *tmp_bytes = sb;
    if (e != hipSuccess) return fl_fail(FL_ERR_HIP, "radix sort: %s", hipGetErrorString(e));
    return FL_OK;
}

}  // namespace fl

using namespace fl;

extern "C" {

size_t fl_csr_build_side_gpu_bytes(int64_t edges, int64_t nodes) {
    if (edges < 0 || nodes < 0) return 0;
    return csr_ws(edges, nodes, nullptr).bytes;
}

int fl_csr_build_side_gpu(void *stream, int64_t edges, int64_t nodes, const int64_t *source, const int64_t *target,
                          const int64_t *relation, int32_t *row_ptr, int32_t *columns, int16_t *edge_rel,
                          int32_t *order, int32_t *group_ptr, int16_t *group_rel, int32_t *group_start,
                          int32_t *group_count, int64_t *info, void *workspace, size_t workspace_bytes) {
    if (edges < 0 || nodes < 0 || nodes > INT32_MAX || edges > INT32_MAX || nodes >= ((int64_t)1 << 48))
        return fl_fail(FL_ERR_ARG, "CSR requires equal 1D arrays and int32-sized graph");
    if (!row_ptr || !group_ptr || !info || (edges > 0 && (!source || !target || !relation || !columns ||
                                                          !edge_rel || !order || !group_rel || !group_start ||
                                                          !group_count)))
        return fl_fail(FL_ERR_ARG, "csr_build_side_gpu: null argument");
    hipStream_t st = (hipStream_t)stream;
    // info: {number of groups, error (1: an id outside the supported range)}
    FL_LAUNCH("k_csr_zero", k_csr_zero, dim3(1), dim3(64), 0, st, info, 2);
    if (edges == 0) {
        FL_LAUNCH("k_csr_empty", k_csr_empty, dim3((unsigned)((nodes + 1 + CSR_NT - 1) / CSR_NT)), dim3(CSR_NT), 0,
                  st, nodes, row_ptr, group_ptr, info);
        return fl_check_launch("csr_build_side_gpu");
    }
    if (!workspace || workspace_bytes < fl_csr_build_side_gpu_bytes(edges, nodes))
        return fl_fail(FL_ERR_ARG, "csr_build_side_gpu: workspace too small");
    CsrWs w = csr_ws(edges, nodes, (char *)workspace);
    const unsigned grid = (unsigned)((edges + CSR_NT - 1) / CSR_NT);
    FL_LAUNCH("k_csr_keys", k_csr_keys, dim3(grid), dim3(CSR_NT), 0, st, source, target, relation, edges, nodes,
              w.keys, w.ids, info + 1);
    size_t sb = w.sort_bytes;
    const hipError_t e = rocprim::radix_sort_pairs(w.sort_tmp, sb, w.keys, w.skeys, w.ids, (uint32_t *)order,
                                                   (unsigned)edges, 0, (unsigned)key_bits(nodes), st);
    if (e != hipSuccess) return fl_fail(FL_ERR_HIP, "csr_build_side_gpu: radix sort: %s", hipGetErrorString(e));
    FL_LAUNCH("k_csr_fill", k_csr_fill, dim3(grid), dim3(CSR_NT), 0, st, w.skeys, (const uint32_t *)order, target,
              edges, nodes, columns, edge_rel, row_ptr, w.flags);
    int rc = exclusive_scan(st, w.flags, w.gid, edges, w.tmp);
    if (rc != FL_OK) return rc;
    FL_LAUNCH("k_csr_groups", k_csr_groups, dim3(grid), dim3(CSR_NT), 0, st, w.skeys, w.flags, w.gid, edges, nodes,
              group_start, group_rel, group_ptr, info);
    FL_LAUNCH("k_csr_counts", k_csr_counts, dim3(grid), dim3(CSR_NT), 0, st, group_start, w.gid, edges,
              group_count);
    return fl_check_launch("csr_build_side_gpu");
}

}  // extern "C"
