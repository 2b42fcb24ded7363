// Host-side parts of the C-ABI: error state, CSR construction and the
// destination-major pull index.  Plain C++ (no device code).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "fl_abi.h"

namespace fl {

static thread_local std::string g_last_error;

int fl_fail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int fl_check_launch(const char *what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fl_fail(FL_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return FL_OK;
}

struct ProfRec {
    std::string name;
    hipEvent_t start, stop;
};
static bool g_prof_on = false;
static std::vector<ProfRec> g_prof;

int prof_begin(const char *kernel, hipStream_t stream) {
    if (!g_prof_on) return -1;
    ProfRec r{kernel, nullptr, nullptr};
    if (hipEventCreate(&r.start) != hipSuccess || hipEventCreate(&r.stop) != hipSuccess) return -1;
    (void)hipEventRecord(r.start, stream);
    g_prof.push_back(r);
    return (int)g_prof.size() - 1;
}

void prof_end(int token, hipStream_t stream) {
    if (token < 0 || token >= (int)g_prof.size()) return;
    (void)hipEventRecord(g_prof[token].stop, stream);
}

static void prof_clear() {
    for (auto &r : g_prof) {
        (void)hipEventDestroy(r.start);
        (void)hipEventDestroy(r.stop);
    }
    g_prof.clear();
}

}  // namespace fl

extern "C" {

// Enables (1) or disables (0) per-kernel event timing; either call discards
// earlier records.  Not thread-safe: for single-threaded benchmarking.
int fl_prof_enable(int on) {
    fl::prof_clear();
    fl::g_prof_on = on != 0;
    return FL_OK;
}

// Sum of event-timed durations (ms) and launch count of `kernel` since the
// last fl_prof_enable; waits for the recorded events.
int fl_prof_read(const char *kernel, double *total_ms, int64_t *launches) {
    double tot = 0.0;
    int64_t cnt = 0;
    for (auto &r : fl::g_prof) {
        if (r.name != kernel) continue;
        if (hipEventSynchronize(r.stop) != hipSuccess) return fl::fl_fail(FL_ERR_HIP, "prof_read: event wait failed");
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess) return fl::fl_fail(FL_ERR_HIP, "prof_read: elapsed failed");
        tot += ms;
        ++cnt;
    }
    *total_ms = tot;
    *launches = cnt;
    return FL_OK;
}

const char *fl_last_error(void) { return fl::g_last_error.c_str(); }

size_t fl_side_bytes(void) { return sizeof(fl_side); }
size_t fl_sparse_hop_bytes(void) { return sizeof(fl_sparse_hop); }
size_t fl_ground_graph_bytes(void) { return sizeof(fl_ground_graph); }

// csr.cpp:12-69: positions ordered by (source, relation, edge id) through a
// stable bucket pass by relation followed by a stable bucket pass by source;
// groups are the maximal runs of equal (source, relation).
int fl_csr_build_side(int64_t edges, int64_t nodes, const int64_t *source, const int64_t *target,
                      const int64_t *relation, int32_t *row_ptr, int32_t *columns,
                      int16_t *edge_rel, int32_t *order, int32_t *group_ptr, int16_t *group_rel,
                      int32_t *group_start, int32_t *group_count, int64_t *num_groups) {
    if (edges < 0 || nodes < 0 || nodes > INT32_MAX || edges > INT32_MAX)
        return fl::fl_fail(FL_ERR_ARG, "CSR requires equal 1D arrays and int32-sized graph");
    int64_t relations = 0;
    for (int64_t i = 0; i < edges; ++i) {
        if (source[i] < 0 || source[i] >= nodes || target[i] < 0 || target[i] >= nodes ||
            relation[i] < 0 || relation[i] > INT16_MAX)
            return fl::fl_fail(FL_ERR_ARG, "CSR entity or relation ID outside supported range");
        if (relation[i] + 1 > relations) relations = relation[i] + 1;
    }
    std::vector<int64_t> bucket(std::max<int64_t>(relations, nodes) + 1, 0);
    std::vector<int32_t> by_rel((size_t)edges);
    for (int64_t i = 0; i < edges; ++i) ++bucket[relation[i]];
    int64_t run = 0;
    for (int64_t r = 0; r < relations; ++r) { int64_t c = bucket[r]; bucket[r] = run; run += c; }
    for (int64_t i = 0; i < edges; ++i) by_rel[bucket[relation[i]]++] = (int32_t)i;
    std::fill(bucket.begin(), bucket.end(), 0);
    for (int64_t i = 0; i < edges; ++i) ++bucket[source[i]];
    run = 0;
    for (int64_t v = 0; v < nodes; ++v) { int64_t c = bucket[v]; row_ptr[v] = (int32_t)run; bucket[v] = run; run += c; }
    row_ptr[nodes] = (int32_t)edges;
    for (int64_t k = 0; k < edges; ++k) { int32_t i = by_rel[k]; order[bucket[source[i]]++] = i; }
    std::memset(group_ptr, 0, sizeof(int32_t) * (size_t)(nodes + 1));
    int64_t g = -1;
    for (int64_t j = 0; j < edges; ++j) {
        const int32_t i = order[j];
        columns[j] = (int32_t)target[i];
        edge_rel[j] = (int16_t)relation[i];
        const bool fresh = j == 0 || source[i] != source[order[j - 1]] || relation[i] != relation[order[j - 1]];
        if (fresh) {
            if (g >= 0) group_count[g] = (int32_t)(j - group_start[g]);
            ++g;
            group_start[g] = (int32_t)j;
            group_rel[g] = (int16_t)relation[i];
            ++group_ptr[source[i] + 1];
        }
    }
    if (g >= 0) group_count[g] = (int32_t)(edges - group_start[g]);
    for (int64_t v = 0; v < nodes; ++v) group_ptr[v + 1] += group_ptr[v];
    *num_groups = g + 1;
    return FL_OK;
}

// Destination-major index of one CSR side: a stable counting sort of the
// positions by destination, so each destination's slots list its incoming
// positions in ascending CSR order.
int fl_pull_index_build(int64_t nodes, int64_t edges, int64_t groups, const int32_t *columns,
                        const int32_t *row_group_ptr, const int16_t *group_rel,
                        const int32_t *group_start, const int32_t *group_count, int32_t *pull_ptr,
                        int32_t *pull_pos, int32_t *pull_src, int16_t *pull_rel) {
    if (nodes < 0 || edges < 0 || groups < 0 || edges > INT32_MAX)
        return fl::fl_fail(FL_ERR_ARG, "pull_index_build: bad sizes");
    std::vector<int32_t> src(edges, -1);
    std::vector<int16_t> rel(edges, 0);
    for (int64_t v = 0; v < nodes; ++v) {
        for (int64_t g = row_group_ptr[v]; g < row_group_ptr[v + 1]; ++g) {
            if (g < 0 || g >= groups) return fl::fl_fail(FL_ERR_ARG, "pull_index_build: group pointer out of range");
            const int64_t s = group_start[g], c = group_count[g];
            if (s < 0 || c < 0 || s + c > edges) return fl::fl_fail(FL_ERR_ARG, "pull_index_build: group range out of bounds");
            for (int64_t p = s; p < s + c; ++p) { src[p] = (int32_t)v; rel[p] = group_rel[g]; }
        }
    }
    std::vector<int64_t> cursor(nodes + 1, 0);
    for (int64_t p = 0; p < edges; ++p) {
        if (columns[p] < 0 || columns[p] >= nodes) return fl::fl_fail(FL_ERR_ARG, "pull_index_build: column out of range");
        if (src[p] < 0) return fl::fl_fail(FL_ERR_ARG, "pull_index_build: position %lld not in any group", (long long)p);
        ++cursor[columns[p]];
    }
    int64_t run = 0;
    for (int64_t v = 0; v < nodes; ++v) { int64_t c = cursor[v]; pull_ptr[v] = (int32_t)run; cursor[v] = run; run += c; }
    pull_ptr[nodes] = (int32_t)edges;
    for (int64_t p = 0; p < edges; ++p) {
        const int64_t slot = cursor[columns[p]]++;
        pull_pos[slot] = (int32_t)p;
        pull_src[slot] = src[p];
        pull_rel[slot] = rel[p];
    }
    return FL_OK;
}

// Heavy destinations (more than FL_SEG slots), their FL_SEG-slot segments
// and FL_SUP-segment supersegments, in destination order.
int fl_pull_segments(int64_t nodes, const int32_t *pull_ptr, int64_t *nseg, int64_t *nheavy, int64_t *nsup,
                     int32_t *seg_dst, int32_t *seg_start, int32_t *seg_h, int32_t *heavy_dst,
                     int32_t *heavy_seg_ptr, int32_t *heavy_sup_ptr, int32_t *sup_h, int32_t *sup_seg0) {
    if (nodes < 0 || !pull_ptr || !nseg || !nheavy || !nsup)
        return fl::fl_fail(FL_ERR_ARG, "pull_segments: bad arguments");
    const bool fill = seg_dst != nullptr;
    int64_t ns = 0, nh = 0, nu = 0;
    for (int64_t v = 0; v < nodes; ++v) {
        const int64_t deg = (int64_t)pull_ptr[v + 1] - pull_ptr[v];
        if (deg <= FL_SEG) continue;
        const int64_t segs = (deg + FL_SEG - 1) / FL_SEG;
        const int64_t sups = (segs + FL_SUP - 1) / FL_SUP;
        if (fill) {
            heavy_dst[nh] = (int32_t)v;
            heavy_seg_ptr[nh] = (int32_t)ns;
            heavy_sup_ptr[nh] = (int32_t)nu;
            for (int64_t k = 0; k < segs; ++k) {
                seg_dst[ns + k] = (int32_t)v;
                seg_start[ns + k] = (int32_t)(pull_ptr[v] + k * FL_SEG);
                seg_h[ns + k] = (int32_t)nh;
            }
            for (int64_t k = 0; k < sups; ++k) {
                sup_h[nu + k] = (int32_t)nh;
                sup_seg0[nu + k] = (int32_t)(ns + k * FL_SUP);
            }
        }
        ns += segs;
        nu += sups;
        ++nh;
    }
    if (fill) {
        heavy_seg_ptr[nh] = (int32_t)ns;
        heavy_sup_ptr[nh] = (int32_t)nu;
    }
    *nseg = ns;
    *nheavy = nh;
    *nsup = nu;
    return FL_OK;
}

}  // extern "C"
