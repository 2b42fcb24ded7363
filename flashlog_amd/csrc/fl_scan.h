// Device-wide exclusive scan shared by the sparse kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fl {
// Bytes of `tmp` needed by exclusive_scan over n elements.
size_t scan_tmp_bytes(int64_t n);
// out[i] = sum of in[0..i), out[n] = total (out holds n+1 entries; for
// int64 input out may alias in).  Enqueued on st; FL_OK or an error code.
int exclusive_scan(hipStream_t st, const int32_t *in, int64_t *out, int64_t n, int64_t *tmp);
int exclusive_scan(hipStream_t st, const int64_t *in, int64_t *out, int64_t n, int64_t *tmp);

// Stable LSD radix sort of (uint32 key, float value) pairs on the low `bits`
// key bits (rocPRIM, in fl_csr.hip): equal keys keep their input order.
// With tmp null, *tmp_bytes receives the scratch size; else it is the size
// of tmp.  FL_OK or an error code.
int radix_sort_u32_f32(hipStream_t st, void *tmp, size_t *tmp_bytes, const uint32_t *keys_in, uint32_t *keys_out,
                       const float *vals_in, float *vals_out, int64_t n, int bits);
}  // namespace fl
