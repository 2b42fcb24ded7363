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
}  // namespace fl
