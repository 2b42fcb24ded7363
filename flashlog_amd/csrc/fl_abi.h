// Host-side helpers shared by the C-ABI translation units.
#pragma once
#include <hip/hip_runtime.h>
#include "../../include/flashlog_hip.h"

namespace fl {
// Records a formatted message for fl_last_error() and returns `code`.
int fl_fail(int code, const char *fmt, ...);
// Checks the last HIP launch error; FL_OK or FL_ERR_HIP with the message.
int fl_check_launch(const char *what);

// Per-kernel HIP-event timing (off unless fl_prof_enable(1) was called).
// prof_begin records a start event on `stream` and returns a token;
// prof_end records the matching stop event.
int prof_begin(const char *kernel, hipStream_t stream);
void prof_end(int token, hipStream_t stream);
}  // namespace fl

// Launch `kernel` on `stream`, bracketed by timing events when profiling.
#define FL_LAUNCH(name, kernel, grid, block, lds, stream, ...)                 \
    do {                                                                       \
        int _fl_tok = fl::prof_begin(name, stream);                            \
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);     \
        fl::prof_end(_fl_tok, stream);                                         \
    } while (0)
