// Host-side helpers shared by the C-ABI translation units.
#pragma once
#include <hip/hip_runtime.h>
#include "../../include/flashlog_hip.h"

namespace fl {
// Records a formatted message for fl_last_error() and returns `code`.
int fl_fail(int code, const char *fmt, ...);
// Checks the last HIP launch error; FL_OK or FL_ERR_HIP with the message.
int fl_check_launch(const char *what);
}  // namespace fl
