// Status codes and error messages of the C ABI, shared by the source files
// that define entry points. The message of the last failing call on a thread
// is kept for tgs_last_error().
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/tinygs_amd.h"

namespace tgs {

// Records the formatted message for tgs_last_error() and returns code.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

}  // namespace tgs

#define TGS_HIP(call)                                                                                        \
    do {                                                                                                     \
        hipError_t e_ = (call);                                                                              \
        if (e_ != hipSuccess)                                                                                \
            return ::tgs::fail(TGS_ERR_HIP, "%s failed at %s:%d: %s", #call, __FILE__, __LINE__,            \
                               hipGetErrorString(e_));                                                       \
    } while (0)

#define TGS_CHECK_LAUNCH()                                                                                   \
    do {                                                                                                     \
        hipError_t e_ = hipGetLastError();                                                                   \
        if (e_ != hipSuccess)                                                                                \
            return ::tgs::fail(TGS_ERR_HIP, "kernel launch failed at %s:%d: %s", __FILE__, __LINE__,        \
                               hipGetErrorString(e_));                                                       \
    } while (0)

#define TGS_TRY(expr)                  \
    do {                               \
        int rc_ = (expr);              \
        if (rc_ != TGS_OK) return rc_; \
    } while (0)
