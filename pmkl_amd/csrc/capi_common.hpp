// Error reporting and dtype helpers shared by the C ABI sources of
// libpmkl_attn.so (attn_capi.hip, softmax_capi.hip).
//
// The reference reports a failed check by throwing pmkl::utils::Error from
// CHECK_FAIL (pmkl/core/utils/exception.h:121-161).  At the C boundary a
// failed check returns a status code and leaves "[pmkl check failed at
// file:line] message" in a thread-local buffer read by pmkl_last_error().
#pragma once

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "pmkl_attn.h"

namespace pmkl_capi {

// One buffer per thread for the whole library (an inline variable, so both
// translation units share it).
inline thread_local char g_err[512] = "";

inline int fail(int code, const char *file, int line, const char *fmt, ...) {
    char msg[400];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof(msg), fmt, ap);
    va_end(ap);
    const char *base = strrchr(file, '/');
    snprintf(g_err, sizeof(g_err), "[pmkl check failed at %s:%d] %s", base ? base + 1 : file, line, msg);
    return code;
}

inline size_t dtype_size(int32_t dt) { return dt == PMKL_DTYPE_F32 ? 4 : 2; }

inline bool dtype_valid(int32_t dt) {
    return dt == PMKL_DTYPE_F32 || dt == PMKL_DTYPE_F16 || dt == PMKL_DTYPE_BF16;
}

}  // namespace pmkl_capi

#define PMKL_FAIL(code, ...) return pmkl_capi::fail((code), __FILE__, __LINE__, __VA_ARGS__)
#define PMKL_REQUIRE(cond, code, ...) \
    do {                              \
        if (!(cond)) PMKL_FAIL((code), __VA_ARGS__); \
    } while (0)
