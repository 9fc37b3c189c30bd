// Host-side plumbing shared by the translation units of librdna4q:
// thread-local error text, argument checks and HIP status mapping.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/r4q.h"

namespace r4q {

// Records printf-style text as this thread's last error; returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Converts the pending launch status (hipGetLastError) into a return code.
int launch_status(const char* what);

}  // namespace r4q

#define R4Q_REQUIRE(cond, ...)                                  \
  do {                                                          \
    if (!(cond)) return ::r4q::fail(R4Q_EINVAL, __VA_ARGS__);   \
  } while (0)

#define R4Q_HIP_TRY(call)                                                   \
  do {                                                                      \
    hipError_t e_ = (call);                                                 \
    if (e_ != hipSuccess)                                                   \
      return ::r4q::fail(R4Q_EHIP, "%s failed: %s", #call,                  \
                         hipGetErrorString(e_));                            \
  } while (0)

#define R4Q_TRY(expr)            \
  do {                           \
    int rc_ = (expr);            \
    if (rc_ != R4Q_OK) return rc_; \
  } while (0)
