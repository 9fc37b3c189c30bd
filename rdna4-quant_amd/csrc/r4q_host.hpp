// Host-side plumbing shared by the translation units of librdna4q:
// thread-local error text, argument checks and HIP status mapping.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "../../include/r4q.h"

namespace r4q {

// Records printf-style text as this thread's last error; returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Converts the pending launch status (hipGetLastError) into a return code.
int launch_status(const char* what);

// Launch-shape overrides for measurement sweeps; 0 = the built-in choice.
// Initial values come from the environment, read once per process (first
// use) and validated there; r4q_tune() changes them later.  A value outside
// its range is ignored (environment) or rejected (r4q_tune).
//   gemv_lpr      R4Q_GEMV_LPR      lanes per GEMV row: 16, 32, 64, 128, 256
//   gemv_wgs      R4Q_GEMV_WGS      GEMV workgroup cap: 1 .. 65536
//   gemv_ub       R4Q_GEMV_UB       GEMV steps in flight per lane: 1 or 2
//   attn_splits   R4Q_ATTN_SPLITS   flash-decode splits: 1 .. 128
//   skinny_splits R4Q_SKINNY_SPLITS skinny-GEMM K splits: 1 .. 8
//   gemm_splits   R4Q_GEMM_SPLITS   ring GEMM: 1 whole tiles, 2 .. 16 stream-K workgroups per tile
//   gemm_kernel   R4Q_GEMM_KERNEL   GEMM for M >= 256: 1 the ring kernel (the default), 2 the
//                                   specialised-wave kernel where it applies (INT4, N % 128 == 0,
//                                   K % 256 == 0)
//   gemv_skew     R4Q_GEMV_SKEW     GEMV on an even grid of more than 256 equal shares: the
//                                   first half takes value - 1 steps more, the second half
//                                   value - 1 fewer (1 = equal shares)
//   split_reduce  R4Q_SPLIT_REDUCE  1: batched decode steps reduce the split-K partials of the
//                                   qkv, o and down projections in their own launches instead
//                                   of in the consumer (attention prologue, row norm)
struct Tuning {
  std::atomic<int> gemv_lpr{0}, gemv_wgs{0}, gemv_ub{0};
  std::atomic<int> attn_splits{0}, skinny_splits{0}, gemm_splits{0};
  std::atomic<int> split_reduce{0}, gemm_kernel{0}, gemv_skew{0};
};
Tuning& tuning();

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
