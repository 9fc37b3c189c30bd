// Error state, ABI version and launch-shape overrides of librdna4q.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <new>

#include "r4q_ctx.hpp"
#include "r4q_host.hpp"

namespace r4q {
namespace {
thread_local char g_err[512] = {0};
}

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = 0; }

int launch_status(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(R4Q_EHIP, "%s: launch failed: %s", what, hipGetErrorString(e));
  return R4Q_OK;
}

namespace {
struct Knob {
  const char* name;  // r4q_tune name; the environment variable is R4Q_<NAME>
  const char* env;
  std::atomic<int> Tuning::*field;
  int lo, hi;
  bool pow2;
};
const Knob kKnobs[] = {
    {"gemv_lpr", "R4Q_GEMV_LPR", &Tuning::gemv_lpr, 16, 256, true},
    {"gemv_wgs", "R4Q_GEMV_WGS", &Tuning::gemv_wgs, 1, 65536, false},
    {"gemv_ub", "R4Q_GEMV_UB", &Tuning::gemv_ub, 1, 2, false},
    {"attn_splits", "R4Q_ATTN_SPLITS", &Tuning::attn_splits, 1, 128, false},
    {"skinny_splits", "R4Q_SKINNY_SPLITS", &Tuning::skinny_splits, 1, 8, false},
    {"gemm_splits", "R4Q_GEMM_SPLITS", &Tuning::gemm_splits, 1, 16, false},
    {"split_reduce", "R4Q_SPLIT_REDUCE", &Tuning::split_reduce, 1, 1, false},
    {"gemm_kernel", "R4Q_GEMM_KERNEL", &Tuning::gemm_kernel, 1, 2, false},
    {"gemv_skew", "R4Q_GEMV_SKEW", &Tuning::gemv_skew, 1, 8, false},
};

bool knob_ok(const Knob& k, long x) {
  return x >= k.lo && x <= k.hi && (!k.pow2 || (x & (x - 1)) == 0);
}

// Value of the knob's environment variable when it parses completely and
// is in range, else 0.
int env_knob(const Knob& k) {
  const char* v = getenv(k.env);
  if (!v || !*v) return 0;
  char* end = nullptr;
  const long x = strtol(v, &end, 10);
  return (*end == 0 && knob_ok(k, x)) ? (int)x : 0;
}
}  // namespace

Tuning& tuning() {
  static Tuning t;
  static const bool init = [] {
    for (const Knob& k : kKnobs) (t.*k.field).store(env_knob(k));
    return true;
  }();
  (void)init;
  return t;
}

int DevBuf::reserve(size_t need) {
  if (need <= bytes) return R4Q_OK;
  if (epoch) ++*epoch;
  if (ptr) {
    (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
  }
  const size_t cap = (need + 0xFFFFF) & ~(size_t)0xFFFFF;  // 1 MiB granules
  if (hipMalloc(&ptr, cap) != hipSuccess) {
    ptr = nullptr;
    return fail(R4Q_ENOMEM, "hipMalloc(%zu) failed", cap);
  }
  bytes = cap;
  return R4Q_OK;
}

void DevBuf::release() {
  if (!ptr) return;
  if (epoch) ++*epoch;
  (void)hipFree(ptr);
  ptr = nullptr;
  bytes = 0;
}

}  // namespace r4q

extern "C" const char* r4q_last_error(void) { return r4q::g_err; }

extern "C" int r4q_abi_version(void) { return 1; }

extern "C" int r4q_tune(const char* name, int value) {
  R4Q_REQUIRE(name, "tune: null name");
  for (const r4q::Knob& k : r4q::kKnobs) {
    if (strcmp(name, k.name) != 0) continue;
    R4Q_REQUIRE(value == 0 || r4q::knob_ok(k, value), "tune: %s=%d outside [%d, %d]%s", name,
                value, k.lo, k.hi, k.pow2 ? " (power of two)" : "");
    (r4q::tuning().*k.field).store(value);
    return R4Q_OK;
  }
  return r4q::fail(R4Q_EINVAL, "tune: unknown knob '%s'", name);
}

extern "C" int r4q_ctx_create(r4q_ctx** out) {
  R4Q_REQUIRE(out, "ctx_create: null output pointer");
  r4q_ctx* c = new (std::nothrow) r4q_ctx();
  if (!c) return r4q::fail(R4Q_ENOMEM, "ctx_create: out of host memory");
  if (hipGetDevice(&c->device) != hipSuccess) {
    delete c;
    return r4q::fail(R4Q_EHIP, "ctx_create: hipGetDevice failed");
  }
  *out = c;
  return R4Q_OK;
}

extern "C" int r4q_ctx_destroy(r4q_ctx* ctx) {
  if (!ctx) return R4Q_OK;
  (void)hipDeviceSynchronize();
  r4q::destroy_graphs(ctx);
  ctx->attn.release();
  ctx->step.release();
  ctx->prefill.release();
  ctx->misc.release();
  ctx->sample.release();
  delete ctx;
  return R4Q_OK;
}
