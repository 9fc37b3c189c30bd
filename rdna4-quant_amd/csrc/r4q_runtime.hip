// Error state and ABI version of librdna4q.
#include <stdarg.h>
#include <stdio.h>

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

}  // namespace r4q

extern "C" const char* r4q_last_error(void) { return r4q::g_err; }

extern "C" int r4q_abi_version(void) { return 1; }

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
