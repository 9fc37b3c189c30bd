// The opaque r4q_ctx: device scratch owned by one context (one stream).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/r4q.h"

namespace r4q {

// A grow-only device buffer.
struct DevBuf {
  void* ptr = nullptr;
  size_t bytes = 0;
  int reserve(size_t need);  // R4Q_OK / R4Q_ENOMEM; never called during capture
  void release();
};

struct GraphCache;  // captured decode steps (r4q_decode.hip)

}  // namespace r4q

struct r4q_ctx {
  int device = -1;
  r4q::DevBuf attn;      // flash-decode partials
  r4q::DevBuf step;      // decode-step activations
  r4q::DevBuf prefill;   // prefill activations
  r4q::DevBuf misc;      // device-side position / counters
  r4q::GraphCache* graphs = nullptr;
};

namespace r4q {

// Flash-decode internals used by the decode step.
// Chooses the split count for `seq_len` positions over B*Hk heads.
int attn_num_splits(int64_t seq_len, int64_t B, int64_t Hk);
// Bytes of partial-result scratch for a launch.
size_t attn_ws_bytes(int64_t B, int64_t H, int nsplit);
// Enqueues partial + combine; seq_len_dev != nullptr: length read on device
// (nsplit must then cover the largest length: seq_len <= 256 * nsplit).
int launch_flash_decode(const void* q, int64_t q_stride, const void* k_cache, const void* v_cache,
                        const float* k_scale, const float* v_scale, void* out, int64_t out_stride,
                        int64_t B, int64_t H, int64_t Hk, int64_t max_seq, int64_t seq_len,
                        const int* seq_len_dev, int nsplit, int fwht, float* ws, hipStream_t st);

}  // namespace r4q

namespace r4q {
// Frees the captured graphs of a context (r4q_decode.hip).
void destroy_graphs(r4q_ctx* ctx);
}  // namespace r4q
