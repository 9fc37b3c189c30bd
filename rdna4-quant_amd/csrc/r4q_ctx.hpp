// The opaque r4q_ctx: device scratch owned by one context (one stream).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/r4q.h"

namespace r4q {

// A grow-only device buffer.  Every (re)allocation and release adds one to
// *epoch (the owning context's count), so that a captured graph, whose key
// holds that count, is never replayed after one of its buffers could have
// moved.
struct DevBuf {
  void* ptr = nullptr;
  size_t bytes = 0;
  uint64_t* epoch = nullptr;
  int reserve(size_t need);  // R4Q_OK / R4Q_ENOMEM; never called during capture
  void release();
};

struct GraphCache;  // captured decode steps (r4q_decode.hip)

}  // namespace r4q

struct r4q_ctx {
  int device = -1;
  // reallocations of this context's buffers (DevBuf::epoch); a graph key
  // holds it, so growing another context's buffers invalidates no graph here
  uint64_t buf_epoch = 0;
  r4q::DevBuf attn;      // flash-decode partials
  r4q::DevBuf step;      // decode-step activations
  void* tail_zeroed = nullptr;  // batched gate/up tail counters known to be zero
  r4q::DevBuf prefill;   // prefill activations
  r4q::DevBuf misc;      // device-side position / counters
  r4q::DevBuf sample;    // sampling tables (kept zeroed between calls)
  size_t sample_zeroed = 0;  // bytes of `sample` known to be zero
  r4q::GraphCache* graphs = nullptr;
  r4q_ctx() {
    for (r4q::DevBuf* b : {&attn, &step, &prefill, &misc, &sample}) b->epoch = &buf_epoch;
  }
};

namespace r4q {

// Flash-decode internals used by the decode step.
// Chooses the split count for `seq_len` positions over B*Hk heads.
int attn_num_splits(int64_t seq_len, int64_t B, int64_t Hk);
// Sampling workspace for B rows, zeroed on (re)allocation.
int sample_reserve(r4q_ctx* ctx, int64_t B, hipStream_t st, void** ws);
// Bytes of partial-result scratch for a launch.
size_t attn_ws_bytes(int64_t B, int64_t H, int nsplit);
// Enqueues partial + combine; seq_len_dev != nullptr: length read on device
// (any length up to max_seq; nsplit is chosen from the capacity).
// Fused decode-step prologue (NORMQ): q of the workgroup's query heads and
// the new position's K/V come raw from the QKV projection row; the
// workgroup applies the head RMSNorm + RoPE (head_norm_rope_pair, the
// arithmetic of the standalone kernel) and the one holding position L-1
// writes that position's FP8 K/V codes and uses them for its own tile.
struct AttnQK {
  const uint16_t* qw;  // [128] q norm weight
  const uint16_t* kw;  // [128] k norm weight
  const uint16_t* cs;  // RoPE tables [positions, 64]
  const uint16_t* sn;
  uint8_t* kc;         // caches to write at position L-1
  uint8_t* vc;
  float eps;
  // nsum >= 2: the raw QKV rows are the split sums fp16(sum over s < nsum of
  // part[s * plane + row offset]) of a split-K projection (nsum <= kMaxQkvSplits)
  const float* part = nullptr;
  int64_t plane = 0;
  int nsum = 0;
};
constexpr int kMaxQkvSplits = 4;

// qk == nullptr: q rows are final (normed, rotated) queries.  Otherwise q
// rows are raw QKV projection rows and the fused prologue above runs.
int launch_flash_decode(const void* q, int64_t q_stride, const void* k_cache, const void* v_cache,
                        const float* k_scale, const float* v_scale, void* out, int64_t out_stride,
                        int64_t B, int64_t H, int64_t Hk, int64_t max_seq, int64_t seq_len,
                        const int* seq_len_dev, int nsplit, int fwht, float* ws, hipStream_t st,
                        const AttnQK* qk = nullptr);

}  // namespace r4q

namespace r4q {
// Frees the captured graphs of a context (r4q_decode.hip).
void destroy_graphs(r4q_ctx* ctx);
}  // namespace r4q
