// Internal launchers shared between translation units (decode step, prefill).
// Arguments are validated by the callers; these only enqueue work.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace r4q {

// mode: 0 rmsnorm, 1 residual+rmsnorm, 2 rmsnorm+FWHT, 3 residual+rmsnorm+FWHT
int launch_rownorm(int mode, const void* a, const void* b, const void* w, void* y,
                   void* res_out, int64_t rows, int64_t D, float eps, hipStream_t st);
// Mode 3 with a = fp16(split-order sum of S fp32 planes ap[s * plane + row * D + i])
// (a split-K projection's partials), equal to its reduce followed by mode 3.
bool rownorm_psum_ok(int64_t D, int S);
int launch_rownorm_psum(const float* ap, int64_t plane, int S, const void* b, const void* w,
                        void* y, void* res_out, int64_t rows, int64_t D, float eps,
                        hipStream_t st);
int launch_silu(bool fwht, const void* g, const void* u, void* y, int64_t rows, int64_t I,
                int64_t in_stride, int64_t out_stride, hipStream_t st);
int check_head_norm_rope_kv(const void* qkv, const void* qw, const void* kw, const void* q_out,
                            const void* k_cache, const void* v_cache, const void* cos_t,
                            const void* sin_t, int64_t B, int64_t H, int64_t Hk, int64_t D,
                            int64_t max_seq, int64_t pos);
// pos_dev != nullptr: position read from device memory (graph replay).
// prefill_rows: row b is position pos + b of cache sequence 0 (else every
// row is at `pos` in cache sequence b).  Null caches skip the KV write.
int launch_head_norm_rope_kv(const void* qkv, int64_t qkv_stride, const void* qw, const void* kw,
                             void* q_out, int64_t q_out_stride, void* k_cache, void* v_cache,
                             const float* k_scale, const float* v_scale, const void* cos_t,
                             const void* sin_t, int64_t B, int64_t H, int64_t Hk, float eps,
                             int64_t max_seq, int64_t pos, const int* pos_dev, hipStream_t st,
                             bool prefill_rows = false);

// Device-side state of a captured decode loop (int words): the position
// being decoded, the sequence length seen by attention, the step index.
enum { kPos = 0, kSeq = 1, kStep = 2, kStateWords = 4 };

// Temperature / top-p sampling (temperature > 0, 0 < top_p; top_p >= 1 keeps
// every token), uniform draw from (seed, counter, row).
struct SampleCfg {
  float temperature;
  float top_p;
  uint64_t seed;
};
// Workspace for B <= 1024 rows: the selection words, then a zeroed
// 65,536-bin table per row (left zeroed by every call; see sample_reserve).
size_t sample_ws_bytes(int64_t B);
// ids[b] = sampled token of row b of logits [B, stride] fp16 (V used).
// counter_dev (device int) overrides counter_host.  With embed != nullptr
// the token's embedding row goes to h[b] and tokens_out[step * B + b] = id
// (step from state[kStep] when state != nullptr, else step_host).
int launch_sample(const void* logits, int64_t B, int64_t V, int64_t stride, const SampleCfg& cfg,
                  const int* counter_dev, int64_t counter_host, void* ws, int64_t* ids,
                  const void* embed, int64_t D, void* h, int64_t* tokens_out, const int* state,
                  int step_host, hipStream_t st);

// out[m] = table[ids[m]] for M rows of D fp16 (ids already range-checked).
int launch_embed_gather(const int64_t* ids, const void* table, void* out, int64_t M, int64_t D,
                        hipStream_t st);
// Causal GQA self-attention over M prompt rows of qkv (q | k | v heads,
// head_dim 128, row stride `stride`), FWHT-32 of each head's output,
// out [M, out_stride] fp16.
int launch_prefill_attention(const void* qkv, int64_t stride, void* out, int64_t out_stride,
                             int64_t M, int64_t H, int64_t Hk, hipStream_t st);

}  // namespace r4q
