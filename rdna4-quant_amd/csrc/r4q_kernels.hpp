// Internal launchers shared between translation units (decode step, prefill).
// Arguments are validated by the callers; these only enqueue work.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace r4q {

// mode: 0 rmsnorm, 1 residual+rmsnorm, 2 rmsnorm+FWHT, 3 residual+rmsnorm+FWHT
int launch_rownorm(int mode, const void* a, const void* b, const void* w, void* y,
                   void* res_out, int64_t rows, int64_t D, float eps, hipStream_t st);
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

// out[m] = table[ids[m]] for M rows of D fp16 (ids already range-checked).
int launch_embed_gather(const int64_t* ids, const void* table, void* out, int64_t M, int64_t D,
                        hipStream_t st);
// Causal GQA self-attention over M prompt rows of qkv (q | k | v heads,
// head_dim 128, row stride `stride`), FWHT-32 of each head's output,
// out [M, out_stride] fp16.
int launch_prefill_attention(const void* qkv, int64_t stride, void* out, int64_t out_stride,
                             int64_t M, int64_t H, int64_t Hk, hipStream_t st);

}  // namespace r4q
