/*
 * r4q.h — C ABI of the MI355X (gfx950) decode-step library `librdna4q.so`.
 *
 * Every entry point takes raw device pointers, int64 sizes and a HIP stream
 * handle passed as `void*` (NULL = the legacy default stream), and returns an
 * int status: R4Q_OK (0) or a negative R4Q_E* code.  The text of the last
 * failure on the calling thread is available from r4q_last_error().  No C++
 * exception crosses this boundary and no entry point takes a torch type.
 *
 * Tensor conventions (all row-major, contiguous):
 *   fp16 values are IEEE binary16 carried as uint16_t bit patterns.
 *   INT4 weight  w  [N, K/2]  uint8, byte = q[2j] | q[2j+1] << 4, q in 0..15
 *   INT8 weight  w  [N, K]    uint8, q in 0..255 (symmetric int8 checkpoints:
 *                              q = int8 + 128 with zero-point 128)
 *   FP16 weight  w  [N, K]    fp16
 *   scale/zero  sz  [N, K/32, 2] fp16, interleaved (scale, zero-point) per
 *                              32-element block; unused for FP16 weights.
 *   dequantised weight = fp16( (float(q) - float(zp)) * float(scale) )
 *   FP8 KV cache [B, Hk, max_seq, head_dim] uint8, E4M3 codes written by the
 *   reference recipe (see r4q_fp16_to_fp8), optional per-head fp32 scale:
 *   stored = fp8(value * (1/scale)), read back as fp8_value * scale.
 *
 * `wbits` selects the weight format: 4 (INT4 asym), 8 (INT8 asym), 16 (FP16).
 *
 * Reference interfaces replaced (JohnTDI-cpu/rdna4-quant,
 * hip_int4/int4_decode_step.hip, pybind table at :3620-3636):
 *   r4q_dequant_int4     <- dequant_int4            (:3590-3603)
 *   r4q_fp16_to_fp8      <- fp16_to_fp8             (:3611-3618)
 *   r4q_gemv             <- dbg_gemv / launch_gemv  (:3541-3550, :230-235)
 *   r4q_gemm             <- dbg_gemm / dequant_matmul_out (:3552-3561, :1973-1988)
 *   r4q_res_rmsnorm_fwht_gemv <- fused_res_norm_fwht + launch_gemv pair
 *                           inside the decode step
 *   r4q_gate_up_silu_fwht <- launch_gemv (gate_up) + silu_hadamard_ds pair
 *   r4q_rmsnorm          <- dbg_rmsnorm             (:3473-3484)
 *   r4q_res_rmsnorm      <- dbg_fused_res_norm      (:3524-3539)
 *   r4q_rmsnorm_fwht     <- fused_rmsnorm_fwht      (:1195-1237)
 *   r4q_res_rmsnorm_fwht <- fused_res_norm_fwht     (:1143-1192)
 *   r4q_fwht32           <- hadamard_rotate_batched (:766-786)
 *   r4q_silu_mul_fwht    <- silu_hadamard_ds        (:1031-1051)
 *   r4q_silu_mul         <- silu_mul_batched        (:2112-2122)
 *   r4q_head_rmsnorm     <- dbg_head_rmsnorm        (:3486-3504)
 *   r4q_rope             <- dbg_rope                (:3506-3522)
 *   r4q_head_norm_rope_kv<- head_rmsnorm_rope_kv    (:1620-1683)
 *   r4q_flash_decode     <- launch_flash_decode     (:1547-1593)
 *   r4q_flash_decode_qkv <- head_rmsnorm_rope_kv + launch_flash_decode
 *                           pair of the decode step (:1620-1683, :2487-2500)
 *   r4q_decode_step      <- decode_step / decode_step_logits (:2343-2595),
 *                           as called once per token by the engine
 *                           (int4_engine_v5.py:272)
 *   r4q_decode_step_graph <- the same, replayed from a hipGraph
 *   r4q_decode_bench     <- decode_bench / decode_bench_graph (:2601-3041),
 *                           and decode_loop (:3284-3466) via tokens_out
 *   r4q_decode_profile   <- decode_profile          (:3047-3273)
 *   r4q_prefill_logits   <- prefill_logits          (:2127-2320)
 *   r4q_prefill_attention <- its causal SDPA + FWHT-32 (:2254-2269)
 *   r4q_decode_generate, r4q_sample <- the Python sampling of the engine
 *                           (int4_engine_v5.py:330-335, 387-399)
 */
#ifndef R4Q_H
#define R4Q_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Only the entry points below are exported from librdna4q.so. */
#if defined(__GNUC__)
#define R4Q_API __attribute__((visibility("default")))
#else
#define R4Q_API
#endif

#define R4Q_OK            0
#define R4Q_EINVAL       -1   /* bad pointer, size, shape or format */
#define R4Q_EUNSUPPORTED -2   /* valid request this build does not implement */
#define R4Q_EHIP         -3   /* a HIP runtime call failed */
#define R4Q_ENOMEM       -4   /* device allocation failed */

/* Text of the last error on this thread ("" if none). */
R4Q_API const char* r4q_last_error(void);
/* ABI version: bumped when a signature or struct layout changes. */
R4Q_API int r4q_abi_version(void);

/* ---------------------------------------------------------------- codecs */

/* out[N,K] fp16 = dequant(packed INT4 [N,K/2], sz [N,K/32,2]).  K % 32 == 0. */
R4Q_API int r4q_dequant_int4(const void* packed, const void* sz, void* out,
                     int64_t N, int64_t K, void* stream);
/* out[N,K] fp16 = dequant(INT8 q [N,K], sz [N,K/32,2]).  K % 32 == 0. */
R4Q_API int r4q_dequant_int8(const void* q, const void* sz, void* out,
                     int64_t N, int64_t K, void* stream);
/* dst[n] uint8 = E4M3 code of src[n] (fp16) by the reference recipe
 * (hip:47-68): clamp to +-448 (NaN -> 448), exponent rebias, keep 3 mantissa
 * bits rounding up when fp32 mantissa bit 19 is set, |x| < 2^-6 -> +-0,
 * exponent >= 15 -> +-0x7E (448).  No scaling. */
R4Q_API int r4q_fp16_to_fp8(const void* src, void* dst, int64_t n, void* stream);
/* dst[n] fp16 = value of E4M3 code src[n] (exact for every emitted code). */
R4Q_API int r4q_fp8_to_fp16(const void* src, void* dst, int64_t n, void* stream);

/* ---------------------------------------------------------------- linear */

/* y[N] fp16 = W x with W given by (w, sz, wbits), x[K] fp16, fp32 accumulate.
 * K % 32 == 0, N >= 1. */
R4Q_API int r4q_gemv(const void* x, const void* w, const void* sz, void* y,
             int64_t N, int64_t K, int wbits, void* stream);
/* y[M,N] fp16 = x[M,K] W^T (same weight formats), fp32 accumulate.
 * Small M streams the weights once for all rows; large M dequantises tiles
 * on the fly into an MFMA GEMM. */
R4Q_API int r4q_gemm(const void* x, const void* w, const void* sz, void* y,
             int64_t M, int64_t N, int64_t K, int wbits, void* stream);
/* Device workspace (bytes, written to *bytes; 0: none) that lets r4q_gemm_ws
 * split K loops over more workgroups: for M >= 256 (INT4 / INT8 / FP16) the
 * output tiles of the full rounds of 256 workgroups are computed whole and
 * the K units of the remaining tiles are shared evenly by the CUs
 * (stream-K; none when the tiles fill their rounds to 7/8 or more; with at
 * most 128 tiles each tile is split into floor(256 / tiles) equal pieces),
 * for 2 <= M <= 16 the weight tiles split along K.  Split tiles keep partials
 * in the workspace (M >= 256: fp16 per segment; M <= 16: fp32), summed in
 * fp32 in a fixed order (deterministic for a given shape and workspace
 * size; M >= 256 within fp16 rounding of each segment of the unsplit
 * product).  Same role
 * as the rocBLAS workspace behind the reference's at::mm_out in
 * dequant_matmul_out (hip:1973-1988). */
R4Q_API int r4q_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int wbits,
                                     size_t* bytes);
/* r4q_gemm with a caller-owned workspace of ws_bytes (NULL / 0: no split). */
R4Q_API int r4q_gemm_ws(const void* x, const void* w, const void* sz, void* y,
                        int64_t M, int64_t N, int64_t K, int wbits, void* ws,
                        size_t ws_bytes, void* stream);
/* Batched gate/up projection with the SiLU gate: y[M,I] fp16 =
 * FWHT-32(silu(g) * u), [g; u] = x W^T over W's 2I rows [gate; up],
 * bit-identical to r4q_gemm_ws with the same workspace into [M, 2I]
 * followed by r4q_silu_mul_fwht (in/out strides 2I / I).  For 2 <= M <= 16
 * and I % 32 == 0.  With a workspace that splits K (r4q_gemm_workspace_bytes
 * (M, 2I, K)) the split-K partial sum, the gate and the FWHT run in one
 * reduce kernel; for M <= 8 without one (NULL / too small to split) the
 * GEMM runs unsplit over tiles of 32 gate rows and the 32 up rows of the
 * same indices, with the gate and the FWHT in its epilogue.  Other cases
 * are rejected.  Replaces the batched decode step's launch_gemv
 * (gate_up) + silu_hadamard_ds pair (hip:1031-1051, hip:2508-2516). */
R4Q_API int r4q_gemm_silu_fwht_ws(const void* x, const void* w, const void* sz, void* y,
                                  int64_t M, int64_t I, int64_t K, int wbits, void* ws,
                                  size_t ws_bytes, void* stream);

/* y[N] = W x with x = FWHT32(fp16(a [+ b]) * rrms * gamma) (the activation
 * of r4q_res_rmsnorm_fwht / r4q_rmsnorm_fwht, bit-identical) computed inside
 * the GEMV; res_out = fp16(a + b) when b != NULL.  Batch 1, K <= 8192.
 * Replaces the launch_res_norm_fwht -> launch_gemv pairs of the reference's
 * decode step (hip:2505-2509 and the next layer's 2481 after :2518-2520;
 * launchers :1300-1313, :230-235). */
R4Q_API int r4q_res_rmsnorm_fwht_gemv(const void* a, const void* b, const void* gamma,
                              void* res_out, float eps, const void* w, const void* sz,
                              void* y, int64_t N, int64_t K, int wbits, void* stream);

/* The gate/up projection with the SiLU-gate folded in: [g; u] = W x with
 * W's rows [gate (I); up (I)], x = r4q_res_rmsnorm_fwht_gemv's activation
 * (gamma != NULL) or a itself (gamma == NULL, b and res_out unused), then
 * y[I] = fp16(FWHT32(silu(fp16(g)) * fp16(u))) -- bit-identical to the GEMV
 * followed by r4q_silu_mul_fwht.  Batch 1; I % 32 == 0; INT4 / INT8 with
 * K <= 5120-style rows (at most 64 lanes of 5 chunks per row).
 * Replaces the launch_gemv (gate_up) -> silu_hadamard_ds pair of the
 * reference's decode step (hip:2509-2513). */
R4Q_API int r4q_gate_up_silu_fwht(const void* a, const void* b, const void* gamma,
                          void* res_out, float eps, const void* w, const void* sz,
                          void* y, int64_t I, int64_t K, int wbits, void* stream);

/* The same pair split at a point, as the decode step runs it.
 * r4q_gate_up_silu writes y[i] = fp16(FWHT32(silu(fp16(g)) * fp16(u)))[i]
 * for i < split (fp16, as r4q_gate_up_silu_fwht) and h[i] = silu(fp16(g_i)) *
 * fp16(u_i) as fp32 for i >= split (no FWHT); split is a multiple of 32 in
 * [0, I], y and h are [I] arrays (only their own part is written; h 16-byte
 * aligned).  r4q_fwht_gemv computes y = W x with x[i] = x16[i] below split
 * and x = fp16(FWHT32(h)) per 32 elements above it, so x is bit-identical
 * to r4q_silu_mul_fwht's output and y to r4q_gemv of it.
 * The elements below the split go in 64-row units (32 gate + 32 up rows,
 * one workgroup each), the rest as pairs spread over every workgroup;
 * r4q_gate_up_silu_split returns the split that keeps whole units in
 * multiples of the CU count.
 * Replace the launch_gemv (gate_up) -> silu_hadamard_ds -> launch_gemv (down)
 * chain of the reference's decode step (hip:2508-2516). */
R4Q_API int r4q_gate_up_silu_split(int64_t I, int64_t* split);
R4Q_API int r4q_gate_up_silu(const void* a, const void* b, const void* gamma, void* res_out,
                     float eps, const void* w, const void* sz, void* y, float* h,
                     int64_t split, int64_t I, int64_t K, int wbits, void* stream);
R4Q_API int r4q_fwht_gemv(const void* x16, const float* h, int64_t split, const void* w,
                  const void* sz, void* y, int64_t N, int64_t K, int wbits, void* stream);

/* ------------------------------------------------------ norms / rotations */

/* y = fp16(x * rrms * w), rrms = 1/sqrt(mean(x^2) + eps), per row of D. */
R4Q_API int r4q_rmsnorm(const void* x, const void* w, void* y,
                int64_t rows, int64_t D, float eps, void* stream);
/* r = fp16(x + res) -> res_out; y = fp16(float(r) * rrms * w) with rrms from
 * the fp32 sum (x + res). */
R4Q_API int r4q_res_rmsnorm(const void* x, const void* res, const void* w, void* y,
                    void* res_out, int64_t rows, int64_t D, float eps,
                    void* stream);
/* y = fp16(H32 (x * rrms * w) / sqrt(32)) per 32-element chunk (D % 32 == 0). */
R4Q_API int r4q_rmsnorm_fwht(const void* x, const void* w, void* y,
                     int64_t rows, int64_t D, float eps, void* stream);
/* residual + RMSNorm + FWHT-32 in one pass: res_out = fp16(a + b);
 * y = FWHT32(float(res_out) * rrms * w) with rrms from the fp32 sum. */
R4Q_API int r4q_res_rmsnorm_fwht(const void* a, const void* b, const void* w,
                         void* y, void* res_out, int64_t rows, int64_t D,
                         float eps, void* stream);
/* y = fp16(H32 x / sqrt(32)) per 32-element chunk of n elements (n % 32 == 0). */
R4Q_API int r4q_fwht32(const void* x, void* y, int64_t n, void* stream);
/* y[r, i] = fp16(FWHT32(silu(g[r,i]) * u[r,i])), i < I; g/u row stride
 * `in_stride`, y row stride `out_stride` (elements).  y may alias g. */
R4Q_API int r4q_silu_mul_fwht(const void* g, const void* u, void* y, int64_t rows,
                      int64_t I, int64_t in_stride, int64_t out_stride,
                      void* stream);
/* y[r, i] = fp16(silu(g[r,i]) * u[r,i]) (no rotation). */
R4Q_API int r4q_silu_mul(const void* g, const void* u, void* y, int64_t rows,
                 int64_t I, int64_t in_stride, int64_t out_stride,
                 void* stream);

/* ---------------------------------------------------------- attention I/O */

/* Per-head RMSNorm of q [H, D] and k [Hk, D] into q_out / k_out (fp16). */
R4Q_API int r4q_head_rmsnorm(const void* q, const void* k, const void* qw,
                     const void* kw, void* q_out, void* k_out, int64_t H,
                     int64_t Hk, int64_t D, float eps, void* stream);
/* Half-split RoPE at position `pos` (tables cos/sin [P, D/2] fp16). */
R4Q_API int r4q_rope(const void* q, const void* k, const void* cos_t,
             const void* sin_t, void* q_out, void* k_out, int64_t H,
             int64_t Hk, int64_t D, int64_t pos, void* stream);
/* Decode-step QK-norm + RoPE + FP8 KV write for B sequences at one position.
 * q/k/v: row b at qkv + b*qkv_stride (q [H,D] | k [Hk,D] | v [Hk,D]).
 * q_out/k_out (fp16, may alias q/k) get the normed+rotated vectors; the K and
 * V caches [B, Hk, max_seq, D] get FP8 codes at `pos` (both NULL: no KV
 * write, max_seq unused).  k_scale / v_scale are [Hk] fp32 or NULL (scale 1).
 * Requires D == 128. */
R4Q_API int r4q_head_norm_rope_kv(const void* qkv, int64_t qkv_stride, const void* qw,
                          const void* kw, void* q_out, int64_t q_out_stride,
                          void* k_cache, void* v_cache, const float* k_scale,
                          const float* v_scale, const void* cos_t,
                          const void* sin_t, int64_t B, int64_t H, int64_t Hk,
                          int64_t D, float eps, int64_t max_seq, int64_t pos,
                          void* stream);

/* --------------------------------------------------------------- context */

typedef struct r4q_ctx r4q_ctx;
/* A context owns device scratch (attention partials, decode-step buffers,
 * captured graphs) for one device.  Not thread-safe; use one per stream. */
R4Q_API int r4q_ctx_create(r4q_ctx** out);
R4Q_API int r4q_ctx_destroy(r4q_ctx* ctx);

/* Split-K flash-decode over an FP8 KV cache for B sequences at seq_len
 * positions: out[b, h*D + d] = softmax(q k^T / sqrt(D)) v for query head h
 * and KV head h / (H/Hk).  q row b at q + b*q_stride.  When `fwht` != 0 the
 * output gets the FWHT-32 rotation (the O-projection input).  Requires
 * D == 128, H % Hk == 0. */
R4Q_API int r4q_flash_decode(r4q_ctx* ctx, const void* q, int64_t q_stride,
                     const void* k_cache, const void* v_cache,
                     const float* k_scale, const float* v_scale, void* out,
                     int64_t B, int64_t H, int64_t Hk, int64_t D,
                     int64_t max_seq, int64_t seq_len, int fwht, void* stream);

/* r4q_flash_decode without a context and without any device allocation.
 * No counterpart in the reference: for callers that cannot allocate (code
 * under hipGraph capture, serving loops and harnesses that forbid
 * hipMalloc).  The split partials live in a fixed 4 MiB device array per GPU
 * (held until the process ends), shared by every call on that GPU: calls
 * that overlap on one GPU race and must be serialised by the caller.  A
 * launch whose partials (B * H * splits * 528 bytes) exceed 4 MiB is
 * rejected with R4Q_EINVAL; the default split counts stay below it for any
 * GQA ratio up to 8.  The first call on each device looks up the array's
 * device address (hipGetSymbolAddress), no allocation.  Same results as
 * r4q_flash_decode, bit for bit. */
R4Q_API int r4q_flash_decode_noalloc(const void* q, int64_t q_stride, const void* k_cache,
                                     const void* v_cache, const float* k_scale,
                                     const float* v_scale, void* out, int64_t B, int64_t H,
                                     int64_t Hk, int64_t D, int64_t max_seq, int64_t seq_len,
                                     int fwht, void* stream);

/* The decode step's attention with its fused prologue, for one new position
 * `pos` of B sequences: qkv row b (at qkv + b*qkv_stride) holds the raw QKV
 * projection (q [H,D] | k [Hk,D] | v [Hk,D]); the kernel applies the
 * per-head RMSNorm + RoPE of r4q_head_norm_rope_kv to q and k (bit-identical
 * arithmetic), writes the FP8 codes of k and v at `pos` into the caches, and
 * attends over positions 0..pos (the split count follows the cache capacity
 * max_seq, as in the decode step).  out as r4q_flash_decode.  Replaces the
 * head_rmsnorm_rope_kv -> launch_flash_decode pair of the reference's decode
 * step (hip:1620-1683, hip:1547-1593, called at hip:2487-2500). */
R4Q_API int r4q_flash_decode_qkv(r4q_ctx* ctx, const void* qkv, int64_t qkv_stride,
                                 const void* q_norm, const void* k_norm, const void* cos_t,
                                 const void* sin_t, float eps, void* k_cache, void* v_cache,
                                 const float* k_scale, const float* v_scale, void* out,
                                 int64_t B, int64_t H, int64_t Hk, int64_t D, int64_t max_seq,
                                 int64_t rope_len, int64_t pos, int fwht, void* stream);

/* ----------------------------------------------------------- decode model */

/* One decoder layer's tensors.  *_bits is 4, 8 or 16 per matrix.
 * qkv = cat(q, k, v) rows; gate_up = cat(gate, up) rows. */
typedef struct r4q_layer {
  const void* qkv_w;  const void* qkv_s;  int64_t qkv_N;  int32_t qkv_bits;
  const void* o_w;    const void* o_s;    int64_t o_N;    int32_t o_bits;
  const void* gu_w;   const void* gu_s;   int64_t gu_N;   int32_t gu_bits;
  const void* down_w; const void* down_s; int64_t down_N; int32_t down_bits;
  const void* in_norm; const void* post_norm; const void* q_norm;
  const void* k_norm;
  void* k_cache; void* v_cache;              /* [B, Hk, max_seq, D] uint8 */
  const float* k_scale; const float* v_scale;/* [Hk] fp32 or NULL        */
} r4q_layer;

typedef struct r4q_model {
  int32_t n_layers, n_heads, n_kv_heads, head_dim, hidden, inter;
  float eps;
  int32_t max_seq;         /* KV cache capacity (positions)            */
  int32_t rope_len;        /* rows of the RoPE tables                  */
  const r4q_layer* layers; /* n_layers entries                         */
  const void* rope_cos; const void* rope_sin; /* [rope_len, D/2] fp16   */
  const void* final_norm;  /* [hidden] fp16 (NULL: no LM head)         */
  const void* lm_w; const void* lm_s; int64_t lm_N, lm_K; int32_t lm_bits;
  const void* embed;       /* [vocab, hidden] fp16 or NULL             */
  int64_t vocab;
} r4q_model;

/* One decode step for B sequences at position `pos` (same for all rows).
 * hidden_in [B, hidden] fp16.  Writes hidden_out [B, hidden] (may be NULL)
 * and, when logits != NULL and the model has an LM head, logits [B, lm_N]
 * fp16.  KV caches are written at `pos`; positions < pos must be filled. */
R4Q_API int r4q_decode_step(r4q_ctx* ctx, const r4q_model* m, const void* hidden_in,
                    int64_t B, int64_t pos, void* hidden_out, void* logits,
                    void* stream);
/* r4q_decode_step replayed from a captured hipGraph: the first call for a
 * (model, B, buffers) combination captures the step with the position held
 * in device memory, later calls at any position set that position and replay
 * it (about 250 launches become one).  Bit-identical results to
 * r4q_decode_step.  On a stream that the caller is capturing it records the
 * eager launches instead.  A caller that waits for every token before the
 * next (the engine's per-token decode_step_logits, int4_engine_v5.py:272 ->
 * hip:2534-2595) is faster with r4q_decode_step: the GPU starts on the
 * first eager launch, but on a replay only once hipGraphLaunch returns. */
R4Q_API int r4q_decode_step_graph(r4q_ctx* ctx, const r4q_model* m, const void* hidden_in,
                                  int64_t B, int64_t pos, void* hidden_out, void* logits,
                                  void* stream);
/* How the decode step runs a model at batch B, without running it (no
 * counterpart in the reference; for tests and measurement):
 * out[0] = attention split count (from the cache capacity),
 * out[1] = layers whose gate/up projection applies the SiLU gate + FWHT-32
 * in the same launch (batch 1: the GEMV's SiLU epilogue; batch > 1: the
 * split-K reduce of the skinny GEMM); with n >= 3, out[2] = projections
 * (qkv, o, down over all layers) whose split-K partials are summed by the
 * kernel consuming them -- attention prologue, row norm -- with no reduce
 * launch (batch > 1).  n >= 2. */
R4Q_API int r4q_decode_plan(const r4q_model* m, int64_t B, int32_t* out, int64_t n);
/* Run `num_tokens` steps from start_pos.  use_graph != 0 captures one step
 * into a hipGraph and replays it with the position held in device memory.
 * Greedy next token (argmax + embedding gather) runs on the device between
 * steps when the model has an embedding; token ids (int64 [num_tokens, B])
 * are written to `tokens_out` when it is not NULL.  B sequences.  At most
 * two steps are queued ahead of the GPU (a deeper queue of steps runs them
 * slower), so the call returns once all but the last two steps have run. */
R4Q_API int r4q_decode_bench(r4q_ctx* ctx, const r4q_model* m, const void* hidden_in,
                     int64_t B, int64_t num_tokens, int64_t start_pos,
                     int use_graph, void* tokens_out, void* stream);
/* r4q_decode_bench with temperature / top-p sampling of each next token on
 * the device (the reference samples in Python, int4_engine_v5.py:387-399):
 * temperature > 0 draws from softmax(logits / temperature) restricted to
 * the tokens whose cumulative probability before them (descending order,
 * ties by index) is < top_p (top_p >= 1 keeps all); the uniform draw of row
 * b at position pos is splitmix64(splitmix64(seed ^ pos) ^ b) >> 40 / 2^24.
 * temperature == 0 is the greedy loop of r4q_decode_bench. */
R4Q_API int r4q_decode_generate(r4q_ctx* ctx, const r4q_model* m, const void* hidden_in,
                                int64_t B, int64_t num_tokens, int64_t start_pos,
                                int use_graph, float temperature, float top_p, uint64_t seed,
                                void* tokens_out, void* stream);
/* Next token of each of B rows of fp16 logits [B, row_stride] (first V used)
 * with the rule of r4q_decode_generate, `counter` in place of the position;
 * temperature <= 0 is argmax (lowest index of the maximum).  Replaces the
 * reference's Python sampling (int4_engine_v5.py:330-335, 387-399);
 * ids_out: int64 [B] on the device.  Logits must not be NaN. */
R4Q_API int r4q_sample(r4q_ctx* ctx, const void* logits, int64_t B, int64_t V, int64_t row_stride,
                       float temperature, float top_p, uint64_t seed, int64_t counter,
                       int64_t* ids_out, void* stream);
/* Time one step by kernel category with HIP events:
 * out_ms[5] = {total, gemv, attention, norm, rest}. */
R4Q_API int r4q_decode_profile(r4q_ctx* ctx, const r4q_model* m, const void* hidden_in,
                       int64_t pos, float* out_ms, void* stream);

/* Measurement aid with no counterpart in the reference: overrides one
 * launch-shape choice for the whole process (value 0 restores the built-in
 * choice).  Knobs: "gemv_lpr" (lanes per GEMV row: 16..256, power of two),
 * "gemv_wgs" (GEMV workgroup cap, 1..65536), "gemv_ub" (GEMV steps in flight
 * per lane, 1..2), "attn_splits" (flash-decode splits, 1..128), "skinny_splits"
 * (skinny GEMM K splits, 1..8), "gemm_splits" (ring GEMM: 1 = whole tiles
 * only, 2..16 = stream-K with about that many workgroups per tile),
 * "split_reduce" (1 = batched decode steps reduce the split-K partials of
 * the qkv, o and down projections in their own launches, not in the
 * attention prologue / row norm that consume them), "gemm_kernel" (GEMM for
 * M >= 256: 1 = the ring kernel (the default), 2 = the specialised-wave
 * kernel where it applies: INT4, N % 128 == 0, K % 256 == 0), "gemv_skew"
 * (GEMV on an even grid of more than 256 equal shares: the first half of the
 * workgroups takes value - 1 steps more and the second half value - 1 fewer;
 * 1 = equal shares; default 2 on a 512-workgroup grid of at least 4 steps
 * each).
 * Initial values come from R4Q_GEMV_LPR, R4Q_GEMV_WGS, R4Q_GEMV_UB,
 * R4Q_ATTN_SPLITS, R4Q_SKINNY_SPLITS, R4Q_GEMM_SPLITS, R4Q_SPLIT_REDUCE,
 * R4Q_GEMM_KERNEL, R4Q_GEMV_SKEW, read once.  Results do
 * not depend on these choices beyond fp32 summation order (split counts) --
 * they exist for sweeps and tests.  Captured decode graphs are keyed by the
 * values in force. */
R4Q_API int r4q_tune(const char* name, int value);

/* Measurement aid with no counterpart in the reference: reads `bytes` bytes
 * at src (16-byte aligned) once, with the fastest plain-read layout measured
 * on MI355X, so that a kernel's duration can be set against the HBM read
 * floor for the same byte count.  sink: device scratch of >= 8192 bytes,
 * normally left untouched. */
R4Q_API int r4q_hbm_read(const void* src, int64_t bytes, void* sink, int64_t sink_bytes,
                         void* stream);

/* Prefill M tokens from position 0: embedding of ids (int64 [M]) through all
 * layers; writes logits [M, lm_N] fp16 (NULL: skip the LM head) and, when
 * write_kv != 0, the FP8 KV caches at positions 0..M-1. */
R4Q_API int r4q_prefill_logits(r4q_ctx* ctx, const r4q_model* m, const void* ids,
                       int64_t M, void* logits, int write_kv, void* stream);
/* The prefill's causal GQA self-attention alone (the step r4q_prefill_logits
 * runs after the head norm + RoPE): qkv rows [M, stride] fp16 hold H query
 * heads, then Hk key and Hk value heads of head_dim 128; out[M, out_stride]
 * gets FWHT32(softmax_{j<=m}(q_m . k_j / sqrt(128)) V) per query head.
 * Replaces the causal SDPA of int4_prefill_logits (hip:2254-2265) and the
 * FWHT-32 after it (hip:2269). */
R4Q_API int r4q_prefill_attention(const void* qkv, int64_t stride, void* out,
                                  int64_t out_stride, int64_t M, int64_t H, int64_t Hk,
                                  void* stream);

#ifdef __cplusplus
}
#endif
#endif /* R4Q_H */
