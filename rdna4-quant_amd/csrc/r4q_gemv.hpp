// Internal interface of the GEMV translation unit (used by the decode step).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace r4q {

// Validates a batch-1 GEMV request; returns R4Q_OK or an R4Q_E* code.
int gemv_check(const void* x, const void* w, const void* sz, const void* y, int64_t N,
               int64_t K, int wbits);
// Enqueues y = W x on `st` (arguments already validated).
int gemv_launch(const void* x, const void* w, const void* sz, void* y, int64_t N, int64_t K,
                int wbits, hipStream_t st);

// y = W x with x = FWHT32(fp16(a [+ b]) * rrms * gamma) computed in the
// GEMV's activation staging (residual + RMSNorm + FWHT-32 fused); workgroup 0
// writes res_out = fp16(a + b) when b != NULL.  gamma == NULL: plain x = a.
// K <= 8192 with a norm, batch 1.  silu (W's rows [gate; up], N = 2I, g and
// u the fp16-rounded rows; needs gemv_silu_ok(N, K, wbits)):
//   kUnit:  y[I] = fp16(FWHT32(silu(g) * u)), the SiLU-gate kernel fused
//           into the epilogue (one workgroup per 64-row unit);
//   kSplit: the same for elements [0, split) (one workgroup per 64-row unit,
//           split / 32 of them), and h[i] = silu(g_i) * u_i as fp32 for
//           i >= split, without the FWHT: gemv_fwht_launch applies it in the
//           next GEMV's staging.  gemv_silu_split() gives a split whose
//           units spread evenly over the CUs.
enum class SiluEpi { kNone, kUnit, kSplit };
int gemv_norm_launch(const void* a, const void* b, const void* gamma, void* res_out, float eps,
                     const void* w, const void* sz, void* y, int64_t N, int64_t K, int wbits,
                     hipStream_t st, SiluEpi silu = SiluEpi::kNone, float* h = nullptr,
                     int64_t split = 0);
bool gemv_silu_ok(int64_t N, int64_t K, int wbits);
int64_t gemv_silu_split(int64_t I);
// y = W x with x[i] = x16[i] for i < split and fp16(FWHT32(h)) per 32
// elements above (K % 32 == 0): the down projection after a kSplit gate/up
// GEMV, x bit-identical to the SiLU-gate kernel's output.
int gemv_fwht_launch(const void* x16, const float* h, int64_t split, const void* w,
                     const void* sz, void* y, int64_t N, int64_t K, int wbits, hipStream_t st);

// Row counts up to this use the weight-streaming GEMV path; above it the
// MFMA tile GEMM with on-the-fly dequantisation.
constexpr int64_t kSkinnyMaxRows = 16;

// MFMA GEMM (r4q_gemm.hip), arguments validated by the caller.  ws
// (ws_bytes of device memory, may be null) holds the fp32 partials of a
// split-K launch; gemm_splits() gives the split count a workspace allows
// (1: none needed).
constexpr int kMaxGemmSplits = 16;
int gemm_splits(int64_t M, int64_t N, int64_t K, int wbits, size_t ws_bytes);
// Workspace bytes for the best split count of a shape (0: none needed).
size_t gemm_ws_bytes(int64_t M, int64_t N, int64_t K, int wbits);
int gemm_mfma_launch(const void* x, const void* w, const void* sz, void* y, int64_t M, int64_t N,
                     int64_t K, int wbits, hipStream_t st, void* ws = nullptr,
                     size_t ws_bytes = 0);

// Skinny MFMA GEMM for 2 <= M <= 16 rows (weights streamed once); usable
// when gemm_skinny_ok(M, N, K, wbits).  With a workspace of at least
// skinny_ws_bytes() narrow shapes are split along K (fp32 partials).
bool gemm_skinny_ok(int64_t M, int64_t N, int64_t K, int wbits);
size_t skinny_ws_bytes(int64_t M, int64_t N, int64_t K, int wbits);
// K split count the skinny GEMM takes for a shape given ws_bytes of workspace.
int skinny_splits(int64_t M, int64_t N, int64_t K, int wbits, size_t ws_bytes);
int gemm_skinny_launch(const void* x, const void* w, const void* sz, void* y, int64_t M,
                       int64_t N, int64_t K, int wbits, hipStream_t st, void* ws = nullptr,
                       size_t ws_bytes = 0);
// The same GEMM without its split reduce: *S = the K split count; S > 1
// leaves the S fp32 planes part[s][m][n] (part = ws) for the consumer to sum
// in split order and round to fp16 (what the reduce stores); S == 1 writes y.
int gemm_skinny_part_launch(const void* x, const void* w, const void* sz, void* y, int64_t M,
                            int64_t N, int64_t K, int wbits, hipStream_t st, void* ws,
                            size_t ws_bytes, int* S);
// The same GEMM over N = 2I gate/up columns with the SiLU gate and FWHT-32
// fused: y (M x I fp16) = FWHT-32(silu(gate) * up), equal to the plain GEMM
// with the same workspace followed by silu_mul_fwht.  A workspace that
// splits K puts the gate in the split sum; without one (M <= 8) it runs in
// the unsplit GEMM's epilogue (gemm_skinny_silu_ok).
bool gemm_skinny_silu_ok(int64_t M, int64_t I, int64_t K, int wbits, size_t ws_bytes);
int gemm_skinny_silu_launch(const void* x, const void* w, const void* sz, void* y, int64_t M,
                            int64_t I, int64_t K, int wbits, hipStream_t st, void* ws,
                            size_t ws_bytes);
// The same unsplit SiLU GEMM (M <= 8) with the units past the last whole
// round of 256 cut along K into pieces spread over the CUs; tail_ws holds
// skinny_silu_tail_bytes(I, K, wbits) bytes, of which the first
// skinny_silu_tail_cnt_bytes(I) (arrival counters, the same for every
// width) are zero before the call and after it.  tail_ws == NULL: the
// plain unsplit launch.
size_t skinny_silu_tail_bytes(int64_t I, int64_t K, int wbits);
size_t skinny_silu_tail_cnt_bytes(int64_t I);
int gemm_skinny_silu_tail_launch(const void* x, const void* w, const void* sz, void* y, int64_t M,
                                 int64_t I, int64_t K, int wbits, hipStream_t st, void* tail_ws);

// Workspace bytes gemm_launch can use for a shape (0: none), over both the
// skinny (M <= 16) and the tiled paths.
size_t gemm_ws_need(int64_t M, int64_t N, int64_t K, int wbits);

// y[M,N] = x[M,K] W^T; rows of x and y contiguous.  ws: optional split-K
// workspace (see gemm_mfma_launch).
int gemm_launch(const void* x, const void* w, const void* sz, void* y, int64_t M, int64_t N,
                int64_t K, int wbits, hipStream_t st, void* ws = nullptr, size_t ws_bytes = 0);

}  // namespace r4q
