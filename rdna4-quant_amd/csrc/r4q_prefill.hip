// Kernels of the prompt (prefill) pass that the decode step does not have:
// the embedding gather and causal self-attention over the prompt's own
// fp16 Q/K/V.
//
// Reference: int4_prefill_logits (hip:2127-2320) gathers embeddings with
// torch::embedding (:2172) and runs causal SDPA with GQA on the fp16
// head-normed, RoPE'd Q/K and raw V (:2254-2265), followed by the FWHT-32
// of the attention output (:2269).  Here the FWHT runs in the attention
// kernel's epilogue, before the single fp16 rounding.
#include <math.h>

#include "r4q_device.hpp"
#include "r4q_host.hpp"
#include "r4q_kernels.hpp"

namespace r4q {
namespace {

// out[m, :] = table[ids[m], :] (fp16 rows of D elements, D % 8 == 0).
// ids are range-checked on the host before launch.
__global__ __launch_bounds__(256) void embed_gather_kernel(const int64_t* __restrict__ ids,
                                                           const uint16_t* __restrict__ table,
                                                           uint16_t* __restrict__ out, int D) {
  const int64_t m = blockIdx.x;
  const u4_t* src = reinterpret_cast<const u4_t*>(table + ids[m] * (int64_t)D);
  u4_t* dst = reinterpret_cast<u4_t*>(out + m * (int64_t)D);
  for (int i = threadIdx.x; i < D / 8; i += blockDim.x) dst[i] = src[i];
}

// Causal GQA flash attention on the matrix cores (v_mfma_f32_16x16x32_f16).
// A workgroup (4 waves) takes 64 query rows of one query head; wave w owns
// rows q0 + 16w .. +15.  Rows of `qkv` (stride `stride` elements) hold q
// heads at h*128, k heads at (H + kh)*128 and v heads at (H + Hk + kh)*128,
// kh = h / (H/Hk).  out[m, h*128 + d] =
//   FWHT32(softmax_{j <= m}(q_m . k_j / sqrt(128)) V)[d].
// Keys go in blocks of 32 through LDS (K row-major, V transposed), the next
// block's global loads in flight during the current block's arithmetic.
// Per block and wave (lane l: column n = l % 16, group g = l / 16):
//  * S^T = K Q^T for two 16-key halves: A = K (lane: key n of the half,
//    dims 32k + 8g .. over the 4 k-steps), B = Q^T (lane: query row n, the
//    same dims, held in registers for the whole loop).  C: lane holds query
//    n at keys 4g .. 4g+3 of the half;
//  * online softmax per query across the 4 lanes holding it, probabilities
//    rounded to fp16, keys past the query (or the prompt) masked;
//  * O += P V: A = P (lane: query n; k-slots = its 8 keys 4g + r and
//    16 + 4g + r), B = V (lane: dim 16j + n of N-block j, the same keys,
//    two 8-byte reads of the transposed block).  C: lane holds dim 16j + n
//    of queries 4g .. 4g+3.
// Epilogue: O / l, FWHT-32 per 32-dim chunk (the 16-dim step inside the
// lane, steps 1 .. 8 across lanes xor 1 .. 8), one fp16 rounding.
constexpr int kFaKRow = 136;  // halves per K row in LDS (128 + 8 pad)
constexpr int kFaVRow = 36;   // halves per transposed-V row (32 keys + 4 pad)

__global__ __launch_bounds__(256) void prefill_fa_kernel(const uint16_t* __restrict__ qkv,
                                                         int64_t stride,
                                                         uint16_t* __restrict__ out,
                                                         int64_t out_stride, int M, int H,
                                                         int Hk) {
  __shared__ __align__(16) uint16_t ks[32 * kFaKRow];
  __shared__ __align__(16) uint16_t vt[128 * kFaVRow];
  const int h = blockIdx.x, q0 = blockIdx.y * 64;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int col = lane & 15, g = lane >> 4;
  const int kh = h / (H / Hk);
  const uint16_t* kbase = qkv + (int64_t)(H + kh) * 128;
  const uint16_t* vbase = qkv + (int64_t)(H + Hk + kh) * 128;
  const int r0 = q0 + 16 * wave;  // this wave's first query row
  const int kend = min(q0 + 64, M);  // the workgroup needs keys [0, kend)
  const int nkb = (kend + 31) / 32;

  // Q^T fragments: qb[k] = Q[row r0 + col][32k + 8g .. +7] (rows past M clamped)
  u4_t qb[4];
  {
    const uint16_t* qr = qkv + (int64_t)min(r0 + col, M - 1) * stride + h * 128 + 8 * g;
#pragma unroll
    for (int k = 0; k < 4; ++k) qb[k] = *reinterpret_cast<const u4_t*>(qr + 32 * k);
  }
  // block staging: piece t and t + 256 of 512 16-byte pieces (key t / 16,
  // dims 8 (t % 16) ..) for K and for V; keys past the prompt clamped
  u4_t kp[2], vp[2];
  auto load_block = [&](int kb) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int pc = t + 256 * i, key = min(32 * kb + (pc >> 4), M - 1), d8 = 8 * (pc & 15);
      kp[i] = *reinterpret_cast<const u4_t*>(kbase + (int64_t)key * stride + d8);
      vp[i] = *reinterpret_cast<const u4_t*>(vbase + (int64_t)key * stride + d8);
    }
  };
  auto store_block = [&]() {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int pc = t + 256 * i, key = pc >> 4, d8 = 8 * (pc & 15);
      *reinterpret_cast<u4_t*>(ks + key * kFaKRow + d8) = kp[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vt[(d8 + 2 * e) * kFaVRow + key] = (uint16_t)(vp[i][e] & 0xFFFFu);
        vt[(d8 + 2 * e + 1) * kFaVRow + key] = (uint16_t)(vp[i][e] >> 16);
      }
    }
  };

  const float sscale = 0.08838834764831845f;  // 1 / sqrt(128)
  const uint32_t ones = 0x3C003C00u;           // fp16 (1, 1)
  float m_run = -INFINITY, l_run = 0.f;        // query col; l over this lane's keys
  f4_t o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = f4_t{0.f, 0.f, 0.f, 0.f};
  auto kpos = [&](int s) { return s < 4 ? 4 * g + s : 16 + 4 * g + (s - 4); };

  load_block(0);
  for (int kb = 0; kb < nkb; ++kb) {
    __syncthreads();  // the previous block's LDS reads are done
    store_block();
    __syncthreads();
    if (kb + 1 < nkb) load_block(kb + 1);  // in flight during this block
    if (32 * kb > r0 + 15) continue;       // wave-uniform: block entirely past this wave's rows
    // ---- S^T = K Q^T
    f4_t sacc[2];
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      sacc[bb] = f4_t{0.f, 0.f, 0.f, 0.f};
      const uint16_t* kr = ks + (16 * bb + col) * kFaKRow + 8 * g;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        sacc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            __builtin_bit_cast(h8_t, *reinterpret_cast<const u4_t*>(kr + 32 * k)),
            __builtin_bit_cast(h8_t, qb[k]), sacc[bb], 0, 0, 0);
    }
    // ---- online softmax for query r0 + col over keys 32 kb + kpos(s)
    const int qabs = r0 + col;
    float sv[8];
#pragma unroll
    for (int s = 0; s < 8; ++s)
      sv[s] = (32 * kb + kpos(s) <= qabs) ? sacc[s >> 2][s & 3] * sscale : -INFINITY;
    float mx = sv[0];
#pragma unroll
    for (int s = 1; s < 8; ++s) mx = fmaxf(mx, sv[s]);
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mn = fmaxf(m_run, mx);  // finite: key 32 kb <= r0 <= qabs is unmasked
    const float alpha = (m_run == -INFINITY) ? 0.f : __expf(m_run - mn);
    u4_t pa;  // fp16 probabilities, k-slot s = key kpos(s)
    float lp = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p0 = __expf(sv[2 * i] - mn), p1 = __expf(sv[2 * i + 1] - mn);
      pa[i] = cvt_pk_h(p0, p1);
      lp = __builtin_amdgcn_fdot2(as_h2(pa[i]), as_h2(ones), lp, false);
    }
    l_run = __builtin_fmaf(l_run, alpha, lp);
    m_run = mn;
    float ar[4];  // alpha of the C rows' queries 4g + r (lane 4g + r holds that query)
#pragma unroll
    for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, 4 * g + r);
    // ---- O += P V
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint16_t* vr = vt + (16 * j + col) * kFaVRow + 4 * g;
      const u2_t lo = *reinterpret_cast<const u2_t*>(vr);
      const u2_t hi = *reinterpret_cast<const u2_t*>(vr + 16);
      const u4_t vb = u4_t{lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
      for (int r = 0; r < 4; ++r) o[j][r] *= ar[r];
      o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, pa),
                                                    __builtin_bit_cast(h8_t, vb), o[j], 0, 0, 0);
    }
  }
  // ---- O / l, FWHT-32, fp16 out (rows 4g + r of the wave's 16)
  float lsum = l_run + __shfl_xor(l_run, 16);
  lsum += __shfl_xor(lsum, 32);
  float inv[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) inv[r] = 1.0f / __shfl(lsum, 4 * g + r);
#pragma unroll
  for (int c = 0; c < 4; ++c) {  // 32-dim chunk c = N-blocks 2c, 2c+1
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float a = o[2 * c][r] * inv[r], b = o[2 * c + 1][r] * inv[r];
      {  // element bit 4 (dims 16 apart) inside the lane
        const float t0 = a + b, t1 = a - b;
        a = t0;
        b = t1;
      }
#pragma unroll
      for (int bit = 1; bit <= 8; bit <<= 1) {  // element bits 0..3 across lanes
        const float oa = __shfl_xor(a, bit), ob = __shfl_xor(b, bit);
        if (col & bit) {
          a = oa - a;
          b = ob - b;
        } else {
          a = a + oa;
          b = b + ob;
        }
      }
      const int row = r0 + 4 * g + r;
      if (row < M) {
        uint16_t* dst = out + (int64_t)row * out_stride + h * 128 + 32 * c + col;
        dst[0] = f2h(a * kInvSqrt32);
        dst[16] = f2h(b * kInvSqrt32);
      }
    }
  }
}

}  // namespace

int launch_embed_gather(const int64_t* ids, const void* table, void* out, int64_t M, int64_t D,
                        hipStream_t st) {
  if (M == 0) return R4Q_OK;
  hipLaunchKernelGGL(embed_gather_kernel, dim3((unsigned)M), dim3(256), 0, st, ids,
                     static_cast<const uint16_t*>(table), static_cast<uint16_t*>(out), (int)D);
  return launch_status("embed_gather");
}

int launch_prefill_attention(const void* qkv, int64_t stride, void* out, int64_t out_stride,
                             int64_t M, int64_t H, int64_t Hk, hipStream_t st) {
  if (M == 0) return R4Q_OK;
  hipLaunchKernelGGL(prefill_fa_kernel, dim3((unsigned)H, (unsigned)((M + 63) / 64)), dim3(256),
                     0, st, static_cast<const uint16_t*>(qkv), stride,
                     static_cast<uint16_t*>(out), out_stride, (int)M, (int)H, (int)Hk);
  return launch_status("prefill_attention");
}

}  // namespace r4q

extern "C" int r4q_prefill_attention(const void* qkv, int64_t stride, void* out,
                                     int64_t out_stride, int64_t M, int64_t H, int64_t Hk,
                                     void* stream) {
  R4Q_REQUIRE(qkv && out, "prefill_attention: null pointer");
  R4Q_REQUIRE(M >= 1 && M < (1LL << 31), "prefill_attention: bad row count");
  R4Q_REQUIRE(H >= 1 && Hk >= 1 && H % Hk == 0, "prefill_attention: bad head counts");
  R4Q_REQUIRE(stride >= (H + 2 * Hk) * 128 && stride % 8 == 0 && out_stride >= H * 128 &&
                  (reinterpret_cast<uintptr_t>(qkv) & 15) == 0,
              "prefill_attention: rows must be 16-byte aligned and hold H + 2 Hk heads of 128");
  return r4q::launch_prefill_attention(qkv, stride, out, out_stride, M, H, Hk,
                                       r4q::as_stream(stream));
}
