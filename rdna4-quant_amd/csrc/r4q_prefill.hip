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

// Causal GQA attention for one (query row m, query head h) per wave.
// Rows of `qkv` (stride `stride` elements) hold q heads at h*128, k heads at
// (H + kh)*128 and v heads at (H + Hk + kh)*128, kh = h / (H/Hk).
// out[m, h*128 + d] = FWHT32(softmax_j<=m(q_m . k_j / sqrt(128)) v_j)[d].
//  * keys in blocks of 64, lane j scores key j0+j with the whole q row in
//    registers (64 fp16 pairs, v_dot2_f32_f16), online softmax in fp32;
//  * P V: lane l owns dims 2l and 2l+1; each key's probability is broadcast
//    with v_readlane; all V loads of a block are issued before the FMAs
//    (rows past the causal end are clamped and carry p = 0);
//  * the FWHT-32 butterflies run across lanes (a 32-dim chunk spans 16
//    lanes) with the same operations per element as the register version.
__global__ __launch_bounds__(256) void prefill_attn_kernel(const uint16_t* __restrict__ qkv,
                                                           int64_t stride,
                                                           uint16_t* __restrict__ out,
                                                           int64_t out_stride, int M, int H,
                                                           int Hk) {
  const int h = blockIdx.x;
  const int m = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (m >= M) return;  // whole wave; the kernel has no barriers
  const int kh = h / (H / Hk);
  const uint16_t* kbase = qkv + (int64_t)(H + kh) * 128;
  const uint16_t* vbase = qkv + (int64_t)(H + Hk + kh) * 128;

  uint32_t qv[64];
  {
    const u4_t* qr = reinterpret_cast<const u4_t*>(qkv + (int64_t)m * stride + h * 128);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const u4_t v = qr[i];
      qv[4 * i] = v[0];
      qv[4 * i + 1] = v[1];
      qv[4 * i + 2] = v[2];
      qv[4 * i + 3] = v[3];
    }
  }
  const float scale = 0.08838834764831845f;  // 1 / sqrt(128)
  float m_run = -INFINITY, l_run = 0.f, o0 = 0.f, o1 = 0.f;
  for (int j0 = 0; j0 <= m; j0 += 64) {
    const int j = j0 + lane;
    const bool valid = j <= m;
    const u4_t* kr = reinterpret_cast<const u4_t*>(kbase + (int64_t)min(j, m) * stride);
    uint32_t vv[64];
#pragma unroll
    for (int t = 0; t < 64; ++t)  // clamped rows: loads stay inside the prompt
      vv[t] = *reinterpret_cast<const uint32_t*>(vbase + (int64_t)min(j0 + t, m) * stride +
                                                 2 * lane);
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const u4_t k = kr[i];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        s = __builtin_amdgcn_fdot2(as_h2(k[e]), as_h2(qv[4 * i + e]), s, false);
    }
    dot_dpp_fence();
    s = valid ? s * scale : -INFINITY;
    const float mn = fmaxf(m_run, wave_max(s));  // finite: key j0 <= m is valid
    const float alpha = __expf(m_run - mn);
    const float p = valid ? __expf(s - mn) : 0.f;
    l_run = __builtin_fmaf(l_run, alpha, wave_sum(p));
    o0 *= alpha;
    o1 *= alpha;
#pragma unroll
    for (int t = 0; t < 64; ++t) {
      const float pt = readlane_f(p, t);
      o0 = __builtin_fmaf(pt, h2f((uint16_t)(vv[t] & 0xFFFFu)), o0);
      o1 = __builtin_fmaf(pt, h2f((uint16_t)(vv[t] >> 16)), o1);
    }
    m_run = mn;
  }
  const float inv = 1.0f / l_run;
  float a = o0 * inv, b = o1 * inv;
  // FWHT-32: step 1 inside the lane, steps 2..16 across lanes xor 1..8
  {
    const float t0 = a + b, t1 = a - b;
    a = t0;
    b = t1;
  }
#pragma unroll
  for (int bit = 1; bit <= 8; bit <<= 1) {
    const float oa = __shfl_xor(a, bit), ob = __shfl_xor(b, bit);
    if (lane & bit) {
      a = oa - a;
      b = ob - b;
    } else {
      a = a + oa;
      b = b + ob;
    }
  }
  a *= kInvSqrt32;
  b *= kInvSqrt32;
  *reinterpret_cast<uint32_t*>(out + (int64_t)m * out_stride + h * 128 + 2 * lane) =
      (uint32_t)f2h(a) | ((uint32_t)f2h(b) << 16);
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
  hipLaunchKernelGGL(prefill_attn_kernel, dim3((unsigned)H, (unsigned)((M + 3) / 4)), dim3(256),
                     0, st, static_cast<const uint16_t*>(qkv), stride,
                     static_cast<uint16_t*>(out), out_stride, (int)M, (int)H, (int)Hk);
  return launch_status("prefill_attention");
}

}  // namespace r4q
