// Weight dequantisation and FP8 KV codec kernels.
//
// dequant_int4 replaces the reference's dequant_int4_kernel (hip:3568-3603),
// fp16_to_fp8 its fp16_to_fp8_kernel (hip:3606-3618).  The dequantised value
// is fp16(float(q - zp) * float(scale)): the fp32 product is exact (at most
// 9 + 11 significant bits) so the single fp16 rounding makes the result
// bit-identical to the reference's torch path (int4_quant_v2.py:105-127).
#include "r4q_device.hpp"
#include "r4q_host.hpp"

namespace r4q {
namespace {

// One thread per 32-element block: 16 B of nibbles (INT4) or 32 B (INT8) in,
// 64 B of fp16 out, all 128-bit accesses.
template <int WBITS>
__global__ __launch_bounds__(256) void dequant_kernel(
    const uint8_t* __restrict__ w, const uint32_t* __restrict__ sz,
    uint16_t* __restrict__ out, int64_t nblocks_total, int64_t K) {
  const int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (blk >= nblocks_total) return;
  const uint32_t s2 = sz[blk];
  const float scale = h2f((uint16_t)(s2 & 0xFFFFu));
  const float zp = h2f((uint16_t)(s2 >> 16));
  uint32_t q[32];
  if constexpr (WBITS == 4) {
    const u4_t p = *reinterpret_cast<const u4_t*>(w + blk * 16);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int t = 0; t < 8; ++t) q[8 * j + t] = (p[j] >> (4 * t)) & 0xFu;
  } else {
    const u4_t p0 = *reinterpret_cast<const u4_t*>(w + blk * 32);
    const u4_t p1 = *reinterpret_cast<const u4_t*>(w + blk * 32 + 16);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        q[4 * j + t] = (p0[j] >> (8 * t)) & 0xFFu;
        q[16 + 4 * j + t] = (p1[j] >> (8 * t)) & 0xFFu;
      }
  }
  u4_t o[4];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float plo = ((float)q[2 * i] - zp) * scale;  // exact in fp32
    const float phi = ((float)q[2 * i + 1] - zp) * scale;
    o[i / 4][i % 4] = (uint32_t)f2h(plo) | ((uint32_t)f2h(phi) << 16);
  }
  u4_t* dst = reinterpret_cast<u4_t*>(out + blk * 32);
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[i] = o[i];
  (void)K;
}

__global__ __launch_bounds__(256) void fp16_to_fp8_kernel(
    const uint16_t* __restrict__ src, uint8_t* __restrict__ dst, int64_t n) {
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i0 + 4 <= n) {
    const u2_t v = *reinterpret_cast<const u2_t*>(src + i0);
    const uint32_t c0 = fp8_encode(h2f((uint16_t)(v[0] & 0xFFFF)));
    const uint32_t c1 = fp8_encode(h2f((uint16_t)(v[0] >> 16)));
    const uint32_t c2 = fp8_encode(h2f((uint16_t)(v[1] & 0xFFFF)));
    const uint32_t c3 = fp8_encode(h2f((uint16_t)(v[1] >> 16)));
    *reinterpret_cast<uint32_t*>(dst + i0) = c0 | (c1 << 8) | (c2 << 16) | (c3 << 24);
  } else {
    for (int64_t i = i0; i < n; ++i) dst[i] = (uint8_t)fp8_encode(h2f(src[i]));
  }
}

__global__ __launch_bounds__(256) void fp8_to_fp16_kernel(
    const uint8_t* __restrict__ src, uint16_t* __restrict__ dst, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint32_t h = fp8x2_to_h2_div256(src[i]);
  dst[i] = f2h(h2f((uint16_t)(h & 0xFFFF)) * 256.0f);
}

bool aligned(const void* p, int a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

template <int WBITS>
int dequant(const void* w, const void* sz, void* out, int64_t N, int64_t K, void* stream) {
  R4Q_REQUIRE(w && sz && out, "dequant_int%d: null pointer", WBITS);
  R4Q_REQUIRE(N > 0 && K > 0 && K % 32 == 0,
              "dequant_int%d: need N > 0 and K %% 32 == 0 (N=%lld K=%lld)", WBITS,
              (long long)N, (long long)K);
  R4Q_REQUIRE(aligned(w, 16) && aligned(sz, 4) && aligned(out, 16),
              "dequant_int%d: misaligned pointer", WBITS);
  const int64_t nb = N * (K / 32);
  const int64_t grid = (nb + 255) / 256;
  hipLaunchKernelGGL((dequant_kernel<WBITS>), dim3((unsigned)grid), dim3(256), 0,
                     as_stream(stream), static_cast<const uint8_t*>(w),
                     static_cast<const uint32_t*>(sz), static_cast<uint16_t*>(out), nb, K);
  return launch_status(WBITS == 4 ? "dequant_int4" : "dequant_int8");
}

}  // namespace
}  // namespace r4q

extern "C" int r4q_dequant_int4(const void* packed, const void* sz, void* out, int64_t N,
                                int64_t K, void* stream) {
  return r4q::dequant<4>(packed, sz, out, N, K, stream);
}

extern "C" int r4q_dequant_int8(const void* q, const void* sz, void* out, int64_t N,
                                int64_t K, void* stream) {
  return r4q::dequant<8>(q, sz, out, N, K, stream);
}

extern "C" int r4q_fp16_to_fp8(const void* src, void* dst, int64_t n, void* stream) {
  R4Q_REQUIRE(n >= 0, "fp16_to_fp8: negative size");
  if (n == 0) return R4Q_OK;
  R4Q_REQUIRE(src && dst, "fp16_to_fp8: null pointer");
  R4Q_REQUIRE(r4q::aligned(src, 8) && r4q::aligned(dst, 4), "fp16_to_fp8: misaligned pointer");
  const int64_t threads = (n + 3) / 4;
  hipLaunchKernelGGL(r4q::fp16_to_fp8_kernel, dim3((unsigned)((threads + 255) / 256)),
                     dim3(256), 0, r4q::as_stream(stream),
                     static_cast<const uint16_t*>(src), static_cast<uint8_t*>(dst), n);
  return r4q::launch_status("fp16_to_fp8");
}

extern "C" int r4q_fp8_to_fp16(const void* src, void* dst, int64_t n, void* stream) {
  R4Q_REQUIRE(n >= 0, "fp8_to_fp16: negative size");
  if (n == 0) return R4Q_OK;
  R4Q_REQUIRE(src && dst, "fp8_to_fp16: null pointer");
  hipLaunchKernelGGL(r4q::fp8_to_fp16_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256),
                     0, r4q::as_stream(stream), static_cast<const uint8_t*>(src),
                     static_cast<uint16_t*>(dst), n);
  return r4q::launch_status("fp8_to_fp16");
}
