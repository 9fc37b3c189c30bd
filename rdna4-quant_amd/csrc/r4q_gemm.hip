// Prefill GEMM Y[M,N] = X[M,K] W[N,K]^T with the weight dequantised on the
// fly (INT4 / INT8 block-32 asymmetric, or FP16) into LDS and multiplied on
// the matrix cores with v_mfma_f32_16x16x32_f16 (fp32 accumulate).
//
// Replaces the reference's prefill projection dequant_matmul_out
// (hip:1973-1988), which materialises the whole fp16 weight with
// dequant_int4_kernel and then calls rocBLAS through at::mm_out: here each
// weight byte is read from HBM once per M-tile and never written back.
//
// Tiling: a workgroup (4 waves) owns a 128 x 128 output tile and walks K in
// steps of 32 (one quantisation block).  Per step the X tile (128 x 32 fp16)
// and the dequantised W tile (128 x 32 fp16) are staged in LDS (rows padded
// to 80 B against bank conflicts); each wave computes a 64 x 64 sub-tile as
// 4 x 4 MFMA 16x16x32 tiles.  The next step's global loads are issued before
// the current step's MFMAs.  Dequantised values equal r4q_dequant_int4/8
// bit-for-bit (fp16((q - zp) * scale) from an exact fp32 product).
#include "r4q_device.hpp"
#include "r4q_gemv.hpp"
#include "r4q_host.hpp"

namespace r4q {
namespace {

constexpr int BM = 128, BN = 128, BK = 32;
constexpr int LDS_ROW = 40;  // halves per LDS row (32 + 8 pad)

// Raw global data one thread stages per K step.
template <int WBITS>
struct Stage {
  u4_t a[2];        // two 16-byte chunks of X
  u4_t w[2];        // weight bytes for 16 elements (INT4: w[0].xy used)
  uint32_t sz;      // (scale, zero) of the row's block
};

template <int WBITS>
__device__ __forceinline__ void load_stage(Stage<WBITS>& s, const uint16_t* __restrict__ X,
                                           const uint8_t* __restrict__ W,
                                           const uint32_t* __restrict__ SZ, int M, int N, int K,
                                           int m0, int n0, int k0, int t) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = t + 256 * i;       // 512 chunks of 8 halves
    const int row = c >> 2, kc = c & 3;
    const int m = m0 + row;
    s.a[i] = (m < M) ? *reinterpret_cast<const u4_t*>(X + (int64_t)m * K + k0 + 8 * kc)
                     : u4_t{0, 0, 0, 0};
  }
  const int row = t >> 1, half = t & 1;  // 2 threads per weight row, 16 elements each
  const int n = n0 + row;
  const bool ok = n < N;
  const int64_t nn = ok ? n : 0;
  if constexpr (WBITS == 4) {
    const u2_t v = ok ? *reinterpret_cast<const u2_t*>(W + nn * (K / 2) + k0 / 2 + 8 * half)
                      : u2_t{0, 0};
    s.w[0] = u4_t{v[0], v[1], 0, 0};
    s.sz = ok ? SZ[nn * (K / 32) + k0 / 32] : 0u;
  } else if constexpr (WBITS == 8) {
    s.w[0] = ok ? *reinterpret_cast<const u4_t*>(W + nn * K + k0 + 16 * half) : u4_t{0, 0, 0, 0};
    s.sz = ok ? SZ[nn * (K / 32) + k0 / 32] : 0u;
  } else {
    const u4_t* p = reinterpret_cast<const u4_t*>(W + (nn * K + k0 + 16 * half) * 2);
    s.w[0] = ok ? p[0] : u4_t{0, 0, 0, 0};
    s.w[1] = ok ? p[1] : u4_t{0, 0, 0, 0};
    s.sz = 0u;
  }
}

template <int WBITS>
__device__ __forceinline__ void store_stage(const Stage<WBITS>& s, uint16_t* As, uint16_t* Bs,
                                            int t) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = t + 256 * i;
    const int row = c >> 2, kc = c & 3;
    *reinterpret_cast<u4_t*>(As + row * LDS_ROW + 8 * kc) = s.a[i];
  }
  const int row = t >> 1, half = t & 1;
  u4_t o[2];
  if constexpr (WBITS == 16) {
    o[0] = s.w[0];
    o[1] = s.w[1];
  } else {
    const float scale = h2f((uint16_t)(s.sz & 0xFFFFu));
    const float zp = h2f((uint16_t)(s.sz >> 16));
    uint32_t q[16];
    if constexpr (WBITS == 4) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) q[8 * j + e] = (s.w[0][j] >> (4 * e)) & 0xFu;
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) q[4 * j + e] = (s.w[0][j] >> (8 * e)) & 0xFFu;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float lo = ((float)q[2 * i] - zp) * scale;
      const float hi = ((float)q[2 * i + 1] - zp) * scale;
      o[i >> 2][i & 3] = (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
    }
  }
  u4_t* dst = reinterpret_cast<u4_t*>(Bs + row * LDS_ROW + 16 * half);
  dst[0] = o[0];
  dst[1] = o[1];
}

template <int WBITS>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(const uint16_t* __restrict__ X,
                                                        const uint8_t* __restrict__ W,
                                                        const uint32_t* __restrict__ SZ,
                                                        uint16_t* __restrict__ Y, int M, int N,
                                                        int K) {
  __shared__ __align__(16) uint16_t As[BM * LDS_ROW];
  __shared__ __align__(16) uint16_t Bs[BN * LDS_ROW];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int fr = lane & 15, fk = 8 * (lane >> 4);  // fragment row / k offset

  f4_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  Stage<WBITS> st;
  load_stage<WBITS>(st, X, W, SZ, M, N, K, m0, n0, 0, t);
  for (int k0 = 0; k0 < K; k0 += BK) {
    __syncthreads();  // previous step's fragments consumed
    store_stage<WBITS>(st, As, Bs, t);
    __syncthreads();
    if (k0 + BK < K) load_stage<WBITS>(st, X, W, SZ, M, N, K, m0, n0, k0 + BK, t);
    h8_t a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      a[i] = *reinterpret_cast<const h8_t*>(As + (wm + 16 * i + fr) * LDS_ROW + fk);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      b[j] = *reinterpret_cast<const h8_t*>(Bs + (wn + 16 * j + fr) * LDS_ROW + fk);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
  }
  // C fragment: lane holds rows 4*(lane/16)+r, column lane%16
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = n0 + wn + 16 * j + fr;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm + 16 * i + 4 * (lane >> 4) + r;
        if (row < M && col < N) Y[(int64_t)row * N + col] = f2h(acc[i][j][r]);
      }
    }
}

}  // namespace

int gemm_mfma_launch(const void* x, const void* w, const void* sz, void* y, int64_t M, int64_t N,
                     int64_t K, int wbits, hipStream_t st) {
  const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* wp = static_cast<const uint8_t*>(w);
  const auto* sp = static_cast<const uint32_t*>(sz);
  auto* yp = static_cast<uint16_t*>(y);
  switch (wbits) {
    case 4:
      hipLaunchKernelGGL(gemm_mfma_kernel<4>, grid, dim3(256), 0, st, xp, wp, sp, yp, (int)M,
                         (int)N, (int)K);
      break;
    case 8:
      hipLaunchKernelGGL(gemm_mfma_kernel<8>, grid, dim3(256), 0, st, xp, wp, sp, yp, (int)M,
                         (int)N, (int)K);
      break;
    default:
      hipLaunchKernelGGL(gemm_mfma_kernel<16>, grid, dim3(256), 0, st, xp, wp, sp, yp, (int)M,
                         (int)N, (int)K);
  }
  return launch_status("gemm_mfma");
}

}  // namespace r4q
