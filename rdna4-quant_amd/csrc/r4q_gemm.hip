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

// ---------------------------------------------------------------------
// Skinny GEMM for 2..16 activation rows (batched decode): the weights are
// streamed once for all rows.  v_mfma_f32_16x16x32_f16 with A = the x rows
// (padded to 16 by repeating the last row) and B = dequantised weights.
//
// One iteration of a wave: every lane loads one 16-byte chunk of a weight
// row (lane l: row n0 + l%16, chunk group g = l/16), so the 4 lane groups
// hold 4 consecutive chunks of each of 16 rows (64 contiguous bytes per row).
// The MFMA contraction index k is only a label: lane group g's 8 k-slots of
// MFMA d carry elements of chunk g, and the A fragment of that lane group
// holds the x values of exactly those elements.  Because the weights are
// fully dequantised before the MFMA -- fp16((q - zp) * s) by an exact packed
// fp16 subtraction and one rounded packed multiply, bit-identical to the
// dequant kernel -- the accumulation may run across blocks.
//   INT4: chunk = one 32-element block, 4 MFMAs per iteration; nibble pairs
//         (q_p, q_p+4) come from (w >> 4p) & 0x000F000F | 0x64006400, so x is
//         permuted to (x_p, x_p+4) pairs;
//   INT8: chunk = half a block, 2 MFMAs; byte pairs by v_perm, natural order;
//   FP16: chunk = 8 weights, 1 MFMA.
// A workgroup (4 waves) owns 16*T weight rows; wave w takes iterations
// w, w+4, ...; the 4 partial tiles meet in LDS.
template <int WBITS>
struct Skinny;
template <>
struct Skinny<4> {
  static constexpr int kKPI = 128;  // k per iteration (4 lane groups)
  static constexpr int kMfma = 4;
};
template <>
struct Skinny<8> {
  static constexpr int kKPI = 64;
  static constexpr int kMfma = 2;
};
template <>
struct Skinny<16> {
  static constexpr int kKPI = 32;
  static constexpr int kMfma = 1;
};

// B fragment of MFMA d from the lane's 16-byte chunk.
template <int WBITS>
__device__ __forceinline__ h8_t skinny_b(const u4_t w, uint32_t s2, int d) {
  if constexpr (WBITS == 16) {
    return __builtin_bit_cast(h8_t, w);
  } else {
    const uint32_t sb = s2 & 0xFFFFu;
    const h2_t sc = as_h2(sb | (sb << 16));
    const uint32_t zb = s2 >> 16;
    // -(1024 + zp) as an fp16 pair (exact: an integer below 2048)
    const h2_t nz = -(as_h2(0x64006400u) + as_h2(zb | (zb << 16)));
    uint32_t pr[4];
    if constexpr (WBITS == 4) {
      const uint32_t wd = w[d];
#pragma unroll
      for (int p = 0; p < 4; ++p) pr[p] = ((wd >> (4 * p)) & 0x000F000Fu) | 0x64006400u;
    } else {
      const uint32_t w0 = w[2 * d], w1 = w[2 * d + 1];
      pr[0] = __builtin_amdgcn_perm(w0, 0x64646464u, 0x00050004u);
      pr[1] = __builtin_amdgcn_perm(w0, 0x64646464u, 0x00070006u);
      pr[2] = __builtin_amdgcn_perm(w1, 0x64646464u, 0x00050004u);
      pr[3] = __builtin_amdgcn_perm(w1, 0x64646464u, 0x00070006u);
    }
    u4_t o;
#pragma unroll
    for (int p = 0; p < 4; ++p) o[p] = as_u32((as_h2(pr[p]) + nz) * sc);
    return __builtin_bit_cast(h8_t, o);
  }
}

// A fragment of MFMA d: the 8 x values whose labels match skinny_b's slots.
template <int WBITS>
__device__ __forceinline__ h8_t skinny_a(const uint16_t* __restrict__ xrow, int kchunk, int d) {
  if constexpr (WBITS == 4) {
    const u4_t v = *reinterpret_cast<const u4_t*>(xrow + kchunk + 8 * d);
    // (x0 x1) (x2 x3) (x4 x5) (x6 x7) -> (x0 x4) (x1 x5) (x2 x6) (x3 x7)
    u4_t o;
    o[0] = (v[0] & 0xFFFFu) | (v[2] << 16);
    o[1] = (v[0] >> 16) | (v[2] & 0xFFFF0000u);
    o[2] = (v[1] & 0xFFFFu) | (v[3] << 16);
    o[3] = (v[1] >> 16) | (v[3] & 0xFFFF0000u);
    return __builtin_bit_cast(h8_t, o);
  } else {
    return __builtin_bit_cast(h8_t, *reinterpret_cast<const u4_t*>(xrow + kchunk + 8 * d));
  }
}

template <int WBITS, int T>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(const uint16_t* __restrict__ X,
                                                          const uint8_t* __restrict__ W,
                                                          const uint32_t* __restrict__ SZ,
                                                          uint16_t* __restrict__ Y, int M, int N,
                                                          int K) {
  constexpr int KPI = Skinny<WBITS>::kKPI;
  constexpr int NM = Skinny<WBITS>::kMfma;
  constexpr int CK = KPI / 4;  // elements per lane chunk
  __shared__ __align__(16) float red[4][T][64][4];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int g = lane >> 4, r16 = lane & 15;
  const int n0 = blockIdx.x * 16 * T;
  const int iters = K / KPI;
  const int64_t row_bytes = (int64_t)K * WBITS / 8;
  const int nb = K / 32;
  const uint16_t* xrow = X + (int64_t)min(r16, M - 1) * K;  // A row of this lane

  f4_t acc[T];
#pragma unroll
  for (int i = 0; i < T; ++i) acc[i] = f4_t{0.f, 0.f, 0.f, 0.f};

  // U iterations per batch: all their loads are issued before any MFMA
  // (iterations past the end load the last one again and are not computed)
  constexpr int U = 4;
  for (int it0 = wave; it0 < iters; it0 += 4 * U) {
    u4_t wv[U][T];
    uint32_t s2[U][T];
    h8_t a[U][NM];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int it = min(it0 + 4 * u, iters - 1);
      const int kchunk = it * KPI + g * CK;  // first element of this lane's chunk
#pragma unroll
      for (int i = 0; i < T; ++i) {
        const int64_t n = min(n0 + 16 * i + r16, N - 1);  // clamped: in bounds
        wv[u][i] = __builtin_nontemporal_load(
            reinterpret_cast<const u4_t*>(W + n * row_bytes + (int64_t)kchunk * WBITS / 8));
        s2[u][i] = (WBITS == 16) ? 0u : SZ[n * nb + kchunk / 32];
      }
#pragma unroll
      for (int d = 0; d < NM; ++d) a[u][d] = skinny_a<WBITS>(xrow, kchunk, d);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (it0 + 4 * u < iters) {  // wave-uniform
#pragma unroll
        for (int i = 0; i < T; ++i)
#pragma unroll
          for (int d = 0; d < NM; ++d)
            acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                a[u][d], skinny_b<WBITS>(wv[u][i], s2[u][i], d), acc[i], 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < T; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][i][lane][r] = acc[i][r];
  __syncthreads();
  // C fragment: lane holds rows m = 4*(lane/16) + r, column n = lane % 16
  for (int e = t; e < T * 64 * 4; e += 256) {
    const int i = e / 256, l = (e / 4) & 63, r = e & 3;
    const int m = 4 * (l >> 4) + r, n = n0 + 16 * i + (l & 15);
    const float v = (red[0][i][l][r] + red[1][i][l][r]) + (red[2][i][l][r] + red[3][i][l][r]);
    if (m < M && n < N) Y[(int64_t)m * N + n] = f2h(v);
  }
}

}  // namespace

bool gemm_skinny_ok(int64_t M, int64_t K, int wbits) {
  const int kpi = wbits == 4 ? Skinny<4>::kKPI : wbits == 8 ? Skinny<8>::kKPI : Skinny<16>::kKPI;
  return M >= 2 && M <= 16 && K % kpi == 0;
}

int gemm_skinny_launch(const void* x, const void* w, const void* sz, void* y, int64_t M,
                       int64_t N, int64_t K, int wbits, hipStream_t st) {
  constexpr int T = 2;
  const dim3 grid((unsigned)((N + 16 * T - 1) / (16 * T)));
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* wp = static_cast<const uint8_t*>(w);
  const auto* sp = static_cast<const uint32_t*>(sz);
  auto* yp = static_cast<uint16_t*>(y);
  switch (wbits) {
    case 4:
      hipLaunchKernelGGL((gemm_skinny_kernel<4, T>), grid, dim3(256), 0, st, xp, wp, sp, yp,
                         (int)M, (int)N, (int)K);
      break;
    case 8:
      hipLaunchKernelGGL((gemm_skinny_kernel<8, T>), grid, dim3(256), 0, st, xp, wp, sp, yp,
                         (int)M, (int)N, (int)K);
      break;
    default:
      hipLaunchKernelGGL((gemm_skinny_kernel<16, T>), grid, dim3(256), 0, st, xp, wp, sp, yp,
                         (int)M, (int)N, (int)K);
  }
  return launch_status("gemm_skinny");
}

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
