// Batch-1 GEMV y = W x for block-32 asymmetric INT4 / INT8 and FP16 weights.
//
// Replaces the reference's gemv_warp<4> (hip:116-170, launcher hip:230-235):
// y[n] = sum_b scale[n,b] * sum_{i<32} x[32b+i] * (q[n,32b+i] - zp[n,b]),
// fp32 accumulation, fp16 output.
//
// gfx950 design
//  * A "chunk" is 16 bytes of one weight row (INT4: one 32-element block,
//    INT8: half a block, FP16: 8 values).  The chunks of a row are spread over
//    LR = gcd(chunks_per_row, 64) lanes, so a wave covers 64/LR rows per step
//    and every wave-level dwordx4 load reads contiguous 512-1024 B runs.
//  * Weights are streamed with nontemporal 128-bit loads (read once).
//  * Nibbles become fp16 without per-element converts: (w & 0x000F000F) |
//    0x64006400 is the fp16 pair (1024+q0, 1024+q4); the 0x00F000F0 mask gives
//    (1024+16 q1, 1024+16 q5).  v_dot2_f32_f16 multiplies them with x pairs
//    arranged in that order, and the 1024 / 16 offsets and the zero-point are
//    removed per block with precomputed sums of x:
//      sum x*(q-zp) = A + B/16 - (1024*S_even + 64*S_odd) - zp*(S_even+S_odd)
//    where A/B are the even/odd-element dot accumulators.  INT8 bytes use
//    v_perm to form (1024+q) pairs the same way.
//  * The activation is arranged once per workgroup into LDS in that pair
//    order, with the per-chunk sums; waves keep it in registers when a row is
//    short (K=5120) and stream it from LDS otherwise (K=17408).
//  * Row partials are reduced across the LR lanes with DPP row operations and
//    v_readlane; no LDS round trip.
#include <stdlib.h>

#include "r4q_device.hpp"
#include "r4q_gemv.hpp"
#include "r4q_host.hpp"

namespace r4q {
namespace {

template <int WBITS>
struct Fmt;
template <>
struct Fmt<4> {
  static constexpr int kElems = 32;  // elements per 16-byte chunk
  static constexpr int kXDw = 20;    // prepared-x dwords per chunk
};
template <>
struct Fmt<8> {
  static constexpr int kElems = 16;
  static constexpr int kXDw = 12;
};
template <>
struct Fmt<16> {
  static constexpr int kElems = 8;
  static constexpr int kXDw = 4;
};

constexpr uint32_t kMagic = 0x64006400u;  // fp16 pair (1024, 1024)

__device__ __forceinline__ uint32_t pack_h(uint32_t lo16, uint32_t hi16) {
  return (lo16 & 0xFFFFu) | (hi16 << 16);
}

// Arranges chunk c of x (fp16) into the prepared layout at dst.
template <int WBITS>
__device__ __forceinline__ void prep_chunk(const uint16_t* __restrict__ x, int c,
                                           uint32_t* __restrict__ dst) {
  constexpr int E = Fmt<WBITS>::kElems;
  const u4_t* src = reinterpret_cast<const u4_t*>(x + (int64_t)c * E);
  if constexpr (WBITS == 4) {
    uint32_t raw[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u4_t v = src[i];
      raw[4 * i + 0] = v[0];
      raw[4 * i + 1] = v[1];
      raw[4 * i + 2] = v[2];
      raw[4 * i + 3] = v[3];
    }
    float se = 0.f, so = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      se += h2f((uint16_t)(raw[k] & 0xFFFFu));
      so += h2f((uint16_t)(raw[k] >> 16));
    }
    // word j of the weight chunk holds elements 8j..8j+7; raw[4j + m] holds
    // elements (8j+2m, 8j+2m+1).
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t r0 = raw[4 * j], r1 = raw[4 * j + 1], r2 = raw[4 * j + 2],
                     r3 = raw[4 * j + 3];
      dst[4 * j + 0] = pack_h(r0, r2 & 0xFFFFu);            // (x0, x4)
      dst[4 * j + 1] = pack_h(r0 >> 16, r2 >> 16);          // (x1, x5)
      dst[4 * j + 2] = pack_h(r1, r3 & 0xFFFFu);            // (x2, x6)
      dst[4 * j + 3] = pack_h(r1 >> 16, r3 >> 16);          // (x3, x7)
    }
    dst[16] = __float_as_uint(se + so);
    dst[17] = __float_as_uint(1024.0f * se + 64.0f * so);
    dst[18] = 0u;
    dst[19] = 0u;
  } else if constexpr (WBITS == 8) {
    const u4_t a = src[0], b = src[1];
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      dst[k] = a[k];
      dst[4 + k] = b[k];
      s += h2f((uint16_t)(a[k] & 0xFFFFu)) + h2f((uint16_t)(a[k] >> 16));
      s += h2f((uint16_t)(b[k] & 0xFFFFu)) + h2f((uint16_t)(b[k] >> 16));
    }
    dst[8] = __float_as_uint(s);
    dst[9] = dst[10] = dst[11] = 0u;
  } else {
    const u4_t a = src[0];
#pragma unroll
    for (int k = 0; k < 4; ++k) dst[k] = a[k];
  }
}

// acc + scale * sum over the chunk of x * (q - zp)   (FP16: acc + x . w)
template <int WBITS>
__device__ __forceinline__ float chunk_dot(const u4_t wq, uint32_t s2,
                                           const uint32_t* __restrict__ xp, float acc) {
  if constexpr (WBITS == 4) {
    // Masks and magic live in VGPRs so each pair is one v_and_or_b32 (a
    // VOP3 on gfx9 can read only one scalar/literal operand).
    uint32_t mlo = 0x000F000Fu, mhi = 0x00F000F0u, mag = kMagic;
    asm volatile("" : "+v"(mlo), "+v"(mhi), "+v"(mag));
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w0 = wq[j], w8 = wq[j] >> 8;
      a = __builtin_amdgcn_fdot2(as_h2((w0 & mlo) | mag), as_h2(xp[4 * j + 0]), a, false);
      b = __builtin_amdgcn_fdot2(as_h2((w0 & mhi) | mag), as_h2(xp[4 * j + 1]), b, false);
      a = __builtin_amdgcn_fdot2(as_h2((w8 & mlo) | mag), as_h2(xp[4 * j + 2]), a, false);
      b = __builtin_amdgcn_fdot2(as_h2((w8 & mhi) | mag), as_h2(xp[4 * j + 3]), b, false);
    }
    const float scale = h2f((uint16_t)(s2 & 0xFFFFu));
    const float zp = h2f((uint16_t)(s2 >> 16));
    const float d = __builtin_fmaf(b, 0.0625f, a) -
                    __builtin_fmaf(zp, __uint_as_float(xp[16]), __uint_as_float(xp[17]));
    return __builtin_fmaf(scale, d, acc);
  } else if constexpr (WBITS == 8) {
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a = __builtin_amdgcn_fdot2(as_h2(__builtin_amdgcn_perm(wq[j], 0x64646464u, 0x00050004u)),
                                 as_h2(xp[2 * j]), a, false);
      a = __builtin_amdgcn_fdot2(as_h2(__builtin_amdgcn_perm(wq[j], 0x64646464u, 0x00070006u)),
                                 as_h2(xp[2 * j + 1]), a, false);
    }
    const float scale = h2f((uint16_t)(s2 & 0xFFFFu));
    const float zp = h2f((uint16_t)(s2 >> 16));
    const float d = __builtin_fmaf(-(zp + 1024.0f), __uint_as_float(xp[8]), a);
    return __builtin_fmaf(scale, d, acc);
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      acc = __builtin_amdgcn_fdot2(as_h2(wq[j]), as_h2(xp[j]), acc, false);
    return acc;
  }
}

__device__ __forceinline__ u4_t load_nt(const u4_t* p) {
  return __builtin_nontemporal_load(p);
}

// Reduces `v` over aligned groups of `lr` lanes (power of two <= 64); the
// result is valid in the first lane of each group.
__device__ __forceinline__ float reduce_lr(float v, int lr) {
  dot_dpp_fence();
  if (lr >= 2) v += dpp<kDppQuadXor1>(v);
  if (lr >= 4) v += dpp<kDppQuadXor2>(v);
  if (lr >= 8) v += dpp<kDppHalfMirror>(v);
  if (lr >= 16) v += dpp<kDppRowMirror>(v);
  if (lr >= 32) {
    const float r0 = readlane_f(v, 0), r1 = readlane_f(v, 16);
    const float r2 = readlane_f(v, 32), r3 = readlane_f(v, 48);
    if (lr == 32)
      v = (lane_id() < 32) ? (r0 + r1) : (r2 + r3);
    else
      v = (r0 + r1) + (r2 + r3);
  }
  return v;
}

template <int XD>
__device__ __forceinline__ void lds_copy(const uint32_t* __restrict__ src, uint32_t* dst) {
#pragma unroll
  for (int k = 0; k < XD; k += 4) {
    const u4_t v = *reinterpret_cast<const u4_t*>(src + k);
    dst[k] = v[0];
    dst[k + 1] = v[1];
    dst[k + 2] = v[2];
    dst[k + 3] = v[3];
  }
}

// Shared prologue: arrange x into LDS (every thread of the workgroup).
template <int WBITS>
__device__ __forceinline__ void stage_x(const uint16_t* __restrict__ x, uint32_t* xs, int cpr) {
  for (int c = threadIdx.x; c < cpr; c += blockDim.x)
    prep_chunk<WBITS>(x, c, xs + c * Fmt<WBITS>::kXDw);
  __syncthreads();
}

template <int WBITS>
__device__ __forceinline__ uint32_t load_sz(const uint32_t* __restrict__ srow, int c) {
  if constexpr (WBITS == 4) return srow[c];
  else if constexpr (WBITS == 8) return srow[c >> 1];
  else return 0u;
}

// Register-resident activation: each lane owns exactly CPL chunk columns
// (cpr == CPL * lr), holds their prepared x in VGPRs and sweeps rows.
template <int WBITS, int CPL>
__global__ __launch_bounds__(256) void gemv_xreg_kernel(const uint16_t* __restrict__ x,
                                                        const uint8_t* __restrict__ w,
                                                        const uint32_t* __restrict__ sz,
                                                        uint16_t* __restrict__ y, int N, int K,
                                                        int lr, int upw) {
  constexpr int E = Fmt<WBITS>::kElems;
  constexpr int XD = Fmt<WBITS>::kXDw;
  extern __shared__ __align__(16) uint32_t xs[];
  const int cpr = K / E;
  const int nb = K / 32;
  stage_x<WBITS>(x, xs, cpr);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rpu = 64 / lr;
  const int rl = lane / lr;
  const int cl = lane % lr;
  uint32_t xr[CPL * XD];
#pragma unroll
  for (int i = 0; i < CPL; ++i) lds_copy<XD>(xs + (cl + lr * i) * XD, xr + i * XD);

  const int64_t row_bytes = (int64_t)K * WBITS / 8;
  const int units = (N + rpu - 1) / rpu;
  const int u0 = (blockIdx.x * (blockDim.x >> 6) + wave) * upw;
  const int u1 = min(u0 + upw, units);
  for (int u = u0; u < u1; ++u) {
    const int row = u * rpu + rl;
    const int rowc = min(row, N - 1);  // clamped: loads stay in bounds
    const u4_t* wrow = reinterpret_cast<const u4_t*>(w + (int64_t)rowc * row_bytes) + cl;
    const uint32_t* srow = sz + (int64_t)rowc * nb;
    u4_t wq[CPL];
    uint32_t s2[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      wq[i] = load_nt(wrow + lr * i);
      s2[i] = load_sz<WBITS>(srow, cl + lr * i);
    }
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) acc = chunk_dot<WBITS>(wq[i], s2[i], xr + i * XD, acc);
    const float total = reduce_lr(acc, lr);
    if (row < N && cl == 0) y[row] = f2h(total);
  }
}

// LDS-resident activation for long rows: batches of NB chunk slots, the
// prepared x of each chunk read from LDS as it is consumed.
template <int WBITS, int NB>
__global__ __launch_bounds__(256) void gemv_stream_kernel(const uint16_t* __restrict__ x,
                                                          const uint8_t* __restrict__ w,
                                                          const uint32_t* __restrict__ sz,
                                                          uint16_t* __restrict__ y, int N,
                                                          int K, int lr, int upw) {
  constexpr int E = Fmt<WBITS>::kElems;
  constexpr int XD = Fmt<WBITS>::kXDw;
  extern __shared__ __align__(16) uint32_t xs[];
  const int cpr = K / E;
  const int cpl = cpr / lr;
  const int nb = K / 32;
  stage_x<WBITS>(x, xs, cpr);

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int rpu = 64 / lr;
  const int rl = lane / lr;
  const int cl = lane % lr;

  const int64_t row_bytes = (int64_t)K * WBITS / 8;
  const int units = (N + rpu - 1) / rpu;
  const int u0 = (blockIdx.x * (blockDim.x >> 6) + wave) * upw;
  const int u1 = min(u0 + upw, units);
  for (int u = u0; u < u1; ++u) {
    const int row = u * rpu + rl;
    const int rowc = min(row, N - 1);
    const u4_t* wrow = reinterpret_cast<const u4_t*>(w + (int64_t)rowc * row_bytes) + cl;
    const uint32_t* srow = sz + (int64_t)rowc * nb;
    float acc = 0.f;
    for (int i0 = 0; i0 < cpl; i0 += NB) {
      const int nslot = min(NB, cpl - i0);  // wave-uniform
      u4_t wq[NB];
      uint32_t s2[NB];
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const int slot = i0 + min(i, nslot - 1);  // clamped: always in bounds
        wq[i] = load_nt(wrow + lr * slot);
        s2[i] = load_sz<WBITS>(srow, cl + lr * slot);
      }
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        if (i < nslot) {
          uint32_t xp[XD];
          lds_copy<XD>(xs + (cl + lr * (i0 + i)) * XD, xp);
          acc = chunk_dot<WBITS>(wq[i], s2[i], xp, acc);
        }
      }
    }
    const float total = reduce_lr(acc, lr);
    if (row < N && cl == 0) y[row] = f2h(total);
  }
}

int gcd_int(int a, int b) {
  while (b) {
    const int t = a % b;
    a = b;
    b = t;
  }
  return a;
}

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  if (!v || !*v) return dflt;
  return atoi(v);
}

template <int WBITS>
int launch_gemv_fmt(const void* x, const void* w, const void* sz, void* y, int64_t N, int64_t K,
                    hipStream_t st) {
  constexpr int E = Fmt<WBITS>::kElems;
  constexpr int XD = Fmt<WBITS>::kXDw;
  const int cpr = (int)(K / E);
  const int lr = gcd_int(cpr, 64);
  const int cpl = cpr / lr;
  const int rpu = 64 / lr;
  const int64_t units = (N + rpu - 1) / rpu;
  const size_t lds = (size_t)cpr * XD * 4;
  R4Q_REQUIRE(lds <= 64 * 1024, "gemv: K=%lld too large for the LDS activation stage",
              (long long)K);
  // Units per wave: aim at ~2048 waves over the chip (256 CUs x 8).
  static const int target_waves = env_int("R4Q_GEMV_WAVES", 2048);
  int upw = (int)((units + target_waves - 1) / target_waves);
  if (upw < 1) upw = 1;
  const int64_t waves = (units + upw - 1) / upw;
  const int64_t grid = (waves + 3) / 4;
  const dim3 g((unsigned)grid), b(256);
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* wp = static_cast<const uint8_t*>(w);
  const auto* sp = static_cast<const uint32_t*>(sz);
  auto* yp = static_cast<uint16_t*>(y);
#define R4Q_XREG(C)                                                                       \
  case C:                                                                                 \
    hipLaunchKernelGGL((gemv_xreg_kernel<WBITS, C>), g, b, lds, st, xp, wp, sp, yp, (int)N, \
                       (int)K, lr, upw);                                                  \
    break;
  switch (cpl) {
    R4Q_XREG(1)
    R4Q_XREG(2)
    R4Q_XREG(3)
    R4Q_XREG(4)
    R4Q_XREG(5)
    default:
      if constexpr (WBITS == 16) {
        if (cpl == 10) {
          hipLaunchKernelGGL((gemv_xreg_kernel<WBITS, 10>), g, b, lds, st, xp, wp, sp, yp,
                             (int)N, (int)K, lr, upw);
          break;
        }
      }
      hipLaunchKernelGGL((gemv_stream_kernel<WBITS, 9>), g, b, lds, st, xp, wp, sp, yp, (int)N,
                         (int)K, lr, upw);
  }
#undef R4Q_XREG
  return launch_status("gemv");
}

}  // namespace

int gemv_check(const void* x, const void* w, const void* sz, const void* y, int64_t N,
               int64_t K, int wbits) {
  R4Q_REQUIRE(x && w && y, "gemv: null pointer");
  R4Q_REQUIRE(wbits == 4 || wbits == 8 || wbits == 16, "gemv: wbits must be 4, 8 or 16 (got %d)",
              wbits);
  R4Q_REQUIRE(wbits == 16 || sz, "gemv: null scale/zero pointer");
  R4Q_REQUIRE(N > 0 && K > 0 && K % 32 == 0 && N < (1LL << 31) && K < (1LL << 24),
              "gemv: need N > 0, K > 0, K %% 32 == 0 (N=%lld K=%lld)", (long long)N,
              (long long)K);
  R4Q_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(w) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(sz) & 3) == 0 &&
                  (reinterpret_cast<uintptr_t>(y) & 1) == 0,
              "gemv: x and w must be 16-byte aligned");
  return R4Q_OK;
}

int gemv_launch(const void* x, const void* w, const void* sz, void* y, int64_t N, int64_t K,
                int wbits, hipStream_t st) {
  switch (wbits) {
    case 4: return launch_gemv_fmt<4>(x, w, sz, y, N, K, st);
    case 8: return launch_gemv_fmt<8>(x, w, sz, y, N, K, st);
    default: return launch_gemv_fmt<16>(x, w, sz, y, N, K, st);
  }
}

int gemm_launch(const void* x, const void* w, const void* sz, void* y, int64_t M, int64_t N,
                int64_t K, int wbits, hipStream_t st) {
  if (M > kSkinnyMaxRows) return gemm_mfma_launch(x, w, sz, y, M, N, K, wbits, st);
  const auto* xp = static_cast<const uint16_t*>(x);
  auto* yp = static_cast<uint16_t*>(y);
  for (int64_t m = 0; m < M; ++m) R4Q_TRY(gemv_launch(xp + m * K, w, sz, yp + m * N, N, K, wbits, st));
  return R4Q_OK;
}

}  // namespace r4q

extern "C" int r4q_gemv(const void* x, const void* w, const void* sz, void* y, int64_t N,
                        int64_t K, int wbits, void* stream) {
  R4Q_TRY(r4q::gemv_check(x, w, sz, y, N, K, wbits));
  return r4q::gemv_launch(x, w, sz, y, N, K, wbits, r4q::as_stream(stream));
}

extern "C" int r4q_gemm(const void* x, const void* w, const void* sz, void* y, int64_t M,
                        int64_t N, int64_t K, int wbits, void* stream) {
  R4Q_REQUIRE(M >= 1, "gemm: M must be >= 1");
  R4Q_TRY(r4q::gemv_check(x, w, sz, y, N, K, wbits));
  return r4q::gemm_launch(x, w, sz, y, M, N, K, wbits, r4q::as_stream(stream));
}
