// Batch-1 GEMV y = W x for block-32 asymmetric INT4 / INT8 and FP16 weights.
//
// Replaces the reference's gemv_warp<4> (hip:116-170, launcher hip:230-235):
// y[n] = sum_b scale[n,b] * sum_{i<32} x[32b+i] * (q[n,32b+i] - zp[n,b]),
// fp32 accumulation, fp16 output.
//
// gfx950 design
//  * A "chunk" is 16 bytes of one weight row (INT4: one 32-element block,
//    INT8: half a block, FP16: 8 values).  LPR lanes share a row (16..64
//    inside a wave, 128/256 over 2/4 waves) and lane c owns chunk columns
//    c + LPR*i, so every wave-level dwordx4 load reads contiguous runs.
//  * Weights are streamed with nontemporal 128-bit loads (read once).
//  * Nibbles become fp16 without per-element converts: (w & 0x000F000F) |
//    0x64006400 is the fp16 pair (1024+q0, 1024+q4); the 0x00F000F0 mask gives
//    (1024+16 q1, 1024+16 q5).  v_dot2_f32_f16 multiplies them with x pairs
//    arranged in that order, and the 1024 / 16 offsets and the zero-point are
//    removed per block with precomputed sums of x:
//      sum x*(q-zp) = A + B/16 - (1024*S_even + 64*S_odd) - zp*(S_even+S_odd)
//    where A/B are the even/odd-element dot accumulators.  INT8 bytes use
//    v_perm to form (1024+q) pairs the same way.
//  * The first step's weight loads are issued before the activation is
//    arranged (once per workgroup, in LDS, in that pair order with the
//    per-chunk sums) and copied into registers.  Then each chunk register is
//    refilled with the next step's chunk as soon as it has been consumed
//    (rolling prefetch): one step in flight per lane, no idle gap between
//    steps.
//  * Row partials are reduced across lanes with DPP row operations and
//    v_readlane; rows spread over waves combine per-wave partials through
//    LDS once, at the end of the workgroup.
#include <stdlib.h>

#include <algorithm>

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
  static constexpr int kCpl = 5;     // chunk columns per lane (x in VGPRs)
};
template <>
struct Fmt<8> {
  static constexpr int kElems = 16;
  static constexpr int kXDw = 12;
  static constexpr int kCpl = 5;
};
template <>
struct Fmt<16> {
  static constexpr int kElems = 8;
  static constexpr int kXDw = 4;
  static constexpr int kCpl = 10;
};

constexpr uint32_t kMagic = 0x64006400u;  // fp16 pair (1024, 1024)

__device__ __forceinline__ uint32_t pack_h(uint32_t lo16, uint32_t hi16) {
  return (lo16 & 0xFFFFu) | (hi16 << 16);
}

// Arranges one chunk of x (E fp16 values as E/2 dwords in `raw`) into the
// prepared layout at dst.
template <int WBITS>
__device__ __forceinline__ void prep_raw(const uint32_t* raw, uint32_t* __restrict__ dst) {
  // sums of x in element order; a v_dot2_f32_f16 with (1, 0) / (0, 1) / (1, 1)
  // adds exact products, i.e. one rounding per step as in a scalar sum
  const uint32_t one_lo = 0x00003C00u, one_hi = 0x3C000000u, one_both = 0x3C003C00u;
  if constexpr (WBITS == 4) {
    float se = 0.f, so = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      se = __builtin_amdgcn_fdot2(as_h2(raw[k]), as_h2(one_lo), se, false);
      so = __builtin_amdgcn_fdot2(as_h2(raw[k]), as_h2(one_hi), so, false);
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
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      dst[k] = raw[k];
      dst[4 + k] = raw[4 + k];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k)
      s = __builtin_amdgcn_fdot2(as_h2(raw[k]), as_h2(one_both), s, false);
    dst[8] = __float_as_uint(s);
    dst[9] = dst[10] = dst[11] = 0u;
  } else {
    (void)one_lo;
    (void)one_hi;
    (void)one_both;
#pragma unroll
    for (int k = 0; k < 4; ++k) dst[k] = raw[k];
  }
}

// Arranges chunk c of x (fp16 in global memory) into the prepared layout.
template <int WBITS>
__device__ __forceinline__ void prep_chunk(const uint16_t* __restrict__ x, int c,
                                           uint32_t* __restrict__ dst) {
  constexpr int E = Fmt<WBITS>::kElems;
  const u4_t* src = reinterpret_cast<const u4_t*>(x + (int64_t)c * E);
  uint32_t raw[E / 2];
#pragma unroll
  for (int i = 0; i < E / 8; ++i) {
    const u4_t v = src[i];
    raw[4 * i + 0] = v[0];
    raw[4 * i + 1] = v[1];
    raw[4 * i + 2] = v[2];
    raw[4 * i + 3] = v[3];
  }
  prep_raw<WBITS>(raw, dst);
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

// Plain staging: x as fp16.  Thread t arranges chunks t, t + 256, ... (at
// most NPC); their loads are requested before the first weight steps (see
// NormIn), at clamped addresses so that they are straight-line code.
template <int WBITS, int LPR, int CPL>
struct PlainIn {
  static constexpr int XD = Fmt<WBITS>::kXDw;
  static constexpr int kRow = (LPR * CPL + 255) / 256;      // chunks a row of this shape has
  static constexpr int kLds = (65536 / (XD * 4) + 255) / 256;  // chunks the LDS stage holds
  static constexpr int NPC = kRow < kLds ? kRow : kLds;
  static constexpr int W = Fmt<WBITS>::kElems / 2;  // dwords per chunk
  uint32_t raw[NPC][W];
};

template <int WBITS, int LPR, int CPL>
__device__ __forceinline__ void plain_issue(const uint16_t* __restrict__ x,
                                            PlainIn<WBITS, LPR, CPL>& in, int cpr) {
  using P = PlainIn<WBITS, LPR, CPL>;
#pragma unroll
  for (int i = 0; i < P::NPC; ++i) {
    const int c = min((int)threadIdx.x + 256 * i, cpr - 1);
    const u4_t* src = reinterpret_cast<const u4_t*>(x + (int64_t)c * Fmt<WBITS>::kElems);
#pragma unroll
    for (int q = 0; q < P::W / 4; ++q) {
      const u4_t v = src[q];
      in.raw[i][4 * q] = v[0];
      in.raw[i][4 * q + 1] = v[1];
      in.raw[i][4 * q + 2] = v[2];
      in.raw[i][4 * q + 3] = v[3];
    }
  }
}

// The plain staging's counterpart of norm_pin.
template <int WBITS, int LPR, int CPL>
__device__ __forceinline__ void plain_pin(PlainIn<WBITS, LPR, CPL>& in) {
  using P = PlainIn<WBITS, LPR, CPL>;
#pragma unroll
  for (int i = 0; i < P::NPC; ++i)
#pragma unroll
    for (int k = 0; k < P::W; ++k) asm volatile("" : "+v"(in.raw[i][k])::"memory");
}

template <int WBITS, int LPR, int CPL>
__device__ __forceinline__ void stage_x(const PlainIn<WBITS, LPR, CPL>& in, uint32_t* xs,
                                        int cpr) {
  using P = PlainIn<WBITS, LPR, CPL>;
#pragma unroll
  for (int i = 0; i < P::NPC; ++i) {
    const int c = threadIdx.x + 256 * i;
    if (c < cpr) prep_raw<WBITS>(in.raw[i], xs + c * P::XD);
  }
  __syncthreads();
}

// Activation of a fused-norm GEMV: x = FWHT32(fp16(a [+ b]) * rrms * gamma)
// per 32-element chunk, rrms = 1 / sqrt(sum (a [+ b])^2 / K + eps), with
// the arithmetic (and reduction order) of the standalone row-norm kernel, so
// the prepared activation is bit-identical to norm-then-GEMV.  Workgroup 0
// stores the rounded residual fp16(a + b) to res_out.  One chunk per
// thread: K <= 32 * blockDim.x.
struct GemvNorm {
  const uint16_t* b;      // residual input (NULL: plain RMSNorm of x)
  const uint16_t* gamma;  // [K] norm weight
  uint16_t* res_out;      // [K] fp16(x + b), when b != NULL
  float eps;
  // SiLU split epilogue / mixed staging: fp32 products of elements
  // [split, I) (indexed by element) and the split point (a multiple of 32)
  float* h;
  int split;
  // linear map only: the first half of the workgroups take `skew` steps
  // more than an equal share, the second half `skew` fewer
  int skew = 0;
};

// Inputs of the fused-norm staging, requested before the first weight steps:
// loads retire in issue order, so activation loads issued after the weights
// would hold the staging arithmetic until every prefetched weight step had
// landed.  Every thread loads (its chunk clamped to the last one, and x in
// place of a missing residual), so the loads are straight-line code.
struct NormIn {
  uint32_t g[16], a[16], b[16];
};

__device__ __forceinline__ void norm_issue(const uint16_t* __restrict__ x, const GemvNorm& nm,
                                           NormIn& in, int K) {
  const int c = min((int)threadIdx.x, K / 32 - 1);
  load16w(nm.gamma + c * 32, in.g);
  load16w(x + c * 32, in.a);
  load16w((nm.b ? nm.b : x) + c * 32, in.b);
}

// Marks the fused-norm inputs as consumed here: the empty asm statements
// (memory clobber) keep the weight loads issued above them and the norm
// arithmetic below, so the wait they imply covers only the earlier
// activation loads.
__device__ __forceinline__ void norm_pin(NormIn& in) {
  asm volatile("" : "+v"(in.g[0]), "+v"(in.g[1]), "+v"(in.g[2]), "+v"(in.g[3]), "+v"(in.g[4]),
               "+v"(in.g[5]), "+v"(in.g[6]), "+v"(in.g[7]), "+v"(in.g[8]), "+v"(in.g[9]),
               "+v"(in.g[10]), "+v"(in.g[11]), "+v"(in.g[12]), "+v"(in.g[13]), "+v"(in.g[14]),
               "+v"(in.g[15])::"memory");
  asm volatile("" : "+v"(in.a[0]), "+v"(in.a[1]), "+v"(in.a[2]), "+v"(in.a[3]), "+v"(in.a[4]),
               "+v"(in.a[5]), "+v"(in.a[6]), "+v"(in.a[7]), "+v"(in.a[8]), "+v"(in.a[9]),
               "+v"(in.a[10]), "+v"(in.a[11]), "+v"(in.a[12]), "+v"(in.a[13]), "+v"(in.a[14]),
               "+v"(in.a[15])::"memory");
  asm volatile("" : "+v"(in.b[0]), "+v"(in.b[1]), "+v"(in.b[2]), "+v"(in.b[3]), "+v"(in.b[4]),
               "+v"(in.b[5]), "+v"(in.b[6]), "+v"(in.b[7]), "+v"(in.b[8]), "+v"(in.b[9]),
               "+v"(in.b[10]), "+v"(in.b[11]), "+v"(in.b[12]), "+v"(in.b[13]), "+v"(in.b[14]),
               "+v"(in.b[15])::"memory");
}

template <int WBITS>
__device__ __forceinline__ void stage_x_norm(const NormIn& in, const GemvNorm& nm, uint32_t* xs,
                                             float* red, int K) {
  constexpr int E = Fmt<WBITS>::kElems;
  constexpr int XD = Fmt<WBITS>::kXDw;
  const int c = threadIdx.x;
  const bool act = c < K / 32;
  // Without a residual, b is -0: fp16 a + (-0) == a and fp32(a) + (-0) ==
  // fp32(a) exactly, so one code path serves both.  Every thread computes
  // (idle ones on a clamped chunk, masked below): the loads are used
  // unconditionally and cannot sink behind the weight loads.
  uint32_t b[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) b[k] = nm.b ? in.b[k] : 0x80008000u;
  uint32_t r[16];
  float ss = norm_chunk_sumsq<true>(in.a, b, r, 0.f);
  ss = act ? ss : 0.f;
  const float tot = block_sum(ss, red);
  const float rrms = 1.0f / __builtin_sqrtf(tot / (float)K + nm.eps);
  if (act) {
    // the residual is rounded to fp16 before normalisation
    if (nm.b && blockIdx.x == 0) store16w(nm.res_out + c * 32, r);
    uint32_t raw[16];
    norm_chunk_scale<true>(r, in.g, rrms, raw);
#pragma unroll
    for (int sub = 0; sub < 32 / E; ++sub)
      prep_raw<WBITS>(raw + sub * (E / 2), xs + (c * (32 / E) + sub) * XD);
  }
  __syncthreads();
}

// Activation of the down projection after the split SiLU-gate epilogue:
// elements below `split` are fp16 already (x); above it x = fp16(FWHT32(h))
// per 32-element piece from the fp32 products h, with the butterflies,
// scaling and rounding of silu_kernel<true> (fwht32, store32h), so the
// staged activation is bit-identical to that kernel's output.  Thread t
// stages pieces t, t + 256, ... (at most NPF); all of them are requested
// before the first weight steps (see NormIn), at clamped addresses: a round
// of 256 pieces wholly below the split as 16 dwords of x each, any other as
// 32 dwords, from h for an fp32 piece or from x (its 16 dwords read twice)
// for an fp16 one, without per-thread branches.
template <int WBITS, int LPR, int CPL>
struct FwhtIn {
  static constexpr int XD = Fmt<WBITS>::kXDw;
  static constexpr int kRow = (LPR * CPL * Fmt<WBITS>::kElems / 32 + 255) / 256;
  static constexpr int kLds =
      (65536 / (XD * 4) * Fmt<WBITS>::kElems / 32 + 255) / 256;  // pieces the LDS stage holds
  static constexpr int NPF = kRow < kLds ? kRow : kLds;
  uint32_t raw[NPF][32];
};

template <int WBITS, int LPR, int CPL>
__device__ __forceinline__ void fwht_issue(const uint16_t* __restrict__ x,
                                           const float* __restrict__ h, int split,
                                           FwhtIn<WBITS, LPR, CPL>& in, int K) {
  const int wv = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
#pragma unroll
  for (int i = 0; i < FwhtIn<WBITS, LPR, CPL>::NPF; ++i) {
    const int p = min((int)threadIdx.x + 256 * i, K / 32 - 1);
    if (i > 0 && 256 * i + 64 * wv >= K / 32) {
      // wave-uniform: no piece of this wave in this round (none staged), and
      // the wave has loads of earlier rounds in flight on either path
#pragma unroll
      for (int k = 0; k < 32; ++k) in.raw[i][k] = 0u;
    } else if (256 * i + 256 <= split / 32) {
      // the whole round is fp16 (workgroup-uniform; the SiLU split puts
      // whole rounds of 256 pieces below it): 16 dwords per piece
      const u4_t* src = reinterpret_cast<const u4_t*>(x + (int64_t)p * 32);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u4_t v = src[q];
        in.raw[i][4 * q] = v[0];
        in.raw[i][4 * q + 1] = v[1];
        in.raw[i][4 * q + 2] = v[2];
        in.raw[i][4 * q + 3] = v[3];
      }
#pragma unroll
      for (int k = 16; k < 32; ++k) in.raw[i][k] = 0u;  // unused by fp16 pieces
    } else {
      const bool half = 32 * p < split;
      const u4_t* src = half ? reinterpret_cast<const u4_t*>(x + (int64_t)p * 32)
                             : reinterpret_cast<const u4_t*>(h + (int64_t)p * 32);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const u4_t v = src[half ? (q & 3) : q];
        in.raw[i][4 * q] = v[0];
        in.raw[i][4 * q + 1] = v[1];
        in.raw[i][4 * q + 2] = v[2];
        in.raw[i][4 * q + 3] = v[3];
      }
    }
  }
}

template <int WBITS, int LPR, int CPL>
__device__ __forceinline__ void fwht_pin(FwhtIn<WBITS, LPR, CPL>& in) {
#pragma unroll
  for (int i = 0; i < FwhtIn<WBITS, LPR, CPL>::NPF; ++i)
#pragma unroll
    for (int k = 0; k < 32; ++k) asm volatile("" : "+v"(in.raw[i][k])::"memory");
}

template <int WBITS, int LPR, int CPL>
__device__ __forceinline__ void stage_x_fwht(FwhtIn<WBITS, LPR, CPL>& in, int split, uint32_t* xs,
                                             int K) {
  constexpr int E = Fmt<WBITS>::kElems;
  constexpr int XD = Fmt<WBITS>::kXDw;
#pragma unroll
  for (int i = 0; i < FwhtIn<WBITS, LPR, CPL>::NPF; ++i) {
    const int c = threadIdx.x + 256 * i;
    if (c >= K / 32) break;
    uint32_t* raw = in.raw[i];
    if (32 * c >= split) {
      float v[32];
#pragma unroll
      for (int k = 0; k < 32; ++k) v[k] = __uint_as_float(raw[k]);
      fwht32(v);
#pragma unroll
      for (int k = 0; k < 16; ++k)
        raw[k] = (uint32_t)f2h(v[2 * k]) | ((uint32_t)f2h(v[2 * k + 1]) << 16);
    }
#pragma unroll
    for (int sub = 0; sub < 32 / E; ++sub)
      prep_raw<WBITS>(raw + sub * (E / 2), xs + (c * (32 / E) + sub) * XD);
  }
  __syncthreads();
}

// Input modes of the GEMV: x as fp16, the fused residual + RMSNorm + FWHT
// of GemvNorm, or fp32 SiLU products through stage_x_fwht.
constexpr int kXPlain = 0, kXNorm = 1, kXFwht = 2;
// Epilogues: fp16 rows; the SiLU unit map (64-row units, fp16 FWHT32 of the
// gated products); the SiLU split map (whole units first, then pairs of
// the remaining rows as fp32 gated products, no FWHT).
constexpr int kEpiRows = 0, kEpiSiluUnit = 1, kEpiSiluPair = 2;

template <int WBITS>
__device__ __forceinline__ uint32_t load_sz(const uint32_t* __restrict__ srow, int c) {
  if constexpr (WBITS == 4) return srow[c];
  else if constexpr (WBITS == 8) return srow[c >> 1];
  else return 0u;
}

// Rows are processed in "steps" of RPS = 256/LPR rows per workgroup: LPR
// lanes share a row (LPR <= 64: inside one wave; 128/256: 2/4 waves) and
// lane `cl` of a row owns chunk columns cl + LPR*i, i < CPL (columns past the
// row end are masked).  A RowMap gives the first row of the workgroup's k-th
// step.  The tile is a ring of UB register slots, one step each; the first
// UB steps are requested before the activation is staged, so that staging
// hides behind the weight stream.
template <int WBITS, int LPR, int CPL, int UB>
struct GemvTile {
  static constexpr int RPS = 256 / LPR;
  u4_t wq[UB][CPL];
  uint32_t s2[UB][CPL];
};

// Linear map: workgroup g takes global steps g, g + G, ...  SiLU unit map
// (gate / up halves of a [2I] output): a unit is 32 gate rows and the 32 up
// rows of the same indices; workgroup g takes units g, g + G, ..., each as
// SPU consecutive steps (gate rows first).  SiLU split map: workgroup g < F
// first takes unit g as above; the rows from 32 F on go in pair steps of RPS
// gate rows and the RPS up rows of the same indices, taken as two
// consecutive local steps (gate, then up) by the same lanes; workgroup g
// takes pair steps g, g + G, ... of those.
template <int RPS, int EPI>
struct RowMap {
  int g, G, nsteps;  // linear
  int skew = 0, per = 0;  // linear, skewed: per = nsteps / G exactly
  int I, nunits;     // SiLU: I = N / 2; nunits = I / 32 (unit) or F (split)
  int npairs;        // split: pair steps after the units
  float* h;          // split: fp32 products, indexed by element
  static constexpr int SPU = 64 / RPS;
  __device__ int nunit_steps() const { return g < nunits ? SPU : 0; }
  __device__ int nlocal() const {
    if constexpr (EPI == kEpiSiluUnit) return g < nunits ? ((nunits - g + G - 1) / G) * SPU : 0;
    else if constexpr (EPI == kEpiSiluPair)
      return nunit_steps() + (g < npairs ? ((npairs - g + G - 1) / G) * 2 : 0);
    else if (skew > 0) return g < G / 2 ? per + skew : per - skew;
    else return g < nsteps ? (nsteps - g + G - 1) / G : 0;
  }
  __device__ int row0(int k) const {
    if constexpr (EPI == kEpiSiluUnit) {
      const int u = g + G * (k / SPU), sub = k % SPU;
      return sub < SPU / 2 ? 32 * u + RPS * sub : I + 32 * u + RPS * (sub - SPU / 2);
    } else if constexpr (EPI == kEpiSiluPair) {
      const int us = nunit_steps();
      if (k < us) return k < SPU / 2 ? 32 * g + RPS * k : I + 32 * g + RPS * (k - SPU / 2);
      const int kk = k - us;
      const int p0 = 32 * nunits + RPS * (g + G * (kk >> 1));
      return (kk & 1) ? I + p0 : p0;
    } else {
      if (skew > 0 && k >= per - skew)  // past the common steps: first half only
        return ((per - skew) * G + (k - (per - skew)) * (G / 2) + g) * RPS;
      return (g + G * k) * RPS;
    }
  }
};

template <int WBITS, int LPR, int CPL, int UB, class Map>
__device__ __forceinline__ void gemv_load(GemvTile<WBITS, LPR, CPL, UB>& t,
                                          const uint8_t* __restrict__ w,
                                          const uint32_t* __restrict__ sz, int64_t row_bytes,
                                          int nb, int cpr, int N, const Map& map, int k0,
                                          int nloc, int rs, int cl) {
  // each weight chunk with its (scale, zero) word, so that the first chunks'
  // arithmetic can start while the rest of the step is in flight
#pragma unroll
  for (int j = 0; j < UB; ++j) {
    const int k = max(0, min(k0 + j, nloc - 1));  // clamped: in bounds
    const int rowc = min(map.row0(k) + rs, N - 1);
    const u4_t* wrow = reinterpret_cast<const u4_t*>(w + (int64_t)rowc * row_bytes);
    const uint32_t* srow = sz + (int64_t)rowc * nb;
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = min(cl + LPR * i, cpr - 1);
      t.wq[j][i] = load_nt(wrow + c);
      t.s2[j][i] = load_sz<WBITS>(srow, c);
    }
  }
}

// y[32u + i] = fp16(FWHT32(silu(g_i) * u_i)) for one SiLU unit whose
// fp16-rounded gate/up rows sit in ut[0..31] / ut[32..63]; the arithmetic of
// silu_kernel<true>, with the butterflies across lanes 0..31 of wave 0.
__device__ __forceinline__ void silu_unit(const float* ut, uint16_t* __restrict__ y, int u) {
#pragma clang fp contract(off)  // g / (1 + e^-g) * u in separately rounded steps
  if (threadIdx.x >= 64) return;
  const int i = threadIdx.x & 31;
  const float gv = ut[i], uv = ut[32 + i];
  float v = gv / (1.0f + expf(-gv)) * uv;
#pragma unroll
  for (int bit = 1; bit <= 16; bit <<= 1) {
    const float o = __shfl_xor(v, bit);
    v = (i & bit) ? o - v : v + o;
  }
  v *= kInvSqrt32;
  if (threadIdx.x < 32) y[32 * u + i] = f2h(v);
}

// silu(g) * u as silu_kernel computes it (separately rounded fp32 steps).
__device__ __forceinline__ float silu_mul(float g, float u) {
#pragma clang fp contract(off)
  return g / (1.0f + expf(-g)) * u;
}

// Finishes step k (the k-th of this workgroup) from the lane partials
// `acc`.  Rows spread over several waves leave one partial per (step, wave)
// in `red`; they are combined once, after the last step.  In the SiLU map
// each row's fp16-rounded result goes to the unit buffer `ut`, and the
// unit's last step writes its 32 outputs.  In the pair steps of the SiLU
// split map the gate step parks each row's fp16-rounded value in
// ut[128 + row slot] (the same lane reads it back), and the up step writes
// silu(g) * u as fp32 to h.
template <int LPR, class Map, int EPI>
__device__ __forceinline__ void gemv_finish(float acc, uint16_t* __restrict__ y, float* red,
                                            float* ut, int N, const Map& map, int k, int rs,
                                            int cl) {
  constexpr int RPS = 256 / LPR;
  if constexpr (LPR <= 64) {
    const float total = reduce_lr(acc, LPR);
    if (EPI == kEpiSiluPair && k >= map.nunit_steps()) {  // workgroup-uniform
      if (cl == 0) {
        const float v = h2f(f2h(total));
        if (((k - map.nunit_steps()) & 1) == 0) {
          ut[128 + rs] = v;
        } else {
          const int row = map.row0(k) - map.I + rs;
          map.h[row] = silu_mul(ut[128 + rs], v);
        }
      }
    } else if constexpr (EPI == kEpiSiluUnit || EPI == kEpiSiluPair) {
      constexpr int SPU = Map::SPU;
      const int sub = k % SPU;
      const int slot = (k / SPU) & 1;
      const int idx = sub < SPU / 2 ? RPS * sub + rs : 32 + RPS * (sub - SPU / 2) + rs;
      if (cl == 0) ut[slot * 64 + idx] = h2f(f2h(total));
      if (sub == SPU - 1) {  // unit complete (workgroup-uniform)
        __syncthreads();
        silu_unit(ut + slot * 64, y, map.g + map.G * (k / SPU));
      }
    } else {
      const int row = map.row0(k) + rs;
      if (row < N && cl == 0) y[row] = f2h(total);
    }
  } else {
    const float total = reduce_lr(acc, 64);
    if ((threadIdx.x & 63) == 0) red[k * 4 + (threadIdx.x >> 6)] = total;
  }
}

// One step from a slot of the register ring (wq / s2: CPL chunks and their
// (scale, zero) words) with a rolling refill: as soon as chunk i of step k
// has been consumed, its register receives chunk i of step kn, so the loads
// of the steps ahead overlap this step's arithmetic.
template <int WBITS, int LPR, int CPL, class Map, int EPI, bool NEXT>
__device__ __forceinline__ void gemv_step_roll(u4_t (&wq)[CPL], uint32_t (&s2)[CPL],
                                               const uint32_t* __restrict__ xr,
                                               const uint8_t* __restrict__ w,
                                               const uint32_t* __restrict__ sz,
                                               int64_t row_bytes, int nb,
                                               uint16_t* __restrict__ y, float* red, float* ut,
                                               int cpr, int N, const Map& map, int k, int kn,
                                               int rs, int cl) {
  constexpr int XD = Fmt<WBITS>::kXDw;
  const u4_t* wrow = nullptr;
  const uint32_t* srow = nullptr;
  if constexpr (NEXT) {
    const int rown = min(map.row0(kn) + rs, N - 1);
    wrow = reinterpret_cast<const u4_t*>(w + (int64_t)rown * row_bytes);
    srow = sz + (int64_t)rown * nb;
  }
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    if (LPR * CPL <= cpr || cl + LPR * i < cpr)
      acc = chunk_dot<WBITS>(wq[i], s2[i], xr + i * XD, acc);
    if constexpr (NEXT) {
      const int c = min(cl + LPR * i, cpr - 1);
      wq[i] = load_nt(wrow + c);
      s2[i] = load_sz<WBITS>(srow, c);
    }
  }
  gemv_finish<LPR, Map, EPI>(acc, y, red, ut, N, map, k, rs, cl);
}

template <int WBITS, int LPR, int CPL, int UB, int XM, int EPI>
__global__ __launch_bounds__(256) void gemv_kernel(const uint16_t* __restrict__ x,
                                                   const uint8_t* __restrict__ w,
                                                   const uint32_t* __restrict__ sz,
                                                   uint16_t* __restrict__ y, int N, int K,
                                                   GemvNorm nm) {
  static_assert(EPI == kEpiRows || LPR <= 64, "the SiLU epilogues need rows inside one wave");
  constexpr int XD = Fmt<WBITS>::kXDw;
  constexpr int RPS = 256 / LPR;
  constexpr int WPR = LPR > 64 ? LPR / 64 : 1;  // waves per row
  extern __shared__ __align__(16) uint32_t xs[];
  __shared__ float ut[EPI == kEpiSiluUnit ? 128 : EPI == kEpiSiluPair ? 128 + RPS : 1];
  const int cpr = K / Fmt<WBITS>::kElems;
  const int nb = K / 32;
  const int64_t row_bytes = (int64_t)K * WBITS / 8;
  const int rs = threadIdx.x / LPR, cl = threadIdx.x % LPR;
  RowMap<RPS, EPI> map;
  map.g = blockIdx.x;
  map.G = gridDim.x;
  map.nsteps = (N + RPS - 1) / RPS;
  map.I = N / 2;
  map.nunits = EPI == kEpiSiluPair ? nm.split / 32 : N / 64;
  map.npairs = (N / 2 - nm.split) / RPS;
  map.h = nm.h;
  if constexpr (EPI == kEpiRows) {
    map.skew = nm.skew;
    map.per = map.nsteps / map.G;
  }
  const int nloc = map.nlocal();

  NormIn nin;
  PlainIn<WBITS, LPR, CPL> pin;
  FwhtIn<WBITS, LPR, CPL> fin;
  if constexpr (XM == kXNorm) norm_issue(x, nm, nin, K);
  else if constexpr (XM == kXPlain) plain_issue(x, pin, cpr);
  else fwht_issue(x, nm.h, nm.split, fin, K);
  // the first UB steps (unconditional and clamped, so that the compiler's
  // wait counts stay exact: a workgroup without steps re-reads a valid row)
  GemvTile<WBITS, LPR, CPL, UB> ta;
  gemv_load(ta, w, sz, row_bytes, nb, cpr, N, map, 0, nloc, rs, cl);

  if constexpr (XM == kXNorm) {
    __shared__ float nred[4];
    norm_pin(nin);
    stage_x_norm<WBITS>(nin, nm, xs, nred, K);
  } else if constexpr (XM == kXFwht) {
    fwht_pin(fin);
    stage_x_fwht(fin, nm.split, xs, K);
  } else {
    plain_pin(pin);
    stage_x(pin, xs, cpr);
  }
  uint32_t xr[CPL * XD];
#pragma unroll
  for (int i = 0; i < CPL; ++i) lds_copy<XD>(xs + min(cl + LPR * i, cpr - 1) * XD, xr + i * XD);
  // the staging area becomes the cross-wave partial buffer
  float* red = reinterpret_cast<float*>(xs);
  if constexpr (WPR > 1) __syncthreads();

  // Rolling prefetch over a ring of UB steps: step k is computed from slot
  // k % UB, which then receives step k + UB, so UB steps stay in flight per
  // lane.  The first UB steps were requested before the activation staging.
  // One step in flight (UB = 1) is the default: it keeps the chip near the
  // ~8-16 MB in flight at which HBM streams best.  Measured in the 40-layer
  // step with the activation loads issued first: 2, 3 and 4 steps in flight
  // made every projection slower (qkv + norm 8.0 -> 8.2 / 10.2 us, gate_up
  // 20.2 -> 21.2 / 26.5 us, down 12.6 -> 13.3 / 20.1 us); load-then-compute
  // batches were slower still (11.9 vs 10.4 us for 17408 x 5120 INT4).
  // Steady-state blocks of UB steps refill every slot; only the last
  // 2 UB - 1 steps test for the end.
  int k0 = 0;
  for (; k0 + 2 * UB <= nloc; k0 += UB) {
#pragma unroll
    for (int j = 0; j < UB; ++j)
      gemv_step_roll<WBITS, LPR, CPL, RowMap<RPS, EPI>, EPI, true>(
          ta.wq[j], ta.s2[j], xr, w, sz, row_bytes, nb, y, red, ut, cpr, N, map, k0 + j,
          k0 + j + UB, rs, cl);
  }
#pragma unroll
  for (int jj = 0; jj < 2 * UB - 1; ++jj) {
    const int k = k0 + jj, j = jj % UB;
    if (k >= nloc) break;  // workgroup-uniform
    if (k + UB < nloc)
      gemv_step_roll<WBITS, LPR, CPL, RowMap<RPS, EPI>, EPI, true>(
          ta.wq[j], ta.s2[j], xr, w, sz, row_bytes, nb, y, red, ut, cpr, N, map, k, k + UB, rs,
          cl);
    else
      gemv_step_roll<WBITS, LPR, CPL, RowMap<RPS, EPI>, EPI, false>(
          ta.wq[j], ta.s2[j], xr, w, sz, row_bytes, nb, y, red, ut, cpr, N, map, k, 0, rs, cl);
  }
  if constexpr (WPR > 1) {
    __syncthreads();
    for (int e = threadIdx.x; e < nloc * RPS; e += 256) {
      const int kk = e / RPS, r = e % RPS;
      const int row = map.row0(kk) + r;
      const float* p = red + kk * 4 + r * WPR;
      const float total = WPR == 2 ? p[0] + p[1] : (p[0] + p[1]) + (p[2] + p[3]);
      if (row < N) y[row] = f2h(total);
    }
  }
}

template <int WBITS>
int launch_gemv_fmt(const void* x, const void* w, const void* sz, void* y, int64_t N, int64_t K,
                    const GemvNorm* norm, int xm, int epi, hipStream_t st) {
  constexpr int E = Fmt<WBITS>::kElems;
  constexpr int XD = Fmt<WBITS>::kXDw;
  constexpr int kCpl = Fmt<WBITS>::kCpl;
  const int cpr = (int)(K / E);
  const size_t lds = (size_t)cpr * XD * 4;
  R4Q_REQUIRE(lds <= 64 * 1024, "gemv: K=%lld too large for the LDS activation stage",
              (long long)K);
  // lanes per row: the fewest (>= 16) that keep every lane at <= 5 chunks,
  // or at <= kCpl when 256 lanes cannot
  int lpr = 16;
  while (lpr < 256 && lpr * 5 < cpr) lpr *= 2;
  if (const int v = tuning().gemv_lpr.load()) lpr = v;  // measurement override (r4q_tune)
  R4Q_REQUIRE(lpr * kCpl >= cpr, "gemv: K=%lld needs more than 256 lanes per row", (long long)K);
  const int rps = 256 / lpr;
  if (epi != kEpiRows)
    R4Q_REQUIRE(lpr <= 64 && N % 64 == 0,
                "gemv: SiLU epilogue needs N %% 64 == 0 and rows inside a wave");
  // work items: steps of rps rows; SiLU unit map: units of 64 rows; SiLU
  // split map: one workgroup per whole unit below the split (F of them),
  // else pair steps (rps gate rows + their rps up rows)
  const int64_t F = epi == kEpiSiluPair ? norm->split / 32 : 0;
  const int64_t nsteps = epi == kEpiSiluUnit   ? N / 64
                         : epi == kEpiSiluPair ? (F > 0 ? F : (N / 2 - norm->split) / rps)
                                               : (N + rps - 1) / rps;
  // Workgroups: about the resident capacity (measured best: 4 per CU for
  // rows inside one wave, 2-3 per CU for rows spread over waves), with an
  // equal number of steps each.  A fused-norm prologue is paid once per
  // workgroup and the workgroups of a CU compute it on the same SIMDs: at
  // most one per CU (measured 9.1 -> 8.2 us for 7168 x 5120 INT4), except
  // in the SiLU maps: the unit map needs one workgroup per 64-row unit (as
  // does the split map when it has units); pair steps alone measured best
  // at 768.  Two exceptions, measured on MI355X (cold weights, graph-replayed):
  // a plain GEMV of at most 3 x 256 steps runs one workgroup per CU (5120 x
  // 5120 INT4: 214 workgroups of 3 steps 4.74 us, 640 of 1: 5.22 us, 320 of
  // 2: 5.65 us), and a fused-norm GEMV at 64 lanes per row two per CU (7168 x
  // 5120 INT8: 448 workgroups of 4 steps 9.59 us, 256 of 7: 10.5 us).
  // Plain GEMVs at <= 32 lanes per row follow the most loaded CU's work,
  // ceil(workgroups / 256) x (steps per workgroup + 1, for the workgroup's
  // activation staging and tail): that count is minimised (at most 12 steps
  // each), with the fewest workgroups among equal counts (17408 x 5120 INT4:
  // 242 workgroups of 9 steps 9.95 us, 726 of 3: 10.46, 272 of 8: 12.60;
  // 34816 x 5120: 484 of 9 18.1 us, 871 of 5: 19.4, 544 of 8: 21.4).
  const bool nrm = xm == kXNorm;
  int dflt = nrm ? (lpr == 128 ? 512 : epi != kEpiRows ? 768 : lpr == 64 ? 512 : 256)
                 : (lpr <= 64 ? 1024 : lpr == 128 ? 512 : 768);
  if (xm == kXPlain && epi == kEpiRows && (nsteps + 255) / 256 <= 3) dflt = 256;
  const int wgs_o = tuning().gemv_wgs.load(), ub_o = tuning().gemv_ub.load();
  const int max_wg = wgs_o ? wgs_o : dflt;
  int64_t per = F > 0 ? 1 : (nsteps + max_wg - 1) / max_wg;
  if (!wgs_o && xm == kXPlain && epi == kEpiRows && lpr <= 32) {
    int64_t best = INT64_MAX;
    for (int64_t p = 1; p <= 12; ++p) {
      const int64_t cost = ((nsteps + p - 1) / p + 255) / 256 * (p + 1);
      if (cost <= best) {
        best = cost;
        per = p;
      }
    }
  }
  const int64_t grid = (nsteps + per - 1) / per;
  // steps in flight per lane: at most the steps a workgroup has (a deeper
  // ring would re-read its last step)
  const int64_t spw = epi == kEpiSiluUnit   ? (64 / rps) * per
                      : epi == kEpiSiluPair ? (F > 0 ? 64 / rps : 0) +
                                                  2 * (((N / 2 - norm->split) / rps + grid - 1) / grid)
                                            : per;
  const int ub = (int)std::max<int64_t>(1, std::min<int64_t>(ub_o ? ub_o : 1, spw));
  // Two workgroups per CU: the CU's second workgroup (the second half of
  // the grid, dispatched once every CU holds one) stages its activation
  // beside the first and finishes its equal share ~1.4 us later (in-kernel
  // stamps, 512-workgroup down projection: first half's exits median 9.3-9.4
  // us, second half's 10.8 us).  So a grid of two equal shares per CU gives
  // the first half one step more and the second half one step less (40-layer
  // step 2.637 -> 2.623 ms; two steps: 2.632 ms).  gemv_skew overrides the
  // difference: value - 1 steps (1 = equal shares) on any even grid of
  // more than 256 equal shares.
  int skew = per >= 4 && grid == 2 * 256 ? 1 : 0;
  if (const int v = tuning().gemv_skew.load()) skew = v - 1;
  if (!(epi == kEpiRows && grid > 256 && grid % 2 == 0 && grid * per == nsteps && skew < per))
    skew = 0;
  // the staging area also holds one partial per (step, wave) of the workgroup
  const size_t lds_all = lds > (size_t)(per + skew) * 16 ? lds : (size_t)(per + skew) * 16;
  R4Q_REQUIRE(lds_all <= 64 * 1024, "gemv: N=%lld too large for one launch", (long long)N);
  const dim3 gd((unsigned)grid), bd(256);
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* wp = static_cast<const uint8_t*>(w);
  const auto* sp = static_cast<const uint32_t*>(sz);
  auto* yp = static_cast<uint16_t*>(y);
  if (nrm) R4Q_REQUIRE(K <= 32 * 256, "gemv: fused norm needs K <= 8192 (K=%lld)", (long long)K);
  if (xm == kXFwht)
    R4Q_REQUIRE(norm && norm->split >= 0 && norm->split <= K && norm->split % 32 == 0 &&
                    (norm->h || norm->split == K) && (x || norm->split == 0),
                "gemv: bad FWHT staging split");
  GemvNorm nm = norm ? *norm : GemvNorm{nullptr, nullptr, nullptr, 0.f};
  nm.skew = skew;
#define R4Q_GEMV_K(L, U, XM, EPI)                                                             \
  hipLaunchKernelGGL((gemv_kernel<WBITS, L, kCpl, U, XM, EPI>), gd, bd, lds_all, st, xp, wp, sp, \
                     yp, (int)N, (int)K, nm)
  // rows inside one wave: every input mode; SiLU epilogues after the fp16
  // or fused-norm input
#define R4Q_GEMV(L, U)                                                                       \
  if (lpr == L && ub == U) {                                                                 \
    if (epi == kEpiSiluUnit && nrm) R4Q_GEMV_K(L, U, kXNorm, kEpiSiluUnit);                  \
    else if (epi == kEpiSiluUnit) R4Q_GEMV_K(L, U, kXPlain, kEpiSiluUnit);                   \
    else if (epi == kEpiSiluPair && nrm) R4Q_GEMV_K(L, U, kXNorm, kEpiSiluPair);             \
    else if (epi == kEpiSiluPair) R4Q_GEMV_K(L, U, kXPlain, kEpiSiluPair);                   \
    else if (nrm) R4Q_GEMV_K(L, U, kXNorm, kEpiRows);                                        \
    else if (xm == kXFwht) R4Q_GEMV_K(L, U, kXFwht, kEpiRows);                               \
    else R4Q_GEMV_K(L, U, kXPlain, kEpiRows);                                                \
    return launch_status("gemv");                                                            \
  }
  R4Q_GEMV(16, 1) R4Q_GEMV(32, 1) R4Q_GEMV(64, 1)
  R4Q_GEMV(16, 2) R4Q_GEMV(32, 2) R4Q_GEMV(64, 2)
#undef R4Q_GEMV
  // rows over 2 or 4 waves: fp16 rows from every input mode
#define R4Q_GEMV(L, U)                                                                       \
  if (lpr == L && ub == U) {                                                                 \
    if (nrm) R4Q_GEMV_K(L, U, kXNorm, kEpiRows);                                             \
    else if (xm == kXFwht) R4Q_GEMV_K(L, U, kXFwht, kEpiRows);                               \
    else R4Q_GEMV_K(L, U, kXPlain, kEpiRows);                                                \
    return launch_status("gemv");                                                            \
  }
  R4Q_GEMV(128, 1) R4Q_GEMV(256, 1) R4Q_GEMV(128, 2) R4Q_GEMV(256, 2)
#undef R4Q_GEMV
#undef R4Q_GEMV_K
  return fail(R4Q_EUNSUPPORTED, "gemv: no kernel for %d lanes/row, %d steps in flight", lpr, ub);
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
    case 4: return launch_gemv_fmt<4>(x, w, sz, y, N, K, nullptr, kXPlain, kEpiRows, st);
    case 8: return launch_gemv_fmt<8>(x, w, sz, y, N, K, nullptr, kXPlain, kEpiRows, st);
    default: return launch_gemv_fmt<16>(x, w, sz, y, N, K, nullptr, kXPlain, kEpiRows, st);
  }
}

int gemv_norm_launch(const void* a, const void* b, const void* gamma, void* res_out, float eps,
                     const void* w, const void* sz, void* y, int64_t N, int64_t K, int wbits,
                     hipStream_t st, SiluEpi silu, float* h, int64_t split) {
  R4Q_REQUIRE(a && (!b || (gamma && res_out)), "gemv_norm: null pointer");
  if (silu == SiluEpi::kSplit)
    R4Q_REQUIRE(split >= 0 && split <= N / 2 && split % 32 == 0 && (h || split == N / 2) &&
                    (y || split == 0),
                "gemv_norm: bad SiLU split %lld", (long long)split);
  const GemvNorm nm{static_cast<const uint16_t*>(b), static_cast<const uint16_t*>(gamma),
                    static_cast<uint16_t*>(res_out), eps, h, (int)split};
  const GemvNorm* np = (gamma || silu == SiluEpi::kSplit) ? &nm : nullptr;
  const int xm = gamma ? kXNorm : kXPlain;
  const int epi = silu == SiluEpi::kNone   ? kEpiRows
                  : silu == SiluEpi::kUnit ? kEpiSiluUnit
                                           : kEpiSiluPair;  // kSplit
  switch (wbits) {
    case 4: return launch_gemv_fmt<4>(a, w, sz, y, N, K, np, xm, epi, st);
    case 8: return launch_gemv_fmt<8>(a, w, sz, y, N, K, np, xm, epi, st);
    default: return launch_gemv_fmt<16>(a, w, sz, y, N, K, np, xm, epi, st);
  }
}

int gemv_fwht_launch(const void* x, const float* h, int64_t split, const void* w,
                     const void* sz, void* y, int64_t N, int64_t K, int wbits, hipStream_t st) {
  const GemvNorm nm{nullptr, nullptr, nullptr, 0.f, const_cast<float*>(h), (int)split};
  switch (wbits) {
    case 4: return launch_gemv_fmt<4>(x, w, sz, y, N, K, &nm, kXFwht, kEpiRows, st);
    case 8: return launch_gemv_fmt<8>(x, w, sz, y, N, K, &nm, kXFwht, kEpiRows, st);
    default: return launch_gemv_fmt<16>(x, w, sz, y, N, K, &nm, kXFwht, kEpiRows, st);
  }
}

int64_t gemv_silu_split(int64_t I) {
  // whole 64-row units in multiples of the 256 CUs (every CU gets the same
  // number), the rest as pair steps spread over all workgroups
  const int64_t units = I / 32;
  return 32 * (units >= 256 ? units - units % 256 : units);
}

bool gemv_silu_ok(int64_t N, int64_t K, int wbits) {
  const int64_t cpr = K / (wbits == 4 ? 32 : wbits == 8 ? 16 : 8);
  return N % 64 == 0 && cpr <= 64 * 5;  // rows inside one wave (lanes per row <= 64)
}

size_t gemm_ws_need(int64_t M, int64_t N, int64_t K, int wbits) {
  if (M > kSkinnyMaxRows) return gemm_ws_bytes(M, N, K, wbits);
  return gemm_skinny_ok(M, N, K, wbits) ? skinny_ws_bytes(M, N, K, wbits) : 0;
}

int gemm_launch(const void* x, const void* w, const void* sz, void* y, int64_t M, int64_t N,
                int64_t K, int wbits, hipStream_t st, void* ws, size_t ws_bytes) {
  if (M > kSkinnyMaxRows) return gemm_mfma_launch(x, w, sz, y, M, N, K, wbits, st, ws, ws_bytes);
  if (gemm_skinny_ok(M, N, K, wbits))
    return gemm_skinny_launch(x, w, sz, y, M, N, K, wbits, st, ws, ws_bytes);
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

extern "C" int r4q_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int wbits,
                                        size_t* bytes) {
  R4Q_REQUIRE(bytes, "gemm_workspace_bytes: null output");
  R4Q_REQUIRE(M >= 1 && N >= 1 && K >= 32 && K % 32 == 0 &&
                  (wbits == 4 || wbits == 8 || wbits == 16),
              "gemm_workspace_bytes: bad shape or format");
  *bytes = r4q::gemm_ws_need(M, N, K, wbits);
  return R4Q_OK;
}

extern "C" int r4q_gemm_ws(const void* x, const void* w, const void* sz, void* y, int64_t M,
                           int64_t N, int64_t K, int wbits, void* ws, size_t ws_bytes,
                           void* stream) {
  R4Q_REQUIRE(M >= 1, "gemm: M must be >= 1");
  R4Q_TRY(r4q::gemv_check(x, w, sz, y, N, K, wbits));
  R4Q_REQUIRE(ws || ws_bytes == 0, "gemm: workspace size without a workspace");
  R4Q_REQUIRE((reinterpret_cast<uintptr_t>(ws) & 15) == 0, "gemm: workspace must be 16-byte aligned");
  return r4q::gemm_launch(x, w, sz, y, M, N, K, wbits, r4q::as_stream(stream), ws, ws_bytes);
}

extern "C" int r4q_gemm_silu_fwht_ws(const void* x, const void* w, const void* sz, void* y,
                                     int64_t M, int64_t I, int64_t K, int wbits, void* ws,
                                     size_t ws_bytes, void* stream) {
  R4Q_REQUIRE(M >= 1 && I >= 1, "gemm_silu_fwht: bad shape");
  R4Q_TRY(r4q::gemv_check(x, w, sz, y, 2 * I, K, wbits));
  R4Q_REQUIRE(ws || ws_bytes == 0, "gemm_silu_fwht: workspace size without a workspace");
  R4Q_REQUIRE((reinterpret_cast<uintptr_t>(ws) & 15) == 0,
              "gemm_silu_fwht: workspace must be 16-byte aligned");
  R4Q_REQUIRE(r4q::gemm_skinny_silu_ok(M, I, K, wbits, ws ? ws_bytes : 0),
              "gemm_silu_fwht: M = %lld, I = %lld, K = %lld does not take the split skinny path "
              "(2 <= M <= 16, I %% 32 == 0, workspace of r4q_gemm_workspace_bytes(M, 2I, K))",
              (long long)M, (long long)I, (long long)K);
  return r4q::gemm_skinny_silu_launch(x, w, sz, y, M, I, K, wbits, r4q::as_stream(stream), ws,
                                      ws_bytes);
}

extern "C" int r4q_res_rmsnorm_fwht_gemv(const void* a, const void* b, const void* gamma,
                                         void* res_out, float eps, const void* w, const void* sz,
                                         void* y, int64_t N, int64_t K, int wbits,
                                         void* stream) {
  R4Q_TRY(r4q::gemv_check(a, w, sz, y, N, K, wbits));
  R4Q_REQUIRE(gamma && (!b || res_out), "res_rmsnorm_fwht_gemv: null norm pointer");
  R4Q_REQUIRE((reinterpret_cast<uintptr_t>(gamma) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(b) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(res_out) & 15) == 0,
              "res_rmsnorm_fwht_gemv: pointers must be 16-byte aligned");
  return r4q::gemv_norm_launch(a, b, gamma, res_out, eps, w, sz, y, N, K, wbits,
                               r4q::as_stream(stream));
}

extern "C" int r4q_gate_up_silu_fwht(const void* a, const void* b, const void* gamma,
                                     void* res_out, float eps, const void* w, const void* sz,
                                     void* y, int64_t I, int64_t K, int wbits, void* stream) {
  R4Q_REQUIRE(I > 0 && I % 32 == 0, "gate_up_silu_fwht: I must be a positive multiple of 32");
  R4Q_TRY(r4q::gemv_check(a, w, sz, y, 2 * I, K, wbits));
  R4Q_REQUIRE(wbits != 16 && r4q::gemv_silu_ok(2 * I, K, wbits),
              "gate_up_silu_fwht: INT4 / INT8 rows of at most 320 chunks only");
  R4Q_REQUIRE(!gamma || !b || res_out, "gate_up_silu_fwht: residual output required");
  R4Q_REQUIRE((reinterpret_cast<uintptr_t>(gamma) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(b) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(res_out) & 15) == 0,
              "gate_up_silu_fwht: pointers must be 16-byte aligned");
  return r4q::gemv_norm_launch(a, gamma ? b : nullptr, gamma, gamma ? res_out : nullptr, eps, w,
                               sz, y, 2 * I, K, wbits, r4q::as_stream(stream),
                               r4q::SiluEpi::kUnit);
}

extern "C" int r4q_gate_up_silu_split(int64_t I, int64_t* split) {
  R4Q_REQUIRE(split && I > 0 && I % 32 == 0, "gate_up_silu_split: need I %% 32 == 0 and a result");
  *split = r4q::gemv_silu_split(I);
  return R4Q_OK;
}

extern "C" int r4q_gate_up_silu(const void* a, const void* b, const void* gamma, void* res_out,
                                float eps, const void* w, const void* sz, void* y, float* h,
                                int64_t split, int64_t I, int64_t K, int wbits, void* stream) {
  R4Q_REQUIRE(I > 0 && I % 32 == 0, "gate_up_silu: I must be a positive multiple of 32");
  R4Q_REQUIRE(split >= 0 && split <= I && split % 32 == 0,
              "gate_up_silu: split must be a multiple of 32 in [0, I] (got %lld)", (long long)split);
  R4Q_REQUIRE((split == 0 || y) && (split == I || h), "gate_up_silu: null output");
  R4Q_TRY(r4q::gemv_check(a, w, sz, split > 0 ? y : static_cast<void*>(h), 2 * I, K, wbits));
  R4Q_REQUIRE(wbits != 16 && r4q::gemv_silu_ok(2 * I, K, wbits),
              "gate_up_silu: INT4 / INT8 rows of at most 320 chunks only");
  R4Q_REQUIRE(!gamma || !b || res_out, "gate_up_silu: residual output required");
  R4Q_REQUIRE((reinterpret_cast<uintptr_t>(gamma) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(b) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(res_out) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(h) & 3) == 0 &&
                  (reinterpret_cast<uintptr_t>(y) & 1) == 0,
              "gate_up_silu: pointers must be aligned (16 bytes; h: 4; y: 2)");
  return r4q::gemv_norm_launch(a, gamma ? b : nullptr, gamma, gamma ? res_out : nullptr, eps, w,
                               sz, y, 2 * I, K, wbits, r4q::as_stream(stream),
                               r4q::SiluEpi::kSplit, h, split);
}

extern "C" int r4q_fwht_gemv(const void* x, const float* h, int64_t split, const void* w,
                             const void* sz, void* y, int64_t N, int64_t K, int wbits,
                             void* stream) {
  R4Q_REQUIRE(split >= 0 && split <= K && split % 32 == 0,
              "fwht_gemv: split must be a multiple of 32 in [0, K] (got %lld)", (long long)split);
  R4Q_REQUIRE((split == 0 || x) && (split == K || h), "fwht_gemv: null input");
  R4Q_REQUIRE((reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                  (reinterpret_cast<uintptr_t>(h) & 15) == 0,
              "fwht_gemv: x and h must be 16-byte aligned");
  R4Q_TRY(r4q::gemv_check(split > 0 ? x : static_cast<const void*>(h), w, sz, y, N, K, wbits));
  return r4q::gemv_fwht_launch(x, h, split, w, sz, y, N, K, wbits, r4q::as_stream(stream));
}
