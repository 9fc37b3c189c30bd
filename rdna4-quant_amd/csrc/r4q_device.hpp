// Device-side building blocks shared by every gfx950 kernel of librdna4q.
//
// Numerics follow the reference decode path (JohnTDI-cpu/rdna4-quant,
// hip_int4/int4_decode_step.hip, cited as hip:LINE).  Everything here is
// wave64 CDNA4 code: cross-lane traffic uses DPP and v_readlane, never LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace r4q {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr float kInvSqrt32 = 0.17677669529663689f;  // 1/sqrt(32) as fp32

__device__ __forceinline__ float h2f(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}
// fp32 -> fp16, round-to-nearest-even, from a rounded fp32 value.  The
// empty asm keeps `f` opaque: otherwise a preceding multiply is fused into
// v_fma_mix*_f16, which rounds the exact product once (skipping the fp32
// rounding the oracle models) and turns a -0 product into +0.
__device__ __forceinline__ uint16_t f2h(float f) {
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
// fp16 -> fp32 kept in a VGPR as a plain fp32 operand, so later multiplies
// are IEEE v_mul_f32 (no v_fma_mix with a +0 addend, which loses -0).
__device__ __forceinline__ float h2f_ieee(uint16_t b) {
  float f = (float)__builtin_bit_cast(_Float16, b);
  asm volatile("" : "+v"(f));
  return f;
}
__device__ __forceinline__ h2_t as_h2(uint32_t u) { return __builtin_bit_cast(h2_t, u); }
__device__ __forceinline__ uint32_t as_u32(h2_t h) { return __builtin_bit_cast(uint32_t, h); }

// ---------------------------------------------------------------- FP8 E4M3
// Encoder restating the reference recipe (hip:47-68) in integer steps:
//  * clamp to [-448, 448] with NaN mapping to +448 (fminf/fmaxf ignore NaN),
//  * fp32 exponent e == 0 (zero / fp32 denormal) -> signed zero,
//  * E = e - 120; keep the top 3 mantissa bits and add one when fp32
//    mantissa bit 19 is set (ties round away from zero), carrying into E,
//  * E <= 0 -> signed zero (no E4M3 subnormals are ever produced),
//  * E >= 15 -> sign | 0x7E (448): the whole 256..448 binade saturates.
__device__ __forceinline__ uint32_t fp8_encode(float v) {
  v = fmaxf(-448.0f, fminf(448.0f, v));
  const uint32_t f = __float_as_uint(v);
  const uint32_t sign = (f >> 24) & 0x80u;
  const int e = (int)((f >> 23) & 0xFFu);
  const uint32_t man = f & 0x7FFFFFu;
  int E = e - 120;
  int M = (int)(man >> 20) + (int)((man >> 19) & 1u);
  E += M >> 3;  // mantissa carry (M == 8)
  M &= 7;
  uint32_t code = sign | ((uint32_t)E << 3) | (uint32_t)M;
  code = (E >= 15) ? (sign | 0x7Eu) : code;
  code = (e == 0 || E <= 0) ? sign : code;
  return code;
}

// Two E4M3 codes (bytes 0 and 1 of `c`) -> packed fp16 pair scaled by 2^-8:
// the E4M3 fields are placed into the fp16 exponent/mantissa fields (bias 15
// instead of 7), which is exact for every code, subnormals included.
// Multiply by 256 (or fold 256 into a scale) to get the E4M3 value.
__device__ __forceinline__ uint32_t fp8x2_to_h2_div256(uint32_t c) {
  // spread byte0 -> bits 0..7, byte1 -> bits 16..23
  const uint32_t s = __builtin_amdgcn_perm(0u, c, 0x0c010c00u);
  return ((s << 8) & 0x80008000u) | ((s << 7) & 0x3F803F80u);
}

// ---------------------------------------------------------------- FWHT-32
// In-register Walsh-Hadamard transform of 32 values, Sylvester order,
// butterfly stages step = 1, 2, 4, 8, 16 ({a+b, a-b}), then * 1/sqrt(32)
// (same stage order and scaling as the reference, hip:87-102).
__device__ __forceinline__ void fwht32(float* v) {
#pragma unroll
  for (int step = 1; step < 32; step <<= 1) {
#pragma unroll
    for (int i = 0; i < 32; i += 2 * step) {
#pragma unroll
      for (int j = i; j < i + step; ++j) {
        const float a = v[j], b = v[j + step];
        v[j] = a + b;
        v[j + step] = a - b;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 32; ++i) v[i] *= kInvSqrt32;
}

// ------------------------------------------------------- wave reductions
// DPP controls (GFX9 encoding).
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

// Wait states between a v_dot2* result and a DPP read of it.  The compiler
// pads VALU->DPP reads with 2 wait states, which is not enough after a dot
// instruction on gfx950 (the DPP then sees the pre-dot value); call this
// after dot-product accumulation and before any DPP reduction of the result.
__device__ __forceinline__ void dot_dpp_fence() { asm volatile("s_nop 4" ::: "memory"); }

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of G lanes (G in 1,2,4,8,16); afterwards every lane
// of a group holds the group sum.  Pairing is xor-1, xor-2, then mirror
// within 8 and within 16 (equivalent to xor-4 / xor-8 once the smaller groups
// are uniform), so the fp32 addition tree is fixed.
template <int G>
__device__ __forceinline__ float group_sum16(float v) {
  if constexpr (G >= 2) v += dpp<kDppQuadXor1>(v);
  if constexpr (G >= 4) v += dpp<kDppQuadXor2>(v);
  if constexpr (G >= 8) v += dpp<kDppHalfMirror>(v);
  if constexpr (G >= 16) v += dpp<kDppRowMirror>(v);
  return v;
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Canonical wave64 sum: 16-lane row sums by group_sum16<16>, then
// (row0 + row1) + (row2 + row3).  Result is wave-uniform.
__device__ __forceinline__ float wave_sum(float v) {
  v = group_sum16<16>(v);
  return (readlane_f(v, 0) + readlane_f(v, 16)) +
         (readlane_f(v, 32) + readlane_f(v, 48));
}

// Max over the wave (order irrelevant for max).
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<kDppQuadXor1>(v));
  v = fmaxf(v, dpp<kDppQuadXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppRowMirror>(v));
  return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)),
               fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Per-head RMSNorm factor, one wave per head of 128 where lane l owns
// elements l and l + 64: 1 / sqrt(sum x^2 / 128 + eps) with the canonical
// wave reduction.
__device__ __forceinline__ float head_rrms(float x0, float x1, float eps) {
#pragma clang fp contract(off)
  const float t = x0 * x0 + x1 * x1;
  const float ss = wave_sum(t);
  return 1.0f / __builtin_sqrtf(ss / 128.0f + eps);
}

// Head RMSNorm + half-split RoPE of elements (l, l + 64), no fused
// multiply-add: ne = (x0*rr)*w0, no = (x1*rr)*w1, lo = ne*c - no*s,
// hi = no*c + ne*s.
__device__ __forceinline__ void head_norm_rope_pair(float x0, float x1, float w0, float w1,
                                                    float c, float s, float eps, float& lo,
                                                    float& hi) {
#pragma clang fp contract(off)
  const float rr = head_rrms(x0, x1, eps);
  const float ne = (x0 * rr) * w0;
  const float no = (x1 * rr) * w1;
  lo = ne * c - no * s;
  hi = no * c + ne * s;
}

// 32 consecutive fp16 values <-> fp32 registers (128-bit accesses).
__device__ __forceinline__ void load32h(const uint16_t* __restrict__ p, float* v) {
  const u4_t* s = reinterpret_cast<const u4_t*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u4_t d = s[i];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[8 * i + 2 * k] = h2f((uint16_t)(d[k] & 0xFFFFu));
      v[8 * i + 2 * k + 1] = h2f((uint16_t)(d[k] >> 16));
    }
  }
}

__device__ __forceinline__ void store32h(uint16_t* __restrict__ p, const float* v) {
  u4_t* d = reinterpret_cast<u4_t*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    u4_t o;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      o[k] = (uint32_t)f2h(v[8 * i + 2 * k]) | ((uint32_t)f2h(v[8 * i + 2 * k + 1]) << 16);
    d[i] = o;
  }
}

// Workgroup-wide sum in a fixed order (wave sums, then waves 0, 1, ... in
// sequence); every thread gets the result.  `red` holds one float per wave.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  const int nw = (blockDim.x + 63) >> 6;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < nw; ++i) t += red[i];
  __syncthreads();
  return t;
}

}  // namespace r4q
