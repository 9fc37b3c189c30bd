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

// ------------------------------------------ row-norm chunk arithmetic
// One 32-element chunk of a (residual) RMSNorm [+ FWHT] row kept as 16
// packed fp16 pairs, with the rounding sequence of
//   v = fp32(a) + fp32(b);  ss += v * v;  r = fp16(v);
//   y = fp16([FWHT32](fp32(r) * rrms * fp32(gamma)))
// in fewer instructions: v_fma_mix_f32 reads fp16 halves directly (a * 1 + b
// and r * rrms + (-0) round exactly once, like the fp32 add / multiply, and
// the -0 addend keeps the sign of a zero product); r comes from
// v_pk_add_f16, which equals fp16(fp32(a + b)) because rounding an fp16 sum
// to fp32 first is innocuous (24 >= 2 * 11 + 2 bits); v_cvt_pk_f16_f32
// rounds two values to nearest-even.  Both the row-norm kernel and the
// fused-norm GEMV staging use these, so their activations stay bit-identical.
template <bool HI>
__device__ __forceinline__ float mix_add(uint32_t a, uint32_t b) {  // fp32(a.h) + fp32(b.h)
  float r;
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,1] op_sel_hi:[1,0,1]"
        : "=v"(r) : "v"(a), "v"(b));
  else
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,1]" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
template <bool HI>
__device__ __forceinline__ float mix_sq_acc(uint32_t a, float acc) {  // fp32(a.h)^2 + acc
  float r;
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, %1, %2 op_sel:[1,1,0] op_sel_hi:[1,1,0]"
        : "=v"(r) : "v"(a), "v"(acc));
  else
    asm("v_fma_mix_f32 %0, %1, %1, %2 op_sel_hi:[1,1,0]" : "=v"(r) : "v"(a), "v"(acc));
  return r;
}
template <bool HI>
__device__ __forceinline__ float mix_mul_hf(uint32_t h, float s, float mz) {  // fp32(h.h) * s
  float r;
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
        : "=v"(r) : "v"(h), "v"(s), "v"(mz));
  else
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(s), "v"(mz));
  return r;
}
template <bool HI>
__device__ __forceinline__ float mix_mul_fh(float s, uint32_t h, float mz) {  // s * fp32(h.h)
  float r;
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
        : "=v"(r) : "v"(s), "v"(h), "v"(mz));
  else
    asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel_hi:[0,1,0]" : "=v"(r) : "v"(s), "v"(h), "v"(mz));
  return r;
}
__device__ __forceinline__ uint32_t pk_add_h(uint32_t a, uint32_t b) {  // fp16 a + b, per half
  uint32_t r;
  asm("v_pk_add_f16 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ uint32_t cvt_pk_h(float lo, float hi) {  // (fp16(lo), fp16(hi))
  uint32_t r;
  asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(r) : "v"(lo), "v"(hi));
  return r;
}

__device__ __forceinline__ void load16w(const uint16_t* __restrict__ p, uint32_t* w) {
  const u4_t* s = reinterpret_cast<const u4_t*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const u4_t d = s[i];
    w[4 * i] = d[0];
    w[4 * i + 1] = d[1];
    w[4 * i + 2] = d[2];
    w[4 * i + 3] = d[3];
  }
}
__device__ __forceinline__ void store16w(uint16_t* __restrict__ p, const uint32_t* w) {
  u4_t* d = reinterpret_cast<u4_t*>(p);
#pragma unroll
  for (int i = 0; i < 4; ++i) d[i] = u4_t{w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
}

// Phase 1: r = fp16(a + b) (RES) or a, and the sum over the chunk, in
// element order, of squares of fp32(a + b) (or fp32(a)), added to ss.
template <bool RES>
__device__ __forceinline__ float norm_chunk_sumsq(const uint32_t* a, const uint32_t* b,
                                                  uint32_t* r, float ss) {
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    if constexpr (RES) {
      const float lo = mix_add<false>(a[k], b[k]), hi = mix_add<true>(a[k], b[k]);
      ss = __builtin_fmaf(lo, lo, ss);
      ss = __builtin_fmaf(hi, hi, ss);
      r[k] = pk_add_h(a[k], b[k]);
    } else {
      ss = mix_sq_acc<false>(a[k], ss);
      ss = mix_sq_acc<true>(a[k], ss);
      r[k] = a[k];
    }
  }
  return ss;
}

// Phase 2: y = fp16 pairs of [FWHT32](fp32(r) * rrms * fp32(g)).
template <bool FWHT>
__device__ __forceinline__ void norm_chunk_scale(const uint32_t* r, const uint32_t* g, float rrms,
                                                 uint32_t* y) {
  float mz = -0.0f;
  asm volatile("" : "+v"(mz));
  float v[32];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    v[2 * k] = mix_mul_fh<false>(mix_mul_hf<false>(r[k], rrms, mz), g[k], mz);
    v[2 * k + 1] = mix_mul_fh<true>(mix_mul_hf<true>(r[k], rrms, mz), g[k], mz);
  }
  if constexpr (FWHT) fwht32(v);
#pragma unroll
  for (int k = 0; k < 16; ++k) y[k] = cvt_pk_h(v[2 * k], v[2 * k + 1]);
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
