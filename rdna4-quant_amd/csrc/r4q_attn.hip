// Split-K flash-decode over the FP8 E4M3 KV cache (GQA), with the log-sum-exp
// merge and the optional FWHT-32 output rotation.
//
// Replaces the reference's launch_flash_decode (hip:1547-1593) with its
// flash_decode_partial (hip:1326-1412), flash_decode_reduce (hip:1416-1463)
// and flash_decode_fused (hip:1471-1542); softmax semantics follow SDPA
// (int4_engine_v5.py:245).  Unlike the reference, Q stays fp16 (the
// reference's FP8 quantisation of Q costs ~2.7e-2 rel-L2 and its
// dot4_f32_fp8_fp8 instruction does not exist on gfx950), and K/V carry an
// optional per-head fp32 scale.
//
// attn_mfma_kernel computes one (split, KV head, sequence) per workgroup on
// the matrix cores; attn_merge_kernel combines the splits per query head:
// m* = max_s m_s, out = sum_s e^(m_s-m*) o_s / sum_s e^(m_s-m*) l_s, with the
// FWHT-32 already applied to each o_s (it is linear).  A single split writes
// the fp16 output directly.
#include <math.h>
#include <stdlib.h>

#include <atomic>
#include <mutex>

#include "r4q_ctx.hpp"
#include "r4q_device.hpp"
#include "r4q_host.hpp"

namespace r4q {
namespace {

constexpr int kMaxSplits = 128;  // partials per (sequence, head)
constexpr int kPart = 132;       // floats per (seq, head, split): m, l, pad, pad, o[128]
constexpr int kXcds = 8;         // workgroup i is dispatched to XCD i % 8

// ------------------------------------------------ MFMA flash-decode partials
// E4M3 bytes 0-1 (HI: 2-3) of w -> fp16 pair, v_cvt_scalef32_pk_f16_fp8 with
// scale 1: exact and equal to the reference decoder (hip:71-81) for every
// code the reference encoder emits (it flushes E <= 0 to +-0 and saturates
// at 0x7E, so the E4M3 subnormal and 0x7F codes, which decode differently,
// never occur in a cache).
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_h2(uint32_t w) {
  return as_u32(__builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, HI));
}

// 4x4 byte transpose: out[d] = byte d of in[0], in[1], in[2], in[3].
__device__ __forceinline__ void transpose4x4(const uint32_t* in, uint32_t* out) {
  const uint32_t a0 = __builtin_amdgcn_perm(in[1], in[0], 0x05010400u);  // in0.b0 in1.b0 in0.b1 in1.b1
  const uint32_t a1 = __builtin_amdgcn_perm(in[1], in[0], 0x07030602u);  // in0.b2 in1.b2 in0.b3 in1.b3
  const uint32_t b0 = __builtin_amdgcn_perm(in[3], in[2], 0x05010400u);
  const uint32_t b1 = __builtin_amdgcn_perm(in[3], in[2], 0x07030602u);
  out[0] = __builtin_amdgcn_perm(b0, a0, 0x05040100u);
  out[1] = __builtin_amdgcn_perm(b0, a0, 0x07060302u);
  out[2] = __builtin_amdgcn_perm(b1, a1, 0x05040100u);
  out[3] = __builtin_amdgcn_perm(b1, a1, 0x07060302u);
}

__device__ __forceinline__ f4_t mfma16(u4_t a, u4_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8_t, a),
                                                __builtin_bit_cast(h8_t, b), c, 0, 0, 0);
}

// Flash-decode partials on the matrix cores (v_mfma_f32_16x16x32_f16), one
// workgroup per (split, KV head, sequence).  The sequence is cut into
// 32-position chunks dealt round-robin to the splits; each of the 4 waves
// walks its split's chunks wave, wave + 4, ... with its own online-softmax
// state, and the waves merge once at the end through LDS.
// Lane l has column n = l % 16 and group g = l / 16.  Per chunk:
//  * S^T = K Q^T for two 16-position blocks: A = K (lane: position n of the
//    block, dims 32g .. 32g+31 over the 4 k-steps), B = Q^T (lane: head n,
//    the same dims; heads >= G are zero).  C: lane holds head n at positions
//    4g .. 4g+3 of the block;
//  * online softmax per head across the 4 lanes holding it (the running
//    output is rescaled only when a head's maximum rises), probabilities
//    rounded to fp16 as in the reference kernel;
//  * O += P V: A = P (lane: head n; k-slots = its 8 positions 4g+r and
//    16+4g+r), B = V (lane: dim 8n + j for N-block j, the same positions):
//    each lane loads 8 bytes (dims 8n .. 8n+7) of its 8 position rows and
//    transposes them to per-dim bytes with v_perm.  C: lane holds dim 8n + j
//    for heads 4g .. 4g+3.
// K rows load as 32 contiguous bytes per lane and V rows as 8 (16 lanes
// cover a 128-byte row); the next chunk's K (V) loads are issued as soon as
// this chunk's K (V) registers are converted.
// Prologue (NORMQ): per-head RMSNorm + RoPE of q and k, FP8 write of the new
// K/V at position L-1 by the workgroup holding that position, which patches
// the codes into its own (earlier issued) loads.  Epilogue: FWHT-32 per
// 32-dim chunk, then the fp32 partial (m, l, o) or, with one split, the
// normalised fp16 output.
// QS (NORMQ only): 0 = raw fp16 QKV rows, 2..kMaxQkvSplits = that many fp32
// split planes of the qkv projection to sum (exactly QS loads per element).
template <int G, bool NORMQ, int QS = 0>
__global__ __launch_bounds__(256) void attn_mfma_kernel(
    const uint16_t* __restrict__ q, int64_t q_stride, const uint8_t* __restrict__ kc,
    const uint8_t* __restrict__ vc, const float* __restrict__ ksc, const float* __restrict__ vsc,
    float* __restrict__ part, uint16_t* __restrict__ outp, int64_t out_stride, int fwht, int H,
    int Hk, int max_seq, int L_host, const int* __restrict__ L_dev, int nsplit, AttnQK qk) {
  static_assert(G >= 1 && G <= 16, "query heads per KV head must fit 16 MFMA columns");
  // XCD-grouped order when the (sequence, KV head) pairs fill whole rounds
  // of the 8 XCDs: the grid is (8 nsplit, pairs / 8), workgroups go to the
  // XCDs round-robin in x-fastest order, so every split of pair p sits on
  // XCD p % 8, where the pair's merge workgroups run too (measured 9 us
  // faster per 40-layer step than splits spread over the XCDs); otherwise
  // the grid is (nsplit, pairs)
  const bool grouped = (int)gridDim.x != nsplit;
  const int sp = grouped ? (int)blockIdx.x / kXcds : (int)blockIdx.x;
  const int pair = grouped ? (int)blockIdx.y * kXcds + (int)blockIdx.x % kXcds : (int)blockIdx.y;
  const int kh = pair % Hk;
  const int64_t b = pair / Hk;
  const int L = L_dev ? *L_dev : L_host;
  // 32-position chunks are dealt to the splits round-robin (split sp takes
  // chunks sp, sp + nsplit, ...), so that at any moment the workgroups of a
  // head read one contiguous window of the cache (a plain stream for HBM)
  // instead of nsplit separate ranges; the softmax merge does not depend on
  // which positions a split holds.
  const int nct = (L + 31) / 32;
  const int nchunk = sp < nct ? (nct - 1 - sp) / nsplit + 1 : 0;  // this split's chunks
  auto cpos = [&](int c) { return 32 * (sp + nsplit * c); };  // first position of local chunk c

  __shared__ __align__(16) uint16_t qs[NORMQ ? G : 1][128];
  __shared__ __align__(16) uint8_t knew[128], vnew[128];
  __shared__ float wst[4][G][2];  // per wave: max, sum
  // per wave: unnormalised O by (component r, dims 8 col + 0..3 / 4..7,
  // lane) of the MFMA output layout (see the epilogue); only the lane groups
  // holding heads < G
  constexpr int kOGroups = (G + 3) / 4;
  __shared__ __align__(16) f4_t wo[4][4][2][16 * kOGroups];

  // wave index as a scalar: the chunk loops and the per-chunk guards are
  // then scalar branches (an MFMA computes its whole tile whatever EXEC holds)
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int col = lane & 15, g = lane >> 4;
  const float ks = ksc ? ksc[kh] : 1.0f;
  const float vs = vsc ? vsc[kh] : 1.0f;
  const int64_t head_off = (b * Hk + kh) * (int64_t)max_seq * 128;
  const uint8_t* kbase = kc + head_off;
  const uint8_t* vbase = vc + head_off;

  // local chunk c: K rows cpos(c) + 16bb + col (32 bytes from dim 32g), V
  // rows cpos(c) + vpos(s) (8 bytes from dim 8col); rows past the sequence
  // end are clamped to its last row and masked.
  auto vpos = [&](int s) { return s < 4 ? 4 * g + s : 16 + 4 * g + (s - 4); };
  // One register set per wave: the next chunk's K (V) loads are issued as
  // soon as this chunk's K (V) registers are converted.  They are issued
  // unconditionally (past the wave's last chunk they read the clamped last
  // row again): loads issued on only some paths make the compiler wait for
  // every load in flight before the next use of the set, which would stall
  // each chunk on its successor's loads.  Byte offsets are 32-bit from the
  // workgroup's uniform row base.
  u4_t kr0[2][2];
  u2_t vr0[8];
  auto load_k = [&](u4_t (&kr)[2][2], int c) {
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      const uint32_t p = (uint32_t)min(cpos(c) + 16 * bb + col, L - 1);
      const u4_t* src = reinterpret_cast<const u4_t*>(kbase + (p * 128u + 32u * g));
      kr[bb][0] = __builtin_nontemporal_load(src);
      kr[bb][1] = __builtin_nontemporal_load(src + 1);
    }
  };
  auto load_v = [&](u2_t (&vr)[8], int c) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const uint32_t p = (uint32_t)min(cpos(c) + vpos(s), L - 1);
      vr[s] = __builtin_nontemporal_load(
          reinterpret_cast<const u2_t*>(vbase + (p * 128u + 8u * col)));
    }
  };
  // ---- query: B operands qb[j] = Q[head col][32g + 8j .. +7] (0 for col >= G)
  // NORMQ: tasks 0 .. G-1 are the query heads, G the new K row and G+1 the
  // new V row (the last two only in the workgroup holding position L-1);
  // wave w takes tasks w, w+4, ...  Every prologue input is loaded before
  // the wave's first KV chunk, so that the norm and RoPE run while the chunk
  // is in flight (loads return in issue order).
  constexpr int kSlots = (G + 2 + 3) / 4;
  const int pos = L - 1;
  const bool owner = NORMQ && (pos >> 5) % nsplit == sp;  // holds the new position's chunk
  const int ntask = G + (owner ? 2 : 0);
  uint16_t px[kSlots][2], pw[kSlots][2];  // raw fp16, widened after the KV loads issue
  static_assert(QS == 0 || (NORMQ && QS >= 2 && QS <= kMaxQkvSplits), "split planes to sum");
  float pf[NORMQ && QS >= 2 ? kSlots : 1][2][QS >= 2 ? QS : 1];  // split partials
  uint16_t pc = 0, ps = 0;
  if constexpr (NORMQ) {
    // branch-free, so that all of them are in flight together (slots past
    // the wave's tasks read head 0 and are not used)
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int task = wave + 4 * i;
      const int head = task >= ntask ? 0 : task < G ? kh * G + task : task == G ? H + kh : H + Hk + kh;
      const int64_t off = b * q_stride + (int64_t)head * 128;  // raw QKV row: q | k | v heads
      if constexpr (QS >= 2) {
#pragma unroll
        for (int z = 0; z < QS; ++z) {
          const float* src = qk.part + z * qk.plane + off;
          pf[i][0][z] = src[lane];
          pf[i][1][z] = src[lane + 64];
        }
      } else {
        px[i][0] = q[off + lane];
        px[i][1] = q[off + lane + 64];
      }
      const uint16_t* w = task < G ? qk.qw : qk.kw;
      pw[i][0] = w[lane];
      pw[i][1] = w[lane + 64];
    }
    pc = qk.cs[(int64_t)pos * 64 + lane];
    ps = qk.sn[(int64_t)pos * 64 + lane];
  }
  u4_t qb[4];
  if constexpr (!NORMQ) {  // q rows ahead of the KV loads (head 0 stands in for col >= G)
    const uint16_t* qh = q + b * q_stride + (int64_t)(kh * G + min(col, G - 1)) * 128 + 32 * g;
#pragma unroll
    for (int j = 0; j < 4; ++j) qb[j] = *reinterpret_cast<const u4_t*>(qh + 8 * j);
  }
  // first chunk in flight during the query prologue; unconditional (a wave
  // without chunks reads the clamped last row) so that the prologue waits
  // only for its own, earlier loads
  load_k(kr0, wave);
  load_v(vr0, wave);

  if constexpr (NORMQ) {
    // widened in straight-line code: every slot's loads are consumed here,
    // before any branch (none is sunk behind the KV loads)
    const float c = h2f_ieee(pc), sn = h2f_ieee(ps);
    if constexpr (QS >= 2) {  // the split reduce's sum, in split order, rounded to fp16
#pragma unroll
      for (int i = 0; i < kSlots; ++i)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          float v = pf[i][e][0];
#pragma unroll
          for (int z = 1; z < QS; ++z) v += pf[i][e][z];
          px[i][e] = f2h(v);
        }
    }
    float fx[kSlots][2], fw[kSlots][2];
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      fx[i][0] = h2f_ieee(px[i][0]);
      fx[i][1] = h2f_ieee(px[i][1]);
      fw[i][0] = h2f_ieee(pw[i][0]);
      fw[i][1] = h2f_ieee(pw[i][1]);
    }
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int task = wave + 4 * i;
      if (task >= ntask) break;  // wave-uniform
      const float x0 = fx[i][0], x1 = fx[i][1];
      if (task < G) {
        float lo, hi;
        head_norm_rope_pair(x0, x1, fw[i][0], fw[i][1], c, sn, qk.eps, lo, hi);
        qs[task][lane] = f2h(lo);
        qs[task][lane + 64] = f2h(hi);
      } else if (task == G) {
        float lo, hi;
        head_norm_rope_pair(x0, x1, fw[i][0], fw[i][1], c, sn, qk.eps, lo, hi);
        const float inv = ksc ? 1.0f / ksc[kh] : 1.0f;
        const uint8_t c0 = (uint8_t)fp8_encode(lo * inv), c1 = (uint8_t)fp8_encode(hi * inv);
        uint8_t* kp = qk.kc + ((b * Hk + kh) * (int64_t)max_seq + pos) * 128;
        kp[lane] = c0;
        kp[lane + 64] = c1;
        knew[lane] = c0;
        knew[lane + 64] = c1;
      } else {
        const float inv = vsc ? 1.0f / vsc[kh] : 1.0f;
        const uint8_t c0 = (uint8_t)fp8_encode(x0 * inv);
        const uint8_t c1 = (uint8_t)fp8_encode(x1 * inv);
        uint8_t* vp = qk.vc + ((b * Hk + kh) * (int64_t)max_seq + pos) * 128;
        vp[lane] = c0;
        vp[lane + 64] = c1;
        vnew[lane] = c0;
        vnew[lane + 64] = c1;
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j)
      qb[j] = col < G ? *reinterpret_cast<const u4_t*>(&qs[col][32 * g + 8 * j]) : u4_t{0, 0, 0, 0};
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (col >= G) qb[j] = u4_t{0, 0, 0, 0};
  }
  // position whose K/V sit in knew/vnew (written by the owner workgroup only)
  const int pos_new = NORMQ ? L - 1 : -1;

  const float sscale = ks * 0.08838834764831845f;  // k_scale / sqrt(128)
  const uint32_t ones = 0x3C003C00u;               // fp16 (1, 1)
  float m_run = -INFINITY, l_run = 0.f;            // head col; l over this lane's positions
  f4_t o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = f4_t{0.f, 0.f, 0.f, 0.f};

  // one chunk c from the register set (kr, vr), which then receives chunk
  // cn.  A chunk past the split's last one (c >= nchunk) starts at or after
  // position L, so every score is masked to -inf: it adds nothing (p = 0,
  // alpha = 1 once a real chunk has set the running max)
  auto step = [&](u4_t (&kr)[2][2], u2_t (&vr)[8], int c, int cn) {
    // ---- K -> fp16 A operands, S^T = K Q^T, then the set's next K in flight
    f4_t sacc[2];
#pragma unroll
    for (int bb = 0; bb < 2; ++bb) {
      u4_t ka[4];
      u4_t r0 = kr[bb][0], r1 = kr[bb][1];
      if constexpr (NORMQ) {
        if (owner && min(cpos(c) + 16 * bb + col, L - 1) == pos_new) {
          r0 = *reinterpret_cast<const u4_t*>(&knew[32 * g]);
          r1 = *reinterpret_cast<const u4_t*>(&knew[32 * g + 16]);
        }
      }
      const uint32_t w[8] = {r0[0], r0[1], r0[2], r0[3], r1[0], r1[1], r1[2], r1[3]};
#pragma unroll
      for (int j = 0; j < 4; ++j)
        ka[j] = u4_t{fp8x2_h2<false>(w[2 * j]), fp8x2_h2<true>(w[2 * j]),
                     fp8x2_h2<false>(w[2 * j + 1]), fp8x2_h2<true>(w[2 * j + 1])};
      sacc[bb] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j) sacc[bb] = mfma16(ka[j], qb[j], sacc[bb]);
    }
    load_k(kr, cn);

    // ---- online softmax for head col over positions 32c + vpos(s)
    float sv[8];
    if (cpos(c) + 32 <= L) {  // wave-uniform: a full chunk
#pragma unroll
      for (int s = 0; s < 8; ++s) sv[s] = sacc[s >> 2][s & 3] * sscale;
    } else {
#pragma unroll
      for (int s = 0; s < 8; ++s)
        sv[s] = (cpos(c) + vpos(s) < L) ? sacc[s >> 2][s & 3] * sscale : -INFINITY;
    }
    float mx = sv[0];
#pragma unroll
    for (int s = 1; s < 8; ++s) mx = fmaxf(mx, sv[s]);
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float mn = fmaxf(m_run, mx);
    const float alpha = (m_run == -INFINITY) ? 0.f : __expf(m_run - mn);
    // O needs rescaling only where a head's running max rose (O is zero
    // before the first finite max); exp(0) == 1 exactly elsewhere
    const bool rescale =
        __builtin_amdgcn_ballot_w64(m_run != -INFINITY && mn != m_run) != 0;  // wave-uniform
    u4_t pa;  // fp16 probabilities, k-slot s = position vpos(s)
    float lp = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p0 = (mn == -INFINITY) ? 0.f : __expf(sv[2 * i] - mn);
      const float p1 = (mn == -INFINITY) ? 0.f : __expf(sv[2 * i + 1] - mn);
      pa[i] = cvt_pk_h(p0, p1);
      lp = __builtin_amdgcn_fdot2(as_h2(pa[i]), as_h2(ones), lp, false);
    }
    l_run = __builtin_fmaf(l_run, alpha, lp);
    m_run = mn;

    // ---- V -> per-dim fp16 B operands, next chunk's V in flight, O += P V
    uint32_t vlo[8], vhi[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      vlo[s] = vr[s][0];
      vhi[s] = vr[s][1];
      if constexpr (NORMQ) {
        if (owner && min(cpos(c) + vpos(s), L - 1) == pos_new) {
          vlo[s] = reinterpret_cast<const uint32_t*>(vnew)[2 * col];
          vhi[s] = reinterpret_cast<const uint32_t*>(vnew)[2 * col + 1];
        }
      }
    }
    uint32_t tr[8][2];  // tr[d][h]: dim 8col + d, bytes of k-slots 4h .. 4h+3
    {
      uint32_t x[4];
      transpose4x4(vlo, x);
      for (int d = 0; d < 4; ++d) tr[d][0] = x[d];
      transpose4x4(vlo + 4, x);
      for (int d = 0; d < 4; ++d) tr[d][1] = x[d];
      transpose4x4(vhi, x);
      for (int d = 0; d < 4; ++d) tr[4 + d][0] = x[d];
      transpose4x4(vhi + 4, x);
      for (int d = 0; d < 4; ++d) tr[4 + d][1] = x[d];
    }
    // the transposes above are the set's last reads: the empty asm (inputs:
    // every transposed word; memory clobber) keeps them before the next
    // chunk's loads, so that the loads refill the same registers (a load
    // hoisted above them needs other registers and a copy back at the loop
    // end, which waits for it)
#pragma unroll
    for (int d = 0; d < 8; ++d) asm volatile("" : "+v"(tr[d][0]), "+v"(tr[d][1])::"memory");
    load_v(vr, cn);
    if (rescale) {
      float ar[4];  // alpha of the C rows' heads 4g + r (lane 4g + r holds that head)
#pragma unroll
      for (int r = 0; r < 4; ++r) ar[r] = __shfl(alpha, 4 * g + r);
#pragma unroll
      for (int d = 0; d < 8; ++d)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[d][r] *= ar[r];
    }
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      const u4_t vb = u4_t{fp8x2_h2<false>(tr[d][0]), fp8x2_h2<true>(tr[d][0]),
                           fp8x2_h2<false>(tr[d][1]), fp8x2_h2<true>(tr[d][1])};
      o[d] = mfma16(pa, vb, o[d]);
    }
  };
  // The first chunk is peeled: every path into the loop then comes from a
  // step, which issues the next K before the next V, so the loop's first K
  // wait leaves the V loads in flight (the prologue's order may differ).
  // (A second register set, chunk c + 8 in flight while c and c + 4 are
  // computed, measured no faster at 32K positions and slower at 8K.)
  if (wave < nchunk) {
    step(kr0, vr0, wave, wave + 4);
    for (int c = wave + 4; c < nchunk; c += 4) step(kr0, vr0, c, c + 4);
  }

  // ---- merge the 4 waves.  Lane (col, g) holds O[head 4g + r][dim 8 col + j]
  // in o[j][r]; every wave leaves its O and its (max, sum) per head in LDS,
  // then wave w finishes component r = w, i.e. head 4g + w of each lane
  // group: the waves' O combined in wave order (e^(m_w - M) weights, as one
  // fma chain from 0), scaled, FWHT-32 across the lane's 8 dims (index bits
  // 0-2) and the 4 lanes of its quad (bits 3-4: dims 32q .. 32q+31 sit in
  // cols 4q .. 4q+3), i.e. the butterflies of fwht32 on the same values, in
  // the same order.
  float lsum = l_run + __shfl_xor(l_run, 16);
  lsum += __shfl_xor(lsum, 32);
  if (g == 0 && col < G) {
    wst[wave][col][0] = m_run;
    wst[wave][col][1] = lsum;
  }
  if (g < kOGroups) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      wo[wave][r][0][lane] = f4_t{o[0][r], o[1][r], o[2][r], o[3][r]};
      wo[wave][r][1][lane] = f4_t{o[4][r], o[5][r], o[6][r], o[7][r]};
    }
  }
  __syncthreads();
  const int h = 4 * g + wave;
  if (h >= G) return;  // no global stores follow for this lane
  float mw[4], lw[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    mw[w] = wst[w][h][0];
    lw[w] = wst[w][h][1];
  }
  float M = mw[0];
#pragma unroll
  for (int w = 1; w < 4; ++w) M = fmaxf(M, mw[w]);
  float ew[4], l = 0.f;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    ew[w] = (mw[w] == -INFINITY) ? 0.f : __expf(mw[w] - M);
    l = __builtin_fmaf(ew[w], lw[w], l);
  }
  const float oscale = vs;
  f4_t ow[4][2];  // component r = wave of every wave's O
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    ow[w][0] = wo[w][wave][0][lane];
    ow[w][1] = wo[w][wave][1][lane];
  }
  float v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float acc = 0.f;
#pragma unroll
    for (int w = 0; w < 4; ++w) acc = __builtin_fmaf(ew[w], ow[w][j >> 2][j & 3], acc);
    v[j] = acc * oscale;
  }
  if (fwht) {
#pragma unroll
    for (int step = 1; step < 8; step <<= 1) {
#pragma unroll
      for (int i = 0; i < 8; i += 2 * step) {
#pragma unroll
        for (int jj = i; jj < i + step; ++jj) {
          const float a = v[jj], bb = v[jj + step];
          v[jj] = a + bb;
          v[jj + step] = a - bb;
        }
      }
    }
    // partner p, own value u: the lower lane keeps u + p, the upper p - u,
    // both as fma(+-1, u, p) (an exact product, one rounding: the same
    // values as the add and subtract)
    const float s1 = (col & 1) ? -1.0f : 1.0f, s2 = (col & 2) ? -1.0f : 1.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = __builtin_fmaf(s1, v[j], dpp<kDppQuadXor1>(v[j]));
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = __builtin_fmaf(s2, v[j], dpp<kDppQuadXor2>(v[j]));
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] *= kInvSqrt32;
  }
  if (nsplit == 1) {
    const float inv = l > 0.f ? 1.0f / l : 0.f;
    u4_t w;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      w[jj] = (uint32_t)f2h(v[2 * jj] * inv) | ((uint32_t)f2h(v[2 * jj + 1] * inv) << 16);
    *reinterpret_cast<u4_t*>(outp + b * out_stride + (int64_t)(kh * G + h) * 128 + 8 * col) = w;
  } else {
    float* dst = part + ((b * H + (int64_t)kh * G + h) * nsplit + sp) * kPart;
    *reinterpret_cast<f4_t*>(dst + 4 + 8 * col) = f4_t{v[0], v[1], v[2], v[3]};
    *reinterpret_cast<f4_t*>(dst + 8 + 8 * col) = f4_t{v[4], v[5], v[6], v[7]};
    if (col == 0) {
      dst[0] = M;
      dst[1] = l;
    }
  }
}

// Split merge, one wave per (query head, sequence):
//   m* = max_s m_s,  out = sum_s e^(m_s-m*) o_s / sum_s e^(m_s-m*) l_s.
// The two half-waves take the even and the odd splits, lane j of a half
// owning dims 4j .. 4j+3 (16-byte loads: one instruction reads two splits'
// o), and add their sums at the end.  CH splits per round (8, 16, 18, 24,
// 32 or 64: the smallest covering the split count) with a running maximum;
// every load of a round is issued before any arithmetic; slots past the
// last split re-read it and get weight 0, so CH does not change the result.
template <int CH>
__global__ __launch_bounds__(64) void attn_merge_kernel(const float* __restrict__ part,
                                                        uint16_t* __restrict__ outp,
                                                        int64_t out_stride, int H, int G,
                                                        int nsplit) {
  static_assert(CH % 2 == 0 && CH <= 64, "two splits per load, one (m, l) per lane");
  // on the XCD of the pair's partial workgroups (attn_mfma_kernel's order):
  // grid (8 G, pairs / 8) or (G, pairs)
  const bool grouped = (int)gridDim.x != G;
  const int hq = grouped ? (int)blockIdx.x / kXcds : (int)blockIdx.x;
  const int pair = grouped ? (int)blockIdx.y * kXcds + (int)blockIdx.x % kXcds : (int)blockIdx.y;
  const int h = (pair % (H / G)) * G + hq;
  const int64_t b = pair / (H / G);
  const int lane = threadIdx.x, hh = lane >> 5, j = lane & 31;
  const float* pb = part + (b * H + h) * (int64_t)nsplit * kPart;
  float M = -INFINITY, Ls = 0.f;
  f4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int c0 = 0; c0 < nsplit; c0 += CH) {
    const int nc = min(CH, nsplit - c0);
    // (m, l) of split c0 + lane, and the o of splits c0 + 2t + hh, loaded
    // unconditionally from clamped splits
    float2 ml = *reinterpret_cast<const float2*>(pb + (int64_t)(c0 + min(lane, nc - 1)) * kPart);
    f4_t ov[CH / 2];
#pragma unroll
    for (int t = 0; t < CH / 2; ++t)
      ov[t] = *reinterpret_cast<const f4_t*>(pb + (int64_t)(c0 + min(2 * t + hh, nc - 1)) * kPart +
                                             4 + 4 * j);
    // Every load of the round precedes the first wait: the empty asm takes
    // every loaded register (a memory clobber would not order these loads:
    // the partials are read-only and restrict-qualified).
    asm volatile("" : "+v"(ml.x), "+v"(ml.y));
#pragma unroll
    for (int t = 0; t < CH / 2; ++t)
      asm volatile("" : "+v"(ov[t][0]), "+v"(ov[t][1]), "+v"(ov[t][2]), "+v"(ov[t][3]));
    const float ms = lane < nc ? ml.x : -INFINITY, ls = lane < nc ? ml.y : 0.f;
    const float Mn = fmaxf(M, wave_max(ms));
    const float r = (M == -INFINITY) ? 0.f : __expf(M - Mn);  // rescale of earlier rounds
    const float w = (ms == -INFINITY) ? 0.f : __expf(ms - Mn);
    Ls = __builtin_fmaf(Ls, r, wave_sum(w * ls));
    acc *= r;
#pragma unroll
    for (int t = 0; t < CH / 2; ++t) {
      const float we = readlane_f(w, 2 * t), wo = readlane_f(w, 2 * t + 1);  // 0 past the end
      const float ws = hh ? wo : we;
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[k] = __builtin_fmaf(ws, ov[t][k], acc[k]);
    }
    M = Mn;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) acc[k] += __shfl_xor(acc[k], 32);  // even + odd splits
  if (hh == 0) {
    const float inv = Ls > 0.f ? 1.0f / Ls : 0.f;
    const uint32_t lo = (uint32_t)f2h(acc[0] * inv) | ((uint32_t)f2h(acc[1] * inv) << 16);
    const uint32_t hi = (uint32_t)f2h(acc[2] * inv) | ((uint32_t)f2h(acc[3] * inv) << 16);
    *reinterpret_cast<u2_t*>(outp + b * out_stride + (int64_t)h * 128 + 4 * j) = u2_t{lo, hi};
  }
}

}  // namespace

int attn_num_splits(int64_t cap_len, int64_t B, int64_t Hk) {
  // About 128 positions of the cache capacity per split, at most 32 splits
  // and at most 256 workgroups (one per CU); measured on MI355X with cold
  // caches at 2K-32K contexts (32 splits against 64: 10.5 vs 10.9 us at 8K,
  // 18.3 vs 19.0 us at 32K) and in the batched decode step at ctx 2048,
  // where a 512-workgroup cap was slower (ms per step, 256 against 512:
  // batch 2 3.534 / 3.542, batch 4 3.639 / 3.665, batch 8 3.814 / 3.828,
  // at ctx 8192 4.373 / 4.411, batch 16 4.639 / 4.665).  Depends only on
  // the cache capacity, so a captured graph stays valid as the sequence
  // grows.
  if (const int v = tuning().attn_splits.load()) return v;  // measurement override (r4q_tune)
  int64_t n = (cap_len + 127) / 128;
  if (n > 32) n = 32;
  const int64_t by_wg = 256 / (B * Hk > 0 ? B * Hk : 1);
  if (n > by_wg) n = by_wg;
  return (int)(n < 1 ? 1 : n);
}

size_t attn_ws_bytes(int64_t B, int64_t H, int nsplit) {
  return nsplit > 1 ? (size_t)B * H * nsplit * kPart * sizeof(float) : 0;
}

int launch_flash_decode(const void* q, int64_t q_stride, const void* k_cache, const void* v_cache,
                        const float* k_scale, const float* v_scale, void* out, int64_t out_stride,
                        int64_t B, int64_t H, int64_t Hk, int64_t max_seq, int64_t seq_len,
                        const int* seq_len_dev, int nsplit, int fwht, float* ws, hipStream_t st,
                        const AttnQK* qk) {
  const int G = (int)(H / Hk);
  if (nsplit < 1 || nsplit > kMaxSplits)
    return fail(R4Q_EUNSUPPORTED, "flash_decode: %d splits outside [1, %d]", nsplit, kMaxSplits);
  if (nsplit > 1 && !ws) return fail(R4Q_EINVAL, "flash_decode: no split workspace");
  if (qk && qk->nsum > kMaxQkvSplits)
    return fail(R4Q_EUNSUPPORTED, "flash_decode: %d qkv split planes (at most %d)", qk->nsum,
                kMaxQkvSplits);
  const int npair = (int)(B * Hk);  // (sequence, KV head) pairs
  const bool grouped = npair % kXcds == 0;  // the kernels' XCD-grouped order
  const dim3 grid(grouped ? (unsigned)(kXcds * nsplit) : (unsigned)nsplit,
                  grouped ? (unsigned)(npair / kXcds) : (unsigned)npair);
  float* part = ws;
  const auto* qp = static_cast<const uint16_t*>(q);
  const auto* kp = static_cast<const uint8_t*>(k_cache);
  const auto* vp = static_cast<const uint8_t*>(v_cache);
  bool launched = false;
#define R4Q_ATTN_QK(GG, QQ)                                                                   \
  hipLaunchKernelGGL((attn_mfma_kernel<GG, true, QQ>), grid, dim3(256), 0, st, qp, q_stride,   \
                     kp, vp, k_scale, v_scale, part, static_cast<uint16_t*>(out), out_stride,  \
                     fwht, (int)H, (int)Hk, (int)max_seq, (int)seq_len, seq_len_dev, nsplit,  \
                     *qk)
#define R4Q_ATTN_MFMA(GG)                                                                     \
  if (!launched && G == GG) {                                                                 \
    if (qk) {                                                                                 \
      if (qk->nsum < 2) R4Q_ATTN_QK(GG, 0);                                                   \
      else if (qk->nsum == 2) R4Q_ATTN_QK(GG, 2);                                             \
      else if (qk->nsum == 3) R4Q_ATTN_QK(GG, 3);                                             \
      else R4Q_ATTN_QK(GG, 4);                                                                \
    } else                                                                                    \
      hipLaunchKernelGGL((attn_mfma_kernel<GG, false>), grid, dim3(256), 0, st, qp, q_stride,  \
                         kp, vp, k_scale, v_scale, part, static_cast<uint16_t*>(out),         \
                         out_stride, fwht, (int)H, (int)Hk, (int)max_seq, (int)seq_len,       \
                         seq_len_dev, nsplit, AttnQK{});                                      \
    launched = true;                                                                          \
  }
  R4Q_ATTN_MFMA(1) R4Q_ATTN_MFMA(2) R4Q_ATTN_MFMA(4) R4Q_ATTN_MFMA(5) R4Q_ATTN_MFMA(8)
#undef R4Q_ATTN_MFMA
#undef R4Q_ATTN_QK
  if (!launched)
    return fail(R4Q_EUNSUPPORTED, "flash_decode: GQA ratio %d not built (1, 2, 4, 5, 8)", G);
  if (nsplit > 1) {
    const dim3 mg(grouped ? (unsigned)(kXcds * G) : (unsigned)G,
                  grouped ? (unsigned)(npair / kXcds) : (unsigned)npair);
    auto* o16 = static_cast<uint16_t*>(out);
    if (nsplit <= 8)
      hipLaunchKernelGGL(attn_merge_kernel<8>, mg, dim3(64), 0, st, part, o16, out_stride, (int)H,
                         G, nsplit);
    else if (nsplit <= 16)
      hipLaunchKernelGGL(attn_merge_kernel<16>, mg, dim3(64), 0, st, part, o16, out_stride, (int)H,
                         G, nsplit);
    else if (nsplit <= 18)
      hipLaunchKernelGGL(attn_merge_kernel<18>, mg, dim3(64), 0, st, part, o16, out_stride, (int)H,
                         G, nsplit);
    else if (nsplit <= 24)
      hipLaunchKernelGGL(attn_merge_kernel<24>, mg, dim3(64), 0, st, part, o16, out_stride, (int)H,
                         G, nsplit);
    else if (nsplit <= 32)
      hipLaunchKernelGGL(attn_merge_kernel<32>, mg, dim3(64), 0, st, part, o16, out_stride, (int)H,
                         G, nsplit);
    else
      hipLaunchKernelGGL(attn_merge_kernel<64>, mg, dim3(64), 0, st, part, o16, out_stride, (int)H,
                         G, nsplit);
  }
  return launch_status("flash_decode");
}

}  // namespace r4q

extern "C" int r4q_flash_decode(r4q_ctx* ctx, const void* q, int64_t q_stride,
                                const void* k_cache, const void* v_cache, const float* k_scale,
                                const float* v_scale, void* out, int64_t B, int64_t H, int64_t Hk,
                                int64_t D, int64_t max_seq, int64_t seq_len, int fwht,
                                void* stream) {
  R4Q_REQUIRE(ctx, "flash_decode: null context");
  R4Q_REQUIRE(q && k_cache && v_cache && out, "flash_decode: null pointer");
  R4Q_REQUIRE(D == 128, "flash_decode: head_dim must be 128");
  R4Q_REQUIRE(B >= 1 && H >= 1 && Hk >= 1 && H % Hk == 0, "flash_decode: bad head counts");
  R4Q_REQUIRE(seq_len >= 1 && seq_len <= max_seq, "flash_decode: seq_len %lld outside [1, %lld]",
              (long long)seq_len, (long long)max_seq);
  R4Q_REQUIRE(q_stride >= H * D && (q_stride % 8) == 0 &&
                  (reinterpret_cast<uintptr_t>(q) & 15) == 0,
              "flash_decode: q rows must be 16-byte aligned with stride >= H*D");
  R4Q_REQUIRE((reinterpret_cast<uintptr_t>(out) & 15) == 0, "flash_decode: out must be 16-byte aligned");
  const int nsplit = r4q::attn_num_splits(seq_len, B, Hk);
  R4Q_TRY(ctx->attn.reserve(r4q::attn_ws_bytes(B, H, nsplit)));
  return r4q::launch_flash_decode(q, q_stride, k_cache, v_cache, k_scale, v_scale, out, H * D, B,
                                  H, Hk, max_seq, seq_len, nullptr, nsplit, fwht,
                                  static_cast<float*>(ctx->attn.ptr), r4q::as_stream(stream));
}

extern "C" int r4q_flash_decode_qkv(r4q_ctx* ctx, const void* qkv, int64_t qkv_stride,
                                    const void* q_norm, const void* k_norm, const void* cos_t,
                                    const void* sin_t, float eps, void* k_cache, void* v_cache,
                                    const float* k_scale, const float* v_scale, void* out,
                                    int64_t B, int64_t H, int64_t Hk, int64_t D, int64_t max_seq,
                                    int64_t rope_len, int64_t pos, int fwht, void* stream) {
  R4Q_REQUIRE(ctx, "flash_decode_qkv: null context");
  R4Q_REQUIRE(qkv && q_norm && k_norm && cos_t && sin_t && k_cache && v_cache && out,
              "flash_decode_qkv: null pointer");
  R4Q_REQUIRE(D == 128, "flash_decode_qkv: head_dim must be 128");
  R4Q_REQUIRE(B >= 1 && H >= 1 && Hk >= 1 && H % Hk == 0, "flash_decode_qkv: bad head counts");
  R4Q_REQUIRE(pos >= 0 && pos < max_seq && pos < rope_len,
              "flash_decode_qkv: pos %lld outside the cache (%lld) or RoPE table (%lld rows)",
              (long long)pos, (long long)max_seq, (long long)rope_len);
  R4Q_REQUIRE(qkv_stride >= (H + 2 * Hk) * D, "flash_decode_qkv: qkv stride < (H + 2 Hk) * D");
  R4Q_REQUIRE((reinterpret_cast<uintptr_t>(out) & 15) == 0,
              "flash_decode_qkv: out must be 16-byte aligned");
  // split count from the cache capacity, as in the decode step
  const int nsplit = r4q::attn_num_splits(max_seq, B, Hk);
  R4Q_TRY(ctx->attn.reserve(r4q::attn_ws_bytes(B, H, nsplit)));
  const r4q::AttnQK qk{static_cast<const uint16_t*>(q_norm), static_cast<const uint16_t*>(k_norm),
                       static_cast<const uint16_t*>(cos_t), static_cast<const uint16_t*>(sin_t),
                       static_cast<uint8_t*>(k_cache), static_cast<uint8_t*>(v_cache), eps};
  return r4q::launch_flash_decode(qkv, qkv_stride, k_cache, v_cache, k_scale, v_scale, out, H * D,
                                  B, H, Hk, max_seq, pos + 1, nullptr, nsplit, fwht,
                                  static_cast<float*>(ctx->attn.ptr), r4q::as_stream(stream), &qk);
}

// ------------------------------------------------ allocation-free variant
namespace r4q {
namespace {
// Split partials of r4q_flash_decode_noalloc: one array per GPU, alive until
// the process ends, shared by every call on that GPU (calls that overlap on
// one GPU race on it).  Every launch writes all the partials it reads, so
// nothing has to start zeroed.
constexpr size_t kNoAllocScratchBytes = 4u << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (the host-side name is
// only a stand-in): looked up once per device with hipGetSymbolAddress.
int scratch_on_current_device(void** out) {
  int dev = -1;
  R4Q_HIP_TRY(hipGetDevice(&dev));
  R4Q_REQUIRE(dev >= 0 && dev < kMaxDevices, "flash_decode_noalloc: device %d out of range", dev);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      R4Q_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
      R4Q_REQUIRE(p, "flash_decode_noalloc: null scratch address");
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return R4Q_OK;
}
}  // namespace
}  // namespace r4q

extern "C" int r4q_flash_decode_noalloc(const void* q, int64_t q_stride, const void* k_cache,
                                        const void* v_cache, const float* k_scale,
                                        const float* v_scale, void* out, int64_t B, int64_t H,
                                        int64_t Hk, int64_t D, int64_t max_seq, int64_t seq_len,
                                        int fwht, void* stream) {
  R4Q_REQUIRE(q && k_cache && v_cache && out, "flash_decode_noalloc: null pointer");
  R4Q_REQUIRE(D == 128, "flash_decode_noalloc: head_dim must be 128");
  R4Q_REQUIRE(B >= 1 && H >= 1 && Hk >= 1 && H % Hk == 0, "flash_decode_noalloc: bad head counts");
  R4Q_REQUIRE(seq_len >= 1 && seq_len <= max_seq,
              "flash_decode_noalloc: seq_len %lld outside [1, %lld]", (long long)seq_len,
              (long long)max_seq);
  R4Q_REQUIRE(q_stride >= H * D && (q_stride % 8) == 0 &&
                  (reinterpret_cast<uintptr_t>(q) & 15) == 0,
              "flash_decode_noalloc: q rows must be 16-byte aligned with stride >= H*D");
  R4Q_REQUIRE((reinterpret_cast<uintptr_t>(out) & 15) == 0,
              "flash_decode_noalloc: out must be 16-byte aligned");
  const int nsplit = r4q::attn_num_splits(seq_len, B, Hk);
  const size_t need = r4q::attn_ws_bytes(B, H, nsplit);
  R4Q_REQUIRE(need <= r4q::kNoAllocScratchBytes,
              "flash_decode_noalloc: %d splits x %lld heads x %lld sequences need %zu bytes of "
              "partials, above the %zu-byte scratch",
              nsplit, (long long)H, (long long)B, need, r4q::kNoAllocScratchBytes);
  void* ws = nullptr;
  R4Q_TRY(r4q::scratch_on_current_device(&ws));
  return r4q::launch_flash_decode(q, q_stride, k_cache, v_cache, k_scale, v_scale, out, H * D, B,
                                  H, Hk, max_seq, seq_len, nullptr, nsplit, fwht,
                                  static_cast<float*>(ws), r4q::as_stream(stream));
}
