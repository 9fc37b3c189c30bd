// Split-K flash-decode over the FP8 E4M3 KV cache (GQA), with the log-sum-exp
// merge and the optional FWHT-32 output rotation fused into the same launch.
//
// Replaces the reference's launch_flash_decode (hip:1547-1593) with its
// flash_decode_partial (hip:1326-1412), flash_decode_reduce (hip:1416-1463)
// and flash_decode_fused (hip:1471-1542); softmax semantics follow SDPA
// (int4_engine_v5.py:245).  Unlike the reference, Q stays fp16 (the
// reference's FP8 quantisation of Q costs ~2.7e-2 rel-L2 and its
// dot4_f32_fp8_fp8 instruction does not exist on gfx950), and K/V carry an
// optional per-head fp32 scale.
//
// One workgroup (4 waves) per (split, kv head, sequence) walks its split in
// 256-position tiles:
//  * every K and V load of a tile is issued before any arithmetic (one
//    memory latency per tile);
//  * QK: 4 lanes per position, each owning 32 head dims; the position's 32 K
//    bytes arrive in two 128-bit loads and are widened to fp16 by placing the
//    E4M3 fields into fp16 fields (exact, value / 256); the GQA group's query
//    heads live in registers as fp16 pairs so every K byte feeds all of them
//    through v_dot2_f32_f16; the 4 partial dots are combined with DPP.
//  * scores -> LDS; online softmax per head: tile max, running max/sum and
//    the rescale factor of earlier tiles, fp16-rounded probabilities of
//    position pairs -> LDS.
//  * PV: each lane owns 4 head dims; two positions' V bytes are interleaved
//    with v_perm so v_dot2 contracts over the position pair; the running
//    accumulators are rescaled per tile and reduced across half-waves and
//    waves through LDS at the end.
// Merge: the last workgroup to finish for a (sequence, kv head) -- found with
// a self-resetting arrival counter, no waiting -- combines the (at most 64)
// splits while they are in cache with 128-bit loads: m* = max_s m_s,
// out = sum_s e^(m_s-m*) o_s / sum_s e^(m_s-m*) l_s, then the FWHT-32 in
// registers (one thread per 32-dim chunk).
#include <math.h>
#include <stdlib.h>

#include "r4q_ctx.hpp"
#include "r4q_device.hpp"
#include "r4q_host.hpp"

namespace r4q {
namespace {

constexpr int kMaxSplits = 128;  // partials per (sequence, head)
constexpr int kMergeChunk = 64;  // splits merged per round (one per lane)
constexpr int kPart = 132;       // floats per (seq, head, split): m, l, pad, pad, o[128]

// Four E4M3 bytes (b0 b1 b2 b3) -> fp16 pairs (b0, b2) and (b1, b3), each
// value divided by 256 (exact).
__device__ __forceinline__ void fp8x4_to_h2_div256(uint32_t w, uint32_t& h02, uint32_t& h13) {
  uint32_t m1 = 0x80008000u, m2 = 0x3F803F80u;
  asm volatile("" : "+v"(m1), "+v"(m2));
  h02 = ((w << 8) & m1) | ((w << 7) & m2);
  h13 = (w & m1) | ((w >> 1) & m2);
}

template <int G, int TILE, bool NORMQ>
__global__ __launch_bounds__(256) void attn_partial_kernel(
    const uint16_t* __restrict__ q, int64_t q_stride, const uint8_t* __restrict__ kc,
    const uint8_t* __restrict__ vc, const float* __restrict__ ksc, const float* __restrict__ vsc,
    float* __restrict__ part, uint16_t* __restrict__ outp,
    int64_t out_stride, int fwht, int H, int Hk, int max_seq, int L_host,
    const int* __restrict__ L_dev, int nsplit, AttnQK qk) {
  const int sp = blockIdx.x, kh = blockIdx.y;
  const int64_t b = blockIdx.z;
  const int L = L_dev ? *L_dev : L_host;
  const int S = (L + nsplit - 1) / nsplit;
  const int s0 = sp * S;
  const int n = max(0, min(L, s0 + S) - s0);

  // 128-bit LDS accesses below need 16-byte aligned rows
  __shared__ __align__(16) float sc[G][TILE < 128 ? 128 : TILE];  // also the output stage
  __shared__ __align__(16) uint32_t pp[G][TILE / 2];
  __shared__ __align__(16) float red[8][32][G * 4];
  __shared__ float stat[G][4];  // running max, running sum, tile rescale
  __shared__ __align__(16) uint16_t qs[NORMQ ? G : 1][128];
  __shared__ __align__(16) uint8_t knew[128], vnew[128];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const float ks = ksc ? ksc[kh] : 1.0f;
  const float vs = vsc ? vsc[kh] : 1.0f;
  const int64_t head_off = ((b * Hk + kh) * (int64_t)max_seq + s0) * 128;
  const uint8_t* kbase = kc + head_off;
  const uint8_t* vbase = vc + head_off;

  const int dq = t & 3;
  const int d4 = lane & 31, half = lane >> 5;

  // ---- K and V loads of a tile.  Rows past the tile end are clamped to its
  // last row; their scores become -inf and their probabilities 0.
  constexpr int kPass = TILE / 64;   // 64 positions per QK pass
  constexpr int kPairs = TILE / 16;  // position pairs per (wave, half) slot
  u4_t kw[kPass][2];
  uint32_t va[kPairs], vb[kPairs];
  auto load_k = [&](int base, int nt) {
#pragma unroll
    for (int pass = 0; pass < kPass; ++pass) {
      const int p = min(pass * 64 + (t >> 2), nt - 1);
      const u4_t* kr = reinterpret_cast<const u4_t*>(kbase + (int64_t)(base + p) * 128 + 32 * dq);
      kw[pass][0] = __builtin_nontemporal_load(kr);
      kw[pass][1] = __builtin_nontemporal_load(kr + 1);
    }
  };
  auto load_v = [&](int base, int nt) {
#pragma unroll
    for (int k = 0; k < kPairs; ++k) {
      const int i = 2 * wave + half + 8 * k;
      const int r0 = min(2 * i, nt - 1), r1 = min(2 * i + 1, nt - 1);
      va[k] = __builtin_nontemporal_load(
          reinterpret_cast<const uint32_t*>(vbase + (int64_t)(base + r0) * 128 + 4 * d4));
      vb[k] = __builtin_nontemporal_load(
          reinterpret_cast<const uint32_t*>(vbase + (int64_t)(base + r1) * 128 + 4 * d4));
    }
  };

  uint32_t qraw[G][16];
  if constexpr (NORMQ) {
    // first tile in flight while the prologue normalises q (and K/V)
    if (n > 0) {
      load_k(0, min(TILE, n));
      load_v(0, min(TILE, n));
    }
    const int pos = L - 1;
    const bool owner = n > 0 && pos >= s0 && pos < s0 + n;  // workgroup-uniform
    const uint16_t* row = q + b * q_stride;  // raw QKV row: q | k | v heads
    const float c = h2f_ieee(qk.cs[(int64_t)pos * 64 + lane]);
    const float sn = h2f_ieee(qk.sn[(int64_t)pos * 64 + lane]);
    const int ntask = G + (owner ? 2 : 0);
    for (int task = wave; task < ntask; task += 4) {
      if (task < G) {
        const uint16_t* src = row + (int64_t)(kh * G + task) * 128;
        float lo, hi;
        head_norm_rope_pair(h2f_ieee(src[lane]), h2f_ieee(src[lane + 64]), h2f_ieee(qk.qw[lane]),
                            h2f_ieee(qk.qw[lane + 64]), c, sn, qk.eps, lo, hi);
        qs[task][lane] = f2h(lo);
        qs[task][lane + 64] = f2h(hi);
      } else if (task == G) {
        const uint16_t* src = row + (int64_t)(H + kh) * 128;
        float lo, hi;
        head_norm_rope_pair(h2f_ieee(src[lane]), h2f_ieee(src[lane + 64]), h2f_ieee(qk.kw[lane]),
                            h2f_ieee(qk.kw[lane + 64]), c, sn, qk.eps, lo, hi);
        const float inv = ksc ? 1.0f / ksc[kh] : 1.0f;
        const uint8_t c0 = (uint8_t)fp8_encode(lo * inv), c1 = (uint8_t)fp8_encode(hi * inv);
        uint8_t* kp = qk.kc + ((b * Hk + kh) * (int64_t)max_seq + pos) * 128;
        kp[lane] = c0;
        kp[lane + 64] = c1;
        knew[lane] = c0;
        knew[lane + 64] = c1;
      } else {
        const uint16_t* src = row + (int64_t)(H + Hk + kh) * 128;
        const float inv = vsc ? 1.0f / vsc[kh] : 1.0f;
        const uint8_t c0 = (uint8_t)fp8_encode(h2f_ieee(src[lane]) * inv);
        const uint8_t c1 = (uint8_t)fp8_encode(h2f_ieee(src[lane + 64]) * inv);
        uint8_t* vp = qk.vc + ((b * Hk + kh) * (int64_t)max_seq + pos) * 128;
        vp[lane] = c0;
        vp[lane + 64] = c1;
        vnew[lane] = c0;
        vnew[lane + 64] = c1;
      }
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const u4_t* qr = reinterpret_cast<const u4_t*>(&qs[g][32 * dq]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u4_t v = qr[i];
        qraw[g][4 * i] = v[0];
        qraw[g][4 * i + 1] = v[1];
        qraw[g][4 * i + 2] = v[2];
        qraw[g][4 * i + 3] = v[3];
      }
    }
  } else {
    // query rows first, then the first tile: both in flight together
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const u4_t* qr = reinterpret_cast<const u4_t*>(q + b * q_stride +
                                                     (int64_t)(kh * G + g) * 128 + 32 * dq);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const u4_t v = qr[i];
        qraw[g][4 * i] = v[0];
        qraw[g][4 * i + 1] = v[1];
        qraw[g][4 * i + 2] = v[2];
        qraw[g][4 * i + 3] = v[3];
      }
    }
    if (n > 0) {
      load_k(0, min(TILE, n));
      load_v(0, min(TILE, n));
    }
  }
  const int pos_new = NORMQ ? L - 1 : -1;  // position whose K/V sit in knew/vnew

  // ---- query pairs matching the K decode order:
  // K dword j holds dims 4j..4j+3 -> pairs (4j, 4j+2), (4j+1, 4j+3)
  uint32_t qp[G][16];
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t a = qraw[g][2 * j], c = qraw[g][2 * j + 1];
      qp[g][2 * j] = (a & 0xFFFFu) | (c << 16);
      qp[g][2 * j + 1] = (a >> 16) | (c & 0xFFFF0000u);
    }
  }
  if (t < G) {
    stat[t][0] = -INFINITY;
    stat[t][1] = 0.f;
  }

  float o[G][4];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 4; ++j) o[g][j] = 0.f;

  const float sscale = ks * 22.627416997969522f;  // 256 / sqrt(128)
  for (int base = 0; base < n; base += TILE) {
    const int nt = min(TILE, n - base);
    // (this tile's K and V were requested before the previous tile's
    // arithmetic, or before the query prep for the first tile)
    // ---- Q K^T, 4 lanes per position, 64 positions per pass
#pragma unroll
    for (int pass = 0; pass < kPass; ++pass) {
      const int p = pass * 64 + (t >> 2);
      float acc[G];
#pragma unroll
      for (int g = 0; g < G; ++g) acc[g] = 0.f;
      uint32_t k8[8] = {kw[pass][0][0], kw[pass][0][1], kw[pass][0][2], kw[pass][0][3],
                        kw[pass][1][0], kw[pass][1][1], kw[pass][1][2], kw[pass][1][3]};
      if constexpr (NORMQ) {  // the new position: codes from this launch
        if (s0 + base + min(p, nt - 1) == pos_new) {
#pragma unroll
          for (int j = 0; j < 8; ++j) k8[j] = reinterpret_cast<const uint32_t*>(knew)[8 * dq + j];
        }
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        uint32_t h02, h13;
        fp8x4_to_h2_div256(k8[j], h02, h13);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          acc[g] = __builtin_amdgcn_fdot2(as_h2(h02), as_h2(qp[g][2 * j]), acc[g], false);
          acc[g] = __builtin_amdgcn_fdot2(as_h2(h13), as_h2(qp[g][2 * j + 1]), acc[g], false);
        }
      }
      dot_dpp_fence();
#pragma unroll
      for (int g = 0; g < G; ++g) {
        acc[g] += dpp<kDppQuadXor1>(acc[g]);
        acc[g] += dpp<kDppQuadXor2>(acc[g]);
      }
      if (dq == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) sc[g][p] = (p < nt) ? acc[g] * sscale : -INFINITY;
      }
    }
    const int nb = base + TILE;  // next tile
    if (nb < n) load_k(nb, min(TILE, n - nb));
    __syncthreads();

    // ---- online softmax: tile max, rescale of the running state, fp16
    // probabilities of position pairs.  Lane j holds positions PPL*j ...
    constexpr int PPL = TILE >= 256 ? 4 : 2;
    const bool act = lane * PPL < TILE;
    for (int g = wave; g < G; g += 4) {
      float v[PPL];
#pragma unroll
      for (int i = 0; i < PPL; ++i) v[i] = act ? sc[g][PPL * lane + i] : -INFINITY;
      float vm = v[0];
#pragma unroll
      for (int i = 1; i < PPL; ++i) vm = fmaxf(vm, v[i]);
      const float mt = wave_max(vm);
      const float mo = stat[g][0];
      const float mn = fmaxf(mo, mt);
      const float alpha = (mo == -INFINITY) ? 0.f : __expf(mo - mn);
      float pr[PPL], ps = 0.f;
#pragma unroll
      for (int i = 0; i < PPL; ++i) {
        pr[i] = (mn == -INFINITY) ? 0.f : h2f(f2h(__expf(v[i] - mn)));
        ps += pr[i];
      }
      const float l = wave_sum(ps);
      if (act) {
#pragma unroll
        for (int j = 0; j < PPL / 2; ++j)
          pp[g][(PPL / 2) * lane + j] =
              (uint32_t)f2h(pr[2 * j]) | ((uint32_t)f2h(pr[2 * j + 1]) << 16);
      }
      if (lane == 0) {
        stat[g][0] = mn;
        stat[g][1] = __builtin_fmaf(stat[g][1], alpha, l);
        stat[g][2] = alpha;
      }
    }
    __syncthreads();

    // ---- P V: lane d4 owns dims 4*d4 .. 4*d4+3 of position pairs
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float a = stat[g][2];
#pragma unroll
      for (int j = 0; j < 4; ++j) o[g][j] *= a;
    }
#pragma unroll
    for (int k = 0; k < kPairs; ++k) {
      const int i = 2 * wave + half + 8 * k;
      uint32_t av = va[k], bv = vb[k];
      if constexpr (NORMQ) {  // the new position: codes from this launch
        const uint32_t nv = reinterpret_cast<const uint32_t*>(vnew)[d4];
        if (s0 + base + min(2 * i, nt - 1) == pos_new) av = nv;
        if (s0 + base + min(2 * i + 1, nt - 1) == pos_new) bv = nv;
      }
      // (a0 a1 c0 c1) and (a2 a3 c2 c3): decode gives (a_d, c_d) pairs per dim
      const uint32_t x0 = __builtin_amdgcn_perm(bv, av, 0x05040100u);
      const uint32_t x1 = __builtin_amdgcn_perm(bv, av, 0x07060302u);
      uint32_t h0, h1, h2, h3;
      fp8x4_to_h2_div256(x0, h0, h1);
      fp8x4_to_h2_div256(x1, h2, h3);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const h2_t pg = as_h2(pp[g][i]);
        o[g][0] = __builtin_amdgcn_fdot2(as_h2(h0), pg, o[g][0], false);
        o[g][1] = __builtin_amdgcn_fdot2(as_h2(h1), pg, o[g][1], false);
        o[g][2] = __builtin_amdgcn_fdot2(as_h2(h2), pg, o[g][2], false);
        o[g][3] = __builtin_amdgcn_fdot2(as_h2(h3), pg, o[g][3], false);
      }
    }
    if (nb < n) load_v(nb, min(TILE, n - nb));
    __syncthreads();  // sc / pp / stat rescale reused by the next tile
  }

#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int j = 0; j < 4; ++j) red[2 * wave + half][d4][4 * g + j] = o[g][j];
  __syncthreads();

  // ---- reduce over the 8 (wave, half) slots into ostage[G][128]
  float* ostage = &sc[0][0];
  const float oscale = vs * 256.0f;
  for (int e = t; e < G * 128; e += 256) {
    const int g = e >> 7, d = e & 127;
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < 8; ++r) s += red[r][d >> 2][4 * g + (d & 3)];
    ostage[e] = s * oscale;
  }
  __syncthreads();

  // ---- one thread per 32-dim chunk: FWHT-32 in registers (it is linear,
  // so it commutes with the split merge), then either the final fp16 output
  // (single split) or the fp32 partial (m, l, o).
  if (t < 4 * G) {
    const int g = t >> 2, c = t & 3;
    float v[32];
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
      const f4_t x = *reinterpret_cast<const f4_t*>(&ostage[g * 128 + 32 * c + i]);
      v[i] = x[0];
      v[i + 1] = x[1];
      v[i + 2] = x[2];
      v[i + 3] = x[3];
    }
    if (fwht) fwht32(v);
    if (nsplit == 1) {
      const float l = stat[g][1];
      const float inv = l > 0.f ? 1.0f / l : 0.f;
      uint16_t* dst = outp + b * out_stride + (int64_t)(kh * G + g) * 128 + 32 * c;
#pragma unroll
      for (int i = 0; i < 32; i += 8) {
        u4_t w;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          w[j] = (uint32_t)f2h(v[i + 2 * j] * inv) | ((uint32_t)f2h(v[i + 2 * j + 1] * inv) << 16);
        *reinterpret_cast<u4_t*>(dst + i) = w;
      }
    } else {
      float* dst = part + ((b * H + (int64_t)kh * G + g) * nsplit + sp) * kPart;
#pragma unroll
      for (int i = 0; i < 32; i += 4) {
        const f4_t x = {v[i], v[i + 1], v[i + 2], v[i + 3]};
        *reinterpret_cast<f4_t*>(dst + 4 + 32 * c + i) = x;
      }
      if (c == 0) {
        dst[0] = stat[g][0];
        dst[1] = stat[g][1];
      }
    }
  }
}

// Split merge, one wave per (query head, sequence); lane j owns dims 2j and
// 2j+1.  Every load is issued before any arithmetic:
//   m* = max_s m_s,  out = sum_s e^(m_s-m*) o_s / sum_s e^(m_s-m*) l_s.
__global__ __launch_bounds__(64) void attn_merge_kernel(const float* __restrict__ part,
                                                        uint16_t* __restrict__ outp,
                                                        int64_t out_stride, int H, int nsplit) {
  const int h = blockIdx.x;
  const int64_t b = blockIdx.y;
  const int lane = threadIdx.x;
  const float* pb = part + (b * H + h) * (int64_t)nsplit * kPart;
  // splits in chunks of 64 (lane s holds split c0+s's m and l) with a
  // running maximum; every load of a chunk is issued before its arithmetic
  float M = -INFINITY, Ls = 0.f, a0 = 0.f, a1 = 0.f;
  for (int c0 = 0; c0 < nsplit; c0 += kMergeChunk) {
    const int nc = min(kMergeChunk, nsplit - c0);
    float ms = -INFINITY, ls = 0.f;
    if (lane < nc) {
      ms = pb[(int64_t)(c0 + lane) * kPart];
      ls = pb[(int64_t)(c0 + lane) * kPart + 1];
    }
    float2 ov[kMergeChunk];
#pragma unroll
    for (int s = 0; s < kMergeChunk; ++s)
      ov[s] = *reinterpret_cast<const float2*>(pb + (int64_t)(c0 + min(s, nc - 1)) * kPart + 4 +
                                               2 * lane);
    const float Mn = fmaxf(M, wave_max(ms));
    const float r = (M == -INFINITY) ? 0.f : __expf(M - Mn);  // rescale of earlier chunks
    const float w = (ms == -INFINITY) ? 0.f : __expf(ms - Mn);
    Ls = __builtin_fmaf(Ls, r, wave_sum(w * ls));
    a0 *= r;
    a1 *= r;
#pragma unroll
    for (int s = 0; s < kMergeChunk; ++s) {
      const float ws = readlane_f(w, s);  // 0 past the chunk end
      a0 = __builtin_fmaf(ws, ov[s].x, a0);
      a1 = __builtin_fmaf(ws, ov[s].y, a1);
    }
    M = Mn;
  }
  const float inv = Ls > 0.f ? 1.0f / Ls : 0.f;
  *reinterpret_cast<uint32_t*>(outp + b * out_stride + (int64_t)h * 128 + 2 * lane) =
      (uint32_t)f2h(a0 * inv) | ((uint32_t)f2h(a1 * inv) << 16);
}

}  // namespace

int attn_num_splits(int64_t cap_len, int64_t B, int64_t Hk) {
  // About 128 positions of the cache capacity per split, at most 64 splits
  // (measured on MI355X at 2K-32K contexts, batch 1 and 8: more splits add
  // merge traffic and per-workgroup fixed cost faster than they add
  // parallelism).  Depends only on the cache capacity, so a captured graph
  // stays valid as the sequence grows.
  (void)B;
  (void)Hk;
  if (const char* e = getenv("R4Q_ATTN_SPLITS")) {  // tuning override
    const int v = atoi(e);
    if (v >= 1 && v <= kMaxSplits) return v;
  }
  int64_t n = (cap_len + 127) / 128;
  if (n > 64) n = 64;
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
  const dim3 grid((unsigned)nsplit, (unsigned)Hk, (unsigned)B);
  float* part = ws;
  const auto* qp = static_cast<const uint16_t*>(q);
  const auto* kp = static_cast<const uint8_t*>(k_cache);
  const auto* vp = static_cast<const uint8_t*>(v_cache);
  // tile: the shortest that holds the longest split this launch can see
  const int64_t lmax = seq_len_dev ? max_seq : seq_len;
  const int64_t smax = (lmax + nsplit - 1) / nsplit;
  const int tile = smax <= 64 ? 64 : smax <= 128 ? 128 : 256;
#define R4Q_ATTN(GG, TT)                                                                      \
  if (G == GG && tile == TT) {                                                                \
    if (qk)                                                                                   \
      hipLaunchKernelGGL((attn_partial_kernel<GG, TT, true>), grid, dim3(256), 0, st, qp,       \
                         q_stride, kp, vp, k_scale, v_scale, part,                            \
                         static_cast<uint16_t*>(out), out_stride, fwht, (int)H, (int)Hk,      \
                         (int)max_seq, (int)seq_len, seq_len_dev, nsplit, *qk);               \
    else                                                                                      \
      hipLaunchKernelGGL((attn_partial_kernel<GG, TT, false>), grid, dim3(256), 0, st, qp,      \
                         q_stride, kp, vp, k_scale, v_scale, part,                            \
                         static_cast<uint16_t*>(out), out_stride, fwht, (int)H, (int)Hk,      \
                         (int)max_seq, (int)seq_len, seq_len_dev, nsplit, AttnQK{});           \
    launched = true;                                                                          \
  }
  bool launched = false;
  R4Q_ATTN(1, 64) R4Q_ATTN(1, 128) R4Q_ATTN(1, 256)
  R4Q_ATTN(2, 64) R4Q_ATTN(2, 128) R4Q_ATTN(2, 256)
  R4Q_ATTN(4, 64) R4Q_ATTN(4, 128) R4Q_ATTN(4, 256)
  R4Q_ATTN(5, 64) R4Q_ATTN(5, 128) R4Q_ATTN(5, 256)
  R4Q_ATTN(8, 64) R4Q_ATTN(8, 128) R4Q_ATTN(8, 256)
  if (!launched)
    return fail(R4Q_EUNSUPPORTED, "flash_decode: GQA ratio %d not built (1, 2, 4, 5, 8)", G);
#undef R4Q_ATTN
  if (nsplit > 1)
    hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)H, (unsigned)B), dim3(64), 0, st, part,
                       static_cast<uint16_t*>(out), out_stride, (int)H, nsplit);
  return launch_status("flash_decode");
}

int DevBuf::reserve(size_t need) {
  if (need <= bytes) return R4Q_OK;
  if (ptr) {
    (void)hipFree(ptr);
    ptr = nullptr;
    bytes = 0;
  }
  const size_t cap = (need + 0xFFFFF) & ~(size_t)0xFFFFF;  // 1 MiB granules
  if (hipMalloc(&ptr, cap) != hipSuccess) {
    ptr = nullptr;
    return fail(R4Q_ENOMEM, "hipMalloc(%zu) failed", cap);
  }
  bytes = cap;
  return R4Q_OK;
}

void DevBuf::release() {
  if (ptr) (void)hipFree(ptr);
  ptr = nullptr;
  bytes = 0;
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
