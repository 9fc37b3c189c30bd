// Prefill GEMM Y[M,N] = X[M,K] W[N,K]^T with the weight dequantised on the
// fly (INT4 / INT8 block-32 asymmetric, or FP16) and multiplied on the
// matrix cores with v_mfma_f32_16x16x32_f16 (fp32 accumulate).
//
// Replaces the reference's prefill projection dequant_matmul_out
// (hip:1973-1988), which materialises the whole fp16 weight with
// dequant_int4_kernel and then calls rocBLAS through at::mm_out: here each
// weight byte is read from HBM once per M-tile and never written back.
//
// Three kernels, by shape:
//  * gemm_ring_kernel (M >= 256, INT4 / INT8): 256 x 256 tiles, X and the
//    raw weights copied global -> LDS through a multi-stage ring, the
//    weights dequantised once per workgroup into an fp16 B tile, optional
//    deterministic split-K over a caller workspace (see its comment);
//  * gemm_mfma_kernel (17 <= M < 256, and FP16 weights): 128 x 128 tiles,
//    X and the dequantised W staged in LDS per 32-wide K step;
//  * gemm_skinny_kernel (2 <= M <= 16): weights streamed once for all rows
//    through an LDS ring (split along K for narrow N).
// Dequantised values equal r4q_dequant_int4/8 bit-for-bit
// (fp16((q - zp) * scale) from an exact product, one rounding).
#include <stdint.h>
#include <stdlib.h>

#include <algorithm>

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

// 128 x 128 tile: a workgroup (4 waves) walks K in steps of 32 (one
// quantisation block).  Per step the X tile (128 x 32 fp16) and the
// dequantised W tile (128 x 32 fp16) are staged in LDS (rows padded to
// 80 B); each wave computes a 64 x 64 sub-tile as 4 x 4 MFMA 16x16x32
// tiles.  The next step's global loads are issued before the current
// step's MFMAs (one step in flight: latency-bound at large K, which is why
// M >= 256 takes the ring kernel).
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
// Weight fragments of the skinny GEMM (below).  The MFMA contraction index k
// is only a label: lane group g's 8 k-slots of an MFMA carry 8 weight
// elements, and the A fragment of that lane group holds the activation
// values of exactly those elements.  Because the weights are fully
// dequantised before the MFMA -- fp16((q - zp) * s) by an exact packed fp16
// subtraction and one rounded packed multiply, bit-identical to the dequant
// kernel -- the accumulation may run across blocks.
//   INT4: 4 MFMAs per 16 weight bytes; nibble pairs (q_p, q_p+4) come from
//         (w >> 4p) & 0x000F000F | 0x64006400, so the activation is permuted
//         to (x_p, x_p+4) pairs;
//   INT8: 2 MFMAs per 16 bytes; byte pairs by v_perm, natural order;
//   FP16: 1 MFMA per 16 bytes.
// B fragment of MFMA d from 16 weight bytes w and the block's (scale, zero) s2.
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

// ---------------------------------------------------------------------
// Prefill GEMM for M >= 256 with INT4 / INT8 weights: a workgroup of 8 waves
// (2 per SIMD) owns a 256 x 256 output tile, each wave a 128 x 64 sub-tile
// (8 x 4 MFMA tiles, 128 fp32 accumulators per lane).
// The K loop of the 128 x 128 kernel above is bound by global-load latency
// (one 32-wide K step in flight, ~1.3 us per step on MI355X).  Here X and
// the raw weight bytes (plus the (scale, zero) words) of a K step land in
// LDS by direct global->LDS copies (global_load_lds_dwordx4 / _dword) in a
// ring of Ring::kStages stages, so that several steps are in flight while
// one is multiplied, without holding them in VGPRs.
// Each wave dequantises its own B fragments straight from the raw bytes in
// LDS into registers (one 4-byte INT4 / 8-byte INT8 read per fragment
// instead of 16 bytes of fp16), one step ahead, interleaved with the MFMAs
// of the current step; the fp16 values equal r4q_dequant_int4/8 bit for bit.
// LDS layouts are bank-conflict-free for their fragment reads (measured on
// MI355X with a read-throughput probe):
//  * X rows are 64 bytes per step; the 16-byte piece p of row r sits in slot
//    p ^ ((r >> 1) & 3) of the row;
//  * INT4 weight rows are 16 bytes per step; dword d of row r sits in slot
//    d ^ (((r >> 3) & 1) << 1) (rows 8 apart would share banks otherwise);
//  * INT8 weight rows are 32 bytes per step (two 16-byte pieces, unswizzled).
// One barrier per K step i: before it each wave waits for its own copies of
// step i+1; after it every wave's copies are visible and every wave is done
// with step i-1, whose ring slot then receives step i+kStages-1.  Every
// wave issues the same number of copies per stage (the wait counts are per
// wave): the scale words take one copy of waves 0-3, and waves 4-7 repeat
// theirs into a spare area.
// Work split (1-D grid, tiles numbered M-tile-major): blocks 0 .. full-1
// each compute a whole tile and write fp16; the remaining nst tiles are
// split S ways along K -- block full + S j + s covers K steps
// [s*kps, (s+1)*kps) of tile full + j and writes its fp32 partial to
// part[s][j] (256 x 256) -- and gemm_splitk_reduce_kernel sums the S
// partials of each split tile in split order (deterministic).  With
// full = 0 every tile is split; with full a multiple of the CU count only
// the last round's tiles are, so that round keeps every CU busy.
constexpr int RBM = 256, RBN = 256, RBK = 32;
constexpr int kRingThreads = 512;

template <int WBITS>
struct Ring {
  static constexpr int kStages = WBITS == 4 ? 6 : 5;
  static constexpr int kX = RBM * RBK * 2;          // X: 16 KB
  static constexpr int kW = RBN * RBK * WBITS / 8;  // raw weights: 4 KB (INT4) / 8 KB (INT8)
  static constexpr int kS = RBN * 4;                // (scale, zero) per row
  static constexpr int kStage = kX + kW + 2 * kS;   // + spare area for waves 4-7
  static constexpr int kPerStage = 2 + (WBITS == 4 ? 2 : 1) + 1;  // copies per wave per stage
};

// Global -> LDS copy of 16 (4) bytes per lane: lane l's bytes land at
// lds + 16 l (4 l).  Written as inline assembly so that the compiler's
// wait-count tracking does not see the copies: it would otherwise wait for
// every copy in flight before any LDS read of the ring; the kernel counts
// and waits for its own copies (wait_copies) instead.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)((const __attribute__((address_space(3))) void*)p));
}
__device__ __forceinline__ void copy16(const void* g, void* lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_addr(lds)),
               "v"(g)
               : "memory");
}
__device__ __forceinline__ void copy4(const void* g, void* lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(lds_addr(lds)),
               "v"(g)
               : "memory");
}

// Copies K step kb (32 elements) of the workgroup's 256 X rows and 256
// weight rows into one ring stage; every source row is clamped into the
// matrix (rows past M / N are computed and not stored).  Wave w copies X
// rows 32w .. 32w+31 (2 copies of 16 rows x 64 bytes) and weight rows
// 32w .. 32w+31.
template <int WBITS>
__device__ __forceinline__ void ring_issue(uint8_t* stage, const uint16_t* __restrict__ X,
                                           const uint8_t* __restrict__ W,
                                           const uint32_t* __restrict__ SZ, int M, int N, int K,
                                           int m0, int n0, int kb, int wave, int lane) {
  using R = Ring<WBITS>;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int r0 = 32 * wave + 16 * q;  // first row of this copy
    const int row = r0 + (lane >> 2);
    const int p = (lane & 3) ^ ((row >> 1) & 3);  // global piece held by LDS slot lane & 3
    const int m = min(m0 + row, M - 1);
    copy16(X + (int64_t)m * K + kb * RBK + 8 * p, stage + r0 * 64);
  }
  uint8_t* wst = stage + R::kX;
  if constexpr (WBITS == 4) {  // 16 bytes per row: 2 copies of 16 rows x 4 dwords
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int r0 = 32 * wave + 16 * q;  // a multiple of 16: row bit 3 is lane bit 5
      const int64_t n = min(n0 + r0 + (lane >> 2), N - 1);
      const int d = (lane & 3) ^ (((lane >> 5) & 1) << 1);  // dword held by slot lane & 3
      copy4(W + n * (K / 2) + kb * 16 + 4 * d, wst + r0 * 16);
    }
  } else {  // 32 bytes per row: 32 rows x 2 pieces of 16 bytes
    const int r0 = 32 * wave;
    const int64_t n = min(n0 + r0 + (lane >> 1), N - 1);
    copy16(W + n * K + kb * 32 + 16 * (lane & 1), wst + r0 * 32);
  }
  {  // scale words: waves 0-3 rows 64w .. 64w+63; waves 4-7 repeat into the spare area
    const int r0 = 64 * (wave & 3);
    const int64_t n = min(n0 + r0 + lane, N - 1);
    copy4(SZ + n * (K / 32) + kb, stage + R::kX + R::kW + (wave >> 2) * R::kS + r0 * 4);
  }
}

// B fragments of one ring stage for a wave: fragment j is column c of the
// wave's 16-column block j (weight row wn + 16 j + c) at k labels
// 8 g .. 8 g + 7, dequantised to fp16 as fp16((q - zp) * scale) computed as
// ((1024 + q) - (1024 + zp)) * scale in fp16 pairs (the difference is exact,
// one rounding in the product).  The raw reads are issued first (frag_load),
// the arithmetic later (frag_dequant), so that it can interleave with MFMAs.
template <int WBITS>
struct BRaw {
  uint32_t w[4][WBITS == 4 ? 1 : 2];
  uint32_t s2[4];
};

template <int WBITS>
__device__ __forceinline__ void frag_load(const uint8_t* stage, BRaw<WBITS>& r, int wn, int c,
                                          int g) {
  using R = Ring<WBITS>;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = wn + 16 * j + c;
    if constexpr (WBITS == 4) {
      r.w[j][0] = *reinterpret_cast<const uint32_t*>(stage + R::kX + row * 16 +
                                                     4 * (g ^ (((c >> 3) & 1) << 1)));
    } else {
      const u2_t v = *reinterpret_cast<const u2_t*>(stage + R::kX + row * 32 + 8 * g);
      r.w[j][0] = v[0];
      r.w[j][1] = v[1];
    }
    r.s2[j] = *reinterpret_cast<const uint32_t*>(stage + R::kX + R::kW + row * 4);
  }
}

template <int WBITS>
__device__ __forceinline__ void frag_dequant(const BRaw<WBITS>& r, h8_t* bf) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t sb = r.s2[j] & 0xFFFFu, zb = r.s2[j] >> 16;
    const h2_t sc = as_h2(sb | (sb << 16));
    const h2_t nz = -(as_h2(0x64006400u) + as_h2(zb | (zb << 16)));  // -(1024 + zp), exact
    uint32_t pr[4];  // (1024 + q_2k, 1024 + q_2k+1) as fp16 pairs
    if constexpr (WBITS == 4) {
      typedef uint16_t us2 __attribute__((ext_vector_type(2)));
      const us2 sh = {0, 4};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        // byte k in both halves, the high half shifted down by 4
        const uint32_t tb =
            __builtin_amdgcn_perm(0u, r.w[j][0], (k | 0x0C00u | (k << 16) | 0x0C000000u));
        const uint32_t nib = __builtin_bit_cast(uint32_t, __builtin_bit_cast(us2, tb) >> sh);
        pr[k] = (nib & 0x000F000Fu) | 0x64006400u;
      }
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        pr[k] = __builtin_amdgcn_perm(r.w[j][k >> 1], 0x64646464u,
                                      (k & 1) ? 0x00070006u : 0x00050004u);
    }
    u4_t o;
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = as_u32((as_h2(pr[k]) + nz) * sc);
    bf[j] = __builtin_bit_cast(h8_t, o);
  }
}

template <int N>
__device__ __forceinline__ void wait_copies() {  // at most N of this wave's copies outstanding
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Workgroup barrier that, unlike __syncthreads, does not first wait for
// every outstanding global access (the copies still in flight): only for
// this wave's LDS accesses.
__device__ __forceinline__ void ring_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int WBITS>
__global__ __launch_bounds__(kRingThreads) void gemm_ring_kernel(
    const uint16_t* __restrict__ X, const uint8_t* __restrict__ W,
    const uint32_t* __restrict__ SZ, uint16_t* __restrict__ Y, float* __restrict__ part, int M,
    int N, int K, int full, int nsplit, int kps) {
  using R = Ring<WBITS>;
  constexpr int S = R::kStages;
  __shared__ __align__(16) uint8_t ring[S * R::kStage];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int b = blockIdx.x;
  const bool split = b >= full;  // workgroup-uniform
  const int slot = split ? (b - full) / nsplit : 0, sp = split ? (b - full) % nsplit : 0;
  const int tile = split ? full + slot : b, ntn = (N + RBN - 1) / RBN;
  const int n0 = (tile % ntn) * RBN, m0 = (tile / ntn) * RBM;
  const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;
  const int c = lane & 15, g = lane >> 4;
  const int kb0 = split ? sp * kps : 0;
  const int nk = split ? min(K / RBK - kb0, kps) : K / RBK;  // K steps of this block (>= 1)
  const int nst = (int)(gridDim.x - full) / nsplit;  // split tiles

  f4_t acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};

  int xoff[8];  // per-lane fragment offsets
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = wm + 16 * i + c;
    xoff[i] = row * 64 + 16 * (g ^ ((row >> 1) & 3));
  }

  // stages past the split's end repeat its last step (same copy counts in
  // every iteration; their data is never multiplied)
#pragma unroll
  for (int s = 0; s < S - 1; ++s)
    ring_issue<WBITS>(ring + s * R::kStage, X, W, SZ, M, N, K, m0, n0, kb0 + min(s, nk - 1), wave,
                      lane);
  wait_copies<(S - 2) * R::kPerStage>();  // step 0
  ring_barrier();
  // Two register sets (A fragments and dequantised B fragments) alternate
  // between even and odd steps, so that no step overwrites registers the
  // previous step's MFMAs may still be reading.
  h8_t bf0[4], bf1[4];
  {
    BRaw<WBITS> r0;
    frag_load<WBITS>(ring, r0, wn, c, g);
    frag_dequant<WBITS>(r0, bf0);
  }
  auto kstep = [&](int i, h8_t (&bf)[4], h8_t (&bn)[4]) {
    wait_copies<(S - 3) * R::kPerStage>();  // this wave's copies of step i+1 landed
    ring_barrier();
    ring_issue<WBITS>(ring + ((i + S - 1) % S) * R::kStage, X, W, SZ, M, N, K, m0, n0,
                      kb0 + min(i + S - 1, nk - 1), wave, lane);
    const uint8_t* st = ring + (i % S) * R::kStage;
    h8_t af[8];
#pragma unroll
    for (int i8 = 0; i8 < 8; ++i8) af[i8] = *reinterpret_cast<const h8_t*>(st + xoff[i8]);
    // step i+1's B fragments (raw reads now, dequantised between the MFMAs)
    BRaw<WBITS> rn;
    frag_load<WBITS>(ring + ((i + 1) % S) * R::kStage, rn, wn, c, g);
#pragma unroll
    for (int i8 = 0; i8 < 8; ++i8)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i8][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i8], bf[j], acc[i8][j], 0, 0, 0);
    frag_dequant<WBITS>(rn, bn);
    __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);  // DS reads
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // VALU
    }
  };
  int i = 0;
  for (; i + 1 < nk; i += 2) {
    kstep(i, bf0, bf1);
    kstep(i + 1, bf1, bf0);
  }
  if (i < nk) kstep(i, bf0, bf1);
  wait_copies<0>();  // no copy may land after the workgroup's LDS is released
  // C fragment: lane holds rows 4g + r of an M-block, column c of an N-block
#pragma unroll
  for (int i8 = 0; i8 < 8; ++i8)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = n0 + wn + 16 * j + c;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = m0 + wm + 16 * i8 + 4 * g + r;
        if (split)  // the whole 256 x 256 partial tile (the reduction skips the outside)
          part[(((int64_t)sp * nst + slot) * RBM + (row - m0)) * RBN + (col - n0)] = acc[i8][j][r];
        else if (row < M && col < N)
          Y[(int64_t)row * N + col] = f2h(acc[i8][j][r]);
      }
    }
}

// Y = fp16(sum over s = 0 .. S-1 of part[s][slot]) for the nst split tiles
// (tiles full .. full+nst-1), in split order (deterministic); one block per
// (split tile, tile row), one thread per column.
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const float* __restrict__ part,
                                                                 uint16_t* __restrict__ Y, int M,
                                                                 int N, int full, int nst,
                                                                 int S) {
  const int slot = blockIdx.x / RBM, r = blockIdx.x % RBM, c = threadIdx.x;
  const int tile = full + slot, ntn = (N + RBN - 1) / RBN;
  const int row = (tile / ntn) * RBM + r, col = (tile % ntn) * RBN + c;
  if (row >= M || col >= N) return;
  const int64_t plane = (int64_t)nst * RBM * RBN;
  const float* p = part + ((int64_t)slot * RBM + r) * RBN + c;
  float v = p[0];
  for (int z = 1; z < S; ++z) v += p[z * plane];
  Y[(int64_t)row * N + col] = f2h(v);
}

// ---------------------------------------------------------------------
// Skinny GEMM for 2 <= M <= 16 rows (batched decode) through an LDS ring.
// A workgroup (4 waves) owns 64 weight rows (16 per wave) and a range of K
// steps; each step stages, by global->LDS copies, 128 bytes of every weight
// row (8 rows x 128 B per copy instruction: whole cache lines, which reads
// the weights at ~5.6-6 TB/s where 16 rows x 64 B per instruction -- the
// MFMA B-fragment layout loaded straight into registers -- measured
// 4.4-4.9 TB/s), the rows' (scale, zero) words and the matching slice of the
// MR activation rows.  kSkStages steps are in flight; one barrier per step
// (the ring of gemm_ring_kernel).  Per step each wave runs KS/32 MFMA
// 16x16x32 tiles: B = its 16 weight rows dequantised from LDS (skinny_b),
// A = the activation rows (skinny_a's element order), C = 16 activation
// rows x 16 weight rows.  Lane group g of MFMA j holds the k labels
// k0 + (KS/4) g + 8 j .. +7 in both operands, so each lane reads its 32
// weight bytes of the step with two 16-byte LDS reads.  The 16-byte pieces
// of a row sit in LDS slot piece ^ (row & 7) (bank spread).
// Split-K (S > 1): the workgroup covers steps [s kps, (s+1) kps) and writes
// fp32 partials part[s][m][n]; gemm_skinny_reduce_kernel sums them in order.
constexpr int kSkTile = 64;   // weight rows per workgroup
constexpr int kSkStages = 3;  // steps in flight
constexpr int kSkMaxSplits = 8;

template <int WBITS, int MR>
struct SkRing {
  static constexpr int kKS = 1024 / WBITS;          // k per step: 128 B of each weight row
  static constexpr int kSteps = kKS / 32;           // MFMA k-steps per step
  static constexpr int kW = kSkTile * 128;          // weights: 8 KB
  static constexpr int kSRow = WBITS == 16 ? 0 : (kKS / 32) * 4;  // (scale, zero) bytes per row
  static constexpr int kS = kSkTile * kSRow;        // 2 KB (INT4) / 1 KB (INT8) / 0
  static constexpr int kXRow = kKS * 2;             // activation bytes per row per step
  static constexpr int kX = MR * kXRow;
  static constexpr int kStage = kW + kS + kX;
  static constexpr bool kX16 = kX >= 4096;          // activation as 1 KB copies (else 256 B)
  static constexpr int kCX = kX16 ? kX / 4096 : kX / 1024;  // activation copies per wave
  static constexpr int kCS = WBITS == 4 ? 2 : WBITS == 8 ? 1 : 0;  // scale copies (256 B) per wave
  static constexpr int kPer = 2 + kCS + kCX;        // copies per wave per step
  static_assert(kX % (kX16 ? 4096 : 1024) == 0 && kCX >= 1, "activation copies must split evenly");
};

// Copies step kb of the workgroup's weight rows, scales and activation rows
// into ring stage `stage` (rows past N / M clamped to the last one).
template <int WBITS, int MR>
__device__ __forceinline__ void sk_issue(uint8_t* stage, const uint16_t* __restrict__ X,
                                         const uint8_t* __restrict__ W,
                                         const uint32_t* __restrict__ SZ, int M, int N, int K,
                                         int n0, int kb, int wave, int lane) {
  using R = SkRing<WBITS, MR>;
  const int64_t row_bytes = (int64_t)K * WBITS / 8;
#pragma unroll
  for (int i = 0; i < 2; ++i) {  // weights: copy c covers tile rows 8c .. 8c+7
    const int c = 2 * wave + i, r = 8 * c + (lane >> 3);
    const int piece = (lane & 7) ^ (r & 7);
    const int64_t n = min(n0 + r, N - 1);
    copy16(W + n * row_bytes + (int64_t)kb * 128 + 16 * piece, stage + 1024 * c);
  }
  if constexpr (WBITS != 16) {
    const int nb = K / 32;
    constexpr int wpr = R::kSRow / 4;   // scale words per row per step
    constexpr int rpc = 64 / wpr;       // rows per 256-byte copy
#pragma unroll
    for (int i = 0; i < R::kCS; ++i) {
      const int c = R::kCS * wave + i, r = rpc * c + lane / wpr;
      const int64_t n = min(n0 + r, N - 1);
      copy4(SZ + n * nb + (int64_t)kb * wpr + lane % wpr, stage + R::kW + 256 * c);
    }
  }
  const uint16_t* xs = X + (int64_t)kb * R::kKS;
#pragma unroll
  for (int i = 0; i < R::kCX; ++i) {
    const int c = R::kCX * wave + i;
    if constexpr (R::kX16) {  // 1 KB per copy, 16 bytes per lane
      const int off = 1024 * c + 16 * lane;
      const int r = off / R::kXRow, slot = (off % R::kXRow) / 16;
      const int64_t m = min(r, M - 1);
      copy16(xs + m * K + 8 * (slot ^ (r & 7)), stage + R::kW + R::kS + 1024 * c);
    } else {  // 256 B per copy, 4 bytes per lane
      const int off = 256 * c + 4 * lane;
      const int r = off / R::kXRow, slot = (off % R::kXRow) / 16;
      const int64_t m = min(r, M - 1);
      copy4(xs + m * K + 8 * (slot ^ (r & 7)) + 2 * (lane & 3),
            stage + R::kW + R::kS + 256 * c);
    }
  }
}

template <int WBITS, int MR>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(const uint16_t* __restrict__ X,
                                                          const uint8_t* __restrict__ W,
                                                          const uint32_t* __restrict__ SZ,
                                                          uint16_t* __restrict__ Y,
                                                          float* __restrict__ part, int M, int N,
                                                          int K, int ntiles, int kps) {
  using R = SkRing<WBITS, MR>;
  constexpr int D = kSkStages;
  __shared__ __align__(16) uint8_t ring[D * R::kStage];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x % ntiles, sp = blockIdx.x / ntiles;
  const int n0 = tile * kSkTile;
  const int kt = K / R::kKS;
  const int kb0 = sp * kps, nk = min(kt - kb0, kps);  // >= 1 (host)
  const int col = lane & 15, g = lane >> 4;
  const int wrow = 16 * wave + col;                   // this lane's weight row in the tile
  const int xr = col % MR;                            // activation row (rows >= MR: duplicates)

  f4_t acc = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < D - 1; ++s)
    sk_issue<WBITS, MR>(ring + s * R::kStage, X, W, SZ, M, N, K, n0, kb0 + min(s, nk - 1), wave,
                        lane);
  for (int i = 0; i < nk; ++i) {
    wait_copies<(D - 2) * R::kPer>();  // this wave's copies of step i have landed
    ring_barrier();                    // every wave's; every wave is done with step i-1
    sk_issue<WBITS, MR>(ring + ((i + D - 1) % D) * R::kStage, X, W, SZ, M, N, K, n0,
                        kb0 + min(i + D - 1, nk - 1), wave, lane);
    const uint8_t* st = ring + (i % D) * R::kStage;
    // weight bytes [32 g, 32 g + 32) of row wrow: pieces 2g, 2g+1
    const u4_t b0 = *reinterpret_cast<const u4_t*>(st + 128 * wrow + 16 * ((2 * g) ^ (wrow & 7)));
    const u4_t b1 =
        *reinterpret_cast<const u4_t*>(st + 128 * wrow + 16 * ((2 * g + 1) ^ (wrow & 7)));
    uint32_t sw0 = 0u, sw1 = 0u;
    if constexpr (WBITS == 4) {  // blocks 2g, 2g+1 of the step
      const uint2 v = *reinterpret_cast<const uint2*>(st + R::kW + R::kSRow * wrow + 8 * g);
      sw0 = v.x;
      sw1 = v.y;
    } else if constexpr (WBITS == 8) {  // block g
      sw0 = *reinterpret_cast<const uint32_t*>(st + R::kW + R::kSRow * wrow + 4 * g);
    }
    const uint8_t* xst = st + R::kW + R::kS + R::kXRow * xr;
#pragma unroll
    for (int j = 0; j < R::kSteps; ++j) {
      // activation piece holding k labels k0 + (KS/4) g + 8 j .. +7
      const int piece = (R::kKS / 32) * g + j;
      const u4_t av = *reinterpret_cast<const u4_t*>(xst + 16 * (piece ^ (xr & 7)));
      h8_t a;
      if constexpr (WBITS == 4) {  // (x0 x1)(x2 x3)(x4 x5)(x6 x7) -> (x0 x4)(x1 x5)(x2 x6)(x3 x7)
        u4_t o;
        o[0] = (av[0] & 0xFFFFu) | (av[2] << 16);
        o[1] = (av[0] >> 16) | (av[2] & 0xFFFF0000u);
        o[2] = (av[1] & 0xFFFFu) | (av[3] << 16);
        o[3] = (av[1] >> 16) | (av[3] & 0xFFFF0000u);
        a = __builtin_bit_cast(h8_t, o);
      } else {
        a = __builtin_bit_cast(h8_t, av);
      }
      h8_t b;
      if constexpr (WBITS == 4) b = skinny_b<4>(j < 4 ? b0 : b1, j < 4 ? sw0 : sw1, j & 3);
      else if constexpr (WBITS == 8) b = skinny_b<8>(j < 2 ? b0 : b1, sw0, j & 1);
      else b = __builtin_bit_cast(h8_t, j == 0 ? b0 : b1);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
    }
  }
  wait_copies<0>();  // no copy into LDS outlives the workgroup
  // C: lane holds activation rows 4g + r, weight row n0 + 16 wave + col
  const int n = n0 + 16 * wave + col;
  if (n < N) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = 4 * g + r;
      if (m < M) {
        if (part) part[((int64_t)sp * M + m) * N + n] = acc[r];
        else Y[(int64_t)m * N + n] = f2h(acc[r]);
      }
    }
  }
}

// Y[m][n] = fp16(sum over s of part[s][m][n]), in split order.
__global__ __launch_bounds__(256) void gemm_skinny_reduce_kernel(const float* __restrict__ part,
                                                                 uint16_t* __restrict__ Y, int M,
                                                                 int N, int S) {
  const int n = blockIdx.x * 256 + threadIdx.x, m = blockIdx.y;
  if (n >= N) return;
  const int64_t plane = (int64_t)M * N;
  const float* p = part + (int64_t)m * N + n;
  float v = p[0];
  for (int z = 1; z < S; ++z) v += p[z * plane];
  Y[(int64_t)m * N + n] = f2h(v);
}

// Split sum fused with the SiLU gate of a gate/up projection (N = 2I
// columns: gate 0..I-1, up I..2I-1).  Thread c of row m sums the 32 gate and
// 32 up columns of chunk c over the splits in order and rounds each sum to
// fp16 (what gemm_skinny_reduce_kernel stores), then stores
// FWHT-32(silu(g) * u) in fp16 as silu_kernel<true> does.  64-thread
// workgroups: a row holds only I / 32 chunks.
__device__ __forceinline__ void skinny_sum32(const float* __restrict__ p, int64_t plane, int S,
                                             float* v) {
  const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 t = q[i];
    v[4 * i] = t.x, v[4 * i + 1] = t.y, v[4 * i + 2] = t.z, v[4 * i + 3] = t.w;
  }
  for (int z = 1; z < S; ++z) {
    q = reinterpret_cast<const float4*>(p + z * plane);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 t = q[i];
      v[4 * i] += t.x, v[4 * i + 1] += t.y, v[4 * i + 2] += t.z, v[4 * i + 3] += t.w;
    }
  }
}

__global__ __launch_bounds__(64) void gemm_skinny_reduce_silu_kernel(
    const float* __restrict__ part, uint16_t* __restrict__ Y, int M, int I, int S) {
#pragma clang fp contract(off)  // g / (1 + e^-g) * u in separately rounded steps
  const int c = blockIdx.x * 64 + threadIdx.x, m = blockIdx.y;
  if (c * 32 >= I) return;
  const int64_t plane = (int64_t)M * 2 * I;
  const float* pg = part + (int64_t)m * 2 * I + c * 32;
  float a[32], b[32];
  skinny_sum32(pg, plane, S, a);
  skinny_sum32(pg + I, plane, S, b);
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const float g = h2f(f2h(a[i])), u = h2f(f2h(b[i]));
    a[i] = g / (1.0f + expf(-g)) * u;
  }
  fwht32(a);
  store32h(Y + (int64_t)m * I + c * 32, a);
}

}  // namespace

bool gemm_skinny_ok(int64_t M, int64_t K, int wbits) {
  const int64_t ks = 1024 / (wbits == 4 ? 4 : wbits == 8 ? 8 : 16);  // k per ring step
  return M >= 2 && M <= 16 && K % ks == 0;
}

// Split count of the skinny ring.  A CU streams its workgroups' weight
// tiles at about the same rate whether it holds one or several, so the step
// ends with the most-loaded CU: cost(S) = ceil(ntiles S / CUs) * kps + S,
// the last term charging each split its fp32 partials and share of the
// reduce.  S runs over 1..8 with at most 8 workgroups per CU (past that the
// quantisation the model prices is smoothed out and splitting loses: FP16
// 151936 x 5120 at M = 8, 2 splits 279 us against 268); ties go to more
// splits.  Measured at M = 8 (us, chosen / unsplit / old rule): INT4 o
// 5120 x 5120 3 splits 10.5 / 17.1 / 12.1, qkv 7168 x 5120 2: 12.9 / 17.8,
// gate_up 34816 x 5120 3: 34.8 / 39.4, down 5120 x 17408 3: 23.1 / 51.6 /
// 23.2; INT8 o 3: 11.5 / 18.7 / 13.1, qkv 2: 14.0 / 19.3 / 17.3, down 3:
// 25.7 / 55.1 / 29.9.  S > 1 needs S * M * N fp32 of workspace.
int skinny_splits(int64_t M, int64_t N, int64_t K, int wbits, size_t ws_bytes) {
  constexpr int64_t kCUs = 256;  // MI355X
  const int64_t ntiles = (N + kSkTile - 1) / kSkTile;
  const int64_t kt = K / (1024 / wbits);
  int64_t S = 1, best = INT64_MAX;
  for (int64_t s = 1; s <= std::min<int64_t>(kSkMaxSplits, kt); ++s) {
    const int64_t kps = (kt + s - 1) / s;
    const int64_t se = (kt + kps - 1) / kps;  // splits left non-empty
    if (se > 1 && ntiles * se > 8 * kCUs) break;
    const int64_t c = (ntiles * se + kCUs - 1) / kCUs * kps + se;
    if (c <= best) best = c, S = se;
  }
  if (const int v = tuning().skinny_splits.load()) S = v;  // measurement override (r4q_tune)
  if (S < 2) return 1;
  // every split non-empty
  const int64_t kps = (kt + S - 1) / S;
  S = (kt + kps - 1) / kps;
  if ((size_t)S * M * N * 4 > ws_bytes) return 1;
  return (int)S;
}

size_t skinny_ws_bytes(int64_t M, int64_t N, int64_t K, int wbits) {
  const int S = skinny_splits(M, N, K, wbits, SIZE_MAX);
  return S > 1 ? (size_t)S * M * N * 4 : 0;
}

namespace {
// silu_I > 0: N = 2 silu_I gate/up columns, split (S > 1, checked by the
// caller) and reduced by gemm_skinny_reduce_silu_kernel into y (M x silu_I).
int skinny_run(const void* x, const void* w, const void* sz, void* y, int64_t M, int64_t N,
               int64_t K, int wbits, hipStream_t st, void* ws, size_t ws_bytes, int64_t silu_I) {
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* wp = static_cast<const uint8_t*>(w);
  const auto* sp = static_cast<const uint32_t*>(sz);
  auto* yp = static_cast<uint16_t*>(y);
  const int S = skinny_splits(M, N, K, wbits, ws ? ws_bytes : 0);
  const int64_t ntiles = (N + kSkTile - 1) / kSkTile;
  const int64_t kt = K / (1024 / wbits);
  const int kps = (int)((kt + S - 1) / S);
  float* part = S > 1 ? static_cast<float*>(ws) : nullptr;
  const dim3 grid((unsigned)(ntiles * S));
#define R4Q_SKINNY(WB, MRR)                                                                    \
  hipLaunchKernelGGL((gemm_skinny_kernel<WB, MRR>), grid, dim3(256), 0, st, xp, wp, sp, yp,    \
                     part, (int)M, (int)N, (int)K, (int)ntiles, kps)
  const bool m8 = M <= 8;
  switch (wbits) {
    case 4:
      if (m8) R4Q_SKINNY(4, 8);
      else R4Q_SKINNY(4, 16);
      break;
    case 8:
      if (m8) R4Q_SKINNY(8, 8);
      else R4Q_SKINNY(8, 16);
      break;
    default:
      if (m8) R4Q_SKINNY(16, 8);
      else R4Q_SKINNY(16, 16);
  }
#undef R4Q_SKINNY
  R4Q_TRY(launch_status("gemm_skinny"));
  if (silu_I > 0) {
    hipLaunchKernelGGL(gemm_skinny_reduce_silu_kernel,
                       dim3((unsigned)((silu_I / 32 + 63) / 64), (unsigned)M), dim3(64), 0, st,
                       part, yp, (int)M, (int)silu_I, S);
    R4Q_TRY(launch_status("gemm_skinny_reduce_silu"));
  } else if (S > 1) {
    hipLaunchKernelGGL(gemm_skinny_reduce_kernel, dim3((unsigned)((N + 255) / 256), (unsigned)M),
                       dim3(256), 0, st, part, yp, (int)M, (int)N, S);
    R4Q_TRY(launch_status("gemm_skinny_reduce"));
  }
  return R4Q_OK;
}
}  // namespace

int gemm_skinny_launch(const void* x, const void* w, const void* sz, void* y, int64_t M,
                       int64_t N, int64_t K, int wbits, hipStream_t st, void* ws,
                       size_t ws_bytes) {
  return skinny_run(x, w, sz, y, M, N, K, wbits, st, ws, ws_bytes, 0);
}

bool gemm_skinny_silu_ok(int64_t M, int64_t I, int64_t K, int wbits, size_t ws_bytes) {
  return gemm_skinny_ok(M, K, wbits) && I > 0 && I % 32 == 0 &&
         skinny_splits(M, 2 * I, K, wbits, ws_bytes) > 1;
}

int gemm_skinny_silu_launch(const void* x, const void* w, const void* sz, void* y, int64_t M,
                            int64_t I, int64_t K, int wbits, hipStream_t st, void* ws,
                            size_t ws_bytes) {
  R4Q_REQUIRE(gemm_skinny_silu_ok(M, I, K, wbits, ws ? ws_bytes : 0),
              "gate_up_silu: shape or workspace does not take the split path");
  return skinny_run(x, w, sz, y, M, 2 * I, K, wbits, st, ws, ws_bytes, I);
}

bool gemm_ring_ok(int64_t M, int wbits) { return M >= RBM && wbits != 16; }

// Work split of the ring kernel: `full` tiles computed whole, the other
// nst = tiles - full split S ways along K (kps steps each).
struct RingPlan {
  int full = 0, S = 1, kps = 0, nst = 0;
  size_t ws = 0;  // fp32 partials: S * nst * 256 * 256 * 4 bytes
};

RingPlan ring_plan(int64_t M, int64_t N, int64_t K, size_t ws_bytes) {
  // Estimated time: rounds of one workgroup per CU (256), a whole tile's K
  // loop at ~3.7 TFLOP/s per CU (measured), split tiles taking 1/S of it,
  // plus the partials written and read back at ~5 TB/s.  Candidates: no
  // split; every tile split S ways (few tiles); only the tiles of a last,
  // partial round split S ways (full = the tiles of the complete rounds).
  const int64_t tiles = ((N + RBN - 1) / RBN) * ((M + RBM - 1) / RBM);
  const int64_t nk = K / RBK;
  const double tile_us = 2.0 * RBM * RBN * (double)K / 3.7e6;
  const double part_us = (double)RBM * RBN * 8 / 5e6;  // one partial tile, out and back
  RingPlan best;
  best.full = (int)tiles;
  best.kps = (int)nk;
  double best_us = (double)((tiles + 255) / 256) * tile_us;
  auto consider = [&](int64_t full, int S) {
    const int64_t nst = tiles - full;
    if (S < 2 || nst <= 0 || nk / S < 8) return;
    const size_t ws = (size_t)S * nst * RBM * RBN * 4;
    if (ws > ws_bytes) return;
    const int64_t rounds_full = (full + 255) / 256, rounds_split = (nst * S + 255) / 256;
    const double us = rounds_full * tile_us + rounds_split * tile_us / S + S * nst * part_us;
    if (us < best_us) {
      best_us = us;
      best.full = (int)full;
      best.S = S;
      best.nst = (int)nst;
      best.ws = ws;
    }
  };
  for (int S = 2; S <= kMaxGemmSplits; ++S) {
    consider(0, S);
    if (tiles > 256 && tiles % 256) consider(tiles - tiles % 256, S);
  }
  if (const int v = tuning().gemm_splits.load()) {  // measurement override: every tile split
    const size_t ws = (size_t)v * tiles * RBM * RBN * 4;
    if (v >= 2 && v <= kMaxGemmSplits && nk / v >= 1 && ws <= ws_bytes) {
      best.full = 0;
      best.S = v;
      best.nst = (int)tiles;
      best.ws = ws;
    } else if (v == 1) {
      best = RingPlan();
      best.full = (int)tiles;
    }
  }
  best.kps = best.S > 1 ? (int)((nk + best.S - 1) / best.S) : (int)nk;
  if (best.S > 1) best.S = (int)((nk + best.kps - 1) / best.kps);  // every split non-empty
  if (best.S == 1) {
    best.full = (int)tiles;
    best.nst = 0;
    best.ws = 0;
  } else {
    best.ws = (size_t)best.S * best.nst * RBM * RBN * 4;
  }
  return best;
}

int gemm_splits(int64_t M, int64_t N, int64_t K, int wbits, size_t ws_bytes) {
  return gemm_ring_ok(M, wbits) ? ring_plan(M, N, K, ws_bytes).S : 1;
}

size_t gemm_ws_bytes(int64_t M, int64_t N, int64_t K, int wbits) {
  return gemm_ring_ok(M, wbits) ? ring_plan(M, N, K, (size_t)-1).ws : 0;
}

int gemm_mfma_launch(const void* x, const void* w, const void* sz, void* y, int64_t M, int64_t N,
                     int64_t K, int wbits, hipStream_t st, void* ws, size_t ws_bytes) {
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* wp = static_cast<const uint8_t*>(w);
  const auto* sp = static_cast<const uint32_t*>(sz);
  auto* yp = static_cast<uint16_t*>(y);
  if (gemm_ring_ok(M, wbits)) {
    const RingPlan pl = ring_plan(M, N, K, ws ? ws_bytes : 0);
    float* part = pl.S > 1 ? static_cast<float*>(ws) : nullptr;
    const unsigned blocks = (unsigned)(pl.full + (int64_t)pl.nst * pl.S);
    if (wbits == 4)
      hipLaunchKernelGGL(gemm_ring_kernel<4>, dim3(blocks), dim3(kRingThreads), 0, st, xp, wp, sp,
                         yp, part, (int)M, (int)N, (int)K, pl.full, pl.S, pl.kps);
    else
      hipLaunchKernelGGL(gemm_ring_kernel<8>, dim3(blocks), dim3(kRingThreads), 0, st, xp, wp, sp,
                         yp, part, (int)M, (int)N, (int)K, pl.full, pl.S, pl.kps);
    R4Q_TRY(launch_status("gemm_ring"));
    if (pl.S > 1) {
      hipLaunchKernelGGL(gemm_splitk_reduce_kernel, dim3((unsigned)(pl.nst * RBM)), dim3(256), 0,
                         st, part, yp, (int)M, (int)N, pl.full, pl.nst, pl.S);
      R4Q_TRY(launch_status("gemm_splitk_reduce"));
    }
    return R4Q_OK;
  }
  const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
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
