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
//  * gemm_ring_kernel (M >= 256, INT4 / INT8 / FP16): 256 x 256 tiles, X
//    and the raw weights copied global -> LDS through a ring, the weights
//    dequantised per wave in registers (FP16: read as they are), the K
//    units of the tiles beyond the full rounds of 256 shared evenly by the
//    CUs (stream-K) or, with at most 128 tiles, each tile split into equal
//    pieces (deterministic reduce over a caller workspace; see its comment);
//  * gemm_mfma_kernel (17 <= M < 256): 128 x 128 tiles, X and the
//    dequantised W staged in LDS per 32-wide K step;
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

// (1024 + q_2p, 1024 + q_2p+1) as an fp16 pair from byte p of a packed INT4
// word w (w4 = w >> 4): v_perm puts byte p of w in byte 0 and byte p of w4 in
// byte 2, one v_and_or keeps the low nibbles and sets the 0x64 exponent bytes
// (written out: with two literal operands, which VOP3 cannot encode on this
// target, the compiler emits a separate AND and OR).
__device__ __forceinline__ uint32_t nib_pair(uint32_t w, uint32_t w4, int p) {
  const uint32_t t = __builtin_amdgcn_perm(w4, w, (uint32_t)(p | (p + 4) << 16));
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(t), "s"(0x000F000Fu), "v"(0x64006400u));
  return r;
}

// ---------------------------------------------------------------------
// Weight fragments of the skinny GEMM (below).  The MFMA contraction index k
// is only a label: lane group g's 8 k-slots of an MFMA carry 8 weight
// elements, and the A fragment of that lane group holds the activation
// values of exactly those elements.  Because the weights are fully
// dequantised before the MFMA -- fp16((q - zp) * s) by an exact packed fp16
// subtraction and one rounded packed multiply, bit-identical to the dequant
// kernel -- the accumulation may run across blocks.
//   INT4: 4 MFMAs per 16 weight bytes; the nibble pair (q_2j, q_2j+1) of
//         byte j of a word w is byte j of w and of w >> 4 (v_perm), masked
//         and tagged 0x6400 in one v_and_or: natural k order, so the
//         activation is used as loaded;
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
      const uint32_t wd = w[d], wd4 = wd >> 4;
#pragma unroll
      for (int p = 0; p < 4; ++p) pr[p] = nib_pair(wd, wd4, p);
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
// Prefill GEMM for M >= 256 with INT4 / INT8 / FP16 weights: a workgroup of 4 waves
// (one per SIMD) owns a 256 x 256 output tile, each wave 256 rows x 64
// columns (16 x 4 MFMA tiles, 256 fp32 accumulators per lane, in AGPRs).
// The K loop of the 128 x 128 kernel above is bound by global-load latency
// (one 32-wide K step in flight, ~1.3 us per step on MI355X); here the
// operands arrive through LDS rings filled by direct global->LDS copies, so
// that several steps are in flight without holding them in VGPRs.
// X of a K step (16 KB) lands in LDS by direct global->LDS copies
// (global_load_lds_dwordx4) in a ring of kXStages stages; the raw weights
// and their (scale, zero) words arrive per super-step of Ring::KS K steps
// (128 bytes of each weight row: whole cache lines, where one step's 16 / 32
// bytes of 256 rows would touch 256 lines per step) into two alternating
// buffers, requested a super-step ahead.
// Each wave dequantises its own B fragments straight from the raw bytes in
// LDS into registers (one 4-byte INT4 / 8-byte INT8 read per fragment
// instead of 16 bytes of fp16), one step ahead, interleaved with the MFMAs
// of the current step; the fp16 values equal r4q_dequant_int4/8 bit for bit.
// FP16 weights have no super-steps: each X stage also holds the step's 64
// bytes of the 256 weight rows, laid out like X, and the B fragments are
// read from it like X fragments.
// Each X fragment register is refilled with the next step's fragment right
// after its MFMAs, so that each step starts its MFMAs without waiting for LDS.
// LDS layouts are bank-conflict-free for their fragment reads (measured on
// MI355X with a read-throughput probe):
//  * X rows are 64 bytes per step; the 16-byte piece p of row r sits in slot
//    p ^ ((r >> 1) & 3) of the row;
//  * weight rows are 128 bytes per super-step; chunk q (16 bytes) of row r
//    sits in slot q ^ wswz(r);
//  * scale words are in natural order (rows 8 apart share a bank: a 2-way
//    conflict on 4 of the 12 reads per step).
// One barrier per K step i: before it each wave waits for its own copies of
// step i+1; after it every wave's copies are visible and every wave is done
// with step i-1, whose X stage then receives step i+kXStages-1.  Every
// wave issues the same number of copies per step position (the wait counts
// are per wave).
// Work split: tiles of 256 x 256 outputs, each a K loop of U units (one
// unit = one weight super-step, below).  Blocks [0, dp) compute tiles
// 0 .. dp-1 whole.  The sk stream-K workgroups share the units of tiles
// dp .. T-1 evenly: workgroup w takes the flattened units
// [floor(w * TU / sk), floor((w + 1) * TU / sk)) (TU = (T - dp) * U), i.e. the
// tail of one tile, whole tiles, the head of another.  A tile done by one
// workgroup is written as fp16 directly; a tile shared by several writes one
// fp16 partial per workgroup (segment j = w - the first workgroup on the
// tile; fp16 halves the partial traffic, written and read back, at one
// extra rounding of each segment's sum) and gemm_splitk_reduce_kernel sums
// them in fp32 in segment order, so the result does not depend on timing.
constexpr int RBM = 256, RBN = 256, RBK = 32;
constexpr int kRingWaves = 4;  // one per SIMD; wave w owns output columns 64w .. 64w+63
constexpr int kRingThreads = 64 * kRingWaves;
constexpr int kRingRows = RBM / kRingWaves;  // rows of X / W each wave copies
constexpr int kXStages = 4;                   // X ring depth (one K step per stage)

template <int WBITS>
struct Ring {
  static constexpr bool kF16 = WBITS == 16;
  // K steps per weight super-step: 128 bytes of every weight row, fetched
  // as whole cache lines (INT4: 8 steps of 16 bytes, INT8: 4 of 32).  FP16
  // weights (64 bytes per row and step) travel with X instead: each X stage
  // holds the step's X (16 KB) and its weights (16 KB).
  static constexpr int KS = WBITS == 4 ? 8 : WBITS == 8 ? 4 : 1;
  static constexpr int kXPart = RBM * RBK * 2;          // X of a step: 16 KB
  static constexpr int kX = kF16 ? 2 * kXPart : kXPart;  // one X stage
  static constexpr int kW = kF16 ? 0 : RBN * 128;        // one super-step of raw weights: 32 KB
  static constexpr int kS = kF16 ? 0 : RBN * KS * 4;     // its (scale, zero) words: 8 KB / 4 KB
  static constexpr int kWOff = kXStages * kX;  // two weight buffers follow the X stages
  static constexpr int kSOff = kWOff + 2 * kW;
  static constexpr int kBytes = kSOff + 2 * kS;  // 144 KB / 136 KB / 128 KB
  // copies per wave per X stage (FP16: X and weights)
  static constexpr int kXCopies = (kF16 ? 2 : 1) * (kRingRows / 16);
  // per wave per super-step: weights (8 rows per copy), scale words
  static constexpr int kWCopies = kF16 ? 0 : kRingRows / 8 + kRingRows * KS / 64;
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
// LDS-qualified byte pointer: ring addresses stay 32-bit LDS offsets (a
// generic pointer into LDS is a 64-bit value the compiler keeps in VGPRs).
typedef __attribute__((address_space(3))) uint8_t lds8;
template <class T>
__device__ __forceinline__ T lds_ld(const lds8* p) {
  return *(const __attribute__((address_space(3))) T*)p;
}
__device__ __forceinline__ uint32_t lds_off(const lds8* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)p);
}

// The same with a uniform 64-bit base in SGPRs and a 32-bit byte offset
// per lane (half the VGPRs of a per-lane address).
__device__ __forceinline__ void copy16s(const void* base, uint32_t off, lds8* lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_off(lds)),
               "v"(off), "s"(base)
               : "memory");
}
__device__ __forceinline__ void copy4s(const void* base, uint32_t off, lds8* lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, %2" ::"s"(lds_off(lds)),
               "v"(off), "s"(base)
               : "memory");
}

// X of K step kb (32 elements) of the workgroup's 256 rows into one X stage;
// rows past M are clamped into the matrix (computed, never stored).  Wave w
// copies rows kRingRows w .. (16 rows x 64 bytes per copy); the 16-byte
// pieces of a row are XOR-swizzled by (row >> 1) & 3 so that the fragment
// reads are free of bank conflicts.
__device__ __forceinline__ void x_issue(lds8* xs, const uint16_t* __restrict__ X, int M, int K,
                                        int m0, int kb, int wave, int lane) {
#pragma unroll
  for (int q = 0; q < kRingRows / 16; ++q) {
    const int r0 = kRingRows * wave + 16 * q;  // first row of this copy
    const int row = r0 + (lane >> 2);
    const int p = (lane & 3) ^ ((row >> 1) & 3);  // global piece held by LDS slot lane & 3
    const int m = min(m0 + row, M - 1);
    copy16s(X, 2u * ((uint32_t)m * K + kb * RBK + 8 * p), xs + r0 * 64);
  }
}

// FP16 weights of K step kb (64 bytes of each of the workgroup's 256 rows)
// into the second half of an X stage, laid out like X.
__device__ __forceinline__ void w16_issue(lds8* xs, const uint8_t* __restrict__ W, int N, int K,
                                          int n0, int kb, int wave, int lane) {
#pragma unroll
  for (int q = 0; q < kRingRows / 16; ++q) {
    const int r0 = kRingRows * wave + 16 * q;
    const int row = r0 + (lane >> 2);
    const int p = (lane & 3) ^ ((row >> 1) & 3);
    const uint32_t n = min(n0 + row, N - 1);
    copy16s(W, 2u * (n * (uint32_t)K + kb * RBK + 8 * p), xs + RBM * RBK * 2 + r0 * 64);
  }
}

// 16-byte chunk swizzle of weight row r in a super-step buffer (128 bytes
// per row): chunk q of the row sits at slot q ^ wswz(r).  With it the 16
// rows a fragment read touches (rows c = 0 .. 15 of a 16-row block, each
// lane group g reading dword g of its chunk) fall on 64 different banks.
__device__ __forceinline__ int wswz(int r) { return (r & 7) ^ ((r >> 3) & 1); }

// Weights and (scale, zero) words of the super-step starting at K step kb
// for the workgroup's 256 weight rows (rows past N clamped into the matrix,
// steps past K clamped to its last step: their data is never multiplied).
// Weights: wave w copies rows kRingRows w .., 8 rows x 128 bytes per copy
// (whole cache lines).  Scale words in natural order: INT4 8 per row (32
// bytes), INT8 4 per row (16 bytes).  Byte offsets fit 32 bits (checked by
// the host).
template <int WBITS>
__device__ __forceinline__ void w_issue(lds8* wb, lds8* sb, const uint8_t* __restrict__ W,
                                        const uint32_t* __restrict__ SZ, int N, int K, int n0,
                                        int kb, int wave, int lane) {
  const int nks = K / RBK;
  const uint32_t ksz = K / 32;  // scale words per row
#pragma unroll
  for (int q = 0; q < kRingRows / 8; ++q) {
    const int r0 = kRingRows * wave + 8 * q;
    const int r = r0 + (lane >> 3);
    const int qg = (lane & 7) ^ wswz(r);  // chunk of the row this lane fetches
    const uint32_t n = min(n0 + r, N - 1);
    uint32_t off;
    if constexpr (WBITS == 4)
      off = n * (uint32_t)(K / 2) + (uint32_t)min(kb + qg, nks - 1) * 16u;
    else
      off = n * (uint32_t)K + (uint32_t)min(kb + (qg >> 1), nks - 1) * 32u + 16u * (qg & 1);
    copy16s(W, off, wb + r0 * 128);
  }
  constexpr int WPR = WBITS == 4 ? 8 : 4;   // scale words per row and super-step
  constexpr int RPC = 64 / WPR;             // rows per copy
#pragma unroll
  for (int q = 0; q < kRingRows / RPC; ++q) {
    const int r0 = kRingRows * wave + RPC * q;
    const uint32_t n = min(n0 + r0 + lane / WPR, N - 1);
    copy4s(SZ, 4u * (n * ksz + (uint32_t)min(kb + lane % WPR, nks - 1)), sb + r0 * WPR * 4);
  }
}

// B fragments of one K step for a wave: fragment j is column c of the
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
__device__ __forceinline__ void frag_dequant(const BRaw<WBITS>& r, h8_t* bf) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t sb = r.s2[j] & 0xFFFFu, zb = r.s2[j] >> 16;
    const h2_t sc = as_h2(sb | (sb << 16));
    const h2_t nz = -(as_h2(0x64006400u) + as_h2(zb | (zb << 16)));  // -(1024 + zp), exact
    uint32_t pr[4];  // (1024 + q_2k, 1024 + q_2k+1) as fp16 pairs
    if constexpr (WBITS == 4) {
      const uint32_t w4 = r.w[j][0] >> 4;
#pragma unroll
      for (int k = 0; k < 4; ++k) pr[k] = nib_pair(r.w[j][0], w4, k);
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

// Pair k (k labels 8g + 2k, 8g + 2k + 1) of B fragment j, the same
// arithmetic as frag_dequant, so that the dequantisation can be spread over
// a step's MFMAs one pair at a time.  nz / sc / w4: fragment j's
// -(1024 + zp) and scale pairs and (INT4) its word shifted by 4, set by the
// pair-0 call.
template <int WBITS>
__device__ __forceinline__ uint32_t dq_pair(const BRaw<WBITS>& r, int j, int k, h2_t& nz,
                                            h2_t& sc, uint32_t& w4) {
  if (k == 0) {
    const uint32_t sb = r.s2[j] & 0xFFFFu, zb = r.s2[j] >> 16;
    sc = as_h2(sb | (sb << 16));
    nz = -(as_h2(0x64006400u) + as_h2(zb | (zb << 16)));  // -(1024 + zp), exact
    if constexpr (WBITS == 4) w4 = r.w[j][0] >> 4;
  }
  uint32_t pr;
  if constexpr (WBITS == 4) {
    pr = nib_pair(r.w[j][0], w4, k);
  } else {
    pr = __builtin_amdgcn_perm(r.w[j][k >> 1], 0x64646464u, (k & 1) ? 0x00070006u : 0x00050004u);
  }
  return as_u32((as_h2(pr) + nz) * sc);
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

// Stream-K bookkeeping shared by the GEMM and the reduce: first unit of
// workgroup w, and the workgroup holding unit u.
__device__ __forceinline__ int64_t sk_lo(int w, int64_t TU, int sk) {
  return (int64_t)w * TU / sk;
}
__device__ __forceinline__ int sk_owner(int64_t u, int64_t TU, int sk) {
  int w = (int)(u * sk / TU);
  while (w + 1 < sk && sk_lo(w + 1, TU, sk) <= u) ++w;
  while (w > 0 && sk_lo(w, TU, sk) > u) --w;
  return w;
}

// One segment of a tile: K steps [kb0, kb0 + nk) (kb0 a multiple of KS) of
// the 256 x 256 tile at (m0, n0), accumulated into acc.  Wave w computes
// all 256 rows x columns 64w .. 64w+63: 16 x 4 MFMA tiles, 256 fp32
// accumulators per lane, so that each weight column is dequantised once per
// workgroup.  Per step the workgroup waits for its copies of the next step,
// passes one barrier and issues the copies of step + kXStages - 1 (and, at a
// super-step's first step, the weights of the super-step after next); each
// wave then requests the raw B fragments of step + 2 and walks its 16 X
// fragments: 4 MFMAs each, after which the fragment register is refilled
// with the next step's fragment (so every read has a step of MFMAs to land),
// with the next step's B dequantised in between.
// Copies retire in issue order, so one count per step position covers the
// weights as well: they were issued before the X stage being waited for.
template <int WBITS>
struct RingSeg {
  using R = Ring<WBITS>;
  static constexpr int KS = R::KS;
  lds8* ring;
  const uint16_t* X;
  const uint8_t* W;
  const uint32_t* SZ;
  int M, N, K, m0, n0, kb0, nk, wave, lane, wn, c, g, hc, xoff;

  // copies issued after those of X step i+1 when step i waits: the X
  // stages of the steps in between, and a super-step's weights when step
  // i-1 began one (position 1)
  static constexpr int kAfter = R::kXCopies * (kXStages - 3);

  __device__ __forceinline__ lds8* xst(int i) const { return ring + (i % kXStages) * R::kX; }
  __device__ __forceinline__ lds8* wbuf(int s) const { return ring + R::kWOff + (s & 1) * R::kW; }
  __device__ __forceinline__ lds8* sbuf(int s) const { return ring + R::kSOff + (s & 1) * R::kS; }

  __device__ __forceinline__ void issue_x(int i) {
    const int kb = kb0 + min(i, nk - 1);
    x_issue(xst(i), X, M, K, m0, kb, wave, lane);
    if constexpr (R::kF16) w16_issue(xst(i), W, N, K, n0, kb, wave, lane);
  }
  __device__ __forceinline__ void issue_w(int s) {
    if constexpr (!R::kF16)
      w_issue<WBITS>(wbuf(s), sbuf(s), W, SZ, N, K, n0, kb0 + s * KS, wave, lane);
  }
  // FP16 B fragment j of step i: read like an X fragment (rows wn + 16 j + c)
  __device__ __forceinline__ h8_t b16(int i, int j) const {
    return lds_ld<h8_t>(xst(i) + R::kXPart + xoff + wn * 64 + 1024 * j);
  }

  // B fragments of step i (raw reads): position i % KS of super-step i / KS
  __device__ __forceinline__ void load_b(int i, BRaw<WBITS>& r) const {
    if constexpr (R::kF16) return;
    const int s = i / KS, pos = i % KS;
    const lds8* wb = wbuf(s);
    const lds8* sb = sbuf(s) + 4 * pos;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int row = wn + 16 * j + c;  // wswz(row) = wswz(c)
      if constexpr (WBITS == 4) {
        r.w[j][0] = lds_ld<uint32_t>(wb + row * 128 + ((pos << 4) ^ hc) + 4 * g);
        r.s2[j] = lds_ld<uint32_t>(sb + row * 32);
      } else {
        const u2_t v =
            lds_ld<u2_t>(wb + row * 128 + (((2 * pos + (g >> 1)) << 4) ^ hc) + 8 * (g & 1));
        r.w[j][0] = v[0];
        r.w[j][1] = v[1];
        r.s2[j] = lds_ld<uint32_t>(sb + row * 16);
      }
    }
  }

  // Step i; the position in the super-step is a wave-uniform runtime value
  // (an unrolled super-step keeps every position's LDS offsets in VGPRs).
  // Entering: af = step i's X fragments, bf = step i's B (dequantised),
  // rb1 = step i+1's raw B.  Leaving: af = step i+1's X, bf = step i+1's B,
  // rb1 = step i+2's raw B (read two steps ahead, so that the dequantisation
  // has its inputs in registers and can run between the MFMAs).
  __device__ __forceinline__ void step(int i, f4_t (&acc)[16][4], h8_t (&af)[16], h8_t (&bf)[4],
                                       BRaw<WBITS>& rb1) {
    const int pos = i % KS;
    if (pos == 1)  // this wave's copies of step i+1 landed
      wait_copies<kAfter + R::kWCopies>();
    else
      wait_copies<kAfter>();
    ring_barrier();  // everyone's; and every read of step i-1's stage is done
    if (pos == 0) issue_w(i / KS + 1);
    issue_x(i + kXStages - 1);
    BRaw<WBITS> rb2;
    load_b(i + 2, rb2);
    __builtin_amdgcn_sched_barrier(0);
    // 16 groups: 4 MFMAs of X fragment i8, its refill with the next step's
    // fragment, and pair i8 % 4 of the next step's B fragment i8 / 4
    u4_t bw[4];
    h2_t nz, sc;
    uint32_t w4 = 0;
    const lds8* xn = xst(i + 1) + xoff;
#pragma unroll
    for (int i8 = 0; i8 < 16; ++i8) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i8][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i8], bf[j], acc[i8][j], 0, 0, 0);
      af[i8] = lds_ld<h8_t>(xn + 1024 * i8);
      if constexpr (R::kF16) {  // the next step's fragment j = i8 (groups 0-3)
        if (i8 < 4) bw[i8] = __builtin_bit_cast(u4_t, b16(i + 1, i8));
      } else {
        bw[i8 >> 2][i8 & 3] = dq_pair<WBITS>(rb1, i8 >> 2, i8 & 3, nz, sc, w4);
        // consumed here, so that the pair is computed inside its group
        asm volatile("" ::"v"(bw[i8 >> 2][i8 & 3]));
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    h8_t bn[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) bn[j] = __builtin_bit_cast(h8_t, bw[j]);
#pragma unroll
    for (int j = 0; j < 4; ++j) bf[j] = bn[j];
    rb1 = rb2;
  }

  // the segment's first copies: super-step 0's weights, X steps 0 .. kXStages-2
  __device__ __forceinline__ void start() {
    issue_w(0);
#pragma unroll
    for (int s = 0; s < kXStages - 1; ++s) issue_x(s);
  }

  // the segment's K loop, after start(); nothing else may have been issued
  // to global memory since start() but stores (they retire before the count
  // below is reached only if they were issued earlier, which costs time, not
  // correctness)
  __device__ void run(f4_t (&acc)[16][4]) {
    wait_copies<R::kXCopies * (kXStages - 2)>();  // X step 0 (and the weights) landed
    ring_barrier();
    h8_t af[16], bf[4];
#pragma unroll
    for (int i8 = 0; i8 < 16; ++i8) af[i8] = lds_ld<h8_t>(xst(0) + xoff + 1024 * i8);
    BRaw<WBITS> rb1;
    if constexpr (R::kF16) {
#pragma unroll
      for (int j = 0; j < 4; ++j) bf[j] = b16(0, j);
    } else {
      BRaw<WBITS> r0;
      load_b(0, r0);
      frag_dequant<WBITS>(r0, bf);
      load_b(1, rb1);  // step 1 is in super-step 0 (KS >= 4)
    }
    for (int i = 0; i < nk; ++i) step(i, acc, af, bf, rb1);
    wait_copies<0>();  // no copy may land after the ring is reused or released
    ring_barrier();    // every wave's last fragment reads done before the next segment
  }
};

template <int WBITS>
__global__ __launch_bounds__(kRingThreads, 1) void gemm_ring_kernel(
    const uint16_t* __restrict__ X, const uint8_t* __restrict__ W,
    const uint32_t* __restrict__ SZ, uint16_t* __restrict__ Y, uint16_t* __restrict__ part, int M,
    int N, int K, int dp, int sk, int U, int maxseg) {
  using R = Ring<WBITS>;
  __shared__ __align__(16) uint8_t ring[R::kBytes];
  RingSeg<WBITS> sg;
  // the ring's base as a value the compiler cannot see: it is LDS address 0,
  // and with that known the per-stage offsets become per-lane registers
  // instead of immediate offsets of the LDS reads
  lds8* rb = (lds8*)ring;
  asm volatile("" : "+s"(rb));
  sg.ring = rb;
  sg.X = X;
  sg.W = W;
  sg.SZ = SZ;
  sg.M = M;
  sg.N = N;
  sg.K = K;
  const int t = threadIdx.x;
  sg.lane = t & 63;
  sg.wave = t >> 6;
  sg.wn = sg.wave * 64;
  sg.c = sg.lane & 15;
  sg.g = sg.lane >> 4;
  sg.hc = wswz(sg.c) << 4;
  // fragment i8 of a stage: rows 16 i8 + c, k labels 8g .. 8g+7 (piece g of
  // the row, swizzled by (row >> 1) & 3 = (c >> 1) & 3) at xoff + 1024 i8
  sg.xoff = sg.c * 64 + 16 * (sg.g ^ ((sg.c >> 1) & 3));
  const int ntn = (N + RBN - 1) / RBN;
  const int tiles = ntn * ((M + RBM - 1) / RBM);
  const int nks = K / RBK;
  const int b = blockIdx.x;
  // unit range over the flattened (tile, unit) space of this block
  int64_t lo, hi, TU = 0;
  int w = 0;
  if (b < dp) {
    lo = (int64_t)b * U;
    hi = lo + U;
  } else {
    // stream-K workgroup; consecutive workgroups (adjacent units, shared
    // tiles and X rows) are placed on one XCD (blocks go to XCDs round-robin)
    const int bb = b - dp;
    w = (sk % 8 == 0) ? (b % 8) * (sk / 8) + bb / 8 : bb;
    TU = (int64_t)(tiles - dp) * U;
    lo = (int64_t)dp * U + sk_lo(w, TU, sk);
    hi = (int64_t)dp * U + sk_lo(w + 1, TU, sk);
  }
  // segment starting at unit u: sets the ring's tile and K range
  auto set_seg = [&](int64_t u, int64_t& ue, int& ua, int& ub, int& tile) {
    tile = (int)(u / U);
    ue = min(hi, (int64_t)(tile + 1) * U);
    ua = (int)(u - (int64_t)tile * U);
    ub = (int)(ue - (int64_t)tile * U);
    sg.m0 = (tile / ntn) * RBM;
    sg.n0 = (tile % ntn) * RBN;
    sg.kb0 = ua * R::KS;
    sg.nk = min(ub * R::KS, nks) - sg.kb0;
  };
  int64_t u = lo, ue = lo;
  int ua = 0, ub = 0, tile = 0;
  if (u < hi) {
    set_seg(u, ue, ua, ub, tile);
    sg.start();
  }
  while (u < hi) {
    f4_t acc[16][4];
#pragma unroll
    for (int i = 0; i < 16; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};
    sg.run(acc);
    const int ctile = tile, cm0 = sg.m0, cn0 = sg.n0;
    const bool whole = ua == 0 && ub == U;
    // the next segment's first copies go out before this one's results
    u = ue;
    if (u < hi) {
      set_seg(u, ue, ua, ub, tile);
      sg.start();
    }
    // The lane index is re-read through an empty asm so that the compiler
    // does not keep the store offsets live across the segment loop.
    int tq = t;
    asm volatile("" : "+v"(tq));
    if (!whole) {
      // fp16 partial in the accumulator layout: the 8 values of N-blocks
      // 2 jp and 2 jp + 1 of (wave, i8, lane) as one 16-byte piece at
      // ((wave * 16 + i8) * 2 + jp) * 64 + lane (1 KB per wave
      // instruction); gemm_splitk_reduce_kernel reads the same layout
      const int tl = ctile - dp;
      const int j = w - sk_owner((int64_t)tl * U, TU, sk);
      u4_t* pt = reinterpret_cast<u4_t*>(part + ((int64_t)tl * maxseg + j) * (RBM * RBN));
      pt += (tq >> 6) * (16 * 2 * 64) + (tq & 63);
#pragma unroll
      for (int i8 = 0; i8 < 16; ++i8)
#pragma unroll
        for (int jp = 0; jp < 2; ++jp) {
          const f4_t a = acc[i8][2 * jp], c = acc[i8][2 * jp + 1];
          pt[(i8 * 2 + jp) * 64] = u4_t{cvt_pk_h(a[0], a[1]), cvt_pk_h(a[2], a[3]),
                                        cvt_pk_h(c[0], c[1]), cvt_pk_h(c[2], c[3])};
        }
    } else {
      // C fragment: lane holds rows 4g + r of an M-block, column c of an N-block
      const int ec = tq & 15, eg = (tq >> 4) & 3, ewn = (tq >> 6) * 64;
#pragma unroll
      for (int i8 = 0; i8 < 16; ++i8)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int col = cn0 + ewn + 16 * jj + ec;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = cm0 + 16 * i8 + 4 * eg + r;
            if (row < M && col < N) Y[(int64_t)row * N + col] = f2h(acc[i8][jj][r]);
          }
        }
    }
  }
}

// Y = fp16(sum over the segments of each shared tile, in segment order, in
// fp32).  Partials are fp16 in the accumulator layout of gemm_ring_kernel
// (16-byte pieces of (wave, i8, jp, lane): N-blocks 2 jp and 2 jp + 1 of a
// lane); a thread takes lanes 16g + 4q .. + 3 of one (wave, i8, jp) -- 64
// contiguous bytes, rows 16 i8 + 4g .. + 3 x columns 64 wave + 16 j + 4q ..
// + 3 for j = 2 jp, 2 jp + 1 -- and writes 4 x 8 outputs.  The loads of up
// to 4 segments are in flight before they are added in order.
constexpr int kRedThreadsPerTile = RBM * RBN / 32;
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const uint16_t* __restrict__ part,
                                                                 uint16_t* __restrict__ Y, int M,
                                                                 int N, int dp, int sk, int U,
                                                                 int maxseg) {
  const int gt = blockIdx.x * 256 + threadIdx.x;
  const int tl = gt / kRedThreadsPerTile, x = gt % kRedThreadsPerTile;
  const int q = x & 3, g = (x >> 2) & 3, jp = (x >> 4) & 1, i8 = (x >> 5) & 15, wv = x >> 9;
  const int ntn = (N + RBN - 1) / RBN;
  const int tiles = ntn * ((M + RBM - 1) / RBM);
  const int64_t TU = (int64_t)(tiles - dp) * U;
  const int w0 = sk_owner((int64_t)tl * U, TU, sk);
  const int w1 = sk_owner((int64_t)tl * U + U - 1, TU, sk);
  if (w1 == w0) return;  // written whole by one workgroup
  const int tile = dp + tl;
  const int row0 = (tile / ntn) * RBM + 16 * i8 + 4 * g;
  const int colb = (tile % ntn) * RBN + 64 * wv + 32 * jp + 4 * q;  // N-block 2 jp
  if (row0 >= M || colb >= N) return;
  const int nseg = w1 - w0 + 1;
  const u4_t* p = reinterpret_cast<const u4_t*>(part + (int64_t)tl * maxseg * (RBM * RBN)) +
                  ((wv * 16 + i8) * 2 + jp) * 64 + 16 * g + 4 * q;
  constexpr int64_t kSeg = RBM * RBN / 8;  // 16-byte pieces per segment
  // v[b][l][r]: N-block 2 jp + b, column 4q + l, row 4g + r
  float v[2][4][4];
  auto add = [&](const u4_t (&t)[4], bool first) {
#pragma unroll
    for (int l = 0; l < 4; ++l)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t wd = t[l][2 * b + h];
          const float lo = h2f((uint16_t)(wd & 0xFFFFu)), hi = h2f((uint16_t)(wd >> 16));
          v[b][l][2 * h] = first ? lo : v[b][l][2 * h] + lo;
          v[b][l][2 * h + 1] = first ? hi : v[b][l][2 * h + 1] + hi;
        }
  };
  {
    u4_t t[4];
#pragma unroll
    for (int l = 0; l < 4; ++l) t[l] = p[l];
    add(t, true);
  }
  for (int j0 = 1; j0 < nseg; j0 += 4) {
    u4_t t[4][4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int l = 0; l < 4; ++l) t[s][l] = p[(int64_t)min(j0 + s, nseg - 1) * kSeg + l];
#pragma unroll
    for (int s = 0; s < 4; ++s)
      if (j0 + s < nseg) add(t[s], false);
  }
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int col0 = colb + 16 * b;
    if (col0 >= N) break;
    const bool vec = col0 + 4 <= N && (N & 3) == 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (row0 + r >= M) break;
      uint16_t* y = Y + (int64_t)(row0 + r) * N + col0;
      if (vec) {
        const uint32_t lo = (uint32_t)f2h(v[b][0][r]) | ((uint32_t)f2h(v[b][1][r]) << 16);
        const uint32_t hi = (uint32_t)f2h(v[b][2][r]) | ((uint32_t)f2h(v[b][3][r]) << 16);
        *reinterpret_cast<u2_t*>(y) = u2_t{lo, hi};
      } else {
#pragma unroll
        for (int l = 0; l < 4; ++l)
          if (col0 + l < N) y[l] = f2h(v[b][l][r]);
      }
    }
  }
}

// ---------------------------------------------------------------------
// Prefill GEMM with specialised waves (INT4, M >= 256, N % 128 == 0,
// K % 256 == 0; selected by the gemm_kernel knob, see use_spec for how it
// measures against the ring kernel).  A workgroup of 8 waves owns a 256 x
// 128 output tile:
//  * waves 0-3 ("MFMA waves") copy X of every K step global -> LDS
//    (global_load_lds, 64 rows each) and otherwise only read fragments from
//    LDS and issue MFMAs: wave c computes rows 128 (c >> 1) .. +127 x
//    columns 64 (c & 1) .. +63 (8 x 4 v_mfma_f32_16x16x32_f16 tiles, 128
//    fp32 accumulators per lane);
//  * waves 4-7 ("dequantisation waves") copy the raw weights and (scale,
//    zero) words of every super-step of 8 K steps (128 bytes of each weight
//    row: whole cache lines) global -> LDS, and dequantise: each lane turns
//    half a row's 32-element block of K step g + 3 into fp16 in a ring of B
//    stages, from raw bytes it read from LDS in the step before (its own
//    wave's copies: rows 32 p .. 32 p + 31 of wave p).
// Waves c and c + 4 share a SIMD, so the dequantisation of one runs while
// the other's MFMAs execute instead of serialising with them in one wave.
// One barrier per K step for all 8 waves; the ring stages are indexed by
// the workgroup's running K step, so the pipeline runs on across the tiles
// of a stream-K range.  Invariants (barrier B_g opens step g):
//  * X and B of step g + 1 are complete at B_g (the MFMA waves read them
//    during step g); X copies of step g + 4 go out in step g into the stage
//    step g used; B of step g + 3 is written in step g into the stage of
//    step g - 1 and waited for one step later (its consumers read it after
//    B_g+2);
//  * the raw weights of super-step s + 1 go out in step 8 s - 4, after the
//    last raw read of the buffer they replace (super-step s - 1), and are
//    waited for in step 8 s + 4, before the first read of their own.
// The dequantised values equal r4q_dequant_int4 bit for bit and every
// output element sees the same MFMA sequence as in gemm_ring_kernel, so
// whole tiles are bit-identical to it.  Shared tiles leave fp16 partials in
// the accumulator layout, summed by gemm_spec_reduce_kernel in segment
// order.
constexpr int SBM = 256, SBN = 128;
constexpr int kSpecWaves = 8;  // 4 MFMA waves, then 4 dequantisation waves
constexpr int kSpecThreads = 64 * kSpecWaves;
constexpr int kSpecKS = 8;     // K steps per weight super-step (INT4: 128 bytes of a row)
constexpr int kSpecXSt = 4;    // X stages: copies of step g + 4 issued in step g
constexpr int kSpecBSt = 4;    // dequantised B stages: step g + 3 written in step g
struct SpecRing {
  static constexpr int kX = SBM * RBK * 2;             // 16 KB
  static constexpr int kB = SBN * RBK * 2;             // 8 KB
  static constexpr int kW = SBN * 128;                 // 16 KB of raw INT4 per super-step
  static constexpr int kS = SBN * kSpecKS * 4;         // 4 KB of (scale, zero) words
  static constexpr int kBOff = kSpecXSt * kX;
  static constexpr int kWOff = kBOff + kSpecBSt * kB;
  static constexpr int kSOff = kWOff + 2 * kW;
  static constexpr int kBytes = kSOff + 2 * kS;        // 136 KB
  static constexpr int kXc = SBM / 4 / 16;             // X copies per MFMA wave per step: 4
  static constexpr int kWc = SBN / 4 / 8 + SBN / 4 * kSpecKS * 4 / 256;  // per super-step: 4 + 4
};

// Raw weights and (scale, zero) words of the super-step starting at K step
// kb for tile rows 32 p .. 32 p + 31 (dequantisation wave p): 8 rows x 128
// bytes per copy, chunk q of row r at slot q ^ wswz(r); the words of a row
// in natural order (32 bytes per row).
__device__ __forceinline__ void spec_w_issue(lds8* wb, lds8* sb, const uint8_t* __restrict__ W,
                                             const uint32_t* __restrict__ SZ, int N, int K,
                                             int n0, int kb, int p, int lane) {
  const uint32_t ksz = K / 32;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r0 = 32 * p + 8 * q;
    const int r = r0 + (lane >> 3);
    const int qg = (lane & 7) ^ wswz(r);
    const uint32_t n = min(n0 + r, N - 1);
    copy16s(W, n * (uint32_t)(K / 2) + (uint32_t)(kb + qg) * 16u, wb + r0 * 128);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int r0 = 32 * p + 8 * q;
    const uint32_t n = min(n0 + r0 + (lane >> 3), N - 1);
    copy4s(SZ, 4u * (n * ksz + (uint32_t)(kb + (lane & 7))), sb + r0 * 32);
  }
}

// Raw input of one lane's dequantisation: 16 nibbles and the block's
// (scale, zero) word.
struct SpecRaw {
  u2_t w;
  uint32_t s2;
};

// Position pos of a super-step (one K step) for tile row r = 32 p + lane /
// 2, elements 16 h .. 16 h + 15 of its block (h = lane & 1).
__device__ __forceinline__ SpecRaw spec_raw(const lds8* wb, const lds8* sb, int pos, int p,
                                            int lane) {
  const int r = 32 * p + (lane >> 1), h = lane & 1;
  return SpecRaw{lds_ld<u2_t>(wb + r * 128 + ((pos ^ wswz(r)) << 4) + 8 * h),
                 lds_ld<uint32_t>(sb + r * 32 + 4 * pos)};
}

// fp16 weights of a lane's raw input as pieces 2 h and 2 h + 1 of row r in
// a B stage (64 bytes per row, piece P at slot P ^ ((r >> 1) & 3): the X
// layout, so that the MFMA waves read B fragments like X fragments).
__device__ __forceinline__ void spec_dequant(lds8* bs, const SpecRaw& in, int p, int lane) {
  const int r = 32 * p + (lane >> 1), h = lane & 1;
  const uint32_t sbits = in.s2 & 0xFFFFu, zb = in.s2 >> 16;
  const h2_t sc = as_h2(sbits | (sbits << 16));
  const h2_t nz = -(as_h2(0x64006400u) + as_h2(zb | (zb << 16)));  // -(1024 + zp), exact
  u4_t o[2];
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    const uint32_t w = in.w[d], w4 = w >> 4;
#pragma unroll
    for (int k = 0; k < 4; ++k) o[d][k] = as_u32((as_h2(nib_pair(w, w4, k)) + nz) * sc);
  }
  const int sw = (r >> 1) & 3;
  lds8* row = bs + r * 64;
  *(__attribute__((address_space(3))) u4_t*)(row + 16 * ((2 * h) ^ sw)) = o[0];
  *(__attribute__((address_space(3))) u4_t*)(row + 16 * ((2 * h + 1) ^ sw)) = o[1];
}

// Unit range of a ring / specialised workgroup: blocks [0, dp) take tile b
// whole, the sk stream-K workgroups share the units of the other tiles
// (consecutive ones on one XCD); w = the stream-K index.
__device__ __forceinline__ void sk_range(int b, int dp, int sk, int U, int tiles, int64_t& lo,
                                         int64_t& hi, int64_t& TU, int& w) {
  TU = 0;
  w = 0;
  if (b < dp) {
    lo = (int64_t)b * U;
    hi = lo + U;
  } else {
    const int bb = b - dp;
    w = (sk % 8 == 0) ? (b % 8) * (sk / 8) + bb / 8 : bb;
    TU = (int64_t)(tiles - dp) * U;
    lo = (int64_t)dp * U + sk_lo(w, TU, sk);
    hi = (int64_t)dp * U + sk_lo(w + 1, TU, sk);
  }
}

// Position in a workgroup's K steps as (tile, unit of the tile, step of the
// unit), advanced one step at a time without divisions.
struct SpecCursor {
  int tile, unit, pos;
  __device__ __forceinline__ void init(int u, int U) {
    tile = u / U;
    unit = u - tile * U;
    pos = 0;
  }
  __device__ __forceinline__ void next(int U) {
    if (++pos == kSpecKS) {
      pos = 0;
      if (++unit == U) {
        unit = 0;
        ++tile;
      }
    }
  }
  __device__ __forceinline__ int kb() const { return unit * kSpecKS + pos; }
};

// Barrier that waits only for this wave's LDS accesses older than its last N.
template <int N>
__device__ __forceinline__ void ring_barrier_lgkm() {
  asm volatile("s_waitcnt lgkmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

__global__ __launch_bounds__(kSpecThreads, 1) void gemm_spec_kernel(
    const uint16_t* __restrict__ X, const uint8_t* __restrict__ W,
    const uint32_t* __restrict__ SZ, uint16_t* __restrict__ Y, uint16_t* __restrict__ part, int M,
    int N, int K, int dp, int sk, int U, int maxseg) {
  using R = SpecRing;
  __shared__ __align__(16) uint8_t ring[R::kBytes];
  lds8* rb = (lds8*)ring;
  asm volatile("" : "+s"(rb));  // a value the compiler cannot see (see gemm_ring_kernel)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int ntn = N / SBN;
  const int tiles = ntn * ((M + SBM - 1) / SBM);
  int64_t lo, hi, TU;
  int w;
  sk_range(blockIdx.x, dp, sk, U, tiles, lo, hi, TU, w);
  // K steps of this workgroup: whole units of kSpecKS steps (K % 256 == 0)
  const int G = (int)(hi - lo) * kSpecKS;
  if (G <= 0) return;  // workgroup-uniform: no wave reaches a barrier
  const int ulo = (int)lo;
  if (wave >= 4) {
    // ----------------------------------------------- dequantisation waves
    const int p = wave - 4;
    const int S = G / kSpecKS;  // super-steps
    auto wcopy = [&](int s) {   // raw weights of super-step s (clamped) into buffer s & 1
      const int u = ulo + min(s, S - 1), tile = u / U;
      spec_w_issue(rb + R::kWOff + (s & 1) * R::kW, rb + R::kSOff + (s & 1) * R::kS, W, SZ, N, K,
                   (tile % ntn) * SBN, (u - tile * U) * kSpecKS, p, lane);
    };
    auto raw = [&](int g) {  // this lane's raw input of step g
      const int s = g / kSpecKS;
      return spec_raw(rb + R::kWOff + (s & 1) * R::kW, rb + R::kSOff + (s & 1) * R::kS,
                      g % kSpecKS, p, lane);
    };
    auto bstage = [&](int g) { return rb + R::kBOff + (g % kSpecBSt) * R::kB; };
    wcopy(0);
    wcopy(1);
    wait_copies<R::kWc>();  // super-step 0 (this wave's rows)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      if (j < G) spec_dequant(bstage(j), raw(j), p, lane);
    SpecRaw nx = raw(min(3, G - 1));  // step 3 is in super-step 0
    ring_barrier();                    // B_-1: B of steps 0-2 complete
    // Every step issues the same 4 LDS accesses (2 writes, 2 reads; past
    // the last step they repeat step G - 1 into stages nobody reads again),
    // so that the barrier's count below is exact.
    for (int g = 0; g < G; ++g) {
      // B of step g + 1 (written in step g - 2) complete; the 4 accesses of
      // step g - 1 may still be in flight
      ring_barrier_lgkm<4>();  // B_g
      // keeps the dequantisation below the barrier: hoisted above it, its
      // wait for the raw reads would also wait for the previous step's writes
      __builtin_amdgcn_sched_barrier(0);
      spec_dequant(bstage(g + 3), nx, p, lane);
      // the raw buffer of super-step (g + 4) / 8 - 1 was last read in step
      // g - 1 (its registers were consumed just above); past the last
      // super-step the copies repeat it (the same bytes)
      if (g >= 4 && (g + 4) % kSpecKS == 0) wcopy((g + 4) / kSpecKS + 1);
      // the first raw read of a super-step: its copies (issued 8 steps
      // ago) landed; only the next super-step's may be in flight
      if (g + 4 < G && (g + 4) % kSpecKS == 0) wait_copies<R::kWc>();
      nx = raw(min(g + 4, G - 1));
    }
    wait_copies<0>();  // no copy may land after the workgroup ends
    return;
  }
  // -------------------------------------------------------------- MFMA waves
  const int c = lane & 15, gq = lane >> 4;
  const int sw = 16 * (gq ^ ((c >> 1) & 3));
  const int cm = 128 * (wave >> 1), cn = 64 * (wave & 1);
  const int xoff = (cm + c) * 64 + sw;  // A fragment i8 at + 1024 i8
  const int boff = (cn + c) * 64 + sw;  // B fragment j at + 1024 j
  // X copies: rows 64 wave + 16 q + lane / 4, the 16-byte piece held by LDS
  // slot lane & 3 (X layout); per-lane byte offsets for the current M tile
  // (rows clamped into the matrix), the K step on the scalar base
  uint32_t xo[R::kXc];
  int xm0 = -1;
  auto xcopy = [&](const SpecCursor& cur, int g) {
    const int m0 = (cur.tile / ntn) * SBM;
    if (m0 != xm0) {
      xm0 = m0;
#pragma unroll
      for (int q = 0; q < R::kXc; ++q) {
        const int row = 64 * wave + 16 * q + (lane >> 2);
        const int pc = (lane & 3) ^ ((row >> 1) & 3);
        xo[q] = 2u * ((uint32_t)min(m0 + row, M - 1) * (uint32_t)K + 8u * pc);
      }
    }
    const uint16_t* xb = X + (int64_t)__builtin_amdgcn_readfirstlane(cur.kb()) * RBK;
    lds8* st = rb + (g % kSpecXSt) * R::kX + 64 * 64 * wave;
#pragma unroll
    for (int q = 0; q < R::kXc; ++q) copy16s(xb, xo[q], st + 1024 * q);
  };
  SpecCursor xc, cc;  // X copy step, compute step
  xc.init(ulo, U);
  cc.init(ulo, U);
  int ng = 0;  // the step xc stands at (stops at G - 1)
#pragma unroll
  for (int s = 0; s < kSpecXSt; ++s) {
    xcopy(xc, s);
    if (ng < G - 1) {
      xc.next(U);
      ++ng;
    }
  }
  f4_t acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};
  // End of step g: the last step of a unit that closes the tile or the
  // workgroup's range ends a segment, whose results go out (whole tile:
  // fp16 outputs; shared tile: an fp16 partial) before the accumulators
  // restart.
  auto finish = [&](int g) {
    const SpecCursor cur = cc;
    cc.next(U);
    if (cur.pos != kSpecKS - 1 || (cur.unit != U - 1 && g + 1 != G)) return;
    const int tile = cur.tile;
    const int64_t ua = max<int64_t>(lo, (int64_t)tile * U);
    const int64_t ub = (int64_t)tile * U + cur.unit + 1;
    const int m0 = (tile / ntn) * SBM, n0 = (tile % ntn) * SBN;
    int tq = lane;
    asm volatile("" : "+v"(tq));
    if (ua == (int64_t)tile * U && ub == (int64_t)(tile + 1) * U) {
      // C fragment: lane holds rows 4 g + r of an M-block, column c of an N-block
      const int ec = tq & 15, eg = tq >> 4;
#pragma unroll
      for (int i8 = 0; i8 < 8; ++i8)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int col = n0 + cn + 16 * j + ec;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int row = m0 + cm + 16 * i8 + 4 * eg + r;
            if (row < M) Y[(int64_t)row * N + col] = f2h(acc[i8][j][r]);
          }
        }
    } else {
      // fp16 partial in the accumulator layout: the 8 values of N-blocks 2 jp
      // and 2 jp + 1 of (wave, i8, lane) as one 16-byte piece at
      // ((wave * 8 + i8) * 2 + jp) * 64 + lane; gemm_spec_reduce_kernel reads it
      const int tl = tile - dp;
      const int j = w - sk_owner((int64_t)tl * U, TU, sk);
      u4_t* pt = reinterpret_cast<u4_t*>(part + ((int64_t)tl * maxseg + j) * (SBM * SBN));
      pt += wave * (8 * 2 * 64) + tq;
#pragma unroll
      for (int i8 = 0; i8 < 8; ++i8)
#pragma unroll
        for (int jp = 0; jp < 2; ++jp) {
          const f4_t a = acc[i8][2 * jp], d = acc[i8][2 * jp + 1];
          pt[(i8 * 2 + jp) * 64] = u4_t{cvt_pk_h(a[0], a[1]), cvt_pk_h(a[2], a[3]),
                                        cvt_pk_h(d[0], d[1]), cvt_pk_h(d[2], d[3])};
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f4_t{0.f, 0.f, 0.f, 0.f};
  };
  // A step: the fragments of step g + 1 are requested first (into the other
  // register set, so that nothing waits for them before the next barrier),
  // then the 32 MFMAs of step g.
  struct Frag {
    h8_t a[8], b[4];
  };
  auto cstep = [&](int g, const Frag& cur, Frag& nxt) {
    // X of step g + 1 landed (younger: the copies of steps g + 2 .. g + kSpecXSt - 1)
    wait_copies<(kSpecXSt - 2) * R::kXc>();
    ring_barrier();  // B_g: step g + 1's stages complete, this wave's reads of step g done
    xcopy(xc, g + kSpecXSt);  // into the stage step g used (clamped to step G - 1)
    if (ng < G - 1) {
      xc.next(U);
      ++ng;
    }
    // fragments of step g + 1 (after the last step: a stage nobody writes
    // any more, read and never used)
    const lds8* xs = rb + ((g + 1) % kSpecXSt) * R::kX + xoff;
    const lds8* bs = rb + R::kBOff + ((g + 1) % kSpecBSt) * R::kB + boff;
#pragma unroll
    for (int i8 = 0; i8 < 8; ++i8) nxt.a[i8] = lds_ld<h8_t>(xs + 1024 * i8);
#pragma unroll
    for (int j = 0; j < 4; ++j) nxt.b[j] = lds_ld<h8_t>(bs + 1024 * j);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i8 = 0; i8 < 8; ++i8)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[i8][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cur.a[i8], cur.b[j], acc[i8][j], 0, 0, 0);
    finish(g);
  };
  Frag f0, f1;
  wait_copies<(kSpecXSt - 1) * R::kXc>();  // X of step 0
  ring_barrier();                           // B_-1
#pragma unroll
  for (int i8 = 0; i8 < 8; ++i8) f0.a[i8] = lds_ld<h8_t>(rb + xoff + 1024 * i8);
#pragma unroll
  for (int j = 0; j < 4; ++j) f0.b[j] = lds_ld<h8_t>(rb + R::kBOff + boff + 1024 * j);
  for (int g = 0; g < G; g += 2) {  // G is a multiple of kSpecKS
    cstep(g, f0, f1);
    cstep(g + 1, f1, f0);
  }
}

// Y = fp16(sum over the segments of each shared 256 x 128 tile, in segment
// order, in fp32) from the partials of gemm_spec_kernel: a thread takes
// lanes 16 g + 4 q .. + 3 of one (wave, i8, jp) piece row -- rows 128 (wave
// >> 1) + 16 i8 + 4 g .. + 3 x columns 64 (wave & 1) + 16 j + 4 q .. + 3 for
// j = 2 jp, 2 jp + 1 -- and writes 4 x 8 outputs (the arithmetic of
// gemm_splitk_reduce_kernel).
constexpr int kSpecRedThreadsPerTile = SBM * SBN / 32;
__global__ __launch_bounds__(256) void gemm_spec_reduce_kernel(const uint16_t* __restrict__ part,
                                                               uint16_t* __restrict__ Y, int M,
                                                               int N, int dp, int sk, int U,
                                                               int maxseg) {
  const int gt = blockIdx.x * 256 + threadIdx.x;
  const int tl = gt / kSpecRedThreadsPerTile, x = gt % kSpecRedThreadsPerTile;
  const int q = x & 3, g = (x >> 2) & 3, jp = (x >> 4) & 1, i8 = (x >> 5) & 7, wv = x >> 8;
  const int ntn = N / SBN;
  const int tiles = ntn * ((M + SBM - 1) / SBM);
  const int64_t TU = (int64_t)(tiles - dp) * U;
  const int w0 = sk_owner((int64_t)tl * U, TU, sk);
  const int w1 = sk_owner((int64_t)tl * U + U - 1, TU, sk);
  if (w1 == w0) return;  // written whole by one workgroup
  const int tile = dp + tl;
  const int row0 = (tile / ntn) * SBM + 128 * (wv >> 1) + 16 * i8 + 4 * g;
  const int colb = (tile % ntn) * SBN + 64 * (wv & 1) + 32 * jp + 4 * q;  // N-block 2 jp
  if (row0 >= M) return;
  const int nseg = w1 - w0 + 1;
  const u4_t* p = reinterpret_cast<const u4_t*>(part + (int64_t)tl * maxseg * (SBM * SBN)) +
                  ((wv * 8 + i8) * 2 + jp) * 64 + 16 * g + 4 * q;
  constexpr int64_t kSeg = SBM * SBN / 8;  // 16-byte pieces per segment
  float v[2][4][4];  // v[b][l][r]: N-block 2 jp + b, column 4q + l, row 4g + r
  auto add = [&](const u4_t (&t)[4], bool first) {
#pragma unroll
    for (int l = 0; l < 4; ++l)
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint32_t wd = t[l][2 * b + h];
          const float lo = h2f((uint16_t)(wd & 0xFFFFu)), hi = h2f((uint16_t)(wd >> 16));
          v[b][l][2 * h] = first ? lo : v[b][l][2 * h] + lo;
          v[b][l][2 * h + 1] = first ? hi : v[b][l][2 * h + 1] + hi;
        }
  };
  {
    u4_t t[4];
#pragma unroll
    for (int l = 0; l < 4; ++l) t[l] = p[l];
    add(t, true);
  }
  for (int j0 = 1; j0 < nseg; j0 += 4) {
    u4_t t[4][4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int l = 0; l < 4; ++l) t[s][l] = p[(int64_t)min(j0 + s, nseg - 1) * kSeg + l];
#pragma unroll
    for (int s = 0; s < 4; ++s)
      if (j0 + s < nseg) add(t[s], false);
  }
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    const int col0 = colb + 16 * b;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if (row0 + r >= M) break;
      uint16_t* y = Y + (int64_t)(row0 + r) * N + col0;
      const uint32_t lo = (uint32_t)f2h(v[b][0][r]) | ((uint32_t)f2h(v[b][1][r]) << 16);
      const uint32_t hi = (uint32_t)f2h(v[b][2][r]) | ((uint32_t)f2h(v[b][3][r]) << 16);
      *reinterpret_cast<u2_t*>(y) = u2_t{lo, hi};
    }
  }
}

// ---------------------------------------------------------------------
// Skinny GEMM for 2 <= M <= 16 rows (batched decode) through an LDS ring.
// A workgroup (4 waves) owns 64 weight rows (16 per wave) and a range of K
// steps; each step stages, by global->LDS copies, 128 bytes of every weight
// row (8 rows x 128 B per copy instruction: whole cache lines, which reads
// the weights at ~5.6-6 TB/s where 16 rows x 64 B per instruction -- the
// MFMA B-fragment layout loaded straight into registers -- measured
// 4.4-4.9 TB/s), the rows' (scale, zero) words and the matching slice of the
// MR activation rows.  kSkStages ring stages, stages - 1 steps in flight
// (kSkDeepStages stages when the grid has at most one workgroup per CU, whose
// LDS then allows it); one barrier per step
// (the ring of gemm_ring_kernel).  Per step each wave runs KS/32 MFMA
// 16x16x32 tiles: B = its 16 weight rows dequantised from LDS (skinny_b),
// A = the activation rows (skinny_a's element order), C = 16 activation
// rows x 16 weight rows.  Lane group g of MFMA j holds the k labels
// k0 + (KS/4) g + 8 j .. +7 in both operands, so each lane reads its 32
// weight bytes of the step with two 16-byte LDS reads.  The 16-byte pieces
// of a row sit in LDS slot piece ^ (row & 7) (bank spread).
// Split-K (S > 1): the workgroup covers steps [s kps, (s+1) kps) and writes
// fp32 partials part[s][m][n]; gemm_skinny_reduce_kernel sums them in order.
// SiLU epilogue (SILU, unsplit, M <= 8; W = [gate; up] over 2I rows): tile t
// holds gate rows 32t .. 32t+31 (waves 0, 1) and the up rows I + 32t ..
// of the same indices (waves 2, 3); its fp16-rounded results meet in LDS
// and each of the 256 threads finishes one (activation row, element):
// y[m][32t + i] = fp16(FWHT32(silu(g) * u)) with the butterflies across 32
// lanes -- the arithmetic of silu_kernel<true>.  A weight row's MFMA chain
// does not depend on the tile it sits in, so the result equals the unsplit
// GEMM followed by that kernel bit for bit.
constexpr int kSkTile = 64;   // weight rows per workgroup
constexpr int kSkStages = 3;      // ring stages (stages - 1 steps in flight)
// at most one workgroup per CU; against 3 stages the batch-8 step measured
// -19 us with 4, +44 us with 5 and +100 us with 6
constexpr int kSkDeepStages = 4;
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

// Per-lane source offsets of the copies of one ring step (bytes from the
// step's uniform bases W + 128 kb, SZ + kb * words, X + kb * kKS; rows past N /
// M clamped to the last one), computed once per workgroup: a step's copies
// then cost no vector arithmetic.  Tile rows 0..31 are weight rows n0 ..,
// tile rows 32..63 are n1 .. (n1 = n0 + 32 except in the SiLU map).
template <int WBITS, int MR>
struct SkCopy {
  using R = SkRing<WBITS, MR>;
  static constexpr int kWpr = R::kSRow / 4;  // scale words per row per step
  uint32_t wo[2], so[R::kCS > 0 ? R::kCS : 1], xo[R::kCX];

  __device__ __forceinline__ void init(int M, int N, int K, int n0, int n1, int wave, int lane) {
    const uint32_t row_bytes = (uint32_t)K * WBITS / 8;
    auto row = [&](int r) { return min(r < 32 ? n0 + r : n1 + (r - 32), N - 1); };
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // weights: copy c covers tile rows 8c .. 8c+7
      const int c = 2 * wave + i, r = 8 * c + (lane >> 3);
      const int piece = (lane & 7) ^ (r & 7);
      wo[i] = (uint32_t)row(r) * row_bytes + 16 * piece;
    }
    if constexpr (WBITS != 16) {
      constexpr int rpc = 64 / kWpr;  // rows per 256-byte copy
#pragma unroll
      for (int i = 0; i < R::kCS; ++i) {
        const int c = R::kCS * wave + i, r = rpc * c + lane / kWpr;
        so[i] = 4u * ((uint32_t)row(r) * (uint32_t)(K / 32) + lane % kWpr);
      }
    }
#pragma unroll
    for (int i = 0; i < R::kCX; ++i) {
      const int c = R::kCX * wave + i;
      if constexpr (R::kX16) {  // 1 KB per copy, 16 bytes per lane
        const int off = 1024 * c + 16 * lane;
        const int r = off / R::kXRow, slot = (off % R::kXRow) / 16;
        xo[i] = 2u * ((uint32_t)min(r, M - 1) * K + 8 * (slot ^ (r & 7)));
      } else {  // 256 B per copy, 4 bytes per lane
        const int off = 256 * c + 4 * lane;
        const int r = off / R::kXRow, slot = (off % R::kXRow) / 16;
        xo[i] = 2u * ((uint32_t)min(r, M - 1) * K + 8 * (slot ^ (r & 7)) + 2 * (lane & 3));
      }
    }
  }

  // step kb of the workgroup's weight rows, scale words and activation rows
  // into ring stage `stage`
  __device__ __forceinline__ void issue(lds8* stage, const uint16_t* __restrict__ X,
                                        const uint8_t* __restrict__ W,
                                        const uint32_t* __restrict__ SZ, int kb,
                                        int wave) const {
    const uint8_t* wb = W + (int64_t)kb * 128;
#pragma unroll
    for (int i = 0; i < 2; ++i) copy16s(wb, wo[i], stage + 1024 * (2 * wave + i));
    if constexpr (WBITS != 16) {
      const uint32_t* sb = SZ + (int64_t)kb * kWpr;
#pragma unroll
      for (int i = 0; i < R::kCS; ++i) copy4s(sb, so[i], stage + R::kW + 256 * (R::kCS * wave + i));
    }
    const uint16_t* xs = X + (int64_t)kb * R::kKS;
#pragma unroll
    for (int i = 0; i < R::kCX; ++i) {
      const int c = R::kCX * wave + i;
      if constexpr (R::kX16) copy16s(xs, xo[i], stage + R::kW + R::kS + 1024 * c);
      else copy4s(xs, xo[i], stage + R::kW + R::kS + 256 * c);
    }
  }
};

// The K loop of one workgroup.  The ring stage of a step is a template
// argument (the loop is unrolled by the ring depth), so that the LDS reads
// address each stage through their immediate offset from per-lane offsets
// computed once.
template <int WBITS, int MR, int D>
struct SkLoop {
  using R = SkRing<WBITS, MR>;
  static_assert(D >= 3 && (D - 2) * R::kPer <= 63, "ring depth: copy waits fit vmcnt");
  lds8* ring;
  const uint16_t* X;
  const uint8_t* W;
  const uint32_t* SZ;
  SkCopy<WBITS, MR> cp;
  int kb0, nk, wave;
  uint32_t ob0, ob1, osw, ox[R::kSteps];  // per-lane LDS offsets within a stage
  f4_t acc;

  template <int ST>
  __device__ __forceinline__ void step(int i) {
    wait_copies<(D - 2) * R::kPer>();  // this wave's copies of step i have landed
    ring_barrier();                    // every wave's; every wave is done with step i-1
    cp.issue(ring + ((ST + D - 1) % D) * R::kStage, X, W, SZ, kb0 + min(i + D - 1, nk - 1),
             wave);
    const lds8* st = ring + ST * R::kStage;
    const u4_t b0 = lds_ld<u4_t>(st + ob0);
    const u4_t b1 = lds_ld<u4_t>(st + ob1);
    uint32_t sw0 = 0u, sw1 = 0u;
    if constexpr (WBITS == 4) {  // blocks 2g, 2g+1 of the step
      const u2_t v = lds_ld<u2_t>(st + osw);
      sw0 = v[0];
      sw1 = v[1];
    } else if constexpr (WBITS == 8) {  // block g
      sw0 = lds_ld<uint32_t>(st + osw);
    }
#pragma unroll
    for (int j = 0; j < R::kSteps; ++j) {
      // activation piece holding k labels k0 + (KS/4) g + 8 j .. +7
      const h8_t a = lds_ld<h8_t>(st + ox[j]);
      h8_t b;
      if constexpr (WBITS == 4) b = skinny_b<4>(j < 4 ? b0 : b1, j < 4 ? sw0 : sw1, j & 3);
      else if constexpr (WBITS == 8) b = skinny_b<8>(j < 2 ? b0 : b1, sw0, j & 1);
      else b = __builtin_bit_cast(h8_t, j == 0 ? b0 : b1);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
    }
  }

  // steps i, i+1, ... from ring stage ST to D-1 (one round of the ring)
  template <int ST>
  __device__ __forceinline__ void round_from(int i) {
    step<ST>(i);
    if constexpr (ST + 1 < D) round_from<ST + 1>(i + 1);
  }
  // the last nk - i < D steps, from stage 0
  template <int ST>
  __device__ __forceinline__ void tail_from(int i) {
    if (i < nk) {
      step<ST>(i);
      if constexpr (ST + 2 < D) tail_from<ST + 1>(i + 1);
    }
  }

  __device__ __forceinline__ void run() {
#pragma unroll
    for (int s = 0; s < D - 1; ++s)
      cp.issue(ring + s * R::kStage, X, W, SZ, kb0 + min(s, nk - 1), wave);
    int i = 0;
    for (; i + D <= nk; i += D) round_from<0>(i);
    tail_from<0>(i);
  }
};

// Balanced SiLU tail (SILU, tail.part != NULL): units 0 .. umain-1 (whole
// rounds of 256) run one workgroup each over all of K; each of the other
// units is cut along K into S pieces of kps steps (workgroups umain + u' S +
// s), which leave fp32 partials and count in on the unit's counter; the last
// piece to arrive sums the S partials in piece order and finishes the unit.
// Without it the units past the last whole round (544 = 2 x 256 + 32 at I =
// 17408) ran as a third workgroup on 32 CUs, which then finished a whole
// unit after the rest.
struct SkTail {
  float* part = nullptr;  // [tail units][S][8 rows][64 tile rows] fp32
  int* cnt = nullptr;     // [tail units] arrivals, zero before and after a launch
  int umain = 0, S = 1, kps = 0;
};

// Device-coherent 32-bit load and store (agent scope: past the caches of the
// other XCDs), for partials that workgroups hand to each other in a launch.
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int WBITS, int MR, bool SILU, int D = kSkStages>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(const uint16_t* __restrict__ X,
                                                          const uint8_t* __restrict__ W,
                                                          const uint32_t* __restrict__ SZ,
                                                          uint16_t* __restrict__ Y,
                                                          float* __restrict__ part, int M, int N,
                                                          int K, int ntiles, int kps, int silu_I,
                                                          SkTail tail) {
  static_assert(!SILU || MR == 8, "the SiLU epilogue maps 8 rows x 32 elements to 256 threads");
  using R = SkRing<WBITS, MR>;
  __shared__ __align__(16) uint8_t ring[D * R::kStage];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  int tile = blockIdx.x % ntiles, sp = blockIdx.x / ntiles;
  // SiLU tail piece: unit tile, piece sp of tail.S (workgroup-uniform)
  const bool piece = SILU && tail.part && (int)blockIdx.x >= tail.umain;
  if (piece) {
    const int j = (int)blockIdx.x - tail.umain;
    tile = tail.umain + j / tail.S;
    sp = j % tail.S;
    kps = tail.kps;
  }
  const int n0 = SILU ? 32 * tile : tile * kSkTile;
  const int n1 = SILU ? silu_I + 32 * tile : n0 + 32;
  const int kt = K / R::kKS;
  const int col = lane & 15, g = lane >> 4;
  const int wrow = 16 * wave + col;                   // this lane's weight row in the tile
  const int xr = col % MR;                            // activation row (rows >= MR: duplicates)

  SkLoop<WBITS, MR, D> lp;
  lp.ring = (lds8*)ring;
  lp.X = X;
  lp.W = W;
  lp.SZ = SZ;
  lp.kb0 = sp * kps;
  lp.nk = min(kt - lp.kb0, kps);  // >= 1 (host)
  lp.wave = wave;
  lp.cp.init(M, N, K, n0, n1, wave, lane);
  // weight bytes [32 g, 32 g + 32) of row wrow: pieces 2g, 2g+1
  lp.ob0 = 128 * wrow + 16 * ((2 * g) ^ (wrow & 7));
  lp.ob1 = 128 * wrow + 16 * ((2 * g + 1) ^ (wrow & 7));
  lp.osw = R::kW + R::kSRow * wrow + (WBITS == 4 ? 8 * g : 4 * g);
#pragma unroll
  for (int j = 0; j < R::kSteps; ++j)
    lp.ox[j] = R::kW + R::kS + R::kXRow * xr + 16 * ((R::kSteps * g + j) ^ (xr & 7));
  lp.acc = f4_t{0.f, 0.f, 0.f, 0.f};
  lp.run();
  const f4_t acc = lp.acc;
  wait_copies<0>();  // no copy into LDS outlives the workgroup
  // C: lane holds activation rows 4g + r (rows >= MR repeat rows < MR), tile
  // row 16 wave + col
  if constexpr (SILU) {
#pragma clang fp contract(off)  // g / (1 + e^-g) * u in separately rounded steps
    __syncthreads();  // every wave is done with the ring, which now holds
    float* us = reinterpret_cast<float*>(ring);  // us[m][tile row], 8 x 64
    const int m = threadIdx.x >> 5, i = threadIdx.x & 31;
    float gv, uv;
    if (piece) {
      // partials out as device-coherent stores, which every wave waits for
      // before thread 0 counts the piece in; the last of the unit's S pieces
      // resets the counter for the next launch and sums the partials
      const int tu = tile - tail.umain;
      float* tp = tail.part + ((int64_t)tu * tail.S + sp) * 512;
      if (g < 2) {
#pragma unroll
        for (int r = 0; r < 4; ++r) st_agent(tp + (4 * g + r) * 64 + 16 * wave + col, acc[r]);
      }
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      int* last = reinterpret_cast<int*>(us + 512);
      if (threadIdx.x == 0) {
        int* c = tail.cnt + tu;
        const int prev = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *last = prev == tail.S - 1;
        if (prev == tail.S - 1) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      __syncthreads();
      if (*last == 0) return;
      // the split reduce's arithmetic: fp32 sums in piece order, one fp16 rounding
      const float* tb = tail.part + (int64_t)tu * tail.S * 512 + m * 64 + i;
      float ga = ld_agent(tb), ua = ld_agent(tb + 32);
      for (int z = 1; z < tail.S; ++z) {
        ga += ld_agent(tb + z * 512);
        ua += ld_agent(tb + z * 512 + 32);
      }
      gv = h2f(f2h(ga));
      uv = h2f(f2h(ua));
    } else {
      if (g < 2) {
#pragma unroll
        for (int r = 0; r < 4; ++r) us[(4 * g + r) * 64 + 16 * wave + col] = h2f(f2h(acc[r]));
      }
      __syncthreads();
      gv = us[m * 64 + i];
      uv = us[m * 64 + 32 + i];
    }
    float v = gv / (1.0f + expf(-gv)) * uv;
#pragma unroll
    for (int bit = 1; bit <= 16; bit <<= 1) {
      const float o = __shfl_xor(v, bit);
      v = (i & bit) ? o - v : v + o;
    }
    v *= kInvSqrt32;
    if (m < M) Y[(int64_t)m * silu_I + 32 * tile + i] = f2h(v);
    return;
  }
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
// columns: gate 0..I-1, up I..2I-1), four lanes per 32-column chunk: lane q
// of chunk c of row m sums gate and up columns 32c + 8q .. + 7 over the
// splits in order and rounds each sum to fp16 (what gemm_skinny_reduce_kernel
// stores), applies silu(g) * u as silu_kernel<true> does, then runs the
// butterfly stages 1, 2, 4 of the FWHT-32 in registers and stages 8 and 16
// with the lanes q ^ 1 and q ^ 2 -- the stage order and (a + b, a - b) pairs
// of fwht32, so the fp16 output is the same bit for bit.  (One thread per
// chunk left 72 waves on the chip for I = 17408 and took 6.2 us.)
__device__ __forceinline__ void skinny_sum8(const float* __restrict__ p, int64_t plane, int S,
                                            float* v) {
  const float4* q = reinterpret_cast<const float4*>(p);
  float4 t0 = q[0], t1 = q[1];
  v[0] = t0.x, v[1] = t0.y, v[2] = t0.z, v[3] = t0.w;
  v[4] = t1.x, v[5] = t1.y, v[6] = t1.z, v[7] = t1.w;
  for (int z = 1; z < S; ++z) {
    q = reinterpret_cast<const float4*>(p + z * plane);
    t0 = q[0];
    t1 = q[1];
    v[0] += t0.x, v[1] += t0.y, v[2] += t0.z, v[3] += t0.w;
    v[4] += t1.x, v[5] += t1.y, v[6] += t1.z, v[7] += t1.w;
  }
}

constexpr int kSiluRedThreads = 256;
__global__ __launch_bounds__(kSiluRedThreads) void gemm_skinny_reduce_silu_kernel(
    const float* __restrict__ part, uint16_t* __restrict__ Y, int M, int I, int S) {
#pragma clang fp contract(off)  // g / (1 + e^-g) * u in separately rounded steps
  const int tid = blockIdx.x * kSiluRedThreads + threadIdx.x, m = blockIdx.y;
  const int c = tid >> 2, q = tid & 3;
  // lanes past the row read chunk 0 and store nothing, but take part in the
  // cross-lane stages of their chunk group
  const bool live = c * 32 < I;
  const int64_t plane = (int64_t)M * 2 * I;
  const float* pg = part + (int64_t)m * 2 * I + (live ? c : 0) * 32 + 8 * q;
  float a[8], b[8];
  skinny_sum8(pg, plane, S, a);
  skinny_sum8(pg + I, plane, S, b);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float g = h2f(f2h(a[i])), u = h2f(f2h(b[i]));
    a[i] = g / (1.0f + expf(-g)) * u;
  }
#pragma unroll
  for (int step = 1; step < 8; step <<= 1) {
#pragma unroll
    for (int i = 0; i < 8; i += 2 * step) {
#pragma unroll
      for (int j = i; j < i + step; ++j) {
        const float x = a[j], y = a[j + step];
        a[j] = x + y;
        a[j + step] = x - y;
      }
    }
  }
#pragma unroll
  for (int lm = 1; lm <= 2; lm <<= 1) {  // stages 8 and 16: partner lane q ^ lm
    const bool upper = (q & lm) != 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float o = __shfl_xor(a[j], lm);
      a[j] = upper ? o - a[j] : a[j] + o;
    }
  }
  if (!live) return;
  u4_t w;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    w[k] = (uint32_t)f2h(a[2 * k] * kInvSqrt32) | ((uint32_t)f2h(a[2 * k + 1] * kInvSqrt32) << 16);
  *reinterpret_cast<u4_t*>(Y + (int64_t)m * I + c * 32 + 8 * q) = w;
}

}  // namespace

bool gemm_skinny_ok(int64_t M, int64_t N, int64_t K, int wbits) {
  const int64_t ks = 1024 / (wbits == 4 ? 4 : wbits == 8 ? 8 : 16);  // k per ring step
  // the copies address the weights with 32-bit byte offsets
  return M >= 2 && M <= 16 && K % ks == 0 && N * K * wbits / 8 < ((int64_t)1 << 32);
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
size_t skinny_tail_part_bytes(int64_t T, int64_t S) {
  return ((size_t)T * S * 512 * 4 + 255) & ~(size_t)255;
}
size_t skinny_tail_cnt_bytes(int64_t T) { return ((size_t)T * 4 + 255) & ~(size_t)255; }

// Tail plan of the unsplit SiLU GEMM (see SkTail) for I / 32 units over 256
// CUs: the units past the last whole round of 256, each cut into S pieces
// of kps K steps with S about 128 / tail units (measured at 32 tail units:
// 4 pieces each 3.845 ms per batch-8 step, 2 / 3 / 8 / 16 pieces 3.935 /
// 3.877 / 3.852 / 3.892 ms).  No tail
// (part == NULL) without a workspace, below one round, on whole rounds, or
// when a unit would not be cut.  Workspace: the counters, then the partials.
SkTail skinny_tail_plan(int64_t I, int64_t K, int wbits, void* ws) {
  SkTail t;
  const int64_t units = I / 32, kt = K / (1024 / wbits);
  const int64_t T = units % 256;
  if (!ws || units <= 256 || T == 0) return t;
  const int64_t S0 = std::min<int64_t>(kt, std::max<int64_t>(1, 128 / T));
  const int64_t kps = (kt + S0 - 1) / S0, S = (kt + kps - 1) / kps;  // every piece non-empty
  if (S < 2) return t;
  t.umain = (int)(units - T);
  t.S = (int)S;
  t.kps = (int)kps;
  t.cnt = static_cast<int*>(ws);  // counters first: the same place for every width
  t.part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + skinny_tail_cnt_bytes(T));
  return t;
}

// silu_I > 0: N = 2 silu_I gate/up columns into y (M x silu_I) gated by
// SiLU + FWHT-32: split (S > 1) and reduced by
// gemm_skinny_reduce_silu_kernel, or unsplit (S == 1, M <= 8: checked by the
// caller) with the gate in the GEMM's epilogue.  keep_part: no reduce, the
// S fp32 partial planes stay in ws (S > 1) for the consumer to sum.
int skinny_run(const void* x, const void* w, const void* sz, void* y, int64_t M, int64_t N,
               int64_t K, int wbits, hipStream_t st, void* ws, size_t ws_bytes, int64_t silu_I,
               bool keep_part = false, void* tail_ws = nullptr) {
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
  const bool m8 = M <= 8;
  if (silu_I > 0 && S == 1) {  // unsplit: the SiLU gate in the epilogue
    R4Q_REQUIRE(M <= 8 && silu_I % 32 == 0 && N == 2 * silu_I,
                "gate_up_silu: the unsplit epilogue takes at most 8 rows (M=%lld)", (long long)M);
    const SkTail tl = skinny_tail_plan(silu_I, K, wbits, tail_ws);
    const int64_t units = silu_I / 32;
    const int64_t wgs = tl.part ? tl.umain + (units - tl.umain) * tl.S : units;
#define R4Q_SKINNY_SILU(WB)                                                                      \
  hipLaunchKernelGGL((gemm_skinny_kernel<WB, 8, true>), dim3((unsigned)wgs), dim3(256), 0, st,   \
                     xp, wp, sp, yp, nullptr, (int)M, (int)N, (int)K, (int)units, kps,           \
                     (int)silu_I, tl)
    if (wbits == 4) R4Q_SKINNY_SILU(4);
    else if (wbits == 8) R4Q_SKINNY_SILU(8);
    else R4Q_SKINNY_SILU(16);
#undef R4Q_SKINNY_SILU
    return launch_status("gemm_skinny_silu");
  }
  const bool deep = ntiles * S <= 256;  // one workgroup per CU: LDS for a deeper ring
#define R4Q_SKINNY_D(WB, MRR, DD)                                                              \
  hipLaunchKernelGGL((gemm_skinny_kernel<WB, MRR, false, DD>), grid, dim3(256), 0, st, xp, wp, \
                     sp, yp, part, (int)M, (int)N, (int)K, (int)ntiles, kps, 0, SkTail{})
#define R4Q_SKINNY(WB, MRR)                                                                    \
  if (deep) R4Q_SKINNY_D(WB, MRR, kSkDeepStages);                                            \
  else R4Q_SKINNY_D(WB, MRR, kSkStages)
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
#undef R4Q_SKINNY_D
  R4Q_TRY(launch_status("gemm_skinny"));
  if (keep_part) return R4Q_OK;
  if (silu_I > 0) {
    hipLaunchKernelGGL(gemm_skinny_reduce_silu_kernel,
                       dim3((unsigned)((silu_I / 8 + kSiluRedThreads - 1) / kSiluRedThreads),
                            (unsigned)M),
                       dim3(kSiluRedThreads), 0, st, part, yp, (int)M, (int)silu_I, S);
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

int gemm_skinny_part_launch(const void* x, const void* w, const void* sz, void* y, int64_t M,
                            int64_t N, int64_t K, int wbits, hipStream_t st, void* ws,
                            size_t ws_bytes, int* S) {
  R4Q_REQUIRE(gemm_skinny_ok(M, N, K, wbits), "skinny GEMM: unsupported shape");
  *S = skinny_splits(M, N, K, wbits, ws ? ws_bytes : 0);
  return skinny_run(x, w, sz, y, M, N, K, wbits, st, ws, ws_bytes, 0, true);
}

bool gemm_skinny_silu_ok(int64_t M, int64_t I, int64_t K, int wbits, size_t ws_bytes) {
  return gemm_skinny_ok(M, 2 * I, K, wbits) && I > 0 && I % 32 == 0 &&
         (M <= 8 || skinny_splits(M, 2 * I, K, wbits, ws_bytes) > 1);
}

int gemm_skinny_silu_launch(const void* x, const void* w, const void* sz, void* y, int64_t M,
                            int64_t I, int64_t K, int wbits, hipStream_t st, void* ws,
                            size_t ws_bytes) {
  R4Q_REQUIRE(gemm_skinny_silu_ok(M, I, K, wbits, ws ? ws_bytes : 0),
              "gate_up_silu: needs I %% 32 == 0, and above 8 rows a workspace that splits K");
  return skinny_run(x, w, sz, y, M, 2 * I, K, wbits, st, ws, ws_bytes, I);
}

size_t skinny_silu_tail_bytes(int64_t I, int64_t K, int wbits) {
  int dummy = 0;
  const SkTail t = skinny_tail_plan(I, K, wbits, &dummy);
  if (!t.part) return 0;
  const int64_t T = I / 32 - t.umain;
  return skinny_tail_cnt_bytes(T) + skinny_tail_part_bytes(T, t.S);
}

size_t skinny_silu_tail_cnt_bytes(int64_t I) {
  const int64_t units = I / 32;
  return units > 256 && units % 256 ? skinny_tail_cnt_bytes(units % 256) : 0;
}

int gemm_skinny_silu_tail_launch(const void* x, const void* w, const void* sz, void* y, int64_t M,
                                 int64_t I, int64_t K, int wbits, hipStream_t st, void* tail_ws) {
  R4Q_REQUIRE(M <= 8 && gemm_skinny_silu_ok(M, I, K, wbits, 0),
              "gate_up_silu: the unsplit epilogue takes at most 8 rows and I %% 32 == 0");
  return skinny_run(x, w, sz, y, M, 2 * I, K, wbits, st, nullptr, 0, I, false, tail_ws);
}

// The ring kernel addresses X, W and the scale words with 32-bit byte offsets.
bool gemm_ring_ok(int64_t M, int64_t N, int64_t K, int wbits) {
  const int64_t lim = (int64_t)1 << 32;
  return M >= RBM && M * K * 2 < lim && N * K * wbits / 8 < lim &&
         N * (K / 32) * 4 < lim;
}

// Work split of the ring kernel (see gemm_ring_kernel): dp whole tiles,
// then sk stream-K workgroups over the other tiles.
struct RingPlan {
  int dp = 0, sk = 0, U = 1, maxseg = 1;
  size_t ws = 0;  // fp16 partials: (tiles - dp) * maxseg * 256 * 256 * 2 bytes
};

constexpr int kRingCUs = 256;  // MI355X compute units: one ring workgroup each (LDS-bound)

// Host restatement of sk_lo / sk_owner (the kernel's unit split).
static int64_t host_sk_lo(int64_t w, int64_t TU, int64_t sk) { return w * TU / sk; }
static int64_t host_sk_owner(int64_t u, int64_t TU, int64_t sk) {
  int64_t w = u * sk / TU;
  while (w + 1 < sk && host_sk_lo(w + 1, TU, sk) <= u) ++w;
  while (w > 0 && host_sk_lo(w, TU, sk) > u) --w;
  return w;
}

// dp / sk split of `tiles` tiles of U units each (see ring_plan), with fp16
// partials of tile_elems elements per (shared tile, segment).
static RingPlan split_plan(int64_t tiles, int U, int64_t tile_elems, size_t ws_bytes) {
  // Every CU gets the same number of K units: the tiles of the full rounds
  // of 256 workgroups are computed whole, the remaining tiles' units are
  // shared by 256 stream-K workgroups (each then writes at most two fp32
  // partials: 512 x 34816 x 5120, 272 tiles, INT4 271 -> 238 us against
  // sharing every tile out).  Whole tiles throughout when their rounds are
  // at least 7/8 full: the partials and their reduce then cost what the idle
  // CUs would (the LM head of a 512-token prompt, 1188 tiles in 5 rounds:
  // 1109 us whole, 1116 us shared).
  RingPlan pl;
  pl.U = U;
  int64_t dp = tiles, sk = 0;
  const int v = tuning().gemm_splits.load();  // measurement override
  if (v >= 2) {                                // about v segments per tile, all tiles shared
    dp = 0;
    sk = std::min<int64_t>(tiles * v, tiles * pl.U);
  } else if (v == 1 || 8 * tiles >= 7 * kRingCUs * ((tiles + kRingCUs - 1) / kRingCUs)) {
    dp = tiles;
  } else if (tiles > kRingCUs) {
    dp = (tiles / kRingCUs) * kRingCUs;
    // no more stream-K workgroups than shared units: every one owns at
    // least one, so every partial slot the reduce reads is written
    sk = std::min<int64_t>(kRingCUs, (tiles - dp) * pl.U);
  } else if (kRingCUs / tiles >= 2) {
    // at most 128 tiles: each split into floor(256 / tiles) equal pieces, so
    // that every workgroup stays inside one tile and writes one partial
    // (M = 512: 7168 x 5120 INT4 81.6 -> 67.7 us, 5120 x 17408 125.6 -> 119.7)
    dp = 0;
    sk = std::min<int64_t>(tiles * (kRingCUs / tiles), tiles * pl.U);
  } else {
    dp = 0;
    sk = std::min<int64_t>(kRingCUs, tiles * pl.U);
  }
  if (sk > 0) {
    const int64_t TU = (tiles - dp) * pl.U;
    int64_t maxseg = 1;
    for (int64_t t = 0; t < tiles - dp; ++t)
      maxseg = std::max(maxseg, host_sk_owner(t * pl.U + pl.U - 1, TU, sk) -
                                    host_sk_owner(t * pl.U, TU, sk) + 1);
    const size_t ws = maxseg > 1 ? (size_t)(tiles - dp) * maxseg * tile_elems * 2 : 0;
    if (ws <= ws_bytes) {
      pl.dp = (int)dp;
      pl.sk = (int)sk;
      pl.maxseg = (int)maxseg;
      pl.ws = ws;
      return pl;
    }
  }
  pl.dp = (int)tiles;  // whole tiles only
  return pl;
}

RingPlan ring_plan(int64_t M, int64_t N, int64_t K, int wbits, size_t ws_bytes) {
  const int64_t tiles = ((N + RBN - 1) / RBN) * ((M + RBM - 1) / RBM);
  const int KS = wbits == 4 ? Ring<4>::KS : wbits == 8 ? Ring<8>::KS : Ring<16>::KS;
  return split_plan(tiles, (int)((K / RBK + KS - 1) / KS), RBM * RBN, ws_bytes);
}

// The specialised-wave kernel: INT4, whole 128-column tiles, whole super-steps.
bool gemm_spec_ok(int64_t M, int64_t N, int64_t K, int wbits) {
  return wbits == 4 && gemm_ring_ok(M, N, K, wbits) && N % SBN == 0 &&
         K % (RBK * kSpecKS) == 0;
}

RingPlan spec_plan(int64_t M, int64_t N, int64_t K, size_t ws_bytes) {
  const int64_t tiles = (N / SBN) * ((M + SBM - 1) / SBM);
  return split_plan(tiles, (int)(K / (RBK * kSpecKS)), SBM * SBN, ws_bytes);
}

// Kernel for M >= 256: the ring kernel, or the specialised-wave kernel where
// it applies when the gemm_kernel knob is 2.  Measured on config 3 (M = 512,
// INT4, five A/B pairs on one box) the latter is the slower of the two (3a
// 140-146 against 132-137 us, 3b 131-141 against 126-131 us): the 256 x 128
// tile that the register budget of two waves per SIMD allows copies twice
// the X bytes per FLOP of the ring kernel's 256 x 256 tile, and the X copies
// (16 KB per K step per CU) then bound its K step as the single-wave issue
// bounds the ring kernel's.
bool use_spec(int64_t M, int64_t N, int64_t K, int wbits) {
  return tuning().gemm_kernel.load() == 2 && gemm_spec_ok(M, N, K, wbits);
}

int gemm_splits(int64_t M, int64_t N, int64_t K, int wbits, size_t ws_bytes) {
  if (use_spec(M, N, K, wbits)) return spec_plan(M, N, K, ws_bytes).maxseg;
  return gemm_ring_ok(M, N, K, wbits) ? ring_plan(M, N, K, wbits, ws_bytes).maxseg : 1;
}

// Workspace for the larger of the two kernels' plans, so that a workspace
// sized once serves either choice of the gemm_kernel knob.
size_t gemm_ws_bytes(int64_t M, int64_t N, int64_t K, int wbits) {
  if (!gemm_ring_ok(M, N, K, wbits)) return 0;
  size_t ws = ring_plan(M, N, K, wbits, (size_t)-1).ws;
  if (gemm_spec_ok(M, N, K, wbits)) ws = std::max(ws, spec_plan(M, N, K, (size_t)-1).ws);
  return ws;
}

int gemm_mfma_launch(const void* x, const void* w, const void* sz, void* y, int64_t M, int64_t N,
                     int64_t K, int wbits, hipStream_t st, void* ws, size_t ws_bytes) {
  const auto* xp = static_cast<const uint16_t*>(x);
  const auto* wp = static_cast<const uint8_t*>(w);
  const auto* sp = static_cast<const uint32_t*>(sz);
  auto* yp = static_cast<uint16_t*>(y);
  if (use_spec(M, N, K, wbits)) {
    const RingPlan pl = spec_plan(M, N, K, ws ? ws_bytes : 0);
    uint16_t* part = pl.ws ? static_cast<uint16_t*>(ws) : nullptr;
    hipLaunchKernelGGL(gemm_spec_kernel, dim3((unsigned)(pl.dp + pl.sk)), dim3(kSpecThreads), 0,
                       st, xp, wp, sp, yp, part, (int)M, (int)N, (int)K, pl.dp, pl.sk, pl.U,
                       pl.maxseg);
    R4Q_TRY(launch_status("gemm_spec"));
    if (pl.ws) {
      const int64_t tiles = (N / SBN) * ((M + SBM - 1) / SBM);
      const unsigned rb = (unsigned)((tiles - pl.dp) * (kSpecRedThreadsPerTile / 256));
      hipLaunchKernelGGL(gemm_spec_reduce_kernel, dim3(rb), dim3(256), 0, st, part, yp, (int)M,
                         (int)N, pl.dp, pl.sk, pl.U, pl.maxseg);
      R4Q_TRY(launch_status("gemm_spec_reduce"));
    }
    return R4Q_OK;
  }
  if (gemm_ring_ok(M, N, K, wbits)) {
    const RingPlan pl = ring_plan(M, N, K, wbits, ws ? ws_bytes : 0);
    uint16_t* part = pl.ws ? static_cast<uint16_t*>(ws) : nullptr;
    const unsigned blocks = (unsigned)(pl.dp + pl.sk);
    if (wbits == 4)
      hipLaunchKernelGGL(gemm_ring_kernel<4>, dim3(blocks), dim3(kRingThreads), 0, st, xp, wp, sp,
                         yp, part, (int)M, (int)N, (int)K, pl.dp, pl.sk, pl.U, pl.maxseg);
    else if (wbits == 8)
      hipLaunchKernelGGL(gemm_ring_kernel<8>, dim3(blocks), dim3(kRingThreads), 0, st, xp, wp, sp,
                         yp, part, (int)M, (int)N, (int)K, pl.dp, pl.sk, pl.U, pl.maxseg);
    else
      hipLaunchKernelGGL(gemm_ring_kernel<16>, dim3(blocks), dim3(kRingThreads), 0, st, xp, wp,
                         sp, yp, part, (int)M, (int)N, (int)K, pl.dp, pl.sk, pl.U, pl.maxseg);
    R4Q_TRY(launch_status("gemm_ring"));
    if (pl.ws) {
      const int64_t tiles = ((N + RBN - 1) / RBN) * ((M + RBM - 1) / RBM);
      const unsigned rb = (unsigned)((tiles - pl.dp) * (kRedThreadsPerTile / 256));
      hipLaunchKernelGGL(gemm_splitk_reduce_kernel, dim3(rb), dim3(256), 0, st, part, yp, (int)M,
                         (int)N, pl.dp, pl.sk, pl.U, pl.maxseg);
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
