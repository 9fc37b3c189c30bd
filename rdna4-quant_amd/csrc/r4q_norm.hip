// RMSNorm / residual / FWHT-32 / SiLU-gate and the per-head QK-norm + RoPE
// + FP8 KV-cache write of the decode step.
//
// Reference kernels replaced: fused_res_norm_fwht (hip:1143-1192),
// fused_rmsnorm_fwht (hip:1195-1237), rmsnorm_ds / fused_res_norm
// (hip:795-846), hadamard_rotate_batched (hip:766-786), silu_hadamard_ds
// (hip:1031-1051), silu_mul_batched (hip:2112-2122), head_rmsnorm / rope_ds
// (hip:849-911) and head_rmsnorm_rope_kv (hip:1620-1683).
//
// Row kernels: one workgroup per row, one thread per 32-element chunk; the
// chunk is loaded with 128-bit accesses, the FWHT-32 runs in that thread's
// registers, the sum of squares is reduced with DPP + v_readlane inside each
// wave and through 16 floats of LDS across waves.
#include "r4q_device.hpp"
#include "r4q_host.hpp"
#include "r4q_kernels.hpp"

namespace r4q {
namespace {

// MODE bit 0: residual input b (res_out = fp16(a + b)); bit 1: FWHT output.
template <int MODE>
__global__ __launch_bounds__(1024) void rownorm_kernel(const uint16_t* __restrict__ a,
                                                        const uint16_t* __restrict__ b,
                                                        const uint16_t* __restrict__ w,
                                                        uint16_t* __restrict__ y,
                                                        uint16_t* __restrict__ res_out, int D,
                                                        float eps) {
  constexpr bool RES = MODE & 1;
  constexpr bool FWHT = MODE & 2;
  __shared__ float red[16];
  const int64_t row = blockIdx.x;
  const int nch = D / 32;
  constexpr int kMaxChunks = 2;  // chunks per thread (D <= 2 * 32 * 1024)
  uint32_t r[kMaxChunks][16];  // fp16 pairs: a, or the rounded residual fp16(a + b)
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxChunks; ++j) {
    const int c = threadIdx.x + j * blockDim.x;
    if (c < nch) {
      uint32_t av[16], bv[16];
      load16w(a + row * D + c * 32, av);
      if constexpr (RES) load16w(b + row * D + c * 32, bv);
      ss = norm_chunk_sumsq<RES>(av, bv, r[j], ss);
    }
  }
  const float tot = block_sum(ss, red);
  const float rrms = 1.0f / __builtin_sqrtf(tot / (float)D + eps);
#pragma unroll
  for (int j = 0; j < kMaxChunks; ++j) {
    const int c = threadIdx.x + j * blockDim.x;
    if (c < nch) {
      uint32_t g[16], o[16];
      load16w(w + c * 32, g);
      // the residual is rounded to fp16 before normalisation (hip:1151-1153,
      // 1178): stored, and normalised from the rounded value
      if constexpr (RES) store16w(res_out + row * D + c * 32, r[j]);
      norm_chunk_scale<FWHT>(r[j], g, rrms, o);
      store16w(y + row * D + c * 32, o);
    }
  }
}

// rownorm_kernel<3> (residual + RMSNorm + FWHT-32) whose input a is the
// split-K sum of a projection, a = fp16(sum over s < S of ap[s * plane +
// row * D + i]) in split order -- the arithmetic of gemm_skinny_reduce_kernel
// -- so the outputs equal that reduce followed by rownorm_kernel<3>.  One
// workgroup per row, its waves in two roles, so that every load instruction
// carries a full wave of useful bytes (the kernel is bound by the rate at
// which its loads issue, not by their bytes):
//  * the first 5/8 of the threads (PT) read the S planes coalesced (KF
//    float4 per thread and plane), add them in split order and stage the
//    fp16 row in LDS;
//  * the other CT threads, one per 32-element chunk, load their residual
//    and weight chunks meanwhile, then run the chunk norm as rownorm_kernel
//    does from the staged row (the sum of squares over the waves in order:
//    the plane waves add exact zeros).
// D <= 4 KF PT and D / 32 <= CT.
constexpr int kPsumMaxS = 4;
template <int NT, int KF, int S>
__global__ __launch_bounds__(NT) void rownorm_psum_kernel(
    const float* __restrict__ ap, int64_t plane, const uint16_t* __restrict__ b,
    const uint16_t* __restrict__ w, uint16_t* __restrict__ y, uint16_t* __restrict__ res_out,
    int D, float eps) {
  constexpr int PT = NT / 8 * 5;  // plane threads (whole waves)
  __shared__ float red[NT / 64];
  __shared__ __align__(16) uint32_t as[2 * KF * PT];  // the fp16 row
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x, nch = D / 32, nf = D / 4;
  const int wv = __builtin_amdgcn_readfirstlane(t >> 6);
  typedef float f4v __attribute__((ext_vector_type(4)));
  uint32_t bv[16], g[16];
  if (wv < PT / 64) {
    const float* pr = ap + row * D;
    f4v v[KF][S];
#pragma unroll
    for (int k = 0; k < KF; ++k) {
      const int f = min(t + k * PT, nf - 1);  // clamped, unused past nf
#pragma unroll
      for (int z = 0; z < S; ++z) v[k][z] = *reinterpret_cast<const f4v*>(pr + z * plane + 4 * f);
    }
#pragma unroll
    for (int k = 0; k < KF; ++k) {
      const int f = t + k * PT;
      if (f < nf) {
        f4v a = v[k][0];
#pragma unroll
        for (int z = 1; z < S; ++z) a += v[k][z];
        as[2 * f] = (uint32_t)f2h(a[0]) | ((uint32_t)f2h(a[1]) << 16);
        as[2 * f + 1] = (uint32_t)f2h(a[2]) | ((uint32_t)f2h(a[3]) << 16);
      }
    }
  } else {
    const int c = min(t - PT, nch - 1);
    load16w(b + row * D + c * 32, bv);
    load16w(w + c * 32, g);
  }
  __syncthreads();
  const int c = t - PT;
  const bool act = c >= 0 && c < nch;
  uint32_t r[16];
  float ss = 0.f;
  if (act) {
    uint32_t av[16];
    const u4_t* s4 = reinterpret_cast<const u4_t*>(as + 16 * c);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u4_t d = s4[i];
      av[4 * i] = d[0];
      av[4 * i + 1] = d[1];
      av[4 * i + 2] = d[2];
      av[4 * i + 3] = d[3];
    }
    ss = norm_chunk_sumsq<true>(av, bv, r, ss);
  }
  const float tot = block_sum(ss, red);
  const float rrms = 1.0f / __builtin_sqrtf(tot / (float)D + eps);
  if (act) {
    uint32_t o[16];
    store16w(res_out + row * D + c * 32, r);
    norm_chunk_scale<true>(r, g, rrms, o);
    store16w(y + row * D + c * 32, o);
  }
}

__global__ __launch_bounds__(256) void fwht32_kernel(const uint16_t* __restrict__ x,
                                                     uint16_t* __restrict__ y, int64_t nch) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= nch) return;
  float v[32];
  load32h(x + c * 32, v);
  fwht32(v);
  store32h(y + c * 32, v);
}

// y = fp16([FWHT](silu(g) * u)); one thread per 32-chunk.  y may alias g:
// each thread reads its whole chunk before writing it.
template <bool FWHT>
__global__ __launch_bounds__(256) void silu_kernel(const uint16_t* g, const uint16_t* u,
                                                   uint16_t* y, int I, int64_t in_stride,
                                                   int64_t out_stride) {
#pragma clang fp contract(off)  // g / (1 + e^-g) * u in separately rounded steps
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = blockIdx.y;
  if (c * 32 >= I) return;
  float a[32], b[32];
  load32h(g + row * in_stride + c * 32, a);
  load32h(u + row * in_stride + c * 32, b);
#pragma unroll
  for (int i = 0; i < 32; ++i) a[i] = a[i] / (1.0f + expf(-a[i])) * b[i];
  if constexpr (FWHT) fwht32(a);
  store32h(y + row * out_stride + c * 32, a);
}

// ------------------------------------------------------------ per-head ops
// One wave per head of 128: lane l owns elements l and l + 64 (head_rrms in
// r4q_device.hpp).

__global__ __launch_bounds__(64) void head_rmsnorm_kernel(const uint16_t* __restrict__ q,
                                                          const uint16_t* __restrict__ k,
                                                          const uint16_t* __restrict__ qw,
                                                          const uint16_t* __restrict__ kw,
                                                          uint16_t* __restrict__ qo,
                                                          uint16_t* __restrict__ ko, int H,
                                                          float eps) {
#pragma clang fp contract(off)
  const int h = blockIdx.x, l = threadIdx.x;
  const bool isq = h < H;
  const uint16_t* src = isq ? q + h * 128 : k + (h - H) * 128;
  const uint16_t* w = isq ? qw : kw;
  uint16_t* dst = isq ? qo + h * 128 : ko + (h - H) * 128;
  const float x0 = h2f(src[l]), x1 = h2f(src[l + 64]);
  const float rr = head_rrms(x0, x1, eps);
  dst[l] = f2h((x0 * rr) * h2f(w[l]));
  dst[l + 64] = f2h((x1 * rr) * h2f(w[l + 64]));
}

__global__ __launch_bounds__(64) void rope_kernel(const uint16_t* __restrict__ q,
                                                  const uint16_t* __restrict__ k,
                                                  const uint16_t* __restrict__ cs,
                                                  const uint16_t* __restrict__ sn,
                                                  uint16_t* __restrict__ qo,
                                                  uint16_t* __restrict__ ko, int H) {
#pragma clang fp contract(off)
  const int h = blockIdx.x, l = threadIdx.x;
  const bool isq = h < H;
  const uint16_t* src = isq ? q + h * 128 : k + (h - H) * 128;
  uint16_t* dst = isq ? qo + h * 128 : ko + (h - H) * 128;
  const float e = h2f(src[l]), o = h2f(src[l + 64]);
  const float c = h2f(cs[l]), s = h2f(sn[l]);
  dst[l] = f2h(e * c - o * s);
  dst[l + 64] = f2h(o * c + e * s);
}

// QK RMSNorm + half-split RoPE + FP8 KV write; grid (H + Hk, B), one wave.
// Operation order (no contraction): t = x_l^2 + x_{l+64}^2, canonical wave
// sum, rrms = 1/sqrt(ss/128 + eps), ne = (x_l*rrms)*w_l,
// no = (x_{l+64}*rrms)*w_{l+64}, lo = ne*c - no*s, hi = no*c + ne*s;
// K code = fp8(lo * (1/k_scale)), V code = fp8(v * (1/v_scale)).
__global__ __launch_bounds__(64) void head_norm_rope_kv_kernel(
    const uint16_t* __restrict__ qkv, int64_t qkv_stride, const uint16_t* __restrict__ qw,
    const uint16_t* __restrict__ kw, uint16_t* __restrict__ qo, int64_t qo_stride,
    uint8_t* __restrict__ kc, uint8_t* __restrict__ vc, const float* __restrict__ ksc,
    const float* __restrict__ vsc, const uint16_t* __restrict__ cs,
    const uint16_t* __restrict__ sn, int H, int Hk, float eps, int max_seq, int pos_host,
    const int* __restrict__ pos_dev, int row_pos_step, int row_kv_step) {
#pragma clang fp contract(off)
  const int h = blockIdx.x, l = threadIdx.x;
  const int64_t b = blockIdx.y;
  // decode: every row at the same position, row b -> cache sequence b;
  // prefill: row b at position pos + b of cache sequence 0
  const int pos = (pos_dev ? *pos_dev : pos_host) + (int)b * row_pos_step;
  const int64_t kvb = b * row_kv_step;
  const uint16_t* row = qkv + b * qkv_stride;
  const float c = h2f_ieee(cs[(int64_t)pos * 64 + l]), s = h2f_ieee(sn[(int64_t)pos * 64 + l]);
  if (h < H + Hk) {
    const bool isq = h < H;
    const uint16_t* src = row + h * 128;  // q heads, then k heads
    const uint16_t* w = isq ? qw : kw;
    float lo, hi;
    head_norm_rope_pair(h2f_ieee(src[l]), h2f_ieee(src[l + 64]), h2f_ieee(w[l]),
                        h2f_ieee(w[l + 64]), c, s, eps, lo, hi);
    uint16_t* dst = qo + b * qo_stride + h * 128;
    dst[l] = f2h(lo);
    dst[l + 64] = f2h(hi);
    if (!isq && kc) {
      const int kh = h - H;
      const float inv = ksc ? 1.0f / ksc[kh] : 1.0f;
      uint8_t* kp = kc + ((kvb * Hk + kh) * (int64_t)max_seq + pos) * 128;
      kp[l] = (uint8_t)fp8_encode(lo * inv);
      kp[l + 64] = (uint8_t)fp8_encode(hi * inv);
    }
  } else if (vc) {
    const int kh = h - H - Hk;
    const uint16_t* src = row + (H + Hk + kh) * 128;
    const float inv = vsc ? 1.0f / vsc[kh] : 1.0f;
    uint8_t* vp = vc + ((kvb * Hk + kh) * (int64_t)max_seq + pos) * 128;
    vp[l] = (uint8_t)fp8_encode(h2f_ieee(src[l]) * inv);
    vp[l + 64] = (uint8_t)fp8_encode(h2f_ieee(src[l + 64]) * inv);
  }
}

}  // namespace

namespace {
bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <int MODE>
int rownorm(const void* a, const void* b, const void* w, void* y, void* res_out, int64_t rows,
            int64_t D, float eps, void* stream, const char* name) {
  R4Q_REQUIRE(a && w && y && rows >= 0, "%s: null pointer or negative rows", name);
  R4Q_REQUIRE(!(MODE & 1) || (b && res_out), "%s: residual pointers required", name);
  R4Q_REQUIRE(D > 0 && D % 32 == 0 && D <= 2 * 32 * 1024,
              "%s: D must be a positive multiple of 32 and <= 65536 (D=%lld)", name,
              (long long)D);
  R4Q_REQUIRE(al16(a) && al16(w) && al16(y) && (!(MODE & 1) || (al16(b) && al16(res_out))),
              "%s: pointers must be 16-byte aligned", name);
  if (rows == 0) return R4Q_OK;
  const int nch = (int)(D / 32);
  int threads = nch > 1024 ? 1024 : ((nch + 63) / 64) * 64;
  hipLaunchKernelGGL((rownorm_kernel<MODE>), dim3((unsigned)rows), dim3(threads), 0,
                     as_stream(stream), static_cast<const uint16_t*>(a),
                     static_cast<const uint16_t*>(b), static_cast<const uint16_t*>(w),
                     static_cast<uint16_t*>(y), static_cast<uint16_t*>(res_out), (int)D, eps);
  return launch_status(name);
}
}  // namespace

int launch_rownorm(int mode, const void* a, const void* b, const void* w, void* y,
                   void* res_out, int64_t rows, int64_t D, float eps, hipStream_t st) {
  switch (mode) {
    case 0: return rownorm<0>(a, b, w, y, res_out, rows, D, eps, st, "rmsnorm");
    case 1: return rownorm<1>(a, b, w, y, res_out, rows, D, eps, st, "res_rmsnorm");
    case 2: return rownorm<2>(a, b, w, y, res_out, rows, D, eps, st, "rmsnorm_fwht");
    default: return rownorm<3>(a, b, w, y, res_out, rows, D, eps, st, "res_rmsnorm_fwht");
  }
}

// Threads per rownorm_psum workgroup: 512 up to D = 5120 (4 float4 per plane
// thread, 192 chunk threads), 1024 up to D = 10240.
int psum_threads(int64_t D) { return D <= 5120 ? 512 : 1024; }

bool rownorm_psum_ok(int64_t D, int S) {
  return D % 32 == 0 && D > 0 && D <= 10240 && S >= 2 && S <= kPsumMaxS;
}

int launch_rownorm_psum(const float* ap, int64_t plane, int S, const void* b, const void* w,
                        void* y, void* res_out, int64_t rows, int64_t D, float eps,
                        hipStream_t st) {
  R4Q_REQUIRE(ap && b && w && y && res_out && rows >= 0, "res_rmsnorm_fwht (split sum): null pointer");
  R4Q_REQUIRE(rownorm_psum_ok(D, S), "res_rmsnorm_fwht (split sum): D=%lld S=%d unsupported",
              (long long)D, S);
  R4Q_REQUIRE(plane >= rows * D && al16(ap) && al16(b) && al16(w) && al16(y) && al16(res_out),
              "res_rmsnorm_fwht (split sum): bad plane or alignment");
  if (rows == 0) return R4Q_OK;
  const int nt = psum_threads(D), pt = nt / 8 * 5;
  const int kf = (int)((D / 4 + pt - 1) / pt);
#define R4Q_PSUM(NT, KF, SS)                                                                   \
  hipLaunchKernelGGL((rownorm_psum_kernel<NT, KF, SS>), dim3((unsigned)rows), dim3(NT), 0, st, \
                     ap, plane, static_cast<const uint16_t*>(b),                               \
                     static_cast<const uint16_t*>(w), static_cast<uint16_t*>(y),               \
                     static_cast<uint16_t*>(res_out), (int)D, eps)
#define R4Q_PSUM_S(NT, KF)            \
  switch (S) {                        \
    case 2: R4Q_PSUM(NT, KF, 2); break; \
    case 3: R4Q_PSUM(NT, KF, 3); break; \
    default: R4Q_PSUM(NT, KF, 4);       \
  }
#define R4Q_PSUM_K(NT)                \
  switch (kf) {                       \
    case 1: R4Q_PSUM_S(NT, 1); break; \
    case 2: R4Q_PSUM_S(NT, 2); break; \
    case 3: R4Q_PSUM_S(NT, 3); break; \
    default: R4Q_PSUM_S(NT, 4);       \
  }
  if (nt == 512) {
    R4Q_PSUM_K(512)
  } else {
    R4Q_PSUM_K(1024)
  }
#undef R4Q_PSUM_K
#undef R4Q_PSUM_S
#undef R4Q_PSUM
  return launch_status("res_rmsnorm_fwht (split sum)");
}

int launch_silu(bool fwht, const void* g, const void* u, void* y, int64_t rows, int64_t I,
                int64_t in_stride, int64_t out_stride, hipStream_t st) {
  R4Q_REQUIRE(g && u && y && rows >= 0, "silu_mul: null pointer");
  R4Q_REQUIRE(I > 0 && I % 32 == 0 && in_stride >= I && out_stride >= I &&
                  in_stride % 8 == 0 && out_stride % 8 == 0,
              "silu_mul: need I %% 32 == 0 and strides >= I, multiples of 8");
  R4Q_REQUIRE(al16(g) && al16(u) && al16(y), "silu_mul: pointers must be 16-byte aligned");
  if (rows == 0) return R4Q_OK;
  const int nch = (int)(I / 32);
  const dim3 grid((nch + 255) / 256, (unsigned)rows);
  if (fwht)
    hipLaunchKernelGGL((silu_kernel<true>), grid, dim3(256), 0, st,
                       static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(u),
                       static_cast<uint16_t*>(y), (int)I, in_stride, out_stride);
  else
    hipLaunchKernelGGL((silu_kernel<false>), grid, dim3(256), 0, st,
                       static_cast<const uint16_t*>(g), static_cast<const uint16_t*>(u),
                       static_cast<uint16_t*>(y), (int)I, in_stride, out_stride);
  return launch_status("silu_mul");
}

int check_head_norm_rope_kv(const void* qkv, const void* qw, const void* kw, const void* q_out,
                            const void* k_cache, const void* v_cache, const void* cos_t,
                            const void* sin_t, int64_t B, int64_t H, int64_t Hk, int64_t D,
                            int64_t max_seq, int64_t pos) {
  R4Q_REQUIRE(qkv && qw && kw && q_out && cos_t && sin_t, "head_norm_rope_kv: null pointer");
  R4Q_REQUIRE((k_cache == nullptr) == (v_cache == nullptr),
              "head_norm_rope_kv: pass both caches or neither");
  R4Q_REQUIRE(D == 128, "head_norm_rope_kv: head_dim must be 128 (got %lld)", (long long)D);
  R4Q_REQUIRE(B >= 1 && H >= 1 && Hk >= 1 && H % Hk == 0, "head_norm_rope_kv: bad head counts");
  R4Q_REQUIRE(pos >= 0 && (!k_cache || pos < max_seq),
              "head_norm_rope_kv: pos %lld outside the cache (max_seq %lld)", (long long)pos,
              (long long)max_seq);
  return R4Q_OK;
}

int launch_head_norm_rope_kv(const void* qkv, int64_t qkv_stride, const void* qw, const void* kw,
                             void* q_out, int64_t q_out_stride, void* k_cache, void* v_cache,
                             const float* k_scale, const float* v_scale, const void* cos_t,
                             const void* sin_t, int64_t B, int64_t H, int64_t Hk, float eps,
                             int64_t max_seq, int64_t pos, const int* pos_dev, hipStream_t st,
                             bool prefill_rows) {
  hipLaunchKernelGGL(head_norm_rope_kv_kernel, dim3((unsigned)(H + 2 * Hk), (unsigned)B),
                     dim3(64), 0, st, static_cast<const uint16_t*>(qkv), qkv_stride,
                     static_cast<const uint16_t*>(qw), static_cast<const uint16_t*>(kw),
                     static_cast<uint16_t*>(q_out), q_out_stride, static_cast<uint8_t*>(k_cache),
                     static_cast<uint8_t*>(v_cache), k_scale, v_scale,
                     static_cast<const uint16_t*>(cos_t), static_cast<const uint16_t*>(sin_t),
                     (int)H, (int)Hk, eps, (int)max_seq, (int)pos, pos_dev,
                     prefill_rows ? 1 : 0, prefill_rows ? 0 : 1);
  return launch_status("head_norm_rope_kv");
}

}  // namespace r4q

using namespace r4q;

extern "C" int r4q_rmsnorm(const void* x, const void* w, void* y, int64_t rows, int64_t D,
                           float eps, void* stream) {
  return launch_rownorm(0, x, nullptr, w, y, nullptr, rows, D, eps, as_stream(stream));
}

extern "C" int r4q_res_rmsnorm(const void* x, const void* res, const void* w, void* y,
                               void* res_out, int64_t rows, int64_t D, float eps, void* stream) {
  return launch_rownorm(1, x, res, w, y, res_out, rows, D, eps, as_stream(stream));
}

extern "C" int r4q_rmsnorm_fwht(const void* x, const void* w, void* y, int64_t rows, int64_t D,
                                float eps, void* stream) {
  return launch_rownorm(2, x, nullptr, w, y, nullptr, rows, D, eps, as_stream(stream));
}

extern "C" int r4q_res_rmsnorm_fwht(const void* a, const void* b, const void* w, void* y,
                                    void* res_out, int64_t rows, int64_t D, float eps,
                                    void* stream) {
  return launch_rownorm(3, a, b, w, y, res_out, rows, D, eps, as_stream(stream));
}

extern "C" int r4q_fwht32(const void* x, void* y, int64_t n, void* stream) {
  R4Q_REQUIRE(x && y, "fwht32: null pointer");
  R4Q_REQUIRE(n > 0 && n % 32 == 0, "fwht32: n must be a positive multiple of 32");
  R4Q_REQUIRE(al16(x) && al16(y), "fwht32: pointers must be 16-byte aligned");
  const int64_t nch = n / 32;
  hipLaunchKernelGGL(fwht32_kernel, dim3((unsigned)((nch + 255) / 256)), dim3(256), 0,
                     as_stream(stream), static_cast<const uint16_t*>(x),
                     static_cast<uint16_t*>(y), nch);
  return launch_status("fwht32");
}

extern "C" int r4q_silu_mul_fwht(const void* g, const void* u, void* y, int64_t rows, int64_t I,
                                 int64_t in_stride, int64_t out_stride, void* stream) {
  return launch_silu(true, g, u, y, rows, I, in_stride, out_stride, as_stream(stream));
}

extern "C" int r4q_silu_mul(const void* g, const void* u, void* y, int64_t rows, int64_t I,
                            int64_t in_stride, int64_t out_stride, void* stream) {
  return launch_silu(false, g, u, y, rows, I, in_stride, out_stride, as_stream(stream));
}

extern "C" int r4q_head_rmsnorm(const void* q, const void* k, const void* qw, const void* kw,
                                void* q_out, void* k_out, int64_t H, int64_t Hk, int64_t D,
                                float eps, void* stream) {
  R4Q_REQUIRE(q && k && qw && kw && q_out && k_out, "head_rmsnorm: null pointer");
  R4Q_REQUIRE(D == 128, "head_rmsnorm: head_dim must be 128");
  R4Q_REQUIRE(H >= 1 && Hk >= 0, "head_rmsnorm: bad head counts");
  hipLaunchKernelGGL(head_rmsnorm_kernel, dim3((unsigned)(H + Hk)), dim3(64), 0,
                     as_stream(stream), static_cast<const uint16_t*>(q),
                     static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(qw),
                     static_cast<const uint16_t*>(kw), static_cast<uint16_t*>(q_out),
                     static_cast<uint16_t*>(k_out), (int)H, eps);
  return launch_status("head_rmsnorm");
}

extern "C" int r4q_rope(const void* q, const void* k, const void* cos_t, const void* sin_t,
                        void* q_out, void* k_out, int64_t H, int64_t Hk, int64_t D, int64_t pos,
                        void* stream) {
  R4Q_REQUIRE(q && k && cos_t && sin_t && q_out && k_out, "rope: null pointer");
  R4Q_REQUIRE(D == 128, "rope: head_dim must be 128");
  R4Q_REQUIRE(pos >= 0 && H >= 1 && Hk >= 0, "rope: bad arguments");
  const uint16_t* c = static_cast<const uint16_t*>(cos_t) + pos * 64;
  const uint16_t* s = static_cast<const uint16_t*>(sin_t) + pos * 64;
  hipLaunchKernelGGL(rope_kernel, dim3((unsigned)(H + Hk)), dim3(64), 0, as_stream(stream),
                     static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), c, s,
                     static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_out), (int)H);
  return launch_status("rope");
}

extern "C" int r4q_head_norm_rope_kv(const void* qkv, int64_t qkv_stride, const void* qw,
                                     const void* kw, void* q_out, int64_t q_out_stride,
                                     void* k_cache, void* v_cache, const float* k_scale,
                                     const float* v_scale, const void* cos_t, const void* sin_t,
                                     int64_t B, int64_t H, int64_t Hk, int64_t D, float eps,
                                     int64_t max_seq, int64_t pos, void* stream) {
  R4Q_TRY(check_head_norm_rope_kv(qkv, qw, kw, q_out, k_cache, v_cache, cos_t, sin_t, B, H, Hk,
                                  D, max_seq, pos));
  R4Q_REQUIRE(qkv_stride >= (H + 2 * Hk) * D && q_out_stride >= (H + Hk) * D,
              "head_norm_rope_kv: row strides too small");
  return launch_head_norm_rope_kv(qkv, qkv_stride, qw, kw, q_out, q_out_stride, k_cache, v_cache,
                                  k_scale, v_scale, cos_t, sin_t, B, H, Hk, eps, max_seq, pos,
                                  nullptr, as_stream(stream));
}
