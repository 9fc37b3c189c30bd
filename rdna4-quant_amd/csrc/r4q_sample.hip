// Temperature + top-p (nucleus) sampling of the next token on the device.
//
// Semantics of the reference's Python sampler (int4_engine_v5.py:387-399):
//   z = float(logits) / temperature;
//   if top_p < 1: sort z descending, drop every token whose cumulative
//                 softmax probability *before* it is >= top_p;
//   draw one token from softmax over the kept tokens.
// temperature <= 0 is the greedy argmax (int4_engine_v5.py:352-353), served
// by the argmax kernels of the decode step.
//
// gfx950 design.  fp16 logits take at most 65,536 distinct values, and the
// order-preserving 16-bit key of a value ranks it exactly, so
//  * sample_hist_kernel builds an integer histogram of the keys (one
//    65,536-bin table per row; atomics on integers are order-independent, so
//    every result below is deterministic);
//  * sample_select_kernel (one 1024-thread workgroup per row) scans the bins
//    from the largest key down: per-bin mass = count * exp(z_b - z_max), the
//    top-p cutoff per bin (tokens tied in a bin are ranked by index, like a
//    stable descending sort), the kept mass, and the draw: u * kept mass
//    lands in one bin at one tie rank.  It zeroes its bins for the next call;
//  * sample_pick_kernel finds the token with that key and tie rank (lowest
//    index first), writes its id and, for the decode loop, gathers its
//    embedding row into the next step's hidden state.
// u is a counter-based uniform draw: x = splitmix64(seed ^ counter), then
// splitmix64(x ^ row), u = top 24 bits / 2^24 -- reproducible from (seed,
// position, row) without any RNG state.
#include <math.h>

#include "r4q_ctx.hpp"
#include "r4q_device.hpp"
#include "r4q_host.hpp"
#include "r4q_kernels.hpp"

namespace r4q {
namespace {

constexpr int kBins = 65536;
constexpr int kSelThreads = 1024;
constexpr int kBinsPerThread = kBins / kSelThreads;  // 64
constexpr int kHistBlocks = 64;
// Workspace layout, independent of B so that a table written zero by one
// call is still zero for a call with more rows: the selection words of up
// to kMaxRows rows first, then one table per row.
constexpr int kMaxRows = 1024;
constexpr size_t kSelBytes = (size_t)kMaxRows * 8;

// Order-preserving key of an fp16 bit pattern: larger value, larger key;
// -0 is taken as +0 so that equal values share a key (NaN is not a valid
// logit).
__device__ __forceinline__ uint32_t key16(uint32_t h) {
  if (h == 0x8000u) h = 0u;
  return (h & 0x8000u) ? (~h & 0xFFFFu) : (h | 0x8000u);
}
__device__ __forceinline__ uint32_t unkey16(uint32_t k) {
  return (k & 0x8000u) ? (k & 0x7FFFu) : (~k & 0xFFFFu);
}

// splitmix64 finalizer (S. Vigna, public domain).
__device__ __forceinline__ uint64_t mix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

__global__ __launch_bounds__(256) void sample_hist_kernel(const uint16_t* __restrict__ logits,
                                                          int64_t V, int64_t stride,
                                                          uint32_t* __restrict__ hist) {
  const int64_t b = blockIdx.y;
  const int64_t per = (V + gridDim.x - 1) / gridDim.x;
  const int64_t lo = blockIdx.x * per, hi = min(V, lo + per);
  uint32_t* hb = hist + b * kBins;
  for (int64_t i = lo + threadIdx.x; i < hi; i += blockDim.x)
    atomicAdd(&hb[key16(logits[b * stride + i])], 1u);
}

// Exclusive scan of one float per thread in a fixed order (thread order),
// returning the prefix and setting *total.
__device__ float block_exclusive_scan(float v, float* buf, float* total) {
  const int t = threadIdx.x;
  buf[t] = v;
  __syncthreads();
  // Hillis-Steele over 1024 entries; each step's adds happen in a fixed order
  for (int off = 1; off < kSelThreads; off <<= 1) {
    const float add = t >= off ? buf[t - off] : 0.f;
    __syncthreads();
    buf[t] += add;
    __syncthreads();
  }
  const float incl = buf[t];
  *total = buf[kSelThreads - 1];
  __syncthreads();
  return incl - v;
}

// Per row: cutoff, kept mass, the draw.  sel[b] = {key, tie rank}.  Thread
// t owns bins r = 64t .. 64t+63 in descending key order (key = 65535 - r);
// every pass re-reads its counts (the table stays in L2) and recomputes the
// same per-bin quantities, so nothing per bin is held in registers.
__global__ __launch_bounds__(kSelThreads) void sample_select_kernel(
    uint32_t* __restrict__ hist, float temperature, float top_p, uint64_t seed,
    const int* __restrict__ counter_dev, int64_t counter_host, int* __restrict__ sel) {
  const int b = blockIdx.x, t = threadIdx.x;
  uint32_t* hb = hist + (int64_t)b * kBins;
  __shared__ float buf[kSelThreads];
  __shared__ int kmax_s, owner;
  const int r0 = kBinsPerThread * t;
  auto count = [&](int j) { return hb[kBins - 1 - (r0 + j)]; };
  auto zval = [&](int r) {  // logit / temperature of the bin at descending rank r
    return h2f((uint16_t)unkey16((uint32_t)(kBins - 1 - r))) / temperature;
  };
  // largest occupied key (the logits are finite: some bin is occupied)
  int first = kBins;
  for (int j = kBinsPerThread - 1; j >= 0; --j)
    if (count(j)) first = r0 + j;
  if (t == 0) {
    kmax_s = kBins;
    owner = -1;
  }
  __syncthreads();
  atomicMin(&kmax_s, first);
  __syncthreads();
  if (temperature <= 0.f) {  // greedy: the largest value at tie rank 0 (lowest index)
    if (t == 0) {
      sel[2 * b] = kBins - 1 - kmax_s;
      sel[2 * b + 1] = 0;
    }
    __syncthreads();
    for (int j = 0; j < kBinsPerThread; ++j)
      if (count(j)) hb[kBins - 1 - (r0 + j)] = 0u;
    return;
  }
  const float zmax = zval(kmax_s);
  // pass 1: this thread's softmax mass (unnormalised) and the row total Z
  float mass = 0.f;
  for (int j = 0; j < kBinsPerThread; ++j) {
    const uint32_t c = count(j);
    if (c) mass = __builtin_fmaf((float)c, __expf(zval(r0 + j) - zmax), mass);
  }
  float Z;
  const float before = block_exclusive_scan(mass, buf, &Z);
  // pass 2: tokens kept by top-p.  The token at tie rank k of a bin with
  // per-token mass w and mass S before the bin is kept iff S + k w < top_p Z.
  const bool cut = top_p < 1.0f;
  const float lim = top_p * Z;
  auto kept_in = [&](uint32_t c, float w, float S) {
    if (w == 0.f) return 0;  // underflowed: no mass to draw
    if (!cut) return (int)c;
    const float r = (lim - S) / w;  // ranks k < r are kept
    return r <= 0.f ? 0 : (r >= (float)c ? (int)c : (int)ceilf(r));
  };
  float S = before, kept = 0.f;
  for (int j = 0; j < kBinsPerThread; ++j) {
    const uint32_t c = count(j);
    if (c) {
      const float w = __expf(zval(r0 + j) - zmax);
      kept = __builtin_fmaf((float)kept_in(c, w, S), w, kept);
      S = __builtin_fmaf((float)c, w, S);
    }
  }
  float K;
  const float kbefore = block_exclusive_scan(kept, buf, &K);
  // pass 3: the draw, target = u * K in kept mass, walked in descending key
  // order and, inside a bin, by tie rank
  const uint64_t ctr = counter_dev ? (uint64_t)(int64_t)*counter_dev : (uint64_t)counter_host;
  const uint64_t x = mix64(mix64(seed ^ ctr) ^ (uint64_t)b);
  const float u = (float)(x >> 40) * (1.0f / 16777216.0f);
  const float target = u * K;
  // owner: the last thread with kept mass whose range starts at or below the
  // target (rounding at a range end falls to that thread's last kept token)
  if (kept > 0.f && kbefore <= target) atomicMax(&owner, t);
  __syncthreads();
  if (t == owner) {
    float Sb = before, C = kbefore;
    int jb = -1, rank = 0, jlast = -1, klast = 0;
    for (int j = 0; j < kBinsPerThread && jb < 0; ++j) {
      const uint32_t c = count(j);
      if (!c) continue;
      const float w = __expf(zval(r0 + j) - zmax);
      const int k = kept_in(c, w, Sb);
      Sb = __builtin_fmaf((float)c, w, Sb);
      if (k == 0) continue;
      jlast = j;
      klast = k;
      const float end = __builtin_fmaf((float)k, w, C);
      if (target < end) {
        jb = j;
        const int q = (int)floorf((target - C) / w);
        rank = q < 0 ? 0 : (q >= k ? k - 1 : q);
      }
      C = end;
    }
    if (jb < 0) {  // past the last kept bin by rounding
      jb = jlast;
      rank = klast - 1;
    }
    sel[2 * b] = kBins - 1 - (r0 + jb);
    sel[2 * b + 1] = rank;
  }
  __syncthreads();
  // leave the table zeroed for the next call (each thread clears its bins)
  for (int j = 0; j < kBinsPerThread; ++j)
    if (count(j)) hb[kBins - 1 - (r0 + j)] = 0u;
}

// The token of key sel[b].x with tie rank sel[b].y (lowest index first).
__global__ __launch_bounds__(kSelThreads) void sample_pick_kernel(
    const uint16_t* __restrict__ logits, int64_t V, int64_t stride, const int* __restrict__ sel,
    int64_t* __restrict__ ids, const uint16_t* __restrict__ embed, int D, uint16_t* __restrict__ h,
    int64_t* __restrict__ tokens_out, const int* __restrict__ state, int step_host, int B) {
  const int b = blockIdx.x, t = threadIdx.x;
  const uint32_t key = (uint32_t)sel[2 * b];
  const int rank = sel[2 * b + 1];
  const int64_t per = (V + kSelThreads - 1) / kSelThreads;
  const int64_t lo = t * per, hi = min(V, lo + per);
  const uint16_t* row = logits + (int64_t)b * stride;
  int n = 0;
  for (int64_t i = lo; i < hi; ++i) n += key16(row[i]) == key;
  __shared__ float buf[kSelThreads];
  float tot;
  const int before = (int)block_exclusive_scan((float)n, buf, &tot);  // counts < 2^24: exact
  __shared__ int tok;
  if (t == 0) tok = 0;
  __syncthreads();
  if (n > 0 && before <= rank && rank < before + n) {
    int k = rank - before;
    for (int64_t i = lo; i < hi; ++i)
      if (key16(row[i]) == key && k-- == 0) {
        tok = (int)i;
        break;
      }
  }
  __syncthreads();
  if (t == 0) {
    ids[b] = tok;
    const int step = state ? state[kStep] : step_host;
    if (tokens_out) tokens_out[(int64_t)step * B + b] = tok;
  }
  if (embed) {
    const u4_t* src = reinterpret_cast<const u4_t*>(embed + (int64_t)tok * D);
    u4_t* dst = reinterpret_cast<u4_t*>(h + (int64_t)b * D);
    for (int i = t; i < D / 8; i += kSelThreads) dst[i] = src[i];
  }
}

__global__ void zero_u32_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0u;
}

}  // namespace

size_t sample_ws_bytes(int64_t B) { return kSelBytes + (size_t)B * kBins * 4; }

int sample_reserve(r4q_ctx* ctx, int64_t B, hipStream_t st, void** ws) {
  const size_t need = sample_ws_bytes(B);
  const void* old = ctx->sample.ptr;
  R4Q_TRY(ctx->sample.reserve(need));
  if (ctx->sample.ptr != old || ctx->sample_zeroed < need) {
    const int64_t n = (int64_t)(ctx->sample.bytes / 4);
    hipLaunchKernelGGL(zero_u32_kernel, dim3(256), dim3(256), 0, st,
                       static_cast<uint32_t*>(ctx->sample.ptr), n);
    R4Q_TRY(launch_status("sample_reserve"));
    ctx->sample_zeroed = ctx->sample.bytes;
  }
  *ws = ctx->sample.ptr;
  return R4Q_OK;
}

int launch_sample(const void* logits, int64_t B, int64_t V, int64_t stride, const SampleCfg& cfg,
                  const int* counter_dev, int64_t counter_host, void* ws, int64_t* ids,
                  const void* embed, int64_t D, void* h, int64_t* tokens_out, const int* state,
                  int step_host, hipStream_t st) {
  R4Q_REQUIRE(cfg.top_p > 0.f, "sample: top_p must be > 0");
  R4Q_REQUIRE(V >= 1 && V < (1LL << 31) && stride >= V, "sample: bad vocabulary size / stride");
  R4Q_REQUIRE(!embed || (D % 8 == 0), "sample: embedding width must be a multiple of 8");
  R4Q_REQUIRE(B <= kMaxRows, "sample: at most %d rows per call (got %lld)", kMaxRows,
              (long long)B);
  int* sel = static_cast<int*>(ws);
  uint32_t* hist = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(ws) + kSelBytes);
  const auto* lg = static_cast<const uint16_t*>(logits);
  hipLaunchKernelGGL(sample_hist_kernel, dim3(kHistBlocks, (unsigned)B), dim3(256), 0, st, lg, V,
                     stride, hist);
  R4Q_TRY(launch_status("sample_hist"));
  hipLaunchKernelGGL(sample_select_kernel, dim3((unsigned)B), dim3(kSelThreads), 0, st, hist,
                     cfg.temperature, cfg.top_p, cfg.seed, counter_dev, counter_host, sel);
  R4Q_TRY(launch_status("sample_select"));
  hipLaunchKernelGGL(sample_pick_kernel, dim3((unsigned)B), dim3(kSelThreads), 0, st, lg, V,
                     stride, sel, ids, static_cast<const uint16_t*>(embed), (int)D,
                     static_cast<uint16_t*>(h), tokens_out, state, step_host, (int)B);
  return launch_status("sample_pick");
}

}  // namespace r4q

extern "C" int r4q_sample(r4q_ctx* ctx, const void* logits, int64_t B, int64_t V, int64_t stride,
                          float temperature, float top_p, uint64_t seed, int64_t counter,
                          int64_t* ids_out, void* stream) {
  R4Q_REQUIRE(ctx && logits && ids_out, "sample: null argument");
  R4Q_REQUIRE(B >= 1, "sample: B must be >= 1");
  R4Q_REQUIRE((reinterpret_cast<uintptr_t>(logits) & 1) == 0, "sample: logits must be fp16");
  const hipStream_t st = r4q::as_stream(stream);
  void* ws = nullptr;
  R4Q_TRY(r4q::sample_reserve(ctx, B, st, &ws));
  const int rc = r4q::launch_sample(logits, B, V, stride, r4q::SampleCfg{temperature, top_p, seed},
                                    nullptr, counter, ws, ids_out, nullptr, 0, nullptr, nullptr,
                                    nullptr, 0, st);
  if (rc != R4Q_OK) ctx->sample_zeroed = 0;  // a partial run may leave counts behind
  return rc;
}
