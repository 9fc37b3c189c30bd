// Decode-step orchestration: one token (or B tokens, one per sequence)
// through every layer, the LM head, on-device greedy sampling, hipGraph
// capture/replay and the per-category HIP-event profile.
//
// Replaces int4_decode_step / int4_decode_step_logits (hip:2343-2595),
// int4_decode_bench (hip:2601-2795), int4_decode_bench_graph (hip:2801-3041),
// int4_decode_profile (hip:3047-3273) and int4_decode_loop (hip:3284-3466).
//
// Per layer (same dataflow as the reference, hip:2474-2524):
//   rot -> QKV linear -> QK-norm + RoPE + FP8 KV write -> flash-decode
//   (+FWHT) -> O linear -> residual + post-norm + FWHT -> gate/up linear ->
//   SiLU-gate + FWHT -> down linear -> residual + next layer's input norm +
//   FWHT.
// Every decode path splits attention by the cache capacity (split length =
// ceil(len / nsplit), computed on the device), so the eager step, the eager
// loop and the captured graph run the same arithmetic for a given position.
// The graph path keeps the position, sequence length and step counter in
// device memory; argmax, the embedding gather and the position advance run
// inside the graph, so replaying N tokens needs no host work per token.
#include <string.h>

#include <algorithm>
#include <cstddef>
#include <utility>
#include <vector>

#include "r4q_ctx.hpp"
#include "r4q_device.hpp"
#include "r4q_gemv.hpp"
#include "r4q_host.hpp"
#include "r4q_kernels.hpp"

namespace r4q {

// Captured graphs of a context, keyed by everything they bake in (model,
// shape, buffer addresses); the least recently used one is dropped when the
// cache is full.  All replay on one private stream.
struct GraphCache {
  static constexpr size_t kMax = 4;
  struct Entry {
    std::vector<uint8_t> key;
    hipGraphExec_t exec = nullptr;
    uint64_t used = 0;
  };
  hipStream_t stream = nullptr;
  hipEvent_t ev_in = nullptr, ev_out = nullptr;  // caller stream -> graph stream -> caller
  std::vector<Entry> entries;
  uint64_t clock = 0;
  hipGraphExec_t find(const std::vector<uint8_t>& key) {
    for (Entry& e : entries)
      if (e.key == key) {
        e.used = ++clock;
        return e.exec;
      }
    return nullptr;
  }
  void insert(std::vector<uint8_t> key, hipGraphExec_t exec) {
    if (entries.size() >= kMax) {
      size_t lru = 0;
      for (size_t i = 1; i < entries.size(); ++i)
        if (entries[i].used < entries[lru].used) lru = i;
      // replays of the evicted graph may still be queued on the stream
      // (the decode loops return with up to kInFlight of them in flight)
      (void)hipStreamSynchronize(stream);
      (void)hipGraphExecDestroy(entries[lru].exec);
      entries.erase(entries.begin() + (std::ptrdiff_t)lru);
    }
    entries.push_back(Entry{std::move(key), exec, ++clock});
  }
  ~GraphCache() {
    for (Entry& e : entries) (void)hipGraphExecDestroy(e.exec);
    if (ev_in) (void)hipEventDestroy(ev_in);
    if (ev_out) (void)hipEventDestroy(ev_out);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

void destroy_graphs(r4q_ctx* ctx) {
  delete ctx->graphs;
  ctx->graphs = nullptr;
}

namespace {

struct Dims {
  int L, H, Hk, hd, D, I, qkvN, qd;
  float eps;
  int max_seq;
};

struct Bufs {
  uint16_t *h, *r, *rot, *qkv, *o, *gu, *y, *d, *logits;
  void* ws = nullptr;  // split-K partials of the batched projections
  size_t ws_bytes = 0;
  void* tail = nullptr;  // batched gate/up: tail-piece counters + partials
  float* attn;
  int* state;
  int64_t* ids;
  float* amax;  // argmax partials
};

constexpr int kArgmaxBlocks = 64;  // <= 64: stage 2 reduces them in one wave

int validate(const r4q_model* m, int64_t B, Dims& dm) {
  R4Q_REQUIRE(m && m->layers, "decode: null model");
  R4Q_REQUIRE(B >= 1 && B <= 64, "decode: batch must be in [1, 64] (got %lld)", (long long)B);
  dm.L = m->n_layers;
  dm.H = m->n_heads;
  dm.Hk = m->n_kv_heads;
  dm.hd = m->head_dim;
  dm.D = m->hidden;
  dm.I = m->inter;
  dm.eps = m->eps;
  dm.max_seq = m->max_seq;
  R4Q_REQUIRE(dm.L >= 1 && dm.H >= 1 && dm.Hk >= 1 && dm.H % dm.Hk == 0,
              "decode: bad layer/head counts");
  R4Q_REQUIRE(dm.hd == 128, "decode: head_dim must be 128");
  R4Q_REQUIRE(dm.D % 32 == 0 && dm.I % 32 == 0 && dm.D > 0 && dm.I > 0,
              "decode: hidden and intermediate sizes must be multiples of 32");
  R4Q_REQUIRE(m->rope_cos && m->rope_sin && m->rope_len >= 1, "decode: missing RoPE tables");
  dm.qd = dm.H * dm.hd;
  dm.qkvN = (dm.H + 2 * dm.Hk) * dm.hd;
  for (int li = 0; li < dm.L; ++li) {
    const r4q_layer& y = m->layers[li];
    R4Q_REQUIRE(y.qkv_N == dm.qkvN && y.o_N == dm.D && y.gu_N == 2 * (int64_t)dm.I &&
                    y.down_N == dm.D,
                "decode: layer %d output sizes do not match the model dims", li);
    R4Q_TRY(gemv_check(y.qkv_w, y.qkv_w, y.qkv_s, y.qkv_w, y.qkv_N, dm.D, y.qkv_bits));
    R4Q_TRY(gemv_check(y.o_w, y.o_w, y.o_s, y.o_w, y.o_N, dm.qd, y.o_bits));
    R4Q_TRY(gemv_check(y.gu_w, y.gu_w, y.gu_s, y.gu_w, y.gu_N, dm.D, y.gu_bits));
    R4Q_TRY(gemv_check(y.down_w, y.down_w, y.down_s, y.down_w, y.down_N, dm.I, y.down_bits));
    R4Q_REQUIRE(y.in_norm && y.post_norm && y.q_norm && y.k_norm && y.k_cache && y.v_cache,
                "decode: layer %d has a null norm weight or cache", li);
  }
  if (m->final_norm) {
    R4Q_REQUIRE(m->lm_K == dm.D, "decode: lm_K must equal hidden");
    R4Q_TRY(gemv_check(m->lm_w, m->lm_w, m->lm_s, m->lm_w, m->lm_N, m->lm_K, m->lm_bits));
  }
  return R4Q_OK;
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// Workspace of the batched projections (split-K partials): the largest any
// of the step's matrices asks for (none at batch 1).
size_t step_gemm_ws(const r4q_model* m, const Dims& dm, int64_t B) {
  size_t gws = 0;
  if (B > 1) {
    auto need = [&](int64_t N, int64_t K, int bits) {
      gws = std::max(gws, gemm_ws_need(B, N, K, bits));
    };
    for (int li = 0; li < dm.L; ++li) {
      const r4q_layer& y = m->layers[li];
      need(dm.qkvN, dm.D, y.qkv_bits);
      need(dm.D, dm.qd, y.o_bits);
      need(2 * (int64_t)dm.I, dm.D, y.gu_bits);
      need(dm.D, dm.I, y.down_bits);
    }
    if (m->final_norm) need(m->lm_N, m->lm_K, m->lm_bits);
  }
  return gws;
}

// Batched gate/up with the SiLU epilogue: workspace of its tail pieces (the
// largest any layer's width asks for; 0 when no layer has a tail).
size_t step_tail_ws(const r4q_model* m, const Dims& dm, int64_t B) {
  size_t t = 0;
  if (B > 1 && B <= 8)
    for (int li = 0; li < dm.L; ++li) {
      const int bits = m->layers[li].gu_bits;
      if (bits != 16) t = std::max(t, skinny_silu_tail_bytes(dm.I, dm.D, bits));
    }
  return t;
}

__global__ void zero_words_kernel(uint32_t* p, int64_t n) {
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0u;
}

int reserve(r4q_ctx* ctx, const r4q_model* m, const Dims& dm, int64_t B, int nsplit, hipStream_t st,
            Bufs& bf) {
  const size_t D = dm.D, I = dm.I;
  const size_t lmN = m->final_norm ? (size_t)m->lm_N : 0;
  const size_t rotw = dm.qd > dm.D ? dm.qd : dm.D;
  const size_t sizes[] = {B * D, B * D, B * rotw, B * (size_t)dm.qkvN, B * D, B * 2 * I,
                          B * I, B * D, B * lmN};
  size_t total = 0;
  for (size_t s : sizes) total += align256(s * 2);
  const size_t gws = step_gemm_ws(m, dm, B), tws = step_tail_ws(m, dm, B);
  const void* old = ctx->step.ptr;
  R4Q_TRY(ctx->step.reserve(total + align256(gws) + tws));
  uint16_t** dst[] = {&bf.h, &bf.r, &bf.rot, &bf.qkv, &bf.o, &bf.gu, &bf.y, &bf.d, &bf.logits};
  uint8_t* p = static_cast<uint8_t*>(ctx->step.ptr);
  for (int i = 0; i < 9; ++i) {
    *dst[i] = reinterpret_cast<uint16_t*>(p);
    p += align256(sizes[i] * 2);
  }
  bf.ws = gws ? p : nullptr;
  bf.ws_bytes = gws;
  bf.tail = tws ? p + align256(gws) : nullptr;
  // the tail counters start at zero and every launch leaves them at zero;
  // a layout without them (another batch size) may have put other data there
  if (bf.tail && (ctx->step.ptr != old || ctx->tail_zeroed != bf.tail)) {
    hipLaunchKernelGGL(zero_words_kernel, dim3(1), dim3(256), 0, st,
                       static_cast<uint32_t*>(bf.tail),
                       (int64_t)(skinny_silu_tail_cnt_bytes(dm.I) / 4));
    R4Q_TRY(launch_status("decode workspace"));
  }
  ctx->tail_zeroed = bf.tail;
  R4Q_TRY(ctx->attn.reserve(attn_ws_bytes(B, dm.H, nsplit)));
  bf.attn = static_cast<float*>(ctx->attn.ptr);
  const size_t misc = align256(kStateWords * 4) + align256(B * 8) +
                      align256((size_t)B * kArgmaxBlocks * 8);
  R4Q_TRY(ctx->misc.reserve(misc));
  uint8_t* q = static_cast<uint8_t*>(ctx->misc.ptr);
  bf.state = reinterpret_cast<int*>(q);
  bf.ids = reinterpret_cast<int64_t*>(q + align256(kStateWords * 4));
  bf.amax = reinterpret_cast<float*>(q + align256(kStateWords * 4) + align256(B * 8));
  return R4Q_OK;
}

// Batched gate/up: the unsplit skinny GEMM with the SiLU gate in its
// epilogue when it has a workgroup per CU or more (I / 32 tiles), else the
// split GEMM whose reduce applies the gate.  Measured at 8 rows, 17408 x
// 5120 (GEMM + gate, us): INT4 31.8 + epilogue against 29.8 + 6.2, INT8
// 52.8 against 48.8 + 6.2.
bool silu_epilogue(int64_t B, int64_t I) { return B <= 8 && I / 32 >= 256; }

int linear(const void* x, const void* w, const void* s, void* y, int64_t B, int64_t N, int64_t K,
           int bits, hipStream_t st, const Bufs& bf) {
  if (B == 1) return gemv_launch(x, w, s, y, N, K, bits, st);
  return gemm_launch(x, w, s, y, B, N, K, bits, st, bf.ws, bf.ws_bytes);
}

// Optional event recorder for the per-category profile.
// Optional per-segment timing: mark(st, cat) records an event that starts a
// segment of category cat (kGemv, kAttn, kNorm, kRest); the segment ends at
// the next mark.
enum ProfCat { kGemv = 0, kAttn = 1, kNorm = 2, kRest = 3, kEnd = -1 };
struct Prof {
  std::vector<hipEvent_t>* ev = nullptr;
  std::vector<int>* cat = nullptr;
  void mark(hipStream_t st, int c) {
    if (!ev) return;
    hipEvent_t e;
    (void)hipEventCreate(&e);
    (void)hipEventRecord(e, st);
    ev->push_back(e);
    cat->push_back(c);
  }
};

// Enqueues one decode step for B rows.  pos_dev/seq_dev: device-held
// position and length (graph replay), else pos_host.  Input hidden states
// must already be in bf.h.
// Batched steps (B > 1): the K-split partials of a skinny projection are
// summed by the kernel consuming them -- the attention prologue (qkv), the
// residual + row norm (o, down) -- when the skinny GEMM splits K into 2..
// that kernel's maximum.  Returns the split count S, or 0 (own reduce).
enum Consumer { kToAttention, kToRowNorm };
int consumer_split(int64_t B, int64_t N, int64_t K, int bits, size_t ws_bytes, Consumer c) {
  if (B == 1 || tuning().split_reduce.load() != 0 || !gemm_skinny_ok(B, N, K, bits)) return 0;
  const int S = skinny_splits(B, N, K, bits, ws_bytes);
  if (S < 2) return 0;
  if (c == kToAttention) return S <= kMaxQkvSplits ? S : 0;
  return rownorm_psum_ok(N, S) ? S : 0;
}

// a projection whose partials its consumer sums: launches the GEMM without
// its reduce and returns S (0: the ordinary launch, y written)
int project(const void* x, const void* w, const void* s, void* y, int64_t B, int64_t N,
            int64_t K, int bits, hipStream_t st, const Bufs& bf, Consumer c, int* S) {
  *S = consumer_split(B, N, K, bits, bf.ws_bytes, c);
  if (*S == 0) return linear(x, w, s, y, B, N, K, bits, st, bf);
  int got = 0;
  R4Q_TRY(gemm_skinny_part_launch(x, w, s, y, B, N, K, bits, st, bf.ws, bf.ws_bytes, &got));
  R4Q_REQUIRE(got == *S, "skinny GEMM split count changed (%d, expected %d)", got, *S);
  return R4Q_OK;
}

// residual + RMSNorm + FWHT-32 of row input a (or of the S split partials of
// the projection that produced it)
int rownorm3(const void* a, int S, const void* b, const void* w, void* y, void* res_out,
             int64_t B, int64_t D, float eps, hipStream_t st, const Bufs& bf) {
  if (S >= 2)
    return launch_rownorm_psum(static_cast<const float*>(bf.ws), B * D, S, b, w, y, res_out, B,
                               D, eps, st);
  return launch_rownorm(3, a, b, w, y, res_out, B, D, eps, st);
}

int enqueue_step(const r4q_model* m, const Dims& dm, int64_t B, int64_t pos_host,
                 const int* pos_dev, const int* seq_dev, int nsplit, const Bufs& bf, bool logits,
                 hipStream_t st, Prof prof = Prof()) {
  const int64_t D = dm.D, I = dm.I;
  const float eps = dm.eps;
  // Batch 1 folds every residual + RMSNorm + FWHT into the activation
  // staging of the GEMV that consumes it (gemv_norm_launch); batches keep
  // the separate row-norm kernel in front of the multi-row linear.
  const bool fused = (B == 1);
  if (!fused) {
    prof.mark(st, kNorm);
    R4Q_TRY(launch_rownorm(2, bf.h, nullptr, m->layers[0].in_norm, bf.rot, nullptr, B, D, eps,
                           st));
  }
  for (int li = 0; li < dm.L; ++li) {
    const r4q_layer& y = m->layers[li];
    prof.mark(st, kGemv);
    // batches: a split-K skinny qkv projection leaves its fp32 partials for
    // the attention prologue to sum (no reduce launch)
    int qkv_nsum = 0;
    if (!fused) {
      R4Q_TRY(project(bf.rot, y.qkv_w, y.qkv_s, bf.qkv, B, dm.qkvN, D, y.qkv_bits, st, bf,
                      kToAttention, &qkv_nsum));
    } else if (li == 0) {  // input hidden state: plain RMSNorm
      R4Q_TRY(gemv_norm_launch(bf.h, nullptr, y.in_norm, nullptr, eps, y.qkv_w, y.qkv_s, bf.qkv,
                               dm.qkvN, D, y.qkv_bits, st));
    } else {  // h = fp16(d + r), then RMSNorm
      R4Q_TRY(gemv_norm_launch(bf.d, bf.r, y.in_norm, bf.h, eps, y.qkv_w, y.qkv_s, bf.qkv,
                               dm.qkvN, D, y.qkv_bits, st));
    }
    // head RMSNorm + RoPE of q/k and the FP8 K/V write at pos run in the
    // attention kernel's prologue (raw QKV rows in)
    prof.mark(st, kAttn);
    const AttnQK qk{static_cast<const uint16_t*>(y.q_norm), static_cast<const uint16_t*>(y.k_norm),
                    static_cast<const uint16_t*>(m->rope_cos),
                    static_cast<const uint16_t*>(m->rope_sin), static_cast<uint8_t*>(y.k_cache),
                    static_cast<uint8_t*>(y.v_cache), eps,
                    qkv_nsum >= 2 ? static_cast<const float*>(bf.ws) : nullptr,
                    B * dm.qkvN, qkv_nsum >= 2 ? qkv_nsum : 0};
    R4Q_TRY(launch_flash_decode(bf.qkv, dm.qkvN, y.k_cache, y.v_cache, y.k_scale, y.v_scale,
                                bf.rot, dm.qd, B, dm.H, dm.Hk, dm.max_seq, pos_host + 1, seq_dev,
                                nsplit, 1, bf.attn, st, &qk));
    prof.mark(st, kGemv);
    int o_nsum = 0;  // batches: o's split partials summed by the row norm below
    R4Q_TRY(project(bf.rot, y.o_w, y.o_s, bf.o, B, D, dm.qd, y.o_bits, st, bf, kToRowNorm,
                    &o_nsum));
    // gate/up: r = fp16(o + h), RMSNorm + FWHT in the staging and, for
    // INT4/INT8, the SiLU-gate in the epilogue: fp16 FWHT'd output for the
    // whole 64-row units below the split (a multiple of the CU count, one
    // workgroup each), fp32 silu(g) * u above it (in bf.gu, unused at batch
    // 1); the down GEMV applies the FWHT-32 to that part in its staging.
    // (A unit map alone has 544 units for 256 CUs at I = 17408.)
    const bool silu_fused = fused && y.gu_bits != 16 && gemv_silu_ok(2 * I, D, y.gu_bits);
    int d_nsum = 0;  // batches: down's split partials summed by the next row norm
    if (silu_fused) {
      // (40-layer step, ctx 2048: 2.925 ms; every element as fp32 pairs:
      // 2.99 ms; every element in units: 3.02 ms)
      const int64_t split = gemv_silu_split(I);
      float* hp = reinterpret_cast<float*>(bf.gu);
      R4Q_TRY(gemv_norm_launch(bf.o, bf.h, y.post_norm, bf.r, eps, y.gu_w, y.gu_s, bf.y, 2 * I,
                               D, y.gu_bits, st, SiluEpi::kSplit, hp, split));
      prof.mark(st, kGemv);
      R4Q_TRY(gemv_fwht_launch(bf.y, hp, split, y.down_w, y.down_s, bf.d, D, I, y.down_bits, st));
    } else {
      bool gated = false;
      if (fused) {
        R4Q_TRY(gemv_norm_launch(bf.o, bf.h, y.post_norm, bf.r, eps, y.gu_w, y.gu_s, bf.gu,
                                 2 * I, D, y.gu_bits, st));
      } else {
        prof.mark(st, kNorm);
        R4Q_TRY(rownorm3(bf.o, o_nsum, bf.h, y.post_norm, bf.rot, bf.r, B, D, eps, st, bf));
        prof.mark(st, kGemv);
        const size_t gu_ws = silu_epilogue(B, I) ? 0 : bf.ws_bytes;
        if (gemm_skinny_silu_ok(B, I, D, y.gu_bits, gu_ws)) {
          // skinny GEMM with the SiLU gate + FWHT-32 in its epilogue
          // (unsplit, with its tail units cut into pieces over the CUs) or
          // in its split reduce
          if (gu_ws)
            R4Q_TRY(gemm_skinny_silu_launch(bf.rot, y.gu_w, y.gu_s, bf.y, B, I, D, y.gu_bits, st,
                                            bf.ws, gu_ws));
          else
            R4Q_TRY(gemm_skinny_silu_tail_launch(bf.rot, y.gu_w, y.gu_s, bf.y, B, I, D,
                                                 y.gu_bits, st, bf.tail));
          gated = true;
        } else {
          R4Q_TRY(linear(bf.rot, y.gu_w, y.gu_s, bf.gu, B, 2 * I, D, y.gu_bits, st, bf));
        }
      }
      if (!gated) {
        prof.mark(st, kNorm);
        R4Q_TRY(launch_silu(true, bf.gu, bf.gu + I, bf.y, B, I, 2 * I, I, st));
      }
      prof.mark(st, kGemv);
      R4Q_TRY(project(bf.y, y.down_w, y.down_s, bf.d, B, D, I, y.down_bits, st, bf, kToRowNorm,
                      &d_nsum));
    }
    if (!fused) {
      prof.mark(st, kNorm);
      const void* nxt = (li + 1 < dm.L) ? m->layers[li + 1].in_norm : m->final_norm;
      R4Q_TRY(rownorm3(bf.d, d_nsum, bf.r, nxt ? nxt : m->layers[0].in_norm, bf.rot, bf.h, B, D,
                       eps, st, bf));
    }
  }
  // h holds the final residual stream (fp16(d + r)) once this block is done
  if (fused && logits) {
    prof.mark(st, kGemv);
    R4Q_TRY(gemv_norm_launch(bf.d, bf.r, m->final_norm, bf.h, eps, m->lm_w, m->lm_s, bf.logits,
                             m->lm_N, m->lm_K, m->lm_bits, st));
  } else if (fused) {
    prof.mark(st, kNorm);
    R4Q_TRY(launch_rownorm(3, bf.d, bf.r, m->layers[0].in_norm, bf.rot, bf.h, B, D, eps, st));
  } else if (logits) {
    prof.mark(st, kGemv);
    R4Q_TRY(linear(bf.rot, m->lm_w, m->lm_s, bf.logits, B, m->lm_N, m->lm_K, m->lm_bits, st, bf));
  }
  prof.mark(st, kEnd);
  return R4Q_OK;
}

// ----------------------------------------------------- on-device sampling
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// (value, index) pair reduction across a wave with `better` (the larger
// value, then the lower index); every lane ends with the wave's best.
__device__ __forceinline__ void wave_best(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o);
    const int oi = __shfl_xor(i, o);
    if (better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}

// Stage 1: per (block, row) max and first index of the max.
__global__ __launch_bounds__(256) void argmax_partial_kernel(const uint16_t* __restrict__ logits,
                                                             int64_t V, float* __restrict__ part) {
  const int64_t b = blockIdx.y;
  const int64_t per = (V + gridDim.x - 1) / gridDim.x;
  const int64_t lo = blockIdx.x * per, hi = min(V, lo + per);
  float bv = -INFINITY;
  int bi = 0x7FFFFFFF;
  for (int64_t i = lo + threadIdx.x; i < hi; i += blockDim.x) {
    const float v = h2f(logits[b * V + i]);
    if (better(v, (int)i, bv, bi)) {
      bv = v;
      bi = (int)i;
    }
  }
  wave_best(bv, bi);
  __shared__ float sv[4];
  __shared__ int si[4];
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < 4; ++w)
      if (better(sv[w], si[w], bv, bi)) {
        bv = sv[w];
        bi = si[w];
      }
    part[(b * gridDim.x + blockIdx.x) * 2] = bv;
    part[(b * gridDim.x + blockIdx.x) * 2 + 1] = __int_as_float(bi);
  }
}

// Stage 2 (one block per row): final argmax over the nblk (<= 64) partials
// by one wave, token id out, embedding gather into the next step's hidden
// state; with `advance` (one row only) also the position / step counters
// that advance_kernel moves otherwise.
__global__ __launch_bounds__(256) void argmax_embed_kernel(
    const float* __restrict__ part, int nblk, const uint16_t* __restrict__ embed, int64_t vocab,
    int D, uint16_t* __restrict__ h, int64_t* __restrict__ ids, int64_t* __restrict__ tokens_out,
    int* __restrict__ state, int step_host, int B, int advance) {
  const int b = blockIdx.x;
  __shared__ int tok;
  if (threadIdx.x < 64) {
    const int k = threadIdx.x;
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;  // blocks past nblk and empty blocks lose every comparison
    if (k < nblk) {
      bv = part[(b * nblk + k) * 2];
      bi = __float_as_int(part[(b * nblk + k) * 2 + 1]);
    }
    wave_best(bv, bi);
    if (threadIdx.x == 0) {
      if (bi >= vocab) bi = 0;
      tok = bi;
      ids[b] = bi;
      const int step = state ? state[kStep] : step_host;
      if (tokens_out) tokens_out[(int64_t)step * B + b] = bi;
      if (advance) {
        state[kPos] += 1;
        state[kSeq] = state[kPos] + 1;
        state[kStep] += 1;
      }
    }
  }
  __syncthreads();
  const u4_t* src = reinterpret_cast<const u4_t*>(embed + (int64_t)tok * D);
  u4_t* dst = reinterpret_cast<u4_t*>(h + (int64_t)b * D);
  for (int i = threadIdx.x; i < D / 8; i += blockDim.x) dst[i] = src[i];
}

// Start of a replayed run: the device position / length / step counters,
// and the caller's hidden states copied into the step's input buffer
// (n16 16-byte pieces; one launch instead of a copy and a kernel).
__global__ void prime_kernel(int* __restrict__ state, int pos, const u4_t* __restrict__ src,
                             u4_t* __restrict__ dst, int64_t n16) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    state[kPos] = pos;
    state[kSeq] = pos + 1;
    state[kStep] = 0;
  }
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n16;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

__global__ void advance_kernel(int* state) {
  state[kPos] += 1;
  state[kSeq] = state[kPos] + 1;
  state[kStep] += 1;
}

// Next token of every row from bf.logits: greedy argmax, or temperature /
// top-p sampling when `scfg` has temperature > 0 (draw counter = the step's
// position: state[kPos] on the device, else pos_host); then its embedding
// into bf.h and, in a captured loop, the position advance.
int enqueue_sample(const r4q_model* m, const Dims& dm, int64_t B, const Bufs& bf,
                   int64_t* tokens_out, bool device_step, int step_host, hipStream_t st,
                   const SampleCfg* scfg = nullptr, void* sample_ws = nullptr,
                   int64_t pos_host = 0) {
  if (scfg && scfg->temperature > 0.f) {
    R4Q_TRY(launch_sample(bf.logits, B, m->lm_N, m->lm_N, *scfg,
                          device_step ? bf.state + kPos : nullptr, pos_host, sample_ws, bf.ids,
                          m->embed, dm.D, bf.h, tokens_out, device_step ? bf.state : nullptr,
                          step_host, st));
    if (device_step) {
      hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, st, bf.state);
      R4Q_TRY(launch_status("advance"));
    }
    return R4Q_OK;
  }
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(kArgmaxBlocks, (unsigned)B), dim3(256), 0, st,
                     bf.logits, m->lm_N, bf.amax);
  R4Q_TRY(launch_status("argmax"));
  // one row: the gather kernel also advances the counters (a single block
  // reads the step before it moves it); several rows: a kernel of its own
  const int fold = device_step && B == 1;
  hipLaunchKernelGGL(argmax_embed_kernel, dim3((unsigned)B), dim3(256), 0, st, bf.amax,
                     kArgmaxBlocks, static_cast<const uint16_t*>(m->embed), m->vocab, dm.D, bf.h,
                     bf.ids, tokens_out, device_step ? bf.state : nullptr, step_host, (int)B,
                     fold);
  R4Q_TRY(launch_status("argmax_embed"));
  if (device_step && !fold) {
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(1), 0, st, bf.state);
    R4Q_TRY(launch_status("advance"));
  }
  return R4Q_OK;
}

int check_positions(const r4q_model* m, int64_t first, int64_t count) {
  R4Q_REQUIRE(first >= 0 && count >= 1, "decode: bad position range");
  R4Q_REQUIRE(first + count <= m->max_seq,
              "decode: positions up to %lld exceed the KV cache (max_seq %d)",
              (long long)(first + count - 1), m->max_seq);
  R4Q_REQUIRE(first + count <= m->rope_len,
              "decode: positions up to %lld exceed the RoPE table (%d rows)",
              (long long)(first + count - 1), m->rope_len);
  return R4Q_OK;
}

// Whether the caller's stream is being captured (a hipStreamIsCapturing
// error, e.g. the null stream while another stream captures, counts as yes:
// no replay is started then).
bool capturing(hipStream_t s) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(s, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return true;
  }
  return cs != hipStreamCaptureStatusNone;
}

// Key of a captured graph: model struct, layer table, launch shape and every
// buffer address the graph bakes in (the context's buffers, the sampling
// workspace, the caller's token array), plus the context's buffer epoch,
// which moves whenever one of its buffers is reallocated.
std::vector<uint8_t> graph_key(const r4q_ctx* ctx, int kind, const r4q_model* m, int64_t B,
                               int nsplit, const void* tokens_out, const Bufs& bf,
                               const SampleCfg& scfg, const void* sample_ws) {
  const void* extra[] = {tokens_out, bf.h, bf.attn, bf.state, bf.ws, sample_ws};
  const uint64_t epoch = ctx->buf_epoch;
  // launch-shape overrides change what a step launches
  const Tuning& tu = tuning();
  const int knobs[] = {tu.gemv_lpr.load(),      tu.gemv_wgs.load(),    tu.gemv_ub.load(),
                       tu.attn_splits.load(),   tu.skinny_splits.load(), tu.gemm_splits.load(),
                       tu.split_reduce.load(),  tu.gemm_kernel.load(), tu.gemv_skew.load()};
  std::vector<uint8_t> k(sizeof(r4q_model) + sizeof(r4q_layer) * m->n_layers + 16 +
                         sizeof(extra) + sizeof(epoch) + sizeof(SampleCfg) + sizeof(knobs));
  uint8_t* p = k.data();
  memcpy(p, m, sizeof(r4q_model));
  p += sizeof(r4q_model);
  memcpy(p, m->layers, sizeof(r4q_layer) * m->n_layers);
  p += sizeof(r4q_layer) * m->n_layers;
  memcpy(p, &B, 8);
  memcpy(p + 8, &nsplit, 4);
  memcpy(p + 12, &kind, 4);
  p += 16;
  memcpy(p, extra, sizeof(extra));
  p += sizeof(extra);
  memcpy(p, &epoch, sizeof(epoch));
  p += sizeof(epoch);
  memcpy(p, &scfg, sizeof(SampleCfg));
  p += sizeof(SampleCfg);
  memcpy(p, knobs, sizeof(knobs));
  return k;
}

enum GraphKind { kGraphLoop = 1, kGraphStep = 2 };

// Keeps at most kInFlight steps (graph replays or eager steps) queued ahead
// of the GPU: the host waits for step t - kInFlight before it enqueues step
// t.  With every replay queued at once, the same graph ran 4-7% slower while
// the queue stayed deep (40-layer step, ctx 2048, batch 1: 2.93 ms per step
// over 64 replays, 2.83 over 128, where the queue fills and the host blocks
// part of the time; 2.73 ms at 1, 2 or 4 in flight, 2 the fastest).
constexpr int kInFlight = 2;
struct Throttle {
  hipEvent_t ev[kInFlight] = {};
  bool on = false;
  // off for runs of at most kInFlight steps and on a stream being captured
  // (no host wait can order captured work)
  int init(int64_t steps, hipStream_t s) {
    if (steps <= kInFlight) return R4Q_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess) {  // e.g. the null stream during a capture
      (void)hipGetLastError();
      return R4Q_OK;
    }
    if (cs != hipStreamCaptureStatusNone) return R4Q_OK;
    for (hipEvent_t& e : ev) R4Q_HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    on = true;
    return R4Q_OK;
  }
  // before step t is enqueued
  int wait(int64_t t) {
    if (on && t >= kInFlight) R4Q_HIP_TRY(hipEventSynchronize(ev[t % kInFlight]));
    return R4Q_OK;
  }
  // after step t is enqueued on s
  int mark(int64_t t, hipStream_t s) {
    if (on) R4Q_HIP_TRY(hipEventRecord(ev[t % kInFlight], s));
    return R4Q_OK;
  }
  ~Throttle() {
    for (hipEvent_t e : ev)
      if (e) (void)hipEventDestroy(e);
  }
};

// Runs a captured graph `reps` times on the context's graph stream, ordered
// after the work already on `st` (and everything enqueued on `st` later waits
// for it), at most kInFlight replays queued ahead of the GPU.  The device
// position state is first set to `pos`.  On a cache miss `record(stream)`
// enqueues the work once under stream capture and the instantiated graph is
// kept under `key`.
template <class Record>
int replay(r4q_ctx* ctx, hipStream_t st, std::vector<uint8_t> key, int* state, int pos,
           const void* hidden_in, void* h, size_t hidden_bytes, int64_t reps,
           const Record& record) {
  if (!ctx->graphs) ctx->graphs = new GraphCache();
  GraphCache& gc = *ctx->graphs;
  if (!gc.stream) R4Q_HIP_TRY(hipStreamCreateWithFlags(&gc.stream, hipStreamNonBlocking));
  if (!gc.ev_in) R4Q_HIP_TRY(hipEventCreateWithFlags(&gc.ev_in, hipEventDisableTiming));
  if (!gc.ev_out) R4Q_HIP_TRY(hipEventCreateWithFlags(&gc.ev_out, hipEventDisableTiming));
  R4Q_HIP_TRY(hipEventRecord(gc.ev_in, st));
  R4Q_HIP_TRY(hipStreamWaitEvent(gc.stream, gc.ev_in, 0));
  const int64_t n16 = (int64_t)(hidden_bytes / 16);
  const unsigned pblocks = (unsigned)std::min<int64_t>(64, std::max<int64_t>(1, (n16 + 255) / 256));
  hipLaunchKernelGGL(prime_kernel, dim3(pblocks), dim3(256), 0, gc.stream, state, pos,
                     static_cast<const u4_t*>(hidden_in), static_cast<u4_t*>(h), n16);
  int rc = launch_status("prime");
  hipGraphExec_t exec = rc == R4Q_OK ? gc.find(key) : nullptr;
  if (rc == R4Q_OK && !exec) {
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamBeginCapture(gc.stream, hipStreamCaptureModeRelaxed);
    if (e != hipSuccess) {
      rc = fail(R4Q_EHIP, "hipStreamBeginCapture: %s", hipGetErrorString(e));
    } else {
      const int rc1 = record(gc.stream);
      e = hipStreamEndCapture(gc.stream, &graph);
      if (rc1 != R4Q_OK) rc = rc1;
      else if (e != hipSuccess) rc = fail(R4Q_EHIP, "hipStreamEndCapture: %s", hipGetErrorString(e));
      else {
        e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
          exec = nullptr;
          rc = fail(R4Q_EHIP, "hipGraphInstantiate: %s", hipGetErrorString(e));
        } else {
          gc.insert(std::move(key), exec);
        }
      }
      if (graph) (void)hipGraphDestroy(graph);
    }
  }
  Throttle th;
  if (rc == R4Q_OK) rc = th.init(reps, gc.stream);
  for (int64_t t = 0; rc == R4Q_OK && t < reps; ++t) {
    rc = th.wait(t);
    if (rc != R4Q_OK) break;
    const hipError_t e = hipGraphLaunch(exec, gc.stream);
    if (e != hipSuccess) rc = fail(R4Q_EHIP, "hipGraphLaunch: %s", hipGetErrorString(e));
    else rc = th.mark(t, gc.stream);
  }
  (void)hipEventRecord(gc.ev_out, gc.stream);
  (void)hipStreamWaitEvent(st, gc.ev_out, 0);
  return rc;
}

}  // namespace
}  // namespace r4q

using namespace r4q;

extern "C" int r4q_decode_plan(const r4q_model* m, int64_t B, int32_t* out, int64_t n) {
  using namespace r4q;
  R4Q_REQUIRE(out && n >= 2, "decode_plan: need room for 2 values");
  Dims dm;
  R4Q_TRY(validate(m, B, dm));
  const size_t gws = step_gemm_ws(m, dm, B);
  int fused = 0, folded = 0;
  for (int li = 0; li < dm.L; ++li) {
    const int bits = m->layers[li].gu_bits;
    fused += B == 1 ? (bits != 16 && gemv_silu_ok(2 * (int64_t)dm.I, dm.D, bits))
                    : gemm_skinny_silu_ok(B, dm.I, dm.D, bits, silu_epilogue(B, dm.I) ? 0 : gws);
    const r4q_layer& y = m->layers[li];
    folded += consumer_split(B, dm.qkvN, dm.D, y.qkv_bits, gws, kToAttention) > 0;
    folded += consumer_split(B, dm.D, dm.qd, y.o_bits, gws, kToRowNorm) > 0;
    folded += consumer_split(B, dm.D, dm.I, y.down_bits, gws, kToRowNorm) > 0;
  }
  out[0] = attn_num_splits(m->max_seq, B, dm.Hk);
  out[1] = fused;
  if (n >= 3) out[2] = folded;
  return R4Q_OK;
}

namespace r4q {
namespace {
int decode_step(r4q_ctx* ctx, const r4q_model* m, const void* hidden_in, int64_t B, int64_t pos,
                void* hidden_out, void* logits, bool use_graph, void* stream) {
  R4Q_REQUIRE(ctx && hidden_in, "decode_step: null context or input");
  Dims dm;
  R4Q_TRY(validate(m, B, dm));
  R4Q_TRY(check_positions(m, pos, 1));
  R4Q_REQUIRE(!logits || m->final_norm, "decode_step: logits requested but the model has no LM head");
  const int nsplit = attn_num_splits(m->max_seq, B, dm.Hk);
  Bufs bf;
  hipStream_t st = as_stream(stream);
  R4Q_TRY(reserve(ctx, m, dm, B, nsplit, st, bf));
  const size_t hbytes = (size_t)B * dm.D * 2;
  const bool want_logits = logits != nullptr;
  // a stream being captured by the caller records the eager launches
  if (use_graph && capturing(st)) use_graph = false;
  // the prime kernel of a replay copies the hidden states in 16-byte pieces
  const bool h16 = (reinterpret_cast<uintptr_t>(hidden_in) & 15) == 0;
  if (use_graph && !h16)
    R4Q_HIP_TRY(hipMemcpyAsync(bf.h, hidden_in, hbytes, hipMemcpyDeviceToDevice, st));
  if (use_graph) {
    // the same step with the position read from device memory; one graph
    // serves every position (the attention split count depends only on the
    // cache capacity)
    auto record = [&](hipStream_t gs) {
      return enqueue_step(m, dm, B, pos, bf.state + kPos, bf.state + kSeq, nsplit, bf,
                          want_logits, gs);
    };
    R4Q_TRY(replay(ctx, st,
                   graph_key(ctx, want_logits ? kGraphStep : -kGraphStep, m, B, nsplit, nullptr,
                             bf, SampleCfg{0.f, 1.f, 0}, nullptr),
                   bf.state, (int)pos, hidden_in, bf.h, h16 ? hbytes : 0, 1, record));
  } else {
    R4Q_HIP_TRY(hipMemcpyAsync(bf.h, hidden_in, hbytes, hipMemcpyDeviceToDevice, st));
    R4Q_TRY(enqueue_step(m, dm, B, pos, nullptr, nullptr, nsplit, bf, want_logits, st));
  }
  if (logits)
    R4Q_HIP_TRY(hipMemcpyAsync(logits, bf.logits, (size_t)B * m->lm_N * 2,
                               hipMemcpyDeviceToDevice, st));
  if (hidden_out)
    R4Q_HIP_TRY(hipMemcpyAsync(hidden_out, bf.h, (size_t)B * dm.D * 2, hipMemcpyDeviceToDevice, st));
  return R4Q_OK;
}
}  // namespace
}  // namespace r4q

extern "C" int r4q_decode_step(r4q_ctx* ctx, const r4q_model* m, const void* hidden_in, int64_t B,
                               int64_t pos, void* hidden_out, void* logits, void* stream) {
  return r4q::decode_step(ctx, m, hidden_in, B, pos, hidden_out, logits, false, stream);
}

extern "C" int r4q_decode_step_graph(r4q_ctx* ctx, const r4q_model* m, const void* hidden_in,
                                     int64_t B, int64_t pos, void* hidden_out, void* logits,
                                     void* stream) {
  return r4q::decode_step(ctx, m, hidden_in, B, pos, hidden_out, logits, true, stream);
}

namespace r4q {
namespace {
// The decode loop behind r4q_decode_bench (greedy) and r4q_decode_generate
// (temperature / top-p): num_tokens steps from start_pos, next token and its
// embedding on the device between steps, optionally captured in a hipGraph.
int decode_loop(r4q_ctx* ctx, const r4q_model* m, const void* hidden_in, int64_t B,
                int64_t num_tokens, int64_t start_pos, int use_graph, void* tokens_out,
                const SampleCfg& scfg, void* stream) {
  R4Q_REQUIRE(ctx && hidden_in, "decode_bench: null context or input");
  Dims dm;
  R4Q_TRY(validate(m, B, dm));
  R4Q_REQUIRE(m->final_norm && m->embed && m->vocab >= m->lm_N,
              "decode_bench: greedy decoding needs an LM head and an embedding table");
  R4Q_REQUIRE(num_tokens >= 1, "decode_bench: num_tokens must be >= 1");
  R4Q_TRY(check_positions(m, start_pos, num_tokens));
  const int nsplit = attn_num_splits(m->max_seq, B, dm.Hk);
  Bufs bf;
  hipStream_t st = as_stream(stream);
  R4Q_TRY(reserve(ctx, m, dm, B, nsplit, st, bf));
  int64_t* toks = static_cast<int64_t*>(tokens_out);
  void* sws = nullptr;
  if (scfg.temperature > 0.f) R4Q_TRY(sample_reserve(ctx, B, st, &sws));
  const size_t hbytes = (size_t)B * dm.D * 2;
  if (!use_graph) {
    R4Q_HIP_TRY(hipMemcpyAsync(bf.h, hidden_in, hbytes, hipMemcpyDeviceToDevice, st));
    Throttle th;
    R4Q_TRY(th.init(num_tokens, st));
    for (int64_t t = 0; t < num_tokens; ++t) {
      const int64_t pos = start_pos + t;
      R4Q_TRY(th.wait(t));
      R4Q_TRY(enqueue_step(m, dm, B, pos, nullptr, nullptr, nsplit, bf, true, st));
      R4Q_TRY(enqueue_sample(m, dm, B, bf, toks, false, (int)t, st, &scfg, sws, pos));
      R4Q_TRY(th.mark(t, st));
    }
    return R4Q_OK;
  }
  // ---- graph path: one captured step + next-token choice + position
  // advance, replayed num_tokens times
  auto record = [&](hipStream_t gs) {
    R4Q_TRY(enqueue_step(m, dm, B, start_pos, bf.state + kPos, bf.state + kSeq, nsplit, bf, true,
                         gs));
    return enqueue_sample(m, dm, B, bf, toks, true, 0, gs, &scfg, sws);
  };
  const bool h16 = (reinterpret_cast<uintptr_t>(hidden_in) & 15) == 0;
  if (!h16) R4Q_HIP_TRY(hipMemcpyAsync(bf.h, hidden_in, hbytes, hipMemcpyDeviceToDevice, st));
  return replay(ctx, st, graph_key(ctx, kGraphLoop, m, B, nsplit, tokens_out, bf, scfg, sws),
                bf.state, (int)start_pos, hidden_in, bf.h, h16 ? hbytes : 0, num_tokens, record);
}
}  // namespace
}  // namespace r4q

extern "C" int r4q_decode_bench(r4q_ctx* ctx, const r4q_model* m, const void* hidden_in, int64_t B,
                                int64_t num_tokens, int64_t start_pos, int use_graph,
                                void* tokens_out, void* stream) {
  return r4q::decode_loop(ctx, m, hidden_in, B, num_tokens, start_pos, use_graph, tokens_out,
                          r4q::SampleCfg{0.f, 1.f, 0}, stream);
}

extern "C" int r4q_decode_generate(r4q_ctx* ctx, const r4q_model* m, const void* hidden_in,
                                   int64_t B, int64_t num_tokens, int64_t start_pos,
                                   int use_graph, float temperature, float top_p, uint64_t seed,
                                   void* tokens_out, void* stream) {
  R4Q_REQUIRE(temperature >= 0.f && top_p > 0.f,
              "decode_generate: need temperature >= 0 and top_p > 0");
  return r4q::decode_loop(ctx, m, hidden_in, B, num_tokens, start_pos, use_graph, tokens_out,
                          r4q::SampleCfg{temperature, top_p, seed}, stream);
}

extern "C" int r4q_decode_profile(r4q_ctx* ctx, const r4q_model* m, const void* hidden_in,
                                  int64_t pos, float* out_ms, void* stream) {
  R4Q_REQUIRE(ctx && hidden_in && out_ms, "decode_profile: null argument");
  Dims dm;
  R4Q_TRY(validate(m, 1, dm));
  R4Q_TRY(check_positions(m, pos, 1));
  const int nsplit = attn_num_splits(m->max_seq, 1, dm.Hk);
  Bufs bf;
  hipStream_t st = as_stream(stream);
  R4Q_TRY(reserve(ctx, m, dm, 1, nsplit, st, bf));
  R4Q_HIP_TRY(hipMemcpyAsync(bf.h, hidden_in, (size_t)dm.D * 2, hipMemcpyDeviceToDevice, st));
  std::vector<hipEvent_t> ev;
  std::vector<int> cat;
  Prof prof;
  prof.ev = &ev;
  prof.cat = &cat;
  int rc = enqueue_step(m, dm, 1, pos, nullptr, nullptr, nsplit, bf, m->final_norm != nullptr, st,
                        prof);
  if (rc == R4Q_OK) {
    (void)hipEventSynchronize(ev.back());
    float by_cat[4] = {0.f, 0.f, 0.f, 0.f}, total = 0.f, ms = 0.f;
    for (size_t i = 0; i + 1 < ev.size(); ++i) {
      (void)hipEventElapsedTime(&ms, ev[i], ev[i + 1]);
      if (cat[i] >= 0) by_cat[cat[i]] += ms;
    }
    (void)hipEventElapsedTime(&total, ev.front(), ev.back());
    out_ms[0] = total;
    out_ms[1] = by_cat[kGemv];
    out_ms[2] = by_cat[kAttn];
    out_ms[3] = by_cat[kNorm];
    out_ms[4] = total - by_cat[kGemv] - by_cat[kAttn] - by_cat[kNorm];
  }
  for (hipEvent_t e : ev) (void)hipEventDestroy(e);
  return rc;
}

extern "C" int r4q_prefill_logits(r4q_ctx* ctx, const r4q_model* m, const void* ids, int64_t M,
                                  void* logits, int write_kv, void* stream) {
  using namespace r4q;
  R4Q_REQUIRE(ctx && ids, "prefill_logits: null argument");
  Dims dm;
  R4Q_TRY(validate(m, 1, dm));
  R4Q_REQUIRE(m->embed && m->vocab >= 1, "prefill_logits: model has no embedding table");
  R4Q_REQUIRE(M >= 1 && M <= m->rope_len, "prefill_logits: M=%lld outside [1, rope_len=%d]",
              (long long)M, m->rope_len);
  R4Q_REQUIRE(!write_kv || M <= m->max_seq,
              "prefill_logits: M=%lld exceeds the KV cache capacity %d", (long long)M, m->max_seq);
  R4Q_REQUIRE(!logits || m->final_norm, "prefill_logits: logits requested without an LM head");
  hipStream_t st = as_stream(stream);
  const int64_t D = dm.D, I = dm.I;
  // token ids are checked on the host: an id outside the table would make
  // the gather read past the embedding
  std::vector<int64_t> hid((size_t)M);
  R4Q_HIP_TRY(hipMemcpyAsync(hid.data(), ids, (size_t)M * 8, hipMemcpyDeviceToHost, st));
  R4Q_HIP_TRY(hipStreamSynchronize(st));
  for (int64_t i = 0; i < M; ++i)
    R4Q_REQUIRE(hid[(size_t)i] >= 0 && hid[(size_t)i] < m->vocab,
                "prefill_logits: token id %lld at row %lld outside [0, %lld)",
                (long long)hid[(size_t)i], (long long)i, (long long)m->vocab);
  // workspace: x, r, rot, qkv, o, gu, y, d
  const size_t rotw = dm.qd > dm.D ? dm.qd : dm.D;
  const size_t sizes[] = {(size_t)(M * D), (size_t)(M * D), M * rotw, (size_t)(M * dm.qkvN),
                          (size_t)(M * D), (size_t)(M * 2 * I), (size_t)(M * I), (size_t)(M * D)};
  size_t total = 0;
  for (size_t sz : sizes) total += align256(sz * 2);
  // split-K partials of the projection GEMMs (the largest any of them uses)
  size_t gws = 0;
  for (int li = 0; li < dm.L; ++li) {
    const r4q_layer& ly = m->layers[li];
    gws = std::max({gws, gemm_ws_need(M, dm.qkvN, D, ly.qkv_bits),
                    gemm_ws_need(M, D, dm.qd, ly.o_bits), gemm_ws_need(M, 2 * I, D, ly.gu_bits),
                    gemm_ws_need(M, D, I, ly.down_bits)});
  }
  if (logits) gws = std::max(gws, gemm_ws_need(M, m->lm_N, m->lm_K, m->lm_bits));
  R4Q_TRY(ctx->prefill.reserve(total + gws));
  uint16_t* buf[8];
  uint8_t* p = static_cast<uint8_t*>(ctx->prefill.ptr);
  for (int i = 0; i < 8; ++i) {
    buf[i] = reinterpret_cast<uint16_t*>(p);
    p += align256(sizes[i] * 2);
  }
  void* ws = gws ? p : nullptr;
  uint16_t *x = buf[0], *r = buf[1], *rot = buf[2], *qkv = buf[3], *o = buf[4], *gu = buf[5],
           *y = buf[6], *d = buf[7];
  const float eps = dm.eps;
  // (hip:2127-2320) embedding -> per layer: norm+FWHT, QKV, head norm +
  // RoPE (+ FP8 KV at positions 0..M-1), causal attention + FWHT, O,
  // residual + norm + FWHT, gate/up, SiLU-gate + FWHT, down, residual +
  // norm + FWHT of the next layer (the last one uses the final norm); LM head
  R4Q_TRY(launch_embed_gather(static_cast<const int64_t*>(ids), m->embed, x, M, D, st));
  R4Q_TRY(launch_rownorm(2, x, nullptr, m->layers[0].in_norm, rot, nullptr, M, D, eps, st));
  for (int li = 0; li < dm.L; ++li) {
    const r4q_layer& ly = m->layers[li];
    R4Q_TRY(gemm_launch(rot, ly.qkv_w, ly.qkv_s, qkv, M, dm.qkvN, D, ly.qkv_bits, st, ws, gws));
    R4Q_TRY(launch_head_norm_rope_kv(qkv, dm.qkvN, ly.q_norm, ly.k_norm, qkv, dm.qkvN,
                                     write_kv ? ly.k_cache : nullptr,
                                     write_kv ? ly.v_cache : nullptr, ly.k_scale, ly.v_scale,
                                     m->rope_cos, m->rope_sin, M, dm.H, dm.Hk, eps, dm.max_seq, 0,
                                     nullptr, st, /*prefill_rows=*/true));
    R4Q_TRY(launch_prefill_attention(qkv, dm.qkvN, rot, dm.qd, M, dm.H, dm.Hk, st));
    R4Q_TRY(gemm_launch(rot, ly.o_w, ly.o_s, o, M, D, dm.qd, ly.o_bits, st, ws, gws));
    R4Q_TRY(launch_rownorm(3, o, x, ly.post_norm, rot, r, M, D, eps, st));
    R4Q_TRY(gemm_launch(rot, ly.gu_w, ly.gu_s, gu, M, 2 * I, D, ly.gu_bits, st, ws, gws));
    R4Q_TRY(launch_silu(true, gu, gu + I, y, M, I, 2 * I, I, st));
    R4Q_TRY(gemm_launch(y, ly.down_w, ly.down_s, d, M, D, I, ly.down_bits, st, ws, gws));
    const void* nxt = (li + 1 < dm.L) ? m->layers[li + 1].in_norm
                                      : (m->final_norm ? m->final_norm : m->layers[0].in_norm);
    R4Q_TRY(launch_rownorm(3, d, r, nxt, rot, x, M, D, eps, st));
  }
  if (logits)
    R4Q_TRY(gemm_launch(rot, m->lm_w, m->lm_s, logits, M, m->lm_N, m->lm_K, m->lm_bits, st, ws,
                        gws));
  return R4Q_OK;
}
