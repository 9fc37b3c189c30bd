"""Drop-in replacement for the reference's `int4_hip` extension module.

Same 15 names, positional signatures and return values as the pybind table
of the reference (hip_int4/int4_decode_step.hip:3620-3636); every call runs
the gfx950 kernels of librdna4q.so through its C ABI on torch's current
stream.  Put this directory on sys.path and `import int4_hip`, exactly as
int4_engine_v5.py:20-21,56-57 does with hip_int4/.

Differences the reference's API cannot express are inferred, not added as
arguments:
  * weight precision per matrix comes from the packed width:
    w.shape[1] * 2 == K -> INT4, w.shape[1] == K -> INT8 (uint8, asymmetric,
    same interleaved (scale, zero) fp16 table), float16 w -> FP16 (LM head);
  * batch = hidden.shape[0] (KV caches [B, Hk, max_seq, D]);
  * per-head FP8 KV scales are 1.0 (the reference's implicit scale); the
    extended `kv_scales=(k_scales, v_scales)` keyword takes per-layer [Hk]
    float32 tensors.
Errors (bad shapes, dtypes, sizes) raise RuntimeError/ValueError before any
device work, unlike the reference which does not check.
"""
from __future__ import annotations

import ctypes as C
import weakref
from typing import List

import torch

import r4q_lib as _R

__all__ = [
    "decode_step", "decode_step_logits", "decode_loop", "decode_bench", "decode_bench_graph",
    "decode_profile", "prefill_logits", "dbg_rmsnorm", "dbg_head_rmsnorm", "dbg_rope",
    "dbg_fused_res_norm", "dbg_gemv", "dbg_gemm", "dequant_int4", "fp16_to_fp8",
]


def _need(cond, msg):
    if not cond:
        raise ValueError(msg)


def _cuda_half(t, name):
    _need(t.is_cuda, f"{name} must be a HIP device tensor")
    _need(t.dtype == torch.float16, f"{name} must be float16 (got {t.dtype})")
    _need(t.is_contiguous(), f"{name} must be contiguous")


def weight_bits(w: torch.Tensor, K: int) -> int:
    """INT4 / INT8 / FP16 from the packed width (the reference API has no
    precision argument)."""
    if w.dtype == torch.float16:
        _need(w.shape[-1] == K, f"fp16 weight width {w.shape[-1]} != K={K}")
        return 16
    _need(w.dtype == torch.uint8, f"weight dtype must be uint8 or float16 (got {w.dtype})")
    if w.shape[-1] * 2 == K:
        return 4
    if w.shape[-1] == K:
        return 8
    raise ValueError(f"packed width {w.shape[-1]} matches neither INT4 nor INT8 for K={K}")


def _stream():
    return _R.stream_handle()


# ----------------------------------------------------------------- utilities
def dequant_int4(packed: torch.Tensor, scales: torch.Tensor, N: int, K: int) -> torch.Tensor:
    """[N, K/2] uint8 + [N, K/16] fp16 interleaved (scale, zero) -> [N, K] fp16
    (hip:3590-3603)."""
    _need(packed.dtype == torch.uint8 and packed.is_contiguous(), "packed must be contiguous uint8")
    _need(packed.numel() == N * K // 2, "packed size != N*K/2")
    _need(scales.numel() == N * K // 16, "scales size != N*K/16")
    out = torch.empty((N, K), dtype=torch.float16, device=packed.device)
    _R.call("r4q_dequant_int4", packed.data_ptr(), scales.data_ptr(), out.data_ptr(), N, K,
            _stream())
    return out


def dequant_int8(q: torch.Tensor, scales: torch.Tensor, N: int, K: int) -> torch.Tensor:
    """INT8 counterpart of dequant_int4 (asymmetric uint8, same sz layout)."""
    _need(q.dtype == torch.uint8 and q.is_contiguous(), "q must be contiguous uint8")
    _need(q.numel() == N * K and scales.numel() == N * K // 16, "size mismatch")
    out = torch.empty((N, K), dtype=torch.float16, device=q.device)
    _R.call("r4q_dequant_int8", q.data_ptr(), scales.data_ptr(), out.data_ptr(), N, K,
            _stream())
    return out


def fp16_to_fp8(src: torch.Tensor) -> torch.Tensor:
    """fp16 -> E4M3 codes (uint8, same shape) by the reference recipe
    (hip:3606-3618)."""
    _cuda_half(src, "src")
    out = torch.empty(src.shape, dtype=torch.uint8, device=src.device)
    _R.call("r4q_fp16_to_fp8", src.data_ptr(), out.data_ptr(), src.numel(), _stream())
    return out


def fp8_to_fp16(src: torch.Tensor) -> torch.Tensor:
    """E4M3 codes -> fp16 values (exact)."""
    _need(src.dtype == torch.uint8 and src.is_contiguous(), "src must be contiguous uint8")
    out = torch.empty(src.shape, dtype=torch.float16, device=src.device)
    _R.call("r4q_fp8_to_fp16", src.data_ptr(), out.data_ptr(), src.numel(), _stream())
    return out


# --------------------------------------------------------------------- debug
def dbg_gemv(X: torch.Tensor, W: torch.Tensor, S: torch.Tensor, N: int, K: int) -> torch.Tensor:
    """Y[N] = W X (hip:3541-3550)."""
    _cuda_half(X, "X")
    _need(X.numel() == K, f"X has {X.numel()} elements, K={K}")
    bits = weight_bits(W, K)
    _need(W.shape[0] == N and W.is_contiguous(), "W must be contiguous with N rows")
    Y = torch.empty((N,), dtype=torch.float16, device=X.device)
    _R.call("r4q_gemv", X.data_ptr(), W.data_ptr(), None if bits == 16 else S.data_ptr(),
            Y.data_ptr(), N, K, bits, _stream())
    return Y


def dbg_gemm(X: torch.Tensor, W: torch.Tensor, S: torch.Tensor, M: int, N: int,
             K: int) -> torch.Tensor:
    """Y[M, N] = X W^T (hip:3552-3561)."""
    _cuda_half(X, "X")
    _need(X.numel() == M * K, "X size != M*K")
    bits = weight_bits(W, K)
    Y = torch.empty((M, N), dtype=torch.float16, device=X.device)
    nws = C.c_size_t(0)
    _R.call("r4q_gemm_workspace_bytes", M, N, K, bits, C.byref(nws))
    ws = torch.empty(nws.value, dtype=torch.uint8, device=X.device) if nws.value else None
    _R.call("r4q_gemm_ws", X.data_ptr(), W.data_ptr(), None if bits == 16 else S.data_ptr(),
            Y.data_ptr(), M, N, K, bits, None if ws is None else ws.data_ptr(), nws.value,
            _stream())
    return Y


def dbg_rmsnorm(X: torch.Tensor, W: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over all of X (hip:3473-3484)."""
    _cuda_half(X, "X")
    Y = torch.empty_like(X)
    D = X.numel()
    _R.call("r4q_rmsnorm", X.data_ptr(), W.data_ptr(), Y.data_ptr(), 1, D, float(eps), _stream())
    return Y


def dbg_fused_res_norm(X: torch.Tensor, Res: torch.Tensor, W: torch.Tensor,
                       eps: float) -> List[torch.Tensor]:
    """[Y, ResOut] with ResOut = X + Res, Y = RMSNorm(ResOut) (hip:3524-3539)."""
    _cuda_half(X, "X")
    _cuda_half(Res, "Res")
    Y = torch.empty_like(X)
    R = torch.empty_like(X)
    _R.call("r4q_res_rmsnorm", X.data_ptr(), Res.data_ptr(), W.data_ptr(), Y.data_ptr(),
            R.data_ptr(), 1, X.numel(), float(eps), _stream())
    return [Y, R]


def dbg_head_rmsnorm(Q, K, QW, KW, H: int, Hk: int, D: int, eps: float) -> List[torch.Tensor]:
    """Per-head RMSNorm of flat Q [H*D] and K [Hk*D] (hip:3486-3504)."""
    _cuda_half(Q, "Q")
    _cuda_half(K, "K")
    Qo = torch.empty_like(Q)
    Ko = torch.empty_like(K)
    _R.call("r4q_head_rmsnorm", Q.data_ptr(), K.data_ptr(), QW.data_ptr(), KW.data_ptr(),
            Qo.data_ptr(), Ko.data_ptr(), H, Hk, D, float(eps), _stream())
    return [Qo, Ko]


def dbg_rope(Q, K, COS, SIN, H: int, Hk: int, D: int) -> List[torch.Tensor]:
    """Half-split RoPE with the cos/sin row passed in (hip:3506-3522)."""
    _cuda_half(Q, "Q")
    _cuda_half(K, "K")
    Qo = torch.empty_like(Q)
    Ko = torch.empty_like(K)
    _R.call("r4q_rope", Q.data_ptr(), K.data_ptr(), COS.data_ptr(), SIN.data_ptr(),
            Qo.data_ptr(), Ko.data_ptr(), H, Hk, D, 0, _stream())
    return [Qo, Ko]


# ------------------------------------------------------------ decode family
class _Model:
    """A C `r4q_model` built from the reference's per-layer tensor lists.

    It holds no strong reference to the caller's tensors (the cache would
    otherwise keep every model ever passed alive, ~11 GB at Qwen3-14B per
    reload): each tensor it points at carries a weak reference whose callback
    drops the cache entry when the tensor is freed, before its memory or its
    id() can be reused."""

    def __init__(self, struct, layers):
        self.struct = struct
        self.layers = layers
        self.refs = []


_models = {}
_ctx = None


def _context():
    global _ctx
    if _ctx is None:
        h = C.c_void_p()
        _R.call("r4q_ctx_create", C.byref(h))
        _ctx = h
    return _ctx


_ptr = torch.Tensor.data_ptr


def _key_of(objs, shaped=()):
    """Cache key of an argument block: tensors by identity and data pointer
    (a storage swapped in place -- set_, .data =, a reallocating resize_ --
    keeps the id but moves the pointer), the tensor lists at positions
    `shaped` also by shape (the KV caches: capacity and batch come from
    them), everything else by value.  A hit is valid because every tensor of
    a cached model is alive (see _Model).  Dtypes and other shapes are
    checked when the model is built; ~70 us for a 40-layer block."""
    key = []
    for i, o in enumerate(objs):
        if isinstance(o, (list, tuple)):
            # tensor lists by identity + pointer, int lists by value
            if o and (o[0] is None or isinstance(o[0], torch.Tensor)):
                key.append(tuple(map(id, o)))
                try:
                    key.append(tuple(map(_ptr, o)))
                except TypeError:  # None entries (no scale table for FP16 weights)
                    key.append(tuple(0 if t is None else t.data_ptr() for t in o))
                if i in shaped:
                    key.append(tuple(t.shape for t in o))
            else:
                key.append(tuple(o))
        elif isinstance(o, torch.Tensor):
            key.append((id(o), o.data_ptr(), tuple(o.shape)))
        else:
            key.append(o)
    return tuple(key)


def _forget(key):
    def cb(_ref):
        _models.pop(key, None)
    return cb


def _watch(m, key, objs):
    cb = _forget(key)
    for o in objs:
        if isinstance(o, torch.Tensor):
            m.refs.append(weakref.ref(o, cb))
        elif isinstance(o, (list, tuple)):
            m.refs.extend(weakref.ref(t, cb) for t in o if isinstance(t, torch.Tensor))


def build_model(qkv_w, qkv_s, qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N, down_w, down_s, down_N,
                in_norm_w, post_norm_w, q_norm_w, k_norm_w, rope_cos, rope_sin,
                num_heads, num_kv_heads, head_dim, hidden_size, intermediate_size, rms_eps,
                k_caches, v_caches, final_norm_w=None, lm_w=None, lm_s=None, lm_N=0, lm_K=0,
                embed_weight=None, kv_scales=None) -> _Model:
    """Validates the reference argument block and returns a cached model
    descriptor (keyed by tensor identity; see _key_of / _Model)."""
    args = [qkv_w, qkv_s, qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N, down_w, down_s, down_N,
            in_norm_w, post_norm_w, q_norm_w, k_norm_w, rope_cos, rope_sin, num_heads,
            num_kv_heads, head_dim, hidden_size, intermediate_size, float(rms_eps), k_caches,
            v_caches, final_norm_w, lm_w, lm_s, lm_N, lm_K, embed_weight,
            None if kv_scales is None else kv_scales[0],
            None if kv_scales is None else kv_scales[1]]
    key = _key_of(args, shaped=(24, 25))  # k_caches, v_caches
    m = _models.get(key)
    if m is not None:
        return m
    L = len(qkv_w)
    D, I, H, Hk, hd = hidden_size, intermediate_size, num_heads, num_kv_heads, head_dim
    lists = dict(qkv_s=qkv_s, o_w=o_w, o_s=o_s, gu_w=gu_w, gu_s=gu_s, down_w=down_w,
                 down_s=down_s, in_norm_w=in_norm_w, post_norm_w=post_norm_w,
                 q_norm_w=q_norm_w, k_norm_w=k_norm_w, k_caches=k_caches, v_caches=v_caches)
    for n, v in lists.items():
        _need(len(v) == L, f"{n} has {len(v)} entries, expected {L}")
    _need(L >= 1, "need at least one layer")
    _need(H % Hk == 0, "num_heads must be a multiple of num_kv_heads")
    _need(hd == 128, "head_dim must be 128")
    _need(k_caches[0].dim() == 4 and k_caches[0].dtype == torch.uint8,
          "KV caches must be uint8 [B, Hk, max_seq, head_dim]")
    max_seq = k_caches[0].shape[2]
    layers = (_R.R4QLayer * L)()
    for li in range(L):
        ly = layers[li]
        specs = (("qkv", qkv_w[li], qkv_s[li], qkv_N[li], D), ("o", o_w[li], o_s[li], o_N[li], H * hd),
                 ("gu", gu_w[li], gu_s[li], gu_N[li], D), ("down", down_w[li], down_s[li], down_N[li], I))
        for nm, w, s, n, k in specs:
            bits = weight_bits(w, k)
            _need(w.shape[0] == n and w.is_contiguous(), f"layer {li} {nm}: weight rows != {n}")
            if bits != 16:
                _need(s.numel() == n * k // 16, f"layer {li} {nm}: scale table size")
            setattr(ly, nm + "_w", w.data_ptr())
            setattr(ly, nm + "_s", None if bits == 16 else s.data_ptr())
            setattr(ly, nm + "_N", n)
            setattr(ly, nm + "_bits", bits)
        _need(qkv_N[li] == (H + 2 * Hk) * hd, f"layer {li}: qkv_N != (H+2Hk)*head_dim")
        _need(o_N[li] == D and down_N[li] == D and gu_N[li] == 2 * I, f"layer {li}: N mismatch")
        ly.in_norm = in_norm_w[li].data_ptr()
        ly.post_norm = post_norm_w[li].data_ptr()
        ly.q_norm = q_norm_w[li].data_ptr()
        ly.k_norm = k_norm_w[li].data_ptr()
        kc, vc = k_caches[li], v_caches[li]
        _need(kc.shape == vc.shape and kc.shape[1] == Hk and kc.shape[3] == hd
              and kc.shape[2] == max_seq and kc.is_contiguous() and vc.is_contiguous(),
              f"layer {li}: KV cache shape {tuple(kc.shape)}")
        ly.k_cache = kc.data_ptr()
        ly.v_cache = vc.data_ptr()
        if kv_scales is not None:
            ks, vs = kv_scales[0][li], kv_scales[1][li]
            _need(ks.dtype == torch.float32 and ks.numel() == Hk, "k scale must be float32 [Hk]")
            _need(vs.dtype == torch.float32 and vs.numel() == Hk, "v scale must be float32 [Hk]")
            ly.k_scale = ks.data_ptr()
            ly.v_scale = vs.data_ptr()
    st = _R.R4QModel()
    st.n_layers, st.n_heads, st.n_kv_heads, st.head_dim = L, H, Hk, hd
    st.hidden, st.inter, st.eps = D, I, float(rms_eps)
    st.max_seq = max_seq
    _need(rope_cos.shape == rope_sin.shape and rope_cos.shape[1] == hd // 2,
          "rope tables must be [P, head_dim/2]")
    st.rope_len = rope_cos.shape[0]
    st.layers = layers
    st.rope_cos, st.rope_sin = rope_cos.data_ptr(), rope_sin.data_ptr()
    if final_norm_w is not None and lm_w is not None:
        _need(lm_K == D, "lm_K must equal hidden_size")
        bits = weight_bits(lm_w, lm_K)
        st.final_norm = final_norm_w.data_ptr()
        st.lm_w = lm_w.data_ptr()
        st.lm_s = None if bits == 16 else lm_s.data_ptr()
        st.lm_N, st.lm_K, st.lm_bits = lm_N, lm_K, bits
    if embed_weight is not None:
        _cuda_half(embed_weight, "embed_weight")
        st.embed = embed_weight.data_ptr()
        st.vocab = embed_weight.shape[0]
    m = _Model(st, layers)
    _watch(m, key, args)
    _models[key] = m
    return m


def _decode_common(hidden_in, layer_args, k_caches, v_caches, final=None, embed=None,
                   kv_scales=None):
    (qkv_w, qkv_s, qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N, down_w, down_s, down_N,
     in_norm_w, post_norm_w, q_norm_w, k_norm_w, rope_cos, rope_sin, pos,
     num_heads, num_kv_heads, head_dim, hidden_size, intermediate_size, rms_eps) = layer_args
    fn, lw, ls, lN, lK = final if final is not None else (None, None, None, 0, 0)
    m = build_model(qkv_w, qkv_s, qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N, down_w, down_s, down_N,
                    in_norm_w, post_norm_w, q_norm_w, k_norm_w, rope_cos, rope_sin, num_heads,
                    num_kv_heads, head_dim, hidden_size, intermediate_size, rms_eps, k_caches,
                    v_caches, fn, lw, ls, lN, lK, embed, kv_scales)
    _cuda_half(hidden_in, "hidden_in")
    B = hidden_in.numel() // hidden_size
    _need(B * hidden_size == hidden_in.numel(), "hidden size mismatch")
    _need(k_caches[0].shape[0] >= B, "KV cache batch smaller than the hidden batch")
    return m, B, int(pos)


def _step_entry(use_graph):
    """The C entry point of one decode step: eager launches unless the caller
    asks for the graph-replayed step (use_graph=True; it runs the eager
    launches itself when the caller is capturing the stream).  A per-token
    caller synchronises on every token (the engine's .item()), so the host
    time before the GPU starts is on the critical path: the first eager
    launch starts the GPU while the rest are enqueued, whereas a replay of
    the ~240-node step graph starts it only after hipGraphLaunch returns.
    Measured on MI355X, engine loop at ctx 2048: 2.86 ms/token eager against
    3.11 ms/token replayed (the graph-replayed multi-step loop: 2.75 ms)."""
    return "r4q_decode_step_graph" if use_graph else "r4q_decode_step"


def decode_step(hidden_in, qkv_w, qkv_s, qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N, down_w, down_s,
                down_N, in_norm_w, post_norm_w, q_norm_w, k_norm_w, rope_cos, rope_sin, pos,
                num_heads, num_kv_heads, head_dim, hidden_size, intermediate_size, rms_eps,
                k_caches, v_caches, hadamard_mat, *, kv_scales=None, use_graph=None):
    """All layers for one token; returns the final hidden state [B, 1, D]
    (hip:2343-2528).  `hadamard_mat` is accepted and unused, as in the
    reference's live kernels.  use_graph=True replays the step from a
    captured hipGraph instead of launching it (bit-identical results)."""
    la = (qkv_w, qkv_s, qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N, down_w, down_s, down_N, in_norm_w,
          post_norm_w, q_norm_w, k_norm_w, rope_cos, rope_sin, pos, num_heads, num_kv_heads,
          head_dim, hidden_size, intermediate_size, rms_eps)
    m, B, pos = _decode_common(hidden_in, la, k_caches, v_caches, kv_scales=kv_scales)
    out = torch.empty((B, 1, hidden_size), dtype=torch.float16, device=hidden_in.device)
    _R.call(_step_entry(use_graph), _context(), C.byref(m.struct), hidden_in.data_ptr(), B, pos,
            out.data_ptr(), None, _stream())
    return out


def decode_step_logits(hidden_in, qkv_w, qkv_s, qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N, down_w,
                       down_s, down_N, in_norm_w, post_norm_w, q_norm_w, k_norm_w, rope_cos,
                       rope_sin, pos, num_heads, num_kv_heads, head_dim, hidden_size,
                       intermediate_size, rms_eps, k_caches, v_caches, final_norm_w, lm_w, lm_s,
                       lm_N, lm_K, hadamard_mat, *, kv_scales=None, use_graph=None):
    """All layers + final norm + LM head; returns logits [B, 1, lm_N] fp16
    (hip:2534-2595).  The engine calls this once per token
    (int4_engine_v5.py:272).  use_graph=True replays the step from a
    captured hipGraph with the position set on the device (bit-identical to
    the eager launches, the default: see _step_entry)."""
    la = (qkv_w, qkv_s, qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N, down_w, down_s, down_N, in_norm_w,
          post_norm_w, q_norm_w, k_norm_w, rope_cos, rope_sin, pos, num_heads, num_kv_heads,
          head_dim, hidden_size, intermediate_size, rms_eps)
    m, B, pos = _decode_common(hidden_in, la, k_caches, v_caches,
                               final=(final_norm_w, lm_w, lm_s, lm_N, lm_K), kv_scales=kv_scales)
    logits = torch.empty((B, 1, lm_N), dtype=torch.float16, device=hidden_in.device)
    _R.call(_step_entry(use_graph), _context(), C.byref(m.struct), hidden_in.data_ptr(), B, pos,
            None, logits.data_ptr(), _stream())
    return logits


def _bench(hidden_in, embed_weight, num_tokens, rest, use_graph, tokens_out=None,
           kv_scales=None, temperature=0.0, top_p=1.0, seed=0):
    (qkv_w, qkv_s, qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N, down_w, down_s, down_N, in_norm_w,
     post_norm_w, q_norm_w, k_norm_w, rope_cos, rope_sin, start_pos, num_heads, num_kv_heads,
     head_dim, hidden_size, intermediate_size, rms_eps, k_caches, v_caches, final_norm_w, lm_w,
     lm_s, lm_N, lm_K, _had) = rest
    la = (qkv_w, qkv_s, qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N, down_w, down_s, down_N, in_norm_w,
          post_norm_w, q_norm_w, k_norm_w, rope_cos, rope_sin, start_pos, num_heads,
          num_kv_heads, head_dim, hidden_size, intermediate_size, rms_eps)
    m, B, pos = _decode_common(hidden_in, la, k_caches, v_caches,
                               final=(final_norm_w, lm_w, lm_s, lm_N, lm_K), embed=embed_weight,
                               kv_scales=kv_scales)
    toks = None if tokens_out is None else tokens_out.data_ptr()
    if temperature > 0:
        _R.call("r4q_decode_generate", _context(), C.byref(m.struct), hidden_in.data_ptr(), B,
                int(num_tokens), pos, 1 if use_graph else 0, float(temperature), float(top_p),
                int(seed) & (2 ** 64 - 1), toks, _stream())
    else:
        _R.call("r4q_decode_bench", _context(), C.byref(m.struct), hidden_in.data_ptr(), B,
                int(num_tokens), pos, 1 if use_graph else 0, toks, _stream())


def decode_bench(hidden_in, embed_weight, num_tokens, *rest, kv_scales=None):
    """num_tokens greedy steps in one C++ loop, argmax + embedding on the
    device between steps (hip:2601-2795)."""
    _bench(hidden_in, embed_weight, num_tokens, rest, False, kv_scales=kv_scales)


def decode_bench_graph(hidden_in, embed_weight, num_tokens, *rest, kv_scales=None):
    """Captures one step in a hipGraph and replays it num_tokens times with
    the position in device memory (hip:2801-3041)."""
    _bench(hidden_in, embed_weight, num_tokens, rest, True, kv_scales=kv_scales)


def decode_loop(embed_weight, final_norm_w, lm_w, lm_s, lm_N, lm_K, first_token_hidden, num_tokens,
                qkv_w, qkv_s, qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N, down_w, down_s, down_N,
                in_norm_w, post_norm_w, q_norm_w, k_norm_w, rope_cos, rope_sin, start_pos,
                num_heads, num_kv_heads, head_dim, hidden_size, intermediate_size, rms_eps,
                k_caches, v_caches, hadamard_mat, *, kv_scales=None, temperature=0.0,
                top_p=1.0, seed=0, use_graph=False):
    """Decode of num_tokens tokens with the next token chosen on the device;
    returns the token ids as a CPU int64 tensor [num_tokens] (hip:3284-3466).
    Greedy by default, as in the reference; temperature > 0 samples with
    top_p on the device (the engine's Python sampling,
    int4_engine_v5.py:387-399) from the counter-based stream of `seed` (see
    `sample`).  use_graph=True replays one captured step per token."""
    B = first_token_hidden.numel() // hidden_size
    toks = torch.empty((int(num_tokens), B), dtype=torch.int64, device=first_token_hidden.device)
    rest = (qkv_w, qkv_s, qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N, down_w, down_s, down_N,
            in_norm_w, post_norm_w, q_norm_w, k_norm_w, rope_cos, rope_sin, start_pos, num_heads,
            num_kv_heads, head_dim, hidden_size, intermediate_size, rms_eps, k_caches, v_caches,
            final_norm_w, lm_w, lm_s, lm_N, lm_K, hadamard_mat)
    _bench(first_token_hidden, embed_weight, num_tokens, rest, use_graph, tokens_out=toks,
           kv_scales=kv_scales, temperature=temperature, top_p=top_p, seed=seed)
    out = toks.to("cpu")
    return out[:, 0] if B == 1 else out


def sample(logits, temperature=0.0, top_p=1.0, seed=0, counter=0):
    """Next token id of each row of fp16 logits [..., V] on the device, as an
    int64 tensor of the leading shape -- the engine's Python sampling
    (int4_engine_v5.py:330-335, 387-399) without the host round trip:
    temperature <= 0 is argmax (lowest index of the maximum); otherwise a
    draw from softmax(logits / temperature) over the tokens whose cumulative
    probability before them (descending, ties by index) is < top_p, with the
    uniform of row b taken from splitmix64(splitmix64(seed ^ counter) ^ b)."""
    _need(logits.is_cuda and logits.dtype == torch.float16, "logits must be cuda float16")
    V = logits.shape[-1]
    rows = logits.reshape(-1, V)
    if rows.stride(-1) != 1 or rows.stride(0) < V:
        rows = rows.contiguous()
    out = torch.empty(rows.shape[0], dtype=torch.int64, device=logits.device)
    _R.call("r4q_sample", _context(), rows.data_ptr(), rows.shape[0], V, rows.stride(0),
            float(temperature), float(top_p), int(seed) & (2 ** 64 - 1), int(counter),
            out.data_ptr(), _stream())
    return out.reshape(logits.shape[:-1])


def decode_profile(hidden_in, embed_weight, qkv_w, qkv_s, qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N,
                   down_w, down_s, down_N, in_norm_w, post_norm_w, q_norm_w, k_norm_w, rope_cos,
                   rope_sin, start_pos, num_heads, num_kv_heads, head_dim, hidden_size,
                   intermediate_size, rms_eps, k_caches, v_caches, final_norm_w, lm_w, lm_s, lm_N,
                   lm_K, hadamard_mat, *, kv_scales=None) -> List[float]:
    """[total, gemv, attention, norm, rest] milliseconds for one step at
    start_pos, from HIP events (hip:3047-3273)."""
    la = (qkv_w, qkv_s, qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N, down_w, down_s, down_N, in_norm_w,
          post_norm_w, q_norm_w, k_norm_w, rope_cos, rope_sin, start_pos, num_heads,
          num_kv_heads, head_dim, hidden_size, intermediate_size, rms_eps)
    m, B, pos = _decode_common(hidden_in, la, k_caches, v_caches,
                               final=(final_norm_w, lm_w, lm_s, lm_N, lm_K), kv_scales=kv_scales)
    out = (C.c_float * 5)()
    _R.call("r4q_decode_profile", _context(), C.byref(m.struct), hidden_in.data_ptr(), pos, out,
            _stream())
    return [float(v) for v in out]


_dummy_caches = {}


def prefill_logits(input_ids, embed_weight, final_norm_w, lm_w, lm_s, lm_N, lm_K, qkv_w, qkv_s,
                   qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N, down_w, down_s, down_N, in_norm_w,
                   post_norm_w, q_norm_w, k_norm_w, rope_cos, rope_sin, num_heads, num_kv_heads,
                   head_dim, hidden_size, intermediate_size, rms_eps, hadamard_mat, *,
                   k_caches=None, v_caches=None, kv_scales=None) -> torch.Tensor:
    """Logits [M, lm_N] for M prompt tokens (hip:2127-2320).  With the
    extended k_caches/v_caches keywords the FP8 KV cache is also filled at
    positions 0..M-1 (the reference's C++ prefill does not write it)."""
    _need(input_ids.dtype == torch.int64 and input_ids.is_cuda, "input_ids must be cuda int64")
    ids = input_ids.reshape(-1).contiguous()
    M = ids.numel()
    write_kv = k_caches is not None
    if not write_kv:
        # The C ABI needs caches to describe the layers; use a one-slot dummy
        # (kept, so repeated calls reuse one model descriptor).
        dkey = (str(input_ids.device), num_kv_heads, head_dim)
        dummy = _dummy_caches.get(dkey)
        if dummy is None:
            dummy = torch.zeros((1, num_kv_heads, 1, head_dim), dtype=torch.uint8,
                                device=input_ids.device)
            _dummy_caches[dkey] = dummy
        k_caches = [dummy] * len(qkv_w)
        v_caches = [dummy] * len(qkv_w)
    m = build_model(qkv_w, qkv_s, qkv_N, o_w, o_s, o_N, gu_w, gu_s, gu_N, down_w, down_s, down_N,
                    in_norm_w, post_norm_w, q_norm_w, k_norm_w, rope_cos, rope_sin, num_heads,
                    num_kv_heads, head_dim, hidden_size, intermediate_size, rms_eps, k_caches,
                    v_caches, final_norm_w, lm_w, lm_s, lm_N, lm_K, embed_weight, kv_scales)
    logits = torch.empty((M, lm_N), dtype=torch.float16, device=input_ids.device)
    _R.call("r4q_prefill_logits", _context(), C.byref(m.struct), ids.data_ptr(), M,
            logits.data_ptr(), 1 if write_kv else 0, _stream())
    return logits
