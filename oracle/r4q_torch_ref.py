"""Torch CPU restatement of the reference's own torch path for the decode /
prompt pass (JohnTDI-cpu/rdna4-quant int4_engine_v5.py, engine_utils.py).

TEST INFRASTRUCTURE, like r4q_oracle: only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg import it.  The product (librdna4q.so and
the rdna4-quant_amd package) never does.

It serves two purposes:
  * an independent route for the oracle's layer composition (the oracle is
    a numpy restatement of the HIP kernels; this one restates the engine's
    torch code: fast_rmsnorm -> .half() -> fast_hadamard, dequant + matmul,
    head_rmsnorm, apply_rope, SDPA, F.silu(g) * u, fp16 residual adds);
  * the CPU baseline that bench.py times: the same torch operations on the
    host cores, with the weights dequantised on the fly per matrix (as
    fast_prefill does, int4_engine_v5.py:214-266) or once, up front.

`mm` is the matrix product in use: `mm_ref` is the reference's literal
`x @ w.T` on fp16 tensors (int4_engine_v5.py:228), timed by the baseline;
`mm_acc32` models the GPU's fp16 GEMM with fp32 accumulation and one final
rounding, which the composition test uses.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

import r4q_oracle as O


def dequant(w: torch.Tensor, sz: torch.Tensor, bits: int) -> torch.Tensor:
    """fp16 [N, K] from packed INT4 [N, K/2] (element 2j in the low nibble)
    or INT8 [N, K] bytes and the interleaved (scale, zero) table [N, K/16]
    (or [N, K/32, 2]): (q - zp) * scale in fp32, then fp16
    (dequantize_int4_asym, int4_quant_v2.py:97-127; the INT8 groups use the
    same asymmetric rule).  FP16 weights (bits 16) pass through."""
    if bits == 16:
        return w
    N = w.shape[0]
    if bits == 4:
        q = torch.stack([w & 0x0F, w >> 4], -1).reshape(N, -1)
    else:
        q = w
    K = q.shape[1]
    t = sz.reshape(N, K // 32, 2).float()
    qf = q.reshape(N, K // 32, 32).float()
    return ((qf - t[..., 1:2]) * t[..., 0:1]).reshape(N, K).half()


def mm_ref(x16: torch.Tensor, w16: torch.Tensor) -> torch.Tensor:
    """`x @ w.T` on fp16 tensors, as the engine writes it (int4_engine_v5.py:228)."""
    return x16 @ w16.T


def mm_acc32(x16: torch.Tensor, w16: torch.Tensor) -> torch.Tensor:
    """x @ w.T as an fp16 GEMM with fp32 accumulation (rocBLAS / hipBLASLt)."""
    return (x16.float() @ w16.float().T).half()


def hadamard_fp16() -> torch.Tensor:
    """The engine's `had_mat`: Sylvester H32 / sqrt(32) in fp16
    (hadamard_utils.py:14-34)."""
    return torch.from_numpy(O.hadamard_matrix(32) / math.sqrt(32)).float().half()


def fast_hadamard(x: torch.Tensor, mm=mm_acc32, had=None) -> torch.Tensor:
    """x.view(-1, 32) @ had_mat (int4_engine_v5.py:202-205)."""
    had = hadamard_fp16() if had is None else had
    return mm(x.reshape(-1, 32), had.T).reshape(x.shape)


def fast_rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """int4_engine_v5.py:208-211."""
    var = x.float().pow(2).mean(-1, keepdim=True)
    return (x.float() * torch.rsqrt(var + eps) * w.float()).half()


def head_rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """int4_engine_v5.py:195-199."""
    var = x.float().pow(2).mean(-1, keepdim=True)
    return (x.float() * torch.rsqrt(var + eps) * w.float()).half()


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
               pos: torch.Tensor) -> torch.Tensor:
    """Half-split RoPE of x [1, heads, M, 128] at positions pos [1, M]
    (engine_utils.py:79-107)."""
    c = cos[pos].unsqueeze(1)
    s = sin[pos].unsqueeze(1)
    x1, x2 = x[..., :64], x[..., 64:]
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], -1)


def fp8_table() -> torch.Tensor:
    """float32 value of every E4M3 code, the reference decoder (hip:71-81)."""
    return torch.from_numpy(O.fp8_decode_ref(np.arange(256, dtype=np.uint8)))


def prefill(layers, embed, final, lm_w, lm_s, ids, cos, sin, *, eps, H, Hk, I, lm_bits=4,
            mm=mm_acc32):
    """The engine's prompt pass, fast_prefill (int4_engine_v5.py:214-266),
    over oracle Layer records (numpy weights); returns (residual stream
    after each layer, logits of every row)."""
    had = hadamard_fp16()
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a))  # noqa: E731
    M = len(ids)
    pos = torch.arange(M).unsqueeze(0)
    x = T(embed)[torch.from_numpy(np.asarray(ids))]
    trace = []
    qd, kd = H * 128, Hk * 128
    for ly in layers:
        normed = fast_hadamard(fast_rmsnorm(x, T(ly.in_norm), eps), mm, had)
        qkv = mm(normed, dequant(T(ly.qkv_w), T(ly.qkv_s), ly.qkv_bits))
        q = head_rmsnorm(qkv[:, :qd].view(M, H, 128), T(ly.q_norm), eps)
        k = head_rmsnorm(qkv[:, qd:qd + kd].view(M, Hk, 128), T(ly.k_norm), eps)
        v = qkv[:, qd + kd:].view(M, Hk, 128)
        q = apply_rope(q.unsqueeze(0).transpose(1, 2), cos, sin, pos)
        k = apply_rope(k.unsqueeze(0).transpose(1, 2), cos, sin, pos)
        v = v.unsqueeze(0).transpose(1, 2)
        att = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True,
                                             enable_gqa=True).half()
        att = att.squeeze(0).transpose(0, 1).reshape(M, qd)
        x = x + mm(fast_hadamard(att, mm, had), dequant(T(ly.o_w), T(ly.o_s), ly.o_bits))
        normed = fast_hadamard(fast_rmsnorm(x, T(ly.post_norm), eps), mm, had)
        gu = mm(normed, dequant(T(ly.gu_w), T(ly.gu_s), ly.gu_bits))
        mlp = F.silu(gu[:, :I]) * gu[:, I:]
        x = x + mm(fast_hadamard(mlp, mm, had), dequant(T(ly.down_w), T(ly.down_s), ly.down_bits))
        trace.append(x.numpy().copy())
    normed = fast_hadamard(fast_rmsnorm(x, T(final), eps), mm, had)
    return trace, mm(normed, dequant(T(lm_w), T(lm_s) if lm_s is not None else None,
                                     lm_bits)).numpy()


def decode_layer(h, ly, pos, kc, vc, cos, sin, *, eps, H, Hk, I, lut, had, mm=mm_ref,
                 wts=None):
    """One layer of a batch-1 decode step on the engine's torch ops, for the
    CPU baseline: h [1, D] fp16; `ly` holds torch tensors (qkv_w, qkv_s,
    qkv_bits, ... , in_norm, post_norm, q_norm, k_norm); kc / vc the layer's
    FP8 code caches [Hk, max_seq, 128] uint8, written at `pos`; `lut` the
    E4M3 decode table.  Weights are dequantised here, per matrix, unless
    `wts` holds them already dequantised ({'qkv': fp16 [N, K], ...})."""
    def W(g):
        if wts is not None:
            return wts[g]
        return dequant(getattr(ly, g + "_w"), getattr(ly, g + "_s"), getattr(ly, g + "_bits"))

    qd, kd = H * 128, Hk * 128
    p = torch.tensor([[pos]])
    normed = fast_hadamard(fast_rmsnorm(h, ly.in_norm, eps), mm, had)
    qkv = mm(normed, W("qkv"))
    q = head_rmsnorm(qkv[:, :qd].view(1, H, 128), ly.q_norm, eps)
    k = head_rmsnorm(qkv[:, qd:qd + kd].view(1, Hk, 128), ly.k_norm, eps)
    v = qkv[:, qd + kd:].view(1, Hk, 128)
    q = apply_rope(q.unsqueeze(0).transpose(1, 2), cos, sin, p)
    k = apply_rope(k.unsqueeze(0).transpose(1, 2), cos, sin, p)
    # FP8 write at pos (fp16_to_fp8 of the rotated fp16 K and of V, hip:3606-3618)
    kc[:, pos] = torch.from_numpy(O.fp8_encode(k[0, :, 0].float().numpy()))
    vc[:, pos] = torch.from_numpy(O.fp8_encode(v[0].float().numpy()))
    kk = lut[kc[:, :pos + 1].long()].unsqueeze(0)
    vv = lut[vc[:, :pos + 1].long()].unsqueeze(0)
    att = F.scaled_dot_product_attention(q.float(), kk, vv, enable_gqa=True).half()
    att = att.reshape(1, qd)
    x = h + mm(fast_hadamard(att, mm, had), W("o"))
    normed = fast_hadamard(fast_rmsnorm(x, ly.post_norm, eps), mm, had)
    gu = mm(normed, W("gu"))
    mlp = F.silu(gu[:, :I]) * gu[:, I:]
    return x + mm(fast_hadamard(mlp, mm, had), W("down"))
