"""Seeded synthetic Qwen3-14B-shaped inputs for tests and benchmarks.

Distributions follow the benchmark configurations:
  * INT4 weights: nibbles uniform 0..15 packed two per byte, per-32-block
    scales fp16(|N(0,1)| * 0.01 + 1e-3), zero-points uniform 6..9;
  * INT8 weights: bytes uniform 0..255, the INT4 scale distribution / 16
    and zero-points uniform 126..129 (the INT4 zero-point range moved to the
    centre of the 8-bit code range), so INT8 layers dequantise to the same
    value range and mean as INT4 layers;
  * FP16 weights (embedding / LM head): 0.02 * N(0,1);
  * norm weights: fp16(1 + 0.02 * N(0,1));
  * activations: N(0,1) fp16, passed through the block-diagonal FWHT-32 when
    they feed a projection.
Tensors are produced with torch generators so the same seed gives the same
bytes on the CPU (for the oracle) and, via .to(device), on the GPU.
"""
from __future__ import annotations

import math

import torch

QWEN3_14B = dict(hidden=5120, inter=17408, heads=40, kv_heads=8, head_dim=128, layers=40,
                 vocab=151936, eps=1e-6, rope_theta=1.0e6)


def gen(seed: int, device="cpu") -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def sz_table(scales: torch.Tensor, zeros: torch.Tensor) -> torch.Tensor:
    """[N, nb] fp16 scales + integer zeros -> interleaved [N, 2*nb] fp16."""
    N = scales.shape[0]
    return torch.stack([scales.half(), zeros.to(torch.float32).half()], dim=-1).reshape(N, -1).contiguous()


def block_scales(N: int, nb: int, g: torch.Generator, device="cpu") -> torch.Tensor:
    return (torch.randn(N, nb, generator=g, device=device).abs() * 0.01 + 1e-3).half()


def int4_weight(N: int, K: int, g: torch.Generator, device="cpu"):
    """(packed uint8 [N, K/2], sz fp16 [N, K/16])."""
    q = torch.randint(0, 16, (N, K), generator=g, device=device, dtype=torch.uint8)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous()
    nb = K // 32
    scales = block_scales(N, nb, g, device)
    zeros = torch.randint(6, 10, (N, nb), generator=g, device=device)
    return packed, sz_table(scales, zeros)


def int8_weight(N: int, K: int, g: torch.Generator, device="cpu"):
    """(q uint8 [N, K], sz fp16 [N, K/16]).  Scales are the INT4 ones / 16 so
    the dequantised weights span the same range as the INT4 layers
    ((q - zp) in +-128 instead of +-8)."""
    q = torch.randint(0, 256, (N, K), generator=g, device=device, dtype=torch.uint8)
    nb = K // 32
    scales = (block_scales(N, nb, g, device).float() / 16).half()
    zeros = torch.randint(126, 130, (N, nb), generator=g, device=device)
    return q.contiguous(), sz_table(scales, zeros)


def fp16_weight(N: int, K: int, g: torch.Generator, device="cpu", std=0.02):
    return (torch.randn(N, K, generator=g, device=device) * std).half().contiguous(), None


def weight(N: int, K: int, bits: int, g: torch.Generator, device="cpu"):
    if bits == 4:
        return int4_weight(N, K, g, device)
    if bits == 8:
        return int8_weight(N, K, g, device)
    if bits == 16:
        return fp16_weight(N, K, g, device)
    raise ValueError(bits)


def hadamard32(device="cpu", dtype=torch.float32) -> torch.Tensor:
    H = torch.ones(1, 1, dtype=torch.float64)
    while H.shape[0] < 32:
        H = torch.cat([torch.cat([H, H], 1), torch.cat([H, -H], 1)], 0)
    return (H / math.sqrt(32)).to(device=device, dtype=dtype)


def rotated_activation(K: int, g: torch.Generator, device="cpu", rows: int = 1) -> torch.Tensor:
    """fp16(FWHT32(x)), x ~ N(0,1) fp16 (float32 rotation)."""
    x = torch.randn(rows, K, generator=g, device=device).half()
    H = hadamard32(device)
    return (x.float().reshape(-1, 32) @ H).reshape(rows, K).half().contiguous()


def norm_weight(D: int, g: torch.Generator, device="cpu") -> torch.Tensor:
    return (1.0 + 0.02 * torch.randn(D, generator=g, device=device)).half().contiguous()


def rope_tables(head_dim: int, max_pos: int, theta: float = 1.0e6, device="cpu"):
    """fp16 cos/sin [max_pos, head_dim/2] built as precompute_rope_freqs does
    (engine_utils.py:70-76): float32 frequencies, positions and angles, cos and
    sin in float32, then fp16 (on the CPU, so the tables do not depend on the
    device)."""
    freqs = 1.0 / (theta ** (torch.arange(0, head_dim, 2).float() / head_dim))
    ang = torch.outer(torch.arange(max_pos).float(), freqs)
    return ang.cos().half().to(device).contiguous(), ang.sin().half().to(device).contiguous()


def precision_mask(n_layers: int, seed: int = 4, frac_int8: float = 0.2):
    """{(layer, group): bits} with exactly round(frac*4L) INT8 matrices chosen
    by torch.randperm(4L, seed); groups = qkv, o, gate_up, down."""
    n = 4 * n_layers
    k = int(round(frac_int8 * n))
    perm = torch.randperm(n, generator=gen(seed))[:k].tolist()
    groups = ("qkv", "o", "gu", "down")
    bits = {(li, gname): 4 for li in range(n_layers) for gname in groups}
    for idx in perm:
        bits[(idx // 4, groups[idx % 4])] = 8
    return bits


def make_layer(D, I, H, Hk, hd, g, device="cpu", bits=None):
    """One decoder layer's tensors as a dict keyed like the int4_hip argument
    lists (qkv_w, qkv_s, qkv_N, ..., in_norm, post_norm, q_norm, k_norm)."""
    bits = bits or {}
    out = {}
    shapes = {"qkv": ((H + 2 * Hk) * hd, D), "o": (D, H * hd), "gu": (2 * I, D), "down": (D, I)}
    for name, (N, K) in shapes.items():
        b = bits.get(name, 4)
        w, s = weight(N, K, b, g, device)
        out[name + "_w"], out[name + "_s"], out[name + "_N"], out[name + "_bits"] = w, s, N, b
    out["in_norm"] = norm_weight(D, g, device)
    out["post_norm"] = norm_weight(D, g, device)
    out["q_norm"] = norm_weight(hd, g, device)
    out["k_norm"] = norm_weight(hd, g, device)
    return out


def random_kv_values(Hk: int, n_fill: int, hd: int, g: torch.Generator, device="cpu",
                     batch: int = 1, scale: float = 1.0) -> torch.Tensor:
    """fp16 [batch, Hk, n_fill, hd] ~ N(0,1) * scale: values to be encoded into
    an FP8 KV cache (by the library's fp16_to_fp8 on the device, or by the
    oracle in CPU tests)."""
    return (torch.randn(batch, Hk, n_fill, hd, generator=g, device=device) * scale).half()


def fp8_caches(n_layers: int, Hk: int, hd: int, ctx: int, capacity: int, batch: int,
               g: torch.Generator, device) -> tuple:
    """Per-layer FP8 K and V caches uint8 [batch, Hk, capacity, hd] whose
    positions [0, ctx) hold the reference encoder's codes of N(0,1) values
    (the library's fp16_to_fp8) and the rest zeros."""
    import int4_hip

    kc, vc = [], []
    for _ in range(n_layers):
        k = torch.zeros(batch, Hk, capacity, hd, dtype=torch.uint8, device=device)
        v = torch.zeros_like(k)
        k[:, :, :ctx] = int4_hip.fp16_to_fp8(random_kv_values(Hk, ctx, hd, g, device, batch))
        v[:, :, :ctx] = int4_hip.fp16_to_fp8(random_kv_values(Hk, ctx, hd, g, device, batch))
        kc.append(k)
        vc.append(v)
    return kc, vc


def qwen3_model(ctx: int, extra: int, batch: int, device, log=None, rope_len: int = 0) -> dict:
    """The BASELINE config-4 model, generated on `device`: 40 Qwen3-14B-shaped
    layers (seed 4; 32 of the 160 projection matrices INT8 by
    precision_mask), FP16 embedding and LM head, FP8 KV caches of capacity
    ctx + extra per layer with positions [0, ctx) holding the reference
    encoder's codes of N(0,1) values (the library's fp16_to_fp8).  The RoPE
    tables have max(ctx + extra, rope_len) rows.  Returns a dict with the
    int4_hip argument lists ("args"), caches ("kc", "vc"), RoPE tables, final
    norm, LM head, embedding, dims and byte counts."""
    c = QWEN3_14B
    D, I, H, Hk, hd, L, V = c["hidden"], c["inter"], c["heads"], c["kv_heads"], c["head_dim"], \
        c["layers"], c["vocab"]
    g = gen(4, device)
    mask = precision_mask(L, seed=4)
    args = {k: [] for k in ("qkv_w", "qkv_s", "qkv_N", "o_w", "o_s", "o_N", "gu_w", "gu_s", "gu_N",
                            "down_w", "down_s", "down_N", "in_norm", "post_norm", "q_norm",
                            "k_norm")}
    wbytes = 0
    for li in range(L):
        bits = {n: mask[(li, n)] for n in ("qkv", "o", "gu", "down")}
        ly = make_layer(D, I, H, Hk, hd, g, device=device, bits=bits)
        for k in args:
            args[k].append(ly[k])
        for n in ("qkv", "o", "gu", "down"):
            N = ly[n + "_N"]
            K = {"qkv": D, "o": H * hd, "gu": D, "down": I}[n]
            wbytes += N * K * ly[n + "_bits"] // 8 + N * (K // 32) * 3
        if log and (li + 1) % 10 == 0:
            log(f"layer {li + 1}/{L} generated")
    max_seq = ctx + extra
    kc, vc = fp8_caches(L, Hk, hd, ctx, max_seq, batch, g, device)
    cos, sin = rope_tables(hd, max(max_seq, rope_len), c["rope_theta"], device)
    final_norm = norm_weight(D, g, device)
    lm_w, _ = fp16_weight(V, D, g, device)
    embed, _ = fp16_weight(V, D, g, device)
    return dict(args=args, kc=kc, vc=vc, cos=cos, sin=sin, final_norm=final_norm, lm_w=lm_w,
                embed=embed, D=D, I=I, H=H, Hk=Hk, hd=hd, L=L, V=V, eps=c["eps"], mask=mask,
                max_seq=max_seq, wbytes=wbytes, lm_bytes=V * D * 2)


def qwen3_bench_args(m: dict, start_pos: int, caches: tuple = None) -> tuple:
    """int4_hip decode_bench / decode_loop argument tail of a qwen3_model
    (layer block at start_pos, caches, final norm, LM head, hadamard);
    `caches` = (k list, v list) replaces the model's own caches."""
    a = m["args"]
    kc, vc = caches if caches is not None else (m["kc"], m["vc"])
    had = m.get("had")
    if had is None:
        had = m["had"] = torch.zeros(32, 32, dtype=torch.float16, device=m["lm_w"].device)
    return (a["qkv_w"], a["qkv_s"], a["qkv_N"], a["o_w"], a["o_s"], a["o_N"], a["gu_w"],
            a["gu_s"], a["gu_N"], a["down_w"], a["down_s"], a["down_N"], a["in_norm"],
            a["post_norm"], a["q_norm"], a["k_norm"], m["cos"], m["sin"], start_pos, m["H"],
            m["Hk"], m["hd"], m["D"], m["I"], m["eps"], kc, vc, m["final_norm"],
            m["lm_w"], None, m["V"], m["D"], had)
