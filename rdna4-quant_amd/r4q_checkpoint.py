"""Loader for the reference's on-disk quantized model directory
(quantized_*/: meta.pt, embed.pt, final_norm.pt, lm_head.pt, layer_XXX.pt;
keys in REPRODUCTION_RECIPE.md:214-283, written by quantize_v4_gptq.py:385-468,
read by int4_engine_v5.py:79-181).

Produces the int4_hip argument lists directly, so a real checkpoint runs
through this library's kernels:
  * INT4 groups `{g}_packed` [N, K/2] u8 + `{g}_scales` [N, K/32] + `{g}_zeros`
    [N, K/32] u8 -> (packed, interleaved (scale, zero) fp16 [N, K/16])
    (interleave_scale_zero, int4_engine_v5.py:95-102).  The writers store
    `{g}_zeros` for every INT4 group (quantize_v4_gptq.py:397-403,
    quantize_v5_pure_int4.py:353-358); the tag `{g}_precision` tells the two
    formats apart: 'int4a' is asymmetric (unsigned nibbles, zero points as
    stored), 'int4' symmetric (two's-complement nibbles, zeros all 0,
    int4_quant_v2.py:240-247), which becomes unsigned nibbles with zero point
    8 (convert_symmetric_to_asymmetric, int4_engine_v5.py:105-118).  Without
    a tag, meta['use_asymmetric'] decides, and without that a missing zeros
    key means symmetric;
  * INT8 groups `{g}_weights` [N, K] int8 + `{g}_scales` (symmetric, the v4
    format the reference engine cannot run) -> uint8 q + 128 with zero point
    128 in the same interleaved table, which the INT8 GEMV consumes;
  * lm_head.pt: asymmetric (packed, scales, zeros) or symmetric INT4
    (packed, scales; quant_format 'int4_symmetric'), converted the same way
    (int4_engine_v5.py:163-176);
  * norms, embedding and final norm cast to fp16.
Every file is read with torch.load(weights_only=True): tensors, numbers,
strings and dicts only, nothing executed from the file.
"""
from __future__ import annotations

import math
from pathlib import Path

import torch

GROUPS = ("qkv", "o", "gate_up", "down")
_ARG = {"qkv": "qkv", "o": "o", "gate_up": "gu", "down": "down"}


def _load(path: Path):
    return torch.load(path, map_location="cpu", weights_only=True)


def interleave_scale_zero(scales: torch.Tensor, zeros: torch.Tensor) -> torch.Tensor:
    """[N, K/32] fp16 scales + [N, K/32] integer zeros -> [N, K/16] fp16 with
    (scale, zero) pairs per block."""
    sz = torch.stack([scales.half(), zeros.to(torch.float16)], dim=-1).contiguous()
    return sz.view(sz.shape[0], -1)


def sym_int4_to_asym(packed: torch.Tensor):
    """Two's-complement nibbles n -> (n + 8) & 0xF (value (n' - 8) * s)."""
    lo = (packed & 0x0F) + 8
    hi = ((packed >> 4) & 0x0F) + 8
    return ((lo & 0x0F) | ((hi & 0x0F) << 4)).to(torch.uint8)


def int4_is_symmetric(precision, zeros, meta) -> bool:
    """Symmetric (two's-complement) or asymmetric INT4 group: the writer's
    `{g}_precision` tag first ('int4' symmetric, 'int4a' asymmetric), then
    the checkpoint-wide meta['use_asymmetric'], then a missing zeros key."""
    if precision in ("int4", "int4a"):
        return precision == "int4"
    if meta is not None and "use_asymmetric" in meta:
        return not bool(meta["use_asymmetric"])
    return zeros is None


def _int4_group(packed, scales, zeros, symmetric, device):
    N = packed.shape[0]
    nb = scales.shape[1]
    if symmetric:
        packed = sym_int4_to_asym(packed)
        zeros = torch.full((N, nb), 8, dtype=torch.uint8)
    elif zeros is None:
        raise ValueError("asymmetric INT4 group without zero points")
    return (packed.contiguous().to(device),
            interleave_scale_zero(scales, zeros).to(device).contiguous())


def _int8_group(weights, scales, device):
    q = (weights.to(torch.int16) + 128).to(torch.uint8)
    zeros = torch.full(scales.shape, 128, dtype=torch.int16)
    return q.contiguous().to(device), interleave_scale_zero(scales, zeros).to(device).contiguous()


def rope_tables(head_dim: int, n_pos: int, theta: float, device):
    """cos/sin [n_pos, head_dim/2] fp16, built as precompute_rope_freqs does
    (engine_utils.py:70-76): float32 frequencies and angles on `device`,
    cos/sin in float32, then rounded to fp16."""
    freqs = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device).float() / head_dim))
    t = torch.arange(n_pos, device=device).float()
    ang = torch.outer(t, freqs)
    return ang.cos().half(), ang.sin().half()


class QuantizedModel:
    """A loaded checkpoint as int4_hip arguments (attributes named like the
    reference engine's lists)."""

    def layer_block(self, pos):
        """The decode-family layer argument block up to rms_eps."""
        return (self.qkv_w, self.qkv_s, self.qkv_N, self.o_w, self.o_s, self.o_N, self.gu_w,
                self.gu_s, self.gu_N, self.down_w, self.down_s, self.down_N, self.in_norm,
                self.post_norm, self.q_norm, self.k_norm, self.rope_cos, self.rope_sin, pos,
                self.num_heads, self.num_kv_heads, self.head_dim, self.hidden_size,
                self.intermediate_size, self.rms_eps)

    def new_kv_caches(self, batch: int = 1, max_seq: int | None = None):
        """Zeroed FP8 KV caches, per layer uint8 [batch, Hk, max_seq, head_dim]."""
        n = max_seq or self.max_seq
        shape = (batch, self.num_kv_heads, n, self.head_dim)
        k = [torch.zeros(shape, dtype=torch.uint8, device=self.device)
             for _ in range(self.num_layers)]
        v = [torch.zeros(shape, dtype=torch.uint8, device=self.device)
             for _ in range(self.num_layers)]
        return k, v


def load_quantized(quant_dir, device="cuda", max_seq: int = 2048,
                   rope_extra: int = 128) -> QuantizedModel:
    """Reads a quantized model directory into device tensors."""
    d = Path(quant_dir)
    meta = _load(d / "meta.pt")
    m = QuantizedModel()
    m.device = torch.device(device)
    m.meta = meta
    for k in ("num_layers", "hidden_size", "intermediate_size", "num_heads", "num_kv_heads",
              "head_dim"):
        setattr(m, k, int(meta[k]))
    m.rms_eps = float(meta["rms_eps"])
    m.rope_theta = float(meta.get("rope_theta", 1.0e6))
    m.max_seq = max_seq
    for name in ("qkv", "o", "gu", "down"):
        for suf in ("_w", "_s", "_N"):
            setattr(m, name + suf, [])
    m.in_norm, m.post_norm, m.q_norm, m.k_norm = [], [], [], []
    m.precision = []
    for li in range(m.num_layers):
        ld = _load(d / f"layer_{li:03d}.pt")
        prec = {}
        for g in GROUPS:
            a = _ARG[g]
            if f"{g}_weights" in ld:  # INT8 (symmetric)
                w, s = _int8_group(ld[f"{g}_weights"], ld[f"{g}_scales"], m.device)
                prec[g] = "int8"
            else:
                zeros = ld.get(f"{g}_zeros")
                sym = int4_is_symmetric(ld.get(f"{g}_precision"), zeros, meta)
                w, s = _int4_group(ld[f"{g}_packed"], ld[f"{g}_scales"], zeros, sym, m.device)
                prec[g] = "int4" if sym else "int4a"
            getattr(m, a + "_w").append(w)
            getattr(m, a + "_s").append(s)
            getattr(m, a + "_N").append(int(ld[f"{g}_N"]))
        m.precision.append(prec)
        for k in ("in_norm", "post_norm", "q_norm", "k_norm"):
            getattr(m, k).append(ld[k].to(torch.float16).contiguous().to(m.device))
        del ld
    lm = _load(d / "lm_head.pt")
    m.lm_N, m.lm_K = int(lm["N"]), int(lm["K"])
    lm_sym = "zeros" not in lm or lm.get("quant_format") == "int4_symmetric"
    m.lm_w, m.lm_s = _int4_group(lm["packed"], lm["scales"], lm.get("zeros"), lm_sym, m.device)
    m.embed = _load(d / "embed.pt").to(torch.float16).contiguous().to(m.device)
    m.final_norm = _load(d / "final_norm.pt").to(torch.float16).contiguous().to(m.device)
    m.vocab = m.embed.shape[0]
    m.rope_cos, m.rope_sin = rope_tables(m.head_dim, max_seq + rope_extra, m.rope_theta,
                                         m.device)
    m.hadamard = torch.zeros(32, 32, dtype=torch.float16, device=m.device)
    h = torch.ones(1, 1, dtype=torch.float32)
    while h.shape[0] < 32:
        h = torch.cat([torch.cat([h, h], 1), torch.cat([h, -h], 1)], 0)
    m.hadamard.copy_((h / math.sqrt(32)).half())  # passed to the API, unused by its kernels
    return m
