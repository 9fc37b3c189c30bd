"""CPU oracle for the decode-step hot path — TEST INFRASTRUCTURE ONLY.

This module restates, in numpy, the arithmetic of the reference decode path
(JohnTDI-cpu/rdna4-quant; `hip:` = hip_int4/int4_decode_step.hip).  It is the
checker for the HIP library: only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import it.  The product path never calls it.

Every function cites the reference lines it follows.  How each function is
pinned (golden vectors, exhaustive tables, library routines, closed forms) is
listed in PINNING below and exercised by tests/test_oracle_*.py.

Conventions
  * fp16 tensors are numpy float16 arrays; INT4 weights are uint8 [N, K/2]
    (byte = q[2j] | q[2j+1] << 4); INT8 weights uint8 [N, K] (q in 0..255);
    scale/zero layout `sz` is float16 [N, K/32, 2] (scale, zero-point).
  * Element-wise steps run in float32 in the order the kernels use (so the
    FP8 KV bytes are reproducible bit-for-bit); dot products and attention
    accumulate in float64.
"""
from __future__ import annotations

import math

import numpy as np

PINNING = {
    "pack_int4/unpack_int4": "exhaustive over 256 bytes + reference roundtrip test "
                             "(tests/test_kernels.py:26-50)",
    "dequant_int4/dequant_int8": "exhaustive closed form over q, zp and every finite fp16 "
                                 "scale (float64 route) + reference test "
                                 "(tests/test_kernels.py:53-70)",
    "fp8_encode": "all 65536 fp16 inputs vs the golden table derived with exact "
                  "rationals (tests/golden/make_fp8_table.py); all 63488 finite fp16 "
                  "inputs vs torch.float8_e4m3fn with every difference classified "
                  "(flush / tie / saturation) and counted",
    "fp8_decode": "all 256 codes vs torch.float8_e4m3fn values",
    "fwht32": "Sylvester matrix (hadamard_utils.py:14-34), H H = I "
              "(tests/test_kernels.py:73-79), unit vectors, float64 matrix product",
    "rmsnorm*/res_rmsnorm*": "torch fast_rmsnorm + fast_hadamard restatement "
                             "(int4_engine_v5.py:202-211), constant-vector closed form",
    "silu_mul_fwht": "torch F.silu(g) * u then Hadamard matrix (int4_engine_v5.py:257)",
    "gemv/gemm": "torch CPU matmul of dequantised weights (int4_engine_v5.py:227-228), "
                 "one-hot inputs select exact weight columns",
    "head_norm_rope_kv": "torch head_rmsnorm + apply_rope restatement "
                         "(int4_engine_v5.py:195-199, engine_utils.py:79-107), "
                         "pos 0 identity",
    "flash_decode": "torch F.scaled_dot_product_attention(enable_gqa=True) on the "
                    "decoded cache (int4_engine_v5.py:245); seq_len 1 closed form",
    "decode_step": "composition of the pinned functions; equals row m of "
                   "prefill_logits(attend_fp8=True) at position m on the same caches "
                   "(rel-L2 <= 5e-3, logits and every layer's hidden state)",
    "decode_step_batch": "row b equals decode_step on row b (same functions, "
                         "projections over all rows at once)",
    "attention_prefill": "torch F.scaled_dot_product_attention(is_causal=True, "
                         "enable_gqa=True) (hip:2262-2264); M=1 closed form (= v)",
    "prefill_logits": "composition of the pinned functions; a torch restatement of "
                      "the reference's own prompt pass (fast_prefill, "
                      "int4_engine_v5.py:214-266) matches every layer's hidden state "
                      "and the logits (rel-L2 <= 5e-3, norm weights 0.5-1.5)",
    "sample_top_p": "kept set vs a literal torch restatement of the reference's top-p "
                    "code (int4_engine_v5.py:387-399: sort, cumsum, mask) in float64; "
                    "draw frequencies vs the renormalised kept distribution "
                    "(chi-square); temperature 0 == torch.argmax; splitmix64 against "
                    "its published test vector",
}

INV_SQRT32 = np.float32(0.17677669529663689)


# --------------------------------------------------------------------- a1/a3
def pack_int4(q: np.ndarray) -> np.ndarray:
    """byte = q[2j] | q[2j+1] << 4  (int4_quant_v2.py:87-94)."""
    q = np.asarray(q, dtype=np.uint8)
    return ((q[..., 0::2] & 0xF) | ((q[..., 1::2] & 0xF) << 4)).astype(np.uint8)


def unpack_int4(p: np.ndarray) -> np.ndarray:
    """element 2j = b & 0xF, element 2j+1 = b >> 4  (int4_quant_v2.py:97-102)."""
    p = np.asarray(p, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = p & 0xF
    out[..., 1::2] = p >> 4
    return out


def interleave_scale_zero(scales: np.ndarray, zeros: np.ndarray) -> np.ndarray:
    """[N, K/32] fp16 scales + uint8 zeros -> [N, K/32, 2] fp16
    (int4_engine_v5.py:95-102)."""
    z = np.asarray(zeros).astype(np.float32).astype(np.float16)
    return np.stack([np.asarray(scales, dtype=np.float16), z], axis=-1)


def sym_int4_to_asym(packed: np.ndarray, scales: np.ndarray):
    """Symmetric two's-complement nibbles -> unsigned with zp = 8
    (int4_engine_v5.py:105-118).  Returns (packed, sz)."""
    p = np.asarray(packed, dtype=np.uint8)
    lo = ((p & 0xF) + 8) & 0xF
    hi = (((p >> 4) & 0xF) + 8) & 0xF
    zeros = np.full(np.asarray(scales).shape, 8, dtype=np.uint8)
    return (lo | (hi << 4)).astype(np.uint8), interleave_scale_zero(scales, zeros)


def sym_int8_to_asym(w_int8: np.ndarray, scales: np.ndarray):
    """Symmetric int8 (value = q * scale, int8_quant.py:52-69) -> unsigned
    q + 128 with zp = 128.  Returns (q_u8, sz)."""
    q = (np.asarray(w_int8, dtype=np.int16) + 128).astype(np.uint8)
    zeros = np.full(np.asarray(scales).shape, 128, dtype=np.uint8)
    return q, interleave_scale_zero(scales, zeros)


# ----------------------------------------------------------------------- a2/a5
def _dequant_blocks(q: np.ndarray, sz: np.ndarray) -> np.ndarray:
    N, K = q.shape
    sz = np.asarray(sz, dtype=np.float16).reshape(N, K // 32, 2)
    s = sz[..., 0].astype(np.float32)[..., None]
    z = sz[..., 1].astype(np.float32)[..., None]
    qb = q.reshape(N, K // 32, 32).astype(np.float32)
    # (q - zp) * scale is exact in fp32; one rounding to fp16 (RNE).
    return ((qb - z) * s).reshape(N, K).astype(np.float16)


def dequant_int4(packed: np.ndarray, sz: np.ndarray) -> np.ndarray:
    """fp16((q - zp) * scale) per 32-block (int4_quant_v2.py:105-127,
    hip:3568-3588)."""
    return _dequant_blocks(unpack_int4(packed), sz)


def dequant_int8(q: np.ndarray, sz: np.ndarray) -> np.ndarray:
    """INT8 asymmetric block-32 (the BASELINE format; symmetric checkpoints
    map through sym_int8_to_asym)."""
    return _dequant_blocks(np.asarray(q, dtype=np.uint8), sz)


def dequant(w: np.ndarray, sz, wbits: int) -> np.ndarray:
    if wbits == 4:
        return dequant_int4(w, sz)
    if wbits == 8:
        return dequant_int8(w, sz)
    if wbits == 16:
        return np.asarray(w, dtype=np.float16)
    raise ValueError(wbits)


# ------------------------------------------------------------------------ a11
def fp8_encode(v) -> np.ndarray:
    """E4M3 code of float32 values by the reference recipe (hip:47-68):
    clamp to +-448 (NaN -> +448), exponent rebias, 3 mantissa bits rounded up
    when fp32 mantissa bit 19 is set, E <= 0 -> signed zero, E >= 15 -> 0x7E."""
    v = np.asarray(v, dtype=np.float32)
    v = np.fmax(np.float32(-448.0), np.fmin(np.float32(448.0), v))
    f = v.view(np.uint32).astype(np.int64)
    sign = (f >> 24) & 0x80
    e = (f >> 23) & 0xFF
    man = f & 0x7FFFFF
    M = (man >> 20) + ((man >> 19) & 1)
    E = e - 120 + (M >> 3)
    M = M & 7
    code = sign | (E << 3) | M
    code = np.where(E >= 15, sign | 0x7E, code)
    code = np.where((e == 0) | (E <= 0), sign, code)
    return code.astype(np.uint8)


def fp8_decode_ref(c) -> np.ndarray:
    """The reference decoder (hip:71-81): sign | (exp+120) << 23 | mant << 20,
    codes with (c & 0x7F) == 0 -> +0.  Exact for every code fp8_encode emits;
    it mis-decodes the E4M3 subnormals 0x01-0x07 (never emitted)."""
    c = np.asarray(c, dtype=np.uint32)
    bits = ((c & 0x80) << 24) | ((((c >> 3) & 0xF) + 120) << 23) | ((c & 0x7) << 20)
    out = bits.astype(np.uint32).view(np.float32)
    return np.where((c & 0x7F) == 0, np.float32(0.0), out).astype(np.float32)


def fp8_value(c) -> np.ndarray:
    """True OCP E4M3 value of a code (subnormals included, 0x7F/0xFF = NaN)."""
    c = np.asarray(c, dtype=np.int64)
    s = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    val = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (e - 7.0))
    val = np.where((c & 0x7F) == 0x7F, np.nan, val)
    return (s * val).astype(np.float64)


# ------------------------------------------------------------------------- a7
def hadamard_matrix(n: int) -> np.ndarray:
    """Unnormalised Sylvester Hadamard matrix (hadamard_utils.py:14-24)."""
    H = np.ones((1, 1))
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return H


def fwht32(x) -> np.ndarray:
    """Block-diagonal FWHT-32 in float32 with the kernels' stage order
    (step 1, 2, 4, 8, 16; {a+b, a-b}) then * fp32(1/sqrt(32)) (hip:87-102)."""
    v = np.asarray(x, dtype=np.float32)
    shp = v.shape
    v = v.reshape(-1, 32).copy()
    step = 1
    while step < 32:
        v = v.reshape(-1, 32 // (2 * step), 2, step)
        a = v[:, :, 0, :].copy()
        b = v[:, :, 1, :].copy()
        v[:, :, 0, :] = a + b
        v[:, :, 1, :] = a - b
        v = v.reshape(-1, 32)
        step *= 2
    return (v * INV_SQRT32).astype(np.float32).reshape(shp)


def fwht32_f64(x) -> np.ndarray:
    """x_rot = x @ H32 / sqrt(32) per 32-chunk in float64
    (hadamard_utils.py:57-88, int4_engine_v5.py:202-205)."""
    H = hadamard_matrix(32) / math.sqrt(32)
    v = np.asarray(x, dtype=np.float64)
    return (v.reshape(-1, 32) @ H).reshape(v.shape)


# ------------------------------------------------------------------------- a8
def _rrms(ss: np.ndarray, D: int, eps: float) -> np.ndarray:
    return np.float32(1.0) / np.sqrt(ss / np.float32(D) + np.float32(eps))


def rmsnorm(x, w, eps: float) -> np.ndarray:
    """fp16(x * rrms * w) per row (fast_rmsnorm int4_engine_v5.py:208-211)."""
    x = np.asarray(x, dtype=np.float16).astype(np.float32)
    D = x.shape[-1]
    ss = (x.astype(np.float64) ** 2).sum(-1, keepdims=True).astype(np.float32)
    r = _rrms(ss, D, eps)
    return (x * r * np.asarray(w, np.float16).astype(np.float32)).astype(np.float16)


def res_rmsnorm(x, res, w, eps: float):
    """r = fp16(x + res); y = fp16(float(r) * rrms * w), rrms from the fp32
    sum (hip:1143-1170 phase 1; int4_engine_v5.py:251-252)."""
    s = np.asarray(x, np.float16).astype(np.float32) + np.asarray(res, np.float16).astype(np.float32)
    r16 = s.astype(np.float16)
    D = s.shape[-1]
    ss = (s.astype(np.float64) ** 2).sum(-1, keepdims=True).astype(np.float32)
    rr = _rrms(ss, D, eps)
    y = (r16.astype(np.float32) * rr * np.asarray(w, np.float16).astype(np.float32))
    return y.astype(np.float16), r16


def rmsnorm_fwht(x, w, eps: float) -> np.ndarray:
    """fp16(FWHT32(x * rrms * w)) (fused_rmsnorm_fwht hip:1195-1237)."""
    x = np.asarray(x, dtype=np.float16).astype(np.float32)
    D = x.shape[-1]
    ss = (x.astype(np.float64) ** 2).sum(-1, keepdims=True).astype(np.float32)
    r = _rrms(ss, D, eps)
    v = x * r * np.asarray(w, np.float16).astype(np.float32)
    return fwht32(v).astype(np.float16)


def res_rmsnorm_fwht(a, b, w, eps: float):
    """res = fp16(a + b); y = fp16(FWHT32(float(res) * rrms * w)) with rrms
    from the fp32 sum (fused_res_norm_fwht hip:1143-1192)."""
    s = np.asarray(a, np.float16).astype(np.float32) + np.asarray(b, np.float16).astype(np.float32)
    r16 = s.astype(np.float16)
    D = s.shape[-1]
    ss = (s.astype(np.float64) ** 2).sum(-1, keepdims=True).astype(np.float32)
    rr = _rrms(ss, D, eps)
    v = r16.astype(np.float32) * rr * np.asarray(w, np.float16).astype(np.float32)
    return fwht32(v).astype(np.float16), r16


# ------------------------------------------------------------------------- a9
def silu_mul(g, u) -> np.ndarray:
    """fp16(silu(g) * u) (silu_mul_batched hip:2112-2122, int4_engine_v5.py:257)."""
    g = np.asarray(g, np.float16).astype(np.float32)
    u = np.asarray(u, np.float16).astype(np.float32)
    return (g / (np.float32(1.0) + np.exp(-g)) * u).astype(np.float16)


def silu_mul_fwht(g, u) -> np.ndarray:
    """fp16(FWHT32(silu(g) * u)) (silu_hadamard_ds hip:1031-1051)."""
    g = np.asarray(g, np.float16).astype(np.float32)
    u = np.asarray(u, np.float16).astype(np.float32)
    return fwht32(g / (np.float32(1.0) + np.exp(-g)) * u).astype(np.float16)


# ---------------------------------------------------------------------- a4-a6
def gemm(x, w, sz, wbits: int, row_chunk: int = 4096) -> np.ndarray:
    """y = fp16(x @ deq(W)^T) with float64 accumulation over fp16 operands
    (gemv_warp hip:116-170; int4_engine_v5.py:227-228)."""
    x = np.asarray(x, dtype=np.float16).astype(np.float64)
    squeeze = x.ndim == 1
    x2 = x.reshape(-1, x.shape[-1])
    N = w.shape[0]
    out = np.empty((x2.shape[0], N), dtype=np.float64)
    for r0 in range(0, N, row_chunk):
        r1 = min(N, r0 + row_chunk)
        W = dequant(w[r0:r1], None if sz is None else sz[r0:r1], wbits).astype(np.float64)
        out[:, r0:r1] = x2 @ W.T
    out = out.astype(np.float16)
    return out[0] if squeeze else out


def gemv(x, w, sz, wbits: int) -> np.ndarray:
    return gemm(x, w, sz, wbits)


# ------------------------------------------------------------------------ a10
def rope_tables(head_dim: int, max_pos: int, theta: float = 1.0e6):
    """cos/sin [max_pos, head_dim/2] fp16 (precompute_rope_freqs
    engine_utils.py:70-76), evaluated in float64 here."""
    inv = 1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim))
    ang = np.outer(np.arange(max_pos, dtype=np.float64), inv)
    return np.cos(ang).astype(np.float16), np.sin(ang).astype(np.float16)


def wave_sum64(t: np.ndarray) -> np.float32:
    """The kernels' canonical float32 reduction of 64 lane values: xor-1,
    xor-2, xor-4, xor-8 butterflies inside each 16-lane row, then
    (row0 + row1) + (row2 + row3)."""
    v = np.asarray(t, dtype=np.float32).reshape(-1, 64).copy()
    idx = np.arange(64)
    for k in (1, 2, 4, 8):
        v = (v + v[:, idx ^ k]).astype(np.float32)
    return ((v[:, 0] + v[:, 16]) + (v[:, 32] + v[:, 48])).astype(np.float32)


def _head_norm_rope(x16: np.ndarray, w16: np.ndarray, c16, s16, eps: float):
    """x16 [nh, 128] -> (lo, hi) float32 halves after RMSNorm + RoPE, in the
    kernel's operation order (hip:1636-1676): lane l owns elements l and
    l+64; sum of squares through wave_sum64; rrms = 1/sqrt(ss/D + eps);
    ne = (x_i*rrms)*w_i, no = (x_{i+64}*rrms)*w_{i+64};
    lo = ne*c - no*s, hi = no*c + ne*s  (no fused multiply-add)."""
    x = x16.astype(np.float32)
    D = x.shape[-1]
    assert D == 128
    t = (x[:, :64] * x[:, :64]).astype(np.float32) + (x[:, 64:] * x[:, 64:]).astype(np.float32)
    ss = wave_sum64(t.astype(np.float32))[:, None]
    rr = (np.float32(1.0) / np.sqrt((ss / np.float32(D)).astype(np.float32) + np.float32(eps))).astype(np.float32)
    w = w16.astype(np.float32)
    ne = ((x[:, :64] * rr).astype(np.float32) * w[:64]).astype(np.float32)
    no = ((x[:, 64:] * rr).astype(np.float32) * w[64:]).astype(np.float32)
    c = c16.astype(np.float32)
    s = s16.astype(np.float32)
    lo = ((ne * c).astype(np.float32) - (no * s).astype(np.float32)).astype(np.float32)
    hi = ((no * c).astype(np.float32) + (ne * s).astype(np.float32)).astype(np.float32)
    return lo, hi


def head_norm_rope_kv(qkv16, qw, kw, cos_t, sin_t, pos: int, H: int, Hk: int, D: int,
                      eps: float, k_scale=None, v_scale=None, return_prequant=False):
    """QK RMSNorm + half-split RoPE + FP8 KV codes for one token
    (head_rmsnorm_rope_kv hip:1620-1683).  K bytes are encoded from the
    float32 rotated value times 1/k_scale, V bytes from fp16 V times
    1/v_scale (scale 1 reproduces the reference).
    Returns (q_out16 [H*D], k_out16 [Hk*D], k_bytes [Hk, D], v_bytes [Hk, D])
    and, with return_prequant, the float32 values that were encoded."""
    qkv16 = np.asarray(qkv16, np.float16)
    q = qkv16[: H * D].reshape(H, D)
    k = qkv16[H * D: (H + Hk) * D].reshape(Hk, D)
    v = qkv16[(H + Hk) * D: (H + 2 * Hk) * D].reshape(Hk, D)
    c = np.asarray(cos_t, np.float16)[pos]
    s = np.asarray(sin_t, np.float16)[pos]
    qlo, qhi = _head_norm_rope(q, np.asarray(qw, np.float16), c, s, eps)
    klo, khi = _head_norm_rope(k, np.asarray(kw, np.float16), c, s, eps)
    q_out = np.concatenate([qlo, qhi], axis=1).astype(np.float16).reshape(-1)
    k32 = np.concatenate([klo, khi], axis=1)
    k_out = k32.astype(np.float16).reshape(-1)
    ks = np.ones(Hk, np.float32) if k_scale is None else np.asarray(k_scale, np.float32)
    vs = np.ones(Hk, np.float32) if v_scale is None else np.asarray(v_scale, np.float32)
    kinv = (np.float32(1.0) / ks).astype(np.float32)[:, None]
    vinv = (np.float32(1.0) / vs).astype(np.float32)[:, None]
    kpre = (k32 * kinv).astype(np.float32)
    vpre = (v.astype(np.float32) * vinv).astype(np.float32)
    kb = fp8_encode(kpre)
    vb = fp8_encode(vpre)
    if return_prequant:
        return q_out, k_out, kb, vb, kpre, vpre
    return q_out, k_out, kb, vb


# ------------------------------------------------------------------------ a12
def attention_decode(q16, k_cache, v_cache, seq_len: int, H: int, Hk: int, D: int,
                     k_scale=None, v_scale=None, fwht: bool = False) -> np.ndarray:
    """Softmax attention of one query token over FP8 cache positions
    [0, seq_len) with GQA (kv head = h // (H/Hk)), float64 math on decoded
    values, score scale 1/sqrt(D) (flash_decode_partial/_reduce
    hip:1326-1463; SDPA int4_engine_v5.py:245 semantics).  Q stays fp16 (the
    reference's FP8 quantisation of Q is not reproduced).  With fwht=True the
    output gets the FWHT-32 rotation the reference's reduce applies.
    k_cache/v_cache: [Hk, max_seq, D] uint8.  Returns fp16 [H*D]."""
    q = np.asarray(q16, np.float16).astype(np.float64).reshape(H, D)
    ks = np.ones(Hk) if k_scale is None else np.asarray(k_scale, np.float64)
    vs = np.ones(Hk) if v_scale is None else np.asarray(v_scale, np.float64)
    g = H // Hk
    out = np.empty((H, D), np.float64)
    for kh in range(Hk):
        K = fp8_decode_ref(k_cache[kh, :seq_len]).astype(np.float64) * ks[kh]
        V = fp8_decode_ref(v_cache[kh, :seq_len]).astype(np.float64) * vs[kh]
        qq = q[kh * g:(kh + 1) * g]
        sc = (qq @ K.T) / math.sqrt(D)
        sc -= sc.max(axis=1, keepdims=True)
        p = np.exp(sc)
        p /= p.sum(axis=1, keepdims=True)
        out[kh * g:(kh + 1) * g] = p @ V
    if fwht:
        out = fwht32_f64(out)
    return out.astype(np.float16).reshape(-1)


def attention_prefill(q16, k16, v16, H: int, Hk: int, fwht: bool = False) -> np.ndarray:
    """Causal GQA self-attention of M prompt rows (SDPA is_causal=True,
    enable_gqa=True as called at hip:2262-2264 / int4_engine_v5.py:245) in
    float64 on fp16 inputs: q16 [M, H, 128], k16/v16 [M, Hk, 128].  With
    fwht=True the output gets the FWHT-32 rotation (hip:2269).
    Returns fp16 [M, H*128]."""
    q = np.asarray(q16, np.float16).astype(np.float64)
    k = np.asarray(k16, np.float16).astype(np.float64)
    v = np.asarray(v16, np.float16).astype(np.float64)
    M, D = q.shape[0], q.shape[-1]
    g = H // Hk
    mask = np.tril(np.ones((M, M), bool))
    out = np.empty((M, H, D), np.float64)
    for h in range(H):
        kh = h // g
        sc = (q[:, h] @ k[:, kh].T) / math.sqrt(D)
        sc = np.where(mask, sc, -np.inf)
        sc -= sc.max(axis=1, keepdims=True)
        p = np.exp(sc)
        p /= p.sum(axis=1, keepdims=True)
        out[:, h] = p @ v[:, kh]
    out = out.reshape(M, H * D)
    if fwht:
        out = fwht32_f64(out)
    return out.astype(np.float16)


# ------------------------------------------------------------------------ a13
class Layer:
    """One decoder layer's tensors (numpy), mirroring int4_hip's arguments."""

    def __init__(self, **kw):
        self.__dict__.update(kw)


def decode_step(layers, hidden16, pos: int, k_caches, v_caches, *, H, Hk, D, hidden, inter,
                eps, rope_cos, rope_sin, final_norm=None, lm_w=None, lm_s=None, lm_bits=4,
                k_scales=None, v_scales=None, trace=None, forced_kv=None, kv_trace=None):
    """One token through all layers (int4_decode_step hip:2343-2528) and,
    with final_norm, the LM head (int4_decode_step_logits hip:2534-2595).
    Mutates k_caches/v_caches ([Hk, max_seq, D] uint8 per layer) at `pos`.
    Returns (hidden_out16, logits16 or None).  `trace` (list) collects the
    per-layer hidden states.  `forced_kv` (per layer (k_bytes, v_bytes)
    [Hk, D]) replaces the oracle's own FP8 codes at `pos` (teacher forcing
    of the quantisation decisions); `kv_trace` then receives per layer
    (own_k, own_v, k_prequant, v_prequant) so callers can check that every
    forced code differs from the oracle's only at a rounding boundary."""
    h = np.asarray(hidden16, np.float16).reshape(-1)
    L = len(layers)
    rot = rmsnorm_fwht(h, layers[0].in_norm, eps)
    q_dim, kv_dim = H * D, Hk * D
    for li, ly in enumerate(layers):
        qkv = gemv(rot, ly.qkv_w, ly.qkv_s, ly.qkv_bits)
        ks = None if k_scales is None else k_scales[li]
        vs = None if v_scales is None else v_scales[li]
        q_out, _, kb, vb, kpre, vpre = head_norm_rope_kv(
            qkv, ly.q_norm, ly.k_norm, rope_cos, rope_sin, pos, H, Hk, D, eps, ks, vs,
            return_prequant=True)
        if kv_trace is not None:
            kv_trace.append((kb, vb, kpre, vpre))
        if forced_kv is not None:
            kb, vb = forced_kv[li]
        k_caches[li][:, pos, :] = kb
        v_caches[li][:, pos, :] = vb
        rot = attention_decode(q_out, k_caches[li], v_caches[li], pos + 1, H, Hk, D, ks, vs,
                               fwht=True)
        o = gemv(rot, ly.o_w, ly.o_s, ly.o_bits)
        rot, r = res_rmsnorm_fwht(o, h, ly.post_norm, eps)
        gu = gemv(rot, ly.gu_w, ly.gu_s, ly.gu_bits)
        y = silu_mul_fwht(gu[:inter], gu[inter:])
        d = gemv(y, ly.down_w, ly.down_s, ly.down_bits)
        nxt = layers[li + 1].in_norm if li + 1 < L else layers[0].in_norm
        rot, h = res_rmsnorm_fwht(d, r, nxt, eps)
        if trace is not None:
            trace.append(h.copy())
    logits = None
    if final_norm is not None:
        rot = rmsnorm_fwht(h, final_norm, eps)
        logits = gemv(rot, lm_w, lm_s, lm_bits)
    return h, logits


def decode_step_batch(layers, hidden16, pos: int, k_caches, v_caches, *, H, Hk, D, hidden,
                      inter, eps, rope_cos, rope_sin, final_norm=None, lm_w=None, lm_s=None,
                      lm_bits=4, k_scales=None, v_scales=None, forced_kv=None, kv_trace=None):
    """decode_step for B independent sequences at one position (the batched
    step of hip:2343-2528 with one row per sequence): hidden16 [B, hidden];
    k_caches/v_caches[li] are [B, Hk, max_seq, D] uint8, mutated at `pos`.
    Each projection dequantises its weights once for all rows; the per-row
    steps (head norm + RoPE + FP8 write, attention) loop over the rows, so
    row b equals decode_step on row b.  forced_kv[li] = (k_bytes, v_bytes)
    [B, Hk, D]; kv_trace receives per layer (own_k, own_v, k_pre, v_pre)
    [B, Hk, D].  Returns (hidden16 [B, hidden], logits16 [B, lm_N] or None)."""
    h = np.asarray(hidden16, np.float16).reshape(-1, hidden)
    B = h.shape[0]
    L = len(layers)
    rot = rmsnorm_fwht(h, layers[0].in_norm, eps)
    for li, ly in enumerate(layers):
        qkv = gemm(rot, ly.qkv_w, ly.qkv_s, ly.qkv_bits)
        ks = None if k_scales is None else k_scales[li]
        vs = None if v_scales is None else v_scales[li]
        att = np.empty((B, H * D), np.float16)
        own = [np.empty((B, Hk, D), np.uint8) for _ in range(2)]
        pre = [np.empty((B, Hk, D), np.float32) for _ in range(2)]
        for b in range(B):
            q_out, _, kb, vb, kpre, vpre = head_norm_rope_kv(
                qkv[b], ly.q_norm, ly.k_norm, rope_cos, rope_sin, pos, H, Hk, D, eps, ks, vs,
                return_prequant=True)
            own[0][b], own[1][b], pre[0][b], pre[1][b] = kb, vb, kpre, vpre
            if forced_kv is not None:
                kb, vb = forced_kv[li][0][b], forced_kv[li][1][b]
            k_caches[li][b, :, pos, :] = kb
            v_caches[li][b, :, pos, :] = vb
            att[b] = attention_decode(q_out, k_caches[li][b], v_caches[li][b], pos + 1, H, Hk, D,
                                      ks, vs, fwht=True)
        if kv_trace is not None:
            kv_trace.append((own[0], own[1], pre[0], pre[1]))
        o = gemm(att, ly.o_w, ly.o_s, ly.o_bits)
        rot, r = res_rmsnorm_fwht(o, h, ly.post_norm, eps)
        gu = gemm(rot, ly.gu_w, ly.gu_s, ly.gu_bits)
        y = silu_mul_fwht(gu[:, :inter], gu[:, inter:])
        d = gemm(y, ly.down_w, ly.down_s, ly.down_bits)
        nxt = layers[li + 1].in_norm if li + 1 < L else layers[0].in_norm
        rot, h = res_rmsnorm_fwht(d, r, nxt, eps)
    logits = None
    if final_norm is not None:
        rot = rmsnorm_fwht(h, final_norm, eps)
        logits = gemm(rot, lm_w, lm_s, lm_bits)
    return h, logits


# ------------------------------------------------------------------------ a15
def prefill_logits(layers, ids, embed, *, H, Hk, D, hidden, inter, eps, rope_cos, rope_sin,
                   final_norm=None, lm_w=None, lm_s=None, lm_bits=4, k_caches=None,
                   v_caches=None, k_scales=None, v_scales=None, kv_trace=None, trace=None,
                   attend_fp8=False):
    """Prompt pass over token ids [M] (int4_prefill_logits hip:2127-2320):
    embedding, then per layer RMSNorm + FWHT, QKV, per-row head RMSNorm +
    RoPE at position m, causal attention + FWHT, O, residual + norm + FWHT,
    gate/up, SiLU-gate + FWHT, down, residual; final norm + FWHT and the LM
    head for every row.  The norms apply the FWHT before the fp16 rounding
    (the decode kernels' order).  With k_caches/v_caches ([Hk, max_seq, D]
    uint8 per layer) the FP8 codes of positions 0..M-1 are written (K from
    the float32 rotated values, as int4_engine_v5.py:237-242 fills the cache
    for decode); kv_trace receives per layer (k_bytes, v_bytes, k_pre, v_pre)
    [M, Hk, D] and `trace` the residual stream [M, hidden] after each layer.
    attend_fp8=True makes the attention read K and V through their FP8 codes
    (decoded, scaled and held as fp16, exact at scale 1) as the decode step
    does, instead of the fp16 values (the reference prompt pass,
    int4_engine_v5.py:245).  Returns (hidden16 [M, hidden], logits16
    [M, lm_N] or None)."""
    ids = np.asarray(ids, np.int64).reshape(-1)
    M = ids.size
    x = np.asarray(embed, np.float16)[ids]
    L = len(layers)
    q_dim, kv_dim = H * D, Hk * D
    rot = rmsnorm_fwht(x, layers[0].in_norm, eps)
    for li, ly in enumerate(layers):
        qkv = gemm(rot, ly.qkv_w, ly.qkv_s, ly.qkv_bits)
        ks = None if k_scales is None else k_scales[li]
        vs = None if v_scales is None else v_scales[li]
        q = np.empty((M, H, D), np.float16)
        k = np.empty((M, Hk, D), np.float16)
        kb_all = np.empty((M, Hk, D), np.uint8)
        vb_all = np.empty((M, Hk, D), np.uint8)
        kp_all = np.empty((M, Hk, D), np.float32)
        vp_all = np.empty((M, Hk, D), np.float32)
        for m in range(M):
            q_out, k_out, kb, vb, kpre, vpre = head_norm_rope_kv(
                qkv[m], ly.q_norm, ly.k_norm, rope_cos, rope_sin, m, H, Hk, D, eps, ks, vs,
                return_prequant=True)
            q[m] = q_out.reshape(H, D)
            k[m] = k_out.reshape(Hk, D)
            kb_all[m], vb_all[m], kp_all[m], vp_all[m] = kb, vb, kpre, vpre
        v = qkv[:, q_dim + kv_dim:].reshape(M, Hk, D)
        if kv_trace is not None:
            kv_trace.append((kb_all, vb_all, kp_all, vp_all))
        if k_caches is not None:
            k_caches[li][:, :M, :] = kb_all.transpose(1, 0, 2)
            v_caches[li][:, :M, :] = vb_all.transpose(1, 0, 2)
        if attend_fp8:
            ksc = np.ones(Hk) if ks is None else np.asarray(ks, np.float64)
            vsc = np.ones(Hk) if vs is None else np.asarray(vs, np.float64)
            k = (fp8_decode_ref(kb_all) * ksc[None, :, None]).astype(np.float16)
            v = (fp8_decode_ref(vb_all) * vsc[None, :, None]).astype(np.float16)
        rot = attention_prefill(q, k, v, H, Hk, fwht=True)
        o = gemm(rot, ly.o_w, ly.o_s, ly.o_bits)
        rot, r = res_rmsnorm_fwht(o, x, ly.post_norm, eps)
        gu = gemm(rot, ly.gu_w, ly.gu_s, ly.gu_bits)
        y = silu_mul_fwht(gu[:, :inter], gu[:, inter:])
        d = gemm(y, ly.down_w, ly.down_s, ly.down_bits)
        if li + 1 < L:
            nxt = layers[li + 1].in_norm
        else:
            nxt = final_norm if final_norm is not None else layers[0].in_norm
        rot, x = res_rmsnorm_fwht(d, r, nxt, eps)
        if trace is not None:
            trace.append(x.copy())
    logits = None
    if final_norm is not None:
        logits = gemm(rot, lm_w, lm_s, lm_bits)
    return x, logits


# ------------------------------------------------------- f3 sampling
_M64 = (1 << 64) - 1


def splitmix64(x: int) -> int:
    """splitmix64 output function (S. Vigna): one step from state x."""
    x = (x + 0x9E3779B97F4A7C15) & _M64
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & _M64
    return x ^ (x >> 31)


def sample_uniform(seed: int, counter: int, row: int) -> np.float32:
    """The draw's uniform u in [0, 1): splitmix64(splitmix64(seed ^ counter)
    ^ row), top 24 bits / 2^24 (the library's counter-based stream)."""
    x = splitmix64(splitmix64((seed ^ (counter & _M64)) & _M64) ^ row)
    return np.float32((x >> 40) / 16777216.0)


def sample_top_p(logits16, temperature: float, top_p: float, u: float,
                 return_info: bool = False):
    """Next token of one row (int4_engine_v5.py:387-399): z = float(logits) /
    temperature; with top_p < 1 the tokens are sorted by z descending (ties
    by ascending index, a stable sort) and a token is dropped when the
    softmax mass before it is >= top_p; one token is drawn from the kept
    tokens' softmax by inverse CDF at u in that same order.  temperature <= 0
    is argmax (the lowest index of the maximum, int4_engine_v5.py:352-353).

    return_info adds the cutoff margin (distance of the nearest cumulative
    mass to top_p) and the draw margin (distance of u * kept mass to the
    nearest CDF step), in probability units, so tests can skip cases whose
    outcome hinges on float rounding."""
    l = np.asarray(logits16, dtype=np.float16).astype(np.float32).ravel()
    V = l.size
    if temperature <= 0:
        tok = int(np.argmax(l))
        info = {"cut_margin": np.inf, "draw_margin": np.inf, "token": tok}
        return (tok, info) if return_info else tok
    z = (l / np.float32(temperature)).astype(np.float32)
    order = np.lexsort((np.arange(V), -z.astype(np.float64)))
    zs = z[order].astype(np.float64)
    p = np.exp(zs - zs[0])
    p /= p.sum()
    before = np.cumsum(p) - p
    if top_p < 1.0:
        keep = before < top_p
        cut_margin = float(np.min(np.abs(before - top_p)))
    else:
        keep = np.ones(V, bool)
        cut_margin = np.inf
    pk = p[keep]
    cdf = np.cumsum(pk)
    target = float(u) * cdf[-1]
    j = int(np.searchsorted(cdf, target, side="right"))
    j = min(j, pk.size - 1)
    tok = int(order[np.flatnonzero(keep)[j]])
    if not return_info:
        return tok
    steps = np.concatenate([[0.0], cdf])
    draw_margin = float(np.min(np.abs(steps - target)))
    return tok, {"cut_margin": cut_margin, "draw_margin": draw_margin,
                 "kept": int(keep.sum()), "order": order, "before": before, "keep": keep,
                 "cdf": cdf / cdf[-1], "u": float(u), "top_p": top_p}


def sample_distance(token: int, info) -> float:
    """How far (probability units) a token chosen by another implementation
    lies from the oracle's outcome: 0 for the oracle's own token; for another
    kept token, the distance of u to that token's CDF interval; for a
    dropped token, the distance of its cumulative mass before it to top_p (a
    cutoff decided by rounding)."""
    if "order" not in info:  # greedy: no rounding-dependent outcome
        return 0.0 if token == info["token"] else np.inf
    pos = int(np.flatnonzero(info["order"] == token)[0])
    if not info["keep"][pos]:
        return float(abs(info["before"][pos] - info["top_p"]))
    j = int(np.flatnonzero(np.flatnonzero(info["keep"]) == pos)[0])
    lo = 0.0 if j == 0 else float(info["cdf"][j - 1])
    hi = float(info["cdf"][j])
    u = info["u"]
    return max(0.0, lo - u, u - hi)

