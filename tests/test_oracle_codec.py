"""Pins the oracle's integer/byte codecs (CPU only).

Nibble packing, dequantisation and the FP8 E4M3 recipe are checked against
closed forms evaluated by a different route, exhaustive enumeration, the
reference's own known-answer tests (tests/test_kernels.py:26-70) and torch's
float8_e4m3fn conversion with every difference classified."""
import numpy as np
import pytest
import torch

import r4q_oracle as O
from conftest import fp8_golden_table

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")


def test_unpack_exhaustive_bytes():
    b = np.arange(256, dtype=np.uint8)[None, :]
    u = O.unpack_int4(b)
    assert u.shape == (1, 512)
    assert np.array_equal(u[0, 0::2], b[0] & 0xF)
    assert np.array_equal(u[0, 1::2], b[0] >> 4)
    assert np.array_equal(O.pack_int4(u), b)


def _restated_rtn_asym(W):
    """Minimal restatement of quantize_to_int4_asymmetric (int4_quant_v2.py:17-46)
    used only to reproduce the reference's known-answer tests."""
    vmin = W.min(-1, keepdims=True)
    vmax = W.max(-1, keepdims=True)
    scale = (vmax - vmin) / 15.0
    scale = np.where(scale > 0, scale, 1.0)
    zp = np.clip(np.round(-vmin / scale), 0, 15)
    q = np.clip(np.round(W / scale + zp), 0, 15).astype(np.uint8)
    recon = (q.astype(np.float32) - zp) * scale
    return q, scale[..., 0].astype(np.float16), zp[..., 0].astype(np.uint8), recon


def test_reference_roundtrip_known_answer():
    """tests/test_kernels.py:26-50: q in [0,15], pack/unpack identity,
    relative MSE < 0.05."""
    rng = np.random.default_rng(42)
    N, K = 128, 256
    W = rng.standard_normal((N, K)).astype(np.float32)
    q, _, _, recon = _restated_rtn_asym(W.reshape(N, K // 32, 32))
    q = q.reshape(N, K)
    assert q.min() >= 0 and q.max() <= 15
    assert np.array_equal(O.unpack_int4(O.pack_int4(q)), q)
    rel = ((W - recon.reshape(N, K)) ** 2).mean() / (W ** 2).mean()
    assert rel < 0.05


def test_reference_dequant_known_answer():
    """tests/test_kernels.py:53-70: dequant(packed) matches the fp32
    reconstruction within 0.01."""
    rng = np.random.default_rng(123)
    N, K = 64, 128
    W = rng.standard_normal((N, K)).astype(np.float32)
    q, s, z, recon = _restated_rtn_asym(W.reshape(N, K // 32, 32))
    sz = O.interleave_scale_zero(s, z)
    deq = O.dequant_int4(O.pack_int4(q.reshape(N, K)), sz)
    assert np.abs(deq.astype(np.float32) - recon.reshape(N, K)).max() < 0.01


def _all_finite_fp16():
    x = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    return x[np.isfinite(x)]


def test_dequant_int4_exhaustive_closed_form():
    """Every (q, zp) pair against every finite fp16 scale: the oracle's fp32
    route equals fp16(float64(q - zp) * float64(scale)) bit-for-bit."""
    scales = _all_finite_fp16()
    N = scales.size
    K = 16 * 32  # block b uses zp = b; each block holds q = 0..15 twice
    q = np.tile(np.concatenate([np.arange(16), np.arange(16)]).astype(np.uint8), 16)
    qm = np.broadcast_to(q, (N, K))
    zeros = np.broadcast_to(np.arange(16, dtype=np.uint8), (N, 16))
    sz = O.interleave_scale_zero(np.broadcast_to(scales[:, None], (N, 16)), zeros)
    got = O.dequant_int4(O.pack_int4(qm), sz)
    d = (q.astype(np.float64) - np.repeat(np.arange(16), 32))[None, :]
    want = (d * scales.astype(np.float64)[:, None]).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_dequant_int8_exhaustive_closed_form():
    scales = _all_finite_fp16()[::3]
    N = scales.size
    zps = np.array([0, 127, 128, 255], dtype=np.uint8)
    q = np.tile(np.arange(256, dtype=np.uint8), 4)  # 8 blocks per zero-point
    K = q.size
    zeros = np.repeat(zps, 8)[None, :].repeat(N, 0)
    sz = O.interleave_scale_zero(np.broadcast_to(scales[:, None], (N, K // 32)), zeros)
    got = O.dequant_int8(np.broadcast_to(q, (N, K)), sz)
    d = q.astype(np.float64) - np.repeat(zps, 256).astype(np.float64)
    want = (d[None, :] * scales.astype(np.float64)[:, None]).astype(np.float16)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_sym_to_asym_conversions():
    """int4_engine_v5.py:105-118 (nibble n -> (n+8)&0xF, zp 8) and the int8
    sym -> asym mapping preserve dequantised values."""
    rng = np.random.default_rng(1)
    N, K = 8, 64
    qs = rng.integers(-8, 8, (N, K))
    packed_sym = O.pack_int4((qs & 0xF).astype(np.uint8))
    scales = (rng.random((N, K // 32)) * 0.1 + 0.01).astype(np.float16)
    p, sz = O.sym_int4_to_asym(packed_sym, scales)
    want = (qs.reshape(N, -1, 32) * scales.astype(np.float32)[..., None]).reshape(N, K)
    assert np.array_equal(O.dequant_int4(p, sz), want.astype(np.float16))
    q8 = rng.integers(-128, 128, (N, K)).astype(np.int8)
    qu, sz8 = O.sym_int8_to_asym(q8, scales)
    want8 = (q8.astype(np.float32).reshape(N, -1, 32) * scales.astype(np.float32)[..., None])
    assert np.array_equal(O.dequant_int8(qu, sz8), want8.reshape(N, K).astype(np.float16))


# ------------------------------------------------------------------- FP8
def test_fp8_encode_all_fp16_vs_torch_classified():
    """All 63488 finite fp16 inputs: equal to torch.float8_e4m3fn except in
    the recipe's documented departures, each checked by its closed form."""
    x = _all_finite_fp16().astype(np.float32)
    ours = O.fp8_encode(x)
    tor = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    ax = np.abs(x)
    sign = np.where(np.signbit(x), 0x80, 0).astype(np.uint8)
    diff = ours != tor
    assert diff.sum() == 24428

    flush = diff & (ax < 2.0 ** -6)
    assert flush.sum() == 8062
    # below 2^-6 the recipe gives +-0, or +-2^-6 when rounding carries into
    # the smallest normal exponent
    assert np.all((ours[flush] == sign[flush]) | (ours[flush] == (sign[flush] | 0x08)))

    sat = diff & (ax >= 248)
    assert np.all(ours[sat] == (sign[sat] | 0x7E))  # 248 and above -> 448
    assert (diff & (ax > 448)).sum() == 14718
    assert (diff & (ax >= 256) & (ax <= 448)).sum() == 1408
    assert (diff & (ax >= 240) & (ax < 256)).sum() == 128

    ties = diff & ~flush & ~sat
    assert ties.sum() == 112
    tv = O.fp8_value(tor[ties])
    ov = O.fp8_value(ours[ties])
    # exact ties, resolved away from zero instead of to even
    assert np.allclose(np.abs(x[ties] - tv), np.abs(ov - x[ties]), rtol=0, atol=0)
    assert np.all(np.abs(ov) > np.abs(tv))


def test_fp8_encode_all_fp16_vs_golden_table():
    """Golden fixture: value-domain derivation (exact rationals, ties away from
    zero, flush/saturate rules) of the reference encoder for all 65,536 fp16
    inputs; the oracle's bit recipe must agree on every code."""
    table = fp8_golden_table()
    assert table.size == 65536
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.fp8_encode(bits.view(np.float16).astype(np.float32))
    assert np.array_equal(got, table)


def test_fp8_encode_special_values():
    v = np.array([np.nan, -np.nan, np.inf, -np.inf, 0.0, -0.0, 448.0, -448.0, 449.0, 1e30,
                  2.0 ** -6, -(2.0 ** -6), 2.0 ** -7, 2.0 ** -10], dtype=np.float32)
    got = O.fp8_encode(v)
    assert list(got) == [0x7E, 0x7E, 0x7E, 0xFE, 0x00, 0x80, 0x7E, 0xFE, 0x7E, 0x7E,
                         0x08, 0x88, 0x00, 0x00]


def test_fp8_encode_fp32_inputs_closed_form():
    """Random fp32 inputs in the normal E4M3 range: arithmetic rounding of
    |x| / 2^(e-3) half away from zero gives the same value as the bit recipe."""
    rng = np.random.default_rng(7)
    mag = np.exp2(rng.uniform(-6, np.log2(240), 200000)).astype(np.float32)
    x = (mag * rng.choice([-1, 1], mag.size)).astype(np.float32)
    # include exact ties at bit 19
    ties = (np.exp2(rng.integers(-6, 7, 2000).astype(np.float64)) *
            (1 + (2 * rng.integers(0, 8, 2000) + 1) / 16.0)).astype(np.float32)
    x = np.concatenate([x, ties, -ties])
    a = np.abs(x).astype(np.float64)
    e = np.floor(np.log2(a))
    m = a / np.exp2(e - 3)
    r = np.floor(m + 0.5)
    val = np.sign(x) * r * np.exp2(e - 3)
    val = np.where(np.abs(val) >= 248, np.sign(x) * 448.0, val)
    want = torch.from_numpy(val.astype(np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(O.fp8_encode(x), want)


def test_fp8_decoders_all_codes():
    c = np.arange(256, dtype=np.uint8)
    tv = torch.from_numpy(c).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    ref = O.fp8_decode_ref(c).astype(np.float64)
    sub = ((c & 0x78) == 0) & ((c & 7) != 0)
    nan = (c & 0x7F) == 0x7F
    assert np.array_equal(ref[~sub & ~nan], tv[~sub & ~nan])
    assert not np.array_equal(ref[sub], tv[sub])  # reference mis-decodes subnormals
    fv = O.fp8_value(c)
    assert np.array_equal(fv[~nan], tv[~nan]) and np.all(np.isnan(fv[nan]))


def test_fp8_roundtrip_emitted_codes():
    """Encoding the decoded value of any emitted code returns the code."""
    emitted = np.unique(O.fp8_encode(_all_finite_fp16().astype(np.float32)))
    assert not np.any(((emitted & 0x78) == 0) & ((emitted & 7) != 0))  # no subnormals
    assert not np.any((emitted & 0x7F) == 0x7F)                        # no NaN
    back = O.fp8_encode(O.fp8_decode_ref(emitted))
    # the reference decoder returns +0 for 0x80, everything else round-trips
    assert np.array_equal(back, np.where(emitted == 0x80, 0, emitted))
