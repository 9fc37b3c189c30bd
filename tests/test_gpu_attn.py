"""GPU parity of the split-K flash-decode against the oracle (float64 softmax
attention on the decoded FP8 cache).  Tolerance rel-L2 <= 5e-3."""
import ctypes as C

import numpy as np
import pytest
import torch

import int4_hip
import r4q_lib as R
import r4q_oracle as O
import r4q_synth as S
from conftest import fp8_golden_table, rel_l2

pytestmark = pytest.mark.gpu
TOL = 5e-3


@pytest.fixture(scope="module")
def ctx():
    h = C.c_void_p()
    R.call("r4q_ctx_create", C.byref(h))
    yield h
    R.call("r4q_ctx_destroy", h)


def _case(dev, ctx, B, H, Hk, L, max_seq, scaled, fwht, seed):
    D = 128
    g = S.gen(seed)
    q = torch.randn(B, H * D, generator=g).half()
    kvals = S.random_kv_values(Hk, L, D, g, batch=B, scale=1.5)
    vvals = S.random_kv_values(Hk, L, D, g, batch=B, scale=1.5)
    kc = np.zeros((B, Hk, max_seq, D), np.uint8)
    vc = np.zeros((B, Hk, max_seq, D), np.uint8)
    kc[:, :, :L] = O.fp8_encode(kvals.float().numpy())
    vc[:, :, :L] = O.fp8_encode(vvals.float().numpy())
    ks = (0.5 + torch.rand(Hk, generator=g)).float() if scaled else None
    vs = (0.5 + torch.rand(Hk, generator=g)).float() if scaled else None
    out = torch.empty(B, H * D, dtype=torch.float16, device=dev)
    Kc, Vc = torch.from_numpy(kc).to(dev), torch.from_numpy(vc).to(dev)
    Ks, Vs = (ks.to(dev), vs.to(dev)) if scaled else (None, None)
    Q = q.to(dev)
    R.call("r4q_flash_decode", ctx, Q.data_ptr(), H * D, Kc.data_ptr(), Vc.data_ptr(), R.ptr(Ks),
           R.ptr(Vs), out.data_ptr(), B, H, Hk, D, max_seq, L, 1 if fwht else 0, R.stream_handle())
    got = out.cpu().numpy()
    for b in range(B):
        want = O.attention_decode(q[b].numpy(), kc[b], vc[b], L, H, Hk, D,
                                  None if ks is None else ks.numpy(),
                                  None if vs is None else vs.numpy(), fwht=fwht)
        assert rel_l2(got[b], want) <= TOL, (b, rel_l2(got[b], want))
    return got


@pytest.mark.parametrize("L", [1, 2, 31, 33, 128, 255, 257, 2048, 8192, 32768])
def test_flash_decode_qwen3_gqa(dev, ctx, L):
    _case(dev, ctx, 1, 40, 8, L, L + 7, scaled=True, fwht=True, seed=L)


@pytest.mark.parametrize("G", [1, 2, 4, 8])
def test_flash_decode_other_group_sizes(dev, ctx, G):
    _case(dev, ctx, 2, 4 * G, 4, 300, 512, scaled=False, fwht=False, seed=G)


def test_flash_decode_batch8_no_rotation(dev, ctx):
    _case(dev, ctx, 8, 40, 8, 700, 1024, scaled=False, fwht=False, seed=8)


@pytest.mark.parametrize("B", [2, 4, 16])
def test_flash_decode_batches_at_the_workgroup_cap(dev, ctx, B):
    """ctx 2048 at the default split count, which keeps B x 8 KV heads x
    splits within one workgroup per CU: 16, 8 and 2 splits for batches 2, 4
    and 16 (XCD-grouped grids, merge rounds of 16 and 8)."""
    _case(dev, ctx, B, 40, 8, 2048, 2048 + 40, scaled=True, fwht=True, seed=100 + B)


@pytest.mark.parametrize("L", [257, 8192])
def test_flash_decode_forced_split_counts(dev, ctx, L):
    """Split counts from 1 to 128 back to back on one context: more than one
    64-split merge round, and splits that hold no positions when there are
    fewer 32-position chunks than splits."""
    try:
        for n in (3, 100, 1, 17, 128, 64, 2):
            R.tune("attn_splits", n)
            _case(dev, ctx, 2, 40, 8, L, L + 1, scaled=True, fwht=True, seed=n + L)
    finally:
        R.tune("attn_splits", 0)


def test_flash_decode_single_position_is_v(dev, ctx):
    """seq_len 1: softmax weight 1, output equals the (scaled) V row."""
    got = _case(dev, ctx, 1, 40, 8, 1, 4, scaled=True, fwht=False, seed=5)
    assert np.all(np.isfinite(got))


def test_flash_decode_widens_every_encoder_code_exactly(dev, ctx):
    """With one position the softmax weight is exactly 1, so the unrotated
    output is fp16(decoded V) bit for bit.  Every E4M3 code except the
    subnormals (0x01-0x07, 0x81-0x87) and 0x7F / 0xFF must widen to the
    reference decoder's value (hip:71-81); the golden encoder table shows
    the reference encoder never emits those excluded codes."""
    excluded = {c for c in range(256) if (c & 0x7F) == 0x7F or ((c >> 3) & 0xF == 0 and c & 7)}
    assert not excluded & set(np.unique(fp8_golden_table()).tolist())
    codes = np.array([c for c in range(256) if c not in excluded], np.uint8)
    want = O.fp8_decode_ref(codes).astype(np.float16)
    q = torch.ones(128, dtype=torch.float16, device=dev)
    out = torch.empty(128, dtype=torch.float16, device=dev)
    kc = torch.zeros(1, 1, 1, 128, dtype=torch.uint8, device=dev)
    for c0 in range(0, codes.size, 128):
        part = codes[c0:c0 + 128]
        row = np.zeros(128, np.uint8)
        row[:part.size] = part
        vc = torch.from_numpy(row.reshape(1, 1, 1, 128)).to(dev)
        R.call("r4q_flash_decode", ctx, q.data_ptr(), 128, kc.data_ptr(), vc.data_ptr(), None,
               None, out.data_ptr(), 1, 1, 1, 128, 1, 1, 0, R.stream_handle())
        got = out.cpu().numpy()[:part.size]
        w = want[c0:c0 + part.size]
        # -0 sums to +0 in the fp32 accumulation: values everywhere, bits off zero
        assert np.array_equal(got, w), c0
        assert np.array_equal(got[w != 0].view(np.uint16), w[w != 0].view(np.uint16)), c0


def test_flash_decode_rejects_bad_arguments(dev, ctx):
    z = torch.zeros(64, dtype=torch.float16, device=dev)
    rc = R.lib().r4q_flash_decode(ctx, z.data_ptr(), 5120, z.data_ptr(), z.data_ptr(), None, None,
                                  z.data_ptr(), 1, 40, 8, 128, 16, 17, 1, None)
    assert rc == R.R4Q_EINVAL
    rc = R.lib().r4q_flash_decode(ctx, z.data_ptr(), 5120, z.data_ptr(), z.data_ptr(), None, None,
                                  z.data_ptr(), 1, 42, 8, 128, 16, 4, 1, None)
    assert rc == R.R4Q_EINVAL


@pytest.mark.parametrize("B", [1, 8])
@pytest.mark.parametrize("pos", [0, 2047, 32767])
@pytest.mark.parametrize("scaled", [False, True])
def test_fused_prologue_kv_bytes_and_output_bit_exact(dev, ctx, B, pos, scaled):
    """The decode step's attention prologue (r4q_flash_decode_qkv: head norm +
    RoPE of raw QKV rows, FP8 K/V write at pos, attention over 0..pos) against
    the two-kernel route (r4q_head_norm_rope_kv, then r4q_flash_decode on its
    q rows and caches) and the oracle:
      * the K/V codes written at pos are bit-identical to the standalone
        kernel's and to the oracle's (K encoded from the fp32 rotated value,
        hip:1667-1675), and no other cache byte changes;
      * with the same split count the attention outputs are bit-identical;
      * with the decode step's own split count (from the cache capacity) the
        output matches the float64 oracle (rel-L2 <= 5e-3)."""
    H, Hk, D = 40, 8, 128
    qkvN = (H + 2 * Hk) * D
    max_seq = pos + 34
    print(f"[prologue] B={B} pos={pos} scaled={scaled}", flush=True)
    g = S.gen(1000 + pos + B + 7 * scaled)
    qkv = (torch.randn(B, qkvN, generator=g) * 2).half()
    qw, kw = S.norm_weight(D, g), S.norm_weight(D, g)
    cos, sin = S.rope_tables(D, max_seq)
    ks = (0.25 + torch.rand(Hk, generator=g)).float() if scaled else None
    vs = (0.25 + torch.rand(Hk, generator=g)).float() if scaled else None
    QKV, QW, KW, COS, SIN = (t.to(dev) for t in (qkv, qw, kw, cos, sin))
    Ks, Vs = (ks.to(dev), vs.to(dev)) if scaled else (None, None)
    # caches: FP8 codes of N(0,1) values (the reference encoder, on the GPU) below pos
    gd = torch.Generator(device=dev)
    gd.manual_seed(pos + B)
    kc0 = torch.zeros(B, Hk, max_seq, D, dtype=torch.uint8, device=dev)
    vc0 = torch.zeros_like(kc0)
    if pos:
        for c in (kc0, vc0):
            vals = torch.randn(B, Hk, pos, D, device=dev, generator=gd).half()
            c[:, :, :pos] = int4_hip.fp16_to_fp8(vals)
            del vals
    kc1, vc1, kc2, vc2 = kc0.clone(), vc0.clone(), kc0.clone(), vc0.clone()
    out1 = torch.empty(B, H * D, dtype=torch.float16, device=dev)
    out2 = torch.empty_like(out1)
    qo = torch.empty(B, (H + Hk) * D, dtype=torch.float16, device=dev)
    nsp = min(32, max(1, (max_seq + 127) // 128))
    try:
        R.tune("attn_splits", nsp)
        R.call("r4q_flash_decode_qkv", ctx, QKV.data_ptr(), qkvN, QW.data_ptr(), KW.data_ptr(),
               COS.data_ptr(), SIN.data_ptr(), C.c_float(1e-6), kc1.data_ptr(), vc1.data_ptr(),
               R.ptr(Ks), R.ptr(Vs), out1.data_ptr(), B, H, Hk, D, max_seq, max_seq, pos, 1,
               R.stream_handle())
        R.call("r4q_head_norm_rope_kv", QKV.data_ptr(), qkvN, QW.data_ptr(), KW.data_ptr(),
               qo.data_ptr(), (H + Hk) * D, kc2.data_ptr(), vc2.data_ptr(), R.ptr(Ks), R.ptr(Vs),
               COS.data_ptr(), SIN.data_ptr(), B, H, Hk, D, C.c_float(1e-6), max_seq, pos,
               R.stream_handle())
        R.call("r4q_flash_decode", ctx, qo.data_ptr(), (H + Hk) * D, kc2.data_ptr(),
               vc2.data_ptr(), R.ptr(Ks), R.ptr(Vs), out2.data_ptr(), B, H, Hk, D, max_seq,
               pos + 1, 1, R.stream_handle())
    finally:
        R.tune("attn_splits", 0)
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    assert torch.equal(out1, out2)
    # only position pos changed
    for c1, c0 in ((kc1, kc0), (vc1, vc0)):
        assert torch.equal(c1[:, :, :pos], c0[:, :, :pos])
        assert torch.equal(c1[:, :, pos + 1:], c0[:, :, pos + 1:])
    # the decode step's own split count, then the oracle
    out3 = torch.empty_like(out1)
    R.call("r4q_flash_decode_qkv", ctx, QKV.data_ptr(), qkvN, QW.data_ptr(), KW.data_ptr(),
           COS.data_ptr(), SIN.data_ptr(), C.c_float(1e-6), kc1.data_ptr(), vc1.data_ptr(),
           R.ptr(Ks), R.ptr(Vs), out3.data_ptr(), B, H, Hk, D, max_seq, max_seq, pos, 1,
           R.stream_handle())
    torch.cuda.synchronize()
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    for b in sorted({0, B - 1}):
        q_out, _, kb, vb = O.head_norm_rope_kv(
            qkv[b].numpy(), qw.numpy(), kw.numpy(), cos.numpy(), sin.numpy(), pos, H, Hk, D,
            1e-6, None if ks is None else ks.numpy(), None if vs is None else vs.numpy())
        assert np.array_equal(kc1[b, :, pos].cpu().numpy(), kb), b
        assert np.array_equal(vc1[b, :, pos].cpu().numpy(), vb), b
        kcb, vcb = kc1[b].cpu().numpy(), vc1[b].cpu().numpy()
        want = O.attention_decode(q_out, kcb, vcb, pos + 1, H, Hk, D,
                                  None if ks is None else ks.numpy(),
                                  None if vs is None else vs.numpy(), fwht=True)
        assert rel_l2(out3[b].cpu().numpy(), want) <= TOL, (b, rel_l2(out3[b].cpu().numpy(), want))
    # the other rows' codes too (cheap: no attention)
    for b in range(B):
        _, _, kb, vb = O.head_norm_rope_kv(
            qkv[b].numpy(), qw.numpy(), kw.numpy(), cos.numpy(), sin.numpy(), pos, H, Hk, D,
            1e-6, None if ks is None else ks.numpy(), None if vs is None else vs.numpy())
        assert np.array_equal(kc1[b, :, pos].cpu().numpy(), kb), b
        assert np.array_equal(vc1[b, :, pos].cpu().numpy(), vb), b


def test_fused_prologue_rejects_bad_arguments(dev, ctx):
    z = torch.zeros(7168, dtype=torch.float16, device=dev)
    c8 = torch.zeros(8 * 16 * 128, dtype=torch.uint8, device=dev)
    args = [ctx, z.data_ptr(), 7168, z.data_ptr(), z.data_ptr(), z.data_ptr(), z.data_ptr(),
            C.c_float(1e-6), c8.data_ptr(), c8.data_ptr(), None, None, z.data_ptr(), 1, 40, 8,
            128, 16, 16, 16, 1, None]
    assert R.lib().r4q_flash_decode_qkv(*args) == R.R4Q_EINVAL  # pos == max_seq
    args[-3] = 15  # pos inside the cache ...
    args[-4] = 8   # ... but past the RoPE table
    assert R.lib().r4q_flash_decode_qkv(*args) == R.R4Q_EINVAL
