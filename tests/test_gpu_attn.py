"""GPU parity of the split-K flash-decode against the oracle (float64 softmax
attention on the decoded FP8 cache).  Tolerance rel-L2 <= 5e-3."""
import ctypes as C

import numpy as np
import pytest
import torch

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


@pytest.mark.parametrize("L", [257, 8192])
def test_flash_decode_forced_split_counts(dev, ctx, monkeypatch, L):
    """Split counts from 1 to 128 back to back on one context: more than one
    64-split merge round, and splits that hold no positions when there are
    fewer 32-position chunks than splits."""
    for n in (3, 100, 1, 17, 128, 64, 2):
        monkeypatch.setenv("R4Q_ATTN_SPLITS", str(n))
        _case(dev, ctx, 2, 40, 8, L, L + 1, scaled=True, fwht=True, seed=n + L)


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
