"""GPU parity of the byte/integer kernels: bit-exact against the oracle."""
import numpy as np
import pytest
import torch

import int4_hip
import r4q_oracle as O
import r4q_synth as S
from conftest import fp8_golden_table

pytestmark = pytest.mark.gpu


def test_fp16_to_fp8_all_bit_patterns(dev):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = torch.from_numpy(bits.view(np.int16)).view(torch.float16).to(dev)
    got = int4_hip.fp16_to_fp8(x).cpu().numpy()
    want = O.fp8_encode(bits.view(np.float16).astype(np.float32))
    assert np.array_equal(got, want)
    assert np.array_equal(got, fp8_golden_table())


@pytest.mark.parametrize("n", [1, 3, 4, 5, 1000003])
def test_fp16_to_fp8_ragged_sizes(dev, n):
    g = S.gen(n)
    x = (torch.randn(n, generator=g) * 50).half()
    got = int4_hip.fp16_to_fp8(x.to(dev)).cpu().numpy()
    assert np.array_equal(got, O.fp8_encode(x.float().numpy()))


def test_fp8_to_fp16_all_codes(dev):
    c = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    got = int4_hip.fp8_to_fp16(c.to(dev)).cpu().float().numpy()
    want = O.fp8_value(c.numpy())
    ok = ~np.isnan(want)
    assert np.array_equal(got[ok].astype(np.float64), want[ok])


@pytest.mark.parametrize("N,K", [(17408, 5120), (5120, 17408), (3, 32), (7, 96)])
def test_dequant_int4_bit_exact(dev, N, K):
    g = S.gen(N + K)
    w, sz = S.int4_weight(N, K, g)
    got = int4_hip.dequant_int4(w.to(dev), sz.to(dev), N, K).cpu().numpy()
    want = O.dequant_int4(w.numpy(), sz.numpy())
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_dequant_int4_exhaustive_scales(dev):
    """All (q, zp) pairs times every finite fp16 scale."""
    x = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    scales = x[np.isfinite(x)]
    N, K = scales.size, 512
    q = np.tile(np.concatenate([np.arange(16), np.arange(16)]).astype(np.uint8), 16)
    packed = O.pack_int4(np.broadcast_to(q, (N, K)))
    zeros = np.broadcast_to(np.arange(16, dtype=np.uint8), (N, 16))
    sz = O.interleave_scale_zero(np.broadcast_to(scales[:, None], (N, 16)), zeros)
    got = int4_hip.dequant_int4(torch.from_numpy(packed).to(dev),
                                torch.from_numpy(np.ascontiguousarray(sz)).to(dev), N, K)
    want = O.dequant_int4(packed, sz)
    assert np.array_equal(got.cpu().numpy().view(np.uint16), want.view(np.uint16))


@pytest.mark.parametrize("N,K", [(5120, 17408), (9, 64)])
def test_dequant_int8_bit_exact(dev, N, K):
    g = S.gen(N * 3 + K)
    w, sz = S.int8_weight(N, K, g)
    got = int4_hip.dequant_int8(w.to(dev), sz.to(dev), N, K).cpu().numpy()
    want = O.dequant_int8(w.numpy(), sz.numpy())
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_dequant_rejects_bad_shape(dev):
    w = torch.zeros(4, 24, dtype=torch.uint8, device=dev)
    s = torch.zeros(4, 3, dtype=torch.float16, device=dev)
    with pytest.raises((RuntimeError, ValueError)):
        int4_hip.dequant_int4(w, s, 4, 48)
