"""GPU parity of the batch-1 GEMV (INT4 / INT8 / FP16) against the oracle.
Tolerance: rel-L2 <= 5e-3 on the fp16 output (fp32 accumulation)."""
import numpy as np
import pytest
import torch

import int4_hip
import r4q_oracle as O
import r4q_synth as S
from conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 5e-3


def _run(dev, bits, N, K, seed):
    g = S.gen(seed)
    w, sz = S.weight(N, K, bits, g)
    x = S.rotated_activation(K, g)[0]
    y = int4_hip.dbg_gemv(x.to(dev), w.to(dev), None if sz is None else sz.to(dev), N, K)
    want = O.gemv(x.numpy(), w.numpy(), None if sz is None else sz.numpy(), bits)
    return y.cpu().numpy(), want, (w, sz, x)


@pytest.mark.parametrize("bits,N,K", [
    (4, 17408, 5120),    # config 0: gate_proj
    (4, 7168, 5120),     # qkv
    (4, 34816, 5120),    # gate_up
    (4, 5120, 17408),    # down (INT4)
    (8, 5120, 17408),    # down (INT8)
    (8, 5120, 5120),     # o (INT8)
    (16, 8192, 5120),    # LM-head slice (FP16)
])
def test_gemv_qwen3_shapes(dev, bits, N, K):
    got, want, _ = _run(dev, bits, N, K, seed=N + K + bits)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, want) <= TOL


def test_gemv_skewed_shares_bit_identical(dev):
    """The INT4 down projection runs 512 workgroups of 5 steps; by default the
    first half of the grid takes one step more and the second half one fewer.
    Every row is still reduced whole by one workgroup, so equal shares and
    skews of 1-3 steps give the same bits, and the default matches the
    oracle."""
    import r4q_lib as R
    got = {}
    try:
        for v in (0, 1, 3, 4):
            R.tune("gemv_skew", v)
            got[v], want, _ = _run(dev, 4, 5120, 17408, seed=41)
    finally:
        R.tune("gemv_skew", 0)
    for v in (0, 3, 4):
        assert np.array_equal(got[v].view(np.uint16), got[1].view(np.uint16)), v
    assert rel_l2(got[0], want) <= TOL


@pytest.mark.parametrize("bits", [4, 8, 16])
@pytest.mark.parametrize("N,K", [(1, 32), (3, 64), (7, 160), (100, 256), (33, 1024), (65, 1536),
                                 (129, 4096), (5, 10240), (2, 2176 * 8)])
def test_gemv_ragged_shapes(dev, bits, N, K):
    got, want, _ = _run(dev, bits, N, K, seed=7 * N + K + bits)
    assert rel_l2(got, want) <= TOL


@pytest.mark.parametrize("bits", [4, 8, 16])
def test_gemv_one_hot_selects_column_exactly(dev, bits):
    N, K = 777, 5120
    g = S.gen(99 + bits)
    w, sz = S.weight(N, K, bits, g)
    W = O.dequant(w.numpy(), None if sz is None else sz.numpy(), bits)
    for k in (0, 31, 32, 4095, 5119):
        x = torch.zeros(K, dtype=torch.float16)
        x[k] = 1.0
        y = int4_hip.dbg_gemv(x.to(dev), w.to(dev), None if sz is None else sz.to(dev), N, K)
        assert np.array_equal(y.cpu().numpy(), W[:, k]), k


def test_gemv_reference_known_answer(dev):
    """tests/test_kernels.py:129-171: N=K=5120, seed 42, RTN-quantised
    N(0,1) weights, cosine similarity > 0.99 vs the fp16 dequant matmul."""
    torch.manual_seed(42)
    N = K = 5120
    W = torch.randn(N, K)
    Wb = W.reshape(N, K // 32, 32)
    vmin, vmax = Wb.amin(-1, keepdim=True), Wb.amax(-1, keepdim=True)
    scale = torch.where((vmax - vmin) / 15 > 0, (vmax - vmin) / 15, torch.ones_like(vmin))
    zp = (-vmin / scale).round().clamp(0, 15)
    q = ((Wb / scale) + zp).round().clamp(0, 15).to(torch.uint8).reshape(N, K)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous()
    sz = S.sz_table(scale.squeeze(-1).half(), zp.squeeze(-1).to(torch.uint8))
    x = torch.randn(1, K).half()
    Wd = torch.from_numpy(O.dequant_int4(packed.numpy(), sz.numpy()))
    ref = (x.float() @ Wd.float().T).squeeze(0)
    y = int4_hip.dbg_gemv(x.squeeze(0).to(dev), packed.to(dev), sz.to(dev), N, K).cpu().float()
    cos = torch.nn.functional.cosine_similarity(ref[None], y[None]).item()
    assert cos > 0.99
    assert rel_l2(y, ref) <= TOL


def test_gemv_zero_point_cancels(dev):
    """q == zp everywhere -> exactly zero output."""
    N, K = 64, 5120
    packed = torch.full((N, K // 2), 0x77, dtype=torch.uint8)
    sz = S.sz_table(torch.full((N, K // 32), 0.01).half(), torch.full((N, K // 32), 7))
    x = S.rotated_activation(K, S.gen(1))[0]
    y = int4_hip.dbg_gemv(x.to(dev), packed.to(dev), sz.to(dev), N, K).cpu().float()
    assert torch.all(y.abs() < 1e-3)


def test_gemv_rejects_bad_k(dev):
    w = torch.zeros(4, 24, dtype=torch.uint8, device=dev)
    s = torch.zeros(4, 4, dtype=torch.float16, device=dev)
    x = torch.zeros(48, dtype=torch.float16, device=dev)
    with pytest.raises((RuntimeError, ValueError)):
        int4_hip.dbg_gemv(x, w, s, 4, 48)


@pytest.mark.parametrize("bits", [4, 8, 16])
@pytest.mark.parametrize("N,K,residual", [(7168, 5120, True), (34816, 5120, False),
                                          (257, 2048, True), (5, 96, True), (3000, 8192, False)])
def test_fused_norm_gemv_bit_exact(dev, bits, N, K, residual):
    """r4q_res_rmsnorm_fwht_gemv == r4q_res_rmsnorm_fwht (or r4q_rmsnorm_fwht)
    followed by r4q_gemv, bit for bit, including the residual output."""
    import r4q_lib as R
    g = S.gen(3 * N + K + bits)
    w, sz = (t if t is None else t.to(dev) for t in S.weight(N, K, bits, g))
    a = (torch.randn(K, generator=g) * 0.7).half().to(dev)
    b = (torch.randn(K, generator=g) * 0.7).half().to(dev) if residual else None
    gam = S.norm_weight(K, g).to(dev)
    eps = 1e-6
    rot = torch.empty(K, dtype=torch.float16, device=dev)
    res1 = torch.empty(K, dtype=torch.float16, device=dev)
    res2 = torch.zeros(K, dtype=torch.float16, device=dev)
    y1 = torch.empty(N, dtype=torch.float16, device=dev)
    y2 = torch.empty(N, dtype=torch.float16, device=dev)
    st = R.stream_handle()
    szp = None if sz is None else sz.data_ptr()
    if residual:
        R.call("r4q_res_rmsnorm_fwht", a.data_ptr(), b.data_ptr(), gam.data_ptr(), rot.data_ptr(),
               res1.data_ptr(), 1, K, eps, st)
    else:
        R.call("r4q_rmsnorm_fwht", a.data_ptr(), gam.data_ptr(), rot.data_ptr(), 1, K, eps, st)
    R.call("r4q_gemv", rot.data_ptr(), w.data_ptr(), szp, y1.data_ptr(), N, K, bits, st)
    R.call("r4q_res_rmsnorm_fwht_gemv", a.data_ptr(), b.data_ptr() if residual else None,
           gam.data_ptr(), res2.data_ptr() if residual else None, eps, w.data_ptr(), szp,
           y2.data_ptr(), N, K, bits, st)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    if residual:
        assert torch.equal(res1.view(torch.int16), res2.view(torch.int16))


def test_fused_norm_gemv_rejects_long_rows(dev):
    import r4q_lib as R
    K, N = 17408, 16
    w = torch.zeros(N, K // 2, dtype=torch.uint8, device=dev)
    sz = torch.zeros(N, K // 16, dtype=torch.float16, device=dev)
    a = torch.zeros(K, dtype=torch.float16, device=dev)
    y = torch.empty(N, dtype=torch.float16, device=dev)
    with pytest.raises(RuntimeError):
        R.call("r4q_res_rmsnorm_fwht_gemv", a.data_ptr(), None, a.data_ptr(), None, 1e-6,
               w.data_ptr(), sz.data_ptr(), y.data_ptr(), N, K, 4, R.stream_handle())


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("I,K,norm", [(17408, 5120, True), (1024, 5120, False), (96, 256, True),
                                      (64, 2048, False)])
def test_gate_up_silu_fwht_bit_exact(dev, bits, I, K, norm):
    """r4q_gate_up_silu_fwht == (fused-norm) GEMV into [g; u] followed by
    r4q_silu_mul_fwht, bit for bit, including the residual output."""
    import r4q_lib as R
    g = S.gen(5 * I + K + bits)
    w, sz = (t.to(dev) for t in S.weight(2 * I, K, bits, g))
    a = (torch.randn(K, generator=g) * 0.7).half().to(dev)
    b = (torch.randn(K, generator=g) * 0.7).half().to(dev)
    gam = S.norm_weight(K, g).to(dev)
    eps = 1e-6
    gu = torch.empty(2 * I, dtype=torch.float16, device=dev)
    y1 = torch.empty(I, dtype=torch.float16, device=dev)
    y2 = torch.empty(I, dtype=torch.float16, device=dev)
    res1 = torch.empty(K, dtype=torch.float16, device=dev)
    res2 = torch.zeros(K, dtype=torch.float16, device=dev)
    st = R.stream_handle()
    if norm:
        R.call("r4q_res_rmsnorm_fwht_gemv", a.data_ptr(), b.data_ptr(), gam.data_ptr(),
               res1.data_ptr(), eps, w.data_ptr(), sz.data_ptr(), gu.data_ptr(), 2 * I, K, bits, st)
        R.call("r4q_gate_up_silu_fwht", a.data_ptr(), b.data_ptr(), gam.data_ptr(),
               res2.data_ptr(), eps, w.data_ptr(), sz.data_ptr(), y2.data_ptr(), I, K, bits, st)
    else:
        R.call("r4q_gemv", a.data_ptr(), w.data_ptr(), sz.data_ptr(), gu.data_ptr(), 2 * I, K,
               bits, st)
        R.call("r4q_gate_up_silu_fwht", a.data_ptr(), None, None, None, eps, w.data_ptr(),
               sz.data_ptr(), y2.data_ptr(), I, K, bits, st)
    R.call("r4q_silu_mul_fwht", gu.data_ptr(), gu[I:].data_ptr(), y1.data_ptr(), 1, I, 2 * I, I, st)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    if norm:
        assert torch.equal(res1.view(torch.int16), res2.view(torch.int16))
    # and against the oracle (its exp is numpy's: last-bit differences)
    want = O.silu_mul_fwht(gu[:I].cpu().numpy(), gu[I:].cpu().numpy())
    assert rel_l2(y2.cpu().numpy(), want) <= 1e-3


@pytest.mark.parametrize("bits,dbits", [(4, 4), (8, 8), (4, 16)])
@pytest.mark.parametrize("I,K,norm", [(17408, 5120, True), (1024, 5120, False), (96, 256, True),
                                      (8448, 2048, False)])
@pytest.mark.parametrize("where", ["lib", "none", "all", "mid"])
def test_gate_up_silu_split_then_fwht_gemv_bit_exact(dev, bits, dbits, I, K, norm, where):
    """r4q_gate_up_silu (fp16 FWHT'd units below the split, fp32 silu(g) * u
    above it) followed by r4q_fwht_gemv (FWHT-32 of the fp32 part in the
    staging) == r4q_gate_up_silu_fwht followed by r4q_gemv, bit for bit on
    the fp16 part, the down projection's output and the residual output;
    the fp32 part against the oracle's SiLU product of the GEMV rows."""
    import ctypes as C
    import r4q_lib as R
    if where == "lib":
        sp = C.c_int64()
        R.call("r4q_gate_up_silu_split", I, C.byref(sp))
        split = sp.value
    else:
        split = {"none": 0, "all": I, "mid": 32 * (I // 64)}[where]
    g = S.gen(7 * I + K + bits + dbits)
    w, sz = (t.to(dev) for t in S.weight(2 * I, K, bits, g))
    N = K  # the down projection maps back to the hidden size
    wd, szd = S.weight(N, I, dbits, g)
    wd = wd.to(dev)
    szd = None if szd is None else szd.to(dev)
    a = (torch.randn(K, generator=g) * 0.7).half().to(dev)
    b = (torch.randn(K, generator=g) * 0.7).half().to(dev)
    gam = S.norm_weight(K, g).to(dev)
    eps = 1e-6
    y16 = torch.empty(I, dtype=torch.float16, device=dev)
    ys = torch.full((I,), float("nan"), dtype=torch.float16, device=dev)
    h = torch.full((I,), float("nan"), dtype=torch.float32, device=dev)
    gu = torch.empty(2 * I, dtype=torch.float16, device=dev)
    d1 = torch.empty(N, dtype=torch.float16, device=dev)
    d2 = torch.empty(N, dtype=torch.float16, device=dev)
    res1 = torch.empty(K, dtype=torch.float16, device=dev)
    res2 = torch.zeros(K, dtype=torch.float16, device=dev)
    st = R.stream_handle()
    szp = None if szd is None else szd.data_ptr()
    if norm:
        R.call("r4q_gate_up_silu_fwht", a.data_ptr(), b.data_ptr(), gam.data_ptr(),
               res1.data_ptr(), eps, w.data_ptr(), sz.data_ptr(), y16.data_ptr(), I, K, bits, st)
        R.call("r4q_gate_up_silu", a.data_ptr(), b.data_ptr(), gam.data_ptr(), res2.data_ptr(),
               eps, w.data_ptr(), sz.data_ptr(), ys.data_ptr(), h.data_ptr(), split, I, K, bits,
               st)
        R.call("r4q_res_rmsnorm_fwht_gemv", a.data_ptr(), b.data_ptr(), gam.data_ptr(),
               res1.data_ptr(), eps, w.data_ptr(), sz.data_ptr(), gu.data_ptr(), 2 * I, K, bits, st)
    else:
        R.call("r4q_gate_up_silu_fwht", a.data_ptr(), None, None, None, eps, w.data_ptr(),
               sz.data_ptr(), y16.data_ptr(), I, K, bits, st)
        R.call("r4q_gate_up_silu", a.data_ptr(), None, None, None, eps, w.data_ptr(),
               sz.data_ptr(), ys.data_ptr(), h.data_ptr(), split, I, K, bits, st)
        R.call("r4q_gemv", a.data_ptr(), w.data_ptr(), sz.data_ptr(), gu.data_ptr(), 2 * I, K,
               bits, st)
    R.call("r4q_gemv", y16.data_ptr(), wd.data_ptr(), szp, d1.data_ptr(), N, I, dbits, st)
    R.call("r4q_fwht_gemv", ys.data_ptr(), h.data_ptr(), split, wd.data_ptr(), szp,
           d2.data_ptr(), N, I, dbits, st)
    torch.cuda.synchronize()
    assert torch.equal(ys[:split].view(torch.int16), y16[:split].view(torch.int16))
    assert torch.isfinite(h[split:]).all()
    assert torch.equal(d1.view(torch.int16), d2.view(torch.int16))
    if norm:
        assert torch.equal(res1.view(torch.int16), res2.view(torch.int16))
    if split < I:
        # the oracle rounds the product to fp16 (and its exp is numpy's)
        want = O.silu_mul(gu[split:I].cpu().numpy(), gu[I + split:].cpu().numpy())
        assert rel_l2(h[split:].cpu().numpy(), want) <= 1e-3


def test_gate_up_silu_split_rejects_bad_split(dev):
    import r4q_lib as R
    I, K = 64, 256
    w = torch.zeros(2 * I, K // 2, dtype=torch.uint8, device=dev)
    sz = torch.zeros(2 * I, K // 32, dtype=torch.int32, device=dev)
    a = torch.zeros(K, dtype=torch.float16, device=dev)
    y = torch.empty(I, dtype=torch.float16, device=dev)
    h = torch.empty(I, dtype=torch.float32, device=dev)
    for split in (-32, 16, I + 32):
        with pytest.raises(RuntimeError):
            R.call("r4q_gate_up_silu", a.data_ptr(), None, None, None, 1e-6, w.data_ptr(),
                   sz.data_ptr(), y.data_ptr(), h.data_ptr(), split, I, K, 4, R.stream_handle())
