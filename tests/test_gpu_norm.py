"""GPU parity of the norm / rotation / SiLU / QK-norm+RoPE+KV kernels.
Bit-exact where the oracle follows the kernel's operation order (residual
sums, FWHT, FP8 KV bytes, QK-norm+RoPE outputs); rel-L2 <= 5e-3 otherwise."""
import ctypes as C

import numpy as np
import pytest
import torch

import int4_hip
import r4q_lib as R
import r4q_oracle as O
import r4q_synth as S
from conftest import rel_l2

pytestmark = pytest.mark.gpu
TOL = 5e-3
EPS = 1e-6


def assert_same(got, want):
    got, want = np.asarray(got), np.asarray(want)
    bad = np.flatnonzero(got.reshape(-1).view(np.uint8 if got.dtype == np.uint8 else np.uint16)
                         != want.reshape(-1).view(np.uint8 if want.dtype == np.uint8 else np.uint16))
    assert bad.size == 0, (f"{bad.size} mismatches; first at {bad[:5].tolist()}: "
                           f"got {got.reshape(-1)[bad[:5]].tolist()} want {want.reshape(-1)[bad[:5]].tolist()}")


def _st():
    return R.stream_handle()


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("rows,D", [(1, 5120), (3, 5120), (2, 128), (512, 5120), (1, 17408),
                                    (4, 2048)])
def test_rownorm_family(dev, rows, D):
    g = S.gen(rows * 7 + D)
    a = (torch.randn(rows, D, generator=g) * 3).half()
    b = (torch.randn(rows, D, generator=g) * 3).half()
    w = S.norm_weight(D, g)
    A, B, W = a.to(dev), b.to(dev), w.to(dev)
    y = torch.empty_like(A)
    r = torch.empty_like(A)
    R.call("r4q_rmsnorm", A.data_ptr(), W.data_ptr(), y.data_ptr(), rows, D, C.c_float(EPS), _st())
    assert rel_l2(y.cpu(), O.rmsnorm(a.numpy(), w.numpy(), EPS)) <= TOL
    R.call("r4q_rmsnorm_fwht", A.data_ptr(), W.data_ptr(), y.data_ptr(), rows, D, C.c_float(EPS),
           _st())
    assert rel_l2(y.cpu(), O.rmsnorm_fwht(a.numpy(), w.numpy(), EPS)) <= TOL
    R.call("r4q_res_rmsnorm", A.data_ptr(), B.data_ptr(), W.data_ptr(), y.data_ptr(), r.data_ptr(),
           rows, D, C.c_float(EPS), _st())
    yo, ro = O.res_rmsnorm(a.numpy(), b.numpy(), w.numpy(), EPS)
    assert np.array_equal(r.cpu().numpy(), ro)
    assert rel_l2(y.cpu(), yo) <= TOL
    R.call("r4q_res_rmsnorm_fwht", A.data_ptr(), B.data_ptr(), W.data_ptr(), y.data_ptr(),
           r.data_ptr(), rows, D, C.c_float(EPS), _st())
    yo, ro = O.res_rmsnorm_fwht(a.numpy(), b.numpy(), w.numpy(), EPS)
    assert np.array_equal(r.cpu().numpy(), ro)
    assert rel_l2(y.cpu(), yo) <= TOL


def test_dbg_wrappers(dev):
    g = S.gen(5)
    D = 5120
    x = torch.randn(D, generator=g).half()
    res = torch.randn(D, generator=g).half()
    w = S.norm_weight(D, g)
    y = int4_hip.dbg_rmsnorm(x.to(dev), w.to(dev), EPS)
    assert rel_l2(y.cpu(), O.rmsnorm(x.numpy(), w.numpy(), EPS)) <= TOL
    y, r = int4_hip.dbg_fused_res_norm(x.to(dev), res.to(dev), w.to(dev), EPS)
    yo, ro = O.res_rmsnorm(x.numpy(), res.numpy(), w.numpy(), EPS)
    assert np.array_equal(r.cpu().numpy(), ro) and rel_l2(y.cpu(), yo) <= TOL


@pytest.mark.parametrize("n", [32, 5120, 17408 * 3])
def test_fwht32_bit_exact(dev, n):
    x = (torch.randn(n, generator=S.gen(n)) * 4).half()
    X = x.to(dev)
    y = torch.empty_like(X)
    R.call("r4q_fwht32", X.data_ptr(), y.data_ptr(), n, _st())
    want = O.fwht32(x.float().numpy()).astype(np.float16)
    assert_same(y.cpu().numpy(), want)


@pytest.mark.parametrize("rows,I", [(1, 17408), (3, 17408), (2, 64)])
def test_silu_mul_fwht(dev, rows, I):
    g = S.gen(I + rows)
    gu = (torch.randn(rows, 2 * I, generator=g) * 2).half()
    GU = gu.to(dev)
    y = torch.empty(rows, I, dtype=torch.float16, device=dev)
    R.call("r4q_silu_mul_fwht", GU.data_ptr(), GU[:, I:].data_ptr(), y.data_ptr(), rows, I, 2 * I,
           I, _st())
    assert rel_l2(y.cpu(), O.silu_mul_fwht(gu[:, :I].numpy(), gu[:, I:].numpy())) <= TOL
    R.call("r4q_silu_mul", GU.data_ptr(), GU[:, I:].data_ptr(), y.data_ptr(), rows, I, 2 * I, I,
           _st())
    assert rel_l2(y.cpu(), O.silu_mul(gu[:, :I].numpy(), gu[:, I:].numpy())) <= TOL
    # in place into the gate half, as the decode step does (hip:2512-2513)
    R.call("r4q_silu_mul_fwht", GU.data_ptr(), GU[:, I:].data_ptr(), GU.data_ptr(), rows, I, 2 * I,
           2 * I, _st())
    assert rel_l2(GU[:, :I].cpu(), O.silu_mul_fwht(gu[:, :I].numpy(), gu[:, I:].numpy())) <= TOL


@pytest.mark.parametrize("pos", [0, 1, 2047, 32767])
@pytest.mark.parametrize("scaled", [False, True])
def test_head_norm_rope_kv_bit_exact(dev, pos, scaled):
    H, Hk, D = 40, 8, 128
    B = 2
    max_seq = pos + 3
    g = S.gen(pos * 2 + scaled)
    qkv = (torch.randn(B, (H + 2 * Hk) * D, generator=g) * 2).half()
    qw, kw = S.norm_weight(D, g), S.norm_weight(D, g)
    cos, sin = S.rope_tables(D, max_seq)
    ks = (0.25 + torch.rand(Hk, generator=g)).float() if scaled else None
    vs = (0.25 + torch.rand(Hk, generator=g)).float() if scaled else None
    kc = torch.zeros(B, Hk, max_seq, D, dtype=torch.uint8, device=dev)
    vc = torch.zeros_like(kc)
    # device copies held in variables: a temporary's memory could be reused
    # before the kernel runs
    QKV, QW, KW, COS, SIN = (t.to(dev) for t in (qkv, qw, kw, cos, sin))
    qo = torch.zeros(B, (H + Hk) * D, dtype=torch.float16, device=dev)
    Ks, Vs = (ks.to(dev), vs.to(dev)) if scaled else (None, None)
    R.call("r4q_head_norm_rope_kv", QKV.data_ptr(), (H + 2 * Hk) * D, QW.data_ptr(),
           KW.data_ptr(), qo.data_ptr(), (H + Hk) * D, kc.data_ptr(), vc.data_ptr(),
           R.ptr(Ks), R.ptr(Vs), COS.data_ptr(), SIN.data_ptr(), B, H, Hk, D,
           C.c_float(EPS), max_seq, pos, _st())
    for b in range(B):
        q_out, k_out, kb, vb = O.head_norm_rope_kv(
            qkv[b].numpy(), qw.numpy(), kw.numpy(), cos.numpy(), sin.numpy(), pos, H, Hk, D, EPS,
            None if ks is None else ks.numpy(), None if vs is None else vs.numpy())
        got = qo[b].cpu().numpy()
        assert_same(got[:H * D], q_out)
        assert_same(got[H * D:], k_out)
        assert_same(kc[b, :, pos].cpu().numpy(), kb)
        assert_same(vc[b, :, pos].cpu().numpy(), vb)
    # nothing else in the caches was touched
    assert int(kc.sum().item()) == int(kc[:, :, pos].sum().item())


def test_head_norm_rope_kv_rejects_position_outside_cache(dev):
    z = torch.zeros(16, dtype=torch.float16, device=dev)
    c8 = torch.zeros(16, dtype=torch.uint8, device=dev)
    rc = R.lib().r4q_head_norm_rope_kv(z.data_ptr(), 7168, z.data_ptr(), z.data_ptr(), z.data_ptr(),
                                       6144, c8.data_ptr(), c8.data_ptr(), None, None,
                                       z.data_ptr(), z.data_ptr(), 1, 40, 8, 128, C.c_float(EPS),
                                       16, 16, None)
    assert rc == R.R4Q_EINVAL


def test_dbg_head_rmsnorm_and_rope(dev):
    H, Hk, D = 40, 8, 128
    g = S.gen(77)
    q = torch.randn(H * D, generator=g).half()
    k = torch.randn(Hk * D, generator=g).half()
    qw, kw = S.norm_weight(D, g), S.norm_weight(D, g)
    qo, ko = int4_hip.dbg_head_rmsnorm(q.to(dev), k.to(dev), qw.to(dev), kw.to(dev), H, Hk, D, EPS)
    want_q = (O.rmsnorm(q.numpy().reshape(H, D), qw.numpy(), EPS)).reshape(-1)
    want_k = (O.rmsnorm(k.numpy().reshape(Hk, D), kw.numpy(), EPS)).reshape(-1)
    assert rel_l2(qo.cpu(), want_q) <= TOL and rel_l2(ko.cpu(), want_k) <= TOL
    cos, sin = S.rope_tables(D, 100)
    qr, kr = int4_hip.dbg_rope(q.to(dev), k.to(dev), cos[37].to(dev), sin[37].to(dev), H, Hk, D)
    c, s = cos[37].float(), sin[37].float()
    qf = q.float().view(H, D)
    want = torch.cat([qf[:, :64] * c - qf[:, 64:] * s, qf[:, 64:] * c + qf[:, :64] * s], 1)
    assert rel_l2(qr.cpu(), want.half()) <= TOL
