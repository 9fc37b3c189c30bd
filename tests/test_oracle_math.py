"""Pins the oracle's floating-point functions (CPU only) against torch
library routines and closed forms: the FWHT against the Sylvester matrix,
norms against the reference's torch helpers (int4_engine_v5.py:195-211),
GEMV against torch matmul, attention against F.scaled_dot_product_attention."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import r4q_oracle as O
from conftest import rel_l2

H32 = torch.from_numpy(O.hadamard_matrix(32) / math.sqrt(32))


def test_hadamard_orthogonality():
    """tests/test_kernels.py:73-79."""
    H = O.hadamard_matrix(32) / math.sqrt(32)
    assert np.abs(H @ H.T - np.eye(32)).max() < 1e-6
    assert np.array_equal(O.hadamard_matrix(2), np.array([[1, 1], [1, -1]]))


def test_hadamard_rotation_invertible():
    """tests/test_kernels.py:82-99: x W^T == rot(x) rot(W)^T."""
    rng = np.random.default_rng(7)
    W = rng.standard_normal((32, 128))
    x = rng.standard_normal((1, 128))
    Wr = O.fwht32_f64(W)
    xr = O.fwht32_f64(x)
    assert np.abs(x @ W.T - xr @ Wr.T).max() < 1e-10


def test_fwht32_stage_order_matches_matrix():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((64, 256)).astype(np.float32)
    assert rel_l2(O.fwht32(x), O.fwht32_f64(x)) < 1e-6
    # unit vectors give the Hadamard columns exactly
    E = np.eye(32, dtype=np.float32)
    want = (O.hadamard_matrix(32).T.astype(np.float32) * O.INV_SQRT32)
    assert np.array_equal(O.fwht32(E), want)
    # involution
    assert rel_l2(O.fwht32(O.fwht32(x)), x) < 1e-6


def _torch_fast_rmsnorm(x, w, eps):
    """int4_engine_v5.py:208-211 on the CPU."""
    variance = x.float().pow(2).mean(-1, keepdim=True)
    return (x.float() * torch.rsqrt(variance + eps) * w.float()).half()


def _torch_fast_hadamard(x):
    """int4_engine_v5.py:202-205 (fp16 Hadamard matrix), on the CPU in fp32."""
    had = H32.float().half().float()
    return (x.float().reshape(-1, 32) @ had).reshape(x.shape).half()


@pytest.mark.parametrize("D", [128, 5120])
def test_rmsnorm_family_vs_reference_torch(D):
    g = torch.Generator().manual_seed(D)
    x = torch.randn(3, D, generator=g).half()
    b = torch.randn(3, D, generator=g).half()
    w = (1 + 0.02 * torch.randn(D, generator=g)).half()
    eps = 1e-6
    ref = _torch_fast_rmsnorm(x, w, eps)
    got = O.rmsnorm(x.numpy(), w.numpy(), eps)
    assert np.abs(got.astype(np.float32) - ref.float().numpy()).max() <= 2e-3
    assert rel_l2(O.rmsnorm_fwht(x.numpy(), w.numpy(), eps), _torch_fast_hadamard(ref)) < 2e-3
    # residual form (x = x + o_out, int4_engine_v5.py:251-252)
    r = (x + b)
    y, r16 = O.res_rmsnorm_fwht(x.numpy(), b.numpy(), w.numpy(), eps)
    assert np.array_equal(r16, r.numpy())
    assert rel_l2(y, _torch_fast_hadamard(_torch_fast_rmsnorm(r, w, eps))) < 3e-3
    y2, r2 = O.res_rmsnorm(x.numpy(), b.numpy(), w.numpy(), eps)
    assert np.array_equal(r2, r.numpy())
    assert rel_l2(y2, _torch_fast_rmsnorm(r, w, eps)) < 2e-3


def test_rmsnorm_constant_vector_closed_form():
    D, c, eps = 256, 0.5, 1e-6
    x = np.full(D, c, np.float16)
    w = np.linspace(0.5, 1.5, D).astype(np.float16)
    want = (w.astype(np.float64) * c / math.sqrt(c * c + eps)).astype(np.float16)
    got = O.rmsnorm(x, w, eps)
    assert np.abs(got.astype(np.float64) - want.astype(np.float64)).max() <= 1e-3


def test_silu_mul_fwht_vs_torch():
    g = torch.Generator().manual_seed(3)
    a = torch.randn(17408, generator=g).half()
    u = torch.randn(17408, generator=g).half()
    ref = _torch_fast_hadamard(F.silu(a.float()) * u.float())
    assert rel_l2(O.silu_mul_fwht(a.numpy(), u.numpy()), ref) < 2e-3
    assert rel_l2(O.silu_mul(a.numpy(), u.numpy()), (F.silu(a.float()) * u.float()).half()) < 1e-3


@pytest.mark.parametrize("bits,N,K", [(4, 300, 5120), (8, 200, 1024), (16, 100, 512)])
def test_gemm_vs_torch_matmul(bits, N, K):
    """int4_engine_v5.py:227-228 (dequant, then x @ w.T)."""
    import r4q_synth as S
    g = S.gen(bits)
    w, sz = S.weight(N, K, bits, g)
    x = S.rotated_activation(K, g, rows=3)
    W = torch.from_numpy(O.dequant(w.numpy(), None if sz is None else sz.numpy(), bits))
    ref = (x.float() @ W.float().T).half()
    got = O.gemm(x.numpy(), w.numpy(), None if sz is None else sz.numpy(), bits)
    assert rel_l2(got, ref) < 1e-3
    # one-hot input selects a dequantised column exactly
    k = K // 3
    e = np.zeros(K, np.float16)
    e[k] = 1.0
    col = O.gemv(e, w.numpy(), None if sz is None else sz.numpy(), bits)
    assert np.array_equal(col, W[:, k].numpy())


def _torch_head_rmsnorm(x, weight, eps):
    """int4_engine_v5.py:195-199."""
    variance = x.float().pow(2).mean(-1, keepdim=True)
    x = x.float() * torch.rsqrt(variance + eps)
    return (x * weight.float()).half()


def _torch_apply_rope(x, cos, sin, pos):
    """engine_utils.py:79-107 for one position, x [heads, D]."""
    half = x.shape[-1] // 2
    c = cos[pos].float()
    s = sin[pos].float()
    x1, x2 = x[..., :half].float(), x[..., half:].float()
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], -1)


@pytest.mark.parametrize("pos", [0, 1, 777, 2047])
def test_head_norm_rope_kv_vs_reference_torch(pos):
    import r4q_synth as S
    H, Hk, D, eps = 40, 8, 128, 1e-6
    g = S.gen(pos + 11)
    qkv = torch.randn((H + 2 * Hk) * D, generator=g).half()
    qw, kw = S.norm_weight(D, g), S.norm_weight(D, g)
    cos, sin = S.rope_tables(D, 2048 + 16)
    q_out, k_out, kb, vb = O.head_norm_rope_kv(qkv.numpy(), qw.numpy(), kw.numpy(), cos.numpy(),
                                               sin.numpy(), pos, H, Hk, D, eps)
    q = _torch_apply_rope(_torch_head_rmsnorm(qkv[:H * D].view(H, D), qw, eps), cos, sin, pos)
    k = _torch_apply_rope(_torch_head_rmsnorm(qkv[H * D:(H + Hk) * D].view(Hk, D), kw, eps),
                          cos, sin, pos)
    assert rel_l2(q_out, q.half()) < 2e-3
    assert rel_l2(k_out, k.half()) < 2e-3
    v = qkv[(H + Hk) * D:].view(Hk, D)
    assert np.array_equal(vb, O.fp8_encode(v.float().numpy()))
    # K bytes: encoding of the torch restatement agrees except at rounding edges
    agree = (kb == O.fp8_encode(k.numpy())).mean()
    assert agree > 0.97
    if pos == 0:  # cos 1, sin 0: RoPE is the identity on the normed values
        qn = _torch_head_rmsnorm(qkv[:H * D].view(H, D), qw, eps)
        assert rel_l2(q_out, qn) < 2e-3


def _sdpa_reference(q16, kc, vc, L, H, Hk, D, ks=None, vs=None):
    K = torch.from_numpy(O.fp8_decode_ref(kc[:, :L])).float()
    V = torch.from_numpy(O.fp8_decode_ref(vc[:, :L])).float()
    if ks is not None:
        K = K * torch.from_numpy(ks)[:, None, None]
        V = V * torch.from_numpy(vs)[:, None, None]
    q = torch.from_numpy(q16.astype(np.float32)).view(1, H, 1, D)
    o = F.scaled_dot_product_attention(q, K[None], V[None], enable_gqa=True)
    return o.reshape(-1).numpy()


@pytest.mark.parametrize("L", [1, 37, 128, 2048])
def test_attention_vs_sdpa(L):
    import r4q_synth as S
    H, Hk, D = 40, 8, 128
    g = S.gen(L)
    q = torch.randn(H * D, generator=g).half().numpy()
    kc = np.zeros((Hk, L + 5, D), np.uint8)
    vc = np.zeros((Hk, L + 5, D), np.uint8)
    kc[:, :L] = O.fp8_encode(torch.randn(Hk, L, D, generator=g).numpy())
    vc[:, :L] = O.fp8_encode(torch.randn(Hk, L, D, generator=g).numpy())
    ks = (0.5 + torch.rand(Hk, generator=g)).numpy().astype(np.float32)
    vs = (0.5 + torch.rand(Hk, generator=g)).numpy().astype(np.float32)
    got = O.attention_decode(q, kc, vc, L, H, Hk, D, ks, vs)
    ref = _sdpa_reference(q, kc, vc, L, H, Hk, D, ks, vs)
    assert rel_l2(got, ref) < 1e-3
    rot = O.attention_decode(q, kc, vc, L, H, Hk, D, ks, vs, fwht=True)
    assert rel_l2(rot, O.fwht32_f64(ref)) < 1e-3
    if L == 1:  # a single position: output is that position's V row
        V0 = O.fp8_decode_ref(vc[:, 0]).astype(np.float64) * vs[:, None]
        want = np.repeat(V0, H // Hk, axis=0).reshape(-1).astype(np.float16)
        assert np.array_equal(got, want)


def test_wave_sum64_tree_order():
    """The canonical reduction is a fixed tree (differs from a sequential sum
    only by rounding)."""
    rng = np.random.default_rng(5)
    t = rng.standard_normal((10, 64)).astype(np.float32)
    s = O.wave_sum64(t)
    assert np.allclose(s, t.astype(np.float64).sum(1), rtol=1e-6)
    one = np.zeros(64, np.float32)
    one[37] = 3.25
    assert O.wave_sum64(one)[0] == np.float32(3.25)


@pytest.mark.parametrize("M,H,Hk", [(1, 4, 2), (7, 4, 4), (33, 8, 2), (70, 5, 1)])
def test_attention_prefill_vs_torch_sdpa(M, H, Hk):
    g = torch.Generator().manual_seed(M * 13 + H)
    q = torch.randn(M, H, 128, generator=g).half()
    k = torch.randn(M, Hk, 128, generator=g).half()
    v = torch.randn(M, Hk, 128, generator=g).half()
    got = O.attention_prefill(q.numpy(), k.numpy(), v.numpy(), H, Hk)
    want = F.scaled_dot_product_attention(
        q.float().permute(1, 0, 2).unsqueeze(0), k.float().permute(1, 0, 2).unsqueeze(0),
        v.float().permute(1, 0, 2).unsqueeze(0), is_causal=True, enable_gqa=True)
    want = want.squeeze(0).permute(1, 0, 2).reshape(M, H * 128).numpy()
    assert rel_l2(got.astype(np.float32), want) <= 2e-3
    if M == 1:  # one key: the output is v itself
        assert np.array_equal(got.reshape(H, 128), v.numpy()[0][np.arange(H) // (H // Hk)])
    rot = O.attention_prefill(q.numpy(), k.numpy(), v.numpy(), H, Hk, fwht=True)
    assert rel_l2(rot.astype(np.float32), O.fwht32_f64(want).astype(np.float32)) <= 2e-3


def test_prefill_row_matches_decode_steps():
    """The oracle's prompt pass: the last row agrees with decode steps 0..m
    run on the KV codes the prompt pass wrote (up to FP8 vs fp16 K/V in
    attention), and prompt prefixes reproduce their rows exactly."""
    rng = np.random.default_rng(5)
    D, I, H, Hk, L, V, M = 64, 96, 2, 1, 2, 50, 5

    def w4(N, K):
        q = rng.integers(0, 16, (N, K), dtype=np.uint8)
        sz = np.stack([(np.abs(rng.standard_normal((N, K // 32))) * 0.02 + 1e-3),
                       rng.integers(6, 10, (N, K // 32))], -1).astype(np.float16)
        return O.pack_int4(q), sz

    layers = []
    for _ in range(L):
        kw = {}
        for n, (N, K) in dict(qkv=((H + 2 * Hk) * 128, D), o=(D, H * 128), gu=(2 * I, D),
                              down=(D, I)).items():
            kw[n + "_w"], kw[n + "_s"] = w4(N, K)
            kw[n + "_bits"] = 4
        for n in ("in_norm", "post_norm"):
            kw[n] = (1 + 0.02 * rng.standard_normal(D)).astype(np.float16)
        for n in ("q_norm", "k_norm"):
            kw[n] = (1 + 0.02 * rng.standard_normal(128)).astype(np.float16)
        layers.append(O.Layer(**kw))
    embed = (rng.standard_normal((V, D)) * 0.5).astype(np.float16)
    fn = (1 + 0.02 * rng.standard_normal(D)).astype(np.float16)
    lm_w, lm_s = w4(V, D)
    cos, sin = O.rope_tables(128, 16)
    ids = rng.integers(0, V, M)
    common = dict(H=H, Hk=Hk, D=128, hidden=D, inter=I, eps=1e-6, rope_cos=cos, rope_sin=sin,
                  final_norm=fn, lm_w=lm_w, lm_s=lm_s, lm_bits=4)
    kc = [np.zeros((Hk, 16, 128), np.uint8) for _ in range(L)]
    vc = [np.zeros((Hk, 16, 128), np.uint8) for _ in range(L)]
    hid, logits = O.prefill_logits(layers, ids, embed, k_caches=kc, v_caches=vc, **common)
    assert logits.shape == (M, V) and np.all(np.isfinite(logits.astype(np.float32)))
    # decode steps over the prefill's own caches reproduce the last row
    kc2 = [np.zeros_like(a) for a in kc]
    vc2 = [np.zeros_like(a) for a in vc]
    for m in range(M):
        h_dec, lg = O.decode_step(layers, embed[ids[m]], m, kc2, vc2,
                                  forced_kv=[(kc[li][:, m], vc[li][:, m]) for li in range(L)],
                                  **common)
    # decode attends over FP8-decoded K/V, the prompt pass over fp16 K/V (as
    # in the reference), so the routes agree only to FP8 precision
    assert rel_l2(lg.astype(np.float32), logits[-1].astype(np.float32)) <= 0.1
    assert rel_l2(h_dec.astype(np.float32), hid[-1].astype(np.float32)) <= 0.1
    # causality: a prefix of the prompt reproduces the same rows exactly
    hp, lp = O.prefill_logits(layers, ids[:3], embed, **common)
    assert np.array_equal(lp, logits[:3]) and np.array_equal(hp, hid[:3])
