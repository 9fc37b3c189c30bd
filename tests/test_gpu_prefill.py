"""Prompt pass (prefill_logits, hip:2127-2320) against the oracle: logits of
every row, the FP8 KV codes it writes (optional), and a decode step that
continues from the prompt's caches.  Tolerance rel-L2 <= 5e-3."""
import numpy as np
import pytest
import torch

import int4_hip
import r4q_oracle as O
from conftest import rel_l2
from decode_util import build, check_forced_kv, gpu_kv_at, oracle_step, step_logits

pytestmark = pytest.mark.gpu
TOL = 5e-3


def prefill_args(m):
    l = m.lists
    return (l["qkv_w"], l["qkv_s"], l["qkv_N"], l["o_w"], l["o_s"], l["o_N"], l["gu_w"], l["gu_s"],
            l["gu_N"], l["down_w"], l["down_s"], l["down_N"], l["in_norm_w"], l["post_norm_w"],
            l["q_norm_w"], l["k_norm_w"], m.cos_d, m.sin_d, m.H, m.Hk, m.hd, m.D, m.I, m.eps)


def gpu_prefill(m, ids, write_kv=False):
    had = torch.zeros(32, 32, dtype=torch.float16, device=m.dev)
    kw = {}
    if write_kv:
        kw = dict(k_caches=m.k_caches, v_caches=m.v_caches, kv_scales=m.kv_scales)
    return int4_hip.prefill_logits(torch.as_tensor(ids, dtype=torch.int64).to(m.dev), m.embed_d,
                                   m.final_norm_d, m.lm_w_d, m.lm_s_d, m.vocab, m.D,
                                   *prefill_args(m), had, **kw)


def oracle_prefill(m, ids, caches=False, kv_trace=None):
    ks = None if m.k_scales is None else [t.numpy() for t in m.k_scales]
    vs = None if m.v_scales is None else [t.numpy() for t in m.v_scales]
    kc = vc = None
    if caches:
        kc = [np.zeros((m.Hk, m.max_seq, m.hd), np.uint8) for _ in range(m.L)]
        vc = [np.zeros_like(a) for a in kc]
    hid, logits = O.prefill_logits(
        m.oracle_layers, ids, m.embed.numpy(), H=m.H, Hk=m.Hk, D=m.hd, hidden=m.D, inter=m.I,
        eps=m.eps, rope_cos=m.cos.numpy(), rope_sin=m.sin.numpy(),
        final_norm=m.final_norm.numpy(), lm_w=m.lm_w.numpy(),
        lm_s=None if m.lm_s is None else m.lm_s.numpy().reshape(m.vocab, -1, 2),
        lm_bits=m.lm_bits, k_caches=kc, v_caches=vc, k_scales=ks, v_scales=vs,
        kv_trace=kv_trace)
    return hid, logits, kc, vc


@pytest.mark.parametrize("M", [1, 5, 16, 17, 40])
def test_prefill_logits_vs_oracle(dev, M):
    bits = {(0, "o"): 8, (1, "gu"): 8}
    m = build(dev, D=256, I=512, H=4, Hk=2, L=2, vocab=300, max_seq=64, seed=50 + M, bits=bits)
    ids = np.random.default_rng(M).integers(0, m.vocab, M)
    got = gpu_prefill(m, ids).cpu().float().numpy()
    _, want, _, _ = oracle_prefill(m, ids)
    assert got.shape == (M, m.vocab) and np.all(np.isfinite(got))
    for row in range(M):
        assert rel_l2(got[row], want[row]) <= TOL, row


def test_prefill_qwen3_width_one_layer(dev):
    m = build(dev, D=5120, I=17408, H=40, Hk=8, L=1, vocab=1024, max_seq=96, seed=61,
              bits={(0, "down"): 8})
    ids = np.random.default_rng(3).integers(0, m.vocab, 48)
    got = gpu_prefill(m, ids).cpu().float().numpy()
    _, want, _, _ = oracle_prefill(m, ids)
    assert rel_l2(got, want) <= TOL
    assert rel_l2(got[-1], want[-1]) <= TOL


@pytest.mark.parametrize("kv_scale", [False, True])
def test_prefill_writes_kv_then_decode_continues(dev, kv_scale):
    m = build(dev, D=256, I=512, H=8, Hk=2, L=2, vocab=200, max_seq=48, seed=70, fill=0,
              kv_scale=kv_scale)
    M = 20
    ids = np.random.default_rng(9).integers(0, m.vocab, M)
    gpu_prefill(m, ids, write_kv=True)
    torch.cuda.synchronize()
    trace = []
    _, want, kc, vc = oracle_prefill(m, ids, caches=True, kv_trace=trace)
    # every code the GPU wrote is the oracle's or a last-bit rounding neighbour
    forced = [(m.k_caches[li][0, :, :M].cpu().numpy().transpose(1, 0, 2),
               m.v_caches[li][0, :, :M].cpu().numpy().transpose(1, 0, 2)) for li in range(m.L)]
    n = check_forced_kv(forced, trace)
    total = sum(k.size + v.size for k, v in forced)
    assert n <= 0.05 * total
    assert np.all(m.k_caches[0][0, :, M:].cpu().numpy() == 0)  # nothing past the prompt
    # decode at position M from the prompt's caches == oracle on the same caches
    h = m.embed[int(ids[-1])].view(1, 1, m.D).contiguous()
    logits = step_logits(m, h.to(dev), M).cpu().float().numpy().reshape(-1)
    kc_g = [m.k_caches[li][0].cpu().numpy().copy() for li in range(m.L)]
    vc_g = [m.v_caches[li][0].cpu().numpy().copy() for li in range(m.L)]
    for li in range(m.L):  # the oracle starts from the GPU's prompt caches
        kc_g[li][:, M] = 0
        vc_g[li][:, M] = 0
    forced_step = gpu_kv_at(m, M)
    step_trace = []
    _, wlog = oracle_step(m, h.numpy().reshape(-1), M, kc_g, vc_g, forced_kv=forced_step,
                          kv_trace=step_trace)
    check_forced_kv(forced_step, step_trace)
    assert rel_l2(logits, wlog) <= TOL


def test_prefill_rejects_bad_token_and_length(dev):
    m = build(dev, D=256, I=512, H=4, Hk=2, L=1, vocab=100, max_seq=16, seed=80)
    with pytest.raises(RuntimeError):
        gpu_prefill(m, np.array([1, 2, 100]))
    with pytest.raises(RuntimeError):
        gpu_prefill(m, np.arange(17) % 100, write_kv=True)  # beyond the cache


@pytest.mark.parametrize("H,Hk", [(40, 8), (4, 4), (8, 2)])
@pytest.mark.parametrize("M", [1, 17, 64, 65, 200, 512])
def test_prefill_attention_vs_oracle(dev, M, H, Hk):
    """The prompt's causal GQA attention (r4q_prefill_attention) alone:
    ragged query blocks (M not a multiple of 64 or of the 32-key block),
    single-row prompts and group sizes 1, 4, 5, against float64 SDPA with
    the FWHT-32 rotation."""
    import r4q_lib as R
    g = torch.Generator().manual_seed(1000 + M + H)
    stride = (H + 2 * Hk) * 128 + 64  # padded rows
    qkv = (torch.randn(M, stride, generator=g) * 1.5).half()
    q = qkv[:, :H * 128].reshape(M, H, 128)
    k = qkv[:, H * 128:(H + Hk) * 128].reshape(M, Hk, 128)
    v = qkv[:, (H + Hk) * 128:(H + 2 * Hk) * 128].reshape(M, Hk, 128)
    want = O.attention_prefill(q.numpy(), k.numpy(), v.numpy(), H, Hk, fwht=True)
    out = torch.empty(M, H * 128 + 32, dtype=torch.float16, device=dev)
    R.call("r4q_prefill_attention", qkv.to(dev).data_ptr(), stride, out.data_ptr(), H * 128 + 32,
           M, H, Hk, R.stream_handle())
    got = out[:, :H * 128].cpu().numpy()
    assert np.all(np.isfinite(got))
    assert rel_l2(got, want) <= TOL
    for r in sorted({0, M // 2, M - 1}):
        assert rel_l2(got[r], want[r]) <= TOL, r
