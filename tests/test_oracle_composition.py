"""Pins the oracle's layer composition (decode_step, decode_step_batch,
prefill_logits) by routes that share no code with it:

  * a torch restatement of the reference's own prompt pass, fast_prefill
    (int4_engine_v5.py:214-266: fast_rmsnorm -> .half() -> fast_hadamard
    (x @ fp16 H32/sqrt(32)), dequant + matmul, head_rmsnorm, apply_rope
    (engine_utils.py:79-107), causal GQA SDPA, F.silu(g) * u, residual adds in
    fp16), compared with O.prefill_logits layer by layer and on the logits;
  * decode steps at positions 0..M-1 against the prompt pass attending over
    the same FP8 codes (O.prefill_logits(attend_fp8=True)), layer by layer;
  * O.decode_step_batch rows against O.decode_step.

Norm weights are spread over 0.5-1.5 so that a norm-weight mix-up (the wrong
layer's or the wrong norm's gamma) moves results far beyond the tolerance.
The two routes round in different places (the reference rounds the norm to
fp16 before the Hadamard matmul, the kernels after), so they agree to
rel-L2 <= 5e-3, not bit for bit."""
import numpy as np
import pytest
import torch

import r4q_oracle as O
import r4q_torch_ref as TR
from conftest import rel_l2

TOL = 5e-3
D, I, H, Hk, L, V, M, EPS = 256, 512, 4, 2, 2, 300, 9, 1e-6


def _model(seed):
    rng = np.random.default_rng(seed)

    def w4(N, K):
        q = rng.integers(0, 16, (N, K), dtype=np.uint8)
        sz = np.stack([(np.abs(rng.standard_normal((N, K // 32))) * 0.02 + 1e-3),
                       rng.integers(6, 10, (N, K // 32))], -1).astype(np.float16)
        return O.pack_int4(q), sz

    def gamma(n):
        return rng.uniform(0.5, 1.5, n).astype(np.float16)

    layers = []
    for _ in range(L):
        kw = {}
        for n, (N, K) in dict(qkv=((H + 2 * Hk) * 128, D), o=(D, H * 128), gu=(2 * I, D),
                              down=(D, I)).items():
            kw[n + "_w"], kw[n + "_s"] = w4(N, K)
            kw[n + "_bits"] = 4
        kw["in_norm"], kw["post_norm"] = gamma(D), gamma(D)
        kw["q_norm"], kw["k_norm"] = gamma(128), gamma(128)
        layers.append(O.Layer(**kw))
    embed = (rng.standard_normal((V, D)) * 0.5).astype(np.float16)
    final = gamma(D)
    lm_w, lm_s = w4(V, D)
    ids = rng.integers(0, V, M)
    return layers, embed, final, lm_w, lm_s, ids


def _t_prefill(layers, embed, final, lm_w, lm_s, ids, cos, sin):
    return TR.prefill(layers, embed, final, lm_w, lm_s, ids, cos, sin, eps=EPS, H=H, Hk=Hk, I=I)


def _common(final, lm_w, lm_s, cos, sin):
    return dict(H=H, Hk=Hk, D=128, hidden=D, inter=I, eps=EPS, rope_cos=cos, rope_sin=sin,
                final_norm=final, lm_w=lm_w, lm_s=lm_s, lm_bits=4)


@pytest.mark.parametrize("seed", [0, 1])
def test_oracle_prefill_matches_torch_restatement_of_fast_prefill(seed):
    layers, embed, final, lm_w, lm_s, ids = _model(seed)
    cos, sin = O.rope_tables(128, 32)
    trace = []
    _, logits = O.prefill_logits(layers, ids, embed, trace=trace,
                                 **_common(final, lm_w, lm_s, cos, sin))
    t_trace, t_logits = _t_prefill(layers, embed, final, lm_w, lm_s, ids,
                                   torch.from_numpy(cos), torch.from_numpy(sin))
    for li in range(L):
        assert rel_l2(trace[li], t_trace[li]) <= TOL, (li, rel_l2(trace[li], t_trace[li]))
    assert rel_l2(logits, t_logits) <= TOL, rel_l2(logits, t_logits)


def test_torch_restatement_detects_a_norm_weight_mixup():
    """Planted in the oracle's inputs: layer 1's post-attention norm weight
    swapped for its input norm weight.  The restatement must then disagree
    by far more than the tolerance (so the comparison above has teeth)."""
    layers, embed, final, lm_w, lm_s, ids = _model(0)
    cos, sin = O.rope_tables(128, 32)
    t_trace, t_logits = _t_prefill(layers, embed, final, lm_w, lm_s, ids,
                                   torch.from_numpy(cos), torch.from_numpy(sin))
    bad = [O.Layer(**vars(ly)) for ly in layers]
    bad[1].post_norm = layers[1].in_norm
    _, logits = O.prefill_logits(bad, ids, embed, **_common(final, lm_w, lm_s, cos, sin))
    assert rel_l2(logits, t_logits) > 10 * TOL


def test_decode_steps_match_prefill_rows_over_fp8_kv():
    """Decode steps at positions 0..M-1 on the KV codes the prompt pass wrote
    equal the prompt pass attending through the same FP8 codes, layer by
    layer and on the logits."""
    layers, embed, final, lm_w, lm_s, ids = _model(3)
    cos, sin = O.rope_tables(128, 32)
    com = _common(final, lm_w, lm_s, cos, sin)
    kc = [np.zeros((Hk, 32, 128), np.uint8) for _ in range(L)]
    vc = [np.zeros((Hk, 32, 128), np.uint8) for _ in range(L)]
    p_trace = []
    _, p_logits = O.prefill_logits(layers, ids, embed, k_caches=kc, v_caches=vc, trace=p_trace,
                                   attend_fp8=True, **com)
    kc2 = [np.zeros_like(a) for a in kc]
    vc2 = [np.zeros_like(a) for a in vc]
    for m in range(M):
        d_trace = []
        _, lg = O.decode_step(layers, embed[ids[m]], m, kc2, vc2, trace=d_trace, **com)
        for li in range(L):
            assert rel_l2(d_trace[li], p_trace[li][m]) <= TOL, (m, li)
        assert rel_l2(lg, p_logits[m]) <= TOL, (m, rel_l2(lg, p_logits[m]))
    # the decode steps rewrote the same KV codes, up to last-bit rounding
    for li in range(L):
        same = (kc2[li][:, :M] == kc[li][:, :M]).mean()
        assert same >= 0.97, (li, same)


def test_decode_step_batch_rows_equal_decode_step():
    layers, embed, final, lm_w, lm_s, ids = _model(4)
    cos, sin = O.rope_tables(128, 32)
    com = _common(final, lm_w, lm_s, cos, sin)
    B, pos = 3, 5
    rng = np.random.default_rng(9)
    kc = [O.fp8_encode(rng.standard_normal((B, Hk, 32, 128)).astype(np.float32)) for _ in range(L)]
    vc = [O.fp8_encode(rng.standard_normal((B, Hk, 32, 128)).astype(np.float32)) for _ in range(L)]
    h = (rng.standard_normal((B, D)) * 0.5).astype(np.float16)
    kcb = [a.copy() for a in kc]
    vcb = [a.copy() for a in vc]
    hb, lb = O.decode_step_batch(layers, h, pos, kcb, vcb, **com)
    for b in range(B):
        kr = [a[b].copy() for a in kc]
        vr = [a[b].copy() for a in vc]
        hr, lr = O.decode_step(layers, h[b], pos, kr, vr, **com)
        assert rel_l2(hb[b], hr) <= 1e-3 and rel_l2(lb[b], lr) <= 1e-3
        for li in range(L):
            assert (kcb[li][b] == kr[li]).mean() > 0.99
