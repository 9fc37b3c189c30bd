"""A checkpoint directory in the reference's on-disk layout, loaded by
r4q_checkpoint, runs through int4_hip: prompt pass and a decode step agree
with the oracle built from the same loaded tensors (rel-L2 <= 5e-3), for
asymmetric ('int4a') and symmetric ('int4', --symmetric) INT4 files."""
import numpy as np
import pytest
import torch

import int4_hip
import r4q_checkpoint as CK
import r4q_oracle as O
from checkpoint_util import write_fake_checkpoint
from conftest import rel_l2
from decode_util import check_forced_kv

pytestmark = pytest.mark.gpu
TOL = 5e-3


def _oracle_layers(m):
    out = []
    for li in range(m.num_layers):
        kw = {}
        for a, K in (("qkv", m.hidden_size), ("o", m.num_heads * m.head_dim),
                     ("gu", m.hidden_size), ("down", m.intermediate_size)):
            w = getattr(m, a + "_w")[li]
            s = getattr(m, a + "_s")[li]
            bits = int4_hip.weight_bits(w, K)
            kw[a + "_w"] = w.cpu().numpy()
            kw[a + "_s"] = s.cpu().numpy().reshape(w.shape[0], -1, 2)
            kw[a + "_bits"] = bits
        for n in ("in_norm", "post_norm", "q_norm", "k_norm"):
            kw[n] = getattr(m, n)[li].cpu().numpy()
        out.append(O.Layer(**kw))
    return out


def _common(m):
    return dict(H=m.num_heads, Hk=m.num_kv_heads, D=m.head_dim, hidden=m.hidden_size,
                inter=m.intermediate_size, eps=m.rms_eps, rope_cos=m.rope_cos.cpu().numpy(),
                rope_sin=m.rope_sin.cpu().numpy(), final_norm=m.final_norm.cpu().numpy(),
                lm_w=m.lm_w.cpu().numpy(), lm_s=m.lm_s.cpu().numpy().reshape(m.lm_N, -1, 2),
                lm_bits=4)


@pytest.mark.parametrize("symmetric", [False, True])
def test_checkpoint_prefill_then_decode(dev, tmp_path, symmetric):
    write_fake_checkpoint(tmp_path, seed=3, symmetric=symmetric)
    m = CK.load_quantized(tmp_path, device=dev, max_seq=32)
    layers = _oracle_layers(m)
    ids = np.random.default_rng(1).integers(0, m.vocab, 9)
    kc, vc = m.new_kv_caches(1, 32)
    blk = m.layer_block(0)
    pre_block = blk[:18] + blk[19:]
    got = int4_hip.prefill_logits(torch.as_tensor(ids).to(dev), m.embed, m.final_norm, m.lm_w,
                                  m.lm_s, m.lm_N, m.lm_K, *pre_block, m.hadamard,
                                  k_caches=kc, v_caches=vc).cpu().float().numpy()
    _, want = O.prefill_logits(layers, ids, m.embed.cpu().numpy(), **_common(m))
    assert rel_l2(got, want) <= TOL
    # decode the next token from the prompt's caches
    pos = len(ids)
    h = m.embed[int(ids[-1])].view(1, 1, -1).contiguous()
    logits = int4_hip.decode_step_logits(h, *m.layer_block(pos), kc, vc, m.final_norm, m.lm_w,
                                         m.lm_s, m.lm_N, m.lm_K, m.hadamard)
    kcs = [t[0].cpu().numpy().copy() for t in kc]
    vcs = [t[0].cpu().numpy().copy() for t in vc]
    forced = [(kcs[li][:, pos].copy(), vcs[li][:, pos].copy()) for li in range(m.num_layers)]
    trace = []
    _, wl = O.decode_step(layers, h.cpu().numpy().reshape(-1), pos, kcs, vcs, forced_kv=forced,
                          kv_trace=trace, **_common(m))
    check_forced_kv(forced, trace)
    assert rel_l2(logits.cpu().float().numpy().reshape(-1), wl) <= TOL
