"""fused_ops drop-in (fused_ops.py:28-215) on the HIP kernels.  The
reference's Triton arithmetic cannot run here (triton is absent), so the
functions are pinned against torch float32 restatements of the same math
(rel-L2 <= 1e-3) and, for the QK-norm + RoPE, bit-exactly against the
oracle's restatement of the decode step's kernel."""
import numpy as np
import pytest
import torch

import fused_ops
import r4q_oracle as O
import r4q_synth as S
from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _rope_ref(x, c, s):
    lo, hi = x[..., :64], x[..., 64:]
    return torch.cat([lo * c - hi * s, hi * c + lo * s], dim=-1)


@pytest.mark.parametrize("shape", [(1, 1, 5120), (4, 7, 256), (3, 128), (2, 17408)])
def test_fused_rmsnorm(dev, shape):
    g = S.gen(sum(shape))
    x = (torch.randn(*shape, generator=g) * 0.8).half()
    w = S.norm_weight(shape[-1], g)
    got = fused_ops.fused_rmsnorm(x.to(dev), w.to(dev), 1e-6).cpu()
    xf = x.float()
    want = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()
    assert got.shape == x.shape and got.dtype == torch.float16
    assert rel_l2(got, want) <= 1e-3


@pytest.mark.parametrize("H,Hk,pos,tensor_pos", [(40, 8, 0, False), (40, 8, 77, True),
                                                  (8, 2, 1023, False)])
def test_fused_rope_decode(dev, H, Hk, pos, tensor_pos):
    g = S.gen(H + pos)
    q = torch.randn(1, H, 1, 128, generator=g).half()
    k = torch.randn(1, Hk, 1, 128, generator=g).half()
    cos, sin = S.rope_tables(128, 1024)
    p = torch.tensor([pos], device=dev) if tensor_pos else pos
    qo, ko = fused_ops.fused_rope_decode(q.to(dev), k.to(dev), cos.to(dev), sin.to(dev), p)
    c, s = cos[pos].float(), sin[pos].float()
    assert qo.shape == q.shape and ko.shape == k.shape
    assert rel_l2(qo.cpu(), _rope_ref(q.float(), c, s)) <= 1e-3
    assert rel_l2(ko.cpu(), _rope_ref(k.float(), c, s)) <= 1e-3
    if pos == 0:  # cos 1, sin 0: identity
        assert torch.equal(qo.cpu(), q) and torch.equal(ko.cpu(), k)


@pytest.mark.parametrize("H,Hk,pos", [(40, 8, 5), (4, 2, 300)])
def test_fused_qknorm_rope_decode(dev, H, Hk, pos):
    g = S.gen(7 * H + pos)
    q = torch.randn(1, H, 1, 128, generator=g).half()
    k = torch.randn(1, Hk, 1, 128, generator=g).half()
    qw, kw = S.norm_weight(128, g), S.norm_weight(128, g)
    cos, sin = S.rope_tables(128, 512)
    qo, ko = fused_ops.fused_qknorm_rope_decode(q.to(dev), k.to(dev), qw.to(dev), kw.to(dev),
                                                cos.to(dev), sin.to(dev),
                                                torch.tensor(pos, device=dev), 1e-6)
    # torch restatement (head_rmsnorm int4_engine_v5.py:195-199 + apply_rope)
    c, s = cos[pos].float(), sin[pos].float()

    def ref(x, w):
        xf = x.float()
        n = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float()
        return _rope_ref(n, c, s)
    assert rel_l2(qo.cpu(), ref(q, qw)) <= 1e-3
    assert rel_l2(ko.cpu(), ref(k, kw)) <= 1e-3
    # bit-exact against the oracle's restatement of the kernel
    row = np.concatenate([q.numpy().reshape(-1), k.numpy().reshape(-1),
                          np.zeros(Hk * 128, np.float16)])
    q_o, k_o, _, _ = O.head_norm_rope_kv(row, qw.numpy(), kw.numpy(), cos.numpy(), sin.numpy(),
                                         pos, H, Hk, 128, 1e-6)
    assert np.array_equal(qo.cpu().numpy().reshape(-1).view(np.uint16), q_o.view(np.uint16))
    assert np.array_equal(ko.cpu().numpy().reshape(-1).view(np.uint16), k_o.view(np.uint16))


def test_fused_ops_rejects_bad_position(dev):
    q = torch.zeros(1, 4, 1, 128, dtype=torch.float16, device=dev)
    k = torch.zeros(1, 2, 1, 128, dtype=torch.float16, device=dev)
    cos, sin = (t.to(dev) for t in S.rope_tables(128, 16))
    with pytest.raises(ValueError):
        fused_ops.fused_rope_decode(q, k, cos, sin, 16)
