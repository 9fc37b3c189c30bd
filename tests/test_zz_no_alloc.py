"""r4q_flash_decode_noalloc (split partials in a fixed per-GPU device array,
no allocation) against r4q_flash_decode (partials in a context buffer): the
same kernels at the same split count, so outputs must be bit-identical.
Two calls in a row, the second with a smaller input (fewer sequences and
positions), then the size limit is enforced."""
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


def _inputs(dev, B, L, max_seq, seed):
    H, Hk, D = 40, 8, 128
    g = S.gen(seed)
    q = torch.randn(B, H * D, generator=g).half().to(dev)
    kc = int4_hip.fp16_to_fp8(S.random_kv_values(Hk, max_seq, D, g, batch=B).to(dev))
    vc = int4_hip.fp16_to_fp8(S.random_kv_values(Hk, max_seq, D, g, batch=B).to(dev))
    ks = (0.5 + torch.rand(Hk, generator=g)).float().to(dev)
    vs = (0.5 + torch.rand(Hk, generator=g)).float().to(dev)
    return q, kc, vc, ks, vs


def test_noalloc_flash_decode_equals_context_flash_decode(dev):
    H, Hk, D = 40, 8, 128
    h = C.c_void_p()
    R.call("r4q_ctx_create", C.byref(h))
    try:
        for B, L, max_seq, seed in ((8, 3000, 3072, 1), (2, 700, 768, 2)):
            print(f"[noalloc] B={B} L={L}", flush=True)
            q, kc, vc, ks, vs = _inputs(dev, B, L, max_seq, seed)
            want = torch.empty(B, H * D, dtype=torch.float16, device=dev)
            got = torch.full_like(want, float("nan"))
            R.call("r4q_flash_decode", h, q.data_ptr(), H * D, kc.data_ptr(), vc.data_ptr(),
                   ks.data_ptr(), vs.data_ptr(), want.data_ptr(), B, H, Hk, D, max_seq, L, 1,
                   R.stream_handle())
            R.call("r4q_flash_decode_noalloc", q.data_ptr(), H * D, kc.data_ptr(),
                   vc.data_ptr(), ks.data_ptr(), vs.data_ptr(), got.data_ptr(), B, H, Hk, D,
                   max_seq, L, 1, R.stream_handle())
            torch.cuda.synchronize()
            assert torch.equal(got, want)
            b = B - 1
            ref = O.attention_decode(q[b].cpu().numpy(), kc[b].cpu().numpy(), vc[b].cpu().numpy(),
                                     L, H, Hk, D, ks.cpu().numpy(), vs.cpu().numpy(), fwht=True)
            assert rel_l2(got[b].cpu().numpy(), ref) <= 5e-3
    finally:
        R.call("r4q_ctx_destroy", h)


def test_noalloc_flash_decode_rejects_partials_beyond_scratch(dev):
    """128 forced splits x 40 heads x 8 sequences need 21.6 MB of partials,
    beyond the 4 MiB array: rejected before any launch."""
    H, Hk, D, B, L = 40, 8, 128, 8, 4096
    q, kc, vc, _, _ = _inputs(dev, B, L, L, 3)
    out = torch.empty(B, H * D, dtype=torch.float16, device=dev)
    try:
        R.tune("attn_splits", 128)
        rc = R.lib().r4q_flash_decode_noalloc(q.data_ptr(), H * D, kc.data_ptr(), vc.data_ptr(),
                                              None, None, out.data_ptr(), B, H, Hk, D, L, L, 1,
                                              R.stream_handle())
    finally:
        R.tune("attn_splits", 0)
    assert rc == R.R4Q_EINVAL
    assert "scratch" in R.last_error()
