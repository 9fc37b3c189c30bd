"""On-disk quantized model directory -> int4_hip arguments (r4q_checkpoint).
Every converted weight must dequantise to exactly the value the stored
format denotes (asymmetric INT4: (q - zp) * s; symmetric INT4: signed nibble
* s; symmetric INT8: q * s), all as fp16 of the exact product."""
import numpy as np
import torch

import r4q_checkpoint as CK
import r4q_oracle as O
from checkpoint_util import DIMS, write_fake_checkpoint


def _expected(ld, g):
    s = ld[f"{g}_scales"].float().numpy()
    if f"{g}_weights" in ld:
        q = ld[f"{g}_weights"].numpy().astype(np.float32)
    else:
        n = O.unpack_int4(ld[f"{g}_packed"].numpy()).astype(np.float32)
        if f"{g}_zeros" in ld:
            q = n - np.repeat(ld[f"{g}_zeros"].numpy().astype(np.float32), 32, axis=1)
        else:
            q = np.where(n >= 8, n - 16, n)
    return (q * np.repeat(s, 32, axis=1)).astype(np.float16)


def test_loader_converts_every_format_exactly(tmp_path):
    kinds = write_fake_checkpoint(tmp_path)
    m = CK.load_quantized(tmp_path, device="cpu", max_seq=64)
    assert m.num_layers == DIMS["num_layers"] and m.vocab == DIMS["vocab"]
    for li in range(m.num_layers):
        ld = torch.load(tmp_path / f"layer_{li:03d}.pt", weights_only=True)
        for g, a in (("qkv", "qkv"), ("o", "o"), ("gate_up", "gu"), ("down", "down")):
            w, sz = getattr(m, a + "_w")[li], getattr(m, a + "_s")[li]
            bits = 8 if kinds[li][g] == "8" else 4
            K = w.shape[1] * (2 if bits == 4 else 1)
            assert sz.shape == (w.shape[0], K // 16) and sz.dtype == torch.float16
            got = O.dequant(w.numpy(), sz.numpy().reshape(w.shape[0], -1, 2), bits)
            assert np.array_equal(got.view(np.uint16), _expected(ld, g).view(np.uint16)), (li, g)
        assert m.in_norm[li].dtype == torch.float16
    lm = torch.load(tmp_path / "lm_head.pt", weights_only=True)
    got = O.dequant(m.lm_w.numpy(), m.lm_s.numpy().reshape(m.lm_N, -1, 2), 4)
    want = _expected({"lm_scales": lm["scales"], "lm_packed": lm["packed"]}, "lm")
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    assert m.embed.dtype == torch.float16 and m.embed.shape == (DIMS["vocab"], DIMS["hidden_size"])
    assert m.rope_cos.shape == (64 + 128, 64)
    assert len(m.layer_block(3)) == 25
