"""On-disk quantized model directory -> int4_hip arguments (r4q_checkpoint).
Every converted weight must dequantise to exactly the value the stored
format denotes (asymmetric INT4 'int4a': (q - zp) * s; symmetric INT4 'int4':
signed two's-complement nibble * s with the stored all-zero zeros ignored;
symmetric INT8: q * s), all as fp16 of the exact product."""
import numpy as np
import pytest
import torch

import r4q_checkpoint as CK
import r4q_oracle as O
import r4q_synth as S
from checkpoint_util import DIMS, write_fake_checkpoint


def _expected(ld, g, kind):
    """Value each stored element denotes, by the writer's own format."""
    s = ld[f"{g}_scales"].float().numpy()
    if kind == "8":
        q = ld[f"{g}_weights"].numpy().astype(np.float32)
    else:
        n = O.unpack_int4(ld[f"{g}_packed"].numpy()).astype(np.float32)
        if kind == "a":
            q = n - np.repeat(ld[f"{g}_zeros"].numpy().astype(np.float32), 32, axis=1)
        else:  # unpack_int4 (int4_quant_v2.py:164-170): nibbles > 7 are negative
            q = np.where(n > 7, n - 16, n)
    return (q * np.repeat(s, 32, axis=1)).astype(np.float16)


@pytest.mark.parametrize("symmetric,tags", [(False, True), (True, True), (True, False),
                                            (False, False)])
def test_loader_converts_every_format_exactly(tmp_path, symmetric, tags):
    kinds = write_fake_checkpoint(tmp_path, symmetric=symmetric, tags=tags)
    m = CK.load_quantized(tmp_path, device="cpu", max_seq=64)
    assert m.num_layers == DIMS["num_layers"] and m.vocab == DIMS["vocab"]
    n_neg = 0
    for li in range(m.num_layers):
        ld = torch.load(tmp_path / f"layer_{li:03d}.pt", weights_only=True)
        for g, a in (("qkv", "qkv"), ("o", "o"), ("gate_up", "gu"), ("down", "down")):
            w, sz = getattr(m, a + "_w")[li], getattr(m, a + "_s")[li]
            kind = kinds[li][g]
            bits = 8 if kind == "8" else 4
            K = w.shape[1] * (2 if bits == 4 else 1)
            assert sz.shape == (w.shape[0], K // 16) and sz.dtype == torch.float16
            got = O.dequant(w.numpy(), sz.numpy().reshape(w.shape[0], -1, 2), bits)
            want = _expected(ld, g, kind)
            assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), (li, g)
            n_neg += int((want < 0).sum())
        assert m.in_norm[li].dtype == torch.float16
    assert n_neg > 0  # negative weights exist (a symmetric file read as asymmetric loses them)
    lm = torch.load(tmp_path / "lm_head.pt", weights_only=True)
    got = O.dequant(m.lm_w.numpy(), m.lm_s.numpy().reshape(m.lm_N, -1, 2), 4)
    want = _expected({"lm_scales": lm["scales"], "lm_packed": lm["packed"]}, "lm", "s")
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    assert m.embed.dtype == torch.float16 and m.embed.shape == (DIMS["vocab"], DIMS["hidden_size"])
    assert m.rope_cos.shape == (64 + 128, 64)
    assert len(m.layer_block(3)) == 25


def test_symmetric_tag_wins_over_stored_zeros():
    """A symmetric group stores zeros = 0 (int4_quant_v2.py:245); read as
    asymmetric with those zeros, nibble 0xF (-1) would decode as +15."""
    assert CK.int4_is_symmetric("int4", torch.zeros(1), {"use_asymmetric": True})
    assert not CK.int4_is_symmetric("int4a", torch.zeros(1), {"use_asymmetric": False})
    assert CK.int4_is_symmetric(None, torch.zeros(1), {"use_asymmetric": False})
    assert not CK.int4_is_symmetric(None, torch.zeros(1), {})
    assert CK.int4_is_symmetric(None, None, {})


def test_rope_tables_built_in_float32_like_the_engine():
    """precompute_rope_freqs (engine_utils.py:70-76) works in float32; at a
    few thousand positions its fp16 tables differ from a float64 build on a
    visible fraction of entries, so this pins the float32 construction."""
    n = 2176
    cos, sin = CK.rope_tables(128, n, 1.0e6, "cpu")
    c2, s2 = S.rope_tables(128, n)
    assert torch.equal(cos, c2) and torch.equal(sin, s2)
    inv = 1.0 / (1.0e6 ** (np.arange(0, 128, 2, dtype=np.float64) / 128))
    ang = np.outer(np.arange(n, dtype=np.float64), inv)
    c64 = np.cos(ang).astype(np.float16)
    frac = float((cos.numpy() != c64).mean())
    assert 0.001 < frac < 0.1, frac
    # position 0 and the first column (frequency 1) are exact in float32
    assert torch.all(cos[0] == 1) and torch.all(sin[0] == 0)
    t = np.arange(n, dtype=np.float64)
    assert np.array_equal(cos[:, 0].numpy(), np.cos(t).astype(np.float16))
