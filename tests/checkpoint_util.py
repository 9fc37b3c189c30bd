"""Writes a small quantized model directory in the reference's on-disk layout
(REPRODUCTION_RECIPE.md:214-283) from seeded random data, key for key as the
reference writers store it (quantize_v4_gptq.py:385-468,
quantize_v5_pure_int4.py:349-415):
  * INT4 groups always carry `{g}_packed`, `{g}_scales` and `{g}_zeros`
    (uint8), tagged `{g}_precision` = 'int4a' (asymmetric: unsigned nibbles,
    zero points 6..9) or 'int4' (symmetric, --symmetric: two's-complement
    nibbles from pack_int4, zeros all 0; int4_quant_v2.py:240-247, 157-161);
  * INT8 groups (v4 mixed precision) `{g}_weights` int8 + `{g}_scales`,
    tagged 'int8';
  * bf16 norms / embedding / final norm, symmetric INT4 LM head (packed,
    scales, quant_format 'int4_symmetric');
  * meta.pt with use_asymmetric and the per-layer precision_map."""
import numpy as np
import torch

import r4q_oracle as O

DIMS = dict(num_layers=2, hidden_size=256, intermediate_size=512, num_heads=4, num_kv_heads=2,
            head_dim=128, vocab=300)


def _scales(rng, N, K, div=1.0):
    return ((np.abs(rng.standard_normal((N, K // 32))) * 0.01 + 1e-3) / div).astype(np.float16)


def _int4_asym(rng, N, K):
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    z = rng.integers(6, 10, (N, K // 32)).astype(np.uint8)
    return torch.from_numpy(O.pack_int4(q)), torch.from_numpy(_scales(rng, N, K)), torch.from_numpy(z)


def _pack_signed(v):
    """pack_int4 (int4_quant_v2.py:157-161): int8 values -8..7, low nibble
    first, two's complement."""
    q = v.astype(np.int8)
    lo = q[..., 0::2].astype(np.uint8) & 0x0F
    hi = q[..., 1::2].astype(np.uint8) & 0x0F
    return (lo | (hi << 4)).astype(np.uint8)


def _int4_sym(rng, N, K):
    v = rng.integers(-8, 8, (N, K))
    return torch.from_numpy(_pack_signed(v)), torch.from_numpy(_scales(rng, N, K))


def _int8_sym(rng, N, K):
    w = rng.integers(-128, 128, (N, K)).astype(np.int8)
    return torch.from_numpy(w), torch.from_numpy(_scales(rng, N, K, div=16))


def write_fake_checkpoint(path, seed=0, symmetric=False, tags=True):
    """symmetric: every INT4 group as the --symmetric writers store it.
    tags=False drops the `{g}_precision` keys (an untagged file: the loader
    must fall back to meta['use_asymmetric']).  Returns per-layer kinds:
    'a' asymmetric INT4, 's' symmetric INT4, '8' INT8."""
    rng = np.random.default_rng(seed)
    D, I, H, Hk, hd = (DIMS[k] for k in ("hidden_size", "intermediate_size", "num_heads",
                                         "num_kv_heads", "head_dim"))
    L, V = DIMS["num_layers"], DIMS["vocab"]
    shapes = {"qkv": ((H + 2 * Hk) * hd, D), "o": (D, H * hd), "gate_up": (2 * I, D),
              "down": (D, I)}
    i4 = "s" if symmetric else "a"
    kinds = [{"qkv": i4, "o": i4, "gate_up": i4, "down": i4},
             {"qkv": i4, "o": "8", "gate_up": i4, "down": "8"}]
    precision_map = {}
    for li in range(L):
        ld = {}
        precision_map[str(li)] = {}
        for g, (N, K) in shapes.items():
            k = kinds[li][g]
            if k == "8":
                w, s = _int8_sym(rng, N, K)
                ld[f"{g}_weights"], ld[f"{g}_scales"] = w, s
                tag = "int8"
            elif k == "s":
                p, s = _int4_sym(rng, N, K)
                ld[f"{g}_packed"], ld[f"{g}_scales"] = p, s
                ld[f"{g}_zeros"] = torch.zeros(N, K // 32, dtype=torch.uint8)
                tag = "int4"
            else:
                p, s, z = _int4_asym(rng, N, K)
                ld[f"{g}_packed"], ld[f"{g}_scales"], ld[f"{g}_zeros"] = p, s, z
                tag = "int4a"
            if tags:
                ld[f"{g}_precision"] = tag
            ld[f"{g}_N"], ld[f"{g}_K"] = N, K
            precision_map[str(li)][g] = "int8" if k == "8" else "int4"
        for n, sz in (("in_norm", D), ("post_norm", D), ("q_norm", hd), ("k_norm", hd)):
            ld[n] = torch.from_numpy(1 + 0.02 * rng.standard_normal(sz)).to(torch.bfloat16)
        torch.save(ld, path / f"layer_{li:03d}.pt")
    p, s = _int4_sym(rng, V, D)
    torch.save({"packed": p, "scales": s, "N": V, "K": D, "rotation": "hadamard",
                "quant_format": "int4_symmetric"}, path / "lm_head.pt")
    torch.save(torch.from_numpy(rng.standard_normal((V, D)) * 0.5).to(torch.bfloat16),
               path / "embed.pt")
    torch.save(torch.from_numpy(1 + 0.02 * rng.standard_normal(D)).to(torch.bfloat16),
               path / "final_norm.pt")
    asym = not symmetric
    meta = dict(model_name="synthetic", num_layers=L, hidden_size=D, intermediate_size=I,
                num_heads=H, num_kv_heads=Hk, head_dim=hd, rms_eps=1e-6, rope_theta=1.0e6,
                method=f"v4_{'asym' if asym else 'sym'}_had_gptq_c4cal", block_size=32,
                quant_format=f"mixed_{'int4a' if asym else 'int4'}_rot_int8",
                use_rotation=True, use_asymmetric=asym, precision_map=precision_map)
    torch.save(meta, path / "meta.pt")
    return kinds
