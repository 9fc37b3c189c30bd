"""Writes a small quantized model directory in the reference's on-disk layout
(REPRODUCTION_RECIPE.md:214-283; quantize_v4_gptq.py:385-468 writer) from
seeded random data: INT4 asymmetric groups (packed, scales, zeros), an INT4
symmetric group (no zeros), an INT8 symmetric group (weights, scales),
bf16 norms / embedding / final norm and a symmetric INT4 LM head."""
import numpy as np
import torch

import r4q_oracle as O

DIMS = dict(num_layers=2, hidden_size=256, intermediate_size=512, num_heads=4, num_kv_heads=2,
            head_dim=128, vocab=300)


def _int4_asym(rng, N, K):
    q = rng.integers(0, 16, (N, K), dtype=np.uint8)
    s = (np.abs(rng.standard_normal((N, K // 32))) * 0.01 + 1e-3).astype(np.float16)
    z = rng.integers(6, 10, (N, K // 32)).astype(np.uint8)
    return torch.from_numpy(O.pack_int4(q)), torch.from_numpy(s), torch.from_numpy(z)


def _int4_sym(rng, N, K):
    v = rng.integers(-8, 8, (N, K))  # two's-complement nibbles
    q = (v & 0xF).astype(np.uint8)
    s = (np.abs(rng.standard_normal((N, K // 32))) * 0.01 + 1e-3).astype(np.float16)
    return torch.from_numpy(O.pack_int4(q)), torch.from_numpy(s)


def _int8_sym(rng, N, K):
    w = rng.integers(-128, 128, (N, K)).astype(np.int8)
    s = ((np.abs(rng.standard_normal((N, K // 32))) * 0.01 + 1e-3) / 16).astype(np.float16)
    return torch.from_numpy(w), torch.from_numpy(s)


def write_fake_checkpoint(path, seed=0):
    rng = np.random.default_rng(seed)
    D, I, H, Hk, hd = (DIMS[k] for k in ("hidden_size", "intermediate_size", "num_heads",
                                         "num_kv_heads", "head_dim"))
    L, V = DIMS["num_layers"], DIMS["vocab"]
    shapes = {"qkv": ((H + 2 * Hk) * hd, D), "o": (D, H * hd), "gate_up": (2 * I, D),
              "down": (D, I)}
    kinds = [{"qkv": "a", "o": "a", "gate_up": "a", "down": "a"},
             {"qkv": "a", "o": "8", "gate_up": "s", "down": "8"}]
    precision_map = {}
    for li in range(L):
        ld = {}
        precision_map[str(li)] = {}
        for g, (N, K) in shapes.items():
            k = kinds[li][g]
            if k == "8":
                w, s = _int8_sym(rng, N, K)
                ld[f"{g}_weights"], ld[f"{g}_scales"] = w, s
                ld[f"{g}_precision"] = "int8"
            elif k == "s":
                p, s = _int4_sym(rng, N, K)
                ld[f"{g}_packed"], ld[f"{g}_scales"] = p, s
                ld[f"{g}_precision"] = "int4"
            else:
                p, s, z = _int4_asym(rng, N, K)
                ld[f"{g}_packed"], ld[f"{g}_scales"], ld[f"{g}_zeros"] = p, s, z
                ld[f"{g}_precision"] = "int4a"
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
    meta = dict(model_name="synthetic", num_layers=L, hidden_size=D, intermediate_size=I,
                num_heads=H, num_kv_heads=Hk, head_dim=hd, rms_eps=1e-6, rope_theta=1.0e6,
                method="v4_asym_had_gptq_c4cal", block_size=32, use_rotation=True,
                use_asymmetric=True, precision_map=precision_map)
    torch.save(meta, path / "meta.pt")
    return kinds
