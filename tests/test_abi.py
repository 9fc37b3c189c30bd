"""C-ABI checks that need no GPU: the library loads, exports every entry
point include/r4q.h declares, the ctypes table matches the header, and
argument validation rejects bad requests before any device work."""
import ctypes as C
import re
from pathlib import Path

import pytest
import torch

import r4q_lib as R

HEADER = Path(__file__).resolve().parents[1] / "include" / "r4q.h"


def header_functions():
    txt = HEADER.read_text()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(r4q_[a-z0-9_]+)\s*\(", txt)))


def test_library_loads_and_exports_every_header_symbol():
    L = R.lib()
    names = header_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, f"declared in r4q.h but not exported: {missing}"
    assert L.r4q_abi_version() == 1


def test_ctypes_table_covers_header():
    names = set(header_functions()) - {"r4q_last_error"}
    assert names == set(R.SIGNATURES), names ^ set(R.SIGNATURES)


def _einval(rc):
    assert rc == R.R4Q_EINVAL, rc
    assert R.last_error()


def test_gemv_rejects_bad_arguments():
    L = R.lib()
    p = C.c_void_p(256)  # never dereferenced: validation fails first
    _einval(L.r4q_gemv(p, p, p, p, 16, 33, 4, None))       # K % 32
    _einval(L.r4q_gemv(p, p, p, p, 16, 64, 5, None))       # wbits
    _einval(L.r4q_gemv(None, p, p, p, 16, 64, 4, None))    # null x
    _einval(L.r4q_gemv(p, p, None, p, 16, 64, 4, None))    # null sz for INT4
    _einval(L.r4q_gemv(p, p, p, p, 0, 64, 4, None))        # N == 0
    _einval(L.r4q_gemv(C.c_void_p(258), p, p, p, 16, 64, 4, None))  # misaligned x
    assert "wbits" in (L.r4q_gemv(p, p, p, p, 16, 64, 3, None) and R.last_error())


def test_codec_rejects_bad_arguments():
    L = R.lib()
    p = C.c_void_p(256)
    _einval(L.r4q_dequant_int4(p, p, p, 4, 48, None))
    _einval(L.r4q_dequant_int8(p, None, p, 4, 64, None))
    _einval(L.r4q_fp16_to_fp8(None, p, 16, None))
    assert L.r4q_fp16_to_fp8(None, None, 0, None) == R.R4Q_OK  # empty is a no-op


def test_norm_and_attention_reject_bad_arguments():
    L = R.lib()
    p = C.c_void_p(256)
    _einval(L.r4q_rmsnorm_fwht(p, p, p, 1, 100, C.c_float(1e-6), None))   # D % 32
    _einval(L.r4q_fwht32(p, p, 31, None))
    _einval(L.r4q_head_norm_rope_kv(p, 7168, p, p, p, 7168, p, p, None, None, p, p,
                                    1, 40, 8, 64, C.c_float(1e-6), 16, 3, None))  # D != 128
    _einval(L.r4q_head_norm_rope_kv(p, 7168, p, p, p, 7168, p, p, None, None, p, p,
                                    1, 40, 8, 128, C.c_float(1e-6), 16, 16, None))  # pos >= max_seq
    _einval(L.r4q_flash_decode(None, p, 5120, p, p, None, None, p, 1, 40, 8, 128, 16, 4, 1, None))


def test_weight_bits_inference():
    import int4_hip
    assert int4_hip.weight_bits(torch.empty(4, 32, dtype=torch.uint8), 64) == 4
    assert int4_hip.weight_bits(torch.empty(4, 64, dtype=torch.uint8), 64) == 8
    assert int4_hip.weight_bits(torch.empty(4, 64, dtype=torch.float16), 64) == 16
    with pytest.raises(ValueError):
        int4_hip.weight_bits(torch.empty(4, 48, dtype=torch.uint8), 64)
    with pytest.raises(ValueError):
        int4_hip.weight_bits(torch.empty(4, 64, dtype=torch.float32), 64)


def test_check_raises_runtime_error():
    with pytest.raises(RuntimeError):
        R.check(R.R4Q_EINVAL, "probe")


def test_fused_ops_surface_matches_reference_signatures():
    """fused_ops.py:28, 155, 184: names and parameter lists."""
    import inspect
    import fused_ops
    sig = {n: list(inspect.signature(getattr(fused_ops, n)).parameters)
           for n in ("fused_rmsnorm", "fused_qknorm_rope_decode", "fused_rope_decode")}
    assert sig["fused_rmsnorm"] == ["x", "weight", "eps"]
    assert sig["fused_qknorm_rope_decode"] == ["q", "k", "q_norm_weight", "k_norm_weight", "cos",
                                               "sin", "position", "eps"]
    assert sig["fused_rope_decode"] == ["q", "k", "cos", "sin", "position"]


def test_gemm_workspace_sizes():
    """Host-side split policy: the skinny GEMM (2-16 rows) asks for S * M * N
    fp32 of partials where splitting K evens the per-CU load (the Qwen3-14B
    projections at M = 8 take the split counts measured fastest); the FP16 LM
    head (2374 tiles, over 8 workgroups per CU once split), one row, and
    shapes off the ring's K step ask for none; M >= 256 follows the tiled
    GEMM's plan: stream-K partials when the 256 x 256 tiles leave CUs idle,
    none when the tiles fill their rounds of 256 workgroups to 7/8 or more
    (the FP16 LM head of a 512-token prompt: 1188 tiles in 5 rounds)."""
    def ws(M, N, K, bits):
        b = C.c_size_t(123)
        R.call("r4q_gemm_workspace_bytes", M, N, K, bits, C.byref(b))
        return b.value
    for bits in (4, 8):
        for (N, K, splits) in ((5120, 17408, 3), (5120, 5120, 3), (7168, 5120, 2),
                               (34816, 5120, 3)):  # down, o, qkv, gate_up
            assert ws(8, N, K, bits) == splits * 8 * N * 4, (bits, N, K)
    assert ws(8, 151936, 5120, 16) == 0               # LM head
    assert ws(1, 5120, 17408, 4) == 0                 # batch 1: GEMV, no workspace
    assert ws(8, 5120, 17408 + 32, 4) == 0            # K off the ring step: per-row path
    assert ws(512, 5120, 17408, 4) > 0                # tiled GEMM, split along K
    assert ws(512, 17408, 5120, 16) > 0               # FP16 weights: the same ring
    assert ws(512, 151936, 5120, 16) == 0             # 1188 tiles: whole tiles
    assert ws(2304, 16384, 768, 8) > 0                # 576 tiles: 2 rounds + stream-K
    with pytest.raises(RuntimeError):
        ws(8, 5120, 100, 4)                           # K % 32 != 0


def test_gate_up_silu_split_point():
    """Whole 64-row units in multiples of 256 (the CU count), the rest as
    fp32 pairs; fewer than 256 units: all units."""
    def split(I):
        v = C.c_int64(-1)
        R.call("r4q_gate_up_silu_split", I, C.byref(v))
        return v.value
    assert split(17408) == 16384
    assert split(8448) == 8192
    assert split(1024) == 1024
    assert split(96) == 96
    with pytest.raises(RuntimeError):
        split(100)


def test_model_cache_key_follows_storage_swaps():
    # A tensor whose storage is swapped in place keeps its id(); the model
    # cache key must still change (a stale key would point the kernels at
    # the old storage).  Host-only: keys are built without device work.
    import int4_hip
    ws = [torch.zeros(8, dtype=torch.uint8) for _ in range(3)]
    kc = [torch.zeros(1, 2, 16, 4, dtype=torch.uint8) for _ in range(3)]
    args = [ws, [1, 2, 3], kc, 0.5]
    k0 = int4_hip._key_of(args, shaped=(2,))
    assert int4_hip._key_of(args, shaped=(2,)) == k0
    ws[1].set_(torch.zeros(8, dtype=torch.uint8))  # new storage, same tensor object
    k1 = int4_hip._key_of(args, shaped=(2,))
    assert k1 != k0
    kc[0].resize_(1, 2, 8, 4)  # shrinks in place: same pointer, other capacity
    assert int4_hip._key_of(args, shaped=(2,)) != k1
    # None entries (FP16 weights carry no scale table) are keyed too
    kn = int4_hip._key_of([[None, ws[0]]])
    assert kn == int4_hip._key_of([[None, ws[0]]])
    ws[0].set_(torch.zeros(8, dtype=torch.uint8))
    assert int4_hip._key_of([[None, ws[0]]]) != kn


# (name, lowest, highest, power of two only) as include/r4q.h documents r4q_tune
KNOBS = [("gemv_lpr", 16, 256, True), ("gemv_wgs", 1, 65536, False), ("gemv_ub", 1, 2, False),
         ("attn_splits", 1, 128, False), ("skinny_splits", 1, 8, False),
         ("gemm_splits", 1, 16, False), ("split_reduce", 1, 1, False),
         ("gemm_kernel", 1, 2, False), ("gemv_skew", 1, 8, False)]


def test_tune_accepts_documented_knobs_and_rejects_the_rest():
    L = R.lib()
    try:
        for name, lo, hi, pow2 in KNOBS:
            n = name.encode()
            assert L.r4q_tune(n, lo) == R.R4Q_OK, name
            assert L.r4q_tune(n, hi) == R.R4Q_OK, name
            _einval(L.r4q_tune(n, lo - 1 if lo > 1 else -1))
            _einval(L.r4q_tune(n, hi + 1))
            if pow2:
                _einval(L.r4q_tune(n, lo + 1))
            assert L.r4q_tune(n, 0) == R.R4Q_OK, name  # back to the built-in choice
        _einval(L.r4q_tune(b"no_such_knob", 1))
        _einval(L.r4q_tune(None, 1))
    finally:
        for name, *_ in KNOBS:
            L.r4q_tune(name.encode(), 0)
