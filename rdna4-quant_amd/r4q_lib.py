"""ctypes binding of librdna4q.so (the C ABI declared in include/r4q.h).

torch is imported first on purpose: torch ships its own libamdhip64.so.7 and
the library must bind to that same HIP runtime instance (both carry the
soname libamdhip64.so.7, so the dynamic loader reuses the loaded copy).
There is no fallback: if the shared library is missing, loading fails loudly.
"""
from __future__ import annotations

import ctypes as C
import os

import torch  # noqa: F401  (must precede loading the HIP library)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librdna4q.so")

R4Q_OK = 0
R4Q_EINVAL = -1
R4Q_EUNSUPPORTED = -2
R4Q_EHIP = -3
R4Q_ENOMEM = -4

_p = C.c_void_p
_i64 = C.c_int64
_i32 = C.c_int32
_f32 = C.c_float
_fp = C.POINTER(C.c_float)


class R4QLayer(C.Structure):
    """Mirror of `struct r4q_layer` (include/r4q.h)."""
    _fields_ = [
        ("qkv_w", _p), ("qkv_s", _p), ("qkv_N", _i64), ("qkv_bits", _i32),
        ("o_w", _p), ("o_s", _p), ("o_N", _i64), ("o_bits", _i32),
        ("gu_w", _p), ("gu_s", _p), ("gu_N", _i64), ("gu_bits", _i32),
        ("down_w", _p), ("down_s", _p), ("down_N", _i64), ("down_bits", _i32),
        ("in_norm", _p), ("post_norm", _p), ("q_norm", _p), ("k_norm", _p),
        ("k_cache", _p), ("v_cache", _p),
        ("k_scale", _p), ("v_scale", _p),
    ]


class R4QModel(C.Structure):
    """Mirror of `struct r4q_model` (include/r4q.h)."""
    _fields_ = [
        ("n_layers", _i32), ("n_heads", _i32), ("n_kv_heads", _i32), ("head_dim", _i32),
        ("hidden", _i32), ("inter", _i32),
        ("eps", _f32),
        ("max_seq", _i32), ("rope_len", _i32),
        ("layers", C.POINTER(R4QLayer)),
        ("rope_cos", _p), ("rope_sin", _p),
        ("final_norm", _p),
        ("lm_w", _p), ("lm_s", _p), ("lm_N", _i64), ("lm_K", _i64), ("lm_bits", _i32),
        ("embed", _p),
        ("vocab", _i64),
    ]


# name -> argtypes (restype is int for all but r4q_last_error)
SIGNATURES = {
    "r4q_abi_version": [],
    "r4q_dequant_int4": [_p, _p, _p, _i64, _i64, _p],
    "r4q_dequant_int8": [_p, _p, _p, _i64, _i64, _p],
    "r4q_fp16_to_fp8": [_p, _p, _i64, _p],
    "r4q_fp8_to_fp16": [_p, _p, _i64, _p],
    "r4q_gemv": [_p, _p, _p, _p, _i64, _i64, C.c_int, _p],
    "r4q_gemm": [_p, _p, _p, _p, _i64, _i64, _i64, C.c_int, _p],
    "r4q_prefill_attention": [_p, _i64, _p, _i64, _i64, _i64, _i64, _p],
    "r4q_gemm_workspace_bytes": [_i64, _i64, _i64, C.c_int, C.POINTER(C.c_size_t)],
    "r4q_gemm_ws": [_p, _p, _p, _p, _i64, _i64, _i64, C.c_int, _p, C.c_size_t, _p],
    "r4q_gemm_silu_fwht_ws": [_p, _p, _p, _p, _i64, _i64, _i64, C.c_int, _p, C.c_size_t, _p],
    "r4q_rmsnorm": [_p, _p, _p, _i64, _i64, _f32, _p],
    "r4q_res_rmsnorm": [_p, _p, _p, _p, _p, _i64, _i64, _f32, _p],
    "r4q_rmsnorm_fwht": [_p, _p, _p, _i64, _i64, _f32, _p],
    "r4q_res_rmsnorm_fwht": [_p, _p, _p, _p, _p, _i64, _i64, _f32, _p],
    "r4q_fwht32": [_p, _p, _i64, _p],
    "r4q_hbm_read": [_p, _i64, _p, _i64, _p],
    "r4q_tune": [C.c_char_p, C.c_int],
    "r4q_silu_mul_fwht": [_p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "r4q_silu_mul": [_p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "r4q_head_rmsnorm": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _f32, _p],
    "r4q_rope": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p],
    "r4q_head_norm_rope_kv": [_p, _i64, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _p,
                              _i64, _i64, _i64, _i64, _f32, _i64, _i64, _p],
    "r4q_res_rmsnorm_fwht_gemv": [_p, _p, _p, _p, _f32, _p, _p, _p, _i64, _i64, C.c_int, _p],
    "r4q_gate_up_silu_fwht": [_p, _p, _p, _p, _f32, _p, _p, _p, _i64, _i64, C.c_int, _p],
    "r4q_gate_up_silu_split": [_i64, C.POINTER(_i64)],
    "r4q_gate_up_silu": [_p, _p, _p, _p, _f32, _p, _p, _p, _p, _i64, _i64, _i64, C.c_int, _p],
    "r4q_fwht_gemv": [_p, _p, _i64, _p, _p, _p, _i64, _i64, C.c_int, _p],
    "r4q_ctx_create": [C.POINTER(_p)],
    "r4q_ctx_destroy": [_p],
    "r4q_flash_decode": [_p, _p, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                         _i64, C.c_int, _p],
    "r4q_flash_decode_noalloc": [_p, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64,
                                 _i64, C.c_int, _p],
    "r4q_flash_decode_qkv": [_p, _p, _i64, _p, _p, _p, _p, _f32, _p, _p, _p, _p, _p, _i64,
                             _i64, _i64, _i64, _i64, _i64, _i64, C.c_int, _p],
    "r4q_decode_step": [_p, C.POINTER(R4QModel), _p, _i64, _i64, _p, _p, _p],
    "r4q_decode_plan": [C.POINTER(R4QModel), _i64, C.POINTER(_i32), _i64],
    "r4q_decode_step_graph": [_p, C.POINTER(R4QModel), _p, _i64, _i64, _p, _p, _p],
    "r4q_decode_bench": [_p, C.POINTER(R4QModel), _p, _i64, _i64, _i64, C.c_int, _p, _p],
    "r4q_decode_generate": [_p, C.POINTER(R4QModel), _p, _i64, _i64, _i64, C.c_int, _f32, _f32,
                            C.c_uint64, _p, _p],
    "r4q_sample": [_p, _p, _i64, _i64, _i64, _f32, _f32, C.c_uint64, _i64, _p, _p],
    "r4q_decode_profile": [_p, C.POINTER(R4QModel), _p, _i64, _fp, _p],
    "r4q_prefill_logits": [_p, C.POINTER(R4QModel), _p, _i64, _p, C.c_int, _p],
}

_lib = None


def lib() -> C.CDLL:
    """Loads librdna4q.so once; raises ImportError if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `make -C {HERE}` "
                "(or __graft_entry__.build()); there is no non-HIP fallback")
        L = C.CDLL(LIB_PATH)
        L.r4q_last_error.restype = C.c_char_p
        L.r4q_last_error.argtypes = []
        for name, args in SIGNATURES.items():
            fn = getattr(L, name, None)
            if fn is None:
                continue  # reported by exported_symbols()/tests
            fn.restype = C.c_int
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    """Names of SIGNATURES entries present in the loaded library."""
    L = lib()
    return [n for n in SIGNATURES if hasattr(L, n)]


def last_error() -> str:
    return lib().r4q_last_error().decode(errors="replace")


def check(rc: int, what: str = "") -> None:
    """Raises RuntimeError for a non-zero ABI status."""
    if rc != R4Q_OK:
        raise RuntimeError(f"librdna4q{(' ' + what) if what else ''}: status {rc}: {last_error()}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


def tune(name: str, value: int) -> None:
    """Process-wide launch-shape override (r4q_tune); 0 restores the default."""
    call("r4q_tune", name.encode(), int(value))


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device=None) -> int:
    """Raw hipStream_t of torch's current stream (torch's raw accessor when it
    has one: a Stream object per call cost ~10 us on the decode path)."""
    if _raw_stream is not None:
        idx = None
        if device is not None:
            idx = device if isinstance(device, int) else torch.device(device).index
        return _raw_stream(torch.cuda.current_device() if idx is None else idx)
    return torch.cuda.current_stream(device).cuda_stream
