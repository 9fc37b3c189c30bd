"""Drop-in for the reference's fused_ops module (fused_ops.py:28-215), backed
by the gfx950 kernels of librdna4q.so instead of Triton.

Same names, arguments and return shapes:
  fused_rmsnorm(x, weight, eps=1e-6)                       (fused_ops.py:28-41)
  fused_qknorm_rope_decode(q, k, q_norm_weight, k_norm_weight, cos, sin,
                           position, eps=1e-6)             (fused_ops.py:155-181)
  fused_rope_decode(q, k, cos, sin, position)              (fused_ops.py:184-215)
engine_utils.py:11-14, 58-63 picks fused_rmsnorm up when `import fused_ops`
succeeds, exactly as with the reference module.

`position` may be an int or a one-element int64 tensor; a device tensor is
read back to the host (one synchronisation), since the C ABI takes the
position by value.  head_dim must be 128 for the two RoPE functions (the
Qwen3 layout the kernels are built for); fused_rmsnorm takes any D that is
a multiple of 32.  There is no CPU fallback: inputs must be on the GPU.
"""
from __future__ import annotations

import torch

import r4q_lib as _R

__all__ = ["fused_rmsnorm", "fused_qknorm_rope_decode", "fused_rope_decode"]


def _need(cond, msg):
    if not cond:
        raise ValueError(msg)


def _pos(position) -> int:
    if isinstance(position, int):
        return position
    return int(position.reshape(-1)[0].item())


def _check_table(t, name, pos):
    _need(t.is_cuda and t.dtype == torch.float16 and t.dim() == 2 and t.shape[1] == 64
          and t.is_contiguous(), f"{name} must be a contiguous cuda float16 [P, 64] table")
    _need(0 <= pos < t.shape[0], f"position {pos} outside the RoPE table ({t.shape[0]} rows)")


def fused_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """y = fp16(x * rsqrt(mean(x^2) + eps) * weight) over the last dim."""
    _need(x.is_cuda and x.dtype == torch.float16, "x must be cuda float16")
    _need(weight.is_cuda and weight.dtype == torch.float16, "weight must be cuda float16")
    D = x.shape[-1]
    _need(weight.numel() == D, "weight must have x.shape[-1] elements")
    x2 = x.reshape(-1, D).contiguous()
    y = torch.empty_like(x2)
    _R.call("r4q_rmsnorm", x2.data_ptr(), weight.contiguous().data_ptr(), y.data_ptr(),
            x2.shape[0], D, float(eps), _R.stream_handle(x.device))
    return y.reshape(x.shape)


def fused_rope_decode(q: torch.Tensor, k: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                      position):
    """Half-split RoPE of q [1, H, 1, D] and k [1, Hk, 1, D] at one position."""
    B, H, S, D = q.shape
    _, Hk, _, _ = k.shape
    _need(B == 1 and S == 1 and D == 128, "q must be [1, H, 1, 128]")
    _need(q.dtype == torch.float16 and k.dtype == torch.float16 and q.is_cuda and k.is_cuda,
          "q and k must be cuda float16")
    pos = _pos(position)
    _check_table(cos, "cos", pos)
    _check_table(sin, "sin", pos)
    qf = q.reshape(H, D).contiguous()
    kf = k.reshape(Hk, D).contiguous()
    q_out = torch.empty_like(qf)
    k_out = torch.empty_like(kf)
    _R.call("r4q_rope", qf.data_ptr(), kf.data_ptr(), cos.data_ptr(), sin.data_ptr(),
            q_out.data_ptr(), k_out.data_ptr(), H, Hk, D, pos, _R.stream_handle(q.device))
    return q_out.reshape(B, H, S, D), k_out.reshape(B, Hk, S, D)


def fused_qknorm_rope_decode(q: torch.Tensor, k: torch.Tensor, q_norm_weight: torch.Tensor,
                             k_norm_weight: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                             position, eps: float = 1e-6):
    """Per-head RMSNorm then half-split RoPE of q [1, H, 1, D] and k
    [1, Hk, 1, D] in one launch (the decode step's kernel, no KV write)."""
    B, H, S, D = q.shape
    _, Hk, _, _ = k.shape
    _need(B == 1 and S == 1 and D == 128, "q must be [1, H, 1, 128]")
    _need(q.dtype == torch.float16 and k.dtype == torch.float16 and q.is_cuda and k.is_cuda,
          "q and k must be cuda float16")
    _need(H % Hk == 0, "H must be a multiple of Hk")
    pos = _pos(position)
    _check_table(cos, "cos", pos)
    _check_table(sin, "sin", pos)
    # the kernel reads one row laid out as q heads | k heads | v heads
    row = torch.empty((H + 2 * Hk) * D, dtype=torch.float16, device=q.device)
    row[:H * D] = q.reshape(-1)
    row[H * D:(H + Hk) * D] = k.reshape(-1)
    out = torch.empty((H + Hk) * D, dtype=torch.float16, device=q.device)
    _R.call("r4q_head_norm_rope_kv", row.data_ptr(), row.numel(),
            q_norm_weight.contiguous().data_ptr(), k_norm_weight.contiguous().data_ptr(),
            out.data_ptr(), out.numel(), None, None, None, None, cos.data_ptr(), sin.data_ptr(),
            1, H, Hk, D, float(eps), 0, pos, _R.stream_handle(q.device))
    return out[:H * D].reshape(B, H, S, D), out[H * D:].reshape(B, Hk, S, D)
