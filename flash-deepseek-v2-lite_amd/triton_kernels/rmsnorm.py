"""RMSNorm (reference: triton_kernels/rmsnorm.py:60-95)."""

from __future__ import annotations

import torch

from . import _hip
from ._checks import require_contiguous, require_cuda, require_dtype


def rmsnorm_triton(hidden_states: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """y = w * bf16(x * rsqrt(mean(x^2) + eps)) over the last dim; bf16 in/out."""
    require_cuda("rmsnorm_triton", hidden_states, weight)
    require_dtype("rmsnorm_triton", hidden_states, torch.bfloat16)
    require_dtype("rmsnorm_triton", weight, torch.bfloat16)
    require_contiguous("rmsnorm_triton", weight)
    n = int(hidden_states.shape[-1])
    if weight.shape != (n,):
        raise ValueError(f"weight shape {tuple(weight.shape)} != ({n},)")
    x = hidden_states.reshape(-1, n)
    if x.stride(1) != 1:
        raise NotImplementedError("rmsnorm_triton requires last dimension to be contiguous")
    y = torch.empty((x.shape[0], n), device=x.device, dtype=x.dtype)
    _hip.call("dsv2_rmsnorm_bf16", x.data_ptr(), x.stride(0), weight.data_ptr(), y.data_ptr(), n, x.shape[0], n,
              float(eps), _hip.stream_ptr(x.device))
    return y.reshape(hidden_states.shape)
