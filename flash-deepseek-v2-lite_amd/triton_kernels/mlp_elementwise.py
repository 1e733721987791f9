"""SwiGLU elementwise (reference: triton_kernels/mlp_elementwise.py:24-45)."""

from __future__ import annotations

import torch

from . import _hip
from ._checks import require_contiguous, require_cuda


def silu_mul_triton(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    require_cuda("silu_mul_triton", gate, up)
    if gate.shape != up.shape:
        raise ValueError("gate and up must have the same shape")
    if gate.dtype != torch.bfloat16 or up.dtype != torch.bfloat16:
        raise NotImplementedError("silu_mul_triton supports bf16 only")
    require_contiguous("silu_mul_triton", gate, up)
    if gate.numel() % 8:
        raise ValueError("silu_mul_triton needs numel % 8 == 0")
    out = torch.empty_like(gate)
    _hip.call("dsv2_silu_mul_bf16", gate.data_ptr(), up.data_ptr(), out.data_ptr(), gate.numel(),
              _hip.stream_ptr(gate.device))
    return out
