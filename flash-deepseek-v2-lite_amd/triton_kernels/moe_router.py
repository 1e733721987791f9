"""Router softmax + top-6 (reference: triton_kernels/moe_router.py:63-86)."""

from __future__ import annotations

import torch

from . import _hip
from ._checks import require_contiguous, require_cuda


def router_softmax_topk6_triton(logits: torch.Tensor, scaling: float) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 logits [B, 64] -> (ids int64 [B, 6] in descending score order, ties to the
    lower index; weights fp32 [B, 6] = score * scaling).  Any B (the reference: B=1)."""
    require_cuda("router_softmax_topk6_triton", logits)
    if logits.dtype != torch.float32:
        raise NotImplementedError("router_softmax_topk6_triton expects fp32 logits")
    if logits.ndim != 2 or logits.shape[1] != 64:
        raise NotImplementedError("router_softmax_topk6_triton is specialized for [B, 64] logits")
    require_contiguous("router_softmax_topk6_triton", logits)
    B = logits.shape[0]
    ids = torch.empty((B, 6), device=logits.device, dtype=torch.long)
    w = torch.empty((B, 6), device=logits.device, dtype=torch.float32)
    _hip.call("dsv2_router_topk6_from_logits", logits.data_ptr(), B, float(scaling), None, ids.data_ptr(),
              w.data_ptr(), _hip.stream_ptr(logits.device))
    return ids, w


def router_topk6_fused(hidden_states: torch.Tensor, norm_weight: torch.Tensor, eps: float,
                       router_weight: torch.Tensor, scaling: float):
    """post-attention RMSNorm + router logits + softmax + top-6 in one kernel
    (replaces _graph_gate_forward, src/run.py:257-275).  Returns (xn, ids int64, weights)."""
    require_cuda("router_topk6_fused", hidden_states, norm_weight, router_weight)
    x = hidden_states.reshape(-1, 2048)
    if x.dtype != torch.bfloat16 or router_weight.dtype != torch.bfloat16 or router_weight.shape != (64, 2048):
        raise NotImplementedError("router_topk6_fused expects bf16 [B, 2048] and bf16 [64, 2048]")
    require_contiguous("router_topk6_fused", x, norm_weight, router_weight)
    B = x.shape[0]
    xn = torch.empty_like(x)
    ids = torch.empty((B, 6), device=x.device, dtype=torch.long)
    w = torch.empty((B, 6), device=x.device, dtype=torch.float32)
    _hip.call("dsv2_router_topk6", x.data_ptr(), 2048, norm_weight.data_ptr(), float(eps), router_weight.data_ptr(),
              float(scaling), B, xn.data_ptr(), None, ids.data_ptr(), w.data_ptr(), _hip.stream_ptr(x.device))
    return xn, ids, w
