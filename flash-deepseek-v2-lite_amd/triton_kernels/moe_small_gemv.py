"""Routed MoE, small family: route-local GEMV (reference:
triton_kernels/moe_small_gemv.py:430-614).  Gate and up rows are paired by
index (row i of gate with row i of up), the packing of pack_routed_experts."""

from __future__ import annotations

import torch

from . import _hip
from .moe_batch import PackedRoutedExperts, _check, pack_routed_experts, packed_routed_moe_eager  # noqa: F401


def batched_grouped_routed_moe_route_gemv(x: torch.Tensor, topk_ids: torch.Tensor, topk_weight: torch.Tensor,
                                          packed: PackedRoutedExperts,
                                          output_dtype: torch.dtype | None = None) -> torch.Tensor:
    """Per token and route: gate_up+SwiGLU GEMV then down GEMV; fixed-order weighted
    top-6 sum inside one workgroup (no atomics, no fp32 partial buffer)."""
    _check("batched_grouped_routed_moe_route_gemv", x, topk_ids, topk_weight, packed)
    if output_dtype not in (None, torch.bfloat16):
        raise NotImplementedError("output_dtype must be bf16")
    x = x.contiguous()
    ids = topk_ids.to(torch.int32).contiguous()
    w = topk_weight.to(torch.float32).contiguous()
    B, I = x.shape[0], packed.intermediate_size
    hbuf = torch.empty(B, 6, I, dtype=torch.bfloat16, device=x.device)
    out = torch.empty(B, 2048, dtype=torch.bfloat16, device=x.device)
    st = _hip.stream_ptr(x.device)
    _hip.call("dsv2_moe_route_gateup", x.data_ptr(), B, ids.data_ptr(), packed.gate_up_weights.data_ptr(), None, I,
              hbuf.data_ptr(), st)
    _hip.call("dsv2_moe_route_down", hbuf.data_ptr(), B, ids.data_ptr(), w.data_ptr(), packed.down_weights.data_ptr(),
              None, I, 6, None, None, out.data_ptr(), st)
    return out


def grouped_routed_moe(x: torch.Tensor, topk_ids: torch.Tensor, topk_weight: torch.Tensor,
                       packed: PackedRoutedExperts, output_dtype: torch.dtype | None = None) -> torch.Tensor:
    if x.ndim != 2 or x.shape[0] != 1:
        raise NotImplementedError("grouped_routed_moe only supports single-token decode")
    if topk_ids.ndim != 2 or topk_ids.shape[0] != 1:
        raise NotImplementedError("topk_ids must have shape [1, topk]")
    return batched_grouped_routed_moe_route_gemv(x, topk_ids, topk_weight, packed, output_dtype)
