"""Routed MoE, batch family: deterministic expert bucketing + expert-grouped
gate_up/SwiGLU and down on bf16 MFMA + fixed-order top-6 combine
(reference: triton_kernels/moe_batch.py:12-30, 324-422, 660-683).

There is no eager/CPU fallback: non-HIP tensors raise NotImplementedError.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _hip
from ._checks import require_cuda


@dataclass
class PackedRoutedExperts:
    # gate_up_weights: [num_experts, 2 * intermediate_size, hidden_size] (per expert [gate; up])
    # down_weights:    [num_experts, hidden_size, intermediate_size]
    gate_up_weights: torch.Tensor
    down_weights: torch.Tensor
    hidden_size: int
    intermediate_size: int
    num_experts: int
    topk: int

    def to(self, *args, **kwargs) -> "PackedRoutedExperts":
        self.gate_up_weights = self.gate_up_weights.to(*args, **kwargs)
        self.down_weights = self.down_weights.to(*args, **kwargs)
        return self


def pack_routed_experts(moe: torch.nn.Module, device: torch.device | str | None = None) -> PackedRoutedExperts:
    """Pack the routed experts of an HF DeepSeek-V2 MoE module.

    Accepts the remote-code layout (``moe.experts`` = list of MLPs with
    gate_proj/up_proj/down_proj) and transformers' native layout
    (``moe.experts.gate_up_proj`` [E, 2I, H], ``moe.experts.down_proj`` [E, H, I])."""
    if getattr(moe, "ep_size", 1) != 1:
        raise NotImplementedError("pack_routed_experts currently only supports ep_size == 1")
    topk = int(getattr(moe, "num_experts_per_tok", None) or getattr(moe.gate, "top_k"))
    ex = moe.experts
    if hasattr(ex, "gate_up_proj"):
        gu = ex.gate_up_proj.detach()
        dn = ex.down_proj.detach()
        device = gu.device if device is None else device
        gu = gu.to(device).contiguous()
        dn = dn.to(device).contiguous()
        E, I2, H = gu.shape
        return PackedRoutedExperts(gu, dn, int(H), int(I2 // 2), int(E), topk)
    experts = [e for e in ex if e is not None]
    if not experts:
        raise ValueError("No local routed experts found to pack")
    first = experts[0]
    device = first.gate_proj.weight.device if device is None else device
    I, H = first.gate_proj.weight.shape
    gu = torch.empty((len(experts), 2 * I, H), device=device, dtype=first.gate_proj.weight.dtype)
    dn = torch.empty((len(experts), H, I), device=device, dtype=first.gate_proj.weight.dtype)
    for i, e in enumerate(experts):
        gu[i, :I].copy_(e.gate_proj.weight)
        gu[i, I:].copy_(e.up_proj.weight)
        dn[i].copy_(e.down_proj.weight)
    return PackedRoutedExperts(gu, dn, int(H), int(I), len(experts), topk)


def _check(name: str, x, topk_ids, topk_weight, packed) -> None:
    if x.ndim != 2 or topk_ids.ndim != 2 or topk_weight.ndim != 2:
        raise ValueError(f"{name} expects x=[B,H], topk tensors=[B,topk]")
    if topk_ids.shape != topk_weight.shape or topk_ids.shape[0] != x.shape[0]:
        raise ValueError("topk_ids/topk_weight must have shape [B, topk]")
    if topk_ids.shape[1] != packed.topk:
        raise ValueError(f"Expected topk={packed.topk}, got {topk_ids.shape[1]}")
    require_cuda(name, x, topk_ids, topk_weight)
    if packed.topk != 6 or packed.num_experts != 64 or packed.hidden_size != 2048 or x.shape[1] != 2048:
        raise NotImplementedError(f"{name} is specialised to 64 experts, top-6, hidden 2048")
    if x.dtype != torch.bfloat16 or packed.gate_up_weights.dtype != torch.bfloat16:
        raise NotImplementedError(f"{name} supports bf16 only")
    if packed.intermediate_size % 64:
        raise NotImplementedError(f"{name} needs intermediate_size % 64 == 0")
    if packed.gate_up_weights.device != x.device or packed.down_weights.device != x.device:
        packed.to(device=x.device)


def batched_grouped_routed_moe_grouped_triton(x: torch.Tensor, topk_ids: torch.Tensor, topk_weight: torch.Tensor,
                                              packed: PackedRoutedExperts,
                                              output_dtype: torch.dtype | None = None) -> torch.Tensor:
    """out[b] = bf16(sum_s w[b,s] * bf16(expert_{ids[b,s]}(x[b])))  (fixed slot order)."""
    _check("batched_grouped_routed_moe", x, topk_ids, topk_weight, packed)
    if output_dtype not in (None, torch.bfloat16):
        raise NotImplementedError("output_dtype must be bf16")
    x = x.contiguous()
    ids = topk_ids.to(torch.int32).contiguous()
    w = topk_weight.to(torch.float32).contiguous()
    B, I = x.shape[0], packed.intermediate_size
    R = B * 6
    if R > 49152:
        raise ValueError("batched_grouped_routed_moe supports at most 8192 tokens per call")
    dev = x.device
    avg = R / 64
    tile = 16 if avg <= 6 else (32 if avg <= 16 else 64)
    max_tiles = math.ceil(R / tile) + 64
    sorted_routes = torch.empty(R, dtype=torch.int32, device=dev)
    route_pos = torch.empty(R, dtype=torch.int32, device=dev)
    tiles = torch.empty(max_tiles, 4, dtype=torch.int32, device=dev)
    ntiles = torch.empty(1, dtype=torch.int32, device=dev)
    hs = torch.empty(R, I, dtype=torch.bfloat16, device=dev)
    ys = torch.empty(R, 2048, dtype=torch.bfloat16, device=dev)
    out = torch.empty(B, 2048, dtype=torch.bfloat16, device=dev)
    st = _hip.stream_ptr(dev)
    _hip.call("dsv2_moe_bucket", ids.data_ptr(), B, tile, sorted_routes.data_ptr(), route_pos.data_ptr(),
              tiles.data_ptr(), ntiles.data_ptr(), st)
    _hip.call("dsv2_moe_grouped_gateup", x.data_ptr(), sorted_routes.data_ptr(), tiles.data_ptr(), ntiles.data_ptr(),
              max_tiles, tile, packed.gate_up_weights.data_ptr(), I, hs.data_ptr(), st)
    _hip.call("dsv2_moe_grouped_down", hs.data_ptr(), tiles.data_ptr(), ntiles.data_ptr(), max_tiles, tile,
              packed.down_weights.data_ptr(), I, ys.data_ptr(), st)
    _hip.call("dsv2_moe_combine", ys.data_ptr(), route_pos.data_ptr(), w.data_ptr(), B, None, None, out.data_ptr(),
              None, 0.0, None, st)
    return out


def batched_grouped_routed_moe(x, topk_ids, topk_weight, packed, output_dtype=None) -> torch.Tensor:
    return batched_grouped_routed_moe_grouped_triton(x, topk_ids, topk_weight, packed, output_dtype)


def packed_routed_moe_eager(x: torch.Tensor, topk_ids: torch.Tensor, topk_weight: torch.Tensor,
                            packed: PackedRoutedExperts) -> torch.Tensor:
    """The reference's per-expert loop (moe_batch.py:366-387): fp32 weighted sum of the
    bf16 expert outputs, one cast to x.dtype.  Kept as a name for its callers; there is no
    eager path here, it runs the same HIP grouped kernels as packed_routed_moe (same math:
    SwiGLU, bf16 expert output, fp32 slot-order sum)."""
    return batched_grouped_routed_moe(x, topk_ids, topk_weight, packed)


def packed_routed_moe(x: torch.Tensor, topk_ids: torch.Tensor, topk_weight: torch.Tensor,
                      packed: PackedRoutedExperts, output_dtype: torch.dtype | None = None) -> torch.Tensor:
    return batched_grouped_routed_moe(x, topk_ids, topk_weight, packed, output_dtype=output_dtype)
