"""Absorbed-MLA decode attention, batch family (reference:
triton_kernels/attention_decode_batch.py:25-35, 214-237, 672-846).

Documented deviation from the reference interface: ``key_cache`` is the
COMPRESSED cache [B, L, 576] bf16 (kv-normalised latent | rotated k_pe) and
``value_cache`` must be None -- the reference caches expanded per-head K/V
[B, 16, L, 192] / [B, 16, L, 128].  Row b's new token is written at
``cache_position`` and attends positions 0..cache_position (src/run.py:196-202).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _hip
from ._checks import require_contiguous, require_cuda

NH, NOPE, ROPE, VD, LAT, HID = 16, 128, 64, 128, 512, 2048
QKVA = NH * (NOPE + ROPE) + LAT + ROPE  # 3648
ROW = LAT + ROPE  # 576


@dataclass
class AttentionPackedWeights:
    w_qkva: torch.Tensor        # [3648, 2048] = cat(q_proj, kv_a_proj_with_mqa)
    kv_norm_weight: torch.Tensor  # [512]
    kv_norm_eps: float
    w_uk: torch.Tensor          # [16, 128, 512]
    w_ukt: torch.Tensor         # [16, 512, 128]
    w_uv: torch.Tensor          # [16, 128, 512]
    w_o: torch.Tensor           # [2048, 2048]


def pack_attention_weights(attn: torch.nn.Module) -> AttentionPackedWeights:
    """Pack an HF DeepseekV2Attention (q_lora_rank=None) for the HIP kernels."""
    if getattr(attn, "q_lora_rank", None) is not None:
        raise NotImplementedError("pack_attention_weights supports q_lora_rank=None (DeepSeek-V2-Lite)")
    q = attn.q_proj.weight.detach()
    kva = attn.kv_a_proj_with_mqa.weight.detach()
    kvb = attn.kv_b_proj.weight.detach().reshape(NH, NOPE + VD, LAT)
    ln = attn.kv_a_layernorm
    eps = float(getattr(ln, "variance_epsilon", getattr(ln, "eps", 1e-6)))
    w_uk = kvb[:, :NOPE].contiguous()
    return AttentionPackedWeights(torch.cat((q, kva)).contiguous(), ln.weight.detach().contiguous(), eps, w_uk,
                                  w_uk.transpose(1, 2).contiguous(), kvb[:, NOPE:].contiguous(),
                                  attn.o_proj.weight.detach().contiguous())


def plan_splits(rows: int, max_ctx: int, target_wgs: int = 256) -> tuple[int, int]:
    """(split_tokens, max_splits) for the split-KV decode: about target_wgs workgroups,
    split_tokens a multiple of 32, at most 64 splits per row.  256 = one workgroup per CU;
    each streams its split with two tiles in flight.  Measured on MI355X over the whole
    decode step against 512: bsz=256 x 2048-token prompts 22.72k vs 22.44k tok/s, bsz=64 x
    U[256,1024] 8.80k vs 8.70k, reference workload 52.6k vs 51.3k (bsz=256) and 22.0k vs
    22.0k (bsz=64); 128 (8.55k at bsz=64) and 1024 (bsz=256 x 2098 tokens: 118 vs 109 us per
    layer) are slower.  Rows of very unequal lengths want more, shorter splits (bsz=128 x
    U[256,8192]: 512 -> 2048-token splits 132 us, 256 -> 4064-token splits 171 us); capping
    the split at 2048 tokens instead cost the equal-length bsz=256 step 8%."""
    per_row = max(1, min(64, math.ceil(target_wgs / max(rows, 1))))
    split = max(32, math.ceil(math.ceil(max_ctx / per_row) / 32) * 32)
    split = max(split, math.ceil(max_ctx / 64 / 32) * 32)
    return split, math.ceil(max_ctx / split)


def _attention_decode(family: str, hidden_states, cos, sin, position_ids, cache_position, key_cache, value_cache,
                      packed: AttentionPackedWeights, softmax_scale: float) -> torch.Tensor:
    name = f"attention_decode[{family}]"
    require_cuda(name, hidden_states, cos, sin, cache_position, key_cache)
    if hidden_states.dtype != torch.bfloat16 or key_cache.dtype != torch.bfloat16:
        raise NotImplementedError(f"{name} supports bf16 only")
    if hidden_states.ndim != 3 or hidden_states.shape[1] != 1 or hidden_states.shape[2] != HID:
        raise ValueError(f"{name} expects hidden_states [B, 1, 2048]")
    B = hidden_states.shape[0]
    if value_cache is not None:
        raise ValueError(f"{name} reads the compressed cache only; pass value_cache=None")
    if key_cache.ndim != 3 or key_cache.shape[0] != B or key_cache.shape[2] != ROW:
        raise ValueError(f"{name} expects key_cache [B, L, 576] (compressed)")
    if cos.dtype != torch.bfloat16 or sin.dtype != torch.bfloat16 or cos.shape[-1] != ROPE or cos.shape != sin.shape:
        raise ValueError(f"{name} expects bf16 cos/sin tables [L, 64]")
    if cache_position.numel() != 1 or cache_position.dtype != torch.long:
        raise ValueError("cache_position must be an int64 tensor with one element")
    require_contiguous(name, key_cache, cos, sin)
    dev = hidden_states.device
    L = key_cache.shape[1]
    cos2, sin2 = cos.reshape(-1, ROPE), sin.reshape(-1, ROPE)
    max_pos = min(cos2.shape[0], L)
    x = hidden_states.reshape(B, HID).contiguous()
    pos = torch.empty(B, dtype=torch.int32, device=dev)
    base = torch.empty(B, dtype=torch.int64, device=dev)
    qkva = torch.empty(B, QKVA, dtype=torch.bfloat16, device=dev)
    q = torch.empty(B, NH, ROW, dtype=torch.bfloat16, device=dev)
    split, nsplit = plan_splits(B, L)
    part_o = torch.empty(B, nsplit, NH, LAT, dtype=torch.float32, device=dev)
    part_ml = torch.empty(B, nsplit, NH, 2, dtype=torch.float32, device=dev)
    attn = torch.empty(B, HID, dtype=torch.bfloat16, device=dev)
    out = torch.empty(B, HID, dtype=torch.bfloat16, device=dev)
    st = _hip.stream_ptr(dev)
    call = _hip.call
    call("dsv2_fill_positions", cache_position.data_ptr(), pos.data_ptr(), base.data_ptr(), L, B, st)
    if family == "small":
        call("dsv2_gemv_bf16", x.data_ptr(), HID, B, HID, packed.w_qkva.data_ptr(), QKVA, None, 0.0, None, 0,
             qkva.data_ptr(), QKVA, 0, st)
        call("dsv2_mla_prepare", qkva.data_ptr(), QKVA, B, pos.data_ptr(), base.data_ptr(),
             packed.kv_norm_weight.data_ptr(), packed.kv_norm_eps, cos2.data_ptr(), sin2.data_ptr(), max_pos,
             packed.w_ukt.data_ptr(), key_cache.data_ptr(), q.data_ptr(), st)
    else:
        call("dsv2_gemm_bf16", x.data_ptr(), HID, 0, B, HID, packed.w_qkva.data_ptr(), 0, QKVA, 1, None, 0,
             qkva.data_ptr(), QKVA, 0, 0, st)
        call("dsv2_mla_prepare", qkva.data_ptr(), QKVA, B, pos.data_ptr(), base.data_ptr(),
             packed.kv_norm_weight.data_ptr(), packed.kv_norm_eps, cos2.data_ptr(), sin2.data_ptr(), max_pos, None,
             key_cache.data_ptr(), q.data_ptr(), st)
        call("dsv2_gemm_bf16", qkva.data_ptr(), QKVA, NOPE + ROPE, B, NOPE, packed.w_ukt.data_ptr(), LAT * NOPE, LAT,
             NH, None, 0, q.data_ptr(), NH * ROW, ROW, 0, st)
    call("dsv2_mla_decode", q.data_ptr(), key_cache.data_ptr(), base.data_ptr(), pos.data_ptr(), B, split, nsplit,
         float(softmax_scale), part_o.data_ptr(), part_ml.data_ptr(), st)
    if family == "small":
        call("dsv2_mla_combine", part_o.data_ptr(), part_ml.data_ptr(), pos.data_ptr(), B, split, nsplit,
             packed.w_uv.data_ptr(), attn.data_ptr(), HID, st)
        call("dsv2_gemv_bf16", attn.data_ptr(), HID, B, HID, packed.w_o.data_ptr(), HID, None, 0.0, None, 0,
             out.data_ptr(), HID, 0, st)
    else:
        olat = torch.empty(B, NH, LAT, dtype=torch.bfloat16, device=dev)
        call("dsv2_mla_combine", part_o.data_ptr(), part_ml.data_ptr(), pos.data_ptr(), B, split, nsplit, None,
             olat.data_ptr(), NH * LAT, st)
        call("dsv2_gemm_bf16", olat.data_ptr(), NH * LAT, LAT, B, LAT, packed.w_uv.data_ptr(), VD * LAT, VD, NH, None,
             0, attn.data_ptr(), HID, VD, 0, st)
        call("dsv2_gemm_bf16", attn.data_ptr(), HID, 0, B, HID, packed.w_o.data_ptr(), 0, HID, 1, None, 0,
             out.data_ptr(), HID, 0, 0, st)
    return out.reshape(B, 1, HID)


def attention_decode_triton(hidden_states, cos, sin, position_ids, cache_position, key_cache, value_cache, packed,
                            softmax_scale: float) -> torch.Tensor:
    """q_len=1 MLA decode for normalised hidden states [B,1,2048] -> o_proj output [B,1,2048]."""
    return _attention_decode("batch", hidden_states, cos, sin, position_ids, cache_position, key_cache, value_cache,
                             packed, softmax_scale)
