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


# caches up to this many tokens per row take one split per row: the engine then runs the
# one-launch decode (dsv2_mla_decode_rows) and no split merge
ONE_SPLIT_MAX_CTX = 256


def plan_splits(rows: int, max_ctx: int, target_wgs: int = 256) -> tuple[int, int]:
    """(split_tokens, max_splits) for the split-KV decode: one split per row for caches of at
    most ONE_SPLIT_MAX_CTX tokens (measured on MI355X, whole decode steps, against the
    multi-split plan below: bsz=64 x 57-token caches 2.809 -> 2.726 ms, bsz=64 x 233 6.958 ->
    6.901, bsz=128 x 233 7.941 -> 7.832; at 433 tokens one split loses, 7.013 -> 7.101);
    else about target_wgs workgroups,
    split_tokens a multiple of 32, at most 64 splits per row.  256 = one workgroup per CU;
    each streams its split with two tiles in flight.  Measured on MI355X over the whole
    decode step against 512: bsz=256 x 2048-token prompts 22.72k vs 22.44k tok/s, bsz=64 x
    U[256,1024] 8.80k vs 8.70k, reference workload 52.6k vs 51.3k (bsz=256) and 22.0k vs
    22.0k (bsz=64); 128 (8.55k at bsz=64) and 1024 (bsz=256 x 2098 tokens: 118 vs 109 us per
    layer) are slower.  Rows of very unequal lengths want more, shorter splits (bsz=128 x
    U[256,8192]: 512 -> 2048-token splits 132 us, 256 -> 4064-token splits 171 us); capping
    the split at 2048 tokens instead cost the equal-length bsz=256 step 8%."""
    if max_ctx <= ONE_SPLIT_MAX_CTX:
        return max(32, math.ceil(max_ctx / 32) * 32), 1
    per_row = max(1, min(64, math.ceil(target_wgs / max(rows, 1))))
    split = max(32, math.ceil(math.ceil(max_ctx / per_row) / 32) * 32)
    split = max(split, math.ceil(max_ctx / 64 / 32) * 32)
    return split, math.ceil(max_ctx / split)


# the small family runs the absorb path (dsv2_qkva_absorb_bf16 + dsv2_mla_attend_parts) while
# the cache is this short, like the engine (dsv2lite.engine.FUSED_MLA_MAX_CTX); longer caches
# take the split-KV decode
FUSED_MAX_CTX = 2048


@dataclass
class AttentionDecodeWorkspace:
    """Per-(device, B, L) buffers of one attention call, cached on the packed weights like
    the reference's workspace (attention_decode_batch.py:641-669); the returned output
    aliases ``out`` and is overwritten by the next call with the same key."""

    pos: torch.Tensor      # [B] int32
    base: torch.Tensor     # [B] int64
    cap: torch.Tensor      # [B] int32
    status: torch.Tensor   # [1] int32: DSV2_DEVERR_* bits of every call so far
    qkva: torch.Tensor     # [B, 3648]
    qlat_part: torch.Tensor  # [B, 16, 8, 512] fp32: partial absorbed queries (small family)
    q: torch.Tensor        # [B, 16, 576]
    split: int
    nsplit: int
    part_o: torch.Tensor   # [B, nsplit, 16, 512] fp32
    part_ml: torch.Tensor  # [B, nsplit, 16, 2] fp32
    olat: torch.Tensor     # [B, 16, 512]
    attn: torch.Tensor     # [B, 2048]
    out: torch.Tensor      # [B, 1, 2048]


def _workspace(packed: AttentionPackedWeights, dev: torch.device, B: int, L: int) -> AttentionDecodeWorkspace:
    key = (dev.index if dev.index is not None else 0, B, L)
    cache = packed.__dict__.setdefault("workspace_by_key", {})
    ws = cache.get(key)
    if ws is None:
        e = lambda *shape, dt=torch.bfloat16: torch.empty(*shape, dtype=dt, device=dev)  # noqa: E731
        split, nsplit = plan_splits(B, L)
        ws = AttentionDecodeWorkspace(
            pos=e(B, dt=torch.int32), base=e(B, dt=torch.int64), cap=e(B, dt=torch.int32),
            status=torch.zeros(1, dtype=torch.int32, device=dev), qkva=e(B, QKVA),
            qlat_part=e(B, NH, NOPE // 16, LAT, dt=torch.float32), q=e(B, NH, ROW), split=split,
            nsplit=nsplit, part_o=e(B, nsplit, NH, LAT, dt=torch.float32), part_ml=e(B, nsplit, NH, 2, dt=torch.float32),
            olat=e(B, NH, LAT), attn=e(B, HID), out=e(B, 1, HID))
        cache[key] = ws
    return ws


def check_cache_status(packed: AttentionPackedWeights) -> None:
    """Raise if an attention call on these weights tried to write its new token at or past
    the cache length L (nothing was written there; synchronises).  The reference raises on
    a cache overflow (src/run.py:131-134)."""
    for ws in packed.__dict__.get("workspace_by_key", {}).values():
        if int(ws.status.item()) & 1:  # DSV2_DEVERR_CACHE_FULL
            ws.status.zero_()
            raise RuntimeError("attention decode: cache_position reached the cache length; the new token was not "
                               "written")


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
    ws = _workspace(packed, dev, B, L)
    attn2, out2 = ws.attn, ws.out.view(B, HID)
    st = _hip.stream_ptr(dev)
    call = _hip.call
    P = lambda t: t.data_ptr()  # noqa: E731
    call("dsv2_fill_positions", P(cache_position), P(ws.pos), P(ws.base), P(ws.cap), L, B, st)
    if family == "small":
        if L <= FUSED_MAX_CTX:
            # the engine's default small-batch MLA: the projection also forms the absorbed query
            call("dsv2_qkva_absorb_bf16", P(x), HID, B, P(packed.w_qkva), None, 0.0, P(packed.w_uk), P(ws.qkva), QKVA,
                 P(ws.qlat_part), P(key_cache), P(ws.base), P(ws.pos), P(ws.cap), st)
            call("dsv2_mla_attend_parts", P(ws.qkva), QKVA, B, P(ws.pos), P(ws.base), P(ws.cap),
                 P(packed.kv_norm_weight), packed.kv_norm_eps, P(cos2), P(sin2), max_pos, P(ws.qlat_part),
                 P(packed.w_uv), P(key_cache), float(softmax_scale), P(attn2), HID, P(ws.status), st)
        else:
            call("dsv2_gemv_bf16", P(x), HID, B, HID, P(packed.w_qkva), QKVA, None, 0.0, None, 0, P(ws.qkva), QKVA, 0,
                 st)
            call("dsv2_mla_prepare", P(ws.qkva), QKVA, B, P(ws.pos), P(ws.base), P(ws.cap), P(packed.kv_norm_weight),
                 packed.kv_norm_eps, P(cos2), P(sin2), max_pos, P(packed.w_ukt), P(key_cache), P(ws.q), P(ws.status),
                 st)
            call("dsv2_mla_decode", P(ws.q), P(key_cache), P(ws.base), P(ws.pos), P(ws.cap), B, ws.split, ws.nsplit,
                 float(softmax_scale), P(ws.part_o), P(ws.part_ml), st)
            call("dsv2_mla_combine", P(ws.part_o), P(ws.part_ml), P(ws.pos), P(ws.cap), B, ws.split, ws.nsplit,
                 P(packed.w_uv), P(attn2), HID, st)
        call("dsv2_gemv_bf16", P(attn2), HID, B, HID, P(packed.w_o), HID, None, 0.0, None, 0, P(out2), HID, 0, st)
        return ws.out
    call("dsv2_gemm_bf16", P(x), HID, 0, B, HID, P(packed.w_qkva), 0, QKVA, 1, None, 0, P(ws.qkva), QKVA, 0, 0, st)
    call("dsv2_mla_prepare", P(ws.qkva), QKVA, B, P(ws.pos), P(ws.base), P(ws.cap), P(packed.kv_norm_weight),
         packed.kv_norm_eps, P(cos2), P(sin2), max_pos, None, P(key_cache), P(ws.q), P(ws.status), st)
    call("dsv2_gemm_bf16", P(ws.qkva), QKVA, NOPE + ROPE, B, NOPE, P(packed.w_ukt), LAT * NOPE, LAT, NH, None, 0,
         P(ws.q), NH * ROW, ROW, 0, st)
    call("dsv2_mla_decode", P(ws.q), P(key_cache), P(ws.base), P(ws.pos), P(ws.cap), B, ws.split, ws.nsplit,
         float(softmax_scale), P(ws.part_o), P(ws.part_ml), st)
    call("dsv2_mla_combine", P(ws.part_o), P(ws.part_ml), P(ws.pos), P(ws.cap), B, ws.split, ws.nsplit, None,
         P(ws.olat), NH * LAT, st)
    call("dsv2_gemm_bf16", P(ws.olat), NH * LAT, LAT, B, LAT, P(packed.w_uv), VD * LAT, VD, NH, None, 0, P(attn2),
         HID, VD, 0, st)
    call("dsv2_gemm_bf16", P(attn2), HID, 0, B, HID, P(packed.w_o), 0, HID, 1, None, 0, P(out2), HID, 0, 0, st)
    return ws.out


def batched_attention_decode_q1_triton(query_states: torch.Tensor, key_states: torch.Tensor,
                                       value_states: torch.Tensor, cache_position: torch.Tensor,
                                       softmax_scale: float) -> torch.Tensor:
    """q_len=1 attention over an expanded per-head cache: query [B, H, 1, Dq], keys
    [B, H, L, Dq], values [B, H, L, Dv] (bf16, last dim contiguous) -> [B, H, 1, Dv]:
    softmax over positions 0..cache_position of scale * q.k, times v, fp32 math.  Positions
    at or past L are not read (the reference reads them unchecked); the call then attends
    the L rows and the overflow is reported by check_expanded_status.
    Reference: attention_decode_batch.py:345-401."""
    require_cuda("batched_attention_decode_q1_triton", query_states, key_states, value_states, cache_position)
    if query_states.dtype != torch.bfloat16 or key_states.dtype != torch.bfloat16 or \
            value_states.dtype != torch.bfloat16:
        raise NotImplementedError("batched_attention_decode_q1_triton supports bf16 only")
    if query_states.ndim != 4 or key_states.ndim != 4 or value_states.ndim != 4:
        raise ValueError("query/key/value states must be rank-4 tensors")
    if query_states.shape[2] != 1:
        raise ValueError("batched_attention_decode_q1_triton only supports q_len=1")
    if cache_position.numel() != 1 or cache_position.dtype != torch.long:
        raise ValueError("cache_position must be CUDA int64 tensor with one element")
    B, H, _, Dq = query_states.shape
    Dv = value_states.shape[3]
    L = key_states.shape[2]
    if key_states.shape[:2] != (B, H) or value_states.shape[:3] != (B, H, L) or key_states.shape[3] != Dq:
        raise ValueError("key/value states must be [B, H, L, Dq] / [B, H, L, Dv] matching the query")
    for t in (query_states, key_states, value_states):
        if t.stride(3) != 1:
            raise NotImplementedError("batched_attention_decode_q1_triton needs a contiguous last dimension")
    out = torch.empty((B, H, 1, Dv), device=query_states.device, dtype=query_states.dtype)
    if B == 0 or L == 0:
        return out
    q, k, v = query_states, key_states, value_states
    _hip.call("dsv2_attention_decode_expanded", q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), k.stride(0),
              k.stride(1), k.stride(2), v.data_ptr(), v.stride(0), v.stride(1), v.stride(2), out.data_ptr(),
              out.stride(0), out.stride(1), B, H, Dq, Dv, L, cache_position.data_ptr(), float(softmax_scale),
              _expanded_status(q.device).data_ptr(), _hip.stream_ptr(q.device))
    return out


_EXPANDED_STATUS: dict = {}


def _expanded_status(dev: torch.device) -> torch.Tensor:
    k = dev.index if dev.index is not None else 0
    if k not in _EXPANDED_STATUS:
        _EXPANDED_STATUS[k] = torch.zeros(1, dtype=torch.int32, device=dev)
    return _EXPANDED_STATUS[k]


def check_expanded_status(device: torch.device | str = "cuda") -> None:
    """Raise if a batched_attention_decode_q1_triton call on `device` had cache_position
    outside [0, L) (synchronises)."""
    st = _expanded_status(torch.device(device))
    if int(st.item()) & 1:  # DSV2_DEVERR_CACHE_FULL
        st.zero_()
        raise RuntimeError("batched_attention_decode_q1_triton: cache_position outside the cache")


def attention_decode_triton(hidden_states, cos, sin, position_ids, cache_position, key_cache, value_cache, packed,
                            softmax_scale: float) -> torch.Tensor:
    """q_len=1 MLA decode for normalised hidden states [B,1,2048] -> o_proj output [B,1,2048]."""
    return _attention_decode("batch", hidden_states, cos, sin, position_ids, cache_position, key_cache, value_cache,
                             packed, softmax_scale)
