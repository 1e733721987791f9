"""Decode input preparation, cache write, residual add
(reference: triton_kernels/attention_prepost.py:113-223)."""

from __future__ import annotations

import torch

from . import _hip
from ._checks import require_contiguous, require_cuda

_STATUS: dict = {}  # device index -> int32 [1] status word of copy_single_token_to_cache


def _status(dev: torch.device) -> torch.Tensor:
    k = dev.index if dev.index is not None else 0
    if k not in _STATUS:
        _STATUS[k] = torch.zeros(1, dtype=torch.int32, device=dev)
    return _STATUS[k]


def check_cache_write_status(device: torch.device | str = "cuda") -> None:
    """Raise if a copy_single_token_to_cache call on `device` had cache_position outside the
    destination's sequence length (that row was not written; synchronises).  The reference's
    GraphCache raises on overflow (src/run.py:131-134)."""
    st = _status(torch.device(device))
    if int(st.item()) & 1:  # DSV2_DEVERR_CACHE_FULL
        st.zero_()
        raise RuntimeError("copy_single_token_to_cache: cache_position outside the cache; nothing was written")


def copy_single_token_to_cache(src: torch.Tensor, dst: torch.Tensor, cache_position: torch.Tensor) -> None:
    """dst[b, pos] = src[b] for each row b, pos = cache_position[0] (device scalar).

    Accepts the reference's expanded layout ([B, H, 1, D] -> [B, H, S, D], per-head
    rows) and the compressed-cache layout ([B, 1, D] -> [B, S, D]).  A pos outside
    [0, S) writes nothing and is reported by check_cache_write_status."""
    require_cuda("copy_single_token_to_cache", src, dst, cache_position)
    if src.dtype != dst.dtype:
        raise ValueError("src and dst dtype must match")
    if cache_position.numel() != 1:
        raise ValueError("cache_position must be a CUDA tensor with one element")
    require_contiguous("copy_single_token_to_cache", src, dst)
    if src.ndim == 4 and dst.ndim == 4 and src.shape[2] == 1 and src.shape[:2] == dst.shape[:2] \
            and src.shape[3] == dst.shape[3]:
        rows = src.shape[0] * src.shape[1]
        row_bytes = src.shape[3] * src.element_size()
        src_bs, dst_bs = row_bytes, dst.shape[2] * row_bytes
        seq = dst.shape[2]
    elif src.ndim == 3 and dst.ndim == 3 and src.shape[1] == 1 and src.shape[0] == dst.shape[0] \
            and src.shape[2] == dst.shape[2]:
        rows = src.shape[0]
        row_bytes = src.shape[2] * src.element_size()
        src_bs, dst_bs = row_bytes, dst.shape[1] * row_bytes
        seq = dst.shape[1]
    else:
        raise NotImplementedError("copy_single_token_to_cache supports [B,H,1,D]->[B,H,S,D] or [B,1,D]->[B,S,D]")
    if row_bytes % 16:
        raise ValueError("row size must be a multiple of 16 bytes")
    if rows == 0 or seq == 0:
        return
    pos = cache_position.reshape(1).to(torch.int64)
    _hip.call("dsv2_copy_token_rows", src.data_ptr(), src_bs, dst.data_ptr(), dst_bs, row_bytes, pos.data_ptr(), seq,
              rows, _status(src.device).data_ptr(), _hip.stream_ptr(src.device))


def prepare_decode_inputs_triton(cache_position: torch.Tensor, attention_mask: torch.Tensor,
                                 position_ids: torch.Tensor, attention_mask_index: torch.Tensor) -> None:
    """mask[b, j] = (attention_mask_index[j] <= pos); position_ids[b] = pos (int64, in place)."""
    require_cuda("prepare_decode_inputs_triton", cache_position, attention_mask, position_ids)
    if cache_position.numel() != 1:
        raise ValueError("cache_position must have one element")
    if attention_mask.ndim != 2:
        raise ValueError("attention_mask must have shape [batch, max_cache_len]")
    if position_ids.ndim != 2 or position_ids.shape[0] != attention_mask.shape[0] or position_ids.shape[1] != 1:
        raise ValueError("position_ids must have shape [batch, 1]")
    if attention_mask_index.ndim != 1 or attention_mask_index.shape[0] != attention_mask.shape[1]:
        raise ValueError("attention_mask_index must be 1D with length max_cache_len")
    if attention_mask.dtype != torch.long or position_ids.dtype != torch.long or cache_position.dtype != torch.long:
        raise ValueError("prepare_decode_inputs_triton requires int64 tensors")
    require_contiguous("prepare_decode_inputs_triton", attention_mask, position_ids)
    idx = attention_mask_index.to(device=attention_mask.device, dtype=torch.long).contiguous()
    if attention_mask.shape[0] == 0:
        return
    _hip.call("dsv2_prepare_decode_inputs", cache_position.data_ptr(), idx.data_ptr(), attention_mask.data_ptr(),
              position_ids.data_ptr(), attention_mask.shape[0], attention_mask.shape[1],
              _hip.stream_ptr(attention_mask.device))


def residual_add_triton(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """out = a + b rounded once from fp32 (bf16 or fp16, same dtype)."""
    require_cuda("residual_add_triton", a, b)
    if a.shape != b.shape:
        raise ValueError("a and b must have the same shape")
    if a.dtype not in (torch.bfloat16, torch.float16) or b.dtype != a.dtype:
        raise NotImplementedError("residual_add_triton supports bf16/fp16 with same dtype")
    require_contiguous("residual_add_triton", a, b)
    if a.numel() % 8:
        raise ValueError("residual_add_triton needs numel % 8 == 0")
    out = torch.empty_like(a)
    fn = "dsv2_residual_add_bf16" if a.dtype == torch.bfloat16 else "dsv2_residual_add_f16"
    _hip.call(fn, a.data_ptr(), b.data_ptr(), out.data_ptr(), a.numel(), _hip.stream_ptr(a.device))
    return out
