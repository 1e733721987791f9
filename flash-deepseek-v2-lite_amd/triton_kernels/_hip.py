"""ctypes binding of libdsv2lite_hip.so (the C ABI declared in include/dsv2lite.h).

The library is loaded after ``import torch`` so that its ``libamdhip64.so.7``
dependency resolves to the HIP runtime torch already loaded: streams, graph
capture and device pointers are then shared.  There is no fallback: if the
library is missing the import raises, naming the build command.
"""

from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdsv2lite_hip.so")
ABI_VERSION = 2

LINEAR_SWIGLU = 1
LINEAR_OUT_F32 = 2
LINEAR_OUT_F32_EXACT = 4

_p = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float

_SIGS = {
    "dsv2_abi_version": ([], _i32),
    "dsv2_last_error_message": ([], ctypes.c_char_p),
    "dsv2_rmsnorm_bf16": ([_p, _i64, _p, _p, _i64, _i32, _i32, _f32, _p], _i32),
    "dsv2_residual_add_bf16": ([_p, _p, _p, _i64, _p], _i32),
    "dsv2_residual_add_f16": ([_p, _p, _p, _i64, _p], _i32),
    "dsv2_silu_mul_bf16": ([_p, _p, _p, _i64, _p], _i32),
    "dsv2_prepare_decode_inputs": ([_p, _p, _p, _p, _i32, _i32, _p], _i32),
    "dsv2_copy_token_rows": ([_p, _i64, _p, _i64, _i64, _p, _i64, _i32, _p, _p], _i32),
    "dsv2_fill_positions": ([_p, _p, _p, _p, _i64, _i32, _p], _i32),
    "dsv2_embed_gather_bf16": ([_p, _p, _i32, _p, _i32, _p], _i32),
    "dsv2_stream_copy": ([_p, _p, _i64, _p], _i32),
    "dsv2_argmax_f32": ([_p, _i32, _i32, _p, _p, _p], _i32),
    "dsv2_gemv_bf16": ([_p, _i64, _i32, _i32, _p, _i32, _p, _f32, _p, _i64, _p, _i64, _i32, _p], _i32),
    "dsv2_lm_head_argmax_workspace_size": ([_i32], _i64),
    "dsv2_lm_head_argmax_bf16": ([_p, _i64, _i32, _p, _i32, _p, _f32, _p, _p, _i64, _p, _p, _p], _i32),
    "dsv2_lm_head_argmax_bf16_noalloc": ([_p, _i64, _i32, _p, _i32, _p, _f32, _p, _p, _p, _p], _i32),
    "dsv2_gemm_bf16": ([_p, _i64, _i64, _i32, _i32, _p, _i64, _i32, _i32, _p, _i64, _p, _i64, _i64, _i32, _p], _i32),
    "dsv2_mla_prepare": ([_p, _i64, _i32, _p, _p, _p, _p, _f32, _p, _p, _i32, _p, _p, _p, _p, _p], _i32),
    "dsv2_mla_prepare_qlat": ([_p, _i64, _i32, _p, _p, _p, _p, _f32, _p, _p, _i32, _p, _p, _p, _p, _p], _i32),
    "dsv2_mla_decode": ([_p, _p, _p, _p, _p, _i32, _i32, _i32, _f32, _p, _p, _p], _i32),
    "dsv2_mla_combine": ([_p, _p, _p, _p, _i32, _i32, _i32, _p, _p, _i64, _p], _i32),
    "dsv2_mla_decode_rows": ([_p, _p, _p, _p, _p, _i32, _f32, _p, _i64, _p], _i32),
    "dsv2_mla_fused": ([_p, _i64, _i32, _p, _p, _p, _p, _f32, _p, _p, _i32, _p, _p, _p, _f32, _p, _i64, _p, _p],
                       _i32),
    "dsv2_attention_decode_expanded": ([_p, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64, _p, _i64, _i64,
                                        _i32, _i32, _i32, _i32, _i32, _p, _f32, _p, _p], _i32),
    "dsv2_mla_prefill_attention": ([_p, _i64, _p, _i64, _i32, _p, _i64, _p, _p, _i64, _i64, _p, _i32, _f32, _p, _i64,
                                    _p], _i32),
    "dsv2_router_logits": ([_p, _i64, _p, _f32, _p, _i32, _p, _p, _p], _i32),
    "dsv2_moe_route_gateup_logits": ([_p, _i32, _p, _f32, _p, _p, _p, _p, _i32, _p, _p], _i32),
    "dsv2_mla_attend": ([_p, _p, _p, _p, _p, _i32, _p, _f32, _p, _i64, _p], _i32),
    "dsv2_mla_spread": ([_p, _i64, _i32, _p, _p, _p, _p, _f32, _p, _p, _i32, _p, _p, _p, _p, _f32, _p, _i64, _p, _p],
                        _i32),
    "dsv2_qkva_absorb_bf16": ([_p, _i64, _i32, _p, _p, _f32, _p, _p, _i64, _p, _p, _p, _p, _p, _p], _i32),
    "dsv2_mla_attend_parts": ([_p, _i64, _i32, _p, _p, _p, _p, _f32, _p, _p, _i32, _p, _p, _p, _f32, _p, _i64, _p,
                               _p], _i32),
    "dsv2_moe_route_gateup_logits_fp8": ([_p, _i32, _p, _f32, _p, _p, _p, _p, _p, _p, _i32, _p, _p], _i32),
    "dsv2_moe_route_down_fp8": ([_p, _i32, _p, _p, _p, _p, _p, _p, _i32, _i32, _p, _p, _p], _i32),
    "dsv2_router_topk6": ([_p, _i64, _p, _f32, _p, _f32, _i32, _p, _p, _p, _p, _p], _i32),
    "dsv2_router_topk6_from_logits": ([_p, _i32, _f32, _p, _p, _p, _p], _i32),
    "dsv2_moe_route_gateup": ([_p, _i32, _p, _p, _p, _i32, _p, _p], _i32),
    "dsv2_moe_route_down": ([_p, _i32, _p, _p, _p, _p, _i32, _i32, _p, _p, _p, _p], _i32),
    "dsv2_moe_bucket": ([_p, _i32, _i32, _p, _p, _p, _p, _p], _i32),
    "dsv2_moe_bucket_workspace_size": ([_i32], _i64),
    "dsv2_moe_bucket_wide": ([_p, _i32, _i32, _p, _p, _p, _p, _p, _i64, _p], _i32),
    "dsv2_moe_grouped_gateup": ([_p, _p, _p, _p, _i32, _i32, _p, _i32, _p, _p], _i32),
    "dsv2_moe_grouped_gateup_shared": ([_p, _i32, _p, _p, _p, _i32, _i32, _p, _p, _i32, _p, _p, _p], _i32),
    "dsv2_moe_grouped_down": ([_p, _p, _p, _i32, _i32, _p, _i32, _p, _p], _i32),
    "dsv2_moe_combine": ([_p, _p, _p, _i32, _p, _p, _p, _p, _f32, _p, _p], _i32),
    "dsv2_moe_grouped_down_shared": ([_p, _i32, _p, _p, _i32, _i32, _p, _p, _p, _i32, _p, _p, _p], _i32),
    "dsv2_moe_grouped_gateup_shared_fp8": ([_p, _i32, _p, _p, _p, _i32, _i32, _p, _p, _p, _p, _i32, _p, _p, _p], _i32),
    "dsv2_moe_grouped_down_shared_fp8": ([_p, _i32, _p, _p, _i32, _i32, _p, _p, _p, _p, _p, _i32, _p, _p, _p], _i32),
    "dsv2_moe_combine_parts": ([_p, _p, _p, _i32, _p, _p, _p, _p, _f32, _p, _p], _i32),
}

EXPORTS = tuple(_SIGS)


class HipKernelError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"HIP library not built: {LIB_PATH} is missing. Run "
            "`python flash-deepseek-v2-lite_amd/csrc/build.py` (or __graft_entry__.build()).")
    lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    for name, (args, res) in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if lib.dsv2_abi_version() != ABI_VERSION:
        raise ImportError(f"libdsv2lite_hip.so ABI {lib.dsv2_abi_version()} != expected {ABI_VERSION}")
    return lib


lib = _load()


def call(name: str, *args) -> None:
    """Invoke an entry point; raise HipKernelError with the library's message on failure."""
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.dsv2_last_error_message().decode(errors="replace")
        raise HipKernelError(f"{name} failed (status {rc}): {msg}")


def stream_ptr(device: torch.device | None = None) -> int:
    """hipStream_t of torch's current stream (the capture stream inside torch.cuda.graph)."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
