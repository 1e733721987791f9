"""Argument checks shared by the wrappers (reference conventions: NotImplementedError
for device/dtype/layout, ValueError for shapes)."""

from __future__ import annotations

import torch


def require_cuda(name: str, *ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and t.device.type != "cuda":
            raise NotImplementedError(f"{name} requires CUDA (HIP) tensors")


def require_dtype(name: str, t: torch.Tensor, *dtypes: torch.dtype) -> None:
    if t.dtype not in dtypes:
        raise NotImplementedError(f"{name}: unsupported dtype {t.dtype}")


def require_contiguous(name: str, *ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_contiguous():
            raise NotImplementedError(f"{name} requires contiguous tensors")
