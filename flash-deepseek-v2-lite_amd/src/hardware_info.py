"""Host/GPU description for the run report (reference: src/hardware_info.py:60-93,
which reads nvidia-smi and torch.version.cuda; this one reports the ROCm side:
gfx architecture, CU count, HBM size, torch.version.hip and the host cores)."""

from __future__ import annotations

import os
import platform

import torch


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def collect_hardware_info(device: torch.device | str | None = None) -> dict:
    info = {
        "cpu": {"model": _cpu_model(), "logical_cores": os.cpu_count(),
                "affinity_cores": len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else None},
        "software": {"python": platform.python_version(), "torch": torch.__version__,
                     "hip": getattr(torch.version, "hip", None)},
    }
    try:
        import psutil

        info["cpu"]["memory_gib"] = round(psutil.virtual_memory().total / 2**30, 1)
    except Exception:  # noqa: BLE001 - optional dependency
        pass
    if torch.cuda.is_available():
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        p = torch.cuda.get_device_properties(dev)
        info["gpu"] = {"name": p.name, "arch": getattr(p, "gcnArchName", None), "compute_units": p.multi_processor_count,
                       "memory_gib": round(p.total_memory / 2**30, 1), "count": torch.cuda.device_count()}
    return info
