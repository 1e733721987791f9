"""Build libdsv2lite_hip.so for gfx950 with hipcc (in-tree, no JIT cache).

    python flash-deepseek-v2-lite_amd/csrc/build.py [-j N]

Each .hip file compiles to an object in parallel, then one shared library is
linked into ``flash-deepseek-v2-lite_amd/triton_kernels/``.  The library links
``libamdhip64.so.7``; loading it after ``import torch`` binds it to the HIP
runtime torch already loaded (same soname), so streams and graphs are shared.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

CSRC = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(CSRC)
ROOT = os.path.dirname(PKG)
INCLUDE = os.path.join(ROOT, "include")
OUT = os.path.join(PKG, "triton_kernels", "libdsv2lite_hip.so")
OBJDIR = os.path.join(PKG, "_build")
SOURCES = ["elementwise.hip", "gemv.hip", "gemm.hip", "mla.hip", "mla_small.hip", "moe.hip", "attention_expanded.hip", "mla_prefill.hip"]
ARCH = os.environ.get("DSV2_OFFLOAD_ARCH", "gfx950")

CXXFLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-I", INCLUDE, "-I", CSRC,
    # packed-FP32 VALU ops off (v_pk_{add,mul,fma}_f32 are not emitted)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    raise RuntimeError("hipcc not found (ROCm is required to build the HIP library)")


def _compile(src: str) -> str:
    obj = os.path.join(OBJDIR, src.replace(".hip", ".o"))
    cmd = [hipcc(), *CXXFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def _check_no_missing_stubs(lib: str) -> None:
    """A kernel whose host launch stub the compiler left undefined links into a library that
    only fails when it is loaded; refuse it at build time."""
    nm = shutil.which("nm")
    if not nm:
        return
    r = subprocess.run([nm, "-D", "--undefined-only", lib], capture_output=True, text=True)
    missing = [ln.split()[-1] for ln in r.stdout.splitlines() if "__device_stub__" in ln]
    if missing:
        os.remove(lib)
        raise RuntimeError(f"undefined kernel launch stubs in the linked library: {missing}")


def build(jobs: int | None = None, verbose: bool = False) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 4, 8)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT + ".tmp"
    # -Bsymbolic: the library's launches bind to its own kernel handles, never to a same-named
    # kernel of a library loaded before it with RTLD_GLOBAL (which would run that kernel on
    # this library's argument layout)
    cmd = [hipcc(), "-shared", "-fPIC", "-Wl,-Bsymbolic", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    _check_no_missing_stubs(tmp)
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}", file=sys.stderr)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=None)
    a = ap.parse_args()
    build(a.j, verbose=True)
