"""Decode-throughput benchmark of the HIP DeepSeek-V2-Lite decode step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config all|1|2|3|4|r64|r256|s8|s64]
                    [--expert-dtype bf16|fp8] [--no-cpu-baseline]

Every config: full 27-layer random-init DeepSeek-V2-Lite bf16 (N(0,0.02), seed 0), eager
prefill of uniform random prompt ids, then K greedy decode steps, the whole step replayed
as one hipGraph.  Prints ONE JSON line.

Default (--config all): the line's value is benchmark config 1 (bsz=1, a 128-token prompt
from seed 1, small kernel family); the metric's other two batch sizes ride along under
"configs" -- C2 (bsz=64, prompt lengths U[256,1024], batch family) and C3 (bsz=256, 2048-
token prompts, batch family) -- timed in the same run on the same weights, each with its
tok/s, ms/step, step roofline and dominant-kernel roofline.  --config N runs one config
alone; r64|r256 are the reference's own published workload (one 24-token prompt replicated
over the batch), whose vs_baseline is value / the published A100 batch-family TPS for it,
and s8|s64 the same workload on the small (GEMV) family, against the published A100
small-GEMV TPS.  The default line carries all of them under "configs", with the isolated
MLA microbenchmark (C4) and configs 1-3 again on e4m3 expert weights (C1_fp8..C3_fp8).
--config 4 is the isolated absorbed-MLA decode microbenchmark (bsz=128, KV lengths
U[256,8192]); its value is compressed-cache GB/s.

Extra fields:
  roofline      -- dominant kernel of the step: algorithmic bytes per launch /
                   average launch time (HIP events around a graph of repeated
                   launches on the engine's stream) vs 8 TB/s; traffic = HBM bytes
                   per launch from the committed PMC summary profiles/traffic_c<N>.json
                   (see --pmc-traffic), null when absent or when it was measured on other
                   source of the kernel; traffic_source says which.
  step_roofline -- algorithmic bytes per step (weights of the experts actually hit,
                   counted from the router output, + compressed KV read) / step time.
  cpu_baseline  -- the CPU oracle (PyTorch eager restatement of the HF math) timed on
                   this host on benchmark config 0 (one MoE layer: prefill 256 + 32
                   decode steps) and scaled to whole-model tokens/s.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "flash-deepseek-v2-lite_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import torch  # noqa: E402

HBM_PEAK = 8.0e12
METRIC = "decode tokens/s at bsz=1/64/256 (1 GPU) + % of HBM roofline per step"

CONFIGS = {
    1: dict(batch=1, family="small", prompt=lambda g: [128], seed=1,
            workload="C1: full 27-layer DeepSeek-V2-Lite, bsz=1, 128-token random prompt, small family, hipGraph"),
    2: dict(batch=64, family="batch", prompt=lambda g: torch.randint(256, 1025, (64,), generator=g).tolist(), seed=2,
            workload="C2: bsz=64, prompt lengths U[256,1024], batch family, hipGraph"),
    3: dict(batch=256, family="batch", prompt=lambda g: [2048] * 256, seed=2,
            workload="C3: bsz=256, prompt 2048, batch family, hipGraph"),
    # The reference's own published workload (src/run.py:733-741): ONE 24-token prompt
    # replicated over the batch, so every row routes to the same 6 experts per layer; the
    # published A100 batch-family decode TPS for it (docs/third_party_baselines.md:90-100)
    # is the baseline of these lines.
    "r64": dict(batch=64, family="batch", prompt=lambda g: [24] * 64, seed=4, replicate=True, published=6237.99,
                workload="reference workload: bsz=64, one 24-token random prompt replicated, batch family, "
                         "hipGraph"),
    "r256": dict(batch=256, family="batch", prompt=lambda g: [24] * 256, seed=4, replicate=True, published=11428.26,
                 workload="reference workload: bsz=256, one 24-token random prompt replicated, batch family, "
                          "hipGraph"),
    # the same workload on the small (GEMV) family above bsz=1; published: the A100 "forced
    # small-GEMV" column of docs/third_party_baselines.md:90-100
    "s8": dict(batch=8, family="small", prompt=lambda g: [24] * 8, seed=4, replicate=True, published=614.82,
               workload="reference workload: bsz=8, one 24-token random prompt replicated, small family, hipGraph"),
    "s64": dict(batch=64, family="small", prompt=lambda g: [24] * 64, seed=4, replicate=True, published=1006.51,
                workload="reference workload: bsz=64, one 24-token random prompt replicated, small family, "
                         "hipGraph"),
}


def step_bytes(cfg, n_exp_per_layer: list[int], ctx_sum_per_layer: float, batch: int,
               expert_fp8: bool = False) -> float:
    """Algorithmic HBM bytes of one decode step (dsv2lite.roofline.step_bytes): every weight
    read once (attention, router, the experts actually hit, shared experts, dense layer 0,
    lm_head, norms), the embedding rows and the compressed KV rows read (1,152 B per token
    per layer)."""
    from dsv2lite.roofline import step_bytes as _sb

    return float(_sb(cfg, n_exp_per_layer, ctx_sum_per_layer, batch, expert_fp8))


def time_dominant_kernel(eng, family: str, reps: int = 4) -> dict:
    """Average duration of the step's dominant kernel: a graph with one launch per MoE layer
    (each on that layer's own weights, so the 26-layer working set streams from HBM rather
    than the 256 MB Infinity Cache), replayed `reps` times between HIP events on the
    current stream, with the step's own activations and routing."""
    from triton_kernels._hip import call, ptr, stream_ptr

    c, b = eng.cfg, eng.buf
    moe_layers = [L for L in eng.w.layers if L.moe]
    B = eng.B
    # small family: each distinct routed expert's and the 2 shared halves' weights once (at
    # bsz=1 every one of the row's 8 routes), the 8 SwiGLU outputs of every row
    n_small = int(torch.unique(b.ids32[:B]).numel()) + 2 if family == "small" else 0
    if family == "small" and eng.expert_dtype == "fp8":
        name = "route_gateup_fp8_kernel<4> (small-family MoE gate_up+SwiGLU on e4m3 weights, 6 routed + 2 shared halves)"
        bytes_per = n_small * 2 * c.moe_inter * (c.hidden + 4) + B * 8 * c.moe_inter * 2

        def launch(L):
            call("dsv2_moe_route_gateup_logits_fp8", ptr(b.xn), B, ptr(b.router_logits), c.routed_scaling,
                 ptr(b.ids32), ptr(b.wts), ptr(L.w_gu8), ptr(L.gu_scale), ptr(L.sh_gu8), ptr(L.sh_gu_scale),
                 c.moe_inter, ptr(b.hbuf), stream_ptr())
    elif family == "small":
        name = "route_gateup_kernel<2, 2> (small-family MoE gate_up+SwiGLU, 6 routed + 2 shared halves)"
        bytes_per = n_small * 2 * c.moe_inter * c.hidden * 2 + B * 8 * c.moe_inter * 2

        def launch(L):
            call("dsv2_moe_route_gateup", ptr(b.xn), B, ptr(b.ids32), ptr(L.w_gu), ptr(L.sh_gu), c.moe_inter,
                 ptr(b.hbuf), stream_ptr())
    elif eng.expert_dtype == "fp8":
        sym = {32: "gemm_f8_kernel<true, 16, 4>", 64: "gemm_f8_kernel<true, 32, 4>"}[b.tile_tokens]
        n_exp = int(torch.unique(b.ids32[:B]).numel())
        # e4m3 weights (1 B) + one fp32 scale per weight row, routed and shared; bf16 outputs
        bytes_per = (n_exp * 2 * c.moe_inter + 2 * c.shared_inter) * (c.hidden + 4) + (B * 6 * c.moe_inter
                                                                                      + B * c.shared_inter) * 2
        name = (f"{sym} via dsv2_moe_grouped_gateup_shared_fp8 (expert-grouped gate_up+SwiGLU on e4m3 weights, "
                f"{b.tile_tokens}-token tiles, + the 2 shared-expert halves)")

        def launch(L):
            call("dsv2_moe_grouped_gateup_shared_fp8", ptr(b.xn), B, ptr(b.sorted), ptr(b.tiles), ptr(b.ntiles),
                 b.max_tiles, b.tile_tokens, ptr(L.w_gu8), ptr(L.gu_scale), ptr(L.sh_gu8), ptr(L.sh_gu_scale),
                 c.moe_inter, ptr(b.hs), ptr(b.shmid), stream_ptr())
    else:
        from dsv2lite.engine import shared_in_grouped

        sym = {16: "gemm_xlds_kernel<1, true, 4, true, 2, 2, 1, false>",
               32: "gemm_xlds_kernel<2, true, 4, true, 2, 4, 2, true>", 64: "gemm_dma_kernel<true, 32, 32, 4, 2>",
               256: "gemm_dma_kernel<true, 64, 128, 2, 4>"}[b.tile_tokens]
        n_exp = int(torch.unique(b.ids32[:B]).numel())
        bytes_per = n_exp * 2 * c.moe_inter * c.hidden * 2 + B * 6 * c.moe_inter * 2
        if shared_in_grouped(B, b.tile_tokens):
            # the step's launch also carries the shared experts' gate_up
            name = (f"{sym} via dsv2_moe_grouped_gateup_shared (expert-grouped gate_up+SwiGLU on MFMA, "
                    f"{b.tile_tokens}-token tiles, + the 2 shared-expert halves)")
            bytes_per += 2 * c.shared_inter * c.hidden * 2 + B * c.shared_inter * 2

            def launch(L):
                call("dsv2_moe_grouped_gateup_shared", ptr(b.xn), B, ptr(b.sorted), ptr(b.tiles), ptr(b.ntiles),
                     b.max_tiles, b.tile_tokens, ptr(L.w_gu), ptr(L.sh_gu), c.moe_inter, ptr(b.hs), ptr(b.shmid),
                     stream_ptr())
        else:
            name = f"{sym} via dsv2_moe_grouped_gateup (expert-grouped gate_up+SwiGLU on MFMA, {b.tile_tokens}-token tiles)"

            def launch(L):
                call("dsv2_moe_grouped_gateup", ptr(b.xn), ptr(b.sorted), ptr(b.tiles), ptr(b.ntiles), b.max_tiles,
                     b.tile_tokens, ptr(L.w_gu), c.moe_inter, ptr(b.hs), stream_ptr())
    avg_s = time_graph(launch, moe_layers, reps)
    ach = bytes_per / avg_s
    return {"kernel": name, "bound": "hbm", "achieved": ach / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": ach / HBM_PEAK, "traffic": None, "bytes_per_launch": bytes_per, "avg_us": avg_s * 1e6}


def time_graph(launch, layers, reps: int = 4) -> float:
    """Average seconds per launch of `launch(L)` over a graph with one launch per entry of
    `layers`, replayed once untimed and `reps` times between HIP events on the current
    stream."""
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        launch(layers[0])
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for L in layers:
            launch(L)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / 1e3 / (len(layers) * reps)


def time_other_kernels(eng, family: str, ctx_rows: list[int]) -> dict:
    """The step's next-largest kernels, each timed like the dominant one (a graph of one
    launch per MoE layer on that layer's weights / cache, after the dominant kernel's graph,
    so their dispatches are the last of their symbol in a profiled run): achieved GB/s of
    the algorithmic bytes.  ctx_rows: cached tokens each row attends (pos + 1)."""
    from dsv2lite.engine import shared_in_grouped
    from triton_kernels._hip import call, ptr, stream_ptr

    c, b, B = eng.cfg, eng.buf, eng.B
    moe = [i for i, L in enumerate(eng.w.layers) if L.moe]
    out = {}

    def entry(name, launch, layers, nbytes):
        t = time_graph(launch, layers)
        out[name] = {"kernel": name, "avg_us": t * 1e6, "bytes_per_launch": nbytes,
                     "achieved_GBps": nbytes / t / 1e9, "frac": nbytes / t / HBM_PEAK}

    kv = sum(ctx_rows) * 1152
    if family == "small":
        def fused(li):
            L = eng.w.layers[li]
            call("dsv2_mla_fused", ptr(b.qkva), c.qkva_dim, B, ptr(eng.cache.pos), ptr(eng.cache.base),
                 ptr(eng.cache.cap), ptr(L.kv_norm), c.eps, ptr(eng.cos), ptr(eng.sin), eng.max_pos, ptr(L.w_ukt),
                 ptr(L.w_uv), ptr(eng.cache.layer(li)), eng.scale, ptr(b.attn), c.hidden, None, stream_ptr())
        if eng.fused_mla:
            entry("mla_quad_kernel (one launch: absorption + new row + attention + W_UV, 64 workgroups per row)",
                  fused, moe,
                  2 * 2 * 16 * 128 * 512 + kv + B * 2048 * 2)

        def prepare(li):
            L = eng.w.layers[li]
            call("dsv2_mla_prepare", ptr(b.qkva), c.qkva_dim, B, ptr(eng.cache.pos), ptr(eng.cache.base),
                 ptr(eng.cache.cap), ptr(L.kv_norm), c.eps, ptr(eng.cos), ptr(eng.sin), eng.max_pos, ptr(L.w_ukt),
                 ptr(eng.cache.layer(li)), ptr(b.q), None, stream_ptr())

        def attend(li):
            L = eng.w.layers[li]
            call("dsv2_mla_attend", ptr(b.q), ptr(eng.cache.layer(li)), ptr(eng.cache.base), ptr(eng.cache.pos),
                 ptr(eng.cache.cap), B, ptr(L.w_uv), eng.scale, ptr(b.attn), c.hidden, stream_ptr())
        if eng.spread_mla:
            entry("mla_prepare_kernel<true> (W_UK absorption over 128 workgroups + new cache row + RoPE)", prepare,
                  moe, 2 * 16 * 128 * 512 + B * 3648 * 2 + B * 16 * 576 * 2)
            entry("mla_attend_kernel (attention + W_UV over heads x W_UV quarters)", attend, moe,
                  2 * 16 * 128 * 512 + kv + B * 16 * 576 * 2 + B * 2048 * 2)

        def qkva_absorb(li):
            L = eng.w.layers[li]
            call("dsv2_qkva_absorb_bf16", ptr(b.h), c.hidden, B, ptr(L.w_qkva), ptr(L.ln_in), c.eps, ptr(L.w_uk),
                 ptr(b.qkva), c.qkva_dim, ptr(b.qlat_part), ptr(eng.cache.layer(li)), ptr(eng.cache.base),
                 ptr(eng.cache.pos), ptr(eng.cache.cap), stream_ptr())

        def attend_parts(li):
            L = eng.w.layers[li]
            call("dsv2_mla_attend_parts", ptr(b.qkva), c.qkva_dim, B, ptr(eng.cache.pos), ptr(eng.cache.base),
                 ptr(eng.cache.cap), ptr(L.kv_norm), c.eps, ptr(eng.cos), ptr(eng.sin), eng.max_pos,
                 ptr(b.qlat_part), ptr(L.w_uv), ptr(eng.cache.layer(li)), eng.scale, ptr(b.attn), c.hidden, None,
                 stream_ptr())
        if eng.absorb_mla:
            entry("qkva_absorb_kernel (q|kv_a projection + W_UK absorption in 8 partial sums per head)",
                  qkva_absorb, moe, 3648 * 2048 * 2 + 2 * 16 * 128 * 512 + B * 16 * 8 * 512 * 4)
            entry("mla_quad_kernel<true> (new row + attention + W_UV from the partial absorbed queries)",
                  attend_parts, moe, 2 * 16 * 128 * 512 + kv + B * 16 * 8 * 512 * 4 + B * 2048 * 2)

        def down(li):
            L = eng.w.layers[li]
            call("dsv2_moe_route_down", ptr(b.hbuf), B, ptr(b.ids32), ptr(b.wts), ptr(L.w_down), ptr(L.sh_down),
                 c.moe_inter, c.top_k + 2, None, ptr(b.h), ptr(b.attn), stream_ptr())

        def down8(li):
            L = eng.w.layers[li]
            call("dsv2_moe_route_down_fp8", ptr(b.hbuf), B, ptr(b.ids32), ptr(b.wts), ptr(L.w_down8),
                 ptr(L.down_scale), ptr(L.sh_down8), ptr(L.sh_down_scale), c.moe_inter, c.top_k + 2, ptr(b.h),
                 ptr(b.attn), stream_ptr())
        n_small = int(torch.unique(b.ids32[:B]).numel()) + 2  # distinct routed experts + 2 shared halves
        if eng.expert_dtype == "fp8":
            entry("route_down_fp8_kernel (6 routed + 2 shared-half down projections on e4m3 weights + combine)",
                  down8, moe, n_small * 2048 * (1408 + 4))
        else:
            entry("route_down_kernel (6 routed + 2 shared-half down projections + combine)", down, moe,
                  n_small * 2048 * 1408 * 2)
        return out
    n_exp = int(torch.unique(b.ids32[:B]).numel())
    R = B * c.top_k
    fp8 = eng.expert_dtype == "fp8"
    shared = fp8 or shared_in_grouped(B, b.tile_tokens)

    def down(li):
        L = eng.w.layers[li]
        if fp8:
            call("dsv2_moe_grouped_down_shared_fp8", ptr(b.hs), B, ptr(b.tiles), ptr(b.ntiles), b.max_tiles,
                 b.tile_tokens, ptr(L.w_down8), ptr(L.down_scale), ptr(b.shmid), ptr(L.sh_down8),
                 ptr(L.sh_down_scale), c.moe_inter, ptr(b.ys), ptr(b.shparts), stream_ptr())
        elif shared:
            call("dsv2_moe_grouped_down_shared", ptr(b.hs), B, ptr(b.tiles), ptr(b.ntiles), b.max_tiles,
                 b.tile_tokens, ptr(L.w_down), ptr(b.shmid), ptr(L.sh_down), c.moe_inter, ptr(b.ys), ptr(b.shparts),
                 stream_ptr())
        else:
            call("dsv2_moe_grouped_down", ptr(b.hs), ptr(b.tiles), ptr(b.ntiles), b.max_tiles, b.tile_tokens,
                 ptr(L.w_down), c.moe_inter, ptr(b.ys), stream_ptr())
    wb = 1 if fp8 else 2  # bytes per weight (e4m3 rows add one fp32 scale each)
    nb = n_exp * 2048 * (1408 * wb + (4 if fp8 else 0)) + R * 1408 * 2 + R * 2048 * 2
    if shared:
        nb += 2048 * (c.shared_inter * wb + (4 if fp8 else 0)) + B * c.shared_inter * 2 + 2 * B * 2048 * 4
    entry("expert-grouped down" + (" on e4m3 weights" if fp8 else "") + (" + the 2 shared-expert halves" if shared else "")
          + f" ({b.tile_tokens}-token tiles)", down, moe, nb)

    if b.max_splits == 1:
        def decode(li):
            call("dsv2_mla_decode_rows", ptr(b.q), ptr(eng.cache.layer(li)), ptr(eng.cache.base), ptr(eng.cache.pos),
                 ptr(eng.cache.cap), B, eng.scale, ptr(b.olat), 16 * 512, stream_ptr())
        entry("mla_decode_kernel<true> (one workgroup per row, normalised o_lat out)", decode, moe,
              kv + B * 16 * 576 * 2 + B * 16 * 512 * 2)
        return out

    def decode(li):
        call("dsv2_mla_decode", ptr(b.q), ptr(eng.cache.layer(li)), ptr(eng.cache.base), ptr(eng.cache.pos),
             ptr(eng.cache.cap), B, b.split_tokens, b.max_splits, eng.scale, ptr(b.part_o), ptr(b.part_ml),
             stream_ptr())
    entry(f"mla_decode_kernel<false> (split-KV, {b.split_tokens}-token splits)", decode, moe,
          kv + B * 16 * 576 * 2 + B * b.max_splits * 16 * 514 * 4)
    return out


CSRC = os.path.join(PKG, "csrc")


def kernel_source_sha(kernel: str) -> str | None:
    """sha256 (16 hex) of the csrc file that defines `kernel` (symbol before any template
    arguments) together with csrc/common.h: a PMC traffic figure measured on other source
    is stale."""
    import hashlib
    import re

    name = kernel.split("<")[0].split(" ")[0]
    pat = re.compile(r"__global__[^;{]*\b" + re.escape(name) + r"\s*\(")
    for fn in sorted(os.listdir(CSRC)):
        if fn.endswith(".hip"):
            txt = open(os.path.join(CSRC, fn), "rb").read()
            if pat.search(txt.decode(errors="replace")):
                h = hashlib.sha256(txt + open(os.path.join(CSRC, "common.h"), "rb").read())
                return h.hexdigest()[:16]
    return None


def measured_traffic(config, kernel: str) -> tuple[float | None, dict]:
    """HBM bytes per launch of the dominant kernel from the committed PMC summary
    profiles/traffic_c<config>.json (written by --pmc-traffic from two rocprofv3 --pmc runs),
    and where that figure comes from.  None when the summary is missing, covers another
    kernel, or was measured on a different source of the kernel (its recorded source sha
    differs from the current file's)."""
    rel = os.path.join("profiles", f"traffic_c{config}.json")
    src = {"profile": rel, "source_sha": kernel_source_sha(kernel)}
    try:
        with open(os.path.join(ROOT, rel)) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None, dict(src, status="missing")
    if not kernel.startswith(t.get("kernel_symbol", "\0")):
        return None, dict(src, status="other kernel")
    if t.get("source_sha") != src["source_sha"]:
        return None, dict(src, status="stale", profiled_source_sha=t.get("source_sha"))
    return t.get("traffic_bytes_per_dispatch"), dict(src, status="measured on this source")


def _csv_rows(path: str):
    import csv
    with open(path, newline="") as f:
        yield from csv.DictReader(f)


# dispatches of the dominant-kernel timing in one bench run: one eager launch, then the
# 26-launch graph replayed 1 + 4 times (time_dominant_kernel)
DOMINANT_DISPATCHES = 1 + 5 * 26


def pmc_traffic(fetch_csv: str, write_csv: str, kernel: str, copy_bytes: int, out: str, command: str) -> dict:
    """Scale the FETCH_SIZE / WRITE_SIZE counters (KiB per dispatch) of the dominant kernel by
    what the same counters read for a plain device copy of copy_bytes (the --copy-calibration
    copies of the profiled run): bytes = counter * copy_bytes / counter(copy).  Only the last
    DOMINANT_DISPATCHES dispatches of the kernel count -- the timing graph's, which `achieved`
    is measured on -- so prefill launches of the same symbol do not mix in."""
    def per_kernel(path: str):
        vals, copies = [], []
        for r in sorted(_csv_rows(path), key=lambda r: int(r["Dispatch_Id"])):
            name = r["Kernel_Name"].replace("void ", "")
            v = float(r["Counter_Value"])
            if name.startswith(kernel):
                vals.append(v)
            elif "copy" in name.lower():
                copies.append(v)
        vals = vals[-DOMINANT_DISPATCHES:]
        copies = sorted(copies[-3:])  # the run ends with the three calibration copies
        if not vals or len(copies) < 3:
            raise SystemExit(f"{path}: no dispatches of {kernel!r} or no calibration copies")
        return sum(vals) / len(vals), len(vals), copies[1]
    f_kib, n_f, f_copy = per_kernel(fetch_csv)
    w_kib, n_w, w_copy = per_kernel(write_csv)
    f_scale, w_scale = copy_bytes / (f_copy * 1024), copy_bytes / (w_copy * 1024)
    res = {"kernel_symbol": kernel, "source_sha": kernel_source_sha(kernel), "command": command,
           "dispatches": [n_f, n_w],
           "fetch_kib_per_dispatch": f_kib, "write_kib_per_dispatch": w_kib,
           "copy_calibration": {"bytes": copy_bytes, "fetch_kib": f_copy, "write_kib": w_copy,
                                "fetch_scale": f_scale, "write_scale": w_scale},
           "traffic_bytes_per_dispatch": f_kib * 1024 * f_scale + w_kib * 1024 * w_scale}
    with open(out, "w") as f:
        json.dump(res, f, indent=1)
        f.write("\n")
    return res


def mfma_summary(counter_csv: str, stats_csv: str, out: str, title: str, command: str, top: int = 12,
                 tail: int | None = None) -> None:
    """rocprofv3 --pmc MfmaUtil SQ_INSTS_VALU_MFMA_MOPS_BF16 counter CSV (one row per dispatch
    and counter) + the kernel_stats.csv of a kernel-trace run of the same command without
    counters -> markdown: per kernel symbol, the MFMA-busy share of the SIMDs (MfmaUtil), the
    bf16 MFMA flops per dispatch (MOPS x 512) and, with the counter-free average duration,
    the achieved TFLOP/s against the 2.5 PFLOP/s dense bf16 peak.  Only the last `tail`
    dispatches of each symbol count (default DOMINANT_DISPATCHES: the bench's timing graph of
    that kernel, after the prefill's dispatches of the same symbol)."""
    import collections

    tail = DOMINANT_DISPATCHES if tail is None else tail
    per = collections.defaultdict(dict)  # name -> dispatch id -> {counter: value}
    for r in _csv_rows(counter_csv):
        name = r["Kernel_Name"].replace("void ", "").split("(")[0]
        per[name].setdefault(int(r["Dispatch_Id"]), {})[r["Counter_Name"]] = float(r["Counter_Value"])
    avg_ns, spans = {}, collections.defaultdict(list)
    for r in _csv_rows(stats_csv):
        if "AverageNs" in r:  # kernel_stats.csv: the average over all dispatches
            avg_ns[r["Name"].replace("void ", "").split("(")[0]] = float(r["AverageNs"])
        else:  # kernel_trace.csv: the last `tail` dispatches, like the counters
            spans[r["Kernel_Name"].replace("void ", "").split("(")[0]].append(
                (int(r["Dispatch_Id"]), int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
    for name, v in spans.items():
        v = sorted(v)[-tail:]
        avg_ns[name] = sum(d for _, d in v) / len(v)
    rows = []
    for name, disp in per.items():
        last = [disp[d] for d in sorted(disp)[-tail:]]
        mops = [x["SQ_INSTS_VALU_MFMA_MOPS_BF16"] for x in last if "SQ_INSTS_VALU_MFMA_MOPS_BF16" in x]
        util = [x["MfmaUtil"] for x in last if "MfmaUtil" in x]
        f = sum(mops) / len(mops) * 512 if mops else 0.0
        u = sum(util) / len(util) if util else float("nan")
        rows.append((f, name, len(last), u, avg_ns.get(name)))
    rows.sort(reverse=True)
    L = [f"# {title}", "", "Commands (from the repo root, on one MI355X):", "", "```", command, "```", "",
         f"Per kernel symbol, the last {tail} dispatches of the counter run (the bench's timing graph of that "
         "kernel: 1 + 5 x 26 launches on the decode step's own activations, after the prefill's dispatches).  "
         "MfmaUtil = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x SIMDs): the share of SIMD cycles the MFMA "
         "unit was busy during the dispatch.  bf16 flops = SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512.  Durations: the "
         f"same last {tail} dispatches of the symbol in the counter-free kernel-trace run.", "",
         "| kernel | dispatches | MfmaUtil % | bf16 MFMA GFLOP / dispatch | avg us | TFLOP/s | % of 2.5 PF |",
         "|---|---:|---:|---:|---:|---:|---:|"]
    for f, name, n, u, ns in rows[:top]:
        if f <= 0:
            continue
        tf = f / (ns * 1e-9) / 1e12 if ns else float("nan")
        L.append(f"| `{name[:70]}` | {n} | {u:.1f} | {f / 1e9:.3f} | "
                 f"{(ns or float('nan')) / 1e3:.1f} | {tf:.1f} | {100 * tf / 2500:.1f} |")
    with open(out, "w") as fh:
        fh.write("\n".join(L) + "\n")


def summarize_trace(db: str, out: str, title: str, command: str, marker: str = "embed_gather") -> None:
    """rocprofv3 rocpd database -> short markdown: per-kernel durations over the whole run and
    one graph-replayed decode step (from one `marker` kernel to the next)."""
    import collections
    import sqlite3
    c = sqlite3.connect(db)
    rows = list(c.execute("select name, start, end from kernels order by start"))

    def short(n: str) -> str:
        return n.split("(")[0].replace("void ", "")[:70]
    st = collections.defaultdict(list)
    for n, a, b in rows:
        st[short(n)].append(b - a)
    tot = sum(sum(v) for v in st.values())
    L = [f"# {title}", "", "Command (from the repo root, on one MI355X):", "", "```", command, "```", "",
         f"Kernel dispatches recorded: {len(rows)}. Durations are rocprofv3 kernel-trace begin/end (ns), averaged "
         "per kernel symbol over the whole run (prefill and the dominant-kernel timing graph included).", "",
         "| kernel | calls | avg us | min us | max us | total ms | % |", "|---|---:|---:|---:|---:|---:|---:|"]
    for n, v in sorted(st.items(), key=lambda kv: -sum(kv[1]))[:25]:
        L.append(f"| `{n}` | {len(v)} | {sum(v) / len(v) / 1e3:.2f} | {min(v) / 1e3:.2f} | {max(v) / 1e3:.2f} | "
                 f"{sum(v) / 1e6:.3f} | {100 * sum(v) / tot:.1f} |")
    idx = [i for i, r in enumerate(rows) if marker in r[0]]
    if len(idx) >= 3:
        a, b = idx[-2], idx[-1]
        seg = rows[a:b]
        wall = seg[-1][2] - seg[0][1]
        per = collections.defaultdict(lambda: [0, 0])
        for r in seg:
            per[short(r[0])][0] += 1
            per[short(r[0])][1] += r[2] - r[1]
        L += ["", f"## One decode step (graph replay {len(idx) - 1} of {len(idx)}, from `{marker}` to the next)", "",
              f"{len(seg)} kernels, {wall / 1e3:.1f} us from first begin to last end "
              f"({sum(r[2] - r[1] for r in seg) / 1e3:.1f} us inside kernels).", "",
              "| kernel | calls/step | us/step |", "|---|---:|---:|"]
        for n, (k, d) in sorted(per.items(), key=lambda kv: -kv[1][1]):
            L.append(f"| `{n}` | {k} | {d / 1e3:.1f} |")
        # one MoE layer in dispatch order (the kernels between the 2nd and 3rd MLA launches)
        mla = [i for i, r in enumerate(seg) if "mla_" in r[0] and ("fused" in r[0] or "prepare" in r[0])]
        if len(mla) >= 3:
            L += ["", "## One MoE layer in dispatch order", "", "| # | kernel | us | gap before us |", "|---:|---|---:|---:|"]
            for k, i in enumerate(range(mla[1], mla[2])):
                r = seg[i]
                gap = (r[1] - seg[i - 1][2]) / 1e3
                L.append(f"| {k} | `{short(r[0])}` | {(r[2] - r[1]) / 1e3:.2f} | {gap:.2f} |")
    with open(out, "w") as f:
        f.write("\n".join(L) + "\n")


def bench_mla_micro(args) -> dict:
    """benchmark config 4: the isolated absorbed-MLA decode (split-KV decode + LSE combine to
    the 16x512 latent output) at bsz=128, per-row KV lengths U[256, 8192] (seed 3), q and the
    compressed cache N(0,1) bf16.  value = cache bytes streamed per second over K graph
    replays of the pair; roofline = the decode kernel alone (HIP events around 26-launch
    graphs, as for the step's dominant kernel)."""
    from triton_kernels._hip import call, ptr, stream_ptr
    from triton_kernels.attention_decode_batch import plan_splits

    import dsv2lite

    cfg = dsv2lite.DSV2Config()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    B = 128
    g = torch.Generator().manual_seed(3)
    lens = torch.randint(256, 8193, (B,), generator=g).tolist()
    base = torch.tensor([0] + list(torch.cumsum(torch.tensor(lens), 0)[:-1].tolist()), dtype=torch.int64)
    cache = torch.randn(sum(lens), 576, generator=g).to(torch.bfloat16).to(dev)
    q = torch.randn(B, 16, 576, generator=g).to(torch.bfloat16).to(dev)
    pos = torch.tensor([n - 1 for n in lens], dtype=torch.int32, device=dev)
    cap = torch.tensor(lens, dtype=torch.int32, device=dev)
    base_d = base.to(dev)
    # the planner with 640 workgroups (5 splits of the longest row), which suits these very
    # unequal lengths (the engine's 256 suits its batches: 320 and 384 made the bsz=64 step
    # 1.5% / 0.7% slower); measured on MI355X, decode kernel: split 1664 (5 splits) 120.3 us,
    # 1728 117.5, 1792 119.6, 1920 121.5, 2048 (4 splits) 126.5, 2304 140.5, 1536 (6 splits)
    # 147.6, 1280 130.3, 3072 169.3
    split, ns = plan_splits(B, max(lens), target_wgs=640)
    if args.mla_split:
        split, ns = args.mla_split, math.ceil(max(lens) / args.mla_split)
    po = torch.empty(B, ns, 16, 512, device=dev)
    pm = torch.empty(B, ns, 16, 2, device=dev)
    olat = torch.empty(B, 16, 512, dtype=torch.bfloat16, device=dev)
    scale = cfg.softmax_scale

    def decode():
        call("dsv2_mla_decode", ptr(q), ptr(cache), ptr(base_d), ptr(pos), ptr(cap), B, split, ns, scale, ptr(po),
             ptr(pm), stream_ptr())

    def pair():
        decode()
        call("dsv2_mla_combine", ptr(po), ptr(pm), ptr(pos), ptr(cap), B, split, ns, None, ptr(olat), 16 * 512,
             stream_ptr())

    def graph_of(fn, n):
        s = torch.cuda.Stream()
        with torch.cuda.stream(s):
            fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for _ in range(n):
                fn()
        return gr

    kb = sum(lens) * 1152 + B * 16 * 576 * 2 + B * ns * 16 * 514 * 4  # cache + q reads, partial writes
    # the K timed steps are one graph of K decode + combine pairs (a graph launch per pair
    # would time the host's launch rate, not the GPU's)
    gw, gk = graph_of(pair, max(args.warmup, 1)), graph_of(pair, args.steps)
    gw.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    gk.replay()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    gd = graph_of(decode, 26)
    gd.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(4):
        gd.replay()
    e1.record()
    torch.cuda.synchronize()
    avg = e0.elapsed_time(e1) / 1e3 / (26 * 4)
    roof = {"kernel": "mla_decode_kernel (split-KV absorbed-MLA decode, MFMA)", "bound": "hbm",
            "achieved": kb / avg / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s", "frac": kb / avg / HBM_PEAK,
            "traffic": None, "bytes_per_launch": kb, "avg_us": avg * 1e6}
    roof["traffic"], roof["traffic_source"] = measured_traffic(4, "mla_decode_kernel")
    value = kb * args.steps / dt / 1e9
    out = {
        "metric": "absorbed-MLA decode kernel: compressed-cache GB/s (benchmark config 4)", "value": round(value, 1),
        "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(dt / args.steps * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic: q and compressed cache N(0,1) bf16, KV lengths U[256,8192] seed 3",
        "config": {"workload": "C4: absorbed-MLA decode microbenchmark, bsz=128, 16 heads, 512+64, split-KV + "
                               "LSE combine", "global_batch": B, "seq_len": max(lens), "kv_tokens": sum(lens),
                   "split_tokens": split, "max_splits": ns, "parallelism": "none (1 GPU)"},
        "roofline": roof,
    }
    if args.copy_calibration:
        _copy_calibration(out, dev)
    if not args.no_cpu_baseline:
        _log("cpu baseline (fp32 attention on the host)")
        torch.set_num_threads(os.cpu_count() or 1)
        qc, cc = q.float().cpu(), cache.float().cpu()
        rows, tc = 0, 0.0
        while tc < 10.0 and rows < B:  # rows in order until about 10 s of host work
            c = cc[int(base[rows]):int(base[rows]) + lens[rows]]
            t0 = time.perf_counter()
            p = torch.softmax((qc[rows] @ c.t()) * scale, dim=-1)
            _ = p @ c[:, :512]
            tc += time.perf_counter() - t0
            rows += 1
        cb = sum(lens[:rows]) * 1152
        out["cpu_baseline"] = {"value": cb / tc / 1e9, "unit": "GB/s", "cores": torch.get_num_threads(),
                               "kind": "port", "sample": f"rows 0-{rows - 1} ({sum(lens[:rows])} cached tokens), "
                                                         f"fp32 torch softmax(q K^T) V on the host, {tc:.2f}s"}
    return out


def device_copy_gbps(dev, nbytes: int = 2**30, reps: int = 10) -> dict:
    """Measured device copy bandwidth (read + write bytes per second of a streaming HBM-to-HBM
    copy, dsv2_stream_copy), the practical ceiling the step fractions are also quoted
    against: a graph of `reps` copies of `nbytes` between HIP events, best of three replays;
    torch's own tensor copy is timed the same way beside it."""
    from triton_kernels._hip import call, ptr, stream_ptr

    src = torch.empty(nbytes // 2, dtype=torch.float16, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    torch_copy = _graph_gbps(lambda: dst.copy_(src), 2 * nbytes, reps)
    gbps = _graph_gbps(lambda: call("dsv2_stream_copy", ptr(src), ptr(dst), nbytes, stream_ptr()), 2 * nbytes, reps)
    ok = bool(torch.equal(dst, src))
    del src, dst
    torch.cuda.empty_cache()
    return {"GBps": gbps, "torch_copy_GBps": torch_copy, "bytes_per_copy": nbytes, "copies": reps, "verified": ok,
            "how": "dsv2_stream_copy (read + write bytes), graph of 10 x 1 GiB, best of 3 replays"}


def _graph_gbps(fn, nbytes: int, reps: int) -> float:
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    best = float("inf")
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        best = min(best, e0.elapsed_time(e1) / 1e3)
    return nbytes * reps / best / 1e9


def in_step_timing(profile: str, kernel: str) -> dict | None:
    """The dominant kernel's average duration inside the graph-replayed step, from the
    committed rocprofv3 step trace (its one-step section), with the source sha the trace was
    recorded on -- beside the live isolated-graph timing of `roofline.avg_us`."""
    path = os.path.join(ROOT, "profiles", profile)
    if not os.path.exists(path):
        return None
    sym = kernel.split(" via ")[0].split(" (")[0].strip()
    in_step = False
    for ln in open(path):
        if ln.startswith("## One decode step"):
            in_step = True
        elif ln.startswith("## "):
            in_step = False
        elif in_step and ln.startswith(f"| `{sym}` |"):  # | kernel | calls/step | us/step |
            cells = [c.strip() for c in ln.strip().strip("|").split("|")]
            try:
                calls, us = int(cells[1]), float(cells[2])
            except (IndexError, ValueError):
                return None
            return {"avg_us": us / calls, "launches_per_step": calls, "profile": f"profiles/{profile}"}
    return None


def _copy_calibration(out: dict, dev) -> None:
    """Three plain 512 MiB device copies at the end of the run: the PMC byte counters of a
    copy of known size scale the dominant kernel's (--pmc-traffic)."""
    src = torch.empty(256 * 2**20, dtype=torch.float16, device=dev).fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    out["copy_calibration_bytes"] = {"read": src.nbytes, "write": dst.nbytes}


def cpu_baseline(max_seconds: float = 30.0) -> dict:
    """Oracle (PyTorch eager, HF math) on the host cores, benchmark config 0."""
    from oracle import dsv2_oracle as O

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    d = O.Dims(n_layers=2)
    w = O.init_weights_cpu(d, n_layers=2, seed=0, with_head=False)
    g = torch.Generator().manual_seed(0)
    m = O.OracleModel(d, w, mode="bf16", max_pos=512)
    moe_w = w["layers"][1]
    cos, sin = m.cos, m.sin
    rb = m.rb
    cache = O.SeqCache()
    h = torch.randn(256, d.hidden, generator=g).to(torch.bfloat16).float()
    t0 = time.perf_counter()
    O.layer_forward(moe_w, d, 1, h, cache, torch.arange(256), cos, sin, rb)
    t_prefill = time.perf_counter() - t0
    steps, t_dec = 0, 0.0
    x = torch.randn(1, d.hidden, generator=g).to(torch.bfloat16).float()
    for i in range(32):
        t0 = time.perf_counter()
        x = O.layer_forward(moe_w, d, 1, x, cache, torch.tensor([256 + i]), cos, sin, rb)
        t_dec += time.perf_counter() - t0
        steps += 1
        if t_dec > max_seconds:
            break
    t_moe = t_dec / steps
    # the dense layer 0 and the lm_head, once each (same oracle), to scale to the whole model
    dense_w = w["layers"][0]
    c0 = O.SeqCache()
    O.layer_forward(dense_w, d, 0, h[:8], c0, torch.arange(8), cos, sin, rb)
    t0 = time.perf_counter()
    O.layer_forward(dense_w, d, 0, x, c0, torch.tensor([8]), cos, sin, rb)
    t_dense = time.perf_counter() - t0
    head = (torch.randn(d.vocab, d.hidden, generator=g) * 0.02).to(torch.bfloat16).float()
    t0 = time.perf_counter()
    _ = O.linear(O.rmsnorm(x, torch.ones(d.hidden), d.eps, rb), head, rb).argmax()
    t_head = time.perf_counter() - t0
    t_tok = 26 * t_moe + t_dense + t_head
    return {"value": 1.0 / t_tok, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": (f"config 0: one MoE layer, prefill 256 ({t_prefill:.2f}s) + {steps} decode steps "
                       f"({t_moe * 1e3:.1f} ms/step); model tok/s = 1/(26*t_moe + t_dense + t_head) with "
                       f"t_dense={t_dense * 1e3:.1f} ms, t_head={t_head * 1e3:.1f} ms; oracle bf16-rounded fp32 math")}


# committed rocprofv3 step traces per config (bench.py --summarize-trace)
STEP_PROFILES = {1: "decode_step_c1_small_bsz1.md", 2: "decode_step_c2_batch_bsz64.md",
                 3: "decode_step_c3_batch_bsz256.md", "r64": "decode_step_r64_reference_workload_bsz64.md",
                 "r256": "decode_step_r256_reference_workload_bsz256.md"}


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def run_config(key, w, args, cfg, dev, expert_dtype: str = "bf16") -> dict:
    """Prefill + K timed graph replays of one benchmark config on already-initialised weights:
    tok/s, ms/step, the step's byte roofline and the dominant kernel's roofline."""
    import dsv2lite

    spec = CONFIGS[key]
    family = args.family or spec["family"]
    g = torch.Generator().manual_seed(spec["seed"])
    lens = spec["prompt"](g)
    if spec.get("replicate"):
        prompts = [torch.randint(0, cfg.vocab, (lens[0],), generator=g)] * len(lens)
    else:
        prompts = [torch.randint(0, cfg.vocab, (n,), generator=g) for n in lens]
    steps, warm = args.steps, args.warmup
    caps = [n + steps + warm + 8 for n in lens]
    eng = dsv2lite.DecodeEngine(w, caps, family=family, mla_path=args.mla_path, expert_dtype=expert_dtype)
    t0 = time.perf_counter()
    eng.prefill([p.to(dev) for p in prompts])
    torch.cuda.synchronize()
    t_prefill = time.perf_counter() - t0
    _log(f"config {key}: prefill of {sum(lens)} tokens done ({t_prefill:.2f}s)")
    snap = eng.snapshot()
    # one recorded eager step: distinct experts per layer (router output) for the byte model
    rec = []
    eng.step(record=rec)
    torch.cuda.synchronize()
    n_exp = [int(torch.unique(r[2]).numel()) for r in rec if r[0] == "router"]
    del rec
    eng.restore(snap)
    for _ in range(warm):
        eng.step()
    torch.cuda.synchronize()
    eng.restore(snap)
    eng.capture()
    eng.restore(snap)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        eng.replay()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    eng.check_errors()
    B = eng.B
    value = B * steps / dt
    ms = dt / steps * 1e3
    # KV rows read per layer per step, averaged over the timed steps (ctx = pos + 1)
    ctx_avg = sum(n + 1 + (steps - 1) / 2 for n in lens)
    sb = step_bytes(cfg, n_exp, ctx_avg, B, expert_dtype == "fp8")
    _log(f"config {key}: timed {steps} graph replays: {ms:.3f} ms/step, {value:.1f} tok/s")
    roof = time_dominant_kernel(eng, family)
    roof["traffic"], roof["traffic_source"] = measured_traffic(key, roof["kernel"])
    prof = STEP_PROFILES.get(key) if expert_dtype == "bf16" else None
    ins = in_step_timing(prof, roof["kernel"]) if prof else None
    if ins:  # the same kernel inside the replayed step (committed trace) beside the live isolated timing
        ins["frac"] = roof["bytes_per_launch"] / (ins["avg_us"] * 1e-6) / HBM_PEAK
        roof["in_step"] = ins
    pos_now = eng.cache.pos.cpu().tolist()
    others = time_other_kernels(eng, family, [p + 1 for p in pos_now])
    res = {"workload": spec["workload"] + (", e4m3 expert weights" if expert_dtype == "fp8" else ""),
           "expert_dtype": expert_dtype, "global_batch": B, "seq_len": max(lens), "kernel_family": family,
           "mla_path": args.mla_path if family == "small" else "split", "prompt_tokens": sum(lens),
           "tok_s": value, "ms_per_step": ms, "steps": steps, "warmup": warm, "kernels_per_step": eng.kernels_per_step,
           "roofline": roof,
           "other_kernels": others,
           "step_roofline": {"bytes_per_step": sb, "achieved_GBps": sb / (ms / 1e3) / 1e9,
                             "frac_of_8TBps": sb / (ms / 1e3) / HBM_PEAK, "distinct_experts_per_layer": n_exp},
           "setup_s": {"prefill": round(t_prefill, 3)}}
    if spec.get("published"):
        res["vs_published_a100"] = round(value / spec["published"], 3)
    del eng
    torch.cuda.empty_cache()
    return res


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=99)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="all", choices=["all"] + [str(k) for k in CONFIGS] + ["4"],
                    help="all (default): config 1 is the line's value, configs 2 and 3 ride along under "
                         "'configs'; N: that config alone")
    ap.add_argument("--family", choices=("small", "batch"), default=None)
    ap.add_argument("--expert-dtype", choices=("bf16", "fp8"), default="bf16",
                    help="one config: MoE expert weights in bf16 or e4m3; 'all' runs C1-C3 both ways")
    ap.add_argument("--mla-path", choices=("fused", "spread", "split", "absorb"), default="absorb",
                    help="small family: the absorption in the q|kv_a projection + one attention launch "
                         "(absorb), prepare + spread attention (two launches), one fused MLA kernel per "
                         "layer, or prepare + split-KV decode + combine")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 3 plain 512 MiB device copies (the reference kernel for scaling the "
                         "FETCH_SIZE / WRITE_SIZE counters of a --pmc run)")
    ap.add_argument("--summarize-trace", nargs=2, metavar=("DB", "OUT_MD"),
                    help="no GPU: summarise a rocprofv3 rocpd database into markdown (with --title/--command)")
    ap.add_argument("--pmc-traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="no GPU: HBM bytes per dispatch of --kernel from two --pmc runs (FETCH_SIZE, WRITE_SIZE) "
                         "scaled by the run's calibration copies; written to --out")
    ap.add_argument("--mfma-summary", nargs=2, metavar=("COUNTER_CSV", "TRACE_CSV"),
                    help="no GPU: MFMA utilisation per kernel from a --pmc MfmaUtil SQ_INSTS_VALU_MFMA_MOPS_BF16 run "
                         "and the kernel_trace.csv of a --kernel-trace run of the same command; markdown to --out")
    ap.add_argument("--mla-split", type=int, default=0, help="config 4: split_tokens override (multiple of 32)")
    ap.add_argument("--kernel", default=None)
    ap.add_argument("--out", default=None)
    ap.add_argument("--title", default="")
    ap.add_argument("--command", default="")
    args = ap.parse_args()
    if args.summarize_trace:
        summarize_trace(args.summarize_trace[0], args.summarize_trace[1], args.title, args.command)
        return
    if args.mfma_summary:
        mfma_summary(args.mfma_summary[0], args.mfma_summary[1], args.out, args.title, args.command)
        return
    if args.pmc_traffic:
        print(json.dumps(pmc_traffic(args.pmc_traffic[0], args.pmc_traffic[1], args.kernel, 512 * 2**20, args.out,
                                     args.command)))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (every box here has one "
              "GPU); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import dsv2lite

    args.config = int(args.config) if args.config.isdigit() else args.config
    if args.config == 4:
        print(json.dumps(bench_mla_micro(args)), flush=True)
        return
    cfg = dsv2lite.DSV2Config()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    t0 = time.perf_counter()
    w = dsv2lite.init_weights(cfg, device=dev, seed=0)
    torch.cuda.synchronize()
    t_init = time.perf_counter() - t0
    _log(f"weights ready ({w.nbytes() / 1e9:.1f} GB, {t_init:.1f}s)")
    head = 1 if args.config == "all" else args.config
    head_dtype = "bf16" if args.config == "all" else args.expert_dtype
    if head_dtype == "fp8":
        dsv2lite.quantize_experts_fp8(w)
    r = run_config(head, w, args, cfg, dev, expert_dtype=head_dtype)
    spec = CONFIGS[head]
    out = {
        "metric": METRIC, "value": round(r["tok_s"], 2), "unit": "tokens/s", "n_gpus": 1, "steps": r["steps"],
        "warmup": r["warmup"], "ms_per_step": round(r["ms_per_step"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": r.get("vs_published_a100"),
        "dtype": "bf16" if head_dtype == "bf16" else "bf16 activations, e4m3 expert weights", "data": "synthetic: random-init weights N(0,0.02) seed 0, uniform random prompt ids"
                                 + (" (one prompt replicated over the batch)" if spec.get("replicate") else ""),
        "config": {"workload": r["workload"], "global_batch": r["global_batch"], "seq_len": r["seq_len"],
                   "kernel_family": r["kernel_family"], "mla_path": r["mla_path"],
                   "prompt_tokens": r["prompt_tokens"], "parallelism": "none (1 GPU)"},
        "roofline": r["roofline"], "step_roofline": r["step_roofline"], "other_kernels": r["other_kernels"],
        "kernels_per_step": r["kernels_per_step"],
        "setup_s": dict(r["setup_s"], init_weights=round(t_init, 2)),
    }
    if args.config == "all":
        # the metric's other two batch sizes, then the reference's own published workload (one
        # prompt replicated over the batch) on the batch family at bsz 64 / 256 and on the small
        # family at bsz 8 / 64 (vs_published_a100 = tok/s / the published A100 figure), timed in
        # the same run on the same weights
        out["configs"] = {}
        for key, name in ((2, "C2"), (3, "C3"), ("r64", "r64"), ("r256", "r256"), ("s8", "s8"), ("s64", "s64")):
            rk = run_config(key, w, args, cfg, dev)
            out["configs"][name] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in rk.items()}
        # benchmark config 4, the isolated absorbed-MLA decode microbenchmark (its own inputs)
        a4 = argparse.Namespace(**vars(args))
        a4.no_cpu_baseline, a4.copy_calibration = True, False
        c4 = bench_mla_micro(a4)
        out["configs"]["C4"] = {k: c4[k] for k in ("metric", "value", "unit", "ms_per_step", "config", "roofline")}
        # configs 1-3 again with the MoE expert weights in e4m3 (per-row power-of-two scales);
        # quantizing rewrites the bf16 experts with their dequantized values, so they run last
        _log("quantizing expert weights to e4m3")
        dsv2lite.quantize_experts_fp8(w)
        for key in (1, 2, 3):
            rk = run_config(key, w, args, cfg, dev, expert_dtype="fp8")
            out["configs"][f"C{key}_fp8"] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in rk.items()}
    # the measured device copy bandwidth and each step's fraction of it (beside the 8 TB/s peak)
    cp = device_copy_gbps(dev)
    out["copy_GBps"] = round(cp["GBps"], 1)
    out["copy"] = cp
    for r in [out] + list(out.get("configs", {}).values()):
        sr = r.get("step_roofline")
        if sr:
            sr["frac_of_copy"] = sr["achieved_GBps"] / cp["GBps"]
    if args.copy_calibration:
        _copy_calibration(out, dev)
    if not args.no_cpu_baseline:
        _log("cpu baseline (oracle, config 0)")
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
