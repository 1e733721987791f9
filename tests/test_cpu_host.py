"""Host-side checks that run without a GPU: the C-ABI library loads and exports every
symbol the header declares, wrappers reject what the reference rejects, and the
product's host math (RoPE tables, softmax scale, split planning, cache layout)
matches the oracle."""

from __future__ import annotations

import math
import os
import re

import pytest
import torch

import oracle.dsv2_oracle as O
from golden_utils import ROOT


def _header_symbols():
    txt = open(os.path.join(ROOT, "include", "dsv2lite.h")).read()
    return sorted(set(re.findall(r"\b(dsv2_[a-z0-9_]+)\s*\(", txt)))


def test_library_exports_every_header_symbol():
    from triton_kernels import _hip

    syms = _header_symbols()
    assert len(syms) >= 20
    for s in syms:
        assert hasattr(_hip.lib, s), s
    assert sorted(_hip.EXPORTS) == syms
    assert _hip.lib.dsv2_abi_version() == _hip.ABI_VERSION


def test_abi_rejects_bad_arguments_without_launching():
    from triton_kernels import _hip

    with pytest.raises(_hip.HipKernelError, match="null pointer"):
        _hip.call("dsv2_rmsnorm_bf16", None, 0, None, None, 0, 1, 2048, 1e-6, None)
    with pytest.raises(_hip.HipKernelError, match="bad shape"):
        _hip.call("dsv2_gemv_bf16", 16, 2048, 1, 2047, 16, 64, None, 0.0, None, 0, 16, 64, 0, None)
    with pytest.raises(_hip.HipKernelError, match="max_splits"):
        _hip.call("dsv2_mla_decode", 16, 16, 16, 16, 16, 1, 32, 65, 0.1, 16, 16, None)
    with pytest.raises(_hip.HipKernelError, match="null pointer"):  # the per-row capacity is required
        _hip.call("dsv2_mla_decode", 16, 16, 16, 16, None, 1, 32, 4, 0.1, 16, 16, None)
    with pytest.raises(_hip.HipKernelError, match="null pointer"):
        _hip.call("dsv2_mla_prepare", 16, 3648, 1, 16, 16, None, 16, 1e-6, 16, 16, 64, None, 16, 16, None, None)
    with pytest.raises(_hip.HipKernelError, match="null pointer"):  # the absorption weights are required
        _hip.call("dsv2_mla_prepare_qlat", 16, 3648, 1, 16, 16, 16, 16, 1e-6, 16, 16, 64, None, 16, 16, None, None)
    with pytest.raises(_hip.HipKernelError, match="rows\\*6"):
        _hip.call("dsv2_moe_bucket", 16, 8193, 32, 16, 16, 16, 16, None)


def test_wrappers_reject_cpu_tensors_like_the_reference():
    from triton_kernels.attention_prepost import residual_add_triton
    from triton_kernels.mlp_elementwise import silu_mul_triton
    from triton_kernels.moe_router import router_softmax_topk6_triton
    from triton_kernels.rmsnorm import rmsnorm_triton

    x = torch.zeros(2, 2048, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        rmsnorm_triton(x, torch.ones(2048, dtype=torch.bfloat16), 1e-6)
    with pytest.raises(NotImplementedError):
        residual_add_triton(x, x)
    with pytest.raises(NotImplementedError):
        silu_mul_triton(x, x)
    with pytest.raises(NotImplementedError):
        router_softmax_topk6_triton(torch.zeros(1, 64), 1.0)


def test_product_rope_and_scale_match_oracle():
    from dsv2lite.config import DSV2Config
    from dsv2lite.rope import cos_sin_tables, inv_freq

    cfg = DSV2Config()
    d = O.Dims()
    assert torch.equal(inv_freq(cfg), O.yarn_inv_freq(d))
    cos, sin = cos_sin_tables(cfg, 3000)
    ocos, osin = O.yarn_cos_sin(d, 3000, mode="bf16")
    assert torch.equal(cos.float(), ocos) and torch.equal(sin.float(), osin)
    assert abs(cfg.softmax_scale - O.softmax_scale(d)) < 1e-12
    assert cfg.qkva_dim == 3648 and cfg.cache_row == 576


@pytest.mark.parametrize("rows,ctx", [(1, 10), (1, 236), (64, 57), (64, 256), (64, 257), (64, 1130), (256, 2160),
                                      (128, 8200), (1024, 2176), (3, 100000)])
def test_plan_splits(rows, ctx):
    from dsv2lite.engine import plan_splits

    split, ns = plan_splits(rows, ctx)
    assert split % 32 == 0 and 1 <= ns <= 64
    assert split * ns >= ctx and split * (ns - 1) < ctx
    if ctx <= 256:  # short caches: one split per row (the one-launch decode, no merge)
        assert ns == 1


def test_moe_tile_choice_and_cache_layout():
    from dsv2lite.cache import CompressedKVCache
    from dsv2lite.engine import moe_tile_tokens

    assert moe_tile_tokens(1) == 16 and moe_tile_tokens(16) == 16 and moe_tile_tokens(64) == 32
    assert moe_tile_tokens(256) == 64 and moe_tile_tokens(512) == 64
    from dsv2lite.engine import routing_load, tile_tokens_for_load

    g = torch.Generator().manual_seed(0)
    uniform = torch.stack([torch.randperm(64, generator=g)[:6] for _ in range(64)])
    same = torch.tensor([7, 16, 25, 34, 43, 52]).repeat(64, 1)
    assert 6 < routing_load(uniform) < 10 and tile_tokens_for_load(routing_load(uniform)) == 32
    assert routing_load(same) == 64 and tile_tokens_for_load(routing_load(same)) == 64
    assert tile_tokens_for_load(24.5) == 64 and tile_tokens_for_load(2.0) == 16
    assert tile_tokens_for_load(384, 2304) == 64 and tile_tokens_for_load(96, 6144) == 256
    assert moe_tile_tokens(853) == 64 and moe_tile_tokens(854) == 256 and moe_tile_tokens(8192) == 256
    from dsv2lite.engine import shared_in_grouped

    assert shared_in_grouped(64, 16) and shared_in_grouped(64, 64) and shared_in_grouped(256, 64)
    assert not shared_in_grouped(256, 32) and not shared_in_grouped(256, 16) and shared_in_grouped(100, 32)
    c = CompressedKVCache(2, [5, 7, 3], device="cpu")
    assert c.base.tolist() == [0, 5, 12] and c.total == 15 and c.data.shape == (2, 15, 576)
    # long rows: starts staggered by (7 b mod 8) 32-token tiles inside slots of capacity + 224
    s = CompressedKVCache(1, [600, 700, 600], device="cpu")
    assert s.base.tolist() == [0, 824 + 224, 824 + 924 + 192] and s.total == 824 + 924 + 824
    ends = [int(b) + c for b, c in zip(s.base.tolist(), s.capacities)]
    assert ends[0] <= s.base[1] and ends[1] <= s.base[2] and ends[2] <= s.total
    c.pos.copy_(torch.tensor([1, 2, 3], dtype=torch.int32))
    snap = c.snapshot()
    c.pos.add_(4)
    c.restore(snap)
    assert c.pos.tolist() == [1, 2, 3]


def test_engine_rejects_unknown_family_and_dims():
    from dsv2lite.config import DSV2Config
    from dsv2lite.engine import DecodeEngine

    with pytest.raises(ValueError, match="Unknown kernel family"):
        DecodeEngine(None, [8], family="tiny")
    with pytest.raises(ValueError, match="specialised"):
        DSV2Config(hidden=1024).check_kernel_dims()


def test_weights_hf_views_roundtrip_cpu():
    from dsv2lite.config import DSV2Config
    from dsv2lite.weights import init_weights, pack_hf_layer

    cfg = DSV2Config(n_layers=1, vocab=128, dense_inter=128)
    w = init_weights(cfg, device="cpu", seed=0)
    hf = w.hf_layer(0)
    assert hf["q_proj"].shape == (3072, 2048) and hf["kv_b_proj"].shape == (4096, 512)
    L = pack_hf_layer(cfg, hf, device="cpu")
    assert torch.equal(L.w_qkva, w.layers[0].w_qkva) and torch.equal(L.w_uk, w.layers[0].w_uk)
    assert torch.equal(L.w_ukt, w.layers[0].w_uk.transpose(1, 2))
    std = float(w.layers[0].w_qkva.float().std())
    assert abs(std - 0.02) < 1e-3


def test_run_cli_parsing_matches_reference_rules():
    """src/run.py keeps the reference's flag rules (run.py:53-57, 239-249)."""
    from src import run as R

    a = R.parse_args(["--batch-sizes", "1, 2，4", "--kernel-family", "small"])
    assert R.parse_batch_sizes(a) == [1, 2, 4]
    assert R.parse_batch_sizes(R.parse_args([])) == [1]
    with pytest.raises(ValueError, match="batch size must be positive"):
        R.parse_batch_sizes(R.parse_args(["--batch-sizes", "2 0"]))
    with pytest.raises(ValueError, match="max_new_tokens must be positive"):
        R.parse_batch_sizes(R.parse_args(["--max-new-tokens", "0"]))
    with pytest.raises(ValueError, match="Unknown kernel family"):
        R.set_kernel_family("tiny")
    with pytest.raises(SystemExit):
        R.parse_args(["--kernel-family", "tiny"])
    c2 = R.parse_args(["--config", "2"])
    assert c2.batch_sizes == [64] and c2.kernel_family == "batch" and c2.prompt_len_range == (256, 1024)
    p = R.make_prompts(c2, 64, 102400)
    assert len(p) == 64 and all(256 <= x.numel() <= 1024 for x in p) and len({x.numel() for x in p}) > 1
    rep = R.make_prompts(R.parse_args(["--prompt-len", "24"]), 3, 1000)
    assert all(torch.equal(rep[0], x) for x in rep) and rep[0].numel() == 24
    r = R.build_result({"batch_size": 2, "path": "hip_batching_graph", "prefill_seconds": 0.5, "decode_seconds": 2.0,
                        "decode_tokens": 198, "generated_ids": [[1], [2]], "step_trace": [], "prompt_lens": [24, 24],
                        "hbm_bytes_per_step": 8e9, "kernels_per_step": 300, "steps": 99},
                       True, False)
    assert r["tps"] == 99.0 and r["ttft_ms"] == 500.0 and r["prompt_lens"] == 24 and "step_trace" not in r
    # the run report's roofline fields: bytes per step / mean step time / 8 TB/s
    assert r["kernels_per_step"] == 300 and math.isclose(r["roofline_fraction"], 8e9 / (2.0 / 99) / 8e12)


def test_run_cli_needs_gpu():
    from src import run as R

    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="GPU is required"):
            R.main([])
        with pytest.raises(RuntimeError, match="GPU is required"):
            R.main(["--model-path", "/data/models/DeepSeek-V2-Lite-Chat"])
    assert R.parse_args([]).prompt == "Write me a 500 word novel."  # the reference's default (run.py:17)


def test_bench_pmc_traffic_scaling_and_tail(tmp_path):
    """bench.py --pmc-traffic: per-dispatch counters of the kernel scaled by the calibration
    copies; only the last DOMINANT_DISPATCHES dispatches of the kernel count (the timing
    graph's), so earlier launches of the same symbol (prefill) do not mix in."""
    import csv
    import importlib
    import sys

    sys.path.insert(0, str(ROOT))
    bench = importlib.import_module("bench")
    n = bench.DOMINANT_DISPATCHES

    def write(path, per_kernel, copy_kib):
        rows, d = [], 0
        for v in [10_000.0] * 7 + [per_kernel] * n:  # 7 prefill launches with other counts
            d += 1
            rows.append({"Dispatch_Id": d, "Kernel_Name": "void mykernel<1>(Args)", "Counter_Value": v})
        for v in copy_kib:
            d += 1
            rows.append({"Dispatch_Id": d, "Kernel_Name": "__amd_rocclr_copyBuffer", "Counter_Value": v})
        with open(path, "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Value"])
            w.writeheader()
            w.writerows(rows)

    fpath, wpath = tmp_path / "f.csv", tmp_path / "w.csv"
    write(fpath, 1000.0, [262144.0, 262145.0, 262146.0])  # 512 MiB copy reads 256 MiB-worth: scale 2
    write(wpath, 10.0, [524288.0] * 3)
    res = bench.pmc_traffic(str(fpath), str(wpath), "mykernel<1>", 512 * 2**20, str(tmp_path / "t.json"), "cmd")
    assert res["dispatches"] == [n, n]
    assert res["fetch_kib_per_dispatch"] == 1000.0 and res["write_kib_per_dispatch"] == 10.0
    f_scale = 512 * 2**20 / (262145.0 * 1024)
    assert math.isclose(res["traffic_bytes_per_dispatch"], 1000.0 * 1024 * f_scale + 10.0 * 1024, rel_tol=1e-12)


def test_bench_refuses_more_than_one_gpu():
    """bench.py --gpus N>1 exits with a message before touching a GPU (this build measures one)."""
    import subprocess
    import sys

    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr and r.stdout == ""


def test_run_cli_config3_draws_one_prompt_per_row():
    """--config 3 (bsz=256 x 2048) gives every row its own random prompt, like bench.py's
    C3; the reference workload (no --config, fixed --prompt-len) replicates one prompt."""
    from src import run as R

    a = R.parse_args(["--config", "3"])
    ps = R.make_prompts(a, 4, 102400)
    assert all(p.numel() == 2048 for p in ps)
    assert len({tuple(p[:16].tolist()) for p in ps}) == 4
    b = R.parse_args(["--batch-size", "3", "--prompt-len", "24"])
    qs = R.make_prompts(b, 3, 102400)
    assert all(torch.equal(q, qs[0]) for q in qs)


def test_engine_capacity_check_is_per_row():
    """A row whose next position reaches its own capacity stops the step even when another
    row still has room (capacities [n+2, n+64]: the first row fills after 2 steps)."""
    from types import SimpleNamespace

    from dsv2lite.engine import DecodeEngine

    eng = object.__new__(DecodeEngine)
    eng.cache = SimpleNamespace(capacities=[12, 74])
    eng._free = set()
    eng._host_pos = [10, 10]
    eng._check_room()  # slot 10 < 12 for row 0
    eng._host_pos = [11, 11]
    eng._check_room()  # slot 11, the last of row 0
    eng._host_pos = [12, 12]
    with pytest.raises(RuntimeError, match="rows \\[0\\]"):
        eng._check_room()


def test_bench_traffic_is_reported_only_for_the_profiled_source(tmp_path, monkeypatch):
    """A committed PMC traffic figure is used only while the kernel's source file (and
    common.h) hash to the sha recorded when it was measured; otherwise traffic is null and
    traffic_source says why."""
    import importlib
    import json
    import sys

    sys.path.insert(0, str(ROOT))
    bench = importlib.import_module("bench")
    sha = bench.kernel_source_sha("route_gateup_kernel<2>")
    assert sha and sha == bench.kernel_source_sha("route_gateup_kernel<1>")
    assert bench.kernel_source_sha("gemm_dma_kernel<true>") != sha  # defined in another file
    assert bench.kernel_source_sha("no_such_kernel") is None
    prof = tmp_path / "profiles"
    prof.mkdir()
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    rec = {"kernel_symbol": "route_gateup_kernel<2>", "source_sha": sha, "traffic_bytes_per_dispatch": 123.0}
    (prof / "traffic_c1.json").write_text(json.dumps(rec))
    t, src = bench.measured_traffic(1, "route_gateup_kernel<2> (small-family MoE)")
    assert t == 123.0 and src["status"] == "measured on this source"
    (prof / "traffic_c1.json").write_text(json.dumps(dict(rec, source_sha="0" * 16)))
    t, src = bench.measured_traffic(1, "route_gateup_kernel<2> (small-family MoE)")
    assert t is None and src["status"] == "stale"
    t, src = bench.measured_traffic(2, "gemm_dma_kernel<true>")
    assert t is None and src["status"] == "missing"


def test_bench_mfma_summary_uses_the_timing_graph_dispatches(tmp_path):
    """--mfma-summary keeps, per kernel symbol, only the last DOMINANT_DISPATCHES dispatches
    (the bench's timing graph), both for the counters and for the trace durations."""
    import csv
    import importlib
    import sys

    sys.path.insert(0, str(ROOT))
    bench = importlib.import_module("bench")
    n = bench.DOMINANT_DISPATCHES
    crow, trow, d = [], [], 0
    for k, (mops, util, dur) in enumerate([(1.0, 90.0, 1000)] * 5 + [(1000.0, 10.0, 2000)] * n):
        d += 1
        crow.append({"Dispatch_Id": d, "Kernel_Name": "void kern<1>(int)", "Counter_Name": "MfmaUtil",
                     "Counter_Value": util})
        crow.append({"Dispatch_Id": d, "Kernel_Name": "void kern<1>(int)", "Counter_Name": "SQ_INSTS_VALU_MFMA_MOPS_BF16",
                     "Counter_Value": mops})
        trow.append({"Dispatch_Id": d, "Kernel_Name": "void kern<1>(int)", "Start_Timestamp": 10 * d,
                     "End_Timestamp": 10 * d + dur})
    for path, rows in ((tmp_path / "c.csv", crow), (tmp_path / "t.csv", trow)):
        with open(path, "w", newline="") as f:
            w = csv.DictWriter(f, fieldnames=list(rows[0]))
            w.writeheader()
            w.writerows(rows)
    out = tmp_path / "m.md"
    bench.mfma_summary(str(tmp_path / "c.csv"), str(tmp_path / "t.csv"), str(out), "t", "cmd")
    line = [ln for ln in out.read_text().splitlines() if ln.startswith("| `kern<1>`")][0]
    cells = [c.strip() for c in line.strip("|").split("|")]
    assert cells[1] == str(n) and cells[2] == "10.0"
    assert float(cells[3]) == round(1000 * 512 / 1e9, 3) and cells[4] == "2.0"


def test_prefill_tiles_cover_every_row_once():
    """The prefill attention's query tiles: <= 128 consecutive rows of one sequence each, every
    chunk row in exactly one tile with its own position and its sequence's cache base; the
    expanded range spans every key any row attends."""
    from dsv2lite.engine import prefill_tiles

    lens = [100, 3, 64, 130]
    bases = [0, 200, 300, 500]
    seq = torch.cat([torch.full((n,), b, dtype=torch.int64) for b, n in enumerate(lens)])
    posv = torch.cat([torch.arange(n, dtype=torch.int32) for n in lens])
    # a chunk that starts inside sequence 0 (positions 40..) and ends inside sequence 3
    s, e = 40, 100 + 3 + 64 + 70
    t, lo, n = prefill_tiles(seq[s:e], posv[s:e], bases)
    seen = torch.zeros(e - s, dtype=torch.int32)
    for r0, nr, p0, sb in t.tolist():
        assert 1 <= nr <= 128
        rows = torch.arange(r0, r0 + nr)
        assert len(set(seq[s:e][rows].tolist())) == 1
        b = int(seq[s + r0])
        assert sb == bases[b] and torch.equal(posv[s:e][rows], torch.arange(p0, p0 + nr, dtype=torch.int32))
        seen[rows] += 1
        assert lo <= sb and sb + p0 + nr <= lo + n  # every key of the tile's rows is expanded
    assert torch.all(seen == 1)
    assert lo == 0 and lo + n == 500 + 70


def test_prefill_groups_bound_the_expansion_by_the_rows_attended():
    """Slots far apart (capacity 32768, 100-token prompts): the chunk's attention is planned in
    groups whose expanded cache range is at most twice the rows they attend plus the slack,
    instead of one range over every slot's unused capacity (64 x 32768 rows); the groups
    together cover every chunk row exactly once.  Slots packed closely stay one group."""
    from dsv2lite.engine import prefill_groups, prefill_tiles

    def plan(lens, caps, slack=4096):
        bases = [0]
        for c in caps[:-1]:
            bases.append(bases[-1] + c)
        seq = torch.cat([torch.full((n,), b, dtype=torch.int64) for b, n in enumerate(lens)])
        posv = torch.cat([torch.arange(n, dtype=torch.int32) for n in lens])
        return seq, posv, bases, prefill_groups(seq, posv, bases, slack=slack)

    lens = [100] * 64
    seq, posv, bases, groups = plan(lens, [32768] * 64)
    seen = torch.zeros(seq.numel(), dtype=torch.int32)
    total_exp = 0
    for tiles, lo, n in groups:
        used = 0
        for r0, nr, p0, sb in tiles.tolist():
            seen[r0:r0 + nr] += 1
            assert lo <= sb and sb + p0 + nr <= lo + n  # every key of the tile's rows is expanded
            used += nr
        assert n <= 2 * used + 4096
        total_exp += n
    assert torch.all(seen == 1)
    assert total_exp <= 64 * 100 + 64 * 4096 and total_exp < 64 * 32768 // 4
    # bench-like capacities (prompt + a few tokens): one group, the same plan as prefill_tiles
    seq, posv, bases, groups = plan([2048] * 4, [2081] * 4)
    assert len(groups) == 1
    t, lo, n = prefill_tiles(seq, posv, bases)
    assert torch.equal(groups[0][0], t) and groups[0][1:] == (lo, n)
