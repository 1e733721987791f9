"""End-to-end decode-step parity on the GPU: the HIP engine (both kernel families,
hipGraph replay) against the CPU oracle on the same seeded random-init weights.

Model: full DeepSeek-V2-Lite widths with 3 layers (layer 0 dense, layers 1-2 MoE)
and the full 102400 vocabulary.  Bars (engine_common): hidden states and logits within
max-rel 2e-2 of both the bf16-rounding and the fp32 oracle; router ids bit-exact wherever
the top-6 margin exceeds 1e-3; greedy tokens identical on >= 95% of teacher-forced steps;
graph replay == eager, bitwise.  Larger batches and contexts: test_gpu_engine_scale.py.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

from engine_common import agree as _agree
from engine_common import build_model
from engine_common import check_trace as _check_trace
from engine_common import close as _close
from engine_common import mean_no_less_exact
from engine_common import oracle_step as _oracle_step
from engine_common import prompts as _prompts

N_LAYERS = 3


@pytest.fixture(scope="module")
def model():
    return build_model(N_LAYERS)


@pytest.mark.parametrize("family,lens,mla", [("small", [16], "split"), ("small", [16], "fused"), ("batch", [16], "split"),
                                             ("small", [16], "spread"), ("small", [5, 11], "spread"),
                                             ("small", [16], "absorb"), ("small", [5, 11], "absorb"),
                                             ("small", [5, 11], "split"), ("small", [5, 11], "fused"),
                                             ("batch", [5, 16, 9, 1], "split")])
def test_engine_decode_vs_oracle(model, family, lens, mla):
    import dsv2lite

    cfg, w, om = model
    B = len(lens)
    eng = dsv2lite.DecodeEngine(w, [n + 16 for n in lens], family=family, mla_path=mla)
    prompts = _prompts(lens, seed=7 + B)
    prec = []
    first = eng.prefill([p.cuda() for p in prompts], record=prec).cpu().clone()
    torch.cuda.synchronize()
    caches = [om.new_cache() for _ in range(B)]
    agree = total = router_checked = 0
    toks = []
    # prefill: first greedy token and last-position logits
    for b in range(B):
        res, tr = _oracle_step(om, caches[b], prompts[b], 0)
        ref = res["logits"][-1]
        _, flipped = _check_trace(om, prec, tr, b, ("prefill", b), res)
        _close(eng.logits[b].cpu(), ref, res["fp32"]["logits"][-1], flipped, ("prefill", b))
        toks.append(int(torch.argmax(ref)))
        agree += _agree(int(first[b]), ref, eng.logits[b].cpu(), ("prefill", b))
        total += 1
    # teacher-forced decode steps: both sides consume the oracle's greedy token
    steps = 6
    for s in range(steps):
        eng.ids.copy_(torch.tensor(toks, dtype=torch.int64))
        rec = []
        eng.step(record=rec)
        torch.cuda.synchronize()
        new = []
        for b in range(B):
            res, trace = _oracle_step(om, caches[b], torch.tensor([toks[b]]), lens[b] + s)
            ref = res["logits"][-1]
            n_clear, flipped = _check_trace(om, rec, trace, b, (family, s, b), res)
            router_checked += n_clear
            _close(eng.logits[b].cpu(), ref, res["fp32"]["logits"][-1], flipped, (family, s, b))
            o_tok = int(torch.argmax(ref))
            agree += _agree(int(eng.ids[b].item()), ref, eng.logits[b].cpu(), (family, s, b))
            total += 1
            new.append(o_tok)
        toks = new
    assert eng.cache.pos.cpu().tolist() == [n + steps for n in lens]
    assert router_checked >= steps * B  # most (layer, step) pairs have a clear top-6
    # every disagreement was verified to be a near-tie in _agree; the >= 95% rate itself is
    # asserted on the longer 40-step run below
    print(f"{family} {lens}: greedy agreement {agree}/{total}", flush=True)


@pytest.mark.parametrize("family,mla", [("small", "fused"), ("small", "spread"), ("small", "absorb"),
                                        ("batch", "split")])
def test_graph_replay_equals_eager_bitwise(model, family, mla):
    import dsv2lite

    cfg, w, _ = model
    lens = [12, 7, 20]
    eng = dsv2lite.DecodeEngine(w, [n + 16 for n in lens], family=family, mla_path=mla)
    assert eng.mla_path == mla
    eng.prefill([p.cuda() for p in _prompts(lens, seed=3)])
    snap = eng.snapshot()
    eager = []
    for _ in range(3):
        eng.step()
        eager.append((eng.logits.clone(), eng.ids.clone()))
    eng.restore(snap)
    eng.capture()
    for rep in range(2):  # replays from the same state, with eager work in between
        eng.restore(snap)
        torch.cuda.synchronize()
        for i in range(3):
            eng.replay()
            torch.cuda.synchronize()
            assert torch.equal(eng.logits, eager[i][0]), (rep, i)
            assert torch.equal(eng.ids, eager[i][1]), (rep, i)
        _ = (eng.logits.sum() * 0).item()
    assert eng.cache.pos.cpu().tolist() == [n + 3 for n in lens]


def test_step_is_deterministic_and_capacity_guard(model):
    import dsv2lite

    cfg, w, _ = model
    eng = dsv2lite.DecodeEngine(w, [10], family="small")
    eng.prefill([_prompts([8], seed=9)[0].cuda()])
    snap = eng.snapshot()
    eng.step()
    a = eng.logits.clone()
    eng.restore(snap)
    eng.step()
    assert torch.equal(a, eng.logits)
    eng.step()  # position 9 = last slot
    with pytest.raises(RuntimeError, match="capacity"):
        eng.step()
    eng.check_errors()  # the host refused the step: nothing reached the kernels
    # positions moved behind the host's back: the kernels skip the write and flag it
    eng._host_pos = [0]
    full = eng.cache.data.clone()
    eng.step()
    torch.cuda.synchronize()
    assert torch.equal(eng.cache.data, full)
    with pytest.raises(RuntimeError, match="capacity exhausted"):
        eng.check_errors()
    eng.check_errors()  # cleared once reported


@pytest.mark.parametrize("family", ["small", "batch"])
def test_greedy_agreement_teacher_forced_40_steps(model, family):
    """greedy tokens identical on >= 95% of (teacher-forced) steps."""
    import dsv2lite

    cfg, w, om = model
    eng = dsv2lite.DecodeEngine(w, [64], family=family)
    prompt = _prompts([12], seed=21)[0]
    eng.prefill([prompt.cuda()])
    cache = om.new_cache()
    res, _ = _oracle_step(om, cache, prompt, 0)
    tok = int(torch.argmax(res["logits"][-1]))
    agree = 0
    steps = 40
    errs: list = []
    for s in range(steps):
        eng.ids.fill_(tok)
        rec = []
        eng.step(record=rec)
        res, tr = _oracle_step(om, cache, torch.tensor([tok]), 12 + s)
        ref = res["logits"][-1]
        _, flipped = _check_trace(om, rec, tr, 0, (family, s), res, errs)
        _close(eng.logits[0].cpu(), ref, res["fp32"]["logits"][-1], flipped, (family, s), errs)
        agree += _agree(int(eng.ids[0].item()), ref, eng.logits[0].cpu(), (family, s))
        tok = int(torch.argmax(ref))
    print(f"{family} ({eng.mla_path} MLA): greedy agreement {agree}/{steps}", flush=True)
    assert agree / steps >= 0.95, (agree, steps)
    mean_no_less_exact(errs, (family, eng.mla_path))


@pytest.mark.parametrize("family,bsz", [("small", 1), ("batch", 3)])
def test_run_cli_end_to_end(family, bsz):
    """src/run.py (the reference's CLI surface) runs the captured decode on the GPU with a
    3-layer random-init model: prefill, graph replays, JSON result with the reference's keys
    and the requested number of generated tokens per row."""
    from src import run as R

    out = R.main(["--kernel-family", family, "--batch-size", str(bsz), "--layers", "3", "--max-new-tokens", "5",
                  "--prompt-len", "16", "--dump-token-ids"])
    assert out["batch_size"] == bsz and out["tps"] > 0 and out["decode_tokens"] > 0
    assert out["path"] == R.PATH_NAMES[family]
    ids = out["generated_token_ids"]
    ids = [ids] if bsz == 1 else ids  # the reference's JSON keeps one row flat (run.py:691-705)
    assert len(ids) == bsz and all(len(r) == 5 for r in ids)
    assert all(0 <= t < 102400 for r in ids for t in r)


def test_bench_json_contract():
    """bench.py (the driver's entry point) prints ONE JSON line with the contract's keys, a
    roofline object for the dominant kernel, the bsz=64 / 256 configs under "configs", and
    (here skipped) no cpu_baseline."""
    import json
    import math
    import os
    import subprocess
    import sys

    from golden_utils import ROOT

    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--steps", "3", "--warmup", "1", "--no-cpu-baseline"],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.strip()]
    assert len(lines) == 1
    d = json.loads(lines[0])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
              "vs_baseline", "dtype", "data", "config", "roofline"):
        assert k in d, k
    assert d["n_gpus"] == 1 and d["steps"] == 3 and d["value"] > 0 and "workload" in d["config"]
    roof = d["roofline"]
    assert roof["bound"] == "hbm" and roof["unit"] == "GB/s" and 0 < roof["frac"] < 1
    assert math.isclose(roof["frac"], roof["achieved"] / roof["peak"], rel_tol=1e-9)
    assert roof["traffic_source"]["status"] in ("measured on this source", "stale", "missing", "other kernel")
    # the metric's bsz=64 and bsz=256 ride along, timed in the same run
    for key, B in (("C2", 64), ("C3", 256)):
        c = d["configs"][key]
        assert c["global_batch"] == B and c["kernel_family"] == "batch" and c["steps"] == 3
        assert math.isclose(c["tok_s"], B * 1e3 / c["ms_per_step"], rel_tol=1e-3)
        r = c["roofline"]
        assert 0 < r["frac"] < 1 and math.isclose(r["frac"], r["achieved"] / r["peak"], rel_tol=1e-3)
        sr = c["step_roofline"]
        assert math.isclose(sr["frac_of_8TBps"], sr["bytes_per_step"] / (c["ms_per_step"] / 1e3) / 8e12, rel_tol=1e-3)
