"""Parity of the model the benchmark times: all 27 layers, full width, the full 102,400-word
vocabulary, random-init weights from seed 0 (bench.py's model), against the CPU oracle.

Two workloads, both with their graph captured and replayed (replay == eager, bitwise, is
checked first; the steps below run eagerly with per-layer records):
  C1 -- bsz=1, the 128-token prompt of seed 1, small kernel family (bench config 1);
  C3 -- bsz=256, 2,048-token prompts of seed 2, batch family (bench config 3); rows 0 and
        137 are checked (every row of the batch runs).

The oracle runs in both modes (HF's bf16 rounding points and exact fp32 math) layer by
layer: each pass pulls one layer's weights from the device to the host in fp32, runs it for
the three checked sequences, and frees it (StreamedOracle), so the host holds ~2.5 GB of
weights at a time instead of ~62 GB.

1. Layer by layer, the north-star bars.  After the prefill and STEPS decode steps, every
   decode step is re-run with each layer's input forced to the oracle's input of that layer
   and the checked rows' compressed cache holding the oracle's rows: each of the 27 layers
   (attention + residual, MoE/MLP + residual), the router and the head (final norm,
   lm_head, argmax on the oracle's last hidden state) are then compared with the oracle's
   same layer on the same input -- hidden states (after the attention and after the MLP)
   and logits within max-rel 2e-2 of the bf16 oracle, router ids exact on the kernel's own
   input where the top-6 margin exceeds 1e-3 and any other flip explained by the two
   inputs' logit difference, greedy tokens equal on >= 95% of the points (every miss a
   verified near-tie).  The distance from exact math is printed, not asserted here: the
   fp32 oracle's layer input is its own trajectory's, not the forced one.

2. Free running (the engine's own hidden states, teacher-forced by token only): bf16
   rounding differences compound over 27 random-init layers for ANY arithmetic -- HF's own
   bf16 arithmetic is up to ~5e-2 from exact math at the last layers, and the same rounding
   points with only the linears' summation order changed drift ~4e-2 from HF (a CPU
   experiment on a model of this shape).  So here every point must stay within
   max(2e-2, 2 x HF's own distance from exact math at that point) of exact math (2.5 x against
   the bf16 oracle), and the mean distance from exact math over all points may exceed HF's
   own mean by at most 10%: the kernels are as accurate as the reference's arithmetic.
   Router flips must be explained by the measured input difference; greedy misses must be
   verified near-ties.  Per-layer maxima / means and every accepted flip are printed.
"""

from __future__ import annotations

import time

import pytest
import torch

pytestmark = pytest.mark.gpu

from engine_common import BAR, FP32_BAR, NEAR_TIE_BAR, StreamedOracle, agree, router_flips
from golden_utils import rel_err

STEPS = 6
C3_ROWS = [0, 137]
DRIFT_POINT = 2.0     # free running: distance from exact math <= this x HF's own, per point
DRIFT_POINT_HF = 2.5  # free running: distance from HF's bf16 arithmetic, per point
DRIFT_MEAN = 1.10     # free running: mean distance from exact math <= this x HF's own mean


@pytest.fixture(scope="module")
def full_model():
    import dsv2lite

    cfg = dsv2lite.DSV2Config()
    w = dsv2lite.init_weights(cfg, device="cuda", seed=0)
    torch.cuda.synchronize()
    return cfg, w


def _bench_prompts(seed: int, lens: list[int], vocab: int) -> list[torch.Tensor]:
    """The prompts bench.py draws for a config (one generator, lengths first)."""
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, vocab, (n,), generator=g) for n in lens]


def _replay_equals_eager(eng, steps: int = 2) -> None:
    snap = eng.snapshot()
    eager = []
    for _ in range(steps):
        eng.step()
        eager.append((eng.logits.clone(), eng.ids.clone()))
    eng.restore(snap)
    eng.capture()
    eng.restore(snap)
    torch.cuda.synchronize()
    for i in range(steps):
        eng.replay()
        torch.cuda.synchronize()
        assert torch.equal(eng.logits, eager[i][0]), ("graph != eager logits", i)
        assert torch.equal(eng.ids, eager[i][1]), ("graph != eager ids", i)
    eng.restore(snap)


def close_at_depth(got, r16, r32, flipped: bool, what, errs: list) -> None:
    """Free-running bar (module docstring, part 2)."""
    e16, e32, floor = rel_err(got, r16), rel_err(got, r32), rel_err(r16, r32)
    errs.append((e16, e32, flipped, floor))
    cap16 = max(NEAR_TIE_BAR if flipped else FP32_BAR, DRIFT_POINT_HF * floor)
    assert e16 <= cap16, (what, "vs HF bf16", e16, floor)
    if not flipped:
        assert e32 <= max(BAR, DRIFT_POINT * floor), (what, "vs exact", e32, floor)


def _free_trace(orc, rec, tr, row, what, res, per_layer: dict, flips_out: list) -> bool:
    """check_trace with the free-running bar: router checks as everywhere, hidden states by
    close_at_depth.  Returns whether a layer's expert set differs from the oracle's."""
    fl = router_flips(orc, rec, tr, row, what, flips_out)
    first = min(fl) if fl else 1 << 30
    for (_, li, h) in (r for r in rec if r[0] == "layer"):
        close_at_depth(h[row].float().cpu(), tr[li]["h_out"], res["fp32"]["layer_out"][li][-1], li >= first,
                       (what, li), per_layer.setdefault(li, []))
    return bool(fl)


def close_forced(got, r16, r32, what, errs: list) -> None:
    """Layer-by-layer bar: within 2e-2 of the bf16 oracle run on the same input.  (The fp32
    oracle's value at this layer comes from exact math's own trajectory, a different input;
    its distance is recorded, not asserted.)"""
    e16, e32, floor = rel_err(got, r16), rel_err(got, r32), rel_err(r16, r32)
    errs.append((e16, e32, False, floor))
    assert e16 <= BAR, (what, "vs HF bf16 on the same input", e16)


def _forced_trace(orc, rec, tr, row, what, res, per_layer: dict, flips_out: list) -> None:
    """Router checks as everywhere; every layer's output (and post-attention state) within
    close_forced of the bf16 oracle's same layer on the same input."""
    router_flips(orc, rec, tr, row, what, flips_out)
    h_attn = {r[1]: r[2][row] for r in rec if r[0] == "attn"}
    for (_, li, h) in (r for r in rec if r[0] == "layer"):
        close_forced(h_attn[li].float().cpu(), tr[li]["h_attn"][-1], tr[li]["h_attn"][-1], (what, li, "attn"), [])
        close_forced(h[row].float().cpu(), tr[li]["h_out"], res["fp32"]["layer_out"][li][-1], (what, li),
                     per_layer.setdefault(li, []))


def _write_oracle_cache(eng, row: int, ocache: list) -> None:
    """The oracle's compressed cache rows (bf16 mode: bf16 values) of one sequence into the
    engine's cache rows of `row`, every layer."""
    base = int(eng.cache.base[row])
    for li, sc in enumerate(ocache):
        rows = torch.cat([torch.cat(sc.c, 0), torch.cat(sc.kpe, 0)], 1).to(torch.bfloat16)
        eng.cache.data[li, base:base + rows.shape[0]].copy_(rows)


def _forced_step(eng, rows: list[int], h_in: list[torch.Tensor], h_final: torch.Tensor, pos: int) -> list:
    """One decode step of every layer with the checked rows' input to layer li set to
    h_in[li] ([len(rows), H]) and the head run on h_final; every row at position `pos`.
    Returns the per-layer record (the format of a recorded step); logits in eng.logits."""
    from triton_kernels import _hip
    from triton_kernels._hip import call, ptr

    c, b, R, fam = eng.cfg, eng.buf, eng.B, eng.family
    st = _hip.stream_ptr()
    rows_d = torch.tensor(rows, dtype=torch.int64, device=eng.device)
    eng.cache.pos.fill_(pos)
    rec = []
    n = len(eng.w.layers)
    for li, L in enumerate(eng.w.layers):
        b.h.index_copy_(0, rows_d, h_in[li].to(torch.bfloat16).to(eng.device))
        if fam == "batch":  # the batch family's attention reads the normalised input
            call("dsv2_rmsnorm_bf16", ptr(b.h), c.hidden, ptr(L.ln_in), ptr(b.xn), c.hidden, R, c.hidden, c.eps, st)
        eng._attention(L, li, b, R, eng.cache.pos, eng.cache.base, eng.cache.cap, fam, st)
        rec.append(("attn", li, b.h[:R].clone()))
        nn = eng.w.layers[li + 1].ln_in if li + 1 < n else eng.w.norm
        eng._mlp(L, li, b, R, fam, nn, st)
        rec.append(("layer", li, b.h[:R].clone()))
        if L.moe:
            rec.append(("router", li, b.ids32[:R].clone(), b.wts[:R].clone()))
    b.h.index_copy_(0, rows_d, h_final.to(torch.bfloat16).to(eng.device))
    if fam == "batch":
        call("dsv2_rmsnorm_bf16", ptr(b.h), c.hidden, ptr(eng.w.norm), ptr(b.xn), c.hidden, R, c.hidden, c.eps, st)
    eng._head(b, fam, st, eng.cache.pos.clone())
    torch.cuda.synchronize()
    return rec


def _table(say, title: str, per_layer: dict) -> None:
    lines = []
    for li in sorted(per_layer):
        es = per_layer[li]
        if not es:
            continue
        clear = [e for e in es if not e[2]]
        src = clear or es
        lines.append(f"L{li}: max {max(e[0] for e in src):.2e} mean {sum(e[0] for e in src) / len(src):.2e} "
                     f"(vs exact: max {max(e[1] for e in src):.2e} mean {sum(e[1] for e in src) / len(src):.2e}; "
                     f"HF vs exact: max {max(e[3] for e in src):.2e} mean {sum(e[3] for e in src) / len(src):.2e}"
                     f"{'; after a flip' if not clear else ''})")
    n = len(per_layer.get(0, []))
    say(f"{title} ({n} points per layer):\n    " + "\n    ".join(lines))


@pytest.mark.timeout(1500)
def test_full_depth_27_layers_vs_oracle(full_model, capsys):
    import dsv2lite

    cfg, w = full_model
    t0 = time.perf_counter()

    def say(msg: str) -> None:
        with capsys.disabled():
            print(f"[full-depth {time.perf_counter() - t0:6.1f}s] {msg}", flush=True)

    # the two engines, prefilled, graphs captured (replay == eager checked)
    p1 = _bench_prompts(1, [128], cfg.vocab)
    e1 = dsv2lite.DecodeEngine(w, [128 + STEPS + 8], family="small")
    pre1 = []
    e1.prefill([p.cuda() for p in p1], record=pre1)
    p3 = _bench_prompts(2, [2048] * 256, cfg.vocab)
    e3 = dsv2lite.DecodeEngine(w, [2048 + STEPS + 8] * 256, family="batch")
    pre3 = []
    e3.prefill([p.cuda() for p in p3], record=pre3)
    torch.cuda.synchronize()
    first = {("C1", 0): (int(e1.ids[0]), e1.logits[0].cpu().clone())}
    for b in C3_ROWS:
        first[("C3", b)] = (int(e3.ids[b]), e3.logits[b].cpu().clone())
    say("prefills done (C1 128 tokens small family, C3 256 x 2048 tokens batch family)")
    _replay_equals_eager(e1)
    _replay_equals_eager(e3)
    say(f"graph replay == eager (C1 {e1.kernels_per_step} kernels per step, C3 {e3.kernels_per_step}, "
        f"MoE tile {e3.buf.tile_tokens})")

    # the checked sequences: (config, engine, row, prompt)
    seqs = [("C1", e1, 0, p1[0])] + [("C3", e3, b, p3[b]) for b in C3_ROWS]
    orc = StreamedOracle(w, max_pos=2048 + STEPS + 16)
    caches = [orc.new_cache() for _ in seqs]
    free = {c: {} for c in ("C1", "C3")}
    flips = {c: [] for c in ("C1", "C3")}
    free_logits: dict = {c: [] for c in ("C1", "C3")}
    failures: list[str] = []
    ag = {"free": 0, "forced": 0}
    tot = {"free": 0, "forced": 0}

    def guard(what, fn):
        try:
            return fn()
        except AssertionError as e:
            failures.append(str(e)[:400])
            say(f"FAILED {what}: {str(e)[:400]}")
            return None

    def check_free(step, outs, records, got_tok, got_logits):
        toks = []
        for (cname, _, b, _), (res, tr), rec, tok, lg in zip(seqs, outs, records, got_tok, got_logits):
            what = (cname, step, b)
            ref = res["logits"][-1]
            n0 = len(flips[cname])
            fl = guard(what, lambda: _free_trace(orc, rec, tr, b, what, res, free[cname], flips[cname]))
            flipped = fl is None or len(flips[cname]) > n0
            guard((what, "logits"), lambda: close_at_depth(lg, ref, res["fp32"]["logits"][-1], flipped,
                                                             (what, "logits"), free_logits[cname]))
            a = guard((what, "greedy"), lambda: agree(tok, ref, lg, what))
            ag["free"] += a or 0
            tot["free"] += 1
            toks.append(int(torch.argmax(ref)))
        return toks

    prog = lambda li: say(f"  oracle layer {li}") if li % 9 == 8 else None  # noqa: E731
    outs = orc.run([(caches[j], s[3], 0) for j, s in enumerate(seqs)], progress=prog)
    say("oracle prefill pass done")
    toks = check_free("prefill", outs, [pre1, pre3, pre3], [first[s[0], s[2]][0] for s in seqs],
                      [first[s[0], s[2]][1] for s in seqs])
    P = {j: s[3].numel() for j, s in enumerate(seqs)}
    step_inputs = []  # per step: (token per seq, oracle outs per seq)
    for step in range(STEPS):
        e1.ids[0] = toks[0]
        nxt3 = e3.ids.clone()
        for j, b in enumerate(C3_ROWS):
            nxt3[b] = toks[1 + j]
        e3.ids.copy_(nxt3)
        r1, r3 = [], []
        e1.step(record=r1)
        e3.step(record=r3)
        torch.cuda.synchronize()
        got_tok = [int(e1.ids[0])] + [int(e3.ids[b]) for b in C3_ROWS]
        got_logits = [e1.logits[0].cpu()] + [e3.logits[b].cpu() for b in C3_ROWS]
        outs = orc.run([(caches[j], torch.tensor([toks[j]]), P[j] + step) for j in range(len(seqs))])
        step_inputs.append((list(toks), outs))
        toks = check_free(step, outs, [r1, r3, r3], got_tok, got_logits)
        say(f"free-running decode step {step} checked")
    e1.check_errors()
    e3.check_errors()

    # 1. layer by layer: every layer's input and the checked rows' cache from the oracle
    forced = {c: {} for c in ("C1", "C3")}
    forced_flips = {c: [] for c in ("C1", "C3")}
    forced_logits: dict = {c: [] for c in ("C1", "C3")}
    for step, (tk, outs) in enumerate(step_inputs):
        for eng, idx in ((e1, [0]), (e3, [1, 2])):
            rows = [seqs[j][2] for j in idx]
            h_in = [torch.cat([(orc.embed[tk[j]].reshape(1, -1) if li == 0 else outs[j][0]["layer_out"][li - 1])
                               for j in idx]) for li in range(len(w.layers))]
            h_fin = torch.cat([outs[j][0]["layer_out"][-1] for j in idx])
            for j in idx:  # every forced step rewrites row P + step from its own input first
                _write_oracle_cache(eng, seqs[j][2], caches[j]["bf16"])
            rec = _forced_step(eng, rows, h_in, h_fin, P[idx[0]] + step)
            for j in idx:
                cname, _, b, _ = seqs[j]
                res, tr = outs[j]
                what = (cname, "forced", step, b)
                guard(what, lambda: _forced_trace(orc, rec, tr, b, what, res, forced[cname], forced_flips[cname]))
                lg, ref = eng.logits[b].cpu(), res["logits"][-1]
                guard((what, "logits"), lambda: close_forced(lg, ref, res["fp32"]["logits"][-1], (what, "logits"),
                                                             forced_logits[cname]))
                a = guard((what, "greedy"), lambda: agree(int(eng.ids[b]), ref, lg, what))
                ag["forced"] += a or 0
                tot["forced"] += 1
        say(f"layer-by-layer decode step {step} checked")

    for cname in ("C1", "C3"):
        _table(say, f"{cname} layer by layer (oracle inputs), error vs the bf16 oracle", forced[cname])
        le = forced_logits[cname] or [(float("nan"),) * 4]
        say(f"{cname} layer by layer: logits max {max(e[0] for e in le):.2e} vs bf16 oracle; router flips "
            f"{[(f[0], round(f[1], 5), round(f[2], 5)) for f in forced_flips[cname]]}")
        _table(say, f"{cname} free running, error vs the bf16 oracle", free[cname])
        pts = [e for li in free[cname] for e in free[cname][li] if not e[2]]
        m32 = sum(e[1] for e in pts) / max(1, len(pts))
        mfl = sum(e[3] for e in pts) / max(1, len(pts))
        le = free_logits[cname] or [(float("nan"),) * 4]
        say(f"{cname} free running: logits max {max(e[0] for e in le):.2e} vs bf16 oracle; mean distance of the "
            f"hidden states from exact math {m32:.3e}, HF's own {mfl:.3e} ({len(pts)} points); router flips "
            f"accepted {len(flips[cname])}, {sum(1 for f in flips[cname] if f[1] > 1e-3)} of them with the "
            f"oracle's top-6 margin > 1e-3: {[(f[0], round(f[1], 5), round(f[2], 5)) for f in flips[cname]]}")
        guard((cname, "free-running mean"), lambda: _assert_mean(m32, mfl, cname))
    say(f"greedy agreement: layer by layer {ag['forced']}/{tot['forced']}, free running {ag['free']}/{tot['free']}")
    assert not failures, failures
    assert ag["forced"] / tot["forced"] >= 0.95, ag


def _assert_mean(m32: float, mfl: float, what) -> None:
    assert m32 <= DRIFT_MEAN * mfl, (what, "mean distance from exact math", m32, mfl)
