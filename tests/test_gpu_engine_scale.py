"""Engine-level GPU parity at the benchmark batch sizes and context lengths: the decode step
at bsz=64 with prompts U[256,1024] (benchmark config 2) and bsz=256 with 2048-token prompts
(config 3), a 256-token prefill followed by 32 decode steps (config 0's shape, one row), and
a prompt that crosses a prefill chunk.  The prefill logits of every sampled row -- the
chunked flash-attention prefill over 2048-token prompts at bsz=256 -- are checked too.  Same 3-layer full-width model and bars
as test_gpu_engine.py (engine_common).

At bsz 64 / 256 the step runs the kernels that only those sizes select: the one-workgroup-
per-token router above 64 rows, the tile size tune_moe_tiles picks from real routing (32-
token tiles at bsz=64, the 64-token direct-to-LDS ring at bsz=256), the shared experts
inside the grouped launches, the ring-GEMM lm_head and the split plan of long contexts.
Four rows per batch (the shortest and the longest prompt and two random ones) are checked
against the oracle, teacher-forced for 3 steps (every row of the batch runs; the sampled
rows are fed the oracle's greedy token, the others their own).  Graph replay must equal
the eager step bitwise for the whole batch.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

from engine_common import agree, build_model, check_trace, close, oracle_step, prompts

N_LAYERS = 3


@pytest.fixture(scope="module")
def model():
    return build_model(N_LAYERS, max_pos=2112)


def _sample(lens, seed):
    g = torch.Generator().manual_seed(seed)
    order = sorted(range(len(lens)), key=lambda b: (lens[b], b))
    rows = [order[0], order[-1]]
    for b in torch.randperm(len(lens), generator=g).tolist():
        if b not in rows:
            rows.append(b)
        if len(rows) == 4:
            break
    return rows[:min(4, len(lens))]


def _graph_equals_eager(eng, snap, steps=2):
    eng.restore(snap)
    eager = []
    for _ in range(steps):
        eng.step()
        eager.append((eng.logits.clone(), eng.ids.clone()))
    eng.restore(snap)
    torch.cuda.synchronize()
    for i in range(steps):
        eng.replay()
        torch.cuda.synchronize()
        assert torch.equal(eng.logits, eager[i][0]), ("graph != eager logits", i)
        assert torch.equal(eng.ids, eager[i][1]), ("graph != eager ids", i)
    eng.restore(snap)


def _parity(model, family, lens, seed, steps=3, rows=None, graph=True, tile=None, chunk=8192):
    import dsv2lite

    cfg, w, om = model
    B = len(lens)
    eng = dsv2lite.DecodeEngine(w, [n + steps + 8 for n in lens], family=family, max_prefill_rows=chunk)
    P = prompts(lens, seed)
    prec = []
    first = eng.prefill([p.cuda() for p in P], record=prec).cpu().clone()
    torch.cuda.synchronize()
    rows = _sample(lens, seed) if rows is None else rows
    first_logits = {b: eng.logits[b].cpu().clone() for b in rows}  # the graph checks overwrite logits
    snap = eng.snapshot()
    if graph:
        eng.capture()  # the batch family picks its MoE tile from real routing first
        if tile is not None:
            assert eng.buf.tile_tokens == tile, eng.buf.tile_tokens
        _graph_equals_eager(eng, snap)
    errs, ag, tot, checked, flipped_steps = [], 0, 0, 0, 0
    caches = {b: om.new_cache() for b in rows}
    toks = eng.ids.cpu().tolist()
    for b in rows:
        res, tr = oracle_step(om, caches[b], P[b], 0, last_logits_only=True)
        ref = res["logits"][-1]
        n_clear, flipped = check_trace(om, prec, tr, b, ("prefill", b), res, errs)
        checked += n_clear
        flipped_steps += flipped
        close(first_logits[b], ref, res["fp32"]["logits"][-1], flipped, ("prefill", b), errs)
        ag += agree(int(first[b]), ref, first_logits[b], ("prefill", b))
        tot += 1
        toks[b] = int(torch.argmax(ref))
    for s in range(steps):
        eng.ids.copy_(torch.tensor(toks, dtype=torch.int64))
        rec = []
        eng.step(record=rec)
        torch.cuda.synchronize()
        nxt = eng.ids.cpu().tolist()
        for b in rows:
            res, tr = oracle_step(om, caches[b], torch.tensor([toks[b]]), lens[b] + s)
            ref = res["logits"][-1]
            n_clear, flipped = check_trace(om, rec, tr, b, (family, s, b), res, errs)
            checked += n_clear
            flipped_steps += flipped
            close(eng.logits[b].cpu(), ref, res["fp32"]["logits"][-1], flipped, (family, s, b), errs)
            ag += agree(int(nxt[b]), ref, eng.logits[b].cpu(), (family, s, b))
            tot += 1
            nxt[b] = int(torch.argmax(ref))
        toks = nxt
    assert eng.cache.pos.cpu().tolist() == [n + steps for n in lens]
    eng.check_errors()
    clear = [e for e in errs if not e[2]]
    print(f"{family} B={B} ctx {min(lens)}..{max(lens)} rows {rows}: greedy {ag}/{tot}, routers checked "
          f"{checked}, max-rel vs bf16 oracle {max(e[0] for e in clear):.3e}, vs fp32 oracle "
          f"{max(e[1] for e in clear):.3e} (bf16 oracle vs fp32 {max(e[3] for e in clear):.3e}); {flipped_steps} "
          f"of {tot} steps with a near-tie router flip", flush=True)
    assert checked >= steps * len(rows)
    return eng


def test_c2_bsz64_varlen_prompts_vs_oracle(model):
    """Benchmark config 2: bsz=64, prompt lengths U[256,1024] from seed 2."""
    g = torch.Generator().manual_seed(2)
    lens = torch.randint(256, 1025, (64,), generator=g).tolist()
    _parity(model, "batch", lens, seed=2, tile=32)


def test_c3_bsz256_2048_prompts_vs_oracle(model):
    """Benchmark config 3: bsz=256, 2048-token prompts (2 prefill chunks per row)."""
    _parity(model, "batch", [2048] * 256, seed=2, tile=64)


@pytest.mark.parametrize("family", ["small", "batch"])
def test_c0_shape_prefill256_then_32_steps(model, family):
    """Config 0's shape on the full path: a 256-token prefill, then 32 teacher-forced decode
    steps of one row, every step against the oracle (the small family captures its graph
    too, so the fused MLA and the route-local MoE run at 256..288 tokens of context)."""
    _parity(model, family, [256], seed=5, steps=32, rows=[0])


def test_prefill_crosses_a_chunk_boundary(model):
    """A 1300-token and a 100-token prompt in 1024-row prefill chunks: the first chunk holds
    the short prompt and the long one's first 924 tokens, the second chunk's queries attend
    keys the first chunk cached."""
    _parity(model, "batch", [100, 1300], seed=6, rows=[0, 1], chunk=1024)


def test_prefill_with_capacities_far_above_the_prompts(model):
    """Slots of capacity 32,768 holding 37..120-token prompts: the prefill plans its attention
    in per-sequence groups (prefill_groups) instead of expanding every slot's unused capacity
    in between, and gives the first tokens and logits of an engine whose capacities just fit
    the prompts (logits within 1e-2; tokens equal or a near-tie)."""
    import dsv2lite

    from golden_utils import rel_err

    cfg, w, _ = model
    lens = [100, 37, 120, 64]
    P = [p.cuda() for p in prompts(lens, seed=8)]
    big = dsv2lite.DecodeEngine(w, [32768] * 4, family="batch")
    tight = dsv2lite.DecodeEngine(w, [n + 8 for n in lens], family="batch")
    ib = big.prefill(P).cpu().clone()
    it = tight.prefill(P).cpu().clone()
    torch.cuda.synchronize()
    for b in range(4):
        assert rel_err(big.logits[b].cpu(), tight.logits[b].cpu()) < 1e-2, b
        agree(int(ib[b]), tight.logits[b].cpu(), big.logits[b].cpu(), ("capacity", b))
    # one decode step on the same input tokens
    big.ids.copy_(tight.ids)
    big.step()
    tight.step()
    torch.cuda.synchronize()
    for b in range(4):
        assert rel_err(big.logits[b].cpu(), tight.logits[b].cpu()) < 2e-2, b


@pytest.mark.parametrize("B", [64, 256])
def test_replicated_prompt_rows_stay_bitwise_identical(model, B):
    """The reference's published workload replicates one prompt over the batch
    (src/run.py:733-741): every row then holds the same sequence and must produce the same
    bits -- the split-KV decode walks every row's tiles in token order (4 splits per row at
    bsz=64, one 600-token split at bsz=256), the cache rows start staggered, and every sum
    has a fixed order -- through the prefill and several graph replays."""
    import dsv2lite

    cfg, w, _ = model
    p = prompts([600], seed=4)[0].cuda()
    eng = dsv2lite.DecodeEngine(w, [600 + 16] * B, family="batch")
    eng.prefill([p] * B)
    torch.cuda.synchronize()
    assert torch.equal(eng.logits, eng.logits[:1].expand_as(eng.logits))
    eng.capture()
    for s in range(4):
        eng.replay()
        torch.cuda.synchronize()
        assert torch.equal(eng.logits, eng.logits[:1].expand_as(eng.logits)), s
        assert torch.equal(eng.ids, eng.ids[:1].expand_as(eng.ids)), s
    eng.check_errors()


@pytest.mark.parametrize("bsz", [8, 64])
def test_small_family_at_larger_batches(model, bsz):
    """The small (GEMV) family above bsz=3, as the reference runs it up to bsz=256
    (attention_decode_small.py:932-1070, moe_small_gemv.py:430-514): ragged prompts, the
    absorbed q|kv_a projection, the one-launch attention and the route-local MoE with 8 and
    64 rows (the lm_head GEMV + argmax above 8 rows).  Two sampled rows (the shortest and the
    longest prompt) against the oracle, teacher-forced for 3 steps; graph == eager for the
    whole batch."""
    g = torch.Generator().manual_seed(20 + bsz)
    lens = torch.randint(24, 600, (bsz,), generator=g).tolist()
    eng = _parity(model, "small", lens, seed=20 + bsz, rows=_sample(lens, 20 + bsz)[:2])
    assert eng.mla_path == "absorb"
