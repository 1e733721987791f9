"""The DeepSeek-V2-Lite q_len=1 decode step on HIP kernels, and its prefill.

One ``step()`` enqueues the whole 27-layer step (embedding gather, per layer
attention + MLP/MoE, final norm, lm_head, greedy argmax, position advance) on
torch's current stream; ``capture()`` records it once into a hipGraph
(torch.cuda.CUDAGraph) and ``replay()`` re-launches it.  Mirrors
``_graph_decode_step`` / ``_run_graph_decode`` (src/run.py:558-688).

Kernel families (``--kernel-family``, src/run.py:53-65):
  small -- VALU GEMV with fused RMSNorm prologue and residual epilogue; fused
           MLA prepare (RoPE + cache write + W_UK absorption) and fused
           combine + W_UV; route-local MoE over 6 routed + 2 shared "half"
           experts with a deterministic in-workgroup top-6 combine.
  batch -- bf16 MFMA grouped GEMM for every projection (heads-batched W_UK /
           W_UV), deterministic expert bucketing, expert-grouped gate_up+SwiGLU
           and down on MFMA, fused combine + shared + residual + next RMSNorm.
Both use the same split-KV absorbed-MLA decode kernel.  Prefill uses the batch
family's projections and MoE with one row per prompt token, and MLA in its expanded
form through a causal flash-attention kernel.
"""

from __future__ import annotations

import math

import torch

from triton_kernels import _hip
from triton_kernels._hip import LINEAR_OUT_F32, LINEAR_OUT_F32_EXACT, LINEAR_SWIGLU, call, ptr
from triton_kernels.attention_decode_batch import plan_splits

from .cache import CompressedKVCache
from .config import DSV2Config
from .rope import cos_sin_tables
from .weights import ModelWeights

BF16 = torch.bfloat16
FAMILIES = ("small", "batch")
FUSED_MLA_MAX_CTX = 2048
# batch family: up to this many rows the router runs as logits over 16 workgroups per token
# plus a one-wave top-6 per row (64 rows: 8.3 us vs 11.1 us for one workgroup per token on
# MI355X); above it one workgroup per token (256 rows: 11.4 us vs 14.7 us)
SPLIT_ROUTER_MAX_ROWS = 64
# from this many rows (prefill chunks) the router runs as RMSNorm + an MFMA logits GEMM + top-6
GEMM_ROUTER_MIN_ROWS = 1024
# prefill chunks from this many rows bucket their routes over many workgroups (one workgroup
# is VALU-bound there: 8192 rows 74 us, against three short launches)
WIDE_BUCKET_MIN_ROWS = 1024
# grouped MoE: from this many routes in a launch the 256-token tiles (256 x 256 ring GEMM, one
# MFMA per 384 B of LDS reads) beat the 64-token ones.  The crossover follows the launch's
# routes rather than their spread over the experts: measured on MI355X, routed gate_up + down,
# uniform routing (all 64 experts) 4096 routes 297 vs 321 us (64 vs 256 tokens), 6144 routes
# 421 vs 358 us, 49152 routes 2264 vs 1155 us; every row on the same 6 experts 3072 routes
# 109 vs 120 us, 6144 routes 213 vs 194 us
BIG_TILE_ROUTES = 5120


def moe_tile_tokens(rows: int, n_experts: int = 64, top_k: int = 6) -> int:
    """Token tile of the expert-grouped MoE GEMMs before any routing has been seen, from the
    mean routes per expert under uniform routing (see tile_tokens_for_load)."""
    return tile_tokens_for_load(rows * top_k / n_experts, rows * top_k)


def tile_tokens_for_load(load: float, routes: int = 0) -> int:
    """Token tile for a mean of `load` routes per routed expert in a launch of `routes` routes
    (256 from BIG_TILE_ROUTES, whatever the spread).  Measured on MI355X, whole
    decode step (the 64-token tiles run on the direct-to-LDS ring GEMM, every size with the
    shared experts folded in where shared_in_grouped allows): bsz=64 random prompts (about
    7 routes per expert) 8.71k tok/s with 32-token tiles vs 8.58k with 16 and 8.13k with 64;
    bsz=256 (about 25) 22.42k with 64 vs 21.79k with 32; every row on the same 6 experts
    (64 or 256 routes per expert) 64."""
    if routes >= BIG_TILE_ROUTES:
        return 256
    return 16 if load <= 3 else (32 if load <= 12 else 64)


def shared_in_grouped(rows: int, tile_tokens: int) -> bool:
    """Whether the shared experts run inside the grouped MoE launches (as two extra experts
    over all rows) rather than as two dense GEMMs.  Each of their token tiles re-reads the
    half's weights, so only few tiles pay: measured on MI355X, 64 rows in 16-token tiles
    8.31k -> 8.58k tok/s; 256 rows in 32-token tiles 21.86k -> 21.63k (kept dense); 64-token
    tiles run on the direct-to-LDS ring, whose dense and grouped forms share the weight reads
    alike (reference workload bsz=64 19.3k -> 22.6k with both launches)."""
    return tile_tokens == 64 or math.ceil(rows / tile_tokens) <= 4


def routing_load(ids: torch.Tensor, n_experts: int = 64) -> float:
    """Mean number of routes in the expert a route goes to (sum c_e^2 / sum c_e over the
    per-expert route counts c_e of one layer's top-k ids): the tile occupancy the grouped
    GEMMs see, ~rows*k/E + 1 for uniform routing, rows for identical rows."""
    c = torch.bincount(ids.reshape(-1).to(torch.int64).cpu(), minlength=n_experts).double()
    return float((c * c).sum() / c.sum().clamp(min=1))


class PrefillPlan:
    """One prefill chunk's attention work, in groups of sequences: each group's query tiles
    (<= 128 consecutive rows of one sequence each: first row, rows, first position, the
    sequence's cache base) and the cache rows [exp_lo, exp_lo + exp_rows) whose keys / values
    the group expands into kexp / vexp."""

    def __init__(self, groups: list[tuple[torch.Tensor, int, int]], kexp: torch.Tensor, vexp: torch.Tensor):
        self.groups = [(t, int(t.shape[0]), lo, n) for t, lo, n in groups]
        self.kexp, self.vexp = kexp, vexp


def _segments(seq: torch.Tensor) -> list[tuple[int, int, int]]:
    """(first chunk row, rows, sequence) of each run of one sequence's rows in a chunk."""
    vals, counts = torch.unique_consecutive(seq, return_counts=True)
    out, r = [], 0
    for s, cnt in zip(vals.tolist(), counts.tolist()):
        out.append((r, cnt, s))
        r += cnt
    return out


def _group_tiles(segs, posv: torch.Tensor, bases: list[int], tile: int) -> tuple[torch.Tensor, int, int]:
    out, lo, hi = [], None, None
    for r, cnt, s in segs:
        p_first = int(posv[r])
        for a in range(0, cnt, tile):
            out.append((r + a, min(tile, cnt - a), p_first + a, bases[s]))
        lo = bases[s] if lo is None else min(lo, bases[s])
        last = bases[s] + p_first + cnt
        hi = last if hi is None else max(hi, last)
    return torch.tensor(out, dtype=torch.int32).reshape(-1, 4), int(lo), int(hi - lo)


def prefill_tiles(seq: torch.Tensor, posv: torch.Tensor, bases: list[int], tile: int = 128) -> tuple[torch.Tensor, int, int]:
    """Query tiles of one chunk (seq[r]: sequence of chunk row r, posv[r]: its position;
    rows of a sequence are consecutive with consecutive positions) and the cache row range
    its attention reads: from the lowest sequence base to the last position of any row."""
    return _group_tiles(_segments(seq), posv, bases, tile)


def prefill_groups(seq: torch.Tensor, posv: torch.Tensor, bases: list[int], tile: int = 128,
                   slack: int = 4096) -> list[tuple[torch.Tensor, int, int]]:
    """prefill_tiles in groups of consecutive sequences whose expanded cache range stays within
    twice the rows they attend (plus `slack`): with slots far apart (capacities much larger
    than the prompts) one range over the whole chunk would expand every slot's unused
    capacity in between.  Each group: (tiles, exp_lo, exp_rows)."""
    groups, cur, lo, hi, used = [], [], 0, 0, 0
    for r, cnt, s in _segments(seq):
        need = int(posv[r]) + cnt
        a, e = bases[s], bases[s] + need
        if cur and max(hi, e) - min(lo, a) <= 2 * (used + need) + slack:
            cur.append((r, cnt, s))
            lo, hi, used = min(lo, a), max(hi, e), used + need
            continue
        if cur:
            groups.append(cur)
        cur, lo, hi, used = [(r, cnt, s)], a, e, need
    groups.append(cur)
    return [_group_tiles(g, posv, bases, tile) for g in groups]


class RowBuffers:
    """Per-row work buffers for `rows` rows of one kernel family (prefill: the batch family
    without the split-KV decode buffers)."""

    def __init__(self, cfg: DSV2Config, rows: int, family: str, max_ctx: int, device, prefill: bool = False):
        self.rows = rows
        self.family = family
        e = lambda *s, dt=BF16: torch.empty(*s, dtype=dt, device=device)  # noqa: E731
        H = cfg.hidden
        self.h = e(rows, H)
        self.xn = e(rows, H)
        self.qkva = e(rows, cfg.qkva_dim)
        self.q = e(rows, cfg.n_heads, cfg.cache_row)
        self.split_tokens, self.max_splits = plan_splits(rows, max_ctx)
        if not prefill:
            self.part_o = e(rows, self.max_splits, cfg.n_heads, cfg.kv_rank, dt=torch.float32)
            self.part_ml = e(rows, self.max_splits, cfg.n_heads, 2, dt=torch.float32)
        self.attn = e(rows, H)
        self.ids32 = e(rows, cfg.top_k, dt=torch.int32)
        self.wts = e(rows, cfg.top_k, dt=torch.float32)
        self.mid = e(rows, cfg.dense_inter)
        self.router_logits = e(rows, cfg.n_experts, dt=torch.float32)
        if family == "small":
            self.hbuf = e(rows, cfg.top_k + 2, cfg.moe_inter)
            if not prefill:  # partial absorbed queries of dsv2_qkva_absorb_bf16 (8 blocks per head)
                self.qlat_part = e(rows, cfg.n_heads, cfg.qk_nope // 16, cfg.kv_rank, dt=torch.float32)
        else:
            R = rows * cfg.top_k
            if not prefill:
                self.olat = e(rows, cfg.n_heads, cfg.kv_rank)
            self._routes, self._n_experts = R, cfg.n_experts
            self.tile_tokens = moe_tile_tokens(rows, cfg.n_experts, cfg.top_k)
            self.max_tiles = math.ceil(R / self.tile_tokens) + cfg.n_experts
            self.sorted = e(R, dt=torch.int32)
            self.route_pos = e(R, dt=torch.int32)
            self.tiles = e(math.ceil(R / 16) + cfg.n_experts, 4, dt=torch.int32)  # room for any tile size
            self.ntiles = e(1, dt=torch.int32)
            self.hs = e(R, cfg.moe_inter)
            self.ys = e(R, H)
            self.shmid = e(rows, cfg.shared_inter)
            self.shout = e(rows, H)
            self.shparts = e(2, rows, H, dt=torch.float32)  # shared down halves (64-token tiles)
            # per-chunk route histograms of dsv2_moe_bucket_wide (prefill chunks)
            self.bucket_ws = (e(_hip.lib.dsv2_moe_bucket_workspace_size(rows), dt=torch.uint8)
                              if prefill and rows >= WIDE_BUCKET_MIN_ROWS else None)


    def set_tile_tokens(self, tile_tokens: int) -> None:
        """Token tile of the grouped MoE launches (16, 32, 64 or 256); the tile table was
        sized for the smallest."""
        if tile_tokens not in (16, 32, 64, 256):
            raise ValueError(f"tile_tokens must be 16, 32, 64 or 256, got {tile_tokens}")
        self.tile_tokens = tile_tokens
        self.max_tiles = math.ceil(self._routes / tile_tokens) + self._n_experts


def _graph_node_count(g: torch.cuda.CUDAGraph) -> int:
    """Nodes of a captured (kept, not yet instantiated) graph, by hipGraphGetNodes of the HIP
    runtime torch loaded (whichever of its sonames resolves); -1 when none does or the call
    fails -- the count is a report, never a reason to fail a capture."""
    import ctypes

    loaded = []  # the runtime already mapped into this process (torch's), never a second copy
    try:
        with open("/proc/self/maps") as f:
            loaded = sorted({ln.split()[-1] for ln in f if "libamdhip64.so" in ln})
    except OSError:
        pass
    for name in loaded + ["libamdhip64.so.7", "libamdhip64.so.6"]:
        try:
            hip = ctypes.CDLL(name)
            break
        except OSError:
            continue
    else:
        return -1
    n = ctypes.c_size_t(0)
    rc = hip.hipGraphGetNodes(ctypes.c_void_p(g.raw_cuda_graph()), None, ctypes.byref(n))
    return int(n.value) if rc == 0 else -1


class DecodeEngine:
    def __init__(self, weights: ModelWeights, capacities: list[int], family: str = "small",
                 max_prefill_rows: int = 8192, device="cuda", mla_path: str = "absorb", moe_tile: int | None = None,
                 expert_dtype: str = "bf16"):
        """capacities: cache tokens of each row (slot).  moe_tile (batch family): fix the
        grouped MoE token tile (16, 32, 64 or 256) instead of choosing it from the routing of one
        eager step at capture -- for a serving loop whose batch changes under one graph.
        expert_dtype "fp8": the decode step reads the e4m3 expert weights of
        quantize_experts_fp8 (small family: the route kernels; batch family: the grouped
        launches, 32- or 64-token tiles); prefill keeps the bf16 kernels on the dequantized
        weights."""
        if family not in FAMILIES:
            raise ValueError(f"Unknown kernel family: {family}")
        if mla_path not in ("split", "fused", "spread", "absorb"):
            raise ValueError(f"Unknown MLA path: {mla_path}")
        if expert_dtype not in ("bf16", "fp8"):
            raise ValueError(f"Unknown expert dtype: {expert_dtype}")
        if expert_dtype == "fp8" and not weights.fp8_experts:
            raise ValueError("fp8 expert weights: run dsv2lite.quantize_experts_fp8(weights) first")
        cfg = weights.cfg
        cfg.check_kernel_dims()
        self.cfg = cfg
        self.w = weights
        self.family = family
        self.expert_dtype = expert_dtype
        self.device = torch.device(device)
        self.B = len(capacities)
        self.cache = CompressedKVCache(cfg.n_layers, capacities, device=device, row=cfg.cache_row)
        self.max_pos = self.cache.max_capacity
        self.cos, self.sin = cos_sin_tables(cfg, self.max_pos, device=device)
        self.scale = cfg.softmax_scale
        self.ids = torch.zeros(self.B, dtype=torch.int64, device=device)
        self.logits = torch.empty(self.B, cfg.vocab, dtype=torch.float32, device=device)
        self.buf = RowBuffers(cfg, self.B, family, self.max_pos, device)
        if family == "batch" and moe_tile is not None:
            self.buf.set_tile_tokens(self._fit_tile(moe_tile))
            self._moe_tiles_tuned = True
        elif family == "batch":
            self.buf.set_tile_tokens(self._fit_tile(self.buf.tile_tokens))
        self._amax = torch.empty(max(0, _hip.lib.dsv2_lm_head_argmax_workspace_size(min(self.B, 8))),
                                 dtype=torch.uint8, device=device)
        # small family: one fused workgroup per (row, head) while contexts are short; the
        # split-KV kernel (parallel over the context) takes over for long contexts
        self.fused_mla = family == "small" and self.max_pos <= FUSED_MLA_MAX_CTX and mla_path == "fused"
        # small family, "spread": mla_prepare (absorption over 128 workgroups) then mla_attend
        # (64 workgroups per row over heads x W_UV quarters)
        self.spread_mla = family == "small" and self.max_pos <= FUSED_MLA_MAX_CTX and mla_path == "spread"
        # small family, "absorb": the q|kv_a projection also forms the absorbed query in partial
        # sums (dsv2_qkva_absorb_bf16), then one attention launch (dsv2_mla_attend_parts)
        self.absorb_mla = family == "small" and self.max_pos <= FUSED_MLA_MAX_CTX and mla_path == "absorb"
        self.mla_path = ("fused" if self.fused_mla else "spread" if self.spread_mla else
                         "absorb" if self.absorb_mla else "split")
        self.max_prefill_rows = max_prefill_rows
        self.graph = None
        self.kernels_per_step = 0  # set by capture()
        self._host_pos = [0] * self.B  # host mirror of cache.pos, for capacity checks only
        self._free: set[int] = set()  # retired slots (continuous batching)

    def _fit_tile(self, tile: int, load: float | None = None) -> int:
        """The decode step's grouped MoE token tile: the e4m3 launches take 32- or 64-token
        tiles (the bf16 ones 16, 32, 64 or 256) -- 32 up to 32 routes per expert (measured on
        MI355X, gate_up + shared halves: 256 rows of uniform routing 105.6 us with 32-token tiles
        against 125.9 us with 64), 64 above."""
        if self.expert_dtype != "fp8":
            return tile
        if load is not None:
            return 32 if load <= 32 else 64
        return min(64, max(32, tile))

    # ------------------------------------------------------------------ layers
    def _attention(self, L, li: int, b: RowBuffers, R: int, pos, base, cap, family: str, st: int,
                   pf: PrefillPlan | None = None) -> None:
        c = self.cfg
        cache = self.cache.layer(li)
        if pf is not None:
            self._attention_prefill(L, cache, b, R, pos, base, cap, st, pf)
            return
        if family == "small" and self.spread_mla and b is self.buf:
            call("dsv2_gemv_bf16", ptr(b.h), c.hidden, R, c.hidden, ptr(L.w_qkva), c.qkva_dim, ptr(L.ln_in), c.eps,
                 None, 0, ptr(b.qkva), c.qkva_dim, 0, st)
            call("dsv2_mla_spread", ptr(b.qkva), c.qkva_dim, R, ptr(pos), ptr(base), ptr(cap), ptr(L.kv_norm),
                 c.eps, ptr(self.cos), ptr(self.sin), self.max_pos, ptr(L.w_ukt), ptr(L.w_uv), ptr(cache), ptr(b.q),
                 self.scale, ptr(b.attn), c.hidden, ptr(self.cache.status), st)
            call("dsv2_gemv_bf16", ptr(b.attn), c.hidden, R, c.hidden, ptr(L.w_o), c.hidden, None, 0.0, ptr(b.h),
                 c.hidden, ptr(b.h), c.hidden, 0, st)
            return
        if family == "small" and self.absorb_mla and b is self.buf:
            call("dsv2_qkva_absorb_bf16", ptr(b.h), c.hidden, R, ptr(L.w_qkva), ptr(L.ln_in), c.eps, ptr(L.w_uk),
                 ptr(b.qkva), c.qkva_dim, ptr(b.qlat_part), ptr(cache), ptr(base), ptr(pos), ptr(cap), st)
            call("dsv2_mla_attend_parts", ptr(b.qkva), c.qkva_dim, R, ptr(pos), ptr(base), ptr(cap), ptr(L.kv_norm),
                 c.eps, ptr(self.cos), ptr(self.sin), self.max_pos, ptr(b.qlat_part), ptr(L.w_uv), ptr(cache),
                 self.scale, ptr(b.attn), c.hidden, ptr(self.cache.status), st)
            call("dsv2_gemv_bf16", ptr(b.attn), c.hidden, R, c.hidden, ptr(L.w_o), c.hidden, None, 0.0, ptr(b.h),
                 c.hidden, ptr(b.h), c.hidden, 0, st)
            return
        if family == "small" and self.fused_mla and b is self.buf:
            call("dsv2_gemv_bf16", ptr(b.h), c.hidden, R, c.hidden, ptr(L.w_qkva), c.qkva_dim, ptr(L.ln_in), c.eps,
                 None, 0, ptr(b.qkva), c.qkva_dim, 0, st)
            call("dsv2_mla_fused", ptr(b.qkva), c.qkva_dim, R, ptr(pos), ptr(base), ptr(cap), ptr(L.kv_norm),
                 c.eps, ptr(self.cos), ptr(self.sin), self.max_pos, ptr(L.w_ukt), ptr(L.w_uv), ptr(cache),
                 self.scale, ptr(b.attn), c.hidden, ptr(self.cache.status), st)
            call("dsv2_gemv_bf16", ptr(b.attn), c.hidden, R, c.hidden, ptr(L.w_o), c.hidden, None, 0.0, ptr(b.h),
                 c.hidden, ptr(b.h), c.hidden, 0, st)
            return
        if family == "small":
            call("dsv2_gemv_bf16", ptr(b.h), c.hidden, R, c.hidden, ptr(L.w_qkva), c.qkva_dim, ptr(L.ln_in), c.eps,
                 None, 0, ptr(b.qkva), c.qkva_dim, 0, st)
            call("dsv2_mla_prepare", ptr(b.qkva), c.qkva_dim, R, ptr(pos), ptr(base), ptr(cap), ptr(L.kv_norm),
                 c.eps, ptr(self.cos), ptr(self.sin), self.max_pos, ptr(L.w_ukt), ptr(cache), ptr(b.q),
                 ptr(self.cache.status), st)
        else:
            call("dsv2_gemm_bf16", ptr(b.xn), c.hidden, 0, R, c.hidden, ptr(L.w_qkva), 0, c.qkva_dim, 1, None, 0,
                 ptr(b.qkva), c.qkva_dim, 0, 0, st)
            # kv-norm + RoPE + cache write, and q_lat[r, h, :512] = W_UK_h^T q_nope[r, h] (16 head
            # groups, K = 128, on MFMA) in one launch
            call("dsv2_mla_prepare_qlat", ptr(b.qkva), c.qkva_dim, R, ptr(pos), ptr(base), ptr(cap),
                 ptr(L.kv_norm), c.eps, ptr(self.cos), ptr(self.sin), self.max_pos, ptr(L.w_ukt), ptr(cache),
                 ptr(b.q), ptr(self.cache.status), st)
        if family == "batch" and b.max_splits == 1:
            # one split per row (~256+ rows fill the GPU): normalised o_lat straight from the decode
            call("dsv2_mla_decode_rows", ptr(b.q), ptr(cache), ptr(base), ptr(pos), ptr(cap), R, self.scale,
                 ptr(b.olat), c.n_heads * c.kv_rank, st)
            call("dsv2_gemm_bf16", ptr(b.olat), c.n_heads * c.kv_rank, c.kv_rank, R, c.kv_rank, ptr(L.w_uv),
                 c.v_dim * c.kv_rank, c.v_dim, c.n_heads, None, 0, ptr(b.attn), c.hidden, c.v_dim, 0, st)
            call("dsv2_gemm_bf16", ptr(b.attn), c.hidden, 0, R, c.hidden, ptr(L.w_o), 0, c.hidden, 1, ptr(b.h),
                 c.hidden, ptr(b.h), c.hidden, 0, 0, st)
            return
        call("dsv2_mla_decode", ptr(b.q), ptr(cache), ptr(base), ptr(pos), ptr(cap), R, b.split_tokens,
             b.max_splits, self.scale, ptr(b.part_o), ptr(b.part_ml), st)
        if family == "small":
            call("dsv2_mla_combine", ptr(b.part_o), ptr(b.part_ml), ptr(pos), ptr(cap), R, b.split_tokens,
                 b.max_splits, ptr(L.w_uv), ptr(b.attn), c.hidden, st)
            call("dsv2_gemv_bf16", ptr(b.attn), c.hidden, R, c.hidden, ptr(L.w_o), c.hidden, None, 0.0, ptr(b.h),
                 c.hidden, ptr(b.h), c.hidden, 0, st)
        else:
            call("dsv2_mla_combine", ptr(b.part_o), ptr(b.part_ml), ptr(pos), ptr(cap), R, b.split_tokens,
                 b.max_splits, None, ptr(b.olat), c.n_heads * c.kv_rank, st)
            # attn[r, h*128 + i] = W_UV_h o_lat[r, h]: 16 head groups, K = 512
            call("dsv2_gemm_bf16", ptr(b.olat), c.n_heads * c.kv_rank, c.kv_rank, R, c.kv_rank, ptr(L.w_uv),
                 c.v_dim * c.kv_rank, c.v_dim, c.n_heads, None, 0, ptr(b.attn), c.hidden, c.v_dim, 0, st)
            call("dsv2_gemm_bf16", ptr(b.attn), c.hidden, 0, R, c.hidden, ptr(L.w_o), 0, c.hidden, 1, ptr(b.h),
                 c.hidden, ptr(b.h), c.hidden, 0, 0, st)

    def _attention_prefill(self, L, cache, b: RowBuffers, R: int, pos, base, cap, st: int, pf: PrefillPlan) -> None:
        """A prefill chunk's attention in the expanded form: the chunk's cache rows and
        RoPE(q_pe) (mla_prepare), k_nope / v of every cache row the chunk attends (W_UK /
        W_UV over the latent: grouped GEMMs over the heads), causal flash attention per
        (128-query tile, head), then o_proj with the residual."""
        c = self.cfg
        H, nh = c.hidden, c.n_heads
        call("dsv2_gemm_bf16", ptr(b.xn), H, 0, R, H, ptr(L.w_qkva), 0, c.qkva_dim, 1, None, 0, ptr(b.qkva),
             c.qkva_dim, 0, 0, st)
        call("dsv2_mla_prepare", ptr(b.qkva), c.qkva_dim, R, ptr(pos), ptr(base), ptr(cap), ptr(L.kv_norm), c.eps,
             ptr(self.cos), ptr(self.sin), self.max_pos, None, ptr(cache), ptr(b.q), ptr(self.cache.status), st)
        for tiles, n_tiles, exp_lo, exp_rows in pf.groups:
            crow = cache.data_ptr() + exp_lo * c.cache_row * cache.element_size()
            # W_UK / W_UV [16, 128, 512] are the [2048, 512] weights of one dense GEMM whose
            # output row is [16, 128] (the heads side by side): the prefill-size ring tiles, not
            # 16 groups of 128 features (C3 prefill: 73 -> ~25 us per expansion)
            for w, out, n in ((L.w_uk, pf.kexp, nh * c.qk_nope), (L.w_uv, pf.vexp, nh * c.v_dim)):
                call("dsv2_gemm_bf16", crow, c.cache_row, 0, exp_rows, c.kv_rank, ptr(w), 0, n, 1, None, 0, ptr(out),
                     n, 0, 0, st)
            call("dsv2_mla_prefill_attention", ptr(b.qkva), c.qkva_dim, ptr(b.q), nh * c.cache_row, R, ptr(cache),
                 cache.shape[0], ptr(pf.kexp), ptr(pf.vexp), exp_lo, exp_rows, ptr(tiles), n_tiles, self.scale,
                 ptr(b.attn), H, st)
        call("dsv2_gemm_bf16", ptr(b.attn), H, 0, R, H, ptr(L.w_o), 0, H, 1, ptr(b.h), H, ptr(b.h), H, 0, 0, st)

    def _mlp(self, L, li: int, b: RowBuffers, R: int, family: str, next_norm, st: int) -> None:
        c = self.cfg
        H = c.hidden
        if family == "small":
            if L.moe:
                call("dsv2_router_logits", ptr(b.h), H, ptr(L.ln_post), c.eps, ptr(L.w_router), R, ptr(b.xn),
                     ptr(b.router_logits), st)
                if self.expert_dtype == "fp8" and b is self.buf:
                    call("dsv2_moe_route_gateup_logits_fp8", ptr(b.xn), R, ptr(b.router_logits), c.routed_scaling,
                         ptr(b.ids32), ptr(b.wts), ptr(L.w_gu8), ptr(L.gu_scale), ptr(L.sh_gu8), ptr(L.sh_gu_scale),
                         c.moe_inter, ptr(b.hbuf), st)
                    call("dsv2_moe_route_down_fp8", ptr(b.hbuf), R, ptr(b.ids32), ptr(b.wts), ptr(L.w_down8),
                         ptr(L.down_scale), ptr(L.sh_down8), ptr(L.sh_down_scale), c.moe_inter, c.top_k + 2, ptr(b.h),
                         ptr(b.h), st)
                    return
                call("dsv2_moe_route_gateup_logits", ptr(b.xn), R, ptr(b.router_logits), c.routed_scaling,
                     ptr(b.ids32), ptr(b.wts), ptr(L.w_gu), ptr(L.sh_gu), c.moe_inter, ptr(b.hbuf), st)
                call("dsv2_moe_route_down", ptr(b.hbuf), R, ptr(b.ids32), ptr(b.wts), ptr(L.w_down), ptr(L.sh_down),
                     c.moe_inter, c.top_k + 2, None, ptr(b.h), ptr(b.h), st)
            else:
                call("dsv2_gemv_bf16", ptr(b.h), H, R, H, ptr(L.w_gu), c.dense_inter, ptr(L.ln_post), c.eps, None, 0,
                     ptr(b.mid), c.dense_inter, LINEAR_SWIGLU, st)
                call("dsv2_gemv_bf16", ptr(b.mid), c.dense_inter, R, c.dense_inter, ptr(L.w_down), H, None, 0.0,
                     ptr(b.h), H, ptr(b.h), H, 0, st)
            return
        if L.moe:
            if R >= GEMM_ROUTER_MIN_ROWS:
                # prefill chunks: the norm, the logits as an MFMA GEMM (unrounded fp32, as the
                # other routers), then the top-6
                call("dsv2_rmsnorm_bf16", ptr(b.h), H, ptr(L.ln_post), ptr(b.xn), H, R, H, c.eps, st)
                call("dsv2_gemm_bf16", ptr(b.xn), H, 0, R, H, ptr(L.w_router), 0, c.n_experts, 1, None, 0,
                     ptr(b.router_logits), c.n_experts, 0, LINEAR_OUT_F32_EXACT, st)
                call("dsv2_router_topk6_from_logits", ptr(b.router_logits), R, c.routed_scaling, ptr(b.ids32), None,
                     ptr(b.wts), st)
            elif R <= SPLIT_ROUTER_MAX_ROWS:
                call("dsv2_router_logits", ptr(b.h), H, ptr(L.ln_post), c.eps, ptr(L.w_router), R, ptr(b.xn),
                     ptr(b.router_logits), st)
                call("dsv2_router_topk6_from_logits", ptr(b.router_logits), R, c.routed_scaling, ptr(b.ids32), None,
                     ptr(b.wts), st)
            else:
                call("dsv2_router_topk6", ptr(b.h), H, ptr(L.ln_post), c.eps, ptr(L.w_router), c.routed_scaling, R,
                     ptr(b.xn), ptr(b.ids32), None, ptr(b.wts), st)
            if b.bucket_ws is not None and R >= WIDE_BUCKET_MIN_ROWS:
                call("dsv2_moe_bucket_wide", ptr(b.ids32), R, b.tile_tokens, ptr(b.sorted), ptr(b.route_pos),
                     ptr(b.tiles), ptr(b.ntiles), ptr(b.bucket_ws), b.bucket_ws.numel(), st)
            else:
                call("dsv2_moe_bucket", ptr(b.ids32), R, b.tile_tokens, ptr(b.sorted), ptr(b.route_pos),
                     ptr(b.tiles), ptr(b.ntiles), st)
            if self.expert_dtype == "fp8" and b is self.buf:
                # e4m3 routed and shared experts, the shared halves in the grouped launches
                call("dsv2_moe_grouped_gateup_shared_fp8", ptr(b.xn), R, ptr(b.sorted), ptr(b.tiles), ptr(b.ntiles),
                     b.max_tiles, b.tile_tokens, ptr(L.w_gu8), ptr(L.gu_scale), ptr(L.sh_gu8), ptr(L.sh_gu_scale),
                     c.moe_inter, ptr(b.hs), ptr(b.shmid), st)
                call("dsv2_moe_grouped_down_shared_fp8", ptr(b.hs), R, ptr(b.tiles), ptr(b.ntiles), b.max_tiles,
                     b.tile_tokens, ptr(L.w_down8), ptr(L.down_scale), ptr(b.shmid), ptr(L.sh_down8),
                     ptr(L.sh_down_scale), c.moe_inter, ptr(b.ys), ptr(b.shparts), st)
                call("dsv2_moe_combine_parts", ptr(b.ys), ptr(b.route_pos), ptr(b.wts), R, ptr(b.shparts),
                     ptr(b.h), ptr(b.h), ptr(next_norm), c.eps, ptr(b.xn), st)
            elif shared_in_grouped(R, b.tile_tokens):
                # the shared experts' two halves ride in the grouped launches as extra tiles
                call("dsv2_moe_grouped_gateup_shared", ptr(b.xn), R, ptr(b.sorted), ptr(b.tiles), ptr(b.ntiles),
                     b.max_tiles, b.tile_tokens, ptr(L.w_gu), ptr(L.sh_gu), c.moe_inter, ptr(b.hs), ptr(b.shmid),
                     st)
                call("dsv2_moe_grouped_down_shared", ptr(b.hs), R, ptr(b.tiles), ptr(b.ntiles), b.max_tiles,
                     b.tile_tokens, ptr(L.w_down), ptr(b.shmid), ptr(L.sh_down), c.moe_inter, ptr(b.ys),
                     ptr(b.shparts), st)
                call("dsv2_moe_combine_parts", ptr(b.ys), ptr(b.route_pos), ptr(b.wts), R, ptr(b.shparts),
                     ptr(b.h), ptr(b.h), ptr(next_norm), c.eps, ptr(b.xn), st)
            else:
                call("dsv2_moe_grouped_gateup", ptr(b.xn), ptr(b.sorted), ptr(b.tiles), ptr(b.ntiles), b.max_tiles,
                     b.tile_tokens, ptr(L.w_gu), c.moe_inter, ptr(b.hs), st)
                call("dsv2_moe_grouped_down", ptr(b.hs), ptr(b.tiles), ptr(b.ntiles), b.max_tiles, b.tile_tokens,
                     ptr(L.w_down), c.moe_inter, ptr(b.ys), st)
                call("dsv2_gemm_bf16", ptr(b.xn), H, 0, R, H, ptr(L.sh_gu), 0, c.shared_inter, 1, None, 0,
                     ptr(b.shmid), c.shared_inter, 0, LINEAR_SWIGLU, st)
                call("dsv2_gemm_bf16", ptr(b.shmid), c.shared_inter, 0, R, c.shared_inter, ptr(L.sh_down), 0, H, 1,
                     None, 0, ptr(b.shout), H, 0, 0, st)
                call("dsv2_moe_combine", ptr(b.ys), ptr(b.route_pos), ptr(b.wts), R, ptr(b.shout), ptr(b.h),
                     ptr(b.h), ptr(next_norm), c.eps, ptr(b.xn), st)
        else:
            call("dsv2_rmsnorm_bf16", ptr(b.h), H, ptr(L.ln_post), ptr(b.xn), H, R, H, c.eps, st)
            call("dsv2_gemm_bf16", ptr(b.xn), H, 0, R, H, ptr(L.w_gu), 0, c.dense_inter, 1, None, 0, ptr(b.mid),
                 c.dense_inter, 0, LINEAR_SWIGLU, st)
            call("dsv2_gemm_bf16", ptr(b.mid), c.dense_inter, 0, R, c.dense_inter, ptr(L.w_down), 0, H, 1, ptr(b.h),
                 H, ptr(b.h), H, 0, 0, st)
            call("dsv2_rmsnorm_bf16", ptr(b.h), H, ptr(next_norm), ptr(b.xn), H, R, H, c.eps, st)

    def _layers(self, b: RowBuffers, R: int, ids: torch.Tensor, pos, base, cap, family: str, st: int,
                record: list | None = None, rows: torch.Tensor | None = None, pf: PrefillPlan | None = None) -> None:
        """Enqueue the embedding gather and every layer for R kernel rows.  With `record`,
        append per layer ("attn", li, h), ("layer", li, h) and ("router", li, ids, weights)
        copies of the rows `rows` (device index tensor; all R rows when None)."""
        sel = (lambda t: t[:R].clone()) if rows is None else (lambda t: t.index_select(0, rows))
        c = self.cfg
        call("dsv2_embed_gather_bf16", ptr(ids), ptr(self.w.embed), c.hidden, ptr(b.h), R, st)
        if family == "batch":
            call("dsv2_rmsnorm_bf16", ptr(b.h), c.hidden, ptr(self.w.layers[0].ln_in), ptr(b.xn), c.hidden, R,
                 c.hidden, c.eps, st)
        n = len(self.w.layers)
        for li, L in enumerate(self.w.layers):
            self._attention(L, li, b, R, pos, base, cap, family, st, pf)
            if record is not None:
                record.append(("attn", li, sel(b.h)))
            next_norm = self.w.layers[li + 1].ln_in if li + 1 < n else self.w.norm
            self._mlp(L, li, b, R, family, next_norm, st)
            if record is not None:
                record.append(("layer", li, sel(b.h)))
                if L.moe:
                    record.append(("router", li, sel(b.ids32), sel(b.wts)))

    def _head(self, b: RowBuffers, family: str, st: int, pos) -> None:
        c = self.cfg
        B = self.B
        if family == "small" and B <= 8:
            call("dsv2_lm_head_argmax_bf16", ptr(b.h), c.hidden, B, ptr(self.w.lm_head), c.vocab, ptr(self.w.norm),
                 c.eps, ptr(self.logits), ptr(self._amax), self._amax.numel(), ptr(self.ids), ptr(pos), st)
            return
        if family == "small":
            call("dsv2_gemv_bf16", ptr(b.h), c.hidden, B, c.hidden, ptr(self.w.lm_head), c.vocab, ptr(self.w.norm),
                 c.eps, None, 0, ptr(self.logits), c.vocab, LINEAR_OUT_F32, st)
        else:  # b.xn already holds the final-normed hidden (fused into the last combine)
            call("dsv2_gemm_bf16", ptr(b.xn), c.hidden, 0, B, c.hidden, ptr(self.w.lm_head), 0, c.vocab, 1, None, 0,
                 ptr(self.logits), c.vocab, 0, LINEAR_OUT_F32, st)
        call("dsv2_argmax_f32", ptr(self.logits), B, c.vocab, ptr(self.ids), ptr(pos), st)

    # ------------------------------------------------------------------ public
    def step(self, record: list | None = None) -> None:
        """Enqueue one decode step for all rows: reads self.ids, writes self.logits and the
        next ids into self.ids, advances cache.pos.  No host synchronisation."""
        self._check_room()
        st = _hip.stream_ptr(self.device)
        self._layers(self.buf, self.B, self.ids, self.cache.pos, self.cache.base, self.cache.cap, self.family, st,
                     record)
        self._head(self.buf, self.family, st, self.cache.pos)
        self._host_pos = [p + 1 for p in self._host_pos]

    def prefill(self, prompts: list[torch.Tensor], record: list | None = None) -> torch.Tensor:
        """Eager prefill of one prompt per row: chunks of <= max_prefill_rows prompt tokens
        (one kernel row each, in sequence order) through the batch-family projections and
        grouped MoE, with the attention in MLA's expanded form (the chunk's cache rows, k_nope
        / v of the cached prefix by grouped GEMMs, causal MFMA flash attention per 128-query
        tile and head).  Writes the compressed cache, sets cache.pos = prompt lengths and
        self.ids = greedy first tokens (returned).  Mirrors _prefill_once (src/run.py:526-544).
        With `record`, it receives the per-layer records of each sequence's LAST prompt token,
        in the format of a recorded decode step (row b = sequence b)."""
        if len(prompts) != self.B:
            raise ValueError(f"need {self.B} prompts, got {len(prompts)}")
        self._free.clear()
        return self._prefill_slots(list(range(self.B)), prompts, record)

    def insert(self, slot: int, prompt: torch.Tensor) -> int:
        """Continuous batching: start a new sequence in `slot` (free, or to be overwritten)
        while the captured graph stays as it is.  The prompt is prefilled into the slot's own
        cache rows only, its position and next id are set in place (the graph reads them from
        the same device tensors), and the slot's first greedy token is returned.  The other
        rows are untouched.  The slot's capacity must hold the prompt plus the tokens it will
        generate."""
        if not 0 <= slot < self.B:
            raise ValueError(f"slot {slot} out of range [0, {self.B})")
        self._prefill_slots([slot], [prompt])
        self._free.discard(slot)
        return int(self.ids[slot].item())

    def retire(self, slot: int) -> None:
        """Continuous batching: end the sequence in `slot`.  The captured step keeps running
        every row, so a free slot goes on decoding throw-away tokens inside its own cache rows;
        its position restarts at 0 now and whenever it would reach its capacity (a device write
        before the replay), so it never stops the batch.  insert() reuses it."""
        if not 0 <= slot < self.B:
            raise ValueError(f"slot {slot} out of range [0, {self.B})")
        self._free.add(slot)
        self._reset_slots([slot])

    @property
    def free_slots(self) -> list[int]:
        return sorted(self._free)

    def _reset_slots(self, slots: list[int]) -> None:
        idx = torch.tensor(slots, dtype=torch.int64, device=self.device)
        self.cache.pos.index_fill_(0, idx, 0)
        for b in slots:
            self._host_pos[b] = 0

    def _prefill_slots(self, slots: list[int], prompts: list[torch.Tensor], record: list | None = None) -> torch.Tensor:
        lens = [int(p.numel()) for p in prompts]
        if not slots or min(lens) < 1:
            raise ValueError("empty prompt")
        if len(set(slots)) != len(slots):
            raise ValueError(f"slots repeat: {slots}")
        for b, n in zip(slots, lens):
            if n >= self.cache.capacities[b]:
                raise ValueError(f"prompt of length {n} does not fit slot {b} (capacity {self.cache.capacities[b]})")
        dev = self.device
        k = len(slots)
        seq = torch.cat([torch.full((n,), j, dtype=torch.int64) for j, n in enumerate(lens)])  # prompt index
        slot_t = torch.tensor(slots, dtype=torch.int64)
        posv = torch.cat([torch.arange(n, dtype=torch.int32) for n in lens])
        ids_all = torch.cat([p.reshape(-1).to(torch.int64).cpu() for p in prompts])
        base_all = self.cache.base.cpu()[slot_t[seq]]
        cap_all = self.cache.cap.cpu()[slot_t[seq]]
        total = seq.numel()
        max_rows = min(self.max_prefill_rows, total)
        pb = RowBuffers(self.cfg, max_rows, "batch", self.max_pos, dev, prefill=True)
        bases = [int(x) for x in self.cache.base.cpu()[slot_t]]
        plans = [prefill_groups(seq[s:s + max_rows], posv[s:s + max_rows], bases) for s in range(0, total, max_rows)]
        n_exp = max(g[2] for p in plans for g in p)
        nh, dk = self.cfg.n_heads, self.cfg.qk_nope
        kexp = torch.empty(n_exp, nh, dk, dtype=BF16, device=dev)
        vexp = torch.empty(n_exp, nh, self.cfg.v_dim, dtype=BF16, device=dev)
        last_h = torch.empty(k, self.cfg.hidden, dtype=BF16, device=dev)
        last_xn = torch.empty_like(last_h)
        st = _hip.stream_ptr(dev)
        acc: dict = {}
        for s in range(0, total, max_rows):
            e = min(total, s + max_rows)
            R = e - s
            ids_c = ids_all[s:e].to(dev)
            pos_c = posv[s:e].to(dev)
            base_c = base_all[s:e].to(dev)
            cap_c = cap_all[s:e].to(dev)
            is_last = (posv[s:e] + 1) == torch.tensor(lens)[seq[s:e]]
            rows = torch.nonzero(is_last).flatten()
            rows_d = rows.to(dev)
            which = seq[s:e][rows].to(dev)
            crec = [] if record is not None else None
            pf = PrefillPlan([(t.to(dev), lo, n) for t, lo, n in plans[s // max_rows]], kexp, vexp)
            self._layers(pb, R, ids_c, pos_c, base_c, cap_c, "batch", st, crec, rows_d, pf)
            for r in crec or ():
                for j, t in enumerate(r[2:]):  # scatter the last-token rows to their sequences
                    key = (r[0], r[1], j)
                    if key not in acc:
                        acc[key] = torch.zeros((self.B,) + tuple(t.shape[1:]), dtype=t.dtype, device=dev)
                    acc[key].index_copy_(0, slot_t.to(dev)[which], t)
            if rows.numel():
                last_h.index_copy_(0, which, pb.h[rows_d])
                last_xn.index_copy_(0, which, pb.xn[rows_d])
        # final norm is fused into the last layer's combine (pb.xn); lm_head + argmax
        c = self.cfg
        whole = slots == list(range(self.B))
        logits = self.logits if whole else torch.empty(k, c.vocab, dtype=torch.float32, device=dev)
        ids = self.ids if whole else torch.empty(k, dtype=torch.int64, device=dev)
        call("dsv2_gemm_bf16", ptr(last_xn), c.hidden, 0, k, c.hidden, ptr(self.w.lm_head), 0, c.vocab, 1, None,
             0, ptr(logits), c.vocab, 0, LINEAR_OUT_F32, st)
        call("dsv2_argmax_f32", ptr(logits), k, c.vocab, ptr(ids), None, st)
        slot_d = slot_t.to(dev)
        if not whole:
            self.logits.index_copy_(0, slot_d, logits)
            self.ids.index_copy_(0, slot_d, ids)
        self.cache.pos.index_copy_(0, slot_d, torch.tensor(lens, dtype=torch.int32, device=dev))
        for b, n in zip(slots, lens):
            self._host_pos[b] = n
        if record is not None:
            for (kind, li, j) in sorted(acc, key=lambda kk: (kk[1], ("attn", "layer", "router").index(kk[0]), kk[2])):
                if j == 0:
                    record.append((kind, li) + tuple(acc[(kind, li, jj)] for jj in range(3) if (kind, li, jj) in acc))
        self.buf.h.index_copy_(0, slot_d, last_h)
        del pb
        return self.ids

    def snapshot(self) -> tuple[torch.Tensor, torch.Tensor, list[int]]:
        return self.cache.snapshot(), self.ids.clone(), list(self._host_pos)

    def restore(self, snap) -> None:
        pos, ids, host = snap
        self.cache.restore(pos)
        self.ids.copy_(ids)
        self._host_pos = list(host)

    def tune_moe_tiles(self) -> int:
        """Batch family: pick the grouped MoE token tile from the routing of one eager step
        (state restored afterwards), like the reference's tile selection before capture
        (moe_batch.py:596-657) but without timing runs: the median over MoE layers of
        routing_load, mapped by tile_tokens_for_load.  Returns the tile."""
        if self.family != "batch":
            return 0
        snap = self.snapshot()
        rec: list = []
        self.step(record=rec)
        self.restore(snap)
        loads = sorted(routing_load(r[2], self.cfg.n_experts) for r in rec if r[0] == "router")
        load = loads[len(loads) // 2] if loads else None
        tile = tile_tokens_for_load(load, self.buf._routes) if loads else self.buf.tile_tokens
        tile = self._fit_tile(tile, load)
        self.buf.set_tile_tokens(tile)
        self._moe_tiles_tuned = True
        return tile

    def capture(self) -> torch.cuda.CUDAGraph:
        """Record one step() into a graph (positions/ids advance on every replay).  The batch
        family first picks its MoE token tile from one eager step (tune_moe_tiles).  Sets
        kernels_per_step to the number of nodes of the captured graph (every node is a kernel
        launch: the step records no copies or memsets)."""
        if self.family == "batch" and not getattr(self, "_moe_tiles_tuned", False):
            self.tune_moe_tiles()
        saved = list(self._host_pos)
        g = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(g):
            self.step()
        self._host_pos = saved
        self.kernels_per_step = _graph_node_count(g)
        g.instantiate()
        self.graph = g
        return g

    def check_errors(self) -> None:
        """Raise if a kernel of the steps so far skipped a cache write past a row's capacity
        (the device status word of the cache; synchronises).  step()/replay() refuse such a
        step on the host first, so this fires only when pos was changed behind their back."""
        self.cache.check_status()

    def _check_room(self) -> None:
        """Every row needs a free slot for its next token: pos[b] + 1 <= capacity[b]
        (the reference raises on overflow, src/run.py:131-134).  Retired slots restart at 0
        (outside graph capture: the reset is an eager device write)."""
        caps = self.cache.capacities
        wrap = [b for b in self._free if self._host_pos[b] + 1 > caps[b]]
        if wrap and not torch.cuda.is_current_stream_capturing():
            self._reset_slots(wrap)
        full = [b for b, (p, c) in enumerate(zip(self._host_pos, caps)) if p + 1 > c]
        if full:
            raise RuntimeError(f"KV cache capacity exhausted for rows {full[:8]} "
                               f"(positions {[self._host_pos[b] for b in full[:8]]}, "
                               f"capacities {[self.cache.capacities[b] for b in full[:8]]})")

    def replay(self) -> None:
        if self.graph is None:
            raise RuntimeError("capture() first")
        self._check_room()
        self.graph.replay()
        self._host_pos = [p + 1 for p in self._host_pos]
