"""CPU oracle for the DeepSeek-V2-Lite q_len=1 decode step.

TEST INFRASTRUCTURE ONLY.  This module is the checker, never the thing that
is measured or shipped: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product path lives in
``flash-deepseek-v2-lite_amd/`` and fails loudly when its HIP library is
missing; nothing there imports this file.

What it restates
----------------
The reference decodes through the HF remote-code DeepSeek-V2 model
(``trust_remote_code``, loaded at ``src/run.py:719-725``; the file itself is
not in the reference tree) with Triton kernels patched in
(``src/run.py:256-502``).  This file restates that math in plain PyTorch on
the CPU, with the remote code's bf16 rounding points made explicit:

* RMSNorm ``w * bf16(x * rsqrt(mean(x^2) + eps))`` in fp32
  (``triton_kernels/rmsnorm.py:24-56`` computes the same in fp32).
* Layer order ``norm -> attn -> +res -> norm -> mlp -> +res``
  (``src/run.py:460-493``).
* MLA attention with the expanded per-head K/V
  (``triton_kernels/attention_decode_batch.py:726-745`` for ``kv_b``,
  ``:240-342`` for the attention core, causal ``n <= pos`` at ``:285``).
* RoPE on de-interleaved pairs: out[i<32] = e*cos - o*sin,
  out[i>=32] = o*cos + e*sin
  (``triton_kernels/attention_decode_small.py:190-229``), with the YaRN
  cos/sin tables of the remote code (bf16 tables, attention factor 1.0 when
  ``mscale == mscale_all_dim``).
* Softmax scale ``192**-0.5 * mscale_all**2`` (``src/run.py:409`` passes the
  module's ``softmax_scale``).
* Router: fp32 logits from fp32 copies of x and W (``src/run.py:268-272``),
  softmax in fp32, top-6 by repeated max with ties to the lower index
  (``triton_kernels/moe_router.py:16-60``), times ``routed_scaling_factor``,
  no renormalisation.
* Experts: ``down(bf16(silu(gate x)) * (up x))`` with bf16 outputs, routed sum
  in fp32 in slot order then one bf16 round
  (``triton_kernels/moe_batch.py:366-387``, ``:56-92``), plus the shared
  experts (``src/run.py:341-352``).
* Greedy argmax over fp32 logits of the bf16 ``lm_head`` output
  (``src/run.py:252-253``, ``:541``).

``mode="fp32"`` drops every bf16 round, which is what the golden vectors of
``tests/golden/`` (made by transformers' native DeepseekV2 run in fp32) pin.

Every function here is pinned by a test in ``tests/test_oracle.py``: against
the transformers goldens, against closed forms (absorbed == expanded MLA in
fp64, constant-cache attention, RoPE as a rotation, YaRN ramp end points), and
against brute force on tiny inputs.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F


@dataclass(frozen=True)
class Dims:
    """Model dimensions; defaults are DeepSeek-V2-Lite (HF config.json)."""

    hidden: int = 2048
    n_heads: int = 16
    qk_nope: int = 128
    qk_rope: int = 64
    v_dim: int = 128
    kv_rank: int = 512
    n_experts: int = 64
    top_k: int = 6
    moe_inter: int = 1408
    n_shared: int = 2
    dense_inter: int = 10944
    vocab: int = 102400
    n_layers: int = 27
    first_dense: int = 1
    eps: float = 1e-6
    rope_theta: float = 10000.0
    yarn_factor: float = 40.0
    yarn_orig_max_pos: int = 4096
    yarn_beta_fast: float = 32.0
    yarn_beta_slow: float = 1.0
    yarn_mscale: float = 0.707
    yarn_mscale_all_dim: float = 0.707
    routed_scaling: float = 1.0

    @property
    def q_head(self) -> int:
        return self.qk_nope + self.qk_rope


def _rounder(mode: str):
    if mode == "bf16":
        return lambda t: t.to(torch.bfloat16).to(torch.float32)
    if mode in ("fp32", "fp64"):
        return lambda t: t
    raise ValueError(f"unknown oracle mode {mode!r}")


# ---------------------------------------------------------------------------
# RoPE (YaRN) -- remote-code DeepseekV2YarnRotaryEmbedding
# ---------------------------------------------------------------------------

def yarn_get_mscale(scale: float, mscale: float) -> float:
    if scale <= 1:
        return 1.0
    return 0.1 * mscale * math.log(scale) + 1.0


def yarn_inv_freq(d: Dims) -> torch.Tensor:
    """Inverse frequencies [rope/2] (fp32) blending interpolation/extrapolation."""
    dim = d.qk_rope
    base = d.rope_theta

    def corr_dim(n_rot: float) -> float:
        return (dim * math.log(d.yarn_orig_max_pos / (n_rot * 2 * math.pi))) / (2 * math.log(base))

    low = max(math.floor(corr_dim(d.yarn_beta_fast)), 0)
    high = min(math.ceil(corr_dim(d.yarn_beta_slow)), dim - 1)
    if low == high:
        high += 0.001
    ramp = torch.clamp((torch.arange(dim // 2, dtype=torch.float32) - low) / (high - low), 0, 1)
    extra_mask = 1.0 - ramp
    freq_extra = 1.0 / (base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    freq_inter = 1.0 / (d.yarn_factor * base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim))
    return freq_inter * (1 - extra_mask) + freq_extra * extra_mask


def yarn_attention_factor(d: Dims) -> float:
    return yarn_get_mscale(d.yarn_factor, d.yarn_mscale) / yarn_get_mscale(d.yarn_factor, d.yarn_mscale_all_dim)


def yarn_cos_sin(d: Dims, n_pos: int, mode: str = "bf16") -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin tables [n_pos, rope] = cat(freqs, freqs); bf16-rounded in bf16 mode."""
    rb = _rounder(mode)
    t = torch.arange(n_pos, dtype=torch.float32)
    freqs = torch.outer(t, yarn_inv_freq(d))
    emb = torch.cat((freqs, freqs), dim=-1)
    af = yarn_attention_factor(d)
    return rb(emb.cos() * af), rb(emb.sin() * af)


def softmax_scale(d: Dims) -> float:
    s = d.q_head ** -0.5
    if d.yarn_mscale_all_dim:
        m = yarn_get_mscale(d.yarn_factor, d.yarn_mscale_all_dim)
        s = s * m * m
    return s


def rope_deinterleave(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, rb) -> torch.Tensor:
    """Remote-code RoPE: de-interleave pairs then rotate_half.

    x [..., R]; cos/sin broadcastable to x.  Returns [evens', odds'] layout.
    """
    r = x.shape[-1]
    x = x.reshape(*x.shape[:-1], r // 2, 2).transpose(-1, -2).reshape(*x.shape[:-1], r)
    half = r // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return rb(rb(x * cos) + rb(rot * sin))


# ---------------------------------------------------------------------------
# building blocks
# ---------------------------------------------------------------------------

def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, rb) -> torch.Tensor:
    var = x.pow(2).mean(-1, keepdim=True)
    return rb(w * rb(x * torch.rsqrt(var + eps)))


def linear(x: torch.Tensor, w: torch.Tensor, rb) -> torch.Tensor:
    return rb(x @ w.t())


def mlp(x: torch.Tensor, w_gate: torch.Tensor, w_up: torch.Tensor, w_down: torch.Tensor, rb) -> torch.Tensor:
    g = linear(x, w_gate, rb)
    u = linear(x, w_up, rb)
    return linear(rb(rb(F.silu(g)) * u), w_down, rb)


def router_topk(x_norm: torch.Tensor, w_router: torch.Tensor, top_k: int, scaling: float):
    """fp32 logits -> softmax -> top-k by repeated max (ties -> lower index).

    Returns (ids int64 [T,k] in descending score order, weights fp32 [T,k],
    scores fp32 [T,E]).
    """
    logits = x_norm.to(torch.float32) @ w_router.to(torch.float32).t()
    scores = torch.softmax(logits, dim=-1, dtype=torch.float32)
    work = scores.clone()
    ids = torch.empty(scores.shape[0], top_k, dtype=torch.int64)
    wts = torch.empty(scores.shape[0], top_k, dtype=torch.float32)
    for s in range(top_k):
        m = work.max(dim=-1).values
        # lowest index among the maxima
        idx = torch.argmax((work == m[:, None]).to(torch.int8), dim=-1)
        ids[:, s] = idx
        wts[:, s] = scores.gather(1, idx[:, None])[:, 0]
        work.scatter_(1, idx[:, None], float("-inf"))
    return ids, wts * scaling, scores


def topk_margin(scores: torch.Tensor, top_k: int) -> torch.Tensor:
    """s_k - s_{k+1} per row (the gap that decides set membership)."""
    srt = torch.sort(scores, dim=-1, descending=True).values
    return srt[:, top_k - 1] - srt[:, top_k]


@dataclass
class SeqCache:
    """Per-sequence compressed cache of one layer (c_norm [L,r], k_pe_rot [L,R])."""

    c: list = field(default_factory=list)
    kpe: list = field(default_factory=list)

    def length(self) -> int:
        return sum(t.shape[0] for t in self.c)


def attention(lw: dict, d: Dims, x_norm: torch.Tensor, cache: SeqCache, positions: torch.Tensor,
              cos: torch.Tensor, sin: torch.Tensor, rb, scale: float | None = None,
              trace: dict | None = None) -> torch.Tensor:
    """Remote-code MLA over the expanded K/V for T new tokens of ONE sequence.

    x_norm [T, hidden]; positions [T] are cache indices (0-based, contiguous
    after the cached tokens).  Appends the new compressed rows to ``cache``.
    """
    T = x_norm.shape[0]
    nh, dn, dr, dv = d.n_heads, d.qk_nope, d.qk_rope, d.v_dim
    q = linear(x_norm, lw["q_proj"], rb).view(T, nh, dn + dr)
    q_nope, q_pe = q[..., :dn], q[..., dn:]
    ckv = linear(x_norm, lw["kv_a_proj_with_mqa"], rb)
    c, k_pe = ckv[:, : d.kv_rank], ckv[:, d.kv_rank:]
    c_n = rmsnorm(c, lw["kv_a_layernorm"], d.eps, rb)
    cs, sn = cos[positions], sin[positions]
    q_pe = rope_deinterleave(q_pe, cs[:, None, :], sn[:, None, :], rb)
    k_pe = rope_deinterleave(k_pe, cs, sn, rb)
    cache.c.append(c_n)
    cache.kpe.append(k_pe)
    if trace is not None:
        trace["c_norm"] = c_n
        trace["k_pe"] = k_pe
        trace["q_pe"] = q_pe
        trace["q_nope"] = q_nope
    c_all = torch.cat(cache.c, 0)
    kpe_all = torch.cat(cache.kpe, 0)
    L = c_all.shape[0]
    kv = linear(c_all, lw["kv_b_proj"], rb).view(L, nh, dn + dv)
    k_nope, v = kv[..., :dn], kv[..., dn:]
    K = torch.cat((k_nope, kpe_all[:, None, :].expand(L, nh, dr)), dim=-1)  # [L, nh, 192]
    Q = torch.cat((q_nope, q_pe), dim=-1)  # [T, nh, 192]
    sc = rb(torch.einsum("thd,lhd->htl", Q, K))
    sc = rb(sc * (softmax_scale(d) if scale is None else scale))
    mask = torch.arange(L)[None, :] > positions[:, None]  # [T, L]
    sc = sc.masked_fill(mask[None], float("-inf"))
    p = rb(torch.softmax(sc, dim=-1, dtype=torch.float64 if sc.dtype == torch.float64 else torch.float32))
    o = rb(torch.einsum("htl,lhd->thd", p, v)).reshape(T, nh * dv)
    return linear(o, lw["o_proj"], rb)


def absorbed_attention(lw: dict, d: Dims, q_nope: torch.Tensor, q_pe_rot: torch.Tensor, c_all: torch.Tensor,
                       kpe_all: torch.Tensor, n_valid: int, scale: float) -> torch.Tensor:
    """Absorbed MLA for ONE query (no rounding): returns o_lat-projected [nh*dv].

    q_lat_h = W_UK_h^T q_nope_h; score = q_lat_h . c + q_pe_h . k_pe;
    out_h = W_UV_h (sum p c).  Used to prove absorbed == expanded in fp64.
    """
    nh, dn, dv = d.n_heads, d.qk_nope, d.v_dim
    wkvb = lw["kv_b_proj"].view(nh, dn + dv, d.kv_rank)
    w_uk, w_uv = wkvb[:, :dn, :], wkvb[:, dn:, :]
    q_lat = torch.einsum("hi,hij->hj", q_nope, w_uk)
    c, kp = c_all[:n_valid], kpe_all[:n_valid]
    s = (q_lat @ c.t() + q_pe_rot @ kp.t()) * scale  # [nh, L]
    p = torch.softmax(s, dim=-1)
    o_lat = p @ c  # [nh, r]
    return torch.einsum("hij,hj->hi", w_uv, o_lat).reshape(nh * dv)


def moe(lw: dict, d: Dims, x_norm: torch.Tensor, rb, trace: dict | None = None) -> torch.Tensor:
    """Routed top-k experts + shared experts for T tokens."""
    ids, wts, scores = router_topk(x_norm, lw["gate"], d.top_k, d.routed_scaling)
    if trace is not None:
        trace["router_ids"] = ids
        trace["router_w"] = wts
        trace["router_scores"] = scores
    T = x_norm.shape[0]
    I = d.moe_inter
    outs = torch.zeros(T, d.top_k, d.hidden, dtype=x_norm.dtype)
    for e in torch.unique(ids).tolist():
        tok, slot = torch.nonzero(ids == e, as_tuple=True)
        gu = lw["experts_gate_up"][e]
        y = mlp(x_norm[tok], gu[:I], gu[I:], lw["experts_down"][e], rb)
        outs[tok, slot] = y
    routed = torch.zeros(T, d.hidden, dtype=x_norm.dtype)
    for s in range(d.top_k):  # fixed slot order, fp32
        routed = routed + wts[:, s: s + 1].to(x_norm.dtype) * outs[:, s]
    routed = rb(routed)
    shared = mlp(x_norm, lw["sh_gate"], lw["sh_up"], lw["sh_down"], rb)
    return rb(routed + shared)


def layer_forward(lw: dict, d: Dims, layer: int, h: torch.Tensor, cache: SeqCache, positions: torch.Tensor,
                  cos: torch.Tensor, sin: torch.Tensor, rb, trace: dict | None = None) -> torch.Tensor:
    xn = rmsnorm(h, lw["input_layernorm"], d.eps, rb)
    a = attention(lw, d, xn, cache, positions, cos, sin, rb, trace=trace)
    h = rb(h + a)
    if trace is not None:
        trace["h_attn"] = h
    xn = rmsnorm(h, lw["post_attention_layernorm"], d.eps, rb)
    if layer < d.first_dense:
        m = mlp(xn, lw["gate_proj"], lw["up_proj"], lw["down_proj"], rb)
    else:
        m = moe(lw, d, xn, rb, trace=trace)
    return rb(h + m)


class OracleModel:
    """Whole-model oracle.  ``weights`` holds HF-named fp32 tensors:

    ``embed``, ``norm``, ``lm_head`` and ``layers[i]`` dicts with ``q_proj``,
    ``kv_a_proj_with_mqa``, ``kv_a_layernorm``, ``kv_b_proj``, ``o_proj``,
    ``input_layernorm``, ``post_attention_layernorm`` and either
    ``gate_proj/up_proj/down_proj`` (dense) or ``gate``, ``experts_gate_up``
    [E, 2I, H], ``experts_down`` [E, H, I], ``sh_gate``, ``sh_up``,
    ``sh_down`` (MoE).
    """

    def __init__(self, dims: Dims, weights: dict, mode: str = "bf16", max_pos: int = 4096):
        self.d = dims
        self.w = weights
        self.mode = mode
        self.rb = _rounder(mode)
        self.cos, self.sin = yarn_cos_sin(dims, max_pos, mode)
        if mode == "fp64":
            self.cos, self.sin = self.cos.double(), self.sin.double()

    def new_cache(self) -> list[SeqCache]:
        return [SeqCache() for _ in range(len(self.w["layers"]))]

    def forward(self, ids: torch.Tensor | None, cache: list[SeqCache], start_pos: int,
                h: torch.Tensor | None = None, trace: list | None = None, last_logits_only: bool = False) -> dict:
        """Run T tokens of ONE sequence from position ``start_pos``.

        Returns {"hidden": [T,H] final (pre-norm) hidden, "logits": [T,V] fp32 (only the
        last token's row, [1,V], with last_logits_only), "layer_out": list of [T,H]}.
        """
        if h is None:
            h = self.w["embed"][ids]
        T = h.shape[0]
        positions = torch.arange(start_pos, start_pos + T)
        outs = []
        for i, lw in enumerate(self.w["layers"]):
            tr = {} if trace is not None else None
            h = layer_forward(lw, self.d, i, h, cache[i], positions, self.cos, self.sin, self.rb, trace=tr)
            outs.append(h)
            if trace is not None:
                trace.append(tr)
        res = {"hidden": h, "layer_out": outs}
        if "lm_head" in self.w:
            xn = rmsnorm(h[-1:] if last_logits_only else h, self.w["norm"], self.d.eps, self.rb)
            res["logits"] = linear(xn, self.w["lm_head"], self.rb).to(torch.float32)
        return res


def greedy(logits: torch.Tensor) -> torch.Tensor:
    """First index of the maximum (torch.argmax semantics)."""
    return torch.argmax(logits, dim=-1)


def init_weights_cpu(d: Dims, n_layers: int, seed: int = 0, std: float = 0.02,
                     with_head: bool = True) -> dict:
    """Seeded N(0, std) weights on the CPU, bf16-representable fp32 (norm weights 1).

    Used for the CPU baseline (timing only) and for CPU-only tests; GPU parity
    tests instead copy the product's device weights back to the host.
    """
    g = torch.Generator().manual_seed(seed)

    def rnd(*shape):
        return (torch.randn(*shape, generator=g) * std).to(torch.bfloat16).to(torch.float32)

    H, nh = d.hidden, d.n_heads
    layers = []
    for i in range(n_layers):
        lw = {
            "q_proj": rnd(nh * d.q_head, H),
            "kv_a_proj_with_mqa": rnd(d.kv_rank + d.qk_rope, H),
            "kv_a_layernorm": torch.ones(d.kv_rank),
            "kv_b_proj": rnd(nh * (d.qk_nope + d.v_dim), d.kv_rank),
            "o_proj": rnd(H, nh * d.v_dim),
            "input_layernorm": torch.ones(H),
            "post_attention_layernorm": torch.ones(H),
        }
        if i < d.first_dense:
            lw.update(gate_proj=rnd(d.dense_inter, H), up_proj=rnd(d.dense_inter, H),
                      down_proj=rnd(H, d.dense_inter))
        else:
            Is = d.moe_inter * d.n_shared
            lw.update(gate=rnd(d.n_experts, H), experts_gate_up=rnd(d.n_experts, 2 * d.moe_inter, H),
                      experts_down=rnd(d.n_experts, H, d.moe_inter), sh_gate=rnd(Is, H), sh_up=rnd(Is, H),
                      sh_down=rnd(H, Is))
        layers.append(lw)
    w = {"layers": layers}
    if with_head:
        w["embed"] = rnd(d.vocab, H)
        w["norm"] = torch.ones(H)
        w["lm_head"] = rnd(d.vocab, H)
    return w
