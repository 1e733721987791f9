"""The decode step's algorithmic HBM bytes: every weight read once (attention, router, the
routed experts actually hit, shared experts, dense layer 0, lm_head, norms), the embedding
rows gathered and the compressed KV rows read (1,152 B per cached token per layer).  Divided
by the step time and the MI355X's 8 TB/s HBM peak it gives the step's roofline fraction."""

from __future__ import annotations

from .config import DSV2Config

HBM_PEAK = 8.0e12  # bytes/s, MI355X HBM3E


def step_bytes(cfg: DSV2Config, n_exp_per_layer: list[int], ctx_sum_per_layer: float, batch: int,
               expert_fp8: bool = False) -> float:
    """n_exp_per_layer: distinct routed experts hit in each MoE layer (from the router output);
    ctx_sum_per_layer: cached tokens read per layer summed over the rows (sum of pos + 1).
    expert_fp8: routed and shared expert weights read as e4m3 (1 byte) plus one fp32 scale
    per row."""
    H = cfg.hidden
    attn_w = H * cfg.qkva_dim + cfg.kv_rank * cfg.n_heads * (cfg.qk_nope + cfg.v_dim) + H * cfg.n_heads * cfg.v_dim
    expert = 3 * H * cfg.moe_inter
    shared = 3 * H * cfg.shared_inter
    dense = 3 * H * cfg.dense_inter
    head = cfg.vocab * H
    norms = 2 * H + cfg.kv_rank  # input / post-attention RMSNorm + kv-norm per layer
    n_moe = sum(1 for i in range(cfg.n_layers) if cfg.is_moe_layer(i))
    moe = sum(n * expert + shared for n in n_exp_per_layer)
    elems = cfg.n_layers * attn_w + cfg.n_layers * norms + (cfg.n_layers - n_moe) * dense + head + H
    router = n_moe * cfg.n_experts * H
    if expert_fp8:
        rows = sum(n * (2 * cfg.moe_inter + H) + 2 * cfg.shared_inter + H for n in n_exp_per_layer)
        moe_bytes = moe + 4 * rows
    else:
        moe_bytes = 2 * moe
    return 2 * (elems + router) + moe_bytes + 2 * H * batch + 2 * cfg.cache_row * ctx_sum_per_layer * cfg.n_layers


def roofline_fraction(nbytes: float, seconds: float) -> float:
    return nbytes / seconds / HBM_PEAK
