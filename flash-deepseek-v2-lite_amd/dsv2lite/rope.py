"""YaRN rotary tables of DeepSeek-V2 (HF remote-code DeepseekV2YarnRotaryEmbedding).

Tables are [n_pos, 64] = cat(freqs, freqs) with freqs = t * inv_freq in fp32,
scaled by mscale(factor, mscale)/mscale(factor, mscale_all_dim) (= 1.0 for
DeepSeek-V2-Lite) and stored in bf16 -- the form the reference passes to its
kernels (src/run.py:372-373).
"""

from __future__ import annotations

import math

import torch

from .config import DSV2Config


def _mscale(scale: float, m: float) -> float:
    return 1.0 if scale <= 1 else 0.1 * m * math.log(scale) + 1.0


def inv_freq(cfg: DSV2Config) -> torch.Tensor:
    dim, base = cfg.qk_rope, cfg.rope_theta

    def correction_dim(rotations: float) -> float:
        return dim * math.log(cfg.yarn_orig_max_pos / (rotations * 2 * math.pi)) / (2 * math.log(base))

    lo = max(math.floor(correction_dim(cfg.yarn_beta_fast)), 0)
    hi = min(math.ceil(correction_dim(cfg.yarn_beta_slow)), dim - 1)
    if lo == hi:
        hi += 0.001
    idx = torch.arange(dim // 2, dtype=torch.float32)
    keep_extrapolated = 1.0 - torch.clamp((idx - lo) / (hi - lo), 0.0, 1.0)
    pos_freq = base ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim)
    return (1.0 / (cfg.yarn_factor * pos_freq)) * (1.0 - keep_extrapolated) + (1.0 / pos_freq) * keep_extrapolated


def cos_sin_tables(cfg: DSV2Config, n_pos: int, device=None) -> tuple[torch.Tensor, torch.Tensor]:
    t = torch.arange(n_pos, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq(cfg))
    emb = torch.cat((freqs, freqs), dim=-1)
    att = _mscale(cfg.yarn_factor, cfg.yarn_mscale) / _mscale(cfg.yarn_factor, cfg.yarn_mscale_all_dim)
    cos = (emb.cos() * att).to(torch.bfloat16)
    sin = (emb.sin() * att).to(torch.bfloat16)
    return cos.to(device).contiguous(), sin.to(device).contiguous()
