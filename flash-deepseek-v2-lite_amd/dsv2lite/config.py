"""DeepSeek-V2-Lite dimensions (the HF config.json of DeepSeek-V2-Lite-Chat).

The HIP kernels are specialised to these shapes; ``n_layers`` and ``vocab`` may
be reduced for tests.  The reference hard-codes the same constants
(triton_kernels/attention_decode_batch.py:13-22) and checks them in its patch
guards (src/run.py:258-267).
"""

from __future__ import annotations

import math
from dataclasses import dataclass


@dataclass(frozen=True)
class DSV2Config:
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

    @property
    def qkva_dim(self) -> int:
        """Fused q_proj | kv_a_proj_with_mqa output width (3072 + 576 = 3648)."""
        return self.n_heads * self.q_head + self.kv_rank + self.qk_rope

    @property
    def cache_row(self) -> int:
        """Compressed cache row: normalised latent + rotated k_pe (576)."""
        return self.kv_rank + self.qk_rope

    @property
    def shared_inter(self) -> int:
        return self.moe_inter * self.n_shared

    @property
    def softmax_scale(self) -> float:
        """q_head**-0.5 * yarn_mscale(factor, mscale_all_dim)**2 (HF DeepseekV2Attention)."""
        m = 0.1 * self.yarn_mscale_all_dim * math.log(self.yarn_factor) + 1.0 if self.yarn_factor > 1 else 1.0
        return self.q_head ** -0.5 * m * m

    def is_moe_layer(self, i: int) -> bool:
        return i >= self.first_dense

    def check_kernel_dims(self) -> None:
        """The HIP kernels hard-code these; anything else is rejected up front."""
        fixed = dict(hidden=2048, n_heads=16, qk_nope=128, qk_rope=64, v_dim=128, kv_rank=512, n_experts=64,
                     top_k=6, moe_inter=1408, n_shared=2)
        bad = {k: getattr(self, k) for k, v in fixed.items() if getattr(self, k) != v}
        if bad:
            raise ValueError(f"HIP kernels are specialised to DeepSeek-V2-Lite dims; unsupported: {bad}")
        if self.dense_inter % 64 or self.vocab % 64:
            raise ValueError("dense_inter and vocab must be multiples of 64")
