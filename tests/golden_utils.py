"""Helpers shared by the tests: load golden fixtures into oracle form."""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
PKG = os.path.join(ROOT, "flash-deepseek-v2-lite_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle.dsv2_oracle import Dims  # noqa: E402

TINY_DIMS = Dims(hidden=64, n_heads=4, qk_nope=16, qk_rope=8, v_dim=16, kv_rank=32, n_experts=8, top_k=3,
                 moe_inter=24, n_shared=2, dense_inter=96, vocab=128, n_layers=3, first_dense=1)


def load_npz(name: str) -> dict:
    z = np.load(os.path.join(GOLDEN, name))  # allow_pickle stays False
    return {k: z[k] for k in z.files}


def tiny_oracle_weights(z: dict, dtype=torch.float32) -> dict:
    def t(k):
        return torch.from_numpy(z["w/" + k]).to(dtype)

    layers = []
    for i in range(TINY_DIMS.n_layers):
        p = f"model.layers.{i}."
        lw = {
            "q_proj": t(p + "self_attn.q_proj.weight"),
            "kv_a_proj_with_mqa": t(p + "self_attn.kv_a_proj_with_mqa.weight"),
            "kv_a_layernorm": t(p + "self_attn.kv_a_layernorm.weight"),
            "kv_b_proj": t(p + "self_attn.kv_b_proj.weight"),
            "o_proj": t(p + "self_attn.o_proj.weight"),
            "input_layernorm": t(p + "input_layernorm.weight"),
            "post_attention_layernorm": t(p + "post_attention_layernorm.weight"),
        }
        if i < TINY_DIMS.first_dense:
            lw.update(gate_proj=t(p + "mlp.gate_proj.weight"), up_proj=t(p + "mlp.up_proj.weight"),
                      down_proj=t(p + "mlp.down_proj.weight"))
        else:
            lw.update(gate=t(p + "mlp.gate.weight"), experts_gate_up=t(p + "mlp.experts.gate_up_proj"),
                      experts_down=t(p + "mlp.experts.down_proj"),
                      sh_gate=t(p + "mlp.shared_experts.gate_proj.weight"),
                      sh_up=t(p + "mlp.shared_experts.up_proj.weight"),
                      sh_down=t(p + "mlp.shared_experts.down_proj.weight"))
        layers.append(lw)
    return {"layers": layers, "embed": t("model.embed_tokens.weight"), "norm": t("model.norm.weight"),
            "lm_head": t("lm_head.weight")}


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """max|a-b| / max|b| -- the relative error used by every parity check."""
    a = a.double()
    b = b.double()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))
