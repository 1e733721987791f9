"""Write the golden vectors that pin the CPU oracle.

Run in the build container only (needs transformers; nothing here travels to
the GPU box as code -- only the .npz data it writes):

    python tests/golden/make_golden.py

Source of truth: transformers 5.15.0's native ``DeepseekV2ForCausalLM``
(``transformers/models/deepseek_v2/modeling_deepseek_v2.py``), built offline
from a ``DeepseekV2Config`` with seeded random weights.  It is mathematically
the HF remote DeepSeek-V2 code the reference runs (router, experts, shared
experts, RMSNorm, YaRN inverse frequencies, softmax scale) except that its RoPE
rotates interleaved pairs, which leaves attention scores unchanged.

Fixtures written:
* ``tiny_model.npz`` -- 3-layer model (1 dense + 2 MoE) with small dims, fp32:
  weights (HF names), token ids, full-sequence logits and per-layer hidden
  states, router top-k sets, and the logits of an incremental decode
  (prefill 8 tokens, then 4 q_len=1 steps through the KV cache).
* ``yarn_real.npz`` -- DeepSeek-V2-Lite RoPE at real dims: inv_freq, cos/sin
  at selected positions, attention factor and softmax scale.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

TINY = dict(
    vocab_size=128, hidden_size=64, intermediate_size=96, moe_intermediate_size=24,
    num_hidden_layers=3, num_attention_heads=4, num_key_value_heads=4, q_lora_rank=None,
    kv_lora_rank=32, qk_nope_head_dim=16, qk_rope_head_dim=8, v_head_dim=16,
    n_routed_experts=8, num_experts_per_tok=3, n_shared_experts=2, first_k_dense_replace=1,
    routed_scaling_factor=1.0, topk_method="greedy", norm_topk_prob=False,
    max_position_embeddings=163840, rms_norm_eps=1e-6, tie_word_embeddings=False,
    hidden_act="silu",
)

YARN = dict(rope_type="yarn", rope_theta=10000.0, factor=40.0, original_max_position_embeddings=4096,
            beta_fast=32.0, beta_slow=1.0, mscale=0.707, mscale_all_dim=0.707)

REAL = dict(
    vocab_size=102400, hidden_size=2048, intermediate_size=10944, moe_intermediate_size=1408,
    num_hidden_layers=27, num_attention_heads=16, num_key_value_heads=16, q_lora_rank=None,
    kv_lora_rank=512, qk_nope_head_dim=128, qk_rope_head_dim=64, v_head_dim=128,
    n_routed_experts=64, num_experts_per_tok=6, n_shared_experts=2, first_k_dense_replace=1,
    max_position_embeddings=163840, rms_norm_eps=1e-6,
)


def _config(**kw):
    from transformers import DeepseekV2Config

    cfg = DeepseekV2Config(**kw, rope_parameters=dict(YARN))
    cfg._attn_implementation = "eager"
    return cfg


def make_tiny() -> None:
    from transformers import DeepseekV2ForCausalLM
    from transformers.cache_utils import DynamicCache

    torch.manual_seed(0)
    cfg = _config(**TINY)
    model = DeepseekV2ForCausalLM(cfg).to(torch.float32).eval()
    g = torch.Generator().manual_seed(1234)
    out = {}
    with torch.no_grad():
        for name, p in sorted(model.named_parameters()):
            if name.endswith("norm.weight") or name.endswith("layernorm.weight"):
                v = 1.0 + 0.1 * torch.randn(p.shape, generator=g)
            else:
                # std 0.15 keeps activations O(1), so the nonlinear terms
                # (SwiGLU asymmetry, softmax shape) move the logits measurably
                v = 0.15 * torch.randn(p.shape, generator=g)
                if "embed_tokens" in name:
                    v = v / 0.15  # O(1) embeddings
            p.copy_(v)
            out["w/" + name] = v.numpy().astype(np.float32)

    ids = torch.randint(0, TINY["vocab_size"], (1, 12), generator=g)
    out["ids"] = ids.numpy()

    # router top-k sets per MoE layer via forward hooks on the router module
    router_sets: dict[int, torch.Tensor] = {}

    def hook(li):
        def f(_mod, _inp, res):
            _, _, idx = res
            router_sets[li] = torch.sort(idx, dim=-1).values.clone()
        return f

    hooks = [layer.mlp.gate.register_forward_hook(hook(i)) for i, layer in enumerate(model.model.layers)
             if hasattr(layer.mlp, "gate")]
    with torch.no_grad():
        res = model(input_ids=ids, output_hidden_states=True, use_cache=False)
    for h in hooks:
        h.remove()
    out["logits"] = res.logits[0].numpy()
    # hidden_states: embeddings + each layer output (last one is after the final norm in HF)
    hs = [t[0].numpy() for t in res.hidden_states]
    out["hidden_embed"] = hs[0]
    for i in range(1, TINY["num_hidden_layers"]):
        out[f"hidden_layer{i - 1}"] = hs[i]
    for li, s in router_sets.items():
        out[f"router_set_layer{li}"] = s.numpy()

    # incremental decode through the cache: prefill 8, then 4 single steps
    with torch.no_grad():
        cache = DynamicCache(config=cfg)
        r = model(input_ids=ids[:, :8], past_key_values=cache, use_cache=True)
        step_logits = [r.logits[0, -1]]
        for t in range(8, 12):
            r = model(input_ids=ids[:, t:t + 1], past_key_values=cache, use_cache=True)
            step_logits.append(r.logits[0, -1])
    out["decode_logits"] = torch.stack(step_logits).numpy()

    # bf16 run of the same model for a looser rounding-order check
    mb = model.to(torch.bfloat16)
    with torch.no_grad():
        rb = mb(input_ids=ids, use_cache=False)
    out["logits_bf16"] = rb.logits[0].float().numpy()

    np.savez_compressed(os.path.join(HERE, "tiny_model.npz"), **out)


def make_yarn_real() -> None:
    from transformers.models.deepseek_v2.modeling_deepseek_v2 import (
        DeepseekV2Attention, DeepseekV2RotaryEmbedding)

    cfg = _config(**REAL)
    rot = DeepseekV2RotaryEmbedding(cfg)
    pos = torch.tensor([[0, 1, 2, 5, 31, 127, 128, 1000, 2047, 2048, 4095, 4096, 8191, 16383]])
    x = torch.zeros(1, 1, 64)
    fc = rot(x, pos)[0]  # complex [P, 32]
    attn = DeepseekV2Attention(cfg, layer_idx=0)
    np.savez_compressed(
        os.path.join(HERE, "yarn_real.npz"),
        inv_freq=rot.inv_freq.numpy(), positions=pos[0].numpy(), cos=fc.real.numpy(), sin=fc.imag.numpy(),
        attention_scaling=np.float64(rot.attention_scaling), softmax_scale=np.float64(attn.scaling),
    )


if __name__ == "__main__":
    make_tiny()
    make_yarn_real()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")), file=sys.stderr)
