"""The checkpoint loader end to end on the GPU: a 2-layer full-width model (dense layer 0 +
one MoE layer, full vocabulary) written to disk in the HF key layout of the published
checkpoint (per-expert MLPs, sharded safetensors, config.json, a tokenizer), loaded back with
dsv2lite.load_weights, must equal the in-memory weights bit for bit and decode to bitwise the
same logits; src/run.py --model-path runs the chat-templated prompt through it."""

from __future__ import annotations

import json
import os

import pytest
import torch

pytestmark = pytest.mark.gpu

from test_checkpoint import LITE_CONFIG, _save_tokenizer


def _write_checkpoint(w, path):
    from safetensors.torch import save_file

    cfg = w.cfg
    sd = {"model.embed_tokens.weight": w.embed, "model.norm.weight": w.norm, "lm_head.weight": w.lm_head}
    I = cfg.moe_inter
    for i in range(cfg.n_layers):
        p = f"model.layers.{i}."
        hf = w.hf_layer(i)
        for k in ("q_proj", "kv_a_proj_with_mqa", "kv_b_proj", "o_proj"):
            sd[p + f"self_attn.{k}.weight"] = hf[k]
        sd[p + "self_attn.kv_a_layernorm.weight"] = hf["kv_a_layernorm"]
        sd[p + "input_layernorm.weight"] = hf["input_layernorm"]
        sd[p + "post_attention_layernorm.weight"] = hf["post_attention_layernorm"]
        if "gate" in hf:
            sd[p + "mlp.gate.weight"] = hf["gate"]
            for e in range(cfg.n_experts):
                q = f"{p}mlp.experts.{e}."
                sd[q + "gate_proj.weight"] = hf["experts_gate_up"][e, :I]
                sd[q + "up_proj.weight"] = hf["experts_gate_up"][e, I:]
                sd[q + "down_proj.weight"] = hf["experts_down"][e]
            for k, n in (("sh_gate", "gate_proj"), ("sh_up", "up_proj"), ("sh_down", "down_proj")):
                sd[p + f"mlp.shared_experts.{n}.weight"] = hf[k]
        else:
            for k in ("gate_proj", "up_proj", "down_proj"):
                sd[p + f"mlp.{k}.weight"] = hf[k]
    names = sorted(sd)
    wm = {}
    os.makedirs(path, exist_ok=True)
    for k in range(2):
        fn = f"model-{k + 1:05d}-of-00002.safetensors"
        part = {n: sd[n].detach().to("cpu").contiguous() for n in names[k::2]}
        save_file(part, os.path.join(path, fn), metadata={"format": "pt"})
        wm.update({n: fn for n in part})
        del part
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(dict(LITE_CONFIG, num_hidden_layers=cfg.n_layers), f)
    _save_tokenizer(path)


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    import dsv2lite

    cfg = dsv2lite.DSV2Config(n_layers=2)
    w = dsv2lite.init_weights(cfg, device="cuda", seed=0)
    path = str(tmp_path_factory.mktemp("dsv2_ckpt"))
    _write_checkpoint(w, path)
    return w, path


def test_loaded_weights_equal_the_written_ones(ckpt):
    import dsv2lite

    w, path = ckpt
    w2 = dsv2lite.load_weights(path, device="cuda")
    assert w2.cfg == w.cfg
    for a, b in ((w.embed, w2.embed), (w.norm, w2.norm), (w.lm_head, w2.lm_head)):
        assert torch.equal(a, b)
    for L, L2 in zip(w.layers, w2.layers):
        for f in ("ln_in", "ln_post", "w_qkva", "kv_norm", "w_uk", "w_ukt", "w_uv", "w_o", "w_gu", "w_down",
                  "w_router", "sh_gu", "sh_down"):
            a, b = getattr(L, f), getattr(L2, f)
            assert (a is None and b is None) or torch.equal(a, b), f
        assert L.moe == L2.moe


@pytest.mark.parametrize("family", ["small", "batch"])
def test_loaded_model_decodes_bitwise_like_the_in_memory_one(ckpt, family):
    import dsv2lite

    w, path = ckpt
    w2 = dsv2lite.load_weights(path, device="cuda")
    g = torch.Generator().manual_seed(11)
    prompt = torch.randint(0, 102400, (20,), generator=g).cuda()
    out = []
    for ww in (w, w2):
        eng = dsv2lite.DecodeEngine(ww, [32, 32], family=family)
        eng.prefill([prompt, prompt[:9]])
        logits = [eng.logits.clone()]
        for _ in range(2):
            eng.step()
            logits.append(eng.logits.clone())
        out.append(torch.stack(logits))
    assert torch.equal(out[0], out[1])


def test_run_cli_with_model_path_and_chat_prompt(ckpt):
    from dsv2lite.checkpoint import chat_prompt_ids, load_tokenizer
    from src import run as R

    _, path = ckpt
    res = R.main(["--model-path", path, "--kernel-family", "small", "--max-new-tokens", "4", "--dump-token-ids",
                  "--prompt", "Write me a 500 word novel."])
    n = chat_prompt_ids(load_tokenizer(path), "Write me a 500 word novel.").numel()
    assert res["prompt_lens"] == n and res["batch_size"] == 1 and len(res["generated_token_ids"]) == 4
    # embed; dense layer: qkv_a with the W_UK absorption, MLA attention, o_proj, gate_up, down;
    # MoE layer: qkv_a + absorption, MLA attention, o_proj, router logits, routed gate_up,
    # routed down; lm_head + argmax
    assert res["kernels_per_step"] == 1 + 5 + 6 + 2
    assert 0 < res["roofline_fraction"] < 1 and 7e8 < res["hbm_bytes_per_step"] < 8e8
