"""The checkpoint loader on the CPU (dsv2lite.checkpoint): the safetensors parser against the
safetensors package byte for byte, the shard index, HF key names -> packed layouts, config.json
-> DSV2Config, and the chat template through a locally built tokenizer.  The reference loads
the same format with transformers (src/run.py:719-737) and packs the experts as
moe_batch.py:324-363."""

from __future__ import annotations

import json
import os

import pytest
import torch

from golden_utils import TINY_DIMS

# DeepSeek-V2-Lite-Chat's config.json fields the loader reads (the published values)
LITE_CONFIG = {
    "model_type": "deepseek_v2", "architectures": ["DeepseekV2ForCausalLM"], "max_position_embeddings": 163840,
    "hidden_size": 2048, "num_attention_heads": 16, "qk_nope_head_dim": 128, "qk_rope_head_dim": 64,
    "v_head_dim": 128, "kv_lora_rank": 512, "q_lora_rank": None, "n_routed_experts": 64, "num_experts_per_tok": 6,
    "moe_intermediate_size": 1408, "n_shared_experts": 2, "intermediate_size": 10944, "vocab_size": 102400,
    "num_hidden_layers": 27, "first_k_dense_replace": 1, "rms_norm_eps": 1e-6, "rope_theta": 10000,
    "rope_scaling": {"type": "yarn", "factor": 40, "original_max_position_embeddings": 4096, "beta_fast": 32,
                     "beta_slow": 1, "mscale": 0.707, "mscale_all_dim": 0.707},
    "routed_scaling_factor": 1.0, "scoring_func": "softmax", "topk_method": "greedy", "norm_topk_prob": False,
}


def _tiny_state(seed=0):
    """HF remote-code key names at the tiny test dims (per-expert MLPs, dense layer 0)."""
    d = TINY_DIMS
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: (torch.randn(*s, generator=g) * 0.02).to(torch.bfloat16)  # noqa: E731
    sd = {"model.embed_tokens.weight": r(d.vocab, d.hidden), "model.norm.weight": r(d.hidden),
          "lm_head.weight": r(d.vocab, d.hidden)}
    for i in range(d.n_layers):
        p = f"model.layers.{i}."
        sd.update({p + "input_layernorm.weight": r(d.hidden), p + "post_attention_layernorm.weight": r(d.hidden),
                   p + "self_attn.q_proj.weight": r(d.n_heads * d.q_head, d.hidden),
                   p + "self_attn.kv_a_proj_with_mqa.weight": r(d.kv_rank + d.qk_rope, d.hidden),
                   p + "self_attn.kv_a_layernorm.weight": r(d.kv_rank),
                   p + "self_attn.kv_b_proj.weight": r(d.n_heads * (d.qk_nope + d.v_dim), d.kv_rank),
                   p + "self_attn.o_proj.weight": r(d.hidden, d.n_heads * d.v_dim)})
        if i < d.first_dense:
            sd.update({p + "mlp.gate_proj.weight": r(d.dense_inter, d.hidden),
                       p + "mlp.up_proj.weight": r(d.dense_inter, d.hidden),
                       p + "mlp.down_proj.weight": r(d.hidden, d.dense_inter)})
        else:
            sd[p + "mlp.gate.weight"] = r(d.n_experts, d.hidden)
            for e in range(d.n_experts):
                q = f"{p}mlp.experts.{e}."
                sd.update({q + "gate_proj.weight": r(d.moe_inter, d.hidden), q + "up_proj.weight": r(d.moe_inter, d.hidden),
                           q + "down_proj.weight": r(d.hidden, d.moe_inter)})
            Is = d.moe_inter * d.n_shared
            sd.update({p + "mlp.shared_experts.gate_proj.weight": r(Is, d.hidden),
                       p + "mlp.shared_experts.up_proj.weight": r(Is, d.hidden),
                       p + "mlp.shared_experts.down_proj.weight": r(d.hidden, Is)})
    return sd


def _write_sharded(sd, path, n_shards=2):
    from safetensors.torch import save_file

    os.makedirs(path, exist_ok=True)
    names = sorted(sd)
    wm = {}
    for k in range(n_shards):
        fn = f"model-{k + 1:05d}-of-{n_shards:05d}.safetensors"
        part = {n: sd[n].contiguous() for n in names[k::n_shards]}
        save_file(part, os.path.join(path, fn), metadata={"format": "pt"})
        wm.update({n: fn for n in part})
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wm}, f)


def test_safetensors_parser_matches_the_package(tmp_path):
    from safetensors import safe_open

    from dsv2lite.checkpoint import Checkpoint, SafetensorsFile

    sd = _tiny_state()
    sd["extra.f32"] = torch.randn(3, 5)
    sd["extra.i64"] = torch.arange(7)
    sd["extra.empty"] = torch.zeros(0, 4, dtype=torch.bfloat16)
    _write_sharded(sd, str(tmp_path), 3)
    ck = Checkpoint(str(tmp_path))
    assert set(ck.where) == set(sd)
    for fn, sf in ck.files.items():
        assert sf.metadata == {"format": "pt"}
        with safe_open(os.path.join(tmp_path, fn), framework="pt") as ref:
            assert sorted(sf.keys()) == sorted(ref.keys())
            for k in ref.keys():
                a, b = sf.get(k), ref.get_tensor(k)
                assert a.dtype == b.dtype and a.shape == b.shape, k
                assert torch.equal(a.view(torch.uint8) if a.numel() else a, b.view(torch.uint8) if b.numel() else b), k
    for k, t in sd.items():
        assert torch.equal(ck.get(k), t), k
    ck.close()
    # a corrupted header length is refused
    bad = tmp_path / "bad"
    bad.mkdir()
    (bad / "x.safetensors").write_bytes((10**9).to_bytes(8, "little") + b"{}")
    with pytest.raises(ValueError, match="header length"):
        SafetensorsFile(str(bad / "x.safetensors"))


def test_hf_keys_map_onto_the_packed_layouts(tmp_path):
    from dsv2lite.checkpoint import Checkpoint, hf_layer_tensors
    from dsv2lite.config import DSV2Config

    d = TINY_DIMS
    sd = _tiny_state(1)
    _write_sharded(sd, str(tmp_path), 2)
    cfg = DSV2Config(hidden=d.hidden, n_heads=d.n_heads, qk_nope=d.qk_nope, qk_rope=d.qk_rope, v_dim=d.v_dim,
                     kv_rank=d.kv_rank, n_experts=d.n_experts, top_k=d.top_k, moe_inter=d.moe_inter,
                     n_shared=d.n_shared, dense_inter=d.dense_inter, vocab=d.vocab, n_layers=d.n_layers,
                     first_dense=d.first_dense)
    ck = Checkpoint(str(tmp_path))
    I = d.moe_inter
    for i in range(d.n_layers):
        t = hf_layer_tensors(ck, cfg, i)
        p = f"model.layers.{i}."
        assert torch.equal(t["q_proj"], sd[p + "self_attn.q_proj.weight"])
        assert torch.equal(t["kv_b_proj"], sd[p + "self_attn.kv_b_proj.weight"])
        if i < d.first_dense:
            assert torch.equal(t["down_proj"], sd[p + "mlp.down_proj.weight"])
            continue
        for e in range(d.n_experts):
            q = f"{p}mlp.experts.{e}."
            assert torch.equal(t["experts_gate_up"][e, :I], sd[q + "gate_proj.weight"])  # [gate; up]
            assert torch.equal(t["experts_gate_up"][e, I:], sd[q + "up_proj.weight"])
            assert torch.equal(t["experts_down"][e], sd[q + "down_proj.weight"])
        assert torch.equal(t["sh_up"], sd[p + "mlp.shared_experts.up_proj.weight"])
        assert torch.equal(t["gate"], sd[p + "mlp.gate.weight"])
    ck.close()
    # transformers' fused expert layout is read as-is
    sd2 = {k: v for k, v in sd.items() if ".experts." not in k}
    p = "model.layers.1."
    sd2[p + "mlp.experts.gate_up_proj"] = torch.stack(
        [torch.cat([sd[f"{p}mlp.experts.{e}.gate_proj.weight"], sd[f"{p}mlp.experts.{e}.up_proj.weight"]])
         for e in range(d.n_experts)])
    sd2[p + "mlp.experts.down_proj"] = torch.stack([sd[f"{p}mlp.experts.{e}.down_proj.weight"]
                                                    for e in range(d.n_experts)])
    for i in range(2, d.n_layers):
        q = f"model.layers.{i}."
        sd2[q + "mlp.experts.gate_up_proj"] = torch.zeros(d.n_experts, 2 * I, d.hidden, dtype=torch.bfloat16)
        sd2[q + "mlp.experts.down_proj"] = torch.zeros(d.n_experts, d.hidden, I, dtype=torch.bfloat16)
    _write_sharded(sd2, str(tmp_path / "native"), 1)
    ck2 = Checkpoint(str(tmp_path / "native"))
    assert torch.equal(hf_layer_tensors(ck2, cfg, 1)["experts_gate_up"], sd2[p + "mlp.experts.gate_up_proj"])
    ck2.close()


def test_config_json_gives_the_lite_dims(tmp_path):
    from dsv2lite.checkpoint import config_from_hf
    from dsv2lite.config import DSV2Config

    (tmp_path / "config.json").write_text(json.dumps(LITE_CONFIG))
    cfg = config_from_hf(str(tmp_path))
    assert cfg == DSV2Config()
    cfg.check_kernel_dims()
    assert abs(cfg.softmax_scale - 0.1147223) < 1e-6
    (tmp_path / "config.json").write_text(json.dumps(dict(LITE_CONFIG, q_lora_rank=1536)))
    with pytest.raises(NotImplementedError, match="q_lora_rank"):
        config_from_hf(str(tmp_path))
    (tmp_path / "config.json").write_text(json.dumps(dict(LITE_CONFIG, norm_topk_prob=True)))
    with pytest.raises(NotImplementedError, match="renormalisation"):
        config_from_hf(str(tmp_path))


def _save_tokenizer(path, chat_template=None):
    from tokenizers import Tokenizer, models, pre_tokenizers, trainers

    tok = Tokenizer(models.BPE(unk_token="<unk>"))
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    trainer = trainers.BpeTrainer(vocab_size=400, special_tokens=["<bos>", "<eos>", "<unk>"],
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet())
    corpus = ["User: Write me a 500 word novel.", "Assistant: Once upon a time", "hello world\n\n"] * 20
    tok.train_from_iterator(corpus, trainer)
    os.makedirs(path, exist_ok=True)
    tok.save(os.path.join(path, "tokenizer.json"))
    cfg = {"tokenizer_class": "LlamaTokenizerFast", "bos_token": {"content": "<bos>", "lstrip": False},
           "eos_token": "<eos>", "unk_token": "<unk>", "add_bos_token": False}
    if chat_template:
        cfg["chat_template"] = chat_template
    with open(os.path.join(path, "tokenizer_config.json"), "w") as f:
        json.dump(cfg, f)


def test_chat_template_prompt_ids(tmp_path):
    """--prompt through the chat template with the generation prompt (run.py:731-735): the
    DeepSeek-V2-Chat template when the tokenizer has none, its own otherwise."""
    from dsv2lite.checkpoint import chat_prompt_ids, load_tokenizer

    _save_tokenizer(str(tmp_path / "a"))
    tok = load_tokenizer(str(tmp_path / "a"))
    text = tok.apply_chat_template([{"role": "user", "content": "Write me a 500 word novel."}],
                                   add_generation_prompt=True, tokenize=False)
    assert text == "<bos>User: Write me a 500 word novel.\n\nAssistant:"
    ids = chat_prompt_ids(tok, "Write me a 500 word novel.")
    assert ids.dtype == torch.int64 and ids.ndim == 1
    assert ids.tolist() == tok(text, add_special_tokens=False)["input_ids"]
    assert ids[0].item() == tok.convert_tokens_to_ids("<bos>")
    assert tok.pad_token_id == tok.eos_token_id  # run.py:728-729
    _save_tokenizer(str(tmp_path / "b"), chat_template="{{ bos_token }}[{{ messages[0]['content'] }}]")
    tok2 = load_tokenizer(str(tmp_path / "b"))
    assert tok2.apply_chat_template([{"role": "user", "content": "hi"}], tokenize=False) == "<bos>[hi]"
