"""Local DeepSeek-V2-Lite checkpoint loading: safetensors shards -> the packed device layouts
of ``weights.py``, config.json -> ``DSV2Config``, and the checkpoint's tokenizer with its chat
template (reference: src/run.py:14, 299-313, 719-737; packing as in moe_batch.py:324-363 and
attention_decode_batch.py:214-237).

safetensors is parsed directly: an 8-byte little-endian header length, a JSON header mapping
each tensor name to {dtype, shape, data_offsets [begin, end)} relative to the end of the
header, then the raw little-endian tensor bytes.  Files are memory-mapped; a tensor is viewed
in place (torch.frombuffer) and copied once, to the device, when it is packed, so host memory
stays at one tensor at a time.  The shard index ``model.safetensors.index.json`` (weight_map:
name -> file) is used when present, else every ``*.safetensors`` file of the directory.

HF key names (remote-code DeepseekV2ForCausalLM, the format of the published checkpoint):
``model.embed_tokens.weight``, ``model.norm.weight``, ``lm_head.weight`` and per layer i under
``model.layers.{i}.``: ``input_layernorm.weight``, ``post_attention_layernorm.weight``,
``self_attn.{q_proj,kv_a_proj_with_mqa,kv_b_proj,o_proj}.weight``,
``self_attn.kv_a_layernorm.weight``, then ``mlp.{gate,up,down}_proj.weight`` (dense layers) or
``mlp.gate.weight``, ``mlp.experts.{e}.{gate,up,down}_proj.weight`` and
``mlp.shared_experts.{gate,up,down}_proj.weight`` (MoE layers).  transformers' native layout
with fused experts (``mlp.experts.gate_up_proj`` [E, 2I, H], ``mlp.experts.down_proj``
[E, H, I]) is accepted too.
"""

from __future__ import annotations

import dataclasses
import json
import mmap
import os
import struct
import warnings

import torch

from .config import DSV2Config
from .weights import ModelWeights, pack_hf_layer

_DTYPES = {"BF16": torch.bfloat16, "F16": torch.float16, "F32": torch.float32, "F64": torch.float64,
           "I64": torch.int64, "I32": torch.int32, "I16": torch.int16, "I8": torch.int8, "U8": torch.uint8,
           "BOOL": torch.bool}

# The published DeepSeek-V2(-Lite)-Chat template (tokenizer_config.json "chat_template"), used
# only when a checkpoint's tokenizer carries none.
DEEPSEEK_V2_CHAT_TEMPLATE = (
    "{% if not add_generation_prompt is defined %}{% set add_generation_prompt = false %}{% endif %}"
    "{{ bos_token }}{% for message in messages %}"
    "{% if message['role'] == 'user' %}{{ 'User: ' + message['content'] + '\n\n' }}"
    "{% elif message['role'] == 'assistant' %}{{ 'Assistant: ' + message['content'] + eos_token }}"
    "{% elif message['role'] == 'system' %}{{ message['content'] + '\n\n' }}{% endif %}{% endfor %}"
    "{% if add_generation_prompt %}{{ 'Assistant:' }}{% endif %}")


class SafetensorsFile:
    """One memory-mapped .safetensors file."""

    def __init__(self, path: str):
        self.path = path
        self._f = open(path, "rb")
        head = self._f.read(8)
        if len(head) != 8:
            raise ValueError(f"{path}: not a safetensors file (shorter than 8 bytes)")
        (n,) = struct.unpack("<Q", head)
        size = os.fstat(self._f.fileno()).st_size
        if n > size - 8:
            raise ValueError(f"{path}: header length {n} exceeds the file")
        self.header = json.loads(self._f.read(n).decode("utf-8"))
        self.metadata = self.header.pop("__metadata__", None)
        self._base = 8 + n
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ) if size > 0 else None
        for name, e in self.header.items():
            b, en = e["data_offsets"]
            dt = _DTYPES.get(e["dtype"])
            if dt is None:
                raise ValueError(f"{path}: tensor {name} has unsupported dtype {e['dtype']}")
            numel = 1
            for d in e["shape"]:
                numel *= int(d)
            if en - b != numel * torch.empty(0, dtype=dt).element_size() or self._base + en > size or b > en:
                raise ValueError(f"{path}: tensor {name} has inconsistent offsets {e['data_offsets']}")

    def keys(self) -> list[str]:
        return list(self.header)

    def get(self, name: str) -> torch.Tensor:
        """The tensor viewed in place (read-only memory map; copy before writing)."""
        e = self.header[name]
        dt = _DTYPES[e["dtype"]]
        b, en = e["data_offsets"]
        shape = [int(d) for d in e["shape"]]
        if en == b:
            return torch.empty(shape, dtype=dt)
        with warnings.catch_warnings():  # the map is read-only; callers copy what they keep
            warnings.simplefilter("ignore", UserWarning)
            t = torch.frombuffer(memoryview(self._mm)[self._base + b:self._base + en], dtype=dt)
        return t.view(shape)

    def close(self) -> None:
        """Release the file; a map that tensors still view stays open until they are freed."""
        if self._mm is not None:
            try:
                self._mm.close()
            except BufferError:  # views handed out by get() are alive
                pass
            self._mm = None
        self._f.close()


class Checkpoint:
    """All tensors of a checkpoint directory, by name."""

    def __init__(self, path: str):
        self.path = path
        index = os.path.join(path, "model.safetensors.index.json")
        self.files: dict[str, SafetensorsFile] = {}
        self.where: dict[str, str] = {}
        if os.path.exists(index):
            with open(index) as f:
                wm = json.load(f)["weight_map"]
            for name, fn in wm.items():
                self.where[name] = fn
            names = sorted(set(wm.values()))
        else:
            names = sorted(fn for fn in os.listdir(path) if fn.endswith(".safetensors"))
        if not names:
            raise FileNotFoundError(f"no .safetensors files in {path}")
        for fn in names:
            sf = SafetensorsFile(os.path.join(path, fn))
            self.files[fn] = sf
            for k in sf.keys():
                if k in self.where and self.where[k] != fn:
                    continue  # the index decides
                self.where.setdefault(k, fn)
        missing = [k for k, fn in self.where.items() if k not in self.files[fn].header]
        if missing:
            raise ValueError(f"index names tensors its shard does not hold: {missing[:4]}")

    def __contains__(self, name: str) -> bool:
        return name in self.where

    def get(self, name: str) -> torch.Tensor:
        if name not in self.where:
            raise KeyError(f"{name} not in checkpoint {self.path}")
        return self.files[self.where[name]].get(name)

    def close(self) -> None:
        for f in self.files.values():
            f.close()


def config_from_hf(path: str) -> DSV2Config:
    """DSV2Config from the checkpoint's config.json (DeepseekV2Config field names)."""
    with open(os.path.join(path, "config.json")) as f:
        c = json.load(f)
    if c.get("q_lora_rank") is not None:
        raise NotImplementedError("q_lora_rank != null (DeepSeek-V2, not -Lite) is not supported")
    if c.get("scoring_func", "softmax") != "softmax" or c.get("topk_method", "greedy") != "greedy" \
            or c.get("norm_topk_prob", False):
        raise NotImplementedError("only softmax scoring, greedy top-k, no top-k renormalisation (DeepSeek-V2-Lite)")
    rs = c.get("rope_scaling") or {}
    if rs and rs.get("type", rs.get("rope_type")) != "yarn":
        raise NotImplementedError(f"rope_scaling {rs} is not YaRN")
    return DSV2Config(
        hidden=c["hidden_size"], n_heads=c["num_attention_heads"], qk_nope=c["qk_nope_head_dim"],
        qk_rope=c["qk_rope_head_dim"], v_dim=c["v_head_dim"], kv_rank=c["kv_lora_rank"],
        n_experts=c["n_routed_experts"], top_k=c["num_experts_per_tok"], moe_inter=c["moe_intermediate_size"],
        n_shared=c["n_shared_experts"], dense_inter=c["intermediate_size"], vocab=c["vocab_size"],
        n_layers=c["num_hidden_layers"], first_dense=c.get("first_k_dense_replace", 0), eps=c["rms_norm_eps"],
        rope_theta=c.get("rope_theta", 10000.0), yarn_factor=rs.get("factor", 1.0),
        yarn_orig_max_pos=rs.get("original_max_position_embeddings", 4096),
        yarn_beta_fast=rs.get("beta_fast", 32.0), yarn_beta_slow=rs.get("beta_slow", 1.0),
        yarn_mscale=rs.get("mscale", 1.0), yarn_mscale_all_dim=rs.get("mscale_all_dim", 0.0),
        routed_scaling=c.get("routed_scaling_factor", 1.0))


def hf_layer_tensors(ck: Checkpoint, cfg: DSV2Config, i: int) -> dict:
    """HF-named tensors of layer i in the layouts pack_hf_layer takes (views of the file;
    the experts are stacked into [E, 2I, H] = per expert [gate; up] and [E, H, I] on the host,
    one layer at a time)."""
    p = f"model.layers.{i}."
    d = {"q_proj": ck.get(p + "self_attn.q_proj.weight"),
         "kv_a_proj_with_mqa": ck.get(p + "self_attn.kv_a_proj_with_mqa.weight"),
         "kv_a_layernorm": ck.get(p + "self_attn.kv_a_layernorm.weight"),
         "kv_b_proj": ck.get(p + "self_attn.kv_b_proj.weight"), "o_proj": ck.get(p + "self_attn.o_proj.weight"),
         "input_layernorm": ck.get(p + "input_layernorm.weight"),
         "post_attention_layernorm": ck.get(p + "post_attention_layernorm.weight")}
    if not cfg.is_moe_layer(i):
        d.update(gate_proj=ck.get(p + "mlp.gate_proj.weight"), up_proj=ck.get(p + "mlp.up_proj.weight"),
                 down_proj=ck.get(p + "mlp.down_proj.weight"))
        return d
    d["gate"] = ck.get(p + "mlp.gate.weight")
    if p + "mlp.experts.gate_up_proj" in ck:
        d["experts_gate_up"] = ck.get(p + "mlp.experts.gate_up_proj")
        d["experts_down"] = ck.get(p + "mlp.experts.down_proj")
    else:
        E, I, H = cfg.n_experts, cfg.moe_inter, cfg.hidden
        gu = torch.empty(E, 2 * I, H, dtype=torch.bfloat16)
        dn = torch.empty(E, H, I, dtype=torch.bfloat16)
        for e in range(E):
            q = f"{p}mlp.experts.{e}."
            gu[e, :I].copy_(ck.get(q + "gate_proj.weight"))
            gu[e, I:].copy_(ck.get(q + "up_proj.weight"))
            dn[e].copy_(ck.get(q + "down_proj.weight"))
        d["experts_gate_up"], d["experts_down"] = gu, dn
    q = p + "mlp.shared_experts."
    d.update(sh_gate=ck.get(q + "gate_proj.weight"), sh_up=ck.get(q + "up_proj.weight"),
             sh_down=ck.get(q + "down_proj.weight"))
    return d


def load_weights(path: str, device="cuda", n_layers: int | None = None) -> ModelWeights:
    """Packed device weights of a local checkpoint directory (config.json + safetensors).
    n_layers < the checkpoint's keeps the first layers only (tests)."""
    cfg = config_from_hf(path)
    if n_layers is not None:
        cfg = dataclasses.replace(cfg, n_layers=n_layers)
    cfg.check_kernel_dims()
    ck = Checkpoint(path)
    try:
        bf = lambda t: t.to(device=device, dtype=torch.bfloat16).contiguous()  # noqa: E731
        layers = [pack_hf_layer(cfg, hf_layer_tensors(ck, cfg, i), device=device) for i in range(cfg.n_layers)]
        embed = bf(ck.get("model.embed_tokens.weight"))
        head = bf(ck.get("lm_head.weight")) if "lm_head.weight" in ck else embed  # tied embeddings
        w = ModelWeights(cfg, embed, bf(ck.get("model.norm.weight")), head, layers)
    finally:
        ck.close()
    for name, t, shape in (("embed_tokens", w.embed, (cfg.vocab, cfg.hidden)),
                           ("lm_head", w.lm_head, (cfg.vocab, cfg.hidden))):
        if tuple(t.shape) != shape:
            raise ValueError(f"{name} has shape {tuple(t.shape)}, config says {shape}")
    return w


def load_tokenizer(path: str):
    """The checkpoint's fast tokenizer: tokenizer.json plus the special tokens and chat
    template of tokenizer_config.json (transformers.PreTrainedTokenizerFast; no remote code,
    no network, and no dependence on the model's config.json).  A tokenizer without a chat
    template gets DeepSeek-V2-Chat's."""
    from transformers import PreTrainedTokenizerFast

    tc = {}
    cfg_path = os.path.join(path, "tokenizer_config.json")
    if os.path.exists(cfg_path):
        with open(cfg_path) as f:
            tc = json.load(f)

    def tok_str(v):
        return v.get("content") if isinstance(v, dict) else v

    special = {k: tok_str(tc[k]) for k in ("bos_token", "eos_token", "unk_token", "pad_token") if tc.get(k)}
    tok = PreTrainedTokenizerFast(tokenizer_file=os.path.join(path, "tokenizer.json"), **special)
    tok.chat_template = tc.get("chat_template") or DEEPSEEK_V2_CHAT_TEMPLATE
    if tok.pad_token_id is None:  # src/run.py:728-729
        tok.pad_token = tok.eos_token
    return tok


def chat_prompt_ids(tok, prompt: str) -> torch.Tensor:
    """The user prompt through the chat template with the generation prompt appended, as
    src/run.py:731-735: int64 [n]."""
    ids = tok.apply_chat_template([{"role": "user", "content": prompt}], add_generation_prompt=True,
                                  return_tensors="pt")
    if isinstance(ids, dict) or hasattr(ids, "input_ids"):
        ids = ids["input_ids"]
    return torch.as_tensor(ids).reshape(-1).to(torch.int64)
