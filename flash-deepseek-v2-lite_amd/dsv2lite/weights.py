"""Seeded random-init DeepSeek-V2-Lite weights, generated straight into the
device layouts the HIP kernels read.

Generation order (one torch.Generator on the target device, N(0, std) in fp32
rounded to bf16; RMSNorm weights = 1): embed_tokens, then per layer q_proj,
kv_a_proj_with_mqa, kv_b_proj, o_proj and either gate_proj, up_proj, down_proj
(dense layer 0) or router gate, experts gate_up [E, 2I, H], experts down
[E, H, I], shared gate_proj, up_proj, down_proj; lm_head last.

Packed layouts (HBM):
  w_qkva [3648, 2048]   = cat(q_proj, kv_a_proj_with_mqa)          (attention_decode_batch.py:214-237)
  w_uk  [16, 128, 512]  = kv_b rows h*256 + [0,128)   (k_nope part)
  w_ukt [16, 512, 128]  = w_uk transposed (A operand of the grouped absorption GEMM)
  w_uv  [16, 128, 512]  = kv_b rows h*256 + [128,256) (value part)
  w_gu  [E, 2I, H]      = per expert [gate; up]                    (moe_batch.py:341-354)
  w_down[E, H, I]
  sh_gu [2*2816, 2048]  = cat(shared gate_proj, shared up_proj); sh_down [2048, 2816]
  dense w_gu [2*10944, 2048], w_down [2048, 10944]

FP8 expert weights (quantize_experts_fp8): the same four MoE layouts in OCP e4m3 bytes
(w_gu8, w_down8, sh_gu8, sh_down8) with one fp32 power-of-two scale per output row
(gu_scale [E, 2I], down_scale [E, H], sh_gu_scale [2*2816], sh_down_scale [2048]).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .config import DSV2Config

BF16 = torch.bfloat16


@dataclass
class LayerWeights:
    ln_in: torch.Tensor
    ln_post: torch.Tensor
    w_qkva: torch.Tensor
    kv_norm: torch.Tensor
    w_uk: torch.Tensor
    w_ukt: torch.Tensor
    w_uv: torch.Tensor
    w_o: torch.Tensor
    moe: bool
    w_gu: torch.Tensor
    w_down: torch.Tensor
    w_router: torch.Tensor | None = None
    sh_gu: torch.Tensor | None = None
    sh_down: torch.Tensor | None = None
    # fp8 (e4m3) copies of the MoE weights and their per-row scales, set by quantize_experts_fp8
    w_gu8: torch.Tensor | None = None
    gu_scale: torch.Tensor | None = None
    w_down8: torch.Tensor | None = None
    down_scale: torch.Tensor | None = None
    sh_gu8: torch.Tensor | None = None
    sh_gu_scale: torch.Tensor | None = None
    sh_down8: torch.Tensor | None = None
    sh_down_scale: torch.Tensor | None = None


@dataclass
class ModelWeights:
    cfg: DSV2Config
    embed: torch.Tensor
    norm: torch.Tensor
    lm_head: torch.Tensor
    layers: list[LayerWeights] = field(default_factory=list)
    fp8_experts: bool = False  # quantize_experts_fp8 has run

    def hf_layer(self, i: int) -> dict:
        """HF-named views of layer i (shared storage; kv_b rebuilt) for checkers."""
        c, L = self.cfg, self.layers[i]
        nq = c.n_heads * c.q_head
        kv_b = torch.cat((L.w_uk, L.w_uv), dim=1).reshape(c.n_heads * (c.qk_nope + c.v_dim), c.kv_rank)
        d = {
            "q_proj": L.w_qkva[:nq], "kv_a_proj_with_mqa": L.w_qkva[nq:], "kv_a_layernorm": L.kv_norm,
            "kv_b_proj": kv_b, "o_proj": L.w_o, "input_layernorm": L.ln_in,
            "post_attention_layernorm": L.ln_post,
        }
        if L.moe:
            Is = c.shared_inter
            d.update(gate=L.w_router, experts_gate_up=L.w_gu, experts_down=L.w_down, sh_gate=L.sh_gu[:Is],
                     sh_up=L.sh_gu[Is:], sh_down=L.sh_down)
        else:
            d.update(gate_proj=L.w_gu[: c.dense_inter], up_proj=L.w_gu[c.dense_inter:], down_proj=L.w_down)
        return d

    def nbytes(self) -> int:
        tot = self.embed.nbytes + self.norm.nbytes + self.lm_head.nbytes
        for L in self.layers:
            for t in (L.ln_in, L.ln_post, L.w_qkva, L.kv_norm, L.w_uk, L.w_uv, L.w_o, L.w_gu, L.w_down,
                      L.w_router, L.sh_gu, L.sh_down):
                if t is not None:
                    tot += t.nbytes
        return tot


class _Rng:
    def __init__(self, device, seed: int, std: float):
        self.g = torch.Generator(device=device)
        self.g.manual_seed(seed)
        self.device = device
        self.std = std

    def fill_(self, out: torch.Tensor) -> torch.Tensor:
        tmp = torch.randn(out.shape, generator=self.g, device=self.device, dtype=torch.float32)
        out.copy_(tmp.mul_(self.std))
        return out

    def new(self, *shape) -> torch.Tensor:
        return self.fill_(torch.empty(*shape, dtype=BF16, device=self.device))


def init_weights(cfg: DSV2Config, device="cuda", seed: int = 0, std: float = 0.02) -> ModelWeights:
    """Random-init DeepSeek-V2-Lite weights in packed device layouts."""
    r = _Rng(device, seed, std)
    H, nh = cfg.hidden, cfg.n_heads
    ones = lambda n: torch.ones(n, dtype=BF16, device=device)  # noqa: E731
    embed = r.new(cfg.vocab, H)
    layers = []
    nq = nh * cfg.q_head
    for i in range(cfg.n_layers):
        w_qkva = torch.empty(cfg.qkva_dim, H, dtype=BF16, device=device)
        r.fill_(w_qkva[:nq])
        r.fill_(w_qkva[nq:])
        kv_b = r.new(nh, cfg.qk_nope + cfg.v_dim, cfg.kv_rank)
        w_uk = kv_b[:, : cfg.qk_nope].contiguous()
        w_uv = kv_b[:, cfg.qk_nope:].contiguous()
        del kv_b
        w_o = r.new(H, nh * cfg.v_dim)
        if cfg.is_moe_layer(i):
            w_router = r.new(cfg.n_experts, H)
            w_gu = r.new(cfg.n_experts, 2 * cfg.moe_inter, H)
            w_down = r.new(cfg.n_experts, H, cfg.moe_inter)
            sh_gu = torch.empty(2 * cfg.shared_inter, H, dtype=BF16, device=device)
            r.fill_(sh_gu[: cfg.shared_inter])
            r.fill_(sh_gu[cfg.shared_inter:])
            sh_down = r.new(H, cfg.shared_inter)
            layers.append(LayerWeights(ones(H), ones(H), w_qkva, ones(cfg.kv_rank), w_uk,
                                       w_uk.transpose(1, 2).contiguous(), w_uv, w_o, True, w_gu, w_down, w_router,
                                       sh_gu, sh_down))
        else:
            w_gu = torch.empty(2 * cfg.dense_inter, H, dtype=BF16, device=device)
            r.fill_(w_gu[: cfg.dense_inter])
            r.fill_(w_gu[cfg.dense_inter:])
            w_down = r.new(H, cfg.dense_inter)
            layers.append(LayerWeights(ones(H), ones(H), w_qkva, ones(cfg.kv_rank), w_uk,
                                       w_uk.transpose(1, 2).contiguous(), w_uv, w_o, False, w_gu, w_down))
    lm_head = r.new(cfg.vocab, H)
    return ModelWeights(cfg, embed, ones(H), lm_head, layers)


def pack_hf_layer(cfg: DSV2Config, hf: dict, device="cuda") -> LayerWeights:
    """Pack one layer given HF-named tensors (e.g. from a checkpoint or a test)."""
    def t(x):
        return x.to(device=device, dtype=BF16).contiguous()

    nh = cfg.n_heads
    kv_b = t(hf["kv_b_proj"]).view(nh, cfg.qk_nope + cfg.v_dim, cfg.kv_rank)
    w_uk = kv_b[:, : cfg.qk_nope].contiguous()
    common = dict(ln_in=t(hf["input_layernorm"]), ln_post=t(hf["post_attention_layernorm"]),
                  w_qkva=torch.cat((t(hf["q_proj"]), t(hf["kv_a_proj_with_mqa"]))), kv_norm=t(hf["kv_a_layernorm"]),
                  w_uk=w_uk, w_ukt=w_uk.transpose(1, 2).contiguous(), w_uv=kv_b[:, cfg.qk_nope:].contiguous(),
                  w_o=t(hf["o_proj"]))
    if "gate" in hf:
        return LayerWeights(**common, moe=True, w_gu=t(hf["experts_gate_up"]), w_down=t(hf["experts_down"]),
                            w_router=t(hf["gate"]), sh_gu=torch.cat((t(hf["sh_gate"]), t(hf["sh_up"]))),
                            sh_down=t(hf["sh_down"]))
    return LayerWeights(**common, moe=False, w_gu=torch.cat((t(hf["gate_proj"]), t(hf["up_proj"]))),
                        w_down=t(hf["down_proj"]))


E4M3_MAX = 448.0  # largest finite OCP e4m3 (float8_e4m3fn) value


def fp8_row_scales(w: torch.Tensor) -> torch.Tensor:
    """Per-row power-of-two scales s (fp32, shape w.shape[:-1]) with max|w| / s <= 448: the
    smallest such power of two, 1 for an all-zero row.  A power of two keeps w / s exact and
    makes e4m3 * s exactly a bf16 value."""
    amax = w.abs().amax(dim=-1).float()
    m, e = torch.frexp(amax / E4M3_MAX)  # amax / 448 = m * 2**e, m in [0.5, 1)
    e = torch.where(m == 0.5, e - 1, e)  # an exact power of two needs no step up
    s = torch.ldexp(torch.ones_like(amax), e)
    return torch.where(amax > 0, s, torch.ones_like(amax))


def quantize_rows_fp8(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(e4m3 bytes as uint8, fp32 row scales) of a bf16 matrix stack [..., K]: each weight
    rounded to the nearest e4m3 value of w / s (ties to even), s from fp8_row_scales."""
    s = fp8_row_scales(w)
    q = (w.float() / s.unsqueeze(-1)).to(torch.float8_e4m3fn)
    return q.view(torch.uint8), s


def dequantize_rows_fp8(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """bf16 value of every e4m3 weight times its row scale (exact: 4 significant bits)."""
    return (q.view(torch.float8_e4m3fn).float() * s.unsqueeze(-1)).to(BF16)


def quantize_experts_fp8(w: ModelWeights) -> ModelWeights:
    """Quantize every MoE layer's routed and shared expert weights to e4m3 with per-row
    power-of-two scales (in place).  The bf16 tensors are overwritten with the dequantized
    values, so the bf16 kernels (prefill, batch family) and any checker see exactly the
    weights the fp8 kernels read.  Returns w."""
    if w.fp8_experts:
        return w
    for L in w.layers:
        if not L.moe:
            continue
        E = L.w_gu.shape[0]
        L.w_gu8 = torch.empty(L.w_gu.shape, dtype=torch.uint8, device=L.w_gu.device)
        L.w_down8 = torch.empty(L.w_down.shape, dtype=torch.uint8, device=L.w_down.device)
        L.gu_scale = torch.empty(L.w_gu.shape[:2], dtype=torch.float32, device=L.w_gu.device)
        L.down_scale = torch.empty(L.w_down.shape[:2], dtype=torch.float32, device=L.w_down.device)
        for e in range(E):  # one expert at a time keeps the fp32 temporaries small
            for src, q8, sc in ((L.w_gu, L.w_gu8, L.gu_scale), (L.w_down, L.w_down8, L.down_scale)):
                q, s = quantize_rows_fp8(src[e])
                q8[e].copy_(q)
                sc[e].copy_(s)
                src[e].copy_(dequantize_rows_fp8(q, s))
        L.sh_gu8, L.sh_gu_scale = quantize_rows_fp8(L.sh_gu)
        L.sh_gu.copy_(dequantize_rows_fp8(L.sh_gu8, L.sh_gu_scale))
        L.sh_down8, L.sh_down_scale = quantize_rows_fp8(L.sh_down)
        L.sh_down.copy_(dequantize_rows_fp8(L.sh_down8, L.sh_down_scale))
    w.fp8_experts = True
    return w
