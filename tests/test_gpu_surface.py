"""The drop-in Python surface on the GPU: every ``triton_kernels`` function the reference's
src/run.py imports (run.py:26-50), plus batched_attention_decode_q1_triton and
packed_routed_moe_eager, called on GPU tensors exactly as the reference's patches call them,
against the CPU oracle or a plain fp32 torch reference on the same inputs.  Also the
scalar-position entry points (dsv2_fill_positions, dsv2_prepare_decode_inputs,
dsv2_copy_token_rows, bit-exact) and the per-row cache capacity guard of the MLA kernels.

Bars: bit-exact for integer work, copies and the residual add; router ids exact where the
top-6 margin exceeds 1e-3; bf16 outputs within max-rel 2e-2 of the oracle (the north-star
bar) -- the kernel-level tests in test_gpu_kernels.py hold the same kernels to 1e-2 vs fp32.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from triton_kernels import _hip
    from triton_kernels._hip import call

import oracle.dsv2_oracle as O
from golden_utils import rel_err

DEV = "cuda"
BF = torch.bfloat16


def st():
    return _hip.stream_ptr()


def rnd(*shape, std=1.0, seed=0, dtype=BF):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=DEV) * std).to(dtype)


def rb(t):
    return t.to(BF).float()


c = lambda t: t.float().cpu()  # noqa: E731


# --------------------------------------------------------------------------- A2 / positions
def test_fill_positions_per_row_arrays():
    cp = torch.tensor([37], dtype=torch.int64, device=DEV)
    B, L = 5, 300
    pos = torch.full((B,), -7, dtype=torch.int32, device=DEV)
    base = torch.full((B,), -7, dtype=torch.int64, device=DEV)
    cap = torch.full((B,), -7, dtype=torch.int32, device=DEV)
    call("dsv2_fill_positions", cp.data_ptr(), pos.data_ptr(), base.data_ptr(), cap.data_ptr(), L, B, st())
    assert pos.tolist() == [37] * B
    assert base.tolist() == [b * L for b in range(B)]
    assert cap.tolist() == [L] * B
    with pytest.raises(_hip.HipKernelError, match="capacity"):
        call("dsv2_fill_positions", cp.data_ptr(), pos.data_ptr(), None, None, 0, B, st())


@pytest.mark.parametrize("pos,permute", [(0, False), (17, False), (255, False), (40, True)])
def test_prepare_decode_inputs_triton_bit_exact(pos, permute):
    """mask[b, j] = index[j] <= pos and position_ids[b] = pos, int64, in place
    (attention_prepost.py:9-36, 152-188)."""
    from triton_kernels.attention_prepost import prepare_decode_inputs_triton

    B, L = 3, 256
    idx = torch.arange(L, device=DEV)
    if permute:
        idx = idx[torch.randperm(L, generator=torch.Generator().manual_seed(5)).to(DEV)]
    mask = torch.full((B, L), 9, dtype=torch.long, device=DEV)
    pid = torch.full((B, 1), 9, dtype=torch.long, device=DEV)
    cp = torch.tensor([pos], dtype=torch.long, device=DEV)
    prepare_decode_inputs_triton(cp, mask, pid, idx)
    ref = (idx[None, :] <= pos).long().expand(B, L)
    assert torch.equal(mask, ref)
    assert torch.equal(pid, torch.full((B, 1), pos, dtype=torch.long, device=DEV))


def test_copy_single_token_to_cache_bit_exact_and_bounded():
    from triton_kernels.attention_prepost import check_cache_write_status, copy_single_token_to_cache

    B, H, S, D = 3, 16, 40, 192
    src = rnd(B, H, 1, D, seed=1)
    dst = rnd(B, H, S, D, seed=2)
    ref = dst.clone()
    cp = torch.tensor([13], dtype=torch.long, device=DEV)
    copy_single_token_to_cache(src, dst, cp)
    ref[:, :, 13] = src[:, :, 0]
    assert torch.equal(dst, ref)
    check_cache_write_status(DEV)  # nothing flagged
    # compressed layout [B, 1, 576] -> [B, S, 576]
    s2 = rnd(B, 1, 576, seed=3)
    d2 = rnd(B, S, 576, seed=4)
    r2 = d2.clone()
    copy_single_token_to_cache(s2, d2, torch.tensor([S - 1], dtype=torch.long, device=DEV))
    r2[:, S - 1] = s2[:, 0]
    assert torch.equal(d2, r2)
    # past the sequence: nothing written, the status reports it
    before = d2.clone()
    copy_single_token_to_cache(s2, d2, torch.tensor([S], dtype=torch.long, device=DEV))
    assert torch.equal(d2, before)
    with pytest.raises(RuntimeError, match="outside the cache"):
        check_cache_write_status(DEV)
    check_cache_write_status(DEV)  # cleared


# --------------------------------------------------------------------------- elementwise
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_residual_add_triton_bit_exact(dtype):
    from triton_kernels.attention_prepost import residual_add_triton

    a = rnd(4, 1, 2048, seed=5, dtype=dtype)
    b = rnd(4, 1, 2048, seed=6, dtype=dtype)
    out = residual_add_triton(a, b)
    assert out.shape == a.shape and out.dtype == dtype
    assert torch.equal(out, (a.float() + b.float()).to(dtype))


def test_silu_mul_and_rmsnorm_triton():
    from triton_kernels.mlp_elementwise import silu_mul_triton
    from triton_kernels.rmsnorm import rmsnorm_triton

    g, u = rnd(3, 2816, seed=7), rnd(3, 2816, seed=8)
    y = silu_mul_triton(g, u)
    ref = torch.nn.functional.silu(c(g)) * c(u)
    assert rel_err(c(y), ref) < 8e-3
    x = rnd(2, 1, 2048, seed=9)
    w = (rnd(2048, seed=10, std=0.1) + 1).to(BF)
    yn = rmsnorm_triton(x, w, 1e-6)
    assert yn.shape == x.shape
    refn = O.rmsnorm(c(x), c(w), 1e-6, rb)
    assert rel_err(c(yn), refn) < 8e-3
    # the kv-norm width (512) as well
    x5 = rnd(3, 512, seed=11)
    w5 = (rnd(512, seed=12, std=0.1) + 1).to(BF)
    assert rel_err(c(rmsnorm_triton(x5, w5, 1e-6)), O.rmsnorm(c(x5), c(w5), 1e-6, rb)) < 8e-3


# --------------------------------------------------------------------------- router
@pytest.mark.parametrize("B", [1, 5])
def test_router_softmax_topk6_triton(B):
    from triton_kernels.moe_router import router_softmax_topk6_triton

    g = torch.Generator().manual_seed(20 + B)
    lg = torch.randn(B, 64, generator=g) * 2
    lg[0, 7] = lg[0, 3] = lg[0].max() + 1.0  # exact tie at the top: the lower index first
    ids, w = router_softmax_topk6_triton(lg.to(DEV), 1.0)
    assert ids.dtype == torch.long and ids.shape == (B, 6) and w.shape == (B, 6)
    sc = torch.softmax(lg, -1)
    for r in range(B):
        order = sorted(range(64), key=lambda e: (-float(sc[r, e]), e))[:6]
        assert ids[r].cpu().tolist() == order
        assert torch.allclose(w[r].cpu(), sc[r, order], rtol=1e-6, atol=1e-7)
    assert ids[0, 0].item() == 3 and ids[0, 1].item() == 7
    # routed_scaling_factor multiplies the weights
    _, w2 = router_softmax_topk6_triton(lg.to(DEV), 2.5)
    assert torch.allclose(w2, w * 2.5, rtol=1e-6)


# --------------------------------------------------------------------------- MoE
class _MLP(torch.nn.Module):
    def __init__(self, gate, up, down):
        super().__init__()
        self.gate_proj = torch.nn.Linear(gate.shape[1], gate.shape[0], bias=False, device=DEV, dtype=BF)
        self.up_proj = torch.nn.Linear(up.shape[1], up.shape[0], bias=False, device=DEV, dtype=BF)
        self.down_proj = torch.nn.Linear(down.shape[1], down.shape[0], bias=False, device=DEV, dtype=BF)
        with torch.no_grad():
            self.gate_proj.weight.copy_(gate)
            self.up_proj.weight.copy_(up)
            self.down_proj.weight.copy_(down)


class _Gate(torch.nn.Module):
    top_k = 6


class _RemoteMoE(torch.nn.Module):
    """HF remote-code DeepseekV2MoE attribute names: experts = ModuleList of MLPs."""

    def __init__(self, gu, dn):
        super().__init__()
        I = gu.shape[1] // 2
        self.experts = torch.nn.ModuleList([_MLP(gu[e, :I], gu[e, I:], dn[e]) for e in range(gu.shape[0])])
        self.gate = _Gate()
        self.num_experts_per_tok = 6
        self.ep_size = 1


class _NativeExperts(torch.nn.Module):
    def __init__(self, gu, dn):
        super().__init__()
        self.gate_up_proj = torch.nn.Parameter(gu.clone(), requires_grad=False)
        self.down_proj = torch.nn.Parameter(dn.clone(), requires_grad=False)


class _NativeMoE(torch.nn.Module):
    """transformers' native DeepseekV2Moe: experts.gate_up_proj [E, 2I, H], down_proj [E, H, I]."""

    def __init__(self, gu, dn):
        super().__init__()
        self.experts = _NativeExperts(gu, dn)
        self.gate = _Gate()
        self.num_experts_per_tok = 6


def _moe_weights(seed):
    return rnd(64, 2 * 1408, 2048, std=0.02, seed=seed), rnd(64, 2048, 1408, std=0.02, seed=seed + 1)


def _routed_ref(xn, ids, w, gu, dn):
    I = 1408
    outs = torch.zeros(xn.shape[0], 6, 2048)
    for t in range(xn.shape[0]):
        for s in range(6):
            e = int(ids[t, s])
            outs[t, s] = O.mlp(xn[t:t + 1], gu[e, :I], gu[e, I:], dn[e], rb)[0]
    routed = torch.zeros(xn.shape[0], 2048)
    for s in range(6):
        routed = routed + w[:, s:s + 1] * outs[:, s]
    return rb(routed)


def test_pack_routed_experts_both_layouts():
    from triton_kernels.moe_batch import pack_routed_experts

    gu, dn = _moe_weights(30)
    for mod in (_RemoteMoE(gu, dn), _NativeMoE(gu, dn)):
        p = pack_routed_experts(mod, device=DEV)
        assert (p.num_experts, p.hidden_size, p.intermediate_size, p.topk) == (64, 2048, 1408, 6)
        assert torch.equal(p.gate_up_weights, gu) and torch.equal(p.down_weights, dn)


@pytest.mark.parametrize("fn,B", [("grouped_routed_moe", 1), ("batched_grouped_routed_moe_route_gemv", 1),
                                  ("batched_grouped_routed_moe_route_gemv", 3), ("packed_routed_moe", 1),
                                  ("packed_routed_moe", 16), ("packed_routed_moe_eager", 5),
                                  ("batched_grouped_routed_moe", 64)])
def test_routed_moe_surface_vs_oracle(fn, B):
    import triton_kernels.moe_batch as MB
    import triton_kernels.moe_small_gemv as MS

    gu, dn = _moe_weights(40)
    packed = MB.pack_routed_experts(_NativeMoE(gu, dn), device=DEV)
    x = rnd(B, 2048, seed=41)
    g = torch.Generator().manual_seed(42 + B)
    ids = torch.stack([torch.randperm(64, generator=g)[:6] for _ in range(B)])
    w = torch.rand(B, 6, generator=g) * 0.3
    f = getattr(MS, fn, None) or getattr(MB, fn)
    args = (x, ids.to(DEV), w.to(DEV), packed)
    out = f(*args) if fn == "packed_routed_moe_eager" else f(*args, output_dtype=BF)
    assert out.shape == (B, 2048) and out.dtype == BF
    sel = list(range(min(B, 8)))
    ref = _routed_ref(c(x)[sel], ids[sel], w[sel], c(gu), c(dn))
    assert rel_err(c(out)[sel], ref) < 2e-2
    assert torch.equal(out, f(*args) if fn == "packed_routed_moe_eager" else f(*args, output_dtype=BF))


# --------------------------------------------------------------------------- attention
class _Lin(torch.nn.Module):
    def __init__(self, w):
        super().__init__()
        self.weight = torch.nn.Parameter(w, requires_grad=False)


class _Norm(torch.nn.Module):
    def __init__(self, w, eps):
        super().__init__()
        self.weight = torch.nn.Parameter(w, requires_grad=False)
        self.variance_epsilon = eps


class _Attn(torch.nn.Module):
    """HF remote-code DeepseekV2Attention attribute names (q_lora_rank=None)."""

    def __init__(self, lw):
        super().__init__()
        self.q_lora_rank = None
        self.q_proj = _Lin(lw["q_proj"])
        self.kv_a_proj_with_mqa = _Lin(lw["kv_a_proj_with_mqa"])
        self.kv_a_layernorm = _Norm(lw["kv_a_layernorm"], 1e-6)
        self.kv_b_proj = _Lin(lw["kv_b_proj"])
        self.o_proj = _Lin(lw["o_proj"])


def _attn_layer(seed):
    return {"q_proj": rnd(3072, 2048, std=0.02, seed=seed), "kv_a_proj_with_mqa": rnd(576, 2048, std=0.02, seed=seed + 1),
            "kv_a_layernorm": (rnd(512, std=0.1, seed=seed + 2) + 1).to(BF),
            "kv_b_proj": rnd(4096, 512, std=0.02, seed=seed + 3), "o_proj": rnd(2048, 2048, std=0.02, seed=seed + 4)}


def _prefill_cache(lw32, d, B, L, pos, seed, cos, sin):
    """Oracle caches of B sequences with `pos` tokens each (random normed hidden states),
    and the same rows as the compressed [B, L, 576] bf16 cache the surface reads."""
    g = torch.Generator().manual_seed(seed)
    caches, kc = [], torch.zeros(B, L, 576, dtype=BF)
    for b in range(B):
        sc = O.SeqCache()
        if pos:
            xs = torch.randn(pos, 2048, generator=g).to(BF).float()
            O.attention(lw32, d, xs, sc, torch.arange(pos), cos, sin, rb)
            rows = torch.cat([torch.cat(sc.c, 0), torch.cat(sc.kpe, 0)], -1)
            kc[b, :pos] = rows.to(BF)
        caches.append(sc)
    return caches, kc.to(DEV)


@pytest.mark.parametrize("fn,B,L,pos", [("attention_decode_only_triton", 1, 64, 40),
                                        ("attention_decode_small_batch_triton", 3, 300, 255),
                                        ("attention_decode_small_batch_triton", 2, 2600, 2100),
                                        ("attention_decode_triton", 4, 200, 0),
                                        ("attention_decode_triton", 3, 1500, 1200)])
def test_attention_decode_surface_vs_oracle(fn, B, L, pos):
    """hidden [B,1,2048] (already input-normed) -> o_proj output, the new token's compressed
    row written at cache_position, through pack_attention_weights of an HF-named module;
    L > 2048 takes the small family's split-KV path."""
    import triton_kernels.attention_decode_batch as AB
    import triton_kernels.attention_decode_small as AS
    from dsv2lite.config import DSV2Config
    from dsv2lite.rope import cos_sin_tables

    lw = _attn_layer(50)
    packed = AB.pack_attention_weights(_Attn(lw))
    assert torch.equal(packed.w_qkva, torch.cat([lw["q_proj"], lw["kv_a_proj_with_mqa"]]))
    d = O.Dims()
    lw32 = {k: c(v) for k, v in lw.items()}
    ocos, osin = O.yarn_cos_sin(d, L, mode="bf16")
    caches, kc = _prefill_cache(lw32, d, B, L, pos, 51, ocos, osin)
    cos, sin = cos_sin_tables(DSV2Config(), L, device=DEV)
    x = rnd(B, 1, 2048, seed=52)
    cp = torch.tensor([pos], dtype=torch.long, device=DEV)
    pid = torch.full((B, 1), pos, dtype=torch.long, device=DEV)
    f = getattr(AS, fn, None) or getattr(AB, fn)
    before = kc.clone()
    out = f(x, cos, sin, pid, cp, kc, None, packed, O.softmax_scale(d))
    assert out.shape == (B, 1, 2048)
    AB.check_cache_status(packed)
    for b in range(B):
        r16 = O.attention(lw32, d, c(x[b]), caches[b], torch.tensor([pos]), ocos, osin, rb)
        assert rel_err(c(out[b]), r16) < 2e-2, (b, rel_err(c(out[b]), r16))
        new = torch.cat([caches[b].c[-1], caches[b].kpe[-1]], -1)[0]
        assert rel_err(c(kc[b, pos]), new) < 8e-3
    mask = torch.ones(L, dtype=torch.bool)
    mask[pos] = False
    assert torch.equal(kc[:, mask], before[:, mask])  # only slot `pos` of each row is written
    # the workspace is reused: a second call with the same shapes returns the same buffer
    out2 = f(x, cos, sin, pid, cp, kc.clone(), None, packed, O.softmax_scale(d))
    assert out2.data_ptr() == out.data_ptr()


@pytest.mark.parametrize("fn", ["attention_decode_only_triton", "attention_decode_triton"])
def test_attention_decode_surface_refuses_overflow(fn):
    """cache_position == L: no row of the cache changes, the status raises, the output is
    finite (the rows that exist are attended)."""
    import triton_kernels.attention_decode_batch as AB
    import triton_kernels.attention_decode_small as AS
    from dsv2lite.config import DSV2Config
    from dsv2lite.rope import cos_sin_tables

    B = 1 if fn == "attention_decode_only_triton" else 2
    L = 48
    packed = AB.pack_attention_weights(_Attn(_attn_layer(60)))
    kc = rnd(B, L, 576, seed=61)
    before = kc.clone()
    cos, sin = cos_sin_tables(DSV2Config(), 64, device=DEV)
    f = getattr(AS, fn, None) or getattr(AB, fn)
    out = f(rnd(B, 1, 2048, seed=62), cos, sin, None, torch.tensor([L], dtype=torch.long, device=DEV), kc, None,
            packed, 0.1147)
    assert torch.isfinite(out.float()).all()
    assert torch.equal(kc, before)
    with pytest.raises(RuntimeError, match="cache length"):
        AB.check_cache_status(packed)


@pytest.mark.parametrize("B,H,L,pos,Dq,Dv", [(2, 16, 100, 99, 192, 128), (3, 16, 700, 311, 192, 128),
                                              (1, 4, 64, 0, 64, 256)])
def test_batched_attention_decode_q1_expanded_vs_fp32(B, H, L, pos, Dq, Dv):
    """The reference's expanded-cache attention (attention_decode_batch.py:241-401): q
    [B,H,1,Dq], K [B,H,L,Dq], V [B,H,L,Dv] as strided views of a larger buffer."""
    from triton_kernels.attention_decode_batch import batched_attention_decode_q1_triton, check_expanded_status

    q = rnd(B, H, 1, Dq, seed=70)
    kbuf = rnd(B, H, L + 5, Dq, seed=71)
    vbuf = rnd(B, H, L + 3, Dv, seed=72)
    k, v = kbuf[:, :, :L], vbuf[:, :, :L]  # non-contiguous in the sequence/head strides
    scale = 0.1147
    out = batched_attention_decode_q1_triton(q, k, v, torch.tensor([pos], dtype=torch.long, device=DEV), scale)
    assert out.shape == (B, H, 1, Dv)
    s = torch.einsum("bhd,bhld->bhl", c(q)[:, :, 0], c(k)[:, :, :pos + 1]) * scale
    ref = torch.einsum("bhl,bhld->bhd", torch.softmax(s, -1), c(v)[:, :, :pos + 1])
    assert rel_err(c(out)[:, :, 0], ref) < 1e-2
    check_expanded_status(DEV)
    # past the cache: attends the L rows, flagged
    out2 = batched_attention_decode_q1_triton(q, k, v, torch.tensor([L + 3], dtype=torch.long, device=DEV), scale)
    s = torch.einsum("bhd,bhld->bhl", c(q)[:, :, 0], c(k)) * scale
    ref2 = torch.einsum("bhl,bhld->bhd", torch.softmax(s, -1), c(v))
    assert rel_err(c(out2)[:, :, 0], ref2) < 1e-2
    with pytest.raises(RuntimeError, match="outside the cache"):
        check_expanded_status(DEV)


# --------------------------------------------------------------------------- capacity guard (C ABI)
def test_mla_kernels_never_touch_another_rows_slots():
    """Row 0 at pos == cap (full), row 1 with room.  The split-KV path (prepare + decode +
    combine), the fused kernel and the attention of the absorb path must: write nothing for
    row 0, write row 1's slot, flag the status, and read nothing outside a row's own slots
    (the slots after row 0's are NaN, so any read of them would poison its output)."""
    from dsv2lite.config import DSV2Config
    from dsv2lite.rope import cos_sin_tables

    cfg = DSV2Config()
    caps = [40, 70]
    B = 2
    base = torch.tensor([0, 48], dtype=torch.int64, device=DEV)  # 8 guard slots between the rows
    capd = torch.tensor(caps, dtype=torch.int32, device=DEV)
    pos = torch.tensor([40, 33], dtype=torch.int32, device=DEV)
    cache = rnd(48 + 70 + 8, 576, seed=80, std=0.5)
    cache[40:48] = float("nan")
    cache[48 + 70:] = float("nan")
    qkva = rnd(B, 3648, seed=81)
    kvw = (rnd(512, seed=82, std=0.1) + 1).to(BF)
    w_uk = rnd(16, 128, 512, std=0.05, seed=83)
    w_ukt = w_uk.transpose(1, 2).contiguous()
    w_uv = rnd(16, 128, 512, std=0.05, seed=84)
    cos, sin = cos_sin_tables(cfg, 128, device=DEV)
    scale = cfg.softmax_scale
    outs = {}
    # the absorb path's partial absorbed queries, formed here from qkva (8 blocks of 16 q_nope rows)
    qn = c(qkva)[:, :3072].view(B, 16, 192)[:, :, :128].reshape(B, 16, 8, 16)
    parts = torch.einsum("bhid,hidc->bhic", qn, c(w_uk).view(16, 8, 16, 512)).contiguous().to(DEV)
    for path in ("split", "fused", "absorb"):
        cch = cache.clone()
        status = torch.zeros(1, dtype=torch.int32, device=DEV)
        out = torch.empty(B, 2048, dtype=BF, device=DEV)
        if path == "split":
            q = torch.empty(B, 16, 576, dtype=BF, device=DEV)
            po = torch.empty(B, 4, 16, 512, device=DEV)
            pm = torch.empty(B, 4, 16, 2, device=DEV)
            call("dsv2_mla_prepare", qkva.data_ptr(), 3648, B, pos.data_ptr(), base.data_ptr(), capd.data_ptr(),
                 kvw.data_ptr(), 1e-6, cos.data_ptr(), sin.data_ptr(), 128, w_ukt.data_ptr(), cch.data_ptr(),
                 q.data_ptr(), status.data_ptr(), st())
            call("dsv2_mla_decode", q.data_ptr(), cch.data_ptr(), base.data_ptr(), pos.data_ptr(), capd.data_ptr(), B,
                 32, 4, scale, po.data_ptr(), pm.data_ptr(), st())
            call("dsv2_mla_combine", po.data_ptr(), pm.data_ptr(), pos.data_ptr(), capd.data_ptr(), B, 32, 4,
                 w_uv.data_ptr(), out.data_ptr(), 2048, st())
        elif path == "fused":
            call("dsv2_mla_fused", qkva.data_ptr(), 3648, B, pos.data_ptr(), base.data_ptr(), capd.data_ptr(),
                 kvw.data_ptr(), 1e-6, cos.data_ptr(), sin.data_ptr(), 128, w_ukt.data_ptr(), w_uv.data_ptr(),
                 cch.data_ptr(), scale, out.data_ptr(), 2048, status.data_ptr(), st())
        else:
            call("dsv2_mla_attend_parts", qkva.data_ptr(), 3648, B, pos.data_ptr(), base.data_ptr(), capd.data_ptr(),
                 kvw.data_ptr(), 1e-6, cos.data_ptr(), sin.data_ptr(), 128, parts.data_ptr(), w_uv.data_ptr(),
                 cch.data_ptr(), scale, out.data_ptr(), 2048, status.data_ptr(), st())
        torch.cuda.synchronize()
        assert status.item() == 1, path
        changed = (cch.view(torch.int16) != cache.view(torch.int16)).any(-1).nonzero().flatten().tolist()
        assert changed == [48 + 33], (path, changed)  # only row 1's slot 33
        assert torch.isfinite(out.float()).all(), path
        outs[path] = out
    # row 1 (within capacity) agrees between the paths; row 0 attended its 40 rows only
    assert rel_err(c(outs["fused"][1]), c(outs["split"][1])) < 2e-2
    assert rel_err(c(outs["absorb"][1]), c(outs["split"][1])) < 2e-2
