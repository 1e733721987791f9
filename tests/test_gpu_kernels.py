"""Kernel-level parity on the GPU: every HIP entry point against a plain PyTorch
fp32 reference (floating point) or the CPU oracle / exact invariants (integer work).

Tolerances (max|a-b| / max|b|): 1e-2 for bf16 GEMV/GEMM/MLA outputs, exact for
residual add, bucketing and router ids where the top-6 margin exceeds 1e-3.
"""

from __future__ import annotations

import math

import pytest
import torch

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from triton_kernels import _hip
    from triton_kernels._hip import LINEAR_OUT_F32, LINEAR_SWIGLU, call

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


def test_abi_loaded():
    assert _hip.lib.dsv2_abi_version() == _hip.ABI_VERSION == 2
    print("native library:", _hip.LIB_PATH, flush=True)


@pytest.mark.parametrize("rows,cols", [(1, 2048), (7, 512), (33, 2048)])
def test_rmsnorm(rows, cols):
    x = rnd(rows, cols, seed=1)
    w = rnd(cols, seed=2, std=0.5) + 1
    w = w.to(BF)
    y = torch.empty_like(x)
    call("dsv2_rmsnorm_bf16", x.data_ptr(), cols, w.data_ptr(), y.data_ptr(), cols, rows, cols, 1e-6, st())
    ref = O.rmsnorm(x.float().cpu(), w.float().cpu(), 1e-6, rb)
    assert rel_err(y.float().cpu(), ref) < 8e-3
    assert (y.float().cpu() == ref).float().mean() > 0.98


def test_residual_add_bit_exact_and_silu_mul():
    a, b = rnd(5, 2048, seed=3), rnd(5, 2048, seed=4)
    out = torch.empty_like(a)
    call("dsv2_residual_add_bf16", a.data_ptr(), b.data_ptr(), out.data_ptr(), a.numel(), st())
    assert torch.equal(out, (a.float() + b.float()).to(BF))
    call("dsv2_silu_mul_bf16", a.data_ptr(), b.data_ptr(), out.data_ptr(), a.numel(), st())
    ref = (torch.nn.functional.silu(a.float()) * b.float()).to(BF)
    assert rel_err(out.float(), ref.float()) < 1e-2


@pytest.mark.parametrize("rows", [1, 3, 8, 11])
@pytest.mark.parametrize("mode", ["plain", "norm", "swiglu", "residual", "f32"])
def test_gemv(rows, mode):
    K, N = 2048, 512
    x = rnd(rows, K, seed=5)
    W = rnd(2 * N if mode == "swiglu" else N, K, std=0.02, seed=6)
    nw = (rnd(K, seed=7, std=0.1) + 1).to(BF) if mode in ("norm", "swiglu") else None
    res = rnd(rows, N, seed=8) if mode == "residual" else None
    flags = LINEAR_SWIGLU if mode == "swiglu" else (LINEAR_OUT_F32 if mode == "f32" else 0)
    y = torch.empty(rows, N, dtype=torch.float32 if mode == "f32" else BF, device=DEV)
    call("dsv2_gemv_bf16", x.data_ptr(), K, rows, K, W.data_ptr(), N, _hip.ptr(nw), 1e-6, _hip.ptr(res), N,
         y.data_ptr(), N, flags, st())
    xf = x.float()
    if nw is not None:
        xf = O.rmsnorm(xf, nw.float(), 1e-6, rb)
    acc = xf @ W.float().t()
    if mode == "swiglu":
        ref = rb(rb(torch.nn.functional.silu(rb(acc[:, :N]))) * rb(acc[:, N:]))
    elif mode == "residual":
        ref = rb(res.float() + rb(acc))
    else:
        ref = rb(acc)
    assert rel_err(y.float(), ref) < 1e-2


@pytest.mark.parametrize("rows", [1, 16, 37, 64, 200, 256])
@pytest.mark.parametrize("mode", ["plain", "swiglu", "residual", "f32"])
def test_gemm_dense(rows, mode):
    K, N = 2048, 384
    x = rnd(rows, K, seed=9)
    W = rnd(2 * N if mode == "swiglu" else N, K, std=0.02, seed=10)
    res = rnd(rows, N, seed=11) if mode == "residual" else None
    flags = LINEAR_SWIGLU if mode == "swiglu" else (LINEAR_OUT_F32 if mode == "f32" else 0)
    y = torch.empty(rows, N, dtype=torch.float32 if mode == "f32" else BF, device=DEV)
    call("dsv2_gemm_bf16", x.data_ptr(), K, 0, rows, K, W.data_ptr(), 0, N, 1, _hip.ptr(res), N, y.data_ptr(), N, 0,
         flags, st())
    acc = x.float() @ W.float().t()
    if mode == "swiglu":
        ref = rb(rb(torch.nn.functional.silu(rb(acc[:, :N]))) * rb(acc[:, N:]))
    elif mode == "residual":
        ref = rb(res.float() + rb(acc))
    else:
        ref = rb(acc)
    assert rel_err(y.float(), ref) < 1e-2


@pytest.mark.parametrize("rows", [3, 64, 200])
@pytest.mark.parametrize("mode", ["residual", "f32", "swiglu"])
def test_gemm_token_lds_shape_epilogues(rows, mode):
    """Launches wide enough for the token-rows-in-LDS shape (>= 512 workgroups), every
    epilogue, ragged token tiles."""
    K, N = 2048, 32768
    x = rnd(rows, K, seed=41)
    W = rnd(2 * N if mode == "swiglu" else N, K, std=0.02, seed=42)
    res = rnd(rows, N, seed=43) if mode == "residual" else None
    flags = LINEAR_SWIGLU if mode == "swiglu" else (LINEAR_OUT_F32 if mode == "f32" else 0)
    y = torch.empty(rows, N, dtype=torch.float32 if mode == "f32" else BF, device=DEV)
    call("dsv2_gemm_bf16", x.data_ptr(), K, 0, rows, K, W.data_ptr(), 0, N, 1, _hip.ptr(res), N, y.data_ptr(), N, 0,
         flags, st())
    acc = x.float() @ W.float().t()
    if mode == "swiglu":
        ref = rb(rb(torch.nn.functional.silu(rb(acc[:, :N]))) * rb(acc[:, N:]))
    elif mode == "residual":
        ref = rb(res.float() + rb(acc))
    else:
        ref = rb(acc)
    assert rel_err(y.float(), ref) < 1e-2


@pytest.mark.parametrize("rows", [5, 100])
@pytest.mark.parametrize("K,N,swiglu", [(128, 512, False), (1408, 2048, False), (2816, 2048, False), (10944, 2048, False),
                                        (2048, 1408, True), (512, 128, False), (2048, 102400, False),
                                        (2048, 65536, True), (1408, 65536, False)])
def test_gemm_k_split_shapes(rows, K, N, swiglu):
    """Every K of the model (uneven per-wave k ranges, multi-batch ranges, one-wave K), and
    output widths large enough for the streaming launch shape (lm_head-sized)."""
    x = rnd(rows, K, seed=K + rows)
    W = rnd(2 * N if swiglu else N, K, std=0.02, seed=K + 1)
    y = torch.empty(rows, N, dtype=BF, device=DEV)
    call("dsv2_gemm_bf16", x.data_ptr(), K, 0, rows, K, W.data_ptr(), 0, N, 1, None, 0, y.data_ptr(), N, 0,
         LINEAR_SWIGLU if swiglu else 0, st())
    acc = x.float() @ W.float().t()
    ref = rb(rb(torch.nn.functional.silu(rb(acc[:, :N]))) * rb(acc[:, N:])) if swiglu else rb(acc)
    assert rel_err(y.float(), ref) < 1e-2


@pytest.mark.parametrize("rows", [16, 64, 130, 256, 600, 1030])
@pytest.mark.parametrize("K,N,mode", [(2048, 3648, "plain"), (2048, 2048, "residual"), (2048, 2816, "swiglu"),
                                      (2816, 2048, "plain"), (2048, 10944, "swiglu"), (10944, 2048, "residual"),
                                      (2048, 2048, "f32"), (2048, 64, "f32")])
def test_gemm_dense_model_shapes(rows, K, N, mode):
    """The batch family's dense projections (qkv_a, o_proj + residual, shared-expert
    gate_up / down, layer-0 MLP gate_up / down + residual, the router logits) at the token
    counts where the one-shot and the token-rows-in-LDS shapes take over from the k-split
    kernel, and at prefill sizes (from 512 rows: 256 x 128 ring tiles, qkv_a with a ragged
    last feature block)."""
    x = rnd(rows, K, seed=K + N + rows)
    W = rnd(2 * N if mode == "swiglu" else N, K, std=0.02, seed=K + N)
    res = rnd(rows, N, seed=3 * rows) if mode == "residual" else None
    flags = LINEAR_SWIGLU if mode == "swiglu" else (LINEAR_OUT_F32 if mode == "f32" else 0)
    y = torch.empty(rows, N, dtype=torch.float32 if mode == "f32" else BF, device=DEV)
    call("dsv2_gemm_bf16", x.data_ptr(), K, 0, rows, K, W.data_ptr(), 0, N, 1, _hip.ptr(res), N, y.data_ptr(), N, 0,
         flags, st())
    acc = x.float() @ W.float().t()
    if mode == "swiglu":
        ref = rb(rb(torch.nn.functional.silu(rb(acc[:, :N]))) * rb(acc[:, N:]))
    elif mode == "residual":
        ref = rb(res.float() + rb(acc))
    else:
        ref = rb(acc)
    assert rel_err(y.float(), ref) < 1e-2


@pytest.mark.parametrize("rows", [200, 256])
@pytest.mark.parametrize("mode", ["plain", "residual", "f32"])
def test_gemm_wide_dense_epilogues(rows, mode):
    """Wide dense outputs at 128+ tokens (the direct-to-LDS ring shape: N = 3648, 64 x 64
    tiles, XCD-aware grid), every epilogue, a partial last token tile at 200 rows."""
    K, N = 2048, 3648
    x = rnd(rows, K, seed=rows + 7)
    W = rnd(N, K, std=0.02, seed=8)
    res = rnd(rows, N, seed=9) if mode == "residual" else None
    flags = LINEAR_OUT_F32 if mode == "f32" else 0
    y = torch.empty(rows, N, dtype=torch.float32 if mode == "f32" else BF, device=DEV)
    call("dsv2_gemm_bf16", x.data_ptr(), K, 0, rows, K, W.data_ptr(), 0, N, 1, _hip.ptr(res), N, y.data_ptr(), N, 0,
         flags, st())
    acc = x.float() @ W.float().t()
    ref = rb(res.float() + rb(acc)) if mode == "residual" else rb(acc)
    assert rel_err(y.float(), ref) < 1e-2


@pytest.mark.parametrize("rows", [1, 5, 64, 200, 256])
def test_gemm_grouped_heads_absorption(rows):
    # q_lat[r, h, :512] = W_UK_h^T q_nope[r, h]   and   attn[r, h*128+i] = W_UV_h o_lat[r, h]
    qkva = rnd(rows, 3648, seed=12)
    w_uk = rnd(16, 128, 512, std=0.05, seed=13)
    w_ukt = w_uk.transpose(1, 2).contiguous()
    q = torch.zeros(rows, 16, 576, dtype=BF, device=DEV)
    call("dsv2_gemm_bf16", qkva.data_ptr(), 3648, 192, rows, 128, w_ukt.data_ptr(), 512 * 128, 512, 16, None, 0,
         q.data_ptr(), 16 * 576, 576, 0, st())
    q_nope = qkva.float().view(rows, 3648)[:, :3072].reshape(rows, 16, 192)[:, :, :128]
    ref = rb(torch.einsum("rhi,hij->rhj", q_nope, w_uk.float()))
    assert rel_err(q[:, :, :512].float(), ref) < 1e-2
    assert torch.all(q[:, :, 512:] == 0)
    olat = rnd(rows, 16, 512, seed=14)
    w_uv = rnd(16, 128, 512, std=0.05, seed=15)
    attn = torch.empty(rows, 2048, dtype=BF, device=DEV)
    call("dsv2_gemm_bf16", olat.data_ptr(), 16 * 512, 512, rows, 512, w_uv.data_ptr(), 128 * 512, 128, 16, None, 0,
         attn.data_ptr(), 2048, 128, 0, st())
    ref = rb(torch.einsum("hij,rhj->rhi", w_uv.float(), olat.float()).reshape(rows, 2048))
    assert rel_err(attn.float(), ref) < 1e-2


def _router_case(rows, seed, unit_norm=True):
    h = rnd(rows, 2048, seed=seed)
    nw = torch.ones(2048, dtype=BF, device=DEV) if unit_norm else (1 + rnd(2048, std=0.1, seed=seed + 2)).to(BF)
    wr = rnd(64, 2048, std=0.02, seed=seed + 1)
    return h, nw, wr


@pytest.mark.parametrize("rows,unit_norm", [(1, True), (64, True), (300, True), (37, False)])
def test_router_topk6(rows, unit_norm):
    """One workgroup per token; 37 rows with a non-trivial norm weight."""
    h, nw, wr = _router_case(rows, 20, unit_norm)
    xn = torch.empty_like(h)
    ids = torch.empty(rows, 6, dtype=torch.int32, device=DEV)
    ids64 = torch.empty(rows, 6, dtype=torch.int64, device=DEV)
    w = torch.empty(rows, 6, dtype=torch.float32, device=DEV)
    call("dsv2_router_topk6", h.data_ptr(), 2048, nw.data_ptr(), 1e-6, wr.data_ptr(), 1.0, rows, xn.data_ptr(),
         ids.data_ptr(), ids64.data_ptr(), w.data_ptr(), st())
    xr = O.rmsnorm(h.float().cpu(), nw.float().cpu(), 1e-6, rb)
    assert rel_err(xn.float().cpu(), xr) < 8e-3
    oid, ow, scores = O.router_topk(xn.float().cpu(), wr.float().cpu(), 6, 1.0)
    margin = O.topk_margin(scores, 6)
    ok = margin > 1e-3
    assert ok.float().mean() > 0.5
    assert torch.equal(ids.cpu().long()[ok], oid[ok])  # same order too (descending, ties -> lower)
    assert torch.equal(ids64.cpu(), ids.cpu().long())
    assert torch.allclose(w.cpu()[ok], ow[ok], rtol=1e-4, atol=1e-6)


def test_router_topk6_exact_ties():
    """W_r rows 9 and 40 identical and aligned with h (so they lead many rows' top-6) and rows
    2 and 3 identical: equal logits, the lower index ranked first with an equal weight, in
    every row that holds both."""
    rows = 40
    h, nw, wr = _router_case(rows, 440, False)
    wr[40] = wr[9] = (h[:8].float().mean(0) * 0.05).to(BF)
    wr[3] = wr[2]
    ids = torch.empty(rows, 6, dtype=torch.int32, device=DEV)
    w = torch.empty(rows, 6, dtype=torch.float32, device=DEV)
    xn = torch.empty_like(h)
    call("dsv2_router_topk6", h.data_ptr(), 2048, nw.data_ptr(), 1e-6, wr.data_ptr(), 1.0, rows, xn.data_ptr(),
         ids.data_ptr(), None, w.data_ptr(), st())
    idl, wl = ids.cpu().tolist(), w.cpu()
    both = 0
    for r in range(rows):
        for a, b in ((9, 40), (2, 3)):
            if a in idl[r] and b in idl[r]:
                both += 1
                ia, ib = idl[r].index(a), idl[r].index(b)
                assert ia + 1 == ib and wl[r, ia] == wl[r, ib], (r, idl[r])
    assert both >= 6
    oid, ow, scores = O.router_topk(xn.float().cpu(), wr.float().cpu(), 6, 1.0)
    for r in range(rows):  # the sets agree with the oracle on the kernel's own xn
        assert sorted(idl[r]) == sorted(oid[r].tolist()) or O.topk_margin(scores[r:r + 1], 6)[0] <= 1e-3


def test_router_from_logits_ties():
    lg = torch.zeros(2, 64, device=DEV)
    lg[0, [5, 9, 40]] = 3.0
    lg[0, [2, 7, 8, 60]] = 1.0
    lg[1] = torch.arange(64, device=DEV, dtype=torch.float32) * 0.01
    ids = torch.empty(2, 6, dtype=torch.int64, device=DEV)
    w = torch.empty(2, 6, dtype=torch.float32, device=DEV)
    call("dsv2_router_topk6_from_logits", lg.data_ptr(), 2, 2.0, None, ids.data_ptr(), w.data_ptr(), st())
    assert ids[0].tolist() == [5, 9, 40, 2, 7, 8]
    assert ids[1].tolist() == [63, 62, 61, 60, 59, 58]
    ref = torch.softmax(lg.cpu(), -1)
    assert torch.allclose(w.cpu(), 2.0 * ref.gather(1, ids.cpu()), rtol=1e-5)


@pytest.mark.parametrize("rows", [1024, 8192])
def test_gemm_router_logits_exact_fp32(rows):
    """The prefill router (RMSNorm, the logits as an MFMA GEMM with DSV2_LINEAR_OUT_F32_EXACT,
    then the top-6) keeps the logits in unrounded fp32 like the decode routers: the logits
    are the fp32 sums of the exact bf16 products (|error| <= 1e-5, where a bf16 round would
    move them by ~2e-4), and the ids and weights equal dsv2_router_topk6's on the same input
    wherever the top-6 logit margin exceeds 1e-4 (the two sum the products in different
    orders)."""
    from triton_kernels._hip import LINEAR_OUT_F32_EXACT

    h, nw, wr = _router_case(rows, 77)
    xn = torch.empty_like(h)
    call("dsv2_rmsnorm_bf16", h.data_ptr(), 2048, nw.data_ptr(), xn.data_ptr(), 2048, rows, 2048, 1e-6, st())
    lg = torch.empty(rows, 64, dtype=torch.float32, device=DEV)
    call("dsv2_gemm_bf16", xn.data_ptr(), 2048, 0, rows, 2048, wr.data_ptr(), 0, 64, 1, None, 0, lg.data_ptr(), 64, 0,
         LINEAR_OUT_F32_EXACT, st())
    ids = torch.empty(rows, 6, dtype=torch.int32, device=DEV)
    w = torch.empty(rows, 6, dtype=torch.float32, device=DEV)
    call("dsv2_router_topk6_from_logits", lg.data_ptr(), rows, 1.0, ids.data_ptr(), None, w.data_ptr(), st())
    xn2 = torch.empty_like(h)
    ids2 = torch.empty_like(ids)
    w2 = torch.empty_like(w)
    call("dsv2_router_topk6", h.data_ptr(), 2048, nw.data_ptr(), 1e-6, wr.data_ptr(), 1.0, rows, xn2.data_ptr(),
         ids2.data_ptr(), None, w2.data_ptr(), st())
    torch.cuda.synchronize()
    exact = xn.double() @ wr.double().t()
    assert float((lg.double() - exact).abs().max()) <= 1e-5
    assert float((rb(exact.float()).double() - exact).abs().max()) > 1e-4  # a bf16 round would show
    srt = torch.sort(exact, dim=-1, descending=True).values
    ok = (srt[:, 5] - srt[:, 6]) > 1e-4
    assert ok.float().mean() > 0.9
    # sets compared in id order (two of the six may hold logits within fp32 rounding)
    def by_id(i, wt):
        o = torch.argsort(i.long(), dim=1)
        return i.gather(1, o), wt.gather(1, o)

    top = torch.sort(exact, dim=-1, descending=True, stable=True).indices[:, :6].to(torch.int32)
    ref_w = torch.softmax(exact, dim=-1).gather(1, top.long()).float()
    (i1, w1), (i0, w0) = by_id(ids, w), by_id(top, ref_w)
    assert torch.equal(i1[ok], i0[ok])
    assert torch.allclose(w1[ok], w0[ok], rtol=1e-5, atol=1e-7)
    # the decode router on the same hidden states: same ids and weights wherever its own
    # normalised input is bitwise the same (its norm sums in another order)
    same = (xn == xn2).all(dim=1) & ok
    assert same.float().mean() > 0.5
    i2, w2s = by_id(ids2, w2)
    assert torch.equal(i1[same], i2[same])
    assert torch.allclose(w1[same], w2s[same], rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("rows,tile", [(1, 16), (64, 16), (256, 64), (1024, 64), (5, 32)])
def test_moe_bucket_invariants(rows, tile):
    g = torch.Generator().manual_seed(rows)
    ids = torch.randint(0, 64, (rows, 6), generator=g, dtype=torch.int32)
    if rows == 256:
        ids[:100] = 7  # a hot expert spanning several tiles
    R = rows * 6
    max_tiles = math.ceil(R / tile) + 64
    d = ids.to(DEV)
    sorted_r = torch.empty(R, dtype=torch.int32, device=DEV)
    rpos = torch.empty(R, dtype=torch.int32, device=DEV)
    tiles = torch.full((max_tiles, 4), -1, dtype=torch.int32, device=DEV)
    nt = torch.empty(1, dtype=torch.int32, device=DEV)
    call("dsv2_moe_bucket", d.data_ptr(), rows, tile, sorted_r.data_ptr(), rpos.data_ptr(), tiles.data_ptr(),
         nt.data_ptr(), st())
    flat = ids.flatten().long()
    ref = sorted(range(R), key=lambda r: (int(flat[r]), r))  # stable counting sort
    assert sorted_r.cpu().tolist() == ref
    assert torch.equal(sorted_r.cpu()[rpos.cpu().long()], torch.arange(R, dtype=torch.int32))
    n = int(nt.item())
    T = tiles.cpu()[:n]
    assert n == sum(math.ceil(int((flat == e).sum()) / tile) for e in range(64))
    covered = torch.zeros(R, dtype=torch.int32)
    for e, s, c, _ in T.tolist():
        assert 1 <= c <= tile
        assert all(int(flat[ref[p]]) == e for p in range(s, s + c))
        covered[s:s + c] += 1
    assert torch.all(covered == 1)


@pytest.mark.parametrize("rows,tile", [(1, 16), (37, 32), (1000, 64), (4096, 256), (8192, 256),
                                       (8192, 64)])
def test_moe_bucket_wide_equals_one_workgroup(rows, tile):
    """dsv2_moe_bucket_wide (three launches, workspace histograms) gives dsv2_moe_bucket's
    outputs bit for bit -- sorted routes, route positions, tile table and count -- at every
    size up to the 49,152 routes of an 8,192-row prefill chunk, with a hot expert spanning
    many chunks; a workspace one byte short is rejected."""
    g = torch.Generator().manual_seed(rows + tile)
    ids = torch.randint(0, 64, (rows, 6), generator=g, dtype=torch.int32)
    if rows >= 1000:
        ids[: rows // 3, 0] = 11
    d = ids.to(DEV)
    R = rows * 6
    max_tiles = math.ceil(R / tile) + 64
    outs = []
    for wide in (False, True):
        sr = torch.full((R,), -1, dtype=torch.int32, device=DEV)
        rp = torch.full((R,), -1, dtype=torch.int32, device=DEV)
        tl = torch.full((max_tiles, 4), -1, dtype=torch.int32, device=DEV)
        nt = torch.full((1,), -1, dtype=torch.int32, device=DEV)
        if wide:
            nb = _hip.lib.dsv2_moe_bucket_workspace_size(rows)
            ws = torch.empty(nb, dtype=torch.uint8, device=DEV)
            with pytest.raises(_hip.HipKernelError):
                call("dsv2_moe_bucket_wide", d.data_ptr(), rows, tile, sr.data_ptr(), rp.data_ptr(), tl.data_ptr(),
                     nt.data_ptr(), ws.data_ptr(), nb - 1, st())
            call("dsv2_moe_bucket_wide", d.data_ptr(), rows, tile, sr.data_ptr(), rp.data_ptr(), tl.data_ptr(),
                 nt.data_ptr(), ws.data_ptr(), nb, st())
        else:
            call("dsv2_moe_bucket", d.data_ptr(), rows, tile, sr.data_ptr(), rp.data_ptr(), tl.data_ptr(),
                 nt.data_ptr(), st())
        n = int(nt.item())
        outs.append((sr.cpu(), rp.cpu(), tl.cpu()[:n], n))
    (a_sr, a_rp, a_tl, a_n), (b_sr, b_rp, b_tl, b_n) = outs
    assert a_n == b_n and torch.equal(a_tl, b_tl)
    assert torch.equal(a_sr, b_sr) and torch.equal(a_rp, b_rp)


def _moe_layer(seed):
    gu = rnd(64, 2 * 1408, 2048, std=0.02, seed=seed)
    dn = rnd(64, 2048, 1408, std=0.02, seed=seed + 1)
    sgu = rnd(2 * 2816, 2048, std=0.02, seed=seed + 2)
    sdn = rnd(2048, 2816, std=0.02, seed=seed + 3)
    return gu, dn, sgu, sdn


def _oracle_moe_parts(xn, ids, w, gu, dn, sgu, sdn):
    """routed (fixed slot order, fp32 sum -> bf16) and shared outputs, bf16 rounding points."""
    I = 1408
    T = xn.shape[0]
    outs = torch.zeros(T, 6, 2048)
    for t in range(T):
        for s in range(6):
            e = int(ids[t, s])
            outs[t, s] = O.mlp(xn[t:t + 1], gu[e, :I], gu[e, I:], dn[e], rb)[0]
    routed = torch.zeros(T, 2048)
    for s in range(6):
        routed = routed + w[:, s:s + 1] * outs[:, s]
    shared = O.mlp(xn, sgu[:2816], sgu[2816:], sdn, rb)
    return rb(routed), shared


@pytest.mark.parametrize("rows", [1, 4])
def test_moe_small_family_route_local(rows):
    gu, dn, sgu, sdn = _moe_layer(30)
    xn = rnd(rows, 2048, seed=34)
    g = torch.Generator().manual_seed(35)
    ids = torch.stack([torch.randperm(64, generator=g)[:6] for _ in range(rows)]).to(torch.int32)
    w = torch.rand(rows, 6, generator=g) * 0.3
    h = rnd(rows, 2048, seed=36)
    hbuf = torch.empty(rows, 8, 1408, dtype=BF, device=DEV)
    out = torch.empty_like(h)
    dids, dw = ids.to(DEV), w.to(DEV)
    call("dsv2_moe_route_gateup", xn.data_ptr(), rows, dids.data_ptr(), gu.data_ptr(), sgu.data_ptr(), 1408,
         hbuf.data_ptr(), st())
    call("dsv2_moe_route_down", hbuf.data_ptr(), rows, dids.data_ptr(), dw.data_ptr(), dn.data_ptr(), sdn.data_ptr(),
         1408, 8, None, h.data_ptr(), out.data_ptr(), st())
    c = lambda t: t.float().cpu()  # noqa: E731
    routed, shared = _oracle_moe_parts(c(xn), ids, w, c(gu), c(dn), c(sgu), c(sdn))
    ref = rb(c(h) + rb(routed + shared))
    assert rel_err(c(out), ref) < 1e-2
    # residual-free, shared-free variant (the reference's routed-only API)
    hb6 = torch.empty(rows, 6, 1408, dtype=BF, device=DEV)
    call("dsv2_moe_route_gateup", xn.data_ptr(), rows, dids.data_ptr(), gu.data_ptr(), None, 1408, hb6.data_ptr(),
         st())
    call("dsv2_moe_route_down", hb6.data_ptr(), rows, dids.data_ptr(), dw.data_ptr(), dn.data_ptr(), None, 1408, 6,
         None, None, out.data_ptr(), st())
    assert rel_err(c(out), routed) < 1e-2
    # precomputed shared output (shared_y) added by the 6-route down == 8-route down
    shy = torch.empty(rows, 2048, dtype=BF, device=DEV)
    call("dsv2_gemv_bf16", hbuf[:, 6:].data_ptr(), 8 * 1408, rows, 2816, sdn.data_ptr(), 2048, None, 0.0, None, 0,
         shy.data_ptr(), 2048, 0, st())
    out2 = torch.empty_like(h)
    call("dsv2_moe_route_down", hbuf.data_ptr(), rows, dids.data_ptr(), dw.data_ptr(), dn.data_ptr(), None, 1408, 8,
         shy.data_ptr(), h.data_ptr(), out2.data_ptr(), st())
    call("dsv2_moe_route_down", hbuf.data_ptr(), rows, dids.data_ptr(), dw.data_ptr(), dn.data_ptr(), sdn.data_ptr(),
         1408, 8, None, h.data_ptr(), out.data_ptr(), st())
    assert rel_err(c(out2), c(out)) < 1e-2


@pytest.mark.parametrize("rows", [3, 64, 256])
def test_moe_batch_family_grouped(rows):
    from triton_kernels.moe_batch import PackedRoutedExperts, packed_routed_moe

    gu, dn, sgu, sdn = _moe_layer(40)
    xn = rnd(rows, 2048, seed=44)
    g = torch.Generator().manual_seed(45)
    ids = torch.stack([torch.randperm(64, generator=g)[:6] for _ in range(rows)])
    if rows == 256:
        ids[:80, 0] = 3  # one expert with 80+ tokens -> several tiles
    w = torch.rand(rows, 6, generator=g) * 0.3
    packed = PackedRoutedExperts(gu, dn, 2048, 1408, 64, 6)
    out = packed_routed_moe(xn, ids.to(DEV), w.to(DEV), packed)
    c = lambda t: t.float().cpu()  # noqa: E731
    sel = list(range(min(rows, 24)))  # oracle on a subset of rows (CPU time)
    routed, _ = _oracle_moe_parts(c(xn)[sel], ids[sel], w[sel], c(gu), c(dn), c(sgu), c(sdn))
    assert rel_err(c(out)[sel], routed) < 1e-2
    # deterministic: a second run is bit-identical
    out2 = packed_routed_moe(xn, ids.to(DEV), w.to(DEV), packed)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("rows,replicated", [(64, True), (200, True), (150, False)])
def test_moe_grouped_tile_sizes(rows, replicated):
    """Bucketing + grouped gate_up / down + combine with 16-, 32-, 64- and 256-token expert
    tiles (64, 256: the direct-to-LDS ring GEMM; replicated rows give full and partial tiles,
    random routing mostly near-empty ones) against the oracle on a subset of rows."""
    gu, dn, sgu, sdn = _moe_layer(60)
    xn = rnd(rows, 2048, seed=61)
    g = torch.Generator().manual_seed(62)
    if replicated:
        ids = torch.randperm(64, generator=g)[:6].repeat(rows, 1)
    else:
        ids = torch.stack([torch.randperm(64, generator=g)[:6] for _ in range(rows)])
    w = torch.rand(rows, 6, generator=g) * 0.3
    ids32, wd = ids.to(torch.int32).to(DEV), w.to(DEV)
    R = rows * 6
    outs = {}
    for tt in (16, 32, 64, 256):
        max_tiles = math.ceil(R / tt) + 64
        srt = torch.empty(R, dtype=torch.int32, device=DEV)
        rpos = torch.empty(R, dtype=torch.int32, device=DEV)
        tiles = torch.empty(max_tiles, 4, dtype=torch.int32, device=DEV)
        nt = torch.empty(1, dtype=torch.int32, device=DEV)
        hs = torch.empty(R, 1408, dtype=BF, device=DEV)
        ys = torch.empty(R, 2048, dtype=BF, device=DEV)
        out = torch.empty(rows, 2048, dtype=BF, device=DEV)
        call("dsv2_moe_bucket", ids32.data_ptr(), rows, tt, srt.data_ptr(), rpos.data_ptr(), tiles.data_ptr(),
             nt.data_ptr(), st())
        call("dsv2_moe_grouped_gateup", xn.data_ptr(), srt.data_ptr(), tiles.data_ptr(), nt.data_ptr(), max_tiles, tt,
             gu.data_ptr(), 1408, hs.data_ptr(), st())
        call("dsv2_moe_grouped_down", hs.data_ptr(), tiles.data_ptr(), nt.data_ptr(), max_tiles, tt, dn.data_ptr(),
             1408, ys.data_ptr(), st())
        call("dsv2_moe_combine", ys.data_ptr(), rpos.data_ptr(), wd.data_ptr(), rows, None, None, out.data_ptr(), None,
             0.0, None, st())
        outs[tt] = out.float().cpu()
    c = lambda t: t.float().cpu()  # noqa: E731
    sel = list(range(0, rows, max(1, rows // 20)))
    routed, _ = _oracle_moe_parts(c(xn)[sel], ids[sel], w[sel], c(gu), c(dn), c(sgu), c(sdn))
    for tt, out in outs.items():
        assert rel_err(out[sel], routed) < 1e-2, tt
        assert rel_err(out, outs[16]) < 1e-2, tt


@pytest.mark.parametrize("rows,replicated,tt", [(64, True, 64), (130, False, 64), (64, False, 16), (37, False, 16),
                                                (200, False, 32), (130, True, 32), (1024, False, 64),
                                                (300, True, 256), (1024, False, 256)])
def test_moe_grouped_gateup_with_shared(rows, replicated, tt):
    """The grouped gate_up / down with the shared halves in the same launches (16-, 32- and
    64-token tiles): routed rows equal the plain grouped launches' bit for bit, the shared
    output matches the fp32 SwiGLU reference and the dense shared gate_up, the fp32 halves
    sum to the shared down projection, and the combine agrees with the oracle."""
    gu, dn, sgu, sdn = _moe_layer(70)
    xn = rnd(rows, 2048, seed=71)
    g = torch.Generator().manual_seed(72)
    if replicated:
        ids = torch.randperm(64, generator=g)[:6].repeat(rows, 1)
    else:
        ids = torch.stack([torch.randperm(64, generator=g)[:6] for _ in range(rows)])
    ids32 = ids.to(torch.int32).to(DEV)
    R = rows * 6
    max_tiles = math.ceil(R / tt) + 64
    srt = torch.empty(R, dtype=torch.int32, device=DEV)
    rpos = torch.empty(R, dtype=torch.int32, device=DEV)
    tiles = torch.empty(max_tiles, 4, dtype=torch.int32, device=DEV)
    nt = torch.empty(1, dtype=torch.int32, device=DEV)
    call("dsv2_moe_bucket", ids32.data_ptr(), rows, tt, srt.data_ptr(), rpos.data_ptr(), tiles.data_ptr(),
         nt.data_ptr(), st())
    hs_ref = torch.empty(R, 1408, dtype=BF, device=DEV)
    call("dsv2_moe_grouped_gateup", xn.data_ptr(), srt.data_ptr(), tiles.data_ptr(), nt.data_ptr(), max_tiles, tt,
         gu.data_ptr(), 1408, hs_ref.data_ptr(), st())
    hs = torch.empty_like(hs_ref)
    sh = torch.empty(rows, 2816, dtype=BF, device=DEV)
    call("dsv2_moe_grouped_gateup_shared", xn.data_ptr(), rows, srt.data_ptr(), tiles.data_ptr(), nt.data_ptr(),
         max_tiles, tt, gu.data_ptr(), sgu.data_ptr(), 1408, hs.data_ptr(), sh.data_ptr(), st())
    assert torch.equal(hs, hs_ref)
    acc = xn.float() @ sgu.float().t()
    ref = rb(rb(torch.nn.functional.silu(rb(acc[:, :2816]))) * rb(acc[:, 2816:]))
    assert rel_err(sh.float(), ref) < 1e-2
    dense = torch.empty_like(sh)
    call("dsv2_gemm_bf16", xn.data_ptr(), 2048, 0, rows, 2048, sgu.data_ptr(), 0, 2816, 1, None, 0, dense.data_ptr(),
         2816, 0, LINEAR_SWIGLU, st())
    assert rel_err(sh.float(), dense.float()) < 1e-2
    # down: routed rows equal dsv2_moe_grouped_down's; the shared halves' fp32 partials sum to
    # the shared down projection; the combine of both paths agrees with the oracle
    ys_ref = torch.empty(R, 2048, dtype=BF, device=DEV)
    call("dsv2_moe_grouped_down", hs.data_ptr(), tiles.data_ptr(), nt.data_ptr(), max_tiles, tt, dn.data_ptr(), 1408,
         ys_ref.data_ptr(), st())
    ys = torch.empty_like(ys_ref)
    parts = torch.empty(2, rows, 2048, dtype=torch.float32, device=DEV)
    call("dsv2_moe_grouped_down_shared", hs.data_ptr(), rows, tiles.data_ptr(), nt.data_ptr(), max_tiles, tt,
         dn.data_ptr(), sh.data_ptr(), sdn.data_ptr(), 1408, ys.data_ptr(), parts.data_ptr(), st())
    assert torch.equal(ys, ys_ref)
    sh_ref = sh.float() @ sdn.float().t()
    assert rel_err(parts[0] + parts[1], sh_ref) < 1e-3
    assert rel_err(parts[1], sh.float()[:, 1408:] @ sdn.float()[:, 1408:].t()) < 1e-3
    w = (torch.rand(rows, 6, generator=g) * 0.3).to(DEV)
    res = rnd(rows, 2048, seed=73)
    out = torch.empty(rows, 2048, dtype=BF, device=DEV)
    call("dsv2_moe_combine_parts", ys.data_ptr(), rpos.data_ptr(), w.data_ptr(), rows, parts.data_ptr(),
         res.data_ptr(), out.data_ptr(), None, 0.0, None, st())
    c = lambda t: t.float().cpu()  # noqa: E731
    sel = list(range(0, rows, max(1, rows // 12)))
    routed, shared = _oracle_moe_parts(c(xn)[sel], ids[sel], c(w)[sel], c(gu), c(dn), c(sgu), c(sdn))
    assert rel_err(c(out)[sel], rb(c(res)[sel] + rb(routed + shared))) < 1e-2


def _mla_reference(q, cache_rows, lens, scale):
    """fp32 softmax(q . c^T * scale) . c[:, :512] per row (o_lat [B, 16, 512])."""
    outs = []
    for b, L in enumerate(lens):
        c = cache_rows[b][:L].float()
        s = (q[b].float() @ c.t()) * scale
        p = torch.softmax(s, dim=-1)
        outs.append(p @ c[:, :512])
    return torch.stack(outs)


@pytest.mark.parametrize("B,lo,hi,seed,split", [(1, 1, 40, 50, None), (3, 1, 300, 51, None), (16, 256, 8192, 3, None),
                                                (128, 256, 8192, 3, None), (128, 256, 8192, 3, "bench"),
                                                (2, 500, 1300, 52, 1056), (3, 40, 200, 53, 128), (4, 1, 97, 54, 96)])
def test_mla_decode_combine_vs_fp32(B, lo, hi, seed, split):
    """Split plan of the engine, the one bench.py's config 4 times ("bench": 640 target
    workgroups), or a fixed one: 33 tiles (odd) / 4 tiles (even, last one partial) / 3 tiles
    per split, so both register stages and the loop exits are covered."""
    from triton_kernels.attention_decode_batch import plan_splits

    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (B,), generator=g).tolist()
    cap = [L + 7 for L in lens]
    base = torch.tensor([0] + list(torch.cumsum(torch.tensor(cap), 0)[:-1].tolist()), dtype=torch.int64)
    cache = (torch.randn(sum(cap), 576, generator=g)).to(BF).to(DEV)
    q = torch.randn(B, 16, 576, generator=g).to(BF).to(DEV)
    pos = torch.tensor([L - 1 for L in lens], dtype=torch.int32, device=DEV)
    scale = O.softmax_scale(O.Dims())
    maxL = max(cap)
    if split is None:
        split, ns = plan_splits(B, maxL)
    elif split == "bench":  # bench.py sizes the plan by the longest row itself
        split, _ = plan_splits(B, max(lens), target_wgs=640)
        ns = math.ceil(maxL / split)
    else:
        ns = math.ceil(maxL / split)
    po = torch.empty(B, ns, 16, 512, device=DEV)
    pm = torch.empty(B, ns, 16, 2, device=DEV)
    base_d = base.to(DEV)  # keep device copies alive until the kernels have run
    cap_d = torch.tensor(cap, dtype=torch.int32, device=DEV)
    call("dsv2_mla_decode", q.data_ptr(), cache.data_ptr(), base_d.data_ptr(), pos.data_ptr(), cap_d.data_ptr(), B,
         split, ns, scale, po.data_ptr(), pm.data_ptr(), st())
    olat = torch.empty(B, 16, 512, dtype=BF, device=DEV)
    call("dsv2_mla_combine", po.data_ptr(), pm.data_ptr(), pos.data_ptr(), cap_d.data_ptr(), B, split, ns, None,
         olat.data_ptr(), 16 * 512, st())
    rows = [cache[int(base[b]):int(base[b]) + lens[b]] for b in range(B)]
    ref = _mla_reference(q, rows, lens, scale)
    assert rel_err(olat.float(), ref) < 1e-2
    # fused W_UV variant
    w_uv = rnd(16, 128, 512, std=0.05, seed=seed + 100)
    out = torch.empty(B, 2048, dtype=BF, device=DEV)
    call("dsv2_mla_combine", po.data_ptr(), pm.data_ptr(), pos.data_ptr(), cap_d.data_ptr(), B, split, ns,
         w_uv.data_ptr(), out.data_ptr(), 2048, st())
    ref2 = torch.einsum("hij,bhj->bhi", w_uv.float(), ref).reshape(B, 2048)
    assert rel_err(out.float(), ref2) < 1e-2


@pytest.mark.parametrize("B,lo,hi,seed", [(1, 1, 40, 70), (5, 1, 300, 71), (256, 2000, 2100, 72), (7, 900, 4200, 73)])
def test_mla_decode_rows_equals_one_split_pair(B, lo, hi, seed):
    """The one-launch decode (a workgroup per row, normalised bf16 o_lat) equals the split
    decode + combine with one split covering every row, bit for bit, and fp32 attention
    within 1e-2; a row of capacity 0 (nothing cached) gives zeros in both.  Lengths cover a
    single partial tile, odd and even tile counts and the bsz=256 shape; o_lat rows are
    written at a stride wider than 8192."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (B,), generator=g).tolist()
    cap = [L + 5 for L in lens]
    if B == 7:
        cap[3] = 0
    base = torch.tensor([0] + list(torch.cumsum(torch.tensor(cap), 0)[:-1].tolist()), dtype=torch.int64)
    cache = torch.randn(max(sum(cap), 1), 576, generator=g).to(BF).to(DEV)
    q = torch.randn(B, 16, 576, generator=g).to(BF).to(DEV)
    pos = torch.tensor([L - 1 for L in lens], dtype=torch.int32, device=DEV)
    scale = O.softmax_scale(O.Dims())
    base_d = base.to(DEV)
    cap_d = torch.tensor(cap, dtype=torch.int32, device=DEV)
    split = math.ceil(max(max(cap), 1) / 32) * 32
    po = torch.empty(B, 1, 16, 512, device=DEV)
    pm = torch.empty(B, 1, 16, 2, device=DEV)
    call("dsv2_mla_decode", q.data_ptr(), cache.data_ptr(), base_d.data_ptr(), pos.data_ptr(), cap_d.data_ptr(), B,
         split, 1, scale, po.data_ptr(), pm.data_ptr(), st())
    pair = torch.full((B, 16, 512), 7.0, dtype=BF, device=DEV)
    call("dsv2_mla_combine", po.data_ptr(), pm.data_ptr(), pos.data_ptr(), cap_d.data_ptr(), B, split, 1, None,
         pair.data_ptr(), 16 * 512, st())
    wide = torch.full((B, 16 * 512 + 64), 7.0, dtype=BF, device=DEV)
    call("dsv2_mla_decode_rows", q.data_ptr(), cache.data_ptr(), base_d.data_ptr(), pos.data_ptr(), cap_d.data_ptr(),
         B, scale, wide.data_ptr(), 16 * 512 + 64, st())
    torch.cuda.synchronize()
    one = wide[:, :16 * 512].reshape(B, 16, 512)
    assert torch.equal(one, pair)
    assert torch.all(wide[:, 16 * 512:] == 7.0)  # nothing past the row's 8192 outputs
    live = [b for b in range(B) if cap[b] > 0]
    rows = [cache[int(base[b]):int(base[b]) + min(lens[b], cap[b])] for b in live]
    ref = _mla_reference(q[live], rows, [min(lens[b], cap[b]) for b in live], scale)
    assert rel_err(one[live].float(), ref) < 1e-2
    for b in range(B):
        if cap[b] == 0:
            assert not one[b].float().any()


def test_mla_constant_cache_returns_value():
    # every cached row identical -> o_lat equals the latent regardless of q
    B, L = 2, 777
    row = torch.randn(576).to(BF)
    cache = row.repeat(B * 800, 1).to(DEV)
    base = torch.tensor([0, 800], dtype=torch.int64, device=DEV)
    pos = torch.tensor([L - 1, 31], dtype=torch.int32, device=DEV)
    q = rnd(B, 16, 576, seed=60)
    cap = torch.tensor([800, 800], dtype=torch.int32, device=DEV)
    po = torch.empty(B, 4, 16, 512, device=DEV)
    pm = torch.empty(B, 4, 16, 2, device=DEV)
    call("dsv2_mla_decode", q.data_ptr(), cache.data_ptr(), base.data_ptr(), pos.data_ptr(), cap.data_ptr(), B, 224, 4,
         0.1147, po.data_ptr(), pm.data_ptr(), st())
    olat = torch.empty(B, 16, 512, dtype=BF, device=DEV)
    call("dsv2_mla_combine", po.data_ptr(), pm.data_ptr(), pos.data_ptr(), cap.data_ptr(), B, 224, 4, None,
         olat.data_ptr(), 16 * 512, st())
    assert torch.allclose(olat.float().cpu(), row[:512].float().expand(B, 16, 512), rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("B", [5, 11])
def test_mla_prepare_vs_oracle(B):
    from dsv2lite.config import DSV2Config
    from dsv2lite.rope import cos_sin_tables

    cfg = DSV2Config()
    qkva = rnd(B, 3648, seed=70)
    kvw = (rnd(512, seed=71, std=0.1) + 1).to(BF)
    w_uk = rnd(16, 128, 512, std=0.05, seed=72)
    cos, sin = cos_sin_tables(cfg, 4096, device=DEV)
    pos = torch.tensor([0, 5, 127, 2048, 4000, 1, 2, 3, 4, 6, 7][:B], dtype=torch.int32, device=DEV)
    base = torch.tensor([0, 10, 200, 3000, 7000, 8000, 8100, 8200, 8300, 8400, 8500][:B], dtype=torch.int64,
                        device=DEV)
    cache = torch.zeros(12000, 576, dtype=BF, device=DEV)
    q = torch.zeros(B, 16, 576, dtype=BF, device=DEV)
    w_ukt = w_uk.transpose(1, 2).contiguous()
    cap = torch.full((B,), 4096, dtype=torch.int32, device=DEV)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    call("dsv2_mla_prepare", qkva.data_ptr(), 3648, B, pos.data_ptr(), base.data_ptr(), cap.data_ptr(), kvw.data_ptr(),
         1e-6, cos.data_ptr(), sin.data_ptr(), 4096, w_ukt.data_ptr(), cache.data_ptr(), q.data_ptr(),
         status.data_ptr(), st())
    assert status.item() == 0
    ocos, osin = O.yarn_cos_sin(O.Dims(), 4096, mode="bf16")
    assert torch.equal(cos.float().cpu(), ocos) and torch.equal(sin.float().cpu(), osin)
    x = qkva.float().cpu()
    p = pos.long().cpu()
    c_n = O.rmsnorm(x[:, 3072:3584], kvw.float().cpu(), 1e-6, rb)
    k_pe = O.rope_deinterleave(x[:, 3584:], ocos[p], osin[p], lambda t: t)
    q_pe = O.rope_deinterleave(x[:, :3072].view(B, 16, 192)[:, :, 128:], ocos[p][:, None], osin[p][:, None],
                               lambda t: t)
    rows = cache.float().cpu()[(base.cpu() + p)]
    assert rel_err(rows[:, :512], c_n) < 8e-3
    assert rel_err(rows[:, 512:], rb(k_pe)) < 8e-3
    assert rel_err(q.float().cpu()[:, :, 512:], rb(q_pe)) < 8e-3
    q_lat = torch.einsum("bhi,hij->bhj", x[:, :3072].view(B, 16, 192)[:, :, :128], w_uk.float().cpu())
    assert rel_err(q.float().cpu()[:, :, :512], q_lat) < 1e-2
    # untouched rows stay zero
    mask = torch.ones(12000, dtype=torch.bool)
    mask[(base.cpu() + p)] = False
    assert torch.all(cache.cpu()[mask] == 0)


@pytest.mark.parametrize("B", [1, 5, 64, 65, 300])
def test_mla_prepare_qlat_matches_two_launches(B):
    """The batch family's one-launch preparation equals, bit for bit, mla_prepare without
    absorption followed by the 16-group absorption GEMM it replaces (both token tiles: 16
    rows up to 64, 32 above), including a row whose position is past its capacity (skipped,
    status flagged) and positions past the RoPE table (clamped)."""
    from dsv2lite.config import DSV2Config
    from dsv2lite.rope import cos_sin_tables

    cfg = DSV2Config()
    qkva = rnd(B, 3648, seed=170)
    kvw = (rnd(512, seed=171, std=0.1) + 1).to(BF)
    w_ukt = rnd(16, 512, 128, std=0.05, seed=172)
    cos, sin = cos_sin_tables(cfg, 1024, device=DEV)
    g = torch.Generator().manual_seed(B)
    pos = torch.randint(0, 1200, (B,), generator=g, dtype=torch.int32)
    cap = torch.full((B,), 1300, dtype=torch.int32)
    cap[B // 2] = int(pos[B // 2])  # full row: skipped, flagged
    base = torch.arange(B, dtype=torch.int64) * 1300
    pos, cap, base = pos.to(DEV), cap.to(DEV), base.to(DEV)
    outs = []
    for fused in (False, True):
        cache = torch.zeros(B * 1300, 576, dtype=BF, device=DEV)
        q = torch.full((B, 16, 576), float("nan"), dtype=BF, device=DEV)
        status = torch.zeros(1, dtype=torch.int32, device=DEV)
        args = (qkva.data_ptr(), 3648, B, pos.data_ptr(), base.data_ptr(), cap.data_ptr(), kvw.data_ptr(), 1e-6,
                cos.data_ptr(), sin.data_ptr(), 1024)
        if fused:
            call("dsv2_mla_prepare_qlat", *args, w_ukt.data_ptr(), cache.data_ptr(), q.data_ptr(),
                 status.data_ptr(), st())
        else:
            call("dsv2_mla_prepare", *args, None, cache.data_ptr(), q.data_ptr(), status.data_ptr(), st())
            call("dsv2_gemm_bf16", qkva.data_ptr(), 3648, 192, B, 128, w_ukt.data_ptr(), 512 * 128, 512, 16, None, 0,
                 q.data_ptr(), 16 * 576, 576, 0, st())
        torch.cuda.synchronize()
        outs.append((cache, q, status.item()))
    (c0, q0, s0), (c1, q1, s1) = outs
    assert s0 == s1 and s0 != 0
    assert torch.equal(c0, c1)
    assert not torch.isnan(q1.float()).any()
    assert torch.equal(q0.view(torch.int16), q1.view(torch.int16))


def test_argmax_first_max_and_position_step():
    lg = torch.randn(3, 102400, device=DEV)
    lg[1, 777] = 50.0
    lg[1, 99999] = 50.0  # tie -> lower index
    ids = torch.empty(3, dtype=torch.int64, device=DEV)
    pos = torch.tensor([4, 5, 6], dtype=torch.int32, device=DEV)
    call("dsv2_argmax_f32", lg.data_ptr(), 3, 102400, ids.data_ptr(), pos.data_ptr(), st())
    assert torch.equal(ids.cpu(), torch.argmax(lg.cpu(), -1))
    assert ids[1].item() == 777
    assert pos.tolist() == [5, 6, 7]


def test_embed_gather_and_api_errors():
    table = rnd(100, 2048, seed=80)
    ids = torch.tensor([3, 99, 0], device=DEV)
    out = torch.empty(3, 2048, dtype=BF, device=DEV)
    call("dsv2_embed_gather_bf16", ids.data_ptr(), table.data_ptr(), 2048, out.data_ptr(), 3, st())
    assert torch.equal(out, table[ids])
    with pytest.raises(_hip.HipKernelError, match="multiple of 8"):
        call("dsv2_residual_add_bf16", table.data_ptr(), table.data_ptr(), out.data_ptr(), 13, st())
    with pytest.raises(_hip.HipKernelError, match="K%64"):
        call("dsv2_gemm_bf16", table.data_ptr(), 2048, 0, 3, 2000, table.data_ptr(), 0, 64, 1, None, 0,
             out.data_ptr(), 2048, 0, 0, st())


@pytest.mark.parametrize("lens", [[1], [231], [40, 7, 300]])
def test_mla_fused_small_family_vs_fp32(lens):
    from dsv2lite.config import DSV2Config
    from dsv2lite.rope import cos_sin_tables

    cfg = DSV2Config()
    B = len(lens)
    g = torch.Generator().manual_seed(sum(lens))
    cap = [L + 5 for L in lens]
    base = torch.tensor([0] + list(torch.cumsum(torch.tensor(cap), 0)[:-1].tolist()), dtype=torch.int64)
    cache = (torch.randn(sum(cap), 576, generator=g) * 0.5).to(BF).to(DEV)
    pos = torch.tensor([L - 1 for L in lens], dtype=torch.int32)  # new token at position L-1
    qkva = rnd(B, 3648, seed=90)
    kvw = (rnd(512, seed=91, std=0.1) + 1).to(BF)
    w_uk = rnd(16, 128, 512, std=0.05, seed=92)
    w_uv = rnd(16, 128, 512, std=0.05, seed=93)
    cos, sin = cos_sin_tables(cfg, 512, device=DEV)
    out = torch.empty(B, 2048, dtype=BF, device=DEV)
    before = cache.clone()
    scale = cfg.softmax_scale
    pos_d, base_d, w_ukt = pos.to(DEV), base.to(DEV), w_uk.transpose(1, 2).contiguous()  # alive across the launch
    cap_d = torch.tensor(cap, dtype=torch.int32, device=DEV)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    call("dsv2_mla_fused", qkva.data_ptr(), 3648, B, pos_d.data_ptr(), base_d.data_ptr(), cap_d.data_ptr(),
         kvw.data_ptr(), 1e-6, cos.data_ptr(), sin.data_ptr(), 512, w_ukt.data_ptr(), w_uv.data_ptr(),
         cache.data_ptr(), scale, out.data_ptr(), 2048, status.data_ptr(), st())
    assert status.item() == 0
    # reference: same prepare math (oracle pieces), fp32 attention over the updated rows
    x = qkva.float().cpu()
    ocos, osin = O.yarn_cos_sin(O.Dims(), 512, mode="bf16")
    p = pos.long()
    c_n = O.rmsnorm(x[:, 3072:3584], kvw.float().cpu(), 1e-6, rb)
    k_pe = rb(O.rope_deinterleave(x[:, 3584:], ocos[p], osin[p], lambda t: t))
    new_rows = torch.cat([c_n, k_pe], -1)
    slots = base + p
    got_rows = cache.float().cpu()[slots]
    assert rel_err(got_rows, new_rows) < 8e-3
    mask = torch.ones(cache.shape[0], dtype=torch.bool)
    mask[slots] = False
    assert torch.equal(cache.cpu()[mask], before.cpu()[mask])  # nothing else written
    q_pe = rb(O.rope_deinterleave(x[:, :3072].view(B, 16, 192)[:, :, 128:], ocos[p][:, None], osin[p][:, None],
                                  lambda t: t))
    q_lat = rb(torch.einsum("bhi,hij->bhj", x[:, :3072].view(B, 16, 192)[:, :, :128], w_uk.float().cpu()))
    q_full = torch.cat([q_lat, q_pe], -1)
    rows = [cache.float().cpu()[int(base[b]):int(base[b]) + lens[b]] for b in range(B)]
    olat = _mla_reference(q_full, rows, lens, scale)
    ref = torch.einsum("hij,bhj->bhi", w_uv.float().cpu(), olat).reshape(B, 2048)
    assert rel_err(out.float().cpu(), ref) < 1e-2


@pytest.mark.parametrize("lens", [[1], [2, 3], [231], [40, 7, 300], [700]])
def test_mla_attend_matches_fused_and_fp32(lens):
    """prepare (absorption) + the spread attend kernel against the fused kernel on the same
    inputs (same cache rows written, outputs within 1e-2) and the fp32 reference, at two
    consecutive positions; the two-launch entry point equals the two calls bit for bit."""
    from dsv2lite.config import DSV2Config
    from dsv2lite.rope import cos_sin_tables

    cfg = DSV2Config()
    B = len(lens)
    g = torch.Generator().manual_seed(7 * sum(lens))
    cap = [L + 5 for L in lens]
    base = torch.tensor([0] + list(torch.cumsum(torch.tensor(cap), 0)[:-1].tolist()), dtype=torch.int64)
    cache0 = (torch.randn(sum(cap), 576, generator=g) * 0.5).to(BF).to(DEV)
    qkva = rnd(B, 3648, seed=190)
    kvw = (rnd(512, seed=191, std=0.1) + 1).to(BF)
    w_uk = rnd(16, 128, 512, std=0.05, seed=192)
    w_uv = rnd(16, 128, 512, std=0.05, seed=193)
    w_ukt = w_uk.transpose(1, 2).contiguous()
    cos, sin = cos_sin_tables(cfg, 1024, device=DEV)
    scale = cfg.softmax_scale
    base_d = base.to(DEV)
    cap_d = torch.tensor(cap, dtype=torch.int32, device=DEV)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    q = torch.empty(B, 16, 576, dtype=BF, device=DEV)
    for step in range(2):
        pos = torch.tensor([L - 1 + step for L in lens], dtype=torch.int32)
        pos_d = pos.to(DEV)
        c_f, c_s = cache0.clone(), cache0.clone()
        out_f = torch.empty(B, 2048, dtype=BF, device=DEV)
        out_s = torch.empty(B, 2048, dtype=BF, device=DEV)
        call("dsv2_mla_fused", qkva.data_ptr(), 3648, B, pos_d.data_ptr(), base_d.data_ptr(), cap_d.data_ptr(),
             kvw.data_ptr(), 1e-6, cos.data_ptr(), sin.data_ptr(), 1024, w_ukt.data_ptr(), w_uv.data_ptr(),
             c_f.data_ptr(), scale, out_f.data_ptr(), 2048, status.data_ptr(), st())
        call("dsv2_mla_prepare", qkva.data_ptr(), 3648, B, pos_d.data_ptr(), base_d.data_ptr(), cap_d.data_ptr(),
             kvw.data_ptr(), 1e-6, cos.data_ptr(), sin.data_ptr(), 1024, w_ukt.data_ptr(), c_s.data_ptr(),
             q.data_ptr(), status.data_ptr(), st())
        call("dsv2_mla_attend", q.data_ptr(), c_s.data_ptr(), base_d.data_ptr(), pos_d.data_ptr(), cap_d.data_ptr(),
             B, w_uv.data_ptr(), scale, out_s.data_ptr(), 2048, st())
        torch.cuda.synchronize()
        assert status.item() == 0
        assert torch.equal(c_f, c_s), step  # the same new rows, nothing else written
        # the attend kernel rounds the softmax weights to bf16 before p.v (as the reference
        # does), the fused kernel keeps them in fp32: both within 1e-2 of fp32 math
        assert rel_err(out_s.float().cpu(), out_f.float().cpu()) < 1e-2, step
        q_full = q.float().cpu()
        n = [L + step for L in lens]
        rows = [c_s.float().cpu()[int(base[b]):int(base[b]) + n[b]] for b in range(B)]
        olat = _mla_reference(q_full, rows, n, scale)
        ref = torch.einsum("hij,bhj->bhi", w_uv.float().cpu(), olat).reshape(B, 2048)
        assert rel_err(out_s.float().cpu(), ref) < 1e-2, step
        # the two-launch entry point: identical cache rows and output
        c_2, out_2, q2 = cache0.clone(), torch.empty_like(out_s), torch.empty_like(q)
        call("dsv2_mla_spread", qkva.data_ptr(), 3648, B, pos_d.data_ptr(), base_d.data_ptr(), cap_d.data_ptr(),
             kvw.data_ptr(), 1e-6, cos.data_ptr(), sin.data_ptr(), 1024, w_ukt.data_ptr(), w_uv.data_ptr(),
             c_2.data_ptr(), q2.data_ptr(), scale, out_2.data_ptr(), 2048, status.data_ptr(), st())
        torch.cuda.synchronize()
        assert torch.equal(c_2, c_s) and torch.equal(q2, q) and torch.equal(out_2, out_s), step


@pytest.mark.parametrize("lens", [[1], [2, 3], [231], [40, 7, 300], [700]])
def test_qkva_absorb_and_attend_parts(lens):
    """The q|kv_a projection with the absorption split over its workgroups: its projection is
    the few-row GEMV's bit for bit, the partial absorbed queries sum to W_UK^T q_nope (fp32),
    and the attention from them writes the fused kernel's cache rows and agrees with it and
    with fp32 math, at two consecutive positions."""
    from dsv2lite.config import DSV2Config
    from dsv2lite.rope import cos_sin_tables

    cfg = DSV2Config()
    B = len(lens)
    g = torch.Generator().manual_seed(11 * sum(lens))
    cap = [L + 5 for L in lens]
    base = torch.tensor([0] + list(torch.cumsum(torch.tensor(cap), 0)[:-1].tolist()), dtype=torch.int64)
    cache0 = (torch.randn(sum(cap), 576, generator=g) * 0.5).to(BF).to(DEV)
    h = rnd(B, 2048, seed=290)
    ln = (rnd(2048, seed=291, std=0.1) + 1).to(BF)
    w_qkva = rnd(3648, 2048, std=0.02, seed=292)
    kvw = (rnd(512, seed=293, std=0.1) + 1).to(BF)
    w_uk = rnd(16, 128, 512, std=0.05, seed=294)
    w_uv = rnd(16, 128, 512, std=0.05, seed=295)
    w_ukt = w_uk.transpose(1, 2).contiguous()
    cos, sin = cos_sin_tables(cfg, 1024, device=DEV)
    scale = cfg.softmax_scale
    base_d = base.to(DEV)
    cap_d = torch.tensor(cap, dtype=torch.int32, device=DEV)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    ref_qkva = torch.empty(B, 3648, dtype=BF, device=DEV)
    call("dsv2_gemv_bf16", h.data_ptr(), 2048, B, 2048, w_qkva.data_ptr(), 3648, ln.data_ptr(), 1e-6, None, 0,
         ref_qkva.data_ptr(), 3648, 0, st())
    for step in range(2):
        pos_d = torch.tensor([L - 1 + step for L in lens], dtype=torch.int32, device=DEV)
        qkva = torch.full((B, 3648), float("nan"), dtype=BF, device=DEV)
        parts = torch.full((B, 16, 8, 512), float("nan"), dtype=torch.float32, device=DEV)
        c_p, c_f = cache0.clone(), cache0.clone()
        call("dsv2_qkva_absorb_bf16", h.data_ptr(), 2048, B, w_qkva.data_ptr(), ln.data_ptr(), 1e-6,
             w_uk.data_ptr(), qkva.data_ptr(), 3648, parts.data_ptr(), c_p.data_ptr(), base_d.data_ptr(),
             pos_d.data_ptr(), cap_d.data_ptr(), st())
        torch.cuda.synchronize()
        assert torch.equal(qkva, ref_qkva), step
        q_nope = qkva.float().cpu()[:, :3072].view(B, 16, 192)[:, :, :128]
        want = torch.einsum("bhd,hdc->bhc", q_nope.double(), w_uk.double().cpu())
        got = parts.double().cpu().sum(2)
        assert (got - want).abs().max() <= 1e-5 * want.abs().max(), step
        out_p = torch.empty(B, 2048, dtype=BF, device=DEV)
        out_f = torch.empty(B, 2048, dtype=BF, device=DEV)
        call("dsv2_mla_attend_parts", qkva.data_ptr(), 3648, B, pos_d.data_ptr(), base_d.data_ptr(),
             cap_d.data_ptr(), kvw.data_ptr(), 1e-6, cos.data_ptr(), sin.data_ptr(), 1024, parts.data_ptr(),
             w_uv.data_ptr(), c_p.data_ptr(), scale, out_p.data_ptr(), 2048, status.data_ptr(), st())
        call("dsv2_mla_fused", qkva.data_ptr(), 3648, B, pos_d.data_ptr(), base_d.data_ptr(), cap_d.data_ptr(),
             kvw.data_ptr(), 1e-6, cos.data_ptr(), sin.data_ptr(), 1024, w_ukt.data_ptr(), w_uv.data_ptr(),
             c_f.data_ptr(), scale, out_f.data_ptr(), 2048, status.data_ptr(), st())
        torch.cuda.synchronize()
        assert status.item() == 0
        assert torch.equal(c_p, c_f), step  # the same new rows, nothing else written
        assert rel_err(out_p.float().cpu(), out_f.float().cpu()) < 1e-2, step
        # fp32 attention from the absorbed query the kernel forms (bf16 of the partial sum)
        ocos, osin = O.yarn_cos_sin(O.Dims(), 1024, mode="bf16")
        p = pos_d.cpu().long()
        x = qkva.float().cpu()
        q_pe = rb(O.rope_deinterleave(x[:, :3072].view(B, 16, 192)[:, :, 128:], ocos[p][:, None], osin[p][:, None],
                                      lambda t: t))
        q_full = torch.cat([rb(got.float()), q_pe], -1)
        n = [L + step for L in lens]
        rows = [c_p.float().cpu()[int(base[b]):int(base[b]) + n[b]] for b in range(B)]
        olat = _mla_reference(q_full, rows, n, scale)
        ref = torch.einsum("hij,bhj->bhi", w_uv.float().cpu(), olat).reshape(B, 2048)
        assert rel_err(out_p.float().cpu(), ref) < 1e-2, step


@pytest.mark.parametrize("rows", [1, 3])
def test_router_logits_split_and_gateup_topk(rows):
    h, nw, wr = _router_case(rows, 95)
    xn = torch.empty_like(h)
    lg = torch.empty(rows, 64, dtype=torch.float32, device=DEV)
    call("dsv2_router_logits", h.data_ptr(), 2048, nw.data_ptr(), 1e-6, wr.data_ptr(), rows, xn.data_ptr(),
         lg.data_ptr(), st())
    xr = O.rmsnorm(h.float().cpu(), nw.float().cpu(), 1e-6, rb)
    assert rel_err(xn.float().cpu(), xr) < 8e-3
    ref_lg = xn.float().cpu() @ wr.float().cpu().t()
    assert torch.allclose(lg.cpu(), ref_lg, rtol=1e-5, atol=1e-5)
    gu, dn, sgu, sdn = _moe_layer(96)
    ids = torch.full((rows, 6), -1, dtype=torch.int32, device=DEV)
    w = torch.empty(rows, 6, dtype=torch.float32, device=DEV)
    hb = torch.empty(rows, 8, 1408, dtype=BF, device=DEV)
    call("dsv2_moe_route_gateup_logits", xn.data_ptr(), rows, lg.data_ptr(), 1.0, ids.data_ptr(), w.data_ptr(),
         gu.data_ptr(), sgu.data_ptr(), 1408, hb.data_ptr(), st())
    oid, ow, _ = O.router_topk(xn.float().cpu(), wr.float().cpu(), 6, 1.0)
    from_lg = torch.softmax(lg.cpu(), -1)
    ref_ids = torch.stack([torch.tensor(sorted(range(64), key=lambda e: (-float(from_lg[r, e]), e))[:6])
                           for r in range(rows)])
    assert torch.equal(ids.cpu().long(), ref_ids)
    assert torch.allclose(w.cpu(), from_lg.gather(1, ref_ids), rtol=1e-5)
    hb2 = torch.empty_like(hb)
    call("dsv2_moe_route_gateup", xn.data_ptr(), rows, ids.data_ptr(), gu.data_ptr(), sgu.data_ptr(), 1408,
         hb2.data_ptr(), st())
    assert torch.equal(hb, hb2)


def test_route_gateup_logits_exact_ties():
    """Planted exact ties inside the top-6 (rank 0/1 and rank 3/4) and at the rank-5/6 edge:
    every routed slot must take the lower index first, in the published ids and in the
    expert each gate_up workgroup streams (compared with the ids-driven entry point)."""
    rows = 2
    g = torch.Generator().manual_seed(321)
    lg = torch.randn(rows, 64, generator=g).float()
    lg[0, 40] = lg[0, 9] = 9.0          # ranks 0 and 1: 9 before 40
    lg[0, 50] = lg[0, 2] = 5.0          # ranks 3 and 4 (after 3 larger ones below)
    lg[0, 33] = 7.0
    lg[1, 63] = lg[1, 0] = lg[1, 31] = 4.0  # a three-way tie across the rank-5/6 edge
    lg[1, 1:6] = torch.tensor([8.0, 7.5, 7.0, 6.5, 6.0])
    lg = lg.to(DEV)
    xn = rnd(rows, 2048, seed=322)
    gu, _, sgu, _ = _moe_layer(323)
    ids = torch.full((rows, 6), -1, dtype=torch.int32, device=DEV)
    w = torch.empty(rows, 6, dtype=torch.float32, device=DEV)
    hb = torch.empty(rows, 8, 1408, dtype=BF, device=DEV)
    call("dsv2_moe_route_gateup_logits", xn.data_ptr(), rows, lg.data_ptr(), 1.0, ids.data_ptr(), w.data_ptr(),
         gu.data_ptr(), sgu.data_ptr(), 1408, hb.data_ptr(), st())
    lc = lg.cpu()
    ref_ids = torch.stack([torch.tensor(sorted(range(64), key=lambda e: (-float(lc[r, e]), e))[:6]) for r in range(rows)])
    assert ref_ids[0, :2].tolist() == [9, 40] and ref_ids[1, 5].item() == 0
    assert torch.equal(ids.cpu().long(), ref_ids)
    hb2 = torch.empty_like(hb)
    call("dsv2_moe_route_gateup", xn.data_ptr(), rows, ids.data_ptr(), gu.data_ptr(), sgu.data_ptr(), 1408,
         hb2.data_ptr(), st())
    assert torch.equal(hb, hb2)


@pytest.mark.parametrize("rows", [1, 2, 5])
def test_lm_head_argmax_matches_gemv_then_argmax(rows):
    x = rnd(rows, 2048, seed=99)
    W = rnd(102400, 2048, std=0.02, seed=100)
    nw = rnd(2048, seed=101, std=0.1) + 1.0
    W[77] = W[4000]  # a planted tie between two vocabulary rows: the lower index must win
    lg = torch.empty(rows, 102400, dtype=torch.float32, device=DEV)
    ids = torch.empty(rows, dtype=torch.int64, device=DEV)
    pos = torch.arange(rows, dtype=torch.int32, device=DEV)
    part = torch.empty(_hip.lib.dsv2_lm_head_argmax_workspace_size(rows), dtype=torch.uint8, device=DEV)
    call("dsv2_lm_head_argmax_bf16", x.data_ptr(), 2048, rows, W.data_ptr(), 102400, nw.data_ptr(), 1e-6,
         lg.data_ptr(), part.data_ptr(), part.numel(), ids.data_ptr(), pos.data_ptr(), st())
    lg2 = torch.empty_like(lg)
    call("dsv2_gemv_bf16", x.data_ptr(), 2048, rows, 2048, W.data_ptr(), 102400, nw.data_ptr(), 1e-6, None, 0,
         lg2.data_ptr(), 102400, LINEAR_OUT_F32, st())
    assert torch.equal(lg, lg2)
    assert torch.equal(ids.cpu(), torch.argmax(lg.cpu(), -1))  # torch: first index of the maximum
    assert pos.tolist() == list(range(1, rows + 1))
    # force the tie to be the maximum of row 0 and check the lower index is returned
    x0 = torch.zeros(rows, 2048, dtype=BF, device=DEV)
    x0[:, :] = W[77].float().sign().to(BF)
    call("dsv2_lm_head_argmax_bf16", x0.data_ptr(), 2048, rows, W.data_ptr(), 102400, nw.data_ptr(), 1e-6,
         lg.data_ptr(), part.data_ptr(), part.numel(), ids.data_ptr(), None, st())
    assert torch.equal(ids.cpu(), torch.argmax(lg.cpu(), -1))
    with pytest.raises(_hip.HipKernelError, match="rows"):
        call("dsv2_lm_head_argmax_bf16", x.data_ptr(), 2048, 9, W.data_ptr(), 102400, nw.data_ptr(), 1e-6,
             lg.data_ptr(), part.data_ptr(), part.numel(), ids.data_ptr(), None, st())


@pytest.mark.parametrize("lens,start", [([70, 150], 0), ([300, 5, 129], 40)])
def test_mla_prefill_attention_vs_fp32(lens, start):
    """Prefill attention (expanded form, causal) against fp32 torch: rows of several
    sequences (a chunk that may start inside the first sequence: its earlier keys come from
    the cache), 128-query tiles with partial last tiles."""
    from dsv2lite.engine import prefill_tiles

    caps = [n + 30 for n in lens]
    bases = [0]
    for cp in caps[:-1]:
        bases.append(bases[-1] + cp)
    ncache = bases[-1] + caps[-1]
    seq = torch.cat([torch.full((n,), b, dtype=torch.int64) for b, n in enumerate(lens)])[start:]
    posv = torch.cat([torch.arange(n, dtype=torch.int32) for n in lens])[start:]
    R = seq.numel()
    tiles, lo, nexp = prefill_tiles(seq, posv, bases)
    cache = rnd(ncache, 576, seed=200)
    kexp = rnd(nexp, 16, 128, seed=201)
    vexp = rnd(nexp, 16, 128, seed=202)
    qkva = rnd(R, 3648, seed=203)
    qrope = rnd(R, 16, 576, seed=204)
    out = torch.full((R, 2048), float("nan"), dtype=BF, device=DEV)
    scale = O.softmax_scale(O.Dims())
    td = tiles.to(DEV)
    call("dsv2_mla_prefill_attention", qkva.data_ptr(), 3648, qrope.data_ptr(), 16 * 576, R, cache.data_ptr(), ncache,
         kexp.data_ptr(), vexp.data_ptr(), lo, nexp, td.data_ptr(), td.shape[0], scale, out.data_ptr(), 2048, st())
    c = lambda t: t.float().cpu()  # noqa: E731
    cc, ke, ve, qa, qr = c(cache), c(kexp), c(vexp), c(qkva), c(qrope)
    ref = torch.empty(R, 16, 128)
    for r in range(R):
        b, p = int(seq[r]), int(posv[r])
        rows = torch.arange(bases[b], bases[b] + p + 1)
        q = torch.cat([qa[r, :3072].view(16, 192)[:, :128], qr[r, :, 512:]], -1)  # [16, 192]
        k = torch.cat([ke[rows - lo], cc[rows, 512:][:, None, :].expand(-1, 16, -1)], -1)  # [n, 16, 192]
        s = torch.einsum("hd,nhd->hn", q, k) * scale
        ref[r] = torch.einsum("hn,nhd->hd", torch.softmax(s, -1), ve[rows - lo])
    assert torch.isfinite(c(out)).all()
    assert rel_err(c(out).view(R, 16, 128), ref) < 1e-2


@pytest.mark.parametrize("nbytes", [16, 4096 * 16 + 48, 64 * 2**20 + 16])
def test_stream_copy_exact(nbytes):
    """dsv2_stream_copy (the copy the benchmark measures its copy bandwidth with) moves every
    byte and nothing past the end, also for sizes that are not a multiple of its 16 KB pass."""
    g = torch.Generator(device=DEV).manual_seed(nbytes % 1000)
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=DEV, generator=g)
    dst = torch.full((nbytes + 64,), 7, dtype=torch.uint8, device=DEV)
    call("dsv2_stream_copy", src.data_ptr(), dst.data_ptr(), nbytes, st())
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src)
    assert torch.all(dst[nbytes:] == 7)
