"""FP8 (OCP e4m3) expert weights on the GPU: the small-family route kernels and the decode
engine with the routed and shared expert weights in e4m3 and one power-of-two fp32 scale
per output row.

The reference has bf16 weights only, so the bar is set here:
- the kernels' e4m3 decoding is exact: with a one-hot input the down kernel returns a
  column of the dequantized matrix (e4m3 value x scale) bit-for-bit against torch's
  float8_e4m3fn conversion, over all 254 finite codes, and the gate_up kernel returns
  what the bf16 kernel returns on the dequantized weights, bit-for-bit;
- on random inputs both kernels are within 1e-2 (max-rel) of the bf16 kernels on the
  dequantized weights and of the fp32 oracle;
- the engine with fp8 experts meets the bf16 engine's bars (hidden states and logits
  2e-2 / 3e-2, router ids, greedy tokens) against the oracle run on the dequantized
  weights: quantization changes the model, not the parity of the step computing it.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from triton_kernels._hip import call, stream_ptr

import oracle.dsv2_oracle as O
from engine_common import agree as _agree
from engine_common import build_model
from engine_common import check_trace as _check_trace
from engine_common import close as _close
from engine_common import oracle_step as _oracle_step
from engine_common import prompts as _prompts
from golden_utils import rel_err

DEV = "cuda"
BF = torch.bfloat16
I, H = 1408, 2048


def rnd(*shape, std=1.0, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=DEV) * std).to(BF)


def _q(w):
    from dsv2lite.weights import dequantize_rows_fp8, quantize_rows_fp8

    q, s = quantize_rows_fp8(w)
    return q.contiguous(), s.contiguous(), dequantize_rows_fp8(q, s)


def _finite_codes(n, seed):
    """n random e4m3 bytes (on the GPU) with the two NaN codes (0x7f, 0xff) replaced by zero."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    b = torch.randint(0, 256, (n,), generator=g, dtype=torch.uint8, device=DEV)
    return b.masked_fill_((b & 0x7F) == 0x7F, 0)


def test_fp8_down_decodes_every_code_exactly():
    rows = 2
    cols = (5, 1400)  # one in each lane chunk range of the down kernel
    g = torch.Generator().manual_seed(901)
    ids = torch.stack([torch.randperm(64, generator=g)[:6] for _ in range(rows)]).to(torch.int32).to(DEV)
    dn8 = torch.zeros(64, H, I, dtype=torch.uint8, device=DEV)
    codes = torch.arange(256, dtype=torch.int32)
    codes[(codes & 0x7F) == 0x7F] = 0
    codes = codes.to(torch.uint8)
    for b in range(rows):
        e = int(ids[b, 0])
        col = torch.cat([codes] * (H // 256))  # every code 8 times down the column
        dn8[e, :, cols[b]] = col.roll(37 * b).to(DEV)
    # row scales: powers of two over a wide range (2^-20 .. 2^4)
    sdn = torch.ldexp(torch.ones(64, H), torch.randint(-20, 5, (64, H), generator=g)).to(DEV)
    hbuf = torch.zeros(rows, 6, I, dtype=BF, device=DEV)
    for b in range(rows):
        hbuf[b, 0, cols[b]] = 1.0
    wts = torch.zeros(rows, 6, dtype=torch.float32, device=DEV)
    wts[:, 0] = 1.0
    out = torch.empty(rows, H, dtype=BF, device=DEV)
    call("dsv2_moe_route_down_fp8", hbuf.data_ptr(), rows, ids.data_ptr(), wts.data_ptr(), dn8.data_ptr(),
         sdn.data_ptr(), None, None, I, 6, None, out.data_ptr(), stream_ptr())
    torch.cuda.synchronize()
    for b in range(rows):
        e = int(ids[b, 0])
        ref = (dn8[e, :, cols[b]].view(torch.float8_e4m3fn).float() * sdn[e]).to(BF)
        assert torch.equal(out[b], ref), b


def test_fp8_gateup_equals_bf16_on_dequantized_one_hot():
    rows = 3
    gu8 = _finite_codes(64 * 2 * I * H, 902).view(64, 2 * I, H)
    g = torch.Generator().manual_seed(903)
    sgu = torch.ldexp(torch.ones(64, 2 * I), torch.randint(-12, -6, (64, 2 * I), generator=g)).to(DEV)
    sh8 = _finite_codes(4 * I * H, 904).view(4 * I, H)
    ssh = torch.ldexp(torch.ones(4 * I), torch.randint(-12, -6, (4 * I,), generator=g)).to(DEV)
    gu = (gu8.view(torch.float8_e4m3fn).float() * sgu.unsqueeze(-1)).to(BF)
    sh = (sh8.view(torch.float8_e4m3fn).float() * ssh.unsqueeze(-1)).to(BF)
    xn = torch.zeros(rows, H, dtype=BF, device=DEV)
    for b, k in enumerate((3, 1111, 2047)):
        xn[b, k] = 1.0
    lg = torch.randn(rows, 64, generator=g).to(DEV)
    ids = torch.empty(rows, 6, dtype=torch.int32, device=DEV)
    wts = torch.empty(rows, 6, dtype=torch.float32, device=DEV)
    hb8 = torch.empty(rows, 8, I, dtype=BF, device=DEV)
    call("dsv2_moe_route_gateup_logits_fp8", xn.data_ptr(), rows, lg.data_ptr(), 1.0, ids.data_ptr(),
         wts.data_ptr(), gu8.data_ptr(), sgu.data_ptr(), sh8.data_ptr(), ssh.data_ptr(), I, hb8.data_ptr(),
         stream_ptr())
    hb = torch.empty_like(hb8)
    call("dsv2_moe_route_gateup", xn.data_ptr(), rows, ids.data_ptr(), gu.data_ptr(), sh.data_ptr(), I,
         hb.data_ptr(), stream_ptr())
    torch.cuda.synchronize()
    assert torch.equal(hb8, hb)
    assert hb.float().abs().amax() > 0


@pytest.mark.parametrize("rows", [1, 4])
def test_fp8_route_kernels_vs_bf16_and_oracle(rows):
    gu = rnd(64, 2 * I, H, std=0.02, seed=910)
    dn = rnd(64, H, I, std=0.02, seed=911)
    sgu = rnd(4 * I, H, std=0.02, seed=912)
    sdn = rnd(H, 2 * I, std=0.02, seed=913)
    gu8, gus, gud = _q(gu)
    dn8, dns, dnd = _q(dn)
    sg8, sgs, sgd = _q(sgu)
    sd8, sds, sdd = _q(sdn)
    xn = rnd(rows, H, seed=914)
    lg = rnd(rows, 64, seed=915).float()
    h = rnd(rows, H, seed=916)
    ids = torch.empty(rows, 6, dtype=torch.int32, device=DEV)
    wts = torch.empty(rows, 6, dtype=torch.float32, device=DEV)
    hb8 = torch.empty(rows, 8, I, dtype=BF, device=DEV)
    hb = torch.empty_like(hb8)
    call("dsv2_moe_route_gateup_logits_fp8", xn.data_ptr(), rows, lg.data_ptr(), 1.0, ids.data_ptr(),
         wts.data_ptr(), gu8.data_ptr(), gus.data_ptr(), sg8.data_ptr(), sgs.data_ptr(), I, hb8.data_ptr(),
         stream_ptr())
    call("dsv2_moe_route_gateup", xn.data_ptr(), rows, ids.data_ptr(), gud.data_ptr(), sgd.data_ptr(), I,
         hb.data_ptr(), stream_ptr())
    out8 = torch.empty_like(h)
    out = torch.empty_like(h)
    call("dsv2_moe_route_down_fp8", hb8.data_ptr(), rows, ids.data_ptr(), wts.data_ptr(), dn8.data_ptr(),
         dns.data_ptr(), sd8.data_ptr(), sds.data_ptr(), I, 8, h.data_ptr(), out8.data_ptr(), stream_ptr())
    call("dsv2_moe_route_down", hb8.data_ptr(), rows, ids.data_ptr(), wts.data_ptr(), dnd.data_ptr(), sdd.data_ptr(),
         I, 8, None, h.data_ptr(), out.data_ptr(), stream_ptr())
    torch.cuda.synchronize()
    c = lambda t: t.float().cpu()  # noqa: E731
    # gate_up: the same products in another summation order -> at most bf16 rounding flips
    assert rel_err(c(hb8), c(hb)) < 1e-2
    assert (hb8 == hb).float().mean() > 0.9
    assert rel_err(c(out8), c(out)) < 1e-2
    # against the fp32-summing oracle on the dequantized weights
    rb = lambda t: t.to(BF).float()  # noqa: E731
    xc, idc, wc = c(xn), ids.cpu(), wts.cpu()
    routed = torch.zeros(rows, H)
    for s in range(6):
        part = torch.stack([O.mlp(xc[t:t + 1], c(gud[int(idc[t, s]), :I]), c(gud[int(idc[t, s]), I:]),
                                  c(dnd[int(idc[t, s])]), rb)[0] for t in range(rows)])
        routed = routed + wc[:, s:s + 1] * part
    shared = O.mlp(xc, c(sgd[:2 * I]), c(sgd[2 * I:]), c(sdd), rb)
    ref = rb(c(h) + rb(rb(routed) + shared))
    assert rel_err(c(out8), ref) < 1e-2


def _bucket(ids, tt):
    rows = ids.shape[0]
    R = rows * 6
    max_tiles = -(-R // tt) + 64
    srt = torch.empty(R, dtype=torch.int32, device=DEV)
    rpos = torch.empty(R, dtype=torch.int32, device=DEV)
    tiles = torch.empty(max_tiles, 4, dtype=torch.int32, device=DEV)
    nt = torch.empty(1, dtype=torch.int32, device=DEV)
    call("dsv2_moe_bucket", ids.to(torch.int32).to(DEV).data_ptr(), rows, tt, srt.data_ptr(), rpos.data_ptr(),
         tiles.data_ptr(), nt.data_ptr(), stream_ptr())
    return srt, rpos, tiles, nt, max_tiles


def _grouped(xn, ids, tt, gu, sgu, dn, sdn, q=None):
    """The grouped gate_up + down with the shared halves: bf16 launches, or with q = (gu8, gus,
    sg8, sgs, dn8, dns, sd8, sds) the e4m3 ones.  Returns (hs, shared_mid, ys, shared_parts)."""
    rows = xn.shape[0]
    R = rows * 6
    srt, rpos, tiles, nt, mt = _bucket(ids, tt)
    hs = torch.empty(R, I, dtype=BF, device=DEV)
    sh = torch.empty(rows, 2 * I, dtype=BF, device=DEV)
    ys = torch.empty(R, H, dtype=BF, device=DEV)
    parts = torch.empty(2, rows, H, dtype=torch.float32, device=DEV)
    if q is None:
        call("dsv2_moe_grouped_gateup_shared", xn.data_ptr(), rows, srt.data_ptr(), tiles.data_ptr(), nt.data_ptr(), mt,
             tt, gu.data_ptr(), sgu.data_ptr(), I, hs.data_ptr(), sh.data_ptr(), stream_ptr())
        call("dsv2_moe_grouped_down_shared", hs.data_ptr(), rows, tiles.data_ptr(), nt.data_ptr(), mt, tt,
             dn.data_ptr(), sh.data_ptr(), sdn.data_ptr(), I, ys.data_ptr(), parts.data_ptr(), stream_ptr())
    else:
        gu8, gus, sg8, sgs, dn8, dns, sd8, sds = q
        call("dsv2_moe_grouped_gateup_shared_fp8", xn.data_ptr(), rows, srt.data_ptr(), tiles.data_ptr(),
             nt.data_ptr(), mt, tt, gu8.data_ptr(), gus.data_ptr(), sg8.data_ptr(), sgs.data_ptr(), I, hs.data_ptr(),
             sh.data_ptr(), stream_ptr())
        call("dsv2_moe_grouped_down_shared_fp8", hs.data_ptr(), rows, tiles.data_ptr(), nt.data_ptr(), mt, tt,
             dn8.data_ptr(), dns.data_ptr(), sh.data_ptr(), sd8.data_ptr(), sds.data_ptr(), I, ys.data_ptr(),
             parts.data_ptr(), stream_ptr())
    torch.cuda.synchronize()
    return hs, sh, ys, parts, srt


@pytest.mark.parametrize("tt", [32, 64])
def test_fp8_grouped_decodes_exactly_on_one_hot_rows(tt):
    """The batch family's e4m3 grouped launches, with every activation row one-hot: each output
    is one product, so it must equal the bf16 launches on the dequantized weights bit for bit
    (gate_up + SwiGLU, the shared halves' SwiGLU) and, for the down projection, the decoded
    weight times its row scale itself -- over random finite codes and row scales 2^-12..2^-6
    for gate_up, 2^-20..2^4 for down, with tiles of 64 experts and both shared halves."""
    rows = 70
    g = torch.Generator().manual_seed(930 + tt)
    gu8 = _finite_codes(64 * 2 * I * H, 931).view(64, 2 * I, H)
    gus = torch.ldexp(torch.ones(64, 2 * I), torch.randint(-12, -6, (64, 2 * I), generator=g)).to(DEV)
    sg8 = _finite_codes(4 * I * H, 932).view(4 * I, H)
    sgs = torch.ldexp(torch.ones(4 * I), torch.randint(-12, -6, (4 * I,), generator=g)).to(DEV)
    dn8 = _finite_codes(64 * H * I, 933).view(64, H, I)
    dns = torch.ldexp(torch.ones(64, H), torch.randint(-20, 5, (64, H), generator=g)).to(DEV)
    sd8 = _finite_codes(H * 2 * I, 934).view(H, 2 * I)
    sds = torch.ldexp(torch.ones(H), torch.randint(-20, 5, (H,), generator=g)).to(DEV)
    deq = lambda q8, sc: (q8.view(torch.float8_e4m3fn).float() * sc.unsqueeze(-1)).to(BF)  # noqa: E731
    gu, sgu, dn, sdn = deq(gu8, gus), deq(sg8, sgs), deq(dn8, dns), deq(sd8, sds)
    ids = torch.stack([torch.randperm(64, generator=g)[:6] for _ in range(rows)])
    xn = torch.zeros(rows, H, dtype=BF, device=DEV)
    xn[torch.arange(rows), torch.randint(0, H, (rows,), generator=g)] = 1.0
    q = (gu8, gus, sg8, sgs, dn8, dns, sd8, sds)
    hs8, sh8, _, _, srt = _grouped(xn, ids, tt, gu, sgu, dn, sdn, q)
    hs, sh, _, _, _ = _grouped(xn, ids, tt, gu, sgu, dn, sdn)
    assert torch.equal(hs8, hs) and torch.equal(sh8, sh)
    assert hs.float().abs().amax() > 0
    # down: one-hot rows of hs / shared_mid pick one column of the decoded weights
    R = rows * 6
    col = torch.randint(0, I, (R,), generator=g)
    hs1 = torch.zeros(R, I, dtype=BF, device=DEV)
    hs1[torch.arange(R), col] = 1.0
    scol = torch.randint(0, 2 * I, (rows,), generator=g)
    sh1 = torch.zeros(rows, 2 * I, dtype=BF, device=DEV)
    sh1[torch.arange(rows), scol] = 1.0
    srt2, _, tiles, nt, mt = _bucket(ids, tt)
    ys = torch.empty(R, H, dtype=BF, device=DEV)
    parts = torch.empty(2, rows, H, dtype=torch.float32, device=DEV)
    call("dsv2_moe_grouped_down_shared_fp8", hs1.data_ptr(), rows, tiles.data_ptr(), nt.data_ptr(), mt, tt,
         dn8.data_ptr(), dns.data_ptr(), sh1.data_ptr(), sd8.data_ptr(), sds.data_ptr(), I, ys.data_ptr(),
         parts.data_ptr(), stream_ptr())
    torch.cuda.synchronize()
    e_of = ids.reshape(-1)[srt2.cpu().long()]  # sorted position p holds route srt[p] = row*6 + slot
    ref = dn[e_of.to(DEV), :, col.to(DEV)]  # [R, H]: column col[p] of expert e_of[p]
    assert torch.equal(ys, ref)
    half = (scol >= I).long()
    ref_sh = sdn[:, scol.to(DEV)].t().float()  # [rows, H]
    got = parts[half.to(DEV), torch.arange(rows, device=DEV)]
    assert torch.equal(got, ref_sh)
    assert torch.all(parts[1 - half.to(DEV), torch.arange(rows, device=DEV)] == 0)


@pytest.mark.parametrize("rows,tt,replicated", [(64, 32, False), (37, 32, False), (256, 64, False),
                                                (64, 64, True), (130, 32, True)])
def test_fp8_grouped_vs_bf16_and_oracle(rows, tt, replicated):
    """Random activations: the e4m3 grouped launches against the bf16 launches on the
    dequantized weights (the same products in another K order within each 64-wide chunk: at
    most bf16 rounding flips) and the combine against the oracle at 1e-2."""
    gu = rnd(64, 2 * I, H, std=0.02, seed=940)
    dn = rnd(64, H, I, std=0.02, seed=941)
    sgu = rnd(4 * I, H, std=0.02, seed=942)
    sdn = rnd(H, 2 * I, std=0.02, seed=943)
    gu8, gus, gud = _q(gu)
    dn8, dns, dnd = _q(dn)
    sg8, sgs, sgd = _q(sgu)
    sd8, sds, sdd = _q(sdn)
    g = torch.Generator().manual_seed(944)
    if replicated:
        ids = torch.randperm(64, generator=g)[:6].repeat(rows, 1)
    else:
        ids = torch.stack([torch.randperm(64, generator=g)[:6] for _ in range(rows)])
    xn = rnd(rows, H, seed=945)
    q = (gu8, gus, sg8, sgs, dn8, dns, sd8, sds)
    hs8, sh8, ys8, parts8, _ = _grouped(xn, ids, tt, gud, sgd, dnd, sdd, q)
    hs, sh, ys, parts, _ = _grouped(xn, ids, tt, gud, sgd, dnd, sdd)
    c = lambda t: t.float().cpu()  # noqa: E731
    for a, b in ((hs8, hs), (sh8, sh), (ys8, ys)):
        assert rel_err(c(a), c(b)) < 1e-2
        assert (a == b).float().mean() > 0.9
    assert rel_err(c(parts8[0] + parts8[1]), c(parts[0] + parts[1])) < 1e-3
    # the combine of the e4m3 path against the oracle on the dequantized weights
    srt, rpos, _, _, _ = _bucket(ids, tt)
    w = (torch.rand(rows, 6, generator=g) * 0.3).to(DEV)
    res = rnd(rows, H, seed=946)
    out = torch.empty(rows, H, dtype=BF, device=DEV)
    call("dsv2_moe_combine_parts", ys8.data_ptr(), rpos.data_ptr(), w.data_ptr(), rows, parts8.data_ptr(),
         res.data_ptr(), out.data_ptr(), None, 0.0, None, stream_ptr())
    torch.cuda.synchronize()
    rb = lambda t: t.to(BF).float()  # noqa: E731
    sel = list(range(0, rows, max(1, rows // 8)))
    xc, wc = c(xn)[sel], c(w)[sel]
    routed = torch.zeros(len(sel), H)
    for s in range(6):
        part = torch.stack([O.mlp(xc[t:t + 1], c(gud[int(ids[r, s]), :I]), c(gud[int(ids[r, s]), I:]),
                                  c(dnd[int(ids[r, s])]), rb)[0] for t, r in enumerate(sel)])
        routed = routed + wc[:, s:s + 1] * part
    shared = O.mlp(xc, c(sgd[:2 * I]), c(sgd[2 * I:]), c(sdd), rb)
    assert rel_err(c(out)[sel], rb(c(res)[sel] + rb(rb(routed) + shared))) < 1e-2


def test_fp8_entry_points_reject_bad_arguments():
    from triton_kernels import _hip

    x = torch.zeros(16, dtype=torch.uint8, device=DEV)
    p = x.data_ptr()
    with pytest.raises(_hip.HipKernelError, match="go together"):  # a shared weight without its scales
        call("dsv2_moe_route_down_fp8", p, 1, p, p, p, p, p, None, I, 8, None, p, stream_ptr())
    with pytest.raises(_hip.HipKernelError, match="go together"):
        call("dsv2_moe_route_gateup_logits_fp8", p, 1, p, 1.0, p, p, p, p, p, None, I, p, stream_ptr())
    with pytest.raises(_hip.HipKernelError, match="bad shape"):  # inter % 16 != 0
        call("dsv2_moe_route_down_fp8", p, 1, p, p, p, p, None, None, I + 8, 6, None, p, stream_ptr())
    with pytest.raises(_hip.HipKernelError, match="bad shape"):  # inter % 4 != 0
        call("dsv2_moe_route_gateup_logits_fp8", p, 1, p, 1.0, p, p, p, p, None, None, I + 2, p, stream_ptr())
    with pytest.raises(_hip.HipKernelError, match="bad shape"):  # 16-token tiles: bf16 launches only
        call("dsv2_moe_grouped_gateup_shared_fp8", p, 1, p, p, p, 8, 16, p, p, p, p, I, p, p, stream_ptr())
    with pytest.raises(_hip.HipKernelError, match="null pointer"):  # the scales are required
        call("dsv2_moe_grouped_down_shared_fp8", p, 1, p, p, 8, 32, p, None, p, p, p, I, p, p, stream_ptr())


N_LAYERS = 3


@pytest.fixture(scope="module")
def model8():
    return build_model(N_LAYERS, fp8=True)


def test_engine_rejects_fp8_without_quantized_weights(model8):
    import dsv2lite

    cfg, w, _ = model8
    w2 = dsv2lite.ModelWeights(cfg, w.embed, w.norm, w.lm_head, w.layers)  # fp8_experts flag unset
    for family in ("small", "batch"):
        with pytest.raises(ValueError):
            dsv2lite.DecodeEngine(w2, [32], family=family, expert_dtype="fp8")
    # the batch family's e4m3 launches take 32- or 64-token tiles
    assert dsv2lite.DecodeEngine(w, [32], family="batch", expert_dtype="fp8").buf.tile_tokens == 32
    assert dsv2lite.DecodeEngine(w, [32], family="batch", expert_dtype="fp8", moe_tile=256).buf.tile_tokens == 64


@pytest.mark.parametrize("family,lens,mla", [("small", [16], "fused"), ("small", [5, 11], "split"),
                                             ("batch", [5, 16, 9, 1], "split"), ("batch", [40] * 64, "split")])
def test_engine_fp8_decode_vs_oracle(model8, family, lens, mla):
    import dsv2lite

    cfg, w, om = model8
    B = len(lens)
    eng = dsv2lite.DecodeEngine(w, [n + 16 for n in lens], family=family, mla_path=mla, expert_dtype="fp8")
    prompts = _prompts(lens, seed=70 + B)
    first = eng.prefill([p.cuda() for p in prompts]).cpu().clone()
    if family == "batch":
        eng.tune_moe_tiles()
    rows = list(range(B)) if B <= 4 else [0, 17, B - 1]  # checked rows (every row runs)
    caches = {b: om.new_cache() for b in rows}
    toks = eng.ids.cpu().tolist()
    agree = total = router_checked = 0
    for b in rows:
        res, _ = _oracle_step(om, caches[b], prompts[b], 0)
        ref = res["logits"][-1]
        toks[b] = int(torch.argmax(ref))
        agree += _agree(int(first[b]), ref, eng.logits[b].cpu(), ("prefill", b))
        total += 1
    steps = 6 if B <= 4 else 3
    for s in range(steps):
        eng.ids.copy_(torch.tensor(toks, dtype=torch.int64))
        rec = []
        eng.step(record=rec)
        torch.cuda.synchronize()
        new = eng.ids.cpu().tolist()
        for b in rows:
            res, trace = _oracle_step(om, caches[b], torch.tensor([toks[b]]), lens[b] + s)
            ref = res["logits"][-1]
            n_clear, flipped = _check_trace(om, rec, trace, b, ("fp8", family, s, b), res)
            router_checked += n_clear
            _close(eng.logits[b].cpu(), ref, res["fp32"]["logits"][-1], flipped, ("fp8", family, s, b))
            agree += _agree(int(eng.ids[b].item()), ref, eng.logits[b].cpu(), ("fp8", family, s, b))
            total += 1
            new[b] = int(torch.argmax(ref))
        toks = new
    assert router_checked >= steps * len(rows)
    print(f"fp8 {family} B={B} {mla}: MoE tile {getattr(eng.buf, 'tile_tokens', '-')}, greedy agreement "
          f"{agree}/{total}", flush=True)


@pytest.mark.parametrize("family", ["small", "batch"])
def test_engine_fp8_graph_replay_equals_eager(model8, family):
    import dsv2lite

    _, w, _ = model8
    lens = [12, 7] if family == "small" else [12, 7, 30, 21] * 16
    eng = dsv2lite.DecodeEngine(w, [n + 16 for n in lens], family=family, expert_dtype="fp8")
    eng.prefill([p.cuda() for p in _prompts(lens, seed=5)])
    eng.tune_moe_tiles()  # the tile capture() would pick, before the eager reference steps
    snap = eng.snapshot()
    eager = []
    for _ in range(3):
        eng.step()
        eager.append((eng.logits.clone(), eng.ids.clone()))
    eng.restore(snap)
    eng.capture()
    for rep in range(2):
        eng.restore(snap)
        torch.cuda.synchronize()
        for i in range(3):
            eng.replay()
            torch.cuda.synchronize()
            assert torch.equal(eng.logits, eager[i][0]), (rep, i)
            assert torch.equal(eng.ids, eager[i][1]), (rep, i)
