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


N_LAYERS = 3


@pytest.fixture(scope="module")
def model8():
    return build_model(N_LAYERS, fp8=True)


def test_engine_rejects_fp8_without_quantized_weights_or_on_batch_family(model8):
    import dsv2lite

    cfg, w, _ = model8
    with pytest.raises(NotImplementedError):
        dsv2lite.DecodeEngine(w, [32], family="batch", expert_dtype="fp8")
    w2 = dsv2lite.ModelWeights(cfg, w.embed, w.norm, w.lm_head, w.layers)  # fp8_experts flag unset
    with pytest.raises(ValueError):
        dsv2lite.DecodeEngine(w2, [32], family="small", expert_dtype="fp8")


@pytest.mark.parametrize("lens,mla", [([16], "fused"), ([5, 11], "split")])
def test_engine_fp8_decode_vs_oracle(model8, lens, mla):
    import dsv2lite

    cfg, w, om = model8
    B = len(lens)
    eng = dsv2lite.DecodeEngine(w, [n + 16 for n in lens], family="small", mla_path=mla, expert_dtype="fp8")
    prompts = _prompts(lens, seed=70 + B)
    first = eng.prefill([p.cuda() for p in prompts]).cpu().clone()
    caches = [om.new_cache() for _ in range(B)]
    toks = []
    agree = total = router_checked = 0
    for b in range(B):
        res, _ = _oracle_step(om, caches[b], prompts[b], 0)
        ref = res["logits"][-1]
        toks.append(int(torch.argmax(ref)))
        agree += _agree(int(first[b]), ref, eng.logits[b].cpu(), ("prefill", b))
        total += 1
    steps = 6
    for s in range(steps):
        eng.ids.copy_(torch.tensor(toks, dtype=torch.int64))
        rec = []
        eng.step(record=rec)
        torch.cuda.synchronize()
        new = []
        for b in range(B):
            res, trace = _oracle_step(om, caches[b], torch.tensor([toks[b]]), lens[b] + s)
            ref = res["logits"][-1]
            n_clear, flipped = _check_trace(om, rec, trace, b, ("fp8", s, b), res)
            router_checked += n_clear
            _close(eng.logits[b].cpu(), ref, res["fp32"]["logits"][-1], flipped, ("fp8", s, b))
            agree += _agree(int(eng.ids[b].item()), ref, eng.logits[b].cpu(), ("fp8", s, b))
            total += 1
            new.append(int(torch.argmax(ref)))
        toks = new
    assert router_checked >= steps * B
    print(f"fp8 {lens} {mla}: greedy agreement {agree}/{total}", flush=True)


def test_engine_fp8_graph_replay_equals_eager(model8):
    import dsv2lite

    _, w, _ = model8
    lens = [12, 7]
    eng = dsv2lite.DecodeEngine(w, [n + 16 for n in lens], family="small", expert_dtype="fp8")
    eng.prefill([p.cuda() for p in _prompts(lens, seed=5)])
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
