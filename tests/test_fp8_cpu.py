"""FP8 expert-weight quantization on the CPU: the e4m3 value table against the OCP 8-bit
floating-point specification (E4M3: bias 7, no infinities, S.1111.111 = NaN, max 448),
the quantizer's rounding against a brute-force nearest-value search, and the byte model."""

from __future__ import annotations

import types

import pytest
import torch

from dsv2lite.weights import E4M3_MAX, dequantize_rows_fp8, fp8_row_scales, quantize_rows_fp8


def _spec_value(code: int) -> float:
    """OCP E4M3 decoding of one byte, written from the specification."""
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 0x7
    if e == 0xF and m == 0x7:
        return float("nan")
    if e == 0:
        return s * (m / 8.0) * 2.0 ** -6
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def _table():
    return torch.tensor([_spec_value(c) for c in range(256)], dtype=torch.float64)


def test_torch_e4m3_decoding_matches_the_specification():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    got = codes.view(torch.float8_e4m3fn).double()
    ref = _table()
    assert torch.equal(torch.isnan(got), torch.isnan(ref))
    fin = ~torch.isnan(ref)
    assert torch.equal(got[fin], ref[fin])
    assert ref[fin].abs().max().item() == E4M3_MAX
    assert int(fin.sum()) == 254


def _nearest_codes(v: torch.Tensor) -> torch.Tensor:
    """Brute force: the finite e4m3 code nearest each value, ties to the even code."""
    tab = _table()
    codes = torch.arange(256)
    fin = ~torch.isnan(tab)
    tab, codes = tab[fin], codes[fin]
    d = (v.double().unsqueeze(-1) - tab).abs()
    best = d.min(dim=-1, keepdim=True).values
    cand = d == best
    # among equally near candidates prefer an even mantissa; +0 over -0
    score = cand.double() * 4 + ((codes & 1) == 0).double() * 2 + (codes == 0).double()
    return codes[score.argmax(dim=-1)]


def test_quantizer_rounds_to_nearest_e4m3_with_pow2_row_scales():
    g = torch.Generator().manual_seed(11)
    w = (torch.randn(24, 512, generator=g) * 0.02).to(torch.bfloat16)
    w[3] = 0  # an all-zero row: scale 1
    w[5, :8] = torch.tensor([448.0, -3.0, 1e-30, 0.5, -448.0, 2.0 ** -20, 7.0, 0.0]).to(torch.bfloat16)
    q, s = quantize_rows_fp8(w)
    assert q.dtype == torch.uint8 and s.dtype == torch.float32 and q.shape == w.shape
    m, e = torch.frexp(s)
    assert torch.all(m == 0.5)  # powers of two
    assert s[3].item() == 1.0
    amax = w.float().abs().amax(-1)
    live = amax > 0
    assert torch.all(amax[live] / s[live] <= E4M3_MAX)
    assert torch.all(amax[live] / s[live] > E4M3_MAX / 2)  # the smallest such power of two
    # every byte is the nearest e4m3 value of w / s
    v = w.float() / s.unsqueeze(-1)
    nearest = _nearest_codes(v.reshape(-1)).reshape(v.shape)
    qv = q.view(torch.float8_e4m3fn).double()
    assert torch.equal(qv, _table()[nearest])
    # dequantized values are exactly e4m3 * scale, representable in bf16
    d = dequantize_rows_fp8(q, s)
    assert d.dtype == torch.bfloat16
    assert torch.equal(d.double(), qv * s.double().unsqueeze(-1))
    # relative error of a normal value at most half an e4m3 ulp (2^-4)
    norm = v.abs() >= 2.0 ** -6
    rel = ((d.float() - w.float()).abs() / w.float().abs())[norm]
    assert rel.max().item() <= 2.0 ** -4


def test_row_scales_exact_powers_and_stacks():
    w = torch.tensor([[448.0, 1.0], [896.0, 0.0], [449.0, 0.0]])
    s = fp8_row_scales(w)
    assert s.tolist() == [1.0, 2.0, 2.0]
    stack = torch.randn(3, 4, 64).to(torch.bfloat16)
    q, s = quantize_rows_fp8(stack)
    assert s.shape == (3, 4) and q.shape == stack.shape


def test_step_bytes_fp8_halves_expert_bytes():
    from dsv2lite import DSV2Config
    from dsv2lite.roofline import step_bytes

    cfg = DSV2Config()
    n_exp = [6] * 26
    b16 = step_bytes(cfg, n_exp, 129.0, 1)
    b8 = step_bytes(cfg, n_exp, 129.0, 1, expert_fp8=True)
    H, I, Is = cfg.hidden, cfg.moe_inter, cfg.shared_inter
    moe_elems = 26 * (6 * 3 * H * I + 3 * H * Is)
    scales = 4 * 26 * (6 * (2 * I + H) + 2 * Is + H)
    assert b16 - b8 == pytest.approx(moe_elems - scales)


def test_engine_rejects_fp8_before_allocating():
    import dsv2lite

    w = types.SimpleNamespace(fp8_experts=False)
    for family in ("small", "batch"):
        with pytest.raises(ValueError, match="quantize_experts_fp8"):
            dsv2lite.DecodeEngine(w, [8], family=family, expert_dtype="fp8")
    with pytest.raises(ValueError):
        dsv2lite.DecodeEngine(w, [8], family="small", expert_dtype="int4")
