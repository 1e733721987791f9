"""dsv2_lm_head_argmax_bf16_noalloc (the entry point with no workspace argument, for
callers that cannot allocate) against dsv2_lm_head_argmax_bf16 (caller workspace) through
the C ABI: bit-identical logits, next ids and position steps on two calls in a row, the
second with fewer rows and a smaller vocabulary, and rows beyond its device scratch
rejected before any launch."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
BF = torch.bfloat16


def _rnd(*shape, std=1.0, seed=0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=DEV) * std).to(BF)


def _both(rows, vocab, seed):
    from triton_kernels import _hip

    st = _hip.stream_ptr()
    x = _rnd(rows, 2048, seed=seed)
    W = _rnd(vocab, 2048, std=0.02, seed=seed + 1)
    nw = (_rnd(2048, std=0.1, seed=seed + 2) + 1).to(BF)
    out = {}
    for name in ("ws", "noalloc"):
        logits = torch.full((rows, vocab), float("nan"), device=DEV)
        ids = torch.full((rows,), -1, dtype=torch.int64, device=DEV)
        pos = torch.arange(rows, dtype=torch.int32, device=DEV) * 10
        if name == "ws":
            ws = torch.empty(_hip.lib.dsv2_lm_head_argmax_workspace_size(rows), dtype=torch.uint8, device=DEV)
            _hip.call("dsv2_lm_head_argmax_bf16", x.data_ptr(), 2048, rows, W.data_ptr(), vocab, nw.data_ptr(), 1e-6,
                      logits.data_ptr(), ws.data_ptr(), ws.numel(), ids.data_ptr(), pos.data_ptr(), st)
        else:
            _hip.call("dsv2_lm_head_argmax_bf16_noalloc", x.data_ptr(), 2048, rows, W.data_ptr(), vocab,
                      nw.data_ptr(), 1e-6, logits.data_ptr(), ids.data_ptr(), pos.data_ptr(), st)
        torch.cuda.synchronize()
        out[name] = (logits.cpu(), ids.cpu(), pos.cpu())
    return out


def test_noalloc_matches_workspace_entry_point_twice():
    for rows, vocab, seed in ((8, 102400, 1), (3, 32000, 7)):  # second call: fewer rows, smaller vocab
        o = _both(rows, vocab, seed)
        assert torch.equal(o["ws"][0], o["noalloc"][0]), (rows, vocab)
        assert torch.equal(o["ws"][1], o["noalloc"][1]), (rows, vocab)
        assert torch.equal(o["ws"][2], o["noalloc"][2]), (rows, vocab)
        assert torch.equal(o["noalloc"][1], torch.argmax(o["noalloc"][0], -1))
        assert torch.equal(o["noalloc"][2], torch.arange(rows, dtype=torch.int32) * 10 + 1)


def test_noalloc_rejects_more_rows_than_its_scratch():
    from triton_kernels import _hip

    with pytest.raises(_hip.HipKernelError, match="1 <= rows <= 8"):
        _hip.call("dsv2_lm_head_argmax_bf16_noalloc", 16, 2048, 9, 16, 102400, 16, 1e-6, 16, 16, None,
                  _hip.stream_ptr())
