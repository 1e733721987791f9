"""Continuous batching under one captured graph (DecodeEngine.insert / retire): a retired
slot keeps decoding throw-away tokens inside its own cache rows without ever stopping the
batch, and a new sequence inserted into it decodes bitwise like the same sequence inserted
into a fresh engine -- nothing of the retired sequence leaks into it -- while the other rows'
caches are untouched by the insertion.  2-layer full-width model (dense + MoE), full vocab."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def weights():
    import dsv2lite

    return dsv2lite.init_weights(dsv2lite.DSV2Config(n_layers=2), device="cuda", seed=0)


def _prompts(lens, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, 102400, (n,), generator=g).cuda() for n in lens]


@pytest.mark.parametrize("family", ["small", "batch"])
def test_retired_slot_reuse_matches_a_fresh_engine_bitwise(weights, family):
    import dsv2lite

    caps = [48, 40, 64, 56]
    tile = 16 if family == "batch" else None
    A = dsv2lite.DecodeEngine(weights, caps, family=family, moe_tile=tile)
    A.prefill(_prompts([10, 7, 20, 12], 1))
    A.capture()
    for _ in range(5):
        A.replay()
    A.retire(2)
    assert A.free_slots == [2]
    for _ in range(3):
        A.replay()  # slot 2 decodes throw-away tokens
    others = {b: A.cache.data[:, int(A.cache.base[b]):int(A.cache.base[b]) + caps[b]].clone() for b in (0, 1, 3)}
    pos_before = A.cache.pos.clone()
    q = _prompts([9], 2)[0]
    first = A.insert(2, q)
    torch.cuda.synchronize()
    assert A.free_slots == [] and int(A.cache.pos[2]) == 9
    for b, t in others.items():  # the insertion touched slot 2's rows only
        assert torch.equal(A.cache.data[:, int(A.cache.base[b]):int(A.cache.base[b]) + caps[b]], t), b
        assert int(A.cache.pos[b]) == int(pos_before[b])
    got = [(first, A.logits[2].clone())]
    for _ in range(6):
        A.replay()
        got.append((int(A.ids[2]), A.logits[2].clone()))
    A.check_errors()

    B = dsv2lite.DecodeEngine(weights, caps, family=family, moe_tile=tile)
    B.capture()
    ref = [(B.insert(2, q), B.logits[2].clone())]
    for _ in range(6):
        B.replay()
        ref.append((int(B.ids[2]), B.logits[2].clone()))
    for i, ((ta, la), (tb, lb)) in enumerate(zip(got, ref)):
        assert ta == tb and torch.equal(la, lb), (family, i)


def test_retired_slot_wraps_inside_its_capacity(weights):
    """A retired slot with a small capacity restarts at 0 whenever it would reach it; the
    active rows decode on, and no kernel ever flags a write past a row's capacity."""
    import dsv2lite

    eng = dsv2lite.DecodeEngine(weights, [80, 12], family="small")
    eng.prefill(_prompts([6, 5], 3))
    eng.capture()
    eng.replay()
    eng.retire(1)
    for _ in range(40):  # > 3 wraps of slot 1's 12 rows
        eng.replay()
        assert 0 <= eng._host_pos[1] <= 12
    torch.cuda.synchronize()
    assert int(eng.cache.pos[0]) == 6 + 41 and int(eng.cache.pos[1]) == eng._host_pos[1]
    eng.check_errors()
    with pytest.raises(ValueError, match="does not fit"):
        eng.insert(1, _prompts([12], 4)[0])
    assert eng.insert(1, _prompts([4], 4)[0]) >= 0 and eng.free_slots == []
