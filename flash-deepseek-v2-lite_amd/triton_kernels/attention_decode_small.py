"""Absorbed-MLA decode attention, small family: GEMV projections, fused
prepare (RoPE + cache write + W_UK absorption) and fused combine + W_UV
(reference: triton_kernels/attention_decode_small.py:553-674, 932-1070).
Same compressed-cache deviation as attention_decode_batch."""

from __future__ import annotations

from .attention_decode_batch import (AttentionPackedWeights, _attention_decode,  # noqa: F401
                                     pack_attention_weights)


def attention_decode_only_triton(hidden_states, cos, sin, position_ids, cache_position, key_cache, value_cache,
                                 packed, softmax_scale: float):
    if hidden_states.shape[0] != 1:
        raise NotImplementedError("attention_decode_only_triton is the bsz=1 path")
    return _attention_decode("small", hidden_states, cos, sin, position_ids, cache_position, key_cache, value_cache,
                             packed, softmax_scale)


def attention_decode_small_batch_triton(hidden_states, cos, sin, position_ids, cache_position, key_cache,
                                        value_cache, packed, softmax_scale: float):
    return _attention_decode("small", hidden_states, cos, sin, position_ids, cache_position, key_cache, value_cache,
                             packed, softmax_scale)
