"""Absorbed-MLA decode attention, small family: the q/kv_a projection with the W_UK
absorption in partial sums, one attention launch (kv-norm + RoPE + cache write, softmax over
the cached rows, W_UV) and the o_proj GEMV while the cache is at most 2048 tokens, else
GEMV + prepare + split-KV decode + combine with W_UV
(reference: triton_kernels/attention_decode_small.py:553-674, 782-840, 932-1070).
Same compressed-cache deviation as attention_decode_batch; batched_attention_decode_q1_triton
(the expanded-cache attention) is shared with it."""

from __future__ import annotations

from .attention_decode_batch import (AttentionPackedWeights, _attention_decode,  # noqa: F401
                                     batched_attention_decode_q1_triton, check_cache_status, pack_attention_weights)


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
