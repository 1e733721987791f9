"""Compressed MLA KV cache in HBM.

Layout: one bf16 tensor [n_layers, total_tokens, 576]; sequence b owns rows
[base[b], base[b] + capacity[b]) of every layer (row starts staggered, see STAGGER_*).  A row is the kv-normalised
512-d latent followed by the 64-d rotated k_pe (1,152 bytes per token per
layer, vs. 10,240 for the reference's expanded K/V cache, src/run.py:81-99).

``pos[b]`` (int32, device) is the number of cached tokens of sequence b, i.e.
the position of its next token; the decode step writes row base+pos and the
argmax kernel advances pos.  Rows at or beyond pos are never read, so
snapshot/restore of the prompt state (src/run.py:161-170, 212-217, 547-555) only
saves and restores ``pos``.

``cap[b]`` (int32, device) is the capacity of sequence b.  The MLA kernels store a
new token only at 0 <= pos < cap and never read past cap; a position at or past cap
writes nothing and sets DSV2_DEVERR_CACHE_FULL in ``status`` (int32, device), which
``check_status`` raises on -- the reference's overflow error (src/run.py:131-134).
"""

from __future__ import annotations

import torch

DEVERR_CACHE_FULL = 1  # DSV2_DEVERR_CACHE_FULL of include/dsv2lite.h

# Staggered row starts: the split-KV decode streams every row's cache tile by tile in token
# order, all rows at once; with every row at one stride some strides put the rows' concurrent
# reads on the same HBM channels (MI355X, bsz=256 x 2,049 cached tokens: a 2,099-token stride
# 158 us per layer against 99-102 us for 2,081 / 2,089 / 2,112 / 2,158).  Row b therefore
# starts (7 b mod 8) tiles of 32 tokens into a slot of capacity + 7 tiles (2,099 with the
# stagger: 101 us; every stride measured stays at 99-102 us).  Caches of short rows skip it.
STAGGER_TILE = 32
STAGGER_PHASES = 8
STAGGER_MIN_CAPACITY = 512


class CompressedKVCache:
    def __init__(self, n_layers: int, capacities: list[int], device="cuda", row: int = 576,
                 stagger: bool | None = None):
        if not capacities or min(capacities) <= 0:
            raise ValueError("capacities must be positive")
        self.n_layers = n_layers
        self.capacities = list(int(c) for c in capacities)
        if stagger is None:
            stagger = max(self.capacities) >= STAGGER_MIN_CAPACITY
        pad = (STAGGER_PHASES - 1) * STAGGER_TILE if stagger else 0
        bases, start = [], 0
        for b, c in enumerate(self.capacities):
            bases.append(start + (((7 * b) % STAGGER_PHASES) * STAGGER_TILE if stagger else 0))
            start += c + pad
        self.total = start
        self.row = row
        self.data = torch.zeros(n_layers, self.total, row, dtype=torch.bfloat16, device=device)
        self.base = torch.tensor(bases, dtype=torch.int64, device=device)
        self.cap = torch.tensor(self.capacities, dtype=torch.int32, device=device)
        self.pos = torch.zeros(len(capacities), dtype=torch.int32, device=device)
        self.status = torch.zeros(1, dtype=torch.int32, device=device)
        self.max_capacity = max(self.capacities)

    @property
    def batch(self) -> int:
        return len(self.capacities)

    def check_status(self) -> None:
        """Raise if a kernel flagged a cache write past a row's capacity (synchronises)."""
        st = int(self.status.item())
        if st & DEVERR_CACHE_FULL:
            self.status.zero_()
            raise RuntimeError("KV cache capacity exhausted: a decode step reached a row's capacity "
                               f"(capacities {self.capacities}); nothing was written past it")

    def layer(self, i: int) -> torch.Tensor:
        return self.data[i]

    def snapshot(self) -> torch.Tensor:
        return self.pos.clone()

    def restore(self, snap: torch.Tensor) -> None:
        self.pos.copy_(snap)

    def rows_of(self, b: int, layer: int, n: int | None = None) -> torch.Tensor:
        """The cached rows of sequence b in a layer (host-synchronising; for checks)."""
        n = int(self.pos[b].item()) if n is None else n
        s = int(self.base[b].item())
        return self.data[layer, s:s + n]
