"""What a model forward sees on a decode step: the op contract of the path.

Counterpart of ``DecodeBatch`` (python/instinct/batches.py:142-253) for the
MI355X kernel: one new token per sequence, page tables packed to
``[batch, width]`` int32 with zero padding (:170-179), ``lengths =
positions + 1`` (:162-164), write rows ``table[pos // P] * P + pos % P``
(:175-178), and :meth:`DecodeBatch.attend`, which writes the new K/V first
and then attends over ``[first, length)`` (:203-226), returning
``[batch, q_heads * head_dim]``.

The packed tables, lengths and write rows are uploaded once per step and
shared by every layer of a group, as in the reference.
"""

from __future__ import annotations

import numpy as np
import torch

from .hip_kernels import paged_decode_attention
from .paged_kv import KVCache


def pack_tables(tables: list[np.ndarray] | list[list[int]], count: int) -> np.ndarray:
    """``[count, width]`` int32 with 0 padding (batches.py:171-174)."""
    width = max(1, max(len(t) for t in tables))
    packed = np.zeros((count, width), dtype=np.int32)
    for row, table in enumerate(tables):
        packed[row, : len(table)] = table
    return packed


class DecodeBatch:
    prefill = False

    def __init__(
        self,
        cache: KVCache,
        tokens: torch.Tensor,
        *,
        positions: np.ndarray,
        tables: dict[str, list[np.ndarray]],
    ) -> None:
        device = cache.device
        self.cache = cache
        self.tokens = tokens
        self.count = int(tokens.shape[0])
        positions = np.asarray(positions).astype(np.int64)
        self.offsets = torch.as_tensor(positions.astype(np.int32), device=device)
        self.lengths = torch.as_tensor((positions + 1).astype(np.int32), device=device)
        self.longest = int(positions.max()) + 1
        page = cache.page_size
        self._write: dict[str, torch.Tensor] = {}
        self._tables: dict[str, torch.Tensor] = {}
        for name in cache.groups:
            packed = pack_tables(tables[name], self.count)
            pages = packed[np.arange(self.count), positions // page]
            rows = (pages.astype(np.int64) * page + positions % page).astype(np.int32)
            self._write[name] = torch.as_tensor(rows, device=device)
            self._tables[name] = torch.as_tensor(packed, device=device)

    @property
    def positions(self) -> torch.Tensor:
        return self.offsets

    def attend(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
               scale: float, softcap: float = 0.0) -> torch.Tensor:
        """Write this step's K/V, then paged decode attention
        (batches.py:203-226). ``q`` is ``[batch, q_heads, head_dim]``; ``k``,
        ``v`` are ``[batch, kv_heads, head_dim]``."""
        group = self.cache.layer_group[layer]
        self.cache.write(layer, self._write[group.name], k, v)
        out = paged_decode_attention(
            q.to(torch.float16).contiguous(),
            self.cache.keys[layer],
            self.cache.values[layer],
            self._tables[group.name],
            self.lengths,
            page_size=self.cache.page_size,
            longest=self.longest,
            scale=scale,
            window=group.window,
            softcap=softcap,
        )
        return out.reshape(self.count, -1)
