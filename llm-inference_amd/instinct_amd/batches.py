"""What a model forward sees on a decode step: the op contract of the path.

Counterpart of ``DecodeBatch`` (python/instinct/batches.py:142-253) for the
MI355X kernel: one new token per sequence, page tables packed to
``[batch, width]`` int32 with zero padding (:170-179), ``lengths =
positions + 1`` (:162-164), write rows ``table[pos // P] * P + pos % P``
(:175-178), :meth:`DecodeBatch.rope` (:195-201) and
:meth:`DecodeBatch.attend`, which writes the new K/V first and then attends
over ``[first, length)`` (:203-226), returning ``[batch, q_heads *
head_dim]``. :meth:`DecodeBatch.rope_attend` does the model's two ``rope``
calls, the write and the attention with the rotation and the write fused into
one launch.

The packed tables, lengths and write rows are uploaded once per step and
shared by every layer of a group, as in the reference.
"""

from __future__ import annotations

from typing import Any

import numpy as np
import torch

from .hip_kernels import (image_spans, paged_decode_attention, paged_prefill_attention, rope,
                          rope_append)
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

    def rope(self, x: torch.Tensor, dims: int, *, base: float | None = None,
             freqs: Any = None) -> torch.Tensor:
        """Rotary embedding of ``[batch, heads, head_dim]`` at each
        sequence's position (batches.py:195-201, portable.py:88-132)."""
        return rope(x.to(self.cache.dtype).contiguous(), self.offsets, dims, base=base,
                    freqs=freqs)

    def rope_attend(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
                    dims: int, scale: float, base: float | None = None, freqs: Any = None,
                    softcap: float = 0.0) -> torch.Tensor:
        """``attend(layer, rope(q), rope(k), v)`` with the rotation of q and k
        and the K/V write in one launch (the model calls of
        backends/dense.py:99-102 and DecodeBatch.attend, batches.py:203-226).
        A bf16 model over an 8-bit cache takes the three steps apart: its
        rotated keys are rounded to bf16 before they are quantized, as the
        reference's are, while the fused 8-bit write rounds them to fp16."""
        group = self.cache.layer_group[layer]
        cache = self.cache
        dtype = cache.compute_dtype
        if dtype != cache.dtype:
            rot = dict(base=base, freqs=freqs)
            return self.attend(layer, self.rope(q, dims, **rot), self.rope(k, dims, **rot), v,
                               scale=scale, softcap=softcap)
        q_rot = rope_append(q.to(dtype).contiguous(), k.to(dtype).contiguous(),
                            v.to(dtype).contiguous(), cache.keys[layer],
                            cache.values[layer], self.offsets, self._write[group.name],
                            page_size=cache.page_size, dims=dims, base=base, freqs=freqs,
                            scales=cache.scales(layer))
        return self._attend_written(layer, q_rot, scale=scale, softcap=softcap)

    def attend(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
               scale: float, softcap: float = 0.0) -> torch.Tensor:
        """Write this step's K/V, then paged decode attention
        (batches.py:203-226). ``q`` is ``[batch, q_heads, head_dim]``; ``k``,
        ``v`` are ``[batch, kv_heads, head_dim]``."""
        group = self.cache.layer_group[layer]
        self.cache.write(layer, self._write[group.name], k, v)
        return self._attend_written(layer, q, scale=scale, softcap=softcap)

    def _attend_written(self, layer: int, q: torch.Tensor, *, scale: float,
                        softcap: float) -> torch.Tensor:
        group = self.cache.layer_group[layer]
        out = paged_decode_attention(
            q.to(self.cache.decode_dtype).contiguous(),
            self.cache.keys[layer],
            self.cache.values[layer],
            self._tables[group.name],
            self.lengths,
            page_size=self.cache.page_size,
            longest=self.longest,
            scale=scale,
            window=group.window,
            softcap=softcap,
            scales=self.cache.scales(layer),
        )
        return out.reshape(self.count, -1).to(self.cache.dtype)


class PrefillBatch:
    """A chunk of one sequence's prompt (batches.py:26-132): positions
    ``start .. start + count - 1``, the chunk's K/V written to the cache
    first, then causal attention over the sequence's pages on the GPU
    (``pda_paged_prefill_attention``, ``_q8`` for an 8-bit cache),
    ``[count, q_heads * head_dim]`` out. ``images``: (at, embeddings) as the
    reference takes them (or (at, length)); their tokens also see the rest of
    their image (batches.py:107-118)."""

    prefill = True

    def __init__(self, cache: KVCache, tokens: torch.Tensor, *, start: int,
                 tables: dict[str, np.ndarray], images: Any = ()) -> None:
        device = cache.device
        self.cache = cache
        self.tokens = tokens
        self.count = int(tokens.shape[0])
        self.start = int(start)
        self.images = list(images)
        end = self.start + self.count
        self._spans = image_spans(
            [(at, x if isinstance(x, int) else int(x.shape[0])) for at, x in self.images], device)
        self.offsets = torch.arange(self.start, end, dtype=torch.int32, device=device)
        self._write: dict[str, torch.Tensor] = {}
        self._tables: dict[str, torch.Tensor] = {}
        for name in cache.groups:
            table = np.asarray(tables[name])
            self._write[name] = torch.as_tensor(cache.rows(table, self.start, end),
                                                device=device)
            self._tables[name] = torch.as_tensor(table.astype(np.int32), device=device)

    @property
    def positions(self) -> torch.Tensor:
        return self.offsets

    def inject(self, x: torch.Tensor) -> torch.Tensor:
        """Put image embeddings in place of their placeholder tokens
        (batches.py:63-68)."""
        for at, embeddings in self.images:
            if isinstance(embeddings, int):
                continue
            offset = at - self.start
            x[offset:offset + int(embeddings.shape[0])] = embeddings.to(x.dtype)
        return x

    def rope(self, x: torch.Tensor, dims: int, *, base: float | None = None,
             freqs: Any = None) -> torch.Tensor:
        """Rotate ``[tokens, heads, head_dim]`` at the chunk's positions
        (batches.py:70-81)."""
        return rope(x.to(self.cache.dtype).contiguous(), self.offsets, dims, base=base,
                    freqs=freqs)

    def attend(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *,
               scale: float, softcap: float = 0.0) -> torch.Tensor:
        """Write the chunk's K/V (quantized in an 8-bit cache), then its
        attention over the dequantized rows (batches.py:84-132,
        paged_kv.py:285-292)."""
        group = self.cache.layer_group[layer]
        self.cache.write(layer, self._write[group.name], k, v)
        out = paged_prefill_attention(
            q.to(self.cache.compute_dtype).contiguous(), self.cache.keys[layer],
            self.cache.values[layer],
            self._tables[group.name], start=self.start, page_size=self.cache.page_size,
            scale=scale, window=group.window, softcap=softcap,
            scales=self.cache.scales(layer),
            images=self._spans if self._spans is not None else ())
        return out.reshape(self.count, -1).to(self.cache.dtype)
