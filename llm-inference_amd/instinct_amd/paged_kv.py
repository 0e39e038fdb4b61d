"""Paged K/V storage in MI355X HBM: the arena and page-pool conventions the
decode kernel reads.

Counterpart of python/instinct/paged_kv.py. Every attention layer keeps its
keys and values in one fp16 arena; a page holds ``page_size`` token rows and
the row of logical position t is ``table[t // P] * P + t % P`` (:259-265).
Two device layouts hold the same rows:

* ``"rows"``: ``[rows, kv_heads, head_dim]``, the reference's arena
  (paged_kv.py:156-235);
* ``"pages"``: ``[pages, kv_heads, page_size, head_dim]`` page tiles, the
  MI355X layout: the rows of one (page, kv head) are one contiguous run
  (4 KiB at head_dim 128, page 16), which the decode kernel reads as whole
  128-byte lines instead of 256-byte pieces strided by kv_heads * head_dim.

The arenas live in device memory as torch tensors, sized once for the whole
page budget: with 288 GB of HBM per MI355X the arena is allocated at its
capacity rather than grown by doubling (:237-250), so the decode path never
reallocates.
"""

from __future__ import annotations

import heapq
from collections.abc import Iterable, Sequence
from dataclasses import dataclass

import numpy as np
import torch


LAYOUTS = ("rows", "pages")


def rows_to_pages(arena: torch.Tensor, page_size: int) -> torch.Tensor:
    """``[rows, kv_heads, head_dim]`` -> ``[pages, kv_heads, page_size,
    head_dim]`` holding the same rows (a copy)."""
    rows, heads, dim = arena.shape
    if rows % page_size:
        raise ValueError("the arena does not hold a whole number of pages")
    return arena.view(rows // page_size, page_size, heads, dim).permute(0, 2, 1, 3).contiguous()


def pages_to_rows(arena: torch.Tensor) -> torch.Tensor:
    """``[pages, kv_heads, page_size, head_dim]`` -> ``[rows, kv_heads,
    head_dim]`` (a copy)."""
    pages, heads, page_size, dim = arena.shape
    return arena.permute(0, 2, 1, 3).reshape(pages * page_size, heads, dim)


@dataclass(frozen=True)
class KVGroup:
    """Attention layers that share a K/V shape and window (paged_kv.py:34-47)."""

    name: str
    layers: tuple[int, ...]
    kv_heads: int
    head_dim: int
    window: int = 0  # 0 for full attention

    def bytes_per_token(self, bits: int = 16) -> int:
        row = self.head_dim * bits // 8 + (2 if bits == 8 else 0)
        return 2 * len(self.layers) * self.kv_heads * row


class PagePool:
    """Physical page ids with reference counts and reservations
    (paged_kv.py:79-153): the lowest free id is handed out first, so the arena
    only has to cover the high-water mark; ``retain``/``release`` let several
    tables hold one page (prefix sharing)."""

    def __init__(self, capacity: int) -> None:
        if capacity <= 0:
            raise ValueError("a page pool needs at least one page")
        self.capacity = capacity
        self._free = list(range(capacity))
        self._refs = np.zeros(capacity, dtype=np.int32)
        self.reserved = 0
        self.high_water = 0

    @property
    def free(self) -> int:
        return len(self._free)

    @property
    def available(self) -> int:
        return len(self._free) - self.reserved

    @property
    def used(self) -> int:
        return self.capacity - len(self._free)

    def reserve(self, count: int) -> bool:
        if count > self.available:
            return False
        self.reserved += count
        return True

    def unreserve(self, count: int) -> None:
        if not 0 <= count <= self.reserved:
            raise RuntimeError("released more pages than were reserved")
        self.reserved -= count

    def allocate(self, *, reserved: bool) -> int:
        """Take one page, from the caller's reservation if ``reserved``."""
        if reserved:
            self.unreserve(1)
        elif self.available <= 0:
            raise RuntimeError("the K/V page pool is exhausted")
        page = heapq.heappop(self._free)
        self._refs[page] = 1
        self.high_water = max(self.high_water, page + 1)
        return page

    def retain(self, pages: Iterable[int]) -> None:
        for page in pages:
            if page >= 0:
                if self._refs[page] <= 0:
                    raise RuntimeError("retained a page that isn't allocated")
                self._refs[page] += 1

    def release(self, pages: Iterable[int]) -> None:
        for page in pages:
            if page < 0:
                continue
            if self._refs[page] <= 0:
                raise RuntimeError("released a page that isn't allocated")
            self._refs[page] -= 1
            if self._refs[page] == 0:
                heapq.heappush(self._free, page)

    def shared(self, page: int) -> bool:
        return bool(self._refs[page] > 1)

    def held_only_by(self, counts: np.ndarray) -> int:
        return int(np.count_nonzero((counts > 0) & (self._refs == counts)))


class KVCache:
    """Per-layer K/V arenas in device memory plus one page pool per group
    (paged_kv.py:156-292), in the ``"pages"`` tile layout by default or the
    reference's ``"rows"`` layout. ``bits`` = 16 stores fp16 rows; ``bits`` =
    8 stores int8 rows with one fp16 scale per (row, kv head) (absmax / 127,
    paged_kv.py:50-55,176-181), the scales ``[rows, kv_heads]`` beside a row
    arena and ``[pages, kv_heads, page_size]`` beside a page-tile arena."""

    def __init__(
        self,
        groups: Sequence[KVGroup],
        *,
        page_size: int,
        capacities: dict[str, int],
        device: torch.device | str = "cuda",
        dtype: torch.dtype = torch.float16,
        layout: str = "pages",
        bits: int = 16,
    ) -> None:
        if layout not in LAYOUTS:
            raise ValueError(f"layout must be one of {LAYOUTS}")
        if bits not in (8, 16):
            raise ValueError("K/V is stored in 16 or 8 bits")
        if dtype not in (torch.float16, torch.bfloat16):
            raise ValueError("the model dtype is float16 or bfloat16")
        self.layout = layout
        self.bits = bits
        self.storage = torch.int8 if bits == 8 else dtype
        self.page_size = page_size
        self.dtype = dtype
        self.device = torch.device(device)
        self.groups = {group.name: group for group in groups}
        self.layer_group = {layer: group for group in groups for layer in group.layers}
        self.pools = {group.name: PagePool(capacities[group.name]) for group in groups}
        self.keys: dict[int, torch.Tensor] = {}
        self.values: dict[int, torch.Tensor] = {}
        self.key_scales: dict[int, torch.Tensor] = {}
        self.value_scales: dict[int, torch.Tensor] = {}
        for group in groups:
            pages = capacities[group.name]
            if layout == "rows":
                shape = (pages * page_size, group.kv_heads, group.head_dim)
            else:
                shape = (pages, group.kv_heads, page_size, group.head_dim)
            for layer in group.layers:
                self.keys[layer] = torch.zeros(shape, dtype=self.storage, device=self.device)
                self.values[layer] = torch.zeros(shape, dtype=self.storage, device=self.device)
                if bits == 8:
                    for store in (self.key_scales, self.value_scales):
                        store[layer] = torch.zeros(shape[:-1], dtype=torch.float16,
                                                   device=self.device)

    @property
    def compute_dtype(self) -> torch.dtype:
        """The element type the kernels take for queries and new K/V: the
        model dtype at 16 bits; fp16 at 8 bits, whose kernels dequantize to
        fp16."""
        return self.dtype if self.bits == 16 else torch.float16

    @property
    def _stores(self) -> tuple[dict[int, torch.Tensor], ...]:
        """Per-layer arrays indexed by row: K, V and, at 8 bits, their scales."""
        if self.bits == 8:
            return self.keys, self.values, self.key_scales, self.value_scales
        return self.keys, self.values

    def scales(self, layer: int) -> tuple[torch.Tensor, torch.Tensor] | None:
        """(key_scales, value_scales) of an 8-bit layer, else None."""
        return (self.key_scales[layer], self.value_scales[layer]) if self.bits == 8 else None

    @property
    def device_bytes(self) -> int:
        return sum(t.numel() * t.element_size()
                   for store in self._stores for t in store.values())

    def rows(self, table: np.ndarray, start: int, end: int) -> np.ndarray:
        """Physical rows of logical positions ``[start, end)`` (paged_kv.py:259-265)."""
        positions = np.arange(start, end, dtype=np.int64)
        pages = np.asarray(table)[positions // self.page_size]
        if np.any(pages < 0):
            raise RuntimeError("K/V range includes a released page")
        return (pages * self.page_size + positions % self.page_size).astype(np.int32)

    def copy_page(self, group: KVGroup, source: int, target: int, count: int) -> None:
        """Copy the first ``count`` rows of a page (copy-on-write of a shared
        tail, paged_kv.py:267-274)."""
        for layer in group.layers:
            for store in self._stores:
                arena = store[layer]
                if self.layout == "rows":
                    src = slice(source * self.page_size, source * self.page_size + count)
                    dst = slice(target * self.page_size, target * self.page_size + count)
                    arena[dst] = arena[src]
                else:
                    arena[target, :, :count] = arena[source, :, :count]

    def _split(self, rows: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        index = rows.long()
        return torch.div(index, self.page_size, rounding_mode="floor"), index % self.page_size

    def write(self, layer: int, rows: torch.Tensor, keys: torch.Tensor,
              values: torch.Tensor) -> None:
        """Scatter new rows ``[n, kv_heads, head_dim]`` into the layer arena
        in place (paged_kv.py:278-283), quantized at 8 bits, with the HIP
        append kernel; rows outside the arena are not written."""
        from .hip_kernels import kv_write

        arena = self.keys[layer]
        if not arena.is_cuda:
            raise ValueError("KVCache.write runs on the GPU; the arenas are on the CPU")
        kv_write(arena, self.values[layer], rows.to(device=arena.device, dtype=torch.int32),
                 keys.to(self.compute_dtype).contiguous(),
                 values.to(self.compute_dtype).contiguous(),
                 page_size=self.page_size, scales=self.scales(layer))

    def _pick(self, store: torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
        if self.layout == "rows":
            return store[rows.long()]
        page, slot = self._split(rows)
        return store[page, :, slot]

    def gather(self, layer: int, rows: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """Rows of the arena, ``[n, kv_heads, head_dim]`` in the model dtype,
        dequantized at 8 bits (paged_kv.py:285-292)."""
        keys, values = self._pick(self.keys[layer], rows), self._pick(self.values[layer], rows)
        if self.bits == 8:
            ks = self._pick(self.key_scales[layer], rows)
            vs = self._pick(self.value_scales[layer], rows)
            keys = (keys.float() * ks.float()[..., None]).to(self.dtype)
            values = (values.float() * vs.float()[..., None]).to(self.dtype)
        return keys, values
