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
    """A set of attention layers whose K/V arenas share one shape, one window
    and one page pool. The fields are the reference's group description
    (paged_kv.py:34-47), so an engine hands its groups over unchanged."""

    name: str
    layers: tuple[int, ...]
    kv_heads: int
    head_dim: int
    window: int = 0  # 0 for full attention

    def bytes_per_token(self, bits: int = 16) -> int:
        """HBM bytes one token costs over the group's layers: a K and a V row
        per kv head, plus one fp16 scale per row at 8 bits."""
        per_head = self.head_dim * bits // 8 + (2 if bits == 8 else 0)
        return len(self.layers) * 2 * self.kv_heads * per_head


_WORD = 64


class PagePool:
    """Physical page ids of one group: reference counts, reservations, and
    the lowest free id handed out first, so the arena only has to cover the
    high-water mark (the reference's contract, paged_kv.py:79-153).

    Design: the free pages are a bitmap of 64-bit words (bit set = free),
    and a Python integer summarises it (bit w set = word w holds a free
    page), so the lowest free id is two lowest-set-bit steps away whatever
    the capacity. Reference counts live in an int32 vector; :meth:`retain`
    and :meth:`release` take whole page lists (a shared prefix of 128
    pages, the pages a window trim drops) and update them with a few vector
    operations. Both check the whole list before changing anything, so a
    bad id leaves the pool as it was. Negative ids (released table entries,
    mlx_engine.py:349-372) are ignored."""

    def __init__(self, capacity: int) -> None:
        if capacity <= 0:
            raise ValueError("a page pool needs at least one page")
        self.capacity = int(capacity)
        words = -(-self.capacity // _WORD)
        self._bits = np.full(words, np.iinfo(np.uint64).max, dtype=np.uint64)
        tail = self.capacity - (words - 1) * _WORD
        if tail < _WORD:
            self._bits[-1] = np.uint64((1 << tail) - 1)
        self._summary = (1 << words) - 1
        self._refs = np.zeros(self.capacity, dtype=np.int32)
        self._free_count = self.capacity
        self.reserved = 0
        self.high_water = 0

    # Counts -------------------------------------------------------------
    @property
    def free(self) -> int:
        """Pages no table holds."""
        return self._free_count

    @property
    def available(self) -> int:
        """Free pages not promised to a reservation."""
        return self._free_count - self.reserved

    @property
    def used(self) -> int:
        return self.capacity - self._free_count

    def refcount(self, page: int) -> int:
        return int(self._refs[page])

    def shared(self, page: int) -> bool:
        """More than one table holds the page (copy-on-write needed)."""
        return bool(self._refs[page] > 1)

    # Reservations --------------------------------------------------------
    def reserve(self, count: int) -> bool:
        """Promise ``count`` free pages to a request; False if they are not there."""
        if count < 0:
            raise ValueError("cannot reserve a negative page count")
        if count > self.available:
            return False
        self.reserved += count
        return True

    def unreserve(self, count: int) -> None:
        if count < 0 or count > self.reserved:
            raise RuntimeError(f"cannot return {count} of {self.reserved} reserved pages")
        self.reserved -= count

    # Allocation -------------------------------------------------------------
    def _take(self, count: int) -> list[int]:
        pages: list[int] = []
        while len(pages) < count:
            w = (self._summary & -self._summary).bit_length() - 1
            word = int(self._bits[w])
            base = w * _WORD
            while word and len(pages) < count:
                low = word & -word
                pages.append(base + low.bit_length() - 1)
                word ^= low
            self._bits[w] = np.uint64(word)
            if not word:
                self._summary &= ~(1 << w)
        return pages

    def allocate_many(self, count: int, *, reserved: bool) -> np.ndarray:
        """The ``count`` lowest free ids, each with one reference; drawn from
        the caller's reservation if ``reserved``."""
        if count < 0:
            raise ValueError("cannot allocate a negative page count")
        if reserved:
            self.unreserve(count)
        elif count > self.available:
            raise RuntimeError(f"the K/V page pool is exhausted ({count} pages asked, "
                               f"{self.available} available)")
        pages = np.asarray(self._take(count), dtype=np.int64)
        self._refs[pages] = 1
        self._free_count -= count
        if count:
            self.high_water = max(self.high_water, int(pages[-1]) + 1)
        return pages

    def allocate(self, *, reserved: bool) -> int:
        """The lowest free id, with one reference."""
        return int(self.allocate_many(1, reserved=reserved)[0])

    # Sharing -----------------------------------------------------------------
    def _held(self, pages: Iterable[int]) -> tuple[np.ndarray, np.ndarray]:
        ids = np.asarray(list(pages) if not isinstance(pages, np.ndarray) else pages,
                         dtype=np.int64).ravel()
        ids = ids[ids >= 0]
        if ids.size and int(ids.max()) >= self.capacity:
            raise RuntimeError(f"page {int(ids.max())} is outside a pool of {self.capacity}")
        unique, counts = np.unique(ids, return_counts=True)
        return unique, counts.astype(np.int32)

    def retain(self, pages: Iterable[int]) -> None:
        """One more reference to each listed page (a table that now shares it)."""
        unique, counts = self._held(pages)
        if np.any(self._refs[unique] <= 0):
            raise RuntimeError("cannot share a page that is not allocated")
        self._refs[unique] += counts

    def held_only_by(self, counts: np.ndarray) -> int:
        """Pages that would come free if ``counts[page]`` of each page's
        references were dropped: those held by exactly that many references
        (the reference's contract, paged_kv.py:150-153; its prefix cache
        weighs evictions with it, prefix_cache.py:193). ``counts`` is indexed
        by page id; entries past the pool's capacity are ignored."""
        counts = np.asarray(counts, dtype=np.int64).ravel()
        n = min(counts.size, self.capacity)
        wanted = counts[:n]
        return int(np.count_nonzero((wanted > 0) & (self._refs[:n] == wanted)))

    def release(self, pages: Iterable[int]) -> None:
        """Drop one reference per listed occurrence; pages left with none
        become free."""
        unique, counts = self._held(pages)
        if np.any(self._refs[unique] < counts):
            raise RuntimeError("cannot release a page more often than it is held")
        self._refs[unique] -= counts
        freed = unique[self._refs[unique] == 0]
        if freed.size:
            words = freed // _WORD
            masks = np.left_shift(np.uint64(1), (freed % _WORD).astype(np.uint64))
            np.bitwise_or.at(self._bits, words, masks)
            for w in np.unique(words).tolist():
                self._summary |= 1 << w
            self._free_count += int(freed.size)


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
        """The element type the append and prefill kernels take for queries
        and new K/V: the model dtype at 16 bits; fp16 at 8 bits, whose
        kernels dequantize to fp16."""
        return self.dtype if self.bits == 16 else torch.float16

    @property
    def decode_dtype(self) -> torch.dtype:
        """The query and output type of the decode call: the model dtype, at
        16 bits and at 8 (the reference's quantized kernel runs on the
        queries' dtype, metal_kernels.py:196-206)."""
        return self.dtype

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
