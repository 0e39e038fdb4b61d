"""Seeded synthetic decode workloads: the five BASELINE configurations and
the reference's own kernel-test shapes.

Page tables and lengths come from ``numpy.random.default_rng(seed)`` on the
host (small); K/V/Q values are drawn with a seeded ``torch.Generator`` on the
target device, so multi-GB arenas are generated in HBM without a host copy.
Arenas are generated in the reference's ``[rows, kv_heads, head_dim]`` fp16
layout (paged_kv.py:156-235); :meth:`Workload.to_layout` converts them to the
page-tile layout with the same rows. Tables are ``[batch, width]`` int32, zero-padded like
``DecodeBatch`` (batches.py:170-179), with -1 for pages released by the
sliding-window trim (mlx_engine.py:349-372).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np
import torch

from .paged_kv import pages_to_rows, rows_to_pages


@dataclass
class Workload:
    name: str
    q: torch.Tensor          # [B, HQ, D] fp16
    keys: torch.Tensor       # [rows, HKV, D] or [pages, HKV, P, D] fp16
    values: torch.Tensor     # same shape as keys
    tables: torch.Tensor     # [B, width] int32
    lengths: torch.Tensor    # [B] int32
    page_size: int
    scale: float
    window: int = 0
    softcap: float = 0.0
    meta: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return int(self.q.shape[0])

    @property
    def q_heads(self) -> int:
        return int(self.q.shape[1])

    @property
    def kv_heads(self) -> int:
        return int(self.keys.shape[1])

    @property
    def head_dim(self) -> int:
        return int(self.q.shape[2])

    @property
    def layout(self) -> str:
        return "pages" if self.keys.dim() == 4 else "rows"

    def to_layout(self, layout: str) -> "Workload":
        """Convert the arenas in place to ``"rows"`` or ``"pages"`` (same
        rows, same results); returns self."""
        if layout == self.layout:
            return self
        if layout == "pages":
            self.keys = rows_to_pages(self.keys, self.page_size)
            self.values = rows_to_pages(self.values, self.page_size)
        elif layout == "rows":
            self.keys = pages_to_rows(self.keys)
            self.values = pages_to_rows(self.values)
        else:
            raise ValueError(f"unknown layout {layout!r}")
        return self

    @property
    def longest(self) -> int:
        """Largest length (the reference's host-side ``longest``), computed
        once: callers pass it on every call without a device sync."""
        if "longest" not in self.meta:
            self.meta["longest"] = int(self.lengths.max().item()) if self.batch else 0
        return self.meta["longest"]

    def spans(self) -> np.ndarray:
        n = self.lengths.cpu().numpy().astype(np.int64)
        return np.minimum(n, self.window) if self.window else n

    def kv_bytes(self) -> int:
        """Algorithmic (logical) K+V bytes one call reads: sum of visible
        spans x kv_heads x head_dim x 2 bytes x 2 (K and V)."""
        return int(self.spans().sum()) * self.kv_heads * self.head_dim * 2 * 2

    def unique_kv_bytes(self) -> int:
        """K+V bytes of distinct physical rows visible to the batch (shared
        prefix pages counted once)."""
        tables = self.tables.cpu().numpy()
        n = self.lengths.cpu().numpy().astype(np.int64)
        rows = set()
        for b in range(self.batch):
            first = max(0, n[b] - self.window) if self.window else 0
            pos = np.arange(first, n[b])
            pages = tables[b][pos // self.page_size]
            ok = pages >= 0
            rows.update((pages[ok].astype(np.int64) * self.page_size
                         + pos[ok] % self.page_size).tolist())
        return len(rows) * self.kv_heads * self.head_dim * 2 * 2

    def numpy(self):
        """Host copies for the oracle: (q, keys, values) as fp16 ndarrays with
        the arenas as ``[rows, kv_heads, head_dim]``, tables and lengths as
        int32."""
        keys, values = self.keys, self.values
        if self.layout == "pages":
            keys, values = pages_to_rows(keys), pages_to_rows(values)
        return (self.q.cpu().numpy(), keys.cpu().numpy(), values.cpu().numpy(),
                self.tables.cpu().numpy(), self.lengths.cpu().numpy())


def _normal(shape, gen: torch.Generator, device, scale: float = 1.0) -> torch.Tensor:
    out = torch.empty(shape, dtype=torch.float16, device=device)
    # Generate in row blocks to bound the float32 temporary.
    flat = out.view(shape[0], -1)
    block = max(1, (1 << 26) // max(1, flat.shape[1]))
    for s in range(0, flat.shape[0], block):
        e = min(flat.shape[0], s + block)
        chunk = torch.randn((e - s, flat.shape[1]), generator=gen, device=device,
                            dtype=torch.float32)
        if scale != 1.0:
            chunk.mul_(scale)
        flat[s:e] = chunk.to(torch.float16)
    return out


def _generator(device, seed: int) -> torch.Generator:
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    return gen


def build(name, *, lengths, tables, arena_pages, q_heads, kv_heads, head_dim, page_size,
          scale, window=0, softcap=0.0, device="cpu", seed=0, kv_scale=1.0,
          meta=None) -> Workload:
    """Assemble a workload from host tables/lengths and seeded device data."""
    device = torch.device(device)
    gen = _generator(device, seed)
    batch = len(lengths)
    rows = arena_pages * page_size
    keys = _normal((rows, kv_heads, head_dim), gen, device, kv_scale)
    values = _normal((rows, kv_heads, head_dim), gen, device, kv_scale)
    q = _normal((batch, q_heads, head_dim), gen, device)
    return Workload(
        name=name, q=q, keys=keys, values=values,
        tables=torch.as_tensor(np.asarray(tables, dtype=np.int32), device=device),
        lengths=torch.as_tensor(np.asarray(lengths, dtype=np.int32), device=device),
        page_size=page_size, scale=scale, window=window, softcap=softcap,
        meta=dict(meta or {}, seed=seed))


def _pack(tables: list[np.ndarray], width: int | None = None) -> np.ndarray:
    width = width or max(len(t) for t in tables)
    packed = np.zeros((len(tables), width), dtype=np.int32)
    for b, t in enumerate(tables):
        packed[b, : len(t)] = t
    return packed


def _permuted_tables(rng, lengths, page_size, arena_pages):
    """Tables of distinct physical pages drawn from one permutation."""
    need = [math.ceil(n / page_size) for n in lengths]
    order = rng.permutation(arena_pages)
    tables, cursor = [], 0
    for count in need:
        tables.append(order[cursor: cursor + count])
        cursor += count
    return tables


# --- the five BASELINE configurations --------------------------------------

def config1(device="cpu", seed=1, batch=8, length=1024) -> Workload:
    """Qwen2.5-0.5B shape: B=8, 14/2 heads, D=64, P=16, every length 1024,
    K/V N(0,1)*0.5, Q N(0,1), scale 1/8."""
    rng = np.random.default_rng(seed)
    P = 16
    pages = batch * (length // P)
    order = rng.permutation(pages)
    tables = order.reshape(batch, -1)
    return build("config1-qwen0.5b", lengths=[length] * batch, tables=tables,
                 arena_pages=pages, q_heads=14, kv_heads=2, head_dim=64, page_size=P,
                 scale=64 ** -0.5, device=device, seed=seed, kv_scale=0.5)


def config2(device="cpu", seed=2, batch=64, low=512, high=8192) -> Workload:
    """Qwen2.5-7B shape: B=64, 28/4 heads (G=7), D=128, P=16, lengths
    U[512, 8192], arena sized to exactly fit, one page permutation."""
    rng = np.random.default_rng(seed)
    P = 16
    lengths = rng.integers(low, high + 1, batch)
    arena = int(sum(math.ceil(n / P) for n in lengths))
    tables = _permuted_tables(rng, lengths, P, arena)
    return build("config2-qwen7b", lengths=lengths, tables=_pack(tables),
                 arena_pages=arena, q_heads=28, kv_heads=4, head_dim=128, page_size=P,
                 scale=128 ** -0.5, device=device, seed=seed)


def config3(device="cpu", seed=3, batch=1, length=32768, planted=8) -> Workload:
    """Long-context split-K stress: 32/8 heads, D=128, P=16, fixed length,
    pages fragmented across a 2x arena, ~8 keys per (sequence, kv head)
    multiplied by 8 to plant large logits."""
    rng = np.random.default_rng(seed)
    P = 16
    lengths = [length] * batch
    need = sum(math.ceil(n / P) for n in lengths)
    arena = 2 * need
    tables = _permuted_tables(rng, lengths, P, arena)
    w = build(f"config3-long-b{batch}-{length}", lengths=lengths, tables=_pack(tables),
              arena_pages=arena, q_heads=32, kv_heads=8, head_dim=128, page_size=P,
              scale=128 ** -0.5, device=device, seed=seed)
    # Plant large keys at random visible positions of each (sequence, kv head).
    for b in range(batch):
        pos = rng.choice(length, size=(8, planted), replace=True)  # [kvh, planted]
        rows = tables[b][pos // P].astype(np.int64) * P + pos % P
        for kvh in range(8):
            idx = torch.as_tensor(rows[kvh], device=w.keys.device)
            w.keys[idx, kvh] *= 8
    w.meta["planted"] = planted
    return w


def config4(device="cpu", seed=4, batch=32, low=4096, high=32768, window=1024) -> Workload:
    """Gemma-3-style sliding window: B=32, 8/4 heads, D=256, P=16, window
    1024, lengths U[4096, 32768]; tables of width 2048 hold only the pages
    covering the window, earlier entries are -1 (released), the rest 0."""
    rng = np.random.default_rng(seed)
    P = 16
    lengths = rng.integers(low, high + 1, batch)
    width = math.ceil(high / P)
    live = []
    for n in lengths:
        first_page = (n - window) // P
        last_page = (n - 1) // P
        live.append((first_page, last_page))
    arena = int(sum(l - f + 1 for f, l in live))
    order = rng.permutation(arena)
    tables = np.zeros((batch, width), dtype=np.int32)
    cursor = 0
    for b, (f, l) in enumerate(live):
        tables[b, :f] = -1
        count = l - f + 1
        tables[b, f: l + 1] = order[cursor: cursor + count]
        cursor += count
    offsets = (lengths - window) % P
    return build("config4-window", lengths=lengths, tables=tables, arena_pages=arena,
                 q_heads=8, kv_heads=4, head_dim=256, page_size=P, scale=256 ** -0.5,
                 window=window, device=device, seed=seed,
                 meta={"nonzero_start_offsets": int(np.count_nonzero(offsets))})


def config5(device="cpu", seed=5, batch=256, low=16, high=65536, shared=64,
            prefix=2048) -> Workload:
    """Continuous-batching mix: B=256, 32/8 heads, D=128, P=16, lengths
    log-uniform in [16, 65536]; ``shared`` sequences map logical pages
    0..prefix/P-1 onto the same physical pages 0..prefix/P-1. Their lengths
    are redrawn log-uniformly in (prefix, 65536] so the whole prefix is
    visible."""
    rng = np.random.default_rng(seed)
    P = 16
    lengths = np.floor(np.exp(rng.uniform(math.log(low), math.log(high), batch))).astype(np.int64)
    lengths = np.clip(lengths, low, high)
    sharers = rng.choice(batch, size=shared, replace=False)
    lengths[sharers] = np.clip(np.floor(np.exp(rng.uniform(
        math.log(prefix + 1), math.log(high), shared))).astype(np.int64), prefix + 1, high)
    prefix_pages = prefix // P
    need_private = []
    for b in range(batch):
        total = math.ceil(lengths[b] / P)
        need_private.append(total - prefix_pages if b in set(sharers.tolist()) else total)
    arena = prefix_pages + int(sum(need_private))
    order = prefix_pages + rng.permutation(arena - prefix_pages)
    sharer_set = set(sharers.tolist())
    tables, cursor = [], 0
    for b in range(batch):
        own = order[cursor: cursor + need_private[b]]
        cursor += need_private[b]
        if b in sharer_set:
            own = np.concatenate([np.arange(prefix_pages), own])
        tables.append(own)
    return build("config5-mix", lengths=lengths, tables=_pack(tables), arena_pages=arena,
                 q_heads=32, kv_heads=8, head_dim=128, page_size=P, scale=128 ** -0.5,
                 device=device, seed=seed, meta={"sharers": sorted(sharer_set)})


CONFIGS = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}


def gemma4_global(device="cpu", seed=6, batch=1, length=261840, q_heads=16, planted=8,
                  dtype=torch.bfloat16) -> Workload:
    """The workload of the reference's one published decode-kernel figure
    (docs/benchmarks.md:102-110): a Gemma 4 global layer, two 512-wide KV
    heads (gemma4.py:3-5, 49-66), bf16, one sequence at 261,840 tokens,
    page 16, pages a seeded permutation of an arena that exactly fits.
    The model attends with scale 1.0 (gemma4.py:161) on normalized
    queries; here queries are drawn N(0,1)/sqrt(512) so that the logits
    have unit variance. ``q_heads`` is a representative 16 (group of 8).
    As in config 3, ``planted`` keys per (sequence, kv head) are multiplied
    by 8: their logits dominate the softmax, so the output is O(1) rather
    than an average of ~1/sqrt(length) over the whole context."""
    rng = np.random.default_rng(seed)
    P, d = 16, 512
    lengths = [length] * batch
    arena = int(sum(math.ceil(n / P) for n in lengths))
    tables = _permuted_tables(rng, lengths, P, arena)
    w = build(f"gemma4-global-b{batch}-{length}", lengths=lengths, tables=_pack(tables),
              arena_pages=arena, q_heads=q_heads, kv_heads=2, head_dim=d, page_size=P,
              scale=1.0, device=device, seed=seed)
    for b in range(batch):
        pos = rng.choice(length, size=(2, planted), replace=True)
        rows = tables[b][pos // P].astype(np.int64) * P + pos % P
        for kvh in range(2):
            w.keys[torch.as_tensor(rows[kvh], device=w.keys.device), kvh] *= 8
    w.q = (w.q.float() * d ** -0.5).to(dtype)
    w.keys = w.keys.to(dtype)
    w.values = w.values.to(dtype)
    w.meta["planted"] = planted
    return w


# --- the reference's kernel-test shapes -----------------------------------

# tests/test_mlx_engine.py:422-431: (q_heads, kv_heads, head_dim, lengths,
# window, softcap). Head dims 80 (at 8 bits) and 4 run the generic kernels.
REFERENCE_TEST_SHAPES = [
    (16, 2, 512, [1, 700, 2049], 0, 0.0),
    (16, 8, 256, [5, 1500, 4000], 1024, 0.0),
    (16, 4, 256, [64, 3333], 0, 0.0),
    (8, 1, 80, [3, 300], 0, 30.0),
    (2, 1, 4, [9], 4, 0.0),
]


def reference_test_case(q_heads, kv_heads, head_dim, lengths, window, softcap,
                        device="cpu", seed=0) -> Workload:
    """Construction of test_mlx_engine.py:438-450: page 16, physical pages a
    ``default_rng(0)`` permutation of ``sum(pages) + 3``, zero-padded tables,
    scale head_dim^-0.5 (values are fp16 here, drawn with torch)."""
    page = 16
    pages = [math.ceil(n / page) for n in lengths]
    order = np.random.default_rng(0).permutation(sum(pages) + 3)
    tables, cursor = [], 0
    for count in pages:
        tables.append(list(order[cursor: cursor + count]) + [0] * (max(pages) - count))
        cursor += count
    return build(f"reftest-{q_heads}-{kv_heads}-{head_dim}", lengths=lengths,
                 tables=np.array(tables, dtype=np.int32), arena_pages=sum(pages) + 3,
                 q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, page_size=page,
                 scale=head_dim ** -0.5, window=window, softcap=softcap, device=device,
                 seed=seed)
