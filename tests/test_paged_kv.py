"""Page pool, arena and table conventions that feed the kernel (CPU only).

PagePool is checked against a brute-force model of its contract (lowest free
id first, reference counts, reservations; paged_kv.py:79-153) and on the
engine's sharing and window-trim patterns (mlx_engine.py:315-372), plus the
block arithmetic of its C++ KVBlockPool test (tests/host_tests.cpp:66-90:
15/16/17 tokens need 1/1/2 pages of 16).
"""

import math
import random

import numpy as np
import pytest
import torch

from instinct_amd.batches import DecodeBatch, pack_tables
from instinct_amd.paged_kv import (LAYOUTS, KVCache, KVGroup, PagePool, pages_to_rows,
                                  rows_to_pages)


class PoolModel:
    """Brute-force model of the pool's contract: a refcount per id, the
    lowest id with no reference comes first, reservations only count."""

    def __init__(self, capacity):
        self.refs = [0] * capacity
        self.reserved = 0
        self.high_water = 0

    @property
    def free(self):
        return self.refs.count(0)

    def allocate(self, count):
        got = [i for i, r in enumerate(self.refs) if r == 0][:count]
        for i in got:
            self.refs[i] = 1
        if got:
            self.high_water = max(self.high_water, got[-1] + 1)
        return got


def agrees(pool, model, rng=None):
    if rng is not None:
        # held_only_by: the pages whose references are all among the given
        # counts, against a count over the model.
        counts = np.array([rng.randint(0, 3) for _ in range(len(model.refs))], dtype=np.int64)
        want = sum(1 for r, c in zip(model.refs, counts) if c > 0 and r == c)
        assert pool.held_only_by(counts) == want
        assert pool.held_only_by(np.asarray(model.refs)) == sum(r > 0 for r in model.refs)
    assert pool.free == model.free
    assert pool.used == pool.capacity - model.free
    assert pool.reserved == model.reserved
    assert pool.available == model.free - model.reserved >= 0
    assert pool.high_water == model.high_water
    assert [pool.refcount(i) for i in range(pool.capacity)] == model.refs


@pytest.mark.parametrize("capacity,seed", [(1, 0), (63, 1), (64, 2), (65, 3), (200, 4),
                                           (1000, 5)])
def test_pool_follows_the_brute_force_model(capacity, seed):
    """Every operation of a long random sequence, including multi-page
    allocations across 64-id word boundaries, repeated ids and released
    (negative) table entries, against the model."""
    rng = random.Random(seed)
    pool, model = PagePool(capacity), PoolModel(capacity)
    held = []  # one entry per reference
    for _ in range(1500):
        op = rng.random()
        if op < 0.3:
            n = rng.randint(0, 5) if rng.random() < 0.8 else rng.randint(0, 80)
            use_reserve = rng.random() < 0.3 and model.reserved >= n
            if not use_reserve and n > model.free - model.reserved:
                with pytest.raises(RuntimeError, match="exhausted"):
                    pool.allocate_many(n, reserved=False)
                continue
            got = pool.allocate_many(n, reserved=use_reserve)
            if use_reserve:
                model.reserved -= n
            assert got.tolist() == model.allocate(n)
            held += got.tolist()
        elif op < 0.45 and held:
            pages = [rng.choice(held) for _ in range(rng.randint(1, 4))] + [-1]
            pool.retain(pages)
            for page in pages:
                if page >= 0:
                    model.refs[page] += 1
                    held.append(page)
        elif op < 0.75 and held:
            pages = [held.pop(rng.randrange(len(held))) for _ in range(min(len(held),
                                                                           rng.randint(1, 6)))]
            pool.release(pages + [-1, -7])
            for page in pages:
                model.refs[page] -= 1
        elif op < 0.85:
            n = rng.randint(0, 6)
            ok = pool.reserve(n)
            assert ok == (n <= model.free - model.reserved)
            model.reserved += n if ok else 0
        elif model.reserved:
            n = rng.randint(0, model.reserved)
            pool.unreserve(n)
            model.reserved -= n
        agrees(pool, model, rng)
    pool.release(held)
    assert pool.free == capacity and pool.used == 0


def test_lowest_free_id_comes_back_first_so_the_arena_stays_compact():
    pool = PagePool(300)
    first = pool.allocate_many(200, reserved=False)
    assert first.tolist() == list(range(200)) and pool.high_water == 200
    pool.release([199, 3, 130, 64])
    assert pool.allocate_many(3, reserved=False).tolist() == [3, 64, 130]
    assert pool.allocate(reserved=False) == 199
    assert pool.allocate(reserved=False) == 200 and pool.high_water == 201


def test_errors_leave_the_pool_unchanged():
    pool = PagePool(10)
    a, b = pool.allocate(reserved=False), pool.allocate(reserved=False)
    pool.retain([a])
    snapshot = [pool.refcount(i) for i in range(10)], pool.free
    with pytest.raises(RuntimeError):
        pool.release([a, b, b])          # b is held once
    with pytest.raises(RuntimeError):
        pool.retain([a, 7])              # 7 is free
    with pytest.raises(RuntimeError):
        pool.release([a, 10])            # outside the pool
    assert ([pool.refcount(i) for i in range(10)], pool.free) == snapshot
    with pytest.raises(RuntimeError):
        pool.unreserve(1)
    with pytest.raises(ValueError):
        PagePool(0)
    assert pool.shared(a) and not pool.shared(b)


def test_reserved_pages_stay_available_to_their_owner_only():
    pool = PagePool(6)
    assert pool.reserve(4) and pool.available == 2
    assert not pool.reserve(3)
    pool.allocate_many(2, reserved=False)
    with pytest.raises(RuntimeError, match="exhausted"):
        pool.allocate(reserved=False)
    assert pool.allocate_many(4, reserved=True).tolist() == [2, 3, 4, 5]
    assert pool.reserved == 0 and pool.free == 0


def test_shared_prefix_and_window_trim():
    """The engine's table producers on one pool (mlx_engine.py:315-372): a
    second request attaches to a 4-page prefix (retain all, copy the
    partial last page into a fresh one); a windowed sequence releases the
    pages that fall before (len - W + 1) // P and marks them -1. Pages come
    free only when their last holder lets go, and a windowed sequence holds
    at most ceil(W / P) + 1 pages however long it grows."""
    P, W = 16, 40
    pool = PagePool(64)
    first = pool.allocate_many(4, reserved=False).tolist()
    second = list(first)
    pool.retain(second)
    tail = pool.allocate(reserved=False)          # copy-on-write of the last page
    pool.release([second[-1]])
    second[-1] = tail
    assert [pool.refcount(p) for p in first] == [2, 2, 2, 1]
    pool.release(first)
    assert pool.free == 64 - 4 and all(pool.refcount(p) == 1 for p in second)
    pool.release(second)
    assert pool.free == 64
    table = []
    for length in range(1, 400):
        if (length - 1) // P >= len(table):
            table.append(pool.allocate(reserved=False))
        drop = (length - W + 1) // P
        gone = [i for i in range(min(drop, len(table))) if table[i] >= 0]
        pool.release([table[i] for i in gone])
        for i in gone:
            table[i] = -1
        assert sum(p >= 0 for p in table) <= math.ceil(W / P) + 1
        assert pool.used == sum(p >= 0 for p in table)
    assert pool.high_water <= math.ceil(W / P) + 2


def test_group_sizes():
    group = KVGroup("full", (3, 7), kv_heads=2, head_dim=512)
    assert group.bytes_per_token() == 2 * 2 * 2 * 512 * 2
    assert group.bytes_per_token(8) == 2 * 2 * 2 * (512 + 2)


@pytest.mark.parametrize("tokens, pages", [(15, 1), (16, 1), (17, 2)])
def test_block_arithmetic(tokens, pages):
    assert math.ceil(tokens / 16) == pages
    pool = PagePool(4)
    table = [pool.allocate(reserved=False) for _ in range(math.ceil(tokens / 16))]
    assert len(table) == pages


def small_cache(layout="rows"):
    groups = [KVGroup("full", (0,), kv_heads=2, head_dim=8),
              KVGroup("local", (1,), kv_heads=2, head_dim=8, window=6)]
    return KVCache(groups, page_size=4, capacities={"full": 8, "local": 8}, device="cpu",
                   layout=layout)


def test_rows_map_positions_through_the_table():
    cache = small_cache()
    table = np.array([5, 2, 7])
    np.testing.assert_array_equal(cache.rows(table, 0, 9),
                                  [20, 21, 22, 23, 8, 9, 10, 11, 28])
    with pytest.raises(RuntimeError, match="released"):
        cache.rows(np.array([-1, 2]), 0, 6)
    np.testing.assert_array_equal(cache.rows(np.array([-1, 2]), 4, 6), [8, 9])


def put_rows(cache, layer, rows, k, v):
    """Test-side scatter (the GPU kernel's write is tested in test_gpu_append)."""
    for arena, data in ((cache.keys[layer], k), (cache.values[layer], v)):
        if cache.layout == "rows":
            arena[rows] = data.half()
        else:
            arena[rows // cache.page_size, :, rows % cache.page_size] = data.half()


def test_write_runs_on_the_gpu_only():
    cache = small_cache()
    with pytest.raises(ValueError, match="GPU"):
        cache.write(0, torch.tensor([1]), torch.zeros(1, 2, 8), torch.zeros(1, 2, 8))


@pytest.mark.parametrize("layout", LAYOUTS)
def test_gather_and_copy_page(layout):
    cache = small_cache(layout)
    rows = torch.tensor([3, 9, 17])
    k = torch.arange(3 * 2 * 8, dtype=torch.float32).view(3, 2, 8)
    v = -k
    put_rows(cache, 0, rows, k, v)
    gk, gv = cache.gather(0, rows)
    assert torch.equal(gk, k.half()) and torch.equal(gv, v.half())
    assert cache.keys[0].abs().sum() == k.abs().sum()
    cache.copy_page(cache.groups["full"], source=2, target=6, count=2)  # rows 8,9 -> 24,25
    assert torch.equal(cache.gather(0, torch.tensor([25]))[0][0], k[1].half())
    assert torch.equal(cache.gather(0, torch.tensor([26]))[1][0], torch.zeros(2, 8).half())
    assert cache.device_bytes == 4 * 32 * 2 * 8 * 2
    # Both layouts hold the same rows: converting one gives the other.
    arena = cache.keys[0]
    as_rows = arena if layout == "rows" else pages_to_rows(arena)
    assert torch.equal(as_rows[9], k[1].half())
    if layout == "pages":
        assert tuple(arena.shape) == (8, 2, 4, 8)
        assert torch.equal(arena[2, :, 1], k[1].half())  # row 9 = page 2, slot 1
        assert torch.equal(pages_to_rows(rows_to_pages(as_rows, 4)), as_rows)


def test_unknown_layout_is_rejected():
    with pytest.raises(ValueError, match="layout"):
        small_cache("columns")


def test_model_dtype_and_kernel_dtype():
    """The arenas hold the model dtype (fp16 or bf16) at 16 bits and int8 at
    8 bits; the kernels take the model dtype at 16 bits and fp16 at 8."""
    groups = [KVGroup("full", (0,), kv_heads=2, head_dim=8)]

    def make(**kw):
        return KVCache(groups, page_size=4, capacities={"full": 2}, device="cpu", **kw)

    bf = make(dtype=torch.bfloat16)
    assert bf.keys[0].dtype == bf.compute_dtype == torch.bfloat16
    q8 = make(dtype=torch.bfloat16, bits=8)
    assert q8.keys[0].dtype == torch.int8 and q8.compute_dtype == torch.float16
    assert make().compute_dtype == torch.float16
    with pytest.raises(ValueError, match="dtype"):
        make(dtype=torch.float32)


def test_decode_batch_packs_tables_and_lengths():
    cache = small_cache()
    positions = np.array([0, 5, 9])
    tables = {"full": [np.array([4]), np.array([1, 6]), np.array([0, 2, 3])],
              "local": [np.array([7]), np.array([-1, 5]), np.array([-1, 1, 2])]}
    packed = pack_tables(tables["full"], 3)
    np.testing.assert_array_equal(packed, [[4, 0, 0], [1, 6, 0], [0, 2, 3]])
    batch = DecodeBatch(cache, torch.zeros(3), positions=positions, tables=tables)
    assert batch.lengths.tolist() == [1, 6, 10] and batch.longest == 10
    # write rows: table[pos // P] * P + pos % P
    assert batch._write["full"].tolist() == [16, 25, 13]
    assert batch._write["local"].tolist() == [28, 21, 9]
    assert batch._tables["local"].tolist() == [[7, 0, 0], [-1, 5, 0], [-1, 1, 2]]
