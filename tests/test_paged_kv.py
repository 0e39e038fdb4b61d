"""Page pool, arena and table conventions that feed the kernel (CPU only).

PagePool invariants follow the reference's tests/test_paged_kv.py (lowest
free page first, reservations, refcounted sharing, random traffic), and the
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


def test_lowest_free_page_first_keeps_the_arena_compact():
    pool = PagePool(8)
    pages = [pool.allocate(reserved=False) for _ in range(3)]
    assert pages == [0, 1, 2] and pool.high_water == 3
    pool.release([1])
    assert pool.allocate(reserved=False) == 1
    assert pool.high_water == 3


def test_reservations_hold_pages_for_their_owner():
    pool = PagePool(4)
    assert pool.reserve(3)
    assert pool.available == 1 and not pool.reserve(2)
    pool.allocate(reserved=True)
    assert pool.reserved == 2 and pool.free == 3 and pool.available == 1
    pool.allocate(reserved=False)
    with pytest.raises(RuntimeError, match="exhausted"):
        pool.allocate(reserved=False)
    pool.unreserve(2)
    assert pool.available == 2
    with pytest.raises(RuntimeError):
        pool.unreserve(1)


def test_shared_pages_return_only_after_the_last_reference():
    pool = PagePool(2)
    page = pool.allocate(reserved=False)
    pool.retain([page, -1])
    assert pool.shared(page)
    pool.release([page])
    assert pool.free == 1 and not pool.shared(page)
    pool.release([page, -1])
    assert pool.free == 2
    with pytest.raises(RuntimeError):
        pool.release([page])
    with pytest.raises(RuntimeError):
        pool.retain([page])


@pytest.mark.parametrize("seed", range(5))
def test_random_traffic_never_loses_or_duplicates_pages(seed):
    rng = random.Random(seed)
    pool = PagePool(32)
    held = []
    for _ in range(500):
        action = rng.random()
        if action < 0.5 and pool.available:
            held.append(pool.allocate(reserved=False))
        elif action < 0.7 and held:
            page = rng.choice(held)
            pool.retain([page])
            held.append(page)
        elif held:
            pool.release([held.pop(rng.randrange(len(held)))])
        assert pool.free + len(set(held)) == pool.capacity
    pool.release(held)
    assert pool.free == pool.capacity


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
