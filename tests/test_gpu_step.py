"""Step-level integration: device-side table packing (pda_pack_decode_step)
against DecodeBatch's host packing (batches.py:148-179), and a whole decode
step captured in a HIP graph (instinct_amd.step.DecodeStepGraph) against the
same step run eagerly with host packing, replayed several times with new
inputs and eager work in between."""

import numpy as np
import pytest
import torch

from instinct_amd import hip_kernels
from instinct_amd.batches import DecodeBatch, pack_tables
from instinct_amd.paged_kv import KVCache, KVGroup
from instinct_amd.step import DecodeStepGraph

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-3
MEAN_ABS = 2e-4


def test_device_packing_matches_the_host_packing(gpu):
    rng = np.random.default_rng(0)
    P, num_slots, stride, width = 16, 40, 64, 48
    seq_tables = rng.integers(0, 5000, (num_slots, stride)).astype(np.int32)
    slots = rng.permutation(num_slots)[:24].astype(np.int32)
    positions = rng.integers(0, width * P, 24).astype(np.int32)
    t = lambda a: torch.as_tensor(a, device=gpu)  # noqa: E731
    tables, lengths, rows = hip_kernels.pack_decode_step(t(seq_tables), t(slots), t(positions),
                                                         width=width, page_size=P)
    torch.cuda.synchronize()
    # Host packing of the reference: each request's pages up to its new
    # token's page, 0 padding, lengths = positions + 1, the write rows.
    lists = [seq_tables[s, : p // P + 1] for s, p in zip(slots, positions)]
    packed = np.zeros((24, width), np.int32)
    packed[:, : pack_tables(lists, 24).shape[1]] = pack_tables(lists, 24)
    want_rows = packed[np.arange(24), positions // P] * P + positions % P
    assert np.array_equal(tables.cpu().numpy(), packed)
    assert np.array_equal(lengths.cpu().numpy(), positions + 1)
    assert np.array_equal(rows.cpu().numpy(), want_rows)
    # A slot outside the array, a negative position, a page past the width.
    bad_slots = t(np.array([-1, num_slots, 3, 4], np.int32))
    bad_pos = t(np.array([5, 5, -2, width * P + 3], np.int32))
    tb, lb, rb = hip_kernels.pack_decode_step(t(seq_tables), bad_slots, bad_pos, width=width,
                                              page_size=P)
    torch.cuda.synchronize()
    assert not tb[:3].any() and lb[:3].tolist() == [0, 0, 0]
    assert rb.tolist()[:3] == [-1, -1, -1] and rb.tolist()[3] == -1
    assert lb[3].item() == width * P + 4


def setup(gpu, layout, bits, layers=2, batch=6, dtype=torch.float16):
    page, heads, hq, d = 16, 4, 28, 128
    groups = [KVGroup("full", tuple(range(layers)), kv_heads=heads, head_dim=d)]
    cache = KVCache(groups, page_size=page, capacities={"full": 1024}, device=gpu,
                    layout=layout, bits=bits, dtype=dtype)
    gen = torch.Generator(device=gpu).manual_seed(1)
    for layer in range(layers):
        if bits == 16:
            cache.keys[layer].normal_(generator=gen)
            cache.values[layer].normal_(generator=gen)
        else:
            for store in (cache.keys, cache.values):
                store[layer].copy_(torch.randn(store[layer].shape, generator=gen, device=gpu)
                                   .mul(36).round().clamp(-127, 127).to(torch.int8))
            for store in (cache.key_scales, cache.value_scales):
                store[layer].fill_(1 / 36)
    pool = cache.pools["full"]
    start = np.array([3, 40, 600, 1000, 2047, 100])[:batch]
    width = (start.max() + 8) // page + 1
    slot_lists = [[pool.allocate(reserved=False) for _ in range(width)] for _ in range(batch)]
    seq_tables = torch.as_tensor(np.array(slot_lists, dtype=np.int32), device=gpu)
    return cache, start, slot_lists, seq_tables, width, hq


@pytest.mark.parametrize("layout,bits,dtype", [
    ("pages", 16, torch.float16), ("rows", 16, torch.float16), ("pages", 8, torch.float16),
    ("pages", 16, torch.bfloat16)])
def test_graph_replays_match_eager_steps(gpu, layout, bits, dtype):
    layers, batch = 2, 6
    cache_g, start, slot_lists, seq_tables, width, hq = setup(gpu, layout, bits, layers, batch,
                                                              dtype)
    cache_e, *_ = setup(gpu, layout, bits, layers, batch, dtype)
    work = cache_g.compute_dtype
    arenas = [(cache_g.keys[l], cache_g.values[l]) + (cache_g.scales(l) or ())
              for l in range(layers)]
    step = DecodeStepGraph(arenas, seq_tables, batch=batch, q_heads=hq, page_size=16,
                           width=width, scale=128 ** -0.5, longest=int(start.max()) + 8,
                           dims=128, base=1e6)
    slots = np.arange(batch, dtype=np.int32)[::-1].copy()  # slot s holds sequence s
    gen = torch.Generator(device=gpu).manual_seed(2)

    def inputs(t):
        return [(torch.randn((batch, hq, 128), generator=gen, device=gpu).to(work),
                 torch.randn((batch, 4, 128), generator=gen, device=gpu).to(work),
                 torch.randn((batch, 4, 128), generator=gen, device=gpu).to(work))
                for _ in range(layers)]

    for t in range(4):
        positions = (start + t).astype(np.int32)[slots]
        qkv = inputs(t)
        step.slots.copy_(torch.as_tensor(slots, device=gpu))
        step.positions.copy_(torch.as_tensor(positions, device=gpu))
        for layer, (q, k, v) in enumerate(qkv):
            step.q[layer].copy_(q)
            step.k[layer].copy_(k)
            step.v[layer].copy_(v)
        if t == 0:
            step.capture()  # runs the first step once eagerly, then captures it
        else:
            step.replay()
        torch.cuda.synchronize()
        # Eager reference: host packing (DecodeBatch), rope + attend per layer.
        batch_e = DecodeBatch(cache_e, torch.zeros(batch, device=gpu), positions=positions,
                              tables={"full": [np.array(slot_lists[s]) for s in slots]})
        for layer, (q, k, v) in enumerate(qkv):
            want = batch_e.rope_attend(layer, q, k, v, dims=128, base=1e6, scale=128 ** -0.5)
            torch.cuda.synchronize()
            got = step.out[layer].reshape(batch, -1)
            assert got.dtype == want.dtype == work
            d = (got.float() - want.float()).abs()
            print(f"step {t} layer {layer}: max={d.max().item():.3e}", flush=True)
            bar = 8 if work == torch.bfloat16 else 1  # bf16: the eps ratio 2^-7 / 2^-10
            assert d.max().item() <= bar * MAX_ABS and d.mean().item() <= bar * MEAN_ABS
            assert torch.equal(cache_g.keys[layer], cache_e.keys[layer])
            assert torch.equal(cache_g.values[layer], cache_e.values[layer])
        # Eager work of the program between replays.
        torch.ones(1 << 20, device=gpu).sum().item()


def test_graph_keeps_its_workspace_when_the_stream_cache_grows(gpu):
    """A captured step records its decode workspace's address. Calls outside
    the graph on the same stream may grow (replace) the stream's cached
    workspace, e.g. a prefill chunk over a long prefix, and the allocator may
    hand the old buffer to new tensors. The graph owns its workspace, so a
    replay after that writes nothing into those tensors and still matches
    the eager step."""
    layers, batch = 2, 6
    # Start from an empty stream cache (earlier tests may have grown it).
    hip_kernels._workspaces.clear()
    torch.cuda.empty_cache()
    cache_g, start, slot_lists, seq_tables, width, hq = setup(gpu, "pages", 16, layers, batch)
    cache_e, *_ = setup(gpu, "pages", 16, layers, batch)
    arenas = [(cache_g.keys[l], cache_g.values[l]) for l in range(layers)]
    # An eager decode call first, so the stream's cache holds a decode-sized buffer.
    q0 = torch.randn((batch, hq, 128), device=gpu, dtype=torch.float16)
    t0 = torch.as_tensor(np.array(slot_lists, dtype=np.int32), device=gpu)
    l0 = torch.as_tensor(start.astype(np.int32) + 1, device=gpu)
    hip_kernels.paged_decode_attention(q0, cache_g.keys[0], cache_g.values[0], t0, l0,
                                       page_size=16, longest=int(l0.max()), scale=0.1)
    torch.cuda.synchronize()
    step = DecodeStepGraph(arenas, seq_tables, batch=batch, q_heads=hq, page_size=16,
                           width=width, scale=128 ** -0.5, longest=int(start.max()) + 8,
                           dims=128, base=1e6)
    slots = np.arange(batch, dtype=np.int32)
    gen = torch.Generator(device=gpu).manual_seed(5)

    def load_step(t):
        positions = (start + t).astype(np.int32)
        step.slots.copy_(torch.as_tensor(slots, device=gpu))
        step.positions.copy_(torch.as_tensor(positions, device=gpu))
        qkv = []
        for layer in range(layers):
            q = torch.randn((batch, hq, 128), generator=gen, device=gpu).half()
            k = torch.randn((batch, 4, 128), generator=gen, device=gpu).half()
            v = torch.randn((batch, 4, 128), generator=gen, device=gpu).half()
            step.q[layer].copy_(q)
            step.k[layer].copy_(k)
            step.v[layer].copy_(v)
            qkv.append((q, k, v))
        return positions, qkv

    def check(positions, qkv):
        batch_e = DecodeBatch(cache_e, torch.zeros(batch, device=gpu), positions=positions,
                              tables={"full": [np.array(slot_lists[s]) for s in slots]})
        for layer, (q, k, v) in enumerate(qkv):
            want = batch_e.rope_attend(layer, q, k, v, dims=128, base=1e6, scale=128 ** -0.5)
            torch.cuda.synchronize()
            d = (step.out[layer].reshape(batch, -1).float() - want.float()).abs()
            assert d.max().item() <= MAX_ABS and d.mean().item() <= MEAN_ABS

    positions, qkv = load_step(0)
    step.capture()
    torch.cuda.synchronize()
    check(positions, qkv)
    before = hip_kernels.stream_workspace(gpu, 0)
    old_bytes, old_ptr = before.numel(), before.data_ptr()
    del before
    # A 512-token prefill chunk over a 32256-token prefix in 8 key ranges:
    # its partials (8 x 512 x 28 x 128 floats) need a workspace larger than
    # the decode call's, so the stream's cached buffer is replaced (and the
    # old one returned to the allocator).
    P, hkv, d, pos0, count = 16, 4, 128, 32256, 512
    pages = (pos0 + count) // P
    pk = torch.randn((pages, hkv, P, d), device=gpu, dtype=torch.float16)
    pv = torch.randn_like(pk)
    table = torch.as_tensor(np.random.default_rng(3).permutation(pages).astype(np.int32),
                            device=gpu)
    pq = torch.randn((count, hq, d), device=gpu, dtype=torch.float16)
    hip_kernels.paged_prefill_attention(pq, pk, pv, table, start=pos0, page_size=P,
                                        scale=d ** -0.5, splits=8)
    torch.cuda.synchronize()
    grown = hip_kernels.stream_workspace(gpu, 0)
    assert grown.numel() > old_bytes and grown.data_ptr() != old_ptr
    del grown
    # New tensors that may take the old buffer's memory, holding a pattern.
    sentinels = [torch.full((old_bytes // 4,), 7.0, device=gpu) for _ in range(3)]
    torch.cuda.synchronize()
    for t in (1, 2):
        positions, qkv = load_step(t)
        step.replay()
        torch.cuda.synchronize()
        check(positions, qkv)
        for s in sentinels:
            assert bool((s == 7.0).all()), "a replay wrote into memory it does not own"
