"""Parity of the paged prefill attention (pda_paged_prefill_attention via the
C-ABI) with the float64 prefill oracle (oracle/paged_attention.
paged_prefill_dense, pinned by tests/test_prefill_oracle.py) on the same
seeded inputs. Bar: max-abs 2e-3, mean-abs 2e-4 (the north star's FP16
bar), in both arena layouts."""

import numpy as np
import pytest
import torch

from instinct_amd.batches import PrefillBatch
from instinct_amd.hip_kernels import paged_prefill_attention
from instinct_amd.paged_kv import KVCache, KVGroup, pages_to_rows, rows_to_pages
from oracle import kv8
from oracle import paged_attention as pa

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-3
MEAN_ABS = 2e-4


def case(gpu, *, hq, hkv, d, start, count, page=16, layout="pages", seed=0, released=()):
    rng = np.random.default_rng(seed)
    pages = (start + count + page - 1) // page
    arena_pages = pages + 5
    table = rng.permutation(arena_pages)[:pages].astype(np.int32)
    for i in released:
        table[i] = -1
    keys = rng.standard_normal((arena_pages * page, hkv, d)).astype(np.float16)
    values = rng.standard_normal((arena_pages * page, hkv, d)).astype(np.float16)
    q = rng.standard_normal((count, hq, d)).astype(np.float16)
    k_dev = torch.as_tensor(keys, device=gpu)
    v_dev = torch.as_tensor(values, device=gpu)
    if layout == "pages":
        k_dev, v_dev = rows_to_pages(k_dev, page), rows_to_pages(v_dev, page)
    return dict(q=q, keys=keys, values=values, table=table, page=page, start=start,
                t=(torch.as_tensor(q, device=gpu), k_dev, v_dev,
                   torch.as_tensor(table, device=gpu)))


def check(c, *, scale, window=0, softcap=0.0, splits=0, images=(), what=""):
    q, k, v, table = c["t"]
    got = paged_prefill_attention(q, k, v, table, start=c["start"], page_size=c["page"],
                                  scale=scale, window=window, softcap=softcap, splits=splits,
                                  images=images)
    torch.cuda.synchronize()
    got = got.float().cpu().numpy()
    assert np.isfinite(got).all(), f"{what}: non-finite"
    want = pa.paged_prefill_dense(c["q"], c["keys"], c["values"], c["table"], start=c["start"],
                                  page_size=c["page"], scale=scale, window=window,
                                  softcap=softcap, images=images)
    err_max, err_mean = pa.error_stats(got, want)
    print(f"{what}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}", flush=True)
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS, (what, err_max, err_mean)


@pytest.mark.parametrize("layout", ["pages", "rows"])
@pytest.mark.parametrize("hq,hkv,d", [(28, 4, 128), (14, 2, 64), (8, 4, 256), (32, 8, 128)])
def test_head_shapes(gpu, layout, hq, hkv, d):
    c = case(gpu, hq=hq, hkv=hkv, d=d, start=37, count=300, layout=layout, seed=d + hq)
    check(c, scale=d ** -0.5, what=f"{hq}/{hkv} D{d} {layout}")


@pytest.mark.parametrize("start,count", [(0, 1), (0, 5), (0, 128), (0, 129), (1000, 64),
                                         (5, 1024), (4095, 1)])
def test_chunk_positions(gpu, start, count):
    c = case(gpu, hq=28, hkv=4, d=128, start=start, count=count, seed=start + count)
    check(c, scale=128 ** -0.5, what=f"start {start} count {count}")


@pytest.mark.parametrize("layout", ["pages", "rows"])
@pytest.mark.parametrize("page,d", [(8, 128), (32, 128), (48, 128), (64, 128), (128, 128),
                                    (16, 256), (64, 256), (48, 64)])
def test_page_sizes(gpu, layout, page, d):
    """Page sizes that divide the key tile (the page cursor steps by a
    constant) and that do not (it divides per tile), with and without key
    ranges."""
    c = case(gpu, hq=8, hkv=2, d=d, start=333, count=260, page=page, layout=layout,
             seed=page + d)
    check(c, scale=d ** -0.5, what=f"page {page} D{d} {layout}")
    check(c, scale=d ** -0.5, splits=3, what=f"page {page} D{d} {layout} splits 3")


def test_window_softcap_and_released_pages(gpu):
    c = case(gpu, hq=8, hkv=4, d=256, start=900, count=200, seed=7)
    check(c, scale=256 ** -0.5, window=128, what="window 128")
    check(c, scale=256 ** -0.5, window=1, what="window 1 (only itself)")
    c = case(gpu, hq=16, hkv=2, d=128, start=0, count=400, seed=8)
    check(c, scale=128 ** -0.5, softcap=30.0, what="softcap")
    # Pages released before the window of every query are never visible.
    c = case(gpu, hq=8, hkv=4, d=128, start=2000, count=64, seed=9, released=(0, 1, 2, 3))
    check(c, scale=128 ** -0.5, window=512, what="released pages outside the window")


@pytest.mark.parametrize("splits", [2, 3, 7, 64])
def test_forced_key_ranges(gpu, splits):
    """The key split and its merge: any number of ranges, including more
    ranges than key tiles (empty ranges), gives the oracle's result."""
    c = case(gpu, hq=28, hkv=4, d=128, start=37, count=300, seed=20 + splits)
    check(c, scale=128 ** -0.5, splits=splits, what=f"splits {splits}")


@pytest.mark.parametrize("d", [64, 96, 256, 512])
def test_forced_key_ranges_head_dims(gpu, d):
    c = case(gpu, hq=8, hkv=2, d=d, start=500, count=200, seed=d)
    check(c, scale=d ** -0.5, splits=3, what=f"D{d} splits 3")
    # More ranges than key tiles: empty ranges leave m = -inf partials.
    check(c, scale=d ** -0.5, splits=64, what=f"D{d} splits 64")


def test_key_ranges_with_window_and_released_pages(gpu):
    # Ranges wholly outside every query's window, or on released pages, are
    # empty partials (max -inf) that the merge skips.
    c = case(gpu, hq=8, hkv=4, d=128, start=2000, count=64, seed=21, released=(0, 1, 2, 3))
    check(c, scale=128 ** -0.5, window=512, splits=5, what="window 512, released, splits 5")
    c = case(gpu, hq=16, hkv=2, d=128, start=0, count=400, seed=22)
    check(c, scale=128 ** -0.5, softcap=30.0, splits=4, what="softcap, splits 4")


def test_long_prefix_chunk_splits_automatically(gpu):
    """A chunk over a long prefix (the reference prefills 512-token chunks,
    mlx_engine.py:74,430): the library splits the keys on its own."""
    from instinct_amd import _lib

    splits, _ = _lib.prefill_workspace_bytes(3000, 256, 8, 128)
    assert splits > 1
    c = case(gpu, hq=8, hkv=2, d=128, start=3000, count=256, seed=23)
    check(c, scale=128 ** -0.5, what=f"start 3000 count 256 (auto, {splits} ranges)")


def test_long_chunk(gpu):
    c = case(gpu, hq=28, hkv=4, d=128, start=0, count=4096, seed=10)
    check(c, scale=128 ** -0.5, what="4096-token chunk")


@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_prefill_batch_chunks_then_decode(gpu, layout):
    """PrefillBatch in two chunks writes the prompt's K/V and attends like the
    oracle over the whole prompt (batches.py:84-132)."""
    page, hq, hkv, d = 16, 14, 2, 64
    groups = [KVGroup("full", (0,), kv_heads=hkv, head_dim=d)]
    cache = KVCache(groups, page_size=page, capacities={"full": 64}, device=gpu, layout=layout)
    n = 300
    table = np.array([cache.pools["full"].allocate(reserved=False)
                      for _ in range((n + page - 1) // page)])
    gen = torch.Generator(device=gpu).manual_seed(6)
    q = torch.randn((n, hq, d), generator=gen, device=gpu).half()
    k = torch.randn((n, hkv, d), generator=gen, device=gpu).half()
    v = torch.randn((n, hkv, d), generator=gen, device=gpu).half()
    outs = []
    for a, b in ((0, 170), (170, n)):
        chunk = PrefillBatch(cache, torch.zeros(b - a, device=gpu), start=a,
                             tables={"full": table})
        outs.append(chunk.attend(0, q[a:b], k[a:b], v[a:b], scale=d ** -0.5))
    torch.cuda.synchronize()
    got = torch.cat(outs).view(n, hq, d).float().cpu().numpy()
    keys, values = cache.keys[0], cache.values[0]
    if layout == "pages":
        keys, values = pages_to_rows(keys), pages_to_rows(values)
    want = pa.paged_prefill_dense(q.cpu().numpy(), keys.cpu().numpy(), values.cpu().numpy(),
                                  table, start=0, page_size=page, scale=d ** -0.5)
    err_max, err_mean = pa.error_stats(got, want)
    print(f"PrefillBatch {layout}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}")
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS


def scales_to_pages(scales: torch.Tensor, page_size: int) -> torch.Tensor:
    """[rows, kv_heads] -> [pages, kv_heads, page_size]."""
    rows, heads = scales.shape
    return scales.view(rows // page_size, page_size, heads).permute(0, 2, 1).contiguous()


@pytest.mark.parametrize("layout", ["pages", "rows"])
@pytest.mark.parametrize("hq,hkv,d,splits,window,page", [
    (28, 4, 128, 0, 0, 16), (28, 4, 128, 3, 0, 16), (14, 2, 64, 2, 0, 48),
    (8, 4, 256, 0, 0, 16), (16, 8, 256, 2, 512, 64), (8, 2, 128, 0, 100, 128),
])
def test_8bit_cache(gpu, layout, hq, hkv, d, splits, window, page):
    """An 8-bit cache (int8 rows, one fp16 scale per (row, kv head), as
    KVCache(bits=8) holds them, paged_kv.py:50-55): attention over the rows
    the reference's gather dequantizes (oracle kv8.gather_dequantize)."""
    rng = np.random.default_rng(d + hq + page)
    start, count = 700, 300
    pages = (start + count + page - 1) // page
    arena_pages = pages + 3
    table = rng.permutation(arena_pages)[:pages].astype(np.int32)
    rows = arena_pages * page
    kq, ks = kv8.quantize(rng.standard_normal((rows, hkv, d)).astype(np.float16))
    vq, vs = kv8.quantize(rng.standard_normal((rows, hkv, d)).astype(np.float16))
    q = rng.standard_normal((count, hq, d)).astype(np.float16)
    keys, values = torch.as_tensor(kq, device=gpu), torch.as_tensor(vq, device=gpu)
    k_s, v_s = torch.as_tensor(ks, device=gpu), torch.as_tensor(vs, device=gpu)
    if layout == "pages":
        keys, values = rows_to_pages(keys, page), rows_to_pages(values, page)
        k_s, v_s = scales_to_pages(k_s, page), scales_to_pages(v_s, page)
    got = paged_prefill_attention(torch.as_tensor(q, device=gpu), keys, values,
                                  torch.as_tensor(table, device=gpu), start=start,
                                  page_size=page, scale=d ** -0.5, window=window,
                                  splits=splits, scales=(k_s, v_s))
    torch.cuda.synchronize()
    want = pa.paged_prefill_dense(q, kv8.gather_dequantize(kq, ks),
                                  kv8.gather_dequantize(vq, vs), table, start=start,
                                  page_size=page, scale=d ** -0.5, window=window)
    err_max, err_mean = pa.error_stats(got.float().cpu().numpy(), want)
    print(f"8-bit {hq}/{hkv} D{d} page {page} {layout}: max_abs={err_max:.3e} "
          f"mean_abs={err_mean:.3e}", flush=True)
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS


@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_prefill_batch_8bit(gpu, layout):
    """PrefillBatch over KVCache(bits=8): the chunks' K/V are quantized on
    write (pda_rope_append_q8, rows = the chunk's positions), then attended
    over the dequantized rows; two chunks against the oracle on the cache's
    own int8 rows and scales."""
    page, hq, hkv, d = 16, 14, 2, 64
    groups = [KVGroup("full", (0,), kv_heads=hkv, head_dim=d)]
    cache = KVCache(groups, page_size=page, capacities={"full": 64}, device=gpu, layout=layout,
                    bits=8)
    n = 300
    table = np.array([cache.pools["full"].allocate(reserved=False)
                      for _ in range((n + page - 1) // page)])
    gen = torch.Generator(device=gpu).manual_seed(7)
    q = torch.randn((n, hq, d), generator=gen, device=gpu).half()
    k = torch.randn((n, hkv, d), generator=gen, device=gpu).half()
    v = torch.randn((n, hkv, d), generator=gen, device=gpu).half()
    outs = []
    for a, b in ((0, 130), (130, n)):
        chunk = PrefillBatch(cache, torch.zeros(b - a, device=gpu), start=a,
                             tables={"full": table})
        outs.append(chunk.attend(0, q[a:b], k[a:b], v[a:b], scale=d ** -0.5))
    torch.cuda.synchronize()
    got = torch.cat(outs).view(n, hq, d).float().cpu().numpy()
    keys, values = cache.keys[0], cache.values[0]
    k_s, v_s = cache.key_scales[0], cache.value_scales[0]
    if layout == "pages":
        keys, values = pages_to_rows(keys), pages_to_rows(values)
        k_s = k_s.permute(0, 2, 1).reshape(-1, hkv)
        v_s = v_s.permute(0, 2, 1).reshape(-1, hkv)
    kq, vq = keys.cpu().numpy(), values.cpu().numpy()
    ks, vs = k_s.cpu().numpy(), v_s.cpu().numpy()
    # The write quantized the chunks' rows as the oracle does.
    rows = np.concatenate([table[p // page] * page + np.arange(p % page, min(page, n - p))
                           for p in range(0, n, page)])
    want_kq, want_ks = kv8.quantize(k.cpu().numpy())
    np.testing.assert_array_equal(vq[rows], kv8.quantize(v.cpu().numpy())[0])
    np.testing.assert_array_equal(ks[rows], want_ks)
    assert np.abs(kq[rows].astype(int) - want_kq.astype(int)).max() <= 0
    want = pa.paged_prefill_dense(q.cpu().numpy(), kv8.gather_dequantize(kq, ks),
                                  kv8.gather_dequantize(vq, vs), table, start=0,
                                  page_size=page, scale=d ** -0.5)
    err_max, err_mean = pa.error_stats(got, want)
    print(f"PrefillBatch 8-bit {layout}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}")
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS


@pytest.mark.parametrize("splits", [0, 3])
@pytest.mark.parametrize("hq,hkv,d", [(28, 4, 128), (14, 2, 64), (8, 4, 256)])
def test_image_spans(gpu, hq, hkv, d, splits):
    """Image tokens see their whole image (batches.py:107-118): spans inside
    one wave's queries, across waves and across 128-query workgroup tiles,
    one at the chunk's end, with and without key ranges."""
    c = case(gpu, hq=hq, hkv=hkv, d=d, start=100, count=420, seed=30 + d + splits)
    images = [(110, 7), (150, 40), (220, 200), (500, 20)]
    check(c, scale=d ** -0.5, splits=splits, images=images,
          what=f"images {hq}/{hkv} D{d} splits {splits}")


def test_image_spans_with_window_and_8bit(gpu):
    # An image longer than the window: its tokens see all of it.
    c = case(gpu, hq=8, hkv=2, d=128, start=1000, count=300, seed=41)
    check(c, scale=128 ** -0.5, window=64, images=[(1010, 150), (1200, 3)],
          what="images with window 64")
    check(c, scale=128 ** -0.5, window=64, splits=4, images=[(1010, 150)],
          what="images with window 64, splits 4")
    # Spans outside the chunk change nothing; an empty span is ignored.
    check(c, scale=128 ** -0.5, images=[(0, 500), (1400, 0)], what="images outside the chunk")


@pytest.mark.parametrize("bits", [16, 8])
def test_prefill_batch_images(gpu, bits):
    """PrefillBatch with an image (as (at, embeddings)): inject puts the
    embeddings in place; attention lets the image's tokens see all of it."""
    page, hq, hkv, d = 16, 8, 2, 128
    groups = [KVGroup("full", (0,), kv_heads=hkv, head_dim=d)]
    cache = KVCache(groups, page_size=page, capacities={"full": 64}, device=gpu, bits=bits)
    n = 260
    table = np.array([cache.pools["full"].allocate(reserved=False)
                      for _ in range((n + page - 1) // page)])
    gen = torch.Generator(device=gpu).manual_seed(9)
    q = torch.randn((n, hq, d), generator=gen, device=gpu).half()
    k = torch.randn((n, hkv, d), generator=gen, device=gpu).half()
    v = torch.randn((n, hkv, d), generator=gen, device=gpu).half()
    embeddings = torch.randn((64, 32), generator=gen, device=gpu)
    batch = PrefillBatch(cache, torch.zeros(n, device=gpu), start=0, tables={"full": table},
                         images=[(70, embeddings)])
    x = torch.zeros((n, 32), device=gpu)
    assert torch.equal(batch.inject(x)[70:134], embeddings) and not x[:70].any()
    got = batch.attend(0, q, k, v, scale=d ** -0.5).view(n, hq, d).float().cpu().numpy()
    keys, values = pages_to_rows(cache.keys[0]), pages_to_rows(cache.values[0])
    kn, vn = keys.cpu().numpy(), values.cpu().numpy()
    if bits == 8:
        ks = cache.key_scales[0].permute(0, 2, 1).reshape(-1, hkv).cpu().numpy()
        vs = cache.value_scales[0].permute(0, 2, 1).reshape(-1, hkv).cpu().numpy()
        kn, vn = kv8.gather_dequantize(kn, ks), kv8.gather_dequantize(vn, vs)
    want = pa.paged_prefill_dense(q.cpu().numpy(), kn, vn, table, start=0, page_size=page,
                                  scale=d ** -0.5, images=[(70, 64)])
    err_max, err_mean = pa.error_stats(got, want)
    print(f"PrefillBatch images {bits}-bit: max_abs={err_max:.3e} mean_abs={err_mean:.3e}")
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS


def test_image_span_at_every_position(gpu):
    """Regression: a query whose only visible keys in a tile come from its
    image span, at every slot of the score layout (spans of 2 and 5 tokens
    at each position of two workgroup tiles, crossing every 4-key group,
    wave and tile boundary)."""
    c = case(gpu, hq=2, hkv=1, d=64, start=0, count=200, seed=12)
    q, k, v, table = c["t"]
    worst = 0.0
    for n in (2, 5):
        for a in range(0, 200 - n + 1):
            got = paged_prefill_attention(q, k, v, table, start=0, page_size=16, scale=0.125,
                                          images=[(a, n)]).float().cpu().numpy()
            want = pa.paged_prefill_dense(c["q"], c["keys"], c["values"], c["table"], start=0,
                                          page_size=16, scale=0.125, images=[(a, n)])
            err = float(np.abs(got - want).max())
            worst = max(worst, err)
            assert err <= MAX_ABS, (a, n, err)
    print(f"image spans at every position: worst max_abs={worst:.3e}")


# --- 512-wide heads (Gemma 4's global layers): four waves split the head dim --

@pytest.mark.parametrize("layout", ["pages", "rows"])
@pytest.mark.parametrize("hq,hkv,start,count", [
    (16, 2, 0, 300), (8, 1, 700, 65), (4, 4, 31, 1), (16, 2, 4000, 96)])
def test_head_dim_512(gpu, layout, hq, hkv, start, count):
    c = case(gpu, hq=hq, hkv=hkv, d=512, start=start, count=count, layout=layout,
             seed=hq + start + count)
    check(c, scale=512 ** -0.5, what=f"D512 {hq}/{hkv} @{start}+{count} {layout}")


def test_head_dim_512_ranges_window_softcap_images(gpu):
    c = case(gpu, hq=8, hkv=2, d=512, start=1500, count=200, page=32, seed=77, released=(0, 3))
    check(c, scale=512 ** -0.5, window=300, softcap=50.0, what="D512 window+softcap")
    for splits in (2, 5):
        check(c, scale=512 ** -0.5, window=300, splits=splits,
              what=f"D512 window, {splits} ranges")
    c = case(gpu, hq=8, hkv=2, d=512, start=100, count=180, seed=78)
    check(c, scale=512 ** -0.5, images=[(110, 7), (150, 70), (270, 10)],
          what="D512 image spans")
    check(c, scale=512 ** -0.5, splits=3, images=[(150, 70)], what="D512 images, 3 ranges")


def test_head_dim_512_long_prefix_splits_automatically(gpu):
    from instinct_amd import _lib

    assert _lib.prefill_workspace_bytes(6000, 64, 8, 512)[0] > 1
    c = case(gpu, hq=8, hkv=1, d=512, start=6000, count=64, seed=79)
    check(c, scale=512 ** -0.5, what="D512 64@6000 auto split")


@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_head_dim_512_8bit_cache(gpu, layout):
    page, hq, hkv, d, start, count = 16, 8, 2, 512, 300, 140
    c = case(gpu, hq=hq, hkv=hkv, d=d, start=start, count=count, seed=80, layout="rows")
    q, k16, v16, table = c["t"]
    s8 = []
    for x in (k16, v16):
        scale = (x.float().abs().amax(-1).clamp(min=1e-4) / 127.0).half()
        s8.append((scale, (x.float() / scale.float()[..., None]).round().clamp(-127, 127)
                   .to(torch.int8)))
    (ks, kq), (vs, vq) = s8
    want = pa.paged_prefill_dense(c["q"], kv8.gather_dequantize(kq.cpu().numpy(), ks.cpu().numpy()),
                                  kv8.gather_dequantize(vq.cpu().numpy(), vs.cpu().numpy()),
                                  c["table"], start=start, page_size=page, scale=d ** -0.5)
    if layout == "pages":
        kq, vq = rows_to_pages(kq, page), rows_to_pages(vq, page)
        ks, vs = scales_to_pages(ks, page), scales_to_pages(vs, page)
    got = paged_prefill_attention(q, kq, vq, table, start=start, page_size=page,
                                  scale=d ** -0.5, scales=(ks, vs))
    torch.cuda.synchronize()
    err_max, err_mean = pa.error_stats(got.float().cpu().numpy(), want)
    print(f"D512 8-bit {layout}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}", flush=True)
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS


@pytest.mark.parametrize("layout", ["pages", "rows"])
@pytest.mark.parametrize("start,count,splits", [(0, 300, 0), (900, 130, 3), (4000, 64, 0)])
def test_head_dim_96(gpu, layout, start, count, splits):
    """96-wide heads (padded V rows, a merge block with idle threads)."""
    c = case(gpu, hq=32, hkv=8, d=96, start=start, count=count, layout=layout,
             seed=start + count)
    check(c, scale=96 ** -0.5, splits=splits,
          what=f"D96 @{start}+{count} s{splits} {layout}")
    check(c, scale=96 ** -0.5, window=200, softcap=30.0, images=[(start + 5, 20)],
          what=f"D96 window+softcap+image {layout}")


@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_global_layer_512_wide_quarter_rotation(gpu, layout):
    """A Gemma 4 global layer end to end (gemma4.py:49-75): 512-wide heads
    whose first quarter of dims is rotated. PrefillBatch in two chunks (the
    model's rope, then attend), then two DecodeBatch.rope_attend steps, each
    against the RoPE oracle and the attention oracle over the arena the
    kernels wrote."""
    from instinct_amd.batches import DecodeBatch
    from oracle import rope_append as ra

    page, hq, hkv, d, dims, base = 16, 8, 2, 512, 128, 1e6
    groups = [KVGroup("full", (0,), kv_heads=hkv, head_dim=d)]
    cache = KVCache(groups, page_size=page, capacities={"full": 32}, device=gpu, layout=layout)
    n = 200
    table = np.array([cache.pools["full"].allocate(reserved=False) for _ in range(16)])
    gen = torch.Generator(device=gpu).manual_seed(12)
    q = torch.randn((n + 2, hq, d), generator=gen, device=gpu).half()
    k = torch.randn((n + 2, hkv, d), generator=gen, device=gpu).half()
    v = torch.randn((n + 2, hkv, d), generator=gen, device=gpu).half()
    inverse = ra.inv_freq(dims, base=base)

    def arena():
        keys, values = cache.keys[0], cache.values[0]
        if layout == "pages":
            keys, values = pages_to_rows(keys), pages_to_rows(values)
        return keys.cpu().numpy(), values.cpu().numpy()

    outs, q_rots = [], []
    for a, b in ((0, 120), (120, n)):
        chunk = PrefillBatch(cache, torch.zeros(b - a, device=gpu), start=a,
                             tables={"full": table})
        q_rot = chunk.rope(q[a:b], dims, base=base)
        k_rot = chunk.rope(k[a:b], dims, base=base)
        pos = np.arange(a, b, dtype=np.int32)
        np.testing.assert_array_equal(
            k_rot.cpu().numpy()[..., dims:], k[a:b].cpu().numpy()[..., dims:])
        assert np.abs(q_rot.cpu().numpy().astype(np.float64)
                      - ra.rope(q[a:b].cpu().numpy(), pos, dims, inverse)).max() <= 2e-3
        q_rots.append(q_rot)
        outs.append(chunk.attend(0, q_rot, k_rot, v[a:b], scale=d ** -0.5))
    torch.cuda.synchronize()
    keys, values = arena()
    want = pa.paged_prefill_dense(torch.cat(q_rots).cpu().numpy(), keys, values, table,
                                  start=0, page_size=page, scale=d ** -0.5)
    err_max, err_mean = pa.error_stats(torch.cat(outs).view(n, hq, d).float().cpu().numpy(),
                                       want)
    print(f"D512 global layer prefill {layout}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}")
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS
    for t in (n, n + 1):
        step = DecodeBatch(cache, torch.zeros(1, device=gpu), positions=np.array([t]),
                           tables={"full": [table]})
        out = step.rope_attend(0, q[t:t + 1], k[t:t + 1], v[t:t + 1], dims=dims, base=base,
                               scale=d ** -0.5)
        torch.cuda.synchronize()
        keys, values = arena()
        q_rot = ra.rope(q[t:t + 1].cpu().numpy(), np.array([t], np.int32), dims, inverse)
        want = pa.paged_decode_dense(q_rot, keys, values, table[None].astype(np.int32),
                                     np.array([t + 1], np.int32), page_size=page,
                                     scale=d ** -0.5)
        err_max, err_mean = pa.error_stats(out.view(1, hq, d).float().cpu().numpy(), want)
        print(f"D512 global layer decode step {t} {layout}: max_abs={err_max:.3e}")
        assert err_max <= MAX_ABS and err_mean <= MEAN_ABS
