"""Prefill at every head dim the decode call takes: any head_dim up to 512
(the reference's PrefillBatch attends with whatever head dim the model has,
batches.py:84-132, and its CUDA test prefills head_dim 4,
tests/cuda_tests.cu:207-262). Head dims without a kernel of their own run
the next wider one (64, 96, 128, 256, 512) with the elements past the head
dim zero; odd ones move single elements (paged_prefill_odd_kernel). Checked against the float64 prefill oracle at the north star's fp16
bar (max-abs 2e-3, mean-abs 2e-4), bf16 at the bar of test_gpu_bf16.py, in
both arena layouts, with key ranges, windows, softcap, images, 8-bit caches,
and the reference's closed form at its own page size."""

import numpy as np
import pytest
import torch

from instinct_amd.batches import PrefillBatch
from instinct_amd.hip_kernels import paged_decode_attention, paged_prefill_attention
from instinct_amd.paged_kv import KVCache, KVGroup, pages_to_rows, rows_to_pages
from oracle import kv8
from oracle import paged_attention as pa

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-3
MEAN_ABS = 2e-4
BF16_MAX_ABS = 1.6e-2
BF16_MEAN_ABS = 1.6e-3


def bf16_round(a):
    return torch.as_tensor(a).to(torch.bfloat16).float().numpy()


def case(gpu, *, hq, hkv, d, start, count, page=16, layout="pages", seed=0, bf16=False):
    rng = np.random.default_rng(seed)
    pages = (start + count + page - 1) // page
    arena_pages = pages + 5
    table = rng.permutation(arena_pages)[:pages].astype(np.int32)
    draw = lambda shape: rng.standard_normal(shape).astype(np.float32)  # noqa: E731
    keys, values = draw((arena_pages * page, hkv, d)), draw((arena_pages * page, hkv, d))
    q = draw((count, hq, d))
    if bf16:
        keys, values, q = bf16_round(keys), bf16_round(values), bf16_round(q)
        dev = lambda a: torch.as_tensor(a, device=gpu).to(torch.bfloat16)  # noqa: E731
    else:
        keys, values, q = (x.astype(np.float16) for x in (keys, values, q))
        dev = lambda a: torch.as_tensor(a, device=gpu)  # noqa: E731
    k_dev, v_dev = dev(keys), dev(values)
    if layout == "pages":
        k_dev, v_dev = rows_to_pages(k_dev, page), rows_to_pages(v_dev, page)
    return dict(q=q, keys=keys, values=values, table=table, page=page, start=start,
                t=(dev(q), k_dev, v_dev, torch.as_tensor(table, device=gpu)))


def check(c, *, scale, window=0, softcap=0.0, splits=0, images=(), what="", bf16=False):
    q, k, v, table = c["t"]
    got = paged_prefill_attention(q, k, v, table, start=c["start"], page_size=c["page"],
                                  scale=scale, window=window, softcap=softcap, splits=splits,
                                  images=images)
    torch.cuda.synchronize()
    assert got.shape == q.shape and got.dtype == q.dtype
    got = got.float().cpu().numpy()
    assert np.isfinite(got).all(), f"{what}: non-finite"
    want = pa.paged_prefill_dense(c["q"], c["keys"], c["values"], c["table"], start=c["start"],
                                  page_size=c["page"], scale=scale, window=window,
                                  softcap=softcap, images=images)
    err_max, err_mean = pa.error_stats(got, want)
    print(f"{what}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}", flush=True)
    bar = (BF16_MAX_ABS, BF16_MEAN_ABS) if bf16 else (MAX_ABS, MEAN_ABS)
    assert err_max <= bar[0] and err_mean <= bar[1], (what, err_max, err_mean)


@pytest.mark.parametrize("layout", ["pages", "rows"])
@pytest.mark.parametrize("d", [2, 4, 36, 48, 80, 100, 112, 160, 200, 320, 510,
                               1, 3, 7, 65, 97, 129, 257, 511])
def test_generic_head_dims(gpu, layout, d):
    hq, hkv = (12, 4) if d <= 256 else (8, 2)
    c = case(gpu, hq=hq, hkv=hkv, d=d, start=300, count=260, layout=layout, seed=d)
    check(c, scale=d ** -0.5, what=f"D{d} {layout}")
    check(c, scale=d ** -0.5, splits=3, what=f"D{d} {layout} splits 3")


@pytest.mark.parametrize("d", [80, 200, 81])
def test_generic_window_softcap_images(gpu, d):
    c = case(gpu, hq=8, hkv=2, d=d, start=1000, count=300, page=32, seed=40 + d)
    check(c, scale=d ** -0.5, window=100, softcap=30.0, what=f"D{d} window 100 softcap")
    check(c, scale=d ** -0.5, window=64, splits=4, images=[(1010, 150), (1200, 3)],
          what=f"D{d} images window 64 splits 4")
    check(c, scale=d ** -0.5, splits=64, what=f"D{d} splits 64 (empty ranges)")


@pytest.mark.parametrize("d", [80, 5])
@pytest.mark.parametrize("page", [1, 5, 48])
def test_generic_page_sizes(gpu, page, d):
    c = case(gpu, hq=6, hkv=2, d=d, start=123, count=200, page=page, layout="rows",
             seed=page + d)
    check(c, scale=d ** -0.5, what=f"D{d} page {page}")
    check(c, scale=d ** -0.5, splits=2, what=f"D{d} page {page} splits 2")


@pytest.mark.parametrize("layout", ["pages", "rows"])
@pytest.mark.parametrize("d,splits", [(80, 0), (36, 3), (200, 2), (320, 0), (7, 0), (129, 3),
                                      (511, 0)])
def test_generic_8bit_cache(gpu, layout, d, splits):
    """int8 rows with one fp16 scale per (row, kv head), dequantized as the
    reference's gather does (oracle kv8.gather_dequantize)."""
    page, hq, hkv, start, count = 16, 8, 2, 500, 200
    rng = np.random.default_rng(d + splits)
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
        k_s = k_s.view(-1, page, hkv).permute(0, 2, 1).contiguous()
        v_s = v_s.view(-1, page, hkv).permute(0, 2, 1).contiguous()
    got = paged_prefill_attention(torch.as_tensor(q, device=gpu), keys, values,
                                  torch.as_tensor(table, device=gpu), start=start,
                                  page_size=page, scale=d ** -0.5, splits=splits,
                                  scales=(k_s, v_s))
    torch.cuda.synchronize()
    want = pa.paged_prefill_dense(q, kv8.gather_dequantize(kq, ks),
                                  kv8.gather_dequantize(vq, vs), table, start=start,
                                  page_size=page, scale=d ** -0.5)
    err_max, err_mean = pa.error_stats(got.float().cpu().numpy(), want)
    print(f"8-bit D{d} splits {splits} {layout}: max_abs={err_max:.3e} "
          f"mean_abs={err_mean:.3e}", flush=True)
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS


@pytest.mark.parametrize("d,splits", [(80, 0), (200, 3), (4, 0), (33, 2), (257, 0)])
def test_generic_bf16(gpu, d, splits):
    c = case(gpu, hq=8, hkv=2, d=d, start=700, count=200, seed=d, bf16=True)
    check(c, scale=d ** -0.5, splits=splits, bf16=True, what=f"bf16 D{d} splits {splits}")


@pytest.mark.parametrize("d", [64, 96, 128, 256, 512])
def test_running_max_moves_and_far_negative_scores(gpu, d):
    """Scores that keep outgrowing the running max (key rows scaled up with
    their position: the lazy max moves again and again mid-chunk, the
    accumulators rescaled each time) and scores far below zero (every score
    near -100 in log2 units, where weights taken against a max of zero would
    all underflow), causal and with a window, against the float64 oracle.
    Such peaked weights make an output nearly one value row, so the rows
    are halved: the fp16 rounding of the output stays well inside the bar."""
    def halve_values(c):
        c["values"] = (c["values"].astype(np.float32) * 0.5).astype(np.float16)
        v_dev = rows_to_pages(torch.as_tensor(c["values"], device=gpu), c["page"])
        c["t"] = (c["t"][0], c["t"][1], v_dev, c["t"][3])

    c = case(gpu, hq=8, hkv=2, d=d, start=300, count=700, seed=5)
    halve_values(c)
    rows = c["keys"].shape[0]
    grow = (1.0 + np.arange(rows, dtype=np.float32) / 96.0)[:, None, None]
    c["keys"] = (c["keys"].astype(np.float32) * grow).astype(np.float16)
    q_dev, _, v_dev, table = c["t"]
    k_dev = rows_to_pages(torch.as_tensor(c["keys"], device=gpu), c["page"])
    c["t"] = (q_dev, k_dev, v_dev, table)
    check(c, scale=d ** -0.5, what=f"D{d} growing keys")
    check(c, scale=d ** -0.5, window=200, splits=3, what=f"D{d} growing keys, window, splits 3")
    c = case(gpu, hq=8, hkv=2, d=d, start=100, count=500, seed=6)
    halve_values(c)
    q, k = c["q"].astype(np.float32), c["keys"].astype(np.float32)
    q[..., 0], k[..., 0] = 24.0, -24.0
    c["q"], c["keys"] = q.astype(np.float16), k.astype(np.float16)
    q_dev = torch.as_tensor(c["q"], device=gpu)
    k_dev = rows_to_pages(torch.as_tensor(c["keys"], device=gpu), c["page"])
    c["t"] = (q_dev, k_dev, c["t"][2], c["t"][3])
    check(c, scale=8.0 * d ** -0.5, what=f"D{d} far negative scores")


def test_closed_form_from_cuda_tests(gpu):
    """tests/cuda_tests.cu:207-262 at its own shape: head_dim 4, page size 2,
    tokens 0, 1 in physical page 1 and token 2 in page 0. The prefill of the
    three tokens (query (1,1,0,0) at token 2) gives the known answer there,
    agrees with the decode call, and token 0 sees only its own value row.
    Tolerance 2^-8: half an fp16 ulp of the output in [4, 8) (2^-9) plus
    the fp16 probabilities' rounding (2^-11 relative, times |v - out| <= 4)."""
    q, keys, values, tables, lengths, page, scale, expected = pa.cuda_closed_form_case()
    tol = 2.0 ** -8
    f16 = lambda a: torch.as_tensor(np.asarray(a, np.float16), device=gpu)  # noqa: E731
    qs = np.concatenate([np.zeros((2, 1, 4)), q], axis=0)
    table = torch.as_tensor(tables[0], device=gpu)
    for layout in ("rows", "pages"):
        k, v = f16(keys), f16(values)
        if layout == "pages":
            k, v = rows_to_pages(k, page), rows_to_pages(v, page)
        out = paged_prefill_attention(f16(qs), k, v, table, start=0, page_size=page,
                                      scale=scale)
        dec = paged_decode_attention(f16(q), k, v, torch.as_tensor(tables, device=gpu),
                                     torch.as_tensor(lengths, device=gpu), page_size=page,
                                     longest=3, scale=scale)
        torch.cuda.synchronize()
        out = out.float().cpu().numpy()
        np.testing.assert_allclose(out[2, 0], expected, atol=tol)
        np.testing.assert_allclose(out[0, 0], [1, 2, 3, 4], atol=tol)
        np.testing.assert_allclose(out[1, 0], [3, 4, 5, 6], atol=tol)  # q = 0: the mean
        np.testing.assert_allclose(dec.float().cpu().numpy()[0, 0], out[2, 0], atol=tol)


@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_prefill_batch_then_decode_head_dim_80(gpu, layout):
    """A head_dim-80 model end to end: PrefillBatch in two chunks writes and
    attends the prompt, then a decode at the next position over the same
    cache; both against the oracle on the cache's rows."""
    page, hq, hkv, d = 16, 10, 2, 80
    groups = [KVGroup("full", (0,), kv_heads=hkv, head_dim=d)]
    cache = KVCache(groups, page_size=page, capacities={"full": 64}, device=gpu, layout=layout)
    n = 300
    table = np.array([cache.pools["full"].allocate(reserved=False)
                      for _ in range((n + page) // page)])
    gen = torch.Generator(device=gpu).manual_seed(11)
    q = torch.randn((n + 1, hq, d), generator=gen, device=gpu).half()
    k = torch.randn((n + 1, hkv, d), generator=gen, device=gpu).half()
    v = torch.randn((n + 1, hkv, d), generator=gen, device=gpu).half()
    outs = []
    for a, b in ((0, 170), (170, n)):
        chunk = PrefillBatch(cache, torch.zeros(b - a, device=gpu), start=a,
                             tables={"full": table})
        outs.append(chunk.attend(0, q[a:b], k[a:b], v[a:b], scale=d ** -0.5))
    torch.cuda.synchronize()
    got = torch.cat(outs).view(n, hq, d).float().cpu().numpy()
    keys, values = cache.keys[0], cache.values[0]
    rows_k = pages_to_rows(keys) if layout == "pages" else keys
    rows_v = pages_to_rows(values) if layout == "pages" else values
    want = pa.paged_prefill_dense(q[:n].cpu().numpy(), rows_k.cpu().numpy(),
                                  rows_v.cpu().numpy(), table, start=0, page_size=page,
                                  scale=d ** -0.5)
    err_max, err_mean = pa.error_stats(got, want)
    print(f"PrefillBatch D80 {layout}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}",
          flush=True)
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS
    # The next token: its K/V into row n, then decode over all n + 1 keys.
    row = table[n // page] * page + n % page
    if layout == "pages":
        keys[table[n // page], :, n % page] = k[n]
        values[table[n // page], :, n % page] = v[n]
    else:
        keys[row] = k[n]
        values[row] = v[n]
    tables = torch.as_tensor(table[None].astype(np.int32), device=gpu)
    lengths = torch.tensor([n + 1], dtype=torch.int32, device=gpu)
    dec = paged_decode_attention(q[n:n + 1], keys, values, tables, lengths, page_size=page,
                                 longest=n + 1, scale=d ** -0.5)
    torch.cuda.synchronize()
    rows_k = pages_to_rows(keys) if layout == "pages" else keys
    rows_v = pages_to_rows(values) if layout == "pages" else values
    want = pa.paged_decode_dense(q[n:n + 1].float().cpu().numpy(), rows_k.float().cpu().numpy(),
                                 rows_v.float().cpu().numpy(), tables.cpu().numpy(),
                                 lengths.cpu().numpy(), page_size=page, scale=d ** -0.5)
    err_max, err_mean = pa.error_stats(dec.float().cpu().numpy(), want)
    print(f"decode after prefill D80 {layout}: max_abs={err_max:.3e}", flush=True)
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS
