"""bf16 queries, K/V and output (the model dtype of the reference's bf16
models, paged_kv.py:156-292): the decode call (pda_paged_decode_attention_bf16
via the C-ABI) and the prefill call (pda_paged_prefill_attention_bf16) against
the float64 oracle on the same bf16 values, the K/V append with rotary
embedding (pda_rope_append_bf16) against the RoPE oracle rounded to bf16, and
a bf16 KVCache through PrefillBatch and DecodeBatch.

Bar: the north star's fp16 bar scaled by the ratio of the two formats'
machine epsilons (bf16 keeps 8 significand bits, fp16 11: 2^-7 / 2^-10 = 8):
max-abs <= 1.6e-2, mean-abs <= 1.6e-3. The output itself is rounded to bf16
(relative error up to 2^-9) and so are the probabilities that weight V."""

import numpy as np
import pytest
import torch

from instinct_amd import workloads
from instinct_amd.hip_kernels import paged_decode_attention
from oracle import paged_attention as pa

pytestmark = pytest.mark.gpu

MAX_ABS = 1.6e-2
MEAN_ABS = 1.6e-3


def as_bf16(w):
    """The workload with q and arenas in bf16 (values rounded from fp16)."""
    w.q = w.q.to(torch.bfloat16)
    w.keys = w.keys.to(torch.bfloat16)
    w.values = w.values.to(torch.bfloat16)
    return w


def host(w):
    """Oracle inputs: the bf16 values as float32, rows layout."""
    from instinct_amd.paged_kv import pages_to_rows

    keys, values = w.keys, w.values
    if w.layout == "pages":
        keys, values = pages_to_rows(keys), pages_to_rows(values)
    f = lambda t: t.float().cpu().numpy()  # noqa: E731
    return f(w.q), f(keys), f(values), w.tables.cpu().numpy(), w.lengths.cpu().numpy()


def check(w, what, **kw):
    out = paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths,
                                 page_size=w.page_size, longest=w.longest, scale=w.scale,
                                 window=w.window, softcap=w.softcap, **kw)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    q, k, v, t, n = host(w)
    want = pa.paged_decode_dense(q, k, v, t, n, page_size=w.page_size, scale=w.scale,
                                 window=w.window, softcap=w.softcap)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all(), what
    err_max, err_mean = pa.error_stats(got, want)
    print(f"{what}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}", flush=True)
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS, (what, err_max, err_mean)


@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_config2_shape_reduced(gpu, layout):
    w = as_bf16(workloads.config2(device=gpu, batch=8, low=512, high=2048).to_layout(layout))
    check(w, f"bf16 config2 {layout}")


@pytest.mark.parametrize("layout", ["pages", "rows"])
@pytest.mark.parametrize("q_heads,kv_heads,head_dim,lengths,window,softcap", [
    (16, 2, 512, [1, 700, 2049], 0, 0.0),
    (16, 8, 256, [5, 1500, 4000], 1024, 0.0),
    (14, 2, 64, [1024, 1024, 17], 0, 0.0),
    (8, 1, 80, [3, 300], 0, 30.0),
    (12, 2, 96, [33, 257, 999], 0, 0.0),
    (28, 4, 128, [3, 300, 4095], 0, 30.0),
])
def test_head_dims(gpu, layout, q_heads, kv_heads, head_dim, lengths, window, softcap):
    w = as_bf16(workloads.reference_test_case(q_heads, kv_heads, head_dim, lengths, window,
                                              softcap, device=gpu).to_layout(layout))
    check(w, f"bf16 {q_heads}/{kv_heads} D{head_dim} {layout}")


def test_split_and_merge_passes(gpu):
    w = as_bf16(workloads.config2(device=gpu, batch=6, low=300, high=3000).to_layout("pages"))
    out = torch.empty_like(w.q)
    for passes in ("split", "merge"):
        paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths,
                               page_size=w.page_size, longest=w.longest, scale=w.scale,
                               out=out, passes=passes)
    torch.cuda.synchronize()
    both = paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths,
                                  page_size=w.page_size, longest=w.longest, scale=w.scale)
    torch.cuda.synchronize()
    assert (out.float() - both.float()).abs().max().item() <= MAX_ABS
    check(w, "bf16 config2 small, both passes")


# --- K/V append with rotary embedding (pda_rope_append_bf16) -----------------

def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 to nearest even, back as float32 (torch's CPU cast)."""
    return torch.as_tensor(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).float().numpy()


def within_bf16_ulp(got: np.ndarray, want: np.ndarray, what: str) -> None:
    """|got - want| <= one bf16 ulp of want + 2^-20. Both round the same
    float32 expression to bf16 to nearest even; the float32 sine and cosine
    of the device and of NumPy may differ in the last bit, which moves a value
    that sits on a rounding tie by one ulp, and moves a result near zero
    (x1 cos ~= x2 sin) by the float32 expression's absolute error, a few
    float32 ulps of |x| <= ~5 (2^-20 bounds it; bf16, unlike fp16, has no
    subnormal spacing that covers it)."""
    assert got.shape == want.shape, what
    if got.size == 0:
        return
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64) * 65536.0 + 2.0 ** -20
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    print(f"{what}: bit-exact {np.mean(got == want):.6f}, max diff {diff.max():.3e}", flush=True)
    assert np.all(diff <= ulp), (what, diff.max())


def append_case(gpu, *, n, hq, hkv, d, layout, page_size=16, seed=0, positions=None):
    rng = np.random.default_rng(seed)
    pages = max(4, 2 * n)
    b = lambda a: bf16_round(a.astype(np.float32))  # noqa: E731
    q = b(rng.standard_normal((n, hq, d))) if hq else None
    k = b(rng.standard_normal((n, hkv, d)))
    v = b(rng.standard_normal((n, hkv, d)))
    if positions is None:
        positions = rng.integers(0, 8192, n)
    positions = np.asarray(positions, np.int32)
    rows = (rng.permutation(pages)[:n] * page_size + positions % page_size).astype(np.int32)
    shape = (pages * page_size, hkv, d) if layout == "rows" else (pages, hkv, page_size, d)
    k_arena, v_arena = b(rng.standard_normal(shape)), b(rng.standard_normal(shape))
    dev = lambda a, dt=torch.bfloat16: (  # noqa: E731
        None if a is None else torch.as_tensor(a, device=gpu).to(dt))
    t = dict(q=dev(q), k=dev(k), v=dev(v), k_arena=dev(k_arena), v_arena=dev(v_arena),
             positions=dev(positions, torch.int32), rows=dev(rows, torch.int32))
    return dict(q=q, k=k, v=v, k_arena=k_arena, v_arena=v_arena, positions=positions,
                rows=rows, layout=layout, page_size=page_size, t=t)


def check_append_bf16(case, *, dims, base=None, freqs=None, in_place=False, what=""):
    from instinct_amd import hip_kernels
    from oracle import rope_append as ra

    t = case["t"]
    inverse = ra.inv_freq(dims, base=base, freqs=freqs) if dims else np.zeros(0, np.float32)
    got_q = hip_kernels.rope_append(t["q"], t["k"], t["v"], t["k_arena"], t["v_arena"],
                                    t["positions"], t["rows"], page_size=case["page_size"],
                                    dims=dims, base=base, freqs=freqs,
                                    q_out=t["q"] if in_place else None)
    torch.cuda.synchronize()
    # The oracle rotates the float32 values and returns float32; rounding that
    # to bf16 is the reference's `.astype(x.dtype)` for a bf16 model.
    want_q, want_k, want_v = ra.rope_append(
        case["q"], case["k"], case["v"], case["k_arena"], case["v_arena"], case["positions"],
        case["rows"], dims=dims, inverse=inverse, layout=case["layout"],
        page_size=case["page_size"])
    got_k = t["k_arena"].float().cpu().numpy()
    got_v = t["v_arena"].float().cpu().numpy()
    assert t["k_arena"].dtype == torch.bfloat16
    assert np.array_equal(got_v, want_v), f"{what}: values"
    within_bf16_ulp(got_k, bf16_round(want_k), f"{what} keys")
    assert np.array_equal(got_k[..., dims:], want_k[..., dims:]), f"{what}: key tail"
    if case["q"] is not None:
        assert got_q.dtype == torch.bfloat16
        if in_place:
            assert got_q.data_ptr() == t["q"].data_ptr()
        gq = got_q.float().cpu().numpy()
        within_bf16_ulp(gq, bf16_round(want_q), f"{what} queries")
        assert np.array_equal(gq[..., dims:], case["q"][..., dims:])
        # Against an exact rotation by the same float32 angles: one bf16
        # rounding (2^-9 relative) of values of size |x| <= ~5.
        half = dims // 2
        angles = (case["positions"].astype(np.float32)[:, None]
                  * inverse[None, :half]).astype(np.float64)
        z = (case["q"][..., :half].astype(np.float64)
             + 1j * case["q"][..., half:dims].astype(np.float64)) * np.exp(1j * angles)[:, None]
        exact = case["q"].astype(np.float64)
        exact[..., :half], exact[..., half:dims] = z.real, z.imag
        err = np.abs(gq - exact).max(initial=0.0)
        print(f"{what}: queries vs float64 rotation max_abs={err:.3e}", flush=True)
        assert err <= MAX_ABS


@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_append_config2_decode_step(gpu, layout):
    """Qwen2.5-7B decode step in bf16: 64 tokens, 28/4 heads, D=128, base 1e6."""
    case = append_case(gpu, n=64, hq=28, hkv=4, d=128, layout=layout, seed=2)
    check_append_bf16(case, dims=128, base=1e6, what=f"bf16 append config2 {layout}")


@pytest.mark.parametrize("d,dims,base,layout", [
    (64, 64, 10000.0, "rows"),
    (80, 80, 10000.0, "pages"),
    (128, 64, 10000.0, "pages"),     # partial rotary
    (256, 256, 10000.0, "rows"),
    (512, 512, 1e6, "pages"),
    (64, 6, 100.0, "pages"),         # odd half
])
def test_append_head_dims(gpu, d, dims, base, layout):
    case = append_case(gpu, n=9, hq=8, hkv=2, d=d, layout=layout, seed=d + dims)
    check_append_bf16(case, dims=dims, base=base, what=f"bf16 append d{d} dims{dims}")


def test_append_in_place_large_positions_and_write_only(gpu):
    positions = [0, 1, 2, 16383, 65535, 131071, 500000, 1 << 20]
    case = append_case(gpu, n=8, hq=4, hkv=2, d=128, layout="pages", positions=positions,
                       seed=5)
    check_append_bf16(case, dims=128, base=10000.0, in_place=True, what="bf16 in place")
    case = append_case(gpu, n=12, hq=0, hkv=4, d=128, layout="rows", seed=12)
    check_append_bf16(case, dims=0, what="bf16 write only")


def test_rope_alone(gpu):
    from instinct_amd import hip_kernels
    from oracle import rope_append as ra

    rng = np.random.default_rng(14)
    x = bf16_round(rng.standard_normal((5, 3, 128)).astype(np.float32))
    positions = np.array([0, 3, 77, 4095, 120000], np.int32)
    got = hip_kernels.rope(torch.as_tensor(x, device=gpu).to(torch.bfloat16),
                           torch.as_tensor(positions, device=gpu), 128, base=1e6)
    assert got.dtype == torch.bfloat16
    want = bf16_round(ra.rope(x, positions, 128, ra.inv_freq(128, base=1e6)))
    within_bf16_ulp(got.float().cpu().numpy(), want, "bf16 rope alone")


# --- paged prefill attention (pda_paged_prefill_attention_bf16) ---------------

def prefill_case(gpu, *, hq, hkv, d, start, count, page=16, layout="pages", seed=0,
                 released=()):
    from instinct_amd.paged_kv import rows_to_pages

    rng = np.random.default_rng(seed)
    pages = (start + count + page - 1) // page
    arena_pages = pages + 5
    table = rng.permutation(arena_pages)[:pages].astype(np.int32)
    for i in released:
        table[i] = -1
    b = lambda shape: bf16_round(rng.standard_normal(shape).astype(np.float32))  # noqa: E731
    keys, values = b((arena_pages * page, hkv, d)), b((arena_pages * page, hkv, d))
    q = b((count, hq, d))
    dev = lambda a: torch.as_tensor(a, device=gpu).to(torch.bfloat16)  # noqa: E731
    k_dev, v_dev = dev(keys), dev(values)
    if layout == "pages":
        k_dev, v_dev = rows_to_pages(k_dev, page), rows_to_pages(v_dev, page)
    return dict(q=q, keys=keys, values=values, table=table, page=page, start=start,
                t=(dev(q), k_dev, v_dev, torch.as_tensor(table, device=gpu)))


def check_prefill(c, *, scale, window=0, softcap=0.0, splits=0, images=(), what=""):
    from instinct_amd.hip_kernels import paged_prefill_attention

    q, k, v, table = c["t"]
    got = paged_prefill_attention(q, k, v, table, start=c["start"], page_size=c["page"],
                                  scale=scale, window=window, softcap=softcap, splits=splits,
                                  images=images)
    torch.cuda.synchronize()
    assert got.dtype == torch.bfloat16
    got = got.float().cpu().numpy()
    assert np.isfinite(got).all(), f"{what}: non-finite"
    want = pa.paged_prefill_dense(c["q"], c["keys"], c["values"], c["table"], start=c["start"],
                                  page_size=c["page"], scale=scale, window=window,
                                  softcap=softcap, images=images)
    err_max, err_mean = pa.error_stats(got, want)
    print(f"{what}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}", flush=True)
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS, (what, err_max, err_mean)


@pytest.mark.parametrize("layout", ["pages", "rows"])
@pytest.mark.parametrize("hq,hkv,d,start,count,splits", [
    (28, 4, 128, 0, 300, 0),
    (28, 4, 128, 700, 200, 3),
    (14, 2, 64, 37, 450, 0),
    (8, 4, 256, 1000, 150, 2),
    (32, 8, 128, 5, 1, 0),
])
def test_prefill_shapes(gpu, layout, hq, hkv, d, start, count, splits):
    c = prefill_case(gpu, hq=hq, hkv=hkv, d=d, start=start, count=count, layout=layout,
                     seed=hq + d + start)
    check_prefill(c, scale=d ** -0.5, splits=splits,
                  what=f"bf16 prefill {hq}/{hkv} D{d} @{start}+{count} s{splits} {layout}")


def test_prefill_window_softcap_images_and_released_pages(gpu):
    c = prefill_case(gpu, hq=8, hkv=2, d=128, start=1000, count=300, page=32, seed=41,
                     released=(0, 1, 5))
    check_prefill(c, scale=128 ** -0.5, window=100, softcap=30.0, what="bf16 window+softcap")
    check_prefill(c, scale=128 ** -0.5, window=64, splits=4, images=[(1010, 150), (1200, 3)],
                  what="bf16 images with window, splits 4")


def test_prefill_long_prefix_splits_automatically(gpu):
    """A 512-token chunk over a 6000-token prefix: the library splits the
    key range (workspace partials merged into bf16)."""
    from instinct_amd import _lib

    assert _lib.prefill_workspace_bytes(6000, 512, 28, 128)[0] > 1
    c = prefill_case(gpu, hq=28, hkv=4, d=128, start=6000, count=512, seed=8)
    check_prefill(c, scale=128 ** -0.5, what="bf16 512@6000 auto split")


@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_bf16_cache_prefill_then_decode(gpu, layout):
    """A bf16 KVCache through PrefillBatch (two chunks: the model's rope
    calls, then attend) and two DecodeBatch rope_attend steps, each against
    the oracle over the arena the kernels wrote (batches.py:26-253)."""
    from instinct_amd.batches import DecodeBatch, PrefillBatch
    from instinct_amd.paged_kv import KVCache, KVGroup, pages_to_rows

    page, hq, hkv, d = 16, 14, 2, 128
    groups = [KVGroup("full", (0,), kv_heads=hkv, head_dim=d)]
    cache = KVCache(groups, page_size=page, capacities={"full": 64}, device=gpu,
                    layout=layout, dtype=torch.bfloat16)
    assert cache.keys[0].dtype == cache.compute_dtype == torch.bfloat16
    n = 300
    table = np.array([cache.pools["full"].allocate(reserved=False) for _ in range(24)])
    gen = torch.Generator(device=gpu).manual_seed(6)
    q = torch.randn((n + 2, hq, d), generator=gen, device=gpu).bfloat16()
    k = torch.randn((n + 2, hkv, d), generator=gen, device=gpu).bfloat16()
    v = torch.randn((n + 2, hkv, d), generator=gen, device=gpu).bfloat16()

    def arena():
        keys, values = cache.keys[0], cache.values[0]
        if layout == "pages":
            keys, values = pages_to_rows(keys), pages_to_rows(values)
        return keys.float().cpu().numpy(), values.float().cpu().numpy()

    outs, qs = [], []
    for a, b in ((0, 170), (170, n)):
        chunk = PrefillBatch(cache, torch.zeros(b - a, device=gpu), start=a,
                             tables={"full": table})
        q_rot = chunk.rope(q[a:b], d, base=1e6)
        k_rot = chunk.rope(k[a:b], d, base=1e6)
        assert q_rot.dtype == k_rot.dtype == torch.bfloat16
        qs.append(q_rot)
        outs.append(chunk.attend(0, q_rot, k_rot, v[a:b], scale=d ** -0.5))
    torch.cuda.synchronize()
    keys, values = arena()
    got = torch.cat(outs).view(n, hq, d).float().cpu().numpy()
    want = pa.paged_prefill_dense(torch.cat(qs).float().cpu().numpy(), keys, values, table,
                                  start=0, page_size=page, scale=d ** -0.5)
    err_max, err_mean = pa.error_stats(got, want)
    print(f"bf16 PrefillBatch {layout}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}")
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS
    for t in (n, n + 1):
        step = DecodeBatch(cache, torch.zeros(1, device=gpu), positions=np.array([t]),
                           tables={"full": [table]})
        out = step.rope_attend(0, q[t:t + 1], k[t:t + 1], v[t:t + 1], dims=d, base=1e6,
                               scale=d ** -0.5)
        torch.cuda.synchronize()
        assert out.dtype == torch.bfloat16
        keys, values = arena()
        q_rot = step.rope(q[t:t + 1], d, base=1e6).float().cpu().numpy()
        want = pa.paged_decode_dense(q_rot, keys, values, table[None].astype(np.int32),
                                     np.array([t + 1], np.int32), page_size=page,
                                     scale=d ** -0.5)
        err_max, err_mean = pa.error_stats(out.view(1, hq, d).float().cpu().numpy(), want)
        print(f"bf16 decode step {t} {layout}: max_abs={err_max:.3e}")
        assert err_max <= MAX_ABS and err_mean <= MEAN_ABS


def test_bf16_model_over_8bit_cache(gpu):
    """KVCache(dtype=bfloat16, bits=8): the kernels take fp16 (bf16 -> fp16
    is exact in fp16's range), rope runs in bf16, rope_attend rounds the
    rotated keys to bf16 before quantizing them (the reference's order,
    paged_kv.py:50-55,278-283), and attention outputs come back in bf16. The
    oracle: the reference's quantization of the bf16 rotated keys and of the
    values, attention over the dequantized rows."""
    from instinct_amd.batches import DecodeBatch, PrefillBatch
    from instinct_amd.paged_kv import KVCache, KVGroup, pages_to_rows
    from oracle import kv8

    page, hq, hkv, d = 16, 14, 2, 128
    groups = [KVGroup("full", (0,), kv_heads=hkv, head_dim=d)]
    cache = KVCache(groups, page_size=page, capacities={"full": 64}, device=gpu,
                    dtype=torch.bfloat16, bits=8)
    assert cache.keys[0].dtype == torch.int8 and cache.compute_dtype == torch.float16
    n = 200
    table = np.array([cache.pools["full"].allocate(reserved=False) for _ in range(16)])
    gen = torch.Generator(device=gpu).manual_seed(9)
    q = torch.randn((n + 2, hq, d), generator=gen, device=gpu).bfloat16()
    k = torch.randn((n + 2, hkv, d), generator=gen, device=gpu).bfloat16()
    v = torch.randn((n + 2, hkv, d), generator=gen, device=gpu).bfloat16()

    def arena():
        keys, values = pages_to_rows(cache.keys[0]), pages_to_rows(cache.values[0])
        k_s = cache.key_scales[0].permute(0, 2, 1).reshape(-1, hkv)
        v_s = cache.value_scales[0].permute(0, 2, 1).reshape(-1, hkv)
        f = lambda t: t.cpu().numpy()  # noqa: E731
        return f(keys), f(values), f(k_s), f(v_s)

    chunk = PrefillBatch(cache, torch.zeros(n, device=gpu), start=0, tables={"full": table})
    q_rot, k_rot = chunk.rope(q[:n], d, base=1e6), chunk.rope(k[:n], d, base=1e6)
    assert q_rot.dtype == k_rot.dtype == torch.bfloat16
    out = chunk.attend(0, q_rot, k_rot, v[:n], scale=d ** -0.5)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    kq, vq, ks, vs = arena()
    rows = np.concatenate([table[p // page] * page + np.arange(page) for p in range(0, n, page)])[:n]
    want_kq, want_ks = kv8.quantize(k_rot.float().cpu().numpy())
    np.testing.assert_array_equal(ks[rows], want_ks)
    np.testing.assert_array_equal(kq[rows], want_kq)
    want = pa.paged_prefill_dense(q_rot.float().cpu().numpy(), kv8.gather_dequantize(kq, ks),
                                  kv8.gather_dequantize(vq, vs), table, start=0,
                                  page_size=page, scale=d ** -0.5)
    err_max, err_mean = pa.error_stats(out.view(n, hq, d).float().cpu().numpy(), want)
    print(f"bf16 model, 8-bit cache, prefill: max_abs={err_max:.3e} mean_abs={err_mean:.3e}")
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS
    for t in (n, n + 1):
        step = DecodeBatch(cache, torch.zeros(1, device=gpu), positions=np.array([t]),
                           tables={"full": [table]})
        out = step.rope_attend(0, q[t:t + 1], k[t:t + 1], v[t:t + 1], dims=d, base=1e6,
                               scale=d ** -0.5)
        torch.cuda.synchronize()
        assert out.dtype == torch.bfloat16
        kq, vq, ks, vs = arena()
        row = table[t // page] * page + t % page
        k_rot = step.rope(k[t:t + 1], d, base=1e6)
        want_kq, want_ks = kv8.quantize(k_rot.float().cpu().numpy())
        np.testing.assert_array_equal(kq[row], want_kq[0])
        np.testing.assert_array_equal(ks[row], want_ks[0])
        q_rot = step.rope(q[t:t + 1], d, base=1e6).float().cpu().numpy()
        want = pa.paged_decode_dense(q_rot, kv8.gather_dequantize(kq, ks),
                                     kv8.gather_dequantize(vq, vs),
                                     table[None].astype(np.int32), np.array([t + 1], np.int32),
                                     page_size=page, scale=d ** -0.5)
        err_max, err_mean = pa.error_stats(out.view(1, hq, d).float().cpu().numpy(), want)
        print(f"bf16 model, 8-bit cache, decode step {t}: max_abs={err_max:.3e}")
        assert err_max <= MAX_ABS and err_mean <= MEAN_ABS


@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_prefill_head_dim_512(gpu, layout):
    c = prefill_case(gpu, hq=8, hkv=2, d=512, start=900, count=130, layout=layout, seed=90)
    check_prefill(c, scale=512 ** -0.5, what=f"bf16 prefill D512 {layout}")
    check_prefill(c, scale=512 ** -0.5, splits=3, window=500,
                  what=f"bf16 prefill D512 3 ranges, window {layout}")


def test_prefill_head_dim_96(gpu):
    c = prefill_case(gpu, hq=32, hkv=8, d=96, start=700, count=200, seed=96)
    check_prefill(c, scale=96 ** -0.5, what="bf16 prefill D96")
    check_prefill(c, scale=96 ** -0.5, splits=4, what="bf16 prefill D96, 4 ranges")
