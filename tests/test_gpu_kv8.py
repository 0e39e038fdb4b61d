"""Parity of the 8-bit K/V decode (pda_paged_decode_attention_q8 via the
C-ABI) with the float64 oracle on the dequantized arena.

The reference's check for its quantized kernel (tests/test_mlx_engine.py:
432-491, bits=8) compares against dense attention over ``int8 * scale``;
the oracle here is the same computation in float64 (oracle/paged_attention.py
on oracle/kv8.py's quantization, both pinned on the CPU). Bar: the north
star's max-abs 2e-3 and mean-abs 2e-4, in both arena layouts.
"""

import numpy as np
import pytest
import torch

from instinct_amd import workloads
from instinct_amd.hip_kernels import paged_decode_attention
from instinct_amd.paged_kv import rows_to_pages
from oracle import kv8
from oracle import paged_attention as pa

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-3
MEAN_ABS = 2e-4


def scales_to_pages(scales: torch.Tensor, page_size: int) -> torch.Tensor:
    """[rows, kv_heads] -> [pages, kv_heads, page_size]."""
    rows, heads = scales.shape
    return scales.view(rows // page_size, page_size, heads).permute(0, 2, 1).contiguous()


class Quantized:
    """A workload's arenas quantized as the reference's KVCache(bits=8) holds
    them (paged_kv.py:50-55, 278-283), on the GPU in either layout."""

    def __init__(self, w, layout, poison_rows=None):
        q, k, v, t, n = w.numpy()
        self.w, self.q, self.t, self.n = w, q, t, n
        self.kq, self.ks = kv8.quantize(k)
        self.vq, self.vs = kv8.quantize(v)
        if poison_rows is not None:
            self.ks[poison_rows] = np.float16(np.nan)
            self.vs[poison_rows] = np.float16(np.inf)
        dev = w.q.device
        P = w.page_size
        keys, values = torch.as_tensor(self.kq, device=dev), torch.as_tensor(self.vq, device=dev)
        ks, vs = torch.as_tensor(self.ks, device=dev), torch.as_tensor(self.vs, device=dev)
        if layout == "pages":
            keys, values = rows_to_pages(keys, P), rows_to_pages(values, P)
            ks, vs = scales_to_pages(ks, P), scales_to_pages(vs, P)
        self.keys, self.values, self.scales = keys, values, (ks, vs)

    def run(self, **kw):
        w = self.w
        out = paged_decode_attention(w.q, self.keys, self.values, w.tables, w.lengths,
                                     page_size=w.page_size, longest=w.longest, scale=w.scale,
                                     window=w.window, softcap=w.softcap, scales=self.scales, **kw)
        torch.cuda.synchronize()
        return out

    def expected(self):
        w = self.w
        return pa.paged_decode_dense(self.q, kv8.dequantize(self.kq, np.nan_to_num(self.ks)),
                                     kv8.dequantize(self.vq, np.nan_to_num(self.vs)), self.t,
                                     self.n, page_size=w.page_size, scale=w.scale,
                                     window=w.window, softcap=w.softcap)


def check(qw, what, **kw):
    got = qw.run(**kw).float().cpu().numpy()
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err_max, err_mean = pa.error_stats(got, qw.expected())
    print(f"{what}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}", flush=True)
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS, (what, err_max, err_mean)
    return got


@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_config2_shape_reduced(gpu, layout):
    w = workloads.config2(device=gpu, batch=8, low=512, high=2048)
    check(Quantized(w, layout), f"config2 q8 {layout}")


@pytest.mark.parametrize("layout", ["pages", "rows"])
@pytest.mark.parametrize("q_heads,kv_heads,head_dim,lengths,window,softcap", [
    (16, 2, 512, [1, 700, 2049], 0, 0.0),
    (16, 8, 256, [5, 1500, 4000], 1024, 0.0),
    (16, 4, 256, [64, 3333], 0, 0.0),
    (14, 2, 64, [1024, 1024, 17], 0, 0.0),
    (28, 4, 128, [3, 300, 4095], 0, 30.0),
])
def test_reference_kernel_shapes(gpu, layout, q_heads, kv_heads, head_dim, lengths, window,
                                 softcap):
    """The reference's bits=8 kernel-test shapes (test_mlx_engine.py:422-431;
    head_dim 80 and 4 run the generic kernels, tests/test_gpu_shapes.py) plus
    config 1's and config 2's head shapes (the matrix-core kernels), with a
    softcap."""
    w = workloads.reference_test_case(q_heads, kv_heads, head_dim, lengths, window, softcap,
                                      device=gpu)
    check(Quantized(w, layout), f"q8 {q_heads}/{kv_heads} D{head_dim} {layout}")


@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_window_poison_and_released_pages(gpu, layout):
    """Rows before the window hold NaN/inf scales (and their pages may be
    released): the output ignores them (portable.py:202-204)."""
    w = workloads.config4(device=gpu, batch=6, low=1100, high=3000)
    _, _, _, t, n = w.numpy()
    first = np.maximum(n - w.window, 0)
    poison = []
    for b in range(w.batch):
        for pos in range(0, int(first[b])):
            page = t[b, pos // w.page_size]
            if page >= 0:
                poison.append(page * w.page_size + pos % w.page_size)
    qw = Quantized(w, layout, poison_rows=np.array(poison, dtype=np.int64))
    check(qw, f"q8 window poison {layout}")


def test_split_and_merge_passes_and_call_to_call(gpu):
    w = workloads.config2(device=gpu, batch=16, low=512, high=4096)
    qw = Quantized(w, "pages")
    whole = qw.run()
    out = torch.empty_like(w.q)
    qw.run(passes="split", out=out)
    qw.run(passes="merge", out=out)
    d = (out.float() - whole.float()).abs()
    assert d.max().item() <= MAX_ABS and d.mean().item() <= MEAN_ABS
    check(qw, "q8 split pages=4", split_pages=4)


# ---------------------------------------------------------------------------
# 8-bit K/V on the matrix cores: GQA groups of 5 or more heads at head dims
# 64, 128, 256 (int8 rows converted in registers, scores times the key
# scale, V rows dequantized to fp16 into the LDS tile).

from instinct_amd.hip_kernels import decode_kernel_names  # noqa: E402


def mf_case(gpu, q_heads, kv_heads, head_dim, lengths, page=16, window=0, softcap=0.0, seed=0):
    rng = np.random.default_rng(seed)
    need = [max(0, -(-n // page)) for n in lengths]
    arena = sum(need) + 3
    order = rng.permutation(arena)
    tables = np.zeros((len(lengths), max(1, max(need))), dtype=np.int32)
    c = 0
    for b, k in enumerate(need):
        tables[b, :k] = order[c:c + k]
        c += k
    return workloads.build(f"mfq8-{q_heads}/{kv_heads}/{head_dim}", lengths=lengths,
                           tables=tables, arena_pages=arena, q_heads=q_heads,
                           kv_heads=kv_heads, head_dim=head_dim, page_size=page,
                           scale=head_dim ** -0.5, window=window, softcap=softcap,
                           device=gpu, seed=seed + 1)


@pytest.mark.parametrize("head_dim", [64, 128, 256, 512])
@pytest.mark.parametrize("q_heads,kv_heads", [(5, 1), (7, 1), (8, 1), (11, 1), (16, 2),
                                              (24, 2), (28, 4)])
def test_matrix_cores_group_sizes(gpu, q_heads, kv_heads, head_dim):
    names = decode_kernel_names(q_heads, kv_heads, head_dim, bits=8)
    assert names["matrix_cores"], names
    w = mf_case(gpu, q_heads, kv_heads, head_dim, [1, 15, 16, 17, 700, 2500, 33],
                seed=q_heads * 10 + head_dim)
    for layout in ("pages", "rows"):
        qw = Quantized(w, layout)
        check(qw, f"mf q8 {q_heads}/{kv_heads} D{head_dim} {layout}")
        check(qw, f"mf q8 {q_heads}/{kv_heads} D{head_dim} {layout} fixed", deterministic=True)


@pytest.mark.parametrize("head_dim", [128, 512])
@pytest.mark.parametrize("page", [1, 5, 12, 24, 64])
def test_matrix_cores_page_sizes(gpu, page, head_dim):
    """Pages that are not a multiple of the 16-key step: the last step of a
    page moves its rows back inside the page and masks the duplicates."""
    w = mf_case(gpu, 14, 2, head_dim, [1, page, page + 1, 777, 1500], page=page, seed=page)
    for layout in ("pages", "rows"):
        check(Quantized(w, layout), f"mf q8 page {page} D{head_dim} {layout}")


@pytest.mark.parametrize("head_dim", [128, 512])
@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_matrix_cores_window_poison_softcap(gpu, layout, head_dim):
    """Rows before the window hold NaN key scales and inf value scales; the
    masked keys' values are zeroed after dequantization, so nothing leaks."""
    P, W = 16, 300
    lengths = [1200, 301, 299, 4000, 9]
    w = mf_case(gpu, 24, 2, head_dim, lengths, window=W, softcap=30.0, seed=8)
    _, _, _, t, n = w.numpy()
    poison = []
    for b, length in enumerate(lengths):
        for pos in range(0, max(0, length - W)):
            poison.append(int(t[b, pos // P]) * P + pos % P)
    qw = Quantized(w, layout, poison_rows=np.array(poison, dtype=np.int64))
    check(qw, f"mf q8 window poison softcap D{head_dim} {layout}")


def test_matrix_cores_fixed_split_is_bitwise_reproducible(gpu):
    w = workloads.config2(device=gpu, batch=16, low=512, high=4096)
    qw = Quantized(w, "pages")
    first = check(qw, "mf q8 config2 fixed", deterministic=True)
    for _ in range(3):
        assert np.array_equal(qw.run(deterministic=True).float().cpu().numpy(), first)


# ---------------------------------------------------------------------------
# The 8-bit write: pda_rope_append_q8 (KVCache.write with bits=8).

from instinct_amd import hip_kernels  # noqa: E402
from instinct_amd.batches import DecodeBatch  # noqa: E402
from instinct_amd.paged_kv import KVCache, KVGroup  # noqa: E402
from oracle import rope_append as ra  # noqa: E402


def scale_slot(scales, row, page_size, layout):
    return scales[row] if layout == "rows" else scales[row // page_size, :, row % page_size]


def arena_slot(arena, row, page_size, layout):
    return arena[row] if layout == "rows" else arena[row // page_size, :, row % page_size]


@pytest.mark.parametrize("layout", ["pages", "rows"])
@pytest.mark.parametrize("d,dims", [(128, 128), (128, 0), (64, 64), (512, 256)])
def test_quantizing_append(gpu, layout, d, dims):
    rng = np.random.default_rng(d + dims)
    n, hq, hkv, P, pages = 12, 7, 2, 16, 32
    q = rng.standard_normal((n, hq, d)).astype(np.float16)
    k = (rng.standard_normal((n, hkv, d)) * rng.uniform(0.01, 8, (n, hkv, 1))).astype(np.float16)
    v = rng.standard_normal((n, hkv, d)).astype(np.float16)
    v[3, 1] = 0  # an all-zero row takes the 1e-4 floor
    positions = rng.integers(0, 70000, n).astype(np.int32)
    rows = (rng.permutation(pages)[:n] * P + positions % P).astype(np.int32)
    rows[5] = -1  # skipped
    shape = (pages * P, hkv, d) if layout == "rows" else (pages, hkv, P, d)
    t = lambda a: torch.as_tensor(a, device=gpu)  # noqa: E731
    keys = torch.full(shape, 7, dtype=torch.int8, device=gpu)
    values = torch.full(shape, -7, dtype=torch.int8, device=gpu)
    ks = torch.full(shape[:-1], 3.0, dtype=torch.float16, device=gpu)
    vs = torch.full(shape[:-1], 3.0, dtype=torch.float16, device=gpu)
    q_out = hip_kernels.rope_append(t(q), t(k), t(v), keys, values, t(positions), t(rows),
                                    page_size=P, dims=dims, base=1e6, scales=(ks, vs))
    torch.cuda.synchronize()
    inv = ra.inv_freq(dims, base=1e6) if dims else np.zeros(0, np.float32)
    k_rot = ra.rope(k, positions, dims, inv) if dims else k
    kq, kscale = kv8.quantize(k_rot)
    vq, vscale = kv8.quantize(v)
    keys, values, ks, vs = (x.cpu().numpy() for x in (keys, values, ks, vs))
    written = set()
    for i, row in enumerate(rows):
        if row < 0:
            continue
        written.add(int(row))
        gk, gv = arena_slot(keys, row, P, layout), arena_slot(values, row, P, layout)
        gks, gvs = scale_slot(ks, row, P, layout), scale_slot(vs, row, P, layout)
        # Values: bit-exact. Keys: the rotation may differ from NumPy's in the
        # last bit of the sine/cosine, which can move a quantized value by one.
        assert np.array_equal(gv, vq[i]) and np.array_equal(gvs, vscale[i]), (i, "values")
        assert np.abs(gk.astype(np.int32) - kq[i].astype(np.int32)).max() <= 1, (i, "keys")
        np.testing.assert_allclose(gks.astype(np.float32), kscale[i].astype(np.float32),
                                   rtol=1e-3)
    # Nothing else changed.
    untouched = [r for r in range(pages * P) if r not in written]
    for r in untouched[:: max(1, len(untouched) // 64)]:
        assert (arena_slot(keys, r, P, layout) == 7).all()
        assert (scale_slot(vs, r, P, layout) == 3.0).all()
    if dims:
        want = ra.rope(q, positions, dims, inv)
        assert np.abs(q_out.cpu().numpy().astype(np.float32) - want.astype(np.float32)).max() <= 2e-3


@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_decode_batch_at_8_bits(gpu, layout):
    """KVCache(bits=8) and DecodeBatch: the write quantizes, the attention
    reads int8 (batches.py:203-226 with scales, paged_kv.py:278-283), and
    rope_attend equals rope, rope, attend."""
    page = 16
    groups = [KVGroup("full", (0, 1), kv_heads=4, head_dim=128)]
    positions = np.array([0, 15, 16, 100, 333, 2047])
    gen = torch.Generator(device=gpu).manual_seed(5)

    def fresh():
        cache = KVCache(groups, page_size=page, capacities={"full": 256}, device=gpu,
                        layout=layout, bits=8)
        pool = cache.pools["full"]
        tables = {"full": [np.array([pool.allocate(reserved=False)
                                     for _ in range(p // page + 1)]) for p in positions]}
        # Rows as quantized N(0, 1) data: int8 ~ N(0, 36^2), scales ~ 1/36
        # (absmax / 127 of a normal row), so the dequantized arena is ~N(0, 1).
        g2 = torch.Generator(device=gpu).manual_seed(11)
        for layer in (0, 1):
            for store in (cache.keys, cache.values):
                store[layer].copy_(torch.randn(store[layer].shape, generator=g2, device=gpu)
                                   .mul(36).round().clamp(-127, 127).to(torch.int8))
            for store in (cache.key_scales, cache.value_scales):
                store[layer].copy_(torch.rand(store[layer].shape, generator=g2, device=gpu)
                                   .mul(0.01).add(1 / 40).half())
        return cache, DecodeBatch(cache, torch.zeros(6, device=gpu), positions=positions,
                                  tables=tables)

    q = torch.randn((6, 28, 128), generator=gen, device=gpu).half()
    k = torch.randn((6, 4, 128), generator=gen, device=gpu).half()
    v = torch.randn((6, 4, 128), generator=gen, device=gpu).half()
    c1, b1 = fresh()
    fused = b1.rope_attend(0, q, k, v, dims=128, base=1e6, scale=128 ** -0.5)
    c2, b2 = fresh()
    plain = b2.attend(0, b2.rope(q, 128, base=1e6), b2.rope(k, 128, base=1e6), v,
                      scale=128 ** -0.5)
    torch.cuda.synchronize()
    for a, b in ((c1.keys[0], c2.keys[0]), (c1.values[0], c2.values[0]),
                 (c1.key_scales[0], c2.key_scales[0]), (c1.value_scales[0], c2.value_scales[0])):
        assert torch.equal(a, b)
    d = (fused.float() - plain.float()).abs()
    assert d.max().item() <= MAX_ABS and d.mean().item() <= MEAN_ABS
    # Against the oracle on the dequantized arena (rows layout on the host).
    keys, values = c1.keys[0], c1.values[0]
    ks, vs = c1.key_scales[0], c1.value_scales[0]
    if layout == "pages":
        from instinct_amd.paged_kv import pages_to_rows
        keys, values = pages_to_rows(keys), pages_to_rows(values)
        ks, vs = ks.permute(0, 2, 1).reshape(-1, 4), vs.permute(0, 2, 1).reshape(-1, 4)
    deq_k = kv8.dequantize(keys.cpu().numpy(), ks.cpu().numpy())
    deq_v = kv8.dequantize(values.cpu().numpy(), vs.cpu().numpy())
    q_rot = b1.rope(q, 128, base=1e6).cpu().numpy()
    expected = pa.paged_decode_dense(q_rot, deq_k, deq_v, b1._tables["full"].cpu().numpy(),
                                     positions + 1, page_size=page, scale=128 ** -0.5)
    err_max, err_mean = pa.error_stats(fused.view(6, 28, 128).float().cpu().numpy(), expected)
    print(f"DecodeBatch bits=8 {layout}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}")
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS
