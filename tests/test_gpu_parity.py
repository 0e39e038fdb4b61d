"""Parity of the MI355X kernel (libpda.so via the C-ABI) with the float64
oracle on the same seeded inputs.

Bar: max-abs error <= 2e-3 and mean-abs error <= 2e-4
for the fp16 output against a float64-accumulated result. The oracle is the
threaded C++ restatement of the reference's portable path
(oracle/cpu_attention.cpp), itself pinned by tests/test_oracle.py.
"""

import math

import numpy as np
import pytest
import torch

from instinct_amd import workloads
from instinct_amd.hip_kernels import paged_decode_attention
from oracle import cpu_oracle
from oracle import paged_attention as pa

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-3
MEAN_ABS = 2e-4


def run(w, split_pages=0, longest=None):
    out = paged_decode_attention(
        w.q, w.keys, w.values, w.tables, w.lengths, page_size=w.page_size,
        longest=w.longest if longest is None else longest, scale=w.scale,
        window=w.window, softcap=w.softcap, split_pages=split_pages)
    torch.cuda.synchronize()
    return out


def run_fixed(w):
    out = paged_decode_attention(
        w.q, w.keys, w.values, w.tables, w.lengths, page_size=w.page_size, longest=w.longest,
        scale=w.scale, window=w.window, softcap=w.softcap, deterministic=True)
    torch.cuda.synchronize()
    return out


def oracle(w):
    q, k, v, t, n = w.numpy()
    return cpu_oracle.decode_f64(q, k, v, t, n, page_size=w.page_size, scale=w.scale,
                                 window=w.window, softcap=w.softcap)


def assert_parity(got, expected, what=""):
    got = got.float().cpu().numpy() if isinstance(got, torch.Tensor) else got
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err_max, err_mean = pa.error_stats(got, expected)
    print(f"{what}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}", flush=True)
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS, (what, err_max, err_mean)


def assert_consistent(a, b, what=""):
    """Two results of the same call agree within the parity bar. The split
    kernel's wave pairs meet wherever their shared page tickets run out, so
    the pieces of a sequence, their running maxima and the fp16 rounding of
    the probabilities can change from call to call."""
    d = (a.float() - b.float()).abs()
    dmax, dmean = d.max().item(), d.mean().item()
    print(f"{what}: call-to-call max={dmax:.3e} mean={dmean:.3e}", flush=True)
    assert dmax <= MAX_ABS and dmean <= MEAN_ABS, (what, dmax, dmean)


def check_layouts(w, what, expected=None, **kw):
    """Parity of both K/V arena layouts (the reference's rows and the page
    tiles) holding the same rows; the kernel does the same arithmetic for
    both, so their outputs agree within the parity bar too. Leaves ``w`` in
    the page layout and returns its output."""
    if expected is None:
        expected = oracle(w)
    got = {}
    for layout in ("rows", "pages"):
        w.to_layout(layout)
        got[layout] = run(w, **kw)
        assert_parity(got[layout], expected, f"{what} [{layout}]")
    assert_consistent(got["rows"], got["pages"], what)
    return got["pages"]


def test_closed_form_from_cuda_tests_at_kernel_page_size(gpu):
    """tests/cuda_tests.cu:207-262 generalised to page 16 and head_dim 64: key
    (1,0,..) at position 0, (0,1,..) at 1..15 (physical page 1), (1,1,..) at 16
    (physical page 0); values (1,2,3,4,..), (5,6,7,8,..), (2,4,6,8,..)."""
    D, P = 64, 16
    keys = torch.zeros((2 * P, 1, D), dtype=torch.float16)
    values = torch.zeros((2 * P, 1, D), dtype=torch.float16)
    k0, k1, k2 = [1, 0, 0, 0], [0, 1, 0, 0], [1, 1, 0, 0]
    v0, v1, v2 = [1, 2, 3, 4], [5, 6, 7, 8], [2, 4, 6, 8]
    keys[P + 0, 0, :4] = torch.tensor(k0)
    values[P + 0, 0, :4] = torch.tensor(v0)
    for t in range(1, P):
        keys[P + t, 0, :4] = torch.tensor(k1)
        values[P + t, 0, :4] = torch.tensor(v1)
    keys[0, 0, :4] = torch.tensor(k2)
    values[0, 0, :4] = torch.tensor(v2)
    q = torch.zeros((1, 2, D), dtype=torch.float16)
    q[0, :, :2] = 1.0
    tables = torch.tensor([[1, 0]], dtype=torch.int32)
    lengths = torch.tensor([17], dtype=torch.int32)
    out = paged_decode_attention(q.to(gpu), keys.to(gpu), values.to(gpu), tables.to(gpu),
                                 lengths.to(gpu), page_size=P, longest=17, scale=0.5)
    e5, e1 = math.exp(0.5), math.exp(1.0)
    expected = (e5 * np.array(v0) + 15 * e5 * np.array(v1) + e1 * np.array(v2)) / (16 * e5 + e1)
    got = out.float().cpu().numpy()
    for h in range(2):
        np.testing.assert_allclose(got[0, h, :4], expected, atol=MAX_ABS)
        assert not got[0, h, 4:].any()


SMALL = {
    1: dict(batch=4, length=1024),
    2: dict(batch=8, low=512, high=2048),
    3: dict(batch=1, length=8192),
    4: dict(batch=6, low=2000, high=5000),
    5: dict(batch=24, low=16, high=8192, shared=6, prefix=1024),
}


@pytest.mark.parametrize("config", [1, 2, 3, 4, 5])
def test_configs_reduced(gpu, config):
    w = workloads.CONFIGS[config](device=gpu, **SMALL[config])
    check_layouts(w, f"config{config}-reduced")


@pytest.mark.parametrize("config", [1, 2, 4])
def test_configs_full_size(gpu, config):
    w = workloads.CONFIGS[config](device=gpu)
    check_layouts(w, f"config{config}-full")


@pytest.mark.parametrize("batch, length", [(1, 32768), (1, 131072), (2, 32768), (2, 131072),
                                           (4, 32768), (4, 131072)])
def test_config3_long_context_full_size(gpu, batch, length):
    """All six points of BASELINE config 3 (B in {1, 2, 4} x {32768, 131072},
    ~8 planted x8 keys per sequence and kv head, pages fragmented over a 2x
    arena); B = 4 x 131072 reads 2.15 GB of K/V per call. The long sequences
    are cut into the most pieces, so the log-sum-exp merge of large planted
    logits is exercised hardest here."""
    w = workloads.config3(device=gpu, batch=batch, length=length)
    assert w.meta["planted"] == 8
    expected = oracle(w)
    got = check_layouts(w, f"config3-b{batch}-{length}", expected)
    # The fixed split gives the same result bit for bit on a second call.
    a = run_fixed(w)
    assert_parity(a, expected, f"config3-b{batch}-{length} fixed")
    assert torch.equal(run_fixed(w), a)
    del got


def test_config5_full_size(gpu):
    w = workloads.config5(device=gpu)
    check_layouts(w, "config5-full")
    assert w.unique_kv_bytes() < w.kv_bytes()


def test_split_size_does_not_change_the_result(gpu):
    """The output is independent of the split plan (fp32 rounding aside)."""
    w = workloads.config2(device=gpu)
    expected = oracle(w)
    w.to_layout("pages")
    outs = []
    for split_pages in (4, 9, 16, 64):
        out = run(w, split_pages=split_pages)
        assert_parity(out, expected, f"config2 split_pages={split_pages}")
        outs.append(out.float())
    for other in outs[1:]:
        assert (other - outs[0]).abs().max().item() <= 2e-3


def test_longest_hint_understated_stays_correct(gpu):
    w = workloads.config2(device=gpu, batch=8, low=512, high=4096)
    assert_parity(run(w, longest=16), oracle(w), "longest=16")


@pytest.mark.parametrize("shape", workloads.REFERENCE_TEST_SHAPES)
def test_reference_kernel_test_shapes(gpu, shape):
    """The five shapes of test_mlx_engine.py:422-431 (16-bit); head_dim 4 runs
    the generic kernel (8-bit versions in test_gpu_shapes.py)."""
    w = workloads.reference_test_case(*shape, device=gpu)
    check_layouts(w, f"reftest{shape[:3]}")


@pytest.mark.parametrize("q_heads, kv_heads, head_dim, page", [
    (8, 8, 64, 16), (14, 2, 64, 16), (16, 2, 64, 32), (12, 4, 80, 16), (24, 4, 96, 64),
    (32, 4, 128, 16), (16, 1, 128, 16), (24, 2, 128, 16), (11, 1, 128, 16),
    (10, 2, 256, 16), (8, 1, 512, 16),
])
def test_head_shapes_and_page_sizes(gpu, q_heads, kv_heads, head_dim, page):
    rng = np.random.default_rng(q_heads * 1000 + head_dim + page)
    lengths = rng.integers(1, 1500, 5)
    lengths[0] = 1
    need = [math.ceil(n / page) for n in lengths]
    arena = sum(need) + 2
    order = rng.permutation(arena)
    tables = np.zeros((5, max(need)), dtype=np.int32)
    c = 0
    for b, n in enumerate(need):
        tables[b, :n] = order[c:c + n]
        c += n
    w = workloads.build("shape", lengths=lengths, tables=tables, arena_pages=arena,
                        q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim,
                        page_size=page, scale=head_dim ** -0.5, device=gpu, seed=7)
    what = f"shape{q_heads}/{kv_heads}/{head_dim}/P{page}"
    expected = oracle(w)
    check_layouts(w, what, expected)
    check_layouts(w, what + " split4", expected, split_pages=4)


def test_edge_lengths_and_empty_sequences(gpu):
    lengths = [0, 1, 15, 16, 17, 31, 32, 33, 255, 256, 257, -3]
    page = 16
    need = [max(0, math.ceil(n / page)) for n in lengths]
    arena = sum(need) + 1
    order = np.random.default_rng(3).permutation(arena)
    tables = np.zeros((len(lengths), max(need)), dtype=np.int32)
    c = 0
    for b, n in enumerate(need):
        tables[b, :n] = order[c:c + n]
        c += n
    w = workloads.build("edges", lengths=lengths, tables=tables, arena_pages=arena,
                        q_heads=28, kv_heads=4, head_dim=128, page_size=page,
                        scale=128 ** -0.5, device=gpu, seed=9)
    expected = oracle(w)
    for split_pages in (0, 4):
        got = check_layouts(w, f"edges split={split_pages}", expected, split_pages=split_pages)
        assert not got[0].any() and not got[-1].any()


def test_window_released_pages_and_poison(gpu):
    """Rows outside every window, released (-1) pages and padding never leak
    into the result, even when they hold NaN/inf (config 4 layout)."""
    w = workloads.config4(device=gpu, batch=8, low=1100, high=6000, window=300)
    clean = run(w).float().cpu()
    tables = w.tables.cpu().numpy()
    n = w.lengths.cpu().numpy()
    visible = torch.zeros(w.keys.shape[0], dtype=torch.bool)
    for b in range(w.batch):
        pos = np.arange(n[b] - w.window, n[b])
        rows = tables[b][pos // 16].astype(np.int64) * 16 + pos % 16
        visible[torch.as_tensor(rows)] = True
    hidden = (~visible).nonzero().squeeze(1).to(gpu)
    w.keys[hidden] = float("nan")
    w.values[hidden] = float("inf")
    poisoned = run(w).float().cpu()
    assert_consistent(clean, poisoned, "poisoned window")
    assert_parity(poisoned, oracle(w), "poisoned window")
    w.to_layout("pages")
    assert_consistent(clean, run(w).float().cpu(), "poisoned window [pages]")


def test_released_page_inside_window_is_masked(gpu):
    w = workloads.config2(device=gpu, batch=4, low=600, high=900)
    t = w.tables.cpu().numpy()
    t[1, 3] = -1
    t[2, 0] = -1
    t[3, 5] = 10**9  # beyond the arena: masked as well
    w.tables = torch.as_tensor(t, device=gpu)
    check_layouts(w, "released inside range")


def test_softcap(gpu):
    w = workloads.config2(device=gpu, batch=6, low=100, high=3000)
    w.softcap = 1.5
    check_layouts(w, "softcap")


def test_repeated_calls_reuse_the_workspace(gpu):
    """The split counters return to zero: alternate shapes on one workspace."""
    a = workloads.config2(device=gpu, batch=6, low=2000, high=6000)
    b = workloads.config5(device=gpu, batch=12, low=16, high=6000, shared=3, prefix=512)
    ea, eb = oracle(a), oracle(b)
    first = run(a, split_pages=4)
    for _ in range(3):
        assert_parity(run(b, split_pages=8), eb, "alt-b")
        again = run(a, split_pages=4)
        assert_consistent(again, first, "alt-a again")
    assert_parity(first, ea, "alt-a")


def test_separate_passes_equal_the_combined_call(gpu):
    """pda_decode_split then pda_decode_merge == pda_paged_decode_attention."""
    w = workloads.config2(device=gpu, batch=12, low=300, high=5000)
    combined = run(w)
    kw = dict(page_size=w.page_size, longest=w.longest, scale=w.scale)
    out = torch.full_like(w.q, float("nan"))
    paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths, out=out,
                           passes="split", **kw)
    paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths, out=out,
                           passes="merge", **kw)
    torch.cuda.synchronize()
    assert_consistent(out, combined, "split + merge")


def test_one_workspace_serves_shapes_with_different_layouts(gpu):
    """Regression: a window/D=256 call with few units leaves float partials
    where a larger batch keeps its split counters unless the counters live in
    a fixed header. Alternate the two layouts on one workspace."""
    from instinct_amd import hip_kernels

    hip_kernels._workspaces.clear()
    a = workloads.config4(device=gpu, batch=6, low=2000, high=5000)
    b = workloads.config5(device=gpu, batch=24, low=16, high=8192, shared=6, prefix=1024)
    ea, eb = oracle(a), oracle(b)
    for i in range(2):
        assert_parity(run(a, split_pages=4), ea, f"layout-a{i}")
        assert_parity(run(b), eb, f"layout-b{i}")


@pytest.mark.parametrize("layout", ["rows", "pages"])
def test_decode_batch_writes_then_attends(gpu, layout):
    """DecodeBatch (batches.py:142-226 counterpart): the new token's K/V is
    scattered into the arena before attention reads it."""
    from instinct_amd.batches import DecodeBatch
    from instinct_amd.paged_kv import KVCache, KVGroup, pages_to_rows

    rng = np.random.default_rng(21)
    page = 16
    groups = [KVGroup("full", (0, 1), kv_heads=2, head_dim=128),
              KVGroup("local", (2,), kv_heads=2, head_dim=128, window=64)]
    cache = KVCache(groups, page_size=page, capacities={"full": 64, "local": 64}, device=gpu,
                    layout=layout)
    positions = np.array([0, 15, 16, 100, 333])
    tables = {}
    for name in ("full", "local"):
        pool = cache.pools[name]
        tables[name] = [np.array([pool.allocate(reserved=False)
                                  for _ in range(p // page + 1)]) for p in positions]
    gen = torch.Generator(device=gpu).manual_seed(0)
    for layer in range(3):
        cache.keys[layer].normal_(generator=gen)
        cache.values[layer].normal_(generator=gen)
    batch = DecodeBatch(cache, torch.zeros(5, device=gpu), positions=positions, tables=tables)
    for layer in range(3):
        group = cache.layer_group[layer]
        q = torch.randn((5, 16, 128), generator=gen, device=gpu).half()
        k = torch.randn((5, 2, 128), generator=gen, device=gpu).half()
        v = torch.randn((5, 2, 128), generator=gen, device=gpu).half()
        out = batch.attend(layer, q, k, v, scale=128 ** -0.5)
        assert out.shape == (5, 16 * 128)
        packed = batch._tables[group.name].cpu().numpy()
        rows = packed[np.arange(5), positions // page] * page + positions % page
        assert torch.equal(cache.gather(layer, torch.as_tensor(rows, device=gpu))[0], k)
        keys, values = cache.keys[layer], cache.values[layer]
        if layout == "pages":
            keys, values = pages_to_rows(keys), pages_to_rows(values)
        expected = cpu_oracle.decode_f64(
            q.cpu().numpy(), keys.cpu().numpy(), values.cpu().numpy(), packed,
            positions + 1, page_size=page, scale=128 ** -0.5, window=group.window)
        assert_parity(out.view(5, 16, 128), expected, f"layer{layer}")


def test_decode_batch_repeats_bit_for_bit(gpu):
    """Two identical decode steps through DecodeBatch give bitwise-equal
    outputs (the default fixed split points; the reference's split ranges are
    fixed too, metal_kernels.py:32-36, and its engine compares token streams
    exactly, tests/test_mlx_engine.py:225-237). Long sequences, so every unit
    is cut over many waves, on the matrix-core (7 heads per kv head) and the
    VALU (4 heads) kernels."""
    from instinct_amd.batches import DecodeBatch
    from instinct_amd.paged_kv import KVCache, KVGroup

    page = 16
    groups = [KVGroup("g7", (0,), kv_heads=4, head_dim=128),
              KVGroup("g4", (1,), kv_heads=8, head_dim=128)]
    cache = KVCache(groups, page_size=page, capacities={"g7": 2048, "g4": 2048}, device=gpu)
    positions = np.array([4000, 1234, 7000, 333, 5555, 2600, 16, 6100])
    tables = {}
    for name in ("g7", "g4"):
        pool = cache.pools[name]
        tables[name] = [np.array([pool.allocate(reserved=False)
                                  for _ in range(p // page + 1)]) for p in positions]
    gen = torch.Generator(device=gpu).manual_seed(3)
    for layer in range(2):
        cache.keys[layer].normal_(generator=gen)
        cache.values[layer].normal_(generator=gen)
    batch = DecodeBatch(cache, torch.zeros(8, device=gpu), positions=positions, tables=tables)
    for layer, hq in ((0, 28), (1, 32)):
        hkv = cache.layer_group[layer].kv_heads
        q = torch.randn((8, hq, 128), generator=gen, device=gpu).half()
        k = torch.randn((8, hkv, 128), generator=gen, device=gpu).half()
        v = torch.randn((8, hkv, 128), generator=gen, device=gpu).half()
        first = batch.attend(layer, q, k, v, scale=128 ** -0.5).clone()
        for step in range(4):
            again = batch.attend(layer, q, k, v, scale=128 ** -0.5)
            assert torch.equal(again, first), f"layer {layer}: step {step + 1} differs"
