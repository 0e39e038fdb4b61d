"""Every shape the reference op accepts, and the fixed-split mode.

The reference decode op takes any head_dim (its IN_HEAD guard,
metal_kernels.py:28-30) and any page size (the PAGE template, :204), and its
kernel test runs head_dim 4 and head_dim 80 at 8 bits
(tests/test_mlx_engine.py:422-432). Here head dims 64, 80, 96, 128, 256 and
512 run tuned kernels and every other even head dim up to 512 a generic one;
page sizes that are not a multiple of a wave step's keys take a partial last
step per page. All of it is checked against the float64 oracle (bar: the
north star's max-abs 2e-3 / mean-abs 2e-4 for fp16; bf16 and 8-bit as in
their own test files), in both arena layouts.

Fixed split points (``deterministic=True``, the default; flags 0 at the
C-ABI) fix where the wave pairs cut the page stream, so repeated calls are
bitwise identical, as the reference's fixed split ranges make its output
(metal_kernels.py:32-36); ``deterministic=False`` passes PDA_DECODE_RACING.
"""

import math

import numpy as np
import pytest
import torch

from instinct_amd import workloads
from instinct_amd.hip_kernels import paged_decode_attention
from instinct_amd.paged_kv import pages_to_rows, rows_to_pages
from oracle import cpu_oracle, kv8
from oracle import paged_attention as pa

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-3
MEAN_ABS = 2e-4
BF16_MAX_ABS = 1.6e-2   # the bf16 bar of test_gpu_bf16.py
BF16_MEAN_ABS = 1.6e-3


def make(gpu, *, q_heads, kv_heads, head_dim, page, lengths, window=0, softcap=0.0, seed=0,
         spare=3):
    """A workload with randomly permuted pages (``spare`` unused pages in the
    arena), zero-padded tables, scale head_dim^-0.5."""
    rng = np.random.default_rng(seed)
    need = [max(0, math.ceil(n / page)) for n in lengths]
    arena = sum(need) + spare
    order = rng.permutation(arena)
    tables = np.zeros((len(lengths), max(1, max(need))), dtype=np.int32)
    c = 0
    for b, n in enumerate(need):
        tables[b, :n] = order[c:c + n]
        c += n
    return workloads.build(f"shape{q_heads}/{kv_heads}/{head_dim}/P{page}", lengths=lengths,
                           tables=tables, arena_pages=arena, q_heads=q_heads,
                           kv_heads=kv_heads, head_dim=head_dim, page_size=page,
                           scale=head_dim ** -0.5, window=window, softcap=softcap,
                           device=gpu, seed=seed + 1)


def run(w, **kw):
    out = paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths,
                                 page_size=w.page_size, longest=w.longest, scale=w.scale,
                                 window=w.window, softcap=w.softcap, **kw)
    torch.cuda.synchronize()
    return out


def stats(got, want, what, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    got = got.float().cpu().numpy()
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err_max, err_mean = pa.error_stats(got, want)
    print(f"{what}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}", flush=True)
    assert err_max <= max_abs and err_mean <= mean_abs, (what, err_max, err_mean)


def check16(w, what, **kw):
    """fp16 parity in both layouts, with and without the fixed split."""
    q, k, v, t, n = w.numpy()
    want = cpu_oracle.decode_f64(q, k, v, t, n, page_size=w.page_size, scale=w.scale,
                                 window=w.window, softcap=w.softcap)
    for layout in ("rows", "pages"):
        w.to_layout(layout)
        stats(run(w, **kw), want, f"{what} [{layout}]")
        stats(run(w, deterministic=True, **kw), want, f"{what} [{layout}, fixed]")


def check_bf16(w, what):
    w.q, w.keys, w.values = (x.to(torch.bfloat16) for x in (w.q, w.keys, w.values))
    keys, values = w.keys, w.values
    if w.layout == "pages":
        keys, values = pages_to_rows(keys), pages_to_rows(values)
    f = lambda x: x.float().cpu().numpy()  # noqa: E731
    want = pa.paged_decode_dense(f(w.q), f(keys), f(values), w.tables.cpu().numpy(),
                                 w.lengths.cpu().numpy(), page_size=w.page_size, scale=w.scale,
                                 window=w.window, softcap=w.softcap)
    out = run(w)
    assert out.dtype == torch.bfloat16
    stats(out, want, what, BF16_MAX_ABS, BF16_MEAN_ABS)


def scales_to_pages(scales, page_size):
    rows, heads = scales.shape
    return scales.view(rows // page_size, page_size, heads).permute(0, 2, 1).contiguous()


def check8(w, what, **kw):
    """8-bit K/V (the reference's quantize, paged_kv.py:50-55) against
    float64 attention over int8 * scale, both layouts."""
    q, k, v, t, n = w.numpy()
    kq, ks = kv8.quantize(k)
    vq, vs = kv8.quantize(v)
    want = pa.paged_decode_dense(q, kv8.dequantize(kq, ks), kv8.dequantize(vq, vs), t, n,
                                 page_size=w.page_size, scale=w.scale, window=w.window,
                                 softcap=w.softcap)
    dev, P = w.q.device, w.page_size
    for layout in ("rows", "pages"):
        keys, values = torch.as_tensor(kq, device=dev), torch.as_tensor(vq, device=dev)
        sk, sv = torch.as_tensor(ks, device=dev), torch.as_tensor(vs, device=dev)
        if layout == "pages":
            keys, values = rows_to_pages(keys, P), rows_to_pages(values, P)
            sk, sv = scales_to_pages(sk, P), scales_to_pages(sv, P)
        for fixed in (False, True):
            out = paged_decode_attention(w.q, keys, values, w.tables, w.lengths, page_size=P,
                                         longest=w.longest, scale=w.scale, window=w.window,
                                         softcap=w.softcap, scales=(sk, sv),
                                         deterministic=fixed, **kw)
            torch.cuda.synchronize()
            stats(out, want, f"{what} q8 [{layout}{', fixed' if fixed else ''}]")


# --- the reference's own kernel-test shapes ---------------------------------

@pytest.mark.parametrize("shape", workloads.REFERENCE_TEST_SHAPES)
@pytest.mark.parametrize("bits", [16, 8])
def test_reference_kernel_test_shapes_at_both_widths(gpu, shape, bits):
    """All five shapes of test_mlx_engine.py:422-431 at bits 16 and 8,
    (2, 1, 4, [9], 4, 0.0) and (8, 1, 80, [3, 300], 0, 30.0) included."""
    w = workloads.reference_test_case(*shape, device=gpu)
    what = f"reftest{shape[:3]}"
    if bits == 16:
        check16(w, what)
    else:
        check8(w, what)


# --- generic head dims --------------------------------------------------------

GENERIC = [  # q_heads, kv_heads, head_dim
    (2, 1, 2), (2, 1, 4), (4, 2, 6), (7, 1, 10), (8, 8, 16), (14, 2, 32), (6, 2, 48),
    (8, 1, 72), (5, 5, 100), (16, 2, 136), (4, 1, 160), (24, 4, 200), (3, 1, 250),
    (8, 2, 384), (2, 2, 510), (12, 4, 34),
]


@pytest.mark.parametrize("q_heads,kv_heads,head_dim", GENERIC)
def test_generic_head_dims(gpu, q_heads, kv_heads, head_dim):
    lengths = [1, 17, 300, 1234, 31]
    w = make(gpu, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, page=16,
             lengths=lengths, seed=head_dim)
    check16(w, f"generic {q_heads}/{kv_heads}/D{head_dim}")
    check16(w, f"generic {q_heads}/{kv_heads}/D{head_dim} split2", split_pages=2)


@pytest.mark.parametrize("q_heads,kv_heads,head_dim,window,softcap", [
    (8, 2, 4, 40, 0.0), (14, 2, 48, 0, 20.0), (8, 1, 200, 300, 0.0), (4, 4, 510, 0, 5.0)])
def test_generic_head_dims_window_softcap(gpu, q_heads, kv_heads, head_dim, window, softcap):
    w = make(gpu, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, page=16,
             lengths=[5, 999, 2100, 64], window=window, softcap=softcap, seed=2 * head_dim)
    check16(w, f"generic D{head_dim} window={window} softcap={softcap}")


@pytest.mark.parametrize("head_dim", [4, 48, 80, 100, 200])
def test_generic_head_dims_bf16(gpu, head_dim):
    w = make(gpu, q_heads=8, kv_heads=2, head_dim=head_dim, page=16,
             lengths=[3, 700, 1500], seed=3 * head_dim)
    check_bf16(w.to_layout("pages"), f"bf16 D{head_dim}")


@pytest.mark.parametrize("q_heads,kv_heads,head_dim,softcap", [
    (8, 1, 80, 30.0), (2, 1, 4, 0.0), (7, 1, 96, 0.0), (14, 2, 48, 0.0), (6, 2, 200, 0.0),
    (4, 2, 510, 0.0)])
def test_generic_head_dims_8bit(gpu, q_heads, kv_heads, head_dim, softcap):
    w = make(gpu, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, page=16,
             lengths=[3, 300, 1800, 17], softcap=softcap, seed=5 * head_dim)
    check8(w, f"8-bit {q_heads}/{kv_heads}/D{head_dim}")


# --- odd head dims ---------------------------------------------------------------
# The reference's IN_HEAD guard takes any head dim (metal_kernels.py:28-30).
# Odd ones run paged_decode_odd_kernel: rows 2-byte aligned (1-byte at 8
# bits), element-wise loads and stores, one query head per unit.

ODD = [  # q_heads, kv_heads, head_dim
    (2, 1, 1), (4, 2, 3), (7, 1, 5), (8, 2, 7), (14, 2, 33), (5, 5, 63), (8, 1, 129),
    (4, 2, 255), (2, 2, 511), (6, 3, 97),
]


@pytest.mark.parametrize("q_heads,kv_heads,head_dim", ODD)
def test_odd_head_dims(gpu, q_heads, kv_heads, head_dim):
    w = make(gpu, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, page=16,
             lengths=[1, 17, 300, 1234, 31], seed=head_dim)
    check16(w, f"odd {q_heads}/{kv_heads}/D{head_dim}")
    check16(w, f"odd {q_heads}/{kv_heads}/D{head_dim} split2", split_pages=2)


@pytest.mark.parametrize("q_heads,kv_heads,head_dim,page,window,softcap", [
    (8, 2, 7, 5, 40, 0.0), (4, 1, 33, 12, 0, 20.0), (6, 2, 129, 1, 300, 0.0),
    (2, 2, 511, 24, 0, 5.0)])
def test_odd_head_dims_pages_window_softcap(gpu, q_heads, kv_heads, head_dim, page, window,
                                           softcap):
    w = make(gpu, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, page=page,
             lengths=[5, 999, 2100, 64], window=window, softcap=softcap, seed=3 * head_dim)
    check16(w, f"odd D{head_dim} P{page} window={window} softcap={softcap}")


@pytest.mark.parametrize("head_dim", [1, 7, 63, 129, 511])
def test_odd_head_dims_bf16(gpu, head_dim):
    w = make(gpu, q_heads=8, kv_heads=2, head_dim=head_dim, page=16,
             lengths=[3, 700, 1500], seed=5 * head_dim)
    check_bf16(w.to_layout("pages"), f"bf16 odd D{head_dim}")


@pytest.mark.parametrize("q_heads,kv_heads,head_dim,softcap", [
    (2, 1, 1, 0.0), (8, 1, 7, 30.0), (6, 2, 65, 0.0), (4, 2, 255, 0.0), (2, 1, 511, 0.0)])
def test_odd_head_dims_8bit(gpu, q_heads, kv_heads, head_dim, softcap):
    w = make(gpu, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, page=16,
             lengths=[3, 300, 1800, 17], softcap=softcap, seed=7 * head_dim)
    check8(w, f"8-bit odd {q_heads}/{kv_heads}/D{head_dim}")


# --- any page size --------------------------------------------------------------

@pytest.mark.parametrize("page", [1, 2, 4, 5, 12, 24, 40])
@pytest.mark.parametrize("q_heads,kv_heads,head_dim", [
    (28, 4, 128), (14, 2, 64), (16, 8, 256), (16, 2, 512), (12, 4, 80), (24, 4, 96),
    (2, 1, 4)])
def test_page_sizes(gpu, page, q_heads, kv_heads, head_dim):
    lengths = [1, page, page + 1, 3 * page - 1, 400, 1000]
    w = make(gpu, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, page=page,
             lengths=lengths, seed=page * 7 + head_dim)
    check16(w, f"P{page} {q_heads}/{kv_heads}/D{head_dim}")


@pytest.mark.parametrize("page", [1, 4, 12])
@pytest.mark.parametrize("head_dim", [64, 128, 256, 512, 80, 4])
def test_page_sizes_8bit(gpu, page, head_dim):
    w = make(gpu, q_heads=8, kv_heads=2, head_dim=head_dim, page=page,
             lengths=[1, page + 3, 333, 900], seed=page + head_dim)
    check8(w, f"P{page} D{head_dim}")


@pytest.mark.parametrize("page", [4, 12])
def test_page_sizes_bf16(gpu, page):
    w = make(gpu, q_heads=28, kv_heads=4, head_dim=128, page=page, lengths=[5, 600, 1111],
             seed=page)
    check_bf16(w.to_layout("pages"), f"bf16 P{page}")


def test_ragged_pages_with_window_released_pages_and_poison(gpu):
    """Page size 12 with a window: pages wholly before the window are
    released (-1), the rows before the window hold NaN/inf, and the keys of a
    page's partial last step past the page belong to the next page (or
    tile) and must not be read."""
    P, W = 12, 100
    lengths = np.array([250, 101, 99, 1000, 7])
    w = make(gpu, q_heads=16, kv_heads=4, head_dim=128, page=P, lengths=list(lengths),
             window=W, seed=44)
    t = w.tables.cpu().numpy()
    visible = np.zeros(w.keys.shape[0], dtype=bool)
    for b, n in enumerate(lengths):
        first = max(0, n - W)
        t[b, : first // P] = -1
        pos = np.arange(first, n)
        visible[t[b][pos // P].astype(np.int64) * P + pos % P] = True
    w.tables = torch.as_tensor(t, device=gpu)
    hidden = torch.as_tensor(np.flatnonzero(~visible), device=gpu)
    w.keys[hidden] = float("nan")
    w.values[hidden] = float("inf")
    check16(w, "ragged window poison")


# --- fixed split: bitwise reproducible -------------------------------------------

@pytest.mark.parametrize("name,kw", [
    ("config2", dict(batch=16, low=512, high=8192)),
    ("config3", dict(batch=1, length=32768)),
    ("config5", dict(batch=48, low=16, high=16384, shared=8, prefix=1024)),
])
def test_fixed_split_is_bitwise_reproducible(gpu, name, kw):
    """Five calls with fixed split points give the same bits, within the
    parity bar of the oracle; config 3 carries the planted x8 keys whose
    large logits make the merge's rescaling matter most."""
    w = getattr(workloads, name)(device=gpu, **kw).to_layout("pages")
    q, k, v, t, n = w.numpy()
    want = cpu_oracle.decode_f64(q, k, v, t, n, page_size=w.page_size, scale=w.scale,
                                 window=w.window, softcap=w.softcap)
    first = run(w, deterministic=True)
    stats(first, want, f"{name} fixed")
    for i in range(4):
        junk = torch.randn(1 << 22, device=gpu)  # other work between the calls
        again = run(w, deterministic=True)
        del junk
        assert torch.equal(again, first), f"{name}: call {i + 1} differs"


def test_fixed_split_8bit_and_bf16_are_reproducible(gpu):
    w = workloads.config2(device=gpu, batch=8, low=1000, high=6000).to_layout("pages")
    _, k, v, _, _ = w.numpy()
    kq, ks = kv8.quantize(k)
    vq, vs = kv8.quantize(v)
    P = w.page_size
    keys = rows_to_pages(torch.as_tensor(kq, device=gpu), P)
    values = rows_to_pages(torch.as_tensor(vq, device=gpu), P)
    scales = (scales_to_pages(torch.as_tensor(ks, device=gpu), P),
              scales_to_pages(torch.as_tensor(vs, device=gpu), P))
    call8 = lambda: paged_decode_attention(  # noqa: E731
        w.q, keys, values, w.tables, w.lengths, page_size=P, longest=w.longest,
        scale=w.scale, scales=scales, deterministic=True)
    a = call8()
    for _ in range(3):
        assert torch.equal(call8(), a)
    wb = workloads.config2(device=gpu, batch=8, low=1000, high=6000).to_layout("pages")
    wb.q, wb.keys, wb.values = (x.to(torch.bfloat16) for x in (wb.q, wb.keys, wb.values))
    b = run(wb, deterministic=True)
    for _ in range(3):
        assert torch.equal(run(wb, deterministic=True), b)


# --- row-sliced merge: few heads, many pieces each ----------------------------

@pytest.mark.parametrize("q_heads,kv_heads,head_dim,lengths,window", [
    (8, 1, 128, [40000], 0),
    (16, 2, 512, [9000, 5], 0),
    (12, 4, 80, [30000], 0),
    (6, 2, 130, [20000, 700], 0),
    (4, 1, 96, [30000], 0),
    (8, 2, 256, [50000], 30000),
    (28, 4, 128, [30000], 0),
])
def test_row_sliced_merge(gpu, q_heads, kv_heads, head_dim, lengths, window):
    """One or two long sequences: the merge's workgroups each take one
    64-element slice of a head's row (a generic head dim's last slices are
    partly or wholly past it), in fp16, bf16 and with the fixed split."""
    from instinct_amd.hip_kernels import decode_kernel_names

    w = make(gpu, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, page=16,
             lengths=lengths, window=window, seed=head_dim + len(lengths))
    names = decode_kernel_names(q_heads, kv_heads, head_dim, batch=w.batch, longest=w.longest,
                                table_width=int(w.tables.shape[1]), window=window)
    assert names["merge_row_sliced"], names
    check16(w, f"sliced merge {q_heads}/{kv_heads}/D{head_dim}")
    check_bf16(w.to_layout("pages"), f"sliced merge bf16 {q_heads}/{kv_heads}/D{head_dim}")


@pytest.mark.parametrize("q_heads,kv_heads,head_dim,lengths", [
    (8, 2, 512, [12000]),
    (8, 1, 80, [20000]),
    (8, 2, 128, [20000, 9]),
])
def test_row_sliced_merge_8bit(gpu, q_heads, kv_heads, head_dim, lengths):
    from instinct_amd.hip_kernels import decode_kernel_names

    w = make(gpu, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, page=16,
             lengths=lengths, seed=3 * head_dim)
    names = decode_kernel_names(q_heads, kv_heads, head_dim, bits=8, batch=w.batch,
                                longest=w.longest, table_width=int(w.tables.shape[1]))
    assert names["merge_row_sliced"], names
    check8(w, f"sliced merge {q_heads}/{kv_heads}/D{head_dim}")
