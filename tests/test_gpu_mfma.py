"""Decode on the matrix cores: GQA groups of 5 or more query heads per kv head
(any group at head dim 512).

The reference serves a whole GQA group from one K/V read whatever its size
(32 x G x R threads per threadgroup, metal_kernels.py:191-192,216-217). Here
groups of 5 to 16 heads (and larger groups as units of up to 16) run
S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_16x16x32 / 16x16x16 at head dims
64, 96, 128, 256 and 512 (four-wave workgroups, accumulators in AGPRs), one
K/V read per unit. Checked against the float64
oracle (max-abs 2e-3, mean-abs 2e-4; bf16 at its own bar,
test_gpu_bf16.py), in both arena layouts, with windows, released pages and
NaN/inf poison, softcap, ragged pages, key ranges split at many points, the
fixed-split mode, and the separate split/merge passes.
"""

import math

import numpy as np
import pytest
import torch

from instinct_amd import workloads
from instinct_amd.hip_kernels import decode_kernel_names, paged_decode_attention
from instinct_amd.paged_kv import pages_to_rows
from oracle import cpu_oracle
from oracle import paged_attention as pa

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-3
MEAN_ABS = 2e-4
BF16_MAX_ABS = 1.6e-2
BF16_MEAN_ABS = 1.6e-3


def make(gpu, *, q_heads, kv_heads, head_dim, lengths, page=16, window=0, softcap=0.0,
         seed=0):
    rng = np.random.default_rng(seed)
    need = [max(0, math.ceil(n / page)) for n in lengths]
    arena = sum(need) + 4
    order = rng.permutation(arena)
    tables = np.zeros((len(lengths), max(1, max(need))), dtype=np.int32)
    c = 0
    for b, n in enumerate(need):
        tables[b, :n] = order[c:c + n]
        c += n
    return workloads.build(f"mf{q_heads}/{kv_heads}/{head_dim}", lengths=lengths,
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


def oracle(w):
    q, k, v, t, n = w.numpy()
    return cpu_oracle.decode_f64(q, k, v, t, n, page_size=w.page_size, scale=w.scale,
                                 window=w.window, softcap=w.softcap)


def check(w, what, **kw):
    names = decode_kernel_names(w.q_heads, w.kv_heads, w.head_dim)
    assert names["matrix_cores"], names
    want = oracle(w)
    for layout in ("rows", "pages"):
        w.to_layout(layout)
        stats(run(w, **kw), want, f"{what} [{layout}]")
        stats(run(w, deterministic=True, **kw), want, f"{what} [{layout}, fixed]")


@pytest.mark.parametrize("head_dim", [64, 96, 128, 256, 512])
@pytest.mark.parametrize("q_heads,kv_heads", [(5, 1), (6, 1), (7, 1), (28, 4), (14, 2),
                                              (8, 1), (16, 2), (9, 1), (11, 1), (12, 1),
                                              (13, 1), (16, 1), (24, 2), (32, 2), (40, 2)])
def test_group_sizes_and_head_dims(gpu, q_heads, kv_heads, head_dim):
    lengths = [1, 15, 16, 17, 600, 2500, 33]
    w = make(gpu, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, lengths=lengths,
             seed=q_heads * 100 + head_dim)
    check(w, f"mf {q_heads}/{kv_heads} D{head_dim}")


@pytest.mark.parametrize("head_dim", [64, 128, 256, 512])
def test_split_into_many_pieces(gpu, head_dim):
    """split_pages 1 and 3: every unit cut into many pieces, merged."""
    w = make(gpu, q_heads=16, kv_heads=1, head_dim=head_dim, lengths=[3000, 50, 1], seed=5)
    check(w, f"mf split1 D{head_dim}", split_pages=1)
    check(w, f"mf split3 D{head_dim}", split_pages=3)


@pytest.mark.parametrize("head_dim", [128, 512])
@pytest.mark.parametrize("page", [1, 4, 12, 24, 64])
def test_page_sizes(gpu, page, head_dim):
    w = make(gpu, q_heads=16, kv_heads=2, head_dim=head_dim, page=page,
             lengths=[1, page, page + 1, 777, 1500], seed=page)
    check(w, f"mf P{page} D{head_dim}")


@pytest.mark.parametrize("head_dim", [128, 512])
def test_window_softcap_released_pages_and_poison(gpu, head_dim):
    P, W = 16, 300
    lengths = np.array([1200, 301, 299, 4000, 9])
    w = make(gpu, q_heads=24, kv_heads=2, head_dim=head_dim, lengths=list(lengths), window=W,
             softcap=30.0, seed=8)
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
    check(w, f"mf window softcap poison D{head_dim}")


def test_planted_large_logits(gpu):
    """Config 3's planted x8 keys with 16 query heads per kv head: large
    logits push the lazy running max up mid-stream."""
    w = make(gpu, q_heads=32, kv_heads=2, head_dim=128, lengths=[32768, 9000], seed=3)
    rng = np.random.default_rng(4)
    t = w.tables.cpu().numpy()
    for b, n in enumerate([32768, 9000]):
        pos = rng.choice(n, size=(2, 8))
        for kvh in range(2):
            rows = t[b][pos[kvh] // 16].astype(np.int64) * 16 + pos[kvh] % 16
            w.keys[torch.as_tensor(rows, device=gpu), kvh] *= 8
    check(w, "mf planted")


def test_fixed_split_is_bitwise_reproducible(gpu):
    w = make(gpu, q_heads=16, kv_heads=1, head_dim=128, lengths=[30000, 4000, 512], seed=6)
    w.to_layout("pages")
    first = run(w, deterministic=True)
    stats(first, oracle(w), "mf fixed")
    for _ in range(4):
        assert torch.equal(run(w, deterministic=True), first)


def test_separate_passes(gpu):
    w = make(gpu, q_heads=16, kv_heads=2, head_dim=128, lengths=[5000, 300, 2222], seed=7)
    w.to_layout("pages")
    whole = run(w)
    kw = dict(page_size=w.page_size, longest=w.longest, scale=w.scale)
    out = torch.full_like(w.q, float("nan"))
    paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths, out=out,
                           passes="split", **kw)
    paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths, out=out,
                           passes="merge", **kw)
    torch.cuda.synchronize()
    d = (out.float() - whole.float()).abs()
    assert d.max().item() <= MAX_ABS and d.mean().item() <= MEAN_ABS


@pytest.mark.parametrize("q_heads,kv_heads,head_dim", [(16, 1, 128), (11, 1, 64), (24, 2, 256),
                                                       (8, 1, 96), (16, 2, 512), (11, 1, 512)])
def test_bf16(gpu, q_heads, kv_heads, head_dim):
    w = make(gpu, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim,
             lengths=[5, 900, 2049], seed=head_dim + q_heads).to_layout("pages")
    w.q, w.keys, w.values = (x.to(torch.bfloat16) for x in (w.q, w.keys, w.values))
    f = lambda x: x.float().cpu().numpy()  # noqa: E731
    want = pa.paged_decode_dense(f(w.q), f(pages_to_rows(w.keys)), f(pages_to_rows(w.values)),
                                 w.tables.cpu().numpy(), w.lengths.cpu().numpy(),
                                 page_size=w.page_size, scale=w.scale)
    out = run(w)
    assert out.dtype == torch.bfloat16
    stats(out, want, f"mf bf16 {q_heads}/{kv_heads} D{head_dim}", BF16_MAX_ABS, BF16_MEAN_ABS)
