"""Seeded random decode calls against the float64 oracle: each seed draws a
shape (kv heads, GQA group, head dim including generic ones, page size
including ragged ones), a batch of lengths (empty, one-token and long
sequences), a window and a softcap, the element type (fp16, bf16 or the
8-bit cache), the arena layout and the split mode, so that the library's
dispatch (VALU or matrix-core kernels, local mode, the whole-row or
row-sliced merge) meets combinations no hand-written case names. The bar is
the north star's (fp16 and 8-bit: max-abs 2e-3, mean-abs 2e-4; 8-bit against
attention over the dequantized rows) and test_gpu_bf16.py's for bf16. Each
case prints itself before it runs."""

import math

import numpy as np
import pytest
import torch

from instinct_amd import workloads
from instinct_amd.hip_kernels import decode_kernel_names, paged_decode_attention
from instinct_amd.paged_kv import rows_to_pages
from oracle import kv8
from oracle import paged_attention as pa

pytestmark = pytest.mark.gpu

BARS = {"f16": (2e-3, 2e-4), "q8": (2e-3, 2e-4), "bf16": (1.6e-2, 1.6e-3)}
DIMS16 = (4, 64, 80, 96, 128, 130, 192, 256, 512)
DIMS8 = (64, 80, 96, 128, 130, 256, 512)


def draw(seed):
    rng = np.random.default_rng(1000 + seed)
    kind = ("f16", "bf16", "q8")[seed % 3]
    dim = int(rng.choice(DIMS8 if kind == "q8" else DIMS16))
    kv_heads = int(rng.choice([1, 2, 4, 8] if dim < 512 else [1, 2]))
    group = int(rng.choice([1, 2, 3, 4, 5, 7, 8, 11, 16]))
    page = int(rng.choice([16, 16, 16, 8, 32, 12, 5]))
    batch = int(rng.integers(1, 7))
    longest = int(rng.choice([300, 2000, 6000]))
    lengths = [int(rng.choice([0, 1, rng.integers(1, longest + 1), longest]))
               for _ in range(batch)]
    if max(lengths) == 0:
        lengths[0] = longest
    window = int(rng.choice([0, 0, 0, 1, 64, 1000]))
    softcap = float(rng.choice([0.0, 0.0, 30.0]))
    layout = str(rng.choice(["rows", "pages"]))
    fixed = bool(rng.integers(0, 2))
    return dict(kind=kind, dim=dim, kv_heads=kv_heads, group=group, page=page,
                lengths=lengths, window=window, softcap=softcap, layout=layout, fixed=fixed)


def build(gpu, c, seed):
    """Randomly permuted pages with a few spare ones, zero-padded tables."""
    rng = np.random.default_rng(seed)
    need = [math.ceil(n / c["page"]) for n in c["lengths"]]
    arena = sum(need) + 3
    order = rng.permutation(arena)
    tables = np.zeros((len(need), max(1, max(need))), dtype=np.int32)
    at = 0
    for b, n in enumerate(need):
        tables[b, :n] = order[at:at + n]
        at += n
    return workloads.build(f"random-{seed}", lengths=c["lengths"], tables=tables,
                           arena_pages=arena, q_heads=c["kv_heads"] * c["group"],
                           kv_heads=c["kv_heads"], head_dim=c["dim"], page_size=c["page"],
                           scale=c["dim"] ** -0.5, window=c["window"], softcap=c["softcap"],
                           device=gpu, seed=seed + 7)


@pytest.mark.parametrize("seed", range(48))
def test_random_decode_call(gpu, seed):
    c = draw(seed)
    w = build(gpu, c, seed)
    P, hkv = c["page"], c["kv_heads"]
    names = decode_kernel_names(w.q_heads, hkv, c["dim"], bits=8 if c["kind"] == "q8" else 16,
                                bf16=c["kind"] == "bf16", batch=w.batch, longest=w.longest,
                                page_size=P, table_width=int(w.tables.shape[1]),
                                window=c["window"])
    print(f"seed {seed}: {c} -> {names['split']} merge {names['merge']}", flush=True)
    q, k, v, t, n = w.numpy()
    kw = dict(page_size=P, longest=w.longest, scale=w.scale, window=c["window"],
              softcap=c["softcap"], deterministic=c["fixed"])
    dense = dict(page_size=P, scale=w.scale, window=c["window"], softcap=c["softcap"])
    pages = c["layout"] == "pages"
    if c["kind"] == "q8":
        kq, ks = kv8.quantize(k)
        vq, vs = kv8.quantize(v)
        want = pa.paged_decode_dense(q, kv8.dequantize(kq, ks), kv8.dequantize(vq, vs), t, n,
                                     **dense)
        arenas = [torch.as_tensor(x, device=gpu) for x in (kq, vq)]
        scales = [torch.as_tensor(x, device=gpu) for x in (ks, vs)]
        if pages:
            arenas = [rows_to_pages(x, P) for x in arenas]
            scales = [x.view(-1, P, hkv).permute(0, 2, 1).contiguous() for x in scales]
        out = paged_decode_attention(w.q, *arenas, w.tables, w.lengths, scales=tuple(scales), **kw)
    else:
        if c["kind"] == "bf16":
            w.q, w.keys, w.values = (x.bfloat16() for x in (w.q, w.keys, w.values))
        f = lambda x: x.float().cpu().numpy()  # noqa: E731
        want = pa.paged_decode_dense(f(w.q), f(w.keys), f(w.values), t, n, **dense)
        if pages:
            w.to_layout("pages")
        out = paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths, **kw)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all(), f"seed {seed}: non-finite output"
    err_max, err_mean = pa.error_stats(got, want)
    print(f"seed {seed}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}", flush=True)
    max_abs, mean_abs = BARS[c["kind"]]
    assert err_max <= max_abs and err_mean <= mean_abs, (seed, c, err_max, err_mean)
