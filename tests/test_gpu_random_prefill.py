"""Seeded random prefill chunks against the float64 prefill oracle: each seed
draws the heads, the head dim (tuned and generic ones), the page size
(ragged ones included), the chunk's start and length, a window, a softcap,
released pages inside the visible range, a forced or automatic key-range
split, the element type (fp16, bf16 or the 8-bit cache) and the arena
layout. Bar: the north star's (fp16 and 8-bit: max-abs 2e-3, mean-abs
2e-4; 8-bit against attention over the rows the reference's gather
dequantizes) and test_gpu_bf16.py's for bf16. Each case prints itself
before it runs."""

import numpy as np
import pytest
import torch

from instinct_amd.hip_kernels import paged_prefill_attention
from instinct_amd.paged_kv import rows_to_pages
from oracle import kv8
from oracle import paged_attention as pa

pytestmark = pytest.mark.gpu

BARS = {"f16": (2e-3, 2e-4), "q8": (2e-3, 2e-4), "bf16": (1.6e-2, 1.6e-3)}


def draw(seed):
    rng = np.random.default_rng(5000 + seed)
    kind = ("f16", "bf16", "q8")[seed % 3]
    d = int(rng.choice([64, 128, 256] if kind == "q8" else [64, 80, 96, 128, 130, 256, 512]))
    hkv = int(rng.choice([1, 2, 4]))
    group = int(rng.choice([1, 2, 4, 7, 8]))
    if d >= 256:
        group = min(group, 4)
    page = int(rng.choice([16, 16, 8, 32, 12, 5]))
    start = int(rng.choice([0, 0, rng.integers(1, 2000)]))
    count = int(rng.choice([1, rng.integers(2, 300), 300]))
    window = int(rng.choice([0, 0, rng.integers(1, 1500)]))
    softcap = float(rng.choice([0.0, 0.0, 30.0]))
    splits = int(rng.choice([0, 0, 2, 3]))
    layout = str(rng.choice(["rows", "pages"]))
    return dict(kind=kind, d=d, hkv=hkv, hq=hkv * group, page=page, start=start, count=count,
                window=window, softcap=softcap, splits=splits, layout=layout)


@pytest.mark.parametrize("seed", range(36))
def test_random_prefill_chunk(gpu, seed):
    c = draw(seed)
    print(f"seed {seed}: {c}", flush=True)
    rng = np.random.default_rng(seed)
    P, d, hq, hkv = c["page"], c["d"], c["hq"], c["hkv"]
    pages = (c["start"] + c["count"] + P - 1) // P
    arena = pages + 3
    table = rng.permutation(arena)[:pages].astype(np.int32)
    if pages > 2 and seed % 4 == 0:
        table[int(rng.integers(0, pages - 1))] = -1  # a released page inside the range
    rows = arena * P
    keys = rng.standard_normal((rows, hkv, d)).astype(np.float16)
    values = rng.standard_normal((rows, hkv, d)).astype(np.float16)
    q = rng.standard_normal((c["count"], hq, d)).astype(np.float16)
    kw = dict(start=c["start"], page_size=P, scale=d ** -0.5, window=c["window"],
              softcap=c["softcap"])
    pages_layout = c["layout"] == "pages"
    if c["kind"] == "q8":
        kq, ks = kv8.quantize(keys)
        vq, vs = kv8.quantize(values)
        want = pa.paged_prefill_dense(q, kv8.gather_dequantize(kq, ks),
                                      kv8.gather_dequantize(vq, vs), table, **kw)
        arenas = [torch.as_tensor(x, device=gpu) for x in (kq, vq)]
        scales = [torch.as_tensor(x, device=gpu) for x in (ks, vs)]
        if pages_layout:
            arenas = [rows_to_pages(x, P) for x in arenas]
            scales = [x.view(-1, P, hkv).permute(0, 2, 1).contiguous() for x in scales]
        got = paged_prefill_attention(torch.as_tensor(q, device=gpu), *arenas,
                                      torch.as_tensor(table, device=gpu), splits=c["splits"],
                                      scales=tuple(scales), **kw)
    else:
        dtype = torch.bfloat16 if c["kind"] == "bf16" else torch.float16
        tq, tk, tv = (torch.as_tensor(x, device=gpu).to(dtype) for x in (q, keys, values))
        f = lambda x: x.float().cpu().numpy()  # noqa: E731
        want = pa.paged_prefill_dense(f(tq), f(tk), f(tv), table, **kw)
        if pages_layout:
            tk, tv = rows_to_pages(tk, P), rows_to_pages(tv, P)
        got = paged_prefill_attention(tq, tk, tv, torch.as_tensor(table, device=gpu),
                                      splits=c["splits"], **kw)
    torch.cuda.synchronize()
    got = got.float().cpu().numpy()
    assert np.isfinite(got).all(), f"seed {seed}: non-finite output"
    err_max, err_mean = pa.error_stats(got, want)
    print(f"seed {seed}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}", flush=True)
    max_abs, mean_abs = BARS[c["kind"]]
    assert err_max <= max_abs and err_mean <= mean_abs, (seed, c, err_max, err_mean)
