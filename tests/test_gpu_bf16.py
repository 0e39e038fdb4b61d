"""bf16 queries, K/V and output (the model dtype of the reference's bf16
models, paged_kv.py:156-292): the decode call (pda_paged_decode_attention_bf16
via the C-ABI) and the prefill call against the float64 oracle on the same
bf16 values.

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
