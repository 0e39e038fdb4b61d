"""8-bit K/V under a bf16 model: bf16 queries in, bf16 out
(pda_paged_decode_attention_q8_bf16 through the C-ABI), as the reference's
quantized kernel runs on T = queries.dtype (metal_kernels.py:134-141,
196-206).

The reference's own check of that kernel (tests/test_mlx_engine.py:422-493)
draws bf16 queries, quantizes bf16 K/V to int8 with fp16 scales and compares
the kernel against float32 attention over ``int8 * scale`` with max-abs
< 2e-2. Here the oracle is that attention in float64 (oracle/paged_attention.py
over oracle/kv8.py's quantization, both pinned on the CPU), at the bf16 bar
of this build: max-abs 1.6e-2, mean-abs 1.6e-3 (the fp16 bar times bf16's
8x larger machine epsilon), on the reference's five kernel-test shapes
(head_dim 512, 256, 80, 4: the matrix-core, VALU and generic kernels),
config 2's head shape and an odd head dim (7), in both arena layouts. Two further checks:

* the bf16 call against the fp16 call (pda_paged_decode_attention_q8) on the
  same queries, which bf16 -> fp16 holds exactly at these magnitudes: the
  two share the arithmetic, so they differ only by the output rounding (at
  most one bf16 ulp plus one fp16 ulp, elementwise);
* queries far outside fp16's range (x 1e6) and far below its normal range
  (x 1e-7): the per-unit power-of-two scaling keeps them exact, where a
  plain cast to fp16 would overflow to inf or flush to zero.
"""

import numpy as np
import pytest
import torch

from instinct_amd import workloads
from instinct_amd.hip_kernels import paged_decode_attention
from oracle import kv8
from oracle import paged_attention as pa
from test_gpu_kv8 import Quantized

pytestmark = pytest.mark.gpu

MAX_ABS = 1.6e-2  # bf16: the fp16 bar x 8 (2^-7 / 2^-10)
MEAN_ABS = 1.6e-3


def run_bf16(qw, q_bf16, **kw):
    w = qw.w
    out = paged_decode_attention(q_bf16, qw.keys, qw.values, w.tables, w.lengths,
                                 page_size=w.page_size, longest=w.longest, scale=w.scale,
                                 window=w.window, softcap=w.softcap, scales=qw.scales, **kw)
    torch.cuda.synchronize()
    assert out.dtype == torch.bfloat16
    return out


def expected(qw, q64):
    w = qw.w
    return pa.paged_decode_dense(q64, kv8.dequantize(qw.kq, qw.ks), kv8.dequantize(qw.vq, qw.vs),
                                 qw.t, qw.n, page_size=w.page_size, scale=w.scale,
                                 window=w.window, softcap=w.softcap)


def check(got, want, what, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    got = got.float().cpu().numpy()
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    err_max, err_mean = pa.error_stats(got, want)
    print(f"{what}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}", flush=True)
    assert err_max <= max_abs and err_mean <= mean_abs, (what, err_max, err_mean)


SHAPES = [
    (16, 2, 512, [1, 700, 2049], 0, 0.0),
    (16, 8, 256, [5, 1500, 4000], 1024, 0.0),
    (16, 4, 256, [64, 3333], 0, 0.0),
    (8, 1, 80, [3, 300], 0, 30.0),
    (2, 1, 4, [9], 4, 0.0),
    (28, 4, 128, [3, 300, 4095, 8000], 0, 0.0),
    (8, 2, 7, [3, 300, 1000], 0, 0.0),  # an odd head dim
]


@pytest.mark.parametrize("layout", ["pages", "rows"])
@pytest.mark.parametrize("q_heads,kv_heads,head_dim,lengths,window,softcap", SHAPES)
def test_reference_kernel_test_shapes(gpu, layout, q_heads, kv_heads, head_dim, lengths, window,
                                      softcap):
    w = workloads.reference_test_case(q_heads, kv_heads, head_dim, lengths, window, softcap,
                                      device=gpu)
    qw = Quantized(w, layout)
    q_bf16 = w.q.float().bfloat16()
    q64 = q_bf16.float().cpu().numpy().astype(np.float64)
    got = run_bf16(qw, q_bf16)
    what = f"q8 bf16 {q_heads}/{kv_heads} D{head_dim} {layout}"
    check(got, expected(qw, q64), what)
    # The fp16 call on the same (exactly representable) queries: the same
    # arithmetic, so only the output rounding differs.
    w.q = q_bf16.half()
    ref16 = qw.run().float()
    diff = (got.float() - ref16).abs()
    ulp = torch.maximum(ref16.abs(), got.float().abs()) * (2.0 ** -8 + 2.0 ** -11) + 2.0 ** -24
    assert bool((diff <= ulp).all()), (what, float(diff.max()))
    # Bitwise repeatable (the default fixed split points).
    assert torch.equal(run_bf16(qw, q_bf16), got)


@pytest.mark.parametrize("factor", [1e6, 1e-7])
def test_queries_outside_the_fp16_range(gpu, factor):
    """Queries x 1e6 (past fp16's 65504) and x 1e-7 (below its 2^-14 normal
    range) with the scale divided by the same factor: the scores, and so the
    output, are those of the unscaled queries."""
    w = workloads.reference_test_case(16, 4, 256, [64, 3333], 0, 0.0, device=gpu)
    qw = Quantized(w, "pages")
    q_bf16 = (w.q.float() * factor).bfloat16()
    q64 = q_bf16.float().cpu().numpy().astype(np.float64)
    w.scale = w.scale / factor
    got = run_bf16(qw, q_bf16)
    check(got, expected(qw, q64), f"q8 bf16 queries x {factor:g}")


def test_config2_shape(gpu):
    """Config 2's head shape (28/4 heads, D = 128, the matrix-core kernel)
    over an 8-bit cache with bf16 queries, 16 sequences of 512-4096 tokens,
    against the float64 oracle."""
    w = workloads.config2(device=gpu, batch=16, low=512, high=4096)
    qw = Quantized(w, "pages")
    q_bf16 = w.q.float().bfloat16()
    q64 = q_bf16.float().cpu().numpy().astype(np.float64)
    check(run_bf16(qw, q_bf16), expected(qw, q64), "q8 bf16 config2 shape")


def test_split_and_merge_passes(gpu):
    w = workloads.config2(device=gpu, batch=16, low=512, high=4096)
    qw = Quantized(w, "pages")
    q_bf16 = w.q.float().bfloat16()
    whole = run_bf16(qw, q_bf16)
    out = torch.empty_like(q_bf16)
    run_bf16(qw, q_bf16, passes="split", out=out)
    run_bf16(qw, q_bf16, passes="merge", out=out)
    assert torch.equal(out, whole)
