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
    head_dim 80 and 4 have no 8-bit kernel) plus config 1's and config 2's
    head shapes, with a softcap."""
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
