"""The VALU decode kernels of shapes that run on the matrix cores by default
(16-bit head dim 512 at every group, 8-bit 512 from 4 heads per kv head,
16-bit groups of 5 or more heads), selected with the library's measurement
knob PDA_MFMA_MIN_GROUP=99. The library reads the knob once per process, so
the check runs in a child process; it compares each call with the float64
oracle at the north star's bar (bf16: the bar of test_gpu_bf16.py; 8-bit:
attention over the dequantized rows) and prints one line per case."""

import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]

CHILD = r"""
import sys
import numpy as np
import torch
from instinct_amd import workloads
from instinct_amd.hip_kernels import decode_kernel_names, paged_decode_attention
from instinct_amd.paged_kv import pages_to_rows, rows_to_pages
from oracle import kv8
from oracle import paged_attention as pa

gpu = torch.device("cuda:0")
bad = []
for hq, hkv, d, lengths, dtype, bits in [
        (16, 2, 512, [1, 700, 2049, 5000], torch.float16, 16),
        (8, 1, 512, [33, 3000], torch.bfloat16, 16),
        (2, 1, 512, [9, 1500], torch.float16, 16),
        (16, 2, 512, [1, 700, 2049], torch.float16, 8),
        (8, 2, 512, [300, 4000], torch.float16, 8),
        (28, 4, 128, [5, 600, 3000], torch.float16, 16),
        (12, 2, 96, [40, 2500], torch.bfloat16, 16)]:
    names = decode_kernel_names(hq, hkv, d, bits=bits, bf16=dtype == torch.bfloat16)
    assert not names["matrix_cores"], names
    w = workloads.reference_test_case(hq, hkv, d, lengths, 0, 0.0, device=gpu)
    q, k, v, t, n = w.numpy()
    if bits == 8:
        kq, ks = kv8.quantize(k)
        vq, vs = kv8.quantize(v)
        want = pa.paged_decode_dense(q, kv8.dequantize(kq, ks), kv8.dequantize(vq, vs), t, n,
                                     page_size=16, scale=w.scale)
        P = 16
        sp = lambda s: torch.as_tensor(s, device=gpu).view(-1, P, hkv).permute(0, 2, 1).contiguous()
        out = paged_decode_attention(w.q, rows_to_pages(torch.as_tensor(kq, device=gpu), P),
                                     rows_to_pages(torch.as_tensor(vq, device=gpu), P), w.tables,
                                     w.lengths, page_size=P, longest=w.longest, scale=w.scale,
                                     scales=(sp(ks), sp(vs)))
        bar = (2e-3, 2e-4)
    else:
        w.q, w.keys, w.values = (x.to(dtype) for x in (w.q, w.keys, w.values))
        f = lambda x: x.float().cpu().numpy()
        want = pa.paged_decode_dense(f(w.q), f(w.keys), f(w.values), t, n, page_size=16,
                                     scale=w.scale)
        w.to_layout("pages")
        out = paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths, page_size=16,
                                     longest=w.longest, scale=w.scale)
        bar = (1.6e-2, 1.6e-3) if dtype == torch.bfloat16 else (2e-3, 2e-4)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    err_max, err_mean = pa.error_stats(got, want)
    ok = np.isfinite(got).all() and err_max <= bar[0] and err_mean <= bar[1]
    print(f"{names['split']} {hq}/{hkv}/D{d} bits {bits}: max_abs={err_max:.3e} "
          f"mean_abs={err_mean:.3e} {'ok' if ok else 'FAIL'}", flush=True)
    if not ok:
        bad.append(names["split"])
sys.exit(1 if bad else 0)
"""


def test_valu_kernels_of_matrix_core_shapes(gpu):
    env = dict(os.environ, PDA_MFMA_MIN_GROUP="99",
               PYTHONPATH=os.pathsep.join([str(ROOT), str(ROOT / "llm-inference_amd"),
                                           os.environ.get("PYTHONPATH", "")]))
    r = subprocess.run([sys.executable, "-c", CHILD], env=env, cwd=ROOT, capture_output=True,
                       text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr[-2000:]
