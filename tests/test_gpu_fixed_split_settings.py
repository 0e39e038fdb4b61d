"""Fixed split points at settings other than the defaults. The first wave of
each pair takes a share of the pair's range (Params::front256: halves at 16
bits, 142/256 at 8 bits) and may steer issue priority; the split kernel and
the merge kernel must agree on where every range is cut, whatever the share.
The library reads its measurement knobs (PDA_FIXED_SHARE, PDA_FIXED_BALANCE)
once per process, so each setting runs in a child process, which checks
against the float64 oracle at the north star's bar (bf16: the bar of
test_gpu_bf16.py; 8-bit: attention over the dequantized rows) on the
matrix-core, VALU, generic and odd-width kernels, 8-bit K/V, local mode and
both merge shapes (whole-row and row-sliced), that repeated calls are
bitwise equal, and that the separate split and merge passes give the bits of
the whole call."""

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
from oracle import paged_attention as pa
from test_gpu_kv8 import Quantized

gpu = torch.device("cuda:0")
bad = []
modes = set()


def call(w, keys, values, scales, **kw):
    out = paged_decode_attention(w.q, keys, values, w.tables, w.lengths, page_size=w.page_size,
                                 longest=w.longest, scale=w.scale, window=w.window,
                                 softcap=w.softcap, scales=scales, **kw)
    torch.cuda.synchronize()
    return out


def check(name, w, bits, dtype=torch.float16):
    info = decode_kernel_names(w.q_heads, w.kv_heads, w.head_dim, bits=bits,
                               bf16=dtype == torch.bfloat16, batch=w.batch, longest=w.longest,
                               page_size=w.page_size, table_width=int(w.tables.shape[1]),
                               window=w.window)
    mode = "local" if info["local"] else "sliced" if info["merge_row_sliced"] else "whole"
    modes.add(mode)
    if bits == 8:
        qw = Quantized(w, "pages")
        want = qw.expected()
        keys, values, scales = qw.keys, qw.values, qw.scales
        bar = (2e-3, 2e-4)
    else:
        _, _, _, t, n = w.numpy()
        w.q, w.keys, w.values = (x.to(dtype) for x in (w.q, w.keys, w.values))
        f = lambda x: x.float().cpu().numpy()
        want = pa.paged_decode_dense(f(w.q), f(w.keys), f(w.values), t, n, page_size=w.page_size,
                                     scale=w.scale, window=w.window, softcap=w.softcap)
        w.to_layout("pages")
        keys, values, scales = w.keys, w.values, None
        bar = (1.6e-2, 1.6e-3) if dtype == torch.bfloat16 else (2e-3, 2e-4)
    out = call(w, keys, values, scales)
    got = out.float().cpu().numpy()
    err_max, err_mean = pa.error_stats(got, want)
    ok = bool(np.isfinite(got).all()) and err_max <= bar[0] and err_mean <= bar[1]
    again = call(w, keys, values, scales)
    ok = ok and torch.equal(again, out)
    parts = torch.empty_like(out)
    call(w, keys, values, scales, passes="split", out=parts)
    call(w, keys, values, scales, passes="merge", out=parts)
    ok = ok and torch.equal(parts, out)
    print(f"{name} [{info['split']}, {mode}]: max_abs={err_max:.3e} mean_abs={err_mean:.3e} {'ok' if ok else 'FAIL'}",
          flush=True)
    if not ok:
        bad.append(name)


check("matrix cores 28/4 D128", workloads.config2(device=gpu, batch=16, low=512, high=4096), 16)
check("matrix cores 28/4 D128, 8-bit",
      workloads.config2(device=gpu, seed=3, batch=16, low=512, high=4096), 8)
check("matrix cores 28/4 D128, bf16",
      workloads.config2(device=gpu, seed=5, batch=8, low=100, high=3000), 16, torch.bfloat16)
check("VALU 32/8 D128", workloads.reference_test_case(32, 8, 128, [64, 3333, 9000], 0, 0.0,
                                                     device=gpu), 16)
check("VALU 16/8 D256, window", workloads.reference_test_case(16, 8, 256, [5, 1500, 4000], 1024,
                                                             0.0, device=gpu), 16)
check("generic 8/1 D80, softcap", workloads.reference_test_case(8, 1, 80, [3, 300, 2000], 0, 30.0,
                                                               device=gpu), 16)
check("8-bit 16/2 D512", workloads.reference_test_case(16, 2, 512, [1, 700, 2049], 0, 0.0,
                                                      device=gpu), 8)
check("local mode 8/4 D256, window", workloads.config4(device=gpu, batch=32), 16)
check("8-bit 8/4 D256, window", workloads.config4(device=gpu, seed=9, batch=32), 8)
check("odd 8/2 D7", workloads.reference_test_case(8, 2, 7, [3, 300, 1000], 0, 0.0, device=gpu), 16)
print("modes:", sorted(modes), flush=True)
sys.exit(1 if bad or modes != {"local", "sliced", "whole"} else 0)
"""


@pytest.mark.parametrize("share, balance", [("40", "1"), ("215", "0"), ("142", "1")])
def test_fixed_split_points_at_other_shares(gpu, share, balance):
    env = dict(os.environ, PDA_FIXED_SHARE=share, PDA_FIXED_BALANCE=balance,
               PYTHONPATH=os.pathsep.join([str(ROOT), str(ROOT / "llm-inference_amd"), str(ROOT / "tests"),
                                           os.environ.get("PYTHONPATH", "")]))
    r = subprocess.run([sys.executable, "-c", CHILD], env=env, cwd=ROOT, capture_output=True,
                       text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr[-2000:]
