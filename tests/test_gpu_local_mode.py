"""Local mode of the decode call: one split workgroup per unit, its waves'
pieces merged in LDS at the end, no merge kernel (the library picks it for
calls of few, short units, such as config 1 and config 4's windows).
PDA_DECODE_LOCAL=1 forces it wherever the pieces fit and =0 turns it off;
the library reads the variable once per process, so each setting runs in a
child process. Every case is checked against the float64 oracle at the
north star's bar (bf16: test_gpu_bf16.py's bar; 8-bit: attention over the
dequantized rows), and the fixed-split mode for bitwise reproducibility.
On the VALU kernels local mode gives each query head its own unit where the
CUs have room; those outputs must equal the GQA units' bit for bit."""

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
from instinct_amd.paged_kv import rows_to_pages
from oracle import kv8
from oracle import paged_attention as pa

want_local = sys.argv[1] == "1"
gpu = torch.device("cuda:0")
P = 16
bad = []


def case(hq, hkv, d, lengths, window=0, softcap=0.0, dtype=torch.float16, bits=16, seed=0,
         released=()):
    w = workloads.reference_test_case(hq, hkv, d, lengths, window, softcap, device=gpu,
                                      seed=seed)
    t = w.tables.cpu().numpy()
    for b, page in released:  # released pages inside the visible range: masked
        t[b, page] = -1
    w.tables = torch.as_tensor(t, device=gpu)
    names = decode_kernel_names(hq, hkv, d, bits=bits, bf16=dtype == torch.bfloat16,
                                batch=w.batch, longest=w.longest, page_size=P,
                                table_width=int(t.shape[1]), window=window)
    assert names["local"] == want_local, names
    q, k, v, tt, n = w.numpy()
    kw = dict(page_size=P, longest=w.longest, scale=w.scale, window=window, softcap=softcap)
    if bits == 8:
        kq, ks = kv8.quantize(k)
        vq, vs = kv8.quantize(v)
        want = pa.paged_decode_dense(q, kv8.dequantize(kq, ks), kv8.dequantize(vq, vs), tt, n,
                                     page_size=P, scale=w.scale, window=window, softcap=softcap)
        sp = lambda s: torch.as_tensor(s, device=gpu).view(-1, P, hkv).permute(0, 2, 1).contiguous()
        keys = rows_to_pages(torch.as_tensor(kq, device=gpu), P)
        values = rows_to_pages(torch.as_tensor(vq, device=gpu), P)
        call = lambda fixed: paged_decode_attention(w.q, keys, values, w.tables, w.lengths,
                                                    scales=(sp(ks), sp(vs)), deterministic=fixed, **kw)
        bar = (2e-3, 2e-4)
    else:
        w.q, w.keys, w.values = (x.to(dtype) for x in (w.q, w.keys, w.values))
        f = lambda x: x.float().cpu().numpy()
        want = pa.paged_decode_dense(f(w.q), f(w.keys), f(w.values), tt, n, page_size=P,
                                     scale=w.scale, window=window, softcap=softcap)
        w.to_layout("pages")
        call = lambda fixed: paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths,
                                                    deterministic=fixed, **kw)
        bar = (1.6e-2, 1.6e-3) if dtype == torch.bfloat16 else (2e-3, 2e-4)
    for fixed in (False, True):
        out = call(fixed)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        err_max, err_mean = pa.error_stats(got, want)
        ok = bool(np.isfinite(got).all()) and err_max <= bar[0] and err_mean <= bar[1]
        if fixed:
            again = [call(True) for _ in range(3)]
            torch.cuda.synchronize()
            ok = ok and all(torch.equal(a, out) for a in again)
        print(f"{names['split']} {hq}/{hkv}/D{d} bits {bits} {dtype} lengths {lengths} "
              f"window {window}{' fixed' if fixed else ''}: max_abs={err_max:.3e} "
              f"mean_abs={err_mean:.3e} {'ok' if ok else 'FAIL'}", flush=True)
        if not ok:
            bad.append(names["split"])


case(14, 2, 64, [1024] * 8)                                   # config 1's shape, matrix cores
case(14, 2, 64, [1, 2, 17, 0, 63, 300])                       # tiny units, an empty sequence
case(8, 4, 256, [4100, 5000, 9000], window=1024, seed=3)      # config 4's shape, VALU
case(28, 4, 128, [5, 600, 1000], softcap=30.0, seed=4)        # matrix cores, softcap
case(6, 2, 128, [700, 900], seed=5, released=((0, 3), (1, 10)))
case(12, 2, 96, [33, 257, 999], dtype=torch.bfloat16, seed=6)
case(8, 1, 80, [3, 300], bits=8, seed=7)                      # generic 8-bit
case(16, 2, 128, [40, 800, 1500], bits=8, seed=8)             # 8-bit matrix cores
case(4, 2, 130, [9, 700], seed=9)                             # generic head dim
case(2, 1, 4, [9], window=4, seed=10)                         # the reference's head_dim 4 case
sys.exit(1 if bad else 0)
"""


@pytest.mark.parametrize("mode", ["1", "0"])
def test_local_mode_against_the_oracle(gpu, mode):
    env = dict(os.environ, PDA_DECODE_LOCAL=mode,
               PYTHONPATH=os.pathsep.join([str(ROOT), str(ROOT / "llm-inference_amd"),
                                           os.environ.get("PYTHONPATH", "")]))
    r = subprocess.run([sys.executable, "-c", CHILD, mode], env=env, cwd=ROOT,
                       capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr[-3000:]


HEADS_CHILD = r"""
import hashlib
import torch
from instinct_amd import workloads
from instinct_amd.hip_kernels import decode_kernel_names, paged_decode_attention

gpu = torch.device("cuda:0")
for hq, hkv, d, lengths, window, dtype, seed in (
        (8, 4, 256, [4100, 5000, 9000], 1024, torch.float16, 3),   # config 4's shape
        (16, 4, 128, [300, 700, 1000], 0, torch.float16, 4),       # 4 heads per kv head
        (8, 2, 128, [50, 301], 0, torch.bfloat16, 5),
        (12, 6, 96, [33, 257, 999], 200, torch.float16, 6),
        (4, 2, 80, [9, 700], 0, torch.float16, 7)):                # generic head dim
    w = workloads.reference_test_case(hq, hkv, d, lengths, window, 0.0, device=gpu, seed=seed)
    w.q, w.keys, w.values = (x.to(dtype) for x in (w.q, w.keys, w.values))
    w.to_layout("pages")
    info = decode_kernel_names(hq, hkv, d, bf16=dtype == torch.bfloat16, batch=w.batch,
                               longest=w.longest, page_size=16,
                               table_width=int(w.tables.shape[1]), window=window)
    assert info["local"], info
    out = paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths, page_size=16,
                                 longest=w.longest, scale=w.scale, window=window)
    torch.cuda.synchronize()
    digest = hashlib.sha256(out.view(torch.int16).cpu().numpy().tobytes()).hexdigest()[:16]
    print(f"{hq}/{hkv}/D{d} {dtype} heads/unit {info['heads_per_unit']} {digest}", flush=True)
"""


def test_local_head_units_match_gqa_units(gpu):
    # Local mode on the VALU kernels takes a unit per query head where the
    # CUs have room (PDA_LOCAL_HEAD_UNITS=0 keeps the GQA units). Each head's
    # arithmetic does not depend on its unit, so both give the same bits.
    runs = {}
    for setting in ("", "0"):
        env = dict(os.environ, PDA_DECODE_LOCAL="1",
                   PYTHONPATH=os.pathsep.join([str(ROOT), str(ROOT / "llm-inference_amd"),
                                               os.environ.get("PYTHONPATH", "")]))
        env.pop("PDA_LOCAL_HEAD_UNITS", None)
        if setting:
            env["PDA_LOCAL_HEAD_UNITS"] = setting
        r = subprocess.run([sys.executable, "-c", HEADS_CHILD], env=env, cwd=ROOT,
                           capture_output=True, text=True, timeout=300)
        print(r.stdout)
        assert r.returncode == 0, r.stdout + r.stderr[-3000:]
        runs[setting] = [line.split() for line in r.stdout.strip().splitlines()]
    for heads, gqa in zip(runs[""], runs["0"]):
        assert heads[-1] == gqa[-1], (heads, gqa)          # the same output bits
        assert heads[-2] == "1" and gqa[-2] != "1", (heads, gqa)  # the policy took effect
