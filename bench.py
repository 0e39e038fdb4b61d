"""Benchmark of split-K paged decode attention on one MI355X.

Workload (default): BASELINE config 2, the Qwen2.5-7B decode shape — batch 64,
28 query / 4 KV heads, head_dim 128, fp16 K/V in a paged arena (page 16),
context lengths U[512, 8192], randomly permuted pages. One step = one call of
the hot path (one layer's decode attention for the whole batch) with inputs
resident in HBM.

Timing: W warmup calls, then K timed calls, each bracketed by HIP events on
the stream the kernel runs on. Between timed calls a 1 GiB buffer is written
and another 1 GiB read, so the 256 MB Infinity Cache and the L2s hold none of
the arena and no dirty lines (flushed = HBM numbers); a second pass without
the flush is reported as "warm".
value = algorithmic K/V bytes / median call time (GB/s). The CPU baseline is
the oracle's threaded C++ float32 restatement of the reference's MLX CPU
(portable) decode path, gather then dense attention, timed on a bounded
sample of the same workload on this host's cores; the restatement of the
reference's split-K algorithm is timed beside it as a second record.
Also reported: the step before the call, RoPE of the new queries and keys
plus the K/V append into the arena (one launch, "append"), and one layer's
decode attention step (append then call, "layer_step_us"), both flushed, and
the prefill attention of one prompt chunk ("prefill", matrix-core bound).

Prints ONE JSON line. Only --gpus 1 is supported (a one-GPU build).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "llm-inference_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 matrix cores, published
METRIC = "decode-attention effective K/V GB/s (% of HBM peak) + µs/layer-step"
TRAFFIC_FILE = ROOT / "profiles" / "decode_traffic.json"
SPIN_CYCLES = 2_000_000  # torch.cuda._sleep before each timed call


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=2, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--batch", type=int, default=0,
                    help="config 3: sequences (1, 2 or 4; default 1)")
    ap.add_argument("--context", type=int, default=0,
                    help="config 3: tokens per sequence (32768 or 131072; default 32768)")
    ap.add_argument("--group", type=int, default=0,
                    help="query heads per kv head (0 = the config's): the config's lengths, "
                         "tables and K/V with a larger or smaller GQA group, for the "
                         "matrix-core vs VALU study")
    ap.add_argument("--split-pages", type=int, default=0)
    ap.add_argument("--deterministic", action="store_true", default=True,
                    help="fixed split points (the library's default, flags 0): bitwise "
                         "reproducible output")
    ap.add_argument("--racing", dest="deterministic", action="store_false",
                    help="racing wave pairs instead of fixed split points: the two waves of "
                         "a pair meet wherever their shared counter runs out (output bits may "
                         "differ between calls)")
    ap.add_argument("--latency-configs", default="1,3,4,5",
                    help="other configs timed in the same run, comma-separated ('' = none): "
                         "GPU call time (flushed) beside the CPU baseline on the same "
                         "workload; BASELINE pairs config 1 with the CPU path (config 3: "
                         "its B=1 x 32768 point)")
    ap.add_argument("--layout", choices=["pages", "rows"], default="pages",
                    help="K/V arena layout: page tiles (MI355X) or the reference's rows")
    ap.add_argument("--step-layers", type=int, default=28,
                    help="layers of the whole-step timing (0 = skip): append + attention "
                         "per layer, eager and as one captured HIP graph")
    ap.add_argument("--kv-bits", type=int, choices=[16, 8], default=16,
                    help="K/V storage: fp16, or int8 with a scale per (row, kv head)")
    ap.add_argument("--dtype", choices=["f16", "bf16"], default="f16",
                    help="model dtype of queries, K/V and outputs at 16 bits (bf16: the "
                         "reference's bf16 models)")
    ap.add_argument("--prefill", default="4096@0,512@32256",
                    help="prefill chunks to time, TOKENS@START comma-separated ('' = skip): "
                         "one sequence at the workload's heads, causal; the reference prefills "
                         "512-token chunks (mlx_engine.py:74)")
    ap.add_argument("--prefill-wide", default="4096@0,4096@28672,4096@258048",
                    help="prefill chunks at 512-wide heads, TOKENS@START ('' = skip): the "
                         "global layers of the reference's Gemma 4 (gemma4.py:49-66), whose "
                         "4096-token chunks at 256K context the reference names as its "
                         "prefill bottleneck (docs/benchmarks.md:102-105, roadmap.md:36)")
    ap.add_argument("--wide-heads", default="16/2",
                    help="query/kv heads of the 512-wide legs (a representative shape)")
    ap.add_argument("--published", default="261840",
                    help="context length of the reference's published decode workload, "
                         "timed in the same run ('' = skip): a Gemma 4 global layer, 2 x "
                         "512-wide bf16 KV heads, one sequence (docs/benchmarks.md:102-110)")
    ap.add_argument("--no-flush", action="store_true", help="skip the flushed pass")
    ap.add_argument("--flushed-only", action="store_true",
                    help="every decode launch follows a cache flush (warmups included, no warm "
                         "pass): for kernel traces whose averages match the flushed timings")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="approximate CPU time budget of the CPU-baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip every CPU-baseline timing")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (rocprof counter scale)")
    return ap.parse_args()


def kernel_label(names):
    """The split kernel and the merge kernel of a call (local mode: merged in
    the split kernel's workgroups, no merge kernel)."""
    if names["merge"] is None:
        return f"{names['split']} (local: one workgroup per unit, merged in LDS)"
    return f"{names['split']} + {names['merge']}"


def merge_shape_of(w):
    """What the merge launch depends on besides the heads (row slicing)."""
    return dict(batch=w.batch, longest=w.longest, page_size=w.page_size,
                table_width=int(w.tables.shape[1]), window=w.window)


def time_calls(passes, steps, flush=None):
    """K timed steps. Each step runs the callables in `passes` back to back on
    the kernels' stream, with a HIP event before the first and after each
    one. Returns per-pass durations (ms, list per pass) and the loop's wall
    time."""
    import torch

    stream = torch.cuda.current_stream()
    n = len(passes)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(n + 1)] for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        if flush is not None:
            flush()
        # A bounded spin keeps the queue busy while the host enqueues the
        # events and the call, so no host time falls between the events.
        torch.cuda._sleep(SPIN_CYCLES)
        ev[i][0].record(stream)
        for j, fn in enumerate(passes):
            fn()
            ev[i][j + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_pass = [[e[j].elapsed_time(e[j + 1]) for e in ev] for j in range(n)]
    return per_pass, wall


def append_inputs(w):
    """This step's new queries, keys and values for every sequence of the
    workload, at position length - 1, and the arena rows they go to
    (table[pos // P] * P + pos % P, batches.py:175-178)."""
    import torch

    dev = w.q.device
    gen = torch.Generator(device=dev).manual_seed(7)
    q = torch.randn(w.q.shape, generator=gen, device=dev).to(w.q.dtype)
    k = torch.randn((w.batch, w.kv_heads, w.head_dim), generator=gen, device=dev).to(w.q.dtype)
    v = torch.randn((w.batch, w.kv_heads, w.head_dim), generator=gen, device=dev).to(w.q.dtype)
    positions = (w.lengths - 1).clamp(min=0).to(torch.int32)
    pages = w.tables.long().gather(1, (positions.long() // w.page_size)[:, None])[:, 0]
    rows = (pages * w.page_size + positions.long() % w.page_size).to(torch.int32)
    q_out = torch.empty_like(q)
    bytes_moved = 2 * q.numel() * 2 + 2 * (k.numel() + v.numel()) * 2
    return q, k, v, positions, rows, q_out, bytes_moved


def decode_step(w, scales, layers, steps):
    """One decode step's attention work for `layers` layers of this workload:
    table packing on the device, then per layer the RoPE + K/V append and the
    decode call, run eagerly (launched from Python) and replayed as one
    captured HIP graph. The layers cycle over four copies of the arena (2.4
    GB of K/V at config 2), so a layer's K/V are not in the caches."""
    import torch

    from instinct_amd.step import DecodeStepGraph

    copies = 4
    arenas = []
    for i in range(min(copies, layers)):
        extra = tuple(x.clone() for x in scales) if scales is not None else ()
        arenas.append((w.keys.clone(), w.values.clone()) + extra)
    per_layer = [arenas[i % len(arenas)] for i in range(layers)]
    step = DecodeStepGraph(per_layer, w.tables, batch=w.batch, q_heads=w.q_heads,
                           page_size=w.page_size, width=int(w.tables.shape[1]), scale=w.scale,
                           longest=w.longest, dims=w.head_dim, base=1e6, window=w.window,
                           softcap=w.softcap)
    step.slots.copy_(torch.arange(w.batch, dtype=torch.int32, device=w.q.device))
    step.positions.copy_((w.lengths - 1).clamp(min=0))
    gen = torch.Generator(device=w.q.device).manual_seed(3)
    for i in range(layers):
        step.q[i].copy_(torch.randn(step.q[i].shape, generator=gen, device=w.q.device))
        step.k[i].copy_(torch.randn(step.k[i].shape, generator=gen, device=w.q.device))
        step.v[i].copy_(torch.randn(step.v[i].shape, generator=gen, device=w.q.device))
    step.capture()

    def timed(fn, n):
        times = []
        for _ in range(n):
            torch.cuda._sleep(SPIN_CYCLES)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1) * 1e3)
        return statistics.median(times)

    def back_to_back(fn, n):
        """n steps issued one after another with no spin in front: the GPU
        time per step, or the host's launch time where that is longer."""
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e6 / n
        return e0.elapsed_time(e1) * 1e3 / n, wall

    n = max(5, min(steps, 20))
    eager = timed(step.run, n)
    graph = timed(step.replay, n)
    b2b_eager, wall_eager = back_to_back(step.run, n)
    b2b_graph, wall_graph = back_to_back(step.replay, n)
    del step, arenas, per_layer
    torch.cuda.empty_cache()
    return {"layers": layers, "launches_per_step": 1 + 3 * layers,
            "eager_us": round(eager, 1), "graph_us": round(graph, 1),
            "graph_us_per_layer": round(graph / layers, 2),
            "back_to_back": {
                "note": f"{n} steps issued back to back, no spin: per-step time between events "
                        "and per-step host wall time",
                "eager_us": round(b2b_eager, 1), "graph_us": round(b2b_graph, 1),
                "eager_wall_us": round(wall_eager, 1), "graph_wall_us": round(wall_graph, 1)}}


def blas_threads() -> int:
    """Threads numpy's OpenBLAS runs with (its environment variables, else
    the host's cores)."""
    for name in ("OPENBLAS_NUM_THREADS", "OMP_NUM_THREADS"):
        if os.environ.get(name, "").isdigit():
            return int(os.environ[name])
    return os.cpu_count() or 1


def prefill_cpu_baseline(w, tokens, start, budget_s):
    """The oracle's dense prefill attention in float32 (the portable path's
    arithmetic, portable.py:173-188) on the chunk's last queries (the ones
    with the most keys), the sample doubled until one call takes a third of
    budget_s; FLOP/s on the same count as the GPU leg. Each call gathers the
    whole visible prefix (as the portable path does once per chunk), so a
    small sample understates the CPU's rate on a whole chunk."""
    import numpy as np

    from oracle import paged_attention as pa

    P, hq, hkv, d = w.page_size, w.q_heads, w.kv_heads, w.head_dim
    end = start + tokens
    pages = (end + P - 1) // P
    rng = np.random.default_rng(5)
    keys = rng.standard_normal((pages * P, hkv, d)).astype(np.float16)
    values = rng.standard_normal((pages * P, hkv, d)).astype(np.float16)
    table = rng.permutation(pages)
    sample, took = 8, 0.0
    while True:
        n = min(sample, tokens)
        q = rng.standard_normal((n, hq, d)).astype(np.float16)
        t0 = time.perf_counter()
        pa.paged_prefill_dense(q, keys, values, table, start=end - n, page_size=P,
                               scale=w.scale, window=w.window, softcap=w.softcap,
                               dtype=np.float32)
        took = time.perf_counter() - t0
        if took >= budget_s / 3 or n == tokens:
            break
        sample *= 2
    pos = np.arange(end - n, end, dtype=np.float64)
    seen = pos + 1 if w.window <= 0 else np.minimum(pos + 1, w.window)
    flops = 4.0 * d * hq * seen.sum()
    return {"value": round(float(flops / took / 1e12), 5), "unit": "TFLOP/s",
            "cores": blas_threads(), "kind": "port",
            "sample": (f"last {n} of the {tokens} queries ({flops / 1e9:.1f} GFLOP, "
                       f"{took:.2f} s, the gather of {end} key rows included): oracle "
                       "paged_prefill_dense in float32, NumPy/OpenBLAS, restating "
                       "PrefillBatch.attend (batches.py:84-132)")}


def append_cpu_baseline(w, budget_s):
    """The oracle's RoPE + K/V write (oracle/rope_append.py, restating
    portable.py:115-132 and paged_kv.py:278-283) on the same 64-token step,
    repeated for ~budget_s; GB/s on the same byte count as the GPU leg."""
    import numpy as np

    from oracle import rope_append as ra

    rng = np.random.default_rng(6)
    n, hq, hkv, d, P = w.batch, w.q_heads, w.kv_heads, w.head_dim, w.page_size
    q = rng.standard_normal((n, hq, d)).astype(np.float16)
    k = rng.standard_normal((n, hkv, d)).astype(np.float16)
    v = rng.standard_normal((n, hkv, d)).astype(np.float16)
    pages = n
    k_arena = np.zeros((pages, hkv, P, d), np.float16)
    v_arena = np.zeros_like(k_arena)
    positions = rng.integers(0, 8192, n)
    rows = rng.permutation(pages * P)[:n]
    inverse = ra.inv_freq(d, base=1e6)
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or reps < 3:
        ra.rope_append(q, k, v, k_arena, v_arena, positions, rows, dims=d, inverse=inverse,
                       layout="pages", page_size=P)
        reps += 1
    took = (time.perf_counter() - t0) / reps
    nbytes = 2 * q.size * 2 + 2 * (k.size + v.size) * 2
    return {"value": round(nbytes / took / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": (f"the {n}-token step x {reps} calls ({took * 1e6:.0f} us each): oracle "
                       "rope_append in NumPy (its arena copies included)")}


def prefill_leg(w, tokens, steps, start=0):
    """One prompt chunk of `tokens` tokens at positions start.. of one
    sequence, at the workload's heads and page size, through
    pda_paged_prefill_attention (PrefillBatch.attend's attention,
    batches.py:84-132). Algorithmic work: query p sees n_p = p + 1 keys (or
    the window), 4 D n_p flops per query head (QK^T and PV, a multiply-add =
    2 flops); roofline = fp16 dense matrix-core peak."""
    import numpy as np
    import torch

    from instinct_amd.hip_kernels import paged_prefill_attention
    from instinct_amd.paged_kv import rows_to_pages

    dev = w.q.device
    P, hq, hkv, d = w.page_size, w.q_heads, w.kv_heads, w.head_dim
    pages = (start + tokens + P - 1) // P
    gen = torch.Generator(device=dev).manual_seed(11)
    dtype = w.q.dtype
    keys = torch.randn((pages * P, hkv, d), generator=gen, device=dev).to(dtype)
    values = torch.randn((pages * P, hkv, d), generator=gen, device=dev).to(dtype)
    if w.layout == "pages":
        keys, values = rows_to_pages(keys, P), rows_to_pages(values, P)
    table = torch.as_tensor(np.random.default_rng(11).permutation(pages).astype(np.int32),
                            device=dev)
    q = torch.randn((tokens, hq, d), generator=gen, device=dev).to(dtype)
    out = torch.empty_like(q)

    def call():
        paged_prefill_attention(q, keys, values, table, start=start, page_size=P,
                                scale=w.scale, window=w.window, softcap=w.softcap, out=out)

    for _ in range(3):
        call()
    (ms,), _ = time_calls([call], max(5, min(steps, 20)))
    from instinct_amd import _lib
    splits, _ = _lib.prefill_workspace_bytes(start, tokens, hq, d, w.window)
    pos = np.arange(start, start + tokens, dtype=np.float64)
    seen = pos + 1 if w.window <= 0 else np.minimum(pos + 1, w.window)
    flops = 4.0 * d * hq * seen.sum()
    med = statistics.median(ms)
    tflops = flops / (med * 1e-3) / 1e12
    bf16 = dtype == torch.bfloat16
    width = next(x for x in (64, 96, 128, 256, 512) if d <= x)  # the kernel that serves d
    return {"kernel": f"paged_prefill_kernel<{width},false,{str(bf16).lower()},"
                      f"{str(width != d).lower()}> "
                      f"(pda_paged_prefill_attention{'_bf16' if bf16 else ''})",
            "tokens": tokens, "start": start, "key_ranges": splits, "q_heads": hq,
            "kv_heads": hkv, "head_dim": d,
            "us_median": round(med * 1e3, 2), "flops": flops,
            "TFLOP_per_s": round(tflops, 2), "peak_TFLOP_per_s": MFMA_F16_PEAK_TFLOPS,
            "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
            "tokens_per_s": round(tokens / (med * 1e-3), 1)}


def config_leg(cfg, args, flush):
    """Another BASELINE config in the same run: the whole call (split and
    merge) timed with HIP events around it, caches flushed between calls,
    and the same CPU baseline as the headline leg on that workload."""
    import torch

    from instinct_amd import workloads
    from instinct_amd.hip_kernels import decode_kernel_names, paged_decode_attention

    device = torch.device("cuda:0")
    w = workloads.CONFIGS[cfg](device=device).to_layout(args.layout)
    out = torch.empty_like(w.q)

    def call():
        paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths,
                               page_size=w.page_size, longest=w.longest, scale=w.scale,
                               window=w.window, softcap=w.softcap, out=out,
                               deterministic=args.deterministic)

    for _ in range(args.warmup):
        call()
    (ms,), _ = time_calls([call], args.steps, flush)
    med = statistics.median(ms)
    kv_bytes = w.kv_bytes()
    names = decode_kernel_names(w.q_heads, w.kv_heads, w.head_dim, **merge_shape_of(w))
    leg = {"workload": w.name, "batch": w.batch, "q_heads": w.q_heads,
           "kv_heads": w.kv_heads, "head_dim": w.head_dim, "kv_bytes": kv_bytes,
           "kernel": kernel_label(names),
           "us_median": round(med * 1e3, 2), "us_mean": round(statistics.fmean(ms) * 1e3, 2),
           "GB_per_s": round(kv_bytes / (med * 1e-3) / 1e9, 2),
           "pct_hbm_peak": round(100 * kv_bytes / (med * 1e-3) / 1e9 / HBM_PEAK_GBS, 2)}
    if w.meta.get("sharers") is not None:
        leg["unique_kv_bytes"] = w.unique_kv_bytes()
    if not args.no_cpu:
        leg["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds / 2)
    del w, out
    torch.cuda.empty_cache()
    return leg


def published_leg(args, flush):
    """The reference's one published decode-kernel figure, re-measured here on
    its own workload: a Gemma 4 global layer (two 512-wide KV heads, bf16)
    with one sequence at 261,840 tokens. The reference reports ~6.7 ms per
    layer and "about 320 GB/s" of K/V on an Apple M3 Max (MLX 0.32.2, Metal;
    docs/benchmarks.md:102-110); K+V of that layer is 1.07 GB, so 6.7 ms is
    160 GB/s by this file's accounting. The time ratio is the comparable
    figure. Caches flushed between calls (the arena is 4x the last-level
    cache anyway)."""
    import torch

    from instinct_amd import workloads
    from instinct_amd.hip_kernels import decode_kernel_names, paged_decode_attention

    hq, _ = (int(x) for x in args.wide_heads.split("/"))
    w = workloads.gemma4_global(device=torch.device("cuda:0"), length=int(args.published),
                                q_heads=hq).to_layout(args.layout)
    out = torch.empty_like(w.q)

    def call():
        paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths,
                               page_size=w.page_size, longest=w.longest, scale=w.scale,
                               out=out, deterministic=args.deterministic)

    for _ in range(args.warmup):
        call()
    (ms,), _ = time_calls([call], args.steps, flush)
    med = statistics.median(ms)
    kv_bytes = w.kv_bytes()
    names = decode_kernel_names(w.q_heads, w.kv_heads, w.head_dim, bf16=True,
                                **merge_shape_of(w))
    rate = kv_bytes / (med * 1e-3) / 1e9
    leg = {"workload": w.name, "dtype": "bf16", "batch": w.batch, "q_heads": w.q_heads,
           "kv_heads": w.kv_heads, "head_dim": w.head_dim, "context": int(args.published),
           "kv_bytes": kv_bytes, "kernel": kernel_label(names),
           "us_median": round(med * 1e3, 2), "us_mean": round(statistics.fmean(ms) * 1e3, 2),
           "GB_per_s": round(rate, 2), "pct_hbm_peak": round(100 * rate / HBM_PEAK_GBS, 2)}
    # The same layer with the 8-bit cache (KVCache(bits=8): int8 rows, an
    # fp16 scale per row and kv head), queries in fp16.
    def quantize(x):
        s8 = (x.float().abs().amax(-1).clamp(min=1e-4) / 127.0).half()
        return (x.float() / s8.float()[..., None]).round().clamp(-127, 127).to(torch.int8), s8

    (keys8, kscale), (values8, vscale) = quantize(w.keys), quantize(w.values)
    q16 = w.q.half()
    out16 = torch.empty_like(q16)

    def call8():
        paged_decode_attention(q16, keys8, values8, w.tables, w.lengths,
                               page_size=w.page_size, longest=w.longest, scale=w.scale,
                               out=out16, scales=(kscale, vscale),
                               deterministic=args.deterministic)

    for _ in range(args.warmup):
        call8()
    (ms8,), _ = time_calls([call8], args.steps, flush)
    med8 = statistics.median(ms8)
    bytes8 = int(w.spans().sum()) * w.kv_heads * (w.head_dim + 2) * 2
    names8 = decode_kernel_names(w.q_heads, w.kv_heads, w.head_dim, bits=8,
                                 **merge_shape_of(w))
    leg["kv8"] = {"kernel": kernel_label(names8),
                  "us_median": round(med8 * 1e3, 2), "kv_bytes": bytes8,
                  "GB_per_s": round(bytes8 / (med8 * 1e-3) / 1e9, 2)}
    del keys8, values8, kscale, vscale
    if not args.no_cpu:
        # The CPU restatement takes fp16 rows: the same layer rounded to fp16.
        import dataclasses

        w16 = dataclasses.replace(w, q=w.q.half(), keys=w.keys.half(), values=w.values.half())
        leg["cpu_baseline"] = cpu_baseline(w16, args.cpu_seconds / 2)
        del w16
    if int(args.published) == 261840:
        leg["reference_published"] = {
            "ms_per_layer": 6.7, "GB_per_s_as_published": 320,
            "GB_per_s_same_accounting": round(kv_bytes / 6.7e-3 / 1e9, 1),
            "hardware": "Apple M3 Max (128 GB), MLX 0.32.2, Metal",
            "source": "docs/benchmarks.md:102-110"}
        leg["time_ratio_vs_published"] = round(6.7 / med, 1)
    del w, out
    torch.cuda.empty_cache()
    return leg


def cpu_model() -> str:
    """The host CPU's model name (Linux), for the CPU-baseline records."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(w, budget_s, splitk=False):
    """A CPU restatement of the reference's decode path on a sample of
    sequences of the same workload, all host cores; returns the dict for the
    JSON line. Default: the path BASELINE.json names, the reference's MLX CPU
    (portable) decode: gather the visible rows, then dense attention in
    float32 (portable.py:155-205, batches.py:228-246), C++ over std::thread.
    `splitk`: the C++ float32 restatement of the Metal split-K kernel
    (metal_kernels.py:18-124), a second record."""
    import numpy as np

    from oracle import cpu_oracle

    cores = cpu_oracle.host_cores()
    q, k, v, t, n = w.numpy()
    spans = w.spans()
    per_seq = spans * w.kv_heads * w.head_dim * 4  # K+V bytes per sequence
    fn = cpu_oracle.decode_splitk if splitk else cpu_oracle.decode_f32
    # Calibrate on one sequence, then size the sample to the budget.
    def run(idx):
        t0 = time.perf_counter()
        fn(q[idx], k, v, t[idx], n[idx], page_size=w.page_size, scale=w.scale,
           window=w.window, softcap=w.softcap, threads=cores)
        return time.perf_counter() - t0

    first = np.arange(min(4, w.batch))
    dt = run(first)
    rate = per_seq[first].sum() / max(dt, 1e-9)
    target_bytes = rate * max(budget_s, 0.5) / 2
    count = int(np.searchsorted(np.cumsum(per_seq), target_bytes)) + 1
    count = max(1, min(w.batch, count))
    idx = np.arange(count)
    reps, total_t, total_b = 0, 0.0, 0
    while total_t < budget_s / 2 or reps < 1:
        total_t += run(idx)
        total_b += int(per_seq[idx].sum())
        reps += 1
    what = ("C++ float32 restatement of the reference split-K kernel "
            "(metal_kernels.py:18-124), std::thread over (sequence, kv head, split)" if splitk else
            "C++ float32 restatement of the reference's MLX CPU (portable) decode path: gather "
            "the visible rows, then dense float32 attention (portable.py:155-205, "
            "batches.py:228-246), std::thread over (sequence, kv head)")
    return {
        "value": round(total_b / total_t / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"first {count} of {w.batch} sequences of {w.name} "
                   f"({int(per_seq[idx].sum())} K/V bytes) x {reps} calls; {what}"),
        "cpu_model": cpu_model(),
        "seconds": round(total_t, 2),
    }


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (--gpus 1); "
              "multi-GPU sharding is a design note, not a measured path.", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        # A plain copy of known size: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on
        # this run gives the factor between counter readings and bytes moved.
        n = args.copy_calibration << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(max(1, args.steps)):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n, "launches": max(1, args.steps)}))
        return

    from instinct_amd import _lib, workloads
    from instinct_amd.hip_kernels import decode_kernel_names, paged_decode_attention

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    bf16 = args.dtype == "bf16"
    if bf16 and args.kv_bits == 8:
        print("bench.py: the 8-bit cache takes fp16 queries (--dtype f16)", file=sys.stderr)
        sys.exit(2)
    cfg_kw = {}
    if args.config == 3:
        cfg_kw = dict(batch=args.batch or 1, length=args.context or 32768)
    elif args.batch or args.context:
        print("bench.py: --batch/--context choose among config 3's points", file=sys.stderr)
        sys.exit(2)
    w = workloads.CONFIGS[args.config](device=device, **cfg_kw).to_layout(args.layout)
    if args.group:
        # Same lengths, tables and K/V; G query heads per kv head.
        gen = torch.Generator(device=device).manual_seed(100 + args.group)
        w.q = torch.randn((w.batch, args.group * w.kv_heads, w.head_dim), generator=gen,
                          device=device).to(w.q.dtype)
        w.name += f"-g{args.group}"
    if bf16:
        # The same seeded values rounded to bf16: a bf16 model's cache.
        w.q, w.keys, w.values = w.q.bfloat16(), w.keys.bfloat16(), w.values.bfloat16()
        torch.cuda.empty_cache()
    kv_bytes = w.kv_bytes()
    fp16_bytes = kv_bytes
    scales = None
    if args.kv_bits == 8:
        # The same rows quantized as KVCache(bits=8) stores them (absmax / 127
        # per row and kv head); the bytes read are int8 rows plus fp16 scales.
        scales = []
        for name in ("keys", "values"):
            x = getattr(w, name)
            s8 = (x.abs().amax(-1).float().clamp(min=1e-4) / 127.0).half()
            q8 = (x.float() / s8.float()[..., None]).round().clamp(-127, 127).to(torch.int8)
            setattr(w, name, q8)
            scales.append(s8)
            del x
        scales = tuple(scales)
        kv_bytes = int(w.spans().sum()) * w.kv_heads * (w.head_dim + 2) * 2
        torch.cuda.empty_cache()
    out = torch.empty_like(w.q)

    def call(passes="both"):
        paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths,
                               page_size=w.page_size, longest=w.longest, scale=w.scale,
                               window=w.window, softcap=w.softcap,
                               split_pages=args.split_pages, out=out, passes=passes,
                               scales=scales, deterministic=args.deterministic)

    def split():
        call("split")

    def merge():
        call("merge")

    flush_buf = torch.empty(1 << 30, dtype=torch.uint8, device=device)
    read_buf = torch.ones(1 << 28, dtype=torch.float32, device=device)

    def flush():
        # Write 1 GiB, then read 1 GiB: the caches end up holding clean lines
        # of neither the arena nor the write (whose write-back would otherwise
        # land inside the timed region).
        flush_buf.fill_(1)
        read_buf.sum()

    for _ in range(args.warmup):
        if args.flushed_only:
            flush()
        call()
    torch.cuda.synchronize()

    # The metric and the roofline: whole calls (split + merge, one C-ABI
    # call), HIP events on the kernels' stream. A second loop issues the two
    # passes separately (an event between them) to show where the time goes.
    flushing = None if args.no_flush else flush
    (call_ms,), wall = time_calls([call], args.steps, flushing)
    (split_ms, merge_ms), _ = time_calls([split, merge], args.steps, flushing)
    call_w = None if args.flushed_only else time_calls([call], args.steps)[0][0]
    ms = call_ms
    med = statistics.median(ms)
    value = kv_bytes / (med * 1e-3) / 1e9
    call_mean = statistics.fmean(ms)
    split_mean = statistics.fmean(split_ms)
    achieved = kv_bytes / (call_mean * 1e-3) / 1e9
    waves, _ = _lib.plan(w.batch, w.q_heads, w.kv_heads, w.head_dim, w.page_size,
                         int(w.tables.shape[1]), w.longest, w.window, args.split_pages)
    names = decode_kernel_names(w.q_heads, w.kv_heads, w.head_dim, bits=args.kv_bits,
                                bf16=bf16, split_pages=args.split_pages, **merge_shape_of(w))
    traffic_key = f"{w.name}/{w.layout}/{'bf16' if bf16 else 'f16'}/kv{args.kv_bits}"
    if not args.deterministic:
        traffic_key += "/racing"
    traffic = None
    if TRAFFIC_FILE.exists():
        traffic = json.loads(TRAFFIC_FILE.read_text()).get(traffic_key, {}).get(
            "hbm_bytes_per_call")
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(med, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("bf16" if bf16 else "f16") if args.kv_bits == 16 else "i8 K/V, f16 math",
        "matrix_cores": names["matrix_cores"],
        "data": "synthetic (seeded N(0,1) K/V/Q, random page permutation)",
        "config": {
            "workload": w.name,
            "batch": w.batch, "q_heads": w.q_heads, "kv_heads": w.kv_heads,
            "head_dim": w.head_dim, "page_size": w.page_size, "window": w.window,
            "layout": w.layout, "kv_bits": args.kv_bits,
            "longest": w.longest, "kv_bytes": kv_bytes,
            "split_pages": args.split_pages, "stream_waves_max": waves,
            "fixed_split": args.deterministic,
            "cache": "warm (no flush)" if args.no_flush else "flushed (1 GiB write + 1 GiB read between calls)",
        },
        "us_per_layer_step": round(med * 1e3, 2),
        "steps_per_s": round(1e3 / med, 1),
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "warm": None if args.flushed_only else {
            "us_median": round(statistics.median(call_w) * 1e3, 2),
            "GB_per_s": round(kv_bytes / (statistics.median(call_w) * 1e-3) / 1e9, 2)},
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": f"{TRAFFIC_FILE.relative_to(ROOT)}[{traffic_key}]",
            "kernel": kernel_label(names) + " (one call, events around it)",
            "us_mean": round(call_mean * 1e3, 2),
            "split_us_mean": round(split_mean * 1e3, 2),
            "merge_us_mean": round(statistics.fmean(merge_ms) * 1e3, 2),
            "head_groups_per_kv_head": names["head_groups_per_kv_head"],
        },
    }
    if w.meta.get("sharers") is not None:
        line["config"]["unique_kv_bytes"] = w.unique_kv_bytes()
    if args.kv_bits == 8:
        # Keys per second in fp16 terms: the fp16 bytes of the same rows / time.
        line["fp16_equivalent_GB_per_s"] = round(fp16_bytes / (med * 1e-3) / 1e9, 2)
    line["wall_s_timed_loop"] = round(wall, 3)
    # The CPU baselines time the fp16 oracle; a bf16 run has none.
    if not args.no_cpu and args.kv_bits == 16 and not bf16:
        line["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
        line["cpu_baseline_splitk"] = cpu_baseline(w, args.cpu_seconds / 2, splitk=True)
    others = [int(c) for c in args.latency_configs.split(",") if c.strip()]
    if args.kv_bits == 16 and not bf16:
        line["other_configs"] = {str(c): config_leg(c, args, flushing)
                                 for c in others if c != args.config}
    if args.published and args.kv_bits == 16:
        line["published_workload"] = published_leg(args, flushing)

    # The step before the attention call: RoPE of the new queries and keys and
    # the K/V append (one launch), timed alone and followed by the call (one
    # layer's decode attention step). Runs last: it writes into the arena.
    from instinct_amd.hip_kernels import rope_append

    aq, ak, av, apos, arows, aq_out, abytes = append_inputs(w)

    def append():
        rope_append(aq, ak, av, w.keys, w.values, apos, arows, page_size=w.page_size,
                    dims=w.head_dim, base=1e6, q_out=aq_out, scales=scales)

    def append_and_call():
        append()
        call()

    for _ in range(args.warmup):
        append_and_call()
    (app_ms,), _ = time_calls([append], args.steps, flushing)
    (step_ms,), _ = time_calls([append_and_call], args.steps, flushing)
    app_med = statistics.median(app_ms)
    line["append"] = {
        "kernel": (f"rope_append_kernel<{'bf16' if bf16 else 'f16'}> (pda_rope_append"
                   f"{'_bf16' if bf16 else ''}: RoPE of q and k, K/V write)"
                   if args.kv_bits == 16 else
                   "rope_append_q8_kernel (pda_rope_append_q8: RoPE, quantized K/V write)"),
        "tokens": w.batch,
        "us_median": round(app_med * 1e3, 2),
        "bytes": abytes,
        "GB_per_s": round(abytes / (app_med * 1e-3) / 1e9, 2),
    }
    if not args.no_cpu and args.kv_bits == 16 and not bf16:
        line["append"]["cpu_baseline"] = append_cpu_baseline(w, 2.0)
    line["layer_step_us"] = round(statistics.median(step_ms) * 1e3, 2)
    if args.step_layers > 0:
        line["decode_step"] = decode_step(w, scales, args.step_layers, args.steps)
        if args.config != 1 and args.kv_bits == 16 and not bf16 and 1 in others:
            # The small shape, where the host's launch work per layer is longer
            # than the GPU's: the step graph's case.
            w1 = workloads.config1(device=device).to_layout(args.layout)
            line["decode_step_config1"] = decode_step(w1, None, args.step_layers, args.steps)
            del w1
            torch.cuda.empty_cache()
    if args.prefill and args.kv_bits == 16:
        line["prefill"] = []
        for case in args.prefill.split(","):
            tokens, start = (int(x) for x in case.split("@"))
            leg = prefill_leg(w, tokens, args.steps, start=start)
            if not args.no_cpu and not bf16:
                leg["cpu_baseline"] = prefill_cpu_baseline(w, tokens, start, 6.0)
            line["prefill"].append(leg)
    if args.prefill_wide and args.kv_bits == 16:
        from types import SimpleNamespace

        hq, hkv = (int(x) for x in args.wide_heads.split("/"))
        wide = SimpleNamespace(q=w.q[:1], page_size=w.page_size, q_heads=hq, kv_heads=hkv,
                               head_dim=512, scale=512 ** -0.5, window=0, softcap=0.0,
                               layout=w.layout)
        line["prefill_wide"] = []
        for case in args.prefill_wide.split(","):
            tokens, start = (int(x) for x in case.split("@"))
            leg = prefill_leg(wide, tokens, min(args.steps, 10), start=start)
            # The float32 oracle gathers the whole prefix per call: only the
            # shorter prefixes are sampled on the CPU.
            if not args.no_cpu and not bf16 and start + tokens <= 65536:
                leg["cpu_baseline"] = prefill_cpu_baseline(wide, tokens, start, 6.0)
            line["prefill_wide"].append(leg)
            torch.cuda.empty_cache()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
