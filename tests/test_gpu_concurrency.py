"""Calls that overlap on one GPU: decode and prefill calls on two streams at
once, and from two host threads at once, each stream with its own
workspace (the C-ABI's contract: only calls that share a workspace must not
overlap). With fixed split points every result must equal, bit for bit, the
same call run alone. Streams keep the default priority."""

import threading

import numpy as np
import pytest
import torch

from instinct_amd import workloads
from instinct_amd.hip_kernels import paged_decode_attention, paged_prefill_attention
from instinct_amd.paged_kv import rows_to_pages

pytestmark = pytest.mark.gpu


def decode_case(gpu, config, **kw):
    w = getattr(workloads, f"config{config}")(device=gpu, **kw).to_layout("pages")

    def call(out):
        return paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths, out=out,
                                      page_size=w.page_size, longest=w.longest, scale=w.scale,
                                      window=w.window, softcap=w.softcap, deterministic=True)
    return w, call


def prefill_case(gpu):
    rng = np.random.default_rng(0)
    P, hq, hkv, d, start, count = 16, 28, 4, 128, 3000, 256
    pages = (start + count + P - 1) // P
    table = torch.as_tensor(rng.permutation(pages + 3)[:pages].astype(np.int32), device=gpu)
    keys = rows_to_pages(torch.randn(((pages + 3) * P, hkv, d), device=gpu).half(), P)
    values = rows_to_pages(torch.randn(((pages + 3) * P, hkv, d), device=gpu).half(), P)
    q = torch.randn((count, hq, d), device=gpu).half()

    def call(out):
        return paged_prefill_attention(q, keys, values, table, start=start, page_size=P,
                                       scale=d ** -0.5, out=out, splits=4)
    return q, call


def test_two_streams_at_once(gpu):
    wa, call_a = decode_case(gpu, 2, batch=16, low=512, high=4096)
    wb, call_b = decode_case(gpu, 4, batch=8, low=1100, high=3000)
    qp, call_p = prefill_case(gpu)
    alone = [call_a(None), call_b(None), call_p(None)]
    torch.cuda.synchronize()
    outs = [[torch.empty_like(x) for x in alone] for _ in range(4)]
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    main = torch.cuda.current_stream()
    s1.wait_stream(main)
    s2.wait_stream(main)
    for i in range(4):
        with torch.cuda.stream(s1):
            call_a(outs[i][0])
            call_p(outs[i][2])
        with torch.cuda.stream(s2):
            call_b(outs[i][1])
            call_a(torch.empty_like(alone[0]))  # the same inputs read from both streams
    main.wait_stream(s1)
    main.wait_stream(s2)
    torch.cuda.synchronize()
    for i in range(4):
        for got, want, what in zip(outs[i], alone, ("decode A", "decode B", "prefill")):
            assert torch.equal(got, want), f"{what}, round {i}: differs from the call alone"


def test_two_host_threads_at_once(gpu):
    wa, call_a = decode_case(gpu, 2, batch=16, low=512, high=4096)
    wb, call_b = decode_case(gpu, 3, batch=1, length=8192)
    want = {"a": call_a(None), "b": call_b(None)}
    torch.cuda.synchronize()
    errors, got = [], {}
    barrier = threading.Barrier(2)

    def worker(name, call):
        try:
            torch.cuda.set_device(gpu)
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                barrier.wait()
                outs = [call(None) for _ in range(8)]
            stream.synchronize()
            got[name] = outs
        except Exception as exc:  # noqa: BLE001 — reported below
            errors.append(f"{name}: {exc!r}")

    threads = [threading.Thread(target=worker, args=("a", call_a)),
               threading.Thread(target=worker, args=("b", call_b))]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker did not finish"
    assert not errors, errors
    for name in ("a", "b"):
        for out in got[name]:
            assert torch.equal(out, want[name]), f"thread {name}: differs from the call alone"
