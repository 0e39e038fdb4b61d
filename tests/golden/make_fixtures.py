"""Writes the committed parity fixtures (tests/golden/*.npz).

Each fixture holds one small decode-attention call: fp16 queries, the layer's
K/V arena (only the pages the call touches), int32 page tables and lengths,
the scalars, and the expected output computed in float64 (stored as
float32) by the restated oracle (oracle/paged_attention.py, the reference's portable path). These are
"restated oracle" vectors: the reference ships no golden data for this path
and its MLX implementation cannot run here, so none of them is MLX output.

Shapes follow the five BASELINE configurations, scaled down, plus the
known answer of the reference's tests/cuda_tests.cu:207-262 embedded at the
kernel's page size. Regenerate with: python tests/golden/make_fixtures.py
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import paged_attention as pa  # noqa: E402


def arena_case(rng, lengths, q_heads, kv_heads, dim, page, *, window=0, released=False,
               shared_prefix=0, sharers=(), kv_scale=1.0, planted=0):
    lengths = np.asarray(lengths, dtype=np.int64)
    batch = len(lengths)
    need = [math.ceil(n / page) for n in lengths]
    prefix_pages = shared_prefix // page
    own = [n - (prefix_pages if b in sharers else 0) for b, n in enumerate(need)]
    arena = prefix_pages + sum(own) + 1  # one page nobody maps
    order = prefix_pages + rng.permutation(arena - prefix_pages)
    width = max(need)
    tables = np.zeros((batch, width), dtype=np.int32)
    cursor = 0
    for b in range(batch):
        pages = order[cursor: cursor + own[b]]
        cursor += own[b]
        if b in sharers:
            pages = np.concatenate([np.arange(prefix_pages), pages])
        tables[b, : need[b]] = pages
        if released and window:
            tables[b, : max(0, (lengths[b] - window) // page)] = -1
    keys = (rng.standard_normal((arena * page, kv_heads, dim)) * kv_scale).astype(np.float16)
    values = (rng.standard_normal((arena * page, kv_heads, dim)) * kv_scale).astype(np.float16)
    for b in range(batch):
        for _ in range(planted):
            t = int(rng.integers(0, lengths[b]))
            row = int(tables[b][t // page]) * page + t % page
            kvh = int(rng.integers(0, kv_heads))
            keys[row, kvh] = (keys[row, kvh].astype(np.float32) * 8).astype(np.float16)
    q = rng.standard_normal((batch, q_heads, dim)).astype(np.float16)
    return q, keys, values, tables, lengths.astype(np.int32)


def closed_form():
    """cuda_tests.cu:207-262 at page 16, head_dim 64 (see test_gpu_parity)."""
    D, P = 64, 16
    keys = np.zeros((2 * P, 1, D), dtype=np.float16)
    values = np.zeros((2 * P, 1, D), dtype=np.float16)
    keys[P, 0, :4] = [1, 0, 0, 0]
    values[P, 0, :4] = [1, 2, 3, 4]
    keys[P + 1: 2 * P, 0, :4] = [0, 1, 0, 0]
    values[P + 1: 2 * P, 0, :4] = [5, 6, 7, 8]
    keys[0, 0, :4] = [1, 1, 0, 0]
    values[0, 0, :4] = [2, 4, 6, 8]
    q = np.zeros((1, 2, D), dtype=np.float16)
    q[0, :, :2] = 1.0
    return q, keys, values, np.array([[1, 0]], dtype=np.int32), np.array([17], dtype=np.int32)


CASES = {
    # name: (builder, page, scale, window, softcap)
    "closed_form_p16": (lambda rng: closed_form(), 16, 0.5, 0, 0.0),
    "config1_small": (lambda rng: arena_case(rng, [64, 64], 14, 2, 64, 16, kv_scale=0.5),
                      16, 64 ** -0.5, 0, 0.0),
    "config2_small": (lambda rng: arena_case(rng, [17, 33, 40], 28, 4, 128, 16),
                      16, 128 ** -0.5, 0, 0.0),
    "config3_small": (lambda rng: arena_case(rng, [48], 32, 8, 128, 16, planted=4),
                      16, 128 ** -0.5, 0, 0.0),
    "config4_small": (lambda rng: arena_case(rng, [45, 40], 8, 4, 256, 16, window=24,
                                             released=True),
                      16, 256 ** -0.5, 24, 0.0),
    "config5_small": (lambda rng: arena_case(rng, [36, 20, 3, 33], 32, 8, 128, 16,
                                             shared_prefix=32, sharers=(0, 3)),
                      16, 128 ** -0.5, 0, 0.0),
    "softcap_small": (lambda rng: arena_case(rng, [5, 50], 8, 1, 80, 16),
                      16, 80 ** -0.5, 0, 30.0),
}


def main():
    for i, (name, (build, page, scale, window, softcap)) in enumerate(CASES.items()):
        rng = np.random.default_rng(1000 + i)
        q, keys, values, tables, lengths = build(rng)
        expected = pa.paged_decode_dense(q, keys, values, tables, lengths, page_size=page,
                                         scale=scale, window=window, softcap=softcap)
        np.savez_compressed(HERE / f"{name}.npz", q=q, keys=keys, values=values,
                            tables=tables, lengths=lengths, expected=expected.astype(np.float32),
                            page_size=page, scale=scale, window=window, softcap=softcap)
        print(name, q.shape, keys.shape, tables.shape, (HERE / f"{name}.npz").stat().st_size)


if __name__ == "__main__":
    main()
