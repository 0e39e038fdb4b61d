"""Pins the prefill oracle (oracle/paged_attention.paged_prefill_dense) on
the CPU: the known answer of the reference's CUDA test (its prefill of the
three tokens agrees with its decode, tests/cuda_tests.cu:207-262), agreement
with the decode oracle at every position, brute force, chunking and window
invariances, and planted mistakes."""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import paged_attention as pa


def test_cuda_closed_form_prefill_agrees_with_decode():
    q, keys, values, tables, lengths, page, scale, expected = pa.cuda_closed_form_case()
    # Prefill of tokens 0..2 with the decode query at the last position.
    qs = np.concatenate([np.zeros((2, 1, 4)), q], axis=0)
    out = pa.paged_prefill_dense(qs, keys, values, tables[0], start=0, page_size=page,
                                 scale=scale)
    np.testing.assert_allclose(out[2, 0], expected, rtol=1e-12)
    # Token 0 sees only itself: its value row.
    np.testing.assert_allclose(out[0, 0], [1, 2, 3, 4], rtol=1e-12)


def arena(rng, rows, heads, dim):
    return (rng.standard_normal((rows, heads, dim)), rng.standard_normal((rows, heads, dim)))


@pytest.mark.parametrize("window,softcap", [(0, 0.0), (7, 0.0), (0, 20.0)])
def test_every_query_equals_a_decode_at_its_position(window, softcap):
    rng = np.random.default_rng(window + int(softcap))
    P, hq, hkv, d = 4, 6, 2, 8
    table = rng.permutation(12)
    keys, values = arena(rng, 12 * P, hkv, d)
    start, count = 9, 13
    q = rng.standard_normal((count, hq, d))
    out = pa.paged_prefill_dense(q, keys, values, table, start=start, page_size=P, scale=0.4,
                                 window=window, softcap=softcap)
    for t in range(count):
        want = pa.paged_decode_dense(q[t][None], keys, values, table[None],
                                     np.array([start + t + 1]), page_size=P, scale=0.4,
                                     window=window, softcap=softcap)
        np.testing.assert_allclose(out[t], want[0], rtol=1e-10, atol=1e-12)


def test_brute_force_and_chunking():
    rng = np.random.default_rng(3)
    P, hq, hkv, d = 2, 4, 1, 4
    table = np.array([3, 0, 2, 1, 4])
    keys, values = arena(rng, 10, hkv, d)
    q = rng.standard_normal((7, hq, d))
    out = pa.paged_prefill_dense(q, keys, values, table, start=2, page_size=P, scale=0.7)
    for t in range(7):
        p = 2 + t
        for h in range(hq):
            scores = []
            for kpos in range(p + 1):
                row = table[kpos // P] * P + kpos % P
                scores.append(0.7 * sum(q[t, h, i] * keys[row, 0, i] for i in range(d)))
            top = max(scores)
            w = [math.exp(s - top) for s in scores]
            acc = [0.0] * d
            for kpos, wk in enumerate(w):
                row = table[kpos // P] * P + kpos % P
                for i in range(d):
                    acc[i] += wk * values[row, 0, i]
            np.testing.assert_allclose(out[t, h], np.array(acc) / sum(w), rtol=1e-10)
    # Two chunks give the one-chunk result.
    a = pa.paged_prefill_dense(q[:3], keys, values, table, start=2, page_size=P, scale=0.7)
    b = pa.paged_prefill_dense(q[3:], keys, values, table, start=5, page_size=P, scale=0.7)
    np.testing.assert_allclose(np.concatenate([a, b]), out, rtol=1e-12)


def test_planted_mistakes_change_the_result():
    """A mask without the causal limit, or one off by one, fails."""
    rng = np.random.default_rng(4)
    P, hq, d = 4, 2, 8
    table = rng.permutation(6)
    keys, values = arena(rng, 24, 1, d)
    q = rng.standard_normal((5, hq, d))
    good = pa.paged_prefill_dense(q, keys, values, table, start=3, page_size=P, scale=0.5)
    # "Non-causal": every query sees the whole chunk = the last query's keys.
    last = pa.paged_decode_dense(q[0][None], keys, values, table[None], np.array([8]),
                                 page_size=P, scale=0.5)
    assert np.abs(good[0] - last[0]).max() > 1e-3
    # "Off by one": query p sees keys up to p - 1.
    shifted = pa.paged_decode_dense(q[2][None], keys, values, table[None], np.array([5]),
                                    page_size=P, scale=0.5)
    assert np.abs(good[2] - shifted[0]).max() > 1e-3


def test_image_spans_brute_force_and_invariants():
    """Image spans (batches.py:107-118): a query inside a span also sees the
    span's later keys, even outside the window; others stay causal."""
    rng = np.random.default_rng(11)
    P, hq, hkv, d = 4, 2, 1, 4
    table = rng.permutation(8)
    keys, values = arena(rng, 32, hkv, d)
    start, count = 5, 14
    q = rng.standard_normal((count, hq, d))
    images = [(7, 4), (13, 3)]
    out = pa.paged_prefill_dense(q, keys, values, table, start=start, page_size=P, scale=0.6,
                                 window=3, images=images)
    for t in range(count):
        p = start + t
        seen = [k for k in range(p + 1) if k > p - 3]
        for at, n in images:
            if at <= p < at + n:
                seen = sorted(set(seen) | set(range(at, at + n)))
        for h in range(hq):
            scores = [0.6 * sum(q[t, h, i] * keys[table[k // P] * P + k % P, 0, i]
                                for i in range(d)) for k in seen]
            top = max(scores)
            wts = [math.exp(x - top) for x in scores]
            acc = [sum(wk * values[table[k // P] * P + k % P, 0, i] for wk, k in zip(wts, seen))
                   for i in range(d)]
            np.testing.assert_allclose(out[t, h], np.array(acc) / sum(wts), rtol=1e-10)
    # A one-token image changes nothing; queries outside every image are causal.
    plain = pa.paged_prefill_dense(q, keys, values, table, start=start, page_size=P, scale=0.6,
                                   window=3)
    one = pa.paged_prefill_dense(q, keys, values, table, start=start, page_size=P, scale=0.6,
                                 window=3, images=[(9, 1)])
    np.testing.assert_allclose(one, plain, rtol=1e-12)
    outside = [t for t in range(count)
               if not any(at <= start + t < at + n for at, n in images)]
    np.testing.assert_allclose(out[outside], plain[outside], rtol=1e-12)
    # Identical queries inside one span see the same keys: identical outputs.
    q2 = q.copy()
    q2[2:6] = q2[2]
    out2 = pa.paged_prefill_dense(q2, keys, values, table, start=start, page_size=P, scale=0.6,
                                  images=[(7, 4)])
    np.testing.assert_allclose(out2[3:6], np.broadcast_to(out2[2], out2[3:6].shape), rtol=1e-12)
