"""Pins the rotary-embedding / K/V-append oracle (oracle/rope_append.py) on the
CPU: the known answers of the reference's CUDA test, an independent complex
formulation, rotation invariants, brute force and planted mistakes."""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import rope_append as ra


def cuda_test_inputs():
    """tests/cuda_tests.cu:155-171: 2 tokens, 2 query heads, 1 kv head,
    head_dim 4, block of 4 tokens, base 10000."""
    hq, hkv, d = 2, 1, 4
    q = (0.1 * (np.arange(2 * hq * d) + 1)).astype(np.float16).reshape(2, hq, d)
    k = (0.2 * (np.arange(2 * hkv * d) + 1)).astype(np.float16).reshape(2, hkv, d)
    v = (1.0 + np.arange(2 * hkv * d)).astype(np.float16).reshape(2, hkv, d)
    return q, k, v


def test_cuda_known_answers_prefill_and_decode():
    q, k, v = cuda_test_inputs()
    inv = ra.inv_freq(4, base=10000.0)
    positions = np.array([0, 1])
    rows = np.array([0, 1])  # table {0}: page 0, offsets 0 and 1
    k_arena = np.zeros((1, 1, 4, 4), np.float16)  # one page tile [pages, kv, P, D]
    v_arena = np.zeros_like(k_arena)
    q_out, k_arena, v_arena = ra.rope_append(q, k, v, k_arena, v_arena, positions, rows,
                                             dims=4, inverse=inv, layout="pages", page_size=4)
    # "RoPE position zero" (:179): unchanged.
    assert abs(float(q_out[0, 0, 0]) - float(q[0, 0, 0])) < 1e-3
    # "RoPE position one" (:180-184): first * cos 1 - second * sin 1.
    first, second = float(q[1, 0, 0]), float(q[1, 0, 2])
    assert abs(float(q_out[1, 0, 0]) - (first * math.cos(1.0) - second * math.sin(1.0))) < 2e-3
    # "prefill K cache write", "prefill V cache write" (:185-187).
    assert abs(float(k_arena[0, 0, 0, 0]) - float(k[0, 0, 0])) < 1e-3
    assert abs(float(v_arena[0, 0, 0, 0]) - float(v[0, 0, 0])) < 1e-3
    # Decode (:189-200): one token at position 2 lands in slot 2 of page 0.
    dq = np.full((1, 2, 4), 0.5, np.float16)
    dk = np.full((1, 1, 4), 0.25, np.float16)
    dv = np.full((1, 1, 4), 3.0, np.float16)
    _, k2, v2 = ra.rope_append(dq, dk, dv, k_arena, v_arena, np.array([2]), np.array([2]),
                               dims=4, inverse=inv, layout="pages", page_size=4)
    assert abs(float(v2[0, 0, 2, 0]) - 3.0) < 1e-3
    # Only slot 2 changed.
    assert np.array_equal(np.delete(v2, 2, axis=2), np.delete(v_arena, 2, axis=2))


@pytest.mark.parametrize("mistake", ["traditional", "sign"])
def test_planted_mistakes_fail_the_known_answer(mistake):
    """A rotation of adjacent pairs (the 'traditional' layout) or of the other
    sense gives a different first element at position one."""
    q, _, _ = cuda_test_inputs()
    x = q[1, 0].astype(np.float64)
    if mistake == "traditional":
        got = x[0] * math.cos(1.0) - x[1] * math.sin(1.0)
    else:
        got = x[0] * math.cos(1.0) + x[2] * math.sin(1.0)
    want = x[0] * math.cos(1.0) - x[2] * math.sin(1.0)
    assert abs(got - want) > 2e-3


def test_inverse_frequencies():
    np.testing.assert_allclose(ra.inv_freq(8, base=10000.0), [1.0, 0.1, 0.01, 0.001], rtol=1e-6)
    for dims, base in ((128, 10000.0), (64, 1e6), (24, 500000.0)):
        exact = base ** (-np.arange(dims // 2) * 2.0 / dims)
        np.testing.assert_allclose(ra.inv_freq(dims, base=base), exact, rtol=2e-6)
    f = ra.inv_freq(12, freqs=[1.0, 4.0, 90.0, 1e4, np.inf, np.inf])
    np.testing.assert_allclose(f, [1.0, 0.25, 1 / 90.0, 1e-4, 0.0, 0.0], rtol=1e-7)
    assert f.dtype == np.float32


def random_case(rng, n, heads, d, dims, max_pos):
    x = rng.standard_normal((n, heads, d)).astype(np.float16)
    positions = rng.integers(0, max_pos, n)
    return x, positions


@pytest.mark.parametrize("d,dims,base", [(128, 128, 10000.0), (64, 32, 1e6), (24, 12, 500.0)])
def test_matches_the_complex_formulation(d, dims, base):
    rng = np.random.default_rng(d + dims)
    x, positions = random_case(rng, 9, 3, d, dims, 2048)
    inv = ra.inv_freq(dims, base=base)
    got = ra.rope(x, positions, dims, inv).astype(np.float64)
    want = ra.rope_complex(x, positions, dims, inv)
    assert np.abs(got - want).max() < 2e-3
    assert np.array_equal(got[..., dims:], x[..., dims:].astype(np.float64))


def test_large_positions_follow_the_float32_angle():
    """At positions near 2^17 the angle is only known to float32 rounding
    (about 0.008 rad): the oracle rounds position * inv_freq to float32 as the
    reference does, and the complex form on those same angles agrees."""
    rng = np.random.default_rng(7)
    x, _ = random_case(rng, 6, 2, 64, 64, 10)
    positions = np.array([0, 1, 65535, 100000, 120000, 131071])
    inv = ra.inv_freq(64, base=10000.0)
    got = ra.rope(x, positions, 64, inv).astype(np.float64)
    angles32 = (positions.astype(np.float32)[:, None] * inv[None, :]).astype(np.float64)
    z = (x[..., :32].astype(np.float64) + 1j * x[..., 32:].astype(np.float64))
    z = z * np.exp(1j * angles32)[:, None, :]
    want = np.concatenate([z.real, z.imag], axis=-1)
    assert np.abs(got - want).max() < 2e-3


def test_rotation_invariants():
    rng = np.random.default_rng(3)
    dims = 64
    inv = ra.inv_freq(dims, base=10000.0)
    q = rng.standard_normal((1, 1, dims))
    k = rng.standard_normal((1, 1, dims))
    # Pair norms are kept.
    r = ra.rope_complex(q, np.array([37]), dims, inv)
    np.testing.assert_allclose(r[..., :32] ** 2 + r[..., 32:] ** 2,
                               q[..., :32] ** 2 + q[..., 32:] ** 2, rtol=1e-12)
    # The score of rotated q and k depends only on the position difference.
    def score(p1, p2):
        return float((ra.rope_complex(q, np.array([p1]), dims, inv)
                      * ra.rope_complex(k, np.array([p2]), dims, inv)).sum())
    assert abs(score(10, 3) - score(1010, 1003)) < 1e-9
    assert abs(score(10, 3) - score(10, 4)) > 1e-3
    # Rotations compose.
    twice = ra.rope_complex(ra.rope_complex(q, np.array([5]), dims, inv), np.array([8]), dims, inv)
    np.testing.assert_allclose(twice, ra.rope_complex(q, np.array([13]), dims, inv), atol=1e-12)
    # Position 0 and infinite frequencies are the identity.
    x16 = rng.standard_normal((2, 2, 16)).astype(np.float16)
    assert np.array_equal(ra.rope(x16, np.array([0, 0]), 16, ra.inv_freq(16, base=1e4)), x16)
    frozen = ra.inv_freq(16, freqs=[np.inf] * 8)
    assert np.array_equal(ra.rope(x16, np.array([5, 9]), 16, frozen), x16)


def test_brute_force_on_tiny_inputs():
    rng = np.random.default_rng(5)
    x, positions = random_case(rng, 3, 2, 10, 6, 50)  # odd half = 3, two copied elements
    inv = ra.inv_freq(6, base=100.0)
    got = ra.rope(x, positions, 6, inv).astype(np.float64)
    want = ra.rope_brute(x, positions, 6, inv)
    assert np.abs(got - want).max() < 2e-3


@pytest.mark.parametrize("layout", ra.LAYOUTS)
def test_write_rows_in_both_layouts(layout):
    rng = np.random.default_rng(11)
    pages, heads, p, d = 5, 2, 4, 8
    data = rng.standard_normal((4, heads, d)).astype(np.float16)
    rows = np.array([0, 7, 19, -1])  # the last is outside the arena: skipped
    flat = np.zeros((pages * p, heads, d), np.float16)
    if layout == "rows":
        arena = flat.copy()
    else:
        arena = np.zeros((pages, heads, p, d), np.float16)
    ra.write_rows(arena, rows, data, layout=layout, page_size=p)
    as_rows = arena if layout == "rows" else arena.transpose(0, 2, 1, 3).reshape(-1, heads, d)
    for t, row in enumerate(rows[:3]):  # brute force
        assert np.array_equal(as_rows[row], data[t])
    assert np.count_nonzero(as_rows.any(axis=(1, 2))) == 3
    before = arena.copy()
    ra.write_rows(arena, np.array([pages * p]), data[:1], layout=layout, page_size=p)
    assert np.array_equal(arena, before)
