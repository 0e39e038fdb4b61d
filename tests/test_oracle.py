"""Pins the CPU oracle (oracle/) before anything is checked against it.

Every check here is independent of the oracle's own formulas: a closed-form
known answer from the reference (tests/cuda_tests.cu:207-262), brute-force
Python loops, torch's scaled_dot_product_attention, special cases with exact
answers, invariants the mathematics fixes (split count, page permutation,
windows, shared pages, GQA), and planted mistakes that these checks must
catch.
"""

import math

import numpy as np
import pytest
import torch

from oracle import cpu_oracle
from oracle import paged_attention as pa


def random_case(rng, *, batch=3, q_heads=8, kv_heads=2, dim=16, page=4, lengths=None,
                window=0, spare=3, released=False):
    lengths = np.array(lengths if lengths is not None else rng.integers(1, 40, batch))
    batch = len(lengths)
    need = [math.ceil(n / page) for n in lengths]
    arena = sum(need) + spare
    order = rng.permutation(arena)
    width = max(need)
    tables = np.zeros((batch, width), dtype=np.int32)
    cursor = 0
    for b, c in enumerate(need):
        tables[b, :c] = order[cursor:cursor + c]
        cursor += c
    if released and window:
        for b, n in enumerate(lengths):
            tables[b, : max(0, (n - window) // page)] = -1
    keys = rng.standard_normal((arena * page, kv_heads, dim)).astype(np.float16)
    values = rng.standard_normal((arena * page, kv_heads, dim)).astype(np.float16)
    q = rng.standard_normal((batch, q_heads, dim)).astype(np.float16)
    return q, keys, values, tables, lengths.astype(np.int32)


def brute_force(q, keys, values, tables, lengths, page, scale, window=0, softcap=0.0):
    """Plain Python loops with math.exp, one (sequence, head) at a time."""
    batch, hq, dim = q.shape
    hkv = keys.shape[1]
    group = hq // hkv
    out = np.zeros((batch, hq, dim))
    for b in range(batch):
        n = int(lengths[b])
        first = max(0, n - window) if window else 0
        for h in range(hq):
            kvh = h // group
            scores, vals = [], []
            for t in range(first, n):
                pg = int(tables[b][t // page])
                if pg < 0:
                    continue
                row = pg * page + t % page
                s = sum(float(q[b, h, d]) * scale * float(keys[row, kvh, d]) for d in range(dim))
                if softcap:
                    s = math.tanh(s / softcap) * softcap
                scores.append(s)
                vals.append([float(values[row, kvh, d]) for d in range(dim)])
            if not scores:
                continue
            top = max(scores)
            ws = [math.exp(s - top) for s in scores]
            tot = sum(ws)
            for d in range(dim):
                out[b, h, d] = sum(w * v[d] for w, v in zip(ws, vals)) / tot
    return out


def test_closed_form_from_cuda_tests():
    q, keys, values, tables, lengths, page, scale, expected = pa.cuda_closed_form_case()
    kw = dict(page_size=page, scale=scale)
    dense = pa.paged_decode_dense(q, keys, values, tables, lengths, **kw)
    np.testing.assert_allclose(dense[0, 0], expected, rtol=0, atol=1e-12)
    for splits in (1, 2, 3):
        split = pa.paged_decode_splitk(q, keys, values, tables, lengths, splits=splits, **kw)
        np.testing.assert_allclose(split[0, 0], expected, rtol=0, atol=1e-12)
    c64 = cpu_oracle.decode_f64(q.astype(np.float16), keys.astype(np.float16),
                                values.astype(np.float16), tables, lengths, **kw)
    np.testing.assert_allclose(c64[0, 0], expected, rtol=0, atol=1e-12)
    c16 = cpu_oracle.decode_splitk(q, keys, values, tables, lengths, **kw)
    np.testing.assert_allclose(c16[0, 0].astype(np.float64), expected, atol=4e-3)
    c32 = cpu_oracle.decode_f32(q, keys, values, tables, lengths, **kw)
    np.testing.assert_allclose(c32[0, 0].astype(np.float64), expected, atol=4e-3)


@pytest.mark.parametrize("seed", range(4))
def test_dense_matches_brute_force(seed):
    rng = np.random.default_rng(seed)
    window = [0, 0, 7, 13][seed]
    softcap = [0.0, 5.0, 0.0, 2.0][seed]
    case = random_case(rng, batch=3, q_heads=4, kv_heads=2, dim=6, page=4,
                       lengths=[1, 9, 23], window=window, released=seed == 3)
    scale = 0.37
    expected = brute_force(*case, 4, scale, window, softcap)
    got = pa.paged_decode_dense(*case, page_size=4, scale=scale, window=window, softcap=softcap)
    np.testing.assert_allclose(got, expected, rtol=0, atol=1e-12)
    got_c = cpu_oracle.decode_f64(*case, page_size=4, scale=scale, window=window, softcap=softcap)
    np.testing.assert_allclose(got_c, expected, rtol=0, atol=1e-12)


def test_dense_matches_torch_sdpa():
    rng = np.random.default_rng(11)
    q, keys, values, tables, lengths = random_case(rng, batch=4, q_heads=8, kv_heads=2,
                                                   dim=32, page=8, lengths=[5, 64, 77, 130])
    scale = 32 ** -0.5
    got = pa.paged_decode_dense(q, keys, values, tables, lengths, page_size=8, scale=scale)
    for b, n in enumerate(lengths):
        rows = [int(tables[b][t // 8]) * 8 + t % 8 for t in range(n)]
        k = torch.tensor(keys[rows].astype(np.float64)).permute(1, 0, 2)  # [HKV, n, D]
        v = torch.tensor(values[rows].astype(np.float64)).permute(1, 0, 2)
        k = k.repeat_interleave(4, dim=0)
        v = v.repeat_interleave(4, dim=0)
        qq = torch.tensor(q[b].astype(np.float64))[:, None, :]  # [HQ, 1, D]
        ref = torch.nn.functional.scaled_dot_product_attention(qq, k, v, scale=scale)
        np.testing.assert_allclose(got[b], ref[:, 0, :].numpy(), rtol=0, atol=1e-12)


def test_single_key_returns_its_value_row():
    rng = np.random.default_rng(2)
    q, keys, values, tables, lengths = random_case(rng, lengths=[1, 1], page=4)
    got = pa.paged_decode_dense(q, keys, values, tables, lengths, page_size=4, scale=0.5)
    for b in range(2):
        row = int(tables[b][0]) * 4
        for h in range(q.shape[1]):
            np.testing.assert_array_equal(got[b, h], values[row, h // 4].astype(np.float64))


def test_identical_keys_average_the_values():
    rng = np.random.default_rng(3)
    q, keys, values, tables, lengths = random_case(rng, lengths=[10], page=4, kv_heads=1,
                                                   q_heads=2)
    keys[:] = keys[0]
    got = pa.paged_decode_dense(q, keys, values, tables, lengths, page_size=4, scale=0.5)
    rows = [int(tables[0][t // 4]) * 4 + t % 4 for t in range(10)]
    mean = values[rows, 0].astype(np.float64).mean(axis=0)
    np.testing.assert_allclose(got[0, 0], mean, atol=1e-12)


def test_dominant_key_selects_its_value():
    rng = np.random.default_rng(4)
    q, keys, values, tables, lengths = random_case(rng, lengths=[50], page=4, kv_heads=1,
                                                   q_heads=1, dim=8)
    q[:] = 1.0
    keys[:] = 0.0
    row = int(tables[0][37 // 4]) * 4 + 37 % 4
    keys[row, 0] = 8.0  # score 64 * scale = 64 against 0 for every other key
    got = pa.paged_decode_dense(q, keys, values, tables, lengths, page_size=4, scale=1.0)
    np.testing.assert_allclose(got[0, 0], values[row, 0].astype(np.float64), atol=1e-12)


@pytest.mark.parametrize("splits", [1, 2, 3, 7, 64, 128])
def test_split_count_does_not_change_the_result(splits):
    rng = np.random.default_rng(5)
    case = random_case(rng, lengths=[1, 17, 100, 257], page=8, window=0)
    dense = pa.paged_decode_dense(*case, page_size=8, scale=0.3)
    split = pa.paged_decode_splitk(*case, page_size=8, scale=0.3, splits=splits)
    np.testing.assert_allclose(split, dense, rtol=0, atol=1e-12)


def test_reference_split_rule():
    assert pa.reference_splits(1) == 1
    assert pa.reference_splits(512) == 1
    assert pa.reference_splits(513) == 2
    assert pa.reference_splits(10**6) == 128
    assert pa.reference_splits(100000, window=1024) == 2


def test_page_permutation_does_not_change_the_result():
    rng = np.random.default_rng(6)
    q, keys, values, tables, lengths = random_case(rng, lengths=[30, 45], page=4, spare=0)
    base = pa.paged_decode_dense(q, keys, values, tables, lengths, page_size=4, scale=0.4)
    perm = rng.permutation(keys.shape[0] // 4)
    # Move physical page p to perm[p]; rewrite the tables to match.
    k2 = np.empty_like(keys)
    v2 = np.empty_like(values)
    for p_old, p_new in enumerate(perm):
        k2[p_new * 4:(p_new + 1) * 4] = keys[p_old * 4:(p_old + 1) * 4]
        v2[p_new * 4:(p_new + 1) * 4] = values[p_old * 4:(p_old + 1) * 4]
    t2 = perm[tables]
    t2[:, :] = np.where(tables >= 0, perm[tables], tables)
    got = pa.paged_decode_dense(q, k2, v2, t2, lengths, page_size=4, scale=0.4)
    np.testing.assert_array_equal(got, base)


def test_window_equals_full_attention_on_the_last_keys_and_ignores_poison():
    rng = np.random.default_rng(7)
    q, keys, values, tables, lengths = random_case(rng, lengths=[40, 33], page=4,
                                                   window=10, released=True)
    got = pa.paged_decode_dense(q, keys, values, tables, lengths, page_size=4, scale=0.5,
                                window=10)
    for b, n in enumerate(lengths):
        # Rebuild a dense sequence of just the window, in fresh pages.
        pos = np.arange(n - 10, n)
        rows = tables[b][pos // 4].astype(np.int64) * 4 + pos % 4
        k = keys[rows]
        v = values[rows]
        ref = pa.attention_plain(q[b][None, :, None, :], k.transpose(1, 0, 2)[None],
                                 v.transpose(1, 0, 2)[None], scale=0.5)
        np.testing.assert_allclose(got[b], ref[0, :, 0, :], atol=1e-12)
    # Poison every row the windows cannot see: the result must not move.
    visible = set()
    for b, n in enumerate(lengths):
        for t in range(n - 10, n):
            visible.add(int(tables[b][t // 4]) * 4 + t % 4)
    k3, v3 = keys.copy(), values.copy()
    for row in range(keys.shape[0]):
        if row not in visible:
            k3[row] = np.nan
            v3[row] = np.inf
    got3 = pa.paged_decode_dense(q, k3, v3, tables, lengths, page_size=4, scale=0.5, window=10)
    np.testing.assert_array_equal(got3, got)
    got4 = cpu_oracle.decode_f64(q, k3, v3, tables, lengths, page_size=4, scale=0.5, window=10)
    np.testing.assert_allclose(got4, got, atol=1e-12)


def test_released_page_inside_the_range_is_masked():
    rng = np.random.default_rng(8)
    q, keys, values, tables, lengths = random_case(rng, lengths=[24], page=4, q_heads=2,
                                                   kv_heads=1)
    masked = tables.copy()
    masked[0, 2] = -1  # positions 8..11 disappear
    got = pa.paged_decode_dense(q, keys, values, masked, lengths, page_size=4, scale=0.5)
    keep = [t for t in range(24) if t // 4 != 2]
    rows = [int(tables[0][t // 4]) * 4 + t % 4 for t in keep]
    ref = pa.attention_plain(q[0][None, :, None, :], keys[rows].transpose(1, 0, 2)[None],
                             values[rows].transpose(1, 0, 2)[None], scale=0.5)
    np.testing.assert_allclose(got[0], ref[0, :, 0, :], atol=1e-12)


def test_shared_pages_equal_private_copies():
    rng = np.random.default_rng(9)
    q, keys, values, tables, lengths = random_case(rng, lengths=[20, 28], page=4, spare=10)
    shared = tables.copy()
    shared[1, :3] = shared[0, :3]  # sequence 1 reuses sequence 0's first 3 pages
    got = pa.paged_decode_dense(q, keys, values, shared, lengths, page_size=4, scale=0.5)
    # Same computation with private copies of the shared pages in spare pages.
    k2, v2, private = keys.copy(), values.copy(), shared.copy()
    unused = sorted(set(range(keys.shape[0] // 4)) - set(tables.ravel().tolist()))
    for i in range(3):
        src = shared[0, i]
        dst = unused[i]
        k2[dst * 4:(dst + 1) * 4] = keys[src * 4:(src + 1) * 4]
        v2[dst * 4:(dst + 1) * 4] = values[src * 4:(src + 1) * 4]
        private[1, i] = dst
    ref = pa.paged_decode_dense(q, k2, v2, private, lengths, page_size=4, scale=0.5)
    np.testing.assert_array_equal(got, ref)


def test_gqa_heads_share_their_kv_head():
    rng = np.random.default_rng(10)
    q, keys, values, tables, lengths = random_case(rng, lengths=[15, 31], page=4, q_heads=6,
                                                   kv_heads=2)
    q[:, 1] = q[:, 0]  # heads 0 and 1 share kv head 0 and the same query
    got = pa.paged_decode_dense(q, keys, values, tables, lengths, page_size=4, scale=0.5)
    np.testing.assert_array_equal(got[:, 1], got[:, 0])
    # G = 3 equals the same computation with HQ = HKV on repeated K/V.
    k_rep = np.repeat(keys, 3, axis=1)
    v_rep = np.repeat(values, 3, axis=1)
    ref = pa.paged_decode_dense(q, k_rep, v_rep, tables, lengths, page_size=4, scale=0.5)
    np.testing.assert_allclose(got, ref, atol=1e-12)


def test_empty_sequence_gives_zeros():
    rng = np.random.default_rng(12)
    q, keys, values, tables, lengths = random_case(rng, lengths=[0, 5], page=4)
    got = pa.paged_decode_dense(q, keys, values, tables, lengths, page_size=4, scale=0.5)
    assert not got[0].any()
    got_c = cpu_oracle.decode_f64(q, keys, values, tables, lengths, page_size=4, scale=0.5)
    assert not got_c[0].any()
    np.testing.assert_allclose(got_c, got, atol=1e-12)


@pytest.mark.parametrize("seed", range(3))
def test_c_oracles_match_the_numpy_restatement(seed):
    rng = np.random.default_rng(100 + seed)
    window = [0, 24, 0][seed]
    softcap = [0.0, 0.0, 3.0][seed]
    case = random_case(rng, batch=5, q_heads=12, kv_heads=4, dim=64, page=16,
                       lengths=rng.integers(1, 300, 5), window=window, released=bool(window))
    scale = 64 ** -0.5
    ref = pa.paged_decode_dense(*case, page_size=16, scale=scale, window=window, softcap=softcap)
    c64 = cpu_oracle.decode_f64(*case, page_size=16, scale=scale, window=window, softcap=softcap)
    np.testing.assert_allclose(c64, ref, rtol=0, atol=1e-11)
    for splits in (0, 1, 5):
        c16 = cpu_oracle.decode_splitk(*case, page_size=16, scale=scale, window=window,
                                       softcap=softcap, splits=splits)
        err_max, err_mean = pa.error_stats(c16, ref)
        assert err_max <= 2e-3 and err_mean <= 2e-4, (err_max, err_mean)
    c32 = cpu_oracle.decode_f32(*case, page_size=16, scale=scale, window=window,
                                softcap=softcap)
    err_max, err_mean = pa.error_stats(c32, ref)
    assert err_max <= 2e-3 and err_mean <= 2e-4, (err_max, err_mean)
    # The float32 path step by step in NumPy (gather, scores, softmax, then
    # the product, each in float32): equal up to the summation order of the
    # float32 dot products, i.e. within one fp16 ulp.
    q, keys, values, tables, lengths = case
    want = np.zeros(q.shape, dtype=np.float16)
    group = q.shape[1] // keys.shape[1]
    for b in range(q.shape[0]):
        n = int(lengths[b])
        first = max(0, n - window) if window else 0
        pos = np.arange(first, n)
        pages = tables[b, pos // 16]
        ok = pages >= 0
        rows = np.where(ok, pages * 16 + pos % 16, 0)
        for h in range(q.shape[1]):
            kr = keys[rows, h // group].astype(np.float32)
            vr = values[rows, h // group].astype(np.float32)
            s = kr @ (q[b, h].astype(np.float32) * np.float32(scale))
            if softcap:
                s = np.tanh(s / np.float32(softcap)) * np.float32(softcap)
            s = np.where(ok, s, -np.inf).astype(np.float32)
            e = np.exp(s - s.max()).astype(np.float32)
            p = (e / e.sum(dtype=np.float32)).astype(np.float32)
            want[b, h] = (p @ vr).astype(np.float16)
    ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
    assert (np.abs(c32.astype(np.float64) - want.astype(np.float64)) <= ulp + 1e-7).all()


def test_fp16_conversions_round_to_nearest_even():
    lib = cpu_oracle.library()
    bits = np.arange(65536, dtype=np.uint16)
    floats = np.zeros(65536, dtype=np.float32)
    lib.oracle_half_to_float(bits.ctypes.data, floats.ctypes.data, 65536)
    np.testing.assert_array_equal(floats.view(np.uint32),
                                  bits.view(np.float16).astype(np.float32).view(np.uint32))
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * s
                        for s in (1e-7, 1e-5, 1e-3, 1, 1e3, 6e4)])
    back = np.zeros(x.size, dtype=np.uint16)
    lib.oracle_float_to_half(x.ctypes.data, back.ctypes.data, x.size)
    np.testing.assert_array_equal(back, x.astype(np.float16).view(np.uint16))


# --- planted mistakes: each must be caught by the checks above ----------------

_decode_rows = pa.decode_rows


def _wrong_rows(tables, lengths, *, page_size, span):
    rows, valid = _decode_rows(tables, lengths, page_size=page_size, span=span)
    return rows ^ 1, valid  # swaps neighbouring rows inside every page


def _dropped_mask(tables, lengths, *, page_size, span):
    rows, valid = _decode_rows(tables, lengths, page_size=page_size, span=span)
    return rows, np.ones_like(valid)  # forgets that released/absent rows are masked


@pytest.mark.parametrize("mistake", [_wrong_rows, _dropped_mask])
def test_planted_mistakes_are_caught(monkeypatch, mistake):
    monkeypatch.setattr(pa, "decode_rows", mistake)
    q, keys, values, tables, lengths, page, scale, expected = pa.cuda_closed_form_case()
    got = pa.paged_decode_dense(q, keys, values, tables, lengths, page_size=page, scale=scale)
    caught = not np.allclose(got[0, 0], expected, atol=1e-6)
    if not caught:  # the closed form has no masked rows: use the released-page case
        rng = np.random.default_rng(8)
        qq, kk, vv, tt, ll = random_case(rng, lengths=[24], page=4, q_heads=2, kv_heads=1)
        tt[0, 2] = -1
        expected2 = brute_force(qq, kk, vv, tt, ll, 4, 0.5)
        got2 = pa.paged_decode_dense(qq, kk, vv, tt, ll, page_size=4, scale=0.5)
        caught = not np.allclose(got2, expected2, atol=1e-6)
    assert caught
