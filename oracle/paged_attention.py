"""CPU oracle for split-K paged decode attention — TEST INFRASTRUCTURE ONLY.

This module restates, in NumPy float64, what the reference computes on its
paged decode path (KavinP21/LLM-Inference, "Instinct"). Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import it,
and only as the checker: the product path (``instinct_amd``) never calls it.

Functions and the reference lines they follow:

* :func:`decode_rows` — ``portable.decode_rows``
  (python/instinct/backends/portable.py:194-205): right-aligned last ``span``
  positions of each sequence, valid when the position is >= 0 and its page id
  is >= 0 (released pages are masked), rows = page * P + position % P.
* :func:`attention_plain` — ``portable._attention_plain`` (portable.py:173-188):
  GQA repeat of K/V, scores (q * scale) @ K^T in float, optional softcap
  ``tanh(s / c) * c``, masked to -inf, softmax, @ V.
* :func:`paged_decode_dense` — the portable ("MLX CPU") decode,
  ``DecodeBatch._attend_dense`` (python/instinct/batches.py:228-246) with the
  span of ``DecodeBatch.__init__`` (:183-189): gather, then dense attention.
  Rows that are all masked (length 0) give zeros, as the Metal kernel writes
  (metal_kernels.py:88).
* :func:`paged_decode_splitk` — the Metal kernel's algorithm
  (metal_kernels.py:18-124): per split an online softmax over its key range,
  unnormalised partials (acc, running max, sum), then the log-sum-exp merge
  that skips splits whose max is -inf. ``splits`` defaults to the reference
  rule ``clamp(ceil(span / 512), 1, 128)`` (metal_kernels.py:126-127,193-194).
* :func:`paged_prefill_dense` — ``PrefillBatch.attend`` (batches.py:84-132):
  one prompt chunk's causal (and windowed) attention over the keys gathered
  from its page table, in float64.
* :func:`cuda_closed_form_case` — the known answer of
  tests/cuda_tests.cu:207-262 (decode over 3 keys in 2 out-of-order pages).

Pinning (tests/test_oracle.py): the closed form above, brute-force Python
loops on tiny inputs, torch's scaled_dot_product_attention on CPU, special
cases (one key, identical keys, a dominant key), split-count invariance,
window/poison invariance, and shared-page equivalence.
"""

from __future__ import annotations

import math

import numpy as np

KEYS_PER_SPLIT = 512  # metal_kernels.py:126
MAX_SPLITS = 128  # metal_kernels.py:127


def decode_rows(tables: np.ndarray, lengths: np.ndarray, *, page_size: int, span: int):
    """Rows and validity of each sequence's last ``span`` positions
    (portable.py:194-205). ``tables`` is ``[B, width]``; negative pages are
    released. Returns ``rows [B, span]`` int64 and ``valid [B, span]`` bool."""
    tables = np.asarray(tables)
    lengths = np.asarray(lengths).astype(np.int64)
    positions = lengths[:, None] - span + np.arange(span)[None, :]
    valid = positions >= 0
    clipped = np.maximum(positions, 0)
    page_index = clipped // page_size
    # The reference indexes the table with take_along_axis; positions past the
    # table width cannot be valid keys, so they are masked here.
    inside = page_index < tables.shape[1]
    pages = np.take_along_axis(tables, np.minimum(page_index, tables.shape[1] - 1), axis=1)
    valid = valid & inside & (pages >= 0)
    rows = np.where(valid, pages.astype(np.int64) * page_size + clipped % page_size, 0)
    return rows, valid


def attention_plain(q, k, v, *, scale: float, mask=None, softcap: float = 0.0,
                    dtype=np.float64):
    """``[B, H, Q, D]`` attention with K/V ``[B, HKV, N, D]`` (portable.py:173-188),
    in float64 (``dtype=np.float32``: the portable path's own float32
    arithmetic, used only for bench's CPU-baseline timing). ``mask`` is a
    boolean array broadcastable to the scores."""
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    batch, heads, count, dim = q.shape
    hkv = k.shape[1]
    # Query head h reads kv head h // groups: the group's queries are stacked
    # as rows of one product per kv head instead of repeating K and V.
    grouped = (q * scale).reshape(batch, hkv, (heads // hkv) * count, dim)
    scores = (grouped @ np.swapaxes(k, -1, -2)).reshape(batch, heads, count, -1)
    if softcap:
        scores = np.tanh(scores / softcap) * softcap
    if mask is not None:
        scores = np.where(mask, scores, -np.inf)
    top = np.max(scores, axis=-1, keepdims=True)
    top = np.where(np.isfinite(top), top, 0.0)
    weights = np.exp(scores - top)
    total = np.sum(weights, axis=-1, keepdims=True)
    probs = np.divide(weights, total, out=np.zeros_like(weights), where=total > 0)
    probs = probs.reshape(batch, hkv, (heads // hkv) * count, -1)
    return (probs @ v).reshape(batch, heads, count, dim)


def paged_decode_dense(q, keys, values, tables, lengths, *, page_size: int, scale: float,
                       window: int = 0, softcap: float = 0.0, longest: int | None = None):
    """Portable decode (batches.py:183-189,228-246) in float64.

    ``q [B, HQ, D]``, ``keys/values [rows, HKV, D]`` (one layer's arena),
    ``tables [B, width]`` int, ``lengths [B]`` int. Returns ``[B, HQ, D]``
    float64. Sequence by sequence so that memory stays proportional to one
    sequence's span."""
    q = np.asarray(q)
    lengths = np.asarray(lengths).astype(np.int64)
    batch, hq, dim = q.shape
    hkv = keys.shape[1]
    if hq % hkv:
        raise ValueError("query heads must be a multiple of kv heads")
    out = np.zeros((batch, hq, dim), dtype=np.float64)
    for b in range(batch):
        n = int(max(lengths[b], 0))
        span = min(n, window) if window else n
        if span <= 0:
            continue
        rows, valid = decode_rows(tables[b : b + 1], lengths[b : b + 1],
                                  page_size=page_size, span=span)
        k = np.asarray(keys)[rows[0]].astype(np.float64)  # [span, HKV, D]
        v = np.asarray(values)[rows[0]].astype(np.float64)
        k = np.where(valid[0][:, None, None], k, 0.0).transpose(1, 0, 2)[None]
        v = np.where(valid[0][:, None, None], v, 0.0).transpose(1, 0, 2)[None]
        o = attention_plain(q[b][None, :, None, :], k, v, scale=scale,
                            mask=valid[0][None, None, None, :], softcap=softcap)
        out[b] = o[0, :, 0, :]
    return out


def paged_prefill_dense(q, keys, values, table, *, start: int, page_size: int, scale: float,
                        window: int = 0, softcap: float = 0.0, images=(), dtype=np.float64):
    """Prefill attention of one chunk (``PrefillBatch.attend``,
    python/instinct/batches.py:84-132, no images) in float64: queries
    ``[count, HQ, D]`` at positions ``start ..``, keys/values the arena
    ``[rows, HKV, D]``, ``table`` the sequence's pages. Query p sees keys
    ``[first, p]``, ``first = max(0, start - window + 1)`` for the chunk and
    the causal mask aligned to the newest key, plus ``key > p - window``
    with a window; pages with a negative id are masked. ``images``: (at,
    length) spans of image tokens; a query inside a span also sees every key
    of that span (batches.py:107-118), whatever the causal limit and the
    window. Returns ``[count, HQ, D]`` float64 (``dtype``: as for
    :func:`attention_plain`)."""
    q = np.asarray(q)
    count, hq, dim = q.shape
    end = start + count
    first = max(0, start - window + 1) if window else 0
    positions = np.arange(first, end)
    table = np.asarray(table)
    pages = table[positions // page_size]
    usable = pages >= 0
    rows = np.where(usable, pages.astype(np.int64) * page_size + positions % page_size, 0)
    k = np.where(usable[:, None, None], np.asarray(keys)[rows].astype(dtype), dtype(0))
    v = np.where(usable[:, None, None], np.asarray(values)[rows].astype(dtype), dtype(0))
    qpos = np.arange(start, end)[:, None]
    kpos = positions[None, :]
    mask = (kpos <= qpos) & usable[None, :]
    if window:
        mask &= kpos > qpos - window
    for at, length in images:
        inside = (qpos >= at) & (qpos < at + length)
        mask |= inside & (kpos >= at) & (kpos < at + length) & usable[None, :]
    out = attention_plain(q.transpose(1, 0, 2)[None], k.transpose(1, 0, 2)[None],
                          v.transpose(1, 0, 2)[None], scale=scale, mask=mask[None, None],
                          softcap=softcap, dtype=dtype)
    return out[0].transpose(1, 0, 2)


def reference_splits(longest: int, window: int = 0) -> int:
    """The reference's batch-wide split count (metal_kernels.py:193-194)."""
    span = min(longest, window) if window else longest
    return max(1, min(MAX_SPLITS, math.ceil(span / KEYS_PER_SPLIT)))


def paged_decode_splitk(q, keys, values, tables, lengths, *, page_size: int, scale: float,
                        window: int = 0, softcap: float = 0.0, splits: int | None = None,
                        longest: int | None = None):
    """The Metal kernel's split-K algorithm (metal_kernels.py:18-124), float64.

    Each (sequence, kv head, split) covers ``[begin, end)`` with
    ``per = ceil((len - first) / splits)`` (:32-36); its partial is the
    unnormalised accumulator with the running max and sum (:54-60, :93-101);
    the merge (:103-124) skips splits whose max is -inf and normalises, giving
    0 where the total is 0 (:122). Released pages (negative ids) are masked as
    in the portable path. Returns ``[B, HQ, D]`` float64."""
    q = np.asarray(q, dtype=np.float64)
    lengths = np.asarray(lengths).astype(np.int64)
    batch, hq, dim = q.shape
    hkv = keys.shape[1]
    if hq % hkv:
        raise ValueError("query heads must be a multiple of kv heads")
    group = hq // hkv
    if splits is None:
        splits = reference_splits(int(longest if longest is not None else lengths.max()), window)
    out = np.zeros((batch, hq, dim), dtype=np.float64)
    for b in range(batch):
        n = int(lengths[b])
        first = max(0, n - window) if window else 0
        per = -(-(n - first) // splits) if n > first else 0
        part_o = np.zeros((splits, hq, dim))
        part_m = np.full((splits, hq), -np.inf)
        part_l = np.zeros((splits, hq))
        for s in range(splits):
            begin = first + s * per
            end = min(n, begin + per)
            if end <= begin:
                continue
            pos = np.arange(begin, end)
            page_index = pos // page_size
            inside = page_index < tables.shape[1]
            pages = np.asarray(tables[b])[np.minimum(page_index, tables.shape[1] - 1)]
            ok = inside & (pages >= 0)
            if not ok.any():
                continue
            rows = pages[ok].astype(np.int64) * page_size + pos[ok] % page_size
            k = np.asarray(keys)[rows].astype(np.float64)  # [n, HKV, D]
            v = np.asarray(values)[rows].astype(np.float64)
            for h in range(hq):
                kvh = h // group
                sc = (k[:, kvh, :] @ (q[b, h] * scale))
                if softcap:
                    sc = np.tanh(sc / softcap) * softcap
                top = sc.max()
                p = np.exp(sc - top)
                part_m[s, h] = top
                part_l[s, h] = p.sum()
                part_o[s, h] = p @ v[:, kvh, :]
        for h in range(hq):
            live = part_m[:, h] != -np.inf
            if not live.any():
                continue
            top = part_m[live, h].max()
            wgt = np.exp(part_m[live, h] - top)
            total = (part_l[live, h] * wgt).sum()
            acc = (part_o[live, h] * wgt[:, None]).sum(axis=0)
            out[b, h] = acc / total if total > 0 else 0.0
    return out


def cuda_closed_form_case():
    """Known answer of tests/cuda_tests.cu:207-262, as decode inputs.

    Page size 2, one kv head, head_dim 4; tokens 0 and 1 live in physical page
    1 (offsets 0, 1) and token 2 in physical page 0 (offset 0); table {1, 0};
    keys (1,0,0,0), (0,1,0,0), (1,1,0,0); values (1,2,3,4), (5,6,7,8),
    (2,4,6,8); the decoding query of head 0 is (1,1,0,0) with scale 1/sqrt(4).
    Expected output: (e^.5 v0 + e^.5 v1 + e^1 v2) / (2 e^.5 + e^1) (:245-247).
    Returns (q, keys, values, tables, lengths, page_size, scale, expected)."""
    page_size, dim = 2, 4
    keys = np.zeros((4, 1, dim))
    values = np.zeros((4, 1, dim))
    token_rows = [1 * page_size + 0, 1 * page_size + 1, 0 * page_size + 0]
    k_tok = np.array([[1, 0, 0, 0], [0, 1, 0, 0], [1, 1, 0, 0]], dtype=np.float64)
    v_tok = np.array([[1, 2, 3, 4], [5, 6, 7, 8], [2, 4, 6, 8]], dtype=np.float64)
    for t, row in enumerate(token_rows):
        keys[row, 0] = k_tok[t]
        values[row, 0] = v_tok[t]
    q = np.array([[[1.0, 1.0, 0.0, 0.0]]])
    tables = np.array([[1, 0]], dtype=np.int32)
    lengths = np.array([3], dtype=np.int32)
    e5, e1 = math.exp(0.5), math.exp(1.0)
    expected = (e5 * v_tok[0] + e5 * v_tok[1] + e1 * v_tok[2]) / (2 * e5 + e1)
    return q, keys, values, tables, lengths, page_size, 0.5, expected


def error_stats(got, expected):
    """(max-abs, mean-abs) error of ``got`` against ``expected`` in float64."""
    diff = np.abs(np.asarray(got, dtype=np.float64) - np.asarray(expected, dtype=np.float64))
    return float(diff.max(initial=0.0)), float(diff.mean()) if diff.size else 0.0
