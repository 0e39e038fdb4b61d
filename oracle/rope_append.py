"""CPU oracle for the K/V append with rotary embedding — TEST INFRASTRUCTURE ONLY.

Restates, in NumPy, what the reference does between the K/V projections and
the paged attention call of a decode step (KavinP21/LLM-Inference,
"Instinct"). Only ``tests/`` and ``bench.py``'s CPU-baseline leg may import
it, and only as the checker: the product path (``instinct_amd``) never calls
it.

Functions and the reference lines they follow:

* :func:`inv_freq` — the inverse frequencies of ``portable._rope_plain``
  (python/instinct/backends/portable.py:117-121): ``base ** (-arange(0, half)
  * 2 / dims)`` in float32, or ``1 / freqs`` when explicit frequencies are
  given (``freqs`` = inf gives 0: the pair is not rotated).
* :func:`rope` — ``portable._rope_plain`` (portable.py:115-132) for one
  position per token (``DecodeBatch.rope``, python/instinct/batches.py:
  195-201): angle = float32(position) * inv_freq in float32; element i pairs
  with i + dims / 2: ``[x1 cos - x2 sin, x2 cos + x1 sin]`` in float32,
  elements from ``dims`` on unchanged, cast back to the input dtype.
* :func:`write_rows` — ``KVCache.write`` (python/instinct/paged_kv.py:278-283):
  scatter rows into the arena, here in either device layout (rows
  ``[rows, kv_heads, D]`` or page tiles ``[pages, kv_heads, P, D]``); rows
  outside the arena are skipped (the library's documented behaviour).
* :func:`rope_append` — the two together, in the order of
  ``DecodeBatch.attend`` (batches.py:203-207) after the model's
  ``batch.rope`` calls (e.g. backends/dense.py:99-102).
* :func:`rope_complex` — an independent float64 formulation (complex
  multiplication by e^(i angle)), used to pin the sign convention and the
  pairing.

Pinning (tests/test_rope_oracle.py): the known answers of the reference's
CUDA test (tests/cuda_tests.cu:155-206: position 0 is the identity; position
1, head_dim 4, base 10000 gives ``first cos 1 - second sin 1``; the rotated
key and the value land at the token's cache row), the complex formulation,
rotation invariants (pair norms; the score of rotated q and k depends only on
the position difference; rotations compose), and brute-force loops on tiny
inputs.
"""

from __future__ import annotations

import numpy as np

LAYOUTS = ("rows", "pages")


def inv_freq(dims: int, *, base: float | None = None, freqs=None) -> np.ndarray:
    """float32 ``[dims // 2]`` inverse frequencies (portable.py:117-121)."""
    half = dims // 2
    f32 = np.float32
    if freqs is None:
        if base is None:
            raise ValueError("rope needs base or freqs")
        exponent = (-np.arange(0, half, dtype=f32) * f32(2)) / f32(dims)
        return np.power(f32(base), exponent, dtype=f32)
    with np.errstate(divide="ignore"):
        return (f32(1) / np.asarray(freqs, dtype=f32)[:half]).astype(f32)


def rope(x: np.ndarray, positions: np.ndarray, dims: int, inverse: np.ndarray) -> np.ndarray:
    """Rotate ``[n, heads, D]`` (fp16) by one position per token
    (portable.py:115-132); returns fp16."""
    f32 = np.float32
    half = dims // 2
    values = x.astype(f32)
    angles = positions.astype(f32)[:, None] * inverse[None, :half].astype(f32)  # [n, half]
    cos = np.cos(angles).astype(f32)[:, None, :]
    sin = np.sin(angles).astype(f32)[:, None, :]
    first, second = values[..., :half], values[..., half:dims]
    out = values.copy()
    out[..., :half] = first * cos - second * sin
    out[..., half:dims] = second * cos + first * sin
    return out.astype(x.dtype)


def rope_complex(x: np.ndarray, positions: np.ndarray, dims: int, inverse: np.ndarray) -> np.ndarray:
    """float64 restatement: pair (x[i], x[i + dims/2]) as the complex number
    x[i] + 1j x[i + dims/2], multiplied by exp(1j * position * inv_freq[i])."""
    half = dims // 2
    values = x.astype(np.float64)
    z = values[..., :half] + 1j * values[..., half:dims]
    angles = positions.astype(np.float64)[:, None] * inverse[None, :half].astype(np.float64)
    z = z * np.exp(1j * angles)[:, None, :]
    out = values.copy()
    out[..., :half] = z.real
    out[..., half:dims] = z.imag
    return out


def arena_slots(rows: np.ndarray, page_size: int):
    rows = np.asarray(rows, dtype=np.int64)
    return rows // page_size, rows % page_size


def write_rows(arena: np.ndarray, rows: np.ndarray, data: np.ndarray, *, layout: str,
               page_size: int) -> None:
    """Scatter ``data[t]`` (``[n, kv_heads, D]``) into arena row ``rows[t]``
    in place (paged_kv.py:278-283); rows outside the arena are skipped."""
    if layout not in LAYOUTS:
        raise ValueError(layout)
    total = arena.shape[0] if layout == "rows" else arena.shape[0] * page_size
    rows = np.asarray(rows, dtype=np.int64)
    keep = (rows >= 0) & (rows < total)
    if layout == "rows":
        arena[rows[keep]] = data[keep]
    else:
        page, slot = arena_slots(rows[keep], page_size)
        arena[page, :, slot] = data[keep]


def rope_append(q, k, v, k_arena, v_arena, positions, rows, *, dims, inverse, layout,
                page_size):
    """Rotated queries, and the arenas with the rotated keys and the values
    written at ``rows`` (copies; the inputs are not modified)."""
    q_out = rope(q, positions, dims, inverse) if q is not None else None
    k_arena = k_arena.copy()
    v_arena = v_arena.copy()
    k_rot = rope(k, positions, dims, inverse)
    write_rows(k_arena, rows, k_rot, layout=layout, page_size=page_size)
    write_rows(v_arena, rows, v, layout=layout, page_size=page_size)
    return q_out, k_arena, v_arena


def rope_brute(x: np.ndarray, positions, dims: int, inverse) -> np.ndarray:
    """Element-by-element Python loops over a tiny input (float64)."""
    import math

    n, heads, d = x.shape
    half = dims // 2
    out = x.astype(np.float64).copy()
    for t in range(n):
        for h in range(heads):
            for i in range(half):
                a = float(positions[t]) * float(inverse[i])
                x1, x2 = float(x[t, h, i]), float(x[t, h, i + half])
                out[t, h, i] = x1 * math.cos(a) - x2 * math.sin(a)
                out[t, h, i + half] = x2 * math.cos(a) + x1 * math.sin(a)
    return out
