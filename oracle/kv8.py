"""CPU oracle for 8-bit K/V — TEST INFRASTRUCTURE ONLY.

Restates, in NumPy, the reference's 8-bit K/V cache (KavinP21/LLM-Inference,
"Instinct"). Only ``tests/`` and ``bench.py``'s CPU-baseline leg may import
it, and only as the checker: the product path (``instinct_amd``) never calls
it.

Functions and the reference lines they follow:

* :func:`quantize` — ``paged_kv.quantize`` (python/instinct/paged_kv.py:50-55):
  per row (the last axis), ``scale = fp16(max(absmax, 1e-4) / 127)`` in
  float32, ``q = clip(round(x / float32(scale)), -127, 127)`` as int8, rounding
  half to even.
* :func:`dequantize` — what the reference's checks compare against
  (tests/test_mlx_engine.py:465-467): ``int8 * scale`` in float32.
* :func:`gather_dequantize` — ``KVCache.gather`` at 8 bits
  (paged_kv.py:285-292): the same product cast to fp16, what prefill
  attention reads.
* The attention itself is the fp16 path's oracle applied to the dequantized
  arena: the Metal kernel multiplies the score by the key's scale and the
  probability that weights the value row by the value's scale
  (metal_kernels.py:52,58 with the ``KEY_SCALE`` / ``VALUE_SCALE``
  substitutions of :134-141), which equals attention over ``int8 * scale``.

Pinning (tests/test_kv8_oracle.py): hand-computed rows (exact scales, ties
rounding to even, the 1e-4 floor, clipping), round-trip error bounds
(|x - dequantize(quantize(x))| <= scale / 2), scale invariance, brute
force on tiny rows, and gather_dequantize against exact rational products
rounded half-to-even to fp16 (every int8 value, normal and subnormal
scales).
"""

from __future__ import annotations

import numpy as np


def quantize(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """``x[..., D]`` -> (int8 ``[..., D]``, fp16 scales ``[...]``)."""
    f32 = np.float32
    x = np.asarray(x).astype(f32)
    scale = (np.maximum(np.abs(x).max(axis=-1), f32(1e-4)) / f32(127.0)).astype(np.float16)
    q = np.rint(x / scale.astype(f32)[..., None])
    return np.clip(q, -127, 127).astype(np.int8), scale


def dequantize(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """int8 rows times their fp16 scales, float32."""
    return q.astype(np.float32) * scale.astype(np.float32)[..., None]


def gather_dequantize(q: np.ndarray, scale: np.ndarray) -> np.ndarray:
    """The rows the reference's 8-bit ``KVCache.gather`` hands to prefill
    attention (python/instinct/paged_kv.py:285-292): ``int8 * scale`` in
    float32, cast to the model dtype (fp16). The float32 product is exact
    (8-bit times 11-bit significands), so this is one rounding to fp16."""
    return dequantize(q, scale).astype(np.float16)


def quantize_brute(row) -> tuple[list[int], float]:
    """One row, element by element, in float32 steps."""
    f32 = np.float32
    top = f32(0)
    for value in row:
        top = max(top, abs(f32(value)))
    scale = np.float16(max(top, f32(1e-4)) / f32(127.0))
    out = []
    for value in row:
        r = np.rint(f32(value) / f32(scale))
        out.append(int(min(127, max(-127, r))))
    return out, float(scale)
