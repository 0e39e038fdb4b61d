"""instinct_amd — MI355X-native split-K paged decode attention.

Drop-in for the decode-attention path of KavinP21/LLM-Inference ("Instinct"):
``paged_decode_attention`` (python/instinct/backends/metal_kernels.py:164-248)
and the ``DecodeBatch`` / ``KVCache`` conventions that feed it. The compute
runs in hand-written HIP kernels for gfx950 (``csrc/pda_kernels.hip``) behind
the C-ABI ``include/pda.h``.
"""

from .hip_kernels import paged_decode_attention

__all__ = ["paged_decode_attention"]
