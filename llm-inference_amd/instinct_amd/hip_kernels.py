"""Paged decode attention on MI355X, behind the reference's operator API.

:func:`paged_decode_attention` keeps the signature and meaning of the
reference's ``paged_decode_attention`` (python/instinct/backends/
metal_kernels.py:164-248) with torch tensors on the GPU in place of MLX
arrays: queries ``[batch, q_heads, head_dim]``, a layer's whole K/V arena,
page tables ``[batch, width]`` int32 and lengths ``[batch]`` int32 (the new
key included). It returns ``[batch, q_heads, head_dim]`` in the queries'
dtype (fp16). The arena is either the reference's ``[rows, kv_heads,
head_dim]`` (3-D) or the page-tile layout ``[pages, kv_heads, page_size,
head_dim]`` (4-D, see :mod:`instinct_amd.paged_kv`), which the kernel reads
as whole contiguous tiles.

The work happens in hand-written HIP kernels (libpda.so, see
``csrc/pda_kernels.hip``) called through the C-ABI of ``include/pda.h``; this
module only validates, allocates the output and the split workspace, and
passes device pointers and the current stream.
"""

from __future__ import annotations

import ctypes
from typing import Any

import torch

from . import _lib

_workspaces: dict[tuple[int, int], torch.Tensor] = {}


def workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A cached, 256-byte aligned device workspace of at least ``nbytes``,
    grown on demand and shared by calls of any shape (it holds nothing
    between calls)."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, 0)
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        size = max(nbytes, 1 << 20)
        if buf is not None:
            size = max(size, 2 * buf.numel())
        buf = torch.empty(size, dtype=torch.uint8, device=device)
        _workspaces[key] = buf
    return buf


def paged_decode_attention(
    queries: torch.Tensor,
    keys: torch.Tensor,
    values: torch.Tensor,
    tables: torch.Tensor,
    lengths: torch.Tensor,
    *,
    page_size: int,
    longest: int,
    scale: float,
    window: int = 0,
    softcap: float = 0.0,
    scales: tuple[Any, Any] | None = None,
    split_pages: int = 0,
    out: torch.Tensor | None = None,
    passes: str = "both",
) -> torch.Tensor:
    """Attention for one new token per sequence over its paged keys
    (metal_kernels.py:164-186). ``split_pages`` is the fewest pages a wave
    reads before the batch is spread over fewer waves (0 = default); the
    result does not depend on it. ``passes`` = "split" or "merge" launches
    one of the two kernels only (the output is complete after the merge)."""
    if scales is not None:
        raise NotImplementedError("8-bit K/V (scales) has no MI355X kernel yet")
    batch, q_heads, head_dim = (int(n) for n in queries.shape)
    kv_heads = int(keys.shape[1])
    if keys.dim() == 3:
        layout, arena_rows, width = _lib.PDA_LAYOUT_ROWS, int(keys.shape[0]), int(keys.shape[2])
    elif keys.dim() == 4:
        if int(keys.shape[2]) != page_size:
            raise ValueError("page-tile arena must be [pages, kv_heads, page_size, head_dim]")
        layout = _lib.PDA_LAYOUT_PAGES
        arena_rows, width = int(keys.shape[0]) * page_size, int(keys.shape[3])
    else:
        raise ValueError("keys must be [rows, kv_heads, head_dim] or "
                         "[pages, kv_heads, page_size, head_dim]")
    if q_heads % kv_heads:
        raise ValueError("query heads must be a multiple of kv heads")
    for name, t in (("queries", queries), ("keys", keys), ("values", values)):
        if t.dtype != torch.float16:
            raise TypeError(f"{name} must be float16, got {t.dtype}")
        if not t.is_cuda:
            raise ValueError(f"{name} must be on a GPU")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if tuple(keys.shape) != tuple(values.shape) or width != head_dim:
        raise ValueError("keys and values must have the same shape and head_dim")
    if tables.dtype != torch.int32 or lengths.dtype != torch.int32:
        raise TypeError("tables and lengths must be int32")
    if tables.dim() != 2 or tables.shape[0] != batch or lengths.shape != (batch,):
        raise ValueError("tables must be [batch, width] and lengths [batch]")
    tables = tables.contiguous()
    lengths = lengths.contiguous()
    device = queries.device
    if out is None:
        out = torch.empty_like(queries)
    if batch == 0:
        return out
    stride = int(tables.shape[1])
    need = _lib.workspace_bytes(batch, q_heads, kv_heads, head_dim, page_size, stride,
                                int(longest), int(window), int(split_pages))
    ws = workspace(device, need)
    stream = torch.cuda.current_stream(device).cuda_stream
    entry = {"both": "pda_paged_decode_attention", "split": "pda_decode_split",
             "merge": "pda_decode_merge"}[passes]
    rc = getattr(_lib.library(), entry)(
        queries.data_ptr(), keys.data_ptr(), values.data_ptr(), tables.data_ptr(),
        lengths.data_ptr(), out.data_ptr(), batch, q_heads, kv_heads, head_dim,
        int(page_size), stride, arena_rows, layout, int(longest), float(scale),
        int(window), float(softcap), int(split_pages), ws.data_ptr(),
        ws.numel(), ctypes.c_void_p(stream))
    _lib.check(rc)
    return out
