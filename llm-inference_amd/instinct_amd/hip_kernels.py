"""Paged decode attention and the K/V append on MI355X, behind the
reference's operator API.

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

The step before it, the rotary embedding of the new queries and keys
(``DecodeBatch.rope``, python/instinct/batches.py:195-201 ->
backends/portable.py:88-132) and the write of the new keys and values into
the arena (``KVCache.write``, paged_kv.py:278-283), is :func:`rope_append`
(one launch), with :func:`rope` and :func:`kv_write` as its two halves.

The work happens in hand-written HIP kernels (libpda.so, see
``csrc/pda_kernels.hip`` and ``csrc/pda_append.hip``) called through the
C-ABI of ``include/pda.h``; this module only validates, allocates outputs and
the split workspace, and passes device pointers and the current stream.
"""

from __future__ import annotations

import ctypes
import os
from collections import OrderedDict
from typing import Any

import numpy as np
import torch

from . import _lib

# Cached workspaces, most recently used last: at most _WORKSPACE_STREAMS
# streams keep one; the least recently used one is dropped past that.
_workspaces: "OrderedDict[tuple[int, int], torch.Tensor]" = OrderedDict()
_WORKSPACE_STREAMS = 4


def new_workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """A workspace for the library's calls: ``nbytes`` of device memory (it
    needs no initialisation; the caching allocator's blocks are 512-byte
    aligned)."""
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def stream_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A cached, 256-byte aligned device workspace of at least ``nbytes``
    for the current stream of ``device``, grown on demand and
    shared by calls of any shape on that stream (calls on one stream never
    overlap). Calls on different streams get different buffers; the cache
    keeps those of the four streams used last (a dropped buffer goes back to
    the caching allocator, which only reuses it for work ordered after it on
    its stream).

    Growing replaces the stream's buffer; the caching allocator only reuses
    the old one for work ordered after the replacement on the same stream.
    Code that records a workspace address for later (a captured graph) must
    pass a workspace it owns instead (``workspace=`` of the calls), as
    :class:`instinct_amd.step.DecodeStepGraph` does."""
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, int(torch.cuda.current_stream(index).cuda_stream))
    buf = _workspaces.get(key)
    if buf is None or buf.numel() < nbytes:
        size = max(nbytes, 1 << 20)
        if buf is not None:
            size = max(size, 2 * buf.numel())
        buf = new_workspace(size, device)
    _workspaces[key] = buf
    _workspaces.move_to_end(key)
    while len(_workspaces) > _WORKSPACE_STREAMS:
        _workspaces.popitem(last=False)
    return buf


def _given_workspace(ws: torch.Tensor, device: torch.device, nbytes: int) -> torch.Tensor:
    """A caller's workspace: a contiguous uint8 tensor on ``device``, 256-byte
    aligned, of at least ``nbytes``."""
    if ws.dtype != torch.uint8 or not ws.is_contiguous() or ws.device != device:
        raise ValueError("workspace must be a contiguous uint8 tensor on the queries' device")
    if ws.numel() < nbytes:
        raise ValueError(f"workspace of {nbytes} bytes needed, {ws.numel()} given")
    if ws.data_ptr() % 256:
        raise ValueError("workspace must be 256-byte aligned")
    return ws


def decode_kernel_names(q_heads: int, kv_heads: int, head_dim: int, *, bits: int = 16,
                        bf16: bool = False, batch: int = 0, longest: int = 0,
                        page_size: int = 16, table_width: int = 0, window: int = 0,
                        split_pages: int = 0) -> dict[str, Any]:
    """The kernels a decode call of this shape launches, as the library
    reports them (``pda_decode_describe``, the dispatch the call itself runs):
    the split kernel ``<D, G, Q8, BF, GEN, MF>`` and the merge kernel
    ``<D, G, BF, GEN>`` or its row-sliced form (None in local mode, where one
    workgroup per unit merges in LDS), whether the matrix cores run it, the
    query heads one unit serves, the units per kv head (each reads the kv
    head's K/V once), the ring depth and the grid. Local mode and the merge
    shape depend on the batch, the longest length and the table width;
    ``batch`` 0 reports the shape's split kernel only (``merge`` None, no
    local mode)."""
    width = table_width or -(-max(longest, 1) // page_size)
    info = _lib.describe(max(batch, 1), q_heads, kv_heads, head_dim, page_size, width,
                         longest, window, split_pages, kv_bits=bits, bf16=bf16)
    real = batch > 0
    return {"split": info["split_kernel"],
            "merge": info["merge_kernel"] if real else None,
            "local": real and bool(info["local"]),
            "merge_row_sliced": real and info["merge"] == 2,
            "matrix_cores": bool(info["matrix_cores"]),
            "heads_per_unit": info["unit_heads"],
            "head_groups_per_kv_head": info["units_per_kv_head"],
            "ring": info["ring"], "split_waves": info["split_waves"],
            "grid_groups": info["grid_groups"],
            "merge_waves": info["merge_waves"] if real else 0}


def decode_workspace_bytes(queries_shape: tuple[int, int, int], keys: torch.Tensor, *,
                           page_size: int, table_width: int, longest: int, window: int = 0,
                           split_pages: int = 0) -> int:
    """Bytes of workspace :func:`paged_decode_attention` needs for this shape
    (``pda_workspace_bytes``)."""
    batch, q_heads, head_dim = (int(n) for n in queries_shape)
    return _lib.workspace_bytes(batch, q_heads, int(keys.shape[1]), head_dim, int(page_size),
                                int(table_width), int(longest), int(window), int(split_pages))


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
    workspace: torch.Tensor | None = None,
    deterministic: bool = True,
) -> torch.Tensor:
    """Attention for one new token per sequence over its paged keys
    (metal_kernels.py:164-186). ``split_pages`` is the fewest pages a wave
    reads before the batch is spread over fewer waves (0 = default); the
    result does not depend on it. ``passes`` = "split" or "merge" launches
    one of the two kernels only (the output is complete after the merge).
    ``workspace``: a uint8 device tensor the caller owns (at least
    :func:`decode_workspace_bytes`), else the stream's cached one.
    ``deterministic`` (default): fixed split points (the library's default,
    flags 0), so repeated calls on the same inputs give bitwise-identical
    outputs, as the reference's fixed split ranges do
    (metal_kernels.py:32-36). ``deterministic=False`` passes
    ``PDA_DECODE_RACING``: the two waves that share a stretch of pages split
    it wherever they meet (the faster takes more), so the last bits of a
    sequence's output can differ from call to call (within the parity bar).
    Any ``head_dim`` up to 512 and any ``page_size`` are accepted, as by
    the reference op (metal_kernels.py:28-30,204).

    ``scales`` = (key_scales, value_scales) selects 8-bit K/V
    (metal_kernels.py:134-141): ``keys``/``values`` are int8 arenas and the
    scales fp16, one per (row, kv head): ``[rows, kv_heads]`` beside a row
    arena, ``[pages, kv_heads, page_size]`` beside a page-tile arena. The
    queries are fp16 or bf16 (a bf16 model's 8-bit cache) and the output
    takes their dtype, as the reference's quantized kernel does
    (metal_kernels.py:196-206)."""
    q8 = scales is not None
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
    # bf16 queries select a bf16 output and, at 16 bits, bf16 K/V (the model
    # dtype of bf16 models); 8-bit K/V take fp16 or bf16 queries.
    bf16 = queries.dtype == torch.bfloat16
    q_dtype = torch.bfloat16 if bf16 else torch.float16
    kv_dtype = torch.int8 if q8 else q_dtype
    for name, t, dtype in (("queries", queries, q_dtype), ("keys", keys, kv_dtype),
                           ("values", values, kv_dtype)):
        if t.dtype != dtype:
            raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
        if not t.is_cuda:
            raise ValueError(f"{name} must be on a GPU")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if q8:
        scale_shape = ((int(keys.shape[0]), kv_heads) if keys.dim() == 3
                       else (int(keys.shape[0]), kv_heads, page_size))
        for name, t in zip(("key_scales", "value_scales"), scales):
            if t.dtype != torch.float16 or tuple(t.shape) != scale_shape:
                raise ValueError(f"{name} must be float16 {list(scale_shape)}")
            if not t.is_cuda or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous GPU tensor")
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
    ws = (stream_workspace(device, need) if workspace is None
          else _given_workspace(workspace, device, need))
    stream = torch.cuda.current_stream(device).cuda_stream
    if out.dtype != q_dtype or tuple(out.shape) != tuple(queries.shape) or not out.is_cuda:
        raise ValueError("out must match the queries' shape and dtype")
    entry = {"both": "pda_paged_decode_attention", "split": "pda_decode_split",
             "merge": "pda_decode_merge"}[passes] + ("_q8" if q8 else "") + ("_bf16" if bf16 else "")
    extra = (scales[0].data_ptr(), scales[1].data_ptr()) if q8 else ()
    rc = getattr(_lib.library(), entry)(
        queries.data_ptr(), keys.data_ptr(), values.data_ptr(), *extra, tables.data_ptr(),
        lengths.data_ptr(), out.data_ptr(), batch, q_heads, kv_heads, head_dim,
        int(page_size), stride, arena_rows, layout, int(longest), float(scale),
        int(window), float(softcap), int(split_pages),
        0 if deterministic else _lib.PDA_DECODE_RACING, ws.data_ptr(),
        ws.numel(), ctypes.c_void_p(stream))
    _lib.check(rc)
    return out


# ---------------------------------------------------------------------------
# Rotary embedding and K/V append.

_inv_freq_cache: dict[tuple, torch.Tensor] = {}


def rope_inv_freq(dims: int, *, base: float | None = None, freqs: Any = None,
                  device: torch.device | str = "cuda") -> torch.Tensor:
    """float32 ``[dims // 2]`` inverse frequencies on ``device``, as
    ``portable._rope_plain`` forms them (portable.py:117-121):
    ``base ** (-arange(0, dims // 2) * 2 / dims)`` in float32, or
    ``1 / freqs`` (an infinite frequency leaves its pair unrotated). The
    kernel's angle is float32(position) * inv_freq[i]."""
    if dims <= 0 or dims % 2:
        raise ValueError("rope dims must be a positive even number")
    half = dims // 2
    f32 = np.float32
    if freqs is None:
        if base is None:
            raise ValueError("rope needs base or freqs")
        key = ("base", dims, float(base))
    else:
        freqs = np.asarray(freqs.cpu() if isinstance(freqs, torch.Tensor) else freqs,
                           dtype=f32)
        if freqs.shape[0] < half:
            raise ValueError("freqs must hold dims // 2 entries")
        key = ("freqs", dims, freqs[:half].tobytes())
    device = torch.device(device)
    key = key + (str(device),)
    table = _inv_freq_cache.get(key)
    if table is None:
        if freqs is None:
            exponent = (-np.arange(0, half, dtype=f32) * f32(2)) / f32(dims)
            host = np.power(f32(base), exponent, dtype=f32)
        else:
            with np.errstate(divide="ignore"):
                host = (f32(1) / freqs[:half]).astype(f32)
        table = torch.as_tensor(host, device=device)
        _inv_freq_cache[key] = table
    return table


def _check_half(name: str, t: torch.Tensor, dims: int,
                dtype: torch.dtype = torch.float16) -> None:
    """A contiguous GPU tensor of ``dims`` dimensions in a 16-bit float type
    (fp16, or bf16 where the caller asks for it)."""
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {str(dtype).replace('torch.', '')}, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be on a GPU")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.dim() != dims:
        raise ValueError(f"{name} must have {dims} dimensions")


def _arena_geometry(keys: torch.Tensor, page_size: int) -> tuple[int, int, int, int]:
    """(layout, arena_rows, kv_heads, head_dim) of a K/V arena."""
    if keys.dim() == 3:
        return _lib.PDA_LAYOUT_ROWS, int(keys.shape[0]), int(keys.shape[1]), int(keys.shape[2])
    if keys.dim() == 4:
        if int(keys.shape[2]) != page_size:
            raise ValueError("page-tile arena must be [pages, kv_heads, page_size, head_dim]")
        return (_lib.PDA_LAYOUT_PAGES, int(keys.shape[0]) * page_size, int(keys.shape[1]),
                int(keys.shape[3]))
    raise ValueError("arena must be [rows, kv_heads, head_dim] or "
                     "[pages, kv_heads, page_size, head_dim]")


def _launch_rope_append(q, q_out, k, v, keys, values, positions, rows, *, n, q_heads,
                        kv_heads, head_dim, page_size, arena_rows, layout, dims, table,
                        device, scales=None, bf16=False) -> None:
    stream = torch.cuda.current_stream(device).cuda_stream
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    lib = _lib.library()
    head = (ptr(q), ptr(q_out), ptr(k), ptr(v), ptr(keys), ptr(values))
    tail = (ptr(positions), ptr(rows), int(n), int(q_heads), int(kv_heads), int(head_dim),
            int(page_size), int(arena_rows), int(layout), int(dims), ptr(table),
            ctypes.c_void_p(stream))
    if scales is None:
        entry = lib.pda_rope_append_bf16 if bf16 else lib.pda_rope_append
        rc = entry(*head, *tail)
    else:
        rc = lib.pda_rope_append_q8(*head, ptr(scales[0]), ptr(scales[1]), *tail)
    _lib.check(rc)


def _int32_vector(name: str, t: torch.Tensor, n: int) -> torch.Tensor:
    if t.dtype != torch.int32 or t.shape != (n,):
        raise ValueError(f"{name} must be int32 [{n}]")
    if not t.is_cuda:
        raise ValueError(f"{name} must be on a GPU")
    return t.contiguous()


def rope_append(q: torch.Tensor | None, k: torch.Tensor, v: torch.Tensor,
                keys: torch.Tensor, values: torch.Tensor, positions: torch.Tensor,
                rows: torch.Tensor, *, page_size: int, dims: int, base: float | None = None,
                freqs: Any = None, q_out: torch.Tensor | None = None,
                scales: tuple[torch.Tensor, torch.Tensor] | None = None
                ) -> torch.Tensor | None:
    """Rotate this step's queries and keys and write the rotated keys and the
    values into the arena, in one launch: the reference's
    ``q = batch.rope(q, dims, ...)``, ``k = batch.rope(k, dims, ...)``
    (batches.py:195-201) then ``cache.write(layer, rows, k, v)``
    (batches.py:203-207, paged_kv.py:278-283).

    ``q`` ``[n, q_heads, D]`` (or None), ``k``, ``v`` ``[n, kv_heads, D]``
    fp16, or all bf16 (bf16 models: the rotation is rounded to bf16);
    ``keys``/``values`` one layer's arena in either layout, of that dtype;
    ``positions`` and ``rows`` int32 ``[n]`` (rows outside the arena are not
    written). ``dims`` = 0 writes without rotation. Returns the rotated
    queries (``q_out``, new unless given; ``q_out`` may be ``q``).

    ``scales`` = (key_scales, value_scales) writes 8-bit K/V: ``keys`` and
    ``values`` are int8 arenas, the rotated keys and the values are quantized
    per (row, kv head) as ``paged_kv.quantize`` does (paged_kv.py:50-55);
    the 8-bit write takes fp16 ``q``, ``k`` and ``v``."""
    n, kv_heads, head_dim = (int(x) for x in k.shape)
    layout, arena_rows, a_heads, a_dim = _arena_geometry(keys, page_size)
    bf16 = k.dtype == torch.bfloat16 and scales is None
    dtype = torch.bfloat16 if bf16 else torch.float16
    for name, t, d in (("k", k, 3), ("v", v, 3)):
        _check_half(name, t, d, dtype)
    if scales is None:
        for name, t in (("keys", keys), ("values", values)):
            _check_half(name, t, keys.dim(), dtype)
    else:
        scale_shape = ((arena_rows, kv_heads) if layout == _lib.PDA_LAYOUT_ROWS
                       else (arena_rows // page_size, kv_heads, page_size))
        for name, t in (("keys", keys), ("values", values)):
            if t.dtype != torch.int8 or not t.is_cuda or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous int8 GPU tensor")
        for name, t in zip(("key_scales", "value_scales"), scales):
            if (t.dtype != torch.float16 or tuple(t.shape) != scale_shape or not t.is_cuda
                    or not t.is_contiguous()):
                raise ValueError(f"{name} must be a contiguous float16 GPU tensor "
                                 f"{list(scale_shape)}")
    if tuple(v.shape) != tuple(k.shape) or tuple(values.shape) != tuple(keys.shape):
        raise ValueError("k/v and keys/values must have matching shapes")
    if (a_heads, a_dim) != (kv_heads, head_dim):
        raise ValueError("k does not match the arena's kv_heads and head_dim")
    q_heads = 0
    if q is not None:
        _check_half("q", q, 3, dtype)
        if int(q.shape[0]) != n or int(q.shape[2]) != head_dim:
            raise ValueError("q must be [n, q_heads, head_dim]")
        q_heads = int(q.shape[1])
        if q_out is None:
            q_out = torch.empty_like(q)
        _check_half("q_out", q_out, 3, dtype)
        if q_out.shape != q.shape:
            raise ValueError("q_out must have q's shape")
    rows = _int32_vector("rows", rows, n)
    if n == 0:
        return q_out
    table = None
    if dims:
        positions = _int32_vector("positions", positions, n)
        table = rope_inv_freq(dims, base=base, freqs=freqs, device=k.device)
    _launch_rope_append(q, q_out if q is not None else None, k, v, keys, values,
                        positions if dims else None, rows, n=n, q_heads=q_heads,
                        kv_heads=kv_heads, head_dim=head_dim, page_size=page_size,
                        arena_rows=arena_rows, layout=layout, dims=dims, table=table,
                        device=k.device, scales=scales, bf16=bf16)
    return q_out


def rope(x: torch.Tensor, positions: torch.Tensor, dims: int, *, base: float | None = None,
         freqs: Any = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """``DecodeBatch.rope`` (batches.py:195-201): rotate ``[n, heads, D]`` by
    one position per token (non-traditional RoPE, portable.py:88-132);
    ``x`` fp16 or bf16, the result in ``x``'s dtype."""
    bf16 = x.dtype == torch.bfloat16
    _check_half("x", x, 3, torch.bfloat16 if bf16 else torch.float16)
    n, heads, head_dim = (int(s) for s in x.shape)
    if out is None:
        out = torch.empty_like(x)
    positions = _int32_vector("positions", positions, n)
    table = rope_inv_freq(dims, base=base, freqs=freqs, device=x.device)
    _launch_rope_append(x, out, None, None, None, None, positions, None, n=n, q_heads=heads,
                        kv_heads=0, head_dim=head_dim, page_size=0, arena_rows=0,
                        layout=0, dims=dims, table=table, device=x.device, bf16=bf16)
    return out


def kv_write(keys: torch.Tensor, values: torch.Tensor, rows: torch.Tensor, k: torch.Tensor,
             v: torch.Tensor, *, page_size: int,
             scales: tuple[torch.Tensor, torch.Tensor] | None = None) -> None:
    """``KVCache.write`` (paged_kv.py:278-283): scatter ``k``, ``v``
    ``[n, kv_heads, D]`` into arena rows ``rows`` in place, either layout
    (quantized into int8 arenas and their scales when ``scales`` is given)."""
    rope_append(None, k, v, keys, values, rows, rows, page_size=page_size, dims=0,
                scales=scales)


def pack_decode_step(seq_tables: torch.Tensor, slots: torch.Tensor, positions: torch.Tensor, *,
                     width: int, page_size: int, tables: torch.Tensor | None = None,
                     lengths: torch.Tensor | None = None, rows: torch.Tensor | None = None
                     ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``DecodeBatch``'s per-step packing (batches.py:148-179) on the device:
    from the resident per-slot page tables ``seq_tables [num_slots, stride]``
    and the step's ``slots``/``positions`` (int32 ``[B]``), the packed tables
    ``[B, width]`` (0 past the new token's page), ``lengths = positions + 1``
    and the write rows. Outputs may be given (static buffers of a graph)."""
    if seq_tables.dtype != torch.int32 or seq_tables.dim() != 2 or not seq_tables.is_cuda:
        raise ValueError("seq_tables must be an int32 [num_slots, stride] GPU tensor")
    seq_tables = seq_tables.contiguous()
    batch = int(slots.shape[0])
    slots = _int32_vector("slots", slots, batch)
    positions = _int32_vector("positions", positions, batch)
    dev = seq_tables.device
    if tables is None:
        tables = torch.empty((batch, width), dtype=torch.int32, device=dev)
    if lengths is None:
        lengths = torch.empty(batch, dtype=torch.int32, device=dev)
    if rows is None:
        rows = torch.empty(batch, dtype=torch.int32, device=dev)
    if tuple(tables.shape) != (batch, width) or lengths.shape != (batch,) or rows.shape != (batch,):
        raise ValueError("output shapes do not match the step")
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = _lib.library().pda_pack_decode_step(
        seq_tables.data_ptr(), int(seq_tables.shape[1]), int(seq_tables.shape[0]),
        slots.data_ptr(), positions.data_ptr(), batch, int(width), int(page_size),
        tables.data_ptr(), lengths.data_ptr(), rows.data_ptr(), ctypes.c_void_p(stream))
    _lib.check(rc)
    return tables, lengths, rows


def image_spans(images: Any, device: torch.device) -> torch.Tensor | None:
    """Image spans as the prefill call takes them: an int32 ``[n, 2]`` GPU
    tensor of [begin, end) positions (None for none), from (at, length)
    pairs or such a tensor."""
    if isinstance(images, torch.Tensor):
        if images.numel() == 0:
            return None
        if images.dtype != torch.int32 or images.dim() != 2 or images.shape[1] != 2:
            raise ValueError("image spans must be an int32 [n, 2] tensor")
        return images.to(device).contiguous()
    pairs = [(int(at), int(at) + int(length)) for at, length in images if int(length) > 0]
    if not pairs:
        return None
    return torch.tensor(pairs, dtype=torch.int32, device=device)


def paged_prefill_attention(queries: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                            table: torch.Tensor, *, start: int, page_size: int, scale: float,
                            window: int = 0, softcap: float = 0.0, splits: int = 0,
                            scales: tuple[Any, Any] | None = None, images: Any = (),
                            out: torch.Tensor | None = None,
                            workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Attention of one prompt chunk (``PrefillBatch.attend``,
    batches.py:84-132): ``queries`` ``[count, q_heads, D]`` at positions
    ``start ..`` over the sequence's keys in the arena (either layout, the
    chunk's own keys already written), ``table`` the sequence's int32 pages.
    Causal, with the window and softcap of the decode call. ``splits`` 0
    lets the library split long key ranges to fill the GPU; > 0 forces a
    count (results do not depend on it beyond rounding). ``scales`` =
    (key_scales, value_scales) selects an 8-bit cache (int8 arenas, fp16
    scales shaped as for :func:`paged_decode_attention`), dequantized as the
    reference's gather does (paged_kv.py:285-292). ``images``: (at, length)
    spans of image tokens, or an int32 GPU tensor ``[n, 2]`` of [begin, end)
    positions; a query inside one also sees the span's later keys
    (batches.py:107-118). bf16 queries with bf16 arenas (bf16 models) give a
    bf16 output; the 8-bit cache takes fp16 queries. ``workspace``: a uint8
    device tensor the caller owns (at least the ``pda_prefill_workspace_bytes``
    of the call), else the stream's cached one."""
    q8 = scales is not None
    bf16 = queries.dtype == torch.bfloat16 and not q8
    dtype = torch.bfloat16 if bf16 else torch.float16
    _check_half("queries", queries, 3, dtype)
    count, q_heads, head_dim = (int(x) for x in queries.shape)
    layout, arena_rows, kv_heads, a_dim = _arena_geometry(keys, page_size)
    for name, t in (("keys", keys), ("values", values)):
        if q8:
            if t.dtype != torch.int8 or not t.is_cuda or not t.is_contiguous():
                raise TypeError(f"{name} must be a contiguous int8 GPU tensor")
        else:
            _check_half(name, t, keys.dim(), dtype)
    if q8:
        scale_shape = tuple(keys.shape[:-1])
        for name, t in zip(("key_scales", "value_scales"), scales):
            if t.dtype != torch.float16 or tuple(t.shape) != scale_shape:
                raise ValueError(f"{name} must be float16 {list(scale_shape)}")
            if not t.is_cuda or not t.is_contiguous():
                raise ValueError(f"{name} must be a contiguous GPU tensor")
    if tuple(values.shape) != tuple(keys.shape) or a_dim != head_dim:
        raise ValueError("keys and values must match the queries' head_dim")
    if q_heads % kv_heads:
        raise ValueError("query heads must be a multiple of kv heads")
    if table.dtype != torch.int32 or table.dim() != 1 or not table.is_cuda:
        raise ValueError("table must be an int32 GPU vector")
    if table.shape[0] == 0 and count > 0:
        raise ValueError("the table holds no pages")
    table = table.contiguous()
    if out is None:
        out = torch.empty_like(queries)
    else:
        _check_half("out", out, 3, dtype)
        if tuple(out.shape) != tuple(queries.shape):
            raise ValueError("out must have the queries' shape")
    if count == 0:
        return out
    _, need = _lib.prefill_workspace_bytes(int(start), count, q_heads, head_dim, int(window),
                                           int(splits))
    ws = None
    if need:
        ws = (stream_workspace(queries.device, need) if workspace is None
              else _given_workspace(workspace, queries.device, need))
    stream = torch.cuda.current_stream(queries.device).cuda_stream
    spans = image_spans(images, queries.device)
    entry = "pda_paged_prefill_attention" + ("_q8" if q8 else "_bf16" if bf16 else "")
    extra = (scales[0].data_ptr(), scales[1].data_ptr()) if q8 else ()
    rc = getattr(_lib.library(), entry)(
        queries.data_ptr(), keys.data_ptr(), values.data_ptr(), *extra, table.data_ptr(),
        int(table.shape[0]), int(start), count, out.data_ptr(), q_heads, kv_heads, head_dim,
        int(page_size), arena_rows, layout, float(scale), int(window), float(softcap),
        spans.data_ptr() if spans is not None else None,
        int(spans.shape[0]) if spans is not None else 0,
        int(splits), ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0, ctypes.c_void_p(stream))
    _lib.check(rc)
    return out
