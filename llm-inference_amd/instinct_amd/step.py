"""A whole decode step's attention work in one HIP graph.

The reference builds each step on the host: ``DecodeBatch.__init__`` packs
the page tables in Python (python/instinct/batches.py:148-179) and every
layer's ``rope`` + ``attend`` (:195-226) is launched separately, and its
roadmap names the host-side step building as the limit on one user's decode
speed (docs/roadmap.md:11-13,37). :class:`DecodeStepGraph` keeps the
requests' page lists resident on the device (one row per request slot),
packs them with one kernel (``pda_pack_decode_step``) and captures, for every
layer, the fused RoPE + K/V append and the paged decode attention into one
``torch.cuda.CUDAGraph`` (a HIP graph on ROCm). A step is then: write the
step's slots, positions and projected q/k/v into the static buffers, replay.
Nothing of the step crosses PCIe except those inputs, and no kernel is
launched from Python.

Results do not depend on ``longest`` (a sizing hint of the decode call), so
one capture serves every later step whose sequences stay within the arenas;
two replays on the same inputs give the same bits (the decode call's split
points are fixed by the inputs).
"""

from __future__ import annotations

from collections.abc import Sequence
from typing import Any

import torch

from .hip_kernels import (decode_workspace_bytes, new_workspace, pack_decode_step,
                          paged_decode_attention, rope_append)


class DecodeStepGraph:
    """Static buffers and a captured graph for ``batch`` sequences over
    ``len(arenas)`` layers.

    ``arenas``: per layer ``(keys, values)`` or ``(keys, values, key_scales,
    value_scales)`` (8-bit); bf16 arenas take bf16 q/k/v and give bf16
    outputs, fp16 and 8-bit arenas fp16 ones; all layers share ``seq_tables``
    (``[num_slots, stride]`` int32 resident page lists), the page size, the
    window and the head shape. ``dims``/``base``/``freqs``: the rotary
    embedding (``dims`` = 0: none)."""

    def __init__(self, arenas: Sequence[tuple[torch.Tensor, ...]], seq_tables: torch.Tensor, *,
                 batch: int, q_heads: int, page_size: int, width: int, scale: float,
                 longest: int, dims: int = 0, base: float | None = None, freqs: Any = None,
                 window: int = 0, softcap: float = 0.0) -> None:
        keys = arenas[0][0]
        dev = keys.device
        kv_heads = int(keys.shape[1])
        head_dim = int(keys.shape[-1])
        self.arenas = [tuple(a) for a in arenas]
        self.seq_tables = seq_tables
        self.batch, self.page_size, self.width = batch, page_size, width
        self.kw = dict(page_size=page_size, longest=longest, scale=scale, window=window,
                       softcap=softcap)
        self.rope = dict(dims=dims, base=base, freqs=freqs)
        i32 = dict(dtype=torch.int32, device=dev)
        dtype = torch.bfloat16 if keys.dtype == torch.bfloat16 else torch.float16
        f16 = dict(dtype=dtype, device=dev)
        # Step inputs, written before every replay.
        self.slots = torch.zeros(batch, **i32)
        self.positions = torch.zeros(batch, **i32)
        layers = len(arenas)
        self.q = [torch.zeros((batch, q_heads, head_dim), **f16) for _ in range(layers)]
        self.k = [torch.zeros((batch, kv_heads, head_dim), **f16) for _ in range(layers)]
        self.v = [torch.zeros((batch, kv_heads, head_dim), **f16) for _ in range(layers)]
        # Step state and outputs.
        self.tables = torch.zeros((batch, width), **i32)
        self.lengths = torch.zeros(batch, **i32)
        self.rows = torch.zeros(batch, **i32)
        self.q_rot = [torch.zeros_like(q) for q in self.q]
        self.out = [torch.zeros_like(q) for q in self.q]
        # The decode calls' workspace, owned by this object: a captured graph
        # holds its address, so it must live as long as the graph and never
        # be shared with calls outside it (whose workspace may be replaced).
        need = decode_workspace_bytes((batch, q_heads, head_dim), keys, page_size=page_size,
                                      table_width=width, longest=longest, window=window)
        self.workspace = new_workspace(need, dev)
        self.graph: torch.cuda.CUDAGraph | None = None

    def run(self) -> None:
        """The step's launches, in order (eager; also what is captured)."""
        pack_decode_step(self.seq_tables, self.slots, self.positions, width=self.width,
                         page_size=self.page_size, tables=self.tables, lengths=self.lengths,
                         rows=self.rows)
        for layer, arena in enumerate(self.arenas):
            keys, values = arena[0], arena[1]
            scales = (arena[2], arena[3]) if len(arena) == 4 else None
            rope_append(self.q[layer], self.k[layer], self.v[layer], keys, values,
                        self.positions, self.rows, q_out=self.q_rot[layer], scales=scales,
                        page_size=self.page_size, **self.rope)
            paged_decode_attention(self.q_rot[layer], keys, values, self.tables, self.lengths,
                                   out=self.out[layer], scales=scales,
                                   workspace=self.workspace, **self.kw)

    def capture(self) -> None:
        """Capture :meth:`run` (after one eager run outside the capture).
        Every buffer the graph touches belongs to this object or to the
        caller (arenas, resident tables), so nothing it recorded is freed
        while the object lives."""
        self.run()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            self.run()
        torch.cuda.synchronize()
        self.graph = graph

    def replay(self) -> None:
        if self.graph is None:
            raise RuntimeError("capture() first")
        self.graph.replay()
