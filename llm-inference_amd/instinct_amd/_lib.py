"""ctypes binding of libpda.so (the C-ABI declared in include/pda.h).

The library is built in-tree by ``make -C llm-inference_amd`` (or
``__graft_entry__.build()``). There is no fallback: if the library is missing
or does not load, :func:`library` raises.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parent.parent
LIBRARY_PATH = PACKAGE_ROOT / "lib" / "libpda.so"

# Return codes (pda.h).
PDA_OK = 0
PDA_ERR_INVALID_ARGUMENT = -1
PDA_ERR_HEAD_RATIO = -2
PDA_ERR_HEAD_DIM = -3
PDA_ERR_PAGE_SIZE = -4
PDA_ERR_WORKSPACE = -5
PDA_ERR_ALIGNMENT = -6
PDA_ERR_TOO_LONG = -7
PDA_ERR_HIP = -8

# Decode flags (pda.h).
PDA_DECODE_FIXED_SPLIT = 1  # fixed split points: bitwise reproducible output
PDA_DECODE_RACING = 2  # racing wave pairs (opt-in): output bits may differ between calls

# K/V arena layouts (pda.h).
PDA_LAYOUT_ROWS = 0   # [rows, kv_heads, head_dim], the reference's arena
PDA_LAYOUT_PAGES = 1  # [pages, kv_heads, page_size, head_dim] tiles

# Every symbol include/pda.h declares, with its ctypes signature.
SIGNATURES = {
    "pda_version": (ctypes.c_int, []),
    "pda_last_error": (ctypes.c_char_p, []),
    "pda_workspace_bytes": (
        ctypes.c_int,
        [c_int32] * 9 + [ctypes.POINTER(c_size_t)],
    ),
    "pda_plan": (
        ctypes.c_int,
        [c_int32] * 9 + [ctypes.POINTER(c_int32), ctypes.POINTER(c_int32)],
    ),
}
_DECODE_ARGS = ([c_void_p] * 6 + [c_int32] * 6
                + [c_int64, c_int32, c_int32, c_float, c_int32, c_float, c_int32, c_int32,
                   c_void_p, c_size_t, c_void_p])
for _name in ("pda_paged_decode_attention", "pda_decode_split", "pda_decode_merge"):
    SIGNATURES[_name] = (ctypes.c_int, _DECODE_ARGS)
    SIGNATURES[_name + "_bf16"] = (ctypes.c_int, _DECODE_ARGS)
# No workspace: the library's static device scratch (the same arguments
# without the workspace pointer and size).
SIGNATURES["pda_paged_decode_attention_noalloc"] = (
    ctypes.c_int, _DECODE_ARGS[:-3] + [c_void_p])
# 8-bit K/V: key and value scale arenas after the values.
_DECODE_ARGS_Q8 = _DECODE_ARGS[:3] + [c_void_p, c_void_p] + _DECODE_ARGS[3:]
for _name in ("pda_paged_decode_attention_q8", "pda_decode_split_q8", "pda_decode_merge_q8"):
    SIGNATURES[_name] = (ctypes.c_int, _DECODE_ARGS_Q8)
    SIGNATURES[_name + "_bf16"] = (ctypes.c_int, _DECODE_ARGS_Q8)
SIGNATURES["pda_rope_append"] = (
    ctypes.c_int,
    [c_void_p] * 8 + [c_int32] * 5 + [c_int64, c_int32, c_int32, c_void_p, c_void_p],
)
SIGNATURES["pda_rope_append_bf16"] = SIGNATURES["pda_rope_append"]
_PREFILL_TAIL = [c_int64, c_int32, c_float, c_int32, c_float, c_void_p, c_int32, c_int32,
                 c_void_p, c_size_t, c_void_p]
SIGNATURES["pda_paged_prefill_attention"] = (
    ctypes.c_int,
    [c_void_p] * 4 + [c_int32] * 3 + [c_void_p] + [c_int32] * 4 + _PREFILL_TAIL,
)
SIGNATURES["pda_paged_prefill_attention_bf16"] = SIGNATURES["pda_paged_prefill_attention"]
SIGNATURES["pda_paged_prefill_attention_q8"] = (
    ctypes.c_int,
    [c_void_p] * 6 + [c_int32] * 3 + [c_void_p] + [c_int32] * 4 + _PREFILL_TAIL,
)
SIGNATURES["pda_prefill_workspace_bytes"] = (
    ctypes.c_int,
    [c_int32] * 6 + [c_void_p, c_void_p],
)
SIGNATURES["pda_pack_decode_step"] = (
    ctypes.c_int,
    [c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_int32, c_int32, c_int32,
     c_void_p, c_void_p, c_void_p, c_void_p],
)
SIGNATURES["pda_rope_append_q8"] = (
    ctypes.c_int,
    [c_void_p] * 10 + [c_int32] * 5 + [c_int64, c_int32, c_int32, c_void_p, c_void_p],
)



class DecodeInfo(ctypes.Structure):
    """``pda_decode_info`` (pda.h): what a decode call of a shape launches."""

    _fields_ = [(name, c_int32) for name in (
        "kernel_dim", "head_slots", "kv_bits", "bf16", "generic", "matrix_cores",
        "unit_heads", "units_per_kv_head", "split_waves", "ring", "grid_groups", "local",
        "merge", "merge_waves")] + [("split_kernel", ctypes.c_char * 96),
                                    ("merge_kernel", ctypes.c_char * 96)]


SIGNATURES["pda_decode_describe"] = (
    ctypes.c_int,
    [c_int32] * 11 + [ctypes.POINTER(DecodeInfo)],
)

_lib: ctypes.CDLL | None = None


class PdaError(RuntimeError):
    """A non-zero return code from libpda, with the library's message."""

    def __init__(self, code: int, message: str) -> None:
        super().__init__(f"libpda error {code}: {message}")
        self.code = code
        self.message = message


def library() -> ctypes.CDLL:
    """Load libpda.so once; raise if it is missing."""
    global _lib
    if _lib is None:
        path = Path(os.environ.get("PDA_LIBRARY", LIBRARY_PATH))
        if not path.exists():
            raise FileNotFoundError(
                f"{path} is not built; run `make -C {PACKAGE_ROOT}` "
                "or __graft_entry__.build()"
            )
        lib = ctypes.CDLL(str(path))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
    return _lib


def check(code: int) -> None:
    if code != PDA_OK:
        message = library().pda_last_error().decode()
        if code == PDA_ERR_HEAD_RATIO:
            # The reference raises ValueError here (metal_kernels.py:189-190).
            raise ValueError(message)
        raise PdaError(code, message)


def workspace_bytes(batch, q_heads, kv_heads, head_dim, page_size, table_stride,
                    longest, window, split_pages=0) -> int:
    out = c_size_t(0)
    check(library().pda_workspace_bytes(batch, q_heads, kv_heads, head_dim, page_size,
                                        table_stride, longest, window, split_pages,
                                        ctypes.byref(out)))
    return out.value


def prefill_workspace_bytes(start, count, q_heads, head_dim, window=0,
                            splits=0) -> tuple[int, int]:
    """(key ranges, workspace bytes) of a prefill call."""
    used = c_int32(0)
    out = c_size_t(0)
    check(library().pda_prefill_workspace_bytes(start, count, q_heads, head_dim, window,
                                                splits, ctypes.byref(used), ctypes.byref(out)))
    return used.value, out.value


def plan(batch, q_heads, kv_heads, head_dim, page_size, table_stride, longest, window,
         split_pages=0) -> tuple[int, int]:
    pages = c_int32(0)
    splits = c_int32(0)
    check(library().pda_plan(batch, q_heads, kv_heads, head_dim, page_size, table_stride,
                             longest, window, split_pages, ctypes.byref(pages),
                             ctypes.byref(splits)))
    return pages.value, splits.value


def describe(batch, q_heads, kv_heads, head_dim, page_size, table_stride, longest, window,
             split_pages=0, kv_bits=16, bf16=False) -> dict:
    """``pda_decode_describe``: the kernels, grid, local mode and merge shape
    the library launches for a decode call of this shape."""
    info = DecodeInfo()
    check(library().pda_decode_describe(batch, q_heads, kv_heads, head_dim, page_size,
                                        table_stride, longest, window, split_pages, kv_bits,
                                        int(bool(bf16)), ctypes.byref(info)))
    out = {name: getattr(info, name) for name, _ in DecodeInfo._fields_}
    out["split_kernel"] = info.split_kernel.decode()
    out["merge_kernel"] = info.merge_kernel.decode() or None
    return out
