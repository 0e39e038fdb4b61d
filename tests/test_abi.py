"""libpda.so loads, exports every entry point include/pda.h declares, and
validates its arguments on the host (no GPU call is made by these tests:
every rejected call returns before touching HIP)."""

import ctypes
import re
from pathlib import Path

import pytest

from instinct_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "pda.h"
FAKE = 0x10000  # an aligned, never-dereferenced address


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(pda_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_expected_entry_points():
    assert declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.library()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.pda_version() >= 1


def decode(**overrides):
    args = dict(queries=FAKE, keys=FAKE, values=FAKE, tables=FAKE, lengths=FAKE, out=FAKE,
                batch=4, q_heads=28, kv_heads=4, head_dim=128, page_size=16,
                table_stride=64, arena_rows=4096, layout=_lib.PDA_LAYOUT_ROWS,
                longest=1000, scale=0.088, window=0,
                softcap=0.0, split_pages=0, flags=0, workspace=FAKE * 16,
                workspace_bytes=1 << 30, stream=None)
    args.update(overrides)
    lib = _lib.library()
    return lib.pda_paged_decode_attention(*args.values())


@pytest.mark.parametrize("overrides, code", [
    (dict(q_heads=30), _lib.PDA_ERR_HEAD_RATIO),
    (dict(head_dim=513), _lib.PDA_ERR_HEAD_DIM),
    (dict(head_dim=514), _lib.PDA_ERR_HEAD_DIM),
    (dict(head_dim=0), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(flags=4), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(flags=_lib.PDA_DECODE_FIXED_SPLIT | _lib.PDA_DECODE_RACING), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(kv_heads=0), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(batch=-1), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(window=-1), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(queries=None), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(tables=None), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(arena_rows=8), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(layout=2), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(layout=-1), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(head_dim=512, q_heads=64, kv_heads=64, page_size=1 << 16, arena_rows=1 << 17),
     _lib.PDA_ERR_TOO_LONG),
    (dict(scale=float("nan")), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(softcap=-1.0), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(batch=9000), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(keys=FAKE + 2), _lib.PDA_ERR_ALIGNMENT),
    (dict(out=FAKE + 8), _lib.PDA_ERR_ALIGNMENT),
    (dict(lengths=FAKE + 2), _lib.PDA_ERR_ALIGNMENT),
    (dict(workspace=None), _lib.PDA_ERR_WORKSPACE),
    (dict(workspace_bytes=16), _lib.PDA_ERR_WORKSPACE),
    (dict(batch=1, workspace=None, workspace_bytes=0), _lib.PDA_ERR_WORKSPACE),
    (dict(workspace=FAKE + 64), _lib.PDA_ERR_ALIGNMENT),
    (dict(table_stride=1 << 28), _lib.PDA_ERR_TOO_LONG),
])
def test_host_validation_rejects_bad_arguments(overrides, code):
    assert decode(**overrides) == code
    assert _lib.library().pda_last_error().decode() != ""


def test_bad_head_ratio_raises_value_error_like_the_reference():
    with pytest.raises(ValueError, match="multiple of kv heads"):
        _lib.check(decode(q_heads=30))


def test_empty_batch_is_a_no_op():
    assert decode(batch=0, workspace=None, workspace_bytes=0) == _lib.PDA_OK
    assert _lib.library().pda_last_error().decode() == ""


def test_workspace_and_plan_are_consistent():
    waves, per_wave = _lib.plan(64, 28, 4, 128, 16, 512, 8192, 0)
    assert waves == 2048 and per_wave * waves >= 64 * 4 * 512
    # Few pages: the stream uses fewer wave pairs, each wave with about
    # split_pages pages (40 pages: 3 pairs of 7 pages a wave).
    # 40 visible pages: one page per wave by default, two with split_pages=2.
    assert _lib.plan(1, 8, 8, 128, 16, 64, 64, 0) == (40, 1)
    assert _lib.plan(1, 8, 8, 128, 16, 64, 64, 0, split_pages=2) == (20, 2)
    # A window bounds the visible pages whatever the table width.
    assert _lib.plan(32, 8, 4, 256, 16, 2048, 32768, 1024, split_pages=16)[0] == 32 * 4 * 65 // 16
    need = _lib.workspace_bytes(64, 28, 4, 128, 16, 512, 8192, 0)
    slots = 2 * 2048
    assert need >= 65 * 4 + slots * 7 * (128 + 2) * 4
    # The workspace does not grow with the context length.
    assert _lib.workspace_bytes(64, 28, 4, 128, 16, 8192, 131072, 0) == need
    # The partial slots hold one unit's query heads: a 16-head group (one
    # matrix-core unit) needs twice the partial space of an 8-head one, and
    # 32 heads (two units of 16) no more than 16.
    eight = _lib.workspace_bytes(2, 8, 1, 128, 16, 64, 1024, 0)
    sixteen = _lib.workspace_bytes(2, 16, 1, 128, 16, 64, 1024, 0)
    thirty_two = _lib.workspace_bytes(2, 32, 1, 128, 16, 64, 1024, 0)
    one = _lib.workspace_bytes(2, 1, 1, 128, 16, 64, 1024, 0)
    assert thirty_two == sixteen
    assert (sixteen - eight) * 7 == (eight - one) * 8  # partial space per head
    assert sixteen - eight >= slots * 8 * (128 + 2) * 4


def test_batch_limit():
    with pytest.raises(_lib.PdaError) as err:
        _lib.workspace_bytes(8192, 16, 2, 128, 16, 64, 1024, 0)
    assert err.value.code == _lib.PDA_ERR_INVALID_ARGUMENT


def test_page_count_limit():
    with pytest.raises(_lib.PdaError) as err:
        _lib.plan(4096, 64, 8, 128, 16, 1 << 24, 1 << 28, 0)
    assert err.value.code == _lib.PDA_ERR_TOO_LONG


def append(**overrides):
    args = dict(q=FAKE, q_out=FAKE, k=FAKE, v=FAKE, k_arena=FAKE, v_arena=FAKE,
                positions=FAKE, rows=FAKE, n=64, q_heads=28, kv_heads=4, head_dim=128,
                page_size=16, arena_rows=4096, layout=_lib.PDA_LAYOUT_PAGES, rope_dims=128,
                inv_freq=FAKE, stream=None)
    args.update(overrides)
    return _lib.library().pda_rope_append(*args.values())


@pytest.mark.parametrize("overrides", [
    dict(n=-1),
    dict(head_dim=0),
    dict(n=0, head_dim=0),
    dict(head_dim=1024, rope_dims=0),
    dict(rope_dims=7),
    dict(rope_dims=130),
    dict(rope_dims=-2),
    dict(q_out=None),                   # q without q_out
    dict(q_heads=0),
    dict(v=None),                       # a partial K/V write
    dict(rows=None),
    dict(kv_heads=0),
    dict(layout=2),
    dict(arena_rows=0),
    dict(arena_rows=4100),              # not a whole number of page tiles
    dict(page_size=0),
    dict(positions=None),               # rotation without positions
    dict(inv_freq=None),
])
def test_append_validation_rejects_bad_arguments(overrides):
    assert append(**overrides) == _lib.PDA_ERR_INVALID_ARGUMENT
    assert _lib.library().pda_last_error()


def test_append_alignment_and_empty_calls():
    assert append(k=FAKE + 1) == _lib.PDA_ERR_ALIGNMENT
    assert append(rows=FAKE + 2) == _lib.PDA_ERR_ALIGNMENT
    # Nothing to do: no launch, no error.
    assert append(n=0) == _lib.PDA_OK
    assert append(q=None, q_out=None, k=None, v=None, k_arena=None, v_arena=None,
                  rows=None) == _lib.PDA_OK
    # Rows layout needs no page size; rope_dims 0 needs no positions or table.
    assert append(n=0, layout=_lib.PDA_LAYOUT_ROWS, page_size=0) == _lib.PDA_OK
    assert append(n=0, rope_dims=0, positions=None, inv_freq=None) == _lib.PDA_OK


def prefill(**overrides):
    args = dict(q=FAKE, k=FAKE, v=FAKE, table=FAKE, table_len=64, start=0, count=256,
                out=FAKE, q_heads=28, kv_heads=4, head_dim=128, page_size=16, arena_rows=4096,
                layout=_lib.PDA_LAYOUT_PAGES, scale=0.088, window=0, softcap=0.0, images=None,
                num_images=0, splits=1, workspace=None, workspace_bytes=0, stream=None)
    args.update(overrides)
    return _lib.library().pda_paged_prefill_attention(*args.values())


@pytest.mark.parametrize("overrides,code", [
    (dict(count=-1), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(start=-1), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(q_heads=0), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(kv_heads=0), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(page_size=0), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(table_len=-1), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(table_len=0), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(window=-1), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(splits=-1), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(num_images=-1), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(num_images=2), _lib.PDA_ERR_INVALID_ARGUMENT),      # spans missing
    (dict(num_images=2, images=FAKE + 2), _lib.PDA_ERR_ALIGNMENT),
    (dict(splits=4), _lib.PDA_ERR_WORKSPACE),
    (dict(splits=4, workspace=FAKE, workspace_bytes=1 << 20), _lib.PDA_ERR_WORKSPACE),
    (dict(splits=4, workspace=FAKE + 16, workspace_bytes=1 << 30), _lib.PDA_ERR_WORKSPACE),
    (dict(q_heads=30), _lib.PDA_ERR_HEAD_RATIO),
    (dict(head_dim=0), _lib.PDA_ERR_HEAD_DIM),
    (dict(head_dim=514), _lib.PDA_ERR_HEAD_DIM),
    (dict(start=(1 << 31) - 100), _lib.PDA_ERR_TOO_LONG),
    (dict(out=None), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(table=None), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(layout=2), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(arena_rows=8), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(scale=float("nan")), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(scale=float("inf")), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(softcap=-1.0), _lib.PDA_ERR_INVALID_ARGUMENT),
    (dict(q=FAKE + 8), _lib.PDA_ERR_ALIGNMENT),
    (dict(v=FAKE + 2), _lib.PDA_ERR_ALIGNMENT),
    (dict(table=FAKE + 2), _lib.PDA_ERR_ALIGNMENT),
    (dict(count=1 << 30, q_heads=256, kv_heads=1), _lib.PDA_ERR_INVALID_ARGUMENT),
])
def test_prefill_validation_rejects_bad_arguments(overrides, code):
    assert prefill(**overrides) == code
    assert _lib.library().pda_last_error()


def test_prefill_empty_chunk_is_a_no_op():
    assert prefill(count=0) == _lib.PDA_OK
    assert prefill(count=0, q=None, k=None, v=None, table=None, out=None) == _lib.PDA_OK


def test_prefill_split_plan():
    # The reference's 512-token chunk over a 4096-token prefix: 4 query tiles
    # x 28 heads = 112 workgroups; 4 ranges fill the 512 slots (256 CUs x 2)
    # in one round (5 would leave a second round of 48).
    splits, need = _lib.prefill_workspace_bytes(4096, 512, 28, 128)
    assert splits == 4
    assert need == 4 * 512 * 28 * 128 * 4 + 4 * 512 * 28 * 8
    assert _lib.prefill_workspace_bytes(3072, 1024, 28, 128)[0] == 2
    # Enough query tiles: one range, no workspace.
    assert _lib.prefill_workspace_bytes(0, 4096, 28, 128) == (1, 0)
    assert _lib.prefill_workspace_bytes(8192, 2048, 28, 128) == (1, 0)
    # A short prefix: ranges of at least 8 key tiles.
    assert _lib.prefill_workspace_bytes(0, 512, 28, 128) == (1, 0)
    assert _lib.prefill_workspace_bytes(500, 512, 28, 128)[0] == 2
    # Forced counts, capped at 64; empty chunks need nothing.
    assert _lib.prefill_workspace_bytes(0, 100, 8, 64, splits=3)[0] == 3
    assert _lib.prefill_workspace_bytes(0, 100, 8, 64, splits=500)[0] == 64
    assert _lib.prefill_workspace_bytes(0, 0, 8, 64, splits=3) == (1, 0)
    # Head dims without a kernel of their own plan as the next wider kernel.
    # Odd head dims too (element-wise kernels of the same widths).
    for d, width in ((80, 96), (4, 64), (200, 256), (510, 512), (66, 96), (98, 128),
                     (1, 64), (81, 96), (129, 256), (511, 512)):
        assert _lib.prefill_workspace_bytes(3000, 256, 8, d) == \
            _lib.prefill_workspace_bytes(3000, 256, 8, width)
    for d in (0, 513, 514, -2):
        with pytest.raises(_lib.PdaError):
            _lib.prefill_workspace_bytes(0, 10, 8, d)
    # 512-wide heads: 64 queries per workgroup, one workgroup per CU. A
    # 64-token chunk at 8 heads is 8 workgroups; 32 ranges would fill the
    # 256 CUs, but a range keeps at least 8 key tiles: 6064 keys / 32 / 8 = 23.
    assert _lib.prefill_workspace_bytes(6000, 64, 8, 512) == (
        23, 23 * 64 * 8 * 512 * 4 + ((23 * 64 * 8 * 8 + 255) // 256) * 256)
    assert _lib.prefill_workspace_bytes(0, 4096, 16, 512) == (1, 0)
    # A prompt from position 0 that fills at most one round: its tiles' key
    # counts differ up to 32x, and 2 ranges let the long tiles' halves run
    # beside the short ones.
    assert _lib.prefill_workspace_bytes(0, 4096, 14, 64)[0] == 2
    assert _lib.prefill_workspace_bytes(0, 2048, 16, 256)[0] == 2
    assert _lib.prefill_workspace_bytes(0, 2048, 16, 512)[0] == 1  # two rounds
    assert _lib.prefill_workspace_bytes(0, 4096, 14, 64, window=256)[0] == 1  # tiles alike


def test_prefill_q8_validation():
    lib = _lib.library()

    def call(ks=FAKE, vs=FAKE, **overrides):
        args = dict(q=FAKE, k=FAKE, v=FAKE, ks=ks, vs=vs, table=FAKE, table_len=64, start=0,
                    count=256, out=FAKE, q_heads=28, kv_heads=4, head_dim=128, page_size=16,
                    arena_rows=4096, layout=_lib.PDA_LAYOUT_PAGES, scale=0.088, window=0,
                    softcap=0.0, images=None, num_images=0, splits=1, workspace=None,
                    workspace_bytes=0, stream=None)
        args.update(overrides)
        return lib.pda_paged_prefill_attention_q8(*args.values())

    assert call(ks=None) == _lib.PDA_ERR_INVALID_ARGUMENT
    assert call(vs=None) == _lib.PDA_ERR_INVALID_ARGUMENT
    assert call(ks=FAKE + 1) == _lib.PDA_ERR_ALIGNMENT
    assert call(head_dim=513) == _lib.PDA_ERR_HEAD_DIM
    assert call(count=0, ks=None, vs=None) == _lib.PDA_OK


# What each BASELINE configuration launches, as pda_decode_describe reports it
# without a device (MI355X's 256-workgroup grid); these are the kernel names
# the rocprofv3 traces under profiles/ show for the same calls.
DESCRIBED = [
    # (q_heads, kv_heads, head_dim, batch, longest, table_width, window, bits, bf16)
    ((14, 2, 64, 8, 1024, 64, 0, 16, False),  # config 1
     "paged_decode_kernel<64,16,false,false,false,true>",
     "paged_decode_merge_sliced_kernel<64,16,false,false>"),
    ((28, 4, 128, 64, 8138, 512, 0, 16, False),  # config 2
     "paged_decode_kernel<128,16,false,false,false,true>",
     "paged_decode_merge_kernel<128,16,false,false>"),
    ((32, 8, 128, 1, 32768, 2048, 0, 16, False),  # config 3, B=1 x 32K
     "paged_decode_kernel<128,4,false,false,false,false>",
     "paged_decode_merge_sliced_kernel<128,4,false,false>"),
    ((32, 8, 128, 4, 131072, 8192, 0, 16, False),  # config 3, B=4 x 131K
     "paged_decode_kernel<128,4,false,false,false,false>",
     "paged_decode_merge_sliced_kernel<128,4,false,false>"),
    ((8, 4, 256, 32, 32768, 2048, 1024, 16, False),  # config 4: local mode, a unit per head
     "paged_decode_kernel<256,1,false,false,false,false>", None),
    ((32, 8, 128, 256, 65536, 4096, 0, 16, False),  # config 5
     "paged_decode_kernel<128,4,false,false,false,false>",
     "paged_decode_merge_kernel<128,4,false,false>"),
    ((16, 2, 512, 1, 261840, 16365, 0, 16, True),  # the reference's published layer, bf16
     "paged_decode_kernel<512,16,false,true,false,true>",
     "paged_decode_merge_sliced_kernel<512,16,true,false>"),
    ((28, 4, 128, 64, 8138, 512, 0, 8, False),  # config 2 over an 8-bit cache
     "paged_decode_kernel<128,16,true,false,false,true>",
     "paged_decode_merge_kernel<128,16,false,false>"),
]


@pytest.mark.parametrize("shape, split, merge", DESCRIBED)
def test_describe_reports_each_configuration(shape, split, merge):
    hq, hkv, d, batch, longest, width, window, bits, bf16 = shape
    info = _lib.describe(batch, hq, hkv, d, 16, width, longest, window, kv_bits=bits, bf16=bf16)
    assert info["split_kernel"] == split
    assert info["merge_kernel"] == merge
    assert info["local"] == (merge is None)
    assert info["merge"] == (0 if merge is None else 2 if "sliced" in merge else 1)
    assert info["matrix_cores"] == split.endswith("true>")
    assert info["grid_groups"] == 256


def test_describe_validation():
    with pytest.raises(_lib.PdaError):
        _lib.describe(4, 28, 4, 128, 16, 64, 1000, 0, kv_bits=4)
    # bf16 queries over an 8-bit cache: the 8-bit kernels' arithmetic, bf16
    # output (the merge kernels write bf16).
    info = _lib.describe(4, 28, 4, 128, 16, 64, 1000, 0, kv_bits=8, bf16=True)
    assert info["split_kernel"] == "paged_decode_kernel<128,16,true,true,false,true>"
    assert info["merge_kernel"].endswith("<128,16,true,false>")
    with pytest.raises(ValueError):
        _lib.describe(4, 30, 4, 128, 16, 64, 1000, 0)
    # Generic head dims report their padded kernel; units of large groups.
    info = _lib.describe(2, 8, 1, 80, 16, 64, 1000, 0, kv_bits=8)
    assert info["split_kernel"] == "paged_decode_kernel<128,8,true,false,true,false>"
    info = _lib.describe(2, 32, 1, 128, 16, 64, 1000, 0)
    assert (info["unit_heads"], info["units_per_kv_head"], info["head_slots"]) == (16, 2, 16)
    # Local mode on the VALU kernels with CUs to spare: a unit per query head
    # (config 4: 32 sequences x 4 kv heads x 2 heads = 256 workgroups).
    info = _lib.describe(32, 8, 4, 256, 16, 2048, 32768, 1024)
    assert info["local"]
    assert (info["unit_heads"], info["units_per_kv_head"], info["head_slots"]) == (1, 2, 1)
    # Odd head dims (the reference's IN_HEAD guard takes any): the padded
    # generic width, element-wise loads, one query head per unit.
    for d, bits, bf16, dp in ((7, 16, False, 8), (129, 8, False, 256), (511, 16, True, 512),
                              (1, 8, True, 8)):
        info = _lib.describe(2, 8, 2, d, 16, 64, 1000, 0, kv_bits=bits, bf16=bf16)
        q8, bf = ("true" if bits == 8 else "false"), ("true" if bf16 else "false")
        assert info["split_kernel"] == f"paged_decode_odd_kernel<{dp},{q8},{bf}>"
        assert info["merge_kernel"].endswith(f"<{dp},1,{bf},true>")
        assert (info["unit_heads"], info["units_per_kv_head"], info["head_slots"]) == (1, 4, 1)
        assert info["generic"] and not info["matrix_cores"]
