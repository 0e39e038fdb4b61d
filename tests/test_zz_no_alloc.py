"""The no-allocation decode entry point (pda_paged_decode_attention_noalloc,
through the C-ABI) against pda_paged_decode_attention with a caller's
workspace: two calls in a row, the second smaller, in the fixed-split mode
(bitwise equal: the same kernels, grid and split points, only the workspace
differs) and in the default mode (within the north star's max-abs 2e-3 /
mean-abs 2e-4), both also against the float64 oracle; and the clear error
for a shape whose partials do not fit the static scratch."""

import ctypes

import numpy as np
import pytest
import torch

from instinct_amd import _lib, workloads
from instinct_amd.hip_kernels import paged_decode_attention
from oracle import cpu_oracle
from oracle import paged_attention as pa

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-3
MEAN_ABS = 2e-4


def noalloc(w, flags):
    """One call of the no-allocation entry point; returns (rc, out)."""
    out = torch.full_like(w.q, float("nan"))
    layout, rows = ((_lib.PDA_LAYOUT_PAGES, int(w.keys.shape[0]) * w.page_size)
                    if w.keys.dim() == 4 else (_lib.PDA_LAYOUT_ROWS, int(w.keys.shape[0])))
    stream = torch.cuda.current_stream().cuda_stream
    rc = _lib.library().pda_paged_decode_attention_noalloc(
        w.q.data_ptr(), w.keys.data_ptr(), w.values.data_ptr(), w.tables.data_ptr(),
        w.lengths.data_ptr(), out.data_ptr(), w.batch, w.q_heads, w.kv_heads, w.head_dim,
        w.page_size, int(w.tables.shape[1]), rows, layout, w.longest, w.scale, w.window,
        w.softcap, 0, flags, ctypes.c_void_p(stream))
    torch.cuda.synchronize()
    return rc, out


def with_workspace(w, deterministic):
    out = paged_decode_attention(w.q, w.keys, w.values, w.tables, w.lengths,
                                 page_size=w.page_size, longest=w.longest, scale=w.scale,
                                 window=w.window, softcap=w.softcap,
                                 deterministic=deterministic)
    torch.cuda.synchronize()
    return out


def oracle(w):
    q, k, v, t, n = w.numpy()
    return cpu_oracle.decode_f64(q, k, v, t, n, page_size=w.page_size, scale=w.scale,
                                 window=w.window, softcap=w.softcap)


def within_bar(got, want, what):
    got = got.float().cpu().numpy() if isinstance(got, torch.Tensor) else got
    assert np.isfinite(got).all(), what
    err_max, err_mean = pa.error_stats(got, want)
    print(f"{what}: max_abs={err_max:.3e} mean_abs={err_mean:.3e}", flush=True)
    assert err_max <= MAX_ABS and err_mean <= MEAN_ABS, (what, err_max, err_mean)


def test_noalloc_matches_the_workspace_call_on_two_calls(gpu):
    big = workloads.config2(device=gpu, batch=32, low=512, high=8192).to_layout("pages")
    small = workloads.config2(device=gpu, seed=9, batch=5, low=100, high=900)
    for name, w in (("first (B=32)", big), ("second (B=5, smaller)", small)):
        want = oracle(w)
        rc, fixed = noalloc(w, 0)  # the default: fixed split points
        _lib.check(rc)
        ref_fixed = with_workspace(w, True)
        assert torch.equal(fixed, ref_fixed), f"{name}: fixed split differs from the workspace call"
        within_bar(fixed, want, f"{name} fixed vs oracle")
        rc, explicit = noalloc(w, _lib.PDA_DECODE_FIXED_SPLIT)
        _lib.check(rc)
        assert torch.equal(explicit, fixed), f"{name}: PDA_DECODE_FIXED_SPLIT differs from flags 0"
        rc, free = noalloc(w, _lib.PDA_DECODE_RACING)
        _lib.check(rc)
        within_bar(free.float().cpu().numpy(), ref_fixed.float().cpu().numpy(),
                   f"{name} racing vs workspace call")
        within_bar(free, want, f"{name} racing vs oracle")


def test_noalloc_at_512_wide_heads_on_four_wave_workgroups(gpu):
    """The matrix-core kernels at D = 512 run four-wave workgroups; the
    scratch is laid out for that grid (5 query heads per kv head: 2 x CUs x
    4 waves x 5 x 512 floats of partials, within the 32 MiB)."""
    w = workloads.reference_test_case(5, 1, 512, [1, 700, 2049, 6000], 0, 0.0, device=gpu)
    w.to_layout("pages")
    rc, fixed = noalloc(w, _lib.PDA_DECODE_FIXED_SPLIT)
    _lib.check(rc)
    assert torch.equal(fixed, with_workspace(w, True))
    within_bar(fixed, oracle(w), "512-wide, 5 heads, fixed")


def test_noalloc_rejects_a_shape_beyond_its_scratch(gpu):
    """512-wide heads with 8 query heads per kv head: 2 x CUs x 4 waves x 8
    x 512 floats of partials, 32 MiB, plus the pair records: above the
    32 MiB scratch."""
    w = workloads.reference_test_case(16, 2, 512, [1, 700, 2049], 0, 0.0, device=gpu)
    rc, _ = noalloc(w, 0)
    assert rc == _lib.PDA_ERR_WORKSPACE
    assert "no-allocation" in _lib.library().pda_last_error().decode()
    # The same call with a workspace works.
    within_bar(with_workspace(w, False), oracle(w), "512-wide with a workspace")
