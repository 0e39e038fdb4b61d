"""Committed parity fixtures (tests/golden/, made by make_fixtures.py).

CPU: both oracle restatements reproduce every fixture. GPU: the MI355X
kernel matches every fixture within max-abs 2e-3 / mean-abs 2e-4.
"""

from pathlib import Path

import numpy as np
import pytest

from oracle import cpu_oracle
from oracle import paged_attention as pa

GOLDEN = sorted((Path(__file__).resolve().parent / "golden").glob("*.npz"))


def load(path):
    with np.load(path) as z:
        case = {k: z[k] for k in z.files}
    for k in ("page_size", "window"):
        case[k] = int(case[k])
    for k in ("scale", "softcap"):
        case[k] = float(case[k])
    return case


def test_fixture_set_is_present():
    names = {p.stem for p in GOLDEN}
    assert {"closed_form_p16", "config1_small", "config2_small", "config3_small",
            "config4_small", "config5_small", "softcap_small"} <= names


@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.stem)
def test_oracles_reproduce_fixture(path):
    c = load(path)
    kw = dict(page_size=c["page_size"], scale=c["scale"], window=c["window"],
              softcap=c["softcap"])
    args = (c["q"], c["keys"], c["values"], c["tables"], c["lengths"])
    np.testing.assert_allclose(pa.paged_decode_dense(*args, **kw), c["expected"], atol=1e-6)
    np.testing.assert_allclose(cpu_oracle.decode_f64(*args, **kw), c["expected"], atol=1e-6)
    np.testing.assert_allclose(pa.paged_decode_splitk(*args, splits=3, **kw), c["expected"],
                               atol=1e-6)


def test_closed_form_fixture_matches_the_formula():
    c = load(next(p for p in GOLDEN if p.stem == "closed_form_p16"))
    e5, e1 = np.exp(0.5), np.exp(1.0)
    v0, v1, v2 = np.array([1, 2, 3, 4]), np.array([5, 6, 7, 8]), np.array([2, 4, 6, 8])
    expected = (e5 * v0 + 15 * e5 * v1 + e1 * v2) / (16 * e5 + e1)
    np.testing.assert_allclose(c["expected"][0, 0, :4], expected, atol=1e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("layout", ["rows", "pages"])
@pytest.mark.parametrize("path", GOLDEN, ids=lambda p: p.stem)
def test_kernel_matches_fixture(gpu, path, layout):
    import torch

    from instinct_amd.hip_kernels import paged_decode_attention
    from instinct_amd.paged_kv import rows_to_pages

    c = load(path)
    t = {k: torch.as_tensor(c[k]).to(gpu) for k in ("q", "keys", "values", "tables", "lengths")}
    if layout == "pages":
        t["keys"] = rows_to_pages(t["keys"], c["page_size"])
        t["values"] = rows_to_pages(t["values"], c["page_size"])
    out = paged_decode_attention(t["q"], t["keys"], t["values"], t["tables"], t["lengths"],
                                 page_size=c["page_size"], longest=int(c["lengths"].max()),
                                 scale=c["scale"], window=c["window"], softcap=c["softcap"])
    got = out.float().cpu().numpy()
    err_max, err_mean = pa.error_stats(got, c["expected"])
    print(f"{path.stem} [{layout}]: max_abs={err_max:.3e} mean_abs={err_mean:.3e}")
    assert err_max <= 2e-3 and err_mean <= 2e-4
