"""Parity of the K/V append with rotary embedding (pda_rope_append via the
C-ABI) with the oracle (oracle/rope_append.py, pinned by
tests/test_rope_oracle.py) on the same seeded inputs.

Bar: the written values and the elements past the rotary dims are bit-exact;
rotated elements are within one fp16 ulp of the oracle plus 2^-21 times the
largest input magnitude (both round the same float32 expression to nearest
even, but the float32 sine and cosine of the library and of NumPy may differ
in their last bits, and where the two products of a rotated element nearly
cancel that moves the result by more than its own fp16 ulp), and within the
north star's 2e-3 of a float64 rotation by the same float32 angles. Rows
outside the arena are not written; nothing else in the arena changes.
"""

import numpy as np
import pytest
import torch

from instinct_amd import hip_kernels
from instinct_amd.batches import DecodeBatch
from instinct_amd.paged_kv import KVCache, KVGroup
from oracle import rope_append as ra

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-3


def ulp_check(got: np.ndarray, want: np.ndarray, what: str, scale: float = 0.0) -> None:
    """Within one fp16 ulp of `want`, plus 2^-21 x `scale` (the largest
    input magnitude: float32 sine and cosine may differ in their last bits,
    which moves a nearly cancelling result by more than its own ulp)."""
    got = got.astype(np.float16)
    want = want.astype(np.float16)
    assert got.shape == want.shape, what
    if got.size == 0:
        return
    spacing = np.spacing(np.abs(want)).astype(np.float64) + scale * 2.0 ** -21
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    exact = np.mean(got == want)
    print(f"{what}: bit-exact {exact:.6f}, max diff {diff.max():.3e}", flush=True)
    assert np.all(diff <= spacing), (what, diff.max())


def float64_rotation(x: np.ndarray, positions: np.ndarray, dims: int, inverse: np.ndarray):
    half = dims // 2
    angles = (positions.astype(np.float32)[:, None] * inverse[None, :half]).astype(np.float64)
    z = x[..., :half].astype(np.float64) + 1j * x[..., half:dims].astype(np.float64)
    z = z * np.exp(1j * angles)[:, None, :]
    out = x.astype(np.float64).copy()
    out[..., :half], out[..., half:dims] = z.real, z.imag
    return out


def make_case(gpu, *, n, hq, hkv, d, layout, page_size=16, arena_pages=None, seed=0,
              max_pos=8192, positions=None):
    rng = np.random.default_rng(seed)
    arena_pages = arena_pages or max(4, 2 * n)
    q = rng.standard_normal((n, hq, d)).astype(np.float16) if hq else None
    k = rng.standard_normal((n, hkv, d)).astype(np.float16)
    v = rng.standard_normal((n, hkv, d)).astype(np.float16)
    if positions is None:
        positions = rng.integers(0, max_pos, n)
    positions = np.asarray(positions, dtype=np.int32)
    # Distinct rows: each token gets its own page of a permutation, at its
    # position's slot.
    pages = rng.permutation(arena_pages)[:n]
    rows = (pages * page_size + positions % page_size).astype(np.int32)
    shape = ((arena_pages * page_size, hkv, d) if layout == "rows"
             else (arena_pages, hkv, page_size, d))
    k_arena = rng.standard_normal(shape).astype(np.float16)
    v_arena = rng.standard_normal(shape).astype(np.float16)
    dev = lambda a: None if a is None else torch.as_tensor(a, device=gpu)  # noqa: E731
    return dict(q=q, k=k, v=v, positions=positions, rows=rows, k_arena=k_arena,
                v_arena=v_arena, page_size=page_size, layout=layout,
                t={name: dev(a) for name, a in (("q", q), ("k", k), ("v", v),
                                                ("positions", positions), ("rows", rows),
                                                ("k_arena", k_arena), ("v_arena", v_arena))})


def check_append(case, *, dims, base=None, freqs=None, in_place=False, what=""):
    t = case["t"]
    inverse = ra.inv_freq(dims, base=base, freqs=freqs) if dims else np.zeros(0, np.float32)
    q_out = t["q"] if in_place else None
    got_q = hip_kernels.rope_append(t["q"], t["k"], t["v"], t["k_arena"], t["v_arena"],
                                    t["positions"], t["rows"], page_size=case["page_size"],
                                    dims=dims, base=base, freqs=freqs, q_out=q_out)
    torch.cuda.synchronize()
    want_q, want_k, want_v = ra.rope_append(
        case["q"], case["k"], case["v"], case["k_arena"], case["v_arena"], case["positions"],
        case["rows"], dims=dims, inverse=inverse, layout=case["layout"],
        page_size=case["page_size"])
    got_k = t["k_arena"].cpu().numpy()
    got_v = t["v_arena"].cpu().numpy()
    assert np.array_equal(got_v, want_v), f"{what}: values"
    # Keys: rotated elements within one ulp, everything else bit-exact.
    if dims:
        ulp_check(got_k, want_k, f"{what} keys", float(np.abs(case["k"]).max(initial=0.0)))
    assert np.array_equal(got_k[..., dims:], want_k[..., dims:]), f"{what}: key tail"
    untouched = np.ones(got_k.shape[:-1], bool)
    total = got_k.shape[0] * (1 if case["layout"] == "rows" else case["page_size"])
    for row in case["rows"]:
        if 0 <= row < total:
            if case["layout"] == "rows":
                untouched[row] = False
            else:
                untouched[row // case["page_size"], :, row % case["page_size"]] = False
    assert np.array_equal(got_k[untouched], case["k_arena"][untouched]), f"{what}: other rows"
    if case["q"] is not None:
        gq = got_q.cpu().numpy()
        if in_place:
            assert got_q.data_ptr() == t["q"].data_ptr()
        if dims:
            ulp_check(gq, want_q, f"{what} queries", float(np.abs(case["q"]).max(initial=0.0)))
            err = np.abs(gq.astype(np.float64)
                         - float64_rotation(case["q"], case["positions"], dims, inverse)).max(
                             initial=0.0)
            print(f"{what}: queries vs float64 rotation max_abs={err:.3e}", flush=True)
            assert err <= MAX_ABS
        else:
            assert np.array_equal(gq, case["q"])
        assert np.array_equal(gq[..., dims:], case["q"][..., dims:])


@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_config2_decode_step(gpu, layout):
    """Qwen2.5-7B decode shape: 64 tokens, 28/4 heads, D=128, base 1e6."""
    case = make_case(gpu, n=64, hq=28, hkv=4, d=128, layout=layout, seed=2,
                     positions=np.random.default_rng(2).integers(511, 8192, 64))
    check_append(case, dims=128, base=1e6, what=f"config2 {layout}")


@pytest.mark.parametrize("d,dims,base,layout", [
    (64, 64, 10000.0, "pages"),
    (80, 80, 10000.0, "rows"),
    (96, 96, 10000.0, "pages"),
    (128, 64, 10000.0, "rows"),      # partial rotary: 64 of 128 dims
    (256, 256, 10000.0, "pages"),
    (512, 512, 1e6, "pages"),
    (64, 6, 100.0, "rows"),          # odd half (3 pairs), 58 copied dims
])
def test_head_dims_and_partial_rotation(gpu, d, dims, base, layout):
    case = make_case(gpu, n=9, hq=8, hkv=2, d=d, layout=layout, seed=d + dims)
    check_append(case, dims=dims, base=base, what=f"d{d} dims{dims}")


def test_large_positions_and_explicit_frequencies(gpu):
    """Positions up to 2^20 (angles ~10^6 rad need full range reduction) and
    explicit frequencies with infinite entries (those pairs stay put), as
    Gemma-style full-attention layers pass them (batches.py:195-201 freqs)."""
    positions = [0, 1, 2, 16383, 65535, 131071, 500000, 1 << 20]
    case = make_case(gpu, n=len(positions), hq=4, hkv=2, d=128, layout="pages",
                     positions=positions, seed=5)
    check_append(case, dims=128, base=10000.0, what="large positions")
    freqs = np.concatenate([np.geomspace(1.0, 1e4, 48), np.full(16, np.inf)]).astype(np.float32)
    case = make_case(gpu, n=8, hq=4, hkv=2, d=128, layout="rows", positions=positions, seed=6)
    check_append(case, dims=128, freqs=freqs, what="freqs")


def test_in_place_queries_and_rows_outside_the_arena(gpu):
    case = make_case(gpu, n=6, hq=7, hkv=1, d=128, layout="pages", arena_pages=8, seed=9)
    total = 8 * 16
    case["rows"][[1, 4]] = [-3, total + 5]
    case["t"]["rows"] = torch.as_tensor(case["rows"], device=gpu)
    check_append(case, dims=128, base=10000.0, in_place=True, what="in place")


@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_write_without_rotation_and_without_queries(gpu, layout):
    case = make_case(gpu, n=12, hq=0, hkv=4, d=128, layout=layout, seed=12)
    check_append(case, dims=0, what=f"write {layout}")
    case = make_case(gpu, n=12, hq=0, hkv=4, d=128, layout=layout, seed=13)
    check_append(case, dims=128, base=1e4, what=f"keys only {layout}")


def test_empty_step(gpu):
    case = make_case(gpu, n=0, hq=4, hkv=2, d=64, layout="pages", arena_pages=4)
    check_append(case, dims=64, base=1e4, what="empty")


def test_rope_alone(gpu):
    rng = np.random.default_rng(14)
    x = rng.standard_normal((5, 3, 128)).astype(np.float16)
    positions = np.array([0, 3, 77, 4095, 120000], np.int32)
    got = hip_kernels.rope(torch.as_tensor(x, device=gpu), torch.as_tensor(positions, device=gpu),
                           128, base=1e6)
    want = ra.rope(x, positions, 128, ra.inv_freq(128, base=1e6))
    ulp_check(got.cpu().numpy(), want, "rope alone")


@pytest.mark.parametrize("layout", ["pages", "rows"])
def test_decode_batch_rope_attend_equals_rope_then_attend(gpu, layout):
    """DecodeBatch.rope_attend (one launch for both rotations and the write)
    gives the arena and the output of the reference's call sequence
    rope(q), rope(k), attend (backends/dense.py:99-102, batches.py:203-226)."""
    page = 16
    groups = [KVGroup("full", (0, 1), kv_heads=4, head_dim=128)]
    positions = np.array([0, 15, 16, 100, 333, 2047])
    gen = torch.Generator(device=gpu).manual_seed(3)

    def fresh():
        cache = KVCache(groups, page_size=page, capacities={"full": 256}, device=gpu,
                        layout=layout)
        pool = cache.pools["full"]
        tables = {"full": [np.array([pool.allocate(reserved=False)
                                     for _ in range(p // page + 1)]) for p in positions]}
        for layer in (0, 1):
            cache.keys[layer].copy_(torch.arange(cache.keys[layer].numel(), device=gpu)
                                    .view_as(cache.keys[layer]).remainder(17).half() * 0.1)
            cache.values[layer].copy_(cache.keys[layer] * -0.5)
        return cache, DecodeBatch(cache, torch.zeros(6, device=gpu), positions=positions,
                                  tables=tables)

    q = torch.randn((6, 28, 128), generator=gen, device=gpu).half()
    k = torch.randn((6, 4, 128), generator=gen, device=gpu).half()
    v = torch.randn((6, 4, 128), generator=gen, device=gpu).half()
    c1, b1 = fresh()
    fused = b1.rope_attend(0, q, k, v, dims=128, base=1e6, scale=128 ** -0.5)
    c2, b2 = fresh()
    qr, kr = b2.rope(q, 128, base=1e6), b2.rope(k, 128, base=1e6)
    plain = b2.attend(0, qr, kr, v, scale=128 ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(c1.keys[0], c2.keys[0]) and torch.equal(c1.values[0], c2.values[0])
    d = (fused.float() - plain.float()).abs()
    print(f"rope_attend vs rope+attend: max={d.max().item():.3e}", flush=True)
    assert d.max().item() <= MAX_ABS and d.mean().item() <= 2e-4


@pytest.mark.parametrize("seed", range(24))
def test_random_appends(gpu, seed):
    """Seeded random appends: token count, query and kv heads (no queries
    too), head dim, rotary dims (none, partial, full), base, page size,
    layout, positions up to 2^17 and in-place queries, against the oracle
    at this file's bar."""
    rng = np.random.default_rng(9000 + seed)
    d = int(rng.choice([8, 64, 80, 96, 128, 256, 512]))
    dims = int(rng.choice([0, d, d // 2 - (d // 2) % 2, 2 * int(rng.integers(1, d // 2 + 1))]))
    hkv = int(rng.choice([1, 2, 4, 8]))
    hq = int(rng.choice([0, hkv, 4 * hkv, 7 * hkv]))
    n = int(rng.choice([1, int(rng.integers(2, 200))]))
    layout = str(rng.choice(["rows", "pages"]))
    page = int(rng.choice([16, 16, 8, 5, 32]))
    base = float(rng.choice([10000.0, 1e6, 500.0]))
    in_place = bool(hq) and bool(rng.integers(0, 2))
    what = (f"seed {seed}: n {n} heads {hq}/{hkv} d {d} dims {dims} {layout} page {page} "
            f"base {base:g}{' in place' if in_place else ''}")
    print(what, flush=True)
    case = make_case(gpu, n=n, hq=hq, hkv=hkv, d=d, layout=layout, page_size=page, seed=seed,
                     max_pos=1 << 17)
    check_append(case, dims=dims, base=base, in_place=in_place, what=what)
