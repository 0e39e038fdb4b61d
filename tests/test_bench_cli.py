"""bench.py's command line on the CPU: the options parse, a multi-GPU
request exits with a message (this build runs on one GPU), and the
workloads the bench times have the shapes and byte counts it reports."""

import math
import subprocess
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]


def run_bench(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT,
                          capture_output=True, text=True, timeout=120)


def test_help_lists_the_legs():
    r = run_bench("--help")
    assert r.returncode == 0, r.stderr
    for option in ("--published", "--latency-configs", "--kv-bits", "--prefill-wide",
                   "--deterministic", "--racing", "--copy-calibration"):
        assert option in r.stdout


def test_more_than_one_gpu_is_refused():
    r = run_bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_published_workload_shape():
    """The Gemma 4 global layer of the reference's published figure
    (docs/benchmarks.md:102-110): 2 kv heads x 512, one sequence of 261,840
    tokens, 1,072,496,640 bytes of K+V; small length here, same geometry."""
    sys.path[:0] = [str(ROOT), str(ROOT / "llm-inference_amd")]
    from instinct_amd import workloads

    w = workloads.gemma4_global(length=1000)
    assert (w.batch, w.q_heads, w.kv_heads, w.head_dim, w.page_size) == (1, 16, 2, 512, 16)
    assert w.kv_bytes() == 1000 * 2 * 512 * 2 * 2
    assert 261840 * 2 * 512 * 2 * 2 == 1072496640
    tables = w.tables.numpy()[0]
    assert sorted(tables.tolist()) == list(range(math.ceil(1000 / 16)))  # a permutation
    keys = w.keys.float().numpy()
    # Planted keys: rows multiplied by 8 stand out of N(0, 1).
    assert np.abs(keys).max() > 8
