"""bench.py's host-side contract: the one-GPU guard and the timing summaries (no GPU needed)."""
import subprocess
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and not r.stdout


def test_dist_us_percentiles():
    ms = [i / 1000 for i in range(1, 102)]  # 1 .. 101 us
    d = bench.dist_us(ms)
    assert d == {"mean": 51.0, "median": 51.0, "p10": 11.0, "p90": 91.0, "n": 101}


def test_cpu_time_bounds_runs():
    calls = []
    med, p10, p90, n = bench._cpu_time(lambda: calls.append(1), budget_s=0.0, min_runs=7, warmup=2)
    assert n == 7 and len(calls) == 9
    assert 0 <= p10 <= med <= p90


def test_random_cq_shapes():
    packed, norms, cb = bench.random_cq(np.random.default_rng(0), 2, 16, 64, 2, 32)
    assert packed.shape == (2, 16, 16) and packed.dtype == np.uint8
    assert norms.shape == (2, 16, 2) and norms.dtype == np.float16
    assert (norms >= np.float16(0.005)).all() and (norms <= np.float16(0.05)).all()
    np.testing.assert_array_equal(cb, [-2, -1, 0, 1])
