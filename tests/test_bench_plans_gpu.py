"""The launches bench.py times, checked against the oracle.

bench.py's figures come from multi-matrix plans built by its ``Stack``: 16
CQ4 (or CQ2) 8192 x 8192 group-32 matrices at batch 1 on the FP32 path (the
headline), and 64 CQ4 4096 x 4096 group-32 matrices at batch 1, 4 and 16 on
the int8 path. These tests build the same stacks through the same code (one
rotation instead of three), run each plan once, and compare every matrix's
output with the oracle: bit-exact on both paths.
"""
import os

import numpy as np
import pytest

import bench
import oracle
from openneedle_amd.device import Stream

pytestmark = pytest.mark.gpu

CORES = max(1, min(16, len(os.sched_getaffinity(0))))


def run_stack(bits, count, rows, batch, int8, seed):
    packed, norms, cb = bench.random_cq(np.random.default_rng(seed), count, rows, rows, bits, 32)
    st = bench.Stack(packed, norms, cb, bits, 32, batch=batch, rot=1, int8=int8)
    with Stream() as stream:
        st.plans[0].run(stream)
        stream.synchronize()
    xs = [d.to_host(np.float32, (batch, rows)) for d in st.x]
    ys = [d.to_host(np.float32, (batch, rows)) for d in st.y]
    return packed, norms, cb, xs, ys


@pytest.mark.parametrize("bits", [4, 2])
def test_fp32_stack_16x8192(bits):
    packed, norms, cb, xs, ys = run_stack(bits, 16, 8192, 1, False, seed=20261201 + bits)
    for i in range(16):
        print(f"matrix {i}", flush=True)
        expected = oracle.cq_linear(packed[i], norms[i], (8192, 8192), bits, 32, cb, xs[i], CORES)
        np.testing.assert_array_equal(ys[i], expected, err_msg=f"matrix {i}")


@pytest.mark.parametrize("batch", [1, 4, 16])
def test_int8_stack_64x4096(batch):
    packed, norms, cb, xs, ys = run_stack(4, 64, 4096, batch, True, seed=20261203 + batch)
    for i in range(64):
        expected = oracle.sdot_linear(packed[i], norms[i], (4096, 4096), 4, 32, cb, xs[i], CORES)
        np.testing.assert_array_equal(ys[i], expected, err_msg=f"matrix {i}")
