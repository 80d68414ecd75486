"""Candidate rows (Engine::project_candidates, needle2/csrc/engine.cpp:1302-1349) on the GPU.

The reference's own contract (tests/test_candidate_projection_dense.py in the
reference) is that a candidate projection equals the full projection indexed
by the candidates, exactly, keeping order and duplicates. Here every result is
compared bit for bit with the full GEMV of the same matrix and with the oracle,
on both sides of the switch between gathering candidate rows (fewer than half
of the rows) and running the whole matrix.
"""
import ctypes as ct

import numpy as np
import pytest

import oracle
from openneedle_amd.cq import CQMatrix
from openneedle_amd._ffi import GpuError, last_error
from openneedle_amd.device import DeviceArray, synchronize
from tests.cases import activations, baseline, example

pytestmark = pytest.mark.gpu


def candidate_ids(rng, rows, count):
    ids = rng.permutation(rows)[:count].astype(np.int32) if count <= rows else rng.integers(0, rows, count,
                                                                                            dtype=np.int32)
    ids[-1] = ids[0]  # duplicates and order must survive the gather
    return ids


@pytest.mark.parametrize("count", [1, 2, 7, 142, 255, 257, 4095, 4096, 7679, 8192, 9000])
def test_lm_head_candidates_fp32(count):
    """The LM-head geometry (8192 x 512 CQ4 g32)."""
    packed, norms, cb, _ = baseline(4, 8192, 512, seed=91)
    q = CQMatrix(packed, norms, (8192, 512), 4, 32, cb)
    x = activations(512, seed=count)
    ids = candidate_ids(np.random.default_rng(count), 8192, count)
    full = q.matvec(x)
    got = q.select(x, ids)
    np.testing.assert_array_equal(got, full[ids])
    np.testing.assert_array_equal(got, oracle.cq_linear(packed, norms, (8192, 512), 4, 32, cb, x, 8)[ids])


@pytest.mark.parametrize("count", [3, 142, 4096, 8192])
def test_lm_head_candidates_int8(count):
    packed, norms, cb, _ = baseline(4, 8192, 512, seed=92)
    q = CQMatrix(packed, norms, (8192, 512), 4, 32, cb)
    x = activations(512, seed=count + 1)
    ids = candidate_ids(np.random.default_rng(count + 1), 8192, count)
    got = q.select(x, ids, int8=True)
    np.testing.assert_array_equal(got, q.matvec_int8(x)[ids])
    np.testing.assert_array_equal(got, oracle.sdot_linear(packed, norms, (8192, 512), 4, 32, cb, x[None], 8)[0][ids])


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
@pytest.mark.parametrize("group", [8, 16, 32, 64, 128, 256, 512])
def test_ragged_candidates_fp32(bits, group):
    packed, norms, cb, dense = example(bits, rows=700, dim=1000, group=group, seed=bits * 100 + group)
    q = CQMatrix(packed, norms, dense.shape, bits, group, cb)
    x = activations(1000, seed=group)
    expected = oracle.cq_linear(packed, norms, dense.shape, bits, group, cb, x, 4)
    rng = np.random.default_rng(bits + group)
    for count in (5, 300, 700):  # two compact tiles (300 of 700 rows), then the whole matrix
        ids = candidate_ids(rng, 700, count)
        np.testing.assert_array_equal(q.select(x, ids), expected[ids])


@pytest.mark.parametrize("bits,group", [(4, 8), (4, 32), (4, 128), (2, 16), (2, 64), (2, 256)])
def test_ragged_candidates_int8(bits, group):
    packed, norms, cb, dense = example(bits, rows=700, dim=1000, group=group, seed=bits * 10 + group)
    q = CQMatrix(packed, norms, dense.shape, bits, group, cb)
    x = activations(1000, seed=group + 2)
    expected = oracle.sdot_linear(packed, norms, dense.shape, bits, group, cb, x[None])[0]
    rng = np.random.default_rng(group)
    for count in (9, 300, 699):
        ids = candidate_ids(rng, 700, count)
        np.testing.assert_array_equal(q.select(x, ids, int8=True), expected[ids])


def test_candidate_validation():
    packed, norms, cb, dense = example(4, rows=9, dim=257, group=32)
    q = CQMatrix(packed, norms, dense.shape, 4, 32, cb)
    x = activations(257, seed=1)
    with pytest.raises(GpuError, match="candidates must be nonempty"):
        q.select(x, [])
    with pytest.raises(ValueError, match="integer"):
        q.select(x, [1.0, 2.0])
    with pytest.raises(GpuError, match="outside vocabulary"):
        q.select(x, [0, 9])
    with pytest.raises(GpuError, match="outside vocabulary"):
        q.select(x, [-1], int8=True)
    # the C entry point makes the same checks itself
    lib = q._lib
    y = np.zeros(2, np.float32)
    for ids, message in ((np.array([3, 9], np.int32), "candidate outside vocabulary"),
                         (np.array([3, -2], np.int32), "candidate outside vocabulary")):
        assert lib.needle2_gpu_cq_candidates(q.handle, x.ctypes.data, ids.ctypes.data, 2, y.ctypes.data) == -1
        assert last_error() == message
    ok = np.array([3, 3], np.int32)
    assert lib.needle2_gpu_cq_candidates(q.handle, x.ctypes.data, ok.ctypes.data, 0, y.ctypes.data) == -1
    assert last_error() == "candidates must be nonempty"
    assert lib.needle2_gpu_cq_candidates(q.handle, x.ctypes.data, ok.ctypes.data, 2, y.ctypes.data) == 0
    np.testing.assert_array_equal(y, q.matvec(x)[[3, 3]])


@pytest.mark.parametrize("int8", [False, True])
def test_device_candidates(int8):
    """Device ids and outputs; an id outside the matrix yields NaN (and reads nothing)."""
    packed, norms, cb, _ = baseline(4, 2048, 512, seed=93)
    q = CQMatrix(packed, norms, (2048, 512), 4, 32, cb)
    x = activations(512, seed=5)
    full = q.matvec_int8(x) if int8 else q.matvec(x)
    d_x = DeviceArray.from_host(x)
    for count in (100, 1500):  # compact rows, then the whole matrix
        ids = candidate_ids(np.random.default_rng(count), 2048, count)
        bad = ids.copy()
        bad[7] = 2048
        bad[11] = -5
        d_ids = DeviceArray.from_host(bad)
        d_y = DeviceArray(4 * count)
        q.select_device(d_x.ptr, d_ids.ptr, count, d_y.ptr, int8=int8)
        synchronize()
        got = d_y.download(np.empty(count, np.float32))
        assert np.isnan(got[7]) and np.isnan(got[11])
        keep = np.ones(count, bool)
        keep[[7, 11]] = False
        np.testing.assert_array_equal(got[keep], full[ids][keep])
