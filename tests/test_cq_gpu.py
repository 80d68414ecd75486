"""GPU parity of the FP32 CQ path against the oracle (same seeded inputs).

Bar: bit-identical to the oracle (which is bit-identical to the reference's
own portable build, tests/test_oracle.py) for every bit width - stronger than
the 1e-5 relative / 1e-6 absolute per-output requirement. Results are also
checked against the fp64 dense closed form with the reference test's
tolerance (atol=3e-6, rtol=2e-5, tests/test_native.py:40 in the reference).
"""
import numpy as np
import pytest

import oracle
from openneedle_amd import formats
from openneedle_amd.native import DeviceArray, NativeCQ, Plan, synchronize
from tests.cases import activations, baseline, example

pytestmark = pytest.mark.gpu

def check(got, expected, bits):
    np.testing.assert_array_equal(got, expected)


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
def test_reference_example_all_modes(bits):
    packed, norms, cb, dense = example(bits)
    q = NativeCQ(packed, norms, dense.shape, bits, 128, cb)
    x = activations((2, 3, 257))
    expected = oracle.cq_linear(packed, norms, dense.shape, bits, 128, cb, x)
    for threads in (1, 2):
        for lookup in (0, 1, 2, 3):
            got = q.linear(x, threads, lookup=lookup)
            assert got.shape == (2, 3, 9)
            check(got, expected, bits)
            np.testing.assert_allclose(got, x.astype(np.float64) @ dense.T, atol=3e-6, rtol=2e-5)
    assert np.all(got[..., 0] == 0)
    ids = np.array([[8, 2], [0, 2]])
    np.testing.assert_array_equal(q.rows(ids), oracle.cq_rows(packed, norms, dense.shape, bits, 128, cb, ids))
    np.testing.assert_allclose(q.dequantize(), dense, atol=2e-7, rtol=3e-5)
    np.testing.assert_allclose(q.rows(2), dense[2], atol=2e-7, rtol=3e-5)


def test_bounds_and_empty_batch():
    packed, norms, cb, dense = example(2)
    q = NativeCQ(packed, norms, dense.shape, 2, 128, cb)
    with pytest.raises(IndexError):
        q.rows([-1])
    with pytest.raises(IndexError):
        q.rows([q.shape[0]])
    with pytest.raises(TypeError):
        q.rows([1.5])
    with pytest.raises(ValueError):
        q.linear(np.ones(256))
    assert q.linear(np.empty((0, 257))).shape == (0, 9)


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
@pytest.mark.parametrize("group", [8, 16, 32, 64, 128, 256, 512, 1024])
@pytest.mark.parametrize("rows,dim", [(33, 200), (300, 1000)])
def test_groups_and_ragged_shapes(bits, group, rows, dim):
    packed, norms, cb, dense = example(bits, rows=rows, dim=dim, group=group, seed=bits * 1000 + group)
    q = NativeCQ(packed, norms, dense.shape, bits, group, cb)
    x = activations((3, dim), seed=group)
    expected = oracle.cq_linear(packed, norms, dense.shape, bits, group, cb, x, 4)
    check(q.linear(x), expected, bits)


def test_huge_group_global_fwht():
    """group > 16384 runs the FWHT as global-memory butterfly stages."""
    bits, group, dim = 4, 32768, 40000
    packed, norms, cb, dense = example(bits, rows=7, dim=dim, group=group, seed=5)
    q = NativeCQ(packed, norms, dense.shape, bits, group, cb)
    x = activations((2, dim), seed=6)
    np.testing.assert_array_equal(q.linear(x), oracle.cq_linear(packed, norms, dense.shape, bits, group, cb, x, 4))
    np.testing.assert_array_equal(q.rows([3, 0]), oracle.cq_rows(packed, norms, dense.shape, bits, group, cb, [3, 0]))


def test_lloyd_max_codebook():
    for bits in (2, 3, 4):
        packed, norms, _, _ = baseline(bits, 512, 1024, group=128, seed=bits)
        cb = formats.codebook(bits, 128)
        q = NativeCQ(packed, norms, (512, 1024), bits, 128, cb)
        x = activations((2, 1024), seed=bits)
        check(q.linear(x), oracle.cq_linear(packed, norms, (512, 1024), bits, 128, cb, x, 4), bits)


def test_single_token_decode_shape_bit_exact():
    """2048 x 512 CQ4 g32, batch 1 (the CPU-runnable decode GEMV)."""
    packed, norms, cb, _ = baseline(4, 2048, 512)
    q = NativeCQ(packed, norms, (2048, 512), 4, 32, cb)
    x = activations(512, seed=11)
    np.testing.assert_array_equal(q.linear(x), oracle.cq_linear(packed, norms, (2048, 512), 4, 32, cb, x, 8))


@pytest.mark.parametrize("bits", [2, 4])
def test_full_size_8192_matrix(bits):
    """One 8192 x 8192 g32 matrix of the HBM-bound stack, batch 1 and 2."""
    packed, norms, cb, _ = baseline(bits, 8192, 8192, seed=77 + bits)
    q = NativeCQ(packed, norms, (8192, 8192), bits, 32, cb)
    x = activations((2, 8192), seed=12)
    expected = oracle.cq_linear(packed, norms, (8192, 8192), bits, 32, cb, x, 8)
    check(q.linear(x), expected, bits)
    check(q.linear(x[1]), expected[1], bits)


def test_device_entry_and_plan():
    mats, xs, expected = [], [], []
    for i in range(3):
        packed, norms, cb, _ = baseline(4, 1000 + 256 * i, 768, seed=300 + i)
        mats.append(NativeCQ(packed, norms, (1000 + 256 * i, 768), 4, 32, cb))
        x = activations(768, seed=400 + i)
        xs.append(x)
        expected.append(oracle.cq_linear(packed, norms, mats[-1].shape, 4, 32, cb, x))
    d_x = [DeviceArray.from_host(x) for x in xs]
    d_y = [DeviceArray(4 * m.shape[0]) for m in mats]
    for m, dx, dy, e in zip(mats, d_x, d_y, expected):
        m.linear_device(dx.ptr, dy.ptr, 1)
        synchronize()
        np.testing.assert_array_equal(dy.download(np.empty(m.shape[0], np.float32)), e)
    for dy in d_y:
        dy.upload(np.full(dy.nbytes // 4, np.nan, np.float32))
    plan = Plan(mats, [d.ptr for d in d_x], [d.ptr for d in d_y])
    for _ in range(2):
        plan.run()
        synchronize()
        for m, dy, e in zip(mats, d_y, expected):
            np.testing.assert_array_equal(dy.download(np.empty(m.shape[0], np.float32)), e)
