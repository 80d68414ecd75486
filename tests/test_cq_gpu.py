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
from openneedle_amd.cq import CQMatrix, Plan
from openneedle_amd.device import DeviceArray, synchronize
from tests.cases import activations, baseline, example

pytestmark = pytest.mark.gpu

def check(got, expected, bits):
    np.testing.assert_array_equal(got, expected)


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
def test_reference_example_all_modes(bits):
    packed, norms, cb, dense = example(bits)
    q = CQMatrix(packed, norms, dense.shape, bits, 128, cb)
    x = activations((2, 3, 257))
    expected = oracle.cq_linear(packed, norms, dense.shape, bits, 128, cb, x)
    for lookup in (0, 1, 2, 3):
        got = q.matvec(x, mode=lookup)
        assert got.shape == (2, 3, 9)
        check(got, expected, bits)
        np.testing.assert_allclose(got, x.astype(np.float64) @ dense.T, atol=3e-6, rtol=2e-5)
    assert np.all(got[..., 0] == 0)
    ids = np.array([[8, 2], [0, 2]])
    np.testing.assert_array_equal(q.rows(ids), oracle.cq_rows(packed, norms, dense.shape, bits, 128, cb, ids))
    np.testing.assert_allclose(q.dense(), dense, atol=2e-7, rtol=3e-5)
    np.testing.assert_allclose(q.rows(2), dense[2], atol=2e-7, rtol=3e-5)


def test_bounds_and_empty_batch():
    packed, norms, cb, dense = example(2)
    q = CQMatrix(packed, norms, dense.shape, 2, 128, cb)
    from openneedle_amd._ffi import GpuError
    with pytest.raises(GpuError, match="outside"):
        q.rows([-1])
    with pytest.raises(GpuError, match="outside"):
        q.rows([q.shape[0]])
    with pytest.raises(TypeError):
        q.rows([1.5])
    with pytest.raises(ValueError):
        q.matvec(np.ones(256))
    assert q.matvec(np.empty((0, 257))).shape == (0, 9)


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
@pytest.mark.parametrize("group", [8, 16, 32, 64, 128, 256, 512, 1024])
@pytest.mark.parametrize("rows,dim", [(33, 200), (300, 1000), (70, 777)])
def test_groups_and_ragged_shapes(bits, group, rows, dim):
    packed, norms, cb, dense = example(bits, rows=rows, dim=dim, group=group, seed=bits * 1000 + group)
    q = CQMatrix(packed, norms, dense.shape, bits, group, cb)
    x = activations((3, dim), seed=group)
    expected = oracle.cq_linear(packed, norms, dense.shape, bits, group, cb, x, 4)
    check(q.matvec(x), expected, bits)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("group", [8, 16, 32, 64])
@pytest.mark.parametrize("dim", [300, 777])
def test_small_groups_with_and_without_prepass(bits, group, dim, monkeypatch):
    """Groups of 8 .. 64: the quarter-split GEMV transforms the raw input itself (NEEDLE2_GPU_FP32_XF=always;
    by default for inputs of at most 512) or reads the activation pre-pass (never; by default for wider
    inputs); every mode bit-exact, through the host call and a plan."""
    packed, norms, cb, dense = example(bits, rows=300, dim=dim, group=group, seed=bits * 77 + group)
    x = activations((2, dim), seed=group + 5)
    expected = oracle.cq_linear(packed, norms, dense.shape, bits, group, cb, x, 4)
    for mode in ("always", "never", "auto"):
        monkeypatch.setenv("NEEDLE2_GPU_FP32_XF", mode)
        q = CQMatrix(packed, norms, dense.shape, bits, group, cb)
        check(q.matvec(x), expected, bits)
        d_x = DeviceArray.from_host(np.ascontiguousarray(x[1]))
        d_y = DeviceArray(4 * dense.shape[0])
        plan = Plan([q], [d_x.ptr], [d_y.ptr])
        plan.run()
        synchronize()
        check(d_y.download(np.empty(dense.shape[0], np.float32)), expected[1], bits)


@pytest.mark.parametrize("group", [8, 16, 32, 64])
@pytest.mark.parametrize("batch", [2, 3, 5])
@pytest.mark.parametrize("dim", [300, 1000])
def test_batched_rows_in_pairs(group, batch, dim, monkeypatch):
    """4-bit batches of two or more rows take two rows per pass over the codes (cq_gemv_quad_pair_kernel: the
    chunks loaded once for both rows' tables, an odd last row alone), for raw inputs (<= 512 wide) and the
    pre-pass; bit-identical to the oracle and to one row per pass (NEEDLE2_GPU_FP32_PAIRS=never)."""
    packed, norms, cb, dense = example(4, rows=300, dim=dim, group=group, seed=31 * group + batch)
    x = activations((batch, dim), seed=group + batch)
    expected = oracle.cq_linear(packed, norms, dense.shape, 4, group, cb, x, 4)
    for mode in ("auto", "never"):
        monkeypatch.setenv("NEEDLE2_GPU_FP32_PAIRS", mode)
        q = CQMatrix(packed, norms, dense.shape, 4, group, cb)
        check(q.matvec(x), expected, 4)
        d_x = DeviceArray.from_host(np.ascontiguousarray(x))
        d_y = DeviceArray(4 * batch * dense.shape[0])
        plan = Plan([q], [d_x.ptr], [d_y.ptr], batch=batch)
        plan.run()
        synchronize()
        check(d_y.download(np.empty((batch, dense.shape[0]), np.float32)), expected, 4)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("dim", [257, 400, 512])
def test_two_window_inputs_window_parallel(bits, dim, monkeypatch):
    """Groups of 128 over inputs of two windows (257 .. 512 positions: a decode step's attention projections):
    the window-parallel kernel (default) and the split kernel (NEEDLE2_GPU_FP32_WSPLIT=never), batch 1 and 3,
    ragged rows, through the host call and a plan: bit-exact with the oracle."""
    packed, norms, cb, dense = example(bits, rows=300, dim=dim, group=128, seed=bits * 10 + dim)
    x = activations((3, dim), seed=dim)
    expected = oracle.cq_linear(packed, norms, dense.shape, bits, 128, cb, x, 4)
    for mode in ("auto", "never"):
        monkeypatch.setenv("NEEDLE2_GPU_FP32_WSPLIT", mode)
        q = CQMatrix(packed, norms, dense.shape, bits, 128, cb)
        check(q.matvec(x), expected, bits)
        check(q.matvec(x[1:2]), expected[1:2], bits)
        d_x = DeviceArray.from_host(np.ascontiguousarray(x))
        d_y = DeviceArray(4 * 3 * dense.shape[0])
        plan = Plan([q], [d_x.ptr], [d_y.ptr], batch=3)
        plan.run()
        synchronize()
        check(d_y.download(np.empty((3, dense.shape[0]), np.float32)), expected, bits)


@pytest.mark.parametrize("group,dim", [(32, 1000), (128, 1000), (128, 300), (1024, 1500)])
def test_host_calls_in_a_row(group, dim):
    """The host-pointer call reads x from its pinned staging buffer in place (or a device copy of it where a
    GEMV would re-read a wide row) and writes y straight back: successive calls on one handle with new inputs
    and growing batches (the staging reallocated) each match the oracle."""
    packed, norms, cb, dense = example(4, rows=300, dim=dim, group=group, seed=group + dim)
    q = CQMatrix(packed, norms, dense.shape, 4, group, cb)
    for k, batch in enumerate((1, 1, 3, 2, 7, 1)):
        x = activations((batch, dim), seed=100 + k)
        check(q.matvec(x), oracle.cq_linear(packed, norms, dense.shape, 4, group, cb, x, 4), 4)
        if group <= 256 and group >= 16:
            want = oracle.sdot_linear(packed, norms, dense.shape, 4, group, cb, x)
            np.testing.assert_array_equal(q.matvec_int8(x), want)


def test_huge_group_global_fwht():
    """group > 16384 runs the FWHT as global-memory butterfly stages."""
    bits, group, dim = 4, 32768, 40000
    packed, norms, cb, dense = example(bits, rows=7, dim=dim, group=group, seed=5)
    q = CQMatrix(packed, norms, dense.shape, bits, group, cb)
    x = activations((2, dim), seed=6)
    np.testing.assert_array_equal(q.matvec(x), oracle.cq_linear(packed, norms, dense.shape, bits, group, cb, x, 4))
    np.testing.assert_array_equal(q.rows([3, 0]), oracle.cq_rows(packed, norms, dense.shape, bits, group, cb, [3, 0]))


def test_lloyd_max_codebook():
    for bits in (2, 3, 4):
        packed, norms, _, _ = baseline(bits, 512, 1024, group=128, seed=bits)
        cb = formats.codebook(bits, 128)
        q = CQMatrix(packed, norms, (512, 1024), bits, 128, cb)
        x = activations((2, 1024), seed=bits)
        check(q.matvec(x), oracle.cq_linear(packed, norms, (512, 1024), bits, 128, cb, x, 4), bits)


def test_single_token_decode_shape_bit_exact():
    """2048 x 512 CQ4 g32, batch 1 (the CPU-runnable decode GEMV)."""
    packed, norms, cb, _ = baseline(4, 2048, 512)
    q = CQMatrix(packed, norms, (2048, 512), 4, 32, cb)
    x = activations(512, seed=11)
    np.testing.assert_array_equal(q.matvec(x), oracle.cq_linear(packed, norms, (2048, 512), 4, 32, cb, x, 8))


@pytest.mark.parametrize("bits", [2, 4])
def test_full_size_8192_matrix(bits):
    """One 8192 x 8192 g32 matrix of the HBM-bound stack, batch 1 and 2."""
    packed, norms, cb, _ = baseline(bits, 8192, 8192, seed=77 + bits)
    q = CQMatrix(packed, norms, (8192, 8192), bits, 32, cb)
    x = activations((2, 8192), seed=12)
    expected = oracle.cq_linear(packed, norms, (8192, 8192), bits, 32, cb, x, 8)
    check(q.matvec(x), expected, bits)
    check(q.matvec(x[1]), expected[1], bits)


def test_device_entry_and_plan():
    mats, xs, expected = [], [], []
    for i in range(3):
        packed, norms, cb, _ = baseline(4, 1000 + 256 * i, 768, seed=300 + i)
        mats.append(CQMatrix(packed, norms, (1000 + 256 * i, 768), 4, 32, cb))
        x = activations(768, seed=400 + i)
        xs.append(x)
        expected.append(oracle.cq_linear(packed, norms, mats[-1].shape, 4, 32, cb, x))
    d_x = [DeviceArray.from_host(x) for x in xs]
    d_y = [DeviceArray(4 * m.shape[0]) for m in mats]
    for m, dx, dy, e in zip(mats, d_x, d_y, expected):
        m.matvec_device(dx.ptr, dy.ptr, 1)
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


def _many_case(specs, seed):
    """Matrices of the given (rows, bits, group, dim) with their oracle inputs."""
    mats, refs = [], []
    for i, (rows, bits, group, dim) in enumerate(specs):
        packed, norms, cb, dense = example(bits, rows=rows, dim=dim, group=group, seed=seed + i)
        mats.append(CQMatrix(packed, norms, dense.shape, bits, group, cb))
        refs.append((packed, norms, dense.shape, bits, group, cb))
    return mats, refs


@pytest.mark.parametrize("mode", [0, 1, 4])
def test_linear_many_shared_transform(mode):
    """needle2_cq_linear_many (cq.cpp:287-292, 360-366): matrices of one input length and group share one
    transform; runs of one storage geometry share a GEMV launch. Mixed widths, codebooks and row counts
    (group 32: pre-pass FWHT; group 128: FWHT fused in the GEMV)."""
    from openneedle_amd.cq import matvec_many
    for group in (32, 128):
        specs = [(300, 4, group, 700), (257, 4, group, 700), (1000, 2, group, 700), (9, 5, group, 700),
                 (64, 3, group, 700), (513, 4, group, 700)]
        mats, refs = _many_case(specs, seed=900 + group)
        x = activations(700, seed=group)
        for out, ref in zip(matvec_many(mats, x, mode=mode), refs):
            np.testing.assert_array_equal(out, oracle.cq_linear(*ref, x))


def test_linear_many_falls_back_per_matrix():
    """Different groups (or input lengths) cannot share a transform: each matrix runs alone, same outputs."""
    from openneedle_amd.cq import matvec_many
    mats, refs = _many_case([(100, 4, 32, 512), (200, 2, 64, 512), (50, 4, 128, 512)], seed=950)
    x = activations(512, seed=951)
    for out, ref in zip(matvec_many(mats, x), refs):
        np.testing.assert_array_equal(out, oracle.cq_linear(*ref, x))
