"""GPU parity of the int8 ("SDOT") path: bit-exact with the oracle, whose
arithmetic is bit-exact with the reference's own SdotCQ (tests/test_oracle.py),
on identical seeded inputs."""
import numpy as np
import pytest

import oracle
from openneedle_amd.cq import CQMatrix, Plan
from openneedle_amd.device import DeviceArray, synchronize
from tests.cases import activations, baseline, example

pytestmark = pytest.mark.gpu


def special_inputs(dim, seed):
    x = activations((4, dim), seed=seed)
    x[0] = 0           # zero groups: scale 1, q 0
    x[1] = 0
    x[1, 0] = 1        # one-hot
    return x


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("group", [64, 128])
@pytest.mark.parametrize("rows", [9, 129])
def test_reference_domain_bit_exact(bits, group, rows):
    packed, norms, cb, dense = example(bits, rows=rows, dim=257, group=group)
    q = CQMatrix(packed, norms, dense.shape, bits, group, cb)
    x = special_inputs(257, seed=315)
    expected = oracle.sdot_linear(packed, norms, dense.shape, bits, group, cb, x)
    np.testing.assert_array_equal(q.matvec_int8(x, reference_bound=True), expected)
    np.testing.assert_array_equal(q.matvec_int8(x[2], reference_bound=True), expected[2])


def test_reference_group_bounds():
    """needle2_sdot_create keeps the reference's groups (sdot.cpp:351-354); needle2_sdot_linear refuses
    non-finite inputs (the reference's loader does, needle2/native.py:249-250) and poisons y with NaN."""
    from openneedle_amd._ffi import GpuError
    packed, norms, cb, dense = example(4, group=32)
    q = CQMatrix(packed, norms, dense.shape, 4, 32, cb)
    with pytest.raises(GpuError, match="group"):
        q.matvec_int8(np.ones(257, np.float32), reference_bound=True)
    q128 = CQMatrix(*example(4)[:2], (9, 257), 4, 128, example(4)[2])
    with pytest.raises(GpuError, match="finite"):
        q128.matvec_int8(np.full(257, np.nan, np.float32), reference_bound=True)


@pytest.mark.parametrize("bits,group", [(4, 8), (4, 16), (4, 32), (2, 16), (2, 32), (4, 256), (2, 512), (4, 1024)])
def test_extended_groups_bit_exact(bits, group):
    packed, norms, cb, dense = example(bits, rows=300, dim=1000, group=group, seed=group + bits)
    q = CQMatrix(packed, norms, dense.shape, bits, group, cb)
    x = special_inputs(1000, seed=group)
    np.testing.assert_array_equal(q.matvec_int8(x), oracle.sdot_linear(packed, norms, dense.shape, bits, group, cb, x))


@pytest.mark.parametrize("group", [32, 128, 256])
def test_subnormal_scale_guard(group):
    """Subnormal inputs (absmax / 127 underflows to zero: the scale is absmax itself), a zero group and a
    one-hot group, through the one-wave-per-group prepare kernels (groups of up to 64 positions per wave, or
    GROUP / 64 positions per lane for 128 and 256)."""
    dim = 4 * group + 7
    packed, norms, cb, dense = example(4, rows=40, dim=dim, group=group, seed=group)
    q = CQMatrix(packed, norms, dense.shape, 4, group, cb)
    x = np.zeros((2, dim), np.float32)
    x[0, :group] = np.float32(4e-45)
    x[0, group + 8] = np.float32(1e-39)
    x[0, 3 * group + 1] = 1
    x[1] = activations((1, dim), seed=group)[0]
    x[1, group:2 * group] = 0
    np.testing.assert_array_equal(q.matvec_int8(x), oracle.sdot_linear(packed, norms, dense.shape, 4, group, cb, x))
    np.testing.assert_array_equal(q.matvec_int8(x[1]), oracle.sdot_linear(packed, norms, dense.shape, 4, group, cb,
                                                                          x[1:])[0])


@pytest.mark.parametrize("batch", [1, 4, 16])
def test_int8_4096_square_batches(batch):
    """CQ4 4096 x 4096 g32, activations quantized per group after the FWHT."""
    packed, norms, cb, _ = baseline(4, 4096, 4096, seed=33)
    q = CQMatrix(packed, norms, (4096, 4096), 4, 32, cb)
    x = activations((batch, 4096), seed=batch)
    np.testing.assert_array_equal(q.matvec_int8(x), oracle.sdot_linear(packed, norms, (4096, 4096), 4, 32, cb, x, 8))


def test_int8_plan_many_matrices():
    mats, d_x, d_y, expected = [], [], [], []
    for i in range(3):
        packed, norms, cb, _ = baseline(4, 512 + 64 * i, 1024, seed=500 + i)
        m = CQMatrix(packed, norms, (512 + 64 * i, 1024), 4, 32, cb)
        x = activations((2, 1024), seed=600 + i)
        mats.append(m)
        expected.append(oracle.sdot_linear(packed, norms, m.shape, 4, 32, cb, x))
        d_x.append(DeviceArray.from_host(x))
        d_y.append(DeviceArray(2 * 4 * m.shape[0]))
    plan = Plan(mats, [d.ptr for d in d_x], [d.ptr for d in d_y], batch=2, int8=True)
    plan.run()
    synchronize()
    for m, dy, e in zip(mats, d_y, expected):
        np.testing.assert_array_equal(dy.download(np.empty((2, m.shape[0]), np.float32)), e)


@pytest.mark.parametrize("mode", ["tile16", "quad", "always", "never", "ksplit", "ksplit_w8", "ksplit_w16",
                                  "ksplit_r16", "ksplit_r32", "ksplit32", "ksplit32_w16"])
@pytest.mark.parametrize("bits,group,batch", [(4, 32, 3), (4, 32, 9), (4, 32, 17), (4, 32, 33), (4, 32, 64),
                                              (4, 64, 40), (4, 128, 12), (4, 256, 5), (2, 32, 8), (2, 32, 33),
                                              (2, 64, 20), (4, 8, 6), (4, 16, 16), (2, 16, 2), (4, 32, 2)])
def test_int8_batched_tiles_bit_exact(bits, group, batch, mode, monkeypatch):
    """Batches of 2 or more on each kernel, forced here (the library picks by size otherwise): 16 x 16 x 32
    int8 MFMA batch tiles of 16 rows (tile16: ragged last tile; groups below one code chunk fall back to the
    quad kernel), 4 x 4 x 4 int8 MFMA batch tiles of up to 16 rows, one lane per weight row (quad: ragged last
    quad and tile), 32 x 32 x 32 int8 MFMA tiles of 32 batch rows (always), v_dot4 batch tiles (never) and the
    K split on 16 x 16 tiles (ksplit; 4-bit codes, else 32 x 32; over 8 or 16 waves per tile by the group
    count, or forced: ksplit_w8 / ksplit_w16; 16- or 32-row workgroups: ksplit_r16 / ksplit_r32) and on
    32 x 32 tiles (ksplit32, ksplit32_w16); 300 ragged weight rows, zero / one-hot activation rows: bit-exact
    with the oracle."""
    if mode.startswith("ksplit"):  # K split over the waves of a tile (small-matrix path)
        monkeypatch.setenv("NEEDLE2_GPU_INT8_KSPLIT", "always")
        monkeypatch.setenv("NEEDLE2_GPU_INT8_KS16", "never" if mode.startswith("ksplit32") else "auto")
        if "_w" in mode:
            monkeypatch.setenv("NEEDLE2_GPU_INT8_KS16_WAVES", mode.split("_w")[1])
        if "_r" in mode:  # 16- or 32-row workgroups of the 16 x 16 K split
            monkeypatch.setenv("NEEDLE2_GPU_INT8_KS16_ROWS", mode.split("_r")[1])
    else:
        monkeypatch.setenv("NEEDLE2_GPU_INT8_KSPLIT", "never")
        monkeypatch.setenv("NEEDLE2_GPU_INT8_TILE16", "always" if mode == "tile16" else "never")
        if mode == "never":
            monkeypatch.setenv("NEEDLE2_GPU_INT8_QUAD", "never")
        monkeypatch.setenv("NEEDLE2_GPU_INT8_MFMA", "auto" if mode in ("quad", "tile16") else mode)
    packed, norms, cb, dense = example(bits, rows=300, dim=1000, group=group, seed=7 * batch + group)
    q = CQMatrix(packed, norms, dense.shape, bits, group, cb)
    x = activations((batch, 1000), seed=batch)
    x[0] = 0
    if batch > 2:
        x[2] = 0
        x[2, 5] = 1
    np.testing.assert_array_equal(q.matvec_int8(x), oracle.sdot_linear(packed, norms, dense.shape, bits, group, cb, x))


@pytest.mark.parametrize("mode", ["always", "auto", "ksplit32"])
def test_int8_plan_decode_batch(mode, monkeypatch):
    """A layer's Q | K | V projections for 64 sequences in one plan (one prepare and one GEMV launch): the
    16 x 16 K-split kernel (auto), the 32 x 32 K-split kernel (ksplit32), the 32 x 32 x 32 MFMA kernel
    (always)."""
    monkeypatch.setenv("NEEDLE2_GPU_INT8_MFMA", "always" if mode == "always" else "auto")
    if mode == "ksplit32":
        monkeypatch.setenv("NEEDLE2_GPU_INT8_KS16", "never")
    mats, d_x, d_y, expected = [], [], [], []
    x = activations((64, 512), seed=640)
    d_in = DeviceArray.from_host(x)
    for i in range(3):
        packed, norms, cb, _ = baseline(4, 512, 512, seed=700 + i)
        m = CQMatrix(packed, norms, (512, 512), 4, 32, cb)
        mats.append(m)
        expected.append(oracle.sdot_linear(packed, norms, m.shape, 4, 32, cb, x))
        d_y.append(DeviceArray(64 * 4 * 512))
    plan = Plan(mats, [d_in.ptr] * 3, [d.ptr for d in d_y], batch=64, int8=True)
    for _ in range(2):
        plan.run()
        synchronize()
        for dy, e in zip(d_y, expected):
            np.testing.assert_array_equal(dy.download(np.empty((64, 512), np.float32)), e)


@pytest.mark.parametrize("xin", ["auto", "never"])
@pytest.mark.parametrize("bits,group,rows,dim", [(4, 32, 512, 512), (4, 32, 2048, 512), (4, 32, 512, 2048),
                                                 (2, 128, 1536, 512), (4, 64, 300, 1000), (2, 256, 257, 1300),
                                                 (2, 32, 640, 777)])
def test_int8_plan_batch1_input_prepared_in_gemv(bits, group, rows, dim, xin, monkeypatch):
    """Batch-1 plans of small matrices (decode projections) run the 32 x 32 K-split GEMV, which prepares the
    input row itself (auto: no prepare launch) or reads the prepare kernel's output (never): three matrices
    over one input with a zero group and a one-hot group, two runs in a row, bit-exact with the oracle."""
    monkeypatch.setenv("NEEDLE2_GPU_INT8_XIN", xin)
    x = activations((1, dim), seed=rows + dim)
    x[0, :group] = 0
    if dim > 2 * group:
        x[0, group:2 * group] = 0
        x[0, group + 3] = -2.5
    d_in = DeviceArray.from_host(x)
    mats, d_y, expected = [], [], []
    for i in range(3):
        packed, norms, cb, dense = example(bits, rows=rows, dim=dim, group=group, seed=900 + 7 * i + group)
        mats.append(CQMatrix(packed, norms, dense.shape, bits, group, cb))
        expected.append(oracle.sdot_linear(packed, norms, dense.shape, bits, group, cb, x))
        d_y.append(DeviceArray(rows * 4))
    plan = Plan(mats, [d_in.ptr] * 3, [d.ptr for d in d_y], batch=1, int8=True)
    for _ in range(2):
        for d in d_y:
            d.fill(0x7F)
        plan.run()
        synchronize()
        for dy, e in zip(d_y, expected):
            np.testing.assert_array_equal(dy.download(np.empty((1, rows), np.float32)), e)


@pytest.mark.parametrize("prepare", ["oct", "lane"])
@pytest.mark.parametrize("bits,group,dim", [(4, 8, 1000), (4, 16, 777), (4, 32, 4100), (4, 64, 1300), (2, 16, 1000),
                                            (2, 32, 777), (2, 64, 2100)])
def test_int8_prepare_kernels_bit_exact(bits, group, dim, prepare, monkeypatch):
    """Groups of 8 .. 64: the prepare kernel with eight positions per thread (oct, the default for large
    inputs) and with one (lane), forced by NEEDLE2_GPU_INT8_PREPARE, batches 1 and 5 with zero, one-hot and
    ragged rows, through the GEMV: bit-exact with the oracle."""
    monkeypatch.setenv("NEEDLE2_GPU_INT8_PREPARE", prepare)
    monkeypatch.setenv("NEEDLE2_GPU_INT8_XIN", "never")  # batch 1 through the prepare kernel too
    packed, norms, cb, dense = example(bits, rows=200, dim=dim, group=group, seed=dim * 3 + group)
    q = CQMatrix(packed, norms, dense.shape, bits, group, cb)
    x = activations((5, dim), seed=group + bits)
    x[1] = 0
    x[3] = 0
    x[3, dim - 1] = 2.5
    want = oracle.sdot_linear(packed, norms, dense.shape, bits, group, cb, x)
    np.testing.assert_array_equal(q.matvec_int8(x), want)
    np.testing.assert_array_equal(q.matvec_int8(x[3:4]), want[3:4])


@pytest.mark.parametrize("mode", ["auto", "never", "ksplit", "ksplit16"])
@pytest.mark.parametrize("bits,group,dim", [(4, 8, 1000), (4, 32, 1000), (4, 64, 4096), (4, 256, 1300), (2, 16, 1000),
                                            (2, 32, 777), (2, 128, 2048)])
def test_int8_single_row_kernels_bit_exact(bits, group, dim, mode, monkeypatch):
    """Batch 1 (decode): the barrier-free row kernel (auto), the windowed kernel (never) and the K split on
    32 x 32 (ksplit) and 16 x 16 tiles (ksplit16, 4-bit codes), ragged shapes, zero and one-hot inputs,
    bit-exact with the oracle."""
    if mode.startswith("ksplit"):
        if group < 32:
            pytest.skip("the K-split path takes groups of 32 .. 256")
        monkeypatch.setenv("NEEDLE2_GPU_INT8_KSPLIT", "always")
        monkeypatch.setenv("NEEDLE2_GPU_INT8_KS16", "always" if mode == "ksplit16" else "never")
    else:
        monkeypatch.setenv("NEEDLE2_GPU_INT8_KSPLIT", "never")
        monkeypatch.setenv("NEEDLE2_GPU_INT8_ROW", mode)
    packed, norms, cb, dense = example(bits, rows=300, dim=dim, group=group, seed=dim + group)
    q = CQMatrix(packed, norms, dense.shape, bits, group, cb)
    for x in special_inputs(dim, seed=group + 1):
        np.testing.assert_array_equal(q.matvec_int8(x), oracle.sdot_linear(packed, norms, dense.shape, bits, group,
                                                                           cb, x[None])[0])

