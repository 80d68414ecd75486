"""GPU parity of the prefill CQ GEMM (fp16 MFMA, fp32 accumulation).

Bar: normwise relative error ||Y - Y_ref|| / ||Y_ref|| <= 2e-3 against the
oracle's FP32 path (bit-identical to the reference's CQ::linear,
tests/test_oracle.py) on the same seeded inputs; activations and the weights
cb*norm are rounded to fp16 on the way into the MFMA, so a per-element bound
is not meaningful where outputs cancel. Each row of Y is also checked
normwise against the fp64 dense closed form.
"""
import numpy as np
import pytest

import oracle
from openneedle_amd import formats
from openneedle_amd.cq import CQMatrix
from openneedle_amd.device import DeviceArray, synchronize
from tests.cases import activations, baseline, example

pytestmark = pytest.mark.gpu

NORMWISE = 2e-3


def gemm(q, x):
    m = x.shape[0]
    d_x = DeviceArray.from_host(np.ascontiguousarray(x, np.float32))
    d_y = DeviceArray(m * q.shape[0] * 4)
    d_y.upload(np.full((m, q.shape[0]), np.nan, np.float32))
    q.gemm_device(d_x.ptr, d_y.ptr, m)
    synchronize()
    return d_y.download(np.empty((m, q.shape[0]), np.float32))


def normwise(got, ref):
    return float(np.linalg.norm(got - ref) / np.linalg.norm(ref))


def test_prefill_chunk_full_size():
    """512 tokens x K 2048 through a CQ4 8192 x 2048 g32 matrix."""
    packed, norms, cb, _ = baseline(4, 8192, 2048, seed=41)
    q = CQMatrix(packed, norms, (8192, 2048), 4, 32, cb)
    x = activations((512, 2048), seed=42)
    got = gemm(q, x)
    ref = oracle.cq_linear(packed, norms, (8192, 2048), 4, 32, cb, x, 16)
    assert np.isfinite(got).all()
    err = normwise(got, ref)
    assert err <= NORMWISE, err
    rows = np.linalg.norm(got - ref, axis=1) / np.linalg.norm(ref, axis=1)
    assert rows.max() <= NORMWISE, rows.max()


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
@pytest.mark.parametrize("group", [8, 16, 32, 64, 128, 256, 1024])
@pytest.mark.parametrize("m,rows,dim", [(1, 33, 200), (37, 300, 1000), (130, 129, 512)])
def test_ragged_shapes_and_groups(bits, group, m, rows, dim):
    packed, norms, cb, dense = example(bits, rows=rows, dim=dim, group=group, seed=bits * 100 + group + m)
    norms[0] = 1  # no all-zero row: normwise checks per row
    dense = formats.dequantize_dense(packed, norms, (rows, dim), bits, group, cb)
    q = CQMatrix(packed, norms, (rows, dim), bits, group, cb)
    x = activations((m, dim), seed=group + m)
    got = gemm(q, x)
    ref = oracle.cq_linear(packed, norms, (rows, dim), bits, group, cb, x, 4)
    assert normwise(got, ref) <= NORMWISE
    exact = x.astype(np.float64) @ dense.T
    per_row = np.linalg.norm(got - exact, axis=1) / np.linalg.norm(exact, axis=1)
    assert per_row.max() <= NORMWISE, per_row.max()


def test_lloyd_max_codebook():
    packed, norms, _, _ = baseline(4, 1024, 1024, group=128, seed=9)
    cb = formats.codebook(4, 128)
    q = CQMatrix(packed, norms, (1024, 1024), 4, 128, cb)
    x = activations((96, 1024), seed=10)
    ref = oracle.cq_linear(packed, norms, (1024, 1024), 4, 128, cb, x, 8)
    assert normwise(gemm(q, x), ref) <= NORMWISE


def test_released_layer_shapes_cq2():
    """The released model's layer projections are CQ2 g128 (q 512 x 512, k / v 256 x 512): a 32-token chunk."""
    for rows in (512, 256):
        packed, norms, _, _ = baseline(2, rows, 512, group=128, seed=rows)
        cb = formats.codebook(2, 128)
        q = CQMatrix(packed, norms, (rows, 512), 2, 128, cb)
        x = activations((32, 512), seed=rows + 1)
        ref = oracle.cq_linear(packed, norms, (rows, 512), 2, 128, cb, x, 8)
        assert normwise(gemm(q, x), ref) <= NORMWISE
        assert normwise(gemm(q, x), ref) <= NORMWISE  # the widened codes are reused
