"""The int32 accumulators of the int8 path, read directly (needle2_gpu_sdot_dots_device), against the
reference's dot_group arithmetic (sdot.cpp:108-137) as the oracle restates it (nd_sdot_dots, itself pinned
against the integer closed form sum(clip(rint(cb / cs)) * clip(rint(rot / scale))) in tests/test_oracle.py):
bit-exact on every (batch row, weight row, group), on the kernels the GEMV runs for the batch (batch 1: the
row kernel; 2 .. 8: the 4 x 4 x 4 batch-tile MFMA kernel; 9 or more: the 16 x 16 x 32 batch-tile MFMA kernel
where the group holds whole code chunks, else the 4 x 4 x 4 one)."""
import numpy as np
import pytest

import oracle
from openneedle_amd.cq import CQMatrix
from openneedle_amd.device import DeviceArray, synchronize
from tests.cases import activations, baseline, example

pytestmark = pytest.mark.gpu


def device_dots(q, x):
    batch = x.shape[0]
    rows, groups = q.geometry.rows, q.geometry.groups
    with DeviceArray.from_host(np.ascontiguousarray(x, np.float32)) as d_x, \
            DeviceArray(batch * rows * groups * 4) as d_dots:
        d_dots.fill(0x7F)
        q.int8_dots_device(d_x, d_dots, batch)
        synchronize()
        return d_dots.to_host(np.int32, (batch, rows, groups))


def oracle_dots(packed, shape, bits, group, cb, x):
    cent, _ = oracle.sdot_centroids(cb, bits)
    out = []
    for row in x:
        qa, _ = oracle.sdot_prepare(row, group)
        out.append(oracle.sdot_dots(packed, shape, bits, group, cent, qa))
    return np.stack(out)


@pytest.mark.parametrize("batch", [1, 4, 16])
def test_int32_accumulators_cq4_4096(batch):
    """The int8 workload's matrix: CQ4 4096 x 4096 group 32, batch 1 / 4 / 16."""
    packed, norms, cb, _ = baseline(4, 4096, 4096, seed=90 + batch)
    q = CQMatrix(packed, norms, (4096, 4096), 4, 32, cb)
    x = activations((batch, 4096), seed=91 + batch)
    got = device_dots(q, x)
    np.testing.assert_array_equal(got, oracle_dots(packed, (4096, 4096), 4, 32, cb, x))
    assert np.abs(got).max() > 1000  # real accumulators, not a constant


@pytest.mark.parametrize("tile16", ["auto", "never"])
@pytest.mark.parametrize("bits,group,batch", [(4, 8, 5), (4, 16, 1), (4, 32, 9), (4, 64, 12), (4, 128, 20),
                                              (4, 256, 3), (2, 16, 7), (2, 32, 1), (2, 64, 16), (2, 256, 33)])
def test_int32_accumulators_ragged(bits, group, batch, tile16, monkeypatch):
    monkeypatch.setenv("NEEDLE2_GPU_INT8_TILE16", tile16)
    packed, norms, cb, dense = example(bits, rows=300, dim=1000, group=group, seed=bits + group + batch)
    q = CQMatrix(packed, norms, dense.shape, bits, group, cb)
    x = activations((batch, 1000), seed=batch + 3)
    x[0] = 0
    np.testing.assert_array_equal(device_dots(q, x), oracle_dots(packed, dense.shape, bits, group, cb, x))
