"""Chained int8 plans outside the decode-layer shapes (needle2_gpu_plan_run_chained): a producer plan leaves
the next plan's input prepared, fused in the 16 x 16 K-split GEMV's epilogue when the next plan's groups are 32
positions, else by the next plan's own prepare launch. Ragged producer rows (the next input's zero padding),
ragged batches, 2- and 4-bit consumers and groups of 32 / 64 / 128: every output bit-exact with the oracle
applied stage by stage."""
import numpy as np
import pytest

import oracle
from openneedle_amd._ffi import GpuError
from openneedle_amd.cq import CQMatrix, Plan
from openneedle_amd.device import DeviceArray, Teardown, synchronize
from tests.cases import activations, example

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("mid,batch,bits2,group2", [(512, 64, 4, 32), (300, 20, 4, 32), (300, 20, 2, 32),
                                                    (512, 33, 4, 64), (512, 16, 2, 128), (1000, 2, 4, 32),
                                                    (512, 1, 4, 32)])
def test_two_plan_chain(mid, batch, bits2, group2):
    dim, out = 512, 200
    p1, n1, cb1, d1 = example(4, rows=mid, dim=dim, group=32, seed=mid + batch)
    p2, n2, cb2, d2 = example(bits2, rows=out, dim=mid, group=group2, seed=mid * 3 + group2)
    x = activations((batch, dim), seed=batch)
    x[0] = 0
    h = oracle.sdot_linear(p1, n1, d1.shape, 4, 32, cb1, x)
    want = oracle.sdot_linear(p2, n2, d2.shape, bits2, group2, cb2, h)
    with Teardown() as td:
        a = td.add(CQMatrix(p1, n1, d1.shape, 4, 32, cb1))
        b = td.add(CQMatrix(p2, n2, d2.shape, bits2, group2, cb2))
        d_x = td.add(DeviceArray.from_host(x))
        d_h = td.add(DeviceArray(4 * batch * mid))
        d_y = td.add(DeviceArray(4 * batch * out))
        first = td.add(Plan([a], [d_x], [d_h], batch=batch, int8=True))
        second = td.add(Plan([b], [d_h], [d_y], batch=batch, int8=True))
        for _ in range(2):  # the second round reuses staged buffers
            d_h.upload(np.full((batch, mid), np.nan, np.float32))
            d_y.upload(np.full((batch, out), np.nan, np.float32))
            first.run(next=second)
            second.run(prepared=True)
            synchronize()
            np.testing.assert_array_equal(d_h.download(np.empty((batch, mid), np.float32)), h)
            np.testing.assert_array_equal(d_y.download(np.empty((batch, out), np.float32)), want)


def test_chain_refuses_a_mismatched_next_plan():
    with Teardown() as td:
        p1, n1, cb1, d1 = example(4, rows=256, dim=512, group=32, seed=1)
        p2, n2, cb2, d2 = example(4, rows=64, dim=300, group=32, seed=2)
        a = td.add(CQMatrix(p1, n1, d1.shape, 4, 32, cb1))
        b = td.add(CQMatrix(p2, n2, d2.shape, 4, 32, cb2))
        d_x = td.add(DeviceArray(4 * 4 * 512))
        d_h = td.add(DeviceArray(4 * 4 * 300))
        d_y = td.add(DeviceArray(4 * 4 * 64))
        first = td.add(Plan([a], [d_x], [d_h], batch=4, int8=True))
        second = td.add(Plan([b], [d_h], [d_y], batch=4, int8=True))  # reads 300 values, first writes 256
        with pytest.raises(GpuError, match="input shape"):
            first.run(next=second)
        fp32 = td.add(Plan([b], [d_h], [d_y], batch=4))
        with pytest.raises(GpuError, match="FP32 plans"):
            fp32.run(prepared=True)
