"""needle2_gpu_sdot_linear_device_noalloc (the int8 GEMV with its staging in the library's static scratch,
nothing allocated) against needle2_gpu_sdot_linear_device (the same kernels, per-handle allocated staging),
through the C ABI: bit-identical outputs on two calls in a row, the second on a smaller input, both also
equal to the oracle; sizes past the scratch are refused with a message."""
import numpy as np
import pytest

import oracle
from openneedle_amd import _ffi
from openneedle_amd.cq import CQMatrix
from openneedle_amd.device import DeviceArray, synchronize
from tests.cases import activations, baseline

pytestmark = pytest.mark.gpu

# (rows, cols, group, batch): the first fills most of the 4 MiB scratch, the second is smaller in every size
CASES = [(1024, 4096, 32, 700), (1000, 1000, 64, 3)]


def run_both(lib, rows, cols, group, batch, seed):
    packed, norms, cb, _ = baseline(4, rows, cols, group=group, seed=seed)
    q = CQMatrix(packed, norms, (rows, cols), 4, group, cb)
    h = q.int8_handle()
    x = activations((batch, cols), seed=seed + 1)
    with DeviceArray.from_host(x) as d_x, DeviceArray(batch * rows * 4) as y_alloc, \
            DeviceArray(batch * rows * 4) as y_static:
        y_static.fill(0xFF)  # NaN pattern: every output must be written
        print(f"case {rows}x{cols} g{group} batch {batch}: allocating entry point", flush=True)
        _ffi.check(lib.needle2_gpu_sdot_linear_device(h, d_x.ptr, y_alloc.ptr, batch, None), "allocating")
        print(f"case {rows}x{cols} g{group} batch {batch}: no-alloc entry point", flush=True)
        _ffi.check(lib.needle2_gpu_sdot_linear_device_noalloc(h, d_x.ptr, y_static.ptr, batch, None), "no-alloc")
        synchronize()
        got = y_static.to_host(np.float32, (batch, rows))
        want = y_alloc.to_host(np.float32, (batch, rows))
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(got, oracle.sdot_linear(packed, norms, (rows, cols), 4, group, cb, x, 8))
    return q


def test_noalloc_matches_allocating_entry_point():
    lib = _ffi.lib()
    for i, case in enumerate(CASES):
        q = run_both(lib, *case, seed=500 + i)
    # past the scratch: refused before any launch, with the reason
    with DeviceArray(4) as d:
        assert lib.needle2_gpu_sdot_linear_device_noalloc(q.int8_handle(), d.ptr, d.ptr, 1 << 20, None) == -1
    assert "4 MiB scratch" in _ffi.last_error()
