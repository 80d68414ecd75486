"""The library's calibration entry points (needle2_gpu_calib_*): they run, return plausible figures and refuse
bad arguments. Their figures are measurements, so only broad bounds are checked."""
import pytest

from openneedle_amd._ffi import GpuError
from openneedle_amd.device import DeviceArray, Stream, calibrate_launch, calibrate_lds, calibrate_stream

pytestmark = pytest.mark.gpu


def test_launch_floor():
    us = calibrate_launch(200)
    assert 0.05 < us < 100.0


@pytest.mark.parametrize("width", [4, 8, 16])
def test_lds_rate(width):
    rate, ghz = calibrate_lds(width)
    assert 0.5 < ghz < 5.0
    assert 8.0 < rate < 1024.0  # bytes per shader clock per CU


def test_stream_patterns_and_errors():
    nbytes = 3 * 512 * 3 * 16384 * 4  # three regions of 512 tiles of 4 x 48 KiB
    with Stream() as s, DeviceArray(nbytes) as buf:
        for pattern in range(4):
            us = calibrate_stream(buf, nbytes, pattern, s)
            assert 0.0 < us < 1e5
        with pytest.raises(GpuError, match="pattern"):
            calibrate_stream(buf, nbytes, 4, s)
        with pytest.raises(GpuError, match="too small"):
            calibrate_stream(buf, 3 * 512 * 16384, 0, s)
    with pytest.raises(GpuError, match="width"):
        calibrate_lds(2)
