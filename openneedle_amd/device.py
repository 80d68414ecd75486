"""Device memory, streams, events and HIP graphs of the gfx950 library.

Each object owns one library resource and releases it in :meth:`close`
(idempotent; also called by ``__del__`` and by ``with`` blocks). Objects that
refer to each other on the device (a graph that replays launches reading a
plan's job table, a plan reading device buffers) should be released in a
known order rather than in whatever order the garbage collector picks:
:class:`Teardown` collects them and closes them in reverse order of
registration after synchronizing the device.
"""
from __future__ import annotations

import contextlib
import ctypes

import numpy as np

from . import _ffi
from ._ffi import check


class _Owned:
    """A library resource released exactly once."""

    _release_name = ""
    ptr = None

    def close(self) -> None:
        ptr, self.ptr = self.ptr, None
        if ptr:
            getattr(_ffi.lib(), self._release_name)(ptr)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown: the library may already be gone
            pass


class DeviceArray(_Owned):
    """``nbytes`` of device memory."""

    _release_name = "needle2_gpu_free"

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        self.ptr = _ffi.lib().needle2_gpu_malloc(self.nbytes)
        if not self.ptr:
            raise MemoryError(f"device allocation of {self.nbytes} bytes failed: {_ffi.last_error()}")

    @classmethod
    def from_host(cls, a) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.nbytes)
        d.upload(a)
        return d

    def upload(self, a, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        if offset < 0 or offset + a.nbytes > self.nbytes:
            raise ValueError(f"upload of {a.nbytes} bytes at {offset} overruns a {self.nbytes}-byte array")
        check(_ffi.lib().needle2_gpu_memcpy(self.ptr + offset, a.ctypes.data, a.nbytes, 0), "upload")

    def download(self, out: np.ndarray, offset: int = 0) -> np.ndarray:
        if not out.flags.c_contiguous or offset < 0 or offset + out.nbytes > self.nbytes:
            raise ValueError("download target must be C-contiguous and inside the array")
        check(_ffi.lib().needle2_gpu_memcpy(out.ctypes.data, self.ptr + offset, out.nbytes, 1), "download")
        return out

    def to_host(self, dtype, shape) -> np.ndarray:
        return self.download(np.empty(shape, dtype))

    def fill(self, byte: int = 0) -> None:
        check(_ffi.lib().needle2_gpu_memset(self.ptr, int(byte), self.nbytes), "memset")

    def view(self, offset: int, nbytes: int) -> "DeviceView":
        """Bytes [offset, offset + nbytes) of this allocation (the view keeps the allocation alive)."""
        if offset < 0 or offset + nbytes > self.nbytes:
            raise ValueError("view outside the array")
        return DeviceView(self, offset, nbytes)


class DeviceView(DeviceArray):
    """A sub-range of a :class:`DeviceArray`; releases nothing itself."""

    def __init__(self, base: DeviceArray, offset: int, nbytes: int):
        self._base = base
        self.nbytes = int(nbytes)
        self.ptr = base.ptr + int(offset)

    def close(self) -> None:
        self.ptr = None


class Stream(_Owned):
    """A non-blocking HIP stream at the default priority."""

    _release_name = "needle2_gpu_stream_destroy"

    def __init__(self):
        self.ptr = _ffi.lib().needle2_gpu_stream_create()
        if not self.ptr:
            raise _ffi.GpuError(f"stream create: {_ffi.last_error()}")

    def synchronize(self) -> None:
        check(_ffi.lib().needle2_gpu_stream_synchronize(self.ptr), "stream synchronize")


def stream_ptr(stream) -> int | None:
    """A :class:`Stream`, a raw hipStream_t address or None (the callee's own stream)."""
    return stream.ptr if isinstance(stream, Stream) else stream


class Event(_Owned):
    """A timing event recorded without a system-scope fence."""

    _release_name = "needle2_gpu_event_destroy"

    def __init__(self):
        self.ptr = _ffi.lib().needle2_gpu_event_create()
        if not self.ptr:
            raise _ffi.GpuError(f"event create: {_ffi.last_error()}")

    def record(self, stream) -> None:
        check(_ffi.lib().needle2_gpu_event_record(self.ptr, stream_ptr(stream)), "event record")

    def elapsed_ms(self, end: "Event") -> float:
        """Milliseconds from this event to ``end`` (waits for ``end``)."""
        return float(_ffi.lib().needle2_gpu_event_elapsed(self.ptr, end.ptr))


class Graph(_Owned):
    """Launches issued to a stream inside :meth:`capture`, replayed by :meth:`launch`.

    What is captured must have run once eagerly before (its buffers exist) and
    must not read host memory. The graph refers to the device memory of the
    objects whose launches it captured; close it before them (:class:`Teardown`).
    """

    _release_name = "needle2_gpu_graph_destroy"

    @classmethod
    @contextlib.contextmanager
    def capture(cls, stream: Stream):
        g = cls()
        library = _ffi.lib()
        check(library.needle2_gpu_graph_begin(stream.ptr), "graph begin")
        try:
            yield g
        finally:
            g.ptr = library.needle2_gpu_graph_end(stream.ptr)
        if not g.ptr:
            raise _ffi.GpuError(f"graph capture: {_ffi.last_error()}")

    def launch(self, stream: Stream) -> None:
        check(_ffi.lib().needle2_gpu_graph_launch(self.ptr, stream.ptr), "graph launch")


class Teardown:
    """Closes registered objects in reverse order of registration, after a device synchronization.

    Used as ``with Teardown() as td: x = td.add(DeviceArray(...)) ...`` so a
    workload releases its graph before its plans, its plans before their
    buffers, whatever the garbage collector would have done.
    """

    def __init__(self):
        self._objs = []

    def add(self, obj):
        self._objs.append(obj)
        return obj

    def close(self) -> None:
        if not self._objs:
            return
        try:
            synchronize()
        finally:
            while self._objs:
                self._objs.pop().close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def copy_kernel(dst: DeviceArray, src: DeviceArray, nbytes: int, stream: Stream | None = None) -> None:
    """The library's streaming copy kernel (the reference point for byte counters)."""
    if nbytes > dst.nbytes or nbytes > src.nbytes:
        raise ValueError("copy larger than its buffers")
    check(_ffi.lib().needle2_gpu_copy_kernel(dst.ptr, src.ptr, int(nbytes), stream_ptr(stream)), "copy kernel")


def calibrate_launch(launches: int = 2000, stream: Stream | None = None) -> float:
    """Microseconds per launch of an empty kernel issued back to back (the dependent-launch floor)."""
    us = ctypes.c_float()
    check(_ffi.lib().needle2_gpu_calib_launch(int(launches), ctypes.byref(us), stream_ptr(stream)),
          "launch calibration")
    return us.value


def calibrate_lds(width: int, stream: Stream | None = None) -> tuple[float, float]:
    """(LDS read bytes per shader clock per CU for `width`-byte lane reads, shader GHz of the run)."""
    rate, ghz = ctypes.c_float(), ctypes.c_float()
    check(_ffi.lib().needle2_gpu_calib_lds(int(width), ctypes.byref(rate), ctypes.byref(ghz), stream_ptr(stream)),
          "LDS calibration")
    return rate.value, ghz.value


def calibrate_stream(buf: DeviceArray, nbytes: int, pattern: int, stream: Stream | None = None) -> float:
    """Microseconds per pass reading one third of `nbytes` of `buf` (the thirds in turn): pattern 0 / 1 the
    GEMVs' per-tile walk with plain / non-temporal loads, 2 / 3 grid-stride streaming with plain /
    non-temporal loads."""
    if nbytes > buf.nbytes:
        raise ValueError("calibration read larger than its buffer")
    us = ctypes.c_float()
    check(_ffi.lib().needle2_gpu_calib_stream(buf.ptr, int(nbytes), int(pattern), ctypes.byref(us),
                                              stream_ptr(stream)), "stream calibration")
    return us.value


def synchronize() -> None:
    check(_ffi.lib().needle2_gpu_synchronize(), "device synchronize")


def device_info() -> dict:
    buf = ctypes.create_string_buffer(512)
    check(_ffi.lib().needle2_gpu_device_info(buf, 512), "device info")
    name, arch, cus, mem, clk = buf.value.decode().split(";")
    return {"name": name, "arch": arch, "cus": int(cus), "hbm_bytes": int(mem), "clock_khz": int(clk)}
