"""ctypes access to the gfx950 CQ library (``libneedle2_native.so``).

Mirrors ``needle2/native.py`` (NativeCQ, available, features, sdot_available)
with the same names, argument validation and error messages, so code written
against the reference's loader runs unchanged on this library. The library is
selected the same way: ``NEEDLE2_NATIVE_LIBRARY`` if set, otherwise the
in-tree build next to this file. There is no CPU fallback: without the HIP
library every call raises.

Additive (device-resident) API: :class:`DeviceArray`, :class:`Stream`,
:class:`Event`, :meth:`NativeCQ.linear_device`, :class:`Plan` and
:class:`KVCache` (int8 KV cache and batched decode attention).
"""
from __future__ import annotations

import ctypes as ct
import functools
import os
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
DEFAULT_LIBRARY = PKG / "libneedle2_native.so"

_P = ct.c_void_p
_I = ct.c_int


def library_path() -> Path:
    """needle2/native.py:76-84 semantics for NEEDLE2_NATIVE_LIBRARY, else the in-tree build."""
    prebuilt = os.environ.get("NEEDLE2_NATIVE_LIBRARY")
    if prebuilt is not None:
        if not prebuilt.strip():
            raise RuntimeError("NEEDLE2_NATIVE_LIBRARY must name a prebuilt OpenNeedle shared library")
        target = Path(prebuilt).expanduser().resolve()
        if not target.is_file():
            raise RuntimeError(f"Prebuilt OpenNeedle library not found: {target}")
        return target
    if not DEFAULT_LIBRARY.is_file():
        raise RuntimeError(f"gfx950 library not built: {DEFAULT_LIBRARY} (run python -m openneedle_amd.build)")
    return DEFAULT_LIBRARY


def _bind(lib, name, args, res=None):
    f = getattr(lib, name)
    f.argtypes = args
    f.restype = res
    return f


@functools.lru_cache(maxsize=1)
def _library():
    lib = ct.CDLL(str(library_path()))
    # reference ABI (needle2/native.py:128-145)
    _bind(lib, "needle2_native_features", [], ct.c_char_p)
    _bind(lib, "needle2_cq_create", [_P, _P, _I, _I, _I, _I, _P], _P)
    _bind(lib, "needle2_cq_destroy", [_P])
    _bind(lib, "needle2_cq_linear", [_P, _P, _P, _I, _I])
    _bind(lib, "needle2_cq_linear_lookup", [_P, _P, _P, _I, _I, _I])
    _bind(lib, "needle2_sdot_supported", [], _I)
    _bind(lib, "needle2_sdot_create", [_P, _P, _I, _I, _I, _I, _P], _P)
    _bind(lib, "needle2_sdot_destroy", [_P])
    _bind(lib, "needle2_sdot_linear", [_P, _P, _P, _I, _I])
    _bind(lib, "needle2_cq_rows", [_P, _P, _P, _I])
    # additive gfx950 exports
    _bind(lib, "needle2_gpu_error", [], ct.c_char_p)
    _bind(lib, "needle2_gpu_sdot_create", [_P, _P, _I, _I, _I, _I, _P], _P)
    _bind(lib, "needle2_gpu_cq_linear_device", [_P, _P, _P, _I, _P], _I)
    _bind(lib, "needle2_gpu_sdot_linear_device", [_P, _P, _P, _I, _P], _I)
    _bind(lib, "needle2_gpu_cq_create_device", [_P, _P, _I, _I, _I, _I, _P, _P], _P)
    _bind(lib, "needle2_gpu_sdot_create_device", [_P, _P, _I, _I, _I, _I, _P, _P], _P)
    for name in ("needle2_gpu_cq_candidates", "needle2_gpu_sdot_candidates"):
        _bind(lib, name, [_P, _P, _P, _I, _P], _I)
        _bind(lib, name + "_device", [_P, _P, _P, _I, _P, _P], _I)
    _bind(lib, "needle2_gpu_cq_gemm_device", [_P, _P, _P, _I, _P], _I)
    _bind(lib, "needle2_gpu_cq_gemm_timed", [_P, _P, _P, _I, _P, _P, _P, _I], _I)
    _bind(lib, "needle2_gpu_cq_plan_create", [_P, _I, _P, _P, _I], _P)
    _bind(lib, "needle2_gpu_sdot_plan_create", [_P, _I, _P, _P, _I], _P)
    _bind(lib, "needle2_gpu_plan_run", [_P, _P], _I)
    _bind(lib, "needle2_gpu_plan_run_timed", [_P, _P, _P, _P], _I)
    _bind(lib, "needle2_gpu_plan_destroy", [_P])
    _bind(lib, "needle2_gpu_malloc", [ct.c_size_t], _P)
    _bind(lib, "needle2_gpu_free", [_P])
    _bind(lib, "needle2_gpu_memcpy", [_P, _P, ct.c_size_t, _I], _I)
    _bind(lib, "needle2_gpu_memset", [_P, _I, ct.c_size_t], _I)
    _bind(lib, "needle2_gpu_copy_kernel", [_P, _P, ct.c_size_t, _P], _I)
    _bind(lib, "needle2_gpu_synchronize", [], _I)
    _bind(lib, "needle2_gpu_stream_create", [], _P)
    _bind(lib, "needle2_gpu_stream_destroy", [_P])
    _bind(lib, "needle2_gpu_stream_synchronize", [_P], _I)
    _bind(lib, "needle2_gpu_event_create", [], _P)
    _bind(lib, "needle2_gpu_event_destroy", [_P])
    _bind(lib, "needle2_gpu_event_record", [_P, _P], _I)
    _bind(lib, "needle2_gpu_event_elapsed", [_P, _P], ct.c_float)
    _bind(lib, "needle2_gpu_device_info", [ct.c_char_p, _I], _I)
    _bind(lib, "needle2_gpu_kv_create", [_I, _I, _I, _I, _I], _P)
    _bind(lib, "needle2_gpu_kv_destroy", [_P])
    _bind(lib, "needle2_gpu_kv_storage_bytes", [_P], ct.c_size_t)
    _bind(lib, "needle2_gpu_kv_store", [_P, _I, _P, _P, _I, _I, _P, _P], _I)
    _bind(lib, "needle2_gpu_kv_store_device", [_P, _I, _P, _P, _I, _P, _P], _I)
    _bind(lib, "needle2_gpu_graph_begin", [_P], _I)
    _bind(lib, "needle2_gpu_graph_end", [_P], _P)
    _bind(lib, "needle2_gpu_graph_launch", [_P, _P], _I)
    _bind(lib, "needle2_gpu_graph_destroy", [_P])
    _bind(lib, "needle2_gpu_attention", [_P, _I, _P, _P, _I, _I, _P, _P, _I, _P], _I)
    _bind(lib, "needle2_gpu_kv_import", [_P, _I, _I, _P, _P, _P, _P, _I, _I], _I)
    _bind(lib, "needle2_gpu_kv_export", [_P, _I, _I, _P, _P, _P, _P, _I, _I], _I)
    return lib


def available() -> bool:
    try:
        _library()
        return True
    except (OSError, RuntimeError):
        return False


def features() -> str:
    return _library().needle2_native_features().decode()


def sdot_available() -> bool:
    return bool(_library().needle2_sdot_supported())


def last_error() -> str:
    return _library().needle2_gpu_error().decode()


def _check(rc: int, what: str) -> None:
    if rc:
        raise RuntimeError(f"{what}: {last_error()}")


class NativeCQ:
    """A packed ``[out, in]`` matrix resident on the GPU (needle2/native.py:165-279).

    The codebook must already include ``1/sqrt(group_size)`` as in a CACT header.
    ``bits=5`` denotes the official signed ternary crumb storage, with 3 centroids.
    """

    def __init__(self, packed, norms, shape, bits, group_size, codebook, *, device=None, int8: bool = False):
        """``device``: optional (d_packed, d_norms, stream) device pointers holding the same packed codes and
        norms; the handles are then built from them on ``stream`` without copying (the caller synchronizes the
        stream before freeing them or using the matrix elsewhere). ``int8``: also build the int8 (SDOT) handle
        now, for groups the GPU int8 path takes."""
        self.shape = tuple(int(v) for v in shape)
        if len(self.shape) != 2 or min(self.shape) <= 0:
            raise ValueError("NativeCQ requires a positive two-dimensional matrix shape")
        self.bits, self.group_size = int(bits), int(group_size)
        if self.bits not in (2, 3, 4, 5):
            raise ValueError("CQ storage bits must be 2, 3, 4, or ternary marker 5")
        if self.group_size < 8 or self.group_size & (self.group_size - 1):
            raise ValueError("CQ group size must be a power of two >= 8")
        out, dim = self.shape
        limit = np.iinfo(np.int32).max
        if max(out, dim, self.group_size) > limit or dim + self.group_size - 1 > limit:
            raise ValueError("CQ dimensions exceed the native int32 interface")
        padded = ((dim + self.group_size - 1) // self.group_size) * self.group_size
        storage_bits = 2 if self.bits == 5 else self.bits
        if padded * storage_bits > limit:
            raise ValueError("CQ row bit count exceeds the native int32 interface")
        self.packed = np.ascontiguousarray(packed, dtype=np.uint8).reshape(out, padded * storage_bits // 8)
        self.norms = np.ascontiguousarray(norms, dtype=np.float16).reshape(out, padded // self.group_size)
        self.codebook = np.ascontiguousarray(codebook, dtype=np.float32)
        if self.codebook.shape != (3 if self.bits == 5 else 1 << self.bits,):
            raise ValueError("Codebook has incorrect number of centroids")
        if not np.isfinite(self.norms).all() or np.any(self.norms < 0):
            raise ValueError("CQ norms must be finite and nonnegative")
        if not np.isfinite(self.codebook).all() or not np.all(np.diff(self.codebook) > 0):
            raise ValueError("CQ codebook must be finite and strictly sorted")
        if self.bits == 5:
            for shift in (0, 2, 4, 6):
                if np.any(((self.packed >> shift) & 3) == 2):
                    raise ValueError("Invalid ternary crumb code 2")
        self._lib = _library()
        if device is None:
            self._handle = self._lib.needle2_cq_create(self.packed.ctypes.data, self.norms.ctypes.data,
                                                       out, dim, self.bits, self.group_size,
                                                       self.codebook.ctypes.data)
        else:
            d_packed, d_norms, stream = device
            stream = stream.ptr if isinstance(stream, Stream) else stream
            self._handle = self._lib.needle2_gpu_cq_create_device(d_packed, d_norms, out, dim, self.bits,
                                                                  self.group_size, self.codebook.ctypes.data, stream)
        if not self._handle:
            raise MemoryError(f"Could not construct native CQ matrix ({last_error()})")
        if int8 and self.bits in (2, 4) and self.group_size >= (8 if self.bits == 4 else 16):
            if device is None:
                self._sdot(True)
            else:
                self._sdot_handle = self._lib.needle2_gpu_sdot_create_device(
                    d_packed, d_norms, out, dim, self.bits, self.group_size, self.codebook.ctypes.data, stream)
                if not self._sdot_handle:
                    raise RuntimeError(f"could not construct SDOT matrix ({last_error()})")

    @classmethod
    def from_record(cls, record):
        cb = record.codebook
        if record.bits == 5 and cb is None:
            cb = (np.array([-1.2240064, 0., 1.2240064], np.float64) / np.sqrt(record.group_size)).astype(np.float32)
        return cls(record.packed, record.norms, record.shape, record.bits, record.group_size, cb)

    def __del__(self):
        for attr, fn in (("_sdot_handle", "needle2_sdot_destroy"), ("_handle", "needle2_cq_destroy")):
            h = getattr(self, attr, None)
            if h:
                getattr(self._lib, fn)(h)
                setattr(self, attr, None)

    def linear(self, x, threads: int = 1, *, lookup: int = 0):
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim < 1 or x.shape[-1] != self.shape[1]:
            raise ValueError(f"Expected input last dimension {self.shape[1]}; got {x.shape}")
        if not 1 <= int(threads) <= 256:
            raise ValueError("threads must be between 1 and 256")
        if (x.size // self.shape[1]) * self.shape[0] > np.iinfo(np.int32).max:
            raise ValueError("CQ batch output count exceeds the native int32 interface")
        y = np.empty(x.shape[:-1] + (self.shape[0],), dtype=np.float32)
        if lookup not in (0, 1, 2, 3):
            raise ValueError("lookup must be 0 (NEON), 1 (byte table), 2 (nibble table), or 3 (group byte table)")
        if lookup:
            self._lib.needle2_cq_linear_lookup(self._handle, x.ctypes.data, y.ctypes.data,
                                               x.size // self.shape[1], int(threads), int(lookup))
        else:
            self._lib.needle2_cq_linear(self._handle, x.ctypes.data, y.ctypes.data,
                                        x.size // self.shape[1], int(threads))
        err = last_error()
        if err:
            raise RuntimeError(f"CQ linear failed: {err}")
        return y

    def _sdot(self, extended: bool):
        if not getattr(self, "_sdot_handle", None):
            create = self._lib.needle2_gpu_sdot_create if extended else self._lib.needle2_sdot_create
            self._sdot_handle = create(self.packed.ctypes.data, self.norms.ctypes.data,
                                       *self.shape, self.bits, self.group_size, self.codebook.ctypes.data)
            if not self._sdot_handle:
                raise RuntimeError(f"could not construct SDOT matrix ({last_error()})")
        return self._sdot_handle

    def linear_sdot(self, x, threads: int = 1):
        """Approximate DotProd GEMV; additionally rounds rotated inputs and centroids to INT8."""
        if self.bits not in (2, 4) or not 64 <= self.group_size <= 131072:
            raise ValueError("SDOT requires CQ2/CQ4 and group size between 64 and 131072")
        return self._linear_int8(x, threads, extended=False)

    def linear_int8(self, x, threads: int = 1):
        """The SDOT arithmetic for every group the GPU supports (CQ4 g>=8, CQ2 g>=16)."""
        if self.bits not in (2, 4) or self.group_size > 131072 or self.group_size < (8 if self.bits == 4 else 16):
            raise ValueError("int8 path requires CQ4 (group >= 8) or CQ2 (group >= 16), group <= 131072")
        return self._linear_int8(x, threads, extended=True)

    def _linear_int8(self, x, threads, extended):
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.ndim < 1 or x.shape[-1] != self.shape[1] or not np.isfinite(x).all():
            raise ValueError("SDOT input must have the expected last dimension and finite values")
        if not 1 <= int(threads) <= 256:
            raise ValueError("threads must be between 1 and 256")
        handle = self._sdot(extended)
        if (x.size // self.shape[1]) * self.shape[0] > np.iinfo(np.int32).max:
            raise ValueError("SDOT batch output count exceeds the native int32 interface")
        y = np.empty(x.shape[:-1] + (self.shape[0],), dtype=np.float32)
        self._lib.needle2_sdot_linear(handle, x.ctypes.data, y.ctypes.data, x.size // self.shape[1], int(threads))
        err = last_error()
        if err:
            raise RuntimeError(f"SDOT linear failed: {err}")
        return y

    def _candidate_ids(self, x, candidates):
        """needle2/native.py:485-495 checks (same messages) for one input vector and candidate rows."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        if x.shape != (self.shape[1],):
            raise ValueError(f"Expected one input vector of {self.shape[1]} values; got {x.shape}")
        cands = np.asarray(candidates)
        if cands.ndim != 1 or not cands.size or cands.dtype.kind not in "iu":
            raise ValueError("candidates must be a nonempty 1D integer array")
        if np.any((cands < 0) | (cands >= self.shape[0])):
            raise ValueError("candidate outside vocabulary")
        return x, np.ascontiguousarray(cands, dtype=np.int32)

    def candidates(self, x, candidates):
        """Rows `candidates` of the FP32 product for one input vector (Engine::project_candidates' CQ branch,
        needle2/csrc/engine.cpp:1307-1349): bit-identical to linear(x)[candidates]."""
        x, ids = self._candidate_ids(x, candidates)
        y = np.empty(ids.size, dtype=np.float32)
        _check(self._lib.needle2_gpu_cq_candidates(self._handle, x.ctypes.data, ids.ctypes.data, ids.size,
                                                   y.ctypes.data), "CQ candidates")
        return y

    def candidates_int8(self, x, candidates):
        """Rows `candidates` of the int8 product (the SDOT branch): bit-identical to linear_int8(x)[candidates]."""
        x, ids = self._candidate_ids(x, candidates)
        if not np.isfinite(x).all():
            raise ValueError("SDOT input must have the expected last dimension and finite values")
        y = np.empty(ids.size, dtype=np.float32)
        _check(self._lib.needle2_gpu_sdot_candidates(self._sdot(True), x.ctypes.data, ids.ctypes.data, ids.size,
                                                     y.ctypes.data), "SDOT candidates")
        return y

    def rows(self, ids):
        ids = np.asarray(ids)
        if ids.dtype.kind not in "iu":
            raise TypeError("row indices must be integers")
        ids_shape = ids.shape
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        if np.any((ids < 0) | (ids >= self.shape[0])):
            raise IndexError("CQ row index outside matrix")
        result = np.empty(ids_shape + (self.shape[1],), dtype=np.float32)
        self._lib.needle2_cq_rows(self._handle, ids.ctypes.data, result.ctypes.data, ids.size)
        err = last_error()
        if err:
            raise RuntimeError(f"CQ rows failed: {err}")
        return result

    def dequantize(self):
        return self.rows(np.arange(self.shape[0], dtype=np.int64))

    # ---- device-resident entry points ----------------------------------
    def linear_device(self, d_x, d_y, batch: int, stream=None) -> None:
        _check(self._lib.needle2_gpu_cq_linear_device(self._handle, d_x, d_y, int(batch), stream), "cq linear_device")

    def gemm_device(self, d_x, d_y, m: int, stream=None, events=None, repeat: int = 1) -> None:
        """Prefill GEMM on fp16 MFMA: device y[m][out] from device x[m][in] (4-bit codes).

        ``events``: optional (start, stop) :class:`Event` pair recorded around ``repeat`` back-to-back launches
        of the GEMM kernel (a timing aid: per-launch time = elapsed / repeat).
        """
        s = stream.ptr if isinstance(stream, Stream) else stream
        if events is None:
            _check(self._lib.needle2_gpu_cq_gemm_device(self._handle, d_x, d_y, int(m), s), "cq gemm_device")
        else:
            _check(self._lib.needle2_gpu_cq_gemm_timed(self._handle, d_x, d_y, int(m), s, events[0].ptr,
                                                       events[1].ptr, int(repeat)), "cq gemm_device")

    def candidates_device(self, d_x, d_ids, count: int, d_y, stream=None, int8: bool = False) -> None:
        """Device form of candidates / candidates_int8: d_ids int32 [count], d_y [count]."""
        s = stream.ptr if isinstance(stream, Stream) else stream
        if int8:
            _check(self._lib.needle2_gpu_sdot_candidates_device(self._sdot(True), d_x, d_ids, int(count), d_y, s),
                   "sdot candidates_device")
        else:
            _check(self._lib.needle2_gpu_cq_candidates_device(self._handle, d_x, d_ids, int(count), d_y, s),
                   "cq candidates_device")

    def int8_device(self, d_x, d_y, batch: int, stream=None, extended: bool = True) -> None:
        _check(self._lib.needle2_gpu_sdot_linear_device(self._sdot(extended), d_x, d_y, int(batch), stream),
               "sdot linear_device")


# --------------------------------------------------------------------------
# Device helpers
# --------------------------------------------------------------------------
class DeviceArray:
    """A device allocation owned by the library (freed on delete)."""

    def __init__(self, nbytes: int):
        self._lib = _library()
        self.nbytes = int(nbytes)
        self.ptr = self._lib.needle2_gpu_malloc(self.nbytes)
        if not self.ptr:
            raise MemoryError(f"device allocation of {nbytes} bytes failed: {last_error()}")

    @classmethod
    def from_host(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.nbytes)
        d.upload(a)
        return d

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        _check(self._lib.needle2_gpu_memcpy(self.ptr + offset, a.ctypes.data, a.nbytes, 0), "upload")

    def download(self, out: np.ndarray, offset: int = 0) -> np.ndarray:
        assert out.flags.c_contiguous and offset + out.nbytes <= self.nbytes
        _check(self._lib.needle2_gpu_memcpy(out.ctypes.data, self.ptr + offset, out.nbytes, 1), "download")
        return out

    def view(self, offset: int, nbytes: int) -> "DeviceView":
        """Bytes [offset, offset + nbytes) of this allocation (which the view keeps alive)."""
        assert 0 <= offset and offset + nbytes <= self.nbytes
        return DeviceView(self, offset, nbytes)

    def __del__(self):
        if getattr(self, "ptr", None):
            self._lib.needle2_gpu_free(self.ptr)
            self.ptr = None


class DeviceView(DeviceArray):
    """A sub-range of a :class:`DeviceArray`; frees nothing itself."""

    def __init__(self, base: DeviceArray, offset: int, nbytes: int):
        self._lib = base._lib
        self._base = base
        self.nbytes = int(nbytes)
        self.ptr = base.ptr + int(offset)

    def __del__(self):
        self.ptr = None


class Stream:
    def __init__(self):
        self._lib = _library()
        self.ptr = self._lib.needle2_gpu_stream_create()
        if not self.ptr:
            raise RuntimeError(last_error())

    def synchronize(self):
        _check(self._lib.needle2_gpu_stream_synchronize(self.ptr), "stream sync")

    def __del__(self):
        if getattr(self, "ptr", None):
            self._lib.needle2_gpu_stream_destroy(self.ptr)
            self.ptr = None


class Event:
    def __init__(self):
        self._lib = _library()
        self.ptr = self._lib.needle2_gpu_event_create()
        if not self.ptr:
            raise RuntimeError(last_error())

    def record(self, stream: Stream):
        _check(self._lib.needle2_gpu_event_record(self.ptr, stream.ptr), "event record")

    def elapsed_ms(self, end: "Event") -> float:
        return float(self._lib.needle2_gpu_event_elapsed(self.ptr, end.ptr))

    def __del__(self):
        if getattr(self, "ptr", None):
            self._lib.needle2_gpu_event_destroy(self.ptr)
            self.ptr = None


class Graph:
    """Work issued to ``stream`` inside ``with Graph.capture(stream) as g:`` replayed by ``g.launch(stream)``.

    Everything captured must have run once eagerly before (buffers allocated)
    and must not read host memory: plan runs, attention, ``store_device``.
    """

    def __init__(self):
        self._lib = _library()
        self.ptr = None

    @classmethod
    def capture(cls, stream: Stream):
        import contextlib

        g = cls()

        @contextlib.contextmanager
        def cm():
            _check(g._lib.needle2_gpu_graph_begin(stream.ptr), "graph begin")
            try:
                yield g
            finally:
                g.ptr = g._lib.needle2_gpu_graph_end(stream.ptr)
            if not g.ptr:
                raise RuntimeError(f"graph capture failed: {last_error()}")
        return cm()

    def launch(self, stream: Stream) -> None:
        _check(self._lib.needle2_gpu_graph_launch(self.ptr, stream.ptr), "graph launch")

    def __del__(self):
        if getattr(self, "ptr", None):
            self._lib.needle2_gpu_graph_destroy(self.ptr)
            self.ptr = None


def copy_kernel(dst: DeviceArray, src: DeviceArray, nbytes: int, stream: "Stream | None" = None) -> None:
    assert nbytes <= dst.nbytes and nbytes <= src.nbytes
    _check(_library().needle2_gpu_copy_kernel(dst.ptr, src.ptr, int(nbytes), stream.ptr if stream else None), "copy")


def synchronize() -> None:
    _check(_library().needle2_gpu_synchronize(), "synchronize")


def device_info() -> dict:
    buf = ct.create_string_buffer(512)
    _check(_library().needle2_gpu_device_info(buf, 512), "device_info")
    name, arch, cus, mem, clk = buf.value.decode().split(";")
    return {"name": name, "arch": arch, "cus": int(cus), "hbm_bytes": int(mem), "clock_khz": int(clk)}


class Plan:
    """Many same-geometry matrices, each with its own device input, in one GEMV launch."""

    def __init__(self, matrices, d_x, d_y, batch: int = 1, int8: bool = False, extended: bool = True):
        self._lib = _library()
        n = len(matrices)
        handles = (_P * n)(*[m._sdot(extended) if int8 else m._handle for m in matrices])
        xs = (_P * n)(*[int(p) for p in d_x])
        ys = (_P * n)(*[int(p) for p in d_y])
        create = self._lib.needle2_gpu_sdot_plan_create if int8 else self._lib.needle2_gpu_cq_plan_create
        self._keep = (matrices, handles, xs, ys)
        self.ptr = create(handles, n, xs, ys, int(batch))
        if not self.ptr:
            raise RuntimeError(f"plan create failed: {last_error()}")

    def run(self, stream: Stream | None = None, gemv_events=None) -> None:
        s = stream.ptr if stream else None
        if gemv_events is None:
            _check(self._lib.needle2_gpu_plan_run(self.ptr, s), "plan run")
        else:
            start, stop = gemv_events
            _check(self._lib.needle2_gpu_plan_run_timed(self.ptr, s, start.ptr, stop.ptr), "plan run")

    def __del__(self):
        if getattr(self, "ptr", None):
            self._lib.needle2_gpu_plan_destroy(self.ptr)
            self.ptr = None


class KVCache:
    """Device int8 KV cache for ``seqs`` sequences plus batched decode attention.

    The arithmetic is the reference Engine's int8 cache (needle2/csrc/engine.cpp:
    1005-1021 quantize/store, 898-967 compute_attention); the host arrays of
    :meth:`load` / :meth:`read` use its layout, [slots][kvheads][head_dim] int8
    and [slots][kvheads] fp32 scales.
    """

    def __init__(self, layers: int, capacity: int, kvheads: int, head_dim: int, seqs: int = 1):
        self._lib = _library()
        self.layers, self.capacity, self.kvheads, self.head_dim, self.seqs = layers, capacity, kvheads, head_dim, seqs
        self.ptr = self._lib.needle2_gpu_kv_create(layers, capacity, kvheads, head_dim, seqs)
        if not self.ptr:
            raise RuntimeError(f"KV cache create failed: {last_error()}")

    def storage_bytes(self) -> int:
        return int(self._lib.needle2_gpu_kv_storage_bytes(self.ptr))

    def store(self, layer: int, d_k, d_v, count: int, first_slot=0, stream: "Stream | None" = None) -> None:
        """Quantize ``count`` tokens per sequence from device fp32 [seqs][count][kvheads][head_dim].

        ``first_slot``: one int for every sequence, or a sequence of ``seqs`` ints.
        """
        per_seq = None
        if np.ndim(first_slot):
            per_seq = np.ascontiguousarray(first_slot, np.int32)
            if per_seq.shape != (self.seqs,):
                raise ValueError("first_slot needs one entry per sequence")
            first = 0
        else:
            first = int(first_slot)
        _check(self._lib.needle2_gpu_kv_store(self.ptr, layer, int(d_k), int(d_v), int(count), first,
                                              per_seq.ctypes.data if per_seq is not None else None,
                                              stream.ptr if stream else None), "KV store")

    def store_device(self, layer: int, d_k, d_v, count: int, d_first_slot, stream: "Stream | None" = None) -> None:
        """:meth:`store` with the per-sequence first slots in device memory (int32 [seqs]); capturable."""
        _check(self._lib.needle2_gpu_kv_store_device(self.ptr, layer, int(d_k), int(d_v), int(count),
                                                     int(d_first_slot), stream.ptr if stream else None),
               "KV store")

    def attention(self, layer: int, d_q, d_out, heads: int, length: int, d_slots=None, d_lengths=None,
                  splits: int = 0, stream: "Stream | None" = None) -> None:
        """One decode step for every sequence: device q/out fp32 [seqs][heads][head_dim]."""
        _check(self._lib.needle2_gpu_attention(self.ptr, layer, int(d_q), int(d_out), int(heads), int(length),
                                               int(d_slots) if d_slots else None,
                                               int(d_lengths) if d_lengths else None, int(splits),
                                               stream.ptr if stream else None), "attention")

    def load(self, layer: int, seq: int, k, v, ks, vs, first_slot: int = 0) -> None:
        """Copy host int8 rows and fp32 scales (reference layout) into the cache."""
        k = np.ascontiguousarray(k, np.int8)
        v = np.ascontiguousarray(v, np.int8)
        ks = np.ascontiguousarray(ks, np.float32)
        vs = np.ascontiguousarray(vs, np.float32)
        n = k.shape[0]
        if k.shape != (n, self.kvheads, self.head_dim) or v.shape != k.shape or ks.shape != (n, self.kvheads) \
                or vs.shape != ks.shape:
            raise ValueError("KV load: shapes must be [n, kvheads, head_dim] and [n, kvheads]")
        _check(self._lib.needle2_gpu_kv_import(self.ptr, layer, seq, k.ctypes.data, v.ctypes.data, ks.ctypes.data,
                                               vs.ctypes.data, int(first_slot), n), "KV import")

    def read(self, layer: int, seq: int, count: int, first_slot: int = 0):
        """(k int8, v int8, k_scales, v_scales) of ``count`` slots in the reference layout."""
        k = np.empty((count, self.kvheads, self.head_dim), np.int8)
        v = np.empty_like(k)
        ks = np.empty((count, self.kvheads), np.float32)
        vs = np.empty_like(ks)
        _check(self._lib.needle2_gpu_kv_export(self.ptr, layer, seq, k.ctypes.data, v.ctypes.data, ks.ctypes.data,
                                               vs.ctypes.data, int(first_slot), count), "KV export")
        return k, v, ks, vs

    def __del__(self):
        if getattr(self, "ptr", None):
            self._lib.needle2_gpu_kv_destroy(self.ptr)
            self.ptr = None
