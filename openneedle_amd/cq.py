"""CQ matrices in device memory, and plans that run many of them in one launch.

A :class:`CQMatrix` is one handle of the library's C ABI (``needle2_cq_*``,
plus an int8 handle ``needle2_sdot_*`` built on first use). The library
checks the geometry, the norms, the codebook and the ternary codes itself
and refuses a matrix it cannot run, so this class only fixes the dtypes and
checks that the host buffers are as long as the geometry says before their
addresses cross the boundary.

Code written for the reference's ``NativeCQ`` keeps working unchanged by
pointing ``NEEDLE2_NATIVE_LIBRARY`` at this library; this module is the
gfx950 side's own interface, with device-resident entry points the
reference does not have.
"""
from __future__ import annotations

import ctypes as ct
from dataclasses import dataclass

import numpy as np

from . import _ffi
from ._ffi import GpuError, addr, check, check_void
from .device import stream_ptr


@dataclass(frozen=True)
class Geometry:
    """Shape and storage of a CQ matrix: ``bits`` 2/3/4, or 5 for ternary crumbs."""

    rows: int
    cols: int
    bits: int
    group: int

    @property
    def storage_bits(self) -> int:
        return 2 if self.bits == 5 else self.bits

    @property
    def padded(self) -> int:
        return -(-self.cols // self.group) * self.group

    @property
    def row_bytes(self) -> int:
        return self.padded * self.storage_bits // 8

    @property
    def groups(self) -> int:
        return self.padded // self.group

    @property
    def centroids(self) -> int:
        return 3 if self.bits == 5 else 1 << self.bits

    def int8_groups(self, reference_bound: bool) -> bool:
        """Whether the int8 path takes this matrix: the reference's rule (2/4-bit codes, groups 64..131072)
        or, with ``reference_bound`` False, every group the GPU kernels run (CQ4 from 8, CQ2 from 16)."""
        if self.bits not in (2, 4) or self.group > 131072:
            return False
        low = 64 if reference_bound else (8 if self.bits == 4 else 16)
        return self.group >= low


def _host(a, dtype, count: int, what: str) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=dtype)
    if a.size != count:
        raise ValueError(f"{what}: expected {count} values, got {a.size}")
    return a


class CQMatrix:
    """A ``rows x cols`` CQ matrix uploaded to the GPU.

    ``packed``: the row-major LSB-first code bitstream, ``rows x row_bytes``
    bytes; ``norms``: fp16 ``rows x groups``; ``codebook``: the sorted
    centroids, already scaled by ``1/sqrt(group)`` as a CACT header stores
    them. ``device=(d_packed, d_norms, stream)`` builds the matrix from
    device-resident copies of the same arrays instead (no host copy; the
    caller keeps them alive until the stream has run).
    """

    def __init__(self, packed, norms, shape, bits, group, codebook, *, device=None, int8: bool = False):
        rows, cols = (int(v) for v in shape)
        self.geometry = g = Geometry(rows, cols, int(bits), int(group))
        self.codebook = np.ascontiguousarray(codebook, np.float32)
        self._lib = _ffi.lib()
        self._int8 = None
        self._int8_ref = None
        # host arrays (when given) stay referenced: a later int8 handle is built from them
        self.packed = None if packed is None else _host(packed, np.uint8, rows * g.row_bytes, "packed codes")
        self.norms = None if norms is None else _host(norms, np.float16, rows * g.groups, "group norms")
        self._device_src = None
        if device is None:
            if self.packed is None or self.norms is None:
                raise ValueError("CQMatrix needs host packed codes and norms, or device=")
            self._handle = self._lib.needle2_cq_create(self.packed.ctypes.data, self.norms.ctypes.data, rows, cols,
                                                       g.bits, g.group, self.codebook.ctypes.data)
        else:
            d_packed, d_norms, stream = device
            # only valid while the caller's device copies live: used by this constructor alone
            self._device_src = (addr(d_packed), addr(d_norms), stream_ptr(stream))
            self._handle = self._lib.needle2_gpu_cq_create_device(self._device_src[0], self._device_src[1], rows,
                                                                  cols, g.bits, g.group, self.codebook.ctypes.data,
                                                                  self._device_src[2])
        try:
            if not self._handle:
                raise GpuError(f"CQ matrix {rows}x{cols} ({g.bits}-bit, group {g.group}): {_ffi.last_error()}")
            if int8 and g.int8_groups(reference_bound=False):
                self.int8_handle()
        finally:
            self._device_src = None

    @classmethod
    def from_record(cls, record, **kw) -> "CQMatrix":
        """A CQ tensor record of a ``.cact`` archive (:class:`openneedle_amd.archive.TensorRecord`)."""
        return cls(record.packed, record.norms, record.shape, record.bits, record.group_size, record.cq_codebook(),
                   **kw)

    @property
    def shape(self) -> tuple[int, int]:
        return self.geometry.rows, self.geometry.cols

    @property
    def handle(self) -> int:
        """The ``needle2_cq_*`` handle (borrowed by plans and engines; valid until :meth:`close`)."""
        return self._handle

    # ---- lifetime ----------------------------------------------------------
    def close(self) -> None:
        for attr, fn in (("_int8", "needle2_sdot_destroy"), ("_int8_ref", "needle2_sdot_destroy"),
                         ("_handle", "needle2_cq_destroy")):
            h = getattr(self, attr, None)
            setattr(self, attr, None)
            if h:
                getattr(self._lib, fn)(h)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def int8_handle(self, reference_bound: bool = False) -> int:
        """The int8 (``needle2_sdot_*``) handle, built on first use. ``reference_bound``: through
        ``needle2_sdot_create`` (groups 64..131072, the reference's rule) instead of the wider export."""
        attr = "_int8_ref" if reference_bound else "_int8"
        h = getattr(self, attr)
        if h:
            return h
        g = self.geometry
        if reference_bound and not g.int8_groups(True):
            raise GpuError("int8 matrix: the reference's int8 path takes 2/4-bit codes and groups 64..131072")
        if self._device_src is not None:
            d_packed, d_norms, stream = self._device_src
            h = self._lib.needle2_gpu_sdot_create_device(d_packed, d_norms, g.rows, g.cols, g.bits, g.group,
                                                         self.codebook.ctypes.data, stream)
        elif self.packed is not None and self.norms is not None:
            create = self._lib.needle2_sdot_create if reference_bound else self._lib.needle2_gpu_sdot_create
            h = create(self.packed.ctypes.data, self.norms.ctypes.data, g.rows, g.cols, g.bits, g.group,
                       self.codebook.ctypes.data)
        else:
            raise GpuError("int8 matrix: built from device memory without host codes; pass int8=True at creation")
        if not h:
            raise GpuError(f"int8 matrix: {_ffi.last_error()}")
        setattr(self, attr, h)
        return h

    # ---- host-pointer calls (the reference ABI) ----------------------------
    def _batch(self, x) -> tuple[np.ndarray, int]:
        x = np.ascontiguousarray(x, np.float32)
        if x.ndim == 0 or x.shape[-1] != self.geometry.cols:
            raise ValueError(f"input rows must hold {self.geometry.cols} values; got shape {x.shape}")
        return x, x.size // self.geometry.cols

    def matvec(self, x, *, mode: int = 0) -> np.ndarray:
        """FP32 product ``y[..., rows] = W x[..., cols]`` through ``needle2_cq_linear`` (``mode`` > 0:
        ``needle2_cq_linear_lookup``)."""
        x, batch = self._batch(x)
        y = np.empty(x.shape[:-1] + (self.geometry.rows,), np.float32)
        if mode:
            self._lib.needle2_cq_linear_lookup(self._handle, x.ctypes.data, y.ctypes.data, batch, 1, int(mode))
        else:
            self._lib.needle2_cq_linear(self._handle, x.ctypes.data, y.ctypes.data, batch, 1)
        check_void("CQ matvec")
        return y

    def matvec_int8(self, x, *, reference_bound: bool = False) -> np.ndarray:
        """The int8 product (SDOT arithmetic) through ``needle2_sdot_linear``."""
        x, batch = self._batch(x)
        h = self.int8_handle(reference_bound)
        y = np.empty(x.shape[:-1] + (self.geometry.rows,), np.float32)
        self._lib.needle2_sdot_linear(h, x.ctypes.data, y.ctypes.data, batch, 1)
        check_void("int8 matvec")
        return y

    def rows(self, ids) -> np.ndarray:
        """Dequantized rows ``ids`` (any integer shape) through ``needle2_cq_rows``."""
        ids = np.asarray(ids)
        if ids.dtype.kind not in "iu":
            raise TypeError("row ids must be integers")
        flat = np.ascontiguousarray(ids, np.int64).reshape(-1)
        out = np.empty(ids.shape + (self.geometry.cols,), np.float32)
        self._lib.needle2_cq_rows(self._handle, flat.ctypes.data, out.ctypes.data, flat.size)
        check_void("CQ rows")
        return out

    def dense(self) -> np.ndarray:
        return self.rows(np.arange(self.geometry.rows))

    def select(self, x, ids, *, int8: bool = False) -> np.ndarray:
        """Rows ``ids`` of the product for one input vector (candidate projection); bit-identical to
        ``matvec(x)[ids]`` (``matvec_int8`` with ``int8``)."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        if x.size != self.geometry.cols:
            raise ValueError(f"select takes one input vector of {self.geometry.cols} values")
        ids = np.asarray(ids)
        if ids.ndim != 1 or (ids.size and ids.dtype.kind not in "iu"):
            raise ValueError("candidate ids: a one-dimensional integer array")
        ids = np.ascontiguousarray(ids, np.int32)
        y = np.empty(ids.size, np.float32)
        if int8:
            check(self._lib.needle2_gpu_sdot_candidates(self.int8_handle(), x.ctypes.data, ids.ctypes.data,
                                                        ids.size, y.ctypes.data), "int8 select")
        else:
            check(self._lib.needle2_gpu_cq_candidates(self._handle, x.ctypes.data, ids.ctypes.data, ids.size,
                                                      y.ctypes.data), "CQ select")
        return y

    # ---- device-resident calls (addresses of device memory) ----------------
    def matvec_device(self, d_x, d_y, batch: int, stream=None) -> None:
        check(self._lib.needle2_gpu_cq_linear_device(self._handle, addr(d_x), addr(d_y), int(batch),
                                                     stream_ptr(stream)), "CQ matvec (device)")

    def matvec_int8_device(self, d_x, d_y, batch: int, stream=None) -> None:
        check(self._lib.needle2_gpu_sdot_linear_device(self.int8_handle(), addr(d_x), addr(d_y), int(batch),
                                                       stream_ptr(stream)), "int8 matvec (device)")

    def int8_dots_device(self, d_x, d_dots, batch: int, stream=None) -> None:
        """The int32 group dots of the int8 product, ``d_dots[b][row][group]`` (device int32)."""
        check(self._lib.needle2_gpu_sdot_dots_device(self.int8_handle(), addr(d_x), addr(d_dots), int(batch),
                                                     stream_ptr(stream)), "int8 dots (device)")

    def select_device(self, d_x, d_ids, count: int, d_y, stream=None, *, int8: bool = False) -> None:
        if int8:
            check(self._lib.needle2_gpu_sdot_candidates_device(self.int8_handle(), addr(d_x), addr(d_ids),
                                                               int(count), addr(d_y), stream_ptr(stream)),
                  "int8 select (device)")
        else:
            check(self._lib.needle2_gpu_cq_candidates_device(self._handle, addr(d_x), addr(d_ids), int(count),
                                                             addr(d_y), stream_ptr(stream)), "CQ select (device)")

    def gemm_device(self, d_x, d_y, m: int, stream=None, events=None, repeat: int = 1) -> None:
        """Prefill GEMM on fp16 MFMA: device ``y[m][rows]`` from ``x[m][cols]``. ``events``: a (start, stop)
        pair recorded around ``repeat`` back-to-back GEMM launches (per-launch time = elapsed / repeat)."""
        s = stream_ptr(stream)
        if events is None:
            check(self._lib.needle2_gpu_cq_gemm_device(self._handle, addr(d_x), addr(d_y), int(m), s), "GEMM")
        else:
            check(self._lib.needle2_gpu_cq_gemm_timed(self._handle, addr(d_x), addr(d_y), int(m), s,
                                                      events[0].ptr, events[1].ptr, int(repeat)), "GEMM")


def matvec_many(matrices, x, *, mode: int = 0) -> list[np.ndarray]:
    """``needle2_cq_linear_many``: one input vector through several matrices (one transform for all
    matrices of one input geometry)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    outs = [np.empty(m.geometry.rows, np.float32) for m in matrices]
    handles = (ct.c_void_p * len(matrices))(*[m.handle for m in matrices])
    ys = (ct.c_void_p * len(matrices))(*[o.ctypes.data for o in outs])
    for m in matrices:
        if m.geometry.cols != x.size:
            raise ValueError("matvec_many: every matrix must take the input's length")
    _ffi.lib().needle2_cq_linear_many(handles, len(matrices), x.ctypes.data, ys, 1, int(mode))
    check_void("CQ matvec_many")
    return outs


class Plan:
    """Matrices of one input geometry, matrix ``i`` reading device ``xs[i]`` (``[batch][cols]``) and writing
    ``ys[i]`` (``[batch][rows_i]``), run by one prepare launch and one GEMV launch."""

    def __init__(self, matrices, xs, ys, batch: int = 1, int8: bool = False):
        self._lib = _ffi.lib()
        n = len(matrices)
        handles = (ct.c_void_p * n)(*[m.int8_handle() if int8 else m.handle for m in matrices])
        xa = (ct.c_void_p * n)(*[addr(p) for p in xs])
        ya = (ct.c_void_p * n)(*[addr(p) for p in ys])
        create = self._lib.needle2_gpu_sdot_plan_create if int8 else self._lib.needle2_gpu_cq_plan_create
        self._matrices = list(matrices)  # the plan borrows their handles
        self.ptr = create(handles, n, xa, ya, int(batch))
        if not self.ptr:
            raise GpuError(f"plan: {_ffi.last_error()}")

    def run(self, stream=None, gemv_events=None, *, next=None, prepared: bool = False) -> None:
        """One run on ``stream``. Chained int8 plans: with ``prepared`` the run uses the prepared input a chained
        call of its producer (a run with ``next=self``, or :meth:`KVCache.attention` with ``next=self``) left
        since this plan's last run, or prepares it itself when none did; ``next``, a one-matrix int8 plan whose
        input is this plan's output, gets its input prepared for its own run with ``prepared=True``. Outputs
        are those of unchained runs."""
        s = stream_ptr(stream)
        if next is not None or prepared:
            if gemv_events is not None:
                raise ValueError("plan run: timing events are for unchained runs")
            check(self._lib.needle2_gpu_plan_run_chained(self.ptr, next.ptr if next is not None else None,
                                                         int(bool(prepared)), s), "plan run")
        elif gemv_events is None:
            check(self._lib.needle2_gpu_plan_run(self.ptr, s), "plan run")
        else:
            check(self._lib.needle2_gpu_plan_run_timed(self.ptr, s, gemv_events[0].ptr, gemv_events[1].ptr),
                  "plan run")

    def close(self) -> None:
        ptr, self.ptr = getattr(self, "ptr", None), None
        if ptr:
            self._lib.needle2_gpu_plan_destroy(ptr)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
