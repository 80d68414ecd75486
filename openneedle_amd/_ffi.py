"""Locating, loading and typing ``libneedle2_native.so``.

The library is the product; this module only gives Python a typed handle on
it. Every export of ``include/needle2_native.h`` is listed once in
:data:`SIGNATURES` (result type, argument types), and :func:`lib` applies the
whole table when the library is first loaded, so a missing export fails at
load time rather than at first use.

Library choice: ``$NEEDLE2_NATIVE_LIBRARY`` when it is set (the variable the
reference's own loader honours, needle2/native.py:77-84), otherwise the
in-tree build next to this file. Nothing here falls back to a CPU path: with
no library every call raises :class:`LibraryMissing`.
"""
from __future__ import annotations

import ctypes as ct
import functools
import os
from pathlib import Path

HERE = Path(__file__).resolve().parent
IN_TREE = HERE / "libneedle2_native.so"
ENV = "NEEDLE2_NATIVE_LIBRARY"

vp, i32, f32, sz, cstr = ct.c_void_p, ct.c_int, ct.c_float, ct.c_size_t, ct.c_char_p

# name: (restype, argtypes). Grouped as the header groups them.
SIGNATURES: dict[str, tuple] = {
    # reference ABI (needle2/native.py:128-145, cq.cpp:342-371, sdot.cpp:349-360)
    "needle2_native_features": (cstr, []),
    "needle2_cq_create": (vp, [vp, vp, i32, i32, i32, i32, vp]),
    "needle2_cq_destroy": (None, [vp]),
    "needle2_cq_linear": (None, [vp, vp, vp, i32, i32]),
    "needle2_cq_linear_lookup": (None, [vp, vp, vp, i32, i32, i32]),
    "needle2_cq_linear_many": (None, [vp, i32, vp, vp, i32, i32]),
    "needle2_cq_rows": (None, [vp, vp, vp, i32]),
    "needle2_sdot_supported": (i32, []),
    "needle2_sdot_create": (vp, [vp, vp, i32, i32, i32, i32, vp]),
    "needle2_sdot_destroy": (None, [vp]),
    "needle2_sdot_linear": (None, [vp, vp, vp, i32, i32]),
    # engine (needle2/csrc/engine.cpp:1499-1548)
    "needle2_engine_error": (cstr, []),
    "needle2_engine_create": (vp, [vp, vp, i32, i32, i32]),
    "needle2_engine_destroy": (None, [vp]),
    "needle2_engine_set_lookup": (None, [vp, i32]),
    "needle2_engine_set_sdot": (i32, [vp]),
    "needle2_engine_reset": (None, [vp, i32]),
    "needle2_engine_cache_prefix": (i32, [vp]),
    "needle2_engine_reset_to_prefix": (i32, [vp]),
    "needle2_engine_step": (i32, [vp, i32, vp, vp]),
    "needle2_engine_prefill": (i32, [vp, vp, i32, i32, vp, vp]),
    "needle2_engine_step_candidates": (i32, [vp, i32, vp, i32, vp, vp]),
    "needle2_engine_project_candidates": (i32, [vp, vp, i32, vp]),
    "needle2_engine_decode_loop": (i32, [vp, i32, i32, vp, vp, vp]),
    "needle2_engine_import": (i32, [vp, i32, i32, vp, vp, i32, vp, vp]),
    "needle2_engine_set_int8_kv": (i32, [vp, i32]),
    "needle2_engine_kv_storage_bytes": (sz, [vp]),
    # additive exports
    "needle2_gpu_error": (cstr, []),
    "needle2_gpu_sdot_create": (vp, [vp, vp, i32, i32, i32, i32, vp]),
    "needle2_gpu_cq_create_device": (vp, [vp, vp, i32, i32, i32, i32, vp, vp]),
    "needle2_gpu_sdot_create_device": (vp, [vp, vp, i32, i32, i32, i32, vp, vp]),
    "needle2_gpu_cq_linear_device": (i32, [vp, vp, vp, i32, vp]),
    "needle2_gpu_sdot_linear_device": (i32, [vp, vp, vp, i32, vp]),
    "needle2_gpu_sdot_linear_device_noalloc": (i32, [vp, vp, vp, i32, vp]),
    "needle2_gpu_sdot_dots_device": (i32, [vp, vp, vp, i32, vp]),
    "needle2_gpu_cq_candidates": (i32, [vp, vp, vp, i32, vp]),
    "needle2_gpu_cq_candidates_device": (i32, [vp, vp, vp, i32, vp, vp]),
    "needle2_gpu_sdot_candidates": (i32, [vp, vp, vp, i32, vp]),
    "needle2_gpu_sdot_candidates_device": (i32, [vp, vp, vp, i32, vp, vp]),
    "needle2_gpu_cq_gemm_device": (i32, [vp, vp, vp, i32, vp]),
    "needle2_gpu_cq_gemm_timed": (i32, [vp, vp, vp, i32, vp, vp, vp, i32]),
    "needle2_gpu_cq_plan_create": (vp, [vp, i32, vp, vp, i32]),
    "needle2_gpu_sdot_plan_create": (vp, [vp, i32, vp, vp, i32]),
    "needle2_gpu_plan_run": (i32, [vp, vp]),
    "needle2_gpu_plan_run_timed": (i32, [vp, vp, vp, vp]),
    "needle2_gpu_plan_run_chained": (i32, [vp, vp, i32, vp]),
    "needle2_gpu_plan_destroy": (None, [vp]),
    "needle2_gpu_malloc": (vp, [sz]),
    "needle2_gpu_free": (None, [vp]),
    "needle2_gpu_memcpy": (i32, [vp, vp, sz, i32]),
    "needle2_gpu_memset": (i32, [vp, i32, sz]),
    "needle2_gpu_copy_kernel": (i32, [vp, vp, sz, vp]),
    "needle2_gpu_calib_launch": (i32, [i32, vp, vp]),
    "needle2_gpu_calib_lds": (i32, [i32, vp, vp, vp]),
    "needle2_gpu_calib_stream": (i32, [vp, sz, i32, vp, vp]),
    "needle2_gpu_synchronize": (i32, []),
    "needle2_gpu_stream_create": (vp, []),
    "needle2_gpu_stream_destroy": (None, [vp]),
    "needle2_gpu_stream_synchronize": (i32, [vp]),
    "needle2_gpu_event_create": (vp, []),
    "needle2_gpu_event_destroy": (None, [vp]),
    "needle2_gpu_event_record": (i32, [vp, vp]),
    "needle2_gpu_event_elapsed": (f32, [vp, vp]),
    "needle2_gpu_device_info": (i32, [cstr, i32]),
    "needle2_gpu_graph_begin": (i32, [vp]),
    "needle2_gpu_graph_end": (vp, [vp]),
    "needle2_gpu_graph_launch": (i32, [vp, vp]),
    "needle2_gpu_graph_destroy": (None, [vp]),
    "needle2_gpu_kv_create": (vp, [i32, i32, i32, i32, i32]),
    "needle2_gpu_kv_destroy": (None, [vp]),
    "needle2_gpu_kv_storage_bytes": (sz, [vp]),
    "needle2_gpu_kv_store": (i32, [vp, i32, vp, vp, i32, i32, vp, vp]),
    "needle2_gpu_kv_store_device": (i32, [vp, i32, vp, vp, i32, vp, vp]),
    "needle2_gpu_attention": (i32, [vp, i32, vp, vp, i32, i32, vp, vp, i32, vp]),
    "needle2_gpu_attention_chained": (i32, [vp, i32, vp, vp, i32, i32, vp, vp, i32, vp, vp, vp, vp, vp]),
    "needle2_gpu_kv_import": (i32, [vp, i32, i32, vp, vp, vp, vp, i32, i32]),
    "needle2_gpu_kv_export": (i32, [vp, i32, i32, vp, vp, vp, vp, i32, i32]),
}


class LibraryMissing(RuntimeError):
    """The gfx950 library could not be found or loaded."""


class GpuError(RuntimeError):
    """A library call reported failure; the message is the library's own."""


def library_path() -> Path:
    """The shared library this process uses (see the module docstring)."""
    chosen = os.environ.get(ENV)
    if chosen is None:
        if not IN_TREE.is_file():
            raise LibraryMissing(f"{IN_TREE} has not been built; run python -m openneedle_amd.build")
        return IN_TREE
    if not chosen.strip():
        raise LibraryMissing(f"{ENV} is set but empty; it must name a prebuilt library file")
    path = Path(chosen).expanduser().resolve()
    if not path.is_file():
        raise LibraryMissing(f"{ENV} names {path}, which does not exist")
    return path


@functools.lru_cache(maxsize=1)
def lib() -> ct.CDLL:
    """The loaded library with every signature of :data:`SIGNATURES` applied."""
    try:
        handle = ct.CDLL(str(library_path()))
    except OSError as exc:
        raise LibraryMissing(str(exc)) from exc
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype, fn.argtypes = res, args
    return handle


def loadable() -> bool:
    """True when :func:`lib` succeeds (the library exists and exports every symbol)."""
    try:
        lib()
    except (LibraryMissing, AttributeError):
        return False
    return True


def last_error() -> str:
    """Message of the last failed library call on this thread ('' after a success)."""
    return lib().needle2_gpu_error().decode()


def check(status: int, what: str) -> None:
    """Raise :class:`GpuError` for a nonzero status of an ``int`` entry point."""
    if status != 0:
        raise GpuError(f"{what}: {last_error()}")


def check_void(what: str) -> None:
    """After a ``void`` entry point of the reference ABI: raise if it recorded a failure."""
    msg = last_error()
    if msg:
        raise GpuError(f"{what}: {msg}")


def addr(obj) -> int | None:
    """Device or host address of a buffer-like argument (None passes NULL)."""
    if obj is None:
        return None
    if isinstance(obj, int):
        return obj
    ptr = getattr(obj, "ptr", None)
    if ptr is not None:
        return int(ptr)
    return int(obj.ctypes.data)
