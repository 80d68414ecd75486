"""CPU checks of the drop-in boundary, at the C level.

The library must export every symbol ``include/*.h`` declares and every symbol
the reference's loader binds (eagerly: needle2/native.py:128-145; lazily: the
engine, native.py:397-660), with the reference's signatures, so that the
reference's own Python runs on it through ``NEEDLE2_NATIVE_LIBRARY``. Those
checks need no GPU: the library loads on this host and its argument checks
run before any device call. A rejected matrix comes back as NULL with the
reason in ``needle2_gpu_error`` (the reference's convention for
``needle2_cq_create``, cq.cpp:350-352).
"""
import ctypes as ct
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from openneedle_amd import _ffi

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names |= set(re.findall(r"\b(needle2_[a-z0-9_]+)\s*\(", text))
    return names


def exported_symbols(path):
    out = subprocess.run(["nm", "-D", "--defined-only", str(path)], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


# needle2/native.py:128-145 (eager) and :397-660 (lazy engine bindings)
REFERENCE_EAGER = {
    "needle2_native_features", "needle2_cq_create", "needle2_cq_destroy", "needle2_cq_linear",
    "needle2_cq_linear_lookup", "needle2_sdot_supported", "needle2_sdot_create", "needle2_sdot_destroy",
    "needle2_sdot_linear", "needle2_cq_rows",
}
REFERENCE_ENGINE = {
    "needle2_engine_create", "needle2_engine_destroy", "needle2_engine_reset", "needle2_engine_step",
    "needle2_engine_error", "needle2_engine_set_lookup", "needle2_engine_set_sdot", "needle2_engine_set_int8_kv",
    "needle2_engine_kv_storage_bytes", "needle2_engine_cache_prefix", "needle2_engine_reset_to_prefix",
    "needle2_engine_step_candidates", "needle2_engine_prefill", "needle2_engine_import",
    "needle2_engine_decode_loop", "needle2_cq_linear_many", "needle2_engine_project_candidates",
}


def test_library_exports_every_declared_symbol():
    exported = exported_symbols(_ffi.library_path())
    declared = declared_symbols()
    assert declared, "no declarations found in include/"
    assert declared <= exported, sorted(declared - exported)
    assert REFERENCE_EAGER <= exported
    assert REFERENCE_ENGINE <= exported


def test_signature_table_covers_the_header():
    """Every declared export has a ctypes signature, and the table names nothing the header does not declare."""
    assert set(_ffi.SIGNATURES) == declared_symbols()


def header_prototypes():
    """name -> number of parameters, from the declarations in include/*.h."""
    protos = {}
    for header in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        for name, params in re.findall(r"\b(needle2_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
            params = params.strip()
            protos[name] = 0 if params in ("", "void") else params.count(",") + 1
    return protos


def test_signature_arity_matches_the_header():
    protos = header_prototypes()
    for name, (_, args) in _ffi.SIGNATURES.items():
        assert len(args) == protos[name], name


# the reference loader's eager argtypes (needle2/native.py:128-145), by arity and pointer / int positions
REFERENCE_ARGTYPES = {
    "needle2_cq_create": "ppiiiip", "needle2_cq_destroy": "p", "needle2_cq_linear": "pppii",
    "needle2_cq_linear_lookup": "pppiii", "needle2_sdot_create": "ppiiiip", "needle2_sdot_destroy": "p",
    "needle2_sdot_linear": "pppii", "needle2_cq_rows": "pppi", "needle2_native_features": "",
    "needle2_sdot_supported": "",
}


def test_reference_signatures():
    kinds = {ct.c_void_p: "p", ct.c_int: "i", ct.c_char_p: "p"}
    for name, want in REFERENCE_ARGTYPES.items():
        got = "".join(kinds[a] for a in _ffi.SIGNATURES[name][1])
        assert got == want, name


def test_library_loads_and_answers_capability_queries():
    lib = _ffi.lib()
    assert _ffi.loadable()
    assert b"gfx950" in lib.needle2_native_features()
    assert lib.needle2_sdot_supported() == 1


def test_library_selection_env(monkeypatch, tmp_path):
    _ffi.lib.cache_clear()
    try:
        monkeypatch.setenv(_ffi.ENV, "  ")
        with pytest.raises(_ffi.LibraryMissing, match="empty"):
            _ffi.library_path()
        monkeypatch.setenv(_ffi.ENV, str(tmp_path / "missing.so"))
        with pytest.raises(_ffi.LibraryMissing, match="does not exist"):
            _ffi.library_path()
        assert not _ffi.loadable()
        monkeypatch.setenv(_ffi.ENV, str(_ffi.IN_TREE))
        assert _ffi.library_path() == _ffi.IN_TREE.resolve()
    finally:
        monkeypatch.delenv(_ffi.ENV, raising=False)
        _ffi.lib.cache_clear()


def test_engine_create_refuses_a_missing_table():
    lib = _ffi.lib()
    assert not lib.needle2_engine_create(None, None, 0, 1, 0)
    assert b"null" in lib.needle2_engine_error()


# ---- argument checks of needle2_cq_create / needle2_sdot_create (before any device call) ----------------------
def _example(bits=2, group=128):
    from tests.cases import example
    packed, norms, cb, dense = example(bits, group=group)
    return packed, norms.view(np.uint16), dense.shape, bits, group, cb


def _create(packed, norms, shape, bits, group, cb, fn="needle2_cq_create"):
    lib = _ffi.lib()
    cb = np.ascontiguousarray(cb, np.float32)
    h = getattr(lib, fn)(packed.ctypes.data, norms.ctypes.data, shape[0], shape[1], bits, group, cb.ctypes.data)
    return h, _ffi.last_error()


def test_create_rejects_bad_geometry():
    packed, norms, shape, bits, group, cb = _example()
    for args, message in (((0, 5), bits, group), "shape"), (((shape), 6, group), "bits"), \
                         (((shape), bits, 48), "power of two"):
        h, err = _create(packed, norms, args[0], args[1], args[2], cb)
        assert not h and message in err, err


def test_create_rejects_corrupt_norms():
    packed, norms, shape, bits, group, cb = _example()
    for value in (-1.0, np.inf, np.nan):
        bad = norms.view(np.float16).copy()
        bad[1, 0] = value
        h, err = _create(packed, bad.view(np.uint16), shape, bits, group, cb)
        assert not h and "norm" in err, err
    ok = norms.view(np.float16).copy()
    ok[1, 0] = -0.0  # a signed zero is a zero norm
    h, err = _create(packed, ok.view(np.uint16), shape, bits, group, cb)
    assert not h or not err  # accepted (on a host without a GPU the upload itself fails later)


def test_create_rejects_unsorted_or_infinite_codebooks():
    packed, norms, shape, bits, group, cb = _example()
    for codebook in ([np.nan, 0, 1, 2], [-2, -1, 0, np.inf], [2, 1, 0, -1], [0, 0, 1, 2]):
        h, err = _create(packed, norms, shape, bits, group, np.asarray(codebook, np.float32))
        assert not h and "codebook" in err, err


def test_create_rejects_reserved_ternary_crumb():
    packed, norms, shape, bits, group, cb = _example(bits=5)
    bad = packed.copy()
    bad[0, 0] = (bad[0, 0] & ~np.uint8(3)) | np.uint8(2)
    h, err = _create(bad, norms, shape, bits, group, cb)
    assert not h and "ternary" in err, err


def test_sdot_create_keeps_the_reference_bound():
    """needle2_sdot_create takes 2/4-bit codes and groups 64..131072 (sdot.cpp:351-354)."""
    packed, norms, shape, _, _, cb = _example(bits=3, group=128)
    h, err = _create(packed, norms, shape, 3, 128, cb, "needle2_sdot_create")
    assert not h and "CQ2/CQ4" in err
    packed, norms, shape, _, _, cb = _example(bits=4, group=32)
    h, err = _create(packed, norms, shape, 4, 32, cb, "needle2_sdot_create")
    assert not h and "group" in err


def test_python_binding_checks_buffer_lengths():
    """The binding refuses host buffers shorter than the geometry before their addresses cross the boundary."""
    from openneedle_amd.cq import CQMatrix
    packed, norms, shape, bits, group, cb = _example()
    with pytest.raises(ValueError, match="packed codes"):
        CQMatrix(packed[:-1], norms, shape, bits, group, cb)
    with pytest.raises(ValueError, match="group norms"):
        CQMatrix(packed, norms[:-1], shape, bits, group, cb)
