"""CPU checks of the drop-in boundary: the library loads, exports every symbol
declared in include/*.h plus the ones the reference's loader binds, and the
Python mirror validates arguments like the reference (needle2/native.py)."""
import ctypes as ct
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from openneedle_amd import native

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
    path = native.library_path()
    exported = exported_symbols(path)
    declared = declared_symbols()
    assert declared, "no declarations found in include/"
    assert declared <= exported, sorted(declared - exported)
    assert REFERENCE_EAGER <= exported
    assert REFERENCE_ENGINE <= exported


def test_library_loads_and_binds_like_reference_loader():
    lib = native._library()
    for name in REFERENCE_EAGER:
        assert getattr(lib, name)
    assert native.available()
    assert "gfx950" in native.features()
    assert native.sdot_available()


def test_library_selection_env(monkeypatch, tmp_path):
    native._library.cache_clear()
    try:
        monkeypatch.setenv("NEEDLE2_NATIVE_LIBRARY", "  ")
        with pytest.raises(RuntimeError, match="must name a prebuilt"):
            native.library_path()
        monkeypatch.setenv("NEEDLE2_NATIVE_LIBRARY", str(tmp_path / "missing.so"))
        with pytest.raises(RuntimeError, match="not found"):
            native.library_path()
        assert not native.available()
        monkeypatch.setenv("NEEDLE2_NATIVE_LIBRARY", str(native.DEFAULT_LIBRARY))
        assert native.library_path() == native.DEFAULT_LIBRARY.resolve()
    finally:
        monkeypatch.delenv("NEEDLE2_NATIVE_LIBRARY", raising=False)
        native._library.cache_clear()


def test_engine_is_refused_through_the_reference_error_channel():
    lib = native._library()
    lib.needle2_engine_create.restype = ct.c_void_p
    lib.needle2_engine_error.restype = ct.c_char_p
    assert not lib.needle2_engine_create(None, None, 0, 1, 0)
    assert b"engine" in lib.needle2_engine_error()


# Argument validation happens before any device call (needle2/native.py:172-202).
def _args(bits=2, group=128):
    from tests.cases import example
    packed, norms, cb, dense = example(bits, group=group)
    return packed, norms, dense.shape, bits, group, cb


def test_rejects_bad_geometry():
    packed, norms, shape, bits, group, cb = _args()
    with pytest.raises(ValueError, match="positive two-dimensional"):
        native.NativeCQ(packed, norms, (0, 5), bits, group, cb)
    with pytest.raises(ValueError, match="storage bits"):
        native.NativeCQ(packed, norms, shape, 6, group, cb)
    with pytest.raises(ValueError, match="power of two"):
        native.NativeCQ(packed, norms, shape, bits, 48, cb)
    with pytest.raises(ValueError, match="incorrect number of centroids"):
        native.NativeCQ(packed, norms, shape, bits, group, cb[:3])


def test_rejects_corrupt_norms_and_codebooks():
    packed, norms, shape, bits, group, cb = _args()
    for value in (-1.0, np.inf, np.nan):
        bad = norms.copy()
        bad[0, 0] = value
        with pytest.raises(ValueError, match="norms must be finite and nonnegative"):
            native.NativeCQ(packed, bad, shape, bits, group, cb)
    for codebook in ([np.nan, 0, 1, 2], [-2, -1, 0, np.inf], [2, 1, 0, -1], [0, 0, 1, 2]):
        with pytest.raises(ValueError, match="codebook must be finite and strictly sorted"):
            native.NativeCQ(packed, norms, shape, bits, group, codebook)


def test_rejects_reserved_ternary_crumb():
    packed, norms, shape, bits, group, cb = _args(bits=5)
    bad = packed.copy()
    bad[0, 0] = (bad[0, 0] & ~np.uint8(3)) | np.uint8(2)
    with pytest.raises(ValueError, match="Invalid ternary crumb code 2"):
        native.NativeCQ(bad, norms, shape, bits, group, cb)
