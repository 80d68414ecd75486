"""One sequence decoded on the GPU behind ``needle2_engine_*``.

The engine itself is C++ and HIP (``csrc/engine.cpp``); it validates its own
arguments (token and candidate ranges, context length, prefix geometry,
grammar tables) and reports failures through ``needle2_engine_error``. This
module builds what the C ABI takes from a ``.cact`` archive (the engine
configuration and the tensor table, whose ``ctypes`` layouts are the
reference's ABI) and returns the engine's outputs as numpy arrays.

:class:`EngineBinding` speaks to any library that exports the engine ABI, so
the same code drives this library (:class:`GpuEngine`) and, in the tests, the
reference's Engine built from source.
"""
from __future__ import annotations

import ctypes as ct
from pathlib import Path

import numpy as np

from . import _ffi
from .archive import CQ, FP16, FP32, Archive, canonical_shapes


# ---- the reference's ABI structures (needle2/csrc/engine.cpp:14-19, 326-338) --------------------------------
class TensorDesc(ct.Structure):
    _fields_ = [("cq", ct.c_void_p), ("data", ct.c_void_p), ("rows", ct.c_int), ("cols", ct.c_int)]


_CONFIG_INTS = ("vocab", "dim", "heads", "kvheads", "layers", "head_dim", "max_seq", "hada", "lanes", "window",
                "slots", "subdim", "tables", "taps", "dilation", "num_orders")


class EngineConfig(ct.Structure):
    _fields_ = [(n, ct.c_int) for n in _CONFIG_INTS] + \
               [("orders", ct.c_int * 4), ("num_sites", ct.c_int), ("sites", ct.c_int * 4), ("rope_theta", ct.c_float)]


class DFAStateDesc(ct.Structure):
    _fields_ = [("num_states", ct.c_int), ("initial_state", ct.c_int), ("eos_id", ct.c_int), ("stop_id", ct.c_int),
                ("tool_start_id", ct.c_int), ("tool_end_id", ct.c_int), ("state_types", ct.POINTER(ct.c_int)),
                ("fallback_next_states", ct.POINTER(ct.c_int)), ("candidate_offsets", ct.POINTER(ct.c_int)),
                ("candidate_tokens", ct.POINTER(ct.c_int)), ("next_states", ct.POINTER(ct.c_int))]


# archive metadata key of each configuration integer (the header fields of needle2/archive.py)
_METADATA_KEY = dict(vocab="vocab_size", dim="d_model", heads="num_heads", kvheads="num_kv_heads",
                     layers="num_layers", head_dim="head_dim", max_seq="max_seq_len", hada="hada_n",
                     lanes="mhc_lanes", window="kv_window", slots="engram_slots", subdim="engram_sub_dim",
                     tables="num_engram_tables", taps="engram_conv_taps", dilation="engram_conv_dilation")


def engine_config(metadata: dict) -> EngineConfig:
    cfg = EngineConfig()
    for field, key in _METADATA_KEY.items():
        setattr(cfg, field, int(metadata[key]))
    orders, sites = list(metadata["engram_orders"]), list(metadata["engram_layers"])
    cfg.num_orders, cfg.num_sites = len(orders), len(sites)
    cfg.orders = (ct.c_int * 4)(*orders)
    cfg.sites = (ct.c_int * 4)(*sites)
    cfg.rope_theta = float(metadata["rope_theta"])
    return cfg


def engine_tensors(archive: Archive) -> list[str]:
    """The architecture tensors in the order the engine's table lists them (probe heads excluded)."""
    names = list(canonical_shapes(archive.metadata))
    for name in names:
        rec = archive.tensors.get(name)
        if rec is None:
            raise ValueError(f"archive lacks tensor {name}")
        if rec.dtype not in (FP16, FP32, CQ):
            raise ValueError(f"{name} is not a numeric tensor")
    return names


class TensorTable:
    """The tensor table an engine borrows: CQ records as matrix handles made by ``make_cq(record)`` (which
    must have a ``handle``), every other record (and the mHC matrices) as an fp32 host copy."""

    def __init__(self, archive: Archive, make_cq):
        self.owners, descs = [], []
        for name in engine_tensors(archive):
            rec = archive.tensors[name]
            if rec.dtype == CQ and not name.startswith("mhc_"):
                mat = make_cq(rec)
                self.owners.append(mat)
                descs.append(TensorDesc(mat.handle, None, *rec.shape))
                continue
            dense = np.ascontiguousarray(rec.dequantize(), np.float32)
            self.owners.append(dense)
            rows = dense.shape[0] if dense.ndim > 1 else 1
            descs.append(TensorDesc(None, dense.ctypes.data, rows, dense.size // rows))
        self.descs = (TensorDesc * len(descs))(*descs)

    def __len__(self):
        return len(self.descs)


ENGINE_SIGNATURES = {name: sig for name, sig in _ffi.SIGNATURES.items() if name.startswith("needle2_engine_")}


class EngineError(RuntimeError):
    pass


class EngineBinding:
    """An engine of ``library`` over ``archive``; outputs are (logits, hidden) pairs as the ABI writes them.
    ``threads`` is the host thread count the reference's CPU engine takes (the GPU engine ignores it)."""

    def __init__(self, library, archive, make_cq, activation_bits: int = 0, threads: int = 1):
        if isinstance(archive, (str, Path)):
            archive = Archive.load(archive)
        for name, (res, args) in ENGINE_SIGNATURES.items():
            fn = getattr(library, name)
            fn.restype, fn.argtypes = res, args
        self._L = library
        self.archive = archive
        self.meta = archive.metadata
        self.vocab, self.layers, self.dim = (int(self.meta[k]) for k in ("vocab_size", "num_layers", "d_model"))
        self.tensors = TensorTable(archive, make_cq)
        self.config = engine_config(self.meta)
        self.h = library.needle2_engine_create(ct.byref(self.config), self.tensors.descs, len(self.tensors),
                                               int(threads), int(activation_bits))
        if not self.h:
            raise EngineError(self._message())
        self.position = 0
        self.prefix = 0

    def _message(self) -> str:
        return self._L.needle2_engine_error().decode()

    def _ok(self, status: int) -> int:
        if status < 0:
            raise EngineError(self._message())
        return status

    def _hidden(self, want: bool):
        return np.empty((self.layers, self.dim), np.float32) if want else None

    # ---- state ---------------------------------------------------------------------------------------------
    def reset(self, prefix: int = 0) -> None:
        self._L.needle2_engine_reset(self.h, int(prefix))
        self.position, self.prefix = 0, int(prefix)

    def set_int8_kv(self, enabled: bool = True) -> None:
        self._ok(self._L.needle2_engine_set_int8_kv(self.h, int(bool(enabled))))
        self.position = 0

    def set_sdot(self) -> None:
        self._ok(self._L.needle2_engine_set_sdot(self.h))

    @property
    def kv_storage_bytes(self) -> int:
        return int(self._L.needle2_engine_kv_storage_bytes(self.h))

    def cache_prefix(self) -> None:
        self._ok(self._L.needle2_engine_cache_prefix(self.h))

    def reset_to_prefix(self) -> int:
        self.position = self.prefix = self._ok(self._L.needle2_engine_reset_to_prefix(self.h))
        return self.position

    def import_state(self, tokens, positions, keys, values) -> None:
        """The state after ``tokens`` with K / V rows ``[layers][len(positions)][kv_heads][head_dim]``."""
        ids = np.ascontiguousarray(tokens, np.int32)
        pos = np.ascontiguousarray(positions, np.int32)
        k, v = (np.ascontiguousarray(a, np.float32) for a in (keys, values))
        want = (self.layers, pos.size, int(self.meta["num_kv_heads"]), int(self.meta["head_dim"]))
        if k.shape != want or v.shape != want:
            raise ValueError(f"import_state: keys and values of shape {want}")
        self._ok(self._L.needle2_engine_import(self.h, ids.size, self.prefix, ids.ctypes.data, pos.ctypes.data,
                                               pos.size, k.ctypes.data, v.ctypes.data))
        self.position = int(ids.size)

    # ---- forward -------------------------------------------------------------------------------------------
    def step(self, token: int, *, logits: bool = True, hidden: bool = False):
        """One token: (logits [vocab] or None, hidden [layers][d_model] or None)."""
        lg = np.empty(self.vocab, np.float32) if logits else None
        hd = self._hidden(hidden)
        self._ok(self._L.needle2_engine_step(self.h, int(token), _ffi.addr(lg), _ffi.addr(hd)))
        self.position += 1
        return lg, hd

    def step_candidates(self, token: int, candidates, *, hidden: bool = False):
        """One token, projecting only rows ``candidates`` of the LM head: (candidate logits, hidden)."""
        ids = np.ascontiguousarray(candidates, np.int32).reshape(-1)
        out = np.empty(ids.size, np.float32)
        hd = self._hidden(hidden)
        self._ok(self._L.needle2_engine_step_candidates(self.h, int(token), ids.ctypes.data, ids.size,
                                                        out.ctypes.data, _ffi.addr(hd)))
        self.position += 1
        return out, hd

    def project_candidates(self, candidates) -> np.ndarray:
        """Candidate logits of the state as it stands (after a step or a prefill)."""
        ids = np.ascontiguousarray(candidates, np.int32).reshape(-1)
        out = np.empty(ids.size, np.float32)
        self._ok(self._L.needle2_engine_project_candidates(self.h, ids.ctypes.data, ids.size, out.ctypes.data))
        return out

    def prefill(self, tokens, *, last_only: bool = False, hidden: bool = False):
        """A prompt: (logits [tokens][vocab], or [vocab] with ``last_only``; the last token's hidden or None)."""
        ids = np.ascontiguousarray(tokens, np.int32).reshape(-1)
        lg = np.empty(self.vocab if last_only else (ids.size, self.vocab), np.float32)
        hd = self._hidden(hidden)
        self._ok(self._L.needle2_engine_prefill(self.h, ids.ctypes.data, ids.size, int(bool(last_only)),
                                                lg.ctypes.data, _ffi.addr(hd)))
        self.position += int(ids.size)
        return lg, hd

    def decode(self, first_token: int, max_new_tokens: int, grammar: DFAStateDesc | None = None) -> list[int]:
        """Greedy decoding in the library from ``first_token`` (included) until eos / stop, ``max_new_tokens``
        or a terminal grammar state."""
        n = max(int(max_new_tokens), 0)
        out = (ct.c_int * (n + 1))()
        count = ct.c_int(0)
        self._ok(self._L.needle2_engine_decode_loop(self.h, int(first_token), n,
                                                    ct.byref(grammar) if grammar is not None else None, out,
                                                    ct.byref(count)))
        self.position += max(count.value - 1, 0)
        return list(out[:count.value])

    # ---- lifetime ------------------------------------------------------------------------------------------
    def close(self) -> None:
        h, self.h = getattr(self, "h", None), None
        if h:
            self._L.needle2_engine_destroy(h)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GpuEngine(EngineBinding):
    """The GPU engine over ``archive``: ``kv_cache`` "fp32" or "int8", ``matmul`` "fp32" or "int8" (the SDOT
    arithmetic for the 2/4-bit matrices of groups 64..131072), ``activation_bits`` 0 or 8."""

    def __init__(self, archive, *, kv_cache: str = "fp32", matmul: str = "fp32", activation_bits: int = 0):
        from .cq import CQMatrix
        if kv_cache not in ("fp32", "int8") or matmul not in ("fp32", "int8"):
            raise ValueError("kv_cache and matmul are 'fp32' or 'int8'")
        super().__init__(_ffi.lib(), archive, CQMatrix.from_record, activation_bits)
        if matmul == "int8":
            self.set_sdot()
        if kv_cache == "int8":
            self.set_int8_kv(True)
