"""``NativeEngine`` on the GPU: the reference's whole-token decode API over the gfx950 library.

Mirrors needle2/native.py:307-663 (constructor checks, descriptors, step / step_candidates / prefill / reset /
set_int8_kv / kv_storage_bytes and their messages). The engine behind ``needle2_engine_*`` runs one sequence
per instance on the GPU: CQ matrices are the archive's :class:`~openneedle_amd.native.NativeCQ` handles (the
mHC matrices are dequantized to fp32, as the reference passes them), the other tensors fp32 copies.
"""
from __future__ import annotations

import ctypes as ct
from pathlib import Path

import numpy as np

from .archive import CQ, FP16, FP32, LAYER_NAMES, MHC_NAMES, Archive, canonical_shapes
from .native import NativeCQ, _library


class _TensorDesc(ct.Structure):
    """needle2/csrc/engine.cpp:14."""
    _fields_ = [("cq", ct.c_void_p), ("data", ct.c_void_p), ("rows", ct.c_int), ("cols", ct.c_int)]


class _EngineConfig(ct.Structure):
    """needle2/csrc/engine.cpp:15-19."""
    _fields_ = [(n, ct.c_int) for n in ("vocab", "dim", "heads", "kvheads", "layers", "head_dim", "max_seq", "hada",
                                        "lanes", "window", "slots", "subdim", "tables", "taps", "dilation",
                                        "num_orders")] + \
               [("orders", ct.c_int * 4), ("num_sites", ct.c_int), ("sites", ct.c_int * 4), ("rope_theta", ct.c_float)]


def engine_config(m: dict) -> _EngineConfig:
    """The engine configuration of archive metadata (needle2/native.py:373-380)."""
    c = _EngineConfig()
    mapping = dict(vocab="vocab_size", dim="d_model", heads="num_heads", kvheads="num_kv_heads", layers="num_layers",
                   head_dim="head_dim", max_seq="max_seq_len", hada="hada_n", lanes="mhc_lanes", window="kv_window",
                   slots="engram_slots", subdim="engram_sub_dim", tables="num_engram_tables",
                   taps="engram_conv_taps", dilation="engram_conv_dilation")
    for field, key in mapping.items():
        setattr(c, field, int(m[key]))
    c.num_orders, c.num_sites = len(m["engram_orders"]), len(m["engram_layers"])
    c.orders = (ct.c_int * 4)(*m["engram_orders"])
    c.sites = (ct.c_int * 4)(*m["engram_layers"])
    c.rope_theta = m["rope_theta"]
    return c


def engine_tensors(archive: Archive):
    """Names in engine order (needle2/native.py:351-364): the architecture tensors without probe heads."""
    m = archive.metadata
    names = list(canonical_shapes(m))
    for name in names:
        rec = archive.tensors.get(name)
        if rec is None:
            raise ValueError(f"{name}: missing")
        if rec.dtype not in (FP16, FP32, CQ):
            raise ValueError(f"{name}: expected a numeric tensor")
        is_matrix = name == "embedding" or name.startswith("mhc_phi") or name.endswith(("_proj", ".tables"))
        if rec.dtype == CQ and not is_matrix:
            raise ValueError(f"{name}: CQ is only supported for matrix tensors")
    return names


class _DFAStateDesc(ct.Structure):
    """needle2/native.py:291-305: a compiled grammar as needle2_engine_decode_loop reads it."""
    _fields_ = [("num_states", ct.c_int), ("initial_state", ct.c_int), ("eos_id", ct.c_int), ("stop_id", ct.c_int),
                ("tool_start_id", ct.c_int), ("tool_end_id", ct.c_int), ("state_types", ct.POINTER(ct.c_int)),
                ("fallback_next_states", ct.POINTER(ct.c_int)), ("candidate_offsets", ct.POINTER(ct.c_int)),
                ("candidate_tokens", ct.POINTER(ct.c_int)), ("next_states", ct.POINTER(ct.c_int))]


class NativeEngine:
    """Entire token forward on the GPU; one independent unpadded sequence per instance (needle2/native.py:307)."""

    def __init__(self, archive, threads: int = 1, activation_bits: int = 0, projection_lookup: int = -1,
                 matmul: str = "fp32", kv_cache: str = "fp32"):
        if isinstance(archive, (str, Path)):
            archive = Archive.load(archive)
        if not 1 <= int(threads) <= 256:
            raise ValueError("threads must be between 1 and 256")
        if kv_cache not in ("fp32", "int8"):
            raise ValueError("kv_cache must be 'fp32' or 'int8'")
        if matmul not in ("fp32", "sdot"):
            raise ValueError("matmul must be fp32 or sdot")
        if matmul == "sdot" and activation_bits:
            raise ValueError("SDOT already rounds rotated activations; use activation_bits=0")
        if projection_lookup not in (-1, 0, 1, 2, 3, 4):
            raise ValueError("projection_lookup must be -1 (auto), 0, 1, 2, 3, or 4")
        if activation_bits not in (0, 8):
            raise ValueError("activation_bits must be 0 (FP32) or 8")
        m = self.metadata = archive.metadata.copy()
        if m["kv_bits"] != 8:
            raise NotImplementedError("NativeEngine currently supports KV8 archives with FP32 reference KV arithmetic")
        if m["head_dim"] % 2 or m["hada_n"] < m["d_model"] or m["hada_n"] & (m["hada_n"] - 1):
            raise ValueError("invalid native head/Hadamard geometry")
        if m["engram_layers"] and (not m["engram_orders"] or m["num_engram_tables"] % len(m["engram_orders"]) or
                                   m["num_engram_tables"] * m["engram_sub_dim"] != m["d_model"]):
            raise ValueError("inconsistent engram geometry")
        self._archive = archive
        self.kv_cache, self.matmul = kv_cache, matmul
        self.prefix_len = 0
        self._owners = []
        descriptors = []
        for name in engine_tensors(archive):
            rec = archive.tensors[name]
            if rec.dtype == CQ and not name.startswith("mhc_"):
                q = NativeCQ.from_record(rec)
                self._owners.append(q)
                descriptors.append(_TensorDesc(q._handle, None, *rec.shape))
            else:
                a = np.ascontiguousarray(rec.dequantize(), dtype=np.float32)
                self._owners.append(a)
                rows, cols = (a.shape[0], int(np.prod(a.shape[1:]))) if a.ndim > 1 else (1, a.size)
                descriptors.append(_TensorDesc(None, a.ctypes.data, rows, cols))
        self._config = engine_config(m)
        self._descriptors = (_TensorDesc * len(descriptors))(*descriptors)
        lib = self._lib = _library()
        for name, args, res in (
                ("needle2_engine_create", [ct.POINTER(_EngineConfig), ct.POINTER(_TensorDesc), ct.c_int, ct.c_int,
                                           ct.c_int], ct.c_void_p),
                ("needle2_engine_destroy", [ct.c_void_p], None),
                ("needle2_engine_reset", [ct.c_void_p, ct.c_int], None),
                ("needle2_engine_step", [ct.c_void_p, ct.c_int, ct.c_void_p, ct.c_void_p], ct.c_int),
                ("needle2_engine_step_candidates", [ct.c_void_p, ct.c_int, ct.c_void_p, ct.c_int, ct.c_void_p,
                                                    ct.c_void_p], ct.c_int),
                ("needle2_engine_prefill", [ct.c_void_p, ct.c_void_p, ct.c_int, ct.c_int, ct.c_void_p, ct.c_void_p],
                 ct.c_int),
                ("needle2_engine_project_candidates", [ct.c_void_p, ct.c_void_p, ct.c_int, ct.c_void_p], ct.c_int),
                ("needle2_engine_set_int8_kv", [ct.c_void_p, ct.c_int], ct.c_int),
                ("needle2_engine_cache_prefix", [ct.c_void_p], ct.c_int),
                ("needle2_engine_decode_loop", [ct.c_void_p, ct.c_int, ct.c_int, ct.POINTER(_DFAStateDesc),
                                                ct.POINTER(ct.c_int), ct.POINTER(ct.c_int)], ct.c_int),
                ("needle2_engine_import", [ct.c_void_p, ct.c_int, ct.c_int, ct.c_void_p, ct.c_void_p, ct.c_int,
                                           ct.c_void_p, ct.c_void_p], ct.c_int),
                ("needle2_engine_reset_to_prefix", [ct.c_void_p], ct.c_int),
                ("needle2_engine_set_sdot", [ct.c_void_p], ct.c_int),
                ("needle2_engine_set_lookup", [ct.c_void_p, ct.c_int], None),
                ("needle2_engine_kv_storage_bytes", [ct.c_void_p], ct.c_size_t),
                ("needle2_engine_error", [], ct.c_char_p)):
            f = getattr(lib, name)
            f.argtypes, f.restype = args, res
        self._handle = lib.needle2_engine_create(ct.byref(self._config), self._descriptors, len(descriptors),
                                                 int(threads), int(activation_bits))
        if not self._handle:
            raise RuntimeError(lib.needle2_engine_error().decode())
        lib.needle2_engine_set_lookup(self._handle, int(projection_lookup))
        if matmul == "sdot" and lib.needle2_engine_set_sdot(self._handle):
            raise RuntimeError(lib.needle2_engine_error().decode())
        if kv_cache == "int8":
            self.set_int8_kv(True)
        self.position = 0

    def set_int8_kv(self, enabled: bool = True):
        """Select the KV format and reset the sequence, retaining prefix geometry."""
        if self._lib.needle2_engine_set_int8_kv(self._handle, int(bool(enabled))):
            raise RuntimeError(self._lib.needle2_engine_error().decode())
        self.kv_cache = "int8" if enabled else "fp32"
        self.position = 0

    @property
    def kv_storage_bytes(self):
        """Allocated KV array bytes (device memory)."""
        return self._lib.needle2_engine_kv_storage_bytes(self._handle)

    def __del__(self):
        if getattr(self, "_handle", None):
            self._lib.needle2_engine_destroy(self._handle)
            self._handle = None

    def reset(self, prefix_len: int = 0):
        if not 0 <= prefix_len <= self.metadata["max_seq_len"]:
            raise ValueError("prefix_len must lie between 0 and max_seq_len")
        self._lib.needle2_engine_reset(self._handle, int(prefix_len))
        self.position = 0
        self.prefix_len = int(prefix_len)

    def cache_prefix(self):
        """Snapshot the complete pinned prefix (needle2/native.py:447-459): its KV slots, the token history
        and the engram ring, kept in device memory. Requires ``position == prefix_len > 0``; ``reset()``
        discards the snapshot."""
        if self.position <= 0 or self.position != self.prefix_len:
            raise ValueError("prefix snapshot requires position == prefix_len > 0")
        if self._lib.needle2_engine_cache_prefix(self._handle):
            raise RuntimeError(self._lib.needle2_engine_error().decode())

    def reset_to_prefix(self):
        """Restore the snapshot without a forward pass (needle2/native.py:461-470)."""
        position = self._lib.needle2_engine_reset_to_prefix(self._handle)
        if position < 0:
            raise RuntimeError(self._lib.needle2_engine_error().decode())
        self.position = self.prefix_len = position

    def step(self, token_id: int, *, return_hidden: bool = False, compute_logits: bool = True, candidates=None):
        if candidates is not None:
            return self.step_candidates(token_id, candidates, return_hidden=return_hidden)
        if not isinstance(token_id, (int, np.integer)) or not 0 <= token_id < self.metadata["vocab_size"]:
            raise ValueError("token_id must be an integer within the vocabulary")
        logits = np.empty(self.metadata["vocab_size"], dtype=np.float32) if compute_logits else None
        hidden = np.empty((self.metadata["num_layers"], self.metadata["d_model"]),
                          dtype=np.float32) if return_hidden else None
        status = self._lib.needle2_engine_step(self._handle, int(token_id),
                                               logits.ctypes.data if logits is not None else None,
                                               hidden.ctypes.data if hidden is not None else None)
        if status:
            raise RuntimeError(self._lib.needle2_engine_error().decode())
        self.position += 1
        return (logits, hidden) if return_hidden else logits

    def step_candidates(self, token_id: int, candidates, *, return_hidden: bool = False):
        """Project candidate logits; a singleton skips projection and returns [0]."""
        if not isinstance(token_id, (int, np.integer)) or not 0 <= token_id < self.metadata["vocab_size"]:
            raise ValueError("token_id must be an integer within the vocabulary")
        cands = np.asarray(candidates)
        if cands.ndim != 1 or not cands.size or cands.dtype.kind not in "iu":
            raise ValueError("candidates must be a nonempty 1D integer array")
        if np.any((cands < 0) | (cands >= self.metadata["vocab_size"])):
            raise ValueError("candidate outside vocabulary")
        cands = np.ascontiguousarray(cands, dtype=np.int32)
        if len(cands) == 1:
            result = self.step(token_id, compute_logits=False, return_hidden=return_hidden)
            hidden = result[1] if return_hidden else None
            logits = np.array([0.0], dtype=np.float32)
            return (logits, hidden) if return_hidden else logits
        logits = np.empty(len(cands), dtype=np.float32)
        hidden = np.empty((self.metadata["num_layers"], self.metadata["d_model"]),
                          dtype=np.float32) if return_hidden else None
        status = self._lib.needle2_engine_step_candidates(self._handle, int(token_id), cands.ctypes.data, len(cands),
                                                          logits.ctypes.data,
                                                          hidden.ctypes.data if hidden is not None else None)
        if status:
            raise RuntimeError(self._lib.needle2_engine_error().decode())
        self.position += 1
        return (logits, hidden) if return_hidden else logits

    def prefill(self, token_ids, *, last_only: bool = False, backend: str = "native"):
        """Append tokens; ``last_only`` skips unnecessary vocabulary projections."""
        ids = np.asarray(token_ids)
        if ids.ndim != 1 or ids.size == 0 or ids.dtype.kind not in "iu":
            raise ValueError("prefill requires a nonempty one-dimensional integer token sequence")
        if np.any((ids < 0) | (ids >= self.metadata["vocab_size"])):
            raise ValueError("token outside vocabulary")
        if backend != "native":
            raise ValueError("prefill backend must be 'native' on the GPU engine")
        ids_c = np.ascontiguousarray(ids, dtype=np.int32)
        vocab = int(self.metadata["vocab_size"])
        logits = np.empty(vocab if last_only else (ids.size, vocab), dtype=np.float32)
        if self._lib.needle2_engine_prefill(self._handle, ids_c.ctypes.data, int(ids.size), int(bool(last_only)),
                                            logits.ctypes.data, None):
            raise RuntimeError(self._lib.needle2_engine_error().decode())
        self.position += int(ids.size)
        return logits

    def decode(self, first_token: int, max_new_tokens: int = 128, grammar_dfa=None) -> list[int]:
        """Greedy decoding in the library until eos, max_new_tokens or a terminal grammar state
        (needle2/native.py:622-663); ``grammar_dfa`` is an object with a ``_desc`` (_DFAStateDesc) and a
        ``validate(vocab_size)`` method, as the reference's NativeGrammarDFA."""
        if not isinstance(max_new_tokens, (int, np.integer)) or not 0 <= max_new_tokens <= np.iinfo(np.int32).max:
            raise ValueError("max_new_tokens must be a nonnegative int32")
        if not isinstance(first_token, (int, np.integer)) or not 0 <= first_token < self.metadata["vocab_size"]:
            raise ValueError("first_token outside vocabulary")
        if grammar_dfa is not None:
            grammar_dfa.validate(self.metadata["vocab_size"])
        if max_new_tokens == 0:
            return []
        if not self.metadata["kv_window"]:
            max_new_tokens = min(max_new_tokens, self.metadata["max_seq_len"] - self.position + 1)
        output = (ct.c_int * (max_new_tokens + 1))()
        count = ct.c_int(0)
        desc = ct.byref(grammar_dfa._desc) if grammar_dfa is not None else None
        if self._lib.needle2_engine_decode_loop(self._handle, int(first_token), int(max_new_tokens), desc, output,
                                                ct.byref(count)):
            raise RuntimeError(self._lib.needle2_engine_error().decode())
        self.position += count.value - 1
        return [output[i] for i in range(count.value)]

    def import_state(self, token_ids, positions, keys, values):
        """needle2_engine_import (engine.cpp:784-815): the state after ``token_ids`` with the KV rows of
        ``positions`` (keys / values [layers][len(positions)][kv_heads][head_dim] fp32), as the reference's
        torch prefill hands it over (needle2/native.py:558-590)."""
        ids = np.ascontiguousarray(token_ids, np.int32)
        pos = np.ascontiguousarray(positions, np.int32)
        k = np.ascontiguousarray(keys, np.float32)
        v = np.ascontiguousarray(values, np.float32)
        m = self.metadata
        shape = (m["num_layers"], pos.size, m["num_kv_heads"], m["head_dim"])
        if k.shape != shape or v.shape != shape:
            raise ValueError(f"keys and values must have shape {shape}")
        if self._lib.needle2_engine_import(self._handle, ids.size, self.prefix_len, ids.ctypes.data, pos.ctypes.data,
                                           pos.size, k.ctypes.data, v.ctypes.data):
            raise RuntimeError(self._lib.needle2_engine_error().decode())
        self.position = int(ids.size)

    def generate(self, token_ids, max_new_tokens: int = 32, eos_token_id: int | None = None, prefix_len: int = 0):
        """Greedy continuation of a prompt (needle2/native.py:596-616, native prefill)."""
        self.reset(prefix_len)
        logits = self.prefill(token_ids, last_only=True)
        out = []
        for _ in range(int(max_new_tokens)):
            token = int(np.argmax(logits))
            out.append(token)
            if eos_token_id is not None and token == eos_token_id:
                break
            logits = self.step(token)
        return out
