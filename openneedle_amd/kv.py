"""Device int8 KV cache for a batch of sequences, and batched decode attention.

The arithmetic is the reference Engine's int8 cache: quantize and store
(needle2/csrc/engine.cpp:1005-1021), decode attention (engine.cpp:898-967).
The reference keeps that cache inside a single-sequence Engine; here one
cache holds ``seqs`` sequences so one launch serves a whole decode batch.
Host arrays of :meth:`KVCache.load` / :meth:`KVCache.read` use the
reference's layout, ``[slots][kvheads][head_dim]`` int8 and
``[slots][kvheads]`` fp32 scales.
"""
from __future__ import annotations

import numpy as np

from . import _ffi
from ._ffi import GpuError, addr, check
from .device import stream_ptr


class KVCache:
    def __init__(self, layers: int, capacity: int, kvheads: int, head_dim: int, seqs: int = 1):
        self._lib = _ffi.lib()
        self.layers, self.capacity, self.kvheads, self.head_dim, self.seqs = layers, capacity, kvheads, head_dim, seqs
        self.ptr = self._lib.needle2_gpu_kv_create(layers, capacity, kvheads, head_dim, seqs)
        if not self.ptr:
            raise GpuError(f"KV cache: {_ffi.last_error()}")

    def storage_bytes(self) -> int:
        return int(self._lib.needle2_gpu_kv_storage_bytes(self.ptr))

    def store(self, layer: int, d_k, d_v, count: int, first_slot=0, stream=None) -> None:
        """Quantize ``count`` tokens per sequence from device fp32 ``[seqs][count][kvheads][head_dim]``.
        ``first_slot``: one slot for every sequence, or one per sequence."""
        per_seq = None
        first = 0
        if np.ndim(first_slot):
            per_seq = np.ascontiguousarray(first_slot, np.int32)
            if per_seq.shape != (self.seqs,):
                raise ValueError(f"first_slot: one slot per sequence ({self.seqs})")
        else:
            first = int(first_slot)
        check(self._lib.needle2_gpu_kv_store(self.ptr, layer, addr(d_k), addr(d_v), int(count), first,
                                             addr(per_seq), stream_ptr(stream)), "KV store")

    def store_device(self, layer: int, d_k, d_v, count: int, d_first_slot, stream=None) -> None:
        """:meth:`store` with the per-sequence first slots in device memory (int32 ``[seqs]``); capturable."""
        check(self._lib.needle2_gpu_kv_store_device(self.ptr, layer, addr(d_k), addr(d_v), int(count),
                                                    addr(d_first_slot), stream_ptr(stream)), "KV store")

    def attention(self, layer: int, d_q, d_out, heads: int, length: int, d_slots=None, d_lengths=None,
                  splits: int = 0, stream=None, next=None, new=None) -> None:
        """One decode step for every sequence: device q / out fp32 ``[seqs][heads][head_dim]``. ``new``: (device
        k, device v, device slots) of one new token per sequence, stored first (as :meth:`store_device` with
        count 1). ``next``: a one-matrix int8 :class:`~openneedle_amd.cq.Plan` reading ``d_out`` whose input is
        left prepared for its run with ``prepared=True``."""
        if next is None and new is None:
            check(self._lib.needle2_gpu_attention(self.ptr, layer, addr(d_q), addr(d_out), int(heads), int(length),
                                                  addr(d_slots), addr(d_lengths), int(splits), stream_ptr(stream)),
                  "attention")
        else:
            nk, nv, ns = new if new is not None else (None, None, None)
            check(self._lib.needle2_gpu_attention_chained(self.ptr, layer, addr(d_q), addr(d_out), int(heads),
                                                          int(length), addr(d_slots), addr(d_lengths), int(splits),
                                                          addr(nk), addr(nv), addr(ns),
                                                          next.ptr if next is not None else None,
                                                          stream_ptr(stream)), "attention")

    def load(self, layer: int, seq: int, k, v, ks, vs, first_slot: int = 0) -> None:
        """Copy host int8 rows and fp32 scales (reference layout) into one sequence of the cache."""
        k, v = (np.ascontiguousarray(a, np.int8) for a in (k, v))
        ks, vs = (np.ascontiguousarray(a, np.float32) for a in (ks, vs))
        n = k.shape[0]
        if k.shape != (n, self.kvheads, self.head_dim) or v.shape != k.shape or ks.shape != (n, self.kvheads) \
                or vs.shape != ks.shape:
            raise ValueError("KV load: rows [n][kvheads][head_dim] and scales [n][kvheads]")
        check(self._lib.needle2_gpu_kv_import(self.ptr, layer, seq, k.ctypes.data, v.ctypes.data, ks.ctypes.data,
                                              vs.ctypes.data, int(first_slot), n), "KV import")

    def read(self, layer: int, seq: int, count: int, first_slot: int = 0):
        """(k int8, v int8, k_scales, v_scales) of ``count`` slots of one sequence, reference layout."""
        k = np.empty((count, self.kvheads, self.head_dim), np.int8)
        v = np.empty_like(k)
        ks = np.empty((count, self.kvheads), np.float32)
        vs = np.empty_like(ks)
        check(self._lib.needle2_gpu_kv_export(self.ptr, layer, seq, k.ctypes.data, v.ctypes.data, ks.ctypes.data,
                                              vs.ctypes.data, int(first_slot), count), "KV export")
        return k, v, ks, vs

    def close(self) -> None:
        ptr, self.ptr = getattr(self, "ptr", None), None
        if ptr:
            self._lib.needle2_gpu_kv_destroy(ptr)

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
