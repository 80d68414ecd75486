"""ctypes access to the checker libraries (TEST INFRASTRUCTURE ONLY).

* ``lib()``  - ``liboracle.so``, the CPU restatement of the reference arithmetic
  in ``needle2_oracle.c`` (each C function cites the reference file:line).
* ``ref()``  - ``_ref/libref.so``, the reference's own ``needle2/csrc/cq.cpp``
  compiled from source with ``ref_harness.cpp``; ``None`` when it was not built.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
use this package, and only as the checker / reported baseline. The product
library (``openneedle_amd``) never imports it.
"""
from __future__ import annotations

import ctypes as ct
import functools
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
_P = ct.c_void_p
_I = ct.c_int


def build() -> None:
    """Compile liboracle.so and, when the reference sources exist, _ref/libref.so."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)


def _ptr(a):
    return a.ctypes.data if a is not None else None


@functools.lru_cache(maxsize=1)
def lib():
    path = HERE / "liboracle.so"
    if not path.exists():
        build()
    L = ct.CDLL(str(path))
    L.nd_half_float.argtypes = [ct.c_uint16]
    L.nd_half_float.restype = ct.c_float
    L.nd_hadamard.argtypes = [_P, _I]
    L.nd_hadamard.restype = None
    L.nd_index_at.argtypes = [_P, _I, _I]
    L.nd_index_at.restype = ct.c_uint
    for name in ("nd_cq_linear", "nd_sdot_linear"):
        f = getattr(L, name)
        f.argtypes = [_P, _P, _I, _I, _I, _I, _P, _P, _P, _I, _I]
        f.restype = _I
    L.nd_cq_rows.argtypes = [_P, _P, _I, _I, _I, _I, _P, _P, _P, _I]
    L.nd_cq_rows.restype = _I
    L.nd_sdot_centroids.argtypes = [_P, _I, _P, _P]
    L.nd_sdot_centroids.restype = None
    L.nd_sdot_prepare.argtypes = [_P, _I, _I, _P, _P]
    L.nd_sdot_prepare.restype = None
    L.nd_sdot_dots.argtypes = [_P, _I, _I, _I, _I, _P, _P, _P]
    L.nd_sdot_dots.restype = None
    L.nd_kv_quantize.argtypes = [_P, _I, _I, _I, _P, _P]
    L.nd_kv_quantize.restype = None
    L.nd_attention_i8.argtypes = [_P, _I, _I, _I, _P, _P, _P, _P, _P, _I, _P]
    L.nd_attention_i8.restype = _I
    return L


@functools.lru_cache(maxsize=1)
def ref():
    path = HERE / "_ref" / "libref.so"
    if not path.exists():
        return None
    L = ct.CDLL(str(path))
    L.needle2_cq_create.argtypes = [_P, _P, _I, _I, _I, _I, _P]
    L.needle2_cq_create.restype = _P
    L.needle2_cq_destroy.argtypes = [_P]
    L.needle2_cq_destroy.restype = None
    L.needle2_cq_linear.argtypes = [_P, _P, _P, _I, _I]
    L.needle2_cq_linear.restype = None
    L.needle2_cq_linear_lookup.argtypes = [_P, _P, _P, _I, _I, _I]
    L.needle2_cq_linear_lookup.restype = None
    L.needle2_cq_rows.argtypes = [_P, _P, _P, _I]
    L.needle2_cq_rows.restype = None
    L.refh_sdot_create.argtypes = [_P, _P, _I, _I, _I, _I, _P]
    L.refh_sdot_create.restype = _P
    L.refh_sdot_destroy.argtypes = [_P]
    L.refh_sdot_linear.argtypes = [_P, _P, _P, _I, _I]
    L.refh_sdot_prepare.argtypes = [_P, _P, _P, _P]
    L.refh_sdot_centroids.argtypes = [_P, _P, _P, _P]
    L.refh_attn_create.argtypes = [_I, _I, _I, _I, _I]
    L.refh_attn_create.restype = _P
    L.refh_attn_destroy.argtypes = [_P]
    L.refh_attn_import.argtypes = [_P, _P, _P, _I]
    L.refh_attn_import.restype = _I
    L.refh_attn_cache.argtypes = [_P, _P, _P, _P, _P, _I]
    L.refh_attn_compute.argtypes = [_P, _I, _P, _P]
    return L


# --------------------------------------------------------------------------
# Oracle calls (C restatement)
# --------------------------------------------------------------------------

def _geometry(in_dim, group):
    padded = (in_dim + group - 1) // group * group
    return padded, padded // group


def cq_linear(packed, norms, shape, bits, group, cb, x, threads=1):
    """FP32 CQ GEMV, reference order (cq.cpp:165-197). x: [..., in]."""
    out, in_dim = shape
    x = np.ascontiguousarray(x, np.float32)
    batch = x.size // in_dim
    y = np.empty(x.shape[:-1] + (out,), np.float32)
    rc = lib().nd_cq_linear(_ptr(np.ascontiguousarray(packed, np.uint8)),
                            _ptr(np.ascontiguousarray(norms).view(np.uint16)),
                            out, in_dim, bits, group, _ptr(np.ascontiguousarray(cb, np.float32)),
                            _ptr(x), _ptr(y), batch, threads)
    assert rc == 0
    return y


def cq_rows(packed, norms, shape, bits, group, cb, ids):
    out, in_dim = shape
    ids = np.ascontiguousarray(ids, np.int64)
    y = np.empty(ids.shape + (in_dim,), np.float32)
    rc = lib().nd_cq_rows(_ptr(np.ascontiguousarray(packed, np.uint8)),
                          _ptr(np.ascontiguousarray(norms).view(np.uint16)),
                          out, in_dim, bits, group, _ptr(np.ascontiguousarray(cb, np.float32)),
                          _ptr(ids), _ptr(y), ids.size)
    assert rc == 0
    return y


def hadamard(v):
    """Normalized FWHT of the last axis, reference stage order (cq.cpp:30-46)."""
    v = np.array(v, np.float32, copy=True, order="C")
    n = v.shape[-1]
    flat = v.reshape(-1, n)
    for row in flat:
        lib().nd_hadamard(_ptr(row), n)
    return flat.reshape(v.shape)


def half_float(h):
    return lib().nd_half_float(int(h))


def sdot_centroids(cb, bits):
    c = np.zeros(16, np.int8)
    cs = np.zeros(1, np.float32)
    lib().nd_sdot_centroids(_ptr(np.ascontiguousarray(cb, np.float32)), bits, _ptr(c), _ptr(cs))
    return c[: 1 << bits].copy(), np.float32(cs[0])


def sdot_prepare(x, group):
    """int8 activations (natural order) and per-group fp32 scales (sdot.cpp:47-81)."""
    x = np.ascontiguousarray(x, np.float32)
    padded, groups = _geometry(x.shape[-1], group)
    q = np.empty(padded, np.int8)
    s = np.empty(groups, np.float32)
    lib().nd_sdot_prepare(_ptr(x), x.shape[-1], group, _ptr(q), _ptr(s))
    return q, s


def sdot_dots(packed, shape, bits, group, centroids, q):
    out, in_dim = shape
    padded, groups = _geometry(in_dim, group)
    c16 = np.zeros(16, np.int8)
    c16[: len(centroids)] = centroids
    d = np.empty((out, groups), np.int32)
    lib().nd_sdot_dots(_ptr(np.ascontiguousarray(packed, np.uint8)), out, in_dim, bits, group,
                       _ptr(c16), _ptr(np.ascontiguousarray(q, np.int8)), _ptr(d))
    return d


def sdot_linear(packed, norms, shape, bits, group, cb, x, threads=1):
    """int8 'SDOT' GEMV, reference arithmetic (sdot.cpp:35-149, 338-359)."""
    out, in_dim = shape
    x = np.ascontiguousarray(x, np.float32)
    batch = x.size // in_dim
    y = np.empty(x.shape[:-1] + (out,), np.float32)
    rc = lib().nd_sdot_linear(_ptr(np.ascontiguousarray(packed, np.uint8)),
                              _ptr(np.ascontiguousarray(norms).view(np.uint16)),
                              out, in_dim, bits, group, _ptr(np.ascontiguousarray(cb, np.float32)),
                              _ptr(x), _ptr(y), batch, threads)
    assert rc == 0
    return y


def kv_quantize(src):
    """src [tokens, kvheads, head_dim] fp32 -> (int8 same shape, fp32 [tokens, kvheads])."""
    src = np.ascontiguousarray(src, np.float32)
    t, kvh, hd = src.shape
    dst = np.empty(src.shape, np.int8)
    sc = np.empty((t, kvh), np.float32)
    lib().nd_kv_quantize(_ptr(src), t, kvh, hd, _ptr(dst), _ptr(sc))
    return dst, sc


def attention_i8(q, keys, values, k_scales, v_scales, slots=None):
    """q [heads, hd]; caches [slots, kvheads, hd] int8; scales [slots, kvheads]."""
    q = np.ascontiguousarray(q, np.float32)
    heads, hd = q.shape
    kvheads = keys.shape[1]
    if slots is None:
        slots = np.arange(keys.shape[0], dtype=np.int32)
    slots = np.ascontiguousarray(slots, np.int32)
    out = np.empty((heads, hd), np.float32)
    rc = lib().nd_attention_i8(_ptr(q), heads, kvheads, hd,
                               _ptr(np.ascontiguousarray(keys, np.int8)),
                               _ptr(np.ascontiguousarray(values, np.int8)),
                               _ptr(np.ascontiguousarray(k_scales, np.float32)),
                               _ptr(np.ascontiguousarray(v_scales, np.float32)),
                               _ptr(slots), len(slots), _ptr(out))
    assert rc == 0
    return out


# --------------------------------------------------------------------------
# Reference (built from source) calls
# --------------------------------------------------------------------------

class RefCQ:
    """The reference's own CQ (needle2_cq_*) and scalar SdotCQ on this host."""

    def __init__(self, packed, norms, shape, bits, group, cb):
        L = ref()
        if L is None:
            raise RuntimeError("oracle/_ref was not built (reference sources absent)")
        self.L = L
        self.shape = tuple(shape)
        self.bits, self.group = bits, group
        self.packed = np.ascontiguousarray(packed, np.uint8)
        self.norms = np.ascontiguousarray(norms).view(np.uint16)
        self.cb = np.ascontiguousarray(cb, np.float32)
        self.h = L.needle2_cq_create(_ptr(self.packed), _ptr(self.norms), shape[0], shape[1],
                                     bits, group, _ptr(self.cb))
        self.s = None

    @property
    def handle(self):
        return self.h

    @classmethod
    def from_record(cls, rec):
        return cls(rec.packed, rec.norms, rec.shape, rec.bits, rec.group_size, rec.cq_codebook())

    def __del__(self):
        if getattr(self, "h", None):
            self.L.needle2_cq_destroy(self.h)
        if getattr(self, "s", None):
            self.L.refh_sdot_destroy(self.s)

    def linear(self, x, threads=1, lookup=0):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(x.shape[:-1] + (self.shape[0],), np.float32)
        batch = x.size // self.shape[1]
        if lookup:
            self.L.needle2_cq_linear_lookup(self.h, _ptr(x), _ptr(y), batch, threads, lookup)
        else:
            self.L.needle2_cq_linear(self.h, _ptr(x), _ptr(y), batch, threads)
        return y

    def rows(self, ids):
        ids = np.ascontiguousarray(ids, np.int64)
        y = np.empty(ids.shape + (self.shape[1],), np.float32)
        self.L.needle2_cq_rows(self.h, _ptr(ids), _ptr(y), ids.size)
        return y

    def _sdot(self):
        if self.s is None:
            self.s = self.L.refh_sdot_create(_ptr(self.packed), _ptr(self.norms), self.shape[0],
                                             self.shape[1], self.bits, self.group, _ptr(self.cb))
        return self.s

    def sdot_linear(self, x, threads=1):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(x.shape[:-1] + (self.shape[0],), np.float32)
        self.L.refh_sdot_linear(self._sdot(), _ptr(x), _ptr(y), x.size // self.shape[1], threads)
        return y

    def sdot_prepare(self, x):
        padded, groups = _geometry(self.shape[1], self.group)
        q = np.empty(padded, np.int8)
        s = np.empty(groups, np.float32)
        self.L.refh_sdot_prepare(self._sdot(), _ptr(np.ascontiguousarray(x, np.float32)), _ptr(q), _ptr(s))
        return q, s

    def sdot_tables(self):
        padded, groups = _geometry(self.shape[1], self.group)
        c = np.zeros(16, np.int8)
        cs = np.zeros(1, np.float32)
        ns = np.empty((self.shape[0], groups), np.float32)
        self.L.refh_sdot_centroids(self._sdot(), _ptr(c), _ptr(cs), _ptr(ns))
        return c[: 1 << self.bits].copy(), np.float32(cs[0]), ns


class RefAttention:
    """The reference Engine's int8 KV quantizer and compute_attention (one layer)."""

    def __init__(self, heads, kvheads, head_dim, max_seq, threads=1):
        L = ref()
        if L is None:
            raise RuntimeError("oracle/_ref was not built (reference sources absent)")
        self.L = L
        self.heads, self.kvheads, self.hd = heads, kvheads, head_dim
        self.h = L.refh_attn_create(heads, kvheads, head_dim, max_seq, threads)
        assert self.h
        self.count = 0

    def __del__(self):
        if getattr(self, "h", None):
            self.L.refh_attn_destroy(self.h)

    def load(self, k, v):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        self.count = k.shape[0]
        assert self.L.refh_attn_import(self.h, _ptr(k), _ptr(v), self.count) == 0

    def cache(self):
        n, kvh, hd = self.count, self.kvheads, self.hd
        k = np.empty((n, kvh, hd), np.int8)
        v = np.empty((n, kvh, hd), np.int8)
        ks = np.empty((n, kvh), np.float32)
        vs = np.empty((n, kvh), np.float32)
        self.L.refh_attn_cache(self.h, _ptr(k), _ptr(v), _ptr(ks), _ptr(vs), n)
        return k, v, ks, vs

    def attend(self, q):
        q = np.ascontiguousarray(q, np.float32)
        out = np.empty((self.heads, self.hd), np.float32)
        self.L.refh_attn_compute(self.h, self.count - 1, _ptr(q), _ptr(out))
        return out


def RefEngine(archive, activation_bits=0, int8_kv=False, threads=1, sdot=False):
    """The reference's own Engine (engine.cpp, built into oracle/_ref) over an archive, driven through the
    same binding as the GPU engine (``openneedle_amd.engine.EngineBinding``): CQ records through the
    reference's CQ handles, everything else (the mHC matrices too) as dequantized fp32."""
    from openneedle_amd.engine import EngineBinding
    L = ref()
    if L is None:
        raise RuntimeError("oracle/_ref was not built (reference sources absent)")
    eng = EngineBinding(L, archive, RefCQ.from_record, activation_bits, threads)
    if sdot:  # the Engine's int8 matmul path (engine.cpp:424-432 without the ARM feature test)
        L.refh_engine_sdot.argtypes, L.refh_engine_sdot.restype = [ct.c_void_p], ct.c_int
        assert L.refh_engine_sdot(eng.h) == 0
    if int8_kv:
        eng.set_int8_kv(True)
    return eng
