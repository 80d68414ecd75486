"""Seeded test inputs shared by the CPU and GPU suites.

``example`` builds the same kind of matrix the reference's own kernel test
uses (tests/test_native.py:9-29 in the reference): uniform random codes, a
linear codebook ``linspace(-2, 2)/sqrt(group)``, fp16 norms U[0.1, 2] with one
all-zero row, and an fp64 dense closed form ``(cb[idx] * norm) @ H``.
``baseline`` builds the synthetic benchmark matrices (integer codebook
``j - 2**(bits-1)``, fp16 norms U[0.005, 0.05], x ~ N(0, 1)).
"""
from __future__ import annotations

import numpy as np

from openneedle_amd import formats


def example(bits, rows=9, dim=257, group=128, seed=None):
    rng = np.random.default_rng(104 + bits if seed is None else seed)
    padded = formats.padded_width(dim, group)
    n = 3 if bits == 5 else 1 << bits
    cb = np.linspace(-2, 2, n, dtype=np.float32) / np.sqrt(np.float32(group))
    indices = rng.integers(0, n, (rows, padded), dtype=np.uint8)
    packed = formats.pack_ternary(indices) if bits == 5 else formats.pack_indices(indices, bits)
    norms = rng.uniform(0.1, 2, (rows, padded // group)).astype(np.float16)
    norms[0] = 0  # exact zero groups and rows
    dense = (cb.astype(np.float64)[indices].reshape(rows, -1, group) * norms.astype(np.float64)[..., None])
    dense = (dense @ formats.hadamard_matrix(group)).reshape(rows, padded)[:, :dim]
    return packed, norms, cb, dense


def baseline(bits, rows, dim, group=32, seed=20261201):
    rng = np.random.default_rng(seed)
    packed, norms, cb, idx = formats.synthetic_cq(rng, rows, dim, bits, group)
    return packed, norms, cb, idx


def activations(shape, seed=9):
    return np.random.default_rng(seed).normal(size=shape).astype(np.float32)


def permute_like_reference(q, bits, group):
    """Natural-order int8 activations -> the reference's stored order (sdot.cpp:98-100)."""
    q = np.asarray(q)
    out = np.empty_like(q)
    width = 4 if bits == 2 else 2
    chunk = width * 16
    for g0 in range(0, q.size, group):
        i = np.arange(group)
        dst = (i // chunk) * chunk + (i % width) * 16 + (i % chunk) // width
        out[g0 + dst] = q[g0 + i]
    return out


# ---------------------------------------------------------------------------
# .cact archives
# ---------------------------------------------------------------------------
def tiny_archive_bytes():
    """The one-layer, one-engram archive that the reference's archive-validation tests build by hand
    (tests/test_archive_validation.py:10-30 of the reference): CQ2 g8 embedding of 64 zero bytes, every other
    tensor FP32 zeros, linspace(-1, 1, 28) codebook."""
    from openneedle_amd import archive as A
    layer = [(8,), (8, 8), (4, 8), (4, 8), (4,), (4,), (8, 8), (8, 8), (8,), (1,), (8,), (8,), (8,), (8,)]
    mhc = [(1,), (1,), (1,), (1, 2), (1, 2), (1, 2, 2), (2, 16), (2, 16), (4, 16)]
    shapes = [(16, 8)] + layer + mhc + [(8, 4), (8, 8), (8, 8), (4, 8), (8,)]
    header = (A.TAG, len(shapes), 28, 5, 8, 16, 8, 2, 1, 1, 4, 64, 8, 2, 4, 4, 2, 4, 3, 2, 2, 3, 0, 0, 1, 0, 0, 0, 0,
              100000.0)
    records = [(A.CQ, shapes[0], bytes(64), 8, 2)]
    records += [(A.FP32, s, np.zeros(s, "<f4").tobytes(), 0, 0) for s in shapes[1:]]
    return A.pack_archive(header, np.linspace(-1, 1, 28, dtype="<f4"), records)


def official_like_archive(seed=0, tokenizer_bytes=115215):
    from openneedle_amd.archive import synthetic_released
    return synthetic_released(seed, tokenizer_bytes)
