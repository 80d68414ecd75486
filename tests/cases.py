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
