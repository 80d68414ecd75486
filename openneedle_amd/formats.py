"""CQ storage format helpers (host side).

The layout is the one the reference's loader and kernels read
(needle2/quantize.py:54-76, needle2/archive.py:98-106): per matrix row, codes
are an LSB-first little-endian bitstream (``bits`` bits per code, 8 codes per
``bits`` bytes), rows are padded to a whole number of groups, and every group
has one IEEE fp16 L2 norm. Codebooks are sorted fp32 centroids.
"""
from __future__ import annotations

import math

import numpy as np

# Shared 28-entry header codebook of the released model (unit sphere, g=128):
# CQ2 = entries 0..3, CQ3 = 4..11, CQ4 = 12..27 (needle2/quantize.py:12-27).
# These are data constants of the format and must match exactly.
_HEADER_CODEBOOK = np.array([
    -.1331721395254135, -.03990209102630615, .04003528133034706, .13346044719219208,
    -.18926136195659637, -.11788499355316162, -.06614968925714493, -.02101346105337143,
    .022101031616330147, .06678506731987, .11826207488775253, .18982602655887604,
    -.23953154683113098, -.18070605397224426, -.14095793664455414, -.10901255160570145,
    -.08151296526193619, -.056527651846408844, -.03293915092945099, -.010116109624505043,
    .012710800394415855, .03570791706442833, .059458255767822266, .08497702330350876,
    .112741619348526, .1446969211101532, .184239000082016, .2422737032175064,
], dtype=np.float32)
_SLICE = {2: 0, 3: 4, 4: 12}


def check_group(group: int) -> None:
    if group < 8 or group & (group - 1):
        raise ValueError("group_size must be a power of two >= 8")


def codebook(bits: int, group_size: int = 128) -> np.ndarray:
    """Lloyd-Max codebook for ``bits`` scaled to the group size (x sqrt(128/g))."""
    if bits not in _SLICE:
        raise ValueError("CQ supports 2, 3, or 4 bits")
    check_group(group_size)
    start = _SLICE[bits]
    return _HEADER_CODEBOOK[start:start + (1 << bits)].copy() * np.float32(math.sqrt(128 / group_size))


def linear_codebook(bits: int) -> np.ndarray:
    """Integer codebook j - 2**(bits-1): code j stands for the value j-8 (CQ4) or j-2 (CQ2)."""
    n = 1 << bits
    return (np.arange(n, dtype=np.float32) - np.float32(n // 2)).astype(np.float32)


def padded_width(width: int, group: int) -> int:
    return (width + group - 1) // group * group


def pack_indices(indices, bits: int) -> np.ndarray:
    """[rows, n] codes (n a multiple of 8) -> [rows, n*bits/8] bytes, LSB-first."""
    idx = np.asarray(indices)
    if bits not in (2, 3, 4) or idx.ndim != 2 or idx.shape[1] % 8:
        raise ValueError("indices must be [rows, multiple of 8], bits in 2/3/4")
    if np.any(idx < 0) or np.any(idx >= 1 << bits):
        raise ValueError("index outside codebook")
    rows, n = idx.shape
    # bit b of code i lands at stream bit i*bits + b
    planes = ((idx.astype(np.uint8)[..., None] >> np.arange(bits, dtype=np.uint8)) & 1).astype(np.uint8)
    return np.packbits(planes.reshape(rows, n * bits), axis=1, bitorder="little")


def unpack_indices(packed, bits: int, n: int) -> np.ndarray:
    """Inverse of :func:`pack_indices` for ``n`` codes per row."""
    p = np.asarray(packed, dtype=np.uint8)
    if bits not in (2, 3, 4) or n % 8 or p.ndim != 2 or p.shape[1] != n * bits // 8:
        raise ValueError("packed byte count does not match geometry")
    stream = np.unpackbits(p, axis=1, bitorder="little").reshape(p.shape[0], n, bits)
    return (stream.astype(np.uint8) << np.arange(bits, dtype=np.uint8)).sum(-1).astype(np.uint8)


def pack_ternary(values) -> np.ndarray:
    """Ternary codebook indices {0,1,2} -> 2-bit crumbs (0->3, 1->0, 2->1), LSB-first."""
    v = np.asarray(values)
    crumbs = np.where(v == 0, 3, v - 1).astype(np.uint8)
    return pack_indices(crumbs, 2)


def hadamard_matrix(n: int) -> np.ndarray:
    """Dense normalized Sylvester-Hadamard matrix (float64)."""
    check_group(n)
    h = np.ones((1, 1))
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h / math.sqrt(n)


def dequantize_dense(packed, norms, shape, bits: int, group: int, cb) -> np.ndarray:
    """fp64 dense weights W[out, in] = (cb[idx] * norm) @ H per group (closed form)."""
    out, width = shape
    padded = padded_width(width, group)
    cb = np.asarray(cb, dtype=np.float64)
    if bits == 5:
        crumbs = unpack_indices(packed, 2, padded)
        lut = np.array([cb[1], cb[2], 0.0, cb[0]])
        vals = lut[crumbs]
    else:
        vals = cb[unpack_indices(packed, bits, padded)]
    vals = vals.reshape(out, -1, group) * np.asarray(norms, dtype=np.float64).reshape(out, -1, 1)
    return (vals @ hadamard_matrix(group)).reshape(out, padded)[:, :width]


def synthetic_cq(rng: np.random.Generator, out: int, width: int, bits: int, group: int,
                 norm_range=(0.005, 0.05), cb=None):
    """Uniform codes, fp16 norms U[norm_range] and (by default) the linear codebook."""
    padded = padded_width(width, group)
    idx = rng.integers(0, 1 << bits, size=(out, padded), dtype=np.uint8)
    packed = pack_indices(idx, bits)
    norms = rng.uniform(norm_range[0], norm_range[1], size=(out, padded // group)).astype(np.float16)
    cb = linear_codebook(bits) if cb is None else np.asarray(cb, np.float32)
    return packed, norms, cb, idx
