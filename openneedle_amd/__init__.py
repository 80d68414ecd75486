"""gfx950 (MI355X) implementation of OpenNeedle's quantized-matmul hot path.

``openneedle_amd.native`` mirrors the reference's ctypes loader
(``needle2/native.py``) over ``libneedle2_native.so``: CQ2/CQ3/CQ4/ternary FP32
GEMV, the bit-exact int8 ("SDOT") GEMV, row dequantization, plus device-resident
entry points, int8-KV decode attention and the prefill GEMM.
"""
from . import formats  # noqa: F401

__all__ = ["formats", "native"]
