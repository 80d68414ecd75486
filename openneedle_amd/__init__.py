"""gfx950 (MI355X) implementation of OpenNeedle's quantized-matmul hot path.

The product is ``libneedle2_native.so`` (``csrc/``): the reference's C ABI
(``needle2_cq_*``, ``needle2_sdot_*``, ``needle2_engine_*``) plus additive
device-resident exports (``needle2_gpu_*``). The Python modules are this
repository's own interface to it:

- ``_ffi``    locating, loading and typing the library;
- ``device``  device memory, streams, events, HIP graphs, ordered teardown;
- ``cq``      CQ matrices (FP32 and int8 products, rows, candidates, the
              prefill GEMM) and multi-matrix plans;
- ``kv``      the int8 KV cache of a decode batch and its attention;
- ``engine``  the single-sequence decode engine;
- ``archive`` / ``formats``  the ``.cact`` file and the CQ storage format.
"""

__all__ = ["archive", "cq", "device", "engine", "formats", "kv"]
