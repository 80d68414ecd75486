"""The `.cact` model archive: validated, named, zero-copy access and one-shot device upload.

Mirrors the reference's reader (needle2/archive.py:13-232: the same header,
directory and payload rules, tensor names and error messages) over a
read-only memory map instead of a byte copy: a tensor's ``blob`` is a view
into the file, so ``packed`` / ``norms`` are numpy views and a CQ matrix goes
from the page cache to device memory without a host-side copy.
:class:`DeviceModel` uploads every CQ matrix of an archive once (the
reference builds one ``NativeCQ`` per record in ``NativeEngine``,
needle2/native.py:382-391) and keeps the dense tensors as fp32 device arrays.

File layout (little-endian): a 120-byte header ``<29If`` (tag, tensor count,
codebook length 28, KV window, KV bits, 14 geometry fields, engram order
count + 4 orders, engram site count + 4 sites, RoPE theta); the shared fp32
codebook (CQ2 = entries 0..3, CQ3 = 4..11, CQ4 = 12..27); one 44-byte record
``<BBHIIIIQQII`` per tensor (dtype, ndim, reserved, 4 dims, offset, nbytes,
group, bits); payloads at 64-byte aligned offsets. A CQ payload holds every
row's packed codes, then every row's fp16 group norms.
"""
from __future__ import annotations

import math
import mmap
import struct
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from . import formats

TAG = 0x05E12A83
HEADER = struct.Struct("<29If")
RECORD = struct.Struct("<BBHIIIIQQII")
FP16, FP32, CQ, RAW = 1, 2, 3, 4
ALIGN = 64
LAYER_NAMES = ("norm_in", "q_proj", "k_proj", "v_proj", "q_norm", "k_norm", "gate_proj", "out_proj", "post_norm",
               "attn_gate", "pre_hada", "d1", "d2", "d3")
MHC_NAMES = ("mhc_a_pre", "mhc_a_post", "mhc_a_res", "mhc_b_pre", "mhc_b_post", "mhc_b_res", "mhc_phi_pre",
             "mhc_phi_post", "mhc_phi_res")
ENGRAM_NAMES = ("tables", "key_proj", "value_proj", "taps")
GEOMETRY_FIELDS = ("vocab_size", "d_model", "num_heads", "num_kv_heads", "num_layers", "head_dim", "max_seq_len",
                   "hada_n", "mhc_lanes", "engram_slots", "engram_sub_dim", "num_engram_tables", "engram_conv_taps",
                   "engram_conv_dilation")
CODEBOOK_SLICES = {2: (0, 4), 3: (4, 12), 4: (12, 28)}
HEAD_CODES = {1: ("contrastive_head", 4), 2: ("confidence_head", 8)}
_TERNARY = 1.2240064  # centroid magnitude of the ternary (bits = 5) records, before 1/sqrt(group)


def cq_payload_bytes(rows: int, cols: int, group: int, bits: int) -> int:
    """Packed codes (2 bits per ternary code) plus one fp16 norm per group, per row."""
    padded = math.ceil(cols / group) * group
    return rows * (padded * (2 if bits == 5 else bits) // 8 + padded // group * 2)


def _metadata(h) -> dict:
    m = dict(zip(GEOMETRY_FIELDS, h[5:19]))
    m.update(kv_window=h[3], kv_bits=h[4], engram_orders=list(h[20:20 + h[19]]),
             engram_layers=list(h[25:25 + h[24]]), rope_theta=h[29], act_bits=8)
    return m


def _check_geometry(m: dict) -> None:
    """needle2/archive.py:22-43."""
    required = ("d_model", "num_heads", "num_kv_heads", "num_layers", "head_dim", "mhc_lanes", "vocab_size",
                "max_seq_len", "hada_n")
    if min(m[k] for k in required) <= 0 or m["num_heads"] % m["num_kv_heads"]:
        raise ValueError("invalid model geometry")
    if m["head_dim"] % 2 or m["hada_n"] != 1 << (m["d_model"] - 1).bit_length():
        raise ValueError("invalid RoPE/Hadamard geometry")
    if not (math.isfinite(m["rope_theta"]) and m["rope_theta"] > 0):
        raise ValueError("rope_theta must be finite and positive")
    if m["kv_bits"] not in (2, 3, 4, 8):
        raise ValueError("unsupported KV bit width")
    sites, orders = m["engram_layers"], m["engram_orders"]
    if len(sites) != len(set(sites)) or any(s >= m["num_layers"] for s in sites):
        raise ValueError("invalid engram layer indices")
    if orders and min(orders) < 1:
        raise ValueError("engram orders must be positive")
    engram_sizes = ("engram_slots", "engram_sub_dim", "num_engram_tables", "engram_conv_taps", "engram_conv_dilation")
    if sites and (not orders or m["num_engram_tables"] % len(orders) or min(m[k] for k in engram_sizes) <= 0):
        raise ValueError("invalid engram geometry")


def canonical_shapes(m: dict) -> dict:
    """Name -> shape of every architecture tensor, in archive order (needle2/archive.py:46-68)."""
    d, lanes, layers, hd = m["d_model"], m["mhc_lanes"], m["num_layers"], m["head_dim"]
    att, kv, hada = m["num_heads"] * hd, m["num_kv_heads"] * hd, m["hada_n"]
    per_layer = ((d,), (att, d), (kv, d), (kv, d), (hd,), (hd,), (att, d), (d, att), (d,), (1,), (d,), (hada,),
                 (hada,), (hada,))
    shapes = {"embedding": (m["vocab_size"], d)}
    for layer in range(layers):
        for name, shape in zip(LAYER_NAMES, per_layer):
            shapes[f"layer{layer:02d}.{name}"] = shape
    mhc = ((layers,), (layers,), (layers,), (layers, lanes), (layers, lanes), (layers, lanes, lanes),
           (layers * lanes, lanes * d), (layers * lanes, lanes * d), (layers * lanes * lanes, lanes * d))
    shapes.update(zip(MHC_NAMES, mhc))
    width = m["num_engram_tables"] * m["engram_sub_dim"]
    for site in range(len(m["engram_layers"])):
        engram = ((m["num_engram_tables"] * m["engram_slots"], m["engram_sub_dim"]), (d, width), (d, width),
                  (m["engram_conv_taps"], d))
        for name, shape in zip(ENGRAM_NAMES, engram):
            shapes[f"engram{site}.{name}"] = shape
    shapes["final_norm"] = (d,)
    return shapes


@dataclass
class TensorRecord:
    """One tensor; ``blob`` is a read-only view of its payload (needle2/archive.py:86-121)."""
    name: str
    dtype: int
    shape: tuple
    blob: memoryview
    group_size: int = 0
    bits: int = 0
    codebook: np.ndarray | None = None
    offset: int = 0  # of the payload in the archive

    @property
    def rowbytes(self) -> int:
        return self.in_pad * (2 if self.bits == 5 else self.bits) // 8

    @property
    def in_pad(self) -> int:
        return math.ceil(self.shape[1] / self.group_size) * self.group_size

    @property
    def packed(self) -> np.ndarray:
        return np.frombuffer(self.blob, dtype=np.uint8, count=self.shape[0] * self.rowbytes).reshape(self.shape[0],
                                                                                                   -1)

    @property
    def norms(self) -> np.ndarray:
        return np.frombuffer(self.blob, dtype="<f2", offset=self.shape[0] * self.rowbytes).reshape(self.shape[0], -1)

    def cq_codebook(self) -> np.ndarray:
        """The record's centroids; ternary records: +-1.2240064 / sqrt(group) and 0."""
        if self.bits == 5:
            return (np.array([-_TERNARY, 0.0, _TERNARY]) / math.sqrt(self.group_size)).astype(np.float32)
        return self.codebook

    def dequantize(self) -> np.ndarray:
        if self.dtype == RAW:
            raise TypeError("RAW tokenizer is not a numeric tensor")
        if self.dtype in (FP16, FP32):
            return np.frombuffer(self.blob, dtype="<f2" if self.dtype == FP16 else "<f4").reshape(
                self.shape).astype(np.float32)
        if self.bits == 5 and np.any(formats.unpack_indices(self.packed, 2, self.in_pad) == 2):
            raise ValueError("invalid ternary crumb 2")
        return formats.dequantize_dense(self.packed, self.norms, self.shape, self.bits, self.group_size,
                                        self.cq_codebook()).astype(np.float32)


class Archive:
    """A validated `.cact` archive over bytes or a read-only memory map."""

    @classmethod
    def load(cls, path) -> "Archive":
        with open(Path(path), "rb") as f:
            size = f.seek(0, 2)
            if size == 0:
                return cls(b"")
            mapped = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
        return cls(mapped)

    def __init__(self, raw):
        self._owner = raw  # keeps the map (or bytes) alive for the record views
        view = memoryview(raw).cast("B")
        self.raw = view
        if len(view) < HEADER.size:
            raise ValueError("truncated .cact header")
        self.header = h = HEADER.unpack_from(view)
        if h[0] != TAG:
            raise ValueError(f"unsupported .cact tag {h[0]:#x}; expected Needle 2 {TAG:#x}")
        if h[2] != 28 or h[19] > 4 or h[24] > 4:
            raise ValueError("unsupported codebook or engram header geometry")
        count, ncb = h[1], h[2]
        end_dir = HEADER.size + ncb * 4 + count * RECORD.size
        if end_dir > len(view):
            raise ValueError("truncated .cact directory")
        self.metadata = m = _metadata(h)
        _check_geometry(m)
        base = 1 + m["num_layers"] * len(LAYER_NAMES) + len(MHC_NAMES) + len(ENGRAM_NAMES) * len(
            m["engram_layers"]) + 1
        if count not in {base + extra for extra in (0, 1, 4, 5, 7, 8)}:
            raise ValueError("tensor count does not match model geometry")
        self.codebook = np.frombuffer(view, dtype="<f4", count=ncb, offset=HEADER.size).copy()
        if not np.isfinite(self.codebook).all():
            raise ValueError("nonfinite codebook")
        records = [self._record(view, i, HEADER.size + ncb * 4 + i * RECORD.size, end_dir) for i in range(count)]
        spans = sorted((r[1], r[1] + r[2]) for r in records)
        if any(a[1] > b[0] for a, b in zip(spans, spans[1:])):
            raise ValueError("overlapping tensor payloads")
        records = [r[0] for r in records]
        names = self._names(records)
        self.tensors = {}
        for name, record in zip(names, records):
            record.name = name
            self.tensors[name] = record
        self._check_named_shapes()

    def _record(self, view, i, at, end_dir):
        dtype, ndim, reserved, d0, d1, d2, d3, offset, nbytes, group, bits = RECORD.unpack_from(view, at)
        if ndim > 4 or reserved != 0 or dtype not in (FP16, FP32, CQ, RAW):
            raise ValueError(f"invalid tensor record {i}")
        shape = (d0, d1, d2, d3)[:ndim]
        if offset % ALIGN or offset < end_dir or offset + nbytes > len(view):
            raise ValueError(f"out-of-range or unaligned tensor {i}")
        if dtype != RAW and (not shape or 0 in shape):
            raise ValueError("empty numeric tensor")
        if dtype != CQ and (group or bits):
            raise ValueError("non-CQ tensor carries quantization metadata")
        if dtype == RAW and ndim:
            raise ValueError("RAW tokenizer must have an empty shape")
        if dtype in (FP16, FP32):
            expected = math.prod(shape) * (2 if dtype == FP16 else 4)
        elif dtype == CQ:
            if ndim != 2 or group < 8 or group & (group - 1) or bits not in (2, 3, 4, 5):
                raise ValueError("unsupported CQ geometry")
            expected = cq_payload_bytes(shape[0], shape[1], group, bits)
        else:
            expected = nbytes
        if nbytes != expected:
            raise ValueError(f"tensor {i}: wrong payload size")
        cb = None
        if dtype == CQ and bits != 5:
            lo, hi = CODEBOOK_SLICES[bits]
            cb = self.codebook[lo:hi].copy()
            if not np.all(np.diff(cb) > 0):
                raise ValueError("codebook must be sorted")
        return TensorRecord("", dtype, shape, view[offset:offset + nbytes], group, bits, cb, offset), offset, nbytes

    def _names(self, records):
        """Architecture order, then the optional probe heads (manifest first) and the RAW tokenizer last
        (needle2/archive.py:196-222)."""
        m = self.metadata
        names = list(canonical_shapes(m))
        raw_last = int(bool(records) and records[-1].dtype == RAW)
        extra = len(records) - len(names) - raw_last
        if extra:
            if extra < 4 or (extra - 1) % 3 or len(names) >= len(records):
                raise ValueError("invalid optional probe heads layout")
            manifest_record = records[len(names)]
            if manifest_record.dtype not in (FP16, FP32) or len(manifest_record.shape) != 1:
                raise ValueError("head manifest must be a floating-point vector")
            manifest = manifest_record.dequantize().reshape(-1)
            if len(manifest) != (extra - 1) // 3 or len(set(manifest.tolist())) != len(manifest):
                raise ValueError("invalid head manifest")
            names.append("heads.manifest")
            for code in manifest:
                if code not in HEAD_CODES:
                    raise ValueError("unknown probe head code")
                head = HEAD_CODES[int(code)][0]
                names += [f"{head}.probes", f"{head}.proj", f"{head}.bias"]
        if raw_last:
            names.append("tokenizer")
        if len(names) != len(records):
            raise ValueError("tensor count does not match model geometry")
        return names

    def _check_named_shapes(self):
        """needle2/archive.py:71-84."""
        expected = canonical_shapes(self.metadata)
        d = self.metadata["d_model"]
        for head, probes in HEAD_CODES.values():
            if f"{head}.probes" not in self.tensors:
                continue
            proj = self.tensors[f"{head}.proj"]
            if len(proj.shape) != 2:
                raise ValueError(f"{head}.proj: expected a matrix")
            outputs = proj.shape[0] if head == "contrastive_head" else 1
            expected.update({f"{head}.probes": (probes, d), f"{head}.proj": (outputs, probes * d),
                             f"{head}.bias": (outputs,)})
        for name, shape in expected.items():
            record = self.tensors[name]
            if record.dtype == RAW or record.shape != shape:
                raise ValueError(f"{name}: expected numeric tensor {shape}, got dtype={record.dtype} "
                                 f"shape={record.shape}")

    def stats(self) -> dict:
        """Sizes and bits per weight (needle2/archive.py:238-248, without the file hash)."""
        numeric = [t for t in self.tensors.values() if t.dtype != RAW]
        quant = [t for t in numeric if t.dtype == CQ]
        params = sum(math.prod(t.shape) for t in numeric)
        qparams = sum(math.prod(t.shape) for t in quant)
        code_bits = sum(math.prod(t.shape) * (2 if t.bits == 5 else t.bits) for t in quant)
        return dict(bytes=len(self.raw), tensors=len(self.tensors), parameters=params, quantized_parameters=qparams,
                    code_bits_per_quantized_weight=code_bits / qparams if qparams else 0,
                    numeric_payload_bits_per_weight=sum(len(t.blob) * 8 for t in numeric) / params,
                    file_bits_per_weight=len(self.raw) * 8 / params,
                    precision_counts={str(b): sum(t.bits == b for t in quant) for b in sorted({t.bits for t in quant})})


def pack_archive(header, codebook, records) -> bytes:
    """Serialise (header tuple, 28-entry codebook, [(dtype, shape, payload bytes, group, bits)]) with payloads
    at 64-byte aligned offsets in record order. The result is validated by :class:`Archive`."""
    head = bytearray(HEADER.pack(*header) + np.ascontiguousarray(codebook, "<f4").tobytes())
    directory, payload = bytearray(), bytearray()
    pos = len(head) + len(records) * RECORD.size
    for dtype, shape, blob, group, bits in records:
        at = -(-pos // ALIGN) * ALIGN
        payload += bytes(at - pos)
        dims = (list(shape) + [0, 0, 0, 0])[:4]
        directory += RECORD.pack(dtype, len(shape), 0, *dims, at, len(blob), group, bits)
        payload += blob
        pos = at + len(blob)
    out = bytes(head + directory + payload)
    Archive(out)
    return out


# The released model's geometry (its header, docs/reference.md section 3 of the reference).
RELEASED_GEOMETRY = dict(vocab_size=8192, d_model=512, num_heads=8, num_kv_heads=4, num_layers=27, head_dim=64,
                         max_seq_len=2048, hada_n=512, mhc_lanes=4, engram_slots=8192, engram_sub_dim=128,
                         num_engram_tables=4, engram_conv_taps=4, engram_conv_dilation=3)


def synthetic_model(geometry: dict, engram_layers=(), engram_orders=(), kv_window: int = 0, group: int = 128,
                    seed: int = 0, heads: bool = False, tokenizer_bytes: int = 0, rope_theta: float = 100000.0,
                    vector_scale: float = 0.1, layer_bits: int = 2) -> bytes:
    """An archive of the given geometry with the released precision map and random contents.

    embedding and mhc_phi* CQ4, attention and engram matrices CQ2 (``layer_bits``: CQ4 for the layers'
    projections instead; all at ``group``), everything else FP16;
    optional probe heads (contrastive with 128 outputs, confidence) and RAW tokenizer. Codes are uniform random
    bytes, norms fp16 U[0.005, 0.05], FP16 values N(0, vector_scale); the codebook is the released header
    codebook."""
    rng = np.random.default_rng(seed)
    g = dict(geometry)
    d = g["d_model"]
    shapes = canonical_shapes(dict(g, engram_layers=list(engram_layers), engram_orders=list(engram_orders)))
    if heads:
        shapes.update({"heads.manifest": (2,), "contrastive_head.probes": (4, d),
                       "contrastive_head.proj": (128, 4 * d), "contrastive_head.bias": (128,),
                       "confidence_head.probes": (8, d), "confidence_head.proj": (1, 8 * d),
                       "confidence_head.bias": (1,)})
    records = []
    for name, shape in shapes.items():
        if name == "embedding" or name.startswith("mhc_phi"):
            bits = 4
        elif name.startswith(("layer", "engram")) and name.endswith(("_proj", ".tables")):
            bits = layer_bits if name.startswith("layer") else 2
        else:
            bits = 0
        if bits:
            rows, cols = shape
            padded = formats.padded_width(cols, group)
            packed = rng.integers(0, 256, size=(rows, padded * bits // 8), dtype=np.uint8)
            norms = rng.uniform(0.005, 0.05, size=(rows, padded // group)).astype("<f2")
            records.append((CQ, shape, packed.tobytes() + norms.tobytes(), group, bits))
        else:
            values = np.array([1, 2], "<f2") if name == "heads.manifest" else \
                (rng.normal(size=shape) * vector_scale).astype("<f2")
            records.append((FP16, shape, values.tobytes(), 0, 0))
    if tokenizer_bytes:
        records.append((RAW, (), rng.integers(0, 256, tokenizer_bytes, dtype=np.uint8).tobytes(), 0, 0))
    orders = (list(engram_orders) + [0, 0, 0, 0])[:4]
    sites = (list(engram_layers) + [0, 0, 0, 0])[:4]
    header = (TAG, len(records), 28, kv_window, 8, *[g[k] for k in GEOMETRY_FIELDS], len(engram_orders), *orders,
              len(engram_layers), *sites, rope_theta)
    return pack_archive(header, formats._HEADER_CODEBOOK, records)


def synthetic_released(seed: int = 0, tokenizer_bytes: int = 115215) -> bytes:
    """An archive with the released model's geometry and precision map (embedding and mhc_phi* CQ4 g128;
    attention and engram matrices CQ2 g128; everything else FP16; probe heads and a RAW tokenizer), random
    contents: :func:`synthetic_model` with the released header's geometry, KV window 256, engram sites 2 and
    15 of orders 2 and 3."""
    return synthetic_model(RELEASED_GEOMETRY, engram_layers=(2, 15), engram_orders=(2, 3), kv_window=256,
                           group=128, seed=seed, heads=True, tokenizer_bytes=tokenizer_bytes)


@dataclass
class DeviceModel:
    """Every tensor of an archive in device memory, uploaded once.

    The span of the file holding the CQ payloads goes to the device in one copy; each CQ record then becomes a
    :class:`~openneedle_amd.cq.CQMatrix` whose relayout kernels read its codes and norms there (plus its
    int8 twin for CQ2 / CQ4 when ``int8``), and the copy is freed once they have run. The FP16 / FP32 tensors
    go up as one fp32 buffer; ``dense[name]`` is a device view of it. The archive stays referenced: the
    handles keep host views of the mapped file for later lazily built int8 twins."""
    archive: Archive
    int8: bool = False
    matrices: dict = field(default_factory=dict)
    dense: dict = field(default_factory=dict)
    uploaded_bytes: int = 0

    def __post_init__(self):
        from .cq import CQMatrix
        from .device import DeviceArray, Stream
        tensors = self.archive.tensors.values()
        cq = [r for r in tensors if r.dtype == CQ]
        stream = Stream()
        if cq:
            lo = min(r.offset for r in cq)
            hi = max(r.offset + len(r.blob) for r in cq)
            span = DeviceArray(hi - lo)
            span.upload(np.frombuffer(self.archive.raw[lo:hi], dtype=np.uint8))
            for r in cq:
                at = span.ptr + r.offset - lo
                self.matrices[r.name] = CQMatrix.from_record(r, device=(at, at + r.shape[0] * r.rowbytes, stream),
                                                             int8=self.int8)
            stream.synchronize()
            self.uploaded_bytes += hi - lo
            span.close()  # the relayouts that read it have run
        stream.close()
        dense = [r for r in tensors if r.dtype in (FP16, FP32)]
        if dense:
            values = [r.dequantize().reshape(-1) for r in dense]
            flat = np.concatenate(values).astype(np.float32)
            self._dense_buffer = DeviceArray.from_host(flat)
            at = 0
            for r, v in zip(dense, values):
                self.dense[r.name] = self._dense_buffer.view(at * 4, v.size * 4)
                at += v.size
            self.uploaded_bytes += flat.nbytes
