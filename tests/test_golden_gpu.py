"""The HIP library against the reference's own golden vectors (tests/golden).

FP32 GEMV, row dequantization, the int8 path and the KV quantizer are
bit-identical to the reference; attention agrees within atol=1e-6 +
rtol=1e-5 (split-context fp32 sums are reordered).
"""
from pathlib import Path

import numpy as np
import pytest

from openneedle_amd.cq import CQMatrix
from openneedle_amd.device import DeviceArray, synchronize
from openneedle_amd.kv import KVCache

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    return np.load(GOLDEN / f"{name}.npz", allow_pickle=False)


def names(prefix):
    return sorted(p.stem for p in GOLDEN.glob(f"{prefix}*.npz"))


@pytest.mark.parametrize("name", names("cq_b") + names("cq4_decode"))
def test_cq(name):
    f = load(name)
    rows, dim, bits, group = (int(v) for v in f["shape"])
    q = CQMatrix(f["packed"], f["norms"].view(np.float16), (rows, dim), bits, group, f["cb"])
    np.testing.assert_array_equal(q.matvec(f["x"]), f["y"])
    if "ids" in f:
        np.testing.assert_array_equal(q.rows(f["ids"]), f["rows"])


@pytest.mark.parametrize("name", names("sdot_"))
def test_sdot(name):
    f = load(name)
    rows, dim, bits, group = (int(v) for v in f["shape"])
    q = CQMatrix(f["packed"], f["norms"].view(np.float16), (rows, dim), bits, group, f["cb"])
    np.testing.assert_array_equal(q.matvec_int8(f["x"], reference_bound=True), f["y"])


@pytest.mark.parametrize("name", names("attn_"))
def test_attention(name):
    f = load(name)
    n, kvh, hd = f["k"].shape
    heads = f["q"].shape[0]
    kv = KVCache(1, n + 8, kvh, hd, 1)
    d_k, d_v = DeviceArray.from_host(f["k"][None]), DeviceArray.from_host(f["v"][None])
    kv.store(0, d_k.ptr, d_v.ptr, n)
    synchronize()
    k8, v8, ks, vs = kv.read(0, 0, n)
    np.testing.assert_array_equal(k8, f["k8"])
    np.testing.assert_array_equal(v8, f["v8"])
    np.testing.assert_array_equal(ks, f["k_scales"])
    np.testing.assert_array_equal(vs, f["v_scales"])
    d_q = DeviceArray.from_host(f["q"][None])
    d_o = DeviceArray(f["q"].nbytes)
    kv.attention(0, d_q.ptr, d_o.ptr, heads, n)
    synchronize()
    np.testing.assert_allclose(d_o.download(np.empty((heads, hd), np.float32)), f["out"], atol=1e-6, rtol=1e-5)
