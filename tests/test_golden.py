"""The oracle against golden vectors written by the reference itself.

tests/golden/*.npz hold seeded inputs and the outputs of the reference's own
C++ (compiled from its sources by oracle/Makefile; generator:
tests/golden/make_golden.py). These tests need neither the reference sources
nor a GPU: they pin the oracle bit for bit (int8 codes, scales, FP32 and int8
GEMV outputs, row dequantization, attention outputs).
"""
from pathlib import Path

import numpy as np
import pytest

import oracle
from tests.cases import permute_like_reference

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    return np.load(GOLDEN / f"{name}.npz", allow_pickle=False)


def names(prefix):
    return sorted(p.stem for p in GOLDEN.glob(f"{prefix}*.npz"))


def test_fixture_set_is_complete():
    assert len(names("cq_b")) == 8 and names("cq4_decode") and len(names("sdot_")) == 4 and len(names("attn_")) == 2


@pytest.mark.parametrize("name", names("cq_b") + names("cq4_decode"))
def test_cq_linear_and_rows(name):
    f = load(name)
    rows, dim, bits, group = (int(v) for v in f["shape"])
    norms = f["norms"].view(np.float16)
    y = oracle.cq_linear(f["packed"], norms, (rows, dim), bits, group, f["cb"], f["x"], 2)
    np.testing.assert_array_equal(y, f["y"])
    if "ids" in f:
        np.testing.assert_array_equal(oracle.cq_rows(f["packed"], norms, (rows, dim), bits, group, f["cb"], f["ids"]),
                                      f["rows"])


@pytest.mark.parametrize("name", names("sdot_"))
def test_sdot(name):
    f = load(name)
    rows, dim, bits, group = (int(v) for v in f["shape"])
    norms = f["norms"].view(np.float16)
    cent, cs = oracle.sdot_centroids(f["cb"], bits)
    np.testing.assert_array_equal(cent, f["centroids"])
    assert np.float32(cs).view(np.uint32) == f["centroid_scale"].view(np.uint32)[0]
    q, s = oracle.sdot_prepare(f["x"][0], group)
    np.testing.assert_array_equal(permute_like_reference(q, bits, group), f["q0"])
    np.testing.assert_array_equal(s, f["xs0"])
    y = oracle.sdot_linear(f["packed"], norms, (rows, dim), bits, group, f["cb"], f["x"], 2)
    np.testing.assert_array_equal(y, f["y"])


@pytest.mark.parametrize("name", names("attn_"))
def test_kv_quantize_and_attention(name):
    f = load(name)
    k8, ks = oracle.kv_quantize(f["k"])
    v8, vs = oracle.kv_quantize(f["v"])
    np.testing.assert_array_equal(k8, f["k8"])
    np.testing.assert_array_equal(v8, f["v8"])
    np.testing.assert_array_equal(ks, f["k_scales"])
    np.testing.assert_array_equal(vs, f["v_scales"])
    np.testing.assert_array_equal(oracle.attention_i8(f["q"], k8, v8, ks, vs), f["out"])
