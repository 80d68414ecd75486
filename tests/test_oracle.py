"""Pins for the CPU oracle (oracle/needle2_oracle.c).

Each restated function is checked three ways where possible:
  * bit-exact against the reference's own code compiled from source
    (oracle/_ref; skipped when the reference sources were not available);
  * against closed forms that a plausible slip (wrong index, sign, dropped
    term, transposed operand) would break: dense Sylvester-Hadamard, integer
    dot products, fp64 softmax;
  * against the reference tests' own known answers (bitstream, zero rows).
"""
import numpy as np
import pytest

import oracle
from openneedle_amd import formats
from tests.cases import activations, example, permute_like_reference

needs_ref = pytest.mark.skipif(oracle.ref() is None, reason="reference sources not available to build oracle/_ref")


# ---------------------------------------------------------------- fp16 ----
def test_half_float_exhaustive_against_numpy():
    bits = np.arange(1 << 16, dtype=np.uint16)
    expected = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.half_float(b) for b in bits], np.float32)
    nan = np.isnan(expected)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), expected[~nan].view(np.uint32))


# ---------------------------------------------------------------- FWHT ----
@pytest.mark.parametrize("n", [8, 16, 32, 64, 128, 1024])
def test_hadamard_matches_dense_sylvester(n):
    x = activations((5, n), seed=n)
    got = oracle.hadamard(x)
    np.testing.assert_allclose(got, x.astype(np.float64) @ formats.hadamard_matrix(n), atol=2e-6, rtol=0)
    # normalized transform is an involution
    np.testing.assert_allclose(oracle.hadamard(got), x, atol=4e-6)


def test_hadamard_first_column_is_constant():
    e0 = np.zeros(32, np.float32)
    e0[0] = 1
    np.testing.assert_array_equal(oracle.hadamard(e0), np.full(32, np.float32(1) / np.sqrt(np.float32(32))))


# ---------------------------------------------------------------- FP32 GEMV ----
@pytest.mark.parametrize("bits", [2, 3, 4, 5])
def test_cq_linear_matches_dense_closed_form(bits):
    packed, norms, cb, dense = example(bits)
    x = activations((2, 3, 257))
    for threads in (1, 2):
        got = oracle.cq_linear(packed, norms, dense.shape, bits, 128, cb, x, threads)
        np.testing.assert_allclose(got, x.astype(np.float64) @ dense.T, atol=3e-6, rtol=2e-5)
    assert np.all(got[..., 0] == 0)  # the all-zero-norm row


@needs_ref
@pytest.mark.parametrize("bits", [2, 3, 4, 5])
@pytest.mark.parametrize("group", [8, 32, 64, 128])
def test_cq_linear_bit_exact_with_reference(bits, group):
    packed, norms, cb, dense = example(bits, rows=33, dim=200, group=group)
    x = activations((3, 200), seed=group + bits)
    ref = oracle.RefCQ(packed, norms, dense.shape, bits, group, cb)
    for threads in (1, 3):
        got = oracle.cq_linear(packed, norms, dense.shape, bits, group, cb, x, threads)
        np.testing.assert_array_equal(got, ref.linear(x, threads))


@needs_ref
def test_cq_linear_bit_exact_baseline_shape():
    from tests.cases import baseline
    packed, norms, cb, _ = baseline(4, 2048, 512)
    x = activations((512,), seed=3)
    ref = oracle.RefCQ(packed, norms, (2048, 512), 4, 32, cb)
    np.testing.assert_array_equal(oracle.cq_linear(packed, norms, (2048, 512), 4, 32, cb, x, 4), ref.linear(x, 4))


@pytest.mark.parametrize("bits", [2, 3, 4, 5])
def test_cq_rows_matches_dense(bits):
    packed, norms, cb, dense = example(bits)
    ids = np.array([[8, 2], [0, 2]])
    got = oracle.cq_rows(packed, norms, dense.shape, bits, 128, cb, ids)
    np.testing.assert_allclose(got, dense[ids], atol=2e-7, rtol=3e-5)
    if oracle.ref() is not None:
        ref = oracle.RefCQ(packed, norms, dense.shape, bits, 128, cb)
        np.testing.assert_array_equal(got, ref.rows(ids))


# ---------------------------------------------------------------- int8 path ----
# The reference's scalar prepare permutes activations within 64-wide chunks for
# CQ2 (sdot.cpp:99-100), which writes past the group when group < 64; its ABI
# rejects such groups (sdot.cpp:352). CQ2 with group 32 is therefore pinned by
# the integer closed form only.
REF_SDOT_CASES = [(4, 32), (4, 64), (4, 128), (2, 64), (2, 128)]


@needs_ref
@pytest.mark.parametrize("bits,group", REF_SDOT_CASES)
def test_sdot_tables_and_prepare_bit_exact_with_reference(bits, group):
    packed, norms, cb, dense = example(bits, dim=257, group=group)
    ref = oracle.RefCQ(packed, norms, dense.shape, bits, group, cb)
    cent, cs, ns = ref.sdot_tables()
    my_cent, my_cs = oracle.sdot_centroids(cb, bits)
    np.testing.assert_array_equal(my_cent, cent)
    assert np.float32(my_cs).view(np.uint32) == np.float32(cs).view(np.uint32)
    my_ns = np.array([[oracle.half_float(h) for h in row] for row in norms.view(np.uint16)], np.float32) * my_cs
    np.testing.assert_array_equal(my_ns, ns)
    for x in (activations(257, seed=315), np.zeros(257, np.float32), np.eye(1, 257, dtype=np.float32)[0]):
        q, s = oracle.sdot_prepare(x, group)
        rq, rs = ref.sdot_prepare(x)
        np.testing.assert_array_equal(permute_like_reference(q, bits, group), rq)
        np.testing.assert_array_equal(s, rs)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("group", [32, 64, 128])
def test_sdot_integer_closed_form(bits, group):
    """int32 dots = sum cent[idx]*q exactly; outputs within the reference test's tolerance."""
    packed, norms, cb, dense = example(bits, dim=257, group=group)
    x = activations((5, 257), seed=315)
    x[0] = 0
    x[1] = 0
    x[1, 0] = 1
    padded = norms.shape[1] * group
    cent, cs = oracle.sdot_centroids(cb, bits)
    # independent construction of the centroid table and scales (numpy, fp64 checks)
    cmax = np.max(np.abs(cb)) / np.float32(127)
    np.testing.assert_array_equal(cent, np.clip(np.rint(cb / cmax), -127, 127).astype(np.int8))
    idx = formats.unpack_indices(packed, bits, padded).astype(np.int64)
    got = oracle.sdot_linear(packed, norms, dense.shape, bits, group, cb, x)
    for b in range(5):
        q, xs = oracle.sdot_prepare(x[b], group)
        rot = np.pad(x[b], (0, padded - 257)).reshape(-1, group).astype(np.float64) @ formats.hadamard_matrix(group)
        amax = np.abs(rot).max(-1)
        np.testing.assert_allclose(xs, np.where(amax > 0, amax / 127, 1), rtol=1e-6)
        np.testing.assert_array_less(np.abs(q.reshape(-1, group) - rot / xs[:, None].astype(np.float64)), 0.5 + 1e-4)
        dots = oracle.sdot_dots(packed, dense.shape, bits, group, cent, q)
        exact = (cent.astype(np.int64)[idx].reshape(9, -1, group) * q.astype(np.int64).reshape(-1, group)).sum(-1)
        np.testing.assert_array_equal(dots, exact)
        ns = norms.astype(np.float64) * np.float64(cs)
        expected = (dots * ns * xs.astype(np.float64)).sum(-1)
        np.testing.assert_allclose(got[b], expected, atol=2e-6, rtol=2e-5)


@needs_ref
@pytest.mark.parametrize("bits,group", REF_SDOT_CASES)
@pytest.mark.parametrize("rows", [9, 129])
def test_sdot_linear_bit_exact_with_reference(bits, group, rows):
    packed, norms, cb, dense = example(bits, rows=rows, dim=257, group=group)
    ref = oracle.RefCQ(packed, norms, dense.shape, bits, group, cb)
    x = np.stack([activations(257, seed=42), np.zeros(257, np.float32), np.eye(1, 257, dtype=np.float32)[0]])
    for threads in (1, 2, 4):
        np.testing.assert_array_equal(oracle.sdot_linear(packed, norms, dense.shape, bits, group, cb, x, threads),
                                      ref.sdot_linear(x, threads))


@needs_ref
def test_sdot_subnormal_scale_guard_matches_reference():
    """absmax/127 underflows to 0 for tiny subnormal groups; the scale falls back to absmax."""
    packed, norms, cb, dense = example(4, rows=4, dim=64, group=32)
    x = np.zeros(64, np.float32)
    tiny = np.float32(4e-45)  # a few multiples of the smallest subnormal
    x[:32] = tiny
    x[40] = np.float32(1e-39)
    ref = oracle.RefCQ(packed, norms, dense.shape, 4, 32, cb)
    q, s = oracle.sdot_prepare(x, 32)
    rq, rs = ref.sdot_prepare(x)
    np.testing.assert_array_equal(s, rs)
    np.testing.assert_array_equal(permute_like_reference(q, 4, 32), rq)
    assert s[0] > 0 and np.float32(s[0]) / np.float32(127) == 0  # the guarded branch was taken
    np.testing.assert_array_equal(oracle.sdot_linear(packed, norms, dense.shape, 4, 32, cb, x),
                                  ref.sdot_linear(x))


# ---------------------------------------------------------------- int8 KV ----
def _kv(tokens, kvh, hd, seed=7):
    rng = np.random.default_rng(seed)
    k = rng.normal(size=(tokens, kvh, hd)).astype(np.float32)
    v = rng.normal(size=(tokens, kvh, hd)).astype(np.float32)
    k[0, 0] = 0  # max == 0 branch
    return k, v


def test_kv_quantize_closed_form():
    k, _ = _kv(17, 3, 38)
    q, s = oracle.kv_quantize(k)
    amax = np.abs(k).max(-1)
    np.testing.assert_array_equal(s, np.where(amax > 0, amax / np.float32(127), np.float32(1)).astype(np.float32))
    inv = np.where(amax > 0, np.float32(127) / np.where(amax > 0, amax, 1), np.float32(0)).astype(np.float32)
    np.testing.assert_array_equal(q, np.clip(np.rint(k * inv[..., None]), -127, 127).astype(np.int8))
    assert np.all(q[0, 0] == 0) and s[0, 0] == 1


@needs_ref
@pytest.mark.parametrize("kvh,hd", [(8, 64), (2, 32), (3, 38)])
def test_kv_quantize_bit_exact_with_reference(kvh, hd):
    k, v = _kv(33, kvh, hd)
    ref = oracle.RefAttention(kvh, kvh, hd, 64)
    ref.load(k, v)
    rk, rv, rks, rvs = ref.cache()
    qk, sk = oracle.kv_quantize(k)
    qv, sv = oracle.kv_quantize(v)
    np.testing.assert_array_equal(qk, rk)
    np.testing.assert_array_equal(qv, rv)
    np.testing.assert_array_equal(sk, rks)
    np.testing.assert_array_equal(sv, rvs)


# ---------------------------------------------------------------- attention ----
def _attention_fp64(q, k8, v8, ks, vs, heads, kvh):
    hd = q.shape[-1]
    out = np.empty((heads, hd))
    for h in range(heads):
        kh = h // (heads // kvh)
        kf = k8[:, kh].astype(np.float64) * ks[:, kh, None]
        vf = v8[:, kh].astype(np.float64) * vs[:, kh, None]
        s = kf @ q[h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ vf
    return out


@pytest.mark.parametrize("heads,kvh,hd,length", [(8, 8, 64, 300), (8, 2, 64, 65), (4, 4, 38, 17), (6, 3, 32, 1)])
def test_attention_matches_fp64_closed_form(heads, kvh, hd, length):
    k, v = _kv(length, kvh, hd, seed=length)
    k8, ks = oracle.kv_quantize(k)
    v8, vs = oracle.kv_quantize(v)
    q = activations((heads, hd), seed=hd)
    got = oracle.attention_i8(q, k8, v8, ks, vs)
    np.testing.assert_allclose(got, _attention_fp64(q, k8, v8, ks, vs, heads, kvh), atol=2e-6, rtol=2e-5)


@needs_ref
@pytest.mark.parametrize("heads,kvh,hd,length", [(8, 8, 64, 300), (8, 2, 64, 65), (4, 4, 38, 17), (6, 3, 32, 1)])
@pytest.mark.parametrize("threads", [1, 2])
def test_attention_bit_exact_with_reference(heads, kvh, hd, length, threads):
    k, v = _kv(length, kvh, hd, seed=length)
    ref = oracle.RefAttention(heads, kvh, hd, 512, threads)
    ref.load(k, v)
    rk, rv, rks, rvs = ref.cache()
    q = activations((heads, hd), seed=hd)
    np.testing.assert_array_equal(oracle.attention_i8(q, rk, rv, rks, rvs), ref.attend(q))
