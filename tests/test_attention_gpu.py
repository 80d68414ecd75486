"""GPU parity of the int8 KV cache and decode attention against the oracle.

Store: bit-identical int8 codes and fp32 scales (the oracle is bit-identical
to the reference's own Engine, tests/test_oracle.py). Attention: the GPU
splits the slot range and rescales partial softmax sums, so fp32 sums are
reordered; outputs must agree with the oracle (the reference's sequential
arithmetic) within atol=1e-6 + rtol=1e-5 per output, and with the fp64 closed
form within the oracle's own tolerance (atol=2e-6, rtol=2e-5).
"""
import numpy as np
import pytest

import oracle
from openneedle_amd.device import DeviceArray, synchronize
from openneedle_amd.kv import KVCache

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-6, 1e-5


def fp64_attention(q, k8, v8, ks, vs, slots):
    heads, hd = q.shape
    kvh = k8.shape[1]
    out = np.empty((heads, hd))
    for h in range(heads):
        kh = h // (heads // kvh)
        k = k8[slots, kh].astype(np.float64) * ks[slots, kh, None]
        v = v8[slots, kh].astype(np.float64) * vs[slots, kh, None]
        s = k @ q[h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v
    return out


def make_cache(rng, seqs, cap, kvh, hd):
    k = rng.normal(size=(seqs, cap, kvh, hd)).astype(np.float32)
    v = rng.normal(size=(seqs, cap, kvh, hd)).astype(np.float32)
    rows = [(oracle.kv_quantize(k[s]), oracle.kv_quantize(v[s])) for s in range(seqs)]
    return k, v, rows


def run_attention(kv, q, length, slots=None, lengths=None, splits=0):
    seqs, heads, hd = q.shape
    d_q = DeviceArray.from_host(q)
    d_o = DeviceArray(q.nbytes)
    d_o.upload(np.full(q.shape, np.nan, np.float32))
    d_s = DeviceArray.from_host(np.asarray(slots, np.int32)) if slots is not None else None
    d_l = DeviceArray.from_host(np.asarray(lengths, np.int32)) if lengths is not None else None
    kv.attention(0, d_q.ptr, d_o.ptr, heads, length, d_s.ptr if d_s else None, d_l.ptr if d_l else None, splits)
    synchronize()
    return d_o.download(np.empty(q.shape, np.float32))


def test_store_bit_exact_and_storage_bytes():
    rng = np.random.default_rng(1)
    seqs, cap, kvh, hd, count = 3, 40, 4, 64, 17
    kv = KVCache(2, cap, kvh, hd, seqs)
    k = rng.normal(size=(seqs, count, kvh, hd)).astype(np.float32) * 3
    v = rng.normal(size=(seqs, count, kvh, hd)).astype(np.float32)
    k[1, 2, 3] = 0  # an all-zero row: scale 1, inverse 0
    v[0, 5, 1, :7] = 1e-41  # subnormal inputs
    d_k, d_v = DeviceArray.from_host(k), DeviceArray.from_host(v)
    kv.store(1, d_k.ptr, d_v.ptr, count, first_slot=[0, 5, 23])
    synchronize()
    for s, first in enumerate([0, 5, 23]):
        k8, v8, ks, vs = kv.read(1, s, count, first)
        ek, eks = oracle.kv_quantize(k[s])
        ev, evs = oracle.kv_quantize(v[s])
        np.testing.assert_array_equal(k8, ek)
        np.testing.assert_array_equal(v8, ev)
        np.testing.assert_array_equal(ks, eks)
        np.testing.assert_array_equal(vs, evs)
    # untouched slots stay zero
    k8, _, ks, _ = kv.read(1, 1, 5, 0)
    assert not k8.any() and not ks.any()
    # reference: layers * slots * (2 * kvh * hd + 2 * kvh * 4) bytes per sequence
    assert kv.storage_bytes() == 2 * seqs * cap * (2 * kvh * hd + 2 * kvh * 4)


def test_store_matches_reference_engine():
    ref = pytest.importorskip("oracle").ref()
    if ref is None:
        pytest.skip("reference library not built")
    heads, kvh, hd, n = 8, 4, 64, 37
    rng = np.random.default_rng(3)
    k = rng.normal(size=(n, kvh, hd)).astype(np.float32)
    v = rng.normal(size=(n, kvh, hd)).astype(np.float32)
    r = oracle.RefAttention(heads, kvh, hd, n + 4)
    r.load(k.reshape(n, -1), v.reshape(n, -1))
    rk, rv, rks, rvs = r.cache()
    kv = KVCache(1, n + 4, kvh, hd, 1)
    d_k, d_v = DeviceArray.from_host(k[None]), DeviceArray.from_host(v[None])
    kv.store(0, d_k.ptr, d_v.ptr, n)
    synchronize()
    gk, gv, gks, gvs = kv.read(0, 0, n)
    np.testing.assert_array_equal(gk, rk)
    np.testing.assert_array_equal(gv, rv)
    np.testing.assert_array_equal(gks, rks)
    np.testing.assert_array_equal(gvs, rvs)
    q = rng.normal(size=(heads, hd)).astype(np.float32)
    got = run_attention(kv, q[None], n)[0]
    np.testing.assert_allclose(got, r.attend(q), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("heads,kvh", [(8, 8), (8, 4), (8, 2), (8, 1)])
@pytest.mark.parametrize("hd", [32, 64, 128])
@pytest.mark.parametrize("length", [1, 255, 256, 257, 1000])
def test_attention_shapes(heads, kvh, hd, length):
    rng = np.random.default_rng(heads * 1000 + kvh * 100 + hd + length)
    seqs, cap = 2, 1024
    _, _, rows = make_cache(rng, seqs, cap, kvh, hd)
    kv = KVCache(1, cap, kvh, hd, seqs)
    for s, ((k8, ks), (v8, vs)) in enumerate(rows):
        kv.load(0, s, k8, v8, ks, vs)
    q = rng.normal(size=(seqs, heads, hd)).astype(np.float32)
    slots = np.arange(length)
    for splits in (0, 1, 3):
        got = run_attention(kv, q, length, splits=splits)
        for s, ((k8, ks), (v8, vs)) in enumerate(rows):
            ref = oracle.attention_i8(q[s], k8, v8, ks, vs, slots)
            np.testing.assert_allclose(got[s], ref, atol=ATOL, rtol=RTOL)
            np.testing.assert_allclose(got[s], fp64_attention(q[s], k8, v8, ks, vs, slots), atol=2e-6, rtol=2e-5)


def test_slot_lists_lengths_and_empty():
    """A ring-like slot list (prefix sinks then a window), ragged per-sequence
    lengths including zero, and listed slots outside the cache (skipped)."""
    rng = np.random.default_rng(7)
    seqs, cap, kvh, hd, heads = 4, 600, 2, 64, 4
    _, _, rows = make_cache(rng, seqs, cap, kvh, hd)
    kv = KVCache(1, cap, kvh, hd, seqs)
    for s, ((k8, ks), (v8, vs)) in enumerate(rows):
        kv.load(0, s, k8, v8, ks, vs)
    window = (np.arange(300, 300 + 500) % cap)
    slots = np.concatenate([np.arange(4), window]).astype(np.int32)  # 504 entries
    lengths = np.array([504, 0, 1, 333], np.int32)
    q = rng.normal(size=(seqs, heads, hd)).astype(np.float32)
    for splits in (0, 1, 2):
        got = run_attention(kv, q, len(slots), slots=slots, lengths=lengths, splits=splits)
        for s, ((k8, ks), (v8, vs)) in enumerate(rows):
            if lengths[s] == 0:
                np.testing.assert_array_equal(got[s], 0)  # empty softmax: the reference sums nothing
                continue
            ref = oracle.attention_i8(q[s], k8, v8, ks, vs, slots[:lengths[s]])
            np.testing.assert_allclose(got[s], ref, atol=ATOL, rtol=RTOL)
    bad = slots.copy()
    bad[[10, 20]] = [-5, cap + 3]  # skipped, as if absent from the list
    got = run_attention(kv, q, len(bad), slots=bad)
    keep = np.delete(slots, [10, 20])
    for s, ((k8, ks), (v8, vs)) in enumerate(rows):
        np.testing.assert_allclose(got[s], oracle.attention_i8(q[s], k8, v8, ks, vs, keep), atol=ATOL, rtol=RTOL)


def test_decode_batch_full_size():
    """64 sequences x 8 heads x head_dim 64, 2047 cached tokens plus one
    stored this step (the decode-layer workload); every sequence checked."""
    rng = np.random.default_rng(2026)
    seqs, cap, kvh, hd, heads = 64, 2048, 8, 64, 8
    kv = KVCache(1, cap, kvh, hd, seqs)
    k = rng.normal(size=(seqs, cap, kvh, hd)).astype(np.float32)
    v = rng.normal(size=(seqs, cap, kvh, hd)).astype(np.float32)
    d_k, d_v = DeviceArray.from_host(k[:, :cap - 1]), DeviceArray.from_host(v[:, :cap - 1])
    kv.store(0, d_k.ptr, d_v.ptr, cap - 1)
    d_k1, d_v1 = DeviceArray.from_host(k[:, cap - 1:]), DeviceArray.from_host(v[:, cap - 1:])
    kv.store(0, d_k1.ptr, d_v1.ptr, 1, first_slot=cap - 1)
    q = rng.normal(size=(seqs, heads, hd)).astype(np.float32)
    got = run_attention(kv, q, cap)
    slots = np.arange(cap)
    for s in range(seqs):
        k8, v8, ks, vs = kv.read(0, s, cap)
        ek, eks = oracle.kv_quantize(k[s])
        np.testing.assert_array_equal(k8, ek)
        np.testing.assert_array_equal(ks, eks)
        np.testing.assert_allclose(got[s], oracle.attention_i8(q[s], k8, v8, ks, vs, slots), atol=ATOL, rtol=RTOL)


def test_validation_errors():
    kv = KVCache(1, 16, 2, 64, 2)
    d = DeviceArray(4 * 2 * 4 * 2 * 64)
    with pytest.raises(RuntimeError, match="capacity"):
        kv.store(0, d.ptr, d.ptr, 4, first_slot=14)
    with pytest.raises(RuntimeError, match="layer"):
        kv.store(1, d.ptr, d.ptr, 1)
    with pytest.raises(RuntimeError, match="multiple of kvheads"):
        kv.attention(0, d.ptr, d.ptr, 3, 4)
    with pytest.raises(RuntimeError, match="capacity"):
        kv.attention(0, d.ptr, d.ptr, 2, 17)
    with pytest.raises(RuntimeError, match="head_dim"):
        KVCache(1, 16, 2, 48, 1)


@pytest.mark.parametrize("hd", [32, 64, 128])
@pytest.mark.parametrize("splits", [0, 1, 3])
def test_attention_storing_the_new_token(hd, splits):
    """The new token of every sequence stored by the attention launch (at slots inside a first sub-tile, past
    it, past every split's range, at the last slot and outside the cache): cache rows bit-identical to the
    store kernel's (oracle.kv_quantize), outputs as attending the stored cache."""
    rng = np.random.default_rng(hd * 10 + splits)
    seqs, cap, kvh, heads, length = 5, 1024, 2, 4, 700
    _, _, rows = make_cache(rng, seqs, cap, kvh, hd)
    kv = KVCache(1, cap, kvh, hd, seqs)
    for s, ((k8, ks), (v8, vs)) in enumerate(rows):
        kv.load(0, s, k8, v8, ks, vs)
    new_slot = np.array([3, 500, 900, cap - 1, cap + 7], np.int32)
    nk = rng.normal(size=(seqs, kvh, hd)).astype(np.float32)
    nv = rng.normal(size=(seqs, kvh, hd)).astype(np.float32)
    q = rng.normal(size=(seqs, heads, hd)).astype(np.float32)
    d_q, d_o = DeviceArray.from_host(q), DeviceArray(q.nbytes)
    d_o.upload(np.full(q.shape, np.nan, np.float32))
    d_k, d_v, d_s = DeviceArray.from_host(nk), DeviceArray.from_host(nv), DeviceArray.from_host(new_slot)
    kv.attention(0, d_q, d_o, heads, length, splits=splits, new=(d_k, d_v, d_s))
    synchronize()
    got = d_o.download(np.empty(q.shape, np.float32))
    k8n, ksn = oracle.kv_quantize(nk)
    v8n, vsn = oracle.kv_quantize(nv)
    for s, ((k8, ks), (v8, vs)) in enumerate(rows):
        k8, v8, ks, vs = k8.copy(), v8.copy(), ks.copy(), vs.copy()
        if new_slot[s] < cap:
            k8[new_slot[s]], v8[new_slot[s]], ks[new_slot[s]], vs[new_slot[s]] = k8n[s], v8n[s], ksn[s], vsn[s]
        for a, b in zip(kv.read(0, s, cap), (k8, v8, ks, vs)):
            np.testing.assert_array_equal(a, b, err_msg=f"seq {s}: cache after the step")
        ref = oracle.attention_i8(q[s], k8, v8, ks, vs, np.arange(length))
        np.testing.assert_allclose(got[s], ref, atol=ATOL, rtol=RTOL)
