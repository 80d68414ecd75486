"""The composed decode layer the bench times (bench.DecodeLayer: 64 sequences, hidden 512, 8 heads = 8 kv heads
of 64, MLP 2048, int8-path CQ4 g32 projections, int8 KV cache of 2048 slots), one step, every stage against the
oracle on the stage's own GPU input:

- Q | K | V, O, MLP up and down: bit-exact with oracle.sdot_linear (the reference's SdotCQ arithmetic);
- the new token's K / V rows in the cache: bit-exact with oracle.kv_quantize;
- attention over the whole cache as the GPU holds it, per (sequence, head): normwise relative error at most
  1e-5 against both oracle.attention_i8 and the fp64 closed form, and every output within 4e-6 * max|v| of
  fp64 (v: the head's dequantized values). The queries come out of the Q projection with a standard deviation
  of about 3.2 (scores about 3x those of tests/test_attention_gpu.py, where the per-output 1e-6 + 1e-5 bar
  holds); on such inputs the oracle's own sequential fp32 arithmetic reaches 4.8e-6 normwise and
  1.7e-6 * max|v| per output against fp64, so the bars are about twice the reference's own error;
- the slots before the new token are untouched by the step.

The step stores the new token inside the attention launch and runs the projections after the attention as a
chain (each producer leaves the next plan's input prepared); the chained step's outputs and cache rows equal
the unchained step's (separate store launch, every plan preparing its own input) bit for bit, with the store
and preparation fused into the attention and GEMV epilogues and with the fallback launches (other batch sizes,
the attention split, the 16 x 16 K split switched off)."""
import numpy as np
import pytest

import bench
import oracle
from openneedle_amd._ffi import GpuError
from openneedle_amd.cq import Plan
from openneedle_amd.device import DeviceArray, Stream, Teardown, synchronize

pytestmark = pytest.mark.gpu

NORMWISE, PER_VALUE = 1e-5, 4e-6


def fp64_attention(q, k8, v8, ks, vs):
    heads, hd = q.shape
    group = heads // k8.shape[1]
    out, vmax = np.empty((heads, hd)), np.empty(heads)
    for h in range(heads):
        kh = h // group
        k = k8[:, kh].astype(np.float64) * ks[:, kh, None]
        v = v8[:, kh].astype(np.float64) * vs[:, kh, None]
        s = k @ q[h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ v
        vmax[h] = np.abs(v).max()
    return out, vmax


def normwise(a, b):
    return np.linalg.norm(a - b, axis=-1) / np.linalg.norm(b, axis=-1)


def linear(layer, name, x):
    packed, norms, cb = layer.host[name]
    rows = packed.shape[0]
    return oracle.sdot_linear(packed, norms, (rows, x.shape[1]), 4, 32, cb, x, 8)


def test_decode_layer_b64_against_oracle():
    seqs, L = 64, bench.DecodeLayer
    with Teardown() as td:
        stream = td.add(Stream())
        layer = L(seqs, td, stream)
        before = [layer.kv.read(0, s, L.CAP - 1) for s in (0, 37, 63)]
        layer.step()
        synchronize()
        got = {n: layer.download(n) for n in layer.widths}
        for w, xin, out in (("wq", "x", "q"), ("wk", "x", "k"), ("wv", "x", "v"), ("wo", "a", "o"),
                            ("wu", "o", "u"), ("wd", "u", "d")):
            np.testing.assert_array_equal(got[out], linear(layer, w, got[xin]), err_msg=f"{w}: {xin} -> {out}")
        shape = (seqs, L.KVH, L.HD)
        k8, ks = oracle.kv_quantize(got["k"].reshape(shape))
        v8, vs = oracle.kv_quantize(got["v"].reshape(shape))
        for s in range(seqs):
            keys, values, kscale, vscale = layer.kv.read(0, s, L.CAP)
            np.testing.assert_array_equal(keys[-1], k8[s], err_msg=f"seq {s}: new K row")
            np.testing.assert_array_equal(values[-1], v8[s], err_msg=f"seq {s}: new V row")
            np.testing.assert_array_equal(kscale[-1], ks[s])
            np.testing.assert_array_equal(vscale[-1], vs[s])
            qs, att = got["q"][s].reshape(L.HEADS, L.HD), got["a"][s].reshape(L.HEADS, L.HD)
            want = oracle.attention_i8(qs, keys, values, kscale, vscale)
            exact, vmax = fp64_attention(qs, keys, values, kscale, vscale)
            assert normwise(att, want).max() <= NORMWISE, f"seq {s}: attention vs oracle {normwise(att, want)}"
            assert normwise(att, exact).max() <= NORMWISE, f"seq {s}: attention vs fp64 {normwise(att, exact)}"
            per_value = (np.abs(att - exact) / vmax[:, None]).max()
            assert per_value <= PER_VALUE, f"seq {s}: attention vs fp64, {per_value:.2e} of max|v|"
        for s, old in zip((0, 37, 63), before):
            for a, b in zip(layer.kv.read(0, s, L.CAP - 1), old):
                np.testing.assert_array_equal(a, b, err_msg=f"seq {s}: older slots changed")


@pytest.mark.parametrize("seqs,splits,ks16", [(64, 0, "auto"), (20, 0, "auto"), (64, 2, "auto"), (64, 0, "never"),
                                              (64, 0, "w8"), (1, 0, "auto"), (1, 3, "auto"), (1, 1, "auto")])
def test_chained_step_equals_unchained(seqs, splits, ks16, monkeypatch):
    """Chained runs (fused epilogue preparation on 16- or 8-wave K splits, or the fallback prepare launches;
    at one sequence, with the attention's slot range split or not) give the unchained bits."""
    if ks16 == "w8":
        monkeypatch.setenv("NEEDLE2_GPU_INT8_KS16_WAVES", "8")
    elif ks16 != "auto":
        monkeypatch.setenv("NEEDLE2_GPU_INT8_KS16", ks16)
    with Teardown() as td:
        stream = td.add(Stream())
        layer = bench.DecodeLayer(seqs, td, stream)
        layer.splits = splits
        L, outs = bench.DecodeLayer, {}
        zk = np.zeros((1, L.KVH, L.HD), np.int8)
        zs = np.zeros((1, L.KVH), np.float32)
        for mode in ("unchained", "chained", "unchained"):
            for n in ("a", "o", "u", "d"):  # stale outputs would hide a missing write
                layer.buf[n].upload(np.full((seqs, layer.widths[n]), np.nan, np.float32))
            for s in range(seqs):  # and a stale new-token slot a missing store
                layer.kv.load(0, s, zk, zk, zs, zs, first_slot=L.CAP - 1)
            (layer.step if mode == "chained" else layer.unchained_step)()
            synchronize()
            got = {n: layer.download(n) for n in ("q", "k", "v", "a", "o", "u", "d")}
            for s in (0, seqs - 1):
                for i, part in enumerate(layer.kv.read(0, s, 1, first_slot=L.CAP - 1)):
                    got[f"cache{s}.{i}"] = part
            outs.setdefault(mode, []).append(got)
        for n in outs["chained"][0]:
            np.testing.assert_array_equal(outs["chained"][0][n], outs["unchained"][0][n], err_msg=n)
            np.testing.assert_array_equal(outs["unchained"][1][n], outs["unchained"][0][n], err_msg=n)


@pytest.mark.parametrize("seqs", [1, 64])
def test_prepared_run_without_a_producer_prepares_itself(seqs):
    """A run with prepared=True that no chained producer call preceded (or whose producer's input was used by
    an earlier run) prepares its own input: the unchained bits."""
    with Teardown() as td:
        stream = td.add(Stream())
        layer = bench.DecodeLayer(seqs, td, stream)
        layer.unchained_step()
        synchronize()
        want = layer.download("o")
        layer.buf["o"].upload(np.full((seqs, 512), np.nan, np.float32))
        layer.plans["o"].run(stream, prepared=True)
        synchronize()
        np.testing.assert_array_equal(layer.download("o"), want)
        layer.step()  # chained: o's staged input is used by this step's o run ...
        layer.buf["o"].upload(np.full((seqs, 512), np.nan, np.float32))
        layer.plans["o"].run(stream, prepared=True)  # ... so this run prepares again
        synchronize()
        np.testing.assert_array_equal(layer.download("o"), want)


def test_chained_run_refuses_a_plan_not_reading_the_output():
    with Teardown() as td:
        stream = td.add(Stream())
        layer = bench.DecodeLayer(4, td, stream)
        other = td.add(DeviceArray(4 * 512 * 4))
        stray = td.add(Plan([layer.mats["wu"]], [other], [layer.buf["u"]], batch=4, int8=True))
        with pytest.raises(GpuError, match="next plan's input"):
            layer.plans["o"].run(stream, prepared=False, next=stray)
        with pytest.raises(GpuError, match="next plan's input"):
            layer.attention(next=stray)
        with pytest.raises(GpuError, match="one-matrix"):
            layer.plans["o"].run(stream, next=layer.plans["qkv"])
