"""A decode step captured in a HIP graph (int8 Q|K|V plan, KV store from a
device slot table, decode attention, int8 O plan) replays bit-identically to
the same step run eagerly, replay after replay, with eager uploads and
synchronizations between the replays."""
import numpy as np
import pytest

from openneedle_amd.cq import CQMatrix, Plan
from openneedle_amd.device import DeviceArray, Graph, Stream, synchronize
from openneedle_amd.kv import KVCache
from tests.cases import activations, baseline

pytestmark = pytest.mark.gpu

SEQS, CAP, KVH, HD, HEADS, HIDDEN = 4, 64, 2, 64, 4, 128


def layer(seed):
    mats = []
    for i in range(4):
        packed, norms, cb, _ = baseline(4, HIDDEN, HIDDEN, seed=seed + i)
        mats.append(CQMatrix(packed, norms, (HIDDEN, HIDDEN), 4, 32, cb))
    return mats


def prefilled_cache(rng_seed, slots):
    kv = KVCache(1, CAP, KVH, HD, SEQS)
    rng = np.random.default_rng(rng_seed)
    k = DeviceArray.from_host(rng.normal(size=(SEQS, slots, KVH, HD)).astype(np.float32))
    v = DeviceArray.from_host(rng.normal(size=(SEQS, slots, KVH, HD)).astype(np.float32))
    kv.store(0, k.ptr, v.ptr, slots, first_slot=0)
    synchronize()
    return kv


class Step:
    """Buffers and plans of one decode step at slot `pos` for SEQS sequences."""

    def __init__(self, mats, kv, pos):
        self.kv, self.pos = kv, pos
        self.buf = {n: DeviceArray(SEQS * HIDDEN * 4) for n in "xqkvao"}
        self.first = DeviceArray.from_host(np.full(SEQS, pos, np.int32))
        b = self.buf
        self.qkv = Plan(mats[:3], [b["x"].ptr] * 3, [b["q"].ptr, b["k"].ptr, b["v"].ptr], batch=SEQS, int8=True)
        self.o = Plan(mats[3:], [b["a"].ptr], [b["o"].ptr], batch=SEQS, int8=True)

    def run(self, stream, device_slots):
        b = self.buf
        self.qkv.run(stream)
        if device_slots:
            self.kv.store_device(0, b["k"].ptr, b["v"].ptr, 1, self.first.ptr, stream=stream)
        else:
            self.kv.store(0, b["k"].ptr, b["v"].ptr, 1, first_slot=self.pos, stream=stream)
        self.kv.attention(0, b["q"].ptr, b["a"].ptr, HEADS, self.pos + 1, stream=stream)
        self.o.run(stream)

    def out(self):
        return self.buf["o"].download(np.empty((SEQS, HIDDEN), np.float32))


def test_decode_step_graph_replays_match_eager():
    mats = layer(900)
    pos = 40
    stream = Stream()
    graphed = Step(mats, prefilled_cache(5, pos), pos)
    eager = Step(mats, prefilled_cache(5, pos), pos)
    graphed.buf["x"].upload(activations((SEQS, HIDDEN), seed=1))
    graphed.run(stream, device_slots=True)  # eager warm-up: every buffer allocated before the capture
    stream.synchronize()
    with Graph.capture(stream) as g:
        graphed.run(stream, device_slots=True)
    for i in range(4):
        x = activations((SEQS, HIDDEN), seed=10 + i)
        graphed.buf["x"].upload(x)
        eager.buf["x"].upload(x)
        g.launch(stream)
        stream.synchronize()
        eager.run(stream, device_slots=False)
        stream.synchronize()
        np.testing.assert_array_equal(graphed.out(), eager.out())
        k_g = graphed.kv.read(0, 0, pos + 1)
        k_e = eager.kv.read(0, 0, pos + 1)
        for a, b in zip(k_g, k_e):
            np.testing.assert_array_equal(a, b)
