"""Write the golden vectors in this directory from the reference itself.

The reference's C++ (needle2/csrc/cq.cpp with sdot.cpp and engine.cpp) is
compiled from its own sources by oracle/Makefile into oracle/_ref/libref.so;
this script feeds it small seeded inputs and stores inputs and outputs as
.npz files (no pickles). Run from the repository root:

    make -C oracle && python tests/golden/make_golden.py

The fixtures are data only: tests/test_golden.py replays them against the
oracle (CPU) and tests/test_golden_gpu.py against the HIP library.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle  # noqa: E402
from tests.cases import activations, baseline, example  # noqa: E402

SEED = 20261201


def save(name, **arrays):
    np.savez_compressed(HERE / f"{name}.npz", **arrays)
    print(f"wrote {name}.npz ({', '.join(f'{k}{list(v.shape)}' for k, v in arrays.items())})")


def cq_cases():
    # every storage width, a small and a large group, ragged input width
    for bits in (2, 3, 4, 5):
        for group in (16, 128):
            packed, norms, cb, _ = example(bits, rows=33, dim=200, group=group, seed=SEED + bits * 10 + group)
            x = activations((3, 200), seed=SEED + group)
            ref = oracle.RefCQ(packed, norms, (33, 200), bits, group, cb)
            ids = np.array([0, 32, 7, 7], np.int64)
            save(f"cq_b{bits}_g{group}", packed=packed, norms=norms.view(np.uint16), cb=cb, x=x,
                 shape=np.array([33, 200, bits, group], np.int32), y=ref.linear(x), ids=ids, rows=ref.rows(ids))
    # the single-token decode GEMV: CQ4 2048 x 512 g32, integer codebook
    packed, norms, cb, _ = baseline(4, 2048, 512, seed=SEED)
    x = activations(512, seed=SEED + 1)
    ref = oracle.RefCQ(packed, norms, (2048, 512), 4, 32, cb)
    save("cq4_decode_2048x512_g32", packed=packed, norms=norms.view(np.uint16), cb=cb, x=x,
         shape=np.array([2048, 512, 4, 32], np.int32), y=ref.linear(x))


def sdot_cases():
    # the reference's int8 path (scalar branches; its ABI accepts g >= 64)
    for bits, group in ((4, 64), (4, 128), (2, 64), (2, 256)):
        packed, norms, cb, _ = example(bits, rows=40, dim=300, group=group, seed=SEED + 7 * bits + group)
        ref = oracle.RefCQ(packed, norms, (40, 300), bits, group, cb)
        x = activations((2, 300), seed=SEED + 3 * group)
        q0, s0 = ref.sdot_prepare(x[0])
        cent, cs, ns = ref.sdot_tables()
        save(f"sdot_b{bits}_g{group}", packed=packed, norms=norms.view(np.uint16), cb=cb, x=x,
             shape=np.array([40, 300, bits, group], np.int32), y=ref.sdot_linear(x), q0=q0, xs0=s0,
             centroids=cent, centroid_scale=np.array([cs], np.float32), norm_scales=ns)


def attention_cases():
    for heads, kvh, hd, length in ((8, 8, 64, 300), (8, 2, 32, 65)):
        rng = np.random.default_rng(SEED + length)
        k = rng.normal(size=(length, kvh * hd)).astype(np.float32)
        v = rng.normal(size=(length, kvh * hd)).astype(np.float32)
        ref = oracle.RefAttention(heads, kvh, hd, length + 8)
        ref.load(k, v)
        rk, rv, rks, rvs = ref.cache()
        q = activations((heads, hd), seed=SEED + hd)
        save(f"attn_h{heads}_kv{kvh}_hd{hd}_n{length}", k=k.reshape(length, kvh, hd), v=v.reshape(length, kvh, hd),
             k8=rk, v8=rv, k_scales=rks, v_scales=rvs, q=q, out=ref.attend(q))


if __name__ == "__main__":
    oracle.build()
    if oracle.ref() is None:
        sys.exit("oracle/_ref/libref.so is missing: build it from the reference sources (make -C oracle)")
    cq_cases()
    sdot_cases()
    attention_cases()
