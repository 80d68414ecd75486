"""One-shot device upload of a .cact archive (released geometry and precision map, random contents): every CQ
matrix becomes a device handle built from the mapped file's views, with results bit-identical to the oracle on
the record's own packed codes and norms."""
import numpy as np
import pytest

import oracle
from openneedle_amd import archive as A
from tests.cases import activations, official_like_archive

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    path = tmp_path_factory.mktemp("cact") / "model.cact"
    path.write_bytes(official_like_archive(seed=4))
    return A.DeviceModel(A.Archive.load(path), int8=True)


def test_everything_uploaded(model):
    a = model.archive
    assert len(model.matrices) == 145 and len(model.dense) == 259
    cq = [t for t in a.tensors.values() if t.dtype == A.CQ]
    span = max(t.offset + len(t.blob) for t in cq) - min(t.offset for t in cq)  # one copy covers every CQ payload
    assert model.uploaded_bytes == span + 364279 * 4
    for name, t in a.tensors.items():
        if t.dtype == A.CQ:
            assert model.matrices[name]._int8  # int8 twins built from the same device copy
    assert set(model.matrices) == {n for n, t in a.tensors.items() if t.dtype == A.CQ}


@pytest.mark.parametrize("name", ["embedding", "layer00.q_proj", "layer26.k_proj", "layer13.out_proj",
                                  "mhc_phi_res", "engram1.tables", "engram0.value_proj"])
def test_matrices_bit_exact(model, name):
    t = model.archive.tensors[name]
    q = model.matrices[name]
    x = activations((2, t.shape[1]), seed=len(name))
    expected = oracle.cq_linear(t.packed, t.norms, t.shape, t.bits, t.group_size, t.codebook, x, 8)
    np.testing.assert_array_equal(q.matvec(x), expected)
    np.testing.assert_array_equal(q.matvec_int8(x), oracle.sdot_linear(t.packed, t.norms, t.shape, t.bits,
                                                                       t.group_size, t.codebook, x, 8))


def test_lm_head_candidates_from_archive(model):
    """The tied embedding as the LM head: candidate rows equal the full projection's rows."""
    q = model.matrices["embedding"]
    x = activations(512, seed=8)
    ids = np.random.default_rng(2).permutation(8192)[:142].astype(np.int32)
    np.testing.assert_array_equal(q.select(x, ids), q.matvec(x)[ids])


def test_dense_tensors_uploaded(model):
    for name in ("layer05.norm_in", "mhc_b_res", "final_norm", "contrastive_head.proj"):
        t = model.archive.tensors[name]
        got = model.dense[name].download(np.empty(t.shape, np.float32))
        np.testing.assert_array_equal(got, t.dequantize())
