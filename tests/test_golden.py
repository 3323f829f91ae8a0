"""The committed golden fixtures (tests/golden/golden.npz) against the CPU oracle.

The fixtures freeze the oracle's outputs on small seeded inputs
(tests/golden/make_golden.py) plus the two known answers the reference's
examples state (rusty-loader/examples/load_and_run.rs:18-34,
rusty-backend/examples/ops_test.rs:13-17).  The oracle must reproduce every
array bit for bit, so a change to oracle/oracle.c that moves any result is
caught against fixed bytes; tests/test_gpu_golden.py holds the device path to
the same bytes.
"""
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden" / "golden.npz"


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_known_answers_are_the_references(gold):
    # load_and_run.rs:18-34: the f32 tensor [1,2,3,4] dequantized into 4 elements
    assert gold["dq_ka_words"].tolist() == [0x3F800000, 0x40000000, 0x40400000, 0x40800000]
    assert gold["dq_ka_out"].tolist() == [0.0, 0.0, 128.0, 63.0]
    # ops_test.rs:13-17: [[1,2],[3,4]] . I
    assert gold["mm_ka_a"].tolist() == [[1, 2], [3, 4]] and gold["mm_ka_out"].ravel().tolist() == [1, 2, 3, 4]


def test_oracle_reproduces_every_fixture(gold):
    import importlib.util

    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN.parent / "make_golden.py")
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    fresh = mg.cases()
    assert sorted(fresh) == sorted(gold)
    for k, v in gold.items():
        f = fresh[k]
        assert f.dtype == v.dtype and f.shape == v.shape, k
        # bytes, so NaN sentinels and signed zeros compare exactly
        assert f.tobytes() == v.tobytes(), f"oracle output {k} moved from the committed fixture"


def test_fixture_invariants(gold):
    # independent of the oracle: the dequantized bytes are the code bytes;
    # the fused and unfused affine forms differ only by the rounding of u*s
    # (at most one ulp of the product) plus the final rounding
    words, out = gold["dq_words"], gold["dq_out"]
    assert np.array_equal(out, words.view(np.uint8)[:150].astype(np.float32))
    prod = gold["af_u"].ravel().astype(np.float32) * np.repeat(gold["af_s"], 64)[:300]
    diff = np.abs(gold["af_out"].astype(np.float64) - gold["af_out_fma"])
    assert np.all(diff <= np.spacing(np.abs(prod)) + np.spacing(np.abs(gold["af_out"])))
    assert not np.array_equal(gold["af_out"], gold["af_out_fma"]), "the two roundings must be told apart"
    # the matmul fixtures agree with an f64 product to f32 accuracy
    for key, want in (("mm_out", gold["mm_a"].astype(np.float64) @ gold["mm_b"]),
                      ("mmbt_out", gold["mm_a"].astype(np.float64) @ gold["mmbt_b"].T),
                      ("mmat_out", gold["mmat_a"].astype(np.float64).T @ gold["mm_b"])):
        assert np.allclose(gold[key], want, rtol=1e-5, atol=1e-5), key
