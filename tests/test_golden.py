"""The committed fixtures of tests/golden/ (written by make_golden.py from
closed forms: weights packed in ggml's layout from chosen scales and codes,
the Q8 round trip and double products in numpy) pin the CPU oracle: its
dequantisers, Q8 quantiser and reference product must reproduce them."""
from __future__ import annotations

import pathlib
import sys

import numpy as np
import pytest

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
Q4, Q6 = 12, 14


@pytest.fixture(scope="module")
def fixture():
    with np.load(GOLDEN / "q4k_q6k_small.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_generator_reproduces_the_committed_file(fixture):
    """The file is what make_golden.py writes (nothing hand-edited)."""
    sys.path.insert(0, str(GOLDEN))
    import make_golden  # noqa: E402

    built = make_golden.build()
    assert set(built) == set(fixture)
    for k, v in built.items():
        assert np.array_equal(np.asarray(v), fixture[k]), k


@pytest.mark.parametrize("qtype,key", [(Q4, "q4k"), (Q6, "q6k")])
def test_oracle_dequant_matches_fixture_bitwise(oracle, fixture, qtype, key):
    K = int(fixture["K"])
    packed = fixture[key]
    want = fixture[key + "_w"]
    got = oracle.dequantize(packed.ravel(), qtype, packed.shape[0], K).reshape(want.shape)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_fixture_closed_forms(fixture):
    """Spot values the packers' inputs fix: Q4_K row 0 is w = q (0..15), row 1
    w = -m with m = sub-block index, row 3 (d = dmin = 0) zeros; Q6_K rows 0
    and 1 are -32 and 31 everywhere, row 4 (d = 0) zeros."""
    w4, w6 = fixture["q4k_w"], fixture["q6k_w"]
    assert np.all((w4[0] == np.round(w4[0])) & (w4[0] >= 0) & (w4[0] <= 15))
    assert np.array_equal(w4[1], -np.tile(np.repeat(np.arange(8), 32), 2).astype(np.float32))
    assert not np.any(w4[3]) and not np.any(w6[4])
    assert np.all(w6[0] == -32) and np.all(w6[1] == 31)
    assert np.all(w4[2] == np.round(w4[2] * 2.0 ** 24) / 2.0 ** 24)  # multiples of 2^-24


def test_oracle_q8_matches_fixture(oracle, fixture):
    x = fixture["x"]
    codes, scales = oracle.quantize_q8(x)
    assert np.array_equal(codes, fixture["x_codes"].ravel())
    assert np.array_equal(scales.view(np.uint32), fixture["x_scales"].ravel().view(np.uint32))
    rt = oracle.q8_roundtrip(x)
    assert np.array_equal(rt.view(np.uint32), fixture["x_rt"].view(np.uint32))
    assert not np.any(fixture["x_codes"][2, 32:64])  # the all-zero block


@pytest.mark.parametrize("qtype,key", [(Q4, "q4k"), (Q6, "q6k")])
def test_oracle_product_matches_fixture(oracle, fixture, qtype, key):
    K = int(fixture["K"])
    packed = fixture[key]
    want = fixture["y_" + key]
    got = oracle.reference_product(fixture["x"], packed.ravel(), qtype, K, packed.shape[0])
    scale = np.maximum(np.abs(want).max(axis=1, keepdims=True), 1e-300)
    assert np.all(np.abs(got - want) <= 1e-12 * scale)  # double sums in another order
