"""The HIP path against the committed fixtures of tests/golden/ (closed-form
weights in ggml's layout, the formula of the reference's make_input, double
products): dequantisation bit for bit, the Q8 quantiser's codes and scales,
and the product through the mat-vec (M = 1), batched (M = 3) and prefill
(M = 12) kernels within the bars of the other parity tests."""
from __future__ import annotations

import pathlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
Q4, Q6 = 12, 14


@pytest.fixture(scope="module")
def fixture():
    with np.load(GOLDEN / "q4k_q6k_small.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("qtype,key", [(Q4, "q4k"), (Q6, "q6k")])
def test_dequant_matches_fixture_bitwise(gpu, fixture, qtype, key):
    K = int(fixture["K"])
    packed, want = fixture[key], fixture[key + "_w"]
    src = gpu.DeviceBuffer.from_array(packed)
    out = gpu.DeviceBuffer.from_array(np.full(want.size, np.nan, np.float32))
    gpu.dequantize_rows(src, out, packed.shape[0], K, packed.shape[1], qtype)
    gpu.synchronize()
    got = out.download(np.float32).reshape(want.shape)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_quantize_matches_fixture(gpu, fixture):
    x = fixture["x"]
    M, K = x.shape
    q8 = gpu.DeviceBuffer(M * K // 32 * gpu.Q8_BLOCK_BYTES)
    gpu.quantize_q8(gpu.DeviceBuffer.from_array(x), M, K, q8)
    gpu.synchronize()
    blocks = q8.download(np.uint8).view(gpu.Q8_DTYPE)
    assert np.array_equal(blocks["codes"].ravel(), fixture["x_codes"].ravel())
    assert np.array_equal(blocks["scale"].view(np.uint32), fixture["x_scales"].ravel().view(np.uint32))


@pytest.mark.parametrize("qtype,key", [(Q4, "q4k"), (Q6, "q6k")])
@pytest.mark.parametrize("M", [1, 3, 12])
def test_matmul_matches_fixture(gpu, oracle, fixture, qtype, key, M):
    K = int(fixture["K"])
    packed = fixture[key]
    N = packed.shape[0]
    reps = -(-M // 3)
    x = np.tile(fixture["x"], (reps, 1))[:M]
    want = np.tile(fixture["y_" + key], (reps, 1))[:M]
    w = gpu.DeviceBuffer.from_array(packed)
    y = gpu.DeviceBuffer.from_array(np.full(M * N, np.nan, np.float32))
    gpu.matmul(gpu.DeviceBuffer.from_array(x), w, qtype, K, N, y, M)
    gpu.synchronize()
    got = y.download(np.float32).reshape(M, N)
    print(f"[case] golden {key} M={M} launch {gpu.last_launch()}", flush=True)
    err = oracle.row_norm_error(got, want)
    assert err <= 1e-5
    assert oracle.approx_pass_rate(got, want) >= (0.999 if M <= 8 else 0.99)
    zero_rows = [n for n in range(N) if not np.any(fixture[key + "_w"][n])]
    assert zero_rows and all(np.all(got[:, n] == 0.0) for n in zero_rows)  # d = 0: exact zeros
