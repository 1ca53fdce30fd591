"""qk_matmul_noalloc (the prefill workspace in the library's file-scope device
scratch, nothing allocated) against qk_matmul through the C-ABI: two calls in
a row on the same scratch, the second with a smaller input, each bit-identical
to qk_matmul (same kernels, same workspace layout) and within the oracle's
bar; the M <= 8 path; a shape whose workspace exceeds the scratch is rejected."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4, Q6 = 12, 14
SEED = 20261230


def _weight(qk, qtype, N, K, seed):
    w = qk.DeviceBuffer(N * qk.row_bytes(qtype, K))
    qk.synth_superblocks(w, qtype, N, K, seed, 0.01 if qtype == Q4 else 0.005, 0.01)
    return w


@pytest.mark.parametrize("first,second", [
    ((Q6, 9728, 2560, 512), (Q4, 2560, 1000, 77)),   # ffn_down at M = 512 (split K), then smaller
    ((Q4, 2560, 9728, 300), (Q6, 2560, 1024, 9)),
])
def test_noalloc_matches_matmul_on_consecutive_calls(gpu, oracle, first, second):
    lib = gpu.load()
    for qtype, K, N, M in (first, second):
        print(f"[case] noalloc type={qtype} K={K} N={N} M={M}", flush=True)
        assert gpu.matmul_workspace_size(qtype, K, N, M) <= (48 << 20)
        w = _weight(gpu, qtype, N, K, SEED + N)
        x = oracle.synth_normal(M * K, SEED + M)
        xd = gpu.DeviceBuffer.from_array(x)
        y_ref = gpu.DeviceBuffer(4 * M * N)
        y = gpu.DeviceBuffer.from_array(np.full(M * N, np.nan, np.float32))
        gpu.matmul(xd, w, qtype, K, N, y_ref, M)
        status = lib.qk_matmul_noalloc(xd.ptr, w.ptr, qtype, K, N, y.ptr, M, None)
        assert status == 0, lib.qk_last_error()
        gpu.synchronize()
        got, ref = y.download(np.float32), y_ref.download(np.float32)
        assert np.array_equal(got, ref)
        if M * N <= 1 << 20:
            exact = oracle.reference_product(x, w.download(np.uint8), qtype, K, N)
            assert oracle.row_norm_error(got.reshape(M, N), exact) <= 1e-5


def test_noalloc_decode_rows_and_limit(gpu, oracle):
    lib = gpu.load()
    K, N, M = 2560, 4096, 4  # the mat-vec: no workspace at all
    w = _weight(gpu, Q4, N, K, SEED)
    x = gpu.DeviceBuffer.from_array(oracle.synth_normal(M * K, SEED + 1))
    y_ref, y = gpu.DeviceBuffer(4 * M * N), gpu.DeviceBuffer(4 * M * N)
    gpu.matmul(x, w, Q4, K, N, y_ref, M)
    assert lib.qk_matmul_noalloc(x.ptr, w.ptr, Q4, K, N, y.ptr, M, None) == 0
    gpu.synchronize()
    assert np.array_equal(y.download(np.float32), y_ref.download(np.float32))
    # 2048 x 9728 activations need ~80 MB of planes: rejected before any launch
    assert gpu.matmul_workspace_size(Q6, 9728, 2560, 2048) > (48 << 20)
    assert lib.qk_matmul_noalloc(x.ptr, w.ptr, Q6, 9728, 2560, y.ptr, 2048, None) == 1
    assert b"scratch" in lib.qk_last_error()
