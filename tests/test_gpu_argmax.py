"""GPU argmax and the fused lm_head + argmax against the oracle's argmax, which
follows src/cuda/argmax.cu's candidate rules: the largest value, the lowest
index among equal maxima, NaN and -inf never win, 0xFFFFFFFF when nothing
wins. Integer results: bit-exact."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4, Q6 = 12, 14
SEED = 20261206


def workspace(qk):
    n = qk.argmax_workspace_size()
    ws = qk.DeviceBuffer(n)
    qk.check(qk.load().qk_memset_async(ws.ptr, 0, n, None))
    return ws, n


def run_argmax(qk, ws, n, values: np.ndarray) -> int:
    d = qk.DeviceBuffer.from_array(values.astype(np.float32))
    res = qk.DeviceBuffer(4)
    qk.argmax(d, values.size, res, ws, n)
    qk.synchronize()
    return int(res.download(np.uint32)[0])


@pytest.mark.parametrize("count", [1, 7, 1024, 1025, 65536 * 3 + 5, 151936, 1 << 22])
def test_argmax_random(gpu, oracle, count):
    ws, n = workspace(gpu)
    rng = np.random.default_rng(count)
    v = rng.standard_normal(count).astype(np.float32)
    for _ in range(2):  # the workspace is re-armed by every call
        assert run_argmax(gpu, ws, n, v) == oracle.argmax(v)
        v = -v


def test_argmax_workspace_check_reports_and_clears_a_timeout(gpu, oracle):
    """The collector's bounded wait, when it gives up, sets a word after the
    1024 partial slots (byte 8192) and writes an index without that partial;
    qk_argmax_workspace_check reports it once and clears the word and every
    slot (a late partial may have landed after the collector cleared its
    slot). Planted from the host here (no workgroup is made to stall); a
    stale slot planted with it must not reach the next call's index."""
    ws, n = workspace(gpu)
    gpu.argmax_workspace_check(ws)  # a zeroed workspace: nothing to report
    ws.upload(np.array([1], np.uint32), offset=8192)
    stale = np.zeros(2, np.uint64)
    stale[1] = np.uint64(0xFFFFFFFFFFFFFFF0)  # slot 1: a huge key left over from a late publisher
    ws.upload(stale, offset=0)
    with pytest.raises(gpu.QKError, match="argmax collector timed out"):
        gpu.argmax_workspace_check(ws)
    assert not np.any(ws.download(np.uint32))
    gpu.argmax_workspace_check(ws)
    v = np.random.default_rng(5).standard_normal(151936).astype(np.float32)
    assert run_argmax(gpu, ws, n, v) == oracle.argmax(v)
    gpu.argmax_workspace_check(ws)


def test_argmax_ties_nan_inf(gpu, oracle):
    ws, n = workspace(gpu)
    rng = np.random.default_rng(3)
    v = rng.integers(-5, 6, 300000).astype(np.float32)  # many exact ties
    assert run_argmax(gpu, ws, n, v) == oracle.argmax(v) == int(np.argmax(v))
    v = np.full(50000, -np.inf, np.float32)
    v[[7, 30000]] = np.nan
    assert run_argmax(gpu, ws, n, v) == oracle.argmax(v) == 0xFFFFFFFF
    v[40000] = -1e30
    v[45000] = np.nan
    assert run_argmax(gpu, ws, n, v) == 40000
    v = np.array([-0.0, 0.0, -1.0], np.float32)  # -0 == +0: the first wins
    assert run_argmax(gpu, ws, n, v) == oracle.argmax(v) == 0
    v = np.full(1000, 1.0, np.float32)
    v[999] = np.inf
    v[500] = np.inf
    assert run_argmax(gpu, ws, n, v) == 500


def test_argmax_validation(gpu):
    lib = gpu.load()
    ws, n = workspace(gpu)
    d = gpu.DeviceBuffer(64)
    res = gpu.DeviceBuffer(4)
    assert lib.qk_argmax(d.ptr, 0, res.ptr, ws.ptr, n, None) == 1
    assert lib.qk_argmax(d.ptr, 1 << 32, res.ptr, ws.ptr, n, None) == 1
    assert lib.qk_argmax(d.ptr, 4, res.ptr, ws.ptr, n - 8, None) == 1
    assert lib.qk_argmax(d.ptr, 4, None, ws.ptr, n, None) == 1


@pytest.mark.parametrize("qtype,K,N", [(Q6, 2560, 151936), (Q4, 2560, 9728), (Q6, 9728, 2560), (Q4, 256, 77)])
def test_matmul_argmax_matches_matmul_then_argmax(gpu, oracle, qtype, K, N):
    """The fused launch gives the matmul's logits and their argmax; its logits
    are within the bar of the oracle product, and its index is the oracle
    product's argmax whenever the top two are clearly apart (the full lm_head
    151936 x 2560 included)."""
    qk = gpu
    print(f"[case] type={qtype} K={K} N={N}", flush=True)
    w = qk.DeviceBuffer(N * qk.row_bytes(qtype, K))
    qk.synth_superblocks(w, qtype, N, K, SEED + N, 0.01 if qtype == Q4 else 0.005, 0.01)
    x = qk.DeviceBuffer(4 * K)
    qk.synth_normal(x, K, SEED + K)
    ws, n = workspace(qk)
    logits, ref_logits = qk.DeviceBuffer(4 * N), qk.DeviceBuffer(4 * N)
    res, res2 = qk.DeviceBuffer(4), qk.DeviceBuffer(4)
    qk.matmul(x, w, qtype, K, N, ref_logits, 1)
    qk.matmul_argmax(x, w, qtype, K, N, logits, res, ws, n)
    qk.matmul_argmax(x, w, qtype, K, N, None, res2, ws, n)  # logits not written
    qk.synchronize()
    print(f"[case] launch {qk.last_launch()}", flush=True)
    got = logits.download(np.float32)
    mm = ref_logits.download(np.float32)
    assert oracle.row_norm_error(got.reshape(1, N), mm.reshape(1, N).astype(np.float64)) <= 1e-6
    idx = int(res.download(np.uint32)[0])
    assert idx == oracle.argmax(got)
    assert int(res2.download(np.uint32)[0]) == idx
    ref = oracle.reference_product(x.download(np.float32), w.download(np.uint8), qtype, K, N)[0]
    assert oracle.row_norm_error(got.reshape(1, N), ref.reshape(1, N)) <= 1e-5
    top = np.sort(ref)[-2:]
    print(f"[case] oracle top two {top[1]:.6g} {top[0]:.6g}, fused index {idx}, oracle {int(np.argmax(ref))}")
    assert top[1] - top[0] > 1e-4 * abs(top[1])  # these seeds keep the top two 3-15% apart
    assert idx == int(np.argmax(ref))


def test_matmul_argmax_tie_goes_to_the_lower_row(gpu, oracle):
    """Two identical weight rows give identical logits; make them the maximum."""
    qk = gpu
    K, N = 2560, 4096
    rb = qk.row_bytes(Q6, K)
    w = qk.DeviceBuffer(N * rb)
    qk.synth_superblocks(w, Q6, N, K, SEED, 0.005, 0.01)
    x = qk.DeviceBuffer(4 * K)
    qk.synth_normal(x, K, SEED + 1)
    y = qk.DeviceBuffer(4 * N)
    qk.matmul(x, w, Q6, K, N, y, 1)
    qk.synchronize()
    j = int(np.argmax(y.download(np.float32)))
    i = 17 if j != 17 else 18
    host = w.download(np.uint8)
    host[i * rb:(i + 1) * rb] = host[j * rb:(j + 1) * rb]  # row i becomes a copy of the max row
    w.upload(host)
    lo = min(i, j)
    ws, n = workspace(qk)
    res = qk.DeviceBuffer(4)
    qk.matmul_argmax(x, w, Q6, K, N, None, res, ws, n)
    qk.synchronize()
    assert int(res.download(np.uint32)[0]) == lo
