"""GPU parity of qk_ffn, the FFN block of src/Engine.cpp:97-101 (rms_norm of
ffn_norm, gate, up, silu_multiply, down), against the CPU oracle and against
the same block run as separate launches.

At M = 1 with Q4_K gate/up the block is one launch with a grid barrier
between the gate/up phase and the down phase. Bars: h within 1e-5 of the
oracle's double-accumulated SiLU(gate) * up (row-norm error), y within 1e-5 of
the oracle's reference product of the GPU's own h (the down product proper),
and y within the path's 1e-3 of the oracle chain (a last-bit difference in h
can move one Q8 code of the round trip). Since the fused launch runs the same
row partition and the same fixed-order sums as the separate launches, both
outputs are also bit-identical to qk_ffn_gate_up(_norm) + qk_matmul.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4, Q6 = 12, 14
SEED = 20261240
DMAX = {Q4: 0.01, Q6: 0.005}


def _weight(qk, qtype, N, K, seed):
    w = qk.DeviceBuffer(N * qk.row_bytes(qtype, K))
    qk.synth_superblocks(w, qtype, N, K, seed, DMAX[qtype], 0.01)
    return w


def _workspace(qk):
    n = qk.ffn_workspace_size()
    ws = qk.DeviceBuffer(n)
    qk.check(qk.load().qk_memset_async(ws.ptr, 0, n, None))
    return ws, n


class Block:
    def __init__(self, qk, oracle, K, N, down_type, M, norm, seed):
        self.qk, self.K, self.N, self.down_type, self.M = qk, K, N, down_type, M
        self.gate = _weight(qk, Q4, N, K, seed)
        self.up = _weight(qk, Q4, N, K, seed + 1)
        self.down = _weight(qk, down_type, K, N, seed + 2)
        x = oracle.synth_normal(M * K, seed + 3) * np.float32(3.0)
        self.x = x.astype(np.float32)
        self.scale = None
        if norm:
            self.scale = (np.float32(1.0) + np.float32(0.3) * oracle.synth_normal(K, seed + 4)).astype(np.float32)
        self.xd = qk.DeviceBuffer.from_array(self.x)
        self.sd = qk.DeviceBuffer.from_array(self.scale) if norm else None
        self.eps = 1e-6

    def run(self, ws, nbytes, stream=None):
        qk = self.qk
        h = qk.DeviceBuffer.from_array(np.full(self.M * self.N, np.nan, np.float32))
        y = qk.DeviceBuffer.from_array(np.full(self.M * self.K, np.nan, np.float32))
        qk.ffn(self.xd, self.sd, self.eps, self.gate, self.up, Q4, self.down, self.down_type, self.K,
               self.N, h, y, self.M, ws, nbytes, stream)
        launch = qk.last_launch()
        qk.synchronize(stream)
        return (h.download(np.float32).reshape(self.M, self.N), y.download(np.float32).reshape(self.M, self.K),
                launch)

    def separate(self):
        """The same block as separate launches (qk_ffn_gate_up(_norm), qk_matmul)."""
        qk = self.qk
        h = qk.DeviceBuffer(4 * self.M * self.N)
        y = qk.DeviceBuffer(4 * self.M * self.K)
        if self.sd is not None:
            qk.ffn_gate_up_norm(self.xd, self.sd, self.eps, self.gate, self.up, Q4, self.K, self.N, h, self.M)
        else:
            qk.ffn_gate_up(self.xd, self.gate, self.up, Q4, self.K, self.N, h, self.M)
        qk.matmul(h, self.down, self.down_type, self.N, self.K, y, self.M)
        qk.synchronize()
        return h.download(np.float32).reshape(self.M, self.N), y.download(np.float32).reshape(self.M, self.K)

    def oracle_h(self, oracle):
        xn = oracle.rms_norm(self.x, self.scale, self.K, self.eps) if self.scale is not None else self.x
        g = oracle.reference_product(xn, self.gate.download(np.uint8), Q4, self.K, self.N)
        u = oracle.reference_product(xn, self.up.download(np.uint8), Q4, self.K, self.N)
        with np.errstate(over="ignore"):  # exp(-g) overflows to inf for very negative g: SiLU -> -0
            return (g / (1.0 + np.exp(-g))) * u

    def check(self, oracle, h, y):
        h_ref = self.oracle_h(oracle)
        err_h = oracle.row_norm_error(h, h_ref)
        down = self.down.download(np.uint8)
        y_own = oracle.reference_product(h, down, self.down_type, self.N, self.K)
        y_chain = oracle.reference_product(h_ref.astype(np.float32), down, self.down_type, self.N, self.K)
        err_y, err_chain = oracle.row_norm_error(y, y_own), oracle.row_norm_error(y, y_chain)
        rate = oracle.approx_pass_rate(y, y_own)
        print(f"h error {err_h:.3e}; y error vs oracle(h) {err_y:.3e} (Approx {rate:.5f}), vs oracle chain "
              f"{err_chain:.3e}", flush=True)
        assert err_h <= 1e-5
        assert err_y <= 1e-5 and rate >= 0.999
        assert err_chain <= 1e-3


@pytest.mark.parametrize("down_type,norm", [(Q6, False), (Q6, True), (Q4, False), (Q4, True)])
def test_ffn_block_qwen3_shape_one_launch(gpu, oracle, down_type, norm):
    """Qwen3-4B FFN at M = 1: gate/up Q4_K 9728 x 2560, down 2560 x 9728."""
    K, N = 2560, 9728
    blk = Block(gpu, oracle, K, N, down_type, 1, norm, SEED + 10 * down_type + norm)
    ws, nbytes = _workspace(gpu)
    h, y, launch = blk.run(ws, nbytes)
    print(f"[case] ffn K={K} N={N} down={down_type} norm={norm} launch {launch}", flush=True)
    assert launch.startswith("ffn_fused_kernel")
    blk.check(oracle, h, y)
    hs, ys = blk.separate()
    assert np.array_equal(h, hs) and np.array_equal(y, ys)
    for _ in range(3):  # the barrier workspace is re-armed by every call
        h2, y2, _ = blk.run(ws, nbytes)
        assert np.array_equal(h2, h) and np.array_equal(y2, y)
    gpu.ffn_workspace_check(ws)


def test_ffn_workspace_check_reports_and_clears_a_timeout(gpu, oracle):
    """The grid barrier's bounded wait, when it gives up, sets a word in the
    workspace (byte 256: the second 256-byte line) and lets the launch end;
    qk_ffn_workspace_check reports it as QK_ERR_RUNTIME once and clears it.
    The word is planted from the host here (no kernel is made to time out),
    then a real launch on the same workspace runs clean and matches."""
    ws, nbytes = _workspace(gpu)
    gpu.ffn_workspace_check(ws)  # a zeroed workspace: nothing to report
    ws.upload(np.array([1], np.uint32), offset=256)
    with pytest.raises(gpu.QKError, match="grid barrier timed out"):
        gpu.ffn_workspace_check(ws)
    assert int(ws.download(np.uint32, 1, offset=256)[0]) == 0
    gpu.ffn_workspace_check(ws)  # cleared by the report
    blk = Block(gpu, oracle, 512, 1024, Q6, 1, True, SEED + 7)
    h, y, launch = blk.run(ws, nbytes)
    print(f"[case] ffn after a planted timeout word: launch {launch}", flush=True)
    assert launch.startswith("ffn_fused_kernel")
    hs, ys = blk.separate()
    assert np.array_equal(h, hs) and np.array_equal(y, ys)
    gpu.ffn_workspace_check(ws)


def test_ffn_one_workspace_across_shapes_and_row_counts(gpu, oracle):
    """One workspace shared by interleaved calls the way an engine may share
    it: the Qwen3 block at M = 1 (the grid barrier's words), another shape at
    M = 1 (the same words, another grid plan), the batched block at M = 8 (its
    Q8(h) and block counters) and again M = 1, twice round. Every call equals
    its separate-launch form bit for bit, the barrier never times out, and
    the batched block's counters are zero after each call."""
    ws, nbytes = _workspace(gpu)
    blocks = [Block(gpu, oracle, 2560, 9728, Q6, 1, False, SEED + 901),
              Block(gpu, oracle, 1024, 3072, Q6, 1, True, SEED + 902),
              Block(gpu, oracle, 2560, 9728, Q6, 8, True, SEED + 903),
              Block(gpu, oracle, 2048, 6144, Q4, 1, False, SEED + 904)]
    expected = [blk.separate() for blk in blocks]
    arrive_off = nbytes - 8 * 1024
    for rnd in range(2):
        for i, blk in enumerate(blocks):
            h, y, launch = blk.run(ws, nbytes)
            print(f"[case] shared workspace round {rnd} block {i} (K={blk.K} N={blk.N} M={blk.M}): {launch}",
                  flush=True)
            assert np.array_equal(h, expected[i][0]) and np.array_equal(y, expected[i][1]), (rnd, i)
            raw = ws.download(np.uint8)
            assert not raw[arrive_off:arrive_off + 4 * (blk.N // 32)].any(), (rnd, i)
    gpu.ffn_workspace_check(ws)


@pytest.mark.parametrize("K,N,down_type", [(1024, 3072, Q6), (2048, 6144, Q4), (512, 1024, Q6)])
def test_ffn_block_other_shapes_one_launch(gpu, oracle, K, N, down_type):
    blk = Block(gpu, oracle, K, N, down_type, 1, True, SEED + K + N)
    ws, nbytes = _workspace(gpu)
    h, y, launch = blk.run(ws, nbytes)
    print(f"[case] ffn K={K} N={N} down={down_type} launch {launch}", flush=True)
    assert launch.startswith("ffn_fused_kernel")
    blk.check(oracle, h, y)
    hs, ys = blk.separate()
    assert np.array_equal(h, hs) and np.array_equal(y, ys)
    gpu.ffn_workspace_check(ws)


@pytest.mark.parametrize("M,norm,down_type", [(2, True, Q6), (8, False, Q6), (8, True, Q4), (5, True, Q6),
                                               (12, True, Q6)])
def test_ffn_block_batched_rows_take_separate_launches(gpu, oracle, M, norm, down_type):
    """M = 2..8: norm and Q8(h) in the workspace, h quantised once, the down
    mat-vec on Q8 blocks; bit-identical to gate/up + qk_matmul (the same Q8
    codes, row partitions and summation order). M > 8: the prefill path."""
    K, N = 2560, 9728
    blk = Block(gpu, oracle, K, N, down_type, M, norm, SEED + 100 + M + down_type)
    ws, nbytes = _workspace(gpu)
    h, y, launch = blk.run(ws, nbytes)
    print(f"[case] ffn M={M} down={down_type} norm={norm} launch {launch}", flush=True)
    assert not launch.startswith("ffn_fused_kernel")
    if M <= 8:
        blk.check(oracle, h, y)
        hs, ys = blk.separate()
        assert np.array_equal(h, hs) and np.array_equal(y, ys)
    else:  # the prefill GEMM's fp16 split products: within the path's bar
        h_ref = blk.oracle_h(oracle)
        assert oracle.row_norm_error(h, h_ref) <= 1e-5
        y_own = oracle.reference_product(h, blk.down.download(np.uint8), Q6, N, K)
        assert oracle.row_norm_error(y, y_own) <= 1e-5


@pytest.mark.parametrize("M,K,N", [(8, 2560, 9728), (3, 2560, 9728), (8, 1024, 3072)])
def test_ffn_block_batched_q8h_from_gate_up_launch(gpu, oracle, M, K, N):
    """M = 2..8: Q8(h) in the workspace (formed in the gate/up launch by the
    workgroup that completes each 32-value block) equals qk_quantize_q8 of the
    call's own h bit for bit, and every block arrival counter is zero again
    after each call (three calls on one workspace). Workspace layout, as
    qk_ffn_workspace_size documents it: barrier words, Q8(h) 160 KiB, norm rows
    512 KiB, arrival counters 8 KiB."""
    blk = Block(gpu, oracle, K, N, Q6, M, True, SEED + 500 + M + N)
    ws, nbytes = _workspace(gpu)
    q8_off = nbytes - (160 + 512 + 8) * 1024
    arrive_off = nbytes - 8 * 1024
    nq = M * N // 32 * gpu.Q8_BLOCK_BYTES
    for rep in range(3):
        h, y, launch = blk.run(ws, nbytes)
        raw = ws.download(np.uint8)
        hd = gpu.DeviceBuffer.from_array(h.reshape(-1))
        q8 = gpu.DeviceBuffer(nq)
        gpu.quantize_q8(hd, M, N, q8)
        gpu.synchronize()
        assert np.array_equal(raw[q8_off:q8_off + nq], q8.download(np.uint8)), f"call {rep}"
        assert not raw[arrive_off:arrive_off + 4 * (N // 32)].any(), f"call {rep}: counters left set"
    blk.check(oracle, h, y)


@pytest.mark.parametrize("M", [1, 8])
def test_ffn_block_graph_replays(gpu, oracle, M):
    """The block captured in a graph (M = 1: the one launch; M = 8: norm,
    gate/up, Q8(h) and down through the workspace), replayed with eager calls
    and synchronisations in between: every replay equals the eager result."""
    qk = gpu
    K, N = 2560, 9728
    blk = Block(qk, oracle, K, N, Q6, M, True, SEED + 300 + M)
    ws, nbytes = _workspace(qk)
    stream = qk.Stream()
    h = qk.DeviceBuffer(4 * M * N)
    y = qk.DeviceBuffer(4 * M * K)

    def record():
        qk.ffn(blk.xd, blk.sd, blk.eps, blk.gate, blk.up, Q4, blk.down, Q6, K, N, h, y, M, ws, nbytes, stream)

    record()
    stream.synchronize()
    eager = (h.download(np.float32), y.download(np.float32))
    graph = qk.Graph.capture(stream, lambda: [record() for _ in range(3)])
    for rep in range(4):
        y.upload(np.full(M * K, np.nan, np.float32))
        h.upload(np.full(M * N, np.nan, np.float32))
        graph.launch(stream)
        stream.synchronize()
        assert np.array_equal(h.download(np.float32), eager[0]), f"replay {rep}"
        assert np.array_equal(y.download(np.float32), eager[1]), f"replay {rep}"
        record()
        stream.synchronize()
    graph.destroy()
    qk.ffn_workspace_check(ws, stream)
    stream.destroy()


def test_ffn_block_validation(gpu):
    lib = gpu.load()
    ws, nbytes = _workspace(gpu)
    d = gpu.DeviceBuffer(1 << 16)
    args = [d.ptr, None, 0.0, d.ptr, d.ptr, Q4, d.ptr, Q6, 2560, 9728, d.ptr, d.ptr, 1]
    assert lib.qk_ffn(*args, ws.ptr, nbytes - 256, None) == 1          # workspace too small
    assert lib.qk_ffn(*args, ws.ptr + 16, nbytes, None) == 1           # misaligned workspace
    bad = list(args)
    bad[1], bad[2] = d.ptr, 0.0                                        # norm without a positive eps
    assert lib.qk_ffn(*bad, ws.ptr, nbytes, None) == 1
    bad = list(args)
    bad[7] = 13                                                        # Q5_K down
    assert lib.qk_ffn(*bad, ws.ptr, nbytes, None) == 2
    bad = list(args)
    bad[12] = 0                                                        # no rows: nothing to do
    assert lib.qk_ffn(*bad, ws.ptr, nbytes, None) == 0
