"""GPU parity of the prefill path (M > 8 activation rows: an MFMA GEMM whose
weight operands are built from the superblocks in registers) against the CPU
oracle, through the C-ABI.

Bar (the path's stated tolerance): max |y - y_ref| / ||y_ref[m,:]||_2 <= 1e-3 against
the oracle's product of the Q8 round trip of x with the fp32 dequantised
weights (src/tests/reference/MatmulReference.hpp:42-64). At full Qwen3 sizes
the double-precision reference is numpy's float64 product of the oracle's
dequantised weights and Q8 round trip, the same sums in another order.
The GEMM splits the activations' Q8 round trip into fp16 hi + lo (22
significant bits) against exact fp16 weight operands (sc*q; for Q6_K a
rounded part plus an exact remainder) with fp32 accumulation, so it is held
to the mat-vec path's tighter bars: row-norm error <= 1e-5 and the
reference's per-element Approx (eps 1e-4, margin 3e-5) on at least 99% of
the elements."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4, Q6 = 12, 14
ROW_NORM_BAR = 1e-3
SEED = 20261202
DMAX = {Q4: 0.01, Q6: 0.005}


def make_weight(qk, qtype, N, K, seed):
    w = qk.DeviceBuffer(N * qk.row_bytes(qtype, K))
    qk.synth_superblocks(w, qtype, N, K, seed, DMAX[qtype], 0.01)
    qk.synchronize()
    return w


def float64_reference(oracle, x, w_bytes, qtype, K, N, M):
    W = oracle.dequantize(w_bytes, qtype, N, K).reshape(N, K).astype(np.float64)
    xr = oracle.q8_roundtrip(x).reshape(M, K).astype(np.float64)
    return xr @ W.T


def check(oracle, got, ref, label):
    err = oracle.row_norm_error(got, ref)
    rate = oracle.approx_pass_rate(got, ref)
    print(f"[{label}] row-norm error {err:.3e}, Approx pass rate {rate:.4f}", flush=True)
    assert np.all(np.isfinite(got))
    assert err <= ROW_NORM_BAR
    assert err <= 1e-5
    assert rate >= 0.99
    return err


# Qwen3-4B prefill projections at M = 512 tokens (config: K=2560 gate/q/k/v,
# plus attn_output and ffn_down).
PREFILL = [
    ("ffn_gate", Q4, 2560, 9728),
    ("attn_q", Q4, 2560, 4096),
    ("attn_k", Q4, 2560, 1024),
    ("attn_v", Q6, 2560, 1024),
    ("attn_output", Q4, 4096, 2560),
    ("ffn_down", Q6, 9728, 2560),
]


@pytest.mark.parametrize("name,qtype,K,N", PREFILL)
def test_prefill_qwen3_shapes_m512(gpu, oracle, name, qtype, K, N):
    M = 512
    print(f"[case] {name} type={qtype} K={K} N={N} M={M}", flush=True)
    w = make_weight(gpu, qtype, N, K, SEED + 10 + PREFILL.index((name, qtype, K, N)))
    x = oracle.synth_normal(M * K, SEED + 1)
    xd = gpu.DeviceBuffer.from_array(x)
    y = gpu.DeviceBuffer(4 * M * N)
    gpu.matmul(xd, w, qtype, K, N, y, M)
    gpu.synchronize()
    got = y.download(np.float32).reshape(M, N)
    ref = float64_reference(oracle, x, w.download(np.uint8), qtype, K, N, M)
    check(oracle, got, ref, name)


PROMPT_SHAPES = PREFILL + [("lm_head", Q6, 2560, 151936)]


@pytest.mark.parametrize("name,qtype,K,N", PROMPT_SHAPES)
def test_prefill_qwen3_shapes_m23(gpu, oracle, name, qtype, K, N):
    """The reference's own prompt length (README.md:30-37: a 23-token
    templated prompt, src/Engine.cpp:71-111 with tokens = 23) on every Qwen3
    projection shape and the lm_head, through kernels::matmul, allocating and
    with a caller workspace (same bits)."""
    M = 23
    w = make_weight(gpu, qtype, N, K, SEED + 30 + PROMPT_SHAPES.index((name, qtype, K, N)))
    x = oracle.synth_normal(M * K, SEED + 3)
    xd = gpu.DeviceBuffer.from_array(x)
    y = gpu.DeviceBuffer(4 * M * N)
    gpu.matmul(xd, w, qtype, K, N, y, M)
    gpu.synchronize()
    print(f"[case] {name} type={qtype} K={K} N={N} M={M} launch {gpu.last_launch()}", flush=True)
    got = y.download(np.float32).reshape(M, N)
    ref = float64_reference(oracle, x, w.download(np.uint8), qtype, K, N, M)
    check(oracle, got, ref, name)
    need = gpu.matmul_workspace_size(qtype, K, N, M)
    ws = gpu.DeviceBuffer(max(need, 16))
    y2 = gpu.DeviceBuffer(4 * M * N)
    gpu.matmul_ws(xd, w, qtype, K, N, y2, M, ws, need)
    gpu.synchronize()
    assert np.array_equal(y2.download(np.float32).reshape(M, N), got)


@pytest.mark.parametrize("qtype", [Q4, Q6])
def test_prefill_single_column_ill_conditioned(gpu, oracle, qtype):
    """N = 1: the row norm is one |y| value, which cancellation can bring near
    zero (fp16 operands alone would give a relative error of order 1 on such
    rows). Error measured against the row magnitude sum(|x||w|) instead:
    within 1e-6, the size of fp32 accumulation error."""
    M, N, K = 257, 1, 3328
    w = make_weight(gpu, qtype, N, K, SEED + 20 + M + N)
    x = oracle.synth_normal(M * K, SEED + 2 + K)
    xd = gpu.DeviceBuffer.from_array(x)
    y = gpu.DeviceBuffer(4 * M)
    gpu.matmul(xd, w, qtype, K, N, y, M)
    gpu.synchronize()
    got = y.download(np.float32).astype(np.float64)
    wb = w.download(np.uint8)
    ref = oracle.reference_product(x, wb, qtype, K, N)[:, 0]
    W = oracle.dequantize(wb, qtype, N, K).reshape(K).astype(np.float64)
    magnitude = np.abs(oracle.q8_roundtrip(x).reshape(M, K)) @ np.abs(W)
    worst = float(np.max(np.abs(got - ref) / magnitude))
    print(f"max |y - y_ref| / sum|x||w| = {worst:.3e}; row-norm {oracle.row_norm_error(got.reshape(M, 1), ref.reshape(M, 1)):.3e}",
          flush=True)
    assert worst <= 1e-6


@pytest.mark.parametrize("qtype", [Q4, Q6])
@pytest.mark.parametrize("scale", [1e-6, 1e4])
def test_prefill_activation_scale_invariance(gpu, oracle, qtype, scale):
    """Rows of very small or very large activations keep full precision: the
    per-row power-of-two scale keeps the fp16 planes in range."""
    M, N, K = 33, 96, 2560
    w = make_weight(gpu, qtype, N, K, SEED + 60)
    x = (oracle.synth_normal(M * K, SEED + 61) * np.float32(scale)).astype(np.float32)
    xd = gpu.DeviceBuffer.from_array(x)
    y = gpu.DeviceBuffer(4 * M * N)
    gpu.matmul(xd, w, qtype, K, N, y, M)
    gpu.synchronize()
    got = y.download(np.float32).reshape(M, N)
    ref = oracle.reference_product(x, w.download(np.uint8), qtype, K, N)
    check(oracle, got, ref, f"x*{scale:g}")


@pytest.mark.parametrize("qtype", [Q4, Q6])
@pytest.mark.parametrize("M,N,K", [(9, 77, 2560), (100, 1000, 512), (129, 64, 256),
                                   (300, 130, 768), (257, 3, 3328), (16, 64, 16640),
                                   (200, 20000, 512)])
def test_prefill_ragged_against_oracle(gpu, oracle, qtype, M, N, K):
    """Row and column counts off the tilings (32 x 128, or 64 x 128 from 1.5
    tiles per CU for Q4_K, as 200 x 20000 takes, and from half a tile per CU
    for Q6_K), narrow and odd widths (K = 16640 takes the activation prep's
    two-pass path), against the oracle's own double-accumulated product."""
    print(f"[case] type={qtype} M={M} N={N} K={K}", flush=True)
    w = make_weight(gpu, qtype, N, K, SEED + 20 + M + N)
    x = oracle.synth_normal(M * K, SEED + 2 + K)
    xd = gpu.DeviceBuffer.from_array(x)
    y = gpu.DeviceBuffer(4 * (M * N + 2))
    y.upload(np.full(M * N + 2, 123.0, np.float32))
    gpu.matmul(xd, w, qtype, K, N, y, M, y_offset=4)
    gpu.synchronize()
    out = y.download(np.float32)
    assert out[0] == 123.0 and out[-1] == 123.0
    ref = oracle.reference_product(x, w.download(np.uint8), qtype, K, N)
    check(oracle, out[1:-1].reshape(M, N), ref.reshape(M, N), f"{qtype} {M}x{N}x{K}")


@pytest.mark.parametrize("qtype", [Q4, Q6])
@pytest.mark.parametrize("M,N,K,scale", [(23, 200, 2560, 1.0), (32, 128, 768, 1e-6), (9, 300, 256, 1e4),
                                         (31, 1000, 4096, 1.0), (17, 2560, 9728, 1.0)])
def test_prefill_short_prompt_against_oracle(gpu, oracle, qtype, M, N, K, scale):
    """M <= 32 (a short prompt): the GEMM forms its own activation planes, with
    a power-of-two scale per row and superblock, in one launch (plus the split
    reduce). Ragged N, one to 38 superblocks, activations scaled by 1e-6 and
    1e4, against the oracle's double-accumulated product."""
    print(f"[case] short type={qtype} M={M} N={N} K={K} x*{scale:g}", flush=True)
    w = make_weight(gpu, qtype, N, K, SEED + 70 + M + N)
    x = (oracle.synth_normal(M * K, SEED + 71 + K) * np.float32(scale)).astype(np.float32)
    xd = gpu.DeviceBuffer.from_array(x)
    y = gpu.DeviceBuffer(4 * M * N)
    gpu.matmul(xd, w, qtype, K, N, y, M)
    gpu.synchronize()
    print(f"[case] launch {gpu.last_launch()}", flush=True)
    got = y.download(np.float32).reshape(M, N)
    ref = oracle.reference_product(x, w.download(np.uint8), qtype, K, N)
    check(oracle, got, ref.reshape(M, N), f"short {qtype} {M}x{N}x{K}")


@pytest.mark.parametrize("qtype", [Q4, Q6])
def test_prefill_short_prompt_superblocks_of_unequal_size(gpu, oracle, qtype):
    """Rows whose superblocks differ by up to 10^7 in magnitude: each
    superblock gets its own power-of-two scale, so the small ones keep their
    precision (checked element by element: the reference's Approx on >= 99%
    of the elements and, per row, the error of every output within 1e-5 of the
    row norm)."""
    M, N, K = 23, 320, 2560
    w = make_weight(gpu, qtype, N, K, SEED + 80)
    x = oracle.synth_normal(M * K, SEED + 81).reshape(M, K // 256, 256)
    mags = np.float32(10.0) ** np.arange(-3, 7, dtype=np.float32)[: K // 256]
    x = (x * mags[None, :, None]).astype(np.float32).reshape(-1)
    xd = gpu.DeviceBuffer.from_array(x)
    y = gpu.DeviceBuffer(4 * M * N)
    gpu.matmul(xd, w, qtype, K, N, y, M)
    gpu.synchronize()
    got = y.download(np.float32).reshape(M, N)
    ref = oracle.reference_product(x, w.download(np.uint8), qtype, K, N).reshape(M, N)
    check(oracle, got, ref, f"unequal superblocks {qtype}")


@pytest.mark.parametrize("qtype", [Q4, Q6])
def test_prefill_zero_input_and_reuse(gpu, oracle, qtype):
    """src/tests/MatmulTests.cpp:12-82 and :84-132 at M > 8: zero rows give exact zeros,
    a reused output is overwritten, two streams give identical bits."""
    K, N, M = 2560, 200, 40
    w = make_weight(gpu, qtype, N, K, SEED + 30)
    x = oracle.synth_normal(M * K, SEED + 31)
    xd = gpu.DeviceBuffer.from_array(x)
    y1 = gpu.DeviceBuffer.from_array(np.full(M * N, np.nan, np.float32))
    y2 = gpu.DeviceBuffer.from_array(np.full(M * N, 123.0, np.float32))
    s1, s2 = gpu.Stream(), gpu.Stream()
    gpu.matmul(xd, w, qtype, K, N, y1, M, s1)
    gpu.matmul(xd, w, qtype, K, N, y2, M, s2)
    s1.synchronize()
    s2.synchronize()
    a, b = y1.download(np.float32), y2.download(np.float32)
    assert np.array_equal(a, b)
    ref = oracle.reference_product(x, w.download(np.uint8), qtype, K, N)
    check(oracle, a.reshape(M, N), ref.reshape(M, N), "streams")
    xd.fill(0)
    gpu.matmul(xd, w, qtype, K, N, y1, M)
    gpu.synchronize()
    assert np.all(y1.download(np.float32) == 0.0)
    s1.destroy()
    s2.destroy()


@pytest.mark.parametrize("qtype,N,M_wide,M_narrow", [
    (Q4, 9728, 384, 320),   # 456 tiles of 64 x 128 against 760 of 32 x 128
    (Q4, 9728, 512, 256),
    (Q6, 2560, 512, 96),    # ffn_down-like, K = 2560: 64 x 128 against 32 x 128
])
def test_prefill_rows_independent_of_tile_height(gpu, oracle, qtype, N, M_wide, M_narrow):
    """The launcher picks 64- or 32-row tiles from the grid size; an output
    row's sums do not depend on it (nor on M): the first M_narrow rows of a
    launch on 64-row tiles equal a launch of those rows alone on 32-row tiles
    bit for bit."""
    K = 2560
    w = make_weight(gpu, qtype, N, K, SEED + 45)
    x = oracle.synth_normal(M_wide * K, SEED + 46)
    xw, xn = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer.from_array(x[:M_narrow * K])
    yw, yn = gpu.DeviceBuffer(4 * M_wide * N), gpu.DeviceBuffer(4 * M_narrow * N)
    gpu.matmul(xw, w, qtype, K, N, yw, M_wide)
    gpu.synchronize()
    wide = gpu.last_launch()
    gpu.matmul(xn, w, qtype, K, N, yn, M_narrow)
    gpu.synchronize()
    narrow = gpu.last_launch()
    print(f"[case] tile height type={qtype} N={N}: M={M_wide} {wide} | M={M_narrow} {narrow}", flush=True)
    assert wide != narrow  # the two launches took different tile shapes
    got = yw.download(np.float32)[:M_narrow * N]
    assert np.array_equal(got, yn.download(np.float32))


@pytest.mark.parametrize("qtype", [Q4, Q6])
def test_prefill_entry_points_agree_bitwise(gpu, oracle, qtype):
    """qk_matmul (stream-ordered scratch) and qk_matmul_ws (caller workspace)
    run the same kernels; qk_matmul_segments at M > 8 too."""
    K, N, M = 2560, 333, 77
    w = make_weight(gpu, qtype, N, K, SEED + 40)
    x = oracle.synth_normal(M * K, SEED + 41)
    xd = gpu.DeviceBuffer.from_array(x)
    ya, yb, yc = (gpu.DeviceBuffer(4 * M * N) for _ in range(3))
    gpu.matmul(xd, w, qtype, K, N, ya, M)
    need = gpu.matmul_workspace_size(qtype, K, N, M)
    assert need >= M * K * 4 + M * 4 and need % 256 == 0
    ws = gpu.DeviceBuffer(need)
    gpu.matmul_ws(xd, w, qtype, K, N, yb, M, ws, need)
    gpu.matmul_segments(xd, M, K, [(w, qtype, N, yc)])
    gpu.synchronize()
    a = ya.download(np.float32)
    assert np.array_equal(a, yb.download(np.float32))
    assert np.array_equal(a, yc.download(np.float32))
    with pytest.raises(RuntimeError, match="workspace too small"):
        gpu.matmul_ws(xd, w, qtype, K, N, yb, M, ws, need - 256)


@pytest.mark.parametrize("M,K,shapes", [
    (512, 2560, [(Q4, 4096), (Q4, 1024), (Q6, 1024)]),   # attn q, k and v: one launch of both types
    (77, 2560, [(Q6, 333), (Q6, 129), (Q4, 200), (Q4, 64)]),
    (40, 2560, [(Q4, 4096), (Q4, 1024), (Q6, 1024)]),
    (64, 9728, [(Q6, 256), (Q4, 300)]),                    # split K: separate launches
    (20, 256, [(Q6, 300), (Q4, 200), (Q4, 64)]),            # short prompt, one launch of both types
    (23, 2560, [(Q4, 4096), (Q4, 1024), (Q6, 1024)]),       # short prompt, split K: separate launches
])
def test_prefill_segments_pairs_match_single_launches(gpu, oracle, M, K, shapes):
    """qk_matmul_segments at M > 8 runs its matrices in one GEMM launch when
    the combined grid needs no split K (each workgroup takes its matrix's
    type), otherwise same-type pairs or single launches. Every output equals
    its single-matrix qk_matmul bit for bit when that launch does not split K
    (the same tiles, the same sums); when it does (attn k / v alone at
    M = 512), the two differ only by the order of fp32 sums: within 1e-6 of
    the row norm. Both within the bar of the oracle."""
    ws = [make_weight(gpu, q, N, K, SEED + 60 + i) for i, (q, N) in enumerate(shapes)]
    x = oracle.synth_normal(M * K, SEED + 61)
    xd = gpu.DeviceBuffer.from_array(x)
    ys = [gpu.DeviceBuffer(4 * M * N) for _, N in shapes]
    gpu.matmul_segments(xd, M, K, [(w, q, N, y) for w, (q, N), y in zip(ws, shapes, ys)])
    print(f"[case] segments M={M} K={K} {shapes} last launch {gpu.last_launch()}", flush=True)
    singles, split = [gpu.DeviceBuffer(4 * M * N) for _, N in shapes], []
    for w, (q, N), y in zip(ws, shapes, singles):
        gpu.matmul(xd, w, q, K, N, y, M)
        launch = gpu.last_launch()  # gemm_kq_kernel<type,TM,TN,splits> grid=G
        split.append(int(launch.split(">")[0].split(",")[-1]) > 1)
        print(f"[case] single N={N} launch {launch}", flush=True)
    gpu.synchronize()
    for w, (q, N), y, y1, sp in zip(ws, shapes, ys, singles, split):
        got = y.download(np.float32)
        one = y1.download(np.float32)
        if sp:
            assert oracle.row_norm_error(got.reshape(M, N), one.reshape(M, N).astype(np.float64)) <= 1e-6
        else:
            assert np.array_equal(got, one)
        if N <= 1024:
            ref = float64_reference(oracle, x, w.download(np.uint8), q, K, N, M)
            check(oracle, got.reshape(M, N), ref, f"segments q{q} N={N}")


def test_prefill_graph_replay_with_workspace(gpu, oracle):
    """qk_matmul_ws allocates nothing, so a prefill step can be captured; each
    replay, with eager work in between, equals the eager result."""
    qk = gpu
    K, M = 2560, 64
    shapes = [(Q4, 4096), (Q6, 1024)]
    ws_ = [make_weight(qk, q, N, K, SEED + 50 + i) for i, (q, N) in enumerate(shapes)]
    xd = qk.DeviceBuffer.from_array(oracle.synth_normal(M * K, SEED + 51))
    need = qk.matmul_workspace_size(Q4, K, 4096, M)
    scratch = qk.DeviceBuffer(need)
    ys = [qk.DeviceBuffer(4 * M * N) for _, N in shapes]
    stream = qk.Stream()

    def record():
        for (q, N), w, y in zip(shapes, ws_, ys):
            qk.matmul_ws(xd, w, q, K, N, y, M, scratch, need, stream)

    record()
    stream.synchronize()
    eager = [y.download(np.float32) for y in ys]
    graph = qk.Graph.capture(stream, record)
    for rep in range(3):
        for y in ys:
            y.upload(np.full(y.nbytes // 4, np.nan, np.float32))
        graph.launch(stream)
        stream.synchronize()
        for e, y in zip(eager, ys):
            assert np.array_equal(y.download(np.float32), e), f"replay {rep}"
        record()
        stream.synchronize()
    graph.destroy()
    stream.destroy()


def test_split_k_workspace_from_garbage_and_across_plans(gpu, oracle):
    """Launches that split K keep their partial products in the workspace and
    a reduce launch adds them in split order. A workspace that starts as 0xFF
    bytes, reused by calls of different split plans one after another (10, 26
    and 10 splits at M = 23; 2 and 3 at M = 512), gives the bits of a fresh
    allocation every time: nothing read is left over from an earlier call."""
    qk = gpu
    shapes = [(23, "attn_k", Q4, 2560, 1024), (23, "ffn_down", Q6, 9728, 2560),
              (23, "attn_v", Q6, 2560, 1024), (512, "attn_k", Q4, 2560, 1024),
              (512, "ffn_down", Q6, 9728, 2560)]
    need = max(qk.matmul_workspace_size(q, K, N, M) for M, _, q, K, N in shapes)
    ws = qk.DeviceBuffer.from_array(np.full(need, 0xFF, np.uint8))
    cases = []
    for i, (M, name, q, K, N) in enumerate(shapes):
        w = make_weight(qk, q, N, K, SEED + 60 + i)
        xd = qk.DeviceBuffer.from_array(oracle.synth_normal(M * K, SEED + 61 + i))
        y = qk.DeviceBuffer(4 * M * N)
        qk.matmul(xd, w, q, K, N, y, M)
        qk.synchronize()
        cases.append((M, name, q, K, N, w, xd, y.download(np.float32)))
        print(f"[case] {name} M={M} launch {qk.last_launch()}", flush=True)
    for rep in range(2):
        for M, name, q, K, N, w, xd, fresh in cases:
            y = qk.DeviceBuffer(4 * M * N)
            qk.matmul_ws(xd, w, q, K, N, y, M, ws, need)
            qk.synchronize()
            assert np.array_equal(y.download(np.float32), fresh), f"{name} M={M} pass {rep}"
    M, name, q, K, N, w, xd, fresh = cases[0]
    ref = float64_reference(oracle, xd.download(np.float32), w.download(np.uint8), q, K, N, M)
    check(oracle, fresh.reshape(M, N), ref, f"{name} M={M}")


@pytest.mark.parametrize("qtype,K,N,M", [(Q4, 2560, 9728, 64), (Q6, 9728, 2560, 40)])
def test_ffn_gate_up_workspace_variant_and_deep_k(gpu, oracle, qtype, K, N, M):
    """qk_ffn_gate_up_ws equals qk_ffn_gate_up bit for bit; the deep-K shape
    (K = 9728, N = 2560) takes the split-K GEMM for gate and up in separate
    launches, checked against the oracle; a workspace short of
    qk_ffn_gate_up_workspace_size is rejected."""
    gate = make_weight(gpu, qtype, N, K, SEED + 60)
    up = make_weight(gpu, qtype, N, K, SEED + 61)
    x = oracle.synth_normal(M * K, SEED + 62)
    xd = gpu.DeviceBuffer.from_array(x)
    h1, h2 = gpu.DeviceBuffer(4 * M * N), gpu.DeviceBuffer(4 * M * N)
    gpu.ffn_gate_up(xd, gate, up, qtype, K, N, h1, M)
    need = gpu.ffn_gate_up_workspace_size(qtype, K, N, M)
    assert need >= 2 * M * N * 4 + gpu.matmul_workspace_size(qtype, K, N, M)
    ws = gpu.DeviceBuffer(need)
    gpu.ffn_gate_up_ws(xd, gate, up, qtype, K, N, h2, M, ws, need)
    gpu.synchronize()
    a, b = h1.download(np.float32), h2.download(np.float32)
    assert np.array_equal(a, b)
    g = oracle.reference_product(x, gate.download(np.uint8), qtype, K, N)
    u = oracle.reference_product(x, up.download(np.uint8), qtype, K, N)
    with np.errstate(over="ignore"):
        ref = (g / (1.0 + np.exp(-g))) * u
    err = oracle.row_norm_error(a.reshape(M, N), ref)
    print(f"[case] ffn prefill type={qtype} K={K} N={N} M={M} error {err:.3e}", flush=True)
    assert err <= 1e-5
    assert gpu.load().qk_ffn_gate_up_ws(xd.ptr, gate.ptr, up.ptr, qtype, K, N, h2.ptr, M, ws.ptr,
                                        need - 256, None) == 1


def test_segments_workspace_variant(gpu, oracle):
    """qk_matmul_segments_ws (q/k/v at M = 40) equals qk_matmul_segments bit for bit."""
    K, M = 2560, 40
    shapes = [(Q4, 4096), (Q4, 1024), (Q6, 1024)]
    ws_ = [make_weight(gpu, q, N, K, SEED + 70 + i) for i, (q, N) in enumerate(shapes)]
    xd = gpu.DeviceBuffer.from_array(oracle.synth_normal(M * K, SEED + 73))
    y1 = [gpu.DeviceBuffer(4 * M * N) for _, N in shapes]
    y2 = [gpu.DeviceBuffer(4 * M * N) for _, N in shapes]
    gpu.matmul_segments(xd, M, K, [(w, q, N, y) for w, (q, N), y in zip(ws_, shapes, y1)])
    segs = [(w, q, N, y) for w, (q, N), y in zip(ws_, shapes, y2)]
    need = gpu.matmul_segments_workspace_size(M, K, segs)
    assert need == max(gpu.matmul_workspace_size(q, K, N, M) for q, N in shapes)
    work = gpu.DeviceBuffer(need)
    gpu.matmul_segments_ws(xd, M, K, segs, work, need)
    gpu.synchronize()
    for a, b in zip(y1, y2):
        assert np.array_equal(a.download(np.float32), b.download(np.float32))


@pytest.mark.parametrize("M,K,N", [(512, 2560, 9728), (77, 2560, 1000), (40, 512, 300), (33, 9728, 2560)])
def test_ffn_gate_up_matches_separate_kernels(gpu, oracle, M, K, N):
    """qk_ffn_gate_up at M > 8 (gate and up in one GEMM launch unless K splits,
    then the SiLU kernel): h equals qk_matmul(gate), qk_matmul(up) and
    qk_silu_multiply bit for bit, and the oracle's SiLU(x . gate^T) *
    (x . up^T) within the bar."""
    gate = make_weight(gpu, Q4, N, K, SEED + 70)
    up = make_weight(gpu, Q4, N, K, SEED + 71)
    x = oracle.synth_normal(M * K, SEED + 72)
    xd = gpu.DeviceBuffer.from_array(x)
    h = gpu.DeviceBuffer.from_array(np.full(M * N, np.nan, np.float32))
    gpu.ffn_gate_up(xd, gate, up, Q4, K, N, h, M)
    gpu.synchronize()
    print(f"[case] ffn gate/up M={M} K={K} N={N} launch {gpu.last_launch()}", flush=True)
    yg, yu, hs = (gpu.DeviceBuffer(4 * M * N) for _ in range(3))
    gpu.matmul(xd, gate, Q4, K, N, yg, M)
    gpu.matmul(xd, up, Q4, K, N, yu, M)
    gpu.silu_multiply(yg, yu, hs, M * N)
    gpu.synchronize()
    got = h.download(np.float32)
    assert np.array_equal(got, hs.download(np.float32))
    if N <= 1000:
        g = float64_reference(oracle, x, gate.download(np.uint8), Q4, K, N, M)
        u = float64_reference(oracle, x, up.download(np.uint8), Q4, K, N, M)
        with np.errstate(over="ignore"):
            ref = g / (1.0 + np.exp(-g)) * u
        check(oracle, got.reshape(M, N), ref, f"ffn gate/up M={M}")
