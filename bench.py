#!/usr/bin/env python3
"""Benchmark of the Q4_K/Q6_K dequantize-matmul path on one MI355X.

Workload (one "step" = one decoded token's projection sweep): a random-init
Qwen3-4B Q4_K_M layout, 36 layers x {attn_q, attn_k (Q4_K 2560->4096/1024),
attn_v (Q6_K 2560->1024), attn_output (Q4_K 4096->2560), ffn_gate, ffn_up
(Q4_K 2560->9728), ffn_down (Q6_K 9728->2560)} + lm_head (Q6_K 2560->151936)
with the next-token argmax, M = 1 activation row, in the reference engine's
call order (src/Engine.cpp:83-111): Q8 quantize + mat-vec per projection,
SiLU*up before ffn_down, lm_head + argmax in one launch. Weights (2.62 GB)
are generated on the device; activations are N(0,1). The step is captured
once as a graph and replayed.

Prints one JSON line: value = algorithmic GB/s of the whole sweep
(weights + fp32 activations in/out, see gemv_bytes), plus tokens/s, the
roofline of the dominant kernel (per-launch HIP events) and the CPU oracle
timed on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import pathlib
import platform
import sys
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
PKG_DIR = ROOT / "qwen3-4b-q4_k_m-inference-engine_amd"

Q4, Q6 = 12, 14
SB_BYTES = {Q4: 144, Q6: 210}
PEAK_HBM_GBS = 8000.0
PEAK_FP16_TFLOPS = 2500.0  # dense fp16 MFMA
METRIC = "Q4_K/Q6_K GEMV HBM GB/s (% of peak) at M=1; decode tokens/s, 4B shapes"
SEED = 20261205  # 20261201 + config id 4

LAYER = [
    ("attn_q", Q4, 2560, 4096),
    ("attn_k", Q4, 2560, 1024),
    ("attn_v", Q6, 2560, 1024),
    ("attn_output", Q4, 4096, 2560),
    ("ffn_gate", Q4, 2560, 9728),
    ("ffn_up", Q4, 2560, 9728),
    ("ffn_down", Q6, 9728, 2560),
]
LM_HEAD = ("lm_head", Q6, 2560, 151936)
N_LAYERS = 36


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def load_package():
    spec = importlib.util.spec_from_file_location("qk_amd", PKG_DIR / "__init__.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules["qk_amd"] = mod
    spec.loader.exec_module(mod)
    mod.load()
    return mod


def gemv_bytes(qtype: int, K: int, N: int, M: int) -> int:
    """Algorithmic HBM bytes of one mat-vec: packed weights + fp32 x + fp32 y."""
    return N * (K // 256) * SB_BYTES[qtype] + 4 * M * K + 4 * M * N


def weight_bytes(qtype: int, K: int, N: int) -> int:
    return N * (K // 256) * SB_BYTES[qtype]


class Op:
    """One launch of the step: a kernel family name, its algorithmic bytes and the call."""

    def __init__(self, family: str, nbytes: int, call):
        self.family, self.nbytes, self.call = family, nbytes, call


class DecodeSweep:
    """Weights, activations and the per-token launch sequence of the decode sweep."""

    def __init__(self, qk, M: int = 1, weights_of: "DecodeSweep | None" = None, fused_ffn: bool = True,
                 engine_calls: bool = False):
        self.qk, self.M = qk, M
        # engine_calls: the reference engine's own per-layer sequence, unmodified
        # (src/Engine.cpp:83-85,94,98-101,109-110): q, k, v, o, gate, up as
        # separate kernels::matmul calls, silu_multiply, down, then the lm_head
        # matmul into logits and argmax; no fused entry points
        self.engine_calls = engine_calls
        # the FFN block through qk_ffn: M = 1 one launch (gate, up, SiLU*up,
        # down); M = 2..8 gate/up, one Q8 of h into the workspace, down on it
        self.fused_ffn = fused_ffn
        if weights_of is not None:  # same weights, other activation rows
            self.layers, self.lm_head = weights_of.layers, weights_of.lm_head
        else:
            self.layers = []
            tensor = 0
            for _ in range(N_LAYERS):
                layer = {}
                for name, qtype, K, N in LAYER:
                    w = qk.DeviceBuffer(N * qk.row_bytes(qtype, K))
                    qk.synth_superblocks(w, qtype, N, K, SEED + 1000 * tensor, 0.01 if qtype == Q4 else 0.005, 0.01)
                    layer[name] = w
                    tensor += 1
                self.layers.append(layer)
            name, qtype, K, N = LM_HEAD
            self.lm_head = qk.DeviceBuffer(N * qk.row_bytes(qtype, K))
            qk.synth_superblocks(self.lm_head, qtype, N, K, SEED + 1000 * tensor, 0.005, 0.01)
        buf = lambda n: qk.DeviceBuffer(4 * M * n)
        self.x_attn, self.x_o, self.x_ffn = buf(2560), buf(4096), buf(2560)
        qk.synth_normal(self.x_attn, M * 2560, SEED + 1)
        qk.synth_normal(self.x_o, M * 4096, SEED + 2)
        qk.synth_normal(self.x_ffn, M * 2560, SEED + 3)
        self.y = {n: buf(N) for n, _, _, N in LAYER}
        self.h = buf(9728)
        self.gate, self.up = buf(9728), buf(9728)
        self.logits = buf(LM_HEAD[3])
        self.argmax_bytes = qk.argmax_workspace_size()
        self.argmax_ws = qk.DeviceBuffer(self.argmax_bytes)
        qk.check(qk.load().qk_memset_async(self.argmax_ws.ptr, 0, self.argmax_bytes, None))
        self.next_token = qk.DeviceBuffer(4)
        self.y_ffn = buf(2560)
        self.ffn_ws_bytes = qk.ffn_workspace_size()
        self.ffn_ws = qk.DeviceBuffer(self.ffn_ws_bytes)
        qk.check(qk.load().qk_memset_async(self.ffn_ws.ptr, 0, self.ffn_ws_bytes, None))
        qk.synchronize()

    def ops(self, stream):
        """The launches of one step, in the reference engine's order
        (src/Engine.cpp:83-109): q/k/v in one launch, attn_output, gate/up with
        SiLU*up in one launch, ffn_down; then lm_head."""
        qk, M, y = self.qk, self.M, self.y
        out = []
        if self.engine_calls:
            return self.engine_ops(stream)
        for layer in self.layers:
            segs = [(layer[n], q, N, y[n]) for n, q, K, N in LAYER[:3]]
            out.append(Op("attn_qkv", sum(weight_bytes(q, 2560, N) for n, q, K, N in LAYER[:3])
                          + 4 * M * (2560 + 4096 + 1024 + 1024),
                          lambda segs=segs: qk.matmul_segments(self.x_attn, M, 2560, segs, stream)))
            w_o = layer["attn_output"]
            out.append(Op("attn_output", gemv_bytes(Q4, 4096, 2560, M),
                          lambda w=w_o: qk.matmul(self.x_o, w, Q4, 4096, 2560, y["attn_output"], M, stream)))
            g, u, w_d = layer["ffn_gate"], layer["ffn_up"], layer["ffn_down"]
            if self.fused_ffn:
                # weights + x in + h out + y out (h's read-back inside the launch is not counted)
                out.append(Op("ffn_block", 2 * weight_bytes(Q4, 2560, 9728) + weight_bytes(Q6, 9728, 2560)
                              + 4 * M * (2560 + 9728 + 2560),
                              lambda g=g, u=u, d=w_d: qk.ffn(self.x_ffn, None, 0.0, g, u, Q4, d, Q6, 2560, 9728,
                                                             self.h, self.y_ffn, M, self.ffn_ws,
                                                             self.ffn_ws_bytes, stream)))
                continue
            out.append(Op("ffn_gate_up", 2 * weight_bytes(Q4, 2560, 9728) + 4 * M * (2560 + 9728),
                          lambda g=g, u=u: qk.ffn_gate_up(self.x_ffn, g, u, Q4, 2560, 9728, self.h, M, stream)))
            out.append(Op("ffn_down", gemv_bytes(Q6, 9728, 2560, M),
                          lambda w=w_d: qk.matmul(self.h, w, Q6, 9728, 2560, y["ffn_down"], M, stream)))
        name, qtype, K, N = LM_HEAD
        if M == 1:  # the engine's last step: logits of the final position and their argmax
            out.append(Op("lm_head_argmax", weight_bytes(qtype, K, N) + 4 * K + 4,
                          lambda: qk.matmul_argmax(self.x_attn, self.lm_head, qtype, K, N, None,
                                                   self.next_token, self.argmax_ws, self.argmax_bytes, stream)))
        else:
            out.append(Op("lm_head", gemv_bytes(qtype, K, N, M),
                          lambda: qk.matmul(self.x_attn, self.lm_head, qtype, K, N, self.logits, M, stream)))
        return out

    def engine_ops(self, stream):
        """The unmodified engine's launches per token: every projection its own
        kernels::matmul (qk_matmul), SiLU*up in its own kernel, the logits
        written out and reduced by qk_argmax."""
        qk, M, y = self.qk, self.M, self.y
        out = []
        for layer in self.layers:
            for n, q, K, N in LAYER[:3]:
                out.append(Op("engine_matmul", gemv_bytes(q, K, N, M),
                              lambda w=layer[n], q=q, K=K, N=N, n=n: qk.matmul(self.x_attn, w, q, K, N, y[n], M, stream)))
            out.append(Op("engine_matmul", gemv_bytes(Q4, 4096, 2560, M),
                          lambda w=layer["attn_output"]: qk.matmul(self.x_o, w, Q4, 4096, 2560, y["attn_output"], M,
                                                                   stream)))
            for n, dst in (("ffn_gate", self.gate), ("ffn_up", self.up)):
                out.append(Op("engine_matmul", gemv_bytes(Q4, 2560, 9728, M),
                              lambda w=layer[n], dst=dst: qk.matmul(self.x_ffn, w, Q4, 2560, 9728, dst, M, stream)))
            out.append(Op("engine_silu", 3 * 4 * M * 9728,
                          lambda: qk.silu_multiply(self.gate, self.up, self.h, M * 9728, stream)))
            out.append(Op("engine_matmul", gemv_bytes(Q6, 9728, 2560, M),
                          lambda w=layer["ffn_down"]: qk.matmul(self.h, w, Q6, 9728, 2560, y["ffn_down"], M, stream)))
        name, qtype, K, N = LM_HEAD
        out.append(Op("engine_matmul", gemv_bytes(qtype, K, N, M),
                      lambda: qk.matmul(self.x_attn, self.lm_head, qtype, K, N, self.logits, M, stream)))
        out.append(Op("engine_argmax", 4 * N + 4,
                      lambda: qk.argmax(self.logits, N, self.next_token, self.argmax_ws, self.argmax_bytes, stream)))
        return out

    def bytes_per_step(self) -> int:
        return sum(op.nbytes for op in self.ops(None))

    def record(self, stream) -> None:
        for op in self.ops(stream):
            op.call()


def time_graph(qk, graph, stream, warmup: int, steps: int) -> float:
    for _ in range(warmup):
        graph.launch(stream)
    stream.synchronize()
    start, end = qk.Event(), qk.Event()
    start.record(stream)
    for _ in range(steps):
        graph.launch(stream)
    end.record(stream)
    end.synchronize()
    ms = start.elapsed_ms(end)
    start.destroy()
    end.destroy()
    return ms / steps


def kernel_roofline(qk, sweep: DecodeSweep, stream, replays: int = 10):
    """Per kernel family: its launches of one step captured back to back in a
    graph, replayed between two HIP events on the launch stream; the average
    launch duration includes the back-to-back dispatch cost, as rocprof's does.
    A family with fewer than 8 launches per step (the lm_head) is captured
    repeated to 8 launches, so that one graph launch's own overhead is not
    counted as kernel time (its 319 MB exceed the 256 MB MALL: each repeat
    streams from HBM)."""
    families: dict[str, list] = {}
    for op in sweep.ops(stream):
        families.setdefault(op.family, []).append(op)
    out = {}
    for fam, ops in families.items():
        rep = max(1, 8 // len(ops))
        graph = qk.Graph.capture(stream, lambda ops=ops, rep=rep: [op.call() for _ in range(rep) for op in ops])
        reps = max(replays, 40 // (len(ops) * rep))
        ms = time_graph(qk, graph, stream, 2, reps)
        graph.destroy()
        avg_us = 1000.0 * ms / (len(ops) * rep)
        avg_bytes = sum(op.nbytes for op in ops) / len(ops)
        gbs = avg_bytes / (avg_us * 1e3)
        out[fam] = {"launches_per_step": len(ops), "avg_us": round(avg_us, 3), "avg_bytes": int(avg_bytes),
                    "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4),
                    "total_us_per_step": round(avg_us * len(ops), 1)}
    return out


TRAFFIC_FILE = ROOT / "profiles" / "traffic_decode_sweep_m1.json"
COPY_BYTES = 256 << 20


def reference_copy(qk, stream) -> None:
    """A device-to-device copy of COPY_BYTES: the known-size kernel against which
    the FETCH_SIZE / WRITE_SIZE counters of a --pmc run of this script are scaled."""
    src, dst = qk.DeviceBuffer(COPY_BYTES), qk.DeviceBuffer(COPY_BYTES)
    qk.check(qk.load().qk_memcpy_d2d_async(dst.ptr, src.ptr, COPY_BYTES, stream.ptr))
    stream.synchronize()
    src.free()
    dst.free()


def measured_traffic(family: str):
    """HBM bytes per launch of `family` from the committed counter runs, or None."""
    try:
        data = json.loads(TRAFFIC_FILE.read_text())
        return data["families"][family]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


COPIES = 40  # distinct weight copies per single-GEMV config: > 2x the 256 MB MALL


def time_launches(qk, stream, calls, replays: int = 5) -> float:
    """Average microseconds per launch of `calls`, captured back to back in a
    graph and replayed between HIP events on the launch stream."""
    graph = qk.Graph.capture(stream, lambda: [c() for c in calls])
    ms = time_graph(qk, graph, stream, 2, replays)
    graph.destroy()
    return 1000.0 * ms / len(calls)


def single_gemv(qk, stream, qtype: int, K: int, N: int, config_id: int):
    """Configs 0/1: one M=1 mat-vec over COPIES distinct weight copies."""
    seed = 20261201 + config_id
    ws = []
    for c in range(COPIES):
        w = qk.DeviceBuffer(N * qk.row_bytes(qtype, K))
        qk.synth_superblocks(w, qtype, N, K, seed + 7919 * c, 0.01 if qtype == Q4 else 0.005, 0.01)
        ws.append(w)
    x, y = qk.DeviceBuffer(4 * K), qk.DeviceBuffer(4 * N)
    qk.synth_normal(x, K, seed)
    qk.synchronize()
    us = time_launches(qk, stream, [lambda w=w: qk.matmul(x, w, qtype, K, N, y, 1, stream) for w in ws])
    nbytes = gemv_bytes(qtype, K, N, 1)
    for w in ws:
        w.free()
    return {"shape": f"{'Q4_K' if qtype == Q4 else 'Q6_K'} {N}x{K}, M=1, {COPIES} weight copies",
            "avg_us": round(us, 3), "GB/s": round(nbytes / (us * 1e3), 1),
            "frac": round(nbytes / (us * 1e3) / PEAK_HBM_GBS, 4), "GFLOP/s": round(2 * N * K / (us * 1e3), 1)}


def prefill_gemm(qk, stream):
    """Config 3: M=512 prefill projections (gate, q, k, v) on the MFMA GEMM."""
    M, K = 512, 2560
    out = {}
    x = qk.DeviceBuffer(4 * M * K)
    qk.synth_normal(x, M * K, 20261204)
    for name, qtype, N in (("ffn_gate", Q4, 9728), ("attn_q", Q4, 4096), ("attn_k", Q4, 1024), ("attn_v", Q6, 1024)):
        w = qk.DeviceBuffer(N * qk.row_bytes(qtype, K))
        qk.synth_superblocks(w, qtype, N, K, 20261204 + N, 0.01 if qtype == Q4 else 0.005, 0.01)
        y = qk.DeviceBuffer(4 * M * N)
        need = qk.matmul_workspace_size(qtype, K, N, M)
        ws = qk.DeviceBuffer(need)
        qk.synchronize()
        us = time_launches(qk, stream, [lambda w=w, y=y, ws=ws: qk.matmul_ws(x, w, qtype, K, N, y, M, ws, need, stream)] * 10)
        flops = 2 * M * N * K
        out[name] = {"shape": f"M={M} K={K} N={N} {'Q4_K' if qtype == Q4 else 'Q6_K'}",
                     "avg_us": round(us, 2), "TFLOP/s": round(flops / (us * 1e6), 1),
                     "frac_of_fp16_mfma_peak": round(flops / (us * 1e6) / PEAK_FP16_TFLOPS, 4)}
        for b in (w, y, ws):
            b.free()
    # attn q, k and v through qk_matmul_segments_ws (the engine's one call:
    # one activation prep, one GEMM launch of both weight types)
    segs = []
    for i, (qtype, N) in enumerate(((Q4, 4096), (Q4, 1024), (Q6, 1024))):
        w = qk.DeviceBuffer(N * qk.row_bytes(qtype, K))
        qk.synth_superblocks(w, qtype, N, K, 20261210 + i, 0.01 if qtype == Q4 else 0.005, 0.01)
        segs.append((w, qtype, N, qk.DeviceBuffer(4 * M * N)))
    need = qk.matmul_segments_workspace_size(M, K, segs)
    ws = qk.DeviceBuffer(need)
    qk.synchronize()
    us = time_launches(qk, stream, [lambda: qk.matmul_segments_ws(x, M, K, segs, ws, need, stream)] * 10)
    flops = 2 * M * K * (4096 + 1024 + 1024)
    out["attn_qkv_segments"] = {"shape": f"M={M} K={K} q 4096 + k 1024 Q4_K, v 1024 Q6_K, prep + one GEMM launch",
                                "avg_us": round(us, 2), "TFLOP/s": round(flops / (us * 1e6), 1),
                                "frac_of_fp16_mfma_peak": round(flops / (us * 1e6) / PEAK_FP16_TFLOPS, 4)}
    for w, _, _, y in segs:
        w.free()
        y.free()
    ws.free()
    # the fused FFN entry point at M = 512 (gate and up in one GEMM launch,
    # stream-ordered scratch, SiLU*up), timed eagerly: it allocates per call
    N = 9728
    gate, up = (qk.DeviceBuffer(N * qk.row_bytes(Q4, K)) for _ in range(2))
    qk.synth_superblocks(gate, Q4, N, K, 20261207, 0.01, 0.01)
    qk.synth_superblocks(up, Q4, N, K, 20261208, 0.01, 0.01)
    h = qk.DeviceBuffer(4 * M * N)
    qk.synchronize()
    for _ in range(2):
        qk.ffn_gate_up(x, gate, up, Q4, K, N, h, M, stream)
    stream.synchronize()
    start, end = qk.Event(), qk.Event()
    start.record(stream)
    for _ in range(10):
        qk.ffn_gate_up(x, gate, up, Q4, K, N, h, M, stream)
    end.record(stream)
    end.synchronize()
    us = 1000.0 * start.elapsed_ms(end) / 10
    start.destroy()
    end.destroy()
    flops = 2 * 2 * M * N * K
    out["ffn_gate_up_fused"] = {"shape": f"M={M} K={K} 2 x N={N} Q4_K + SiLU*up", "avg_us": round(us, 2),
                                "TFLOP/s": round(flops / (us * 1e6), 1),
                                "frac_of_fp16_mfma_peak": round(flops / (us * 1e6) / PEAK_FP16_TFLOPS, 4)}
    for b in (gate, up, h, x):
        b.free()
    return out


PROMPT_M = 23  # the reference's published first-token prompt (README.md:30-37)


def prefill_small_m(qk, sweep: DecodeSweep, stream, M: int = PROMPT_M):
    """The projections of a short prompt's prefill (src/Engine.cpp:71-111 at
    tokens = M): each shape over the sweep's 36 layers' distinct weights (the
    lm_head repeated 8 times), one kernels::matmul per call with a caller
    workspace, against the same shapes at M = 1. At this M the weights
    dominate the bytes, so the rate is HBM GB/s."""
    out = {}
    xs = {K: qk.DeviceBuffer(4 * M * K) for K in (2560, 4096, 9728)}
    for K, x in xs.items():
        qk.synth_normal(x, M * K, SEED + 23 + K)
    shapes = [(name, qtype, K, N, [layer[name] for layer in sweep.layers]) for name, qtype, K, N in LAYER]
    name, qtype, K, N = LM_HEAD
    shapes.append((name, qtype, K, N, [sweep.lm_head] * 8))
    for name, qtype, K, N, ws in shapes:
        y = qk.DeviceBuffer(4 * M * N)
        need = max(qk.matmul_workspace_size(qtype, K, N, M), 16)
        scratch = qk.DeviceBuffer(need)
        qk.synchronize()
        us_m = time_launches(qk, stream, [lambda w=w: qk.matmul_ws(xs[K], w, qtype, K, N, y, M, scratch, need, stream)
                                          for w in ws])
        launch = qk.last_launch()
        us_1 = time_launches(qk, stream, [lambda w=w: qk.matmul(xs[K], w, qtype, K, N, y, 1, stream) for w in ws])
        nbytes = gemv_bytes(qtype, K, N, M)
        out[name] = {"shape": f"M={M} K={K} N={N} {'Q4_K' if qtype == Q4 else 'Q6_K'}", "kernel": launch,
                     "avg_us": round(us_m, 3), "GB/s": round(nbytes / (us_m * 1e3), 1),
                     "frac": round(nbytes / (us_m * 1e3) / PEAK_HBM_GBS, 4),
                     "TFLOP/s": round(2 * M * N * K / (us_m * 1e6), 2),
                     "m1_avg_us": round(us_1, 3), "ratio_to_m1": round(us_m / us_1, 3)}
        y.free()
        scratch.free()
    for x in xs.values():
        x.free()
    return out


CONFIG_PARTS = ("gemv", "ffn", "prefill", "m23", "m8")


def measure_configs(qk, sweep: DecodeSweep, stream, only=None):
    """The other workloads (single Q4_K / Q6_K mat-vecs, the FFN sweep, the
    prefill GEMMs, the M = 8 decode sweep), reported beside the headline sweep;
    `only` names one part of CONFIG_PARTS (for a profiler run of that part)."""
    out = {}
    run = lambda part: only is None or only == part
    if run("gemv"):
        out["0_q4k_gemv"] = single_gemv(qk, stream, Q4, 2560, 9728, 0)
        out["1_q6k_gemv"] = single_gemv(qk, stream, Q6, 9728, 2560, 1)
    if run("ffn"):
        separate = DecodeSweep(qk, M=1, weights_of=sweep, fused_ffn=False)
        for key, src, fams in (("2_ffn_block_sweep", sweep, ("ffn_block",)),
                               ("2_ffn_block_sweep_two_launches", separate, ("ffn_gate_up", "ffn_down"))):
            ffn = [op for op in src.ops(stream) if op.family in fams]
            us = time_launches(qk, stream, [op.call for op in ffn]) * len(ffn)
            nbytes = sum(op.nbytes for op in ffn)
            out[key] = {"shape": f"36 x (gate+up SiLU, down), M=1, {len(ffn) // 36} launch(es) per layer",
                        "us_per_sweep": round(us, 1), "us_per_layer": round(us / 36, 2),
                        "GB/s": round(nbytes / (us * 1e3), 1), "frac": round(nbytes / (us * 1e3) / PEAK_HBM_GBS, 4)}
    if run("prefill"):
        out["3_prefill_gemm"] = prefill_gemm(qk, stream)
    if run("m23"):
        out["3_prefill_m23"] = prefill_small_m(qk, sweep, stream)
    if run("m8"):
        sweep8 = DecodeSweep(qk, M=8, weights_of=sweep)
        graph = qk.Graph.capture(stream, lambda: sweep8.record(stream))
        ms = time_graph(qk, graph, stream, 2, 10)
        graph.destroy()
        out["4_decode_sweep_m8"] = {"ms_per_step": round(ms, 4), "tokens_per_s": round(8e3 / ms, 1),
                                    "GB/s": round(sweep8.bytes_per_step() / (ms * 1e6), 1),
                                    "kernels": kernel_roofline(qk, sweep8, stream)}
    return out


CPU_LAYERS = 8  # layers cycled by the CPU baseline: 8 x 64 MB, more than a host's L3


def cpu_baseline(qk, sweep: DecodeSweep, budget_s: float):
    """The CPU oracle (OpenMP over output rows, double accumulation) on a
    bounded sample of the same workload. One run = the 7 projections of one
    layer at M = 1 (64 MB of weights); runs cycle over CPU_LAYERS distinct
    layers so the host's caches do not hold the weights; one warm-up run,
    then runs until ~budget_s, reported as the median run's rate."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import qk_oracle  # checker only: CPU baseline leg

    qk_oracle.load()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or os.cpu_count()
    rng_x = {K: qk_oracle.synth_normal(K, SEED + K) for K in (2560, 4096, 9728)}
    layers = [[(qtype, K, N, sweep.layers[l][name].download(np.uint8)) for name, qtype, K, N in LAYER]
              for l in range(CPU_LAYERS)]
    run_bytes = sum(gemv_bytes(qtype, K, N, 1) for _, qtype, K, N in LAYER)

    def run(l, product):
        t0 = time.perf_counter()
        for qtype, K, N, w in layers[l % CPU_LAYERS]:
            product(rng_x[K], w, qtype, K, N, threads=threads)
        return time.perf_counter() - t0

    run(0, qk_oracle.reference_product)  # warm-up
    times, total = [], 0.0
    while total < budget_s or len(times) < 5:
        t = run(len(times) + 1, qk_oracle.reference_product)
        times.append(t)
        total += t
    f32 = [run(l, qk_oracle.reference_product_f32) for l in range(1, 6)]
    gbs = run_bytes / float(np.median(times)) / 1e9
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": f"oracle reference_product (Q8 round trip, dequant, double accumulation) of the 7 "
                  f"projections of one layer at M=1 ({run_bytes / 1e6:.1f} MB), cycling over {CPU_LAYERS} "
                  f"distinct layers; median of {len(times)} runs after 1 warm-up ({total:.1f} s)",
        "runs": len(times), "min_run_GB/s": round(run_bytes / min(times) / 1e9, 3),
        "tokens_per_s": round(gbs * 1e9 / sweep.bytes_per_step(), 3),
        "fp32_accumulation_GB/s": round(run_bytes / float(np.median(f32)) / 1e9, 3),
        "cpu": cpu,
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline budget (0 = skip)")
    ap.add_argument("--no-roofline", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the other workloads")
    ap.add_argument("--only-config", choices=CONFIG_PARTS,
                    help="run only this part of the other workloads and print its results (no headline line)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the path would shard over output rows, with no exchange inside a mat-vec)",
              file=sys.stderr)
        return 2

    qk = load_package()
    info = qk.device_info()
    log(f"device {info}")
    t0 = time.perf_counter()
    sweep = DecodeSweep(qk, M=1)
    log(f"weights ready ({sweep.bytes_per_step() / 1e9:.3f} GB/step) in {time.perf_counter() - t0:.1f} s")
    stream = qk.Stream()
    if args.only_config:
        print(json.dumps({"configs": measure_configs(qk, sweep, stream, only=args.only_config)}), flush=True)
        stream.destroy()
        return 0

    # eager step (host-enqueued launch by launch), for reference
    sweep.record(stream)
    stream.synchronize()
    e0 = time.perf_counter()
    sweep.record(stream)
    stream.synchronize()
    eager_ms = (time.perf_counter() - e0) * 1e3

    reference_copy(qk, stream)
    graph = qk.Graph.capture(stream, lambda: sweep.record(stream))
    ms = time_graph(qk, graph, stream, args.warmup, args.steps)
    bytes_step = sweep.bytes_per_step()
    gbs = bytes_step / (ms * 1e-3) / 1e9
    log(f"graph step {ms:.4f} ms -> {gbs:.1f} GB/s, {1e3 / ms:.1f} tok/s (eager step {eager_ms:.2f} ms)")

    # the same step through the unmodified engine's calls (no fused entry points)
    dropin = DecodeSweep(qk, M=1, weights_of=sweep, engine_calls=True)
    dgraph = qk.Graph.capture(stream, lambda: dropin.record(stream))
    dropin_ms = time_graph(qk, dgraph, stream, args.warmup, args.steps)
    dgraph.destroy()
    log(f"drop-in (engine calls unchanged) step {dropin_ms:.4f} ms")
    # the bounded waits of the timed replays (FFN grid barrier, argmax
    # collector): each check reports and clears a timed-out wait
    timeouts = 0
    for ws, check in ((sweep.ffn_ws, qk.ffn_workspace_check), (sweep.argmax_ws, qk.argmax_workspace_check),
                      (dropin.argmax_ws, qk.argmax_workspace_check)):
        try:
            check(ws, stream)
        except qk.QKError as e:
            timeouts += 1
            log(f"timed-out wait reported: {e}")

    roofline, kernels = None, None
    if not args.no_roofline:
        kernels = kernel_roofline(qk, sweep, stream)
        dominant = max(kernels, key=lambda k: kernels[k]["total_us_per_step"])
        d = kernels[dominant]
        roofline = {"bound": "hbm", "achieved": d["GB/s"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                    "frac": d["frac"], "traffic": measured_traffic(dominant),
                    "traffic_source": "profiles/traffic_decode_sweep_m1.json: FETCH_SIZE and WRITE_SIZE "
                                      "rocprofv3 runs of this script, scaled by a 256 MiB copy (not "
                                      "re-measured in a plain run)",
                    "kernel": dominant,
                    "avg_launch_us": d["avg_us"], "avg_bytes_per_launch": d["avg_bytes"]}
        log(f"kernels: {json.dumps(kernels)}")

    configs = None
    if not args.no_configs:
        configs = measure_configs(qk, sweep, stream)
        log(f"configs: {json.dumps(configs)}")

    baseline = None
    if args.cpu_seconds > 0:
        log("CPU baseline (oracle, OpenMP) ...")
        baseline = cpu_baseline(qk, sweep, args.cpu_seconds)
        log(f"CPU baseline {baseline}")

    graph.destroy()
    stream.destroy()
    line = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "Qwen3-4B Q4_K_M decode projection sweep, M=1: 36 x (q,k,v,o,gate,up,down) "
                               "+ lm_head 151936x2560 Q6_K with next-token argmax, Q8 activations, "
                               "3 launches/layer (qkv, o, FFN block) + 1, graph-replayed",
                   "tokens_per_s": round(1e3 / ms, 2), "bytes_per_step": bytes_step,
                   "dropin_ms_per_step": round(dropin_ms, 5),
                   "dropin_note": "the same step through the engine's unmodified calls (src/Engine.cpp:83-110): "
                                  "9 qk_matmul + qk_silu_multiply per layer, lm_head qk_matmul + qk_argmax",
                   "barrier_timeouts": timeouts,
                   "frac_of_peak_hbm": round(gbs / PEAK_HBM_GBS, 4), "eager_ms_per_step": round(eager_ms, 3),
                   "device": info["name"], "arch": info["arch"]},
        "roofline": roofline,
        "cpu_baseline": baseline,
        "kernels": kernels,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
