"""One Qwen3-4B layer and the lm_head run two ways on the same weights and
activations: the reference engine's calls unchanged (src/Engine.cpp:83-85,94,
98-101,109-110: q, k and v as three kernels::matmul calls, attn_output, gate and
up as two matmuls, silu_multiply, down, the lm_head matmul into logits, then
argmax) and the fused entry points the decode benchmark uses (qk_matmul_segments
for q/k/v, qk_ffn for the FFN block, qk_matmul_argmax for the lm_head).

At one activation row both sequences form every output row from the same
superblock sums in the same fixed order, so they agree bit for bit: q, k, v,
h = SiLU(gate) * up, the block's y and the next-token index. At several rows
(M = 3 and 8: other kernels) the outputs agree within the mat-vec's rounding,
and both are checked against the oracle's product for the narrow projections.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

Q4, Q6 = 12, 14
SEED = 20261300
# (name, type, K, N): the Qwen3-4B Q4_K_M layer of src/Engine.cpp:83-101
LAYER = [("attn_q", Q4, 2560, 4096), ("attn_k", Q4, 2560, 1024), ("attn_v", Q6, 2560, 1024),
         ("attn_output", Q4, 4096, 2560), ("ffn_gate", Q4, 2560, 9728), ("ffn_up", Q4, 2560, 9728),
         ("ffn_down", Q6, 9728, 2560)]
LM_HEAD = (Q6, 2560, 151936)


class Layer:
    def __init__(self, qk, oracle, M, seed):
        self.qk, self.M = qk, M
        self.w = {}
        for i, (name, qtype, K, N) in enumerate(LAYER):
            w = qk.DeviceBuffer(N * qk.row_bytes(qtype, K))
            qk.synth_superblocks(w, qtype, N, K, seed + i, 0.01 if qtype == Q4 else 0.005, 0.01)
            self.w[name] = w
        qtype, K, N = LM_HEAD
        self.lm_head = qk.DeviceBuffer(N * qk.row_bytes(qtype, K))
        qk.synth_superblocks(self.lm_head, qtype, N, K, seed + 99, 0.005, 0.01)
        self.x = {k: (oracle.synth_normal(M * k, seed + 100 + k) * np.float32(2.0)).astype(np.float32)
                  for k in (2560, 4096)}
        self.xd = {k: qk.DeviceBuffer.from_array(v) for k, v in self.x.items()}

    def out(self, n):
        return self.qk.DeviceBuffer.from_array(np.full(self.M * n, np.nan, np.float32))

    def engine_calls(self):
        """src/Engine.cpp's sequence, every call unchanged."""
        qk, M, w = self.qk, self.M, self.w
        r = {}
        for name in ("attn_q", "attn_k", "attn_v"):
            _, qtype, K, N = next(t for t in LAYER if t[0] == name)
            r[name] = self.out(N)
            qk.matmul(self.xd[2560], w[name], qtype, K, N, r[name], M)
        gate, up, act, y = self.out(9728), self.out(9728), self.out(9728), self.out(2560)
        qk.matmul(self.xd[2560], w["ffn_gate"], Q4, 2560, 9728, gate, M)
        qk.matmul(self.xd[2560], w["ffn_up"], Q4, 2560, 9728, up, M)
        qk.silu_multiply(gate, up, act, M * 9728)
        qk.matmul(act, w["ffn_down"], Q6, 9728, 2560, y, M)
        r["h"], r["y"] = act, y
        if M == 1:
            qtype, K, N = LM_HEAD
            logits = qk.DeviceBuffer(4 * N)
            ws_bytes = qk.argmax_workspace_size()
            ws = qk.DeviceBuffer(ws_bytes)
            ws.fill(0)
            result = qk.DeviceBuffer(4)
            qk.matmul(self.xd[2560], self.lm_head, qtype, K, N, logits, 1)
            qk.argmax(logits, N, result, ws, ws_bytes)
            r["next"], r["logits"] = result, logits
        qk.synchronize()
        return {k: v.download(np.float32 if k != "next" else np.uint32) for k, v in r.items()}

    def fused_calls(self):
        """The fused entry points of the decode benchmark."""
        qk, M, w = self.qk, self.M, self.w
        r = {name: self.out(N) for name, _, _, N in LAYER[:3]}
        segs = [(w[name], qtype, N, r[name]) for name, qtype, _, N in LAYER[:3]]
        qk.matmul_segments(self.xd[2560], M, 2560, segs)
        ws_bytes = qk.ffn_workspace_size()
        ws = qk.DeviceBuffer(ws_bytes)
        qk.check(qk.load().qk_memset_async(ws.ptr, 0, ws_bytes, None))
        h, y = self.out(9728), self.out(2560)
        qk.ffn(self.xd[2560], None, 0.0, w["ffn_gate"], w["ffn_up"], Q4, w["ffn_down"], Q6, 2560, 9728, h, y, M,
               ws, ws_bytes)
        r["h"], r["y"] = h, y
        if M == 1:
            qtype, K, N = LM_HEAD
            aws_bytes = qk.argmax_workspace_size()
            aws = qk.DeviceBuffer(aws_bytes)
            aws.fill(0)
            result = qk.DeviceBuffer(4)
            qk.matmul_argmax(self.xd[2560], self.lm_head, qtype, K, N, None, result, aws, aws_bytes)
            r["next"] = result
        qk.synchronize()
        qk.ffn_workspace_check(ws)
        return {k: v.download(np.float32 if k != "next" else np.uint32) for k, v in r.items()}


def test_engine_calls_and_fused_calls_agree_bit_for_bit_at_one_row(gpu, oracle):
    layer = Layer(gpu, oracle, 1, SEED)
    print("[case] one layer + lm_head, M = 1: engine calls", flush=True)
    a = layer.engine_calls()
    print("[case] one layer + lm_head, M = 1: fused calls", flush=True)
    b = layer.fused_calls()
    for name in ("attn_q", "attn_k", "attn_v", "h", "y"):
        assert np.all(np.isfinite(a[name])), name
        assert np.array_equal(a[name].view(np.uint32), b[name].view(np.uint32)), name
    assert int(a["next"][0]) == int(b["next"][0])
    # and the index is the logits' first maximum
    assert int(a["next"][0]) == int(np.argmax(a["logits"]))
    # the narrow projections against the oracle's double-accumulated product
    for name, qtype, K, N in LAYER[1:3]:
        ref = oracle.reference_product(layer.x[K], layer.w[name].download(np.uint8), qtype, K, N)
        assert oracle.row_norm_error(a[name].reshape(1, N), ref) <= 1e-5, name


@pytest.mark.parametrize("M", [3, 8])
def test_engine_calls_and_fused_calls_agree_at_several_rows(gpu, oracle, M):
    layer = Layer(gpu, oracle, M, SEED + 10 * M)
    print(f"[case] one layer, M = {M}: engine calls, then fused calls", flush=True)
    a = layer.engine_calls()
    b = layer.fused_calls()
    for name, N in (("attn_q", 4096), ("attn_k", 1024), ("attn_v", 1024), ("h", 9728), ("y", 2560)):
        assert np.all(np.isfinite(b[name])), name
        assert oracle.row_norm_error(b[name].reshape(M, N), a[name].reshape(M, N)) <= 1e-5, name
    for name, qtype, K, N in LAYER[1:3]:
        ref = oracle.reference_product(layer.x[K], layer.w[name].download(np.uint8), qtype, K, N)
        assert oracle.row_norm_error(b[name].reshape(M, N), ref) <= 1e-5, name
