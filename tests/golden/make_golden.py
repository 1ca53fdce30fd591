"""Writes tests/golden/q4k_q6k_small.npz: small Q4_K / Q6_K fixtures whose
expected values come from closed forms, not from the oracle.

The reference holds no golden vectors (its tests compute references at run
time from a model file), so these are the build's own. Weights are packed
from chosen (d, dmin, scales, codes) with the writer-side packers of
tests/ggml_layout.py (ggml's block_q4_K / block_q6_K layout), and the
expected dequantised weights are formed from those same values:
  Q4_K w = (d*sc)*q - dmin*m     (src/cuda/embedding.cu:20-31; every product
                                  exact in fp32, one rounding in the subtract)
  Q6_K w = (d*sc)*(q - 32)       (src/cuda/embedding.cu:45-58; exact)
The activations are the reference's own make_input formula, sin(i*0.031)*0.1
in float (src/tests/reference/MatmulReference.hpp:31-39), plus a wide-range
row; their Q8 round trip is round(x/amax*127)*(amax/127) in float with
round-half-away-from-zero (MatmulReference.hpp:11-29), and the products are
double sums of the round trip times the weights (MatmulReference.hpp:42-64).
Rows include these closed-form cases: d = 1, dmin = 0, sc = 1 (w
= q); sc = 0, dmin = 1, m = k (w = -k); the smallest fp16 subnormal d; Q6_K
all-zero and all-ones codes (w = -32, w = 31); d = 0; negative int8 scales.

Run from the repository root: python3 tests/golden/make_golden.py
"""
from __future__ import annotations

import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
from ggml_layout import f16_bits, pack_q4k, pack_q6k  # noqa: E402

K = 512          # two superblocks per row
S = K // 256
M = 3            # activation rows
OUT = HERE / "q4k_q6k_small.npz"


def f16(bits: int) -> np.float32:
    return np.float32(np.array([bits], dtype=np.uint16).view(np.float16)[0])


def q4k_rows(rng):
    """(bytes [N, S*144], w [N, K] fp32) for the Q4_K rows."""
    rows = []
    tiny = 1  # fp16 bits of 2^-24

    def add(blocks):
        rows.append(blocks)

    # w = q: d = 1, dmin = 0, sc = 1, m = 0
    add([(f16_bits(1.0), 0, [1] * 8, [0] * 8, list(rng.integers(0, 16, 256))) for _ in range(S)])
    # w = -m: sc = 0, dmin = 1, m = sub-block index
    add([(0x0000, f16_bits(1.0), [0] * 8, list(range(8)), list(rng.integers(0, 16, 256))) for _ in range(S)])
    # smallest subnormal d and dmin, the largest scales and mins
    add([(tiny, tiny, [63] * 8, [63] * 8, list(rng.integers(0, 16, 256))) for _ in range(S)])
    # d = 0, dmin = 0: all zeros
    add([(0, 0, list(rng.integers(0, 64, 8)), list(rng.integers(0, 64, 8)), list(rng.integers(0, 16, 256)))
         for _ in range(S)])
    # random blocks, d and dmin as the synthetic generator draws them
    for _ in range(4):
        add([(f16_bits(float(rng.uniform(0, 0.01))), f16_bits(float(rng.uniform(0, 0.01))),
              list(rng.integers(0, 64, 8)), list(rng.integers(0, 64, 8)), list(rng.integers(0, 16, 256)))
             for _ in range(S)])
    packed = np.zeros((len(rows), S * 144), np.uint8)
    w = np.zeros((len(rows), K), np.float32)
    for n, blocks in enumerate(rows):
        for s, (d, dmin, sc, mn, L) in enumerate(blocks):
            packed[n, 144 * s:144 * (s + 1)] = np.frombuffer(pack_q4k(d, dmin, sc, mn, L), np.uint8)
            for p in range(256):
                g = p // 32
                a = f16(d) * np.float32(sc[g]) * np.float32(L[p])       # exact
                b = f16(dmin) * np.float32(mn[g])                       # exact
                w[n, 256 * s + p] = np.float32(a - b)                   # one rounding
    return packed, w


def q6k_rows(rng):
    rows = []

    def add(blocks):
        rows.append(blocks)

    one = f16_bits(1.0)
    add([([0] * 256, [1] * 16, one) for _ in range(S)])           # codes 0: w = -32
    add([([63] * 256, [1] * 16, one) for _ in range(S)])          # codes 63: w = 31
    add([(list(rng.integers(0, 64, 256)), list(rng.integers(-128, 128, 16)), one) for _ in range(S)])
    add([(list(rng.integers(0, 64, 256)), list(rng.integers(-64, 64, 16)), 1) for _ in range(S)])  # tiny d
    add([(list(rng.integers(0, 64, 256)), list(rng.integers(-64, 64, 16)), 0) for _ in range(S)])  # d = 0
    for _ in range(3):
        add([(list(rng.integers(0, 64, 256)), list(rng.integers(-64, 64, 16)),
              f16_bits(float(rng.uniform(0, 0.005)))) for _ in range(S)])
    packed = np.zeros((len(rows), S * 210), np.uint8)
    w = np.zeros((len(rows), K), np.float32)
    for n, blocks in enumerate(rows):
        for s, (L, scales, d) in enumerate(blocks):
            packed[n, 210 * s:210 * (s + 1)] = np.frombuffer(pack_q6k(L, scales, d), np.uint8)
            for p in range(256):
                w[n, 256 * s + p] = f16(d) * np.float32(scales[p // 16]) * np.float32(L[p] - 32)  # exact
    return packed, w


def q8_roundtrip(x: np.ndarray):
    """(codes int8, block scales fp32, round trip fp32) in float, as the reference."""
    blocks = x.reshape(-1, 32).astype(np.float32)
    amax = np.max(np.abs(blocks), axis=1).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        t = (blocks / amax[:, None]).astype(np.float32) * np.float32(127.0)
    t = t.astype(np.float32).astype(np.float64)  # roundf in double: |t| + 0.5 exact
    codes = np.where(amax[:, None] == 0, 0, np.sign(t) * np.floor(np.abs(t) + 0.5))
    scale = (amax / np.float32(127.0)).astype(np.float32)
    rt = (codes.astype(np.float32) * scale[:, None]).astype(np.float32)
    return codes.astype(np.int8).reshape(x.shape), scale.reshape(x.shape[0], -1), rt.reshape(x.shape)


def activations(rng):
    x = np.zeros((M, K), np.float32)
    i = np.arange(2 * K, dtype=np.float32)
    x[:2] = (np.sin(i * np.float32(0.031)).astype(np.float32) * np.float32(0.1)).reshape(2, K)
    x[2] = (rng.standard_normal(K) * np.exp(rng.uniform(-8, 8, K))).astype(np.float32)
    x[2, 32:64] = 0.0  # an all-zero block
    return x


def build():
    rng = np.random.default_rng(20261201)
    q4, w4 = q4k_rows(rng)
    q6, w6 = q6k_rows(rng)
    x = activations(rng)
    codes, scales, rt = q8_roundtrip(x)
    y4 = rt.astype(np.float64) @ w4.astype(np.float64).T
    y6 = rt.astype(np.float64) @ w6.astype(np.float64).T
    return dict(K=np.int64(K), q4k=q4, q4k_w=w4, q6k=q6, q6k_w=w6, x=x, x_codes=codes, x_scales=scales,
                x_rt=rt, y_q4k=y4, y_q6k=y6)


if __name__ == "__main__":
    np.savez_compressed(OUT, **build())
    print(f"wrote {OUT}")
