"""Pins the CPU oracle (oracle/qk_oracle.c) before it is trusted as the checker.

The reference ships no golden vectors for this path (its tests read the real
model file), so each oracle function is pinned by something that a plausible
mistake would fail:
  - fp16 widening: exhaustive against numpy over all 65536 patterns;
  - superblock layouts: blocks written by ggml-side packers (tests/ggml_layout.py)
    with d = 1 so every weight is a small exact integer;
  - closed-form blocks (zero d, fp16 subnormal d = 2^-24, all-ones codes);
  - Q8: the amax element maps to +-127, zero blocks, half-away-from-zero ties,
    and agreement of the two reference statements (GPU quantize vs CPU round trip);
  - product: exact rational brute force on tiny shapes, a float64 dense matmul,
    and the reference GPU kernel's integer decomposition (src/cuda/matmul.cu)
    as a second, independent statement of the bit layout;
  - the synthetic generator: SplitMix64's published test vector.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest

from ggml_layout import f16_bits, pack_q4k, pack_q6k

Q4, Q6 = 12, 14


# ------------------------------------------------------------------- fp16 --

def test_fp16_widening_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expected = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.fp16_to_fp32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(expected)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), expected[~nan].view(np.uint32))


def test_fp16_narrowing_round_to_nearest_even(oracle):
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.uniform(0, 0.01, 4000).astype(np.float32),            # d ~ U(0, 0.01)
        rng.uniform(0, 6.2e-5, 2000).astype(np.float32),          # fp16 subnormal range
        (rng.standard_normal(2000) * 1000).astype(np.float32),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -26, 2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11],
                 dtype=np.float32),
    ])
    with np.errstate(over="ignore"):
        expected = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.fp32_to_fp16(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, expected)


# ------------------------------------------------------------ Q4_K layout --

def test_q4k_layout_from_ggml_packer(oracle):
    rng = np.random.default_rng(11)
    blocks, expected = [], []
    for _ in range(64):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        L = rng.integers(0, 16, 256)
        blocks.append(pack_q4k(f16_bits(1.0), f16_bits(1.0), sc, mn, L))
        g = np.arange(256) // 32
        expected.append((sc[g] * L - mn[g]).astype(np.float32))
    packed = np.frombuffer(b"".join(blocks), dtype=np.uint8)
    got = oracle.dequantize(packed, Q4, 1, 256 * 64)
    assert np.array_equal(got.ravel(), np.concatenate(expected))


def test_q4k_scale_unpack_is_the_inverse_of_the_packer(oracle):
    rng = np.random.default_rng(12)
    for _ in range(200):
        sc = rng.integers(0, 64, 8)
        mn = rng.integers(0, 64, 8)
        block = pack_q4k(0, 0, sc, mn, [0] * 256)
        for g in range(8):
            assert oracle.scale_min_k4(g, block[4:16]) == (sc[g], mn[g])


def test_q4k_closed_forms(oracle):
    L = np.arange(256) % 16
    # d = 1, dmin = 0, every sc = 1: w = q
    b = pack_q4k(f16_bits(1.0), 0, [1] * 8, [0] * 8, L)
    assert np.array_equal(oracle.dequantize(np.frombuffer(b, np.uint8), Q4, 1, 256)[0], L)
    # qs = 0, dmin = 1, m = k: w = -k
    mn = list(range(3, 11))
    b = pack_q4k(f16_bits(1.0), f16_bits(1.0), [5] * 8, mn, [0] * 256)
    got = oracle.dequantize(np.frombuffer(b, np.uint8), Q4, 1, 256)[0]
    assert np.array_equal(got, -np.repeat(mn, 32).astype(np.float32))
    # d = 0 and dmin = 0: all zeros
    b = pack_q4k(0, 0, [63] * 8, [63] * 8, [15] * 256)
    assert not np.any(oracle.dequantize(np.frombuffer(b, np.uint8), Q4, 1, 256))
    # smallest fp16 subnormal d = 2^-24: w = q * 2^-24 exactly (no flush to zero)
    b = pack_q4k(0x0001, 0, [1] * 8, [0] * 8, L)
    got = oracle.dequantize(np.frombuffer(b, np.uint8), Q4, 1, 256)[0]
    assert np.array_equal(got, (L * 2.0 ** -24).astype(np.float32))


# ------------------------------------------------------------ Q6_K layout --

def test_q6k_layout_from_ggml_packer(oracle):
    rng = np.random.default_rng(13)
    blocks, expected = [], []
    for _ in range(64):
        L = rng.integers(0, 64, 256)
        scales = rng.integers(-128, 128, 16)
        blocks.append(pack_q6k(L, scales, f16_bits(1.0)))
        expected.append((scales[np.arange(256) // 16] * (L - 32)).astype(np.float32))
    packed = np.frombuffer(b"".join(blocks), dtype=np.uint8)
    got = oracle.dequantize(packed, Q6, 1, 256 * 64)
    assert np.array_equal(got.ravel(), np.concatenate(expected))


def test_q6k_closed_forms(oracle):
    zero = bytes(192) + bytes([1] * 16) + bytes([0x00, 0x3C])   # ql=qh=0, sc=1, d=1
    got = oracle.dequantize(np.frombuffer(zero, np.uint8), Q6, 1, 256)[0]
    assert np.all(got == -32.0)
    ones = bytes([0xFF] * 192) + bytes([1] * 16) + bytes([0x00, 0x3C])
    got = oracle.dequantize(np.frombuffer(ones, np.uint8), Q6, 1, 256)[0]
    assert np.all(got == 31.0)
    dzero = bytes([0xA5] * 192) + bytes([7] * 16) + bytes([0, 0])
    assert not np.any(oracle.dequantize(np.frombuffer(dzero, np.uint8), Q6, 1, 256))
    L = np.arange(256) % 64
    sub = pack_q6k(L, [1] * 16, 0x0001)
    got = oracle.dequantize(np.frombuffer(sub, np.uint8), Q6, 1, 256)[0]
    assert np.array_equal(got, ((L - 32) * 2.0 ** -24).astype(np.float32))


def test_dequantize_rows_stride_and_errors(oracle):
    w = oracle.synth_superblocks(Q4, 4, 512, seed=5, dmax=0.01, dminmax=0.01)
    dense = oracle.dequantize(w, Q4, 4, 512)
    padded = np.zeros((4, 400), dtype=np.uint8)  # row stride 400 > 288 packed bytes
    padded[:, :288] = w.reshape(4, 288)
    assert np.array_equal(oracle.dequantize(padded.ravel(), Q4, 4, 512, stride=400), dense)
    lib = oracle.load()
    out = np.empty(256, dtype=np.float32)
    assert lib.qko_dequantize_rows(w.ctypes.data, out.ctypes.data, 0, 256, 144, 99) == 0
    assert lib.qko_dequantize_rows(w.ctypes.data, out.ctypes.data, 1, 256, 144, 99) == 2


# ---------------------------------------------------------------------- Q8 --

def _q8_numpy(x: np.ndarray):
    """float32 statement of src/cuda/matmul.cu:8-22 with explicit half-away rounding."""
    xb = x.reshape(-1, 32).astype(np.float32)
    amax = np.max(np.abs(xb), axis=1).astype(np.float32)
    safe = np.where(amax == 0, np.float32(1), amax)
    t = ((xb / safe[:, None]).astype(np.float32) * np.float32(127)).astype(np.float32)
    r = np.sign(t) * np.floor(np.abs(t).astype(np.float64) + 0.5)
    codes = np.where(amax[:, None] == 0, 0, r).astype(np.int8)
    return codes.ravel(), (amax / np.float32(127)).astype(np.float32)


def test_q8_matches_float32_statement(oracle):
    rng = np.random.default_rng(21)
    x = rng.standard_normal(32 * 4096).astype(np.float32)
    x[:32] = 0.0
    codes, scales = oracle.quantize_q8(x)
    ecodes, escales = _q8_numpy(x)
    assert np.array_equal(codes, ecodes)
    assert np.array_equal(scales.view(np.uint32), escales.view(np.uint32))


def test_q8_properties(oracle):
    rng = np.random.default_rng(22)
    x = rng.standard_normal(32 * 512).astype(np.float32)
    codes, scales = oracle.quantize_q8(x)
    cb = codes.reshape(-1, 32)
    xb = x.reshape(-1, 32)
    at = np.argmax(np.abs(xb), axis=1)
    # the amax element is +-127
    assert np.array_equal(cb[np.arange(len(cb)), at], np.where(xb[np.arange(len(xb)), at] > 0, 127, -127))
    z_codes, z_scales = oracle.quantize_q8(np.zeros(64, np.float32))
    assert not np.any(z_codes) and not np.any(z_scales)


def test_q8_ties_round_away_from_zero(oracle):
    """Find inputs whose fl(fl(x/amax)*127) is exactly k + 0.5 and check the code."""
    rng = np.random.default_rng(23)
    amax = np.float32(1.0)
    found = 0
    for k in range(0, 126):
        for cand in (np.float32((k + 0.5) / 127.0),
                     np.nextafter(np.float32((k + 0.5) / 127.0), np.float32(2)),
                     np.nextafter(np.float32((k + 0.5) / 127.0), np.float32(0))):
            t = np.float32(np.float32(cand / amax) * np.float32(127))
            if t == np.float32(k + 0.5):
                for sign in (1, -1):
                    block = rng.uniform(-0.5, 0.5, 32).astype(np.float32) * 0
                    block[0] = amax
                    block[1] = np.float32(sign * cand)
                    codes, _ = oracle.quantize_q8(block)
                    assert codes[1] == sign * (k + 1)
                    rt = oracle.q8_roundtrip(block)
                    assert rt[1] == np.float32(np.float32(sign * (k + 1)) * np.float32(amax / np.float32(127)))
                found += 1
    assert found >= 10


def test_roundtrip_equals_codes_times_scale(oracle):
    """MatmulReference.hpp's round trip and matmul.cu's codes describe the same numbers."""
    rng = np.random.default_rng(24)
    x = (rng.standard_normal(32 * 2048) * rng.uniform(0.01, 100, 32 * 2048)).astype(np.float32)
    codes, scales = oracle.quantize_q8(x)
    rt = oracle.q8_roundtrip(x)
    expected = (codes.astype(np.float32).reshape(-1, 32) * scales[:, None]).astype(np.float32)
    # equal as numbers; the round trip keeps the sign of a rounded-away -0.0
    assert np.array_equal(rt, expected.ravel())
    nz = expected.ravel() != 0
    assert np.array_equal(rt[nz].view(np.uint32), expected.ravel()[nz].view(np.uint32))


# ----------------------------------------------------------------- product --

@pytest.mark.parametrize("qtype", [Q4, Q6])
def test_reference_product_exact_small(oracle, qtype):
    K, N, M = 256, 3, 2
    w = oracle.synth_superblocks(qtype, N, K, seed=31, dmax=0.01, dminmax=0.01)
    x = oracle.synth_normal(M * K, seed=32)
    y = oracle.reference_product(x, w, qtype, K, N)
    q = oracle.q8_roundtrip(x).reshape(M, K)
    dq = oracle.dequantize(w, qtype, N, K)
    for m in range(M):
        for n in range(N):
            exact = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(q[m], dq[n]))
            assert abs(y[m, n] - float(exact)) <= 1e-12 * max(1.0, abs(float(exact)))


@pytest.mark.parametrize("qtype,K,N,M", [(Q4, 512, 37, 3), (Q6, 768, 29, 4)])
def test_reference_product_matches_dense(oracle, qtype, K, N, M):
    w = oracle.synth_superblocks(qtype, N, K, seed=41, dmax=0.01, dminmax=0.01)
    x = oracle.synth_normal(M * K, seed=42)
    y = oracle.reference_product(x, w, qtype, K, N)
    dense = oracle.q8_roundtrip(x).reshape(M, K).astype(np.float64) @ \
        oracle.dequantize(w, qtype, N, K).astype(np.float64).T
    assert np.allclose(y, dense, rtol=1e-12, atol=1e-12)
    assert np.array_equal(oracle.reference_product(x, w, qtype, K, N, threads=1), y)


@pytest.mark.parametrize("qtype,K,N,M", [(Q4, 2560, 64, 2), (Q6, 2560, 64, 2), (Q6, 9728, 16, 1)])
def test_integer_decomposition_agrees(oracle, qtype, K, N, M):
    """matmul.cu's dp4a decomposition and embedding.cu's dequant formula agree."""
    w = oracle.synth_superblocks(qtype, N, K, seed=51, dmax=0.01, dminmax=0.01)
    x = oracle.synth_normal(M * K, seed=52)
    ref = oracle.reference_product(x, w, qtype, K, N)
    got = oracle.integer_product(x, w, qtype, K, N)
    assert oracle.row_norm_error(got, ref) < 1e-5
    f32 = oracle.reference_product_f32(x, w, qtype, K, N)
    assert oracle.row_norm_error(f32, ref) < 1e-5


@pytest.mark.parametrize("qtype", [Q4, Q6])
def test_zero_input_gives_exact_zero(oracle, qtype):
    w = oracle.synth_superblocks(qtype, 5, 512, seed=61, dmax=0.01, dminmax=0.01)
    x = np.zeros(3 * 512, np.float32)
    assert not np.any(oracle.reference_product(x, w, qtype, 512, 5))
    assert not np.any(oracle.integer_product(x, w, qtype, 512, 5))


def test_product_rejects_bad_shapes(oracle):
    lib = oracle.load()
    x = np.zeros(256, np.float32)
    w = np.zeros(144, np.uint8)
    y = np.zeros(1, np.float64)
    assert lib.qko_reference_product(x.ctypes.data, w.ctypes.data, 99, 256, 1, 1, y.ctypes.data, 1) == 2
    assert lib.qko_reference_product(x.ctypes.data, w.ctypes.data, Q4, 100, 1, 1, y.ctypes.data, 1) == 1
    assert lib.qko_reference_product(x.ctypes.data, w.ctypes.data, Q4, 256, 0, 1, y.ctypes.data, 1) == 1


# -------------------------------------------------------------- synthetic --

def test_splitmix64_published_vector(oracle):
    # SplitMix64 seeded with 1234567 (Vigna's reference implementation)
    expected = [6457827717110365317, 3203168211198807973, 9817491932198370423,
                4593380528125082431, 16408922859458223821]
    assert [oracle.word(1234567, i) for i in range(5)] == expected


def test_synth_layout(oracle):
    seed, dmax, dminmax = 20261201, 0.01, 0.005
    w = oracle.synth_superblocks(Q4, 3, 512, seed, dmax, dminmax).reshape(6, 144)
    for b in range(6):
        u = lambda i: np.float32((oracle.word(seed, 20 * b + i) >> 40) * 2.0 ** -24)
        assert int(w[b, 0]) | int(w[b, 1]) << 8 == f16_bits(np.float32(u(0) * np.float32(dmax)))
        assert int(w[b, 2]) | int(w[b, 3]) << 8 == f16_bits(np.float32(u(1) * np.float32(dminmax)))
        w2 = oracle.word(seed, 20 * b + 2).to_bytes(8, "little")
        assert bytes(w[b, 4:12]) == w2
        assert bytes(w[b, 16:24]) == oracle.word(seed, 20 * b + 4).to_bytes(8, "little")
    w6 = oracle.synth_superblocks(Q6, 2, 512, seed, 0.005).reshape(4, 210)
    sc = w6[:, 192:208].view(np.int8)
    assert sc.min() >= -64 and sc.max() <= 63
    assert bytes(w6[1, 0:8]) == oracle.word(seed, 27 + 0).to_bytes(8, "little")
    x = oracle.synth_normal(100000, 3)
    assert abs(float(x.mean())) < 0.02 and abs(float(x.std()) - 1.0) < 0.02


# -------------------------------------------------------------- neighbours --

def test_silu_and_argmax(oracle):
    rng = np.random.default_rng(71)
    g = rng.standard_normal(4096).astype(np.float32) * 4
    u = rng.standard_normal(4096).astype(np.float32)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert np.allclose(oracle.silu_multiply(g, u), ref, rtol=1e-6, atol=1e-7)
    v = np.array([1, 5, 3, 5, -1], np.float32)
    assert oracle.argmax(v) == 1


def test_argmax_follows_the_reference_candidate_rules(oracle):
    """src/cuda/argmax.cu: start (SIZE_MAX, -inf), replace on strictly greater,
    lower index on ties; the uint32_t return turns SIZE_MAX into 0xFFFFFFFF."""
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    assert oracle.argmax(np.array([nan, 2, nan, 3, 3], np.float32)) == 3      # NaN never wins
    assert oracle.argmax(np.array([-inf, -inf, -7], np.float32)) == 2        # -inf never wins
    assert oracle.argmax(np.array([-inf, nan], np.float32)) == 0xFFFFFFFF    # nothing wins
    assert oracle.argmax(np.array([], np.float32)) == 0xFFFFFFFF
    assert oracle.argmax(np.array([-0.0, 0.0, -1], np.float32)) == 0         # -0 == +0: first
    assert oracle.argmax(np.array([1, inf, inf], np.float32)) == 1
    rng = np.random.default_rng(5)
    for _ in range(20):
        v = rng.integers(-3, 4, 1000).astype(np.float32)   # many ties
        assert oracle.argmax(v) == int(np.argmax(v))       # numpy: first maximal index


def test_rms_norm_oracle(oracle):
    """qko_rms_norm (src/cuda/rms_norm.cu:6-24) pinned by a float64
    restatement, a closed form and two invariants: a constant row a gives
    a / sqrt(a^2 + eps) * w; rows come out with unit RMS (w = 1, small eps);
    eps dominating a tiny row leaves it almost unscaled by the mean."""
    rng = np.random.default_rng(5)
    width, rows, eps = 2560, 3, 1e-6
    x = rng.standard_normal(rows * width).astype(np.float32) * 3.0
    w = rng.uniform(0.5, 1.5, width).astype(np.float32)
    got = oracle.rms_norm(x, w, width, eps).reshape(rows, width)
    xr = x.reshape(rows, width).astype(np.float64)
    ref = xr / np.sqrt(np.mean(xr * xr, axis=1, keepdims=True) + eps) * w.astype(np.float64)
    assert np.max(np.abs(got - ref) / np.abs(ref).max()) < 1e-6
    ones = np.ones(width, np.float32)
    unit = oracle.rms_norm(x, ones, width, eps).reshape(rows, width).astype(np.float64)
    assert np.allclose(np.sqrt(np.mean(unit * unit, axis=1)), 1.0, rtol=1e-5)
    const = oracle.rms_norm(np.full(width, 2.0, np.float32), w, width, 0.25)
    assert np.allclose(const, 2.0 / np.sqrt(4.25) * w, rtol=1e-6)
    tiny = np.full(width, 1e-4, np.float32)
    out = oracle.rms_norm(tiny, ones, width, 1.0)  # mean 1e-8 << eps = 1
    assert np.allclose(out, 1e-4 / np.sqrt(1.0 + 1e-8), rtol=1e-6)


def test_q8_scale_invariance_behind_the_norm_fold(oracle):
    """The fused FFN's RMSNorm fold quantises x * scale and multiplies the row
    totals by inv_rms: it relies on Q8(c * v) = (codes(v), c * scales(v)).
    For c a power of two this holds bit for bit; for a general c > 0 codes
    may step only where 127 * v / amax sits within rounding of a half."""
    rng = np.random.default_rng(11)
    v = (rng.standard_normal(32 * 512) * np.exp(rng.uniform(-8, 8, 32 * 512))).astype(np.float32)
    codes, scales = oracle.quantize_q8(v)
    for c in (2.0 ** -20, 0.5, 8.0, 2.0 ** 30):
        c_codes, c_scales = oracle.quantize_q8(v * np.float32(c))
        assert np.array_equal(c_codes, codes)
        assert np.array_equal(c_scales, (scales * np.float32(c)).astype(np.float32))
    c = np.float32(0.037)
    c_codes, c_scales = oracle.quantize_q8(v * c)
    assert np.allclose(c_scales, scales * c, rtol=2e-7, atol=0)
    t = 127.0 * v.astype(np.float64) / np.repeat(scales.astype(np.float64) * 127.0, 32)
    moved = c_codes != codes
    assert np.all(np.abs(c_codes[moved].astype(int) - codes[moved]) == 1)
    assert np.all(np.abs(np.abs(t[moved] - np.floor(t[moved])) - 0.5) < 1e-4)
    assert moved.mean() < 1e-3
