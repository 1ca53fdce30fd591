"""ctypes binding of the CPU oracle (oracle/libqk_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker of the HIP path. Nothing in the
product imports it. See qk_oracle.h for the reference file:line each function
restates.
"""
from __future__ import annotations

import ctypes
import pathlib

import numpy as np

ORACLE_DIR = pathlib.Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "libqk_oracle.so"

TYPE_Q4_K = 12
TYPE_Q6_K = 14
SUPERBLOCK_BYTES = {TYPE_Q4_K: 144, TYPE_Q6_K: 210}

_P = ctypes.c_void_p
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_int = ctypes.c_int
_size = ctypes.c_size_t
_f = ctypes.c_float

_SIGS = {
    "qko_fp16_to_fp32": ([ctypes.c_uint16], _f),
    "qko_fp32_to_fp16": ([_f], ctypes.c_uint16),
    "qko_get_scale_min_k4": ([_int, _P, ctypes.POINTER(_int), ctypes.POINTER(_int)], None),
    "qko_dequantize_row_q4k": ([_P, _P, _i64], None),
    "qko_dequantize_row_q6k": ([_P, _P, _i64], None),
    "qko_dequantize_rows": ([_P, _P, _i64, _i64, _size, _int], _int),
    "qko_quantize_q8": ([_P, _P, _P, _i64], None),
    "qko_q8_roundtrip": ([_P, _P, _i64], None),
    "qko_reference_product": ([_P, _P, _int, _i64, _i64, _i64, _P, _int], _int),
    "qko_reference_product_f32": ([_P, _P, _int, _i64, _i64, _i64, _P, _int], _int),
    "qko_integer_product": ([_P, _P, _int, _i64, _i64, _i64, _P], _int),
    "qko_silu_multiply": ([_P, _P, _P, _i64], None),
    "qko_rms_norm": ([_P, _P, _P, _i64, _i64, ctypes.c_float], None),
    "qko_argmax": ([_P, _i64], _i64),
    "qko_mix64": ([_u64], _u64),
    "qko_word": ([_u64, _u64], _u64),
    "qko_synth_superblocks": ([_P, _int, _i64, _i64, _u64, _f, _f], None),
    "qko_synth_normal": ([_P, _i64, _u64], None),
}

_LIB = None


def load() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run `make -C oracle`")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in _SIGS.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _LIB = lib
    return _LIB


def _c(a: np.ndarray):
    return a.ctypes.data


def row_bytes(qtype: int, K: int) -> int:
    return (K // 256) * SUPERBLOCK_BYTES[qtype]


def fp16_to_fp32(h: int) -> float:
    return load().qko_fp16_to_fp32(h)


def fp32_to_fp16(f: float) -> int:
    return load().qko_fp32_to_fp16(f)


def scale_min_k4(g: int, scales12: bytes) -> tuple[int, int]:
    buf = np.frombuffer(bytes(scales12), dtype=np.uint8).copy()
    sc, m = _int(0), _int(0)
    load().qko_get_scale_min_k4(g, _c(buf), ctypes.byref(sc), ctypes.byref(m))
    return sc.value, m.value


def dequantize(packed: np.ndarray, qtype: int, rows: int, K: int, stride: int | None = None):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    stride = row_bytes(qtype, K) if stride is None else stride
    out = np.empty(rows * K, dtype=np.float32)
    st = load().qko_dequantize_rows(_c(packed), _c(out), rows, K, stride, qtype)
    if st != 0:
        raise ValueError(f"dequantize status {st}")
    return out.reshape(rows, K)


def quantize_q8(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32).ravel()
    codes = np.empty(x.size, dtype=np.int8)
    scales = np.empty(x.size // 32, dtype=np.float32)
    load().qko_quantize_q8(_c(x), _c(codes), _c(scales), x.size)
    return codes, scales


def q8_roundtrip(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    load().qko_q8_roundtrip(_c(x), _c(out), x.size)
    return out


def reference_product(x: np.ndarray, w: np.ndarray, qtype: int, K: int, N: int,
                      threads: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    M = x.size // K
    w = np.ascontiguousarray(w, dtype=np.uint8)
    y = np.zeros(M * N, dtype=np.float64)
    st = load().qko_reference_product(_c(x), _c(w), qtype, K, N, M, _c(y), threads)
    if st != 0:
        raise ValueError(f"reference_product status {st}")
    return y.reshape(M, N)


def reference_product_f32(x, w, qtype, K, N, threads: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    M = x.size // K
    w = np.ascontiguousarray(w, dtype=np.uint8)
    y = np.zeros(M * N, dtype=np.float32)
    st = load().qko_reference_product_f32(_c(x), _c(w), qtype, K, N, M, _c(y), threads)
    if st != 0:
        raise ValueError(f"reference_product_f32 status {st}")
    return y.reshape(M, N)


def integer_product(x, w, qtype, K, N) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    M = x.size // K
    w = np.ascontiguousarray(w, dtype=np.uint8)
    y = np.zeros(M * N, dtype=np.float32)
    st = load().qko_integer_product(_c(x), _c(w), qtype, K, N, M, _c(y))
    if st != 0:
        raise ValueError(f"integer_product status {st}")
    return y.reshape(M, N)


def silu_multiply(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    gate = np.ascontiguousarray(gate, dtype=np.float32)
    up = np.ascontiguousarray(up, dtype=np.float32)
    out = np.empty_like(gate)
    load().qko_silu_multiply(_c(gate), _c(up), _c(out), gate.size)
    return out


def rms_norm(x: np.ndarray, scale: np.ndarray, width: int, eps: float) -> np.ndarray:
    """src/cuda/rms_norm.cu:6-24 per row of `width` values (qko_rms_norm)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    scale = np.ascontiguousarray(scale, dtype=np.float32)
    out = np.empty_like(x)
    load().qko_rms_norm(_c(x), _c(scale), _c(out), x.size // width, width, eps)
    return out


def argmax(v: np.ndarray) -> int:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return int(load().qko_argmax(_c(v), v.size))


def mix64(z: int) -> int:
    return int(load().qko_mix64(z))


def word(seed: int, i: int) -> int:
    return int(load().qko_word(seed, i))


def synth_superblocks(qtype: int, N: int, K: int, seed: int, dmax: float,
                      dminmax: float = 0.0) -> np.ndarray:
    out = np.empty(N * row_bytes(qtype, K), dtype=np.uint8)
    load().qko_synth_superblocks(_c(out), qtype, N, K, seed, dmax, dminmax)
    return out


def synth_normal(count: int, seed: int) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    load().qko_synth_normal(_c(out), count, seed)
    return out


def row_norm_error(y: np.ndarray, ref: np.ndarray) -> float:
    """max_{m,n} |y - ref| / ||ref[m,:]||_2, the parity metric for outputs."""
    y = np.asarray(y, dtype=np.float64).reshape(ref.shape)
    norms = np.linalg.norm(ref, axis=1, keepdims=True)
    norms = np.where(norms == 0, 1.0, norms)
    return float(np.max(np.abs(y - ref) / norms)) if ref.size else 0.0


def approx_pass_rate(y: np.ndarray, ref: np.ndarray, margin: float = 3e-5,
                     epsilon: float = 1e-4) -> float:
    """Share of outputs passing Catch2 Approx(ref).margin(margin).epsilon(epsilon)
    (src/tests/reference/MatmulReference.hpp:71-78)."""
    y = np.asarray(y, dtype=np.float64).reshape(ref.shape)
    diff = np.abs(y - ref)
    ok = (diff <= margin) | (diff <= epsilon * np.abs(ref))
    return float(np.mean(ok)) if ref.size else 1.0
