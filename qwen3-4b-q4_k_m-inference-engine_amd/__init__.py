"""Python handle on libqk_hip.so, the C-ABI of the gfx950 Q4_K/Q6_K
dequantize-matmul library (include/qk_abi.h).

The product is the HIP library and the C++20 host layer above it
(include/Kernels.hpp, include/Weight.hpp); this module only binds the C-ABI
with ctypes so tests and the benchmark can drive it from Python, the way the
reference's Catch2 tests drive kernels::matmul (src/tests/MatmulTests.cpp).
Device memory, streams and events go through the library's own shims, so no
other GPU runtime is loaded into the process.

Loading fails loudly when the library has not been built: there is no CPU
fallback for any entry point.
"""
from __future__ import annotations

import atexit
import ctypes
import pathlib

import numpy as np

PKG_DIR = pathlib.Path(__file__).resolve().parent
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = BUILD_DIR / "libqk_hip.so"
ENGINE_PATH = BUILD_DIR / "libqk_engine.so"

QK_OK = 0
QK_ERR_INVALID_ARGUMENT = 1
QK_ERR_UNSUPPORTED_TYPE = 2
QK_ERR_RUNTIME = 3
QK_ERR_OUT_OF_MEMORY = 4

TYPE_F32 = 0
TYPE_F16 = 1
TYPE_Q4_K = 12
TYPE_Q6_K = 14
SUPERBLOCK_BYTES = {TYPE_Q4_K: 144, TYPE_Q6_K: 210}
QK = 256
Q8_BLOCK_BYTES = 48

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_size = ctypes.c_size_t
_int = ctypes.c_int
_float = ctypes.c_float

class Segment(ctypes.Structure):
    """qk_segment: one weight matrix of a multi-segment mat-vec."""

    _fields_ = [("w", ctypes.c_void_p), ("type", ctypes.c_int), ("N", ctypes.c_int64),
                ("y", ctypes.c_void_p)]


# name -> argument types (every function returns int status unless listed in _RESTYPES)
_SIGNATURES = {
    "qk_last_error": [],
    "qk_last_launch": [],
    "qk_version": [],
    "qk_matmul": [_c_void_p, _c_void_p, _int, _i64, _i64, _c_void_p, _i64, _c_void_p],
    "qk_matmul_workspace_size": [_int, _i64, _i64, _i64],
    "qk_matmul_noalloc": [_c_void_p, _c_void_p, _int, _i64, _i64, _c_void_p, _i64, _c_void_p],
    "qk_matmul_ws": [_c_void_p, _c_void_p, _int, _i64, _i64, _c_void_p, _i64, _c_void_p, _size,
                     _c_void_p],
    "qk_quantize_q8": [_c_void_p, _i64, _i64, _c_void_p, _c_void_p],
    "qk_matmul_q8": [_c_void_p, _c_void_p, _int, _i64, _i64, _c_void_p, _i64, _c_void_p],
    "qk_matmul_segments": [_c_void_p, _i64, _i64, ctypes.POINTER(Segment), _int, _c_void_p],
    "qk_ffn_gate_up": [_c_void_p, _c_void_p, _c_void_p, _int, _i64, _i64, _c_void_p, _i64,
                       _c_void_p],
    "qk_ffn_gate_up_workspace_size": [_int, _i64, _i64, _i64],
    "qk_ffn_gate_up_ws": [_c_void_p, _c_void_p, _c_void_p, _int, _i64, _i64, _c_void_p, _i64,
                          _c_void_p, _size, _c_void_p],
    "qk_matmul_segments_workspace_size": [_i64, _i64, ctypes.POINTER(Segment), _int],
    "qk_matmul_segments_ws": [_c_void_p, _i64, _i64, ctypes.POINTER(Segment), _int, _c_void_p, _size,
                              _c_void_p],
    "qk_ffn_gate_up_norm": [_c_void_p, _c_void_p, _float, _c_void_p, _c_void_p, _int, _i64, _i64,
                            _c_void_p, _i64, _c_void_p],
    "qk_ffn_workspace_size": [],
    "qk_ffn": [_c_void_p, _c_void_p, _float, _c_void_p, _c_void_p, _int, _c_void_p, _int, _i64, _i64,
               _c_void_p, _c_void_p, _i64, _c_void_p, _size, _c_void_p],
    "qk_ffn_workspace_check": [_c_void_p, _c_void_p],
    "qk_argmax_workspace_check": [_c_void_p, _c_void_p],
    "qk_argmax_workspace_size": [],
    "qk_argmax": [_c_void_p, _i64, _c_void_p, _c_void_p, _size, _c_void_p],
    "qk_matmul_argmax": [_c_void_p, _c_void_p, _int, _i64, _i64, _c_void_p, _c_void_p, _c_void_p,
                         _size, _c_void_p],
    "qk_dequantize_rows": [_c_void_p, _c_void_p, _i64, _i64, _size, _int, _c_void_p],
    "qk_silu_multiply": [_c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p],
    "qk_rms_norm": [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _float, _c_void_p],
    "qk_residual_add": [_c_void_p, _c_void_p, _i64, _c_void_p],
    "qk_check_launch": [],
    "qk_malloc": [ctypes.POINTER(_c_void_p), _size],
    "qk_free": [_c_void_p],
    "qk_malloc_async": [ctypes.POINTER(_c_void_p), _size, _c_void_p],
    "qk_free_async": [_c_void_p, _c_void_p],
    "qk_memcpy_h2d": [_c_void_p, _c_void_p, _size, _c_void_p],
    "qk_memcpy_d2h": [_c_void_p, _c_void_p, _size, _c_void_p],
    "qk_memcpy_d2d_async": [_c_void_p, _c_void_p, _size, _c_void_p],
    "qk_memset_async": [_c_void_p, _int, _size, _c_void_p],
    "qk_stream_create": [ctypes.POINTER(_c_void_p)],
    "qk_stream_destroy": [_c_void_p],
    "qk_stream_synchronize": [_c_void_p],
    "qk_stream_query": [_c_void_p, ctypes.POINTER(_int)],
    "qk_device_synchronize": [],
    "qk_device_count": [ctypes.POINTER(_int)],
    "qk_set_device": [_int],
    "qk_device_info": [ctypes.c_char_p, _size, ctypes.POINTER(_int), ctypes.c_char_p, _size],
    "qk_event_create": [ctypes.POINTER(_c_void_p)],
    "qk_event_destroy": [_c_void_p],
    "qk_event_record": [_c_void_p, _c_void_p],
    "qk_event_synchronize": [_c_void_p],
    "qk_event_elapsed_ms": [ctypes.POINTER(_float), _c_void_p, _c_void_p],
    "qk_stream_begin_capture": [_c_void_p],
    "qk_stream_end_capture": [_c_void_p, ctypes.POINTER(_c_void_p)],
    "qk_graph_launch": [_c_void_p, _c_void_p],
    "qk_graph_destroy": [_c_void_p],
    "qk_synth_superblocks": [_c_void_p, _int, _i64, _i64, _u64, _float, _float, _c_void_p],
    "qk_synth_normal": [_c_void_p, _i64, _u64, _c_void_p],
}
_RESTYPES = {"qk_last_error": ctypes.c_char_p, "qk_last_launch": ctypes.c_char_p,
             "qk_matmul_workspace_size": _size,
             "qk_argmax_workspace_size": _size, "qk_ffn_workspace_size": _size,
             "qk_ffn_gate_up_workspace_size": _size, "qk_matmul_segments_workspace_size": _size}

_LIB = None
_SHUTTING_DOWN = False


def _mark_shutdown() -> None:
    global _SHUTTING_DOWN
    _SHUTTING_DOWN = True


atexit.register(_mark_shutdown)  # no frees from __del__ once the interpreter is exiting


class QKError(RuntimeError):
    """A failing C-ABI call: .code is the qk_status, the message qk_last_error()."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


def library_path() -> pathlib.Path:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load libqk_hip.so (built by __graft_entry__.build()); raise if absent."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() first")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = _RESTYPES.get(name, _int)
    _LIB = lib
    return lib


def declared_symbols() -> list[str]:
    return list(_SIGNATURES)


_LAUNCH_LOG: set[str] | None = None


def record_launches() -> set[str]:
    """Start collecting the distinct kernel instantiations launched by the
    calls of this module (each call's last launch, as last_launch() names it);
    returns the live set."""
    global _LAUNCH_LOG
    if _LAUNCH_LOG is None:
        _LAUNCH_LOG = set()
    return _LAUNCH_LOG


def check(status: int) -> None:
    if status != QK_OK:
        msg = load().qk_last_error()
        raise QKError(status, msg.decode() if msg else "")
    if _LAUNCH_LOG is not None:
        name = last_launch()
        if name:
            _LAUNCH_LOG.add(name)


def last_launch() -> str:
    """The last product kernel launched on this thread ("name<values> grid=G")."""
    text = load().qk_last_launch()
    return text.decode() if text else ""


def row_bytes(qtype: int, K: int) -> int:
    return (K // QK) * SUPERBLOCK_BYTES[qtype]


def device_count() -> int:
    n = _int(0)
    check(load().qk_device_count(ctypes.byref(n)))
    return n.value


def device_info() -> dict:
    name = ctypes.create_string_buffer(256)
    arch = ctypes.create_string_buffer(64)
    cus = _int(0)
    check(load().qk_device_info(name, 256, ctypes.byref(cus), arch, 64))
    return {"name": name.value.decode(), "arch": arch.value.decode(), "compute_units": cus.value}


class DeviceBuffer:
    """Owning device allocation (qk_malloc / qk_free)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        ptr = _c_void_p()
        check(load().qk_malloc(ctypes.byref(ptr), self.nbytes))
        self.ptr = ptr.value or 0

    @classmethod
    def from_array(cls, arr: np.ndarray, stream=None) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr, stream)
        return buf

    def upload(self, arr: np.ndarray, stream=None, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        check(load().qk_memcpy_h2d(self.ptr + offset, arr.ctypes.data, arr.nbytes,
                                   _stream_ptr(stream)))

    def download(self, dtype, count: int | None = None, stream=None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        check(load().qk_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes,
                                   _stream_ptr(stream)))
        return out

    def fill(self, value: int, stream=None) -> None:
        check(load().qk_memset_async(self.ptr, value, self.nbytes, _stream_ptr(stream)))
        synchronize(stream)

    def free(self) -> None:
        if self.ptr:
            check(load().qk_free(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            if self.ptr and _LIB is not None and not _SHUTTING_DOWN:
                _LIB.qk_free(self.ptr)
                self.ptr = 0
        except Exception:
            pass


class Stream:
    """Non-blocking stream (qk_stream_create)."""

    def __init__(self):
        s = _c_void_p()
        check(load().qk_stream_create(ctypes.byref(s)))
        self.ptr = s.value

    def synchronize(self) -> None:
        check(load().qk_stream_synchronize(self.ptr))

    def ready(self) -> bool:
        r = _int(0)
        check(load().qk_stream_query(self.ptr, ctypes.byref(r)))
        return bool(r.value)

    def destroy(self) -> None:
        if self.ptr:
            check(load().qk_stream_destroy(self.ptr))
            self.ptr = None


class Event:
    def __init__(self):
        e = _c_void_p()
        check(load().qk_event_create(ctypes.byref(e)))
        self.ptr = e.value

    def record(self, stream=None) -> None:
        check(load().qk_event_record(self.ptr, _stream_ptr(stream)))

    def synchronize(self) -> None:
        check(load().qk_event_synchronize(self.ptr))

    def elapsed_ms(self, end: "Event") -> float:
        ms = _float(0.0)
        check(load().qk_event_elapsed_ms(ctypes.byref(ms), self.ptr, end.ptr))
        return ms.value

    def destroy(self) -> None:
        if self.ptr:
            check(load().qk_event_destroy(self.ptr))
            self.ptr = None


class Graph:
    """A launch sequence captured on a stream (qk_stream_begin/end_capture)."""

    def __init__(self, ptr):
        self.ptr = ptr

    @classmethod
    def capture(cls, stream: "Stream", record) -> "Graph":
        check(load().qk_stream_begin_capture(stream.ptr))
        try:
            record()
        except BaseException:
            g = _c_void_p()
            load().qk_stream_end_capture(stream.ptr, ctypes.byref(g))
            if g.value:
                load().qk_graph_destroy(g.value)
            raise
        g = _c_void_p()
        check(load().qk_stream_end_capture(stream.ptr, ctypes.byref(g)))
        return cls(g.value)

    def launch(self, stream) -> None:
        check(load().qk_graph_launch(self.ptr, _stream_ptr(stream)))

    def destroy(self) -> None:
        if self.ptr:
            check(load().qk_graph_destroy(self.ptr))
            self.ptr = None


def _stream_ptr(stream):
    if stream is None:
        return None
    return stream.ptr if isinstance(stream, Stream) else stream


def _ptr(buf, offset: int = 0):
    if buf is None:
        return None
    base = buf.ptr if isinstance(buf, DeviceBuffer) else int(buf)
    return base + offset


def synchronize(stream=None) -> None:
    if stream is None:
        check(load().qk_device_synchronize())
    else:
        check(load().qk_stream_synchronize(_stream_ptr(stream)))


# ------------------------------------------------------------- entry points --

def matmul(x, w, qtype: int, K: int, N: int, y, M: int, stream=None, y_offset: int = 0) -> None:
    """y[M x N] = Q8(x)[M x K] . W^T  (qk_matmul; kernels::matmul)."""
    check(load().qk_matmul(_ptr(x), _ptr(w), qtype, K, N, _ptr(y, y_offset), M,
                           _stream_ptr(stream)))


def ffn_workspace_size() -> int:
    return load().qk_ffn_workspace_size()


def ffn(x, norm, eps: float, gate, up, gu_type: int, down, down_type: int, K: int, N: int, h, y,
        M: int, workspace, workspace_bytes: int, stream=None) -> None:
    """qk_ffn: h = SiLU(gate . x') * (up . x'), y = down . h (x' = RMSNorm(x) if norm)."""
    check(load().qk_ffn(_ptr(x), _ptr(norm) if norm is not None else None, eps, _ptr(gate), _ptr(up),
                        gu_type, _ptr(down), down_type, K, N, _ptr(h), _ptr(y), M, _ptr(workspace),
                        workspace_bytes, _stream_ptr(stream)))


def ffn_workspace_check(workspace, stream=None) -> None:
    check(load().qk_ffn_workspace_check(_ptr(workspace), _stream_ptr(stream)))


def matmul_noalloc(x, w, qtype: int, K: int, N: int, y, M: int, stream=None) -> None:
    """qk_matmul_noalloc: qk_matmul with its prefill workspace in the library's device scratch."""
    check(load().qk_matmul_noalloc(_ptr(x), _ptr(w), qtype, K, N, _ptr(y), M, _stream_ptr(stream)))


def matmul_segments(x, M: int, K: int, segments, stream=None) -> None:
    """segments: [(w, qtype, N, y), ...] (qk_matmul_segments; q/k/v in one launch)."""
    arr = (Segment * len(segments))(*[Segment(_ptr(w), qtype, N, _ptr(y)) for w, qtype, N, y in segments])
    check(load().qk_matmul_segments(_ptr(x), M, K, arr, len(segments), _stream_ptr(stream)))


def _segments(segments):
    return (Segment * len(segments))(*[Segment(_ptr(w), qtype, N, _ptr(y)) for w, qtype, N, y in segments])


def matmul_segments_workspace_size(M: int, K: int, segments) -> int:
    return load().qk_matmul_segments_workspace_size(M, K, _segments(segments), len(segments))


def matmul_segments_ws(x, M: int, K: int, segments, workspace, workspace_bytes: int, stream=None) -> None:
    """qk_matmul_segments_ws: qk_matmul_segments with a caller workspace."""
    check(load().qk_matmul_segments_ws(_ptr(x), M, K, _segments(segments), len(segments), _ptr(workspace),
                                       workspace_bytes, _stream_ptr(stream)))


def ffn_gate_up_workspace_size(qtype: int, K: int, N: int, M: int) -> int:
    return load().qk_ffn_gate_up_workspace_size(qtype, K, N, M)


def ffn_gate_up_ws(x, gate, up, qtype: int, K: int, N: int, h, M: int, workspace, workspace_bytes: int,
                   stream=None) -> None:
    """qk_ffn_gate_up_ws: qk_ffn_gate_up with a caller workspace."""
    check(load().qk_ffn_gate_up_ws(_ptr(x), _ptr(gate), _ptr(up), qtype, K, N, _ptr(h), M, _ptr(workspace),
                                   workspace_bytes, _stream_ptr(stream)))


def ffn_gate_up(x, gate, up, qtype: int, K: int, N: int, h, M: int, stream=None) -> None:
    """h = SiLU(x . gate^T) * (x . up^T) (qk_ffn_gate_up)."""
    check(load().qk_ffn_gate_up(_ptr(x), _ptr(gate), _ptr(up), qtype, K, N, _ptr(h), M,
                                _stream_ptr(stream)))


def ffn_gate_up_norm(x, norm, eps: float, gate, up, qtype: int, K: int, N: int, h, M: int,
                     stream=None) -> None:
    """h = SiLU(n . gate^T) * (n . up^T), n = RMSNorm(x) with scale `norm` (qk_ffn_gate_up_norm)."""
    check(load().qk_ffn_gate_up_norm(_ptr(x), _ptr(norm), eps, _ptr(gate), _ptr(up), qtype, K, N,
                                     _ptr(h), M, _stream_ptr(stream)))


def matmul_workspace_size(qtype: int, K: int, N: int, M: int) -> int:
    return int(load().qk_matmul_workspace_size(qtype, K, N, M))


def matmul_ws(x, w, qtype: int, K: int, N: int, y, M: int, workspace, workspace_bytes: int,
              stream=None) -> None:
    check(load().qk_matmul_ws(_ptr(x), _ptr(w), qtype, K, N, _ptr(y), M, _ptr(workspace),
                              workspace_bytes, _stream_ptr(stream)))


def argmax_workspace_size() -> int:
    return int(load().qk_argmax_workspace_size())


def argmax_workspace_check(workspace, stream=None) -> None:
    """Raises QKError if an argmax call on `workspace` timed out (then clears it)."""
    check(load().qk_argmax_workspace_check(_ptr(workspace), _stream_ptr(stream)))


def argmax(logits, count: int, result, workspace, workspace_bytes: int, stream=None) -> None:
    """*result (device uint32) = argmax of logits[0, count) (qk_argmax)."""
    check(load().qk_argmax(_ptr(logits), count, _ptr(result), _ptr(workspace), workspace_bytes,
                           _stream_ptr(stream)))


def matmul_argmax(x, w, qtype: int, K: int, N: int, logits, result, workspace,
                  workspace_bytes: int, stream=None) -> None:
    """lm_head + argmax in one launch (qk_matmul_argmax); logits may be None."""
    check(load().qk_matmul_argmax(_ptr(x), _ptr(w), qtype, K, N, _ptr(logits), _ptr(result),
                                  _ptr(workspace), workspace_bytes, _stream_ptr(stream)))


def quantize_q8(x, M: int, K: int, q8, stream=None) -> None:
    check(load().qk_quantize_q8(_ptr(x), M, K, _ptr(q8), _stream_ptr(stream)))


def matmul_q8(q8, w, qtype: int, K: int, N: int, y, M: int, stream=None) -> None:
    check(load().qk_matmul_q8(_ptr(q8), _ptr(w), qtype, K, N, _ptr(y), M, _stream_ptr(stream)))


def dequantize_rows(packed, out, rows: int, K: int, row_stride: int, qtype: int,
                    stream=None) -> None:
    check(load().qk_dequantize_rows(_ptr(packed), _ptr(out), rows, K, row_stride, qtype,
                                    _stream_ptr(stream)))


def silu_multiply(gate, up, out, count: int, stream=None) -> None:
    check(load().qk_silu_multiply(_ptr(gate), _ptr(up), _ptr(out), count, _stream_ptr(stream)))


def rms_norm(x, scale, out, rows: int, width: int, eps: float, stream=None) -> None:
    """qk_rms_norm: out = x * rsqrt(mean(x^2) + eps) * scale, row by row."""
    check(load().qk_rms_norm(_ptr(x), _ptr(scale), _ptr(out), rows, width, eps, _stream_ptr(stream)))


def residual_add(state, branch, count: int, stream=None) -> None:
    """qk_residual_add: state += branch."""
    check(load().qk_residual_add(_ptr(state), _ptr(branch), count, _stream_ptr(stream)))


def synth_superblocks(w, qtype: int, N: int, K: int, seed: int, dmax: float,
                      dminmax: float = 0.0, stream=None) -> None:
    check(load().qk_synth_superblocks(_ptr(w), qtype, N, K, seed, dmax, dminmax,
                                      _stream_ptr(stream)))


def synth_normal(x, count: int, seed: int, stream=None) -> None:
    check(load().qk_synth_normal(_ptr(x), count, seed, _stream_ptr(stream)))


# Q8 activation block layout (qk_q8_block)
Q8_DTYPE = np.dtype([("codes", np.int8, 32), ("scale", np.float32), ("scaled_sum", np.float32),
                     ("neg32_sum_lo", np.int32), ("neg32_sum_hi", np.int32)])
assert Q8_DTYPE.itemsize == Q8_BLOCK_BYTES
