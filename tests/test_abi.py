"""CPU checks of the drop-in boundary: libqk_hip.so loads, exports every symbol
include/qk_abi.h declares, and validates arguments on the host exactly like
kernels::matmul (src/cuda/matmul.cu:132-137) before touching the device.
No compute call is made: every call here returns before any HIP call."""
from __future__ import annotations

import ctypes
import os
import pathlib
import re
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "qk_abi.h"


def declared_functions(header: pathlib.Path) -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(qk_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(qk):
    names = declared_functions(HEADER)
    assert len(names) >= 30
    lib = ctypes.CDLL(str(qk.library_path()))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(qk.declared_symbols()) == names


def test_engine_library_links_the_c_abi(qk):
    path = qk.ENGINE_PATH
    assert path.exists()
    out = subprocess.run(["nm", "-D", "--undefined-only", str(path)], capture_output=True,
                         text=True, check=True).stdout
    used = set(re.findall(r"\b(qk_[a-z0-9_]+)\b", out))
    assert {"qk_matmul", "qk_malloc_async", "qk_stream_create", "qk_last_error"} <= used
    # the host layer reaches HIP only through the C-ABI
    assert "hipLaunchKernel" not in out and "hipMalloc" not in out


def test_version_and_last_error_start_clean(qk):
    lib = qk.load()
    assert lib.qk_version() >= 100
    assert lib.qk_last_error() == b""


@pytest.mark.parametrize("qtype,K,N,M,code", [
    (13, 2560, 8, 1, 2),        # Q5_K: unsupported type
    (0, 2560, 8, 1, 2),         # F32
    (12, 2500, 8, 1, 1),        # K not a multiple of 256
    (12, 0, 8, 1, 1),           # K = 0
    (14, -256, 8, 1, 1),        # K < 0
    (12, 2560, 0, 1, 1),        # N = 0
    (14, 2560, -3, 1, 1),       # N < 0
    (12, 2560, 8, -1, 1),       # negative rows
    (12, (1 << 30) + 256, 8, 1, 1),  # K beyond the kernels' 32-bit indexing
])
def test_matmul_validation_matches_reference(qk, qtype, K, N, M, code):
    lib = qk.load()
    status = lib.qk_matmul(None, None, qtype, K, N, None, M, None)
    assert status == code
    msg = lib.qk_last_error().decode()
    assert ("Q4_K and Q6_K" in msg) if code == 2 else ("dimensions" in msg or "rows" in msg)
    assert lib.qk_matmul_q8(None, None, qtype, K, N, None, M, None) == code
    assert lib.qk_matmul_ws(None, None, qtype, K, N, None, M, None, 0, None) == code


def test_zero_rows_is_a_no_op(qk):
    lib = qk.load()
    assert lib.qk_matmul(None, None, 12, 2560, 8, None, 0, None) == 0
    assert lib.qk_matmul_q8(None, None, 14, 9728, 8, None, 0, None) == 0
    assert lib.qk_dequantize_rows(None, None, 0, 2560, 1440, 99, None) == 0
    assert lib.qk_silu_multiply(None, None, None, 0, None) == 0


def test_other_validation(qk):
    lib = qk.load()
    assert lib.qk_dequantize_rows(None, None, 1, 2560, 1440, 13, None) == 2
    assert lib.qk_dequantize_rows(None, None, 1, 2560, 1000, 12, None) == 1  # stride < row
    assert lib.qk_matmul(None, None, 12, 2560, 8, None, 1, None) == 1      # null pointers
    assert lib.qk_quantize_q8(None, 1, 100, None, None) == 1
    assert lib.qk_matmul_workspace_size(12, 2560, 8, 3) == 0  # Q8 runs inside the kernel
    # M > 8: two fp16 planes (hi, lo) of M x K plus M row scales, rounded up to 256
    # 9*2560*4 + 36 (hi/lo planes, row scales) -> 92208, + 9*10*32 sub-block sums -> 372*256;
    # M <= 32 splits K down to single superblocks (one tile: 10 splits) -> + 10 x 9 x 8 fp32
    # partials -> 98112, rounded up to 384*256
    assert lib.qk_matmul_workspace_size(12, 2560, 8, 9) == 98304
    # one tile of K = 4096 (16 superblocks): 16 splits -> 152320 + 16 x 9 x 8 fp32 partials
    assert lib.qk_matmul_workspace_size(12, 4096, 8, 9) == 156928
    assert lib.qk_matmul_workspace_size(14, 256, 8, 11) == 11776  # 11*256*4 + 44 -> 11312, + 11*32 -> 46*256
    assert lib.qk_matmul_workspace_size(14, 2500, 8, 11) == 0  # rejected shape
    p = ctypes.c_void_p(256)
    assert lib.qk_matmul_ws(p, p, 12, 2560, 8, p, 9, None, 0, None) == 1  # M > 8 needs scratch
    assert b"workspace" in lib.qk_last_error()
    assert lib.qk_matmul_ws(p, p, 12, 2560, 8, p, 9, p, 92416 - 256, None) == 1
    assert b"too small" in lib.qk_last_error()
    assert lib.qk_matmul_ws(p, ctypes.c_void_p(8), 12, 2560, 8, p, 9, p, 1 << 20, None) == 1
    assert b"aligned" in lib.qk_last_error()
    assert lib.qk_matmul_ws(None, None, 12, 2560, 8, None, 1, None, 0, None) == 1
    seg = (qk.Segment * 2)(qk.Segment(16, 12, 8, 16), qk.Segment(16, 13, 8, 16))
    assert lib.qk_matmul_segments(ctypes.c_void_p(16), 1, 2560, seg, 2, None) == 2
    assert lib.qk_matmul_segments(ctypes.c_void_p(16), 1, 2560, seg, 0, None) == 1
    assert lib.qk_matmul_segments(ctypes.c_void_p(16), 1, 2500, seg, 1, None) == 1
    assert lib.qk_matmul_segments(None, 0, 2560, seg, 1, None) == 0
    assert lib.qk_ffn_gate_up(None, None, None, 13, 2560, 8, None, 1, None) == 2
    assert lib.qk_ffn_gate_up(None, None, None, 12, 2560, 0, None, 1, None) == 1
    assert lib.qk_ffn_gate_up(None, None, None, 12, 2560, 8, None, 0, None) == 0
    assert lib.qk_ffn_gate_up(None, None, None, 12, 2560, 8, None, 1, None) == 1  # null pointers
    # the RMSNorm fold: the reference's `!(epsilon > 0)` check (src/cuda/rms_norm.cu:32)
    p16 = ctypes.c_void_p(16)
    assert lib.qk_ffn_gate_up_norm(p16, p16, 0.0, p16, p16, 12, 2560, 8, p16, 1, None) == 1
    assert b"epsilon" in lib.qk_last_error()
    assert lib.qk_ffn_gate_up_norm(p16, p16, float("nan"), p16, p16, 12, 2560, 8, p16, 1, None) == 1
    assert lib.qk_ffn_gate_up_norm(p16, None, 1e-6, p16, p16, 12, 2560, 8, p16, 1, None) == 1
    assert lib.qk_ffn_gate_up_norm(p16, p16, 1e-6, p16, p16, 13, 2560, 8, p16, 1, None) == 2
    assert lib.qk_ffn_gate_up_norm(p16, p16, 1e-6, p16, p16, 12, 2500, 8, p16, 1, None) == 1
    assert lib.qk_ffn_gate_up_norm(None, None, 0.0, None, None, 12, 2560, 8, None, 0, None) == 0


def test_argmax_validation_on_the_host(qk):
    lib = qk.load()
    n = lib.qk_argmax_workspace_size()
    assert n >= 8 * 1024 + 4
    p = ctypes.c_void_p(256)
    assert lib.qk_argmax(None, 5, p, p, n, None) == 1           # null logits
    assert lib.qk_argmax(p, 0, p, p, n, None) == 1              # empty
    assert lib.qk_argmax(p, 1 << 32, p, p, n, None) == 1        # beyond uint32
    assert lib.qk_argmax(p, 5, None, p, n, None) == 1           # null result
    assert lib.qk_argmax(p, 5, p, p, n - 8, None) == 1          # small workspace
    assert lib.qk_argmax(p, 5, p, ctypes.c_void_p(260), n, None) == 1  # misaligned workspace
    assert b"argmax" in lib.qk_last_error()
    assert lib.qk_matmul_argmax(p, p, 13, 2560, 8, None, p, p, n, None) == 2
    assert lib.qk_matmul_argmax(p, p, 12, 2500, 8, None, p, p, n, None) == 1
    assert lib.qk_matmul_argmax(p, p, 12, 2560, 8, None, None, p, n, None) == 1
    assert lib.qk_matmul_argmax(None, p, 12, 2560, 8, None, p, p, n, None) == 1


def test_cpp_host_layer_validation():
    """tests/cpp/host_tests.cpp: kernels::matmul throws the reference's exception types."""
    exe = ROOT / "qwen3-4b-q4_k_m-inference-engine_amd" / "_build" / "host_tests"
    assert exe.exists(), "build the package first"
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(res.stdout[-2000:], res.stderr[-2000:])
    assert res.returncode == 0


def test_engine_call_sequence_builds_against_the_headers(tmp_path):
    """tests/cpp/engine_calls.cpp: the reference engine's call sequence
    (src/Engine.cpp:55-111) compiles against include/ and links against
    libqk_engine.so with only rope and attention left to the engine."""
    build = ROOT / "qwen3-4b-q4_k_m-inference-engine_amd" / "_build"
    assert (build / "libqk_engine.so").exists(), "build the package first"
    exe = tmp_path / "engine_calls"
    cmd = ["g++", "-std=c++20", "-O0", "-Wall", "-Wextra", "-Werror", "-I", str(ROOT / "include"),
           str(ROOT / "tests" / "cpp" / "engine_calls.cpp"), "-o", str(exe), "-L", str(build),
           "-lqk_engine", "-lqk_hip", f"-Wl,-rpath,{build}"]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    print(res.stdout[-4000:], res.stderr[-4000:])
    assert res.returncode == 0
    assert exe.exists()


def test_rms_norm_and_residual_add_validation(qk):
    """src/cuda/rms_norm.cu:31-34 and src/cuda/residual_add.cu:16: zero rows or
    count return at once; a zero width or non-positive epsilon is rejected."""
    lib = qk.load()
    assert lib.qk_rms_norm(None, None, None, 0, 2560, 1e-6, None) == 0
    assert lib.qk_rms_norm(8, 8, 8, 1, 0, 1e-6, None) == 1
    assert lib.qk_rms_norm(8, 8, 8, 1, 2560, 0.0, None) == 1
    assert lib.qk_rms_norm(8, 8, 8, 1, 2560, float("nan"), None) == 1
    assert lib.qk_rms_norm(None, 8, 8, 1, 2560, 1e-6, None) == 1
    assert lib.qk_residual_add(None, None, 0, None) == 0
    assert lib.qk_residual_add(8, 8, -1, None) == 1
    assert lib.qk_residual_add(None, 8, 5, None) == 1


def _sanitized_run(tmp_path, name, sources, extra):
    exe = tmp_path / name
    cmd = ["g++", "-std=c++20", "-g", "-O1", "-fno-omit-frame-pointer",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           "-I", str(ROOT / "include"), "-I", str(ROOT / "oracle"), *extra, *map(str, sources),
           "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    print(res.stdout[-3000:], res.stderr[-3000:])
    assert res.returncode == 0, "sanitizer build failed"
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    print(res.stdout[-3000:], res.stderr[-3000:])
    assert res.returncode == 0


def test_host_layer_under_address_and_ub_sanitizers(tmp_path):
    """The host layer (host/*.cpp: GGUF reader, Weight, DeviceBuffer, Kernels
    validation, EmbedLookup) and its CPU tests built with -fsanitize=address,
    undefined and run: no device call is made, libqk_hip.so only validates."""
    build = ROOT / "qwen3-4b-q4_k_m-inference-engine_amd" / "_build"
    assert (build / "libqk_hip.so").exists(), "build the package first"
    host = sorted((ROOT / "qwen3-4b-q4_k_m-inference-engine_amd" / "host").glob("*.cpp"))
    _sanitized_run(tmp_path, "host_tests_asan", host + [ROOT / "tests" / "cpp" / "host_tests.cpp"],
                   ["-L", str(build), "-lqk_hip", f"-Wl,-rpath,{build}"])


def test_oracle_under_address_and_ub_sanitizers(tmp_path):
    """oracle/qk_oracle.c and a self-check driver of every function built with
    -fsanitize=address,undefined (as C, -ffp-contract=off) and run."""
    exe = tmp_path / "oracle_asan"
    cmd = ["gcc", "-std=c11", "-g", "-O1", "-fno-omit-frame-pointer", "-ffp-contract=off", "-fopenmp",
           "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-I", str(ROOT / "oracle"),
           str(ROOT / "oracle" / "qk_oracle.c"), str(ROOT / "tests" / "cpp" / "oracle_selfcheck.c"),
           "-lm", "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    print(res.stdout[-3000:], res.stderr[-3000:])
    assert res.returncode == 0, "sanitizer build failed"
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1", OMP_NUM_THREADS="2")
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=env)
    print(res.stdout[-3000:], res.stderr[-3000:])
    assert res.returncode == 0 and "all checks passed" in res.stdout
