"""Runs the C++ GPU test of the host layer (tests/cpp/matmul_tests.cpp):
kernels::matmul, Weight, DeviceBuffer, Stream and the GGUF reader on device 0."""
from __future__ import annotations

import pathlib
import subprocess

import pytest

pytestmark = pytest.mark.gpu

EXE = pathlib.Path(__file__).resolve().parents[1] / "qwen3-4b-q4_k_m-inference-engine_amd" / "_build" / "matmul_tests"


def test_cpp_matmul_contract():
    assert EXE.exists(), "build the package first"
    res = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=110)
    print(res.stdout[-4000:], res.stderr[-2000:])
    assert res.returncode == 0
