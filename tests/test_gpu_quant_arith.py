"""Exhaustive GPU check of the activation quantiser's exact-rounding helpers
(refined reciprocal, Markstein quotients, truncation-based roundf) against the
device's IEEE float division and roundf (tests/cpp/quant_arith_check.hip).
They make the in-kernel Q8 codes and scales equal to the reference's float
formula round(x/amax*127), amax/127 (src/cuda/matmul.cu:8-22,
src/tests/reference/MatmulReference.hpp:20-24)."""
from __future__ import annotations

import pathlib
import subprocess

import pytest

pytestmark = pytest.mark.gpu

EXE = pathlib.Path(__file__).resolve().parents[1] / "qwen3-4b-q4_k_m-inference-engine_amd" / "_build" / "quant_arith_check"


def test_quantiser_rounding_identities_exhaustive():
    assert EXE.exists(), "build the package first"
    res = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=110)
    print(res.stdout, res.stderr)
    assert res.returncode == 0
    assert res.stdout.count(": 0 mismatches") == 4
