"""Shared fixtures: the package handle on libqk_hip.so (`qk`) and the CPU
oracle (`oracle`). GPU tests are marked `gpu`; everything else runs on CPU."""
from __future__ import annotations

import importlib.util
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
PKG_DIR = ROOT / "qwen3-4b-q4_k_m-inference-engine_amd"
ORACLE_DIR = ROOT / "oracle"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_package():
    """Import the package directory (its name is not a Python identifier)."""
    if "qk_amd" in sys.modules:
        return sys.modules["qk_amd"]
    spec = importlib.util.spec_from_file_location("qk_amd", PKG_DIR / "__init__.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules["qk_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def load_oracle():
    if str(ORACLE_DIR) not in sys.path:
        sys.path.insert(0, str(ORACLE_DIR))
    import qk_oracle  # noqa: E402

    qk_oracle.load()
    return qk_oracle


@pytest.fixture(scope="session")
def qk():
    mod = load_package()
    mod.load()
    mod.record_launches()
    return mod


def pytest_terminal_summary(terminalreporter):
    """The distinct kernel instantiations the GPU tests launched through the
    package (shape-determined; listed so a quiet run still records them)."""
    mod = sys.modules.get("qk_amd")
    launches = getattr(mod, "_LAUNCH_LOG", None) or () if mod else ()
    names = sorted({name.split(" grid=")[0] for name in launches})
    if names:
        terminalreporter.write_sep("-", f"{len(names)} kernel instantiations launched")
        for name in names:
            terminalreporter.write_line(name)


@pytest.fixture(scope="session")
def oracle():
    return load_oracle()


@pytest.fixture(scope="session")
def gpu(qk):
    """The package, after checking a gfx950 device is present."""
    if qk.device_count() < 1:
        pytest.fail("no GPU visible to libqk_hip.so")
    info = qk.device_info()
    print(f"[gpu] {info}", flush=True)
    return qk
