"""Shared test setup: the `gpu` marker, repo on sys.path, tolerances, GPU gating.

Tolerances follow the reference's differential harness (reference: tests/conftest.py:75-99):
fp32 (atol 1e-5, rtol 1e-5), fp16 (1e-3, 2e-3), bf16 (1e-2, 1.6e-2); integers exact.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

os.environ.setdefault("ENCELADUS_CACHE_DIR", os.path.join(ROOT, ".ek_cache"))
# every kernel the tests compile has its IR verified after each compiler stage
os.environ.setdefault("ENCELADUS_VERIFY", "1")

TOL = {"float32": (1e-5, 1e-5), "float16": (1e-3, 2e-3), "bfloat16": (1e-2, 1.6e-2)}


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and runs HIP kernels")
    config.addinivalue_line("markers", "slow: long-running")


def _has_gpu():
    try:
        from enceladus_amd.runtime import hip
        return hip.device_count() > 0
    except Exception:  # noqa: BLE001
        return False


def pytest_collection_modifyitems(config, items):
    markexpr = config.getoption("-m") or ""
    if "gpu" in markexpr and "not gpu" not in markexpr:
        return  # explicitly asked for GPU tests: never skip silently
    if not _has_gpu():
        skip = pytest.mark.skip(reason="no GPU visible")
        for it in items:
            if "gpu" in it.keywords:
                it.add_marker(skip)
