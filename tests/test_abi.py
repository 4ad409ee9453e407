"""The C-ABI library loads and exports every entry point include/enceladus_hip.h declares.
No compute calls (CPU only)."""

import ctypes
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    text = (ROOT / "include" / "enceladus_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ek_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_expected_surface():
    syms = declared_symbols()
    for s in ("ek_compile", "ek_module_load", "ek_launch", "ek_stream_sync", "ek_malloc",
              "ek_timed_launch"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    from enceladus_amd.runtime import hip
    lib = hip.load_library()
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    assert set(hip.EXPORTED) <= set(declared_symbols())


def test_version_and_compile_without_gpu():
    from enceladus_amd.runtime import hip
    lib = hip.load_library()
    assert b"gfx950" in lib.ek_version()
    code, _ = hip.compile_source('extern "C" __global__ void k(int* p) { p[threadIdx.x] = 1; }',
                                 "k.hip", ["--offload-arch=gfx950", "-O3"])
    assert code[:4] == b"\x7fELF"


def test_compile_error_is_reported():
    import pytest
    from enceladus_amd.compiler.errors import HipError
    from enceladus_amd.runtime import hip
    with pytest.raises(HipError, match="error"):
        hip.compile_source("this is not C++", "bad.hip", ["--offload-arch=gfx950"])


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    import pytest
    from enceladus_amd.compiler.errors import HipError
    from enceladus_amd.runtime import hip
    monkeypatch.setattr(hip, "_lib", None)
    monkeypatch.setattr(hip, "LIB_PATH", tmp_path / "nope.so")
    with pytest.raises(HipError, match="not built"):
        hip.load_library()


def test_struct_layout_matches_header():
    from enceladus_amd.runtime import hip
    assert ctypes.sizeof(hip.DeviceInfo) == 256 + 64 + 4 * 3 + 4 + 8 * 2 + 4 * 4
    assert ctypes.sizeof(hip.FunctionAttrs) == 16
