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


def test_dlpack_structures_match_the_header():
    """dlpack.h v1.0 layouts, and an unconsumed capsule releases its exporter."""
    import ctypes
    import gc
    from enceladus_amd.runtime import dlpack as D
    assert ctypes.sizeof(D.DLTensor) == 48
    assert ctypes.sizeof(D.DLManagedTensor) == 64
    assert ctypes.sizeof(D.DLManagedTensorVersioned) == 80
    owner = object()
    cap = D.export(owner, 0x1000, (3, 4), (4, 1), "bf16")
    assert D.live_exports() == 1
    del cap
    gc.collect()
    assert D.live_exports() == 0
    cap = D.export(owner, 0x1000, (5,), (1,), "i32", versioned=True)
    assert type(cap).__name__ == "PyCapsule"
    del cap
    gc.collect()
    assert D.live_exports() == 0


def test_hip_kernel_signature_and_packing():
    """The raw-kernel escape hatch reads its argument types from the source and packs
    scalars with natural alignment (no GPU needed)."""
    import struct
    from enceladus_amd.runtime import raw
    src = '''
    #include "enceladus_cdna4.h"
    // a comment with a fake kernel(int x)
    extern "C" __global__ void saxpy(float* __restrict__ out, const float* x,
                                     const _Float16 *y, float a, int n, long long m,
                                     __bf16 b, unsigned char c) { }
    '''
    ps = raw.parse_signature(src, "saxpy")
    assert [p.name for p in ps] == ["out", "x", "y", "a", "n", "m", "b", "c"]
    assert [p.pointer for p in ps] == [True, True, True, False, False, False, False, False]
    assert [p.const for p in ps[:3]] == [False, True, True]
    b = raw.pack(ps, [0x1000, 0x2000, 0x3000, 1.5, -3, 1 << 40, 1.0, 7])
    assert struct.unpack_from("<QQQfiq", b, 0) == (0x1000, 0x2000, 0x3000, 1.5, -3, 1 << 40)
    assert struct.unpack_from("<HB", b, 40) == (0x3F80, 7)     # bf16(1.0), then the byte
    assert len(b) % 8 == 0
    import pytest as _pt
    with _pt.raises(ValueError):
        raw.parse_signature(src, "nothere")
    with _pt.raises(NotImplementedError):
        raw.metal_kernel("kernel void k() {}", "k")
