"""Compile-time environment switches (reference: src/enceladus/runtime/compile.py:6-10,
:151-155): ENCELADUS_DUMP writes the IR and source, ENCELADUS_OVERRIDE_DIR replaces the
generated source with a file of the kernel's name. Compile-only, no GPU."""

import numpy as np

from enceladus_amd.runtime import compile as C


def _compile(monkeypatch, tmp_path, **env):
    from examples.vector_add import add_kernel
    monkeypatch.setenv("ENCELADUS_CACHE_DIR", str(tmp_path / "cache"))
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    x = np.zeros(16, np.float32)
    fn = add_kernel.ir_for(x, x, x, 100, BLOCK=1024)
    return C.compile_ir(fn)


def test_dump_writes_ir_and_source(monkeypatch, tmp_path, capsys):
    ck = _compile(monkeypatch, tmp_path, ENCELADUS_DUMP="1")
    dumped = sorted((tmp_path / "cache" / "dump").iterdir())
    assert [p.suffix for p in dumped] == [".hip", ".ir"]
    assert dumped[0].read_text() == ck.hip and dumped[1].read_text() == ck.ir
    assert "IR and HIP source in" in capsys.readouterr().err


def test_override_dir_replaces_the_generated_source(monkeypatch, tmp_path):
    ck = _compile(monkeypatch, tmp_path)
    ovr = tmp_path / "ovr"
    ovr.mkdir()
    edited = ck.hip.replace("{", "{ /* hand-edited */", 1)
    (ovr / "add_kernel.hip").write_text(edited)
    ck2 = _compile(monkeypatch, tmp_path, ENCELADUS_OVERRIDE_DIR=str(ovr))
    assert ck2.hip == edited
    assert ck2.name == ck.name
    # a directory without a file of the kernel's name leaves the generated source alone
    ck3 = _compile(monkeypatch, tmp_path, ENCELADUS_OVERRIDE_DIR=str(tmp_path))
    assert ck3.hip == ck.hip


def _debug_kernel():
    import enceladus
    import enceladus.language as tl

    @enceladus.jit
    def checked(x_ptr, n, BLOCK: tl.constexpr):
        offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
        x = tl.load(x_ptr + offs, mask=offs < n, other=0.0)
        tl.device_assert(x < 100.0, "x must stay below 100", mask=offs < n)
        tl.device_print("x", x)
    return checked


def test_device_assert_is_compiled_only_with_debug(monkeypatch, tmp_path):
    """ENCELADUS_DEBUG=1 keeps tl.device_assert (an error-buffer argument after the runtime
    arguments); without it the check is compiled out. tl.device_print always lowers to
    printf (reference: codegen/debug.py:84-158, compile.py:10)."""
    monkeypatch.setenv("ENCELADUS_CACHE_DIR", str(tmp_path))
    k = _debug_kernel()
    x = np.zeros(16, np.float32)
    monkeypatch.setenv("ENCELADUS_DEBUG", "1")
    ck = C.compile_ir(k.ir_for(x, 100, BLOCK=64))
    assert "ek::assert_fail(ek_assert_buf, 0" in ck.hip and "printf(" in ck.hip
    assert [a.name for a in ck.args] == ["x_ptr", "n", "ek_assert_buf"]
    assert ck.gen.asserts[0]["msg"] == "x must stay below 100"
    monkeypatch.setenv("ENCELADUS_DEBUG", "0")
    ck2 = C.compile_ir(k.ir_for(x, 100, BLOCK=64))
    assert "assert_fail" not in ck2.hip and "printf(" in ck2.hip
    assert [a.name for a in ck2.args] == ["x_ptr", "n"]
