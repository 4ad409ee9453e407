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
