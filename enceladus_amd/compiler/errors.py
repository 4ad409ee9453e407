"""Compiler and runtime error types (reference: src/enceladus/compiler/errors.py:26-98)."""

from __future__ import annotations


class CompilationError(Exception):
    """A kernel the compiler rejects, located at the kernel source line when known."""

    def __init__(self, msg: str, loc: tuple[str, int] | None = None, src_line: str | None = None):
        self.msg = msg
        self.loc = loc
        text = msg
        if loc is not None:
            text = f"{loc[0]}:{loc[1]}: {msg}"
            if src_line:
                text += f"\n    {src_line.strip()}"
        super().__init__(text)


class DeviceAssertionError(RuntimeError):
    """A `tl.device_assert` that failed on the device."""


class HipError(RuntimeError):
    """An error reported by the HIP runtime or the hiprtc compiler."""
