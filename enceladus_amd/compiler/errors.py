"""Compiler and runtime error types (reference: src/enceladus/compiler/errors.py:26-98)."""

from __future__ import annotations


class CompilationError(Exception):
    """A kernel the compiler rejects, located at the kernel source line when known."""

    def __init__(self, msg: str, loc: tuple[str, int] | None = None, src_line: str | None = None,
                 col: int | None = None):
        self.msg = msg
        self.loc = loc
        text = msg
        if loc is not None:
            text = f"{loc[0]}:{loc[1]}: {msg}"
            if src_line:
                # the kernel's line as written, and a caret under the offending expression
                line = src_line.rstrip("\n").rstrip()
                text += f"\n{line}"
                if col is None:
                    col = len(line) - len(line.lstrip())
                text += "\n" + " " * col + "^"
        super().__init__(text)


class DeviceAssertionError(AssertionError):
    """A `tl.device_assert` failed while a kernel ran (reference: errors.py:77-98).

    Attributes:
        message: the assert's message.
        loc: (file, line) of the `tl.device_assert` call, or None.
        program_id: the (x, y, z) program id of the first failing program.
    """

    def __init__(self, message: str = "", loc: tuple[str, int] | None = None,
                 program_id: tuple[int, int, int] = (0, 0, 0)):
        self.message = message
        self.loc = loc
        self.program_id = tuple(program_id)
        super().__init__(str(self))

    def __str__(self) -> str:
        pid = ", ".join(map(str, self.program_id))
        what = f"device assertion failed in program ({pid})"
        text = f"{what}: {self.message}" if self.message else what
        return f"{self.loc[0]}:{self.loc[1]}: {text}" if self.loc else text


class HipError(RuntimeError):
    """An error reported by the HIP runtime or the hiprtc compiler."""
