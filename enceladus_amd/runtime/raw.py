"""`enceladus.hip_kernel`: launch hand-written HIP C++, the expert escape hatch.

The reference's counterpart compiles hand-written MSL (`runtime/raw.py:144-355`,
`metal_kernel`). Here the source is HIP C++ for gfx950, compiled by hiprtc with the same
options as generated kernels (so `#include "enceladus_cdna4.h"` works), and launched with
`kernel[grid, threads_per_group](*args)`; `grid` counts workgroups, as in the reference.

hiprtc has no argument reflection, so the kernel's signature is read from the source:
`extern "C" __global__ void name(T0 a0, T1 a1, ...)`. A pointer parameter takes an array
(NumPy arrays are copied to HBM and back when the pointer is not `const`; torch-ROCm
tensors and `enceladus.Tensor` pass their device pointer); a scalar parameter takes a
Python number, packed as its C type with natural alignment.
"""

from __future__ import annotations

import ctypes
import math
import re
import struct
from typing import Any

import numpy as np

from enceladus_amd.runtime import compile as C
from enceladus_amd.runtime import device as D
from enceladus_amd.runtime import hip
from enceladus_amd.runtime import tensor as T

# C scalar type (normalised) -> struct format
_SCALARS = {
    "float": "f", "double": "d", "_Float16": "e", "__half": "e", "half": "e",
    "int": "i", "int32_t": "i", "signed": "i", "signed int": "i",
    "unsigned": "I", "unsigned int": "I", "uint32_t": "I",
    "long": "q", "long long": "q", "int64_t": "q", "long int": "q",
    "unsigned long": "Q", "unsigned long long": "Q", "uint64_t": "Q", "size_t": "Q",
    "short": "h", "int16_t": "h", "unsigned short": "H", "uint16_t": "H",
    "char": "b", "signed char": "b", "int8_t": "b", "unsigned char": "B", "uint8_t": "B",
    "bool": "?",
}
_BF16 = ("__bf16", "ek::bf16", "bf16", "hip_bfloat16")
MAX_THREADS = 1024


class Param:
    __slots__ = ("name", "ctype", "pointer", "const")

    def __init__(self, name: str, ctype: str, pointer: bool, const: bool):
        self.name, self.ctype, self.pointer, self.const = name, ctype, pointer, const

    def __repr__(self):
        return f"Param({self.ctype}{' const' if self.const else ''}{'*' if self.pointer else ''} {self.name})"


def parse_signature(source: str, name: str) -> list[Param]:
    """The parameters of `extern "C" __global__ ... name(...)` in `source`.

    Raises:
        ValueError: there is no such kernel, or a parameter has a type that can't be packed.
    """
    src = re.sub(r"//[^\n]*|/\*.*?\*/", " ", source, flags=re.S)
    m = re.search(r"__global__[^;{]*?\b" + re.escape(name) + r"\s*\(([^)]*)\)", src, flags=re.S)
    if m is None:
        raise ValueError(f"no `__global__` kernel named '{name}' in the source")
    body = m.group(1).strip()
    if body in ("", "void"):
        return []
    params = []
    for i, raw in enumerate(body.split(",")):
        s = " ".join(raw.replace("*", " * ").split())
        s = re.sub(r"\b(__restrict__|__restrict|restrict|volatile)\b", " ", s)
        s = " ".join(s.split())
        toks = s.split(" ")
        pointer = "*" in toks
        pname = toks[-1] if toks[-1] != "*" else f"arg{i}"
        tt = [t for t in toks[:-1] if t != "*"] if toks[-1] != "*" else [t for t in toks if t != "*"]
        const = "const" in tt
        ctype = " ".join(t for t in tt if t != "const")
        if not pointer and ctype not in _SCALARS and ctype not in _BF16:
            raise ValueError(f"parameter {i} ('{raw.strip()}') of kernel '{name}' has a type "
                             "that Enceladus can't pack from a Python value")
        params.append(Param(pname, ctype, pointer, const))
    return params


def pack(params: list[Param], values: list) -> bytes:
    """Kernarg bytes: pointers as 8 bytes, scalars as their C type, natural alignment."""
    out = bytearray()
    for p, v in zip(params, values):
        if p.pointer:
            fmt, size = "Q", 8
        elif p.ctype in _BF16:
            f32 = np.float32(v).view(np.uint32)
            bits = int((f32 + 0x7FFF + ((f32 >> 16) & 1)) >> 16) & 0xFFFF   # RNE
            if np.isnan(np.float32(v)):
                bits = 0x7FC0
            fmt, size, v = "H", 2, bits
        else:
            fmt = _SCALARS[p.ctype]
            size = struct.calcsize("<" + fmt)
        out += b"\0" * ((-len(out)) % size)
        try:
            out += struct.pack("<" + fmt, v)
        except OverflowError:
            if fmt not in ("f", "e", "d"):
                raise
            out += struct.pack("<" + fmt, math.copysign(math.inf, float(v)))
    out += b"\0" * ((-len(out)) % 8)
    return bytes(out)


def _dim3(v: Any, what: str) -> tuple[int, int, int]:
    if isinstance(v, (int, np.integer)):
        v = (int(v),)
    v = tuple(int(x) for x in v)
    if not 1 <= len(v) <= 3 or any(x < 0 for x in v):
        raise ValueError(f"{what} must be 1 to 3 non-negative integers, got {v}")
    return v + (1,) * (3 - len(v))


class HipKernel:
    """A compiled hand-written HIP kernel; launch with `kernel[grid, threads_per_group](*args)`."""

    def __init__(self, source: str, name: str, options=()):
        self.name = name
        self.source = source
        self.params = parse_signature(source, name)
        self.code = C.compile_code(source, name, tuple(options))
        self._fn = None

    @property
    def arg_names(self) -> list[str]:
        return [p.name for p in self.params]

    def function(self):
        if self._fn is None:
            m, f = ctypes.c_void_p(), ctypes.c_void_p()
            buf = ctypes.create_string_buffer(self.code, len(self.code))
            hip.call("ek_module_load", buf, len(self.code), ctypes.byref(m))
            hip.call("ek_module_function", m, self.name.encode(), ctypes.byref(f))
            self._module, self._fn = m, f
        return self._fn

    def __getitem__(self, key: Any):
        if not (isinstance(key, tuple) and len(key) == 2):
            raise TypeError("launch a raw kernel with kernel[grid, threads_per_group](*args)")
        grid, tg = _dim3(key[0], "grid"), _dim3(key[1], "threads_per_group")
        if min(tg) < 1 or tg[0] * tg[1] * tg[2] > MAX_THREADS:
            raise ValueError(f"threads_per_group {tg} must be 1..{MAX_THREADS} threads")
        return lambda *args: self.launch(grid, tg, args)

    def launch(self, grid, tg, args) -> None:
        if len(args) != len(self.params):
            raise TypeError(f"kernel '{self.name}' takes {len(self.params)} arguments "
                            f"({', '.join(self.arg_names)}), but {len(args)} were given")
        if 0 in grid:
            return
        vals, bindings = [], []
        for p, a in zip(self.params, args):
            if p.pointer:
                if not T.is_array_like(a):
                    raise TypeError(f"argument '{p.name}' is a pointer; pass an array")
                if isinstance(a, np.ndarray) and not p.const and not a.flags.writeable:
                    raise ValueError(f"'{p.name}' is a read-only NumPy array, and the kernel "
                                     "may write to it (its pointer is not const)")
                b = T.bind_array(a)
                b.writeback = not p.const
                bindings.append(b)
                vals.append(b.ptr)
            else:
                if T.is_array_like(a):
                    raise TypeError(f"argument '{p.name}' is a scalar ({p.ctype})")
                vals.append(a)
        kern = pack(self.params, vals)
        buf = ctypes.create_string_buffer(kern, len(kern))
        stream = D.current_stream()
        from enceladus_amd.runtime import debug
        t0 = debug.before_launch(stream) if debug._active is not None else None
        hip.call("ek_launch", ctypes.c_void_p(stream or None), self.function(), grid[0],
                 grid[1], grid[2], tg[0], tg[1], tg[2], 0, buf, len(kern))
        if t0 is not None:
            debug.after_launch(t0, stream, self.name, grid, tg[0] * tg[1] * tg[2], 0)
        T.complete_bindings(bindings)


def hip_kernel(source: str, name: str, options=()) -> HipKernel:
    """Compiles hand-written HIP C++ for gfx950 and returns a launchable kernel.

    Args:
        source: complete source with an `extern "C" __global__` kernel `name`. The device
            templates are available with `#include "enceladus_cdna4.h"`.
        name: the kernel's name.
        options: extra hiprtc options (the gfx950 target and -O3 are always given).

    Returns:
        A kernel launched with `kernel[grid, threads_per_group](*args)`.

    Raises:
        enceladus.MetalError (HipError): the source doesn't compile.
        ValueError: no such kernel, or a parameter type that can't be packed.
    """
    return HipKernel(source, name, options)


def metal_kernel(source: str, name: str, language_version: Any = None,
                 math_mode: str = "relaxed"):
    """MSL can't run on MI355X: port the kernel to HIP C++ and use `hip_kernel`."""
    raise NotImplementedError("metal_kernel takes Metal Shading Language, which doesn't run on "
                              "MI355X; write the kernel in HIP C++ and use enceladus.hip_kernel")
