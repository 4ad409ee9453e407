"""Compile-time evaluation of elementwise ops on constants, with the language's semantics.

The simplifier folds an op whose operands are all constant into a constant. The value it
computes must be the one the interpreter computes for the same op, bit for bit, so that a
folded kernel and an unfolded one agree with the interpreter (reference:
interpreter/interp.py:501-690 and language/ops.py, whose rules these restate):

- floats compute in float32 and round to the result dtype after each op (fp16 through
  NumPy's cast, bf16 to nearest-even); min/max ignore NaN; `%` is `fmod`;
- integers wrap modulo 2^bits; `//` and `%` truncate toward zero;
- float-to-integer conversion truncates toward zero;
- comparisons give int1.

Cases whose result the language leaves to the hardware stay unfolded (the functions return
None), so the GPU computes them as it would unfolded: integer division or remainder by
zero and the most negative value divided by -1, shifts by a negative amount or by the bit
width or more, negation and `abs` of the most negative integer, and float-to-integer
conversion of NaN, infinities and out-of-range values.

Values are carried as NumPy scalars: integers in their NumPy type, booleans as `np.bool_`,
floats of every width as the `np.float32` holding the dtype's value.
"""

from __future__ import annotations

import math

import numpy as np

from enceladus_amd.language import core

_NP_INT = {core.int8: np.int8, core.int16: np.int16, core.int32: np.int32,
           core.int64: np.int64, core.uint8: np.uint8, core.uint16: np.uint16,
           core.uint32: np.uint32, core.uint64: np.uint64}


def bf16_round(x: np.float32) -> np.float32:
    """The bfloat16 value nearest to float32 `x` (ties to even; NaN stays NaN)."""
    u = int(np.array([x], np.float32).view(np.uint32)[0])
    if (u & 0x7FFFFFFF) > 0x7F800000:
        r = ((u >> 16) | 0x40) << 16
    else:
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return np.array([r & 0xFFFFFFFF], np.uint32).view(np.float32)[0]


def round_float(x, dt: core.dtype) -> np.float32:
    """A float32 computation result rounded to float dtype `dt` (as a float32)."""
    x = np.float32(x)
    if dt is core.float16:
        return np.float32(np.float16(x))
    if dt is core.bfloat16:
        return bf16_round(x)
    return x


def scalar(value, dt: core.dtype):
    """A const op's `value` attribute as a NumPy scalar of dtype `dt`."""
    if dt.is_bool():
        return np.bool_(bool(value))
    if dt.is_floating():
        if dt is core.float16:
            return np.float32(np.float16(float(value)))
        return round_float(np.float32(float(value)), dt)
    v = int(value)
    bits = dt.primitive_bitwidth
    v &= (1 << bits) - 1
    if dt.is_signed() and v >> (bits - 1):
        v -= 1 << bits
    return _NP_INT[dt](v)


def attr(x, dt: core.dtype):
    """A NumPy scalar as the Python value a const op stores."""
    if dt.is_bool():
        return bool(x)
    if dt.is_floating():
        return float(np.float32(x))
    return int(x)


def _int_min(dt):
    return -(1 << (dt.primitive_bitwidth - 1)) if dt.is_signed() else 0


def binary(op: str, a, b, dt: core.dtype):
    """`a op b` for operands of dtype `dt` (comparisons give np.bool_), or None."""
    with np.errstate(all="ignore"):
        if op in ("eq", "ne", "lt", "le", "gt", "ge"):
            f = {"eq": np.equal, "ne": np.not_equal, "lt": np.less, "le": np.less_equal,
                 "gt": np.greater, "ge": np.greater_equal}[op]
            return np.bool_(f(a, b))
        if dt.is_floating():
            x, y = np.float32(a), np.float32(b)
            r = {"add": lambda: x + y, "sub": lambda: x - y, "mul": lambda: x * y,
                 "div": lambda: x / y, "mod": lambda: np.fmod(x, y),
                 "min": lambda: np.fmin(x, y), "max": lambda: np.fmax(x, y)}.get(op)
            return None if r is None else round_float(r(), dt)
        if dt.is_bool():
            x, y = bool(a), bool(b)
            r = {"and": x and y, "or": x or y, "xor": x != y}.get(op)
            return None if r is None else np.bool_(r)
        t = _NP_INT[dt]
        bits = dt.primitive_bitwidth
        x, y = int(a), int(b)
        if op in ("floordiv", "mod"):
            if y == 0 or (dt.is_signed() and x == _int_min(dt) and y == -1):
                return None
            q = abs(x) // abs(y)
            q = q if (x >= 0) == (y >= 0) else -q
            return scalar(q if op == "floordiv" else x - q * y, dt)
        if op in ("shl", "shr"):
            if y < 0 or y >= bits:
                return None
            if op == "shl":
                return scalar(x << y, dt)
            return t(x >> y)         # arithmetic for signed, logical for unsigned
        r = {"add": x + y, "sub": x - y, "mul": x * y, "and": x & y, "or": x | y,
             "xor": x ^ y, "min": min(x, y), "max": max(x, y)}.get(op)
        return None if r is None else scalar(r, dt)


def _erf(a: np.ndarray) -> np.ndarray:
    return np.array([math.erf(float(v)) for v in a], np.float64).astype(np.float32)


_MATH = {"exp": np.exp, "exp2": np.exp2, "log": np.log, "log2": np.log2, "sqrt": np.sqrt,
         "rsqrt": lambda a: np.float32(1.0) / np.sqrt(a), "sin": np.sin, "cos": np.cos,
         "tanh": np.tanh, "sigmoid": lambda a: np.float32(1.0) / (np.float32(1.0) + np.exp(-a)),
         "erf": _erf, "floor": np.floor, "ceil": np.ceil}


def unary(op: str, a, dt: core.dtype):
    """`op(a)` for an operand of dtype `dt`, or None."""
    with np.errstate(all="ignore"):
        if dt.is_floating():
            x = np.float32(a)
            if op == "neg":
                return round_float(-x, dt)
            if op == "abs":
                return round_float(np.abs(x), dt)
            f = _MATH.get(op)
            if f is None:
                return None
            # evaluated on a one-element array, as the interpreter evaluates tiles
            return round_float(f(np.array([x], np.float32))[0], dt)
        if dt.is_bool():
            return np.bool_(not bool(a)) if op == "not" else None
        x = int(a)
        if op in ("neg", "abs") and dt.is_signed() and x == _int_min(dt):
            return None
        r = {"neg": -x, "abs": abs(x), "not": ~x}.get(op)
        return None if r is None else scalar(r, dt)


def cast(a, src: core.dtype, dst: core.dtype):
    """Converts `a` of dtype `src` to `dst`, or None where the result is left to the
    hardware."""
    if src is dst:
        return a
    with np.errstate(all="ignore"):
        if dst.is_bool():
            return np.bool_(a != 0)
        if src.is_floating() and dst.is_int():
            x = float(a)
            if not math.isfinite(x):
                return None
            t = math.trunc(x)
            lo, hi = (_int_min(dst), (1 << (dst.primitive_bitwidth - (1 if dst.is_signed()
                                                                          else 0))) - 1)
            if not lo <= t <= hi:
                return None
            return scalar(t, dst)
        if dst.is_floating():
            if src.is_floating():
                return round_float(np.float32(a), dst)
            if dst is core.float16:       # integers convert to fp16 in one rounding
                return np.float32(np.float16(int(a)))
            return round_float(np.float32(int(a)), dst)
        return scalar(int(a), dst)
