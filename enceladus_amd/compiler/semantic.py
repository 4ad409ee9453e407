"""Type promotion, broadcasting, and the IR helpers that the builtins share.

The promotion rules are the language's (reference: src/enceladus/compiler/semantic.py:1-175):
a Python literal adopts the other operand's dtype when kinds match (an int literal with a
float operand adopts the float type, a float literal with an int operand gives fp32);
float16 with bfloat16 promotes to fp32; int with float gives the float; same-signedness
integers promote to the wider; mixed signedness picks the unsigned type when it is at
least as wide; int1 arithmetic computes in int32; `/` on integers computes in fp32;
`//` and `%` truncate toward zero as in C; `//` on floats is an error.
"""

from __future__ import annotations

import math
from typing import Any

from enceladus_amd.compiler import ir
from enceladus_amd.compiler.errors import CompilationError
from enceladus_amd.language import core

INT32_MIN, INT32_MAX = -(1 << 31), (1 << 31) - 1
ARITH_OPS = frozenset(["add", "sub", "mul", "div", "floordiv", "mod", "min", "max"])
BITWISE_OPS = frozenset(["and", "or", "xor"])
SHIFT_OPS = frozenset(["shl", "shr"])
CMP_OPS = frozenset(ir.CMP_OPS)


def is_literal(x: Any) -> bool:
    return isinstance(x, (bool, int, float)) and not isinstance(x, ir.Value)


def int_range(dt: core.dtype) -> tuple[int, int]:
    bits = dt.primitive_bitwidth
    if dt.is_bool():
        return 0, 1
    if dt.is_signed():
        return -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    return 0, (1 << bits) - 1


def literal_dtype(v) -> core.dtype:
    if isinstance(v, bool):
        return core.int1
    if isinstance(v, int):
        if INT32_MIN <= v <= INT32_MAX:
            return core.int32
        if -(1 << 63) <= v < (1 << 63):
            return core.int64
        if 0 <= v < (1 << 64):
            return core.uint64
        raise CompilationError(f"integer literal {v} doesn't fit in 64 bits")
    return core.float32


def adopt_literal(v, dt: core.dtype) -> core.dtype:
    if isinstance(v, bool) and dt.is_bool():
        return core.int1
    if isinstance(v, float):
        return dt if dt.is_floating() else core.float32
    if dt.is_floating():
        return dt
    if dt.is_bool():
        return literal_dtype(int(v))
    lo, hi = int_range(dt)
    return dt if lo <= int(v) <= hi else literal_dtype(int(v))


def integer_promote(a: core.dtype, b: core.dtype) -> core.dtype:
    if a is b:
        return a
    if a.is_bool():
        return b
    if b.is_bool():
        return a
    if a.is_signed() == b.is_signed():
        return a if a.primitive_bitwidth >= b.primitive_bitwidth else b
    s, u = (a, b) if a.is_signed() else (b, a)
    return u if u.primitive_bitwidth >= s.primitive_bitwidth else s


def float_promote(a: core.dtype, b: core.dtype) -> core.dtype:
    if a is b:
        return a
    if {a, b} == {core.float16, core.bfloat16}:
        return core.float32
    return a if a.primitive_bitwidth >= b.primitive_bitwidth else b


def computation_dtype(op: str, a, b) -> core.dtype:
    """Dtype in which binary op `op` computes, given operand dtypes or literals."""
    if is_literal(a) and is_literal(b):
        a, b = literal_dtype(a), literal_dtype(b)
    elif is_literal(a):
        a = adopt_literal(a, b)
    elif is_literal(b):
        b = adopt_literal(b, a)
    if op in BITWISE_OPS or op in SHIFT_OPS:
        if not (a.is_int() and b.is_int()):
            raise CompilationError(f"`{op}` needs integer operands, but got {a} and {b}")
    if op == "floordiv" and (a.is_floating() or b.is_floating()):
        raise CompilationError(f"`//` needs integer operands, but got {a} and {b}; "
                               "use tl.floor(x / y) for floats")
    if a.is_floating() or b.is_floating():
        if a.is_floating() and b.is_floating():
            return float_promote(a, b)
        return a if a.is_floating() else b
    if op == "div":
        return core.float32
    t = integer_promote(a, b)
    if t.is_bool() and op in ARITH_OPS | SHIFT_OPS:
        return core.int32
    return t


def broadcast_shapes(a, b) -> tuple[int, ...]:
    a, b = tuple(a), tuple(b)
    n = max(len(a), len(b))
    a = (1,) * (n - len(a)) + a
    b = (1,) * (n - len(b)) + b
    out = []
    for i, (x, y) in enumerate(zip(a, b)):
        if x != y and x != 1 and y != 1:
            raise CompilationError(f"can't broadcast shapes {a} and {b} (dimension {i})")
        out.append(max(x, y))
    return tuple(out)


def check_shape(shape, what: str) -> tuple[int, ...]:
    try:
        dims = tuple(int(core.unwrap(s)) for s in shape)
    except (TypeError, ValueError):
        raise CompilationError(f"{what} must be a tuple of compile-time integers, got {shape!r}")
    n = 1
    for d in dims:
        if d < 1 or d & (d - 1):
            raise CompilationError(f"{what} dimensions must be powers of two, got {dims}")
        n *= d
    if n > ir.MAX_TILE_NUMEL:
        raise CompilationError(f"{what} {dims} has {n} elements; the limit is "
                               f"{ir.MAX_TILE_NUMEL}")
    return dims


def coerce_literal(v, dt: core.dtype):
    """Returns literal `v` as a Python value of `dt` (C-cast semantics for ints)."""
    if dt.is_floating():
        return float(v)
    if dt.is_bool():
        return bool(v)
    if isinstance(v, float):
        if not math.isfinite(v):
            raise CompilationError(f"the value {v!r} doesn't fit in {dt}")
        v = math.trunc(v)
    v = int(v)
    bits = dt.primitive_bitwidth
    lo, hi = int_range(dt)
    if lo <= v <= hi:
        return v
    if not -(1 << (bits - 1)) <= v < (1 << bits):
        raise CompilationError(f"the value {v} doesn't fit in {dt}. Use a value in that range "
                               f"[{lo}, {hi}], or convert the {dt} operand with "
                               "`.to(tl.int32)` (or a wider type) first.")
    v &= (1 << bits) - 1
    if dt.is_signed() and v >> (bits - 1):
        v -= 1 << bits
    return v


# ---------------------------------------------------------------------------
# IR helpers
# ---------------------------------------------------------------------------


def const(b: ir.Builder, v, dt: core.dtype, shape=()) -> ir.Value:
    return b.create("const", [], [ir.TType(tuple(shape), dt)],
                    {"value": coerce_literal(v, dt)}).result


def to_value(b: ir.Builder, x, dt: core.dtype | None = None) -> ir.Value:
    """Converts a literal or value to an IR value, casting to `dt` when given."""
    x = core.unwrap(x)
    if isinstance(x, ir.Value):
        return cast(b, x, dt) if dt is not None else x
    if hasattr(x, "item") and not isinstance(x, (list, tuple)):
        x = x.item()
    if not is_literal(x):
        raise CompilationError(f"expected a number or a tile, but got {type(x).__name__} {x!r}")
    return const(b, x, dt or literal_dtype(x))


def cast(b: ir.Builder, v: ir.Value, dt: core.dtype, bitcast: bool = False) -> ir.Value:
    if v.type.ptr:
        raise CompilationError("can't convert a pointer tile to another dtype")
    if isinstance(v.type, ir.DescType):
        raise CompilationError("can't convert a tensor descriptor")
    if v.type.dtype is dt:
        return v
    if bitcast:
        if v.type.dtype.primitive_bitwidth != dt.primitive_bitwidth:
            raise CompilationError(f"bitcast needs equal widths, got {v.type.dtype} and {dt}")
        return b.create("bitcast", [v], [v.type.with_dtype(dt)]).result
    if v.op is not None and v.op.name == "const" and not v.type.shape:
        # Fold literal casts so constants stay constants.
        val = v.op.attrs["value"]
        if dt.is_bool():
            return const(b, val != 0, dt)
        if dt.is_int() and isinstance(val, float):
            if not math.isfinite(val):
                return b.create("cast", [v], [v.type.with_dtype(dt)]).result
            lo, hi = int_range(dt)
            t = math.trunc(val)
            if dt is not core.int64:
                t = min(max(t, lo), hi)
            return const(b, coerce_literal(t, dt), dt)
        if dt.is_floating():
            return b.create("cast", [v], [v.type.with_dtype(dt)]).result
        return const(b, coerce_literal(val, dt), dt)
    return b.create("cast", [v], [v.type.with_dtype(dt)]).result


def expand_dims(b: ir.Builder, v: ir.Value, axis: int) -> ir.Value:
    shape = list(v.type.shape)
    shape.insert(axis, 1)
    return b.create("expand_dims", [v], [v.type.with_shape(shape)], {"axis": axis}).result


def broadcast_to(b: ir.Builder, v: ir.Value, shape) -> ir.Value:
    shape = tuple(shape)
    if v.type.shape == shape:
        return v
    if v.type.is_scalar:
        return b.create("splat", [v], [v.type.with_shape(shape)]).result
    src = v.type.shape
    if len(src) > len(shape):
        raise CompilationError(f"can't broadcast shape {src} to {shape}")
    while len(v.type.shape) < len(shape):
        v = expand_dims(b, v, 0)
    broadcast_shapes(v.type.shape, shape)
    if v.type.shape == shape:
        return v
    return b.create("broadcast", [v], [v.type.with_shape(shape)]).result


def dtype_of(x) -> core.dtype | Any:
    x = core.unwrap(x)
    if isinstance(x, ir.Value):
        return x.type.dtype
    return x


def shape_of(x) -> tuple[int, ...]:
    x = core.unwrap(x)
    return x.type.shape if isinstance(x, ir.Value) else ()


def binary(b: ir.Builder, op: str, x, y) -> ir.Value:
    """Builds `x op y` with promotion and broadcasting. Pointers support +/- ints."""
    x, y = core.unwrap(x), core.unwrap(y)
    xp = isinstance(x, ir.Value) and x.type.ptr
    yp = isinstance(y, ir.Value) and y.type.ptr
    if xp or yp:
        if op == "add" and yp and not xp:
            x, y = y, x
        elif not (xp and not yp and op in ("add", "sub")):
            raise CompilationError("pointers support only `+` and `-` with an integer offset")
        off = to_value(b, y)
        if not off.type.dtype.is_int():
            raise CompilationError(f"pointer offsets must be integers, got {off.type.dtype}")
        if off.type.dtype.is_bool():
            off = cast(b, off, core.int32)
        if op == "sub":
            off = binary(b, "sub", 0, off)
        shape = broadcast_shapes(x.type.shape, off.type.shape)
        x = broadcast_to(b, x, shape)
        off = broadcast_to(b, off, shape)
        return b.create("ptr_add", [x, off], [x.type]).result
    if isinstance(x, ir.DescType) or isinstance(y, ir.DescType):
        raise CompilationError("tensor descriptors don't support arithmetic")
    dt = computation_dtype(op, dtype_of(x), dtype_of(y))
    xv, yv = to_value(b, x, dt), to_value(b, y, dt)
    shape = broadcast_shapes(xv.type.shape, yv.type.shape)
    xv, yv = broadcast_to(b, xv, shape), broadcast_to(b, yv, shape)
    rdt = core.int1 if op in CMP_OPS else dt
    return b.create("binary", [xv, yv], [ir.TType(shape, rdt)], {"op": op}).result


def unary(b: ir.Builder, op: str, x) -> ir.Value:
    x = to_value(b, x)
    dt = x.type.dtype
    if x.type.ptr:
        raise CompilationError(f"`{op}` doesn't apply to pointers")
    if op in ir.MATH_UNARY and not dt.is_floating():
        raise CompilationError(f"tl.{op} needs a floating-point input, but got {dt}")
    if op == "not":
        if not dt.is_int():
            raise CompilationError(f"`~` needs an integer or boolean operand, but got {dt}")
        return b.create("unary", [x], [x.type], {"op": "not"}).result
    if op == "neg" and dt.is_bool():
        x = cast(b, x, core.int32)
    return b.create("unary", [x], [x.type], {"op": op}).result


def select(b: ir.Builder, c, x, y) -> ir.Value:
    c = to_value(b, c)
    if not c.type.dtype.is_bool():
        c = cast(b, c, core.int1)
    x, y = core.unwrap(x), core.unwrap(y)
    xp = isinstance(x, ir.Value) and x.type.ptr
    if xp:
        dt = x.type.dtype
        xv, yv = x, y
        if not (isinstance(y, ir.Value) and y.type.ptr and y.type.dtype is dt):
            raise CompilationError("tl.where needs two pointer operands of the same type")
    else:
        dt = computation_dtype("select", dtype_of(x), dtype_of(y))
        xv, yv = to_value(b, x, dt), to_value(b, y, dt)
    shape = broadcast_shapes(broadcast_shapes(c.type.shape, xv.type.shape), yv.type.shape)
    c, xv, yv = (broadcast_to(b, v, shape) for v in (c, xv, yv))
    return b.create("select", [c, xv, yv], [xv.type.with_shape(shape)]).result
