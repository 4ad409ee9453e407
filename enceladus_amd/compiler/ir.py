"""SSA tile IR.

One `func` per specialization. Values are tiles (shape `()` is a scalar); element types
are tile dtypes or pointers to them; tensor descriptors have their own type. Structured
control flow (`for`, `if`) owns regions whose blocks end in `yield`.

The op vocabulary follows the reference IR's verifier table
(reference: src/enceladus/compiler/ir.py:788-832) in meaning, not in spelling.
"""

from __future__ import annotations

import itertools
from dataclasses import dataclass, field
from typing import Any

from enceladus_amd.language import core

MAX_TILE_NUMEL = 1 << 16
CMP_OPS = ("eq", "ne", "lt", "le", "gt", "ge")
MATH_UNARY = ("exp", "exp2", "log", "log2", "sqrt", "rsqrt", "sin", "cos", "tanh", "sigmoid",
              "erf", "floor", "ceil")


@dataclass(frozen=True)
class TType:
    """A tile type: `shape` (`()` for scalars), element dtype, and pointer flag."""

    shape: tuple[int, ...]
    dtype: core.dtype
    ptr: bool = False

    @property
    def numel(self) -> int:
        n = 1
        for s in self.shape:
            n *= s
        return n

    @property
    def is_scalar(self) -> bool:
        return self.shape == ()

    def with_shape(self, shape) -> "TType":
        return TType(tuple(shape), self.dtype, self.ptr)

    def with_dtype(self, dt: core.dtype, ptr: bool = False) -> "TType":
        return TType(self.shape, dt, ptr)

    def __str__(self) -> str:
        e = f"ptr<{self.dtype.ir_name}>" if self.ptr else self.dtype.ir_name
        if not self.shape:
            return e
        return f"tile<{'x'.join(map(str, self.shape))}x{e}>"


@dataclass(frozen=True)
class DescType:
    """A tensor descriptor over `dtype` elements with a compile-time block shape."""

    dtype: core.dtype
    block_shape: tuple[int, ...]

    @property
    def rank(self) -> int:
        return len(self.block_shape)

    shape = ()
    ptr = False
    is_scalar = True

    def __str__(self) -> str:
        return f"desc<{'x'.join(map(str, self.block_shape))}x{self.dtype.ir_name}>"


_ids = itertools.count()


class Value:
    __slots__ = ("type", "op", "index", "id", "name_hint", "facts")

    def __init__(self, type_, op=None, index=0, name_hint=""):
        self.type = type_
        self.op = op
        self.index = index
        self.id = next(_ids)
        self.name_hint = name_hint
        self.facts: dict[str, Any] = {}

    def __repr__(self) -> str:
        return f"%{self.id}"


class Block:
    def __init__(self, arg_types=()):
        self.args = [Value(t) for t in arg_types]
        self.ops: list[Op] = []


class Op:
    __slots__ = ("name", "operands", "results", "attrs", "regions", "loc")

    def __init__(self, name, operands, result_types=(), attrs=None, regions=(), loc=None):
        self.name = name
        self.operands = list(operands)
        self.results = [Value(t, self, i) for i, t in enumerate(result_types)]
        self.attrs = dict(attrs or {})
        self.regions = list(regions)
        self.loc = loc

    @property
    def result(self) -> Value:
        return self.results[0]


@dataclass
class Func:
    name: str
    args: list[Value]
    arg_names: list[str]
    body: Block
    num_warps: int = 4
    attrs: dict[str, Any] = field(default_factory=dict)


class Builder:
    """Appends ops to the current block."""

    def __init__(self, block: Block):
        self.block = block
        self.loc = None

    def create(self, name, operands, result_types=(), attrs=None, regions=()) -> Op:
        op = Op(name, operands, result_types, attrs, regions, self.loc)
        self.block.ops.append(op)
        return op


def walk(block: Block):
    """Yields every op of `block`, pre-order, including nested regions."""
    for op in block.ops:
        yield op
        for r in op.regions:
            yield from walk(r)


def _fmt_attr(v: Any) -> str:
    if isinstance(v, core.dtype):
        return v.ir_name
    if isinstance(v, float):
        return repr(v)
    return repr(v)


def print_func(fn: Func) -> str:
    """Returns a deterministic text form of the function (used in cache keys and dumps)."""
    names: dict[int, str] = {}
    counter = itertools.count()

    def nm(v: Value) -> str:
        if v.id not in names:
            names[v.id] = f"%{next(counter)}"
        return names[v.id]

    lines = []
    args = ", ".join(f"{nm(a)}: {a.type} {a.facts if a.facts else ''}".rstrip()
                     for a in fn.args)
    lines.append(f"func @{fn.name}({args}) warps={fn.num_warps} {fn.attrs} {{")

    def block(b: Block, ind: int):
        pad = "  " * ind
        for op in b.ops:
            res = ", ".join(nm(r) for r in op.results)
            lhs = f"{res} = " if res else ""
            ops = ", ".join(nm(o) for o in op.operands)
            attrs = ", ".join(f"{k}={_fmt_attr(v)}" for k, v in sorted(op.attrs.items()))
            types = ", ".join(str(r.type) for r in op.results)
            lines.append(f"{pad}{lhs}{op.name}({ops}) {{{attrs}}} : {types}")
            for i, r in enumerate(op.regions):
                ba = ", ".join(nm(a) for a in r.args)
                lines.append(f"{pad}  ^region{i}({ba}):")
                block(r, ind + 2)

    block(fn.body, 1)
    lines.append("}")
    return "\n".join(lines)


# ops without side effects: removable when nothing reads their results
PURE_OPS = frozenset(["const", "binary", "unary", "cast", "bitcast", "select", "splat",
                      "broadcast", "expand_dims", "reshape", "trans", "hint", "arange",
                      "program_id", "num_programs", "fma", "ptr_add", "join", "split",
                      "shift"])


def dce(fn: Func) -> int:
    """Removes pure ops whose results nothing reads (e.g. a loop variable's after-loop
    value that the kernel never uses). Returns how many ops were removed."""
    used: dict[int, int] = {}

    def count(b: Block):
        for op in b.ops:
            for o in op.operands:
                used[o.id] = used.get(o.id, 0) + 1
            for r in op.regions:
                count(r)
    count(fn.body)
    removed = 0

    def sweep(b: Block):
        nonlocal removed
        keep = []
        for op in reversed(b.ops):
            for r in op.regions:
                sweep(r)
            if op.name in PURE_OPS and not op.regions and op.results and \
                    all(used.get(r.id, 0) == 0 for r in op.results):
                for o in op.operands:
                    used[o.id] -= 1
                removed += 1
                continue
            keep.append(op)
        b.ops = keep[::-1]
    sweep(fn.body)
    return removed
