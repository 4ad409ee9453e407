"""Structural and type checks of the tile IR, run between compiler stages.

`verify(fn, stage)` checks that every value is defined once and before its uses (in its
own block or an enclosing one), that regions end with the terminator their op needs, and
each op's operand and result counts, types and shapes against the op's rule below. A
violation raises `CompilationError` naming the stage that produced the IR, the op and its
source line. The compiler runs it after the frontend, the simplifier, index widening, the
attention scale rewrite and dead-code elimination when `ENCELADUS_VERIFY=1` (the test
suite sets it) (reference: src/enceladus/compiler/ir.py:788-851, `ENCELADUS_VERIFY`).
"""

from __future__ import annotations

import os

from enceladus_amd.compiler import ir
from enceladus_amd.compiler.errors import CompilationError
from enceladus_amd.language import core

ARITH = ("add", "sub", "mul", "div", "floordiv", "mod", "and", "or", "xor", "shl", "shr",
         "min", "max", "pow")
UNARY = ("neg", "abs", "not") + ir.MATH_UNARY
INT_ONLY = ("floordiv", "and", "or", "xor", "shl", "shr")


def enabled() -> bool:
    return os.environ.get("ENCELADUS_VERIFY", "0") not in ("", "0")


class _Fail(Exception):
    pass


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise _Fail(msg)


def _tile(v: ir.Value) -> ir.TType:
    _need(isinstance(v.type, ir.TType), f"{v} must be a tile or scalar, not {v.type}")
    return v.type


def _data(v: ir.Value) -> ir.TType:
    t = _tile(v)
    _need(not t.ptr, f"{v} must hold data, not pointers")
    return t


def _ptr(v: ir.Value) -> ir.TType:
    t = _tile(v)
    _need(t.ptr, f"{v} must be a pointer or pointer tile")
    return t


def _scalar_int(v: ir.Value) -> None:
    t = _data(v)
    _need(t.is_scalar and t.dtype.is_int(), f"{v} must be an integer scalar, not {t}")


def _arity(op: ir.Op, n_in, n_out: int) -> None:
    ok = len(op.operands) in n_in if isinstance(n_in, tuple) else len(op.operands) == n_in
    _need(ok, f"takes {n_in} operands, has {len(op.operands)}")
    _need(len(op.results) == n_out, f"has {len(op.results)} results, expected {n_out}")


def _same_shape(op: ir.Op, vals) -> None:
    shapes = {tuple(v.type.shape) for v in vals}
    _need(len(shapes) == 1, f"operand and result shapes differ: {sorted(shapes)}")


def _v_const(op):
    _arity(op, 0, 1)
    _data(op.result)
    _need("value" in op.attrs, "a constant needs a `value`")


def _v_pid(op):
    _arity(op, 0, 1)
    t = _data(op.result)
    _need(t.is_scalar and t.dtype is core.int32, "program ids are int32 scalars")
    _need(op.attrs.get("axis") in (0, 1, 2), "axis must be 0, 1 or 2")


def _v_arange(op):
    _arity(op, 0, 1)
    t = _data(op.result)
    _need(len(t.shape) == 1 and t.dtype is core.int32, "tl.arange gives a 1-D int32 tile")
    n = t.shape[0]
    _need(n > 0 and n & (n - 1) == 0 and n <= ir.MAX_TILE_NUMEL,
          f"tile size {n} is not a power of two up to {ir.MAX_TILE_NUMEL}")


def _v_binary(op):
    _arity(op, 2, 1)
    a, b = (_tile(o) for o in op.operands)
    r = _data(op.result)
    k = op.attrs.get("op")
    _same_shape(op, op.operands + op.results)
    _need(a.dtype is b.dtype, f"operand dtypes differ: {a.dtype}, {b.dtype}")
    if k in ir.CMP_OPS:
        _need(r.dtype is core.int1, "comparisons give int1")
    else:
        _need(k in ARITH, f"unknown binary op `{k}`")
        _need(not a.ptr, "arithmetic on pointers goes through ptr_add")
        _need(r.dtype is a.dtype, f"result dtype {r.dtype} differs from operands' {a.dtype}")
        if k in INT_ONLY:
            _need(r.dtype.is_int(), f"`{k}` needs integers")


def _v_unary(op):
    _arity(op, 1, 1)
    k = op.attrs.get("op")
    _need(k in UNARY, f"unknown unary op `{k}`")
    a, r = _data(op.operands[0]), _data(op.result)
    _same_shape(op, op.operands + op.results)
    _need(a.dtype is r.dtype, "a unary op keeps the dtype")
    if k in ir.MATH_UNARY:
        _need(a.dtype.is_floating(), f"tl.{k} needs a floating-point operand")


def _v_fma(op):
    _arity(op, 3, 1)
    _same_shape(op, op.operands + op.results)
    _need(all(_data(o).dtype is op.result.type.dtype for o in op.operands),
          "fma operands and result share one dtype")


def _v_select(op):
    _arity(op, 3, 1)
    c = _data(op.operands[0])
    _need(c.dtype is core.int1, "the condition must be int1")
    _same_shape(op, op.operands + op.results)
    r = _tile(op.result)
    for v in op.operands[1:]:
        t = _tile(v)
        _need(t.dtype is r.dtype and t.ptr == r.ptr, "both values have the result's type")


def _v_cast(op):
    _arity(op, 1, 1)
    a, r = _data(op.operands[0]), _data(op.result)
    _need(a.shape == r.shape, "a conversion keeps the shape")


def _v_bitcast(op):
    _v_cast(op)
    a, r = op.operands[0].type, op.result.type
    _need(a.dtype.primitive_bitwidth == r.dtype.primitive_bitwidth,
          "a bitcast keeps the bit width")


def _v_splat(op):
    _arity(op, 1, 1)
    a, r = _tile(op.operands[0]), _tile(op.result)
    _need(a.is_scalar and not r.is_scalar, "splat makes a tile of a scalar")
    _need(a.dtype is r.dtype and a.ptr == r.ptr, "splat keeps the element type")


def _v_broadcast(op):
    _arity(op, 1, 1)
    a, r = _tile(op.operands[0]), _tile(op.result)
    _need(len(a.shape) == len(r.shape), "broadcast keeps the rank")
    _need(all(x in (1, y) for x, y in zip(a.shape, r.shape)),
          f"can't broadcast {a.shape} to {r.shape}")
    _need(a.dtype is r.dtype and a.ptr == r.ptr, "broadcast keeps the element type")


def _v_expand_dims(op):
    _arity(op, 1, 1)
    a, r = _tile(op.operands[0]), _tile(op.result)
    ax = op.attrs.get("axis")
    _need(isinstance(ax, int) and 0 <= ax <= len(a.shape), "bad axis")
    want = list(a.shape)
    want.insert(ax, 1)
    _need(tuple(want) == r.shape, f"expand_dims of {a.shape} at {ax} is {tuple(want)}")
    _need(a.dtype is r.dtype and a.ptr == r.ptr, "expand_dims keeps the element type")


def _v_reshape(op):
    _arity(op, 1, 1)
    a, r = _tile(op.operands[0]), _tile(op.result)
    _need(a.numel == r.numel, f"reshape of {a.shape} to {r.shape} changes the element count")
    _need(a.dtype is r.dtype and a.ptr == r.ptr, "reshape keeps the element type")


def _v_trans(op):
    _arity(op, 1, 1)
    a, r = _tile(op.operands[0]), _tile(op.result)
    perm = tuple(op.attrs.get("perm", ()))
    _need(sorted(perm) == list(range(len(a.shape))), f"`perm` {perm} is not a permutation")
    _need(tuple(a.shape[p] for p in perm) == r.shape, "trans shape mismatch")


def _v_join(op):
    _arity(op, 2, 1)
    a, b, r = (_data(v) for v in (op.operands[0], op.operands[1], op.result))
    _need(a == b, "join takes two tiles of one type")
    _need(r.shape == a.shape + (2,) and r.dtype is a.dtype, "join appends a dim of 2")


def _v_split(op):
    _arity(op, 1, 2)
    a = _data(op.operands[0])
    _need(a.shape and a.shape[-1] == 2, "split needs a last dim of 2")
    for r in op.results:
        _need(_data(r).shape == a.shape[:-1] and r.type.dtype is a.dtype,
              "split drops the last dim")


def _v_shift(op):
    _arity(op, 1, 1)
    _need(op.operands[0].type == op.result.type, "shift keeps the type")


def _v_ptr_add(op):
    _arity(op, 2, 1)
    p = _ptr(op.operands[0])
    o = _data(op.operands[1])
    _need(o.dtype.is_int(), "pointer offsets are integers")
    _need(op.result.type == p, "ptr_add keeps the pointer type")
    _need(o.shape in ((), p.shape), "offset and pointer shapes differ")


def _v_load(op):
    _arity(op, (1, 3), 1)
    p = _ptr(op.operands[0])
    r = _data(op.result)
    _need(r.shape == p.shape and r.dtype is p.dtype, "a load gives the pointee tile")
    if len(op.operands) == 3:
        m, o = _data(op.operands[1]), _data(op.operands[2])
        _need(m.dtype is core.int1 and m.shape == p.shape, "the mask is int1 of the shape")
        _need(o.dtype is p.dtype and o.shape == p.shape, "`other` has the pointee type")


def _v_store(op):
    _arity(op, (2, 3), 0)
    p = _ptr(op.operands[0])
    v = _data(op.operands[1])
    _need(v.shape == p.shape and v.dtype is p.dtype, "the stored tile matches the pointers")
    if len(op.operands) == 3:
        m = _data(op.operands[2])
        _need(m.dtype is core.int1 and m.shape == p.shape, "the mask is int1 of the shape")


def _v_make_desc(op):
    _need(len(op.results) == 1 and isinstance(op.result.type, ir.DescType),
          "make_desc gives a descriptor")
    t = op.result.type
    _need(len(op.operands) == 1 + 2 * t.rank, "make_desc takes the base, shape and strides")
    p = _ptr(op.operands[0])
    _need(p.is_scalar and p.dtype is t.dtype, "the base is a scalar pointer to the elements")
    for v in op.operands[1:]:
        _scalar_int(v)


def _v_desc_load(op):
    d = op.operands[0].type
    _need(isinstance(d, ir.DescType), "desc_load reads a descriptor")
    _arity(op, 1 + d.rank, 1)
    for v in op.operands[1:]:
        _scalar_int(v)
    r = _data(op.result)
    _need(r.shape == d.block_shape and r.dtype is d.dtype, "desc_load gives the block")


def _v_desc_store(op):
    d = op.operands[0].type
    _need(isinstance(d, ir.DescType), "desc_store writes a descriptor")
    _arity(op, 2 + d.rank, 0)
    for v in op.operands[1:-1]:
        _scalar_int(v)
    v = _data(op.operands[-1])
    _need(v.shape == d.block_shape and v.dtype is d.dtype, "desc_store takes the block")


def _v_atomic(op):
    _need(len(op.results) == 1, "an atomic gives the old values")
    p = _ptr(op.operands[0])
    r = _data(op.result)
    _need(r.shape == p.shape and r.dtype is p.dtype, "old values have the pointee type")
    for v in op.operands[1:]:
        t = _data(v)
        _need(t.shape == p.shape, "atomic operands have the pointers' shape")


def _v_dot(op):
    _arity(op, 3, 1)
    a, b, c = (_data(v) for v in op.operands)
    r = _data(op.result)
    _need(len(a.shape) == 2 and len(b.shape) == 2, "tl.dot multiplies 2-D tiles")
    m, k = a.shape
    k2, n = b.shape
    _need(k == k2, f"inner dims differ: {a.shape} x {b.shape}")
    _need(r.shape == (m, n) and c.shape == (m, n), "accumulator and result are [M, N]")
    _need(a.dtype is b.dtype, "both operands have one dtype")


def _v_reduce(op):
    _need(len(op.operands) == 1 and len(op.results) == 1, "reduce takes and gives one tile")
    a, r = _data(op.operands[0]), _data(op.result)
    ax = op.attrs.get("axis")
    want = () if ax is None else a.shape[:ax] + a.shape[ax + 1:]
    _need(r.shape == want, f"reduce of {a.shape} over {ax} gives {want}, not {r.shape}")


def _v_scan(op):
    _need(len(op.operands) == 1 and len(op.results) == 1, "scan takes and gives one tile")
    _need(op.operands[0].type.shape == op.result.type.shape, "scan keeps the shape")


def _v_for(op):
    _need(len(op.operands) >= 3 and len(op.regions) == 1, "for: bounds, inits, one body")
    for v in op.operands[:3]:
        _scalar_int(v)
    inits = op.operands[3:]
    body = op.regions[0]
    _need(len(body.args) == 1 + len(inits), "the body takes the index and carried values")
    _need(len(op.results) == len(inits), "one result per carried value")
    for a, i, r in zip(body.args[1:], inits, op.results):
        _need(a.type == i.type == r.type, f"carried types differ: {i.type}, {a.type}, {r.type}")
    y = body.ops[-1] if body.ops else None
    _need(y is not None and y.name == "yield", "the body ends with yield")
    _need([v.type for v in y.operands] == [a.type for a in body.args[1:]],
          "yield types differ from the carried types")


def _v_if(op):
    _need(len(op.operands) == 1 and len(op.regions) == 2, "if: a condition and two regions")
    c = _data(op.operands[0])
    _need(c.is_scalar and c.dtype is core.int1, "the condition is an int1 scalar")
    for blk in op.regions:
        y = blk.ops[-1] if blk.ops else None
        _need(y is not None and y.name == "yield", "each branch ends with yield")
        _need([v.type for v in y.operands] == [r.type for r in op.results],
              "a branch yields values of other types than the results")


def _v_yield(op):
    _need(not op.results, "yield has no results")


def _v_effect(op):
    _need(not op.results, f"`{op.name}` has no results")


def _v_hint(op):
    _arity(op, 1, 1)
    _need(op.operands[0].type == op.result.type, "a hint keeps the type")


RULES = {
    "const": _v_const, "program_id": _v_pid, "num_programs": _v_pid, "arange": _v_arange,
    "binary": _v_binary, "unary": _v_unary, "fma": _v_fma, "select": _v_select,
    "cast": _v_cast, "bitcast": _v_bitcast, "splat": _v_splat, "broadcast": _v_broadcast,
    "expand_dims": _v_expand_dims, "reshape": _v_reshape, "trans": _v_trans,
    "join": _v_join, "split": _v_split, "shift": _v_shift, "ptr_add": _v_ptr_add,
    "load": _v_load, "store": _v_store, "make_desc": _v_make_desc,
    "desc_load": _v_desc_load, "desc_store": _v_desc_store, "atomic_rmw": _v_atomic,
    "atomic_cas": _v_atomic, "dot": _v_dot, "reduce": _v_reduce, "scan": _v_scan,
    "for": _v_for, "if": _v_if, "yield": _v_yield, "barrier": _v_effect,
    "assert": _v_effect, "print": _v_effect, "hint": _v_hint,
}


def verify(fn: ir.Func, stage: str = "") -> None:
    """Raises CompilationError if `fn` is malformed (see the module docstring)."""
    seen: set[int] = set()

    def where(op):
        loc = f" ({op.loc})" if getattr(op, "loc", None) else ""
        after = f" after {stage}" if stage else ""
        return f"invalid IR{after}: `{op.name}`{loc}"

    def define(v: ir.Value, op, visible: set[int]):
        if v.id in seen:
            raise CompilationError(f"{where(op)}: value {v} is defined twice")
        seen.add(v.id)
        visible.add(v.id)

    def block(b: ir.Block, visible: set[int], owner, terminated: bool):
        for a in b.args:
            define(a, owner, visible)
        for i, op in enumerate(b.ops):
            if op.name == "yield" and i != len(b.ops) - 1:
                raise CompilationError(f"{where(op)}: yield must end its region")
            for o in op.operands:
                if o.id not in visible:
                    raise CompilationError(f"{where(op)}: operand {o} is used before its "
                                           "definition or outside its region")
            rule = RULES.get(op.name)
            if rule is None:
                raise CompilationError(f"{where(op)}: unknown op")
            try:
                rule(op)
            except _Fail as e:
                raise CompilationError(f"{where(op)}: {e}") from None
            for r in op.regions:
                block(r, set(visible), op, True)
            for r in op.results:
                define(r, op, visible)
        if terminated and (not b.ops or b.ops[-1].name != "yield"):
            raise CompilationError(f"invalid IR{' after ' + stage if stage else ''}: a "
                                   f"region of `{owner.name}` does not end with yield")
        if not terminated and b.ops and any(op.name == "yield" for op in b.ops):
            raise CompilationError(f"invalid IR{' after ' + stage if stage else ''}: yield "
                                   "in the function body")

    top: set[int] = set()
    for a in fn.args:
        if a.id in seen:
            raise CompilationError(f"invalid IR: argument {a} appears twice")
        seen.add(a.id)
        top.add(a.id)
    block(fn.body, top, None, False)


def maybe_verify(fn: ir.Func, stage: str) -> None:
    if enabled():
        verify(fn, stage)
