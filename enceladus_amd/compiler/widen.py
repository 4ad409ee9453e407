"""64-bit index math for kernels whose array arguments span more than 2^31 elements.

A launch sets the `idx64` fact on an array argument whose last element lies more than
2^31 - 1 elements past its first (an MI355X holds 288 GB, so a 9 GB fp32 array is
enough). For such a kernel this pass recomputes in 64 bits the signed integer math that
feeds pointer offsets, and the comparisons that read it (the mask `offs < n`), so the
address and the mask agree on the exact offset: `pid * BLOCK + tl.arange(0, BLOCK)` no
longer wraps at 2^31 (reference behaviour: compiler/passes/widen_index.py:1-25).

The index slice is every signed 8/16/32-bit value that a `ptr_add` offset, or a
comparison reading the slice, computes from through arithmetic and shape ops:

- such a value computed by a cloneable op (arithmetic, select, shape views, constants)
  gets a 64-bit twin placed right after it, computed from the operands' twins;
- any other one (a kernel argument, `tl.program_id`, `tl.arange`, a load, a loop index
  or a loop-carried value) gets a cast to int64 right after its definition;
- a cast of a slice value to int64 is replaced by the twin.

Uses outside the slice (storing `offs` as data) keep the 32-bit value; values a loop
carries in 32 bits still wrap across iterations (carry a pointer or an int64 instead).
"""

from __future__ import annotations

from enceladus_amd.compiler import ir
from enceladus_amd.compiler.errors import CompilationError
from enceladus_amd.language import core

_NARROW = (core.int8, core.int16, core.int32)
_CMP = ("eq", "ne", "lt", "le", "gt", "ge")
# ops whose twin, built from 64-bit operands, computes the exact value of the original
_CLONE = ("binary", "unary", "select", "splat", "broadcast", "expand_dims", "reshape",
          "trans", "hint", "const")


def _narrow(v: ir.Value) -> bool:
    t = v.type
    return isinstance(t, ir.TType) and not t.ptr and t.dtype in _NARROW


def _cast_source(v: ir.Value):
    """`x` when `v` is a cast of a narrow signed `x` to int64."""
    op = v.op
    if op is not None and op.name == "cast" and isinstance(v.type, ir.TType) and \
            not v.type.ptr and v.type.dtype is core.int64 and _narrow(op.operands[0]):
        return op.operands[0]
    return None


def _is_cmp(op: ir.Op) -> bool:
    return op.name == "binary" and op.attrs.get("op") in _CMP


def needs_idx64(fn: ir.Func) -> bool:
    return any(a.facts.get("idx64") for a in fn.args)


def _check_descriptors(fn: ir.Func) -> None:
    for op in ir.walk(fn.body):
        if op.name != "make_desc":
            continue
        base = op.operands[0]
        while base.op is not None and base.op.name in ("ptr_add", "hint"):
            base = base.op.operands[0]
        if base.facts.get("idx64"):
            raise CompilationError(
                "an array argument spans more than 2^31 elements, and tensor descriptors "
                "address at most 2^31 elements of it. Split the array, or load it through a "
                "pointer tile instead.")


def widen_index_math(fn: ir.Func) -> int:
    """Rewrites `fn` in place; returns how many values got a 64-bit twin."""
    _check_descriptors(fn)
    need: dict[int, ir.Value] = {}
    seen: set[int] = set()

    def visit(v: ir.Value) -> None:
        if v.id in seen:
            return
        seen.add(v.id)
        x = _cast_source(v)
        if x is not None:
            visit(x)
            return
        if not _narrow(v):
            return
        need[v.id] = v
        op = v.op
        if op is not None and op.name in _CLONE:
            for o in (op.operands[1:] if op.name == "select" else op.operands):
                visit(o)

    def in_slice(v: ir.Value) -> bool:
        x = _cast_source(v)
        return v.id in need or (x is not None and x.id in need)

    cmps = []
    for op in ir.walk(fn.body):
        if op.name == "ptr_add":
            visit(op.operands[1])
        elif _is_cmp(op):
            cmps.append(op)
    marked: set[int] = set()
    grew = True
    while grew:
        grew = False
        for op in cmps:
            if id(op) not in marked and any(in_slice(v) for v in op.operands):
                marked.add(id(op))
                for v in op.operands:
                    visit(v)
                grew = True
    if not need:
        return 0

    wide: dict[int, ir.Value] = {}

    def cast_op(v: ir.Value, loc) -> ir.Op:
        op = ir.Op("cast", [v], [v.type.with_dtype(core.int64)], loc=loc)
        wide[v.id] = op.result
        return op

    def twin(v: ir.Value) -> ir.Value:
        if v.id in wide:
            return wide[v.id]
        x = _cast_source(v)
        if x is not None and x.id in wide:
            return wide[x.id]
        return v

    def block(b: ir.Block, loc) -> None:
        out = [cast_op(a, loc) for a in b.args if a.id in need]
        for op in b.ops:
            if op.name == "ptr_add":
                op.operands[1] = twin(op.operands[1])
            elif id(op) in marked:
                a, c = (twin(v) for v in op.operands)
                if a.type.dtype is not c.type.dtype:
                    raise CompilationError("internal: index comparison of mixed widths")
                op.operands = [a, c]
            for r in op.regions:
                block(r, op.loc)
            out.append(op)
            for r in op.results:
                if r.id not in need:
                    continue
                if op.name in _CLONE:
                    ops = [twin(v) if v.id in need or _cast_source(v) is not None else v
                           for v in op.operands]
                    clone = ir.Op(op.name, ops, [r.type.with_dtype(core.int64)],
                                  dict(op.attrs), loc=op.loc)
                    wide[r.id] = clone.result
                    out.append(clone)
                else:
                    out.append(cast_op(r, op.loc))
        b.ops = out

    # kernel arguments are not block arguments of the body: their casts go first
    arg_casts = [cast_op(a, None) for a in fn.args if a.id in need]
    block(fn.body, None)
    fn.body.ops = arg_casts + fn.body.ops
    return len(need)
