"""64-bit index math for kernels whose array arguments span more than 2^31 elements.

A launch sets the `idx64` fact on an array argument whose last element lies more than
2^31 - 1 elements past its first (an MI355X holds 288 GB, so a 9 GB fp32 array is
enough). For such a specialization the address arithmetic must not wrap at 2^31: the
signed integer values that pointer offsets are computed from, and the comparisons that
test them (a mask such as `offs < n`), are evaluated at 64 bits, so an address and its
mask agree on the exact offset (the reference's rule: compiler/passes/widen_index.py:1-25).
Results differ from 32-bit math only where the 32-bit math overflows.

Design. One walk over the function records, for every value, its defining op and its
readers. A worklist then finds the *wide set*: the signed 8/16/32-bit values whose exact
value an address needs. It starts from `ptr_add` offsets; a member computed by an op that
yields the exact result from 64-bit operands (integer arithmetic, select, constants and
shape views) pulls its operands in; a comparison that reads a member is an address test,
so its other operands join too. A rebuild then gives each member a 64-bit definition:

- an op whose every reader takes the 64-bit form (offsets, address tests, sign extensions
  and other members rebuilt the same way) is retyped to int64 where it stands;
- an op that also has 32-bit readers (`offs` stored as data, a value a loop yields) keeps
  its 32-bit result and gets a 64-bit copy beside it;
- any other definition (a kernel argument, `tl.program_id`, `tl.arange`, a load, a loop
  index or carried value) is sign-extended where it is defined.

Sign extensions of members to int64 that the frontend inserted (type promotion of
`offs < n` with an int64 `n`) read the 64-bit member directly. A value a loop carries in
32 bits still wraps across iterations: carry a pointer or an int64 offset instead.
"""

from __future__ import annotations

from enceladus_amd.compiler import ir
from enceladus_amd.compiler.errors import CompilationError
from enceladus_amd.language import core

_SIGNED_NARROW = frozenset([core.int8, core.int16, core.int32])
_COMPARE = frozenset(ir.CMP_OPS)
# ops that compute the exact 64-bit value of their result from 64-bit operands
_EXACT_WIDE = frozenset(["binary", "unary", "select", "splat", "broadcast", "expand_dims",
                         "reshape", "trans", "hint", "const"])


def needs_idx64(fn: ir.Func) -> bool:
    return any(a.facts.get("idx64") for a in fn.args)


def _is_narrow(v: ir.Value) -> bool:
    t = v.type
    return isinstance(t, ir.TType) and not t.ptr and t.dtype in _SIGNED_NARROW


def _is_compare(op: ir.Op) -> bool:
    return op.name == "binary" and op.attrs.get("op") in _COMPARE


def _sext_source(op: ir.Op) -> ir.Value | None:
    """The narrow signed operand of a sign extension to int64, or None."""
    if op.name != "cast":
        return None
    r = op.results[0].type
    if isinstance(r, ir.TType) and not r.ptr and r.dtype is core.int64 and \
            _is_narrow(op.operands[0]):
        return op.operands[0]
    return None


def _index_operands(op: ir.Op) -> list[int]:
    """Operand positions of `op` that carry index values (not a select's condition)."""
    return list(range(1, len(op.operands))) if op.name == "select" else \
        list(range(len(op.operands)))


def _refuse_descriptors(fn: ir.Func) -> None:
    for op in ir.walk(fn.body):
        if op.name != "make_desc":
            continue
        base = op.operands[0]
        while base.op is not None and base.op.name in ("ptr_add", "hint"):
            base = base.op.operands[0]
        if base.facts.get("idx64"):
            raise CompilationError(
                "a tensor descriptor is built on an array argument spanning more than 2^31 "
                "elements; descriptors address at most 2^31 elements. Load that array "
                "through pointer tiles, or pass it in pieces of fewer elements.")


class _Graph:
    """Readers of every value: (op, operand position) pairs, over all regions."""

    def __init__(self, fn: ir.Func):
        self.readers: dict[int, list[tuple[ir.Op, int]]] = {}
        self.order: list[ir.Op] = []
        for op in ir.walk(fn.body):
            self.order.append(op)
            for i, o in enumerate(op.operands):
                self.readers.setdefault(o.id, []).append((op, i))

    def users(self, v: ir.Value):
        return self.readers.get(v.id, ())


def _wide_set(fn: ir.Func, g: _Graph) -> tuple[dict[int, ir.Value], set[int]]:
    """(members by id, ids of comparison ops that test addresses)."""
    members: dict[int, ir.Value] = {}
    tests: set[int] = set()
    work: list[ir.Value] = []

    def add(v: ir.Value) -> None:
        if v.op is not None:
            src = _sext_source(v.op)
            if src is not None:
                add(src)
                return
        if _is_narrow(v) and v.id not in members:
            members[v.id] = v
            work.append(v)

    for op in g.order:
        if op.name == "ptr_add":
            add(op.operands[1])
    while work:
        v = work.pop()
        op = v.op
        if op is not None and op.name in _EXACT_WIDE:
            for i in _index_operands(op):
                add(op.operands[i])
        # comparisons reading the member, directly or through a sign extension
        readers = list(g.users(v))
        for u, _ in list(readers):
            if _sext_source(u) is not None:
                readers += g.users(u.results[0])
        for u, _ in readers:
            if _is_compare(u) and id(u) not in tests:
                tests.add(id(u))
                for o in u.operands:
                    add(o)
    return members, tests


def widen_index_math(fn: ir.Func) -> int:
    """Rewrites `fn` in place; returns the size of the wide set."""
    _refuse_descriptors(fn)
    g = _Graph(fn)
    members, tests = _wide_set(fn, g)
    if not members:
        return 0

    # Which members can be retyped in place: every reader takes the 64-bit form. Readers
    # come after their operands in program order, so one reverse sweep decides.
    in_place: set[int] = set()
    for op in reversed(g.order):
        if op.name not in _EXACT_WIDE:
            continue
        for r in op.results:
            if r.id not in members:
                continue
            ok = True
            for u, pos in g.users(r):
                if (u.name == "ptr_add" and pos == 1) or id(u) in tests or \
                        _sext_source(u) is not None:
                    continue
                if u.name in _EXACT_WIDE and any(x.id in in_place for x in u.results) and \
                        pos in _index_operands(u):
                    continue
                ok = False
                break
            if ok:
                in_place.add(r.id)

    # sign extensions of members, found before any result is retyped
    sexts = {id(op): src for op in g.order
             if (src := _sext_source(op)) is not None and src.id in members}
    wide: dict[int, ir.Value] = {}     # member id -> its 64-bit value
    alias: dict[int, ir.Value] = {}    # removed sign extension result -> 64-bit value

    def w64(v: ir.Value) -> ir.Value:
        if v.id in alias:
            return alias[v.id]
        return wide.get(v.id, v)

    def sext(v: ir.Value, loc) -> ir.Op:
        c = ir.Op("cast", [v], [v.type.with_dtype(core.int64)], loc=loc)
        wide[v.id] = c.result
        return c

    def rebuild(b: ir.Block, loc) -> None:
        out = [sext(a, loc) for a in b.args if a.id in members]
        for op in b.ops:
            if id(op) in sexts:
                alias[op.results[0].id] = w64(sexts[id(op)])
                continue
            ops = [alias.get(o.id, o) for o in op.operands]
            if op.name == "ptr_add":
                ops[1] = w64(ops[1])
            elif id(op) in tests:
                ops = [w64(o) for o in ops]
                if len({o.type.dtype.name for o in ops}) != 1:
                    raise CompilationError("internal: an address comparison mixes widths")
            for r in op.regions:
                rebuild(r, op.loc)
            res = op.results[0] if op.results else None
            if res is not None and res.id in in_place:
                for i in _index_operands(op):
                    ops[i] = w64(ops[i])
                res.type = res.type.with_dtype(core.int64)
                wide[res.id] = res
                op.operands = ops
                out.append(op)
                continue
            op.operands = ops
            out.append(op)
            if res is not None and res.id in members:
                if op.name in _EXACT_WIDE:
                    wops = list(ops)
                    for i in _index_operands(op):
                        wops[i] = w64(wops[i])
                    twin = ir.Op(op.name, wops, [res.type.with_dtype(core.int64)],
                                 dict(op.attrs), loc=op.loc)
                    wide[res.id] = twin.result
                    out.append(twin)
                else:
                    out.append(sext(res, op.loc))
        b.ops = out

    # kernel arguments are not block arguments of the body: theirs come first
    head = [sext(a, None) for a in fn.args if a.id in members]
    rebuild(fn.body, None)
    fn.body.ops = head + fn.body.ops
    return len(members)
