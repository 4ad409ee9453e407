"""The simplifier: constant folding, algebraic identities, loop-invariant hoisting, common
subexpressions and dead code (reference: compiler/passes/simplify.py:336-511).

`simplify(fn)` repeats four rewrites until none applies (at most a few rounds):

- **fold**: an elementwise op (`binary`, `unary`, `cast`, `select`) whose operands are all
  constant becomes a constant, evaluated by `compiler.fold` with the interpreter's
  semantics, so folding never changes a result. A constant is a `const` op or a
  `splat`/`broadcast`/`expand_dims`/`reshape` of one. A `select` on a constant condition,
  or between two identical values, becomes the value it selects; an `if` on a constant
  condition is replaced by the ops of the branch it takes.
- **identities** that hold for every operand value: for integers `x + 0`, `x - 0`, `x * 1`,
  `x // 1`, `x | 0`, `x ^ 0`, `x & -1`, `x << 0`, `x >> 0` give `x`, and `x * 0`, `x - x`
  give zero; for floats `x * 1.0`, `x / 1.0`, `x - 0.0` and `x + -0.0` give `x` (`x + 0.0`
  and `x * 0.0` do not hold for -0.0, NaN and infinities and stay).
- **hoist**: a side-effect-free scalar op inside a `for` body whose operands are all
  defined outside the loop moves in front of the loop (it cannot trap, so computing it for
  a loop that runs zero times is harmless); scalar work then runs once per program.
- **cse**: two side-effect-free ops with the same name, operands, attributes and result
  types compute the same value; later ones read the first (within the block that defines
  the first and the regions nested in it).
- **dce**: `ir.dce` removes what nothing reads anymore.

Folded float constants are compared and keyed by bit pattern (0.0 and -0.0 differ; NaN
equals NaN).
"""

from __future__ import annotations

import struct

import numpy as np

from enceladus_amd.compiler import fold, ir
from enceladus_amd.language import core

# side-effect-free ops that depend only on their operands and attributes
_PURE = frozenset(["const", "binary", "unary", "cast", "bitcast", "select", "splat",
                   "broadcast", "expand_dims", "reshape", "trans", "hint", "arange",
                   "program_id", "num_programs", "fma", "ptr_add", "join", "make_desc"])
_VIEWS = frozenset(["splat", "broadcast", "expand_dims", "reshape"])


def _bits_key(x):
    if isinstance(x, float):
        return ("f", struct.pack("<d", x))
    if isinstance(x, (tuple, list)):
        return tuple(_bits_key(v) for v in x)
    if isinstance(x, dict):
        return tuple(sorted((k, _bits_key(v)) for k, v in x.items()))
    if isinstance(x, core.dtype):
        return ("dt", x.name)
    return (type(x).__name__, x)


def constant_of(v: ir.Value):
    """(NumPy scalar, dtype) when every element of `v` is one known constant, else None."""
    seen = 0
    while v.op is not None and v.op.name in _VIEWS and seen < 64:
        v = v.op.operands[0]
        seen += 1
    op = v.op
    if op is None or op.name != "const" or not isinstance(v.type, ir.TType) or v.type.ptr:
        return None
    dt = v.type.dtype
    return fold.scalar(op.attrs["value"], dt), dt


class _Rewriter:
    def __init__(self, fn: ir.Func):
        self.fn = fn
        self.changed = False
        self.replace: dict[int, ir.Value] = {}

    def sub(self, v: ir.Value) -> ir.Value:
        while v.id in self.replace:
            v = self.replace[v.id]
        return v

    def redirect(self, old: ir.Value, new: ir.Value) -> None:
        if old is not new:
            self.replace[old.id] = new
            self.changed = True

    def const(self, like: ir.Value, x, loc) -> ir.Op:
        dt = like.type.dtype
        return ir.Op("const", [], [like.type], {"value": fold.attr(x, dt)}, loc=loc)

    # -- folding and identities ----------------------------------------------------
    def fold_op(self, op: ir.Op):
        """A replacement (a value, or a new const op) for `op`'s result, or None."""
        n = op.name
        if n == "binary":
            a, b = op.operands
            k = op.attrs["op"]
            ca, cb = constant_of(a), constant_of(b)
            dt = a.type.dtype
            if ca is not None and cb is not None:
                r = fold.binary(k, ca[0], cb[0], dt)
                return None if r is None else self.const(op.result, r, op.loc)
            return self.identity(op, k, a, b, ca, cb, dt)
        if n == "unary":
            c = constant_of(op.operands[0])
            if c is not None:
                r = fold.unary(op.attrs["op"], c[0], c[1])
                return None if r is None else self.const(op.result, r, op.loc)
            return None
        if n == "cast":
            c = constant_of(op.operands[0])
            if c is not None and not op.result.type.ptr:
                r = fold.cast(c[0], c[1], op.result.type.dtype)
                return None if r is None else self.const(op.result, r, op.loc)
            return None
        if n == "select":
            cond, x, y = op.operands
            if x is y:
                return x
            c = constant_of(cond)
            if c is not None:
                return x if bool(c[0]) else y
        return None

    def identity(self, op, k, a, b, ca, cb, dt):
        def is_val(c, v):
            if c is None:
                return False
            if dt.is_floating():
                return np.array([c[0]], np.float32).view(np.uint32)[0] == \
                    np.array([v], np.float32).view(np.uint32)[0]
            return int(c[0]) == v

        if dt.is_int() and not dt.is_bool():
            neg1 = -1 if dt.is_signed() else (1 << dt.primitive_bitwidth) - 1
            if (k in ("add", "or", "xor") and is_val(ca, 0)) or (k == "mul" and is_val(ca, 1)):
                return b
            if (k in ("add", "sub", "or", "xor", "shl", "shr") and is_val(cb, 0)) or \
                    (k in ("mul", "floordiv") and is_val(cb, 1)) or (k == "and" and
                                                                     is_val(cb, neg1)):
                return a
            if k == "and" and is_val(ca, neg1):
                return b
            if (k == "mul" and (is_val(ca, 0) or is_val(cb, 0))) or (k == "sub" and a is b):
                return self.const(op.result, fold.scalar(0, dt), op.loc)
            return None
        if dt.is_floating():
            if (k == "mul" and is_val(cb, 1.0)) or (k == "div" and is_val(cb, 1.0)) or \
                    (k == "sub" and is_val(cb, 0.0)) or (k == "add" and is_val(cb, -0.0)):
                return a
            if (k == "mul" and is_val(ca, 1.0)) or (k == "add" and is_val(ca, -0.0)):
                return b
        return None

    # -- the walk ------------------------------------------------------------------
    def run_block(self, b: ir.Block, avail: dict, visible: set, loop_outside) -> None:
        """One rewriting pass over `b`. `avail` maps CSE keys to the values visible here;
        `visible` holds the ids of the values visible here; `loop_outside`, when `b` is a
        loop body, the ids of the values defined before the loop (hoisting candidates'
        operands must all be among them)."""
        out: list[ir.Op] = []
        hoisted: list[ir.Op] = []
        visible.update(a.id for a in b.args)
        for op in b.ops:
            op.operands = [self.sub(o) for o in op.operands]
            if op.name == "if":
                c = constant_of(op.operands[0])
                if c is not None:
                    taken = op.regions[0 if bool(c[0]) else 1]
                    self.run_block(taken, avail, visible, loop_outside)
                    out.extend(taken.ops[:-1])
                    hoisted.extend(taken.hoisted)
                    for r, v in zip(op.results, taken.ops[-1].operands):
                        self.redirect(r, self.sub(v))
                    self.changed = True
                    continue
            if op.regions:
                for r in op.regions:
                    if op.name == "for":
                        self.run_block(r, dict(avail), set(visible), set(visible))
                        out.extend(r.hoisted)
                        visible.update(x.id for h in r.hoisted for x in h.results)
                    else:
                        self.run_block(r, dict(avail), set(visible), None)
                out.append(op)
                visible.update(x.id for x in op.results)
                continue
            new = self.fold_op(op) if len(op.results) == 1 else None
            if isinstance(new, ir.Value):
                self.redirect(op.result, new)
                continue
            if isinstance(new, ir.Op):
                self.redirect(op.result, new.result)
                op = new
            if op.name in _PURE and op.results:
                key = (op.name, tuple(o.id for o in op.operands), _bits_key(op.attrs),
                       tuple(str(r.type) for r in op.results))
                prev = avail.get(key)
                if prev is not None:
                    for r, p in zip(op.results, prev):
                        self.redirect(r, p)
                    continue
                avail[key] = op.results
                if loop_outside is not None and op.name != "make_desc" and \
                        all(isinstance(r.type, ir.TType) and r.type.is_scalar
                            for r in op.results) and \
                        all(o.id in loop_outside for o in op.operands):
                    hoisted.append(op)
                    loop_outside.update(x.id for x in op.results)
                    visible.update(x.id for x in op.results)
                    self.changed = True
                    continue
            out.append(op)
            visible.update(x.id for x in op.results)
        b.ops = out
        b.hoisted = hoisted

    def run(self) -> bool:
        self.changed = False
        self.run_block(self.fn.body, {}, {a.id for a in self.fn.args}, None)
        self._finish(self.fn.body)
        return self.changed

    def _finish(self, b: ir.Block) -> None:
        for op in b.ops:
            op.operands = [self.sub(o) for o in op.operands]
            for r in op.regions:
                self._finish(r)


def simplify(fn: ir.Func, rounds: int = 4) -> None:
    """Rewrites `fn` in place (see the module docstring)."""
    for _ in range(rounds):
        rw = _Rewriter(fn)
        changed = rw.run()
        removed = ir.dce(fn)
        if not changed and not removed:
            break
