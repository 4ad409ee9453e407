"""Python AST → tile IR.

`build_ir` parses a kernel's source and walks it with `CodeGenerator`. Python values
(ints, floats, bools, tuples, dtypes, constexpr arguments) fold at compile time; runtime
values are `ir.Value`s. `for ... in range(...)` becomes a structured `for` op whose
loop-carried values are the names the body reassigns; `if` on a runtime condition becomes
a structured `if` op; `if` on a compile-time condition picks a branch. Calls to other
`@jit` functions inline. Reference: src/enceladus/compiler/frontend.py:202-1339
(`CodeGenerator`, `run_kernel`, loop-carried inference :571-697, `build_ir` :1244).
"""

from __future__ import annotations

import ast
import builtins
import sys
import types
import inspect
import textwrap
from typing import Any

from enceladus_amd.compiler import ir, semantic
from enceladus_amd.compiler.errors import CompilationError
from enceladus_amd.language import core

_BINOPS = {ast.Add: "add", ast.Sub: "sub", ast.Mult: "mul", ast.Div: "div",
           ast.FloorDiv: "floordiv", ast.Mod: "mod", ast.BitAnd: "and", ast.BitOr: "or",
           ast.BitXor: "xor", ast.LShift: "shl", ast.RShift: "shr"}
_CMPOPS = {ast.Eq: "eq", ast.NotEq: "ne", ast.Lt: "lt", ast.LtE: "le", ast.Gt: "gt",
           ast.GtE: "ge"}
_PY_BIN = {"add": lambda a, b: a + b, "sub": lambda a, b: a - b, "mul": lambda a, b: a * b,
           "div": lambda a, b: a / b, "floordiv": lambda a, b: a // b,
           "mod": lambda a, b: a % b, "and": lambda a, b: a & b, "or": lambda a, b: a | b,
           "xor": lambda a, b: a ^ b, "shl": lambda a, b: a << b, "shr": lambda a, b: a >> b,
           "eq": lambda a, b: a == b, "ne": lambda a, b: a != b, "lt": lambda a, b: a < b,
           "le": lambda a, b: a <= b, "gt": lambda a, b: a > b, "ge": lambda a, b: a >= b}


class _Poison:
    """A name whose value can't be used (reading it raises the stored error)."""

    def __init__(self, msg: str):
        self.msg = msg


class _Return(Exception):
    def __init__(self, value, node=None):
        self.value = value
        self.node = node


class BoundMethod:
    """A method of a runtime value (`x.to`, `desc.load`), resolved at call time."""

    def __init__(self, impl, obj):
        self.impl = impl
        self.obj = obj


def is_builtin(obj: Any) -> bool:
    return getattr(obj, "_ek_frontend", None) is not None


def _is_jit(obj: Any) -> bool:
    return getattr(obj, "_ek_jit", False)


def is_value(x: Any) -> bool:
    return isinstance(x, ir.Value)


class Context:
    """What builtins see: the builder plus launch options."""

    def __init__(self, b: ir.Builder, num_warps: int, options: dict):
        self.b = b
        self.num_warps = num_warps
        self.options = options
        # what the kernel read at compile time outside its arguments: (container, name,
        # value, is_mapping); a launch recompiles when one of them changed (reference:
        # runtime/jit.py:289, 1037-1234)
        self.deps: list = []
        self._dep_seen: set = set()

    def record(self, container, name: str, value, mapping: bool) -> None:
        key = (id(container), name)
        if key in self._dep_seen or isinstance(value, types.ModuleType):
            return
        self._dep_seen.add(key)
        self.deps.append((container, name, value, mapping))

    def is_known_one(self, v) -> bool:
        v = core.unwrap(v)
        if isinstance(v, int) and not isinstance(v, bool):
            return v == 1
        if isinstance(v, ir.Value):
            if v.op is not None and v.op.name == "const":
                return v.op.attrs["value"] == 1
            return bool(v.facts.get("equal_to_1"))
        return False


def _unparse(node) -> str:
    try:
        return ast.unparse(node)
    except Exception:  # pragma: no cover
        return "<expr>"


class CodeGenerator(ast.NodeVisitor):
    def __init__(self, ctx: Context, fn, scope: dict[str, Any], filename: str,
                 line_offset: int, src_lines: list[str]):
        self.ctx = ctx
        self.fn = fn
        self.globals = dict(fn.__globals__)
        self._cells: dict = {}
        if fn.__closure__:
            for name, cell in zip(fn.__code__.co_freevars, fn.__closure__):
                try:
                    self.globals[name] = cell.cell_contents
                    self._cells[name] = cell
                except ValueError:
                    pass
        self.scope = scope
        self.filename = filename
        self.line_offset = line_offset
        self.src_lines = src_lines

    @property
    def b(self) -> ir.Builder:
        return self.ctx.b

    # -- errors --------------------------------------------------------------
    def error(self, node, msg: str) -> CompilationError:
        line = getattr(node, "lineno", 0) + self.line_offset
        src = None
        if 0 < getattr(node, "lineno", 0) <= len(self.src_lines):
            src = self.src_lines[node.lineno - 1]
        return CompilationError(msg, (self.filename, line), src,
                                getattr(node, "col_offset", None))

    def visit(self, node):
        if isinstance(node, ast.stmt):
            # ops created for this statement carry its source location
            self.ctx.b.loc = (self.filename, getattr(node, "lineno", 0) + self.line_offset)
        try:
            return super().visit(node)
        except CompilationError as e:
            if e.loc is None and hasattr(node, "lineno"):
                raise self.error(node, e.msg) from None
            raise
        except (_Return, _BreakScan):
            raise
        except Exception as e:  # noqa: BLE001
            if hasattr(node, "lineno") and not isinstance(e, CompilationError):
                raise self.error(node, f"{type(e).__name__}: {e}") from e
            raise

    def generic_visit(self, node):
        hint = ""
        if isinstance(node, (ast.Dict, ast.Set, ast.DictComp, ast.SetComp)):
            hint = ". Use a compile-time tuple, or pass values as tl.constexpr arguments."
        elif isinstance(node, ast.Lambda):
            hint = ". Define an @enceladus.jit function instead."
        raise self.error(node, f"unsupported syntax: {type(node).__name__} "
                               f"(`{_unparse(node)}`){hint}")

    # -- statements ----------------------------------------------------------
    def visit_stmts(self, stmts):
        for s in stmts:
            self.visit(s)

    def visit_Pass(self, node):
        return None

    def visit_Expr(self, node):
        if isinstance(node.value, ast.Constant) and isinstance(node.value.value, str):
            return None  # docstring
        self.visit(node.value)

    def assign_target(self, target, value, node):
        if isinstance(target, ast.Name):
            v = core.unwrap(value)
            if isinstance(v, ir.Value) and not v.name_hint and v.op is not None:
                v.name_hint = target.id          # for kernel.explain's report
            self.scope[target.id] = value
        elif isinstance(target, (ast.Tuple, ast.List)):
            vals = core.unwrap(value)
            if not isinstance(vals, (tuple, list)):
                raise self.error(node, "can only unpack a tuple")
            if len(vals) != len(target.elts):
                raise self.error(node, f"can't unpack {len(vals)} values into "
                                       f"{len(target.elts)} names")
            for t, v in zip(target.elts, vals):
                self.assign_target(t, v, node)
        else:
            raise self.error(node, f"unsupported assignment target `{_unparse(target)}`")

    def visit_Assign(self, node):
        value = self.visit(node.value)
        for t in node.targets:
            self.assign_target(t, value, node)

    def visit_AnnAssign(self, node):
        if node.value is None:
            return
        value = self.visit(node.value)
        ann = None
        try:
            ann = eval(compile(ast.Expression(node.annotation), "<ann>", "eval"), self.globals)
        except Exception:  # noqa: BLE001
            pass
        if ann is not None and core.is_constexpr_annotation(ann) and is_value(value):
            raise self.error(node, "a constexpr variable needs a compile-time value")
        self.assign_target(node.target, value, node)

    def visit_AugAssign(self, node):
        if not isinstance(node.target, ast.Name):
            raise self.error(node, "augmented assignment needs a plain name")
        cur = self.lookup(node.target.id, node)
        rhs = self.visit(node.value)
        self.scope[node.target.id] = self.binop(_BINOPS[type(node.op)], cur, rhs, node)

    def visit_Return(self, node):
        raise _Return(None if node.value is None else self.visit(node.value), node)

    def visit_Assert(self, node):
        cond = self.visit(node.test)
        if is_value(cond):
            raise self.error(node, "`assert` needs a compile-time condition; use "
                                   "tl.device_assert for runtime checks")
        if not core.unwrap(cond):
            msg = self.visit(node.msg) if node.msg is not None else ""
            raise self.error(node, f"assertion failed: {msg}")

    def visit_test(self, node):
        """A condition whose truth value is all that matters (`if`, `x if c else y`,
        `not`): `and`/`or` combine truth values there, so their operands may have
        different types (reference: compiler/frontend.py:927-931). A compile-time false
        (true) operand of `and` (`or`) decides the result without the later operands."""
        if isinstance(node, ast.BoolOp):
            kind = "and" if isinstance(node.op, ast.And) else "or"
            acc = None
            for v in node.values:
                t = core.unwrap(self.visit_test(v))
                if not is_value(t):
                    if kind == "and" and not t:
                        return False
                    if kind == "or" and t:
                        return True
                    continue
                acc = t if acc is None else semantic.binary(self.b, kind, acc, t)
            return acc if acc is not None else kind == "and"
        if isinstance(node, ast.UnaryOp) and isinstance(node.op, ast.Not):
            t = core.unwrap(self.visit_test(node.operand))
            return (not t) if not is_value(t) else semantic.binary(self.b, "eq", t, False)
        x = core.unwrap(self.visit(node))
        if not is_value(x) or x.type.shape or x.type.ptr or x.type.dtype.is_bool():
            return x
        return semantic.binary(self.b, "ne", x, 0)

    def visit_If(self, node):
        cond = self.visit_test(node.test)
        cond = core.unwrap(cond)
        if not is_value(cond):
            self.visit_stmts(node.body if cond else node.orelse)
            return
        if cond.type.shape != ():
            raise self.error(node, "`if` needs a scalar condition; for a tile condition use "
                                   "tl.where(cond, a, b)")
        self.runtime_if(node, cond)

    def _names_assigned(self, stmts) -> list[str]:
        out: list[str] = []

        class V(ast.NodeVisitor):
            def visit_Name(self, n):
                if isinstance(n.ctx, ast.Store) and n.id not in out:
                    out.append(n.id)

            def visit_FunctionDef(self, n):  # nested defs are not supported anyway
                pass

        for s in stmts:
            V().visit(s)
        return out

    def _run_region(self, stmts, block: ir.Block, scope: dict) -> dict:
        saved_b, saved_scope = self.ctx.b, self.scope
        self.ctx.b = ir.Builder(block)
        self.ctx.b.loc = saved_b.loc
        self.scope = scope
        try:
            self.visit_stmts(stmts)
            return self.scope
        finally:
            self.ctx.b, self.scope = saved_b, saved_scope

    def runtime_if(self, node, cond: ir.Value):
        if not cond.type.dtype.is_bool():
            cond = semantic.binary(self.b, "ne", cond, 0)
        names = [n for n in self._names_assigned(node.body + node.orelse)]
        then_b, else_b = ir.Block(), ir.Block()
        then_scope = self._run_region(node.body, then_b, dict(self.scope))
        else_scope = self._run_region(node.orelse, else_b, dict(self.scope))
        results = []
        for n in names:
            tv, ev = then_scope.get(n), else_scope.get(n)
            if tv is None or ev is None:
                continue
            if tv is ev:
                continue
            if not (is_value(tv) or is_value(ev)):
                if core.unwrap(tv) == core.unwrap(ev):
                    continue
                raise self.error(node, f"`{n}` gets different compile-time values in the "
                                       "branches of a runtime `if`")
            results.append(n)
        then_vals, else_vals, types = [], [], []
        for n in results:
            tv, ev = then_scope[n], else_scope[n]
            tv, ev = self._unify_pair(tv, ev, then_b, else_b, node, n)
            then_vals.append(tv)
            else_vals.append(ev)
            types.append(tv.type)
        ir.Builder(then_b).create("yield", then_vals)
        ir.Builder(else_b).create("yield", else_vals)
        op = self.b.create("if", [cond], types, regions=[then_b, else_b])
        for n, r in zip(results, op.results):
            self.scope[n] = r

    def _unify_pair(self, tv, ev, then_b, else_b, node, name):
        tb, eb = ir.Builder(then_b), ir.Builder(else_b)
        if not is_value(tv):
            tv = semantic.to_value(tb, tv, ev.type.dtype if is_value(ev) else None)
        if not is_value(ev):
            ev = semantic.to_value(eb, ev, tv.type.dtype)
        if tv.type != ev.type:
            if tv.type.ptr or ev.type.ptr or isinstance(tv.type, ir.DescType):
                raise self.error(node, f"`{name}` has types {tv.type} and {ev.type} in the "
                                       "two branches")
            dt = semantic.computation_dtype("select", tv.type.dtype, ev.type.dtype)
            shape = semantic.broadcast_shapes(tv.type.shape, ev.type.shape)
            tv = semantic.broadcast_to(tb, semantic.cast(tb, tv, dt), shape)
            ev = semantic.broadcast_to(eb, semantic.cast(eb, ev, dt), shape)
        return tv, ev

    def visit_For(self, node):
        if node.orelse:
            raise self.error(node, "`for ... else` isn't supported")
        it = node.iter
        if not isinstance(it, ast.Call):
            raise self.error(node, "`for` loops must iterate over range(), tl.range() or "
                                   "tl.static_range()")
        callee = self.visit(it.func)
        args = [self.visit(a) for a in it.args]
        kwargs = {k.arg: self.visit(k.value) for k in it.keywords}
        static = getattr(callee, "_ek_static_range", False)
        is_range = callee is builtins.range or getattr(callee, "_ek_range", False)
        if not (static or is_range):
            # A compile-time iterable (a tuple of constexprs, zip, enumerate, ...).
            vals = callee(*[core.unwrap(a) for a in args], **kwargs)
            for v in vals:
                self.assign_target(node.target, v, node)
                self.visit_stmts(node.body)
            return
        if len(args) == 1:
            lo, hi, step = 0, args[0], 1
        elif len(args) == 2:
            lo, hi, step = args[0], args[1], 1
        elif len(args) == 3:
            lo, hi, step = args
        else:
            raise self.error(node, "range() takes 1 to 3 arguments")
        lo, hi, step = core.unwrap(lo), core.unwrap(hi), core.unwrap(step)
        if static or not any(is_value(v) for v in (lo, hi, step)):
            if any(is_value(v) for v in (lo, hi, step)):
                raise self.error(node, "tl.static_range needs compile-time bounds")
            n_iter = len(range(int(lo), int(hi), int(step)))
            if static or n_iter <= 0:
                for i in range(int(lo), int(hi), int(step)):
                    self.assign_target(node.target, i, node)
                    self.visit_stmts(node.body)
                return
        if not isinstance(node.target, ast.Name):
            raise self.error(node, "the loop variable must be a single name")
        self.runtime_for(node, lo, hi, step, kwargs)

    def runtime_for(self, node, lo, hi, step, kwargs):
        b = self.b
        vals = [semantic.to_value(b, v) for v in (lo, hi, step)]
        for v in vals:
            if v.type.shape != () or not v.type.dtype.is_int():
                raise self.error(node, "range() bounds must be integer scalars")
        dt = core.int32
        for v in vals:
            d = v.type.dtype
            if d in (core.int64, core.uint32, core.uint64):
                dt = core.int64
        lo_v, hi_v, step_v = (semantic.cast(b, v, dt) for v in vals)
        if isinstance(core.unwrap(step), int) and core.unwrap(step) == 0:
            raise self.error(node, "range() arg 3 must not be zero")
        iv_name = node.target.id
        # Pass 1: find which names the body rebinds, and their types.
        assigned = [n for n in self._names_assigned(node.body) if n != iv_name]
        carried = [n for n in assigned if n in self.scope]
        probe_blk = ir.Block([ir.TType((), dt)])
        probe_scope = dict(self.scope)
        probe_scope[iv_name] = probe_blk.args[0]
        probe_scope = self._run_region(node.body, probe_blk, probe_scope)
        init_vals, names = [], []
        for n in carried:
            before, after = self.scope[n], probe_scope.get(n)
            if after is before:
                continue
            if not is_value(before) and not is_value(after):
                if core.unwrap(before) == core.unwrap(after):
                    continue
            if is_value(before) and is_value(after) and after.type != before.type:
                raise self.error(
                    node, f"loop-carried variable `{n}` has type {before.type} before the loop "
                          f"but {after.type} at the end of the body. Convert it with `.to(...)` "
                          "so that the type stays the same, or initialize it with the final type.")
            names.append(n)
            bv = before
            if not is_value(bv):
                want = after.type.dtype if is_value(after) else None
                bv = semantic.to_value(b, bv, want)
            if is_value(after) and after.type != bv.type and not after.type.ptr:
                if after.type.shape != bv.type.shape:
                    bv = semantic.broadcast_to(b, bv, after.type.shape)
                if after.type.dtype != bv.type.dtype:
                    dtp = semantic.computation_dtype("select", bv.type.dtype, after.type.dtype)
                    bv = semantic.cast(b, bv, dtp)
            init_vals.append(bv)
        # Pass 2: the real body with block arguments for the carried names.
        body = ir.Block([ir.TType((), dt)] + [v.type for v in init_vals])
        scope = dict(self.scope)
        scope[iv_name] = body.args[0]
        for n, a in zip(names, body.args[1:]):
            scope[n] = a
        scope = self._run_region(node.body, body, scope)
        yields = []
        bb = ir.Builder(body)
        for n, a in zip(names, body.args[1:]):
            v = scope[n]
            if not is_value(v):
                v = semantic.to_value(bb, v, a.type.dtype)
            if v.type != a.type:
                if v.type.ptr or isinstance(v.type, ir.DescType):
                    raise self.error(node, f"loop-carried `{n}` changes type from {a.type} "
                                           f"to {v.type}")
                if v.type.shape != a.type.shape:
                    v = semantic.broadcast_to(bb, v, a.type.shape)
                if v.type.dtype != a.type.dtype:
                    if semantic.computation_dtype("select", a.type.dtype,
                                                  v.type.dtype) is not a.type.dtype:
                        raise self.error(node, f"loop-carried `{n}` changes type from "
                                               f"{a.type} to {v.type}; convert it before "
                                               "the loop")
                    v = semantic.cast(bb, v, a.type.dtype)
            yields.append(v)
        bb.create("yield", yields)
        attrs = {}
        if kwargs.get("num_stages") is not None:
            attrs["num_stages"] = int(core.unwrap(kwargs["num_stages"]))
        op = b.create("for", [lo_v, hi_v, step_v, *init_vals], [v.type for v in init_vals],
                      attrs, regions=[body])
        for n, r in zip(names, op.results):
            self.scope[n] = r
        # As in Python, the loop variable keeps its last value after the loop, or its value
        # from before the loop when the loop doesn't run.
        # last = lo + ((|hi - lo| - 1) // |step|) * step, for steps of either sign
        cst = core.unwrap(step)
        sub = lambda x, y: semantic.binary(b, "sub", x, y)  # noqa: E731
        up = (sub(sub(hi_v, lo_v), 1), step_v)
        down = (sub(sub(lo_v, hi_v), 1), sub(semantic.to_value(b, 0, dt), step_v))
        if isinstance(cst, int):
            num, den = up if cst > 0 else down
            ran = semantic.binary(b, "lt", lo_v, hi_v) if cst > 0 else \
                semantic.binary(b, "gt", lo_v, hi_v)
        else:
            pos = semantic.binary(b, "gt", step_v, 0)
            num = semantic.select(b, pos, up[0], down[0])
            den = semantic.select(b, pos, up[1], down[1])
            ran = semantic.binary(b, "or", semantic.binary(
                b, "and", pos, semantic.binary(b, "lt", lo_v, hi_v)), semantic.binary(
                b, "and", semantic.binary(b, "lt", step_v, 0), semantic.binary(b, "gt", lo_v, hi_v)))
        last = semantic.binary(b, "add", lo_v, semantic.binary(
            b, "mul", semantic.binary(b, "floordiv", num, den), step_v))
        prior = core.unwrap(self.scope.get(iv_name))
        if prior is not None:
            pdt = prior.type.dtype if is_value(prior) and not isinstance(prior.type, ir.DescType) \
                else None
            same = (pdt is dt and prior.type.shape == ()) if is_value(prior) else (
                isinstance(prior, int) and not isinstance(prior, bool) and
                semantic.adopt_literal(prior, dt) is dt)
            if same:
                last = semantic.select(b, ran, last, prior)
            else:
                last = _Poison(f"`{iv_name}` is {prior!r} before the loop and an integer loop "
                               "counter inside it, so its type after the loop depends on "
                               "whether the loop ran. Give the loop variable a different name.")
        self.scope[iv_name] = last

    def visit_While(self, node):
        raise self.error(node, "`while` loops aren't supported; use `for ... in range(...)`")

    def visit_Break(self, node):
        raise self.error(node, "`break` isn't supported in kernels")

    def visit_Continue(self, node):
        raise self.error(node, "`continue` isn't supported in kernels")

    # -- expressions ---------------------------------------------------------
    def lookup(self, name: str, node):
        if name in self.scope:
            v = self.scope[name]
            if isinstance(v, _Poison):
                raise self.error(node, v.msg)
            return v
        if name in self.globals:
            v = self.globals[name]
            if name in self._cells:
                self.ctx.record(self._cells[name], "cell_contents", v, False)
            else:
                self.ctx.record(self.fn.__globals__, name, v, True)
            return v
        if hasattr(builtins, name):
            return getattr(builtins, name)
        raise self.error(node, f"name `{name}` is not defined")

    def visit_Name(self, node):
        return self.lookup(node.id, node)

    def visit_Constant(self, node):
        return node.value

    def visit_Tuple(self, node):
        return tuple(self.visit(e) for e in node.elts)

    def visit_List(self, node):
        return [self.visit(e) for e in node.elts]

    def visit_JoinedStr(self, node):
        parts = []
        for v in node.values:
            if isinstance(v, ast.Constant):
                parts.append(str(v.value))
            else:
                x = self.visit(v.value)
                parts.append(format(core.unwrap(x), v.format_spec.values[0].value
                                    if v.format_spec else ""))
        return "".join(parts)

    def visit_Attribute(self, node):
        obj = core.unwrap(self.visit(node.value))
        attr = node.attr
        if is_value(obj):
            return value_attr(self.ctx, obj, attr)
        try:
            v = getattr(obj, attr)
        except AttributeError as e:
            raise self.error(node, str(e)) from None
        if isinstance(obj, (types.ModuleType, type)) and not _stable_module(obj):
            self.ctx.record(obj, attr, v, False)
        return v

    def visit_Subscript(self, node):
        obj = core.unwrap(self.visit(node.value))
        idx = self.visit(node.slice)
        if is_value(obj):
            return index_tile(self.b, obj, idx)
        return obj[core.unwrap(idx)]

    def visit_Slice(self, node):
        lo = None if node.lower is None else core.unwrap(self.visit(node.lower))
        hi = None if node.upper is None else core.unwrap(self.visit(node.upper))
        st = None if node.step is None else core.unwrap(self.visit(node.step))
        return slice(lo, hi, st)

    def visit_Index(self, node):  # pragma: no cover - Python < 3.9
        return self.visit(node.value)

    def binop(self, op: str, a, b_, node):
        a, b_ = core.unwrap(a), core.unwrap(b_)
        if not is_value(a) and not is_value(b_):
            return _PY_BIN[op](a, b_)
        return semantic.binary(self.b, op, a, b_)

    def visit_BinOp(self, node):
        a = self.visit(node.left)
        b_ = self.visit(node.right)
        if type(node.op) not in _BINOPS:
            if isinstance(node.op, ast.Pow):
                ca, cb = core.unwrap(a), core.unwrap(b_)
                if not is_value(ca) and not is_value(cb):
                    return ca ** cb
                raise self.error(node, "`**` isn't supported on runtime values. Multiply "
                                       "explicitly (`x * x`), or use tl.exp2/tl.log2.")
            raise self.error(node, f"unsupported operator {type(node.op).__name__}")
        return self.binop(_BINOPS[type(node.op)], a, b_, node)

    def visit_UnaryOp(self, node):
        if isinstance(node.op, ast.Not):
            x = core.unwrap(self.visit_test(node.operand))
            return (not x) if not is_value(x) else semantic.binary(self.b, "eq", x, 0)
        x = core.unwrap(self.visit(node.operand))
        if not is_value(x):
            if isinstance(node.op, ast.USub):
                return -x
            if isinstance(node.op, ast.UAdd):
                return +x
            if isinstance(node.op, ast.Not):
                return not x
            if isinstance(node.op, ast.Invert):
                return ~x
        if isinstance(node.op, ast.USub):
            return semantic.unary(self.b, "neg", x)
        if isinstance(node.op, ast.UAdd):
            return x
        if isinstance(node.op, ast.Not):
            return semantic.binary(self.b, "eq", x, 0)
        if isinstance(node.op, ast.Invert):
            return semantic.unary(self.b, "not", x)
        raise self.error(node, "unsupported unary operator")

    def visit_Compare(self, node):
        left = self.visit(node.left)
        result = None
        for op, comp in zip(node.ops, node.comparators):
            right = self.visit(comp)
            if isinstance(op, (ast.Is, ast.IsNot)):
                l, r = core.unwrap(left), core.unwrap(right)
                c = (l is r) if isinstance(op, ast.Is) else (l is not r)
            elif isinstance(op, (ast.In, ast.NotIn)):
                c = core.unwrap(left) in core.unwrap(right)
                if isinstance(op, ast.NotIn):
                    c = not c
            else:
                c = self.binop(_CMPOPS[type(op)], left, right, node)
            if result is not None and is_value(core.unwrap(c)) and core.unwrap(c).type.shape:
                raise self.error(node, "chained comparisons on tiles have no single truth "
                                       "value in Python. Write `(a < b) & (b < c)`.")
            result = c if result is None else self.logical("and", result, c)
            left = right
        return result

    def logical(self, kind, a, b_):
        a, b_ = core.unwrap(a), core.unwrap(b_)
        if not is_value(a) and not is_value(b_):
            return (a and b_) if kind == "and" else (a or b_)
        op = "and" if kind == "and" else "or"
        if any(is_value(v) and v.type.shape for v in (a, b_)):
            sym = "&" if kind == "and" else "|"
            raise CompilationError(f"`{kind}` on tiles has no single truth value in Python; "
                                   f"use `{sym}` for the elementwise {kind} of masks")
        if all(not is_value(v) or v.type.dtype.is_bool() for v in (a, b_)):
            return semantic.binary(self.b, op, a, b_)
        # Python's value semantics on runtime scalars: `a or b` is a when a is truthy, else
        # b; `a and b` is a when a is falsy, else b. Both sides must share a type.
        ta = a.type.dtype if is_value(a) else None
        tb = b_.type.dtype if is_value(b_) else None
        dt = ta or tb
        for v, t in ((a, ta), (b_, tb)):
            if t is None and semantic.adopt_literal(v, dt) is not dt:
                t = semantic.literal_dtype(v)
            if (t or dt) is not dt:
                raise CompilationError(
                    f"`{kind}` of {ta or semantic.literal_dtype(a)} and "
                    f"{tb or semantic.literal_dtype(b_)}: both need the same type (Python would "
                    "return either one); convert one side with `.to(...)`")
        av, bv = semantic.to_value(self.b, a, dt), semantic.to_value(self.b, b_, dt)
        truthy = semantic.binary(self.b, "ne", av, 0)
        return semantic.select(self.b, truthy, av, bv) if kind == "or" else \
            semantic.select(self.b, truthy, bv, av)

    def visit_BoolOp(self, node):
        kind = "and" if isinstance(node.op, ast.And) else "or"
        val = self.visit(node.values[0])
        for v in node.values[1:]:
            cur = core.unwrap(val)
            if not is_value(cur):
                if kind == "and" and not cur:
                    return cur
                if kind == "or" and cur:
                    return cur
                val = self.visit(v)
                continue
            val = self.logical(kind, val, self.visit(v))
        return val

    def visit_IfExp(self, node):
        cond = core.unwrap(self.visit_test(node.test))
        if not is_value(cond):
            return self.visit(node.body) if cond else self.visit(node.orelse)
        return semantic.select(self.b, cond, self.visit(node.body), self.visit(node.orelse))

    def visit_Call(self, node):
        fn = self.visit(node.func)
        args = []
        for a in node.args:
            if isinstance(a, ast.Starred):
                args.extend(core.unwrap(self.visit(a.value)))
            else:
                args.append(self.visit(a))
        kwargs = {}
        for k in node.keywords:
            if k.arg is None:
                kwargs.update(core.unwrap(self.visit(k.value)))
            else:
                kwargs[k.arg] = self.visit(k.value)
        return self.call(fn, args, kwargs, node)

    def call(self, fn, args, kwargs, node):
        fn = core.unwrap(fn)
        if isinstance(fn, BoundMethod):
            return fn.impl(self.ctx, fn.obj, *args, **kwargs)
        if is_builtin(fn):
            return fn._ek_frontend(self.ctx, *args, **kwargs)
        if _is_jit(fn):
            return self.inline(fn, args, kwargs, node)
        if any(is_value(core.unwrap(a)) for a in [*args, *kwargs.values()]):
            if fn in (builtins.min, builtins.max) and len(args) == 2:
                return semantic.binary(self.b, fn.__name__, args[0], args[1])
            if fn is builtins.float:
                return semantic.cast(self.b, core.unwrap(args[0]), core.float32)
            if fn is builtins.int:
                return semantic.cast(self.b, core.unwrap(args[0]), core.int32)
            if fn is builtins.abs:
                return semantic.unary(self.b, "abs", core.unwrap(args[0]))
            if fn is builtins.print:
                raise self.error(node, "`print` runs when the kernel compiles and can't show "
                                       "runtime values. Use tl.device_print (or "
                                       "tl.static_print for compile-time values).")
            raise self.error(node, f"`{getattr(fn, '__name__', fn)}` can't take runtime values")
        if fn is builtins.print:
            return None
        code = getattr(fn, "__code__", None)
        glb = getattr(fn, "__globals__", None)
        if code is not None and glb is not None and not _stable_module(
                sys.modules.get(getattr(fn, "__module__", ""), None)):
            # a plain Python helper runs now: the globals it names are dependencies too
            for nm in code.co_names:
                if nm in glb:
                    self.ctx.record(glb, nm, glb[nm], True)
        return fn(*[core.unwrap(a) for a in args],
                   **{k: core.unwrap(v) for k, v in kwargs.items()})

    def inline(self, jfn, args, kwargs, node):
        try:
            return inline_jit(self.ctx, jfn, args, kwargs)
        except _BadCall as e:
            raise self.error(node, str(e)) from None


class _BadCall(Exception):
    pass


def inline_jit(ctx: Context, jfn, args, kwargs=None):
    """Emits the body of the @jit function `jfn` called with `args` at the builder's
    current position and returns its return value (a tuple for several values)."""
    fn = jfn.fn
    stack = ctx.__dict__.setdefault("inlining", [])
    if fn in stack:
        raise _BadCall(f"recursion isn't supported: `{fn.__name__}` calls itself (through "
                       f"{' -> '.join(f.__name__ for f in stack)})")
    stack.append(fn)
    try:
        return _inline(ctx, fn, args, kwargs)
    finally:
        stack.pop()


def _inline(ctx: Context, fn, args, kwargs):
    sig = inspect.signature(fn)
    try:
        bound = sig.bind(*args, **(kwargs or {}))
    except TypeError as e:
        raise _BadCall(f"bad call to `{fn.__name__}`: {e}") from None
    bound.apply_defaults()
    scope = dict(bound.arguments)
    tree, fname, off, lines = parse_function(fn)
    gen = CodeGenerator(ctx, fn, scope, fname, off, lines)
    try:
        gen.visit_stmts(tree.body)
    except _Return as r:
        return r.value
    return None


def is_jit(obj: Any) -> bool:
    return _is_jit(obj)


class _BreakScan(Exception):
    pass


# ---------------------------------------------------------------------------
# Value attributes and indexing
# ---------------------------------------------------------------------------

TILE_METHODS: dict[str, Any] = {}
DESC_METHODS: dict[str, Any] = {}


def value_attr(ctx: Context, v: ir.Value, attr: str):
    t = v.type
    if isinstance(t, ir.DescType):
        if attr == "dtype":
            return t.dtype
        if attr == "block_shape":
            return list(t.block_shape)
        if attr in DESC_METHODS:
            return BoundMethod(DESC_METHODS[attr], v)
        raise CompilationError(f"tensor descriptors have no attribute `{attr}`")
    if attr == "dtype":
        return t.dtype
    if attr == "shape":
        return tuple(t.shape)
    if attr == "T":
        return TILE_METHODS["trans"](ctx, v)
    if attr in TILE_METHODS:
        return BoundMethod(TILE_METHODS[attr], v)
    raise CompilationError(f"tiles have no attribute `{attr}`")


def index_tile(b: ir.Builder, v: ir.Value, idx):
    idx = core.unwrap(idx)
    if not isinstance(idx, tuple):
        idx = (idx,)
    out = v
    dim = 0
    for i in idx:
        i = core.unwrap(i)
        if i is None:
            out = semantic.expand_dims(b, out, dim)
            dim += 1
        elif isinstance(i, slice) and i == slice(None, None, None):
            dim += 1
        else:
            raise CompilationError("tiles support only `:` and `None` in subscripts, as in "
                                   "`x[:, None]`")
    if dim != len(v.type.shape) + sum(1 for i in idx if core.unwrap(i) is None):
        # fewer subscripts than dims: the rest are implied `:`
        pass
    return out


# ---------------------------------------------------------------------------
# Entry point
# ---------------------------------------------------------------------------

_PARSE_CACHE: dict[Any, tuple] = {}


def parse_function(fn):
    key = fn.__code__
    hit = _PARSE_CACHE.get(key)
    if hit is not None:
        return hit
    try:
        lines, start = inspect.getsourcelines(fn)
    except (OSError, TypeError) as e:
        raise CompilationError(f"can't read the source of `{fn.__name__}`: {e}") from None
    src = textwrap.dedent("".join(lines))
    tree = ast.parse(src)
    fdef = next(n for n in tree.body if isinstance(n, (ast.FunctionDef, ast.AsyncFunctionDef)))
    filename = inspect.getsourcefile(fn) or "<kernel>"
    out = (fdef, filename, start - 1, src.splitlines())
    _PARSE_CACHE[key] = out
    return out


def build_ir(fn, arg_types: dict[str, Any], arg_facts: dict[str, dict], constexprs: dict,
             num_warps: int = 4, options: dict | None = None) -> ir.Func:
    """Builds the IR of `fn` for one specialization.

    `arg_types` maps runtime parameter names to `ir.TType` (scalars or pointers), in
    declaration order; `constexprs` maps constexpr parameter names to Python values.
    """
    fdef, filename, off, lines = parse_function(fn)
    args = []
    names = []
    body = ir.Block()
    for name, t in arg_types.items():
        v = ir.Value(t, name_hint=name)
        v.facts.update(arg_facts.get(name, {}))
        args.append(v)
        names.append(name)
    scope: dict[str, Any] = {}
    for n, v in zip(names, args):
        scope[n] = v
    scope.update(constexprs)
    ctx = Context(ir.Builder(body), num_warps, options or {})
    gen = CodeGenerator(ctx, fn, scope, filename, off, lines)
    try:
        gen.visit_stmts(fdef.body)
    except _Return as r:
        if r.value is not None:
            if r.node is not None:
                raise gen.error(r.node, "kernels can't return values; store results through "
                                        "a pointer argument") from None
            raise CompilationError("kernels can't return values") from None
    f = ir.Func(fn.__name__, args, names, body, num_warps, dict(options or {}))
    f.deps = ctx.deps
    return f


def _stable_module(m) -> bool:
    """The language's and the runtime's own modules: their attributes don't change."""
    name = getattr(m, "__name__", "") or ""
    return name.split(".")[0] in ("enceladus", "enceladus_amd", "numpy", "math", "builtins")

