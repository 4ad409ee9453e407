"""Contiguity / divisibility / constancy analysis of integer and pointer tiles.

Per dimension: `contig` is the length of runs of consecutive values (+1 per element),
`div` the largest power of two dividing the first value of each run (bytes for pointers),
`const` the length of runs of equal values. These decide vector widths of memory ops.
Rules follow Triton's axis analysis, as the reference does
(reference: src/enceladus/compiler/passes/axis_info.py:123-356).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

from enceladus_amd.compiler import ir

BIG = 1 << 30


def pow2div(v: int) -> int:
    v = abs(int(v))
    if v == 0:
        return BIG
    return min(v & -v, BIG)


@dataclass(frozen=True)
class Info:
    contig: tuple
    div: tuple
    const: tuple


def _scalar(div: int) -> Info:
    return Info((1,), (div,), (1,))


def _default(shape) -> Info:
    n = max(1, len(shape))
    return Info((1,) * n, (1,) * n, (1,) * n)


def _meet(a: Info, b: Info) -> Info:
    return Info(tuple(math.gcd(x, y) for x, y in zip(a.contig, b.contig)),
                tuple(math.gcd(x, y) for x, y in zip(a.div, b.div)),
                tuple(math.gcd(x, y) for x, y in zip(a.const, b.const)))


class AxisAnalysis:
    def __init__(self, fn: ir.Func):
        self.info: dict[int, Info] = {}
        for a in fn.args:
            t = a.type
            if isinstance(t, ir.DescType):
                continue
            if t.ptr:
                self.info[a.id] = _scalar(16 if a.facts.get("divisibility") else t.dtype.itemsize)
            elif t.dtype.is_int():
                self.info[a.id] = _scalar(pow2div(16) if a.facts.get("divisibility") else 1)
            else:
                self.info[a.id] = _scalar(1)
        self.block(fn.body)

    def get(self, v: ir.Value) -> Info:
        i = self.info.get(v.id)
        if i is None:
            i = _default(v.type.shape) if not isinstance(v.type, ir.DescType) else _scalar(1)
            self.info[v.id] = i
        return i

    def block(self, b: ir.Block):
        for op in b.ops:
            self.op(op)

    def op(self, op: ir.Op):
        n = op.name
        if n == "for":
            body = op.regions[0]
            carried = body.args[1:]
            inits = op.operands[3:]
            self.info[body.args[0].id] = _scalar(1)
            for a, i in zip(carried, inits):
                self.info[a.id] = self.get(i)
            for _ in range(3):
                self.block(body)
                y = body.ops[-1]
                changed = False
                for a, v in zip(carried, y.operands):
                    m = _meet(self.get(a), self.get(v))
                    if m != self.info[a.id]:
                        self.info[a.id] = m
                        changed = True
                if not changed:
                    break
            for r, a in zip(op.results, carried):
                self.info[r.id] = self.info[a.id]
            return
        if n == "if":
            for r in op.regions:
                self.block(r)
            ty, ey = op.regions[0].ops[-1], op.regions[1].ops[-1]
            for res, a, b in zip(op.results, ty.operands, ey.operands):
                self.info[res.id] = _meet(self.get(a), self.get(b))
            return
        if not op.results:
            for r in op.regions:
                self.block(r)
            return
        res = op.result
        if isinstance(res.type, ir.DescType):
            return
        shape = res.type.shape
        rank = max(1, len(shape))
        if n == "const":
            v = op.attrs["value"]
            d = pow2div(v) if isinstance(v, int) and not isinstance(v, bool) else 1
            self.info[res.id] = Info((1,) * rank, (d,) * rank, tuple(shape) if shape else (1,))
        elif n == "arange":
            self.info[res.id] = Info((shape[0],), (pow2div(op.attrs["start"]),), (1,))
        elif n in ("program_id", "num_programs"):
            self.info[res.id] = _scalar(1)
        elif n == "splat":
            s = self.get(op.operands[0])
            self.info[res.id] = Info((1,) * rank, (s.div[0],) * rank, tuple(shape))
        elif n == "expand_dims":
            s = self.get(op.operands[0])
            ax = op.attrs["axis"]
            src_rank = len(op.operands[0].type.shape)
            if src_rank == 0:
                self.info[res.id] = Info((1,), s.div, (1,))
                return
            nd = min([d if c == 1 else 1 for c, d in zip(s.contig, s.div)] or [1])
            self.info[res.id] = Info(s.contig[:ax] + (1,) + s.contig[ax:],
                                     s.div[:ax] + (nd,) + s.div[ax:],
                                     s.const[:ax] + (1,) + s.const[ax:])
        elif n == "broadcast":
            s = self.get(op.operands[0])
            src = op.operands[0].type.shape
            c, d, k = list(s.contig), list(s.div), list(s.const)
            for i, (a, b) in enumerate(zip(src, shape)):
                if a == 1 and b != 1:
                    c[i], k[i] = 1, b
            self.info[res.id] = Info(tuple(c), tuple(d), tuple(k))
        elif n == "trans":
            s = self.get(op.operands[0])
            p = op.attrs["perm"]
            self.info[res.id] = Info(tuple(s.contig[i] for i in p), tuple(s.div[i] for i in p),
                                     tuple(s.const[i] for i in p))
        elif n == "hint":
            s = self.get(op.operands[0])
            c, d = list(s.contig), list(s.div)
            if "multiple_of" in op.attrs:
                vals = op.attrs["multiple_of"]
                d = [max(x, pow2div(vals[min(i, len(vals) - 1)])) for i, x in enumerate(d)]
            if "max_contiguous" in op.attrs:
                vals = op.attrs["max_contiguous"]
                c = [max(x, vals[min(i, len(vals) - 1)]) for i, x in enumerate(c)]
            self.info[res.id] = Info(tuple(c), tuple(d), s.const)
        elif n in ("binary", "ptr_add"):
            a, b = self.get(op.operands[0]), self.get(op.operands[1])
            kind = "add" if n == "ptr_add" else op.attrs["op"]
            if n == "ptr_add":
                es = op.operands[0].type.dtype.itemsize
                b = Info(b.contig, tuple(min(x * es, BIG) for x in b.div), b.const)
            const = tuple(math.gcd(x, y) for x, y in zip(a.const, b.const))
            if kind == "add":
                contig = tuple(max(math.gcd(ca, kb), math.gcd(ka, cb))
                               for ca, cb, ka, kb in zip(a.contig, b.contig, a.const, b.const))
                div = tuple(math.gcd(x, y) for x, y in zip(a.div, b.div))
            elif kind == "sub":
                contig = tuple(math.gcd(ca, kb) for ca, kb in zip(a.contig, b.const))
                div = tuple(math.gcd(x, y) for x, y in zip(a.div, b.div))
            elif kind == "mul":
                contig = (1,) * rank
                div = tuple(min(x * y, BIG) for x, y in zip(a.div, b.div))
            else:
                contig, div = (1,) * rank, (1,) * rank
            if op.result.type.dtype.is_bool() or kind in ("eq", "ne", "lt", "le", "gt", "ge"):
                contig, div = (1,) * rank, (1,) * rank
            self.info[res.id] = Info(contig, div, const)
        elif n == "cast":
            s = self.get(op.operands[0])
            if res.type.dtype.is_int() and op.operands[0].type.dtype.is_int() and \
                    res.type.dtype.primitive_bitwidth >= op.operands[0].type.dtype.primitive_bitwidth:
                self.info[res.id] = s
            else:
                self.info[res.id] = Info((1,) * rank, (1,) * rank, s.const)
        elif n in ("unary", "bitcast"):
            s = self.get(op.operands[0])
            self.info[res.id] = Info((1,) * rank, (1,) * rank, s.const)
        elif n == "select":
            a, b, c = (self.get(o) for o in op.operands)
            const = tuple(math.gcd(math.gcd(x, y), z) for x, y, z in zip(a.const, b.const, c.const))
            self.info[res.id] = Info((1,) * rank, (1,) * rank, const)
        else:
            self.info[res.id] = _default(shape)
        for r in op.regions:
            self.block(r)
