"""Tile IR → HIP C++ for gfx950.

Every tile value lives in per-thread register arrays laid out by a wave64 `Layout`.
Values fall in four kinds:

- scalar:   a uniform C++ variable;
- cheap:    a pure function of element coordinates (aranges, splats, index math), emitted
            inline in whatever layout a consumer asks for, so it never moves;
- view:     broadcast / expand_dims / trans of a stored value: a register re-indexing;
- anchored: a register array with a fixed layout (loads, dots, reductions, scans,
            elementwise results of anchored values, loop-carried values).

A consumer that needs an anchored value in another layout gets it through an LDS round
trip (vectorised where both sides allow). Conversions of loop-invariant values are hoisted
in front of the loop. Reductions use in-register trees, DPP/ds_bpermute butterflies over
lane bits and an LDS step over warp bits; scans use a serial-then-wave-then-block scheme;
`tl.dot` lowers onto gfx950 MFMA instructions with operand layouts built for them.

Reference structure: the MSL emitter `_Codegen` (reference: src/enceladus/compiler/codegen/
msl.py:220-1381), `emit_dot` (dot.py:170-307), `emit_reduce` (reduce.py:58-194), `emit_scan`
(scan.py:348-375) and `emit_atomic` (atomic.py:138-177). The kernel ABI keeps the
reference's rules (runtime args in declaration order with constexprs removed, msl.py:1298-
1342) in HIP form: one kernarg struct with natural alignment, block = num_warps*64.
"""

from __future__ import annotations

import math
import struct
from dataclasses import dataclass, field

import numpy as np

from enceladus_amd.compiler import ir
from enceladus_amd.compiler import layout as LY
from enceladus_amd.compiler import lds as LDS
from enceladus_amd.compiler.axis_info import AxisAnalysis
from enceladus_amd.compiler.errors import CompilationError
from enceladus_amd.language import core

MAX_LDS = 160 * 1024

_MATH = {"exp": "expf", "exp2": "ek::exp2_fast", "log": "logf", "log2": "log2f", "sqrt": "sqrtf",
         "sin": "sinf", "cos": "cosf", "tanh": "tanhf", "erf": "ek::erf_as", "floor": "floorf",
         "ceil": "ceilf"}
_INFIX = {"add": "+", "sub": "-", "mul": "*", "div": "/", "and": "&", "or": "|", "xor": "^",
          "eq": "==", "ne": "!=", "lt": "<", "le": "<=", "gt": ">", "ge": ">="}


def _through_trans(v: ir.Value) -> ir.Value:
    while v.op is not None and v.op.name == "trans":
        v = v.op.operands[0]
    return v


def ctype(dt: core.dtype) -> str:
    return dt.cname


def is_half(dt: core.dtype) -> bool:
    return dt in (core.float16, core.bfloat16)


def literal(v, dt: core.dtype) -> str:
    if dt.is_bool():
        return "true" if v else "false"
    if dt.is_floating():
        f = float(v)
        if dt is core.bfloat16:
            bits = int(np.array([f], np.float32).view(np.uint32)[0])
            if (bits & 0x7FFFFFFF) > 0x7F800000:
                b16 = (bits >> 16) | 0x40
            else:
                b16 = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) & 0xFFFF
            return f"ek::bf16{{0x{b16:04x}}}"
        if dt is core.float16:
            f = float(np.float16(f))
        else:
            f = float(np.float32(f))
        if math.isnan(f):
            s = "__builtin_nanf(\"\")"
        elif math.isinf(f):
            s = "__builtin_inff()" if f > 0 else "(-__builtin_inff())"
        else:
            s = f.hex() + "f"
        return f"(_Float16)({s})" if dt is core.float16 else s
    v = int(v)
    if dt.is_signed():
        if dt.primitive_bitwidth == 64:
            return f"(int64_t)({v}LL)" if v > -(1 << 63) else "(int64_t)(-9223372036854775807LL-1)"
        if v == -(1 << 31):
            return "(int32_t)(-2147483647-1)"
        return f"({ctype(dt)})({v})"
    return f"({ctype(dt)})({v}ULL)"


def bits_expr(r: str, pairs: list[tuple[int, int]]) -> str:
    """OR of ((r >> j) & 1) << i over (j, i) pairs, merging runs."""
    if not pairs:
        return "0"
    pairs = sorted(pairs)
    runs = []
    for j, i in pairs:
        if runs and runs[-1][0] + runs[-1][2] == j and runs[-1][1] + runs[-1][2] == i:
            runs[-1][2] += 1
        else:
            runs.append([j, i, 1])
    terms = []
    for j, i, n in runs:
        mask = (1 << n) - 1
        t = f"({r})" if j == 0 else f"(({r}) >> {j})"
        t = f"({t} & {mask})"
        if i:
            t = f"({t} << {i})"
        terms.append(t)
    return " | ".join(terms) if len(terms) > 1 else terms[0]


_STAGE_LAYOUTS: dict = {}


@dataclass
class Scope:
    level: int
    items: list = field(default_factory=list)
    memo: dict = field(default_factory=dict)
    hoist: list | None = None
    indent: str = "  "


@dataclass
class KernelArg:
    name: str
    kind: str          # "ptr" | "scalar"
    dtype: core.dtype
    cparam: str        # C++ parameter type


@dataclass
class GeneratedKernel:
    name: str
    source: str
    args: list
    num_warps: int
    lds_bytes: int
    block: int
    coarsen: int = 0       # workgroups per CU of a coarsened launch (0: one per program)
    asserts: list = field(default_factory=list)   # tl.device_assert sites (message, loc)
    # two-level histogram flush: {"name", "rb" (rows per flush workgroup), "bases" (arg
    # indices), "total" (words per workgroup row of the partial buffer), "chunks" (64-word
    # column chunks)}; the launcher runs `name` on grid (chunks, rows / rb) after the kernel
    flush: dict | None = None
    # what `kernel.explain` reports: {"conversions", "lds", "dots"} recorded by the emitter
    report: dict = field(default_factory=dict)


class Emitter:
    def __init__(self, fn: ir.Func, options: dict | None = None):
        self.fn = fn
        self.opt = options or {}
        self.report: dict = {}
        self.nw = fn.num_warps
        self.nt = 64 * self.nw
        self.axis = AxisAnalysis(fn)
        self.kind: dict[int, str] = {}
        self.lay: dict[int, LY.Layout] = {}
        self.name: dict[int, str] = {}
        self.vals: dict[int, ir.Value] = {}
        self.uses: dict[int, list] = {}
        self.def_level: dict[int, int] = {}
        self.desc: dict[int, dict] = {}
        self.tc: dict[tuple, str] = {}
        self.prologue: list[str] = []
        self.scopes = [Scope(0)]
        self.counter = 0
        self.lds = 0
        self.dot_plans: dict[int, LY.DotPlan] = {}
        self.inplace: set[int] = set()
        self.extra_smem: list[tuple[str, int]] = []
        self.asserts: list[dict] = []
        self.split_bit: dict[int, tuple] = {}
        self.int_dots: set[int] = set()
        # program versioning: the fast copy assumes the uniform edge conditions it guards
        self.fast_mode = False
        self.fast_conds: list[str] = []
        self.fast_side = False
        self.fast_streams = 0
        self.fast_failed = False
        self.edge_only = False       # the general copy runs only for edge programs

    # ------------------------------------------------------------------ utilities
    def fresh(self, hint="v") -> str:
        self.counter += 1
        return f"{hint}{self.counter}"

    @property
    def cur(self) -> Scope:
        return self.scopes[-1]

    def emit(self, line: str):
        self.cur.items.append(self.cur.indent + line)

    def need_lds(self, nbytes: int):
        op = getattr(self, "cur_op", None)
        if op is not None:
            self.report.setdefault("lds", []).append(
                {"op": op.name, "loc": op.loc, "bytes": int(nbytes)})
        self.lds = max(self.lds, nbytes)
        if getattr(self, "in_staged_loop", 0):
            self.scratch_in_stage_loop = True

    def tile(self, v: ir.Value) -> bool:
        return not isinstance(v.type, ir.DescType) and v.type.shape != ()

    def count_uses(self, block: ir.Block):
        for op in block.ops:
            for o in op.operands:
                self.uses.setdefault(o.id, []).append(op)
            for r in op.regions:
                self.count_uses(r)

    # ------------------------------------------------------------------ layouts
    def default_layout(self, v: ir.Value) -> LY.Layout:
        es = 8 if v.type.ptr else v.type.dtype.itemsize
        return LY.default_blocked(v.type.shape, self.nw, es)

    def mem_layout(self, ptr: ir.Value) -> LY.Layout:
        shape = ptr.type.shape
        info = self.axis.get(ptr)
        es = ptr.type.dtype.itemsize
        best = len(shape) - 1
        for d in range(len(shape)):
            if info.contig[d] > info.contig[best]:
                best = d
        vec = min(info.contig[best], max(1, info.div[best] // es), max(1, 16 // es),
                  shape[best])
        vec = 1 << LY.log2(max(1, vec))
        order = [best] + [d for d in reversed(range(len(shape))) if d != best]
        return LY.blocked(shape, order, vec, self.nw)

    def mem_vec(self, ptr: ir.Value, lay: LY.Layout) -> int:
        """Elements per vector access for `ptr` read in `lay` (contiguity, alignment)."""
        info = self.axis.get(ptr)
        es = ptr.type.dtype.itemsize
        d, nb = lay.vec_dim_bits()
        if not lay.reg or nb == 0:
            return 1
        v = min(1 << nb, info.contig[d], max(1, info.div[d] // es), max(1, 16 // es))
        return 1 << LY.log2(max(1, v))

    def wave_run_bytes(self, ptr: ir.Value, lay: LY.Layout) -> int:
        """Bytes one vector access of `ptr` in `lay` covers contiguously across a wave:
        the register vector, then the lane bits that continue the same dim."""
        info = self.axis.get(ptr)
        d, nb = lay.vec_dim_bits()
        if nb == 0 and lay.lane and lay.lane[0] is not None:
            d = lay.lane[0][0]
        v = self.mem_vec(ptr, lay)
        run = v
        if v >= (1 << nb):
            k = 0
            while k < len(lay.lane) and lay.lane[k] == (d, nb + k):
                k += 1
            run = v << k
        return min(run, info.contig[d]) * ptr.type.dtype.itemsize

    def lay_of(self, v: ir.Value):
        return self.lay.get(v.id)

    def assign_block(self, block: ir.Block):
        for op in block.ops:
            self.assign_op(op)

    # -- dot planning ------------------------------------------------------------------
    _EW = ("binary", "unary", "cast", "select", "fma", "bitcast", "hint")

    def _dot_source(self, v: ir.Value, depth=0):
        """The dot whose accumulator `v` derives from elementwise (same shape), if any."""
        if v.op is None or depth > 64:
            return None
        if v.op.name == "dot":
            return v.op
        if v.op.name in self._EW:
            for o in v.op.operands:
                if o.type.shape == v.type.shape:
                    d = self._dot_source(o, depth + 1)
                    if d is not None:
                        return d
        return None

    def plan_dots(self, fn: ir.Func):
        """Chooses warps/MFMA shape per dot, and the transposed orientation with a matching
        k order when one dot's result feeds another dot's A operand (attention's P), so
        the product's registers are the next MFMA's operand registers."""
        dw = self.opt.get("dot_warps")
        dots = []
        base = {}
        for d in (op for op in ir.walk(fn.body) if op.name == "dot"):
            a, b = d.operands[0], d.operands[1]
            adt = a.type.dtype
            if adt.is_int() and (adt is not core.int8 or self.opt.get("no_int8_mfma")):
                self.int_dots.add(d.result.id)   # multiply-adds from LDS
                continue
            try:
                base[d] = LY.plan_dot(a.type.shape[0], b.type.shape[1], a.type.shape[1],
                                      self.nw, adt.name, dw)
            except ValueError:
                # tiles below the MFMA minimums (16x16, K a multiple of the instruction
                # depth): multiply-adds from LDS
                self.int_dots.add(d.result.id)
                continue
            dots.append(d)
        trans, korder = set(), {}
        if not self.opt.get("no_dot_transpose") and not self.opt.get("no_acc_transpose"):
            # 16-bit 32x32x16 dots compute C^T: each lane then holds one row of the result
            # and 4 consecutive columns per 4 registers, so row reductions stay in registers
            # and the result goes to memory in 8-byte runs instead of 2-byte ones (the
            # 4096^3 matmul's epilogue: 8.4 K cycles per wave against 10.6 K in the
            # instruction's own orientation; ENCELADUS_CODEGEN=no_acc_transpose keeps that).
            for d in dots:
                p = base[d]
                if p.inst.m == 32 and p.inst.k == 16 and \
                        d.operands[0].type.dtype in (core.float16, core.bfloat16):
                    trans.add(d)
        if not self.opt.get("no_dot_transpose"):
            for d2 in dots:
                d1 = self._dot_source(d2.operands[0])
                if d1 is None or d1 is d2 or d1 not in base:
                    continue
                p1, p2 = base[d1], base[d2]
                if p1.inst.m != 32 or p2.inst.m != 32 or p2.inst.k != 16:
                    continue
                if (p1.wm, p1.wn) != (p2.wm, p2.wn) or p1.wn != 1 or p1.bm != p2.bm:
                    continue
                trans.update((d1, d2))
                nk = LY.log2(p2.bk)
                if nk >= 4:
                    korder[d2] = (0, 1, 3, 2) + tuple(range(4, nk))
        for d in dots:
            a, b = d.operands[0], d.operands[1]
            self.dot_plans[d.result.id] = LY.plan_dot(
                a.type.shape[0], b.type.shape[1], a.type.shape[1], self.nw, a.type.dtype.name,
                dw, d in trans, korder.get(d, ()))

    def _operand_layout_for(self, v: ir.Value):
        """If `v`'s single use is a dot operand (directly or through trans), the layout that
        operand wants, expressed in `v`'s own shape."""
        us = self.uses.get(v.id, [])
        if len(us) != 1:
            return None
        u = us[0]
        perm = None
        if u.name == "trans" and len(self.uses.get(u.result.id, [])) == 1:
            perm = u.attrs["perm"]
            v2 = u.result
            u = self.uses[v2.id][0]
        else:
            v2 = v
        if u.name != "dot" or u.result.id not in self.dot_plans:
            return None
        plan = self.dot_plans[u.result.id]
        if u.operands[0].id == v2.id:
            lay = LY.mfma_operand(plan, "a")
        elif u.operands[1].id == v2.id:
            lay = LY.mfma_operand(plan, "b")
        else:
            return None
        if perm is not None:
            inv = [0] * len(perm)
            for i, p in enumerate(perm):
                inv[p] = i
            lay = lay.permute(tuple(inv))
        return lay

    def _anch(self, v):
        return self.kind.get(v.id) in ("anchored", "view", "staged", "fused")

    def assign_op(self, op: ir.Op):
        n = op.name
        for r in op.results:
            self.vals[r.id] = r
        if n == "for":
            self.assign_for(op)
            return
        if n == "if":
            for reg in op.regions:
                self.assign_block(reg)
            ty, ey = op.regions[0].ops[-1], op.regions[1].ops[-1]
            for res, a, b in zip(op.results, ty.operands, ey.operands):
                if not self.tile(res):
                    self.kind[res.id] = "scalar"
                    continue
                self.kind[res.id] = "anchored"
                la = self.lay_of(a) if self._anch(a) else None
                lb = self.lay_of(b) if self._anch(b) else None
                self.lay[res.id] = la or lb or self.default_layout(res)
            return
        for reg in op.regions:
            self.assign_block(reg)
        if not op.results:
            return
        res = op.result
        if isinstance(res.type, ir.DescType):
            self.kind[res.id] = "desc"
            return
        if not self.tile(res):
            self.kind[res.id] = "scalar"
            return
        if n in ("const", "arange", "splat"):
            self.kind[res.id] = "cheap"
        elif n in ("broadcast", "expand_dims", "trans", "hint", "reshape"):
            src = op.operands[0]
            if not self._anch(src):
                self.kind[res.id] = "cheap"
            else:
                self.kind[res.id] = "view"
                sl = self.lay[src.id]
                if n == "broadcast":
                    self.lay[res.id] = sl.lift(res.type.shape)
                elif n == "expand_dims":
                    self.lay[res.id] = sl.expand(op.attrs["axis"])
                elif n == "trans":
                    self.lay[res.id] = sl.permute(op.attrs["perm"])
                elif n == "reshape":
                    self.lay[res.id] = sl.reshape(res.type.shape)
                else:
                    self.lay[res.id] = sl
        elif n == "join":
            # the new last dim is register bit 0: res[2r + k] = (a, b)[k][r]
            self.kind[res.id] = "anchored"
            base = next((self.lay[o.id] for o in op.operands
                         if self._anch(o) and self.kind[o.id] == "anchored"), None)
            base = base or self.default_layout(op.operands[0])
            rank = len(base.shape)
            self.lay[res.id] = LY.Layout(res.type.shape, ((rank, 0),) + tuple(base.reg),
                                         base.lane, base.warp)
        elif n == "split":
            x = op.operands[0]
            rank = len(x.type.shape)
            xl = self.lay[x.id] if self._anch(x) else None
            bit = (rank - 1, 0)
            if xl is not None and (bit in xl.reg or bit in xl.lane):
                # a register bit selects registers; a lane bit becomes two shuffles, and
                # both halves are then replicated over that lane bit
                mode = ("reg", xl.reg.index(bit)) if bit in xl.reg else \
                    ("lane", xl.lane.index(bit))
                out = LY.Layout(res.type.shape, tuple(b for b in xl.reg if b != bit),
                                tuple(None if b == bit else b for b in xl.lane),
                                tuple(None if b == bit else b for b in xl.warp))
            else:
                out = self.default_layout(res)
                mode = ("reg", 0)
            for r in op.results:
                self.kind[r.id] = "anchored"
                self.lay[r.id] = out
            self.split_bit[res.id] = mode
        elif n == "shift":
            src = op.operands[0]
            self.kind[res.id] = "anchored"
            self.lay[res.id] = self.lay_of(src) if self._anch(src) and \
                self.kind[src.id] == "anchored" else self.default_layout(res)
        elif n in ("binary", "unary", "cast", "select", "fma", "ptr_add", "bitcast"):
            anch = [o for o in op.operands if self.tile(o) and self._anch(o)]
            if not anch:
                self.kind[res.id] = "cheap"
            else:
                self.kind[res.id] = "anchored"
                pick = next((o for o in anch if self.kind[o.id] == "anchored"), anch[0])
                self.lay[res.id] = self.lay[pick.id]
                if self._fusable(op):
                    self.kind[res.id] = "fused"
        elif n == "load":
            self.kind[res.id] = "anchored"
            lay = self.mem_layout(op.operands[0])
            us = self.uses.get(res.id, [])
            if len(us) == 1 and us[0].name == "scan" and \
                    LY.scan_groups(lay, us[0].attrs["axis"]) is None:
                lay = LY.scan_layout(res.type.shape, us[0].attrs["axis"], self.nw)
            self.lay[res.id] = lay
        elif n == "desc_load" and res.id in self.staged:
            self.kind[res.id] = "staged"
            self.lay[res.id] = self.staged[res.id]["lay"]
        elif n == "desc_load":
            self.kind[res.id] = "anchored"
            es = res.type.dtype.itemsize
            lay = self._operand_layout_for(res)
            if lay is not None:
                d, nb = lay.vec_dim_bits()
                # direct operand loads only when each lane reads >= 16 contiguous bytes
                if not (d == len(lay.shape) - 1 and (1 << nb) * es >= 16):
                    lay = None
            if lay is None:
                lay = LY.blocked(res.type.shape, LY.default_order(res.type.shape),
                                 max(1, 16 // es), self.nw)
            self.lay[res.id] = lay
        elif n == "dot":
            self.kind[res.id] = "anchored"
            if res.id in self.int_dots:
                self.lay[res.id] = self.default_layout(res)
            else:
                self.lay[res.id] = LY.mfma_acc(self.dot_plans[res.id])
        elif n == "reduce":
            src = op.operands[0]
            sl = self.lay[src.id] if self._anch(src) else self.default_layout(src)
            self.kind[res.id] = "anchored"
            self.lay[res.id] = sl.slice(op.attrs["axis"])
        elif n == "scan":
            src = op.operands[0]
            ax = op.attrs["axis"]
            sl = self.lay[src.id] if self._anch(src) else None
            if sl is None or LY.scan_groups(sl, ax) is None:
                sl = LY.scan_layout(src.type.shape, ax, self.nw)
            self.kind[res.id] = "anchored"
            self.lay[res.id] = sl
        elif n in ("atomic_rmw", "atomic_cas"):
            self.kind[res.id] = "anchored"
            self.lay[res.id] = self.mem_layout(op.operands[0])
            if res.id in getattr(self, "priv", {}):
                idx = op.operands[0].op.operands[1]
                if self._anch(idx) and self.lay[idx.id].shape == res.type.shape:
                    self.lay[res.id] = self.lay[idx.id]
        else:
            raise CompilationError(f"the HIP backend doesn't lower `{n}`")

    _EW_OPS = ("binary", "unary", "cast", "select", "fma", "bitcast")
    _CHEAP_BIN = ("add", "sub", "mul", "and", "or", "xor", "min", "max", "eq", "ne", "lt",
                  "le", "gt", "ge")

    def _fusable(self, op: ir.Op) -> bool:
        """Elementwise results consumed only by elementwise ops are emitted inline in their
        consumers (no register array): single-use values always, multi-use ones when cheap."""
        if self.opt.get("no_fusion"):
            return False
        us = self.uses.get(op.result.id, [])
        if len(us) == 1 and us[0].name == "store" and us[0].operands[1] is op.result and \
                op.result not in us[0].operands[2:] and not self.opt.get("no_store_fusion"):
            # the value of a store: computed vector by vector inside the store loop, so
            # each vector's writes go out while the next one's math runs
            return True
        if not us or any(u.name not in self._EW_OPS for u in us):
            return False
        if len(us) == 1:
            return True
        if op.name in ("cast", "select", "bitcast"):
            return True
        if op.name == "binary" and op.attrs["op"] in self._CHEAP_BIN:
            return True
        if op.name == "unary" and op.attrs["op"] in ("neg", "abs", "not"):
            return True
        return False

    def _use_layout(self, body: ir.Block, arg: ir.Value):
        """Layout of the first memory op that reads or writes through `arg`."""
        frontier = {arg.id}
        for op in ir.walk(body):
            if op.name in ("load", "store", "atomic_rmw", "atomic_cas") and \
                    op.operands[0].id in frontier:
                return self.mem_layout(op.operands[0])
            if op.name in ("ptr_add", "binary", "broadcast", "hint") and \
                    op.operands[0].id in frontier and op.results:
                frontier.add(op.result.id)
        return None

    def assign_for(self, op: ir.Op):
        body = op.regions[0]
        iv, carried = body.args[0], body.args[1:]
        inits = op.operands[3:]
        self.kind[iv.id] = "scalar"
        self.vals[iv.id] = iv
        pending = []
        for a, i in zip(carried, inits):
            self.vals[a.id] = a
            if not self.tile(a):
                self.kind[a.id] = "scalar"
            elif self._anch(i):
                self.kind[a.id] = "anchored"
                self.lay[a.id] = self.lay[i.id].lift(a.type.shape) if \
                    self.lay[i.id].shape != a.type.shape else self.lay[i.id]
            else:
                self.kind[a.id] = "cheap"   # provisional
                pending.append(a)
        for _ in range(3):
            self.assign_block(body)
            y = body.ops[-1]
            changed = False
            for a, v in zip(carried, y.operands):
                if a in pending and self._anch(v):
                    self.kind[a.id] = "anchored"
                    self.lay[a.id] = self.lay[v.id]
                    pending.remove(a)
                    changed = True
            if not changed:
                break
        for a in list(pending):
            lay = self._use_layout(body, a) or self.default_layout(a)
            self.kind[a.id] = "anchored"
            self.lay[a.id] = lay
            pending.remove(a)
        self.assign_block(body)
        for r, a in zip(op.results, carried):
            self.vals[r.id] = r
            self.kind[r.id] = self.kind[a.id]
            if a.id in self.lay:
                self.lay[r.id] = self.lay[a.id]

    # ------------------------------------------------------------------ coordinates
    def thread_coord(self, lay: LY.Layout, d: int) -> str:
        key = (lay.key(), d)
        nm = self.tc.get(key)
        if nm is not None:
            return nm
        pairs_l = [(i, b[1]) for i, b in enumerate(lay.lane) if b is not None and b[0] == d]
        pairs_w = [(i, b[1]) for i, b in enumerate(lay.warp) if b is not None and b[0] == d]
        terms = []
        if pairs_l:
            terms.append(bits_expr("ek_lane", pairs_l))
        if pairs_w:
            terms.append(bits_expr("ek_warp", pairs_w))
        if not terms:
            self.tc[key] = "0"
            return "0"
        nm = f"tc{len(self.tc)}"
        self.prologue.append(f"  const int {nm} = {' | '.join(terms)};")
        self.tc[key] = nm
        return nm

    def reg_coord(self, lay: LY.Layout, d: int, r: str) -> str:
        pairs = [(i, b[1]) for i, b in enumerate(lay.reg) if b[0] == d]
        return bits_expr(r, pairs) if pairs else "0"

    def coord(self, lay: LY.Layout, d: int, r: str) -> str:
        t = self.thread_coord(lay, d)
        rc = self.reg_coord(lay, d, r)
        if t == "0":
            return f"({rc})"
        if rc == "0":
            return t
        return f"({t} + ({rc}))"

    def owner_cond(self, lay: LY.Layout) -> str | None:
        lm = sum(1 << i for i, b in enumerate(lay.lane) if b is None)
        wm = sum(1 << i for i, b in enumerate(lay.warp) if b is None)
        conds = []
        if lm:
            conds.append(f"((ek_lane & {lm}) == 0)")
        if wm:
            conds.append(f"((ek_warp & {wm}) == 0)")
        return " && ".join(conds) if conds else None

    # ------------------------------------------------------------------ expressions
    def ew(self, op: ir.Op, xs: list[str]) -> str:
        """Elementwise expression of `op` given operand expressions."""
        n = op.name
        rt = op.result.type.dtype
        if n == "binary":
            k = op.attrs["op"]
            dt = op.operands[0].type.dtype
            a, b = xs
            if is_half(dt):
                a, b = f"ek::f32({a})", f"ek::f32({b})"
            if k in ("eq", "ne", "lt", "le", "gt", "ge"):
                return f"({a} {_INFIX[k]} {b})"
            cdt = "float" if is_half(dt) else ctype(dt)
            if k in ("add", "sub", "mul") and dt in (core.int32, core.int64):
                # signed 32/64-bit math wraps (two's complement), as the language defines
                # it; C++ leaves signed overflow undefined
                e = f"ek::w{k}({a}, {b})"
            elif k == "div" and dt.is_floating() and self._uniform_divisor(op):
                # relaxed math (the language's default, as Metal's relaxed mode): a tile
                # divided by a value repeated along it (a broadcast row statistic) is
                # multiplied by the divisor's reciprocal, one IEEE division per distinct
                # divisor (the compiler shares `1.0f / b` across the elements that read
                # the same b); within 1.5 ulp of the quotient
                e = f"({a} * (1.0f / {b}))"
            elif k in ("add", "sub", "mul", "div"):
                e = f"({a} {_INFIX[k]} {b})"
            elif k in ("and", "or", "xor"):
                e = f"({a} {_INFIX[k]} {b})"
            elif k == "floordiv":
                e = f"ek::idiv<{cdt}>({a}, {b})"
            elif k == "mod":
                e = f"ek::fmodf_({a}, {b})" if dt.is_floating() else f"ek::imod<{cdt}>({a}, {b})"
            elif k == "shl":
                e = f"ek::ishl<{cdt}>({a}, {b})"
            elif k == "shr":
                e = f"ek::ishr<{cdt}>({a}, {b})"
            elif k == "min":
                e = f"__builtin_fminf({a}, {b})" if dt.is_floating() else \
                    f"ek::Min::op<{cdt}>({a}, {b})"
            elif k == "max":
                e = f"__builtin_fmaxf({a}, {b})" if dt.is_floating() else \
                    f"ek::Max::op<{cdt}>({a}, {b})"
            else:
                raise CompilationError(f"unknown binary op {k}")
            if is_half(dt):
                return f"ek::rnd<{ctype(rt)}>({e})"
            return f"(({ctype(rt)}){e})"
        if n == "unary":
            k = op.attrs["op"]
            dt = op.operands[0].type.dtype
            (a,) = xs
            if k == "not":
                return f"(!{a})" if dt.is_bool() else f"(({ctype(dt)})~{a})"
            if dt.is_floating():
                fa = f"ek::f32({a})" if is_half(dt) else a
                if k == "neg":
                    e = f"(-{fa})"
                elif k == "abs":
                    e = f"__builtin_fabsf({fa})"
                elif k == "rsqrt":
                    e = f"(1.0f / sqrtf({fa}))"
                elif k == "sigmoid":
                    e = f"(1.0f / (1.0f + expf(-{fa})))"
                else:
                    e = f"{_MATH[k]}({fa})"
                return f"ek::rnd<{ctype(dt)}>({e})" if is_half(dt) else e
            if k == "neg":
                return f"ek::wneg({a})" if dt in (core.int32, core.int64) else \
                    f"(({ctype(dt)})(-{a}))"
            if k == "abs":
                if dt in (core.int32, core.int64):
                    return f"({a} < 0 ? ek::wneg({a}) : {a})"
                return f"(({ctype(dt)})({a} < 0 ? -{a} : {a}))"
            raise CompilationError(f"`{k}` needs a floating-point input")
        if n == "cast":
            return f"ek::cvt<{ctype(rt)}>({xs[0]})"
        if n == "bitcast":
            return f"__builtin_bit_cast({ctype(rt)}, {xs[0]})"
        if n == "select":
            return f"({xs[0]} ? {xs[1]} : {xs[2]})"
        if n == "fma":
            if is_half(rt):
                return f"ek::rnd<{ctype(rt)}>(__builtin_fmaf(ek::f32({xs[0]}), ek::f32({xs[1]}), " \
                       f"ek::f32({xs[2]})))"
            return f"__builtin_fmaf({xs[0]}, {xs[1]}, {xs[2]})"
        if n == "ptr_add":
            return f"({xs[0]} + {xs[1]})"
        raise CompilationError(f"not an elementwise op: {n}")

    def _uniform_divisor(self, op: ir.Op) -> bool:
        """Whether `op` (a float division) is emitted as a multiplication by the divisor's
        reciprocal: under relaxed math when the divisor is a tile that repeats one value
        along a dimension (a broadcast row statistic, as attention's `acc / l[:, None]`);
        under fast math also for a scalar or splat divisor. Relaxed math keeps the IEEE
        division for a scalar divisor: on a row kernel (softmax, one row per program, the
        row sum splat over the row) the division measured 4% faster than the reciprocal in
        interleaved A/B runs on MI355X. The "precise" setting (an experiment switch of
        ENCELADUS_CODEGEN) keeps every division."""
        mode = self.opt.get("math_mode", "relaxed")
        if mode == "precise" or not op.result.type.shape:
            return False
        d = op.operands[1]
        if not d.type.shape or self.kind.get(d.id) == "scalar":
            return mode == "fast"
        if d.op is not None and d.op.name == "splat":
            return mode == "fast"
        return d.op is not None and d.op.name == "broadcast"

    def cheap(self, v: ir.Value, coords: list[str]) -> str:
        k = self.kind.get(v.id)
        if k == "scalar":
            return self.name[v.id]
        op = v.op
        if op is None:
            raise CompilationError("internal: cheap block argument")
        n = op.name
        if n == "const":
            return literal(op.attrs["value"], v.type.dtype)
        if n == "arange":
            s = op.attrs["start"]
            return f"((int32_t)({s} + {coords[0]}))" if s else f"((int32_t){coords[0]})"
        if n == "splat":
            return self.name[op.operands[0].id]
        if n == "broadcast":
            x = op.operands[0]
            xc = [("0" if x.type.shape[d] == 1 else coords[d]) for d in range(len(coords))]
            return self.cheap(x, xc)
        if n == "expand_dims":
            ax = op.attrs["axis"]
            return self.cheap(op.operands[0], coords[:ax] + coords[ax + 1:])
        if n == "trans":
            perm = op.attrs["perm"]
            xc = [None] * len(perm)
            for i, p in enumerate(perm):
                xc[p] = coords[i]
            return self.cheap(op.operands[0], xc)
        if n == "hint":
            return self.cheap(op.operands[0], coords)
        if n == "reshape":
            # row-major linear index, then the source coordinates (power-of-two dims)
            shp, src = v.type.shape, op.operands[0]
            lin, sh = [], 0
            for d in reversed(range(len(shp))):
                lin.append(f"(({coords[d]}) << {sh})" if sh else f"({coords[d]})")
                sh += LY.log2(shp[d])
            le = "(" + " | ".join(lin) + ")" if lin else "0"
            xc, sh = [None] * len(src.type.shape), 0
            for d in reversed(range(len(src.type.shape))):
                xc[d] = f"(({le} >> {sh}) & {src.type.shape[d] - 1})"
                sh += LY.log2(src.type.shape[d])
            return self.cheap(src, xc)
        xs = []
        for o in op.operands:
            xs.append(self.name[o.id] if not self.tile(o) else self.cheap(o, coords))
        return self.ew(op, xs)

    def resolve(self, v: ir.Value, lay: LY.Layout, r: str):
        """Follows views back to a stored value: (src, layout over src shape, index expr)."""
        while self.kind.get(v.id) == "view":
            op = v.op
            src = op.operands[0]
            if op.name == "broadcast":
                proj = lay.project(src.type.shape)
                kept = [j for j, b in enumerate(lay.reg) if src.type.shape[b[0]] != 1]
                r = bits_expr(r, [(j, t) for t, j in enumerate(kept)])
                lay = proj
            elif op.name == "expand_dims":
                ax = op.attrs["axis"]
                lay = lay._map(lambda b: (b[0] - (b[0] > ax), b[1]),
                               lay.shape[:ax] + lay.shape[ax + 1:])
            elif op.name == "trans":
                perm = op.attrs["perm"]
                inv = [0] * len(perm)
                for i, p in enumerate(perm):
                    inv[p] = i
                lay = lay.permute(tuple(inv))
            elif op.name == "reshape":
                lay = lay.reshape(src.type.shape)
            v = src
        return v, lay, r

    def elem(self, v: ir.Value, lay: LY.Layout, r: str) -> str:
        k = self.kind.get(v.id)
        if k == "scalar":
            return self.name[v.id]
        if k == "fused":
            op = v.op
            xs = [self.elem(o, lay, r) if self.tile(o) else self.name[o.id] for o in op.operands]
            return self.ew(op, xs)
        if k == "cheap":
            return self.cheap(v, [self.coord(lay, d, r) for d in range(len(lay.shape))])
        src, sl, ri = self.resolve(v, lay, r)
        if self.kind.get(src.id) == "cheap":
            return self.cheap(src, [self.coord(sl, d, ri) for d in range(len(sl.shape))])
        if self.kind.get(src.id) == "fused":
            return self.elem(src, sl, ri)
        if self.kind.get(src.id) == "staged":
            return f"{self.read_staged(src, sl)}[{ri}]"
        a = self.lay[src.id]
        nm = self.name[src.id]
        if a.key() == sl.key():
            return f"{nm}[{ri}]"
        if LY.is_view(a, sl):
            return f"{nm}[{bits_expr(ri, LY.reg_index_map(a, sl))}]"
        conv = self.convert(src, sl)
        return f"{conv}[{ri}]"

    def prime(self, *pairs):
        """Materialises any conversion the given (value, layout) reads need, so that the
        code for it is emitted before a loop header rather than inside the loop body."""
        for v, lay in pairs:
            if v is not None and self.tile(v):
                self.elem(v, lay, "0")

    def array(self, v: ir.Value, lay: LY.Layout) -> str:
        """Name of an array holding `v` in exactly `lay` (materialising if needed)."""
        k = self.kind.get(v.id)
        if k == "staged":
            return self.read_staged(v, lay)
        if k == "view":
            src, sl, ri = self.resolve(v, lay, "r")
            if self.kind.get(src.id) == "staged" and ri == "r":
                return self.read_staged(src, sl)
        if k == "anchored" and self.lay[v.id].key() == lay.key():
            return self.name[v.id]
        if k in ("anchored", "view"):
            src, sl, ri = self.resolve(v, lay, "r")
            if self.kind.get(src.id) == "anchored" and ri == "r" and \
                    self.lay[src.id].key() == sl.key():
                return self.name[src.id]
            if self.kind.get(src.id) == "anchored" and ri == "r" and \
                    not LY.is_view(self.lay[src.id], sl):
                return self.convert(src, sl)
        nm = self.fresh("m")
        t = ctype(v.type.dtype) + ("*" if v.type.ptr else "")
        e = self.elem(v, lay, "r")
        self.emit(f"{t} {nm}[{lay.nregs}];")
        self.emit(f"#pragma unroll")
        self.emit(f"for (int r = 0; r < {lay.nregs}; ++r) {nm}[r] = {e};")
        return nm

    # ------------------------------------------------------------------ LDS conversion
    def lds_order(self, a: LY.Layout, b: LY.Layout, es: int = 4):
        rank = len(a.shape)
        if rank == 0:
            return []
        best = None
        for f in dict.fromkeys([b.vec_dim_bits()[0], a.vec_dim_bits()[0]]):
            order = [f] + [d for d in reversed(range(rank)) if d != f]
            cost = a.nregs // self.lds_vec(a, order, es) + b.nregs // self.lds_vec(b, order, es)
            if best is None or cost < best[0]:
                best = (cost, order)
        return best[1]

    def lds_addr(self, shape, order, es: int):
        """Strides (elements) for an LDS image of `shape` with the given dim order,
        padding each fastest-dim row by 16 bytes when rows are >= 128 bytes."""
        strides = [0] * len(shape)
        s = 1
        pad = 0
        for i, d in enumerate(order):
            strides[d] = s
            if i == 0:
                row = shape[d]
                pad = (16 // es) if row * es >= 128 and len(order) > 1 else 0
                s = row + pad
            else:
                s *= shape[d]
        return strides, s

    def lds_index(self, lay: LY.Layout, strides, r: str) -> str:
        terms = []
        for d, st in enumerate(strides):
            if lay.shape[d] == 1:
                continue
            terms.append(f"({self.coord(lay, d, r)}) * {st}")
        return " + ".join(terms) if terms else "0"

    def lds_vec(self, lay: LY.Layout, order, es: int) -> int:
        if not order or not lay.reg:
            return 1
        d, n = lay.vec_dim_bits()
        if d != order[0]:
            return 1
        return min(1 << n, max(1, 16 // es))

    def _target_scope(self, v: ir.Value) -> int:
        return self.def_level.get(v.id, 0)

    def convert(self, src: ir.Value, dst: LY.Layout) -> str:
        key = ("conv", src.id, dst.key())
        lvl = self._target_scope(src)
        for s in reversed(self.scopes[lvl:]):
            if key in s.memo:
                return s.memo[key]
        a = self.lay[src.id]
        t = ctype(src.type.dtype) + ("*" if src.type.ptr else "")
        es = 8 if src.type.ptr else src.type.dtype.itemsize
        order = self.lds_order(a, dst, es)
        strides, total = self.lds_addr(a.shape, order, es)
        nbytes = total * es
        if nbytes > MAX_LDS:
            raise CompilationError(f"a layout conversion of a {a.shape} tile needs {nbytes} "
                                   "bytes of LDS")
        self.need_lds(nbytes)
        op = getattr(self, "cur_op", None)
        self.report.setdefault("conversions", []).append(
            {"value": src, "loc": op.loc if op is not None else None, "bytes": int(nbytes),
             "src": a, "dst": dst})
        nm = self.fresh("cv")
        sname = self.name[src.id]
        lines = []
        wv = self.lds_vec(a, order, es)
        rv = self.lds_vec(dst, order, es)
        lines.append(f"{t} {nm}[{dst.nregs}];")
        lines.append("{")
        lines.append(f"  {t}* sm = reinterpret_cast<{t}*>(ek_smem);")
        lines.append("  __syncthreads();")
        lines.append("  #pragma unroll")
        lines.append(f"  for (int r = 0; r < {a.nregs}; r += {wv}) "
                     f"ek::vstore<{t}, {wv}>(&sm[{self.lds_index(a, strides, 'r')}], &{sname}[r]);")
        lines.append("  __syncthreads();")
        lines.append("  #pragma unroll")
        lines.append(f"  for (int r = 0; r < {dst.nregs}; r += {rv}) "
                     f"ek::vload<{t}, {rv}>(&{nm}[r], &sm[{self.lds_index(dst, strides, 'r')}]);")
        lines.append("}")
        self._emit_at_level(lvl, lines)
        self.scopes[lvl].memo[key] = nm
        return nm

    def _emit_at_level(self, lvl: int, lines: list[str]):
        if lvl >= len(self.scopes) - 1:
            for ln in lines:
                self.emit(ln)
            return
        target = self.scopes[lvl + 1].hoist
        ind = self.scopes[lvl].indent
        for ln in lines:
            target.append(ind + ln)

    # ------------------------------------------------------------------ scopes
    def push_scope(self, header: str):
        parent = self.cur
        hoist: list[str] = []
        parent.items.append(hoist)
        parent.items.append(parent.indent + header)
        s = Scope(parent.level + 1, hoist=hoist, indent=parent.indent + "  ")
        self.scopes.append(s)
        return s

    def pop_scope(self, footer: str = "}"):
        s = self.scopes.pop()
        self.cur.items.append(s.items)
        self.emit(footer)

    def define(self, v: ir.Value, name: str):
        self.name[v.id] = name
        self.def_level[v.id] = len(self.scopes) - 1

    # ------------------------------------------------------------------ ops
    def gen_block(self, block: ir.Block, ops=None):
        for op in (block.ops if ops is None else ops):
            sp = getattr(self, "split_next", None)
            if sp is not None and sp.get("at") is op:
                self._split_barrier(sp)
            self.gen_op(op)

    def _split_barrier(self, sp):
        """Split stages: every wave is done reading the first dot's stage and this wave's
        copies of the second dot's operand have landed; after the barrier everyone's have,
        and the first dot's operand for the next iteration can be copied under the second
        dot."""
        self.emit('asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\\n\\ts_barrier" ::: '
                  '"memory");')
        su, ch = sp["parts"]
        self.deferred_dma = {"lines": ["{"] + ["  " + ln for ln in su + ch] + ["}"],
                             "setup": su, "chunks": ch, "used": False, "scope": self.cur}
        self.split_next = None

    def gen_op(self, op: ir.Op):
        prev = getattr(self, "cur_op", None)
        self.cur_op = op
        try:
            self._gen_op(op)
        finally:
            self.cur_op = prev

    def _gen_op(self, op: ir.Op):
        n = op.name
        fn = getattr(self, f"op_{n}", None)
        if n in ("yield",):
            return
        if fn is not None:
            fn(op)
            return
        if n in ("binary", "unary", "cast", "select", "fma", "ptr_add", "bitcast"):
            self.op_elementwise(op)
            return
        if n in ("const", "arange", "splat", "broadcast", "expand_dims", "trans", "hint",
                 "reshape"):
            res = op.result
            k = self.kind.get(res.id)
            if k == "scalar":
                self.op_elementwise(op)
            self.def_level[res.id] = len(self.scopes) - 1
            return
        raise CompilationError(f"the HIP backend doesn't lower `{n}`")

    def scalar_expr(self, op: ir.Op) -> str:
        n = op.name
        if n == "const":
            return literal(op.attrs["value"], op.result.type.dtype)
        if n == "hint":
            return self.name[op.operands[0].id]
        xs = [self.name[o.id] for o in op.operands]
        return self.ew(op, xs)

    def op_elementwise(self, op: ir.Op):
        res = op.result
        k = self.kind[res.id]
        t = ctype(res.type.dtype) + ("*" if res.type.ptr else "")
        if k == "scalar":
            nm = self.fresh("s")
            self.emit(f"{t} const {nm} = {self.scalar_expr(op)};")
            self.define(res, nm)
            return
        if k in ("cheap", "fused"):
            self.def_level[res.id] = len(self.scopes) - 1
            return
        lay = self.lay[res.id]
        nm = self.fresh("t")
        rs = self._rescale(res, lay)
        if rs is not None:
            # acc * scale[:, None]: a wave whose factors are all exactly 1 skips the multiply
            # (x * 1 == x), the common case in online softmax once the row maxima settle
            ea, es = self.elem(rs[0], lay, "r"), self.elem(rs[1], lay, "r")
            self.emit(f"float {nm}[{lay.nregs}];")
            self.emit("{")
            self.emit("  bool ek_any = false;")
            self.emit("  #pragma unroll")
            self.emit(f"  for (int r = 0; r < {lay.nregs}; ++r) {{ {nm}[r] = {ea}; "
                      f"ek_any |= ({es} != 1.0f); }}")
            self.emit("  if (__builtin_amdgcn_ballot_w64(ek_any) != 0) {")
            self.emit("    #pragma unroll")
            self.emit(f"    for (int r = 0; r < {lay.nregs}; ++r) {nm}[r] *= {es};")
            self.emit("  }")
            self.emit("}")
            self.define(res, nm)
            return
        xs = [self.elem(o, lay, "r") if self.tile(o) else self.name[o.id] for o in op.operands]
        cond = None
        if op.name == "select" and self.tile(op.operands[0]) and \
                not self.opt.get("no_edge_versioning"):
            cond = self.all_true(op.operands[0])
        self.emit(f"{t} {nm}[{lay.nregs}];")
        if cond and self._assume(cond):
            self.emit("#pragma unroll")
            self.emit(f"for (int r = 0; r < {lay.nregs}; ++r) {nm}[r] = {xs[1]};")
            self.define(res, nm)
            return
        if cond and self._edge_copy():
            cond = None
        if cond:
            # Edge versioning: a uniform branch skips the per-element mask when the whole
            # tile is provably selected (interior blocks of a masked loop).
            self.emit(f"if ({cond}) {{")
            self.emit("  #pragma unroll")
            self.emit(f"  for (int r = 0; r < {lay.nregs}; ++r) {nm}[r] = {xs[1]};")
            self.emit("} else {")
            self.emit("  #pragma unroll")
            self.emit(f"  for (int r = 0; r < {lay.nregs}; ++r) {nm}[r] = {self.ew(op, xs)};")
            self.emit("}")
        else:
            self.emit("#pragma unroll")
            self.emit(f"for (int r = 0; r < {lay.nregs}; ++r) {nm}[r] = {self.ew(op, xs)};")
        self.define(res, nm)

    def op_program_id(self, op):
        nm = self.fresh("pid")
        ax = "xyz"[op.attrs["axis"]]
        src = f"ek_pid_{ax}" if (self.remap_pids or self.coarsen) else \
            f"(int32_t)blockIdx.{ax}"
        self.emit(f"const int32_t {nm} = {src};")
        self.define(op.result, nm)

    def op_num_programs(self, op):
        nm = self.fresh("np")
        ax = "xyz"[op.attrs["axis"]]
        src = f"ek_np_{ax}" if self.coarsen else f"(int32_t)gridDim.{ax}"
        self.emit(f"const int32_t {nm} = {src};")
        self.define(op.result, nm)

    def op_barrier(self, op):
        self.emit("__syncthreads();")

    # -- debugging (reference: codegen/debug.py:84-158) ------------------------------------
    def _pid3(self) -> str:
        if self.remap_pids or self.coarsen:
            return "ek_pid_x, ek_pid_y, ek_pid_z"
        return "(int)blockIdx.x, (int)blockIdx.y, (int)blockIdx.z"

    def _debug_layout(self, vals) -> LY.Layout:
        for v in vals:
            if self.tile(v) and v.id in self.lay and self.kind.get(v.id) == "anchored":
                return self.lay[v.id]
        return self.default_layout(vals[0])

    def op_assert(self, op):
        """Records the first failing program in the error buffer `ek_assert_buf` (a kernel
        argument after the runtime ones): flag, assert index, program id."""
        idx = len(self.asserts)
        self.asserts.append({"msg": op.attrs["msg"], "loc": op.loc})
        cond = op.operands[0]
        mask = op.operands[1] if len(op.operands) > 1 else None
        call = f"ek::assert_fail(ek_assert_buf, {idx}, {self._pid3()});"
        if not self.tile(cond):
            c = self.name[cond.id]
            if mask is not None:
                c = f"({c}) || !({self.name[mask.id]})"
            self.emit(f"if (!({c})) {call}")
            return
        lay = self._debug_layout([cond] + ([mask] if mask is not None else []))
        self.prime(*[(v, lay) for v in op.operands])
        e = self.elem(cond, lay, "r")
        m = self.elem(mask, lay, "r") if mask is not None else None
        ok = self.fresh("aok")
        self.emit(f"bool {ok} = true;")
        self.emit("#pragma unroll")
        test = f"({e})" if m is None else f"(({e}) || !({m}))"
        self.emit(f"for (int r = 0; r < {lay.nregs}; ++r) {ok} = {ok} && {test};")
        self.emit(f"if (!{ok}) {call}")

    _PRINTF = {"i1": ("%d", "int"), "i8": ("%d", "int"), "i16": ("%d", "int"),
               "i32": ("%d", "int"), "u8": ("%u", "unsigned"), "u16": ("%u", "unsigned"),
               "u32": ("%u", "unsigned"), "i64": ("%lld", "long long"),
               "u64": ("%llu", "unsigned long long"), "fp16": ("%f", "double"),
               "bf16": ("%f", "double"), "fp32": ("%f", "double"), "fp64": ("%f", "double")}

    def op_print(self, op):
        """printf, one line per element this thread owns (broadcast copies stay silent):
        `pid (x, y, z) idx (i, ...) prefix values`."""
        pre = op.attrs["prefix"].rstrip()
        if pre:
            pre = pre + " " if pre.endswith(":") else pre + ": "
        pre = pre.replace("\\", "\\\\").replace('"', '\\"').replace("%", "%%")
        convs = []
        for v in op.operands:
            c, cast = self._PRINTF[v.type.dtype.name]
            if op.attrs.get("hex") and not v.type.dtype.is_floating():
                c = "0x%llx" if v.type.dtype.itemsize == 8 else "0x%x"
            convs.append((c, cast))
        fmtv = " ".join(c for c, _ in convs)
        vals = list(op.operands)
        if not vals or not self.tile(vals[0]) or not vals[0].type.shape:
            exprs = []
            for v, (_, cast) in zip(vals, convs):
                if self.tile(v):
                    lay = self._debug_layout([v])
                    self.prime((v, lay))
                    x = self.elem(v, lay, "0")
                else:
                    x = self.name[v.id]
                exprs.append(f"({cast})(ek::f32_or_self({x}))")
            fmt = f"pid (%d, %d, %d) {pre}{fmtv}".rstrip()
            args = ", ".join([self._pid3()] + exprs)
            self.emit(f'if (ek_tid == 0) printf("{fmt}\\n", {args});')
            return
        lay = self._debug_layout(vals)
        self.prime(*[(v, lay) for v in vals])
        rank = len(lay.shape)
        own = self.owner_cond(lay)
        fmt = (f"pid (%d, %d, %d) idx ({', '.join(['%d'] * rank)}) {pre}{fmtv}").rstrip()
        if own:
            self.emit(f"if ({own}) {{")
        self.emit(f"for (int r = 0; r < {lay.nregs}; ++r) {{")
        coords = [self.coord(lay, d, "r") for d in range(rank)]
        exprs = [f"({cast})(ek::f32_or_self({self.elem(v, lay, 'r')}))"
                 for v, (_, cast) in zip(vals, convs)]
        args = ", ".join([self._pid3()] + [f"(int)({c})" for c in coords] + exprs)
        self.emit(f'  printf("{fmt}\\n", {args});')
        self.emit("}")
        if own:
            self.emit("}")

    # -- memory ----------------------------------------------------------------------
    def op_load(self, op):
        res = op.result
        ptr = op.operands[0]
        t = ctype(res.type.dtype)
        if not self.tile(res):
            nm = self.fresh("s")
            p = self.name[ptr.id]
            if len(op.operands) > 1:
                m, o = self.name[op.operands[1].id], self.name[op.operands[2].id]
                self.emit(f"const {t} {nm} = {m} ? *{p} : {o};")
            else:
                self.emit(f"const {t} {nm} = *{p};")
            self.define(res, nm)
            return
        lay = self.lay[res.id]
        V = self.mem_vec(ptr, lay)
        self.prime(*[(o, lay) for o in op.operands])
        nm = self.fresh("ld")
        self.emit(f"{t} {nm}[{lay.nregs}];")
        hdr = f"for (int rv = 0; rv < {lay.nregs}; rv += {V}) {{"
        pe = lambda i: self.elem(ptr, lay, f"rv + {i}" if i else "rv")  # noqa: E731
        ld = "vload_nt" if self._streaming_load(op) else "vload"

        def plain():
            self.emit("#pragma unroll")
            self.emit(hdr)
            self.emit(f"  ek::{ld}<{t}, {V}>(&{nm}[rv], {pe(0)});")
            self.emit("}")
        if len(op.operands) == 1:
            plain()
            self.define(res, nm)
            return
        mask, other = op.operands[1], op.operands[2]
        # Edge versioning: a mask that is provably all-true over a uniform runtime interval
        # (e.g. offs < n away from the last program) gets a branch-free unmasked path.
        cond = None if self.opt.get("no_edge_versioning") else self.all_true(mask)
        if cond and self._assume(cond):
            if ld == "vload_nt" and not self.opt.get("no_serial_streams"):
                # One streaming tile load in flight per wave: waiting for the previous one
                # before issuing the next measured +1.5% on vector add (two 1 GiB inputs).
                if self.fast_streams:
                    self.emit("__builtin_amdgcn_s_waitcnt(0x0F70);")
                self.fast_streams += 1
            plain()
            self.define(res, nm)
            return
        if cond and self._edge_copy():
            cond = None
        if cond:
            self.emit(f"if ({cond}) {{")
            plain()
            self.emit("} else {")
        me = lambda i: self.elem(mask, lay, f"rv + {i}" if i else "rv")  # noqa: E731
        oe = lambda i: self.elem(other, lay, f"rv + {i}" if i else "rv")  # noqa: E731
        self.emit("#pragma unroll")
        self.emit(hdr)
        if V > 1:
            allm = " && ".join(f"({me(i)})" for i in range(V))
            self.emit(f"  if ({allm}) {{ ek::{ld}<{t}, {V}>(&{nm}[rv], {pe(0)}); }}")
            self.emit("  else {")
            for i in range(V):
                self.emit(f"    {nm}[rv + {i}] = ({me(i)}) ? *({pe(i)}) : {oe(i)};")
            self.emit("  }")
        else:
            self.emit(f"  {nm}[rv] = ({me(0)}) ? *({pe(0)}) : {oe(0)};")
        self.emit("}")
        if cond:
            self.emit("}")
        self.define(res, nm)

    def _depends_on_pid(self, v: ir.Value, depth=0) -> bool:
        if v.op is None or depth > 48:
            return False
        if v.op.name == "program_id":
            return True
        return any(self._depends_on_pid(o, depth + 1) for o in v.op.operands)

    def _streaming_load(self, op) -> bool:
        """Non-temporal loads for large per-program tiles whose addresses move with the
        program id (each program streams its own rows once). Measured on MI355X: +7% on
        the [4096, 8192] row kernels; small tiles and shared operands keep cached loads."""
        if self.opt.get("nt_loads"):
            return True
        if self.opt.get("no_nt_loads"):
            return False
        ptr = op.operands[0]
        if op.result.type.numel >= 4096 and self._depends_on_pid(ptr):
            return True
        return self._disjoint_stream(ptr)

    def _pid_stride(self, v: ir.Value, depth=0):
        """C when scalar `v` is `program_id * C` plus terms that don't depend on the
        program id; None otherwise."""
        op = v.op
        if op is None or depth > 16:
            return None
        if op.name in ("cast", "hint"):
            return self._pid_stride(op.operands[0], depth + 1)
        if op.name != "binary":
            return None
        k = op.attrs["op"]
        a, b = op.operands
        if k == "mul":
            for x, y in ((a, b), (b, a)):
                if x.op is not None and x.op.name == "program_id" and y.op is not None and \
                        y.op.name == "const":
                    return int(y.op.attrs["value"])
            return None
        if k in ("add", "sub"):
            for x, y in ((a, b), (b, a)):
                c = self._pid_stride(x, depth + 1)
                if c is not None and not self._depends_on_pid(y):
                    return c
        return None

    def _disjoint_stream(self, ptr: ir.Value) -> bool:
        """A 1-D contiguous tile at `base + program_id * C + arange(n)` with C >= n: each
        program reads its own bytes once (vector add, histogram inputs), so the load can
        bypass the caches. Measured on MI355X: +2% on the n = 2^28 vector add."""
        t = ptr.type
        if len(t.shape) != 1 or ptr.op is None or ptr.op.name != "ptr_add":
            return False
        if len(self.pid_axes) != 1:
            return False        # with a 2-D grid, programs along the other axis share tiles
        n = t.shape[0]
        if self.axis.get(ptr).contig[0] < n:
            return False
        base, off = ptr.op.operands
        if self._depends_on_pid(base) or off.op is None or off.op.name != "binary" or \
                off.op.attrs["op"] != "add":
            return False
        for x, y in (off.op.operands, off.op.operands[::-1]):
            while x.op is not None and x.op.name in ("splat", "broadcast", "expand_dims"):
                x = x.op.operands[0]
            c = self._pid_stride(x) if not x.type.shape else None
            if c is not None and c >= n and not self._depends_on_pid(y):
                return True
        return False

    def op_store(self, op):
        ptr, val = op.operands[0], op.operands[1]
        mask = op.operands[2] if len(op.operands) > 2 else None
        t = ctype(val.type.dtype)
        if not self.tile(ptr):
            cond = "ek_tid == 0" + (f" && {self.name[mask.id]}" if mask is not None else "")
            self.emit(f"if ({cond}) *{self.name[ptr.id]} = {self.name[val.id]};")
            self.fast_side = True
            return
        lay = self.mem_layout(ptr)
        if self._anch(val) and self.kind[val.id] in ("anchored", "fused"):
            vl = self.lay[val.id]
            want = self.mem_vec(ptr, lay)
            # keep the value where it is when that stores as wide a vector, or when each
            # store instruction still writes one contiguous 256-byte run per wave: either
            # beats a round trip through LDS
            if vl.shape == lay.shape and (self.mem_vec(ptr, vl) >= want or
                                          self.wave_run_bytes(ptr, vl) >= 256):
                lay = vl
        V = self.mem_vec(ptr, lay)
        own = self.owner_cond(lay)
        self.prime((ptr, lay), (mask, lay), (val, lay))
        pe = lambda i: self.elem(ptr, lay, f"rv + {i}" if i else "rv")  # noqa: E731
        if self.kind.get(val.id) == "fused":
            # computed per vector inside each store loop: `vals` names the vector's
            # temporary, indexed from the vector's first element
            vals, base = self.fresh("sv"), "0"

            def open_vec():
                self.emit(f"  {t} {vals}[{V}];")
                for i in range(V):
                    self.emit(f"  {vals}[{i}] = "
                              f"{self.elem(val, lay, f'rv + {i}' if i else 'rv')};")
        else:
            vals, base = self.array(val, lay), "rv"

            def open_vec():
                pass
        at = lambda i: f"{vals}[{base} + {i}]" if i else f"{vals}[{base}]"  # noqa: E731
        if own:
            self.emit(f"if ({own}) {{")
        st = "vstore" if self.opt.get("no_nt_stores") else "vstore_nt"
        cond = None
        if mask is not None and not self.opt.get("no_edge_versioning"):
            cond = self.all_true(mask)
        if cond and self._assume(cond):
            self._vec_loop(lay.nregs, V)
            open_vec()
            self.emit(f"  ek::{st}<{t}, {V}>({pe(0)}, &{at(0)});")
            self.emit("}")
            if own:
                self.emit("}")
            self.fast_side = True
            return
        if cond and self._edge_copy():
            cond = None
        if cond:
            # edge versioning, as for loads
            self.emit(f"if ({cond}) {{")
            self._vec_loop(lay.nregs, V)
            open_vec()
            self.emit(f"  ek::{st}<{t}, {V}>({pe(0)}, &{at(0)});")
            self.emit("}")
            self.emit("} else {")
        self._vec_loop(lay.nregs, V)
        open_vec()
        if mask is None:
            self.emit(f"  ek::{st}<{t}, {V}>({pe(0)}, &{at(0)});")
        else:
            me = lambda i: self.elem(mask, lay, f"rv + {i}" if i else "rv")  # noqa: E731
            if V > 1:
                allm = " && ".join(f"({me(i)})" for i in range(V))
                self.emit(f"  if ({allm}) {{ ek::{st}<{t}, {V}>({pe(0)}, &{at(0)}); }}")
                self.emit("  else {")
                for i in range(V):
                    self.emit(f"    if ({me(i)}) *({pe(i)}) = {at(i)};")
                self.emit("  }")
            else:
                self.emit(f"  if ({me(0)}) *({pe(0)}) = {at(0)};")
        self.emit("}")
        if cond:
            self.emit("}")
        if own:
            self.emit("}")
        self.fast_side = True

    def op_make_desc(self, op):
        base = op.operands[0]
        vals = [self.name[o.id] for o in op.operands[1:]]
        rank = op.result.type.rank
        info = {"base": self.name[base.id], "shape": vals[:rank], "strides": vals[rank:],
                "base_v": base, "shape_v": op.operands[1:1 + rank],
                "stride_v": op.operands[1 + rank:]}
        self.desc[op.result.id] = info
        self.def_level[op.result.id] = len(self.scopes) - 1

    def _desc_vec(self, d: dict, offs: list[ir.Value], lay: LY.Layout, es: int) -> int:
        """Vector width for a descriptor block access in `lay` (contiguous last dim)."""
        dvec, nb = lay.vec_dim_bits()
        rank = len(lay.shape)
        if dvec != rank - 1 or nb == 0:
            return 1
        v = min(1 << nb, max(1, 16 // es))
        align = self.axis.get(d["base_v"]).div[0]
        for o in offs[-1:]:
            align = math.gcd(align, self.axis.get(o).div[0] * es)
        for s in d["stride_v"][:-1]:
            align = math.gcd(align, self.axis.get(s).div[0] * es)
        v = min(v, max(1, align // es))
        return 1 << LY.log2(max(1, v))

    def _desc_addr(self, d, offs, lay, r):
        rank = len(lay.shape)
        idx = []
        conds = []
        for k in range(rank):
            c = f"({self.name[offs[k].id]} + {self.coord(lay, k, r)})"
            conds.append(f"((unsigned){c} < (unsigned){d['shape'][k]})")
            idx.append(c if k == rank - 1 else f"{c} * {d['strides'][k]}")
        return " + ".join(idx), " && ".join(conds)

    def op_desc_load(self, op):
        if op.result.id in getattr(self, "staged", {}):
            self.def_level[op.result.id] = len(self.scopes) - 1
            return
        desc, offs = op.operands[0], op.operands[1:]
        d = self.desc[desc.id]
        res = op.result
        lay = self.lay[res.id]
        t = ctype(res.type.dtype)
        es = res.type.dtype.itemsize
        V = self._desc_vec(d, offs, lay, es)
        nm = self.fresh("dl")
        self.emit(f"{t} {nm}[{lay.nregs}];")
        self._vec_loop(lay.nregs, V)
        addr, cond = self._desc_addr(d, offs, lay, "rv")
        zero = literal(0, res.type.dtype)
        if V > 1:
            _, cond_last = self._desc_addr(d, offs, lay, f"rv + {V - 1}")
            self.emit(f"  if ({cond} && {cond_last}) {{ ek::vload<{t}, {V}>(&{nm}[rv], "
                      f"{d['base']} + {addr}); }}")
            self.emit("  else {")
            for i in range(V):
                a_i, c_i = self._desc_addr(d, offs, lay, f"rv + {i}")
                self.emit(f"    {nm}[rv + {i}] = ({c_i}) ? {d['base']}[{a_i}] : {zero};")
            self.emit("  }")
        else:
            self.emit(f"  {nm}[rv] = ({cond}) ? {d['base']}[{addr}] : {zero};")
        self.emit("}")
        self.define(res, nm)

    def op_desc_store(self, op):
        desc, offs, val = op.operands[0], op.operands[1:-1], op.operands[-1]
        d = self.desc[desc.id]
        t = ctype(val.type.dtype)
        es = val.type.dtype.itemsize
        lay = LY.blocked(val.type.shape, LY.default_order(val.type.shape), max(1, 16 // es),
                         self.nw)
        V = self._desc_vec(d, offs, lay, es)
        vals = self.array(val, lay)
        self._vec_loop(lay.nregs, V)
        addr, cond = self._desc_addr(d, offs, lay, "rv")
        if V > 1:
            _, cond_last = self._desc_addr(d, offs, lay, f"rv + {V - 1}")
            self.emit(f"  if ({cond} && {cond_last}) {{ ek::vstore_nt<{t}, {V}>({d['base']} + "
                      f"{addr}, &{vals}[rv]); }}")
            self.emit("  else {")
            for i in range(V):
                a_i, c_i = self._desc_addr(d, offs, lay, f"rv + {i}")
                self.emit(f"    if ({c_i}) {d['base']}[{a_i}] = {vals}[rv + {i}];")
            self.emit("  }")
        else:
            self.emit(f"  if ({cond}) {d['base']}[{addr}] = {vals}[rv];")
        self.emit("}")

    # -- interval analysis for edge versioning --------------------------------------------
    def interval(self, v: ir.Value, depth=0):
        """(lo, hi) C++ expressions bounding every element of an integer tile built from
        aranges, splats, constants, + and -, and x constant; None when unknown."""
        if depth > 32:
            return None
        k = self.kind.get(v.id)
        if k == "scalar" and not isinstance(v.type, ir.DescType) and v.type.dtype.is_int() \
                and not v.type.ptr and v.id in self.name:
            nm = self.name[v.id]
            return (nm, nm)
        op = v.op
        if op is None or v.type.ptr or not v.type.dtype.is_int() or v.type.dtype.is_bool():
            return None
        n = op.name
        if n == "const":
            x = str(int(op.attrs["value"]))
            return (x, x)
        if n == "arange":
            st = op.attrs["start"]
            return (str(st), str(st + v.type.shape[0] - 1))
        if n in ("splat", "broadcast", "expand_dims", "hint"):
            return self.interval(op.operands[0], depth + 1)
        if n == "cast":
            # a widening integer cast (64-bit index math) keeps the bounds; the bound
            # expressions are evaluated in the wider type
            x = op.operands[0]
            if x.type.ptr or not x.type.dtype.is_int() or x.type.dtype.is_bool() or \
                    x.type.dtype.primitive_bitwidth > v.type.dtype.primitive_bitwidth or \
                    (x.type.dtype.kind == "uint") != (v.type.dtype.kind == "uint"):
                return None
            a = self.interval(x, depth + 1)
            if a is None:
                return None
            t = ctype(v.type.dtype)
            return (f"(({t})({a[0]}))", f"(({t})({a[1]}))")
        if n == "binary" and op.attrs["op"] in ("add", "sub", "mul"):
            a = self.interval(op.operands[0], depth + 1)
            b = self.interval(op.operands[1], depth + 1)
            if a is None or b is None:
                return None
            kk = op.attrs["op"]
            if kk == "add":
                return (f"({a[0]} + {b[0]})", f"({a[1]} + {b[1]})")
            if kk == "sub":
                return (f"({a[0]} - {b[1]})", f"({a[1]} - {b[0]})")
            for x, y in ((a, b), (b, a)):
                if x[0] == x[1] and x[0].lstrip("-").isdigit() and int(x[0]) >= 0:
                    return (f"({y[0]} * {x[0]})", f"({y[1]} * {x[0]})")
            if a[0] == a[1] and b[0] == b[1]:
                return (f"({a[0]} * {b[0]})", f"({a[0]} * {b[0]})")
        return None

    def _assume(self, cond: str) -> bool:
        """In the fast copy of a versioned program, at the top level: True when the uniform
        condition `cond` may be assumed. The first time a condition appears, the rest of the
        fast copy opens under `if (cond)`, so that a failing guard falls through to the
        general copy; a new condition after a store cannot be guarded (the store would run
        twice), and the fast copy is then abandoned."""
        if not self.fast_mode or self.cur is not self.scopes[0]:
            return False
        if cond not in self.fast_conds:
            if self.fast_side:
                self.fast_failed = True
                return False
            # the rest of the fast copy nests under the guard (structured control flow;
            # a guard that fails falls through to the general copy)
            self.emit(f"if (__builtin_expect(({cond}), 1)) {{")
            self.fast_conds.append(cond)
        return True

    def _vec_loop(self, n: int, V: int):
        """Opens the loop over a thread's vectors (`rv`, closed by the caller's "}"). One
        vector is a plain block: LLVM dropped the non-temporal hint of the store in a
        single-iteration loop of this shape."""
        if n == V:
            self.emit("{ const int rv = 0;")
        else:
            self.emit("#pragma unroll")
            self.emit(f"for (int rv = 0; rv < {n}; rv += {V}) {{")

    def _edge_copy(self) -> bool:
        """In the general copy of a versioned program, at the top level: the copy runs only
        when a guard failed, so its per-access fast paths are left out (the masked paths are
        correct everywhere); this also keeps its stores from merging with the fast copy's."""
        return self.edge_only and self.cur is self.scopes[0]

    def _can_version(self, fn) -> bool:
        """Program versioning applies to straight-line programs of loads, pure tile ops and
        stores (no loops, branches, atomics, dots or debug ops) that are not coarsened."""
        if self.opt.get("no_edge_versioning") or self.opt.get("no_program_versioning") or \
                self.coarsen or self.priv or self.asserts:
            return False
        for op in fn.body.ops:
            if op.regions or op.name in ("dot", "atomic_rmw", "atomic_cas", "assert", "print",
                                         "barrier", "desc_store"):
                return False
        return True

    def all_true(self, m: ir.Value, depth=0):
        """A uniform C++ condition under which every element of boolean tile `m` is true."""
        if depth > 32 or m.op is None:
            return None
        op = m.op
        n = op.name
        if n in ("splat", "broadcast", "expand_dims"):
            return self.all_true(op.operands[0], depth + 1)
        if n == "const":
            return "true" if op.attrs["value"] else None
        if n != "binary":
            return None
        k = op.attrs["op"]
        if k == "and":
            a = self.all_true(op.operands[0], depth + 1)
            b = self.all_true(op.operands[1], depth + 1)
            return f"({a} && {b})" if a and b else None
        if k not in ("lt", "le", "gt", "ge"):
            return None
        if op.operands[0].type.dtype.is_floating():
            return None
        a = self.interval(op.operands[0])
        b = self.interval(op.operands[1])
        if a is None or b is None:
            return None
        if k == "lt":
            return f"({a[1]} < {b[0]})"
        if k == "le":
            return f"({a[1]} <= {b[0]})"
        if k == "gt":
            return f"({a[0]} > {b[1]})"
        return f"({a[0]} >= {b[1]})"

    # -- LDS-privatised histograms ----------------------------------------------------
    def _and_terms(self, v: ir.Value, out: list):
        op = v.op
        if op is not None and op.name == "binary" and op.attrs["op"] == "and" and \
                v.type.dtype.is_bool():
            self._and_terms(op.operands[0], out)
            self._and_terms(op.operands[1], out)
        elif op is not None and op.name in ("broadcast", "expand_dims"):
            self._and_terms(op.operands[0], out)
        else:
            out.append(v)

    def _pos_step(self, op: ir.Op) -> bool:
        """Whether a `for` op's step is a compile-time positive constant (the loop then
        counts up with `iv < hi`; any other step takes the trip-count form)."""
        v = op.operands[2]
        while v.op is not None and v.op.name == "cast":
            v = v.op.operands[0]
        c = self._const_of(v)
        return isinstance(c, int) and not isinstance(c, bool) and c > 0

    def _const_of(self, v: ir.Value):
        while v.op is not None and v.op.name in ("splat", "broadcast", "expand_dims"):
            v = v.op.operands[0]
        if v.op is not None and v.op.name == "const":
            return v.op.attrs["value"]
        return None

    def plan_privatization(self, fn: ir.Func):
        """Finds `tl.atomic_add(base + idx, val, mask=... & (idx >= 0) & (idx < C))` on
        32-bit integers with the result unused, `base` a kernel argument and C a constant
        <= 16384: such bins live in LDS per workgroup and are flushed once at the end."""
        self.priv: dict[int, dict] = {}
        if self.opt.get("no_privatize"):
            return
        args = {a.id for a in fn.args}
        for op in ir.walk(fn.body):
            if op.name != "atomic_rmw" or op.attrs["op"] != "add" or not op.attrs.get("has_mask"):
                continue
            if self.uses.get(op.result.id) or not self.tile(op.result):
                continue
            dt = op.result.type.dtype
            if dt not in (core.int32, core.uint32):
                continue
            ptr, val, mask = op.operands
            p = ptr.op
            if p is None or p.name != "ptr_add":
                continue
            base, idx = p.operands
            while base.op is not None and base.op.name in ("splat", "broadcast"):
                base = base.op.operands[0]
            if base.id not in args:
                continue
            terms = []
            self._and_terms(mask, terms)
            lo_ok = hi = None
            for t in terms:
                o = t.op
                if o is None or o.name != "binary":
                    continue
                a, b = o.operands
                k = o.attrs["op"]
                same = lambda x: x.id == idx.id  # noqa: E731
                if k == "ge" and same(a) and self._const_of(b) == 0:
                    lo_ok = True
                elif k == "le" and same(b) and self._const_of(a) == 0:
                    lo_ok = True
                elif k == "lt" and same(a) and isinstance(self._const_of(b), int):
                    hi = self._const_of(b)
                elif k == "gt" and same(b) and isinstance(self._const_of(a), int):
                    hi = self._const_of(a)
            if lo_ok and hi is not None and 0 < hi <= 16384:
                self.priv[op.result.id] = {"base": base, "bins": hi, "dt": dt,
                                           "name": f"ek_bins{len(self.priv)}"}
        if self.priv:
            # Copies (option `priv_copies`): bin b's copy c sits at word b * C + c and lane
            # l adds into copy l % C. Measured on the 1024-bin histogram, one copy and 8
            # workgroups per CU is fastest: the loop is bound by loads in flight, and extra
            # copies cost occupancy and flush work.
            words = sum(i["bins"] for i in self.priv.values())
            # 32 waves per CU (8 per SIMD) at most: an 8-wave program gets 4 workgroups
            # per CU, all resident at once, rather than 8 of which half would wait for
            # the first half to finish its walk
            wgs = int(self.opt.get("priv_wgs", max(1, min(8, 32 // self.nw))))
            cop = int(self.opt.get("priv_copies", 1))
            self.priv_copies = cop
            self.coarsen = 0 if self.opt.get("no_coarsen") else wgs

    # -- atomics --------------------------------------------------------------------
    def _atomic_call(self, kind: str, t: str, dt: core.dtype, p: str, v: str, cmp=None) -> str:
        """One atomic on element pointer `p`, returning the old value (reference:
        codegen/atomic.py:44-135). 32-bit integer and float add, 32/64-bit integer
        max/min, 32-bit bitwise ops, exchange and integer compare-and-swap are native;
        float max/min (NaN-ignoring, as fmax/fmin), float compare-and-swap (a value compare,
        so -0.0 matches 0.0) and every 8/16-bit element go through `ek::atomic_update`."""
        scope = "__ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT"
        sub = dt.primitive_bitwidth < 32
        fl = dt.is_floating()
        if not sub:
            if kind == "add":
                return f"__hip_atomic_fetch_add({p}, {v}, {scope})"
            if kind in ("and", "or", "xor"):
                return f"__hip_atomic_fetch_{kind}({p}, {v}, {scope})"
            if kind == "xchg":
                return f"__hip_atomic_exchange({p}, {v}, {scope})"
            if kind in ("max", "min") and not fl:
                return f"__hip_atomic_fetch_{kind}({p}, {v}, {scope})"
            if kind == "cas" and not fl:
                return (f"([&]() {{ {t} o = {cmp}; __hip_atomic_compare_exchange_strong({p}, "
                        f"&o, {v}, __ATOMIC_RELAXED, __ATOMIC_RELAXED, "
                        "__HIP_MEMORY_SCOPE_AGENT); return o; })()")
        f32 = (lambda x: f"ek::f32_or_self({x})") if fl else (lambda x: x)
        if kind == "add":
            new = f"({t})(o + {v})"
        elif kind in ("and", "or", "xor"):
            new = f"({t})(o {_INFIX[kind]} {v})"
        elif kind == "xchg":
            new = f"({t})({v})"
        elif kind in ("max", "min") and fl:
            fn = "__builtin_fmaxf" if kind == "max" else "__builtin_fminf"
            new = f"ek::Cvt<{t}>::from({fn}({f32('o')}, {f32(v)}))"
        elif kind in ("max", "min"):
            cmpop = ">" if kind == "max" else "<"
            new = f"(o {cmpop} {v} ? o : ({t})({v}))"
        elif kind == "cas":
            new = f"({f32('o')} == {f32(cmp)} ? ({t})({v}) : o)"
        else:
            raise CompilationError(f"unknown atomic {kind}")
        return f"ek::atomic_update({p}, [&]({t} o) -> {t} {{ return {new}; }})"

    def op_atomic_rmw(self, op):
        self._atomic(op, op.attrs["op"])

    def op_atomic_cas(self, op):
        self._atomic(op, "cas")

    def _atomic(self, op, kind):
        res = op.result
        dt = res.type.dtype
        t = ctype(dt)
        ptr = op.operands[0]
        used = bool(self.uses.get(res.id))
        has_mask = op.attrs.get("has_mask")
        if kind == "cas":
            cmp_v, val_v = op.operands[1], op.operands[2]
            mask = None
        else:
            val_v = op.operands[1]
            cmp_v = None
            mask = op.operands[2] if has_mask else None
        if not self.tile(res):
            nm = self.fresh("s")
            p, v = self.name[ptr.id], self.name[val_v.id]
            c = self.name[cmp_v.id] if cmp_v is not None else None
            m = self.name[mask.id] if mask is not None else "true"
            self.need_lds(8)
            self.emit(f"{t} {nm};")
            self.emit("{")
            self.emit(f"  {t}* sm = reinterpret_cast<{t}*>(ek_smem);")
            self.emit("  __syncthreads();")
            self.emit(f"  if (ek_tid == 0) sm[0] = ({m}) ? {self._atomic_call(kind, t, dt, p, v, c)}"
                      f" : {t}{{}};")
            self.emit("  __syncthreads();")
            self.emit(f"  {nm} = sm[0];")
            self.emit("}")
            self.define(res, nm)
            return
        lay = self.lay[res.id]
        own = self.owner_cond(lay)
        pv = self.priv.get(res.id) if hasattr(self, "priv") else None
        if pv is not None:
            idx = ptr.op.operands[1]
            # Copies of an element replicated over a warp bit sit in whole waves: those
            # waves skip the atomics with a wave-uniform branch. Over a lane bit, and for
            # masked-off elements, a lane adds 0 instead, which keeps the loop one basic
            # block; its dummy address is a bin of its own (its lane number), so the dummy
            # adds of a wave never pile onto one LDS word (all on bin 0 they serialised:
            # an 8-wave launch whose upper four waves were copies ran 3x slower).
            lm = sum(1 << i for i, b in enumerate(lay.lane) if b is None)
            wm = sum(1 << i for i, b in enumerate(lay.warp) if b is None)
            conds = [f"((ek_lane & {lm}) == 0)"] if lm else []
            conds.append(f"({self.elem(mask, lay, 'r')})")
            ie = self.elem(idx, lay, "r")
            ve = self.elem(val_v, lay, "r")
            cop = self.priv_copies
            bins = pv["bins"]
            dummy = "ek_lane" if bins >= 64 else f"(ek_lane % {bins})"
            ie = f"(({' && '.join(conds)}) ? ({ie}) : {dummy})"
            ve = f"(({' && '.join(conds)}) ? ({ve}) : 0)"
            slot = f"{ie} * {cop} + (ek_lane & {cop - 1})" if cop > 1 else ie
            if wm:
                self.emit(f"if ((ek_warp & {wm}) == 0) {{")
            self.emit("#pragma unroll")
            self.emit(f"for (int r = 0; r < {lay.nregs}; ++r) "
                      f"__hip_atomic_fetch_add(&{pv['name']}[{slot}], {ve}, "
                      f"__ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);")
            if wm:
                self.emit("}")
            self.define(res, "ek_unused")
            return
        nm = self.fresh("at")
        p = self.elem(ptr, lay, "r")
        v = self.elem(val_v, lay, "r")
        c = self.elem(cmp_v, lay, "r") if cmp_v is not None else None
        conds = []
        if own:
            conds.append(own)
        if mask is not None:
            conds.append(f"({self.elem(mask, lay, 'r')})")
        self.emit(f"{t} {nm}[{lay.nregs}];")
        self.emit("#pragma unroll")
        self.emit(f"for (int r = 0; r < {lay.nregs}; ++r) {{")
        call = self._atomic_call(kind, t, dt, p, v, c)
        if conds:
            self.emit(f"  {nm}[r] = ({' && '.join(conds)}) ? {call} : {t}{{}};")
        else:
            self.emit(f"  {nm}[r] = {call};")
        self.emit("}")
        if used and own:
            # Replicated elements: only the owner thread ran the atomic, so the old values
            # go through LDS to every thread that holds a copy (reference:
            # codegen/atomic.py:208-231).
            es = dt.itemsize
            order = tuple(reversed(range(len(lay.shape))))
            strides, total = self.lds_addr(lay.shape, order, es)
            self.need_lds(total * es)
            ix = self.lds_index(lay, strides, "r")
            self.emit("{")
            self.emit(f"  {t}* sm = reinterpret_cast<{t}*>(ek_smem);")
            self.emit("  __syncthreads();")
            self.emit("  #pragma unroll")
            self.emit(f"  for (int r = 0; r < {lay.nregs}; ++r) if ({own}) sm[{ix}] = {nm}[r];")
            self.emit("  __syncthreads();")
            self.emit("  #pragma unroll")
            self.emit(f"  for (int r = 0; r < {lay.nregs}; ++r) {nm}[r] = sm[{ix}];")
            self.emit("}")
        self.define(res, nm)

    # -- join / split (reference: language/ops.py:832-902, codegen/msl.py:693-747) --------
    def op_join(self, op):
        res = op.result
        lay = self.lay[res.id]
        base = LY.Layout(op.operands[0].type.shape, tuple(lay.reg[1:]), lay.lane, lay.warp)
        a, b = (self.array(o, base) for o in op.operands)
        nm = self.fresh("jn")
        self.emit(f"{ctype(res.type.dtype)} {nm}[{lay.nregs}];")
        self.emit("#pragma unroll")
        self.emit(f"for (int r = 0; r < {base.nregs}; ++r) {{ {nm}[2 * r] = {a}[r]; "
                  f"{nm}[2 * r + 1] = {b}[r]; }}")
        self.define(res, nm)

    def op_split(self, op):
        x = op.operands[0]
        out = self.lay[op.results[0].id]
        mode, k = self.split_bit[op.results[0].id]
        bit = (len(x.type.shape) - 1, 0)
        t = ctype(x.type.dtype)
        if mode == "lane":
            lane = list(out.lane)
            lane[k] = bit
            xa = self.array(x, LY.Layout(x.type.shape, out.reg, tuple(lane), out.warp))
            for half, r_ in enumerate(op.results):
                src = f"(ek_lane | {1 << k})" if half else f"(ek_lane & ~{1 << k})"
                nm = self.fresh("sp")
                self.emit(f"{t} {nm}[{out.nregs}];")
                self.emit("#pragma unroll")
                self.emit(f"for (int r = 0; r < {out.nregs}; ++r) {nm}[r] = "
                          f"ek::shfl({xa}[r], {src});")
                self.define(r_, nm)
            return
        regs = list(out.reg)
        regs.insert(k, bit)
        xl = LY.Layout(x.type.shape, tuple(regs), out.lane, out.warp)
        xa = self.array(x, xl)
        lo = f"(r & {(1 << k) - 1})" if k else "0"
        for half, r_ in enumerate(op.results):
            nm = self.fresh("sp")
            self.emit(f"{t} {nm}[{out.nregs}];")
            self.emit("#pragma unroll")
            self.emit(f"for (int r = 0; r < {out.nregs}; ++r) {nm}[r] = "
                      f"{xa}[((r >> {k}) << {k + 1}) | ({half} << {k}) | {lo}];")
            self.define(r_, nm)

    # -- shift along an axis (the Hillis-Steele steps of tl.associative_scan) ------------
    def op_shift(self, op):
        """res[..., i, ...] = x[..., i - by, ...] where that is in range, else x itself,
        through one LDS round trip (the tile is written row-major, then read shifted)."""
        x, res = op.operands[0], op.result
        ax, by = op.attrs["axis"], op.attrs["by"]
        lay = self.lay[res.id]
        xa = self.array(x, lay)
        t = ctype(x.type.dtype)
        shp = x.type.shape
        self.need_lds(x.type.numel * max(4, x.type.dtype.itemsize))
        strides, st = [0] * len(shp), 1
        for d in reversed(range(len(shp))):
            strides[d] = st
            st *= shp[d]
        cs = [self.coord(lay, d, "r") for d in range(len(shp))]
        lin = " + ".join(f"({c}) * {strides[d]}" for d, c in enumerate(cs))
        lin_src = " + ".join(f"({c if d != ax else 'c'}) * {strides[d]}"
                             for d, c in enumerate(cs))
        nm = self.fresh("sh")
        self.emit(f"{t} {nm}[{lay.nregs}];")
        self.emit("{")
        self.emit(f"  {t}* sm = reinterpret_cast<{t}*>(ek_smem);")
        self.emit("  __syncthreads();")
        self.emit("  #pragma unroll")
        self.emit(f"  for (int r = 0; r < {lay.nregs}; ++r) sm[{lin}] = {xa}[r];")
        self.emit("  __syncthreads();")
        self.emit("  #pragma unroll")
        self.emit(f"  for (int r = 0; r < {lay.nregs}; ++r) {{")
        self.emit(f"    int c = (int)({cs[ax]}) - ({by});")
        self.emit(f"    {nm}[r] = (c >= 0 && c < {shp[ax]}) ? sm[{lin_src}] : {xa}[r];")
        self.emit("  }")
        self.emit("}")
        self.define(res, nm)

    # -- reductions -------------------------------------------------------------------
    def op_reduce(self, op):
        src, res = op.operands[0], op.result
        ax = op.attrs["axis"]
        kind = op.attrs["kind"]
        dt = src.type.dtype
        sl = self.lay[src.id] if self._anch(src) else self.default_layout(src)
        if self.kind.get(src.id) == "view" or (self._anch(src) and
                                                self.kind.get(src.id) != "anchored"):
            sl = self.lay[src.id]
        arr = self.array(src, sl)
        out = sl.slice(ax)
        acc_t = "float" if is_half(dt) else ctype(dt)
        arg = kind in ("argmax", "argmin")
        comb = {"sum": "ek::Sum", "max": "ek::Max", "min": "ek::Min",
                "argmax": "ek::Max", "argmin": "ek::Min", "first": "ek::First"}[kind]
        if kind == "first" and src.type.shape[ax] != 1:
            raise CompilationError("internal: reduce kind `first` takes a size-1 axis")
        axis_reg = [i for i, b in enumerate(sl.reg) if b[0] == ax]
        keep_reg = [i for i, b in enumerate(sl.reg) if b[0] != ax]
        ro_n = 1 << len(keep_reg)
        ra_n = 1 << len(axis_reg)
        nm = self.fresh("rd")
        rt = ctype(res.type.dtype)
        cvt_in = (lambda x: f"ek::f32({x})") if is_half(dt) else (lambda x: x)
        idx_in = lambda ro, ra: " | ".join(  # noqa: E731
            [bits_expr(ro, [(t, i) for t, i in enumerate(keep_reg)]),
             bits_expr(ra, [(t, i) for t, i in enumerate(axis_reg)])])
        self.emit(f"{acc_t} {nm}_v[{ro_n}];")
        if arg:
            self.emit(f"int32_t {nm}_i[{ro_n}];")
        self.emit("#pragma unroll")
        self.emit(f"for (int ro = 0; ro < {ro_n}; ++ro) {{")
        axc = self.coord(sl, ax, idx_in("ro", "ra"))
        first = cvt_in(arr + "[" + idx_in("ro", "0") + "]")
        nxt = cvt_in(arr + "[" + idx_in("ro", "ra") + "]")
        if arg:
            self.emit(f"  {acc_t} bv = {first};")
            self.emit(f"  int32_t bi = {axc.replace('ra', '0')};")
            self.emit("  #pragma unroll")
            self.emit(f"  for (int ra = 1; ra < {ra_n}; ++ra) {{")
            self.emit(f"    {acc_t} cv = {nxt}; int32_t ci = {axc};")
            self.emit(f"    if ({self._arg_better(kind, dt)}) {{ bv = cv; bi = ci; }}")
            self.emit("  }")
            self.emit(f"  {nm}_v[ro] = bv; {nm}_i[ro] = bi;")
        else:
            self.emit(f"  {acc_t} a = {first};")
            self.emit("  #pragma unroll")
            self.emit(f"  for (int ra = 1; ra < {ra_n}; ++ra) a = {comb}::op<{acc_t}>(a, {nxt});")
            self.emit(f"  {nm}_v[ro] = a;")
        self.emit("}")
        # lanes
        for i, b in enumerate(sl.lane):
            if b is None or b[0] != ax:
                continue
            self.emit("#pragma unroll")
            self.emit(f"for (int ro = 0; ro < {ro_n}; ++ro) {{")
            if arg:
                self.emit(f"  {acc_t} cv = ek::shfl_xor<{1 << i}>({nm}_v[ro]);"
                          f" int32_t ci = ek::shfl_xor<{1 << i}>({nm}_i[ro]);")
                self.emit(f"  {acc_t} bv = {nm}_v[ro]; int32_t bi = {nm}_i[ro];")
                self.emit(f"  if ({self._arg_better(kind, dt)}) {{ {nm}_v[ro] = cv; "
                          f"{nm}_i[ro] = ci; }}")
            else:
                self.emit(f"  {nm}_v[ro] = {comb}::op<{acc_t}>({nm}_v[ro], "
                          f"ek::shfl_xor<{1 << i}>({nm}_v[ro]));")
            self.emit("}")
        # warps
        wbits = [i for i, b in enumerate(sl.warp) if b is not None and b[0] == ax]
        if wbits:
            nwa = 1 << len(wbits)
            nout = max(1, res.type.numel)
            esz = 4 if acc_t in ("float", "int32_t", "uint32_t") else 8
            per = nout * (esz + (4 if arg else 0))
            self.need_lds(nwa * per)
            lane_ax = sum(1 << i for i, b in enumerate(sl.lane) if b is not None and b[0] == ax)
            widx = bits_expr("ek_warp", [(w, t) for t, w in enumerate(wbits)])
            outlin = self._lin(out, "ro")
            self.emit("{")
            self.emit(f"  {acc_t}* sm = reinterpret_cast<{acc_t}*>(ek_smem);")
            if arg:
                self.emit(f"  int32_t* si = reinterpret_cast<int32_t*>(ek_smem + {nwa * nout * esz});")
            self.emit("  __syncthreads();")
            self.emit(f"  if ((ek_lane & {lane_ax}) == 0) {{")
            self.emit("    #pragma unroll")
            self.emit(f"    for (int ro = 0; ro < {ro_n}; ++ro) {{ sm[({widx}) * {nout} + {outlin}]"
                      f" = {nm}_v[ro];" + (f" si[({widx}) * {nout} + {outlin}] = {nm}_i[ro];"
                                           if arg else "") + " }")
            self.emit("  }")
            self.emit("  __syncthreads();")
            self.emit("  #pragma unroll")
            self.emit(f"  for (int ro = 0; ro < {ro_n}; ++ro) {{")
            if arg:
                self.emit(f"    {acc_t} bv = sm[{outlin}]; int32_t bi = si[{outlin}];")
                self.emit(f"    for (int w = 1; w < {nwa}; ++w) {{ {acc_t} cv = sm[w * {nout} + "
                          f"{outlin}]; int32_t ci = si[w * {nout} + {outlin}]; "
                          f"if ({self._arg_better(kind, dt)}) {{ bv = cv; bi = ci; }} }}")
                self.emit(f"    {nm}_v[ro] = bv; {nm}_i[ro] = bi;")
            else:
                self.emit(f"    {acc_t} a = sm[{outlin}];")
                self.emit(f"    for (int w = 1; w < {nwa}; ++w) a = {comb}::op<{acc_t}>(a, "
                          f"sm[w * {nout} + {outlin}]);")
                self.emit(f"    {nm}_v[ro] = a;")
            self.emit("  }")
            self.emit("}")
        src_arr = f"{nm}_i" if arg else f"{nm}_v"
        fin = (lambda x: f"ek::rnd<{rt}>({x})") if is_half(res.type.dtype) else (lambda x: x)
        if res.type.shape == ():
            self.emit(f"const {rt} {nm} = {fin(src_arr + '[0]')};")
        else:
            self.emit(f"{rt} {nm}[{ro_n}];")
            self.emit("#pragma unroll")
            self.emit(f"for (int r = 0; r < {ro_n}; ++r) {nm}[r] = {fin(src_arr + '[r]')};")
        self.define(res, nm)

    def _arg_better(self, kind, dt) -> str:
        gt = ">" if kind == "argmax" else "<"
        if dt.is_floating():
            return (f"((cv {gt} bv) || (cv == bv && ci < bi) || (bv != bv && cv == cv) || "
                    f"(bv != bv && cv != cv && ci < bi))")
        return f"((cv {gt} bv) || (cv == bv && ci < bi))"

    def _lin(self, lay: LY.Layout, r: str) -> str:
        if not lay.shape:
            return "0"
        terms = []
        s = 1
        for d in reversed(range(len(lay.shape))):
            terms.append(f"({self.coord(lay, d, r)}) * {s}")
            s *= lay.shape[d]
        return "(" + " + ".join(terms) + ")"

    # -- scans ------------------------------------------------------------------------
    def op_scan(self, op):
        src, res = op.operands[0], op.result
        ax = op.attrs["axis"]
        rev = op.attrs["reverse"]
        lay = self.lay[res.id]
        dt = res.type.dtype
        acc_t = "float" if is_half(dt) else ctype(dt)
        arr = self.array(src, lay)
        nm = self.fresh("sc")
        R = lay.nregs
        k, gpos = LY.scan_groups(lay, ax)
        run = 1 << k
        outer = R // run
        # the axis segment (group) each run of registers belongs to, and the same run's
        # register-run index in another group
        gbits = [g - k for g in gpos]
        gmask = sum(1 << b for b in gbits)
        G = 1 << len(gbits)

        def grp(o):
            return sum(((o >> b) & 1) << j for j, b in enumerate(gbits))

        def in_grp(o, g):
            return (o & ~gmask) | sum(((g >> j) & 1) << b for j, b in enumerate(gbits))
        cin = (lambda x: f"ek::f32({x})") if is_half(dt) else (lambda x: x)
        self.emit(f"{acc_t} {nm}_x[{R}];")
        self.emit("#pragma unroll")
        self.emit(f"for (int r = 0; r < {R}; ++r) {nm}_x[r] = {cin(arr + '[r]')};")
        # phase 1: serial within each run
        self.emit("#pragma unroll")
        self.emit(f"for (int o = 0; o < {outer}; ++o) {{")
        self.emit("  #pragma unroll")
        if not rev:
            self.emit(f"  for (int i = 1; i < {run}; ++i) {nm}_x[o * {run} + i] += "
                      f"{nm}_x[o * {run} + i - 1];")
        else:
            self.emit(f"  for (int i = {run - 2}; i >= 0; --i) {nm}_x[o * {run} + i] += "
                      f"{nm}_x[o * {run} + i + 1];")
        self.emit("}")
        lane_bits = [i for i, b in enumerate(lay.lane) if b is not None and b[0] == ax]
        warp_bits = [i for i, b in enumerate(lay.warp) if b is not None and b[0] == ax]
        last = run - 1 if not rev else 0
        if lane_bits or warp_bits:
            self.emit(f"{acc_t} {nm}_t[{outer}], {nm}_p[{outer}];")
            self.emit("#pragma unroll")
            self.emit(f"for (int o = 0; o < {outer}; ++o) {{ {nm}_t[o] = {nm}_x[o * {run} + "
                      f"{last}]; {nm}_p[o] = {nm}_t[o]; }}")
            low = 0
            dpp = (lane_bits == list(range(6)) and not rev and acc_t in ("int32_t", "uint32_t",
                                                                         "float") and
                   not self.opt.get("no_dpp_scan"))
            if dpp:
                # all 64 lanes walk the axis in order: one DPP prefix sum per run
                self.emit("#pragma unroll")
                self.emit(f"for (int o = 0; o < {outer}; ++o) {nm}_p[o] = "
                          f"ek::wave_prefix_sum<{acc_t}>({nm}_p[o]);")
            for i in ([] if dpp else lane_bits):
                bit = 1 << i
                if not rev:
                    srcl = f"((ek_lane & ~{bit}) | {low})"
                    cond = f"(ek_lane & {bit})"
                else:
                    srcl = f"((ek_lane | {bit}) & ~{low})"
                    cond = f"!(ek_lane & {bit})"
                self.emit("#pragma unroll")
                self.emit(f"for (int o = 0; o < {outer}; ++o) {{ {acc_t} u = ek::shfl({nm}_p[o], "
                          f"{srcl}); if ({cond}) {nm}_p[o] += u; }}")
                low |= bit
            lane_ax = sum(1 << i for i in lane_bits)
            if G > 1:
                # each segment's total over the lanes and warps that hold the axis
                self.emit(f"{acc_t} {nm}_g[{outer}];")
            # warp totals through LDS
            if warp_bits:
                nwa = 1 << len(warp_bits)
                rows = res.type.numel // res.type.shape[ax]
                esz = 8 if acc_t in ("int64_t", "uint64_t") else 4
                self.need_lds(nwa * G * rows * esz)
                widx = bits_expr("ek_warp", [(w, t) for t, w in enumerate(warp_bits)])
                rowc = self._row_lin(lay, ax, f"o * {run}")
                gsel = "0"
                if G > 1:
                    gsel = " | ".join(f"(((o >> {b}) & 1) << {j})" for j, b in enumerate(gbits))
                slot = f"(({{w}}) * {G} + ({gsel})) * {rows} + {rowc}"
                writer = f"(ek_lane & {lane_ax}) == {lane_ax if not rev else 0}"
                self.emit("{")
                self.emit(f"  {acc_t}* sm = reinterpret_cast<{acc_t}*>(ek_smem);")
                self.emit("  __syncthreads();")
                self.emit(f"  if ({writer}) {{")
                self.emit("    #pragma unroll")
                self.emit(f"    for (int o = 0; o < {outer}; ++o) sm[{slot.format(w=widx)}]"
                          f" = {nm}_p[o];")
                self.emit("  }")
                self.emit("  __syncthreads();")
                self.emit(f"  const int ek_wa = {widx};")
                self.emit("  #pragma unroll")
                self.emit(f"  for (int o = 0; o < {outer}; ++o) {{")
                self.emit(f"    {acc_t} s = 0;")
                if not rev:
                    self.emit(f"    for (int w = 0; w < ek_wa; ++w) s += sm[{slot.format(w='w')}];")
                else:
                    self.emit(f"    for (int w = ek_wa + 1; w < {nwa}; ++w) s += "
                              f"sm[{slot.format(w='w')}];")
                if G > 1:
                    self.emit(f"    {acc_t} a = 0;")
                    self.emit(f"    for (int w = 0; w < {nwa}; ++w) a += sm[{slot.format(w='w')}];")
                    self.emit(f"    {nm}_g[o] = a;")
                self.emit(f"    {nm}_p[o] += s;")
                self.emit("  }")
                self.emit("}")
            elif G > 1:
                # one wave holds the axis: its last lane (first, reversed) has the total
                src_l = f"(ek_lane | {lane_ax})" if not rev else f"(ek_lane & ~{lane_ax})"
                self.emit("#pragma unroll")
                self.emit(f"for (int o = 0; o < {outer}; ++o) {nm}_g[o] = "
                          f"ek::shfl({nm}_p[o], {src_l});")
            if G > 1:
                # segment carries: the totals of the segments before this one (after, reversed)
                for o in range(outer):
                    g = grp(o)
                    prev = [in_grp(o, h) for h in (range(g) if not rev else range(g + 1, G))]
                    terms = " + ".join(f"{nm}_g[{q}]" for q in prev) if prev else "0"
                    self.emit(f"{nm}_p[{o}] += {terms};")
            self.emit("#pragma unroll")
            self.emit(f"for (int o = 0; o < {outer}; ++o) {{ {acc_t} e = {nm}_p[o] - {nm}_t[o];")
            self.emit("  #pragma unroll")
            self.emit(f"  for (int i = 0; i < {run}; ++i) {nm}_x[o * {run} + i] += e; }}")
        rt = ctype(dt)
        fin = (lambda x: f"ek::rnd<{rt}>({x})") if is_half(dt) else (lambda x: x)
        self.emit(f"{rt} {nm}[{R}];")
        self.emit("#pragma unroll")
        self.emit(f"for (int r = 0; r < {R}; ++r) {nm}[r] = {fin(nm + '_x[r]')};")
        self.define(res, nm)

    def _row_lin(self, lay: LY.Layout, ax: int, r: str) -> str:
        terms = []
        s = 1
        for d in reversed(range(len(lay.shape))):
            if d == ax:
                continue
            terms.append(f"({self.coord(lay, d, r)}) * {s}")
            s *= lay.shape[d]
        return "(" + " + ".join(terms) + ")" if terms else "0"

    # -- dot --------------------------------------------------------------------------
    def _staged_operand(self, v: ir.Value, lay: LY.Layout):
        """(info, layout over the staged tile) when `v` is a staged tile or a view of one."""
        k = self.kind.get(v.id)
        if k == "staged":
            return self.staged[v.id], lay
        if k == "view":
            src, sl, ri = self.resolve(v, lay, "r")
            if self.kind.get(src.id) == "staged" and ri == "r":
                return self.staged[src.id], sl
        return None

    def _frag_read(self, info, lay: LY.Layout, first: str, n: int, dst: str, decl=True):
        """Emits LDS reads of registers [first, first+n) of `lay` from a staged tile."""
        T = info["T"]
        sm = (f"(reinterpret_cast<const {T}*>({info['smem']}) + (ek_it{info['loop_idx']} % "
              f"{info['nst']}) * {info['stage_elems']})")
        if decl:
            self.emit(f"      {T} {dst}[{n}];")
        if info.get("dma") and info["mode"] == "trans":
            # transpose reads: run (first + j) / 4 of the fragment comes from one instruction
            src = LY.tr16_source(lay)
            assert src is not None and n % 4 == 0, "fragment layout unfit for transpose reads"
            r = f"(({first} + j) >> 2)"
            idx = info["sl"].cexpr(self.coord(src, 0, r), self.coord(src, 1, r))
            self.emit(f"    #pragma unroll")
            self.emit(f"    for (int j = 0; j < {n}; j += 4) ek::tr_read4<{T}>(&{dst}[j], "
                      f"&{sm}[{idx}]);")
            return
        lay_s = self._stage_view(info, lay)
        d, nb = lay_s.vec_dim_bits()
        V = min(1 << nb, 8, n) if d == info["pos_dim"] else 1
        r = f"({first} + j)"
        idx = info["sl"].cexpr(self.coord(lay_s, info["line_dim"], r),
                               self.coord(lay_s, info["pos_dim"], r))
        self.emit(f"    #pragma unroll")
        self.emit(f"    for (int j = 0; j < {n}; j += {V}) ek::vload<{T}, {V}>(&{dst}[j], "
                  f"&{sm}[{idx}]);")

    def _rescale(self, c: ir.Value, lc):
        """(acc, scale) when `c` is `acc * scale` in fp32, with `acc` a register tile in
        layout `lc` (an accumulator) and `scale` a broadcast of a lower-rank tile (one
        factor per row, as in the online-softmax rescale); None otherwise."""
        if self.opt.get("no_rescale_skip") or c.op is None or c.op.name != "binary" or \
                c.op.attrs.get("op") != "mul" or c.type.dtype is not core.float32 or \
                lc.nregs < 16:
            return None
        for a, b in (c.op.operands, c.op.operands[::-1]):
            if self.kind.get(a.id) != "anchored" or self.lay[a.id].key() != lc.key():
                continue
            x = b
            while x.op is not None and x.op.name in ("broadcast", "expand_dims"):
                x = x.op.operands[0]
            if x is not b and len(x.type.shape) < len(c.type.shape) and x.type.numel <= \
                    c.type.shape[0]:
                return a, b
        return None

    def op_dot_int(self, op):
        """A product without MFMA: integer operands other than int8 (uint8, 16- and 32-bit),
        and tiles below the MFMA minimums (an 8x8 tile, K = 8 with 16-bit floats). Both
        operands go to LDS as 32-bit values (int32, or fp32 for floats; A rows padded by one
        word so a wave's different rows hit different banks), then every thread accumulates
        its own outputs over k: integers in unsigned 32-bit arithmetic, so products and sums
        wrap modulo 2^32 as the integer tl.dot defines; floats with fp32 fma, rounded to the
        accumulator's dtype at the end."""
        a, b, c = op.operands
        res = op.result
        lay = self.lay[res.id]
        M, K = a.type.shape
        N = b.type.shape[1]
        pa = K + 1
        self.need_lds((M * pa + K * N) * 4)
        la = self.lay[a.id] if self.kind.get(a.id) == "anchored" else self.default_layout(a)
        lb = self.lay[b.id] if self.kind.get(b.id) == "anchored" else self.default_layout(b)
        xa, xb = self.array(a, la), self.array(b, lb)
        flt = a.type.dtype.is_floating()
        T = "float" if flt else "int32_t"
        cvt = (lambda x: f"ek::f32({x})") if flt else (lambda x: f"(int32_t){x}")
        nm = self.fresh("acc")
        self.emit(f"{T} {nm}[{lay.nregs}];")
        self.emit("#pragma unroll")
        self.emit(f"for (int r = 0; r < {lay.nregs}; ++r) {nm}[r] = "
                  f"{cvt('(' + self.elem(c, lay, 'r') + ')')};")
        mr, nr = self.coord(lay, 0, "r"), self.coord(lay, 1, "r")
        self.emit("{")
        self.emit(f"  {T}* sa = reinterpret_cast<{T}*>(ek_smem);")
        self.emit(f"  {T}* sb = sa + {M * pa};")
        self.emit("  __syncthreads();")
        self.emit("  #pragma unroll")
        self.emit(f"  for (int r = 0; r < {la.nregs}; ++r) sa[({self.coord(la, 0, 'r')}) * "
                  f"{pa} + ({self.coord(la, 1, 'r')})] = {cvt(xa + '[r]')};")
        self.emit("  #pragma unroll")
        self.emit(f"  for (int r = 0; r < {lb.nregs}; ++r) sb[({self.coord(lb, 0, 'r')}) * "
                  f"{N} + ({self.coord(lb, 1, 'r')})] = {cvt(xb + '[r]')};")
        self.emit("  __syncthreads();")
        self.emit(f"  for (int k = 0; k < {K}; ++k) {{")
        self.emit("    #pragma unroll")
        ea, eb = f"sa[({mr}) * {pa} + k]", f"sb[k * {N} + ({nr})]"
        if flt:
            self.emit(f"    for (int r = 0; r < {lay.nregs}; ++r) {nm}[r] = "
                      f"__builtin_fmaf({ea}, {eb}, {nm}[r]);")
        else:
            self.emit(f"    for (int r = 0; r < {lay.nregs}; ++r) {nm}[r] = (int32_t)("
                      f"(uint32_t){nm}[r] + (uint32_t){ea} * (uint32_t){eb});")
        self.emit("  }")
        self.emit("}")
        cdt = res.type.dtype
        if flt and cdt is not core.float32:
            out = self.fresh("acch")
            self.emit(f"{ctype(cdt)} {out}[{lay.nregs}];")
            self.emit(f"for (int r = 0; r < {lay.nregs}; ++r) {out}[r] = ek::rnd<{ctype(cdt)}>"
                      f"({nm}[r]);")
            nm = out
        self.define(res, nm)

    def op_dot(self, op):
        a, b, c = op.operands
        res = op.result
        if res.id in self.int_dots:
            return self.op_dot_int(op)
        plan = self.dot_plans[res.id]
        la, lb = LY.mfma_operand(plan, "a"), LY.mfma_operand(plan, "b")
        lc = self.lay[res.id]
        ins = plan.inst
        self.report.setdefault("dots", []).append(
            {"loc": op.loc, "plan": plan, "staged": [o for o, st in (("a", a), ("b", b))
                                                     if _through_trans(st).id in
                                                     getattr(self, "staged", {})]})
        sa = self._staged_operand(a, la)
        sb = self._staged_operand(b, lb)
        aa = None if sa else self.array(a, la)
        bb = None if sb else self.array(b, lb)
        cdt = res.type.dtype
        nacc = 16 if ins.m == 32 else 4
        single = len(self.uses.get(c.id, [])) == 1
        if cdt in (core.float32, core.int32) and self.kind.get(c.id) == "anchored" and \
                single and self.lay[c.id].key() == lc.key():
            nm = self.name[c.id]
        elif cdt is core.int32:
            nm = self.fresh("acc")
            e = self.elem(c, lc, "r")
            self.emit(f"int32_t {nm}[{lc.nregs}];")
            self.emit("#pragma unroll")
            self.emit(f"for (int r = 0; r < {lc.nregs}; ++r) {nm}[r] = {e};")
        else:
            nm = self.fresh("acc")
            e = self.elem(c, lc, "r")
            self.emit(f"float {nm}[{lc.nregs}];")
            self.emit("#pragma unroll")
            self.emit(f"for (int r = 0; r < {lc.nregs}; ++r) {nm}[r] = ek::f32({e});")
        tm, tn, tk, kpl = plan.tm, plan.tn, plan.tk, ins.kpl
        sp = getattr(self, "split_next", None)
        if sp is not None and sp["scope"] is self.cur and \
                any(x is not None and x[0] is sp["info"] for x in (sa, sb)):
            self._split_barrier(sp)
        dd = getattr(self, "deferred_dma", None)
        copies = {}
        if (sa or sb) and dd is not None and not dd["used"] and tk > 1 and \
                dd["scope"] is self.cur:
            # The loop's stage copies go out from this dot (one the loop body always runs,
            # not one under a branch), spread over its k steps: copy c
            # after the MFMAs of step c * (tk - 1) // n, so each step's copy issue overlaps
            # the MFMAs already queued instead of stalling the wave in one block (the first
            # fragment reads still go out before any copy).
            dd["used"] = True
            if self.opt.get("dma_block"):
                copies = {0: dd["chunks"]}
            else:
                n = len(dd["chunks"])
                for c_, ln in enumerate(dd["chunks"]):
                    copies.setdefault(c_ * (tk - 1) // n, []).append(ln)
            for ln in dd["setup"]:
                self.emit(ln)
        # Per k step: read every A and B fragment first (staged operands come from LDS),
        # then issue the TM x TN MFMAs, so LDS latency overlaps the previous step's MFMAs.
        self.emit("#pragma unroll")
        self.emit(f"for (int kk = 0; kk < {tk}; ++kk) {{")
        if sa:
            T = sa[0]["T"]
            self.emit(f"  {T} fa[{tm}][{kpl}];")
            self.emit("  #pragma unroll")
            self.emit(f"  for (int im = 0; im < {tm}; ++im) {{")
            self._frag_read(sa[0], sa[1], f"(im * {tk} + kk) * {kpl}", kpl, "fa[im]", decl=False)
            self.emit("  }")
            ea = "fa[im]"
        else:
            ea = f"&{aa}[(im * {tk} + kk) * {kpl}]"
        if sb:
            T = sb[0]["T"]
            self.emit(f"  {T} fb[{tn}][{kpl}];")
            self.emit("  #pragma unroll")
            self.emit(f"  for (int in_ = 0; in_ < {tn}; ++in_) {{")
            self._frag_read(sb[0], sb[1], f"(in_ * {tk} + kk) * {kpl}", kpl, "fb[in_]",
                            decl=False)
            self.emit("  }")
            eb = "fb[in_]"
        else:
            eb = f"&{bb}[(in_ * {tk} + kk) * {kpl}]"
        x, y = (eb, ea) if plan.trans else (ea, eb)
        self.emit("  #pragma unroll")
        self.emit(f"  for (int im = 0; im < {tm}; ++im)")
        self.emit("    #pragma unroll")
        self.emit(f"    for (int in_ = 0; in_ < {tn}; ++in_) "
                  f"ek::{ins.fn}(&{nm}[(im * {tn} + in_) * {nacc}], {x}, {y});")
        for k_, lns in sorted(copies.items()):
            self.emit(f"  if (kk == {k_}) {{")
            for ln in lns:
                self.emit("    " + ln)
            self.emit("  }")
        self.emit("}")
        if cdt not in (core.float32, core.int32):
            out = self.fresh("acch")
            self.emit(f"{ctype(cdt)} {out}[{lc.nregs}];")
            self.emit(f"for (int r = 0; r < {lc.nregs}; ++r) {out}[r] = ek::rnd<{ctype(cdt)}>"
                      f"({nm}[r]);")
            nm = out
        self.define(res, nm)

    # -- staged dot operands --------------------------------------------------------------
    def plan_staging(self, block: ir.Block):
        """Marks descriptor loads inside `for` loops that feed a tl.dot operand and whose
        block offsets are the loop variable or loop-invariant. Those tiles go through a
        double-buffered LDS stage: the next iteration's tile is loaded into registers at the
        top of the body, stored to the other stage at the end, one barrier per iteration;
        the dot reads its operand fragments straight from LDS ("row" stages keep the tile's
        contiguous dim; "trans" stages transpose 8x8 blocks in registers on the way in)."""
        if not hasattr(self, "staged"):
            self.staged: dict[int, dict] = {}
            self.stage_loops: dict[int, list] = {}
        for op in block.ops:
            for r in op.regions:
                self.plan_staging(r)
            if op.name != "for" or self.opt.get("no_staging") or not self._pos_step(op):
                continue
            body = op.regions[0]
            iv = body.args[0]
            inner = set()
            for o in ir.walk(body):
                inner.update(r.id for r in o.results)
            inner.update(a.id for a in body.args)
            found = []
            for ld in body.ops:
                if ld.name != "desc_load":
                    continue
                desc, offs = ld.operands[0], ld.operands[1:]
                if desc.id in inner or len(offs) != 2:
                    continue
                kinds = []
                for o in offs:
                    if o.id == iv.id:
                        kinds.append("iv")
                    elif o.id not in inner:
                        kinds.append("inv")
                    elif o.op is not None and o.op.name == "const":
                        kinds.append("const")
                    else:
                        kinds = None
                        break
                if kinds is None:
                    continue
                res = ld.result
                if res.type.dtype.itemsize != 2:
                    continue
                lay = self._operand_layout_for(res)
                if lay is None:
                    continue
                d, nb = lay.vec_dim_bits()
                R, C = res.type.shape
                if d == 1 and nb >= 2:
                    mode = "row"
                elif d == 0 and nb >= 2 and R % 8 == 0 and C % 8 == 0:
                    mode = "trans"
                else:
                    continue
                info = {"op": ld, "lay": lay, "mode": mode, "kinds": kinds, "R": R, "C": C,
                        "loop": op}
                self.staged[res.id] = info
                found.append(info)
            if found:
                self.stage_loops[id(op)] = found

    def _stage_offsets(self, info, kval: str):
        vals = []
        for o, k in zip(info["op"].operands[1:], info["kinds"]):
            if k == "iv":
                vals.append(kval)
            elif k == "const":
                vals.append(str(int(o.op.attrs["value"])))
            else:
                vals.append(self.name[o.id])
        return vals

    @staticmethod
    def _stage_view(info, lay: LY.Layout) -> LY.Layout:
        """`lay` with the staged position dim's bits renamed to their storage bits."""
        pd, sig = info["pos_dim"], info["sl"].sigma
        return lay._map(lambda b: (pd, sig[b[1]]) if b[0] == pd else b, lay.shape)

    def _stage_layout(self, info, W: int, nvec: int, per: int) -> LDS.StageLayout:
        """Picks the LDS layout of a stage by simulating its stores and the dot's fragment
        reads under the bank model of `lds.py`."""
        R, C, lay = info["R"], info["C"], info["lay"]
        row = info["mode"] == "row"
        lines, length = (R, C) if row else (C, R)
        pd, ld_ = (1, 0) if row else (0, 1)
        if row:
            sigma = LDS.identity_sigma(length)
        else:
            lead = []
            for b in lay.reg:
                if b[0] != 0 or len(lead) == 3:
                    break
                lead.append(b[1])
            sigma = LDS.fragment_sigma(length, lead)
        key = (info["mode"], R, C, W, self.nt, lay.key())
        cache = _STAGE_LAYOUTS
        if key in cache:
            return cache[key][0]
        acc = []
        for w in range(self.nt // 64):
            for i in range(per):
                for q in range(1 if row else W):
                    lanes = []
                    for ln in range(64):
                        c = w * 64 + ln + i * self.nt
                        if c >= nvec:
                            lanes.append(None)
                        elif row:
                            lanes.append((c // (C // 8), (c % (C // 8)) * 8))
                        else:
                            lanes.append(((c % (C // W)) * W + q, (c // (C // W)) * 8))
                    acc.append((16, lanes, True))
        probe = LDS.StageLayout(lines, length, length, sigma=sigma)
        lay_s = self._stage_view({"pos_dim": pd, "sl": probe}, lay)
        d, nb = lay_s.vec_dim_bits()
        V = min(1 << nb, 8) if d == pd else 1
        seen = set()
        for w in range(lay_s.num_warps):
            wc = lay_s.thread_coord(0, w)
            if wc in seen:
                continue
            seen.add(wc)
            for j in range(0, lay_s.nregs, V):
                rc = lay_s.reg_coord(j)
                lanes = []
                for ln in range(64):
                    tc = lay_s.thread_coord(ln, w)
                    lanes.append((tc[ld_] | rc[ld_], tc[pd] | rc[pd]))
                acc.append((2 * V, lanes, False))
        sl, cyc = LDS.choose(lines, length, sigma, acc)
        cache[key] = (sl, cyc, LDS.ideal(acc))
        return sl

    def _stage_dma_ok(self, info) -> bool:
        """Whether a stage can be filled by LDS DMA: buffer-addressable rows of whole 16-byte
        chunks, a loop-invariant column origin, a chunk count that fills whole wave copies,
        and (transposed operands) a fragment layout that ds_read_b64_tr_b16 delivers."""
        if self.opt.get("no_lds_dma"):
            return False
        d = self.desc[info["op"].operands[0].id]
        R, C = info["R"], info["C"]
        if C % 8 or (R * C // 8) % self.nt or info["kinds"][1] == "iv":
            return False
        if not self._stage_buffer_ok(info, d, 8):
            return False
        if info["mode"] == "trans":
            src = LY.tr16_source(info["lay"])
            if src is None:
                return False
            info["tr_src"] = src
        return True

    def _stage_setup_dma(self, info, idx: int, nst: int):
        """A stage filled by LDS DMA keeps the tile's memory rows (row-major, 16-byte chunks
        XOR-swizzled per the bank model); each thread copies `per` chunks per stage. The chunk
        a lane copies is the one the swizzle puts at its LDS position."""
        ld = info["op"]
        d = self.desc[ld.operands[0].id]
        R, C = info["R"], info["C"]
        T = ctype(ld.result.type.dtype)
        info.update({"line_dim": 0, "pos_dim": 1, "W": 8, "dma": True, "nst": nst})
        nvec = R * C // 8
        per = nvec // self.nt
        sl = self._dma_layout(info)
        name = f"ek_stg{idx}"
        info.update({"desc": d, "T": T, "sl": sl, "stage_elems": sl.elems, "nvec": nvec,
                     "per": per, "smem": name})
        self.extra_smem.append((name, nst * sl.elems * 2))
        lsh = sl.pitch.bit_length() - 1
        lensh = C.bit_length() - 1
        o1 = self._stage_offsets(info, "0")[1]
        sh1, s0 = d["shape"][1], d["strides"][0]
        h = (f"((((rw >> {sl.sa}) ^ (rw >> {sl.sb})) & {sl.mask}) << {3 + sl.csh})" if sl.mask
             else "0")
        self.emit(f"int ek_dmo{idx}[{per}];")
        self.emit("#pragma unroll")
        self.emit(f"for (int i = 0; i < {per}; ++i) {{")
        self.emit(f"  const int e = (i * {self.nt} + ek_tid) * 8, rw = e >> {lsh};")
        self.emit(f"  const int vp = (e & {sl.pitch - 1}) ^ {h};")
        self.emit(f"  const int line = rw * {sl.k} + (vp >> {lensh}), gc = {o1} + (vp & {C - 1});")
        self.emit(f"  ek_dmo{idx}[i] = (gc >= 0 && gc + 8 <= {sh1}) ? line * {s0} + gc : -1;")
        self.emit("}")
        # byte offsets relative to the tile's first row, for the resource that starts there
        self.emit(f"int ek_dmb{idx}[{per}];")
        self.emit("#pragma unroll")
        self.emit(f"for (int i = 0; i < {per}; ++i) "
                  f"ek_dmb{idx}[i] = ek_dmo{idx}[i] >= 0 ? ek_dmo{idx}[i] * 2 : ek::kOOB;")
        self.emit(f"const uint32_t ek_dml{idx} = ek::lds_addr({name}) + "
                  f"(uint32_t)__builtin_amdgcn_readfirstlane(ek_warp) * 1024u;")

    def _dma_layout(self, info) -> LDS.StageLayout:
        """Stage layout for a DMA-filled tile: rows of C elements, chunk swizzle chosen by
        simulating the dot's fragment reads (16-byte row reads, or transpose reads)."""
        R, C, lay = info["R"], info["C"], info["lay"]
        key = ("dma", info["mode"], R, C, self.nt, lay.key())
        if key in _STAGE_LAYOUTS:
            return _STAGE_LAYOUTS[key][0]
        acc = []
        seen = set()
        if info["mode"] == "row":
            d, nb = lay.vec_dim_bits()
            V = min(1 << nb, 8) if d == 1 else 1
            for w in range(lay.num_warps):
                wc = lay.thread_coord(0, w)
                if wc in seen:
                    continue
                seen.add(wc)
                for j in range(0, lay.nregs, V):
                    rc = lay.reg_coord(j)
                    lanes = []
                    for ln in range(64):
                        tc = lay.thread_coord(ln, w)
                        lanes.append((tc[0] | rc[0], tc[1] | rc[1]))
                    acc.append((2 * V, lanes, False))
        else:
            src = info["tr_src"]
            for w in range(src.num_warps):
                wc = src.thread_coord(0, w)
                if wc in seen:
                    continue
                seen.add(wc)
                for j in range(src.nregs):
                    rc = src.reg_coord(j)
                    lanes = []
                    for ln in range(64):
                        tc = src.thread_coord(ln, w)
                        lanes.append((tc[0] | rc[0], tc[1] | rc[1]))
                    acc.append((8, lanes, False))
        sigma = LDS.identity_sigma(C)
        best = None
        for i, c in enumerate(LDS.candidates(R, C, sigma)):
            if c.pitch != c.rowlen or (R * C) % c.pitch:
                continue
            k_ = (LDS.cost(c, acc), c.mask != 0, i)
            if best is None or k_ < best[0]:
                best = (k_, c)
        sl = best[1]
        _STAGE_LAYOUTS[key] = (sl, best[0][0], LDS.ideal(acc))
        return sl

    def _split_stages(self, stg: list, body, per_stage: int):
        """(first, second) stage infos when a loop's two staged operands are better served
        by one LDS stage each than by two: each operand feeds its own `tl.dot` at the top
        level of the body, one dot after the other (attention's QK^T, then PV); the
        workgroup has at most 4 waves; and double-buffered stages would take more than half
        of the CU's LDS while single ones fit in half, so two workgroups can share a CU.
        The second operand is then copied under the first dot and the first operand's next
        tile under the second dot, with a barrier between the dots, and the other
        workgroup on the CU covers each one's waits (a 128x128 attention tile, causal:
        547 against 750 us with two stages each, and against 568 us for 256x128 with 8
        waves). None otherwise, or with ENCELADUS_CODEGEN=no_split_stages."""
        force = self.opt.get("split_stages") == "force"
        if self.opt.get("no_split_stages") or len(stg) != 2 or self.nt > 256 or \
                per_stage > 81920 or not (force or 81920 < 2 * per_stage):
            return None
        ids = {info["op"].result.id: info for info in stg}
        order, dots = [], []
        for o in body.ops:
            if o.name != "dot":
                continue
            hit = [ids[_through_trans(x).id] for x in o.operands[:2]
                   if _through_trans(x).id in ids]
            if len(hit) > 1:
                return None
            if hit:
                plan = self.dot_plans.get(o.result.id)
                if plan is None or plan.tk < 2 or hit[0] in order:
                    return None
                order.append(hit[0])
                dots.append(o)
        if len(order) != 2:
            return None
        for info in stg:
            for u in self.uses.get(info["op"].result.id, []):
                if u.name not in ("dot", "trans"):
                    return None
        return order[0], order[1], dots[0], dots[1]

    # ops that read nothing but their operands and memory no op in the loop body writes
    _SINKABLE = frozenset(("binary", "unary", "cast", "select", "fma", "splat", "broadcast",
                           "expand_dims", "trans", "reshape", "const", "arange", "reduce",
                           "desc_load", "hint", "bitcast"))

    def _split_sink(self, body, first, second):
        """The loop body's ops in the order that puts the barrier between the dots of a
        split-stage loop (see `_split_stages`) as late as it can go: the ops between the two
        dots that build the second dot's A operand from a row reduction of the first dot's
        result (attention: `p = exp2(qk * scale - m)` and its cast), and everything that
        uses them (the row sum of p), move after the others (the row max, the rescale
        factor, `acc * alpha`), keeping their relative order. Returns (ops, first moved op),
        the barrier going right before that op, or None when there is nothing to move, an
        op in between has a region or a side effect, or ENCELADUS_CODEGEN=no_split_sink.

        The moved ops then form one basic block with the second dot's MFMAs (the rescale's
        skip branch stays before the barrier), which lets the compiler issue the
        exponentials of key slice k+1 while slice k's MFMAs run (causal 128x128: 3.3%
        faster than the barrier right before the second dot). The same order without a
        barrier in a double-buffered loop (256x128, 8 waves) measured 3% slower non-causal
        and no change causal, so only split-stage loops get it."""
        if self.opt.get("no_split_sink"):
            return None
        ops = body.ops
        i1, i2 = ops.index(first), ops.index(second)
        between = ops[i1 + 1:i2]
        if any(o.name not in self._SINKABLE or o.regions for o in between):
            return None
        inside = {id(o) for o in between}

        def producers(o):
            return [x.op for x in o.operands if x.op is not None and id(x.op) in inside]

        a = second.operands[0]
        anc, todo = set(), [a.op] if a.op is not None and id(a.op) in inside else []
        while todo:
            o = todo.pop()
            if id(o) not in anc:
                anc.add(id(o))
                todo.extend(producers(o))
        after_reduce = set()
        for o in between:
            if o.name == "reduce" or any(id(p) in after_reduce for p in producers(o)):
                after_reduce.add(id(o))
        moved = {id(o) for o in between if id(o) in anc and id(o) in after_reduce and
                 o.name != "reduce" and o.results and o.result.type.shape == a.type.shape}
        if not moved:
            return None
        for o in between:
            if any(id(p) in moved for p in producers(o)):
                moved.add(id(o))
        keep = [o for o in between if id(o) not in moved]
        sunk = [o for o in between if id(o) in moved]
        return ops[:i1 + 1] + keep + sunk + ops[i2:], sunk[0]

    def _stage_dma_parts(self, info, kval: str, stage: str) -> tuple[list[str], list[str]]:
        """Copies the tile at row origin `kval` (or the loop-invariant one) into stage `stage`,
        as (set-up lines, one line per 16-byte copy of this thread) so that the copies can be
        spread over a dot's k steps. Rows outside [0, shape0) fall past the buffer resource
        and arrive as zeros."""
        d = info["desc"]
        o0, _ = self._stage_offsets(info, kval)
        idx = info["smem"][len("ek_stg"):]
        R, per = info["R"], info["per"]
        base, s0, sh0 = d["base"], d["strides"][0], d["shape"][0]
        t = self.fresh("cp")
        # A tile starting at row >= 0 (the usual case) copies through a resource based at its
        # first row, so the per-chunk offsets are the loop-invariant ones; otherwise rows
        # before 0 need the general form with the row offset in each lane's address. The
        # choice is uniform: the resource is a select, the rare general offsets a branch in
        # the set-up, so the copies themselves need no branch.
        setup = [f"const int {t}_r0 = {o0};",
                 f"const uint32_t {t}_ls = ek_dml{idx} + (uint32_t)({stage}) * "
                 f"{info['stage_elems'] * 2}u;",
                 f"const bool {t}_pos = {t}_r0 >= 0;",
                 f"const ek::i32x4 {t}_rs = {t}_pos ? ek::rsrc_words({base} + (int64_t){t}_r0 * "
                 f"{s0}, {t}_r0 < {sh0} ? (uint32_t)({sh0} - {t}_r0) * (uint32_t){s0} * 2u : 0u) "
                 f": ek::rsrc_words({base}, {t}_r0 > -{R} ? (uint32_t){sh0} * (uint32_t){s0} * 2u "
                 ": 0u);",
                 f"int {t}_of[{per}];",
                 "#pragma unroll",
                 f"for (int i = 0; i < {per}; ++i) {t}_of[i] = ek_dmb{idx}[i];",
                 f"if (!{t}_pos) {{",
                 f"  const int {t}_rb = {t}_r0 * {s0};",
                 "  #pragma unroll",
                 f"  for (int i = 0; i < {per}; ++i) {t}_of[i] = ek_dmo{idx}[i] >= 0 ? "
                 f"({t}_rb + ek_dmo{idx}[i]) * 2 : ek::kOOB;",
                 "}"]
        chunks = [f"ek::dma16({t}_rs, {t}_ls + {i * self.nt * 16}u, {t}_of[{i}]);"
                  for i in range(per)]
        return setup, chunks

    def _stage_dma(self, info, kval: str, stage: str) -> list[str]:
        """The whole copy of one tile as a block (loop prologues)."""
        setup, chunks = self._stage_dma_parts(info, kval, stage)
        return ["{"] + ["  " + ln for ln in setup + chunks] + ["}"]

    def _stage_setup(self, info, idx: int):
        ld = info["op"]
        d = self.desc[ld.operands[0].id]
        R, C = info["R"], info["C"]
        T = ctype(ld.result.type.dtype)
        info["nst"] = 2
        if info["mode"] == "row":
            W = 8
            nvec = R * C // 8
            info.update({"line_dim": 0, "pos_dim": 1})
        else:
            W = 8 if (R // 8) * (C // 8) >= self.nt or C % 4 else 4
            nvec = (R // 8) * (C // W)
            info.update({"line_dim": 1, "pos_dim": 0})
        info["W"] = W
        info["buf"] = self._stage_buffer_ok(info, d, W)
        per = (nvec + self.nt - 1) // self.nt
        sl = self._stage_layout(info, W, nvec, per)
        name = f"ek_stg{idx}"
        info.update({"desc": d, "T": T, "sl": sl, "stage_elems": sl.elems,
                     "nvec": nvec, "per": per, "smem": name, "regs": f"ek_pf{idx}"})
        self.extra_smem.append((name, 2 * sl.elems * 2))
        if info["mode"] == "trans" and W == 4:
            self.emit(f"ek::u32x2 {info['regs']}[{per * 8}];")
        else:
            regs = per * (8 if info["mode"] == "trans" else 1)
            self.emit(f"ek::u32x4 {info['regs']}[{regs}];")

    def _stage_buffer_ok(self, info, d, W: int) -> bool:
        """Whether a stage can load through raw buffer loads: 32-bit byte offsets, aligned
        rows, and column chunks of W elements that lie wholly inside or outside the tile."""
        if self.opt.get("no_buffer_loads") or d["base_v"].facts.get("span2g"):
            return False
        div = lambda v: self.axis.get(v).div[0]  # noqa: E731
        if div(d["base_v"]) < 2 * W or div(d["stride_v"][0]) % W:
            return False
        if div(d["shape_v"][1]) % W:
            return False
        o1 = info["op"].operands[2]
        return div(o1) % W == 0

    def _stage_load_buffer(self, info, o0: str, o1: str) -> list[str]:
        """Stage loads through one buffer resource: rows outside [0, shape0) fall past the
        resource and read zeros in hardware, so there is no edge path. A tile that starts
        far outside gets an empty resource, which also keeps the 32-bit offsets from
        wrapping into range."""
        d = info["desc"]
        R, C, per, nvec = info["R"], info["C"], info["per"], info["nvec"]
        base, s0 = d["base"], d["strides"][0]
        sh0, sh1 = d["shape"][0], d["shape"][1]
        regs, W = info["regs"], info["W"]
        o1v = info["op"].operands[2]
        o1c = int(o1v.op.attrs["value"]) if o1v.op is not None and o1v.op.name == "const" else None
        sh1v = d["shape_v"][1]
        sh1c = int(sh1v.op.attrs["value"]) if sh1v.op is not None and sh1v.op.name == "const" \
            else None
        cols_ok = o1c is not None and sh1c is not None and o1c >= 0 and o1c + C <= sh1c
        out = ["{", f"  const int ek_r0 = {o0};",
               f"  const __amdgpu_buffer_rsrc_t ek_rs = ek::buffer_rsrc({base}, "
               f"(ek_r0 > -{R} && ek_r0 < {sh0}) ? (uint32_t){sh0} * (uint32_t){s0} * 2u : 0u);",
               "  #pragma unroll", f"  for (int i = 0; i < {per}; ++i) {{",
               f"    const int c = ek_tid + i * {self.nt};"]
        if nvec % self.nt:
            out.append(f"    if (c >= {nvec}) break;")
        if info["mode"] == "row":
            chk = "" if cols_ok else f"(gc >= 0 && gc + 8 <= {sh1}) ? "
            tail = "" if cols_ok else " : ek::kOOB"
            out += [f"    const int r = c / {C // 8}, cc = (c % {C // 8}) * 8, gc = {o1} + cc;",
                    f"    {regs}[i] = ek::buffer_load16(ek_rs, {chk}((ek_r0 + r) * {s0} + gc) * 2"
                    f"{tail});"]
        else:
            sig = info["sl"].sigma
            rr = bits_expr("rb", [(s_, i_) for i_, s_ in enumerate(sig) if s_ >= 3])
            rj = bits_expr("j", [(s_, i_) for i_, s_ in enumerate(sig) if s_ < 3])
            ld = "buffer_load16" if W == 8 else "buffer_load8"
            chk = "" if cols_ok else f"(gc >= 0 && gc + {W} <= {sh1}) ? "
            tail = "" if cols_ok else " : ek::kOOB"
            out += [f"    const int rb = (c / {C // W}) * 8, cb = (c % {C // W}) * {W}, "
                    f"rr = {rr}, gc = {o1} + cb;",
                    "    #pragma unroll",
                    f"    for (int j = 0; j < 8; ++j) {regs}[i * 8 + j] = ek::{ld}(ek_rs, "
                    f"{chk}((ek_r0 + rr + ({rj})) * {s0} + gc) * 2{tail});"]
        out += ["  }", "}"]
        return out

    def _stage_load(self, info, kval: str) -> list[str]:
        d = info["desc"]
        o0, o1 = self._stage_offsets(info, kval)
        if info.get("buf"):
            return self._stage_load_buffer(info, o0, o1)
        R, C, per, nvec = info["R"], info["C"], info["per"], info["nvec"]
        base, s0 = d["base"], d["strides"][0]
        sh0, sh1 = d["shape"][0], d["shape"][1]
        regs = info["regs"]
        W = info.get("W", 8)
        vt = "ek::u32x4" if (info["mode"] == "row" or W == 8) else "ek::u32x2"
        head = ["#pragma unroll", f"for (int i = 0; i < {per}; ++i) {{",
                f"  const int c = ek_tid + i * {self.nt};"]
        if nvec % self.nt:
            head.append(f"  if (c >= {nvec}) break;")
        scalar = (f"(unsigned)gr < (unsigned){sh0} && (unsigned)(gc + e) < (unsigned){sh1}) ? "
                  f"reinterpret_cast<const uint16_t*>({base})[(int64_t)gr * {s0} + gc + e] : "
                  f"(uint16_t)0;")
        # uniform interior test: the whole R x C block is inside the descriptor
        full = (f"(({o0}) >= 0 && ({o0}) + {R} <= {sh0} && ({o1}) >= 0 && "
                f"({o1}) + {C} <= {sh1})")
        out = [f"if ({full}) {{"]
        if info["mode"] == "row":
            out += ["  " + x for x in head] + [
                f"    const int r = c / {C // 8}, cc = (c % {C // 8}) * 8;",
                f"    {regs}[i] = *reinterpret_cast<const ek::u32x4*>({base} + (int64_t)({o0} + r)"
                f" * {s0} + {o1} + cc);", "  }", "} else {"]
            out += ["  " + x for x in head] + [
                f"    const int r = c / {C // 8}, cc = (c % {C // 8}) * 8;",
                f"    const int gr = {o0} + r, gc = {o1} + cc;",
                f"    if ((unsigned)gr < (unsigned){sh0} && gc >= 0 && gc + 8 <= {sh1}) "
                f"{regs}[i] = *reinterpret_cast<const ek::u32x4*>({base} + (int64_t)gr * {s0} + gc);",
                "    else {", "      uint16_t h[8];",
                f"      for (int e = 0; e < 8; ++e) h[e] = ({scalar}",
                f"      __builtin_memcpy(&{regs}[i], h, 16);", "    }", "  }", "}"]
        else:
            # storage positions rb..rb+7 hold logical rows rr + (the logical offset of j)
            sig = info["sl"].sigma
            rr = bits_expr("rb", [(s_, i_) for i_, s_ in enumerate(sig) if s_ >= 3])
            rj = bits_expr("j", [(s_, i_) for i_, s_ in enumerate(sig) if s_ < 3])
            idx_ = (f"    const int rb = (c / {C // W}) * 8, cb = (c % {C // W}) * {W}, "
                    f"rr = {rr};")
            out += ["  " + x for x in head] + [
                idx_,
                "    #pragma unroll",
                f"    for (int j = 0; j < 8; ++j) {regs}[i * 8 + j] = *reinterpret_cast<const {vt}*>"
                f"({base} + (int64_t)({o0} + rr + ({rj})) * {s0} + {o1} + cb);", "  }", "} else {"]
            out += ["  " + x for x in head] + [
                idx_,
                f"    const int gc = {o1} + cb;",
                "    #pragma unroll", "    for (int j = 0; j < 8; ++j) {",
                f"      const int gr = {o0} + rr + ({rj});",
                f"      if ((unsigned)gr < (unsigned){sh0} && gc >= 0 && gc + {W} <= {sh1}) "
                f"{regs}[i * 8 + j] = *reinterpret_cast<const {vt}*>({base} + (int64_t)gr * {s0} + gc);",
                "      else {", f"        uint16_t h[{W}];",
                f"        for (int e = 0; e < {W}; ++e) h[e] = ({scalar}",
                f"        __builtin_memcpy(&{regs}[i * 8 + j], h, {2 * W});", "      }", "    }",
                "  }", "}"]
        return out

    def _stage_store(self, info, stage: str) -> list[str]:
        C, per, nvec = info["C"], info["per"], info["nvec"]
        regs, sl = info["regs"], info["sl"]
        sm = f"(reinterpret_cast<uint16_t*>({info['smem']}) + ({stage}) * {info['stage_elems']})"
        out = ["#pragma unroll", f"for (int i = 0; i < {per}; ++i) {{",
               f"  const int c = ek_tid + i * {self.nt};"]
        if nvec % self.nt:
            out.append(f"  if (c >= {nvec}) break;")
        if info["mode"] == "row":
            out += [f"  const int r = c / {C // 8}, cc = (c % {C // 8}) * 8;",
                    f"  *reinterpret_cast<ek::u32x4*>({sm} + {sl.cexpr('r', 'cc')}) = {regs}[i];"]
        else:
            W = info["W"]
            out += [f"  const int rb = (c / {C // W}) * 8, cb = (c % {C // W}) * {W};",
                    f"  ek::u32x4 o[{W}];",
                    f"  ek::transpose8x{W}(&{regs}[i * 8], o);",
                    "  #pragma unroll",
                    f"  for (int q = 0; q < {W}; ++q) *reinterpret_cast<ek::u32x4*>({sm} + "
                    f"{sl.cexpr('cb + q', 'rb')}) = o[q];"]
        out.append("}")
        return out

    def read_staged(self, v: ir.Value, lay: LY.Layout) -> str:
        key = ("stg", v.id, lay.key())
        for sc in reversed(self.scopes):
            if key in sc.memo:
                return sc.memo[key]
        info = self.staged[v.id]
        T = info["T"]
        lay_s = self._stage_view(info, lay)
        d, nb = lay_s.vec_dim_bits()
        V = min(1 << nb, 8) if d == info["pos_dim"] else 1
        sm = (f"(reinterpret_cast<const {T}*>({info['smem']}) + (ek_it{info['loop_idx']} % "
              f"{info['nst']}) * {info['stage_elems']})")
        idx = info["sl"].cexpr(self.coord(lay_s, info["line_dim"], "r"),
                               self.coord(lay_s, info["pos_dim"], "r"))
        nm = self.fresh("sr")
        self.emit(f"{T} {nm}[{lay.nregs}];")
        self.emit("#pragma unroll")
        self.emit(f"for (int r = 0; r < {lay.nregs}; r += {V}) ek::vload<{T}, {V}>(&{nm}[r], "
                  f"&{sm}[{idx}]);")
        self.cur.memo[key] = nm
        return nm

    # -- dot loops on the GEMM template ---------------------------------------------------
    def _gemm_match(self, op):
        """Matches `for k in range(lo, hi, BK): acc = dot(dA.load([m0, k]), dB.load([k, n0]),
        acc)` with loop-invariant m0/n0, 16-bit operands and aligned row-major tiles.
        Returns a dict for the template, or None to use the generic lowering."""
        body = op.regions[0]
        iv, carried = body.args[0], body.args[1:]
        if len(carried) != 1:
            return None
        acc = carried[0]
        ops = body.ops[:-1]
        y = body.ops[-1]
        dots = [o for o in ops if o.name == "dot"]
        loads = [o for o in ops if o.name == "desc_load"]
        if len(dots) != 1 or len(loads) != 2:
            return None
        dot = dots[0]
        a, b, c = dot.operands
        if c.id != acc.id or y.operands[0].id != dot.result.id:
            return None
        if len(self.uses.get(acc.id, [])) != 1:
            return None
        la = a.op if a.op in loads else None
        lb = b.op if b.op in loads else None
        if la is None or lb is None:
            return None
        if len(self.uses.get(a.id, [])) != 1 or len(self.uses.get(b.id, [])) != 1:
            return None
        scalar_ops = []
        for o in ops:
            if o in (dot, la, lb):
                continue
            if o.regions or not o.results or self.tile(o.result) or \
                    isinstance(o.result.type, ir.DescType) or o.name in (
                        "load", "atomic_rmw", "atomic_cas", "store", "desc_store"):
                return None
            scalar_ops.append(o)
        dep = {iv.id}
        for o in scalar_ops:
            if any(x.id in dep for x in o.operands):
                dep.add(o.result.id)
        da, db = la.operands[0], lb.operands[0]
        if da.id not in self.desc or db.id not in self.desc:
            return None
        if la.operands[2].id != iv.id or lb.operands[1].id != iv.id:
            return None
        if la.operands[1].id in dep or lb.operands[2].id in dep:
            return None
        dt = a.type.dtype
        if dt not in (core.float16, core.bfloat16) or b.type.dtype is not dt:
            return None
        if c.type.dtype is not core.float32:
            return None
        step = op.operands[2]
        bm, bk = a.type.shape
        bn = b.type.shape[1]
        if not (step.op is not None and step.op.name == "const" and step.op.attrs["value"] == bk):
            return None
        plan = self.dot_plans[dot.result.id]
        if plan.inst.m != 32 or plan.inst.k != 16 or plan.wrep != 1 or \
                tuple(plan.korder) != tuple(range(len(plan.korder))):
            return None
        nt = self.nt
        kc = bk // 8
        if bk % 16 or (bm * kc) % nt or ((kc * (bn // 8)) % nt and kc * (bn // 8) >= nt):
            return None
        if self.lay[acc.id].key() != LY.mfma_acc(plan).key():
            return None
        A, B = self.desc[da.id], self.desc[db.id]
        ok = lambda v, d: self.axis.get(v).div[0] >= d  # noqa: E731
        if not (ok(A["base_v"], 16) and ok(B["base_v"], 16) and ok(A["stride_v"][0], 8)
                and ok(B["stride_v"][0], 8)):
            return None
        return {"plan": plan, "A": A, "B": B, "m0": la.operands[1], "n0": lb.operands[2],
                "scalar_ops": scalar_ops, "dt": dt, "bm": bm, "bn": bn, "bk": bk}

    def _emit_gemm_loop(self, op, g) -> bool:
        self.report["gemm_template"] = op.loc
        body = op.regions[0]
        acc_arg = body.args[1]
        init = op.operands[3]
        lo, hi = (self.name[o.id] for o in op.operands[:2])
        lay = self.lay[acc_arg.id]
        nm = self.fresh("c")
        e = self.elem(init, lay, "r")
        self.emit(f"float {nm}[{lay.nregs}];")
        self.emit("#pragma unroll")
        self.emit(f"for (int r = 0; r < {lay.nregs}; ++r) {nm}[r] = {e};")
        self.emit("{")
        for o in g["scalar_ops"]:
            self.gen_op(o)
        p = g["plan"]
        T = ctype(g["dt"])
        A, B = g["A"], g["B"]
        # Buffer loads (hardware bounds checks) send a 16-byte chunk that is not wholly inside
        # its row out of range, so they need K and N known to be multiples of 8; and no
        # operand may span >= 2 GiB (32-bit byte offsets).
        big = any(v.facts.get("span2g") for v in (A["base_v"], B["base_v"]))
        whole = all(self.axis.get(v).div[0] % 8 == 0 for v in (A["shape_v"][1], B["shape_v"][1]))
        buf = not (big or not whole or self.opt.get("no_buffer_loads"))
        bm, bn, bk = g["bm"], g["bn"], g["bk"]
        stage = (bm * bk + bk * bn) * 2
        dma = (buf and not self.opt.get("no_lds_dma") and (bm * bk // 8) % self.nt == 0
               and (bk * bn // 8) % self.nt == 0 and bn >= 32)
        if dma:
            # Stages: as many (at most 4) as fit the LDS share of a workgroup when a CU keeps
            # 8 waves (2 per SIMD) resident; or the `gemm_stages` option.
            share = 163840 // max(1, 8 // (self.nt // 64))
            nst = int(self.opt.get("gemm_stages", 0)) or max(2, min(4, share // stage))
            d = (bm * bk // 8 + bk * bn // 8) // self.nt
            while nst > 2 and ((nst - 2) * d > 63 or nst * stage > 163840):
                nst -= 1
            split = min(bk // 16, int(self.opt.get("gemm_split", 1)))
            tr = ", true" if p.trans else ""
            tmpl = (f"ek::GemmDma<{T}, {bm}, {bn}, {bk}, {p.wm}, {p.wn}, {self.nt}, {nst}, "
                    f"{split}{tr}>")
            self.need_lds(nst * stage)
        else:
            tr = ", true" if p.trans else ""
            tmpl = (f"ek::Gemm<{T}, {bm}, {bn}, {bk}, {p.wm}, {p.wn}, {self.nt}, "
                    f"{'true' if buf else 'false'}{tr}>")
            self.need_lds(2 * stage)
        self.emit(f"  {tmpl} ek_g;")
        self.emit(f"  ek_g.run({nm}, {A['base']}, {A['strides'][0]}, {B['base']}, "
                  f"{B['strides'][0]}, {A['shape'][0]}, {B['shape'][1]}, {A['shape'][1]}, "
                  f"{self.name[g['m0'].id]}, {self.name[g['n0'].id]}, {lo}, {hi}, ek_smem, ek_tid);")
        self.emit("}")
        self.define(op.results[0], nm)
        self.big_acc = max(getattr(self, "big_acc", 0), lay.nregs)
        return True

    # -- control flow -----------------------------------------------------------------
    def op_for(self, op):
        if not self._pos_step(op):
            return self._general_for(op)
        if not self.opt.get("no_gemm_template"):
            g = self._gemm_match(op)
            if g is not None and self._emit_gemm_loop(op, g):
                return
        body = op.regions[0]
        iv, carried = body.args[0], body.args[1:]
        lo, hi, step = (self.name[o.id] for o in op.operands[:3])
        inits = op.operands[3:]
        names = []
        for a, i in zip(carried, inits):
            t = ctype(a.type.dtype) + ("*" if a.type.ptr else "")
            nm = self.fresh("c")
            names.append(nm)
            if not self.tile(a):
                self.emit(f"{t} {nm} = {self.name[i.id]};")
            else:
                lay = self.lay[a.id]
                e = self.elem(i, lay, "r")
                self.emit(f"{t} {nm}[{lay.nregs}];")
                self.emit("#pragma unroll")
                self.emit(f"for (int r = 0; r < {lay.nregs}; ++r) {nm}[r] = {e};")
        it = ctype(iv.type.dtype)
        ivn = self.fresh("iv")
        stg = self.stage_loops.get(id(op), []) if hasattr(self, "stage_loops") else []
        dma = bool(stg) and all(self._stage_dma_ok(info) for info in stg)
        if dma:
            li = self.counter
            self.emit(f"int ek_it{li} = 0;")
            # stages: 2, or 3 when they fit the LDS share of a workgroup at 8 waves per CU
            per_stage = sum(info["R"] * info["C"] * 2 for info in stg)
            share = 163840 // max(1, 8 // (self.nt // 64))
            nst = int(self.opt.get("stage_count", 0)) or (3 if 3 * per_stage <= share else 2)
            dcount = sum(info["R"] * info["C"] // 8 // self.nt for info in stg)
            while nst > 2 and (nst - 2) * dcount > 63:
                nst -= 1
            split = self._split_stages(stg, body, per_stage)
            if split is not None:
                nst = 1
            for info in stg:
                info["loop_idx"] = li
                self._stage_setup_dma(info, len(self.extra_smem), nst)
            self.emit("__syncthreads();")
            # nothing loaded before the loop is outstanding, so the vmcnt at the top of the
            # body counts this loop's copies only
            self.emit("__builtin_amdgcn_s_waitcnt(0x0F70);")
            if split is not None:
                # split stages: only the first dot's operand is copied ahead of the loop
                for ln in self._stage_dma(split[0], lo, "0"):
                    self.emit(ln)
            for s_ in range(nst - 1):
                for info in stg:
                    kv = f"({lo} + {s_} * {step})" if s_ else lo
                    for ln in self._stage_dma(info, kv, str(s_)):
                        self.emit(ln)
        elif stg:
            li = self.counter
            self.emit(f"int ek_it{li} = 0;")
            for k, info in enumerate(stg):
                info["loop_idx"] = li
                self._stage_setup(info, len(self.extra_smem))
            self.emit("__syncthreads();")
            self.emit(f"if ({lo} < {hi}) {{")
            for info in stg:
                for ln in self._stage_load(info, lo):
                    self.emit("  " + ln)
                for ln in self._stage_store(info, "0"):
                    self.emit("  " + ln)
            self.emit("}")
            self.emit("__syncthreads();")
            # s_waitcnt vmcnt(0): no global load is outstanding at the loop head on any path,
            # so the first use of a register loaded before the loop does not also wait for
            # the next tile's prefetch issued at the top of the body.
            self.emit("__builtin_amdgcn_s_waitcnt(0x0F70);")
        self.push_scope(f"for ({it} {ivn} = {lo}; {ivn} < {hi}; {ivn} += {step}) {{")
        self.define(iv, ivn)
        for a, nm in zip(carried, names):
            self.define(a, nm)
        body_ops = None
        if dma:
            self.in_staged_loop = getattr(self, "in_staged_loop", 0) + 1
            # this wave's copies of the current stage have landed (nst - 2 younger stages may
            # still fly) and its reads of the previous stage are complete; after the barrier
            # everyone's are, so the previous stage can be refilled.
            self.emit(f'asm volatile("s_waitcnt vmcnt({max(0, nst - 2) * dcount}) lgkmcnt(0)'
                      f'\\n\\ts_barrier" ::: "memory");')
            setup, chunks = [], []
            if split is not None:
                # split stages: the second dot's operand for this iteration is copied under
                # the first dot; the first dot's operand for the next iteration is copied
                # under the second dot, after a barrier between them (`op_dot`)
                setup, chunks = self._stage_dma_parts(split[1], ivn, "0")
                prev_split = getattr(self, "split_next", None)
                self.split_next = {"info": split[1], "scope": self.cur,
                                   "parts": self._stage_dma_parts(split[0],
                                                                  f"({ivn} + {step})", "0")}
                sink = self._split_sink(body, split[2], split[3])
                if sink is not None:
                    body_ops, self.split_next["at"] = sink
            for info in (stg if split is None else ()):
                su, ch = self._stage_dma_parts(info, f"({ivn} + {nst - 1} * {step})",
                                               f"(ek_it{li} + {nst - 1}) % {nst}")
                setup += su
                chunks += ch
            lines = ["{"] + ["  " + ln for ln in setup + chunks] + ["}"]
            # The copies for a later stage may go anywhere after the barrier: the first dot
            # that reads a stage issues them after its first k slice (its fragment reads go
            # out first and hide behind the copy issue); otherwise they land here.
            slot: list = []
            self.cur.items.append(slot)
            prev_dma = getattr(self, "deferred_dma", None)
            self.deferred_dma = None if self.opt.get("no_late_dma") else \
                {"lines": lines, "setup": setup, "chunks": chunks, "used": False,
                 "scope": self.cur}
            if self.deferred_dma is None:
                slot.extend(self.cur.indent + ln for ln in lines)
        elif stg:
            self.in_staged_loop = getattr(self, "in_staged_loop", 0) + 1
            self.emit(f"const bool ek_more{li} = {ivn} + {step} < {hi};")
            self.emit(f"if (ek_more{li}) {{")
            for info in stg:
                for ln in self._stage_load(info, f"({ivn} + {step})"):
                    self.emit("  " + ln)
            self.emit("}")
        self.gen_block(body, body_ops)
        if dma:
            d = self.deferred_dma
            if d is not None and not d["used"]:
                slot.extend(self.cur.indent + ln for ln in d["lines"])
            self.deferred_dma = prev_dma
            if split is not None:
                assert self.split_next is None, "split stages: the second dot never ran"
                self.split_next = prev_split
            self.emit(f"++ek_it{li};")
            self.in_staged_loop -= 1
        elif stg:
            self.emit(f"if (ek_more{li}) {{")
            for info in stg:
                for ln in self._stage_store(info, f"(ek_it{li} + 1) & 1"):
                    self.emit("  " + ln)
            self.emit("}")
            self.emit("__syncthreads();")
            self.emit(f"++ek_it{li};")
            self.in_staged_loop -= 1
        y = body.ops[-1]
        self._assign_yield(y.operands, carried, names)
        self.pop_scope()
        if dma:
            # copies issued past the last iteration land before anyone reuses the LDS
            self.emit('asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\\n\\ts_barrier" ::: "memory");')
        for r, nm in zip(op.results, names):
            self.define(r, nm)

    def _general_for(self, op):
        """Python `range` with a runtime or negative step: the trip count is computed once
        in 64-bit unsigned arithmetic (exact for any bounds of the loop type), so the loop
        always ends; a zero step runs no iterations (Python raises instead)."""
        body = op.regions[0]
        iv, carried = body.args[0], body.args[1:]
        lo, hi, step = (self.name[o.id] for o in op.operands[:3])
        names = []
        for a, i in zip(carried, op.operands[3:]):
            t = ctype(a.type.dtype) + ("*" if a.type.ptr else "")
            nm = self.fresh("c")
            names.append(nm)
            if not self.tile(a):
                self.emit(f"{t} {nm} = {self.name[i.id]};")
            else:
                lay = self.lay[a.id]
                self.emit(f"{t} {nm}[{lay.nregs}];")
                self.emit("#pragma unroll")
                self.emit(f"for (int r = 0; r < {lay.nregs}; ++r) {nm}[r] = "
                          f"{self.elem(i, lay, 'r')};")
        it = ctype(iv.type.dtype)
        k = self.fresh("gl")
        self.emit(f"const int64_t {k}_lo = (int64_t)({lo}), {k}_hi = (int64_t)({hi}), "
                  f"{k}_st = (int64_t)({step});")
        self.emit(f"const uint64_t {k}_n = {k}_st > 0 ? ({k}_hi > {k}_lo ? ((uint64_t){k}_hi - "
                  f"(uint64_t){k}_lo - 1) / (uint64_t){k}_st + 1 : 0) : {k}_st < 0 ? ({k}_lo > "
                  f"{k}_hi ? ((uint64_t){k}_lo - (uint64_t){k}_hi - 1) / (0 - (uint64_t){k}_st) "
                  "+ 1 : 0) : 0;")
        ivn = self.fresh("iv")
        self.push_scope(f"for (uint64_t {k}_k = 0; {k}_k < {k}_n; ++{k}_k) {{")
        self.emit(f"const {it} {ivn} = ({it})((uint64_t){k}_lo + {k}_k * (uint64_t){k}_st);")
        self.define(iv, ivn)
        for a, nm in zip(carried, names):
            self.define(a, nm)
        self.gen_block(body)
        self._assign_yield(body.ops[-1].operands, carried, names)
        self.pop_scope()
        for r, nm in zip(op.results, names):
            self.define(r, nm)

    def _assign_yield(self, vals, targets, names):
        tids = {t.id for t in targets}
        need_tmp = False
        for v in vals:
            s = v
            if self.kind.get(v.id) == "view":
                s, _, _ = self.resolve(v, self.lay[v.id], "r")
            if s.id in tids or self.kind.get(s.id) == "fused":
                need_tmp = True
        pend = []
        for v, t, nm in zip(vals, targets, names):
            if v.id == t.id:
                continue
            if not self.tile(t):
                if need_tmp:
                    tmp = self.fresh("y")
                    self.emit(f"const {ctype(t.type.dtype)}{'*' if t.type.ptr else ''} {tmp} = "
                              f"{self.name[v.id]};")
                    pend.append((nm, tmp, None))
                else:
                    self.emit(f"{nm} = {self.name[v.id]};")
                continue
            lay = self.lay[t.id]
            if self.kind.get(v.id) == "anchored" and self.name.get(v.id) == nm:
                continue
            if need_tmp:
                tmp = self.fresh("y")
                tt = ctype(t.type.dtype) + ("*" if t.type.ptr else "")
                e = self.elem(v, lay, "r")
                self.emit(f"{tt} {tmp}[{lay.nregs}];")
                self.emit("#pragma unroll")
                self.emit(f"for (int r = 0; r < {lay.nregs}; ++r) {tmp}[r] = {e};")
                pend.append((nm, tmp, lay.nregs))
            else:
                e = self.elem(v, lay, "r")
                self.emit("#pragma unroll")
                self.emit(f"for (int r = 0; r < {lay.nregs}; ++r) {nm}[r] = {e};")
        for nm, tmp, n in pend:
            if n is None:
                self.emit(f"{nm} = {tmp};")
            else:
                self.emit("#pragma unroll")
                self.emit(f"for (int r = 0; r < {n}; ++r) {nm}[r] = {tmp}[r];")

    def op_if(self, op):
        cond = self.name[op.operands[0].id]
        names = []
        for r in op.results:
            t = ctype(r.type.dtype) + ("*" if r.type.ptr else "")
            nm = self.fresh("f")
            names.append(nm)
            if self.tile(r):
                self.emit(f"{t} {nm}[{self.lay[r.id].nregs}];")
            else:
                self.emit(f"{t} {nm};")
        for i, reg in enumerate(op.regions):
            self.push_scope(f"if ({cond}) {{" if i == 0 else "else {")
            self.gen_block(reg)
            y = reg.ops[-1]
            for v, r, nm in zip(y.operands, op.results, names):
                if self.tile(r):
                    lay = self.lay[r.id]
                    e = self.elem(v, lay, "r")
                    self.emit("#pragma unroll")
                    self.emit(f"for (int r = 0; r < {lay.nregs}; ++r) {nm}[r] = {e};")
                else:
                    self.emit(f"{nm} = {self.name[v.id]};")
            self.pop_scope()
        for r, nm in zip(op.results, names):
            self.define(r, nm)

    # ------------------------------------------------------------------ driver
    def run(self) -> GeneratedKernel:
        fn = self.fn
        self.count_uses(fn.body)
        args = []
        params = []
        for i, (a, nmh) in enumerate(zip(fn.args, fn.arg_names)):
            self.vals[a.id] = a
            t = a.type
            if t.ptr:
                self.kind[a.id] = "scalar"
                cp = f"{ctype(t.dtype)}*"
                args.append(KernelArg(nmh, "ptr", t.dtype, cp))
                params.append(f"{cp} a{i}")
                self.name[a.id] = f"a{i}"
            else:
                self.kind[a.id] = "scalar"
                dt = t.dtype
                cp = "int32_t" if dt.is_bool() else ctype(dt)
                args.append(KernelArg(nmh, "scalar", dt, cp))
                params.append(f"{cp} a{i}")
                self.name[a.id] = f"a{i}" if not dt.is_bool() else f"((bool)a{i})"
            self.def_level[a.id] = 0
        self.plan_dots(fn)
        self.plan_staging(fn.body)
        # workgroups per CU for a coarsened grid (0: one workgroup per program)
        c_ = self.opt.get("coarsen")
        self.coarsen = (4 if c_ is True else int(c_)) if c_ else 0
        self.pid_axes = {op.attrs.get("axis", 0) for op in ir.walk(fn.body)
                         if op.name == "program_id"}
        self.plan_privatization(fn)
        self.assign_block(fn.body)
        self.remap_pids = bool(self.dot_plans) and not self.opt.get("no_pid_remap") and \
            not self.coarsen
        # Program versioning: a straight-line program whose masked accesses are all provably
        # unmasked under a few uniform conditions (every program but the edge ones) runs a
        # fast copy without per-access branches and mask arithmetic; the first failing
        # guard jumps to the general copy before any store has run.
        if self._can_version(fn):
            mark = len(self.scopes[0].items)
            report = {k: list(v) for k, v in self.report.items()}
            self.fast_mode = True
            self.gen_block(fn.body)
            self.fast_mode = False
            fast = self.scopes[0].items[mark:]
            del self.scopes[0].items[mark:]
            self.scopes[0].memo.clear()
            self.report = report
            if not self.fast_failed and self.fast_conds and \
                    all(isinstance(it, str) for it in fast):
                self.scopes[0].items.append("  {")
                self.scopes[0].items.extend("  " + it for it in fast)
                self.scopes[0].items.append("    return;")
                self.scopes[0].items.append("  " + "}" * (len(self.fast_conds) + 1))
                self.edge_only = True
        self.gen_block(fn.body)
        kname = f"ek_{fn.name}"
        if self.asserts:
            params.append("uint32_t* ek_assert_buf")
            args.append(KernelArg("ek_assert_buf", "ptr", core.uint32, "uint32_t*"))
        # Two-level flush of privatised bins: each workgroup stores its bins to a partial
        # buffer row (plain stores), and a second kernel sums a block of RB rows by 64 words
        # and adds each sum with one global atomic. Measured on the 1024-bin histogram: one
        # global atomic per bin per workgroup (2,048 per address) cost about 29 us; 32-row
        # blocks across all bins (64 atomics per address) 7.6 us.
        two = bool(self.priv) and bool(self.coarsen) and self.priv_copies == 1 and \
            self.opt.get("priv_flush", "two_level") != "atomic" and \
            all(i["dt"].primitive_bitwidth == 32 for i in self.priv.values())
        if two:
            off = 0
            for info in self.priv.values():
                info["off"] = off
                off += (info["bins"] + 3) // 4 * 4
            total_words = off
            params.append("int32_t* __restrict__ ek_part")
            args.append(KernelArg("ek_part", "ptr", core.int32, "int32_t*"))
        if self.coarsen:
            params += ["int32_t ek_np_x", "int32_t ek_np_y", "int32_t ek_np_z"]
        out = ['#include "enceladus_cdna4.h"', ""]
        attrs = f"__launch_bounds__({self.nt})"
        if getattr(self, "big_acc", 0) >= 128:
            attrs += " __attribute__((amdgpu_waves_per_eu(1, 1)))"
        elif self.dot_plans and self.nt <= 256 and not self.opt.get("no_occupancy_hint"):
            # Two waves per SIMD for MFMA loops: the second wave covers LDS and barrier
            # latency. hiprtc otherwise settles on one wave when it can use >256 registers.
            attrs += f" __attribute__((amdgpu_waves_per_eu({int(self.opt.get('waves_per_eu', 2))})))"
        out.append(f'extern "C" __global__ void {attrs} {kname}('
                   + ", ".join(params) + ") {")
        # Stage buffers share the LDS block with the scratch used for conversions and
        # reductions when no scratch user runs inside a staged loop (the stage prologue and
        # every scratch user start with a barrier); otherwise they follow the scratch.
        scratch = (self.lds + 15) // 16 * 16
        off = 0 if not getattr(self, "scratch_in_stage_loop", False) else scratch
        stage_offs = []
        for nm_, nb_ in self.extra_smem:
            stage_offs.append((nm_, off))
            off += (nb_ + 15) // 16 * 16
        total = max(scratch, off)
        if total:
            out.append(f"  __shared__ __attribute__((aligned(16))) char ek_smem[{total}];")
        for nm_, o_ in stage_offs:
            out.append(f"  char* const {nm_} = ek_smem + {o_};")
        self.lds = total
        out.append("  const int ek_tid = threadIdx.x;")
        out.append("  const int ek_lane = ek_tid & 63;")
        out.append("  const int ek_warp = ek_tid >> 6;")
        out.append("  (void)ek_lane; (void)ek_warp; (void)ek_tid;")
        if self.remap_pids:
            out.extend(PID_REMAP)
        out.extend(self.prologue)

        def flat(items):
            for it in items:
                if isinstance(it, list):
                    yield from flat(it)
                else:
                    yield it
        body = list(flat(self.scopes[0].items))
        if self.priv:
            cop = self.priv_copies
            for info in self.priv.values():
                t = "int32_t" if info["dt"].name == "i32" else "uint32_t"
                n = info["bins"] * cop
                out.append(f"  __shared__ __attribute__((aligned(16))) {t} {info['name']}[{n}];")
                out.append(f"  for (int i = ek_tid; i < {n}; i += {self.nt}) {info['name']}[i] = 0;")
            out.append("  __syncthreads();")
        if self.coarsen:
            # Program coarsening: a capped grid of workgroups walks the logical program ids
            # (programs are independent; privatised atomics commute). The walk is unrolled
            # by U programs, each in its own scope, so the compiler can issue the U
            # programs' global loads before the first program's LDS atomics: a workgroup
            # keeps U loads in flight instead of one.
            u_ = max(1, int(self.opt.get("coarsen_unroll", 4)))
            # The walk is emitted twice: a 1-D launch (the common case) takes the program id
            # as is, other launches split it with integer divisions per program.
            flat = ["  const int ek_pid_x = ek_p, ek_pid_y = 0, ek_pid_z = 0;",
                    "  (void)ek_pid_x; (void)ek_pid_y; (void)ek_pid_z;"]
            general = ["  const int ek_pid_x = ek_p % ek_np_x;",
                       "  const int ek_pid_y = (ek_p / ek_np_x) % ek_np_y;",
                       "  const int ek_pid_z = ek_p / (ek_np_x * ek_np_y);",
                       "  (void)ek_pid_x; (void)ek_pid_y; (void)ek_pid_z;"]
            out.append("  const int ek_nprog = ek_np_x * ek_np_y * ek_np_z;")
            out.append("  const int ek_g = (int)gridDim.x;")
            for n_, pids in enumerate((flat, general)):
                out.append("  if (ek_np_y == 1 && ek_np_z == 1) {" if n_ == 0 else "  } else {")
                out.append("  int ek_p0 = blockIdx.x;")
                if u_ > 1:
                    out.append(f"  for (; ek_p0 + {u_ - 1} * ek_g < ek_nprog; "
                               f"ek_p0 += {u_} * ek_g) {{")
                    for k_ in range(u_):
                        out.append(f"  {{ const int ek_p = ek_p0 + {k_} * ek_g;")
                        out.extend(pids)
                        out.extend(body)
                        out.append("  }")
                    out.append("  }")
                out.append("  for (int ek_p = ek_p0; ek_p < ek_nprog; ek_p += ek_g) {")
                out.extend(pids)
                out.extend(body)
                out.append("  }")
            out.append("  }")
        else:
            out.extend(body)
        if two:
            out.append("  __syncthreads();")
            for info in self.priv.values():
                out.append(f"  for (int i = ek_tid; i < {info['bins']}; i += {self.nt}) "
                           f"ek_part[(size_t)blockIdx.x * {total_words} + {info['off']} + i] = "
                           f"(int32_t){info['name']}[i];")
        elif self.priv:
            # Flush: a wave reads consecutive words (whole groups of C copies), sums each group
            # with butterfly shuffles and one lane adds the bin's total to global memory.
            out.append("  __syncthreads();")
            cop = self.priv_copies
            for rid, info in self.priv.items():
                base = self.name[info["base"].id]
                n = info["bins"] * cop
                out.append(f"  for (int i = ek_tid; i < {(n + 63) // 64 * 64}; i += {self.nt}) {{")
                out.append(f"    auto v = i < {n} ? {info['name']}[i] : 0;")
                o = 1
                while o < cop:
                    out.append(f"    v += ek::shfl(v, ek_lane ^ {o});")
                    o *= 2
                out.append(f"    if (i < {n} && (i & {cop - 1}) == 0 && v) "
                           f"__hip_atomic_fetch_add({base} + i / {cop}, v, __ATOMIC_RELAXED, "
                           "__HIP_MEMORY_SCOPE_AGENT);")
                out.append("  }")
        out.append("}")
        flush = None
        if two:
            rb = int(self.opt.get("priv_flush_rows", 256))
            fname = f"{kname}_flush"
            T_ = total_words
            infos = list(self.priv.values())
            hs = [f"{ctype(i['dt'])}* ek_h{k}" for k, i in enumerate(infos)]
            out += ["", "// Second level of the privatised-bin flush: workgroup (x, y) sums words "
                    f"[64x, 64x+64) of the partial", f"// rows [y*{rb}, y*{rb}+{rb}), 16 rows at a "
                    "time with 16-byte loads, reduces the 16 row lanes in LDS",
                    "// and adds each non-zero sum to the kernel's bins with one atomic.",
                    f'extern "C" __global__ void __launch_bounds__(256) {fname}('
                    "const int32_t* __restrict__ ek_part, int32_t ek_nwg, " + ", ".join(hs) + ") {",
                    "  __shared__ int32_t ek_red[16][64];",
                    "  const int t = threadIdx.x, seg = t & 15, rl = t >> 4;",
                    "  const int w0 = blockIdx.x * 64 + seg * 4;",
                    f"  const int p0 = blockIdx.y * {rb}, p1 = min(ek_nwg, p0 + {rb});",
                    "  ek::i32x4 s = {0, 0, 0, 0};",
                    f"  if (w0 < {T_}) {{",
                    "    #pragma unroll 8",
                    "    for (int w = p0 + rl; w < p1; w += 16) s += __builtin_nontemporal_load("
                    f"reinterpret_cast<const ek::i32x4*>(ek_part + (size_t)w * {T_} + w0));",
                    "  }",
                    "  #pragma unroll",
                    "  for (int j = 0; j < 4; ++j) ek_red[rl][seg * 4 + j] = s[j];",
                    "  __syncthreads();",
                    "  if (t < 64) {",
                    "    int32_t v = 0;",
                    "    #pragma unroll",
                    "    for (int r = 0; r < 16; ++r) v += ek_red[r][t];",
                    "    const int w = blockIdx.x * 64 + t;",
                    "    if (v) {"]
            for k, info in enumerate(infos):
                B, O = info["bins"], info["off"]
                kw = "if" if k == 0 else "else if"
                out.append(f"      {kw} (w >= {O} && w < {O + B}) __hip_atomic_fetch_add("
                           f"ek_h{k} + (w - {O}), ({ctype(info['dt'])})v, __ATOMIC_RELAXED, "
                           "__HIP_MEMORY_SCOPE_AGENT);")
            out += ["    }", "  }", "}"]
            bases = [fn.args.index(i["base"]) for i in infos]
            flush = {"name": fname, "rb": rb, "bases": bases, "total": total_words,
                     "chunks": (total_words + 63) // 64}
        gk = GeneratedKernel(kname, "\n".join(out) + "\n", args, self.nw, self.lds, self.nt)
        gk.coarsen = int(self.coarsen)
        gk.asserts = list(self.asserts)
        gk.flush = flush
        gk.report = self.report
        return gk


# Program-id remapping for kernels with tl.dot (programs are independent, so any bijection
# of program ids is allowed). Hardware hands consecutive workgroups to the 8 XCDs round
# robin; remapping makes the programs on one XCD consecutive, grouped in bands of 4 rows of
# axis 1, so they share operand tiles in that XCD's L2. Axis 0 runs in reverse so that in
# causal attention the longest programs start first.
PID_REMAP = [
    "  int ek_pid_x, ek_pid_y;",
    "  const int ek_pid_z = blockIdx.z;",
    "  {",
    "    const int gx = gridDim.x, gy = gridDim.y, nb = gx * gy;",
    "    int L = blockIdx.x + gx * blockIdx.y;",
    "    if ((nb & 7) == 0) L = (L & 7) * (nb >> 3) + (L >> 3);",
    "    const int band = 4 * gx, first = (L / band) * 4;",
    "    const int gs = (gy - first) < 4 ? (gy - first) : 4, r = L % band;",
    "    ek_pid_y = first + r % gs;",
    "    ek_pid_x = gx - 1 - r / gs;",
    "  }",
    "  (void)ek_pid_x; (void)ek_pid_y; (void)ek_pid_z;",
]


def generate(fn: ir.Func, options: dict | None = None) -> GeneratedKernel:
    return Emitter(fn, options).run()


def arg_offsets(kargs: list[KernelArg]) -> list[int]:
    """Byte offset of each argument in the kernarg layout that `pack_args` builds."""
    offs, n = [], 0
    for ka in kargs:
        if ka.kind == "ptr":
            size = 8
        else:
            size = {"int32_t": 4, "int64_t": 8, "uint32_t": 4, "uint64_t": 8, "float": 4,
                    "int16_t": 2, "uint16_t": 2, "int8_t": 1, "uint8_t": 1}[ka.cparam]
        n += (-n) % size
        offs.append(n)
        n += size
    return offs


def pack_args(kargs: list[KernelArg], values: list, pad8: bool = True) -> bytes:
    """Packs runtime argument values into the kernarg layout (natural alignment)."""
    buf = bytearray()
    for ka, v in zip(kargs, values):
        if ka.kind == "ptr":
            fmt, size = "Q", 8
            v = int(v)
        else:
            cp = ka.cparam
            fmt, size = {"int32_t": ("i", 4), "int64_t": ("q", 8), "uint32_t": ("I", 4),
                         "uint64_t": ("Q", 8), "float": ("f", 4), "int16_t": ("h", 2),
                         "uint16_t": ("H", 2), "int8_t": ("b", 1), "uint8_t": ("B", 1)}[cp]
            if fmt == "f":
                # C's double -> float conversion (round to nearest even; beyond the float
                # range, +-inf), which struct would refuse with OverflowError
                with np.errstate(over="ignore"):
                    v = float(np.float32(float(v)))
            else:
                v = int(v)
        pad = (-len(buf)) % size
        buf += b"\0" * pad
        buf += struct.pack("<" + fmt, v)
    if pad8:
        buf += b"\0" * ((-len(buf)) % 8)
    else:
        buf += b"\0" * ((-len(buf)) % 4)
    return bytes(buf)
