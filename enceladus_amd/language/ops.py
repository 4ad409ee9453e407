"""The `tl` builtins: each one builds IR when a kernel is compiled.

Calling a builtin outside a kernel raises. Signatures and semantics follow the reference
language (reference: src/enceladus/language/ops.py; op index in SURVEY-listed lines
136-2074: program_id :141, arange :179, full :203, load :305, store :365,
make_tensor_descriptor :437, where :557, to :668, sum :983, max :1015, dot :1244,
atomic_add :1943, cumsum :2064).
"""

from __future__ import annotations

import builtins as _bi
import math as _pymath
from typing import Any

from enceladus_amd.compiler import frontend as F
from enceladus_amd.compiler import ir, semantic
from enceladus_amd.compiler.errors import CompilationError
from enceladus_amd.language import core


class Builtin:
    def __init__(self, name: str, frontend):
        self.__name__ = name
        self._ek_frontend = frontend
        self.__doc__ = frontend.__doc__

    def __call__(self, *args, **kwargs):
        raise RuntimeError(f"tl.{self.__name__} can only be called inside an @enceladus.jit "
                           "kernel")

    def __repr__(self):
        return f"<tl.{self.__name__}>"


def builtin(name: str | None = None):
    def deco(f):
        return Builtin(name or f.__name__.rstrip("_"), f)
    return deco


def _cint(v: Any, what: str) -> int:
    v = core.unwrap(v)
    if isinstance(v, ir.Value) or isinstance(v, bool) or not isinstance(v, int):
        raise CompilationError(f"{what} must be a compile-time integer, but got {v!r}")
    return v


def _dtype(v: Any, what: str = "dtype") -> core.dtype:
    v = core.unwrap(v)
    if isinstance(v, core.dtype):
        return v
    if isinstance(v, str):
        return core.dtype_from_name(v)
    raise CompilationError(f"{what} must be a tl dtype, but got {v!r}")


def _axis(axis: Any, rank: int) -> int:
    a = _cint(axis, "axis")
    if not -rank <= a < rank:
        raise CompilationError(f"axis {a} is out of range for a rank-{rank} tile")
    return a % rank


def _tile(ctx, x, what: str) -> ir.Value:
    x = core.unwrap(x)
    if not isinstance(x, ir.Value):
        x = semantic.to_value(ctx.b, x)
    if isinstance(x.type, ir.DescType):
        raise CompilationError(f"tl.{what} can't take a tensor descriptor")
    return x


def _shape(shape) -> tuple[int, ...]:
    shape = core.unwrap(shape)
    if isinstance(shape, int):
        shape = (shape,)
    return semantic.check_shape(shape, "tile shape")


# -- program structure ----------------------------------------------------------

@builtin()
def program_id(ctx, axis):
    a = _cint(axis, "axis")
    if a not in (0, 1, 2):
        raise CompilationError(f"program_id axis must be 0, 1, or 2, got {a}")
    return ctx.b.create("program_id", [], [ir.TType((), core.int32)], {"axis": a}).result


@builtin()
def num_programs(ctx, axis):
    a = _cint(axis, "axis")
    if a not in (0, 1, 2):
        raise CompilationError(f"num_programs axis must be 0, 1, or 2, got {a}")
    return ctx.b.create("num_programs", [], [ir.TType((), core.int32)], {"axis": a}).result


@builtin()
def arange(ctx, start, end):
    s, e = _cint(start, "arange start"), _cint(end, "arange end")
    n = e - s
    if n <= 0 or n & (n - 1) or n > ir.MAX_TILE_NUMEL:
        raise CompilationError(f"arange({s}, {e}) must have a power-of-two length "
                               f"<= {ir.MAX_TILE_NUMEL}")
    return ctx.b.create("arange", [], [ir.TType((n,), core.int32)], {"start": s}).result


@builtin()
def full(ctx, shape, value, dtype):
    dt = _dtype(dtype)
    shp = _shape(shape)
    v = core.unwrap(value)
    if isinstance(v, ir.Value):
        if v.type.shape != ():
            raise CompilationError("tl.full needs a scalar value")
        return semantic.broadcast_to(ctx.b, semantic.cast(ctx.b, v, dt), shp)
    return semantic.const(ctx.b, v, dt, shp)


@builtin()
def zeros(ctx, shape, dtype):
    return full._ek_frontend(ctx, shape, 0, dtype)


@builtin()
def zeros_like(ctx, input):
    x = _tile(ctx, input, "zeros_like")
    return semantic.const(ctx.b, 0, x.type.dtype, x.type.shape)


@builtin()
def full_like(ctx, input, value, dtype=None):
    x = _tile(ctx, input, "full_like")
    dt = x.type.dtype if dtype is None else _dtype(dtype)
    return full._ek_frontend(ctx, x.type.shape or (1,), value, dt) if x.type.shape else \
        semantic.to_value(ctx.b, value, dt)


# -- memory -------------------------------------------------------------------------

def _check_mask(m: ir.Value):
    if not m.type.dtype.is_bool():
        raise CompilationError(f"a mask must be a boolean (int1) tile, such as `offs < n`, "
                               f"but got {m.type.dtype}")


def _ptr(x, what):
    x = core.unwrap(x)
    if not (isinstance(x, ir.Value) and x.type.ptr):
        raise CompilationError(f"tl.{what} needs a pointer or pointer tile")
    return x


@builtin()
def load(ctx, pointer, mask=None, other=None, boundary_check=(), padding_option="",
         cache_modifier="", eviction_policy="", volatile=False):
    """Loads from a pointer tile; masked-off lanes read `other` (0 by default)."""
    b = ctx.b
    p = _ptr(pointer, "load")
    if boundary_check or padding_option:
        raise CompilationError("block pointers aren't supported; use tl.make_tensor_descriptor")
    elem = p.type.dtype
    mask = core.unwrap(mask)
    rt = ir.TType(p.type.shape, elem)
    if mask is None or mask is True:
        return b.create("load", [p], [rt]).result
    if not isinstance(mask, ir.Value):
        raise CompilationError("`mask` must be a boolean tile")
    _check_mask(mask)
    shape = semantic.broadcast_shapes(p.type.shape, mask.type.shape)
    p = semantic.broadcast_to(b, p, shape)
    mask = semantic.broadcast_to(b, mask, shape)
    o = core.unwrap(other)
    ov = semantic.to_value(b, 0 if o is None else o, elem)
    ov = semantic.broadcast_to(b, ov, shape)
    return b.create("load", [p, mask, ov], [ir.TType(shape, elem)]).result


@builtin()
def store(ctx, pointer, value, mask=None, boundary_check=(), cache_modifier="",
          eviction_policy=""):
    """Stores `value` through a pointer tile where `mask` is true."""
    b = ctx.b
    p = _ptr(pointer, "store")
    v = core.unwrap(value)
    if isinstance(v, ir.Value) and v.type.ptr:
        raise CompilationError("tl.store can't store pointers")
    v = semantic.to_value(b, v, p.type.dtype)
    mask = core.unwrap(mask)
    shape = semantic.broadcast_shapes(p.type.shape, v.type.shape)
    if mask is not None and mask is not True:
        if not isinstance(mask, ir.Value):
            raise CompilationError("`mask` must be a boolean tile")
        _check_mask(mask)
        shape = semantic.broadcast_shapes(shape, mask.type.shape)
    if shape != p.type.shape:
        p = semantic.broadcast_to(b, p, shape)
    v = semantic.broadcast_to(b, v, shape)
    ops = [p, v]
    if mask is not None and mask is not True:
        ops.append(semantic.broadcast_to(b, mask, shape))
    b.create("store", ops)
    return None


@builtin()
def make_tensor_descriptor(ctx, base, shape, strides, block_shape, padding_option="zero"):
    """Describes a strided 2D+ array; `desc.load/store` move whole blocks, zero-padded."""
    b = ctx.b
    base = core.unwrap(base)
    if not (isinstance(base, ir.Value) and base.type.ptr and base.type.shape == ()):
        raise CompilationError("tl.make_tensor_descriptor needs a scalar base pointer")
    shape, strides = list(core.unwrap(shape)), list(core.unwrap(strides))
    block = semantic.check_shape(core.unwrap(block_shape), "tensor descriptor block")
    if not (len(shape) == len(strides) == len(block)):
        raise CompilationError("shape, strides and block_shape need the same rank")
    if padding_option not in ("zero", "", None):
        raise CompilationError('tensor descriptors support only zero padding')
    if not ctx.is_known_one(strides[-1]):
        raise CompilationError("the last stride of a tensor descriptor must be 1")
    vals = []
    for v in [*shape, *strides]:
        v = core.unwrap(v)
        if isinstance(v, ir.Value):
            if v.type.shape != () or not v.type.dtype.is_int():
                raise CompilationError("descriptor shape/stride entries must be integer scalars")
            vals.append(semantic.cast(b, v, core.int64) if v.type.dtype in
                        (core.uint32, core.uint64) else v)
        else:
            vals.append(semantic.to_value(b, int(v)))
    t = ir.DescType(base.type.dtype, block)
    return b.create("make_desc", [base, *vals], [t]).result


def _offsets(ctx, desc, offsets):
    offs = list(core.unwrap(offsets))
    if len(offs) != desc.type.rank:
        raise CompilationError(f"the descriptor has rank {desc.type.rank}, but got "
                               f"{len(offs)} offsets")
    out = []
    for o in offs:
        v = semantic.to_value(ctx.b, o)
        if v.type.shape != () or not v.type.dtype.is_int():
            raise CompilationError("descriptor offsets must be integer scalars")
        out.append(v)
    return out


def _desc_load(ctx, desc, offsets):
    offs = _offsets(ctx, desc, offsets)
    t = ir.TType(desc.type.block_shape, desc.type.dtype)
    return ctx.b.create("desc_load", [desc, *offs], [t]).result


def _desc_store(ctx, desc, offsets, value):
    offs = _offsets(ctx, desc, offsets)
    v = semantic.to_value(ctx.b, value, desc.type.dtype)
    if v.type.shape != desc.type.block_shape:
        v = semantic.broadcast_to(ctx.b, v, desc.type.block_shape)
    ctx.b.create("desc_store", [desc, *offs, v])


F.DESC_METHODS["load"] = _desc_load
F.DESC_METHODS["store"] = _desc_store


# -- elementwise --------------------------------------------------------------------

@builtin()
def where(ctx, condition, x, y):
    return semantic.select(ctx.b, condition, x, y)


@builtin()
def maximum(ctx, x, y):
    return semantic.binary(ctx.b, "max", x, y)


@builtin()
def minimum(ctx, x, y):
    return semantic.binary(ctx.b, "min", x, y)


@builtin()
def fma(ctx, x, y, z):
    b = ctx.b
    dts = [semantic.dtype_of(v) for v in (x, y, z)]
    dt = semantic.computation_dtype("mul", dts[0], dts[1])
    dt = semantic.computation_dtype("add", dt, dts[2])
    if not dt.is_floating():
        return semantic.binary(b, "add", semantic.binary(b, "mul", x, y), z)
    vs = [semantic.to_value(b, v, dt) for v in (x, y, z)]
    shape = ()
    for v in vs:
        shape = semantic.broadcast_shapes(shape, v.type.shape)
    vs = [semantic.broadcast_to(b, v, shape) for v in vs]
    return b.create("fma", vs, [ir.TType(shape, dt)]).result


@builtin(name="abs")
def abs_(ctx, x):
    x = _tile(ctx, x, "abs")
    if x.type.dtype.is_unsigned():
        return x
    return semantic.unary(ctx.b, "abs", x)


@builtin()
def cdiv(ctx, x, div):
    xv, dv = core.unwrap(x), core.unwrap(div)
    if not isinstance(xv, ir.Value) and not isinstance(dv, ir.Value):
        return -(-xv // dv)
    b = ctx.b
    return semantic.binary(b, "floordiv", semantic.binary(b, "sub",
                           semantic.binary(b, "add", x, div), 1), div)


@builtin()
def clamp(ctx, x, min, max):
    b = ctx.b
    return semantic.binary(b, "min", semantic.binary(b, "max", x, min), max)


def _to(ctx, x, dtype, bitcast=False, fp_downcast_rounding=None):
    x = _tile(ctx, x, "to")
    return semantic.cast(ctx.b, x, _dtype(dtype), bool(core.unwrap(bitcast)))


F.TILE_METHODS["to"] = _to


@builtin()
def cast(ctx, input, dtype, bitcast=False, fp_downcast_rounding=None):
    return _to(ctx, input, dtype, bitcast)


for _m in ("exp", "exp2", "log", "log2", "sqrt", "rsqrt", "sin", "cos", "tanh", "sigmoid",
           "erf", "floor", "ceil"):
    def _mk(opname):
        def f(ctx, x):
            return semantic.unary(ctx.b, opname, x)
        f.__name__ = opname
        return Builtin(opname, f)
    globals()[_m] = _mk(_m)
    F.TILE_METHODS[_m] = (lambda opname: (lambda ctx, x: semantic.unary(ctx.b, opname, x)))(_m)


# -- shape ops ----------------------------------------------------------------------

@builtin()
def broadcast_to(ctx, input, *shape):
    if len(shape) == 1 and isinstance(core.unwrap(shape[0]), (tuple, list)):
        shape = tuple(core.unwrap(shape[0]))
    x = _tile(ctx, input, "broadcast_to")
    return semantic.broadcast_to(ctx.b, x, _shape(shape))


@builtin()
def expand_dims(ctx, input, axis):
    x = _tile(ctx, input, "expand_dims")
    axes = core.unwrap(axis)
    axes = list(axes) if isinstance(axes, (tuple, list)) else [axes]
    rank = len(x.type.shape) + len(axes)
    for a in sorted(_axis(a, rank) for a in axes):
        x = semantic.expand_dims(ctx.b, x, a)
    return x


@builtin()
def reshape(ctx, input, *shape, can_reorder=False):
    if len(shape) == 1 and isinstance(core.unwrap(shape[0]), (tuple, list)):
        shape = tuple(core.unwrap(shape[0]))
    x = _tile(ctx, input, "reshape")
    shp = _shape(shape)
    if ir.TType(shp, x.type.dtype).numel != x.type.numel:
        raise CompilationError(f"can't reshape {x.type.shape} to {shp}")
    if shp == x.type.shape:
        return x
    return ctx.b.create("reshape", [x], [x.type.with_shape(shp)]).result


def _trans(ctx, input, *dims):
    x = _tile(ctx, input, "trans")
    rank = len(x.type.shape)
    if len(dims) == 1 and isinstance(core.unwrap(dims[0]), (tuple, list)):
        dims = tuple(core.unwrap(dims[0]))
    if not dims:
        if rank != 2:
            raise CompilationError("tl.trans without dims needs a 2D tile")
        dims = (1, 0)
    perm = tuple(_axis(d, rank) for d in dims)
    if sorted(perm) != list(_bi.range(rank)):
        raise CompilationError(f"{perm} isn't a permutation")
    if perm == tuple(_bi.range(rank)):
        return x
    shape = tuple(x.type.shape[p] for p in perm)
    return ctx.b.create("trans", [x], [x.type.with_shape(shape)], {"perm": perm}).result


F.TILE_METHODS["trans"] = _trans
trans = Builtin("trans", _trans)
permute = Builtin("permute", _trans)


# -- reductions and scans -----------------------------------------------------------

def _sum_input_dtype(dt: core.dtype) -> core.dtype:
    if dt.is_int() and dt.primitive_bitwidth < 32:
        return core.uint32 if dt.kind == "uint" else core.int32
    return dt


def _reduce(ctx, input, axis, kind, keep_dims, dtype=None):
    b = ctx.b
    v = _tile(ctx, input, kind)
    if v.type.ptr:
        raise CompilationError(f"tl.{kind} can't reduce pointers")
    if dtype is not None:
        v = semantic.cast(b, v, _dtype(dtype))
    if kind == "sum":
        v = semantic.cast(b, v, _sum_input_dtype(v.type.dtype))
    rank = len(v.type.shape)
    if rank == 0:
        return v
    axis = core.unwrap(axis)
    if axis is None:
        if rank > 1:
            v = b.create("reshape", [v], [v.type.with_shape((v.type.numel,))]).result
        ax = 0
    else:
        ax = _axis(axis, rank)
    s = list(v.type.shape)
    del s[ax]
    elem = core.int32 if kind in ("argmax", "argmin") else v.type.dtype
    r = b.create("reduce", [v], [ir.TType(tuple(s), elem)], {"axis": ax, "kind": kind}).result
    if core.unwrap(keep_dims):
        if axis is None:
            return semantic.broadcast_to(b, r, (1,) * rank)
        r = semantic.expand_dims(b, r, ax)
    return r


@builtin(name="sum")
def sum_(ctx, input, axis=None, keep_dims=False, dtype=None):
    return _reduce(ctx, input, axis, "sum", keep_dims, dtype)


@builtin(name="max")
def max_(ctx, input, axis=None, return_indices=False, return_indices_tie_break_left=True,
         keep_dims=False):
    if core.unwrap(return_indices):
        return (_reduce(ctx, input, axis, "max", keep_dims),
                _reduce(ctx, input, axis, "argmax", keep_dims))
    return _reduce(ctx, input, axis, "max", keep_dims)


@builtin(name="min")
def min_(ctx, input, axis=None, return_indices=False, return_indices_tie_break_left=True,
         keep_dims=False):
    if core.unwrap(return_indices):
        return (_reduce(ctx, input, axis, "min", keep_dims),
                _reduce(ctx, input, axis, "argmin", keep_dims))
    return _reduce(ctx, input, axis, "min", keep_dims)


@builtin()
def argmax(ctx, input, axis, tie_break_left=True, keep_dims=False):
    return _reduce(ctx, input, axis, "argmax", keep_dims)


@builtin()
def argmin(ctx, input, axis, tie_break_left=True, keep_dims=False):
    return _reduce(ctx, input, axis, "argmin", keep_dims)


for _k in ("sum", "max", "min", "argmax", "argmin"):
    F.TILE_METHODS[_k] = (lambda k: (lambda ctx, x, axis=None, keep_dims=False:
                                     _reduce(ctx, x, axis, k, keep_dims)))(_k)


@builtin()
def cumsum(ctx, input, axis=0, reverse=False, dtype=None):
    b = ctx.b
    v = _tile(ctx, input, "cumsum")
    if dtype is not None:
        v = semantic.cast(b, v, _dtype(dtype))
    v = semantic.cast(b, v, _sum_input_dtype(v.type.dtype))
    rank = len(v.type.shape)
    if rank == 0:
        raise CompilationError("tl.cumsum needs a tile")
    ax = _axis(axis, rank)
    return b.create("scan", [v], [v.type], {"axis": ax, "kind": "sum",
                                              "reverse": bool(core.unwrap(reverse))}).result


F.TILE_METHODS["cumsum"] = lambda ctx, x, axis=0, reverse=False: cumsum._ek_frontend(
    ctx, x, axis, reverse)


# -- dot ----------------------------------------------------------------------------

_DOT_FLOAT = (core.float16, core.bfloat16, core.float32)


@builtin()
def dot(ctx, input, other, acc=None, input_precision=None, allow_tf32=None,
        max_num_imprecise_acc=None, out_dtype=None):
    """Matrix product of two 2D tiles, accumulated in fp32 (floats) or int32 (ints)."""
    b = ctx.b
    a = _tile(ctx, input, "dot")
    bt = _tile(ctx, other, "dot")
    if len(a.type.shape) != 2 or len(bt.type.shape) != 2:
        raise CompilationError(f"tl.dot needs 2D tiles, got {a.type.shape} and "
                               f"{bt.type.shape}")
    if a.type.shape[1] != bt.type.shape[0]:
        raise CompilationError(f"tl.dot inner dimensions differ: {a.type.shape} @ "
                               f"{bt.type.shape}")
    if a.type.dtype is not bt.type.dtype:
        raise CompilationError(f"tl.dot needs operands of the same dtype, got "
                               f"{a.type.dtype} and {bt.type.dtype}")
    m, n = a.type.shape[0], bt.type.shape[1]
    adt = a.type.dtype
    acc = core.unwrap(acc)
    if acc is None:
        if adt.is_int():
            out_dt = core.int32
        else:
            out_dt = core.float32 if out_dtype is None else _dtype(out_dtype)
        accv = semantic.const(b, 0, out_dt, (m, n))
    else:
        accv = _tile(ctx, acc, "dot")
        out_dt = accv.type.dtype
        if accv.type.shape != (m, n):
            raise CompilationError(f"the tl.dot accumulator must be {m}x{n}, got "
                                   f"{accv.type.shape}")
    if adt.is_int():
        if out_dt is not core.int32:
            raise CompilationError("tl.dot accumulates integer operands in int32")
        raise CompilationError("integer tl.dot isn't supported by the MI355X backend yet")
    if adt not in _DOT_FLOAT:
        raise CompilationError(f"tl.dot supports float16, bfloat16 and float32 operands, "
                               f"got {adt}")
    if out_dt not in (core.float32, core.float16):
        raise CompilationError("tl.dot accumulates float operands in float32 or float16")
    return b.create("dot", [a, bt, accv], [ir.TType((m, n), out_dt)]).result


# -- atomics ------------------------------------------------------------------------

_ATOMIC_BITWISE = ("and", "or", "xor")


def _atomic(ctx, kind, pointer, vals, mask, sem, scope):
    b = ctx.b
    p = _ptr(pointer, f"atomic_{kind}")
    dt = p.type.dtype
    if dt.is_bool():
        raise CompilationError(f"tl.atomic_{kind} doesn't support int1 pointers")
    if dt.is_floating() and kind in _ATOMIC_BITWISE:
        raise CompilationError(f"tl.atomic_{kind} needs integer elements")
    if kind == "add" and dt in (core.float16, core.bfloat16):
        raise CompilationError(f"tl.atomic_add doesn't support {dt}")
    if dt.primitive_bitwidth == 64 and not (dt is core.uint64 and kind in ("max", "min")):
        raise CompilationError(f"tl.atomic_{kind} doesn't support {dt}")
    vs = [semantic.to_value(b, v, dt) for v in vals]
    mask = core.unwrap(mask)
    if mask is True:
        mask = None
    if mask is not None:
        if not isinstance(mask, ir.Value):
            raise CompilationError("`mask` must be a boolean tile")
        _check_mask(mask)
    shape = p.type.shape
    for v in [*vs, *([mask] if mask is not None else [])]:
        shape = semantic.broadcast_shapes(shape, v.type.shape)
    ops = [semantic.broadcast_to(b, p, shape)] + [semantic.broadcast_to(b, v, shape) for v in vs]
    if mask is not None:
        ops.append(semantic.broadcast_to(b, mask, shape))
    rt = ir.TType(shape, dt)
    if kind == "cas":
        return b.create("atomic_cas", ops, [rt], {"has_mask": mask is not None}).result
    return b.create("atomic_rmw", ops, [rt], {"op": kind, "has_mask": mask is not None}).result


def _mk_atomic(kind):
    def f(ctx, pointer, val, mask=None, sem=None, scope=None):
        return _atomic(ctx, kind, pointer, [val], mask, sem, scope)
    return Builtin(f"atomic_{kind}", f)


atomic_add = _mk_atomic("add")
atomic_max = _mk_atomic("max")
atomic_min = _mk_atomic("min")
atomic_xchg = _mk_atomic("xchg")
atomic_and = _mk_atomic("and")
atomic_or = _mk_atomic("or")
atomic_xor = _mk_atomic("xor")


@builtin()
def atomic_cas(ctx, pointer, cmp, val, sem=None, scope=None):
    return _atomic(ctx, "cas", pointer, [cmp, val], None, sem, scope)


# -- compile-time helpers -----------------------------------------------------------

class _StaticRange:
    _ek_static_range = True

    def __call__(self, *a):
        raise RuntimeError("tl.static_range can only be used in a kernel `for` loop")


class _Range:
    _ek_range = True

    def __call__(self, *a, **k):
        raise RuntimeError("tl.range can only be used in a kernel `for` loop")


static_range = _StaticRange()
range = _Range()  # noqa: A001 - tl.range


@builtin()
def static_assert(ctx, cond, msg=""):
    c = core.unwrap(cond)
    if isinstance(c, ir.Value):
        raise CompilationError("tl.static_assert needs a compile-time condition")
    if not c:
        raise CompilationError(f"static_assert failed: {core.unwrap(msg)}")


@builtin()
def static_print(ctx, *values, sep=" "):
    print(*[core.unwrap(v) for v in values], sep=sep)


@builtin()
def debug_barrier(ctx):
    ctx.b.create("barrier", [])


@builtin()
def multiple_of(ctx, input, values):
    x = core.unwrap(input)
    if isinstance(x, ir.Value):
        vals = core.unwrap(values)
        vals = list(vals) if isinstance(vals, (list, tuple)) else [vals]
        return ctx.b.create("hint", [x], [x.type], {"multiple_of": tuple(int(v) for v in vals)}).result
    return x


@builtin()
def max_contiguous(ctx, input, values):
    x = core.unwrap(input)
    if isinstance(x, ir.Value):
        vals = core.unwrap(values)
        vals = list(vals) if isinstance(vals, (list, tuple)) else [vals]
        return ctx.b.create("hint", [x], [x.type], {"max_contiguous": tuple(int(v) for v in vals)}).result
    return x


@builtin()
def device_assert(ctx, cond, msg="", mask=None):
    """Checks `cond` (where `mask` is true) on the device when ENCELADUS_DEBUG=1; the first
    failing program is reported as `DeviceAssertionError` when the launch completes. Without
    ENCELADUS_DEBUG the check is compiled out (reference: language/ops.py:1480-1500,
    codegen/debug.py:123-158)."""
    if not ctx.options.get("debug"):
        return None
    b = ctx.b
    c = semantic.to_value(b, cond)
    if not c.type.dtype.is_bool():
        c = semantic.binary(b, "ne", c, 0)
    ops_ = [c]
    if mask is not None:
        m = semantic.to_value(b, mask)
        shape = semantic.broadcast_shapes(c.type.shape, m.type.shape)
        ops_ = [semantic.broadcast_to(b, c, shape), semantic.broadcast_to(b, m, shape)]
    b.create("assert", ops_, [], {"msg": str(core.unwrap(msg))})
    return None


@builtin()
def device_print(ctx, prefix, *args, hex=False):
    """Prints from the device with printf: one line per element a thread owns, as
    `pid (x, y, z) idx (i, ...) prefix: values` (reference: codegen/debug.py:84-120)."""
    b = ctx.b
    vals = [semantic.to_value(b, a) for a in args]
    shape = ()
    for v in vals:
        shape = semantic.broadcast_shapes(shape, v.type.shape)
    vals = [semantic.broadcast_to(b, v, shape) for v in vals]
    b.create("print", vals, [], {"prefix": str(core.unwrap(prefix)),
                                 "hex": bool(core.unwrap(hex))})
    return None
