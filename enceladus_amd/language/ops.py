"""The `tl` builtins: each one builds IR when a kernel is compiled.

Calling a builtin outside a kernel raises. Signatures and semantics follow the reference
language (reference: src/enceladus/language/ops.py, lines 136-2074: program_id :141,
arange :179, full :203, load :305, store :365, make_tensor_descriptor :437, where :557,
to :668, join :840, split :875, sum :983, max :1015, reduce :1100, dot :1244,
atomic_add :1943, cumsum :2064, associative_scan :2097).
"""

from __future__ import annotations

import builtins as _bi
import inspect
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

    @property
    def __signature__(self) -> inspect.Signature:
        """The signature user code calls: the frontend's without the compiler context."""
        sig = inspect.signature(self._ek_frontend)
        return sig.replace(parameters=list(sig.parameters.values())[1:])

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
    if isinstance(v, ir.Value):
        nm = v.name_hint or "it"
        raise CompilationError(
            f"{what} must be a compile-time integer, but `{nm}` is a runtime value. If it is "
            f"a kernel parameter, annotate it as `{nm}: tl.constexpr`.")
    if isinstance(v, bool) or not isinstance(v, int):
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
                               f"<= {ir.MAX_TILE_NUMEL}. Round the block size up to a power "
                               "of two and mask the extra elements.")
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
def cast(ctx, x, dtype, bitcast=False, fp_downcast_rounding=None):
    return _to(ctx, x, dtype, bitcast)


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


# -- join / split (reference: language/ops.py:815-902) -------------------------------

def _no_pointers(fname: str, *xs) -> None:
    for x in xs:
        if isinstance(x, ir.Value) and x.type.ptr:
            raise CompilationError(
                f"tl.{fname} doesn't support tiles of pointers. Apply it to the integer "
                "offsets instead, and add the result to the base pointer.")


def _join_dtype(a, b) -> core.dtype:
    """A Python number takes the other operand's dtype; two runtime operands must already
    share one (as in `tl.where` for literals, as in Triton for the rest)."""
    dt = semantic.computation_dtype("select", a, b)
    for x, other in ((a, b), (b, a)):
        if isinstance(x, core.dtype) and x is not dt:
            what = f"the literal {other!r}" if semantic.is_literal(other) else str(other)
            raise CompilationError(f"tl.join needs two operands of one dtype, but got {x} and "
                                   f"{what}. Convert one operand with `.to(dtype)` first.")
    return dt


def _first(b: ir.Builder, v: ir.Value) -> ir.Value:
    """The only element of a tile of shape (1,), as a scalar."""
    return b.create("reduce", [v], [ir.TType((), v.type.dtype)],
                    {"axis": 0, "kind": "first"}).result


@builtin()
def join(ctx, a, b):
    """Joins `a` and `b` along a new last dimension of size 2: the operands broadcast to
    one shape S and the result has shape (*S, 2), `[..., 0]` from `a` and `[..., 1]` from
    `b`. Two scalars give a tile of shape (2,)."""
    x, y = core.unwrap(a), core.unwrap(b)
    _no_pointers("join", x, y)
    bld = ctx.b
    dt = _join_dtype(semantic.dtype_of(x), semantic.dtype_of(y))
    xv, yv = semantic.to_value(bld, x, dt), semantic.to_value(bld, y, dt)
    shape = semantic.broadcast_shapes(xv.type.shape, yv.type.shape)
    scalar = not shape
    shape = shape or (1,)
    xv, yv = (semantic.broadcast_to(bld, v, shape) for v in (xv, yv))
    out = bld.create("join", [xv, yv], [ir.TType((*shape, 2), dt)]).result
    if scalar:
        out = bld.create("reshape", [out], [out.type.with_shape((2,))]).result
    return out


@builtin()
def split(ctx, a):
    """Splits `a` along its last dimension, which must be 2: returns (a[..., 0],
    a[..., 1]), the inverse of `tl.join`. A tile of shape (2,) gives two scalars."""
    v = _tile(ctx, a, "split")
    _no_pointers("split", v)
    shp = v.type.shape
    if not shp or shp[-1] != 2:
        raise CompilationError(
            f"tl.split needs a tile whose last dimension is 2, but got a tile of shape {shp}. "
            "Reshape the tile first so that its last dimension is 2.")
    b = ctx.b
    rank1 = len(shp) == 1
    if rank1:
        v = b.create("reshape", [v], [v.type.with_shape((1, 2))]).result
    t = v.type.with_shape(v.type.shape[:-1])
    outs = b.create("split", [v], [t, t]).results
    if rank1:
        outs = [_first(b, r) for r in outs]
    return outs[0], outs[1]


# -- reductions and scans with a combine function ---------------------------------------
# Both are lowered here to tile ops the backend already has, in the combination order of
# the reference interpreter: `tl.reduce` halves the axis (combine(x[:h], x[h:]), reference
# ops.py:1061-1096) and `tl.associative_scan` is Hillis-Steele (combine(x[i-s], x[i]) for
# s = 1, 2, 4, ..., reference ops.py:2026-2044), so results match it bit for bit.

def _combine_fn(fn, fname: str):
    fn = core.unwrap(fn)
    if not F.is_jit(fn):
        raise CompilationError(
            f"tl.{fname} needs a @enceladus.jit function as `combine_fn`. Plain Python "
            "functions aren't accepted, because the kernel cache doesn't track their source.")
    return fn


def _combine(ctx, fn, lhs: list, rhs: list, fname: str) -> list:
    b = ctx.b
    res = F.inline_jit(ctx, fn, [*lhs, *rhs])
    res = list(res) if isinstance(res, tuple) else [res]
    if len(res) != len(lhs):
        raise CompilationError(f"combine_fn returns {len(res)} values for {len(lhs)} inputs. "
                               "Return one value per input.")
    out = []
    for i, (r, x) in enumerate(zip(res, lhs)):
        r = core.unwrap(r)
        dt, shape = x.type.dtype, x.type.shape
        if isinstance(r, ir.Value):
            if r.type.dtype is not dt or r.type.ptr:
                raise CompilationError(
                    f"result {i} of combine_fn has dtype {r.type.dtype}, but {dt} is expected "
                    "here. Convert it with `.to(...)`.")
        elif semantic.is_literal(r):
            if isinstance(r, float) and not dt.is_floating():
                raise CompilationError(f"result {i} of combine_fn is the float {r!r}, but the "
                                       f"input is {dt}")
            r = semantic.to_value(b, r, dt)
        else:
            raise CompilationError(f"result {i} of combine_fn isn't a value: {r!r}")
        out.append(semantic.broadcast_to(b, r, shape))
    return out


def _halves(b: ir.Builder, v: ir.Value, ax: int) -> tuple[ir.Value, ir.Value]:
    """(v[..., :n/2, ...], v[..., n/2:, ...]) along `ax`, as views plus one split."""
    shp = v.type.shape
    h = shp[ax] // 2
    s2 = shp[:ax] + (2, h) + shp[ax + 1:]
    v = b.create("reshape", [v], [v.type.with_shape(s2)]).result
    perm = tuple(d for d in _bi.range(len(s2)) if d != ax) + (ax,)
    v = b.create("trans", [v], [v.type.with_shape(tuple(s2[p] for p in perm))],
                 {"perm": perm}).result
    t = v.type.with_shape(v.type.shape[:-1])
    lo, hi = b.create("split", [v], [t, t]).results
    return lo, hi


@builtin(name="reduce")
def reduce_(ctx, input, axis, combine_fn, keep_dims=False):
    """Reduces `input` (a tile, or a tuple of tiles of one shape) along `axis` (all of it
    for None) with `combine_fn(a0, ..., b0, ...)`, a @enceladus.jit function that must be
    associative and commutative."""
    b = ctx.b
    fn = _combine_fn(combine_fn, "reduce")
    single = not isinstance(core.unwrap(input), tuple)
    vals = [_tile(ctx, x, "reduce") for x in ((input,) if single else core.unwrap(input))]
    _no_pointers("reduce", *vals)
    if len({v.type.shape for v in vals}) != 1:
        raise CompilationError("tl.reduce needs inputs of one shape, but got "
                               f"{sorted({v.type.shape for v in vals})}")
    rank = len(vals[0].type.shape)
    if rank == 0:
        return vals[0] if single else tuple(vals)
    axis = core.unwrap(axis)
    if axis is None:
        vals = [b.create("reshape", [v], [v.type.with_shape((v.type.numel,))]).result
                if rank > 1 else v for v in vals]
        ax = 0
    else:
        ax = _axis(axis, rank)
    while vals[0].type.shape[ax] > 1:
        parts = [_halves(b, v, ax) for v in vals]
        vals = _combine(ctx, fn, [p[0] for p in parts], [p[1] for p in parts], "reduce")
    shp = list(vals[0].type.shape)
    del shp[ax]
    if shp:
        outs = [b.create("reshape", [v], [v.type.with_shape(tuple(shp))]).result for v in vals]
    else:
        outs = [_first(b, v) for v in vals]
    if core.unwrap(keep_dims):
        if axis is None:
            outs = [semantic.broadcast_to(b, r, (1,) * rank) for r in outs]
        else:
            outs = [semantic.expand_dims(b, r, ax) for r in outs]
    return outs[0] if single else tuple(outs)


F.TILE_METHODS["reduce"] = lambda ctx, x, axis, combine_fn, keep_dims=False: \
    reduce_._ek_frontend(ctx, x, axis, combine_fn, keep_dims)


@builtin()
def associative_scan(ctx, input, axis, combine_fn, reverse=False):
    """The inclusive scan of `input` (a tile, or a tuple of tiles of one shape) along
    `axis` with `combine_fn(a0, ..., b0, ...)`, where the `a` values come from earlier
    elements (later ones with `reverse=True`). It must be associative; it need not be
    commutative."""
    b = ctx.b
    fn = _combine_fn(combine_fn, "associative_scan")
    single = not isinstance(core.unwrap(input), tuple)
    vals = [_tile(ctx, x, "associative_scan")
            for x in ((input,) if single else core.unwrap(input))]
    _no_pointers("associative_scan", *vals)
    if len({v.type.shape for v in vals}) != 1:
        raise CompilationError("tl.associative_scan needs inputs of one shape, but got "
                               f"{sorted({v.type.shape for v in vals})}")
    shp = vals[0].type.shape
    if not shp:
        raise CompilationError("tl.associative_scan needs a tile")
    if core.unwrap(axis) is None:
        raise CompilationError("tl.associative_scan needs an `axis`, for example `axis=0`")
    ax = _axis(axis, len(shp))
    rev = core.unwrap(reverse)
    if not isinstance(rev, bool):
        raise CompilationError(f"`reverse` must be a compile-time bool, but got {rev!r}")
    n = shp[ax]
    idx = None
    s = 1
    while s < n:
        if idx is None:
            idx = b.create("arange", [], [ir.TType((n,), core.int32)], {"start": 0}).result
            for _ in _bi.range(ax):
                idx = semantic.expand_dims(b, idx, 0)
            for _ in _bi.range(len(shp) - ax - 1):
                idx = semantic.expand_dims(b, idx, len(idx.type.shape))
        by = -s if rev else s
        prev = [b.create("shift", [v], [v.type], {"axis": ax, "by": by}).result for v in vals]
        comb = _combine(ctx, fn, prev, vals, "associative_scan")
        keep = semantic.binary(b, "lt", idx, n - s) if rev else semantic.binary(b, "ge", idx, s)
        vals = [semantic.select(b, keep, c, v) for c, v in zip(comb, vals)]
        s *= 2
    return vals[0] if single else tuple(vals)


F.TILE_METHODS["associative_scan"] = lambda ctx, x, axis, combine_fn, reverse=False: \
    associative_scan._ek_frontend(ctx, x, axis, combine_fn, reverse)
F.TILE_METHODS["join"] = lambda ctx, x, other: join._ek_frontend(ctx, x, other)
F.TILE_METHODS["split"] = lambda ctx, x: split._ek_frontend(ctx, x)
F.TILE_METHODS["reshape"] = lambda ctx, x, *shape, can_reorder=False: reshape._ek_frontend(
    ctx, x, *shape, can_reorder=can_reorder)
F.TILE_METHODS["broadcast_to"] = lambda ctx, x, *shape: broadcast_to._ek_frontend(
    ctx, x, *shape)
F.TILE_METHODS["expand_dims"] = lambda ctx, x, axis: expand_dims._ek_frontend(ctx, x, axis)
# the rest of the reference's tile methods (reference: language/ops.py:1714-1721)
F.TILE_METHODS["permute"] = _trans
F.TILE_METHODS["cast"] = lambda ctx, x, dtype, bitcast=False, fp_downcast_rounding=None: \
    cast._ek_frontend(ctx, x, dtype, bitcast, fp_downcast_rounding)
F.TILE_METHODS["abs"] = lambda ctx, x: abs_._ek_frontend(ctx, x)
F.TILE_METHODS["sum"] = lambda ctx, x, axis=None, keep_dims=False, dtype=None: \
    sum_._ek_frontend(ctx, x, axis, keep_dims, dtype)
F.TILE_METHODS["max"] = lambda ctx, x, axis=None, return_indices=False, \
    return_indices_tie_break_left=True, keep_dims=False: max_._ek_frontend(
        ctx, x, axis, return_indices, return_indices_tie_break_left, keep_dims)
F.TILE_METHODS["min"] = lambda ctx, x, axis=None, return_indices=False, \
    return_indices_tie_break_left=True, keep_dims=False: min_._ek_frontend(
        ctx, x, axis, return_indices, return_indices_tie_break_left, keep_dims)
F.TILE_METHODS["argmax"] = lambda ctx, x, axis, tie_break_left=True, keep_dims=False: \
    argmax._ek_frontend(ctx, x, axis, tie_break_left, keep_dims)
F.TILE_METHODS["argmin"] = lambda ctx, x, axis, tie_break_left=True, keep_dims=False: \
    argmin._ek_frontend(ctx, x, axis, tie_break_left, keep_dims)


# -- dot ----------------------------------------------------------------------------

_DOT_FLOAT = (core.float16, core.bfloat16, core.float32)


@builtin()
def dot(ctx, input, other, acc=None, input_precision=None, allow_tf32=None,
        max_num_imprecise_acc=None, out_dtype=None):
    """Matrix product of two 2D tiles, accumulated in fp32 (floats) or int32 (ints).

    int8 operands run on the i8 MFMAs (v_mfma_i32_32x32x32_i8 and relatives); uint8,
    16- and 32-bit integer operands run as 32-bit multiply-adds from LDS. Integer
    products and sums wrap modulo 2^32, as in the reference (language/ops.py:1244-1270).
    """
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
        if adt.primitive_bitwidth not in (8, 16, 32) or adt.is_bool():
            raise CompilationError(f"tl.dot takes 8-, 16- or 32-bit integer operands, got {adt}")
        if out_dt is not core.int32:
            raise CompilationError("tl.dot accumulates integer operands in int32; create the "
                                   "accumulator with `tl.zeros(..., dtype=tl.int32)`")
        if a.type.shape[1] % 8:
            raise CompilationError(f"tl.dot needs a K dimension that is a multiple of 8, got "
                                   f"{a.type.shape[1]}")
        return b.create("dot", [a, bt, accv], [ir.TType((m, n), out_dt)]).result
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
        raise CompilationError(f"tl.atomic_add doesn't support {dt}. Accumulate in a float32 "
                               "buffer and convert the result afterwards.")
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

    def __call__(self, arg1, arg2=None, step=None):
        raise RuntimeError("tl.static_range can only be used in a kernel `for` loop")


class _Range:
    """`tl.range`: the Triton hints `num_stages`, `loop_unroll_factor`,
    `disallow_acc_multi_buffer`, `flatten` and `warp_specialize` are accepted and have no
    effect (reference: language/ops.py:1299-1311)."""
    _ek_range = True

    def __call__(self, arg1, arg2=None, step=None, num_stages=None, loop_unroll_factor=None,
                 disallow_acc_multi_buffer=False, flatten=False, warp_specialize=False):
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
