"""A from-scratch NumPy restatement of the reference tile-language interpreter.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): the product never imports this.

`run_grid(kernel, grid, *args, **constexprs)` runs the kernel's Python function once per
program id, in row-major (z, y, x) order, with `tl` replaced by this module's NumPy
implementation (reference: interp.py:801-825 `run_grid`, the sequential nested loop
:816-820). Semantics restated:

- tiles are NumPy arrays plus a tile dtype (`OTile`, reference `ITile` interp.py:156);
  fp16/bf16 arithmetic computes in fp32 and rounds after every op (interp.py:45-47,
  :546-548); bf16 values are held as fp32 numbers rounded to bf16 (RNE);
- promotion follows the language rules (reference semantic.py:113-152), restated here;
- integer `//` and `%` truncate toward zero and never trap (`_c_div`, interp.py:600);
- float→int conversion truncates and saturates, int64 wraps modulo 2^64, NaN→0
  (`float_to_int`, interp.py:573-597);
- loads/stores through flat views with element offsets (`IPointer`, interp.py:362) and
  bounds checks on unmasked elements (interp.py:407-419);
- descriptors zero-pad out-of-bounds loads and skip such stores (ops.py:495-530);
- reductions: `np.sum` in the compute dtype, `fmax`/`fmin` for float max/min, argmax as
  the first index of the NaN-ignoring max (ops.py:945-975); narrow ints sum in 32 bits
  (ops.py:910);
- `dot`: fp32 (or int64→int32) matmul of the operands plus the accumulator
  (ops.py:1222-1240);
- atomics: applied in row-major order of the masked elements, one at a time when
  addresses collide (ops.py:1880-1902);
- `cumsum`: `np.cumsum` in the (widened) compute dtype, optionally reversed
  (ops.py:2047-2060).

Pins (tests/test_oracle.py): closed forms for every example (`oracle.reference_np`,
which restates the examples' reference() functions), brute force on tiny inputs,
invariants (cumsum differences recover the input; histogram counts sum to n), the
bf16 rounding table against torch's RNE cast, and the saturating conversion against
hand-picked edge values. Float reduction bit patterns and NumPy's exp ULPs are
"parity unpinned": the reference's own tests check them only to tolerance.
"""

from __future__ import annotations

import builtins
import math as _pymath
import types
from typing import Any

import numpy as np

# ---------------------------------------------------------------------------------------
# dtypes (restated; the product's dtype objects are recognised by name)
# ---------------------------------------------------------------------------------------


class dtype:  # noqa: N801
    def __init__(self, name, kind, bits, npdt):
        self.name, self.kind, self.primitive_bitwidth, self.np = name, kind, bits, npdt

    @property
    def itemsize(self):
        return max(1, self.primitive_bitwidth // 8)

    def is_floating(self):
        return self.kind == "float"

    def is_int(self):
        return self.kind in ("int", "uint", "bool")

    def is_bool(self):
        return self.kind == "bool"

    def is_signed(self):
        return self.kind in ("int", "float")

    @property
    def element_ty(self):
        return self

    def __repr__(self):
        return f"tl.{self.name}"


int1 = dtype("int1", "bool", 1, np.bool_)
int8 = dtype("int8", "int", 8, np.int8)
int16 = dtype("int16", "int", 16, np.int16)
int32 = dtype("int32", "int", 32, np.int32)
int64 = dtype("int64", "int", 64, np.int64)
uint8 = dtype("uint8", "uint", 8, np.uint8)
uint16 = dtype("uint16", "uint", 16, np.uint16)
uint32 = dtype("uint32", "uint", 32, np.uint32)
uint64 = dtype("uint64", "uint", 64, np.uint64)
float16 = dtype("float16", "float", 16, np.float16)
bfloat16 = dtype("bfloat16", "float", 16, np.float32)   # held as bf16-rounded fp32
float32 = dtype("float32", "float", 32, np.float32)
ALL = {d.name: d for d in (int1, int8, int16, int32, int64, uint8, uint16, uint32, uint64,
                           float16, bfloat16, float32)}
_ALIAS = {"i1": int1, "bool": int1, "i8": int8, "i16": int16, "i32": int32, "i64": int64,
          "u8": uint8, "u16": uint16, "u32": uint32, "u64": uint64, "fp16": float16,
          "f16": float16, "bf16": bfloat16, "fp32": float32, "f32": float32}


def as_dtype(d) -> dtype:
    """Maps this module's, the product's, numpy's or a name to an oracle dtype."""
    if isinstance(d, dtype):
        return d
    name = getattr(d, "long_name", None) or getattr(d, "name", None) or str(d)
    if isinstance(d, str):
        name = d
    if name in ALL:
        return ALL[name]
    if name in _ALIAS:
        return _ALIAS[name]
    nd = np.dtype(d)
    for v in ALL.values():
        if v is not bfloat16 and np.dtype(v.np) == nd:
            return v
    raise TypeError(f"no tile dtype for {d!r}")


class constexpr:  # noqa: N801
    def __init__(self, value=None):
        self.value = value


def _uw(x):
    if type(x).__name__ == "constexpr" and hasattr(x, "value"):
        return x.value
    return x


# ---------------------------------------------------------------------------------------
# bf16 rounding (round to nearest even), float->int conversion
# ---------------------------------------------------------------------------------------

def bf16_round(a) -> np.ndarray:
    """fp32 -> nearest bf16 value (ties to even), returned as fp32."""
    f = np.asarray(a, np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, (u >> 16) | 0x40, r).astype(np.uint32) << 16
    return r.astype(np.uint32).view(np.float32).reshape(f.shape)


def bf16_bits(a) -> np.ndarray:
    return (bf16_round(a).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def int_range(dt: dtype):
    bits = dt.primitive_bitwidth
    if dt.is_bool():
        return 0, 1
    if dt.is_signed():
        return -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    return 0, (1 << bits) - 1


def float_to_int(data, dt: dtype) -> np.ndarray:
    """Truncate toward zero; NaN -> 0; saturate (int64: wrap mod 2^64, inf -> 0)."""
    f = np.asarray(data).astype(np.float32).astype(np.float64)
    nan = np.isnan(f)
    t = np.trunc(np.where(nan, 0.0, f))
    if dt is int64:
        with np.errstate(invalid="ignore"):
            r = np.fmod(t, 2.0 ** 64)
        r = np.where(r >= 2.0 ** 63, r - 2.0 ** 64, np.where(r < -(2.0 ** 63), r + 2.0 ** 64, r))
        return np.where(np.isfinite(r), r, 0.0).astype(np.int64)
    lo, hi = int_range(dt)
    if dt.primitive_bitwidth < 64:
        return np.clip(t, lo, hi).astype(dt.np)
    out = np.clip(t, 0.0, np.nextafter(2.0 ** 64, 0.0)).astype(np.uint64)
    return np.where(t >= 2.0 ** 64, np.uint64(hi), out)


def round_to(data, dt: dtype) -> np.ndarray:
    """Rounds computed values (fp32 for floats) to storage of `dt`."""
    if dt is bfloat16:
        return bf16_round(np.asarray(data, np.float32))
    return np.asarray(data).astype(dt.np)


# ---------------------------------------------------------------------------------------
# Values
# ---------------------------------------------------------------------------------------

class OTile:
    __slots__ = ("data", "dtype")
    __array_priority__ = 1000

    def __init__(self, data, dt: dtype):
        self.data = np.asarray(data)
        self.dtype = dt

    @property
    def shape(self):
        return tuple(self.data.shape)

    def __repr__(self):
        return f"OTile({self.data!r}, {self.dtype})"

    def __bool__(self):
        if self.data.ndim:
            raise ValueError("a tile has no single truth value")
        return bool(self.data.item())

    def __index__(self):
        if self.data.ndim or not self.dtype.is_int():
            raise TypeError("only integer scalars can be used as an index")
        return int(self.data.item())

    __int__ = __index__

    def __float__(self):
        return float(self.data.item())

    def __getitem__(self, idx):
        return OTile(self.data[idx], self.dtype)

    @property
    def T(self):  # noqa: N802
        return OTile(self.data.T, self.dtype)

    def to(self, dt, bitcast=False, fp_downcast_rounding=None):
        return _cast(self, as_dtype(_uw(dt)), bitcast)

    def __getattr__(self, name):
        f = _METHODS.get(name)
        if f is None:
            raise AttributeError(name)
        return lambda *a, **k: f(self, *a, **k)


def _binop(op):
    def f(self, o):
        return binary(op, self, o)

    def r(self, o):
        return binary(op, o, self)
    return f, r


for _op, _py in [("add", "add"), ("sub", "sub"), ("mul", "mul"), ("div", "truediv"),
                 ("floordiv", "floordiv"), ("mod", "mod"), ("and", "and"), ("or", "or"),
                 ("xor", "xor"), ("shl", "lshift"), ("shr", "rshift")]:
    _f, _r = _binop(_op)
    setattr(OTile, f"__{_py}__", _f)
    setattr(OTile, f"__r{_py}__", _r)
for _op, _py in [("eq", "eq"), ("ne", "ne"), ("lt", "lt"), ("le", "le"), ("gt", "gt"),
                 ("ge", "ge")]:
    setattr(OTile, f"__{_py}__", _binop(_op)[0])
OTile.__hash__ = None
OTile.__neg__ = lambda self: unary("neg", self)
OTile.__pos__ = lambda self: self
OTile.__invert__ = lambda self: unary("not", self)


class OPointer:
    __slots__ = ("flat", "offsets", "elem", "bf16")

    def __init__(self, flat, offsets, elem: dtype, bf16=False):
        self.flat = flat
        self.offsets = np.asarray(offsets, np.int64)
        self.elem = elem
        self.bf16 = bf16

    @property
    def dtype(self):
        return self.elem

    @property
    def shape(self):
        return tuple(self.offsets.shape)

    def with_offsets(self, off):
        return OPointer(self.flat, off, self.elem, self.bf16)

    def __add__(self, o):
        return _ptr_add(self, o, 1)

    __radd__ = __add__

    def __sub__(self, o):
        return _ptr_add(self, o, -1)

    def __getitem__(self, idx):
        return self.with_offsets(self.offsets[idx])

    def read(self, offs) -> np.ndarray:
        v = self.flat[offs]
        if self.bf16:
            return bf16_from_bits(v)
        return np.array(v)

    def write(self, offs, vals):
        if self.bf16:
            self.flat[offs] = bf16_bits(vals)
        else:
            self.flat[offs] = vals

    def check(self, offs, mask, what):
        n = self.flat.shape[0]
        bad = (offs < 0) | (offs >= n)
        if mask is not None:
            bad &= mask
        if bad.any():
            raise IndexError(f"out-of-bounds {what}: offset {int(offs[bad].flat[0])} outside "
                             f"a buffer of {n} elements")


def _ptr_add(p: OPointer, o, sign):
    o = _uw(o)
    if isinstance(o, OTile):
        if not o.dtype.is_int():
            raise TypeError("pointer offsets must be integers")
        off = o.data.astype(np.int64)
    else:
        off = np.int64(int(o))
    return p.with_offsets(p.offsets + sign * off)


class ODesc:
    def __init__(self, base: OPointer, shape, strides, block):
        self.base = base
        self.shape = tuple(int(s) for s in shape)
        self.strides = tuple(int(s) for s in strides)
        self.block_shape = tuple(int(b) for b in block)

    @property
    def dtype(self):
        return self.base.elem

    def _block(self, offsets):
        rank = len(self.shape)
        off = np.zeros(self.block_shape, np.int64)
        mask = np.ones(self.block_shape, bool)
        for d in range(rank):
            idx = int(offsets[d]) + np.arange(self.block_shape[d], dtype=np.int64)
            view = [1] * rank
            view[d] = self.block_shape[d]
            idx = idx.reshape(view)
            off = off + idx * self.strides[d]
            mask = mask & (idx >= 0) & (idx < self.shape[d])
        return off + self.base.offsets, mask

    def load(self, offsets):
        off, mask = self._block([_uw(o) for o in offsets])
        return load(self.base.with_offsets(off), OTile(mask, int1))

    def store(self, offsets, value):
        off, mask = self._block([_uw(o) for o in offsets])
        v = to_tile(value, self.dtype)
        store(self.base.with_offsets(off), OTile(np.broadcast_to(v.data, off.shape), v.dtype),
              OTile(mask, int1))


# ---------------------------------------------------------------------------------------
# Promotion (restated from the language rules) and elementwise ops
# ---------------------------------------------------------------------------------------

def _is_lit(x):
    return isinstance(x, (bool, int, float, np.generic)) and not isinstance(x, OTile)


def literal_dtype(v) -> dtype:
    if isinstance(v, (bool, np.bool_)):
        return int1
    if isinstance(v, (int, np.integer)):
        v = int(v)
        if -(1 << 31) <= v < (1 << 31):
            return int32
        if -(1 << 63) <= v < (1 << 63):
            return int64
        return uint64
    return float32


def _adopt(v, dt: dtype) -> dtype:
    if isinstance(v, bool) and dt.is_bool():
        return int1
    if isinstance(v, float):
        return dt if dt.is_floating() else float32
    if dt.is_floating():
        return dt
    if dt.is_bool():
        return literal_dtype(int(v))
    lo, hi = int_range(dt)
    return dt if lo <= int(v) <= hi else literal_dtype(int(v))


def _int_promote(a: dtype, b: dtype) -> dtype:
    if a is b:
        return a
    if a.is_bool():
        return b
    if b.is_bool():
        return a
    if a.is_signed() == b.is_signed():
        return a if a.primitive_bitwidth >= b.primitive_bitwidth else b
    s, u = (a, b) if a.is_signed() else (b, a)
    return u if u.primitive_bitwidth >= s.primitive_bitwidth else s


def compute_dtype(op, a, b) -> dtype:
    if _is_lit(a) and _is_lit(b):
        a, b = literal_dtype(a), literal_dtype(b)
    elif _is_lit(a):
        a = _adopt(a, b)
    elif _is_lit(b):
        b = _adopt(b, a)
    if op in ("and", "or", "xor", "shl", "shr") and not (a.is_int() and b.is_int()):
        raise TypeError(f"`{op}` needs integer operands")
    if op == "floordiv" and (a.is_floating() or b.is_floating()):
        raise TypeError("`//` needs integer operands")
    if a.is_floating() or b.is_floating():
        if a.is_floating() and b.is_floating():
            if a is b:
                return a
            if {a, b} == {float16, bfloat16}:
                return float32
            return a if a.primitive_bitwidth >= b.primitive_bitwidth else b
        return a if a.is_floating() else b
    if op == "div":
        return float32
    t = _int_promote(a, b)
    if t.is_bool() and op in ("add", "sub", "mul", "div", "floordiv", "mod", "min", "max",
                              "shl", "shr"):
        return int32
    return t


def _lit_array(v, dt: dtype):
    if dt.is_floating():
        return round_to(np.float32(float(v)), dt)
    if dt.is_bool():
        return np.asarray(bool(v))
    if isinstance(v, float):
        v = _pymath.trunc(v)
    v = int(v)
    bits = dt.primitive_bitwidth
    v &= (1 << bits) - 1
    if dt.is_signed() and v >> (bits - 1):
        v -= 1 << bits
    return np.asarray(v, dt.np)


def to_tile(x, dt: dtype | None = None) -> OTile:
    x = _uw(x)
    if isinstance(x, OTile):
        return _cast(x, dt) if dt is not None else x
    if isinstance(x, np.ndarray) and x.ndim > 0:
        t = OTile(x, as_dtype(x.dtype))
        return _cast(t, dt) if dt is not None else t
    if isinstance(x, np.generic):
        x = x.item()
    dt = dt or literal_dtype(x)
    return OTile(_lit_array(x, dt), dt)


def _cast(x: OTile, dt: dtype, bitcast=False) -> OTile:
    if x.dtype is dt:
        return x
    if bitcast:
        src = x.data
        if x.dtype is bfloat16:
            src = bf16_bits(src)
        if dt is bfloat16:
            return OTile(bf16_from_bits(src.view(np.uint16)), dt)
        return OTile(src.view(dt.np), dt)
    d = x.data
    if dt.is_bool():
        return OTile(d != 0, dt)
    if x.dtype.is_floating() and dt.is_int():
        return OTile(float_to_int(d, dt), dt)
    if dt.is_floating():
        return OTile(round_to(d.astype(np.float32) if dt is not float16 or x.dtype is
                              bfloat16 else d, dt), dt)
    return OTile(d.astype(dt.np), dt)


def _compute(x, dt: dtype) -> np.ndarray:
    t = to_tile(x, dt) if not isinstance(x, OTile) else _cast(x, dt)
    return t.data.astype(np.float32) if dt.is_floating() else t.data


def _c_div(a, b, signed):
    b = np.where(b == 0, 1, b).astype(b.dtype)
    q = np.floor_divide(a, b)
    if signed:
        q = q + ((q < 0) & (q * b != a)).astype(q.dtype)
    return q


def _shift(a, b, left):
    bits = a.dtype.itemsize * 8
    bb = b.astype(np.int64)
    big = (bb >= bits) | (bb < 0)
    safe = np.where(big, 0, bb).astype(a.dtype)
    r = np.left_shift(a, safe) if left else np.right_shift(a, safe)
    if left:
        fill = np.zeros_like(a)
    else:
        fill = np.where(a < 0, -1, 0).astype(a.dtype) if np.issubdtype(a.dtype, np.signedinteger) \
            else np.zeros_like(a)
    return np.where(big, fill, r)


_BIN = {
    "add": lambda a, b, dt: a + b, "sub": lambda a, b, dt: a - b,
    "mul": lambda a, b, dt: a * b, "div": lambda a, b, dt: a / b,
    "floordiv": lambda a, b, dt: _c_div(a, b, dt.is_signed()),
    "mod": lambda a, b, dt: np.fmod(a, b if dt.is_floating() else np.where(b == 0, 1, b)),
    "and": lambda a, b, dt: a & b, "or": lambda a, b, dt: a | b,
    "xor": lambda a, b, dt: a ^ b,
    "shl": lambda a, b, dt: _shift(a, b, True), "shr": lambda a, b, dt: _shift(a, b, False),
    "min": lambda a, b, dt: np.fmin(a, b) if dt.is_floating() else np.minimum(a, b),
    "max": lambda a, b, dt: np.fmax(a, b) if dt.is_floating() else np.maximum(a, b),
    "eq": lambda a, b, dt: a == b, "ne": lambda a, b, dt: a != b,
    "lt": lambda a, b, dt: a < b, "le": lambda a, b, dt: a <= b,
    "gt": lambda a, b, dt: a > b, "ge": lambda a, b, dt: a >= b,
}


def _operand(x):
    x = _uw(x)
    if isinstance(x, OTile):
        return x.dtype
    if isinstance(x, np.generic):
        return x.item()
    return x


def binary(op, x, y):
    x, y = _uw(x), _uw(y)
    if isinstance(y, OPointer) and op == "add":
        return _ptr_add(y, x, 1)
    if isinstance(x, OPointer) and op in ("add", "sub"):
        return _ptr_add(x, y, 1 if op == "add" else -1)
    dt = compute_dtype(op, _operand(x), _operand(y))
    a, b = _compute(x, dt), _compute(y, dt)
    np.broadcast_shapes(a.shape, b.shape)
    with np.errstate(all="ignore"):
        out = _BIN[op](a, b, dt)
    if op in ("eq", "ne", "lt", "le", "gt", "ge"):
        return OTile(np.asarray(out, bool), int1)
    return OTile(round_to(out, dt), dt)


def _erf(a):
    return np.vectorize(_pymath.erf, otypes=[np.float64])(a.astype(np.float64)).astype(a.dtype)


_UN = {"neg": lambda a: -a, "abs": np.abs, "exp": np.exp, "exp2": np.exp2, "log": np.log,
       "log2": np.log2, "sqrt": np.sqrt, "rsqrt": lambda a: 1.0 / np.sqrt(a),
       "sin": np.sin, "cos": np.cos, "tanh": np.tanh,
       "sigmoid": lambda a: 1.0 / (1.0 + np.exp(-a)), "erf": _erf, "floor": np.floor,
       "ceil": np.ceil}
_MATH = ("exp", "exp2", "log", "log2", "sqrt", "rsqrt", "sin", "cos", "tanh", "sigmoid", "erf",
         "floor", "ceil")


def unary(op, x):
    x = to_tile(x)
    dt = x.dtype
    if op in _MATH and not dt.is_floating():
        raise TypeError(f"tl.{op} needs a floating-point input")
    if op == "not":
        return OTile(np.logical_not(x.data) if dt.is_bool() else np.invert(x.data), dt)
    if op == "neg" and dt.is_bool():
        dt = int32
    with np.errstate(all="ignore"):
        return OTile(round_to(_UN[op](_compute(x, dt)), dt), dt)


# ---------------------------------------------------------------------------------------
# The tl surface
# ---------------------------------------------------------------------------------------

class _State:
    pid = (0, 0, 0)
    grid = (1, 1, 1)


STATE = _State()


def program_id(axis):
    return OTile(np.int32(STATE.pid[int(_uw(axis))]), int32)


def num_programs(axis):
    return OTile(np.int32(STATE.grid[int(_uw(axis))]), int32)


def arange(start, end):
    return OTile(np.arange(int(_uw(start)), int(_uw(end)), dtype=np.int32), int32)


def _shape(shape):
    shape = _uw(shape)
    if isinstance(shape, int):
        return (shape,)
    return tuple(int(_uw(s)) for s in shape)


def full(shape, value, dtype):
    dt = as_dtype(_uw(dtype))
    v = _uw(value)
    if isinstance(v, OTile):
        return OTile(np.broadcast_to(_cast(v, dt).data, _shape(shape)).copy(), dt)
    return OTile(np.full(_shape(shape), _lit_array(v, dt), dtype=_lit_array(v, dt).dtype), dt)


def zeros(shape, dtype):
    return full(shape, 0, dtype)


def zeros_like(input):
    return full(input.shape, 0, input.dtype)


def full_like(input, value, dtype=None):
    return full(input.shape, value, dtype or input.dtype)


def load(pointer, mask=None, other=None, boundary_check=(), padding_option="",
         cache_modifier="", eviction_policy="", volatile=False):
    p = pointer
    mask = _uw(mask)
    if mask is None or mask is True:
        p.check(p.offsets, None, "load")
        return OTile(p.read(p.offsets), p.elem)
    m = to_tile(mask)
    offs, mb = np.broadcast_arrays(p.offsets, m.data)
    p.check(offs, mb, "load")
    if p.flat.shape[0] == 0:
        data = np.zeros(offs.shape, np.float32 if p.bf16 else p.elem.np)
    else:
        data = p.read(np.where(mb, offs, 0))
    fill = to_tile(other if _uw(other) is not None else 0, p.elem).data
    data = np.array(data)
    np.copyto(data, np.broadcast_to(fill, data.shape).astype(data.dtype), where=~mb)
    return OTile(data, p.elem)


def store(pointer, value, mask=None, boundary_check=(), cache_modifier="", eviction_policy=""):
    p = pointer
    v = to_tile(value, p.elem)
    mask = _uw(mask)
    arrays = [p.offsets, v.data] + ([] if mask is None or mask is True else [to_tile(mask).data])
    bc = np.broadcast_arrays(*arrays)
    offs, vals = bc[0], bc[1]
    mb = bc[2] if len(bc) > 2 else np.ones(offs.shape, bool)
    p.check(offs, mb, "store")
    p.write(offs[mb], vals[mb])


def make_tensor_descriptor(base, shape, strides, block_shape, padding_option="zero"):
    shp = [int(_uw(s)) for s in _uw(shape)]
    st = [int(_uw(s)) for s in _uw(strides)]
    if st[-1] != 1:
        raise ValueError("the last stride of a tensor descriptor must be 1")
    return ODesc(base, shp, st, _shape(block_shape))


def where(condition, x, y):
    c = to_tile(condition)
    x, y = _uw(x), _uw(y)
    if isinstance(x, OPointer):
        offs = np.where(c.data, x.offsets, y.offsets)
        return x.with_offsets(offs)
    dt = compute_dtype("select", _operand(x), _operand(y))
    a, b = to_tile(x, dt).data, to_tile(y, dt).data
    return OTile(np.where(c.data != 0, a, b), dt)


def maximum(x, y):
    return binary("max", x, y)


def minimum(x, y):
    return binary("min", x, y)


def fma(x, y, z):
    return binary("add", binary("mul", x, y), z)


def abs(x):  # noqa: A001
    return unary("abs", x)


def cdiv(x, div):
    return binary("floordiv", binary("sub", binary("add", x, div), 1), div)


def clamp(x, min, max):  # noqa: A002
    return binary("min", binary("max", x, min), max)


def cast(input, dtype, bitcast=False, fp_downcast_rounding=None):
    return _cast(to_tile(input), as_dtype(_uw(dtype)), bitcast)


def broadcast_to(input, *shape):
    if len(shape) == 1 and isinstance(_uw(shape[0]), (tuple, list)):
        shape = _uw(shape[0])
    x = to_tile(input)
    return OTile(np.broadcast_to(x.data, _shape(shape)), x.dtype)


def expand_dims(input, axis):
    x = to_tile(input)
    return OTile(np.expand_dims(x.data, _uw(axis)), x.dtype)


def reshape(input, *shape, can_reorder=False):
    if len(shape) == 1 and isinstance(_uw(shape[0]), (tuple, list)):
        shape = _uw(shape[0])
    x = to_tile(input)
    return OTile(x.data.reshape(_shape(shape)), x.dtype)


def trans(input, *dims):
    x = to_tile(input)
    if len(dims) == 1 and isinstance(_uw(dims[0]), (tuple, list)):
        dims = _uw(dims[0])
    dims = tuple(int(_uw(d)) for d in dims) or None
    return OTile(np.transpose(x.data, dims), x.dtype)


permute = trans


def _sum_dtype(dt: dtype) -> dtype:
    if dt.is_int() and dt.primitive_bitwidth < 32:
        return uint32 if dt.kind == "uint" else int32
    return dt


def _reduce(input, axis, kind, keep_dims, dtype=None):
    t = to_tile(input)
    if dtype is not None:
        t = _cast(t, as_dtype(_uw(dtype)))
    if kind == "sum":
        t = _cast(t, _sum_dtype(t.dtype))
    axis = _uw(axis)
    keep = bool(_uw(keep_dims))
    data = t.data.astype(np.float32) if t.dtype.is_floating() else t.data
    if kind == "sum":
        return OTile(round_to(np.sum(data, axis=axis, keepdims=keep, dtype=data.dtype), t.dtype),
                     t.dtype)
    flat = data.reshape(-1) if axis is None else data
    a = 0 if axis is None else int(axis)
    uf = {"max": np.fmax, "min": np.fmin} if t.dtype.is_floating() else \
        {"max": np.maximum, "min": np.minimum}
    out = uf[kind.removeprefix("arg")].reduce(flat, axis=a, keepdims=True)
    if kind in ("argmax", "argmin"):
        hit = flat == out
        if t.dtype.is_floating():
            hit |= np.isnan(flat) & np.isnan(out)
        out = np.argmax(hit, axis=a, keepdims=True).astype(np.int32)
    if not keep:
        out = np.squeeze(out, axis=a)
    elif axis is None:
        out = out.reshape((1,) * t.data.ndim)
    if kind in ("argmax", "argmin"):
        return OTile(out, int32)
    return OTile(round_to(out, t.dtype), t.dtype)


def sum(input, axis=None, keep_dims=False, dtype=None):  # noqa: A001
    return _reduce(input, axis, "sum", keep_dims, dtype)


def max(input, axis=None, return_indices=False, return_indices_tie_break_left=True,  # noqa: A001
        keep_dims=False):
    if _uw(return_indices):
        return _reduce(input, axis, "max", keep_dims), _reduce(input, axis, "argmax", keep_dims)
    return _reduce(input, axis, "max", keep_dims)


def min(input, axis=None, return_indices=False, return_indices_tie_break_left=True,  # noqa: A001
        keep_dims=False):
    if _uw(return_indices):
        return _reduce(input, axis, "min", keep_dims), _reduce(input, axis, "argmin", keep_dims)
    return _reduce(input, axis, "min", keep_dims)


def argmax(input, axis, tie_break_left=True, keep_dims=False):
    return _reduce(input, axis, "argmax", keep_dims)


def argmin(input, axis, tie_break_left=True, keep_dims=False):
    return _reduce(input, axis, "argmin", keep_dims)


def cumsum(input, axis=0, reverse=False, dtype=None):
    t = to_tile(input)
    if dtype is not None:
        t = _cast(t, as_dtype(_uw(dtype)))
    t = _cast(t, _sum_dtype(t.dtype))
    ax = int(_uw(axis))
    data = t.data.astype(np.float32) if t.dtype.is_floating() else t.data
    rev = bool(_uw(reverse))
    if rev:
        data = np.flip(data, ax)
    out = np.cumsum(data, axis=ax, dtype=data.dtype)
    if rev:
        out = np.flip(out, ax)
    return OTile(round_to(out, t.dtype), t.dtype)


def dot(input, other, acc=None, input_precision=None, allow_tf32=None,
        max_num_imprecise_acc=None, out_dtype=None):
    a, b = to_tile(input), to_tile(other)
    m, n = a.shape[0], b.shape[1]
    if a.dtype.is_int():
        c = np.zeros((m, n), np.int64) if acc is None else to_tile(acc).data.astype(np.int64)
        r = a.data.astype(np.int64) @ b.data.astype(np.int64) + c
        return OTile(r.astype(np.int32), int32)
    out_dt = float32 if acc is None and out_dtype is None else (
        to_tile(acc).dtype if acc is not None else as_dtype(_uw(out_dtype)))
    c = np.zeros((m, n), np.float32) if acc is None else to_tile(acc).data.astype(np.float32)
    r = a.data.astype(np.float32) @ b.data.astype(np.float32) + c
    return OTile(round_to(r, out_dt), out_dt)


def _apply_atomic(kind, old, val, cmp, dt):
    if kind == "xchg":
        return val
    if kind == "cas":
        return np.where(old == cmp, val, old)
    if kind in ("and", "or", "xor"):
        return {"and": np.bitwise_and, "or": np.bitwise_or, "xor": np.bitwise_xor}[kind](old, val)
    if dt.is_floating():
        out = {"add": np.add, "max": np.fmax, "min": np.fmin}[kind](old.astype(np.float32),
                                                                   val.astype(np.float32))
        return round_to(out, dt)
    return {"add": np.add, "max": np.maximum, "min": np.minimum}[kind](old, val)


def _atomic(kind, pointer, operands, mask):
    p = pointer
    dt = p.elem
    vals = [to_tile(v, dt).data for v in operands]
    arrays = [p.offsets, *vals]
    mask = _uw(mask)
    if mask is not None and mask is not True:
        arrays.append(to_tile(mask).data)
    bc = np.broadcast_arrays(*arrays)
    offs = bc[0]
    mb = bc[1 + len(vals)] if len(bc) > 1 + len(vals) else np.ones(offs.shape, bool)
    p.check(offs, mb, f"atomic_{kind}")
    old = np.zeros(offs.shape, np.float32 if p.bf16 else dt.np)
    o = offs[mb]
    v = bc[len(vals)][mb]
    c = bc[1][mb] if kind == "cas" else None
    if np.unique(o).size == o.size:
        cur = p.read(o)
        old[mb] = cur
        p.write(o, _apply_atomic(kind, cur, v, c, dt))
    else:
        # Colliding addresses apply one at a time in row-major order. Integer adds commute,
        # so the final memory equals a bincount-style accumulation (used for speed).
        if kind == "add" and dt.is_int():
            uniq, inv = np.unique(o, return_inverse=True)
            sums = np.zeros(uniq.shape, np.int64)
            np.add.at(sums, inv, v.astype(np.int64))
            cur = p.read(uniq).astype(np.int64)
            # old values: running prefix per address in row-major order
            order = np.argsort(inv, kind="stable")
            vv = v.astype(np.int64)[order]
            grp = inv[order]
            csum = np.cumsum(vv)
            start = np.concatenate([[0], np.flatnonzero(np.diff(grp)) + 1])
            base = np.repeat(csum[start] - vv[start], np.diff(np.append(start, len(vv))))
            excl = csum - vv - base
            got = np.empty_like(vv)
            got[order] = (cur[grp] + excl)
            new = cur + sums
            bits = dt.primitive_bitwidth
            wrap = lambda x: ((x + (1 << (bits - 1))) % (1 << bits)) - (1 << (bits - 1)) \
                if dt.is_signed() else x % (1 << bits)  # noqa: E731
            p.write(uniq, wrap(new).astype(dt.np))
            old[mb] = wrap(got).astype(dt.np)
        else:
            got = np.empty(o.shape, old.dtype)
            for i in builtins.range(o.size):
                cur = p.read(o[i:i + 1])
                got[i] = cur[0]
                ci = None if c is None else c[i:i + 1]
                p.write(o[i:i + 1], _apply_atomic(kind, cur, v[i:i + 1], ci, dt))
            old[mb] = got
    return OTile(old, dt)


def _mk_atomic(kind):
    def f(pointer, val, mask=None, sem=None, scope=None):
        return _atomic(kind, pointer, [val], mask)
    f.__name__ = f"atomic_{kind}"
    return f


atomic_add = _mk_atomic("add")
atomic_max = _mk_atomic("max")
atomic_min = _mk_atomic("min")
atomic_xchg = _mk_atomic("xchg")
atomic_and = _mk_atomic("and")
atomic_or = _mk_atomic("or")
atomic_xor = _mk_atomic("xor")


def atomic_cas(pointer, cmp, val, sem=None, scope=None):
    return _atomic("cas", pointer, [cmp, val], None)


for _m in _MATH:
    globals()[_m] = (lambda op: (lambda x: unary(op, x)))(_m)


def typed_range(*args, **kwargs):
    vals = [_uw(a) for a in args]
    if not any(isinstance(v, OTile) for v in vals):
        return builtins.range(*[int(v) for v in vals])
    dt = int32
    for v in vals:
        if isinstance(v, OTile) and v.dtype in (int64, uint32, uint64):
            dt = int64
    return (OTile(np.array(i, dt.np), dt) for i in builtins.range(*[int(v) for v in vals]))


range = typed_range  # noqa: A001


def static_range(*args):
    return builtins.range(*[int(_uw(a)) for a in args])


def static_assert(cond, msg=""):
    if not _uw(cond):
        raise AssertionError(msg)


def static_print(*values, sep=" "):
    pass


def debug_barrier():
    pass


def multiple_of(input, values):
    return input


def max_contiguous(input, values):
    return input


def device_assert(cond, msg="", mask=None):
    pass


def device_print(prefix, *args, hex=False):
    pass


_METHODS = {"to": lambda x, dt, bitcast=False, **k: _cast(x, as_dtype(_uw(dt)), bitcast),
            "sum": sum, "max": max, "min": min, "cumsum": cumsum, "argmax": argmax,
            "argmin": argmin, "trans": trans}
for _m in _MATH:
    _METHODS[_m] = globals()[_m]

math = types.SimpleNamespace(**{m: globals()[m] for m in _MATH})

# ---------------------------------------------------------------------------------------
# Grid runner
# ---------------------------------------------------------------------------------------

_TL = types.ModuleType("oracle_tl")
for _k, _v in list(globals().items()):
    if not _k.startswith("_"):
        setattr(_TL, _k, _v)
_TL.range = typed_range
_TL.math = math


def _is_tl_module(v) -> bool:
    return isinstance(v, types.ModuleType) and v.__name__ in (
        "enceladus_amd.language", "enceladus.language")


def _rebind(fn, memo):
    if fn in memo:
        return memo[fn]
    g = dict(fn.__globals__)
    for k, v in list(g.items()):
        if _is_tl_module(v):
            g[k] = _TL
        elif getattr(v, "_ek_jit", False):
            g[k] = None  # filled below
    g["range"] = typed_range
    new = types.FunctionType(fn.__code__, g, fn.__name__, fn.__defaults__, fn.__closure__)
    memo[fn] = new
    for k, v in list(fn.__globals__.items()):
        if getattr(v, "_ek_jit", False):
            g[k] = _rebind(v.fn, memo)
    return new


def _arg(x, is_const: bool):
    if is_const:
        return _uw(x)
    t = __import__("sys").modules.get("torch")
    if t is not None and isinstance(x, t.Tensor):
        if str(x.dtype) == "torch.bfloat16":
            bits = x.detach().cpu().contiguous().view(t.int16).numpy().view(np.uint16)
            return _pointer(bits.reshape(-1), bfloat16, True)
        x = x.detach().cpu().numpy()
    if isinstance(x, np.ndarray):
        return _pointer(x, as_dtype(x.dtype))
    if isinstance(x, (bool, np.bool_)):
        return OTile(np.bool_(x), int1)
    if isinstance(x, (int, np.integer)):
        return to_tile(int(x))
    if isinstance(x, (float, np.floating)):
        return OTile(np.float32(x), float32)
    if isinstance(x, OPointer):
        return x
    raise TypeError(f"unsupported kernel argument {type(x).__name__}")


def _pointer(a: np.ndarray, dt: dtype, bf16=False) -> OPointer:
    item = a.itemsize
    if a.size == 0:
        length = 0
    else:
        length = 1 + builtins.sum((n - 1) * (s // item) for n, s in zip(a.shape, a.strides))
    flat = np.lib.stride_tricks.as_strided(a, shape=(length,), strides=(item,))
    return OPointer(flat, np.int64(0), dt, bf16)


def bf16_pointer(bits: np.ndarray) -> OPointer:
    """A pointer over a uint16 array holding bf16 bit patterns (writes update it)."""
    return _pointer(bits, bfloat16, True)


def run_grid(kernel, grid, *args, programs=None, **kwargs):
    """Runs `kernel` (an @jit function or plain function) once per program.

    `programs`, if given, is an iterable of (x, y, z) program ids to run instead of the
    whole grid (a sample: programs are independent).
    """
    import inspect
    fn = getattr(kernel, "fn", kernel)
    params = list(inspect.signature(fn).parameters.values())
    bound = {}
    for p, a in zip(params, args):
        bound[p.name] = a
    bound.update(kwargs)
    call = {}
    for p in params:
        if p.name not in bound:
            if p.default is inspect.Parameter.empty:
                raise TypeError(f"missing argument {p.name}")
            bound[p.name] = p.default
        ann = p.annotation
        is_c = (getattr(ann, "__name__", "") == "constexpr") or (isinstance(ann, str) and
                                                                   ann.endswith("constexpr"))
        call[p.name] = _arg(bound[p.name], is_c)
    f = _rebind(fn, {})
    grid = tuple(grid) + (1,) * (3 - len(tuple(grid)))
    STATE.grid = grid
    with np.errstate(all="ignore"):
        if programs is not None:
            for pid in programs:
                STATE.pid = tuple(pid) + (0,) * (3 - len(tuple(pid)))
                f(**call)
        else:
            for z in builtins.range(grid[2]):
                for y in builtins.range(grid[1]):
                    for x in builtins.range(grid[0]):
                        STATE.pid = (x, y, z)
                        f(**call)
