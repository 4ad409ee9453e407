"""`@jit`, kernel specialization and the launch front door.

`kernel[grid](*args, num_warps=4, dot_warps=None, **constexprs)` binds arguments, looks up
the specialization (a dict hit when warm), compiles on a miss, packs the kernarg buffer
and launches one workgroup of `num_warps * 64` threads per program. Reference:
src/enceladus/runtime/jit.py (`JITFunction` :214-667, `run` :388, `_lookup` :449,
`arg_type` :97, `arg_facts` :148, `jit` :1237, `cdiv`/`next_power_of_2` :64-71).

`ENCELADUS_INTERPRET=1` (the reference's NumPy interpreter mode) is not part of this
backend: the CPU interpreter is test infrastructure here, so requesting it raises.
"""

from __future__ import annotations

import ctypes
import inspect
import os
import struct
import threading
from dataclasses import dataclass
from typing import Any, Callable

import numpy as np

from enceladus_amd.compiler import ir
from enceladus_amd.compiler.errors import CompilationError, DeviceAssertionError
from enceladus_amd.language import core
from enceladus_amd.runtime import compile as C
from enceladus_amd.runtime import device as D
from enceladus_amd.runtime import hip as _hip
from enceladus_amd.runtime import speccache
from enceladus_amd.runtime import debug as _trace
from enceladus_amd.runtime import timing as _timing
from enceladus_amd.runtime import tensor as T


def _debug() -> bool:
    """ENCELADUS_DEBUG=1 keeps `tl.device_assert` checks (reference: compile.py:10)."""
    return os.environ.get("ENCELADUS_DEBUG", "") not in ("", "0")


def cdiv(x: int, div: int) -> int:
    """`ceil(x / div)` for positive integers: the number of blocks that cover `x`."""
    return (x + div - 1) // div


def next_power_of_2(n: int) -> int:
    n = int(n)
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


def arg_type(value: Any) -> ir.TType:
    if isinstance(value, (bool, np.bool_)):
        return ir.TType((), core.int1)
    if isinstance(value, np.uint64):
        return ir.TType((), core.uint64)
    if isinstance(value, (int, np.integer)):
        v = int(value)
        if -(1 << 31) <= v < (1 << 31):
            return ir.TType((), core.int32)
        if -(1 << 63) <= v < (1 << 63):
            return ir.TType((), core.int64)
        if 0 <= v < (1 << 64):
            return ir.TType((), core.uint64)
        raise TypeError(f"integer argument {v} doesn't fit in 64 bits")
    if isinstance(value, (float, np.floating)):
        return ir.TType((), core.float32)
    if T.is_array_like(value):
        return ir.TType((), T.elem_dtype(value), ptr=True)
    raise TypeError(f"a {type(value).__name__} can't be a runtime kernel argument; annotate "
                    "compile-time parameters as tl.constexpr")


def _data_ptr(value: Any) -> int | None:
    if isinstance(value, np.ndarray):
        return value.__array_interface__["data"][0]
    if isinstance(value, T.Tensor):
        return value.ptr
    p = getattr(value, "data_ptr", None)
    return p() if callable(p) else None


def arg_facts(value: Any) -> dict:
    if isinstance(value, (bool, np.bool_)):
        return {}
    if isinstance(value, (float, np.floating)):
        # the sign of a float (an attention scale) lets the compiler fold it through max
        return {"positive": True} if float(value) > 0 else {}
    if isinstance(value, (int, np.integer)):
        v = int(value)
        f = {}
        if v % 16 == 0:
            f["divisibility"] = 16
        if v == 1:
            f["equal_to_1"] = True
        return f
    if T.is_array_like(value):
        p = _data_ptr(value)
        facts = {}
        if isinstance(value, np.ndarray):
            facts["divisibility"] = 16   # copied into a fresh 16-byte-aligned allocation
        elif p is not None and p % 16 == 0:
            facts["divisibility"] = 16
        last = _last_index(value)
        if (last + 1) * T.elem_dtype(value).itemsize >= (1 << 31) - 64:
            facts["span2g"] = True       # byte offsets may not fit 32 bits: no buffer loads
        if last > MAX_ELEMENT_INDEX:
            facts["idx64"] = True        # element offsets need 64-bit index math
        return facts
    return {}


# The largest element offset from an array argument's first element that 32-bit index
# math reaches; launches with a larger span compile an `idx64` variant with 64-bit index
# math (reference: runtime/launcher.py:42-48).
MAX_ELEMENT_INDEX = (1 << 31) - 1
# facts that stay in the specialization even for do_not_specialize parameters
REQUIRED_FACTS = ("idx64", "span2g")

# -- the warm launch path ------------------------------------------------------------
# A warm launch of a specialization whose arguments are all device arrays and scalars is
# keyed by a tuple computed in one pass over the arguments (dtypes, 16-byte alignment, a
# span class, integer width classes, float signs, constexpr values, launch options and
# the environment switches that change code generation), and packs its kernarg with a
# precomputed `struct.Struct`. Launches with NumPy arrays, assertion buffers, coarsened
# program walks or a second flush kernel take the general path.

_ENV = getattr(os.environ, "_data", None)      # POSIX: bytes keys, updated by os.environ
_ENV_KEYS = (b"ENCELADUS_CODEGEN", b"ENCELADUS_OVERRIDE_DIR", b"ENCELADUS_DEBUG",
             b"ENCELADUS_INTERPRET")


def _env_token() -> tuple:
    e = _ENV
    if e is None:
        return tuple(os.environ.get(k.decode()) for k in _ENV_KEYS)
    return (e.get(b"ENCELADUS_CODEGEN"), e.get(b"ENCELADUS_OVERRIDE_DIR"),
            e.get(b"ENCELADUS_DEBUG"), e.get(b"ENCELADUS_INTERPRET"))


_torch_mod = None


def _torch():
    """torch, once something imported it (this module never imports it)."""
    global _torch_mod
    if _torch_mod is None:
        import sys
        _torch_mod = sys.modules.get("torch")
    return _torch_mod


def _span_class(nbytes_last: int, last: int) -> int:
    """0: small; 1: >= 2 GiB of bytes (no buffer loads); 2: also > 2^31 - 1 elements."""
    if last > MAX_ELEMENT_INDEX:
        return 2
    return 1 if nbytes_last >= (1 << 31) - 64 else 0


def _int_class(v: int) -> int:
    if -(1 << 31) <= v < (1 << 31):
        return 0
    if -(1 << 63) <= v < (1 << 63):
        return 1
    return 2


_FMT = {"int32_t": ("i", 4), "int64_t": ("q", 8), "uint32_t": ("I", 4), "uint64_t": ("Q", 8),
        "float": ("f", 4), "int16_t": ("h", 2), "uint16_t": ("H", 2), "int8_t": ("b", 1),
        "uint8_t": ("B", 1)}


class _FastEntry:
    """A specialization's pre-packed launch: kernarg struct, function, block size."""

    __slots__ = ("lc", "st", "fn", "block")

    def __init__(self, lc, st, fn, block):
        self.lc, self.st, self.fn, self.block = lc, st, fn, block


def _fast_entry(lc) -> "_FastEntry | None":
    g = lc.ck.gen
    if g.flush or g.coarsen or g.asserts:
        return None
    fmt, off = "<", 0
    for ka in lc.ck.args:
        code, size = ("Q", 8) if ka.kind == "ptr" else _FMT[ka.cparam]
        pad = (-off) % size
        fmt += "x" * pad + code
        off += pad + size
    fmt += "x" * ((-off) % 8)
    return _FastEntry(lc, struct.Struct(fmt), lc.ck.function(), g.block)


_tls = threading.local()
_ek_launch_fn = None
_raw_stream_fns = None


def _ek_launch():
    global _ek_launch_fn
    if _ek_launch_fn is None:
        _ek_launch_fn = _hip.load_library().ek_launch
    return _ek_launch_fn


def _launch_stream() -> int:
    """torch's current raw stream on the current device (what `device.current_stream`
    returns) through cached accessors, for the warm path."""
    global _raw_stream_fns
    if _raw_stream_fns is None:
        torch = _torch()
        c = getattr(torch, "_C", None) if torch is not None else None
        if c is None or not torch.cuda.is_initialized() or \
                not hasattr(c, "_cuda_getCurrentRawStream"):
            return D.current_stream()
        _raw_stream_fns = (c._cuda_getCurrentRawStream, c._cuda_getDevice)
    raw, dev = _raw_stream_fns
    return int(raw(dev()))


def _errbuf():
    b = getattr(_tls, "err", None)
    if b is None:
        b = _tls.err = ctypes.create_string_buffer(1024)
    return b


def _last_index(value) -> int:
    """How many elements past the first the last element of array `value` lies (NumPy
    arrays are copied to a contiguous allocation; others use their strides)."""
    shape = tuple(int(d) for d in getattr(value, "shape", ()))
    if 0 in shape:
        return -1
    if isinstance(value, np.ndarray):
        return sum((n - 1) * abs(x) // value.itemsize for n, x in zip(shape, value.strides))
    stride = getattr(value, "stride", None)
    if callable(stride):
        st = tuple(int(x) for x in stride())
        return sum((n - 1) * abs(x) for n, x in zip(shape, st))
    n = 1
    for d in shape:
        n *= d
    return n - 1


@dataclass(frozen=True)
class KernelParam:
    name: str
    index: int
    is_constexpr: bool
    default: Any
    do_not_specialize: bool


def _writes(fn: ir.Func) -> set[int]:
    """Indices of pointer args the kernel may write through."""
    roots = {}
    out = set()
    for i, a in enumerate(fn.args):
        roots[a.id] = i
    for op in ir.walk(fn.body):
        if op.name in ("ptr_add", "broadcast", "splat", "expand_dims", "hint", "select",
                       "trans", "make_desc"):
            for o in op.operands[:1] if op.name != "select" else op.operands[1:]:
                if o.id in roots and op.results:
                    roots[op.result.id] = roots[o.id]
        if op.name == "for":
            body = op.regions[0]
            for a, i in zip(body.args[1:], op.operands[3:]):
                if i.id in roots:
                    roots[a.id] = roots[i.id]
            for r, i in zip(op.results, op.operands[3:]):
                if i.id in roots:
                    roots[r.id] = roots[i.id]
        if op.name in ("store", "atomic_rmw", "atomic_cas", "desc_store"):
            if op.operands[0].id in roots:
                out.add(roots[op.operands[0].id])
    return out


_MISSING = object()


def _same(a, b) -> bool:
    if a is b:
        return True
    if type(a) is not type(b):
        return False
    if isinstance(a, float):
        return struct.pack("<d", a) == struct.pack("<d", b)
    if isinstance(a, (tuple, list)):
        return len(a) == len(b) and all(_same(x, y) for x, y in zip(a, b))
    if isinstance(a, (int, str, bytes, bool, complex)):
        return a == b
    return False


class Launcher:
    """A compiled kernel plus the per-specialization launch plan."""

    def __init__(self, ck: C.CompiledKernel, runtime_names: list[str], writes: set[int],
                 constexprs: dict, deps: list | None = None):
        self.ck = ck
        self.runtime_names = runtime_names
        self.writes = writes
        self.constexprs = constexprs
        self.deps = list(deps or ())

    def current(self) -> bool:
        """Whether every global, module or class attribute the compile read still holds
        the value it read (floats by bit pattern, so 0.0 -> -0.0 is a change)."""
        for container, name, value, mapping in self.deps:
            now = container.get(name, _MISSING) if mapping else \
                getattr(container, name, _MISSING)
            if not _same(now, value):
                return False
        return True

    def __call__(self, grid, values: list, stream: int | None = None):
        arrays = [i for i, v in enumerate(values) if T.is_array_like(v)]
        for i in arrays:
            v = values[i]
            if i in self.writes and isinstance(v, np.ndarray) and not v.flags.writeable:
                raise ValueError(
                    f"argument `{self.runtime_names[i]}` is a read-only NumPy array, and "
                    "the kernel writes it; pass a writable array (for example a copy)")
        ptrs, bindings = T.bind_arrays([values[i] for i in arrays],
                                       {k for k, i in enumerate(arrays) if i in self.writes})
        packed = list(values)
        for i, p in zip(arrays, ptrs):
            packed[i] = p
        if stream is None:
            stream = D.current_stream()
        asserts = self.ck.gen.asserts
        if asserts:
            # ENCELADUS_DEBUG=1: the error buffer rides after the runtime arguments; the
            # launch synchronises and reports the first failing program.
            from enceladus_amd.runtime import hip
            if getattr(self, "_abuf", None) is None:
                self._abuf = T.zeros((5,), core.uint32)
            hip.call("ek_memset", ctypes.c_void_p(self._abuf.ptr), 0, 20, None)
            packed.append(self._abuf.ptr)
        self.ck.launch_raw(grid, self.ck.pack(packed), stream)
        if not asserts:
            T.complete_bindings(bindings)
        else:
            from enceladus_amd.runtime import hip
            T.flush_pending()
            hip.call("ek_device_sync")
            for b in bindings:
                T.finish_binding(b)
            rec = self._abuf.numpy()
            if rec[0]:
                a = asserts[int(rec[1])]
                raise DeviceAssertionError(a["msg"], a["loc"],
                                           (int(rec[2]), int(rec[3]), int(rec[4])))


def _const_canon(v):
    """A constexpr value as a key: type names and float bit patterns, recursively, so
    0.0 and -0.0 give different kernels, one NaN launch reuses another's kernel, and
    `2`, `2.0` and `True` (alone or inside tuples) stay apart. Raises TypeError for an
    unhashable value."""
    if isinstance(v, core.dtype):
        return ("dt", v.name)
    if isinstance(v, (list, tuple)):
        return (type(v).__name__,) + tuple(_const_canon(x) for x in v)
    if isinstance(v, float):
        return ("float", struct.pack("<d", v))
    hash(v)
    return (type(v).__name__, v)


# Float math modes (reference: runtime/jit.py:56). "relaxed" (the default) multiplies by
# the reciprocal of a broadcast row statistic instead of dividing by it; "fast" does so for
# every divisor that is uniform along the divided tile, scalars included.
MATH_MODES = ("relaxed", "fast")


class JITFunction:
    """A kernel or device function created by `@enceladus.jit`."""

    _ek_jit = True

    def __init__(self, fn: Callable, *, interpret=None, do_not_specialize=(),
                 math_mode: str = "relaxed"):
        if math_mode not in MATH_MODES:
            raise ValueError(f"math_mode must be one of {MATH_MODES}, but got {math_mode!r}")
        self.fn = fn
        self.__name__ = fn.__name__
        self.__doc__ = fn.__doc__
        self.math_mode = math_mode
        self.interpret = interpret
        sig = inspect.signature(fn)
        dns = set(do_not_specialize)
        self.params = []
        for i, p in enumerate(sig.parameters.values()):
            self.params.append(KernelParam(
                p.name, i, core.is_constexpr_annotation(p.annotation),
                p.default if p.default is not inspect.Parameter.empty else inspect.Parameter.empty,
                p.name in dns or i in dns))
        self.arg_names = [p.name for p in self.params]
        self._name_set = frozenset(self.arg_names)
        self._cache: dict[Any, Launcher] = {}
        self._fast: dict[Any, _FastEntry] = {}
        self._binders: dict[tuple, Callable] = {}

    def __repr__(self):
        return f"JITFunction({self.fn.__module__}:{self.__name__})"

    def __call__(self, *args, **kwargs):
        raise RuntimeError(f"`{self.__name__}` is an @enceladus.jit kernel: launch it as "
                           f"{self.__name__}[grid](...), or call it from another kernel")

    def __getitem__(self, grid):
        return lambda *args, **kwargs: self.run(*args, grid=grid, **kwargs)

    def _bind(self, args, kwargs):
        vals = {}
        if len(args) > len(self.params):
            raise TypeError(f"{self.__name__} takes {len(self.params)} arguments, got {len(args)}")
        for p, a in zip(self.params, args):
            vals[p.name] = a
        for k, v in kwargs.items():
            if k not in self.arg_names:
                raise TypeError(f"{self.__name__} got an unexpected argument `{k}`")
            vals[k] = v
        for p in self.params:
            if p.name not in vals:
                if p.default is inspect.Parameter.empty:
                    raise TypeError(f"{self.__name__}: missing a required argument: "
                                    f"'{p.name}'")
                vals[p.name] = p.default
        return vals

    def bind(self, args, kwargs):
        """Binds launch arguments to parameter names, applying defaults (reference:
        runtime/jit.py:349)."""
        return self._bind(tuple(args), dict(kwargs))

    def specialize(self, bound: dict):
        """Argument types, specialization facts and constexpr values of bound arguments
        (reference: runtime/jit.py:358)."""
        types, facts, consts = {}, {}, {}
        for p in self.params:
            v = bound[p.name]
            if p.is_constexpr:
                c = core.unwrap(v)
                try:
                    hash(c if not isinstance(c, list) else tuple(c))
                except TypeError:
                    raise TypeError(f"{self.__name__}: constexpr parameter `{p.name}` got an "
                                    f"unhashable {type(c).__name__}; pass a number, a string, "
                                    "a dtype or a tuple of those") from None
                consts[p.name] = c
                continue
            try:
                types[p.name] = arg_type(v)
            except TypeError as e:
                raise TypeError(f"{self.__name__}: argument `{p.name}`: {e}") from None
            f = arg_facts(v)
            if p.do_not_specialize:
                f = {k: x for k, x in f.items() if k in REQUIRED_FACTS}
            facts[p.name] = f
        return types, facts, consts

    def _key(self, types, facts, consts, num_warps, dot_warps):
        return (tuple((k, str(t)) for k, t in types.items()),
                tuple((k, tuple(sorted(f.items()))) for k, f in facts.items()),
                tuple((k, _const_canon(v)) for k, v in consts.items()), num_warps,
                tuple(dot_warps) if dot_warps else None)

    def _options(self, dot_warps) -> dict:
        """The compile options of a specialization: the same for launches, `warmup`, `ir`
        and `explain`, so each describes the kernel a launch runs."""
        options = {"dot_warps": tuple(dot_warps) if dot_warps else None,
                   "math_mode": self.math_mode}
        # ENCELADUS_CODEGEN="flag,flag=value": emitter switches for experiments (e.g.
        # no_staging, no_gemm_template, coarsen); part of the specialization key.
        for item in filter(None, os.environ.get("ENCELADUS_CODEGEN", "").split(",")):
            k, _, v = item.partition("=")
            v = v.strip()
            options[k.strip()] = int(v) if v.isdigit() else (v if v else True)
        # ENCELADUS_DEBUG=1 keeps tl.device_assert checks (part of the key)
        options["debug"] = _debug()
        return options

    def _compile_for(self, types, facts, consts, num_warps, dot_warps) -> Launcher:
        options = self._options(dot_warps)
        # a specialization an earlier process compiled skips the frontend and codegen
        plain = not (os.environ.get("ENCELADUS_OVERRIDE_DIR") or
                     os.environ.get("ENCELADUS_DUMP", "0") not in ("", "0"))
        skey = speccache.spec_key(self, types, facts, consts, num_warps, options) \
            if plain else None
        if skey is not None:
            hit = speccache.load(skey)
            if hit is not None:
                gen, ir_text, names, writes, deps = hit
                ck = C.CompiledKernel(gen, ir_text, C.compile_code(gen.source, gen.name))
                return Launcher(ck, names, writes, consts, deps)
        fn_ir = C.build_module(self, types, facts, consts, num_warps, options)
        ck = C.compile_ir(fn_ir, options)
        runtime_names = list(types.keys())
        writes = _writes(fn_ir)
        if skey is not None:
            speccache.store(skey, fn_ir, ck.gen, runtime_names, writes)
        return Launcher(ck, runtime_names, writes, consts, getattr(fn_ir, "deps", ()))

    def _lookup(self, vals, num_warps, dot_warps) -> Launcher:
        types, facts, consts = self.specialize(vals)
        key = (self._key(types, facts, consts, num_warps, dot_warps),
               os.environ.get("ENCELADUS_CODEGEN", ""),
               os.environ.get("ENCELADUS_OVERRIDE_DIR", ""), _debug())
        lc = self._cache.get(key)
        if lc is None or (lc.deps and not lc.current()):
            lc = self._compile_for(types, facts, consts, num_warps, dot_warps)
            self._cache[key] = lc
        return lc

    def _fast_key(self, args, kwargs, num_warps, dot_warps):
        """(key, runtime values) for the warm path, or None when an argument needs the
        general path (NumPy arrays, unknown or missing arguments, unhashable constexprs)."""
        if len(args) > len(self.params):
            return None                 # the general path raises the TypeError
        for k in kwargs:
            if k not in self._name_set:
                return None
        torch = _torch()
        tt = torch.Tensor if torch else ()
        n = len(args)
        key = [num_warps, dot_warps, _env_token()]
        rt = []
        for p in self.params:
            if p.index < n:
                v = args[p.index]
            elif p.name in kwargs:
                v = kwargs[p.name]
            elif p.default is not inspect.Parameter.empty:
                v = p.default
            else:
                return None
            t = type(v)
            if p.is_constexpr:
                c = core.unwrap(v)
                tc = type(c)
                if tc is float:
                    key.append((tc, struct.pack("<d", c)))
                elif tc in (int, bool, str) or isinstance(c, core.dtype):
                    key.append((tc, c))
                elif tc in (tuple, list):
                    # element types and float bit patterns, as the general key has them:
                    # (1,), (1.0,) and (True,) are different kernels
                    try:
                        key.append(_const_canon(c))
                    except TypeError:
                        return None
                else:
                    return None
                continue
            if t is int:
                key.append((int, v & 15 == 0, v == 1, _int_class(v)))
                rt.append(v)
            elif t is float:
                key.append((float, v > 0))
                rt.append(v)
            elif t is bool:
                key.append((bool,))
                rt.append(int(v))
            elif torch and isinstance(v, tt):
                if not v.is_cuda:
                    return None
                ptr = v.data_ptr()
                es = v.element_size()
                if v.is_contiguous():
                    last = v.numel() - 1
                else:
                    last = _last_index(v)
                key.append((v.dtype, ptr & 15 == 0, _span_class((last + 1) * es, last)))
                rt.append(ptr)
            elif t is T.Tensor:
                ptr = v.ptr
                last = _last_index(v)
                key.append((v.dtype.name, ptr & 15 == 0,
                            _span_class((last + 1) * v.itemsize, last)))
                rt.append(ptr)
            else:
                return None
        return tuple(key), rt

    def _make_binder(self, nargs: int, kwnames: tuple, args, kwargs):
        """A key function for one call shape (the number of positional arguments and the
        keyword names in order), specialised to the Python types the arguments had when the
        shape was first seen. It returns what `_fast_key` returns for the same call (the
        same key tuple, the same runtime values) or None when an argument has another type
        (then `_fast_key` runs). Generated once per shape, it replaces the per-parameter
        dispatch of `_fast_key` with straight-line code."""
        if nargs > len(self.params):
            return lambda *_: None      # the general path raises the TypeError
        torch = _torch()
        ns = {"_env": _env_token, "_ic": _int_class, "_sc": _span_class, "_li": _last_index,
              "_unwrap": core.unwrap, "_pack": struct.pack, "_dtype": core.dtype,
              "_TT_cls": T.Tensor}
        lines = [f"def _bind(args, kwargs, nw, dw):"]
        if nargs:
            lines.append("    " + ", ".join(f"a{i}" for i in range(nargs)) +
                         (", = args" if nargs == 1 else " = args"))
        for k in kwnames:
            if k not in self._name_set:
                return lambda *_: None
            lines.append(f"    k_{k} = kwargs[{k!r}]")
        parts, rts = [], []
        for j, prm in enumerate(self.params):
            if prm.index < nargs:
                v, sample = f"a{prm.index}", args[prm.index]
            elif prm.name in kwnames:
                v, sample = f"k_{prm.name}", kwargs[prm.name]
            elif prm.default is not inspect.Parameter.empty:
                v, sample = f"_D{j}", prm.default
                ns[v] = prm.default
            else:
                return lambda *_: None
            if prm.is_constexpr:
                lines += [f"    c{j} = _unwrap({v})", f"    t{j} = type(c{j})",
                          f"    if t{j} is float:", f"        q{j} = (t{j}, _pack('<d', c{j}))",
                          f"    elif t{j} in (int, bool, str) or isinstance(c{j}, _dtype):",
                          f"        q{j} = (t{j}, c{j})", "    else:", "        return None"]
                parts.append(f"q{j}")
                continue
            ts = type(sample)
            if ts is int:
                lines += [f"    if type({v}) is not int:", "        return None"]
                parts.append(f"(int, {v} & 15 == 0, {v} == 1, _ic({v}))")
                rts.append(v)
            elif ts is float:
                lines += [f"    if type({v}) is not float:", "        return None"]
                parts.append(f"(float, {v} > 0)")
                rts.append(v)
            elif ts is bool:
                lines += [f"    if type({v}) is not bool:", "        return None"]
                parts.append("(bool,)")
                rts.append(f"int({v})")
            elif torch is not None and isinstance(sample, torch.Tensor):
                ns[f"_TT{j}"] = ts
                lines += [f"    if type({v}) is not _TT{j} or not {v}.is_cuda:", "        return None",
                          f"    p{j} = {v}.data_ptr()",
                          f"    l{j} = {v}.numel() - 1 if {v}.is_contiguous() else _li({v})",
                          f"    s{j} = _sc((l{j} + 1) * {v}.element_size(), l{j})"]
                parts.append(f"({v}.dtype, p{j} & 15 == 0, s{j})")
                rts.append(f"p{j}")
            elif ts is T.Tensor:
                lines += [f"    if type({v}) is not _TT_cls:", "        return None",
                          f"    p{j} = {v}.ptr", f"    l{j} = _li({v})"]
                parts.append(f"({v}.dtype.name, p{j} & 15 == 0, "
                             f"_sc((l{j} + 1) * {v}.itemsize, l{j}))")
                rts.append(f"p{j}")
            else:
                return lambda *_: None
        lines.append(f"    return (nw, dw, _env(), {', '.join(parts)}{',' if parts else ''}), "
                     f"[{', '.join(rts)}]")
        exec(compile("\n".join(lines), f"<binder {self.__name__}>", "exec"), ns)
        return ns["_bind"]

    def _fast_launch(self, ent: _FastEntry, rt, args, kwargs, grid, stream):
        if callable(grid):
            grid = grid(dict(self._bind(args, kwargs)))
        if type(grid) is tuple and len(grid) == 1 and type(grid[0]) is int and \
                0 <= grid[0] < 1 << 31:
            gx, gy, gz = grid[0], 1, 1      # the common 1-D grid, already valid
        else:
            grid = tuple(int(g) for g in (grid if isinstance(grid, (tuple, list))
                                          else (grid,)))
            if not 1 <= len(grid) <= 3:
                raise ValueError(f"grid must have 1 to 3 dimensions, got {grid}")
            if grid[0] >= 1 << 31 or any(g > 65535 for g in grid[1:]) or \
                    any(g < 0 for g in grid):
                raise ValueError(f"grid {grid} exceeds the HIP limits (x < 2^31, y, z <= 65535)")
            gx, gy, gz = (grid + (1, 1))[:3]
        if gx == 0 or gy == 0 or gz == 0:
            return ent.lc.ck
        if _trace._active is not None:
            return None                 # `enceladus.capture` records the general path
        try:
            kb = ent.st.pack(*rt)
        except (struct.error, OverflowError):
            return None                 # a float beyond fp32's range: general packing
        if stream is None:
            stream = _launch_stream()
        t = _timing.current()
        if t is not None:
            t.launch(stream, ent.fn, (gx, gy, gz), ent.block, kb, len(kb))
            return ent.lc.ck
        err = _errbuf()
        if _ek_launch()(stream or None, ent.fn, gx, gy, gz, ent.block, 1, 1, 0, kb, len(kb),
                        err, 1024):
            from enceladus_amd.compiler.errors import HipError
            raise HipError(f"ek_launch: {err.value.decode(errors='replace')}")
        return ent.lc.ck

    def run(self, *args, grid, num_warps: int = 4, num_stages=None, dot_warps=None,
            dot_backend: str = "auto", stream=None, **kwargs):
        """Launches the kernel (reference: runtime/jit.py:388). `num_stages` is accepted for
        Triton compatibility and has no effect; `dot_backend` ("auto", "simdgroup", "mpp")
        is checked and every `tl.dot` lowers to MFMA; `stream` (a HIP stream handle)
        defaults to torch's current stream."""
        if dot_backend != "auto":
            check_dot_backend(dot_backend)
        fk = None
        if not self.interpret:
            shape = (len(args), tuple(kwargs))
            b = self._binders.get(shape)
            if b is None:
                b = self._binders[shape] = self._make_binder(shape[0], shape[1], args, kwargs)
            fk = b(args, kwargs, num_warps, dot_warps)
            if fk is None:
                fk = self._fast_key(args, kwargs, num_warps, dot_warps)
        if fk is not None:
            ent = self._fast.get(fk[0])
            if ent is not None and (not ent.lc.deps or ent.lc.current()):
                ck = self._fast_launch(ent, fk[1], args, kwargs, grid, stream)
                if ck is not None:
                    return ck
        if self.interpret or os.environ.get("ENCELADUS_INTERPRET") == "1":
            raise RuntimeError("ENCELADUS_INTERPRET=1 selects the CPU interpreter, which this "
                               "MI355X backend ships only as test infrastructure (oracle/); "
                               "unset it to run on the GPU")
        if num_warps not in (1, 2, 4, 8, 16):
            raise ValueError(f"num_warps must be 1, 2, 4, 8 or 16 (wave64), got {num_warps}")
        vals = self._bind(args, kwargs)
        lc = self._lookup(vals, num_warps, dot_warps)
        if callable(grid):
            grid = grid(dict(vals))
        grid = tuple(int(g) for g in (grid if isinstance(grid, (tuple, list)) else (grid,)))
        if not 1 <= len(grid) <= 3:
            raise ValueError(f"grid must have 1 to 3 dimensions, got {grid}")
        if grid[0] >= 1 << 31 or any(g > 65535 for g in grid[1:]) or any(g < 0 for g in grid):
            raise ValueError(f"grid {grid} exceeds the HIP limits (x < 2^31, y, z <= 65535)")
        values = [vals[n] for n in lc.runtime_names]
        lc(grid, values, stream)
        if fk is not None:
            cur = self._fast.get(fk[0])
            if cur is None or cur.lc is not lc:
                # first launch of this key, or a recompile after a global the kernel reads
                # changed: the warm entry follows the launcher now in use
                ent = _fast_entry(lc)
                if ent is not None:
                    self._fast[fk[0]] = ent
                else:
                    self._fast.pop(fk[0], None)
        return lc.ck

    def warmup(self, *args, grid=None, num_warps: int = 4, dot_warps=None,
               dot_backend: str = "auto", _record: bool = True, **kwargs):
        """Compiles the kernel for these arguments without launching it and returns the
        `CompiledKernel` (`.hip`, `.ir`, `.lds_bytes`, `.num_warps`; reference:
        runtime/jit.py:527). `dot_backend` is checked and otherwise has no effect: every
        `tl.dot` lowers to MFMA."""
        check_dot_backend(dot_backend)
        vals = self._bind(args, kwargs)
        return self._lookup(vals, num_warps, dot_warps).ck

    def ir(self, *args, num_warps: int = 4, dot_warps=None, **kwargs) -> ir.Func:
        """The verified IR of the specialization these arguments select, after the pass
        pipeline, without compiling or launching (reference: runtime/jit.py:378)."""
        vals = self._bind(args, kwargs)
        types, facts, consts = self.specialize(vals)
        return C.build_module(self, types, facts, consts, num_warps, self._options(dot_warps))

    ir_for = ir

    def explain(self, *args, grid=None, num_warps: int = 4, dot_warps=None,
                dot_backend: str = "auto", full: bool = False, **kwargs) -> str:
        """Prints and returns a report of the compiler's decisions for the specialization
        these arguments select (reference: runtime/jit.py:539): MFMA plans, layout
        conversions and LDS by source line. `full=True` appends the IR and the generated
        HIP."""
        from enceladus_amd.compiler import codegen_hip
        from enceladus_amd.compiler import explain as EX
        ck = self.warmup(*args, num_warps=num_warps, dot_warps=dot_warps,
                         dot_backend=dot_backend, **kwargs)
        if ck.gen.report is None:
            # loaded from the specialization cache: regenerate the emitter's report with
            # the options the loaded kernel was compiled with
            fn_ir = self.ir(*args, num_warps=num_warps, dot_warps=dot_warps, **kwargs)
            ck.gen.report = codegen_hip.generate(fn_ir, self._options(dot_warps)).report
        if grid is not None and not callable(grid):
            grid = tuple(grid) if isinstance(grid, (tuple, list)) else (grid,)
        elif callable(grid):
            grid = tuple(grid(dict(self._bind(args, kwargs))))
        text = EX.explain(ck, grid)
        if full:
            text += f"\n\n--- IR ---\n{ck.ir}\n--- HIP ---\n{ck.hip}"
        print(text)
        return text


DOT_BACKENDS = ("auto", "simdgroup", "mpp")


def check_dot_backend(backend: str) -> str:
    """The reference's `tl.dot` backend names (runtime/dot_backend.py:108-116). On MI355X
    every backend lowers to MFMA; an unknown name raises ValueError as there."""
    if backend not in DOT_BACKENDS:
        raise ValueError(f"dot_backend must be one of {DOT_BACKENDS}, not {backend!r}")
    return backend


def jit(fn=None, *, interpret=None, do_not_specialize=(), math_mode: str = "relaxed"):
    def deco(f):
        return JITFunction(f, interpret=interpret, do_not_specialize=do_not_specialize,
                           math_mode=math_mode)
    if fn is not None:
        return deco(fn)
    return deco
