"""The persistent specialization cache: a launch whose specialization a previous process
compiled skips the frontend and the code generator.

The key is computed before any compilation, from what decides the generated code: the
kernel's source text, the specialization (argument types and facts, constexpr values,
`num_warps`, `dot_warps`, code-generation options) and a hash of the compiler (its Python
sources and device headers) and of the HIP runtime version (reference: runtime/compile.py:38-47
and runtime/cache.py:97-144 key on kernel source and specialization the same way). The entry
(`$ENCELADUS_CACHE_DIR/specs/<key>.json`) holds the generated source and the launch metadata
(kernel arguments, block size, flush plan, runtime argument names, written arguments,
IR text), and the fingerprints of the globals and attributes the frontend read while
compiling. The code object itself stays in the code-object cache under its source hash.

A hit is used only when every recorded global or attribute still has the fingerprinted
value in this process: numbers, strings, tuples and dtypes by value, functions and @jit
kernels by the hash of their source text. A compile that read something without a
fingerprint (a closure cell, an arbitrary object) is not stored.
"""

from __future__ import annotations

import hashlib
import inspect
import json
import logging
import os
import struct
import sys
import threading
import weakref
from pathlib import Path

from enceladus_amd.compiler import codegen_hip
from enceladus_amd.language import core

log = logging.getLogger("enceladus")

_lock = threading.Lock()
# function -> (its code object, hash of its source); weak keys, so a collected function's
# entry goes with it and a new function can never inherit it
_src_hash: "weakref.WeakKeyDictionary" = weakref.WeakKeyDictionary()
_COMPILER = None


def hashed_sources(root: Path | None = None) -> list[Path]:
    """Every file whose text decides generated code or launch metadata: all Python sources
    of the package (frontend, passes, emitter, and the runtime's pass pipeline, argument
    facts and specialization rules) and the device headers."""
    root = root or Path(__file__).resolve().parent.parent
    files = [p for p in root.rglob("*.py") if "__pycache__" not in p.parts]
    files += list((root / "csrc" / "include").glob("*.h"))
    return sorted(files, key=lambda p: p.relative_to(root).as_posix())


def tree_hash(root: Path) -> "hashlib._Hash":
    """sha256 over the names and bytes of `hashed_sources(root)`."""
    h = hashlib.sha256()
    for p in hashed_sources(root):
        h.update(p.relative_to(root).as_posix().encode())
        h.update(p.read_bytes())
    return h


def compiler_hash() -> str:
    """Changes whenever any Python source of the package, the device headers or the HIP
    runtime change."""
    global _COMPILER
    if _COMPILER is None:
        h = tree_hash(Path(__file__).resolve().parent.parent)
        try:
            from enceladus_amd.runtime import hip
            lib = hip.load_library()
            v = __import__("ctypes").c_int(0)
            lib.ek_runtime_version(__import__("ctypes").byref(v))
            h.update(f"{lib.ek_version().decode()}|{v.value}".encode())
        except Exception:  # noqa: BLE001 - no shim: the key still covers the compiler
            pass
        _COMPILER = h.hexdigest()[:24]
    return _COMPILER


def _source_hash(fn) -> str | None:
    code = getattr(fn, "__code__", None)
    try:
        hit = _src_hash.get(fn)
    except TypeError:                   # not weak-referenceable: hash it every time
        hit = None
    if hit is not None and hit[0] is code:
        return hit[1]
    try:
        src = inspect.getsource(fn)
    except (OSError, TypeError):
        return None
    h = hashlib.sha256(src.encode()).hexdigest()[:24]
    try:
        _src_hash[fn] = (code, h)
    except TypeError:
        pass
    return h


def _canon(v):
    """A JSON-able canonical form of a specialization component."""
    if isinstance(v, core.dtype):
        return ["dt", v.name]
    if isinstance(v, float):
        return ["f", struct.pack("<d", v).hex()]
    if isinstance(v, (bool, int, str)) or v is None:
        return [type(v).__name__, v]
    if isinstance(v, (tuple, list)):
        return [type(v).__name__] + [_canon(x) for x in v]
    if isinstance(v, dict):
        return ["d"] + [[k, _canon(x)] for k, x in sorted(v.items())]
    if hasattr(v, "shape") and hasattr(v, "dtype"):
        return ["ttype", str(v)]
    return None


def spec_key(jfn, types, facts, consts, num_warps, options) -> str | None:
    src = _source_hash(jfn.fn)
    if src is None:
        return None
    parts = [src, jfn.fn.__module__, jfn.fn.__qualname__,
             [[k, str(t)] for k, t in types.items()], _canon(facts), _canon(consts),
             num_warps, _canon(dict(options)), compiler_hash()]
    if any(p is None for p in parts[4:7]):
        return None
    return hashlib.sha256(json.dumps(parts, sort_keys=True).encode()).hexdigest()


# -- dependency fingerprints ----------------------------------------------------------

def _fingerprint(v):
    v = core.unwrap(v)
    if v is None or isinstance(v, (bool, int, str)):
        return ["lit", type(v).__name__, v]
    if isinstance(v, float):
        return ["f", struct.pack("<d", v).hex()]
    if isinstance(v, core.dtype):
        return ["dt", v.name]
    if isinstance(v, (tuple, list)):
        parts = [_fingerprint(x) for x in v]
        return None if any(p is None for p in parts) else [type(v).__name__] + parts
    fn = getattr(v, "fn", None) if getattr(v, "_ek_jit", False) else None
    target = fn if fn is not None else v
    if inspect.isfunction(target):
        h = _source_hash(target)
        return None if h is None else ["src", h]
    return None


def _owner_name(container) -> list | None:
    """How to find `container` again in another process."""
    if isinstance(container, dict):
        mod = container.get("__name__")
        if isinstance(mod, str) and sys.modules.get(mod) is not None and \
                sys.modules[mod].__dict__ is container:
            return ["globals", mod]
        return None
    if inspect.ismodule(container):
        return ["module", container.__name__]
    if inspect.isclass(container):
        return ["class", container.__module__, container.__qualname__]
    return None


def _resolve(owner):
    kind = owner[0]
    mod = sys.modules.get(owner[1])
    if mod is None:
        return None
    if kind == "globals":
        return mod.__dict__
    if kind == "module":
        return mod
    obj = mod
    for part in owner[2].split("."):
        obj = getattr(obj, part, None)
        if obj is None:
            return None
    return obj


def _fingerprint_deps(deps) -> list | None:
    out = []
    for container, name, value, mapping in deps:
        owner = _owner_name(container)
        fp = _fingerprint(value)
        if owner is None or fp is None:
            return None
        out.append([owner, name, mapping, fp])
    return out


def _live_deps(recorded) -> list | None:
    """The recorded dependencies resolved in this process, when all still match."""
    live = []
    for owner, name, mapping, fp in recorded:
        container = _resolve(owner)
        if container is None:
            return None
        missing = object()
        v = container.get(name, missing) if mapping else getattr(container, name, missing)
        if v is missing or _fingerprint(v) != fp:
            return None
        live.append((container, name, v, mapping))
    return live


# -- entries ---------------------------------------------------------------------------

def _path(key: str) -> Path:
    from enceladus_amd.runtime.compile import cache_dir
    return cache_dir() / "specs" / key[:2] / f"{key}.json"


def _gen_to_json(gen) -> dict | None:
    try:
        asserts = json.loads(json.dumps(gen.asserts))
        flush = json.loads(json.dumps(gen.flush))
    except (TypeError, ValueError):
        return None
    return {"name": gen.name, "source": gen.source, "num_warps": gen.num_warps,
            "lds_bytes": gen.lds_bytes, "block": gen.block, "coarsen": gen.coarsen,
            "asserts": asserts, "flush": flush,
            "args": [[a.name, a.kind, a.dtype.name if a.dtype else None, a.cparam]
                     for a in gen.args]}


def _gen_from_json(d: dict):
    args = [codegen_hip.KernelArg(n, k, core.dtype_from_name(dt) if dt else None, cp)
            for n, k, dt, cp in d["args"]]
    g = codegen_hip.GeneratedKernel(d["name"], d["source"], args, d["num_warps"],
                                    d["lds_bytes"], d["block"])
    g.coarsen = d["coarsen"]
    g.asserts = d["asserts"]
    g.flush = d["flush"]
    g.report = None          # `explain` regenerates the report
    return g


def store(key: str, fn_ir, gen, runtime_names, writes) -> None:
    if os.environ.get("ENCELADUS_ALWAYS_COMPILE") == "1":
        return
    deps = _fingerprint_deps(getattr(fn_ir, "deps", ()))
    g = _gen_to_json(gen)
    if deps is None or g is None:
        return
    from enceladus_amd.compiler import ir
    entry = {"gen": g, "deps": deps, "runtime_names": list(runtime_names),
             "writes": sorted(writes), "ir": ir.print_func(fn_ir)}
    p = _path(key)
    try:
        p.parent.mkdir(parents=True, exist_ok=True)
        tmp = p.with_suffix(f".tmp{os.getpid()}.{threading.get_ident()}")
        tmp.write_text(json.dumps(entry))
        os.replace(tmp, p)
    except OSError as e:
        log.debug("couldn't store specialization %s: %s", key, e)


def load(key: str):
    """(GeneratedKernel, IR text, runtime names, written indices, live deps) or None."""
    if os.environ.get("ENCELADUS_ALWAYS_COMPILE") == "1":
        return None
    p = _path(key)
    try:
        entry = json.loads(p.read_text())
    except (OSError, ValueError):
        return None
    try:
        live = _live_deps(entry["deps"])
        if live is None:
            return None
        return (_gen_from_json(entry["gen"]), entry["ir"], entry["runtime_names"],
                set(entry["writes"]), live)
    except (KeyError, TypeError, ValueError) as e:
        log.debug("unusable specialization entry %s: %s", p, e)
        return None
