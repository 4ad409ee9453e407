"""`@autotune`, `Config` and `heuristics` (reference: src/enceladus/runtime/autotuner.py:54-585).

On the first launch for a key, every candidate config is compiled (in a thread pool:
hiprtc programs are per-call objects) and timed with HIP events on the launch stream:
phase 1 times each config, phase 2 times the few fastest again in interleaved rounds, and
the earliest finalist within `tolerance` of the fastest wins (the reference's rule). The
winner is kept in memory and merged, under a file lock, into
`$ENCELADUS_CACHE_DIR/autotune/<kernel and compiler hash>/<arch>.json`; a saved winner that
is no longer a candidate is re-tuned, and a compiler change starts a new file. Arguments in
`restore_value` are restored and those in `reset_to_zero` zeroed before every timed run
and after tuning, so in-place kernels don't accumulate. Configs that fail to compile or
run are skipped with a warning.
"""

from __future__ import annotations

import contextlib
import hashlib
import inspect
import json
import logging
import os
import statistics
import threading
import warnings
from concurrent.futures import ThreadPoolExecutor
from typing import Any, Callable

import numpy as np

log = logging.getLogger("enceladus.autotune")

FINALISTS = 3          # configs timed again in phase 2
FINALIST_BAND = 0.10   # ... when within this fraction of the phase-1 best
FINAL_ROUNDS = 3


class Config:
    def __init__(self, kwargs: dict, num_warps: int = 4, num_stages=None, dot_warps=None,
                 dot_backend: str = "auto", pre_hook: Callable | None = None):
        self.kwargs = dict(kwargs)
        self.num_warps = num_warps
        self.num_stages = num_stages
        self.dot_warps = tuple(dot_warps) if dot_warps else None
        self.dot_backend = dot_backend
        self.pre_hook = pre_hook

    def _key(self):
        return (tuple(sorted(self.kwargs.items())), self.num_warps, self.dot_warps)

    def __eq__(self, other):
        return isinstance(other, Config) and self._key() == other._key()

    def __hash__(self):
        return hash(self._key())

    def __repr__(self):
        kw = ", ".join(f"{k}={v}" for k, v in self.kwargs.items())
        return f"Config({kw}, num_warps={self.num_warps}, dot_warps={self.dot_warps})"

    def launch_options(self) -> dict:
        out = {"num_warps": self.num_warps}
        if self.dot_warps:
            out["dot_warps"] = self.dot_warps
        return out

    def to_json(self) -> dict:
        return {"kwargs": self.kwargs, "num_warps": self.num_warps,
                "dot_warps": list(self.dot_warps) if self.dot_warps else None}

    @staticmethod
    def from_json(d: dict) -> "Config":
        return Config(dict(d["kwargs"]), int(d["num_warps"]), dot_warps=d.get("dot_warps"))


def _jit_of(fn):
    """The JITFunction under a Heuristics wrapper (or `fn` itself)."""
    return fn.jit if isinstance(fn, Heuristics) else fn


def _named(fn, args, kwargs) -> dict:
    """Launch arguments by name, with the kernel signature's defaults applied."""
    jfn = _jit_of(fn)
    named = {p.name: p.default for p in jfn.params if p.default is not inspect.Parameter.empty}
    named.update(zip(jfn.arg_names, args))
    named.update(kwargs)
    return named


def _key_value(v) -> str:
    """One key argument: arrays contribute their shape, scalars their value (a NumPy
    scalar and the Python number share a key), dtypes their name."""
    if isinstance(v, np.generic):
        return repr(v.item())
    from enceladus_amd.language import core
    if isinstance(v, core.dtype):
        return v.name
    if isinstance(v, (type, np.dtype)) or (isinstance(v, str) and v in _DTYPE_NAMES):
        with contextlib.suppress(Exception):
            return core.dtype_from_numpy(np.dtype(v)).name
    shape = getattr(v, "shape", None)
    if shape is not None and hasattr(v, "dtype"):
        if len(shape) == 0 and hasattr(v, "item"):
            return repr(v.item())
        return str(list(shape))
    return repr(v)


_DTYPE_NAMES = {"float16", "float32", "bfloat16", "int8", "int16", "int32", "int64", "uint8",
                "uint16", "uint32", "uint64", "bool"}


def _compiler_hash() -> str:
    """Changes whenever the code generator or the device templates change."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    h = hashlib.sha256()
    for sub in ("compiler", os.path.join("csrc", "include")):
        d = os.path.join(root, sub)
        for name in sorted(os.listdir(d)):
            if name.endswith((".py", ".h")):
                with open(os.path.join(d, name), "rb") as f:
                    h.update(f.read())
    return h.hexdigest()[:16]


# -- argument state around timed runs ----------------------------------------------

def _snapshot(v):
    if isinstance(v, np.ndarray):
        return v.copy()
    if hasattr(v, "clone") and hasattr(v, "copy_"):
        return v.clone()
    if hasattr(v, "numpy"):
        return v.numpy()
    return None


def _restore(v, snap) -> None:
    if snap is None:
        return
    if isinstance(v, np.ndarray):
        v[...] = snap
    elif hasattr(v, "copy_") and not hasattr(v, "copy_from_numpy"):
        v.copy_(snap)
    elif hasattr(v, "copy_from_numpy"):
        v.copy_from_numpy(snap)


def _zero(v) -> None:
    if isinstance(v, np.ndarray):
        v[...] = 0
    elif hasattr(v, "zero_"):
        v.zero_()
    elif hasattr(v, "copy_from_numpy"):
        from enceladus_amd.runtime import hip
        import ctypes
        if v.nbytes:
            hip.call("ek_memset", ctypes.c_void_p(v.ptr), 0, v.nbytes, None)


class Autotuner:
    def __init__(self, fn, configs, key, prune_configs_by=None, reset_to_zero=None,
                 restore_value=None, warmup_ms=50, rep=20, tolerance=0.01):
        self.fn = fn
        self.configs = list(configs)
        self.key = list(key)
        self.prune = dict(prune_configs_by or {})
        self.reset_to_zero = list(reset_to_zero or [])
        self.restore_value = list(restore_value or [])
        self.warmup_ms = warmup_ms
        self.rep = rep
        self.tolerance = tolerance
        self.best: dict[str, Config] = {}
        self.timings: dict[str, dict] = {}
        self._saved: dict[str, Config] = {}
        self._loaded = False
        self._lock = threading.Lock()
        self.__name__ = getattr(fn, "__name__", "kernel")
        self._ek_jit = False

    @property
    def arg_names(self):
        return _jit_of(self.fn).arg_names

    @property
    def cache(self) -> dict:
        return self.best

    def __getitem__(self, grid):
        return lambda *args, **kwargs: self.run(*args, grid=grid, **kwargs)

    # -- keys and persistence ------------------------------------------------------
    def _key(self, named: dict) -> str:
        from enceladus_amd.runtime import tensor as T
        parts = [_key_value(named.get(k)) for k in self.key]
        dts = [T.elem_dtype(named[n]).name for n in self.arg_names
               if n in named and T.is_array_like(named[n])]
        return "|".join(parts) + "|" + ",".join(dts)

    def _path(self):
        from enceladus_amd.runtime.compile import ARCH, cache_dir
        src = inspect.getsource(_jit_of(self.fn).fn)
        h = hashlib.sha256((src + _compiler_hash()).encode()).hexdigest()[:24]
        return cache_dir() / "autotune" / f"{self.__name__}-{h}" / f"{ARCH}.json"

    def _load(self):
        self._loaded = True
        if os.environ.get("ENCELADUS_ALWAYS_COMPILE") == "1":
            return
        try:
            data = json.loads(self._path().read_text())
        except (OSError, ValueError):
            return
        for k, v in data.items():
            with contextlib.suppress(KeyError, TypeError, ValueError):
                self._saved.setdefault(k, Config.from_json(v))

    def _from_saved(self, key: str, named: dict):
        """The candidate matching the saved winner for `key` (keeping its pre_hook); a
        saved winner that is no longer a candidate is re-tuned."""
        saved = self._saved.pop(key, None)
        if saved is None:
            return None
        return next((c for c in self._candidates(named) if c == saved), None)

    def _save(self):
        import fcntl
        p = self._path()
        try:
            p.parent.mkdir(parents=True, exist_ok=True)
            with open(p.with_suffix(".lock"), "a") as lock:
                fcntl.flock(lock, fcntl.LOCK_EX)
                data: dict = {}
                with contextlib.suppress(OSError, ValueError):
                    loaded = json.loads(p.read_text())
                    if isinstance(loaded, dict):
                        data = loaded
                data.update({k: c.to_json() for k, c in self.best.items()})
                tmp = p.with_suffix(f".tmp{os.getpid()}.{threading.get_ident()}")
                tmp.write_text(json.dumps(data, indent=1, sort_keys=True))
                os.replace(tmp, p)
        except OSError as e:
            log.debug("couldn't save autotuning results: %s", e)

    # -- candidates ----------------------------------------------------------------
    def _candidates(self, named: dict) -> list:
        cfgs = list(self.configs)
        early = self.prune.get("early_config_prune")
        if early is not None:
            cfgs = list(early(cfgs, named))
        model, top_k = self.prune.get("perf_model"), self.prune.get("top_k")
        if model is not None and top_k:
            scored = sorted(cfgs, key=lambda c: model(**{**named, **c.kwargs},
                                                       num_warps=c.num_warps))
            n = int(top_k * len(cfgs)) if isinstance(top_k, float) else int(top_k)
            cfgs = scored[:max(1, n)]
        return cfgs

    def prune_configs(self, named) -> list:
        return self._candidates(named)

    def config_for(self, *args, **kwargs):
        """The tuned config for these launch arguments, or None if not tuned yet."""
        return self.best.get(self._key(_named(self.fn, args, kwargs)))

    def _config_without_tuning(self, args, kwargs) -> Config:
        if not self._loaded:
            self._load()
        named = _named(self.fn, args, kwargs)
        key = self._key(named)
        with self._lock:
            cfg = self.best.get(key)
            if cfg is None:
                cfg = self._from_saved(key, named)
                if cfg is not None:
                    self.best[key] = cfg
        return cfg if cfg is not None else self._candidates(named)[0]

    def warmup(self, *args, **kwargs):
        """Compiles (never benchmarks) with the tuned config, or the first candidate."""
        cfg = self._config_without_tuning(args, kwargs)
        return self.fn.warmup(*args, **kwargs, **cfg.kwargs, **cfg.launch_options())

    def explain(self, *args, **kwargs) -> str:
        cfg = self._config_without_tuning(args, kwargs)
        return self.fn.explain(*args, **kwargs, **cfg.kwargs, **cfg.launch_options())

    # -- launching and tuning ------------------------------------------------------
    def run(self, *args, grid, **kwargs):
        if not self._loaded:
            self._load()
        named = _named(self.fn, args, kwargs)
        key = self._key(named)
        cfg = self.best.get(key)
        if cfg is None:
            with self._lock:
                cfg = self.best.get(key) or self._from_saved(key, named)
                if cfg is None:
                    cfg = self._tune(key, args, kwargs, grid, named)
                self.best[key] = cfg
        if os.environ.get("ENCELADUS_PRINT_AUTOTUNING", "0") not in ("", "0"):
            print(f"autotune {self.__name__} [{key}]: {cfg}")
        if cfg.pre_hook:
            cfg.pre_hook(named)
        return self.fn.run(*args, grid=grid, **cfg.kwargs, **cfg.launch_options(), **kwargs)

    def _tune(self, key, args, kwargs, grid, named) -> Config:
        from enceladus_amd.testing import do_bench
        cfgs = self._candidates(named)
        if not cfgs:
            raise ValueError(f"no autotune configs left for {self.__name__}")
        errors: dict[int, Exception] = {}

        def compile_one(i):
            c = cfgs[i]
            self.fn.warmup(*args, **c.kwargs, **c.launch_options(), **kwargs)
        with ThreadPoolExecutor(max_workers=min(8, len(cfgs))) as ex:
            futs = [ex.submit(compile_one, i) for i in range(len(cfgs))]
            for i, f in enumerate(futs):
                try:
                    f.result()
                except Exception as e:  # noqa: BLE001 - reported below
                    errors[i] = e
        for i, e in errors.items():
            warnings.warn(f"{self.__name__}: skipping {cfgs[i]}: {e}", stacklevel=4)
        saved = {n: _snapshot(named[n]) for n in self.restore_value if n in named}

        def settle():
            for n, snap in saved.items():
                _restore(named[n], snap)
            for n in self.reset_to_zero:
                if n in named:
                    _zero(named[n])

        def launch(c):
            settle()
            if c.pre_hook:
                c.pre_hook(named)
            self.fn.run(*args, grid=grid, **c.kwargs, **c.launch_options(), **kwargs)

        def bench(i, warmup_ms, rep, mode):
            try:
                return do_bench(lambda: launch(cfgs[i]), warmup=warmup_ms, rep=rep,
                                return_mode=mode)
            except Exception as e:  # noqa: BLE001 - a config that fails to launch is skipped
                errors[i] = e
                warnings.warn(f"{self.__name__}: skipping {cfgs[i]}: {e}", stacklevel=5)
                return None

        timings: dict[int, float] = {}
        for i in range(len(cfgs)):
            if i not in errors:
                t = bench(i, self.warmup_ms, self.rep, "median")
                if t is not None:
                    timings[i] = t
        order = sorted(timings, key=timings.get)
        finalists = [i for i in order[:FINALISTS]
                     if timings[i] <= timings[order[0]] * (1 + FINALIST_BAND)] if order else []
        if len(finalists) > 1:
            samples: dict[int, list] = {i: [] for i in finalists}
            for _ in range(FINAL_ROUNDS):
                for i in finalists:
                    if i not in errors:
                        s = bench(i, 0, max(3, self.rep // 4) + 1, "all")
                        if s is not None:
                            samples[i] += s[1:]
            for i in finalists:
                if i in errors or not samples[i]:
                    timings.pop(i, None)
                else:
                    timings[i] = statistics.median(samples[i])
            finalists = [i for i in finalists if i in timings]
        from enceladus_amd.runtime import device as D
        D.synchronize()
        settle()
        if not timings:
            first = next(iter(errors.values()), None)
            raise RuntimeError(f"every autotune config of {self.__name__} failed to compile or "
                               f"run; the first error was: {first}") from first
        pool = finalists if len(finalists) > 1 else list(timings)
        fastest = min(timings[i] for i in pool)
        best_i = min(i for i in pool if timings[i] <= fastest * (1 + self.tolerance))
        best = cfgs[best_i]
        self.best[key] = best
        self.timings[key] = {repr(cfgs[i]): t for i, t in timings.items()}
        self._save()
        return best


def autotune(configs, key, prune_configs_by=None, reset_to_zero=None, restore_value=None,
             warmup_ms=50, rep=20, tolerance=0.01):
    def deco(fn):
        return Autotuner(fn, configs, key, prune_configs_by, reset_to_zero, restore_value,
                         warmup_ms, rep, tolerance)
    return deco


class Heuristics:
    """Computes constexprs from the other launch arguments (reference: autotuner.py:233)."""

    def __init__(self, fn, values: dict):
        self.fn = fn
        self.values = dict(values)
        self.__name__ = getattr(fn, "__name__", "kernel")

    @property
    def jit(self):
        return _jit_of(self.fn)

    @property
    def arg_names(self):
        return self.jit.arg_names

    @property
    def params(self):
        return self.jit.params

    def resolve(self, args, kwargs) -> dict:
        named = _named(self.jit, args, kwargs)
        kw = dict(kwargs)
        for k, f in self.values.items():
            kw[k] = f({**named, **kw})
        return kw

    def __getitem__(self, grid):
        return lambda *args, **kwargs: self.run(*args, grid=grid, **kwargs)

    def run(self, *args, grid, **kwargs):
        return self.fn.run(*args, grid=grid, **self.resolve(args, kwargs))

    def warmup(self, *args, **kwargs):
        return self.fn.warmup(*args, **self.resolve(args, kwargs))

    def explain(self, *args, **kwargs) -> str:
        return self.fn.explain(*args, **self.resolve(args, kwargs))


def heuristics(values: dict[str, Callable]):
    """Computes constexprs from the other arguments before launch."""
    def deco(fn):
        return Heuristics(fn, values)
    return deco
