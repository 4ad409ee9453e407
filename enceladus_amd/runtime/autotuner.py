"""`@autotune`, `Config` and `heuristics` (reference: src/enceladus/runtime/autotuner.py:54-585).

On the first launch for a key, every candidate config is compiled (in a thread pool:
hiprtc programs are per-call objects) and timed with HIP events on the launch stream:
phase 1 times each config, phase 2 times the few fastest again in interleaved rounds, and
the earliest finalist within `tolerance` of the fastest wins (the reference's rule). Each
sample is the GPU time of the launch's dispatches alone (`testing.do_bench`). The winner is
kept in memory and appended to the kernel's tuning log (`TuneLog`,
`$ENCELADUS_CACHE_DIR/autotune/<kernel>-<source and compiler hash>/<arch>.jsonl`); a logged
winner that is no longer a candidate is re-tuned, and a compiler change starts a new log.
One method, `_resolve`, decides every launch's config (memory, then the log, then tuning or,
for `warmup`/`explain`, the first candidate). Arguments in
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


DOT_BACKENDS = ("auto", "simdgroup", "mpp")


class Config:
    """One candidate configuration: constexpr values plus launch options (reference:
    runtime/autotuner.py:54-103, same fields in the same positional order).

    Args:
        kwargs: Constexpr values, for example `{"BM": 64, "BN": 64, "BK": 32}`.
        num_warps: Waves (64 lanes each) per program.
        dot_warps: The (WM, WN) grid of waves for `tl.dot`, or None for the default.
        dot_backend: "auto", "simdgroup" or "mpp"; checked, and every `tl.dot` lowers to
            MFMA on MI355X whichever is named.
        pre_hook: Called with the bound arguments before each launch of this config.
    """

    def __init__(self, kwargs: dict, num_warps: int = 4, dot_warps=None,
                 dot_backend: str = "auto", pre_hook: Callable | None = None):
        if dot_backend not in DOT_BACKENDS:
            raise ValueError(f"dot_backend must be 'auto', 'simdgroup', or 'mpp', not "
                             f"{dot_backend!r}")
        self.kwargs = dict(kwargs)
        self.num_warps = num_warps
        self.dot_warps = tuple(dot_warps) if dot_warps is not None else None
        self.dot_backend = dot_backend
        self.pre_hook = pre_hook

    def _key(self):
        return (tuple(sorted(self.kwargs.items())), self.num_warps, self.dot_warps,
                self.dot_backend)

    def __eq__(self, other):
        return isinstance(other, Config) and self._key() == other._key()

    def __hash__(self):
        return hash(self._key())

    def __repr__(self):
        kw = ", ".join(f"{k}={v}" for k, v in self.kwargs.items())
        tail = f", dot_backend={self.dot_backend!r}" if self.dot_backend != "auto" else ""
        return f"Config({kw}, num_warps={self.num_warps}, dot_warps={self.dot_warps}{tail})"

    def __str__(self):
        parts = [repr(self.kwargs), f"num_warps={self.num_warps}"]
        if self.dot_warps is not None:
            parts.append(f"dot_warps={self.dot_warps}")
        if self.dot_backend != "auto":
            parts.append(f"dot_backend={self.dot_backend!r}")
        return f"enceladus.Config({', '.join(parts)})"

    def launch_options(self) -> dict:
        out = {"num_warps": self.num_warps}
        if self.dot_warps is not None:
            out["dot_warps"] = self.dot_warps
        if self.dot_backend != "auto":
            out["dot_backend"] = self.dot_backend
        return out

    def to_json(self) -> dict:
        """The fields that identify this config (`pre_hook` cannot be serialised)."""
        return {"kwargs": self.kwargs, "num_warps": self.num_warps,
                "dot_warps": list(self.dot_warps) if self.dot_warps else None,
                "dot_backend": self.dot_backend}

    @classmethod
    def from_json(cls, d: dict) -> "Config":
        dw = d.get("dot_warps")
        return cls(dict(d["kwargs"]), int(d["num_warps"]), tuple(dw) if dw else None,
                   d.get("dot_backend", "auto"))


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
    """Changes whenever any Python source of the package, the device headers or the HIP
    runtime change (`speccache.compiler_hash`)."""
    from enceladus_amd.runtime.speccache import compiler_hash
    return compiler_hash()


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


class TuneLog:
    """The tuning results of one kernel source under one compiler, on disk.

    One JSON object per line, appended as results are found: `{"key", "config",
    "timings_ms"}`; a later line for a key supersedes an earlier one. Lines go out with one
    `write` on a descriptor opened for appending, under an exclusive `flock`, so processes
    tuning the same kernel at once interleave whole lines. A compiler change writes a new
    file (the compiler hash is in the path); a line that does not parse is skipped.
    """

    def __init__(self, path):
        self.path = path
        self._records: dict | None = None

    def _read(self) -> dict:
        if self._records is None:
            self._records = {}
            if os.environ.get("ENCELADUS_ALWAYS_COMPILE") != "1":
                try:
                    text = self.path.read_text()
                except OSError:
                    text = ""
                for line in text.splitlines():
                    with contextlib.suppress(ValueError, KeyError, TypeError):
                        rec = json.loads(line)
                        self._records[rec["key"]] = Config.from_json(rec["config"])
        return self._records

    def get(self, key: str):
        return self._read().get(key)

    def put(self, key: str, cfg: "Config", timings: dict) -> None:
        self._read()[key] = cfg
        line = json.dumps({"key": key, "config": cfg.to_json(),
                           "timings_ms": timings}, sort_keys=True) + "\n"
        try:
            import fcntl
            self.path.parent.mkdir(parents=True, exist_ok=True)
            fd = os.open(self.path, os.O_WRONLY | os.O_APPEND | os.O_CREAT, 0o644)
            try:
                fcntl.flock(fd, fcntl.LOCK_EX)
                os.write(fd, line.encode())
            finally:
                os.close(fd)
        except OSError as e:
            log.debug("couldn't record the tuning result: %s", e)

    def entries(self) -> dict:
        return dict(self._read())


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
        self._log: TuneLog | None = None
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

    # -- keys and the tuning log ---------------------------------------------------
    def _key(self, named: dict) -> str:
        from enceladus_amd.runtime import tensor as T
        parts = [_key_value(named.get(k)) for k in self.key]
        dts = [T.elem_dtype(named[n]).name for n in self.arg_names
               if n in named and T.is_array_like(named[n])]
        return "|".join(parts) + "|" + ",".join(dts)

    def log_path(self):
        """`$ENCELADUS_CACHE_DIR/autotune/<kernel>-<hash of its source and the compiler>/
        <arch>.jsonl`."""
        from enceladus_amd.runtime.compile import ARCH, cache_dir
        src = inspect.getsource(_jit_of(self.fn).fn)
        h = hashlib.sha256((src + _compiler_hash()).encode()).hexdigest()[:24]
        return cache_dir() / "autotune" / f"{self.__name__}-{h}" / f"{ARCH}.jsonl"

    @property
    def tune_log(self) -> TuneLog:
        path = self.log_path()
        if self._log is None or self._log.path != path:
            self._log = TuneLog(path)
        return self._log

    def _resolve(self, named: dict, tune):
        """The config for this launch: tuned in this process, recorded in the tuning log
        (when it is still a candidate), tuned now when `tune` is a callable that tunes,
        or else the first candidate."""
        key = self._key(named)
        cfg = self.best.get(key)
        if cfg is not None:
            return cfg
        with self._lock:
            cfg = self.best.get(key)
            if cfg is None:
                logged = self.tune_log.get(key)
                if logged is not None:
                    cfg = next((c for c in self._candidates(named) if c == logged), None)
            if cfg is None and tune is not None:
                cfg = tune(key)
            if cfg is not None:
                self.best[key] = cfg
        return cfg if cfg is not None else self._candidates(named)[0]

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

    def warmup(self, *args, **kwargs):
        """Compiles (never benchmarks) with the tuned or logged config, or the first
        candidate."""
        cfg = self._resolve(_named(self.fn, args, kwargs), None)
        return self.fn.warmup(*args, **kwargs, **cfg.kwargs, **cfg.launch_options())

    def explain(self, *args, **kwargs) -> str:
        cfg = self._resolve(_named(self.fn, args, kwargs), None)
        return self.fn.explain(*args, **kwargs, **cfg.kwargs, **cfg.launch_options())

    # -- launching and tuning ------------------------------------------------------
    def run(self, *args, grid, **kwargs):
        named = _named(self.fn, args, kwargs)
        cfg = self._resolve(named, lambda key: self._tune(key, args, kwargs, grid, named))
        if os.environ.get("ENCELADUS_PRINT_AUTOTUNING", "0") not in ("", "0"):
            print(f"autotune {self.__name__} [{self._key(named)}]: {cfg}")
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
                return do_bench(lambda: launch(cfgs[i]), warmup_ms=warmup_ms, rep=rep,
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
        self.timings[key] = {repr(cfgs[i]): t for i, t in timings.items()}
        self.tune_log.put(key, best, self.timings[key])
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
