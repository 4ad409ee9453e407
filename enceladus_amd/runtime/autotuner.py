"""`@autotune`, `Config` and `heuristics` (reference: src/enceladus/runtime/autotuner.py:54-585).

On the first launch for a key, every config is compiled (in a thread pool: hiprtc
programs are per-call objects), timed with HIP events on the launch stream, and the
fastest one (the earliest config within `tolerance` of the best) is cached in memory and
in `$ENCELADUS_CACHE_DIR/autotune/<kernel>.json`. Configs that fail to compile or run are
skipped.
"""

from __future__ import annotations

import hashlib
import json
import logging
import os
from concurrent.futures import ThreadPoolExecutor
from typing import Any, Callable

log = logging.getLogger("enceladus.autotune")


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


class Autotuner:
    def __init__(self, fn, configs, key, prune_configs_by=None, reset_to_zero=None,
                 restore_value=None, warmup_ms=50, rep=20, tolerance=0.01):
        self.fn = fn
        self.configs = list(configs)
        self.key = list(key)
        self.prune = (prune_configs_by or {}).get("early_config_prune")
        self.reset_to_zero = list(reset_to_zero or [])
        self.restore_value = list(restore_value or [])
        self.warmup_ms = warmup_ms
        self.rep = rep
        self.tolerance = tolerance
        self.cache: dict[Any, Config] = {}
        self.__name__ = getattr(fn, "__name__", "kernel")
        self._ek_jit = False
        self._loaded = False

    def __getitem__(self, grid):
        return lambda *args, **kwargs: self.run(*args, grid=grid, **kwargs)

    def _named(self, args, kwargs) -> dict:
        names = self.fn.arg_names
        named = dict(zip(names, args))
        named.update(kwargs)
        return named

    def _key_of(self, named) -> tuple:
        from enceladus_amd.runtime import tensor as T
        parts = []
        for k in self.key:
            v = named[k]
            parts.append(tuple(v.shape) if hasattr(v, "shape") else v)
        for v in named.values():
            if T.is_array_like(v):
                parts.append(str(T.elem_dtype(v)))
        return tuple(parts)

    def _path(self):
        from enceladus_amd.runtime.compile import cache_dir
        import inspect
        src = inspect.getsource(self.fn.fn)
        h = hashlib.sha256(src.encode()).hexdigest()[:16]
        return cache_dir() / "autotune" / f"{self.__name__}-{h}.json"

    def _load(self):
        if self._loaded:
            return
        self._loaded = True
        try:
            data = json.loads(self._path().read_text())
        except (OSError, ValueError):
            return
        for k, c in data.items():
            cfg = Config(c["kwargs"], c["num_warps"], dot_warps=c.get("dot_warps"))
            self.cache[k] = cfg

    def _save(self, skey, cfg: Config):
        p = self._path()
        try:
            p.parent.mkdir(parents=True, exist_ok=True)
            data = {}
            if p.exists():
                data = json.loads(p.read_text())
            data[skey] = {"kwargs": cfg.kwargs, "num_warps": cfg.num_warps,
                          "dot_warps": list(cfg.dot_warps) if cfg.dot_warps else None}
            tmp = p.with_suffix(f".tmp{os.getpid()}")
            tmp.write_text(json.dumps(data, indent=1, sort_keys=True))
            os.replace(tmp, p)
        except (OSError, ValueError):
            pass

    def prune_configs(self, named) -> list[Config]:
        cfgs = self.configs
        if self.prune is not None:
            cfgs = self.prune(cfgs, named)
        return cfgs

    def run(self, *args, grid, **kwargs):
        named = self._named(args, kwargs)
        key = self._key_of(named)
        skey = repr(key)
        self._load()
        cfg = self.cache.get(skey)
        if cfg is None:
            cfg = self._tune(args, kwargs, grid, named)
            self.cache[skey] = cfg
            self._save(skey, cfg)
        if os.environ.get("ENCELADUS_PRINT_AUTOTUNING") == "1":
            print(f"autotune {self.__name__} {key}: {cfg}")
        if cfg.pre_hook:
            cfg.pre_hook(named)
        return self.fn.run(*args, grid=grid, **cfg.kwargs, **cfg.launch_options(), **kwargs)

    def _tune(self, args, kwargs, grid, named) -> Config:
        from enceladus_amd.testing import do_bench
        cfgs = self.prune_configs(named)
        if not cfgs:
            raise ValueError(f"no autotune configs left for {self.__name__}")

        def compile_one(c):
            try:
                self.fn.warmup(*args, **c.kwargs, **c.launch_options(), **kwargs)
                return c
            except Exception as e:  # noqa: BLE001
                log.debug("config %s failed to compile: %s", c, e)
                return None
        with ThreadPoolExecutor(max_workers=min(8, len(cfgs))) as ex:
            ok = [c for c in ex.map(compile_one, cfgs) if c is not None]
        timings = []
        for c in ok:
            def call(c=c):
                self.fn.run(*args, grid=grid, **c.kwargs, **c.launch_options(), **kwargs)
            try:
                t = do_bench(call, warmup=self.warmup_ms, rep=self.rep)
            except Exception as e:  # noqa: BLE001
                log.debug("config %s failed to run: %s", c, e)
                continue
            timings.append((t, c))
        if not timings:
            raise RuntimeError(f"every autotune config of {self.__name__} failed")
        best = min(t for t, _ in timings)
        for t, c in timings:
            if t <= best * (1 + self.tolerance):
                return c
        return timings[0][1]


def autotune(configs, key, prune_configs_by=None, reset_to_zero=None, restore_value=None,
             warmup_ms=50, rep=20, tolerance=0.01):
    def deco(fn):
        return Autotuner(fn, configs, key, prune_configs_by, reset_to_zero, restore_value,
                         warmup_ms, rep, tolerance)
    return deco


def heuristics(values: dict[str, Callable]):
    """Computes constexprs from the other arguments before launch."""
    def deco(fn):
        class _H:
            def __init__(self):
                self.fn = fn
                self.__name__ = getattr(fn, "__name__", "kernel")

            def __getitem__(self, grid):
                def launch(*args, **kwargs):
                    named = dict(zip(fn.arg_names, args))
                    named.update(kwargs)
                    for k, f in values.items():
                        kwargs[k] = f(named)
                    return fn.run(*args, grid=grid, **kwargs)
                return launch

            @property
            def arg_names(self):
                return fn.arg_names
        return _H()
    return deco
