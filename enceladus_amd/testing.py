"""Benchmark and comparison helpers (reference: src/enceladus/testing.py:14-90).

`do_bench` times a callable with HIP events recorded on the launch stream: warm up for
`warmup` ms, then `rep` timed repetitions; returns the median (or the requested
statistic) in ms.
"""

from __future__ import annotations

import ctypes
import statistics

import numpy as np

from enceladus_amd.runtime import device as D
from enceladus_amd.runtime import hip

_TOL = {"float32": (1e-5, 1e-5), "float16": (1e-3, 2e-3), "bfloat16": (1e-2, 1.6e-2)}


def default_tolerance(dtype) -> tuple[float, float]:
    name = getattr(dtype, "long_name", None) or np.dtype(dtype).name
    return _TOL.get(name, (0.0, 0.0))


def assert_close(actual, expected, atol=None, rtol=None, dtype=None):
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    if atol is None or rtol is None:
        ta, tr = default_tolerance(dtype or np.asarray(expected).dtype)
        atol = ta if atol is None else atol
        rtol = tr if rtol is None else rtol
    np.testing.assert_allclose(a, e, atol=atol, rtol=rtol)


class _Events:
    def __init__(self):
        self.a, self.b = ctypes.c_void_p(), ctypes.c_void_p()
        hip.call("ek_event_new", ctypes.byref(self.a))
        hip.call("ek_event_new", ctypes.byref(self.b))

    def __del__(self):
        try:
            hip.call("ek_event_free", self.a)
            hip.call("ek_event_free", self.b)
        except Exception:  # noqa: BLE001
            pass

    def time(self, fn, stream) -> float:
        s = ctypes.c_void_p(stream or None)
        hip.call("ek_event_record", self.a, s)
        fn()
        hip.call("ek_event_record", self.b, s)
        ms = ctypes.c_float()
        hip.call("ek_event_elapsed_ms", self.a, self.b, ctypes.byref(ms))
        return ms.value


def do_bench(fn, warmup: float = 50, rep: int = 20, return_mode: str = "median",
             stream: int | None = None):
    """Times `fn` on the GPU in ms. Each sample is the GPU time of the dispatches `fn`
    launches through this runtime, from the first one's start to the last one's end
    (`runtime.timing.DispatchTimer`), so host launch latency is excluded; an `fn` that
    launches nothing through the runtime (a torch op) is timed with events around it."""
    from enceladus_amd.runtime.timing import DispatchTimer
    fn()
    D.synchronize()
    ev = _Events()
    timer = DispatchTimer()
    s = D.current_stream() if stream is None else stream

    def sample():
        with timer:
            fn()
        if timer.count:
            return timer.ms()
        return ev.time(fn, s)

    first = sample()
    n_warm = max(1, int(warmup / max(first, 1e-3)))
    for _ in range(min(n_warm, 1000)):
        fn()
    D.synchronize()
    times = [sample() for _ in range(rep)]
    if return_mode == "all":
        return times
    if return_mode == "min":
        return min(times)
    if return_mode == "mean":
        return statistics.fmean(times)
    return statistics.median(times)
