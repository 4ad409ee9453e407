"""Benchmark and comparison helpers (reference: src/enceladus/testing.py:14-90).

`do_bench` times a callable on the GPU: it warms up until `warmup_ms` of GPU time has been
spent, then takes `rep` timed samples and returns their median (or the requested
statistic) in ms. `default_tolerance` and `assert_close` give the reference's public
dtype tolerances. (The test suite's own differential table, which is tighter for fp16 and
bf16, lives in `tests/conftest.py`.)
"""

from __future__ import annotations

import ctypes
import statistics

import numpy as np

from enceladus_amd.runtime import device as D
from enceladus_amd.runtime import hip


def default_tolerance(dtype) -> tuple[float, float]:
    """(atol, rtol) suited to comparing results of `dtype` (reference: testing.py:66-75)."""
    name = getattr(dtype, "long_name", None)
    if name is None:
        if hasattr(dtype, "to_numpy"):
            dtype = dtype.to_numpy()
        dt = np.dtype(dtype)
        name = "bfloat16" if dt.kind == "V" and dt.itemsize == 2 else dt.name
    if name == "bfloat16":
        return 2e-2, 2e-2
    if name == "float16":
        return 2e-3, 2e-3
    if name == "float32":
        return 1e-5, 1e-5
    return 0.0, 0.0


def assert_close(actual, expected, atol=None, rtol=None, *, dtype=None):
    """Asserts that two arrays match within tolerances chosen from `actual`'s dtype (or
    `dtype`) unless given (reference: testing.py:80-90)."""
    a = np.asarray(actual)
    e = np.asarray(expected)
    d_atol, d_rtol = default_tolerance(dtype if dtype is not None else a.dtype)
    np.testing.assert_allclose(
        a.astype(np.float64) if a.dtype.kind in "fV" else a,
        e.astype(np.float64) if e.dtype.kind in "fV" else e,
        atol=d_atol if atol is None else atol, rtol=d_rtol if rtol is None else rtol)


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


def do_bench(fn, warmup_ms: float = 50.0, rep: int = 20, return_mode: str = "median", *,
             stream: int | None = None):
    """Times `fn` on the GPU and returns milliseconds (reference: testing.py:14-63).

    Each sample is the GPU time of the dispatches `fn` launches through this runtime, from
    the first one's start to the last one's end (`runtime.timing.DispatchTimer`), so host
    launch latency is excluded; an `fn` that launches nothing through the runtime (a torch
    op) is timed with HIP events around it on `stream` (torch's current stream by
    default). Before sampling, `fn` runs until `warmup_ms` of GPU time has been spent:
    the clock is low after an idle spell, so cold samples run slow.

    Args:
        fn: A function that launches one or more kernels.
        warmup_ms: GPU time to spend warming up before measuring.
        rep: The number of timed repetitions.
        return_mode: "median", "min", "mean", or "all" (a list of every sample).
    """
    from enceladus_amd.runtime.timing import DispatchTimer
    if return_mode not in ("median", "min", "mean", "all"):
        raise ValueError(f"return_mode must be 'median', 'min', 'mean' or 'all', not "
                         f"{return_mode!r}")
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

    spent = 0.0
    while spent < warmup_ms:
        t = sample()
        if t <= 0.0:
            raise RuntimeError("do_bench measured no GPU work; fn must launch kernels on the "
                               "GPU")
        spent += t
    times = [sample() for _ in range(rep)]
    if return_mode == "all":
        return times
    if return_mode == "min":
        return min(times)
    if return_mode == "mean":
        return statistics.fmean(times)
    return statistics.median(times)
