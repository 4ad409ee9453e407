"""GPU time of the dispatches a piece of host code launches.

Inside `with DispatchTimer() as t:`, every dispatch the runtime launches on this thread
goes through `ek_launch_timed_events`: the first records the timer's start event when it
begins on the GPU and each records the stop event when it ends. `t.ms()` is then the GPU
time from the first dispatch's start to the last one's end, without the host's launch
latency before the first dispatch (the reference times a flushed command buffer's GPU
timestamps the same way: testing.py:14-63, enceladus_rt.mm:626). `t.count` says how many
dispatches were timed; code that launched nothing through this runtime (a torch op) leaves
it at 0, and the caller times it another way.
"""

from __future__ import annotations

import ctypes
import threading

from enceladus_amd.runtime import hip

_tls = threading.local()


def current():
    """The active timer of this thread, or None."""
    return getattr(_tls, "timer", None)


class DispatchTimer:
    def __init__(self):
        self.start, self.stop = ctypes.c_void_p(), ctypes.c_void_p()
        hip.call("ek_event_new", ctypes.byref(self.start))
        hip.call("ek_event_new", ctypes.byref(self.stop))
        self.count = 0

    def __del__(self):
        for e in (getattr(self, "start", None), getattr(self, "stop", None)):
            if e is not None and e.value:
                try:
                    hip.call("ek_event_free", e)
                except Exception:  # noqa: BLE001
                    pass

    def __enter__(self):
        self.count = 0
        self._prev = current()
        _tls.timer = self
        return self

    def __exit__(self, *exc):
        _tls.timer = self._prev
        return False

    def launch(self, stream, fn, grid, block, kernarg, size) -> None:
        """One dispatch with the timer's events (HipError on failure)."""
        hip.call("ek_launch_timed_events", ctypes.c_void_p(stream or None), fn, grid[0],
                 grid[1], grid[2], block, 1, 1, 0, kernarg, size,
                 self.start if self.count == 0 else None, self.stop)
        self.count += 1

    def ms(self) -> float:
        """Milliseconds from the first timed dispatch's start to the last one's end."""
        if not self.count:
            raise RuntimeError("no dispatch was timed")
        out = ctypes.c_float()
        hip.call("ek_event_elapsed_ms", self.start, self.stop, ctypes.byref(out))
        return out.value
