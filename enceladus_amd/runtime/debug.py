"""`enceladus.capture`: a dispatch trace of the GPU work inside a block.

The reference records a Metal `.gputrace` document for Xcode (runtime/debug.py:14-90).
On MI355X the counterpart is a trace of every kernel this runtime launches inside the
block: two HIP events around each dispatch on its stream give its start and duration,
and the trace is written as Chrome trace-event JSON (load it in Perfetto or
chrome://tracing) with the kernel name, grid, workgroup size and LDS bytes of each
dispatch. Hardware counters stay with `rocprofv3`, which needs no cooperation from the
program.
"""

from __future__ import annotations

import contextlib
import ctypes
import json
import os
from typing import Iterator

from enceladus_amd.runtime import hip

_active: list | None = None


def capture_active() -> bool:
    """Whether `enceladus.capture` is recording."""
    return _active is not None


def _event():
    e = ctypes.c_void_p()
    hip.call("ek_event_new", ctypes.byref(e))
    return e


def before_launch(stream: int):
    """Called by launchers while a capture runs: records the start event."""
    e = _event()
    hip.call("ek_event_record", e, ctypes.c_void_p(stream or None))
    return e


def after_launch(start, stream: int, name: str, grid, block: int, lds: int) -> None:
    e = _event()
    hip.call("ek_event_record", e, ctypes.c_void_p(stream or None))
    _active.append((start, e, name, tuple(grid), block, lds, stream))


@contextlib.contextmanager
def capture(path: str | os.PathLike) -> Iterator[str]:
    """Records every kernel launched inside the block into a dispatch trace.

    Example:

        with enceladus.capture("add.trace.json"):
            add_kernel[grid](x, y, out, n, BLOCK=1024)

    Args:
        path: where to write the trace; it must end in `.json` and must not exist.

    Yields:
        The trace path as a string.

    Raises:
        RuntimeError: a capture is already running.
        FileExistsError: `path` already exists.
        ValueError: `path` doesn't end in `.json`.
    """
    global _active
    path = os.fspath(path)
    if not path.endswith(".json"):
        raise ValueError(f"the trace path must end in .json (Chrome trace events), got {path!r}")
    if os.path.exists(path):
        raise FileExistsError(path)
    if _active is not None:
        raise RuntimeError("a capture is already running")
    _active = []
    origin = _event()
    hip.call("ek_event_record", origin, None)
    try:
        yield path
    finally:
        recs, _active = _active, None
        hip.call("ek_device_sync")
        events = []
        ms = ctypes.c_float()
        for start, end, name, grid, block, lds, stream in recs:
            hip.call("ek_event_elapsed_ms", origin, start, ctypes.byref(ms))
            t0 = ms.value * 1e3
            hip.call("ek_event_elapsed_ms", start, end, ctypes.byref(ms))
            events.append({"name": name, "ph": "X", "ts": round(t0, 3),
                           "dur": round(ms.value * 1e3, 3), "pid": 0,
                           "tid": f"stream {stream:#x}" if stream else "null stream",
                           "args": {"grid": list(grid), "workgroup": block, "lds_bytes": lds}})
            hip.call("ek_event_free", start)
            hip.call("ek_event_free", end)
        hip.call("ek_event_free", origin)
        with open(path, "x") as f:
            json.dump({"traceEvents": events, "displayTimeUnit": "ns"}, f, indent=1)


def lazy_mlx(enabled: bool = True) -> None:
    """MLX arrays exist only on Apple silicon (reference: runtime/mlx_lazy.py:61): on
    MI355X the lazy path has nothing to join. `lazy_mlx(False)` is accepted."""
    if enabled:
        raise NotImplementedError("MLX doesn't run on MI355X; pass torch-ROCm tensors, "
                                  "enceladus.Tensor or NumPy arrays (see enceladus.async_numpy)")
