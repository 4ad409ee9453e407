"""Device singleton and capabilities (reference: src/enceladus/runtime/device.py:15-84)."""

from __future__ import annotations

import ctypes
import os
import threading
from dataclasses import dataclass, field

from enceladus_amd.runtime import hip


@dataclass(frozen=True)
class Capabilities:
    """Static facts about the GPU that affect compilation and launch (reference:
    runtime/device.py:15-36, same fields in the same order).

    The reference's Apple-family fields keep their names with the values an AMD GPU has
    (no Apple families, no Metal 3 or 4); the MI355X facts follow as keyword-only fields.
    """

    name: str
    architecture: str
    apple_families: tuple
    metal3: bool
    metal4: bool
    max_threadgroup_memory: int
    max_threads_per_threadgroup: int
    max_buffer_length: int
    recommended_max_working_set: int
    max_concurrent_compilations: int
    compute_units: int = field(default=0, kw_only=True)
    warp_size: int = field(default=64, kw_only=True)
    clock_khz: int = field(default=0, kw_only=True)
    l2_bytes: int = field(default=0, kw_only=True)
    total_mem: int = field(default=0, kw_only=True)

    def supports_apple(self, family: int) -> bool:
        """Whether the device supports `MTLGPUFamilyApple<family>`: never, on AMD."""
        return family in self.apple_families

    @property
    def apple_family(self) -> int:
        return max(self.apple_families, default=0)

    @property
    def arch(self) -> str:
        """The full target name, e.g. `gfx950:sramecc+:xnack-`."""
        return self.architecture

    @property
    def gfx(self) -> str:
        return self.architecture.split(":")[0]

    @property
    def lds_per_block(self) -> int:
        return self.max_threadgroup_memory


class Stream:
    """The stream launches go to: torch's current stream when torch is in use, else the
    null stream (reference: runtime/stream.py:44-124)."""

    def __init__(self, device: "Device"):
        self.device = device

    @property
    def handle(self) -> int:
        return current_stream()

    def synchronize(self) -> None:
        """Waits for the GPU's work and copies back host arrays that asynchronous launches
        wrote."""
        synchronize()


class Device:
    """GPU 0 with its capabilities and stream (reference: runtime/device.py:39-63)."""

    def __init__(self, index: int = 0):
        from enceladus_amd.compiler.errors import HipError
        if hip.device_count() == 0:
            raise HipError("no HIP device is visible; the MI355X backend has no CPU fallback")
        info = hip.device_info(index)
        self.index = index
        self.caps = Capabilities(
            info.name.decode(), info.arch.decode(), (), False, False, info.lds_per_block,
            info.max_threads_per_block, info.total_mem, info.total_mem,
            min(8, os.cpu_count() or 1), compute_units=info.compute_units,
            warp_size=info.warp_size, clock_khz=info.clock_khz, l2_bytes=info.l2_bytes,
            total_mem=info.total_mem)
        self.stream = Stream(self)

    def __repr__(self) -> str:
        return f"<enceladus.Device {self.caps.name} ({self.caps.architecture})>"


_dev = None
_lock = threading.Lock()


def get_device() -> Device:
    """The process-wide default device (GPU 0), created on first use; raises HipError
    when no GPU is visible."""
    global _dev
    if _dev is None:
        with _lock:
            if _dev is None:
                _dev = Device(0)
    return _dev


def has_gpu() -> bool:
    try:
        return hip.device_count() > 0
    except Exception:  # noqa: BLE001
        return False


def synchronize() -> None:
    """Waits for all GPU work, then copies back host arrays that asynchronous launches
    wrote (`enceladus.async_numpy`)."""
    hip.call("ek_device_sync")
    from enceladus_amd.runtime import tensor
    tensor.flush_pending()


_raw_stream = None


def current_stream() -> int:
    """The HIP stream launches go to: torch's current stream when torch is in use."""
    global _raw_stream
    import sys
    torch = sys.modules.get("torch")
    if torch is not None:
        try:
            if torch.cuda.is_initialized():
                if _raw_stream is None:
                    # torch's raw-handle accessor skips building a Stream object
                    _raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", False)
                if _raw_stream:
                    return int(_raw_stream(torch.cuda.current_device()))
                return int(torch.cuda.current_stream().cuda_stream)
        except Exception:  # noqa: BLE001
            pass
    return 0


__all__ = ["Capabilities", "Device", "Stream", "get_device", "has_gpu", "synchronize",
           "current_stream"]
