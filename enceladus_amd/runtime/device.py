"""Device singleton and capabilities (reference: src/enceladus/runtime/device.py:15-84)."""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

from enceladus_amd.runtime import hip


@dataclass(frozen=True)
class Capabilities:
    name: str
    arch: str
    compute_units: int
    warp_size: int
    max_threads_per_block: int
    lds_per_block: int
    total_mem: int
    clock_khz: int
    l2_bytes: int

    @property
    def gfx(self) -> str:
        return self.arch.split(":")[0]


_dev = None


def get_device() -> Capabilities:
    """Returns the capabilities of GPU 0; raises HipError when no GPU is visible."""
    global _dev
    if _dev is None:
        n = hip.device_count()
        if n == 0:
            from enceladus_amd.compiler.errors import HipError
            raise HipError("no HIP device is visible; the MI355X backend has no CPU fallback")
        info = hip.device_info(0)
        _dev = Capabilities(info.name.decode(), info.arch.decode(), info.compute_units,
                            info.warp_size, info.max_threads_per_block, info.lds_per_block,
                            info.total_mem, info.clock_khz, info.l2_bytes)
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


__all__ = ["Capabilities", "get_device", "has_gpu", "synchronize", "current_stream", "ctypes"]
