"""Enceladus tile language on AMD Instinct MI355X (gfx950).

The user surface matches the reference (`@jit`, `kernel[grid](...)`, `tl.*`, constexpr,
autotune, NumPy/torch interop); kernels compile to HIP C++ via hiprtc and launch through
the C-ABI shim `libenceladus_hip.so`. Reference public names: src/enceladus/__init__.py:12-61.
"""

__version__ = "0.1.0"

from enceladus_amd import language  # noqa: F401
from enceladus_amd.compiler.errors import (  # noqa: F401
    CompilationError, DeviceAssertionError, HipError,
)
from enceladus_amd.language.core import constexpr  # noqa: F401
from enceladus_amd.runtime.debug import capture, lazy_mlx  # noqa: F401
from enceladus_amd.runtime.device import Capabilities, get_device, synchronize  # noqa: F401
from enceladus_amd.runtime.jit import JITFunction, cdiv, jit, next_power_of_2  # noqa: F401
from enceladus_amd.runtime.raw import hip_kernel, metal_kernel  # noqa: F401
from enceladus_amd.runtime.tensor import (  # noqa: F401
    Tensor, arange, async_numpy, element_dtype, element_strides, empty, empty_like, from_numpy,
    full, new_empty, new_zeros, ones, rand, randn, zeros, zeros_like,
)

MetalError = HipError  # the reference's runtime error name, kept for drop-in code

_LAZY = ("configs", "testing", "autotune", "Config", "heuristics")


def __getattr__(name):
    if name in ("configs", "testing"):
        import importlib
        return importlib.import_module(f"enceladus_amd.{name}")
    if name in ("autotune", "Config", "heuristics"):
        from enceladus_amd.runtime import autotuner
        return getattr(autotuner, name)
    raise AttributeError(f"module 'enceladus' has no attribute {name!r}")
