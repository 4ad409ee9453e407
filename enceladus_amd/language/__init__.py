"""The tile language, conventionally imported as `import enceladus.language as tl`.

Names follow the reference surface (reference: src/enceladus/language/__init__.py:21-102).
"""

from enceladus_amd.compiler.errors import CompilationError
from enceladus_amd.language import math  # noqa: F401
from enceladus_amd.language.core import (  # noqa: F401
    bfloat16, constexpr, dtype, float16, float32, int1, int8, int16, int32, int64, uint8,
    uint16, uint32, uint64,
)
from enceladus_amd.language.ops import (  # noqa: F401
    arange, argmax, argmin, associative_scan, atomic_add, atomic_and, atomic_cas, atomic_max, atomic_min,
    atomic_or, atomic_xchg, atomic_xor, broadcast_to, cast, cdiv, ceil, clamp, cos, cumsum,
    debug_barrier, device_assert, device_print, dot, erf, exp, exp2, expand_dims, floor, fma,
    full, full_like, join, load, log, log2, make_tensor_descriptor, max_contiguous, maximum,
    minimum, multiple_of, num_programs, permute, program_id, reshape, rsqrt, sigmoid, sin,
    split, sqrt, static_assert, static_print, static_range, store, tanh, trans, where, zeros,
    zeros_like,
)
from enceladus_amd.language.ops import abs_ as abs  # noqa: F401
from enceladus_amd.language.ops import max_ as max  # noqa: F401
from enceladus_amd.language.ops import min_ as min  # noqa: F401
from enceladus_amd.language.ops import range  # noqa: F401
from enceladus_amd.language.ops import reduce_ as reduce  # noqa: F401
from enceladus_amd.language.ops import sum_ as sum  # noqa: F401


class _MissingNameError(CompilationError, AttributeError):
    """A missing `tl` name: a `CompilationError` in a kernel that `hasattr` still handles
    (reference: language/__init__.py:100-115)."""


def __getattr__(name: str):
    if name.startswith("__"):
        raise AttributeError(name)
    if name in ("float64", "double", "fp64"):
        raise _MissingNameError("Enceladus has no float64 type. Use tl.float32 instead.")
    raise _MissingNameError(f"module `enceladus.language` has no attribute `{name}`. Check "
                            "the spelling; some Triton functions don't exist in Enceladus.")
