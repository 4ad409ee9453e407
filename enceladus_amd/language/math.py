"""`tl.math`: the math builtins (reference: src/enceladus/language/math.py:30-55)."""

from enceladus_amd.language.ops import (  # noqa: F401
    ceil, cos, erf, exp, exp2, floor, log, log2, rsqrt, sigmoid, sin, sqrt, tanh,
)
