"""Element types, `constexpr`, and the kernel-side value wrapper.

The dtype table mirrors the reference language's twelve types
(reference: src/enceladus/language/core.py:45-117). NumPy has no bfloat16 without
`ml_dtypes`, so host-side bfloat16 arrays are carried as `uint16` bit patterns (or as
torch tensors); `dtype.to_numpy()` reports `uint16` storage for `bfloat16`, and
`BF16_TAG` (a 2-byte void dtype of kind "V", the kind ml_dtypes' bfloat16 reports) is the
NumPy-side name of the element type (`enceladus.element_dtype`).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import numpy as np


@dataclass(frozen=True, eq=False)
class dtype:  # noqa: N801 - Triton spelling
    """A tile element type such as `tl.float32`.

    Attributes:
        name: short name (`fp32`, `bf16`, `i32`, ...).
        kind: `bool`, `int`, `uint` or `float`.
        primitive_bitwidth: width in bits (`int1` reports 1).
        ir_name: IR scalar name (`f32`, `i32`, ...).
        long_name: `float32`, `int32`, ...
        cname: the HIP C++ spelling used by the emitter.
    """

    name: str
    kind: str
    primitive_bitwidth: int
    ir_name: str
    long_name: str
    cname: str

    @property
    def itemsize(self) -> int:
        return max(1, self.primitive_bitwidth // 8)

    def is_floating(self) -> bool:
        return self.kind == "float"

    def is_int(self) -> bool:
        return self.kind in ("int", "uint", "bool")

    def is_bool(self) -> bool:
        return self.kind == "bool"

    def is_signed(self) -> bool:
        return self.kind in ("int", "float")

    def is_unsigned(self) -> bool:
        return self.kind in ("uint", "bool")

    def is_half(self) -> bool:
        return self.kind == "float" and self.primitive_bitwidth == 16

    @property
    def element_ty(self) -> "dtype":
        return self

    def to_numpy(self) -> np.dtype:
        return _NUMPY[self.name]

    def __repr__(self) -> str:
        return f"tl.{self.long_name}"

    __str__ = __repr__

    def __reduce__(self):
        return (dtype_from_name, (self.name,))


int1 = dtype("i1", "bool", 1, "i1", "int1", "bool")
int8 = dtype("i8", "int", 8, "i8", "int8", "int8_t")
int16 = dtype("i16", "int", 16, "i16", "int16", "int16_t")
int32 = dtype("i32", "int", 32, "i32", "int32", "int32_t")
int64 = dtype("i64", "int", 64, "i64", "int64", "int64_t")
uint8 = dtype("u8", "uint", 8, "u8", "uint8", "uint8_t")
uint16 = dtype("u16", "uint", 16, "u16", "uint16", "uint16_t")
uint32 = dtype("u32", "uint", 32, "u32", "uint32", "uint32_t")
uint64 = dtype("u64", "uint", 64, "u64", "uint64", "uint64_t")
float16 = dtype("fp16", "float", 16, "f16", "float16", "_Float16")
bfloat16 = dtype("bf16", "float", 16, "bf16", "bfloat16", "ek::bf16")
float32 = dtype("fp32", "float", 32, "f32", "float32", "float")

ALL_DTYPES: tuple[dtype, ...] = (
    int1, int8, int16, int32, int64, uint8, uint16, uint32, uint64, float16, bfloat16, float32,
)

_NUMPY = {
    "i1": np.dtype(np.bool_), "i8": np.dtype(np.int8), "i16": np.dtype(np.int16),
    "i32": np.dtype(np.int32), "i64": np.dtype(np.int64), "u8": np.dtype(np.uint8),
    "u16": np.dtype(np.uint16), "u32": np.dtype(np.uint32), "u64": np.dtype(np.uint64),
    "fp16": np.dtype(np.float16), "bf16": np.dtype(np.uint16), "fp32": np.dtype(np.float32),
}
_FROM_NUMPY = {v: k for k, v in _NUMPY.items() if k != "bf16"}
# The NumPy-side name of bfloat16 (kind "V", itemsize 2, tagged by its metadata).
BF16_TAG = np.dtype("V2", metadata={"enceladus_dtype": "bfloat16"})
_BY_NAME: dict[str, dtype] = {}
for _d in ALL_DTYPES:
    _BY_NAME[_d.name] = _d
    _BY_NAME[_d.ir_name] = _d
    _BY_NAME[_d.long_name] = _d
_BY_NAME["bool"] = int1


def dtype_from_numpy(np_dtype: Any) -> dtype:
    d = np.dtype(np_dtype)
    if (d.metadata or {}).get("enceladus_dtype") == "bfloat16":
        return bfloat16
    name = _FROM_NUMPY.get(d) if d.kind != "V" else None
    if name is not None:
        return _BY_NAME[name]
    if d == np.float64:
        raise TypeError("Enceladus has no float64 type. Cast the array to float32 first "
                        "(for example `x.astype(np.float32)`, or `x.float()` for torch).")
    raise TypeError(f"NumPy dtype {d} has no Enceladus equivalent.")


def dtype_from_name(name: str) -> dtype:
    try:
        return _BY_NAME[name]
    except KeyError:
        raise KeyError(f"unknown dtype name {name!r}") from None


def dtype_from_torch(tdt: Any) -> dtype:
    """Maps a torch dtype (by its string form) to a tile dtype."""
    s = str(tdt).removeprefix("torch.")
    table = {"float32": float32, "float16": float16, "bfloat16": bfloat16, "int32": int32,
             "int64": int64, "int16": int16, "int8": int8, "uint8": uint8, "bool": int1,
             "uint16": uint16, "uint32": uint32, "uint64": uint64, "half": float16,
             "float": float32, "int": int32, "long": int64}
    if s not in table:
        raise TypeError(f"torch dtype {tdt} has no Enceladus equivalent")
    return table[s]


class constexpr:  # noqa: N801 - Triton spelling
    """Marks a parameter as compile-time (`BLOCK: tl.constexpr`) or wraps a constant.

    Reference: src/enceladus/language/core.py:193.
    """

    def __init__(self, value: Any = None):
        self.value = value.value if isinstance(value, constexpr) else value

    def __repr__(self) -> str:
        return f"constexpr({self.value!r})"

    def __bool__(self):
        return bool(self.value)

    def __index__(self):
        return int(self.value)

    def __int__(self):
        return int(self.value)

    def __float__(self):
        return float(self.value)

    def __hash__(self):
        return hash(self.value)

    def __eq__(self, other):
        return self.value == unwrap(other)


def unwrap(x: Any) -> Any:
    return x.value if isinstance(x, constexpr) else x


def is_constexpr_annotation(ann: Any) -> bool:
    if ann is constexpr:
        return True
    if isinstance(ann, str):
        return ann.split(".")[-1] == "constexpr"
    return False
