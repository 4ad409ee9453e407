"""Autotune candidate lists for MI355X (the reference's lists: src/enceladus/configs.py:19-127).

Same functions and arguments as the reference (`matmul_configs(dtype)`,
`attention_configs(dtype, head_dim)`, ValueError for an unsupported dtype or head
dimension); the tiles are CDNA4's, not the M4's. `num_warps` counts 64-lane waves.

Matmul (16-bit operands): BM, BN and BK range over {64, 128, 256}, as the north-star sweep
asks, keeping the shapes whose double-buffered LDS stages fit a CU's 160 KB
((BM + BN) * BK * 2 bytes * 2 stages <= 160 KB) and whose fp32 accumulator fits a
wave's 512 registers (BM * BN / (64 * num_warps) <= 256 per lane). 256 x 256 x 64 over 8 waves is the
fastest at 4096^3 (one workgroup per CU, 2 LDS stages); the smaller tiles win on small or
ragged shapes, where 256-wide tiles leave CUs idle. fp32 operands run the 32x32x2 fp32
MFMA: four times the operand bytes per FLOP, so BK stays at 32-64.

Attention: every wave owns 32 whole query rows (`dot_warps=(num_warps, 1)`), so the
softmax row statistics stay inside a wave and P feeds the second dot from registers;
BLOCK_M = 32 * num_warps. BLOCK_N is the key step. fp32 inputs keep BLOCK_N <= 64 (the fp32
operand fragments double the registers of the score tile).
"""

from __future__ import annotations

from typing import Any

import numpy as np

from enceladus_amd.runtime.autotuner import Config

# (BM, BN, BK, num_warps), fastest at 4096^3 first.
_MATMUL_HALF = [
    (256, 256, 64, 8),
    (256, 256, 64, 4),
    (256, 128, 64, 8),
    (128, 256, 64, 8),
    (256, 128, 64, 4),
    (128, 128, 64, 4),
    (128, 128, 128, 4),
    (128, 64, 128, 4),
    (64, 128, 128, 4),
    (64, 64, 128, 4),
    (64, 64, 256, 4),
]
_MATMUL_FP32 = [
    (128, 128, 32, 4),
    (128, 128, 64, 4),
    (256, 128, 32, 8),
    (128, 64, 32, 4),
    (64, 128, 32, 4),
    (64, 64, 64, 4),
]

# (BLOCK_M, BLOCK_N, num_warps)
_ATTENTION = [
    (256, 128, 8),
    (256, 64, 8),
    (128, 128, 4),
    (128, 64, 4),
    (128, 32, 4),
    (64, 64, 2),
    (64, 32, 2),
]
_ATTENTION_FP32 = [
    (128, 64, 4),
    (128, 32, 4),
    (64, 64, 2),
    (64, 32, 2),
]

_FP32_NAMES = ("float32", "fp32", "f32")
_HALF_NAMES = ("float16", "fp16", "f16", "half", "bfloat16", "bf16")


def _dtype_name(dtype: Any) -> str:
    """The bare name of a tl, NumPy or torch dtype, or of a dtype string."""
    if isinstance(dtype, str):
        name = dtype
    elif hasattr(dtype, "long_name"):          # tl dtypes print short names
        name = dtype.long_name
    else:
        try:
            name = np.dtype(dtype).name
        except (TypeError, ValueError):        # torch.float16 prints dotted
            name = str(dtype)
    return name.rsplit(".", 1)[-1]


def matmul_configs(dtype: Any = "float16") -> list[Config]:
    """The matmul candidates for operands of `dtype` (float32, float16 or bfloat16)."""
    name = _dtype_name(dtype)
    if name in _HALF_NAMES:
        shapes = _MATMUL_HALF
    elif name in _FP32_NAMES:
        shapes = _MATMUL_FP32
    else:
        raise ValueError(f"matmul_configs supports float32, float16 and bfloat16, but got "
                         f"{name}. Pass the dtype of the matmul operands.")
    return [Config({"BM": bm, "BN": bn, "BK": bk}, num_warps=nw) for bm, bn, bk, nw in shapes]


def attention_configs(dtype: Any = "float16", head_dim: int = 64) -> list[Config]:
    """The flash-attention candidates (`BLOCK_M`, `BLOCK_N`, `num_warps`, `dot_warps`) for
    q/k/v of `dtype` and head dimension `head_dim` (16, 32, 64 or 128)."""
    name = _dtype_name(dtype)
    if name not in _FP32_NAMES + _HALF_NAMES:
        raise ValueError(f"attention_configs supports float32, float16 and bfloat16, but got "
                         f"{name}. Pass the dtype of q, k and v.")
    if head_dim not in (16, 32, 64, 128):
        raise ValueError(f"attention_configs supports head dimensions 16, 32, 64 and 128, "
                         f"but got {head_dim}")
    shapes = _ATTENTION_FP32 if name in _FP32_NAMES else _ATTENTION
    return [Config({"BLOCK_M": bm, "BLOCK_N": bn}, num_warps=nw, dot_warps=(nw, 1))
            for bm, bn, nw in shapes]
