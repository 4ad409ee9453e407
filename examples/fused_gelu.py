"""Fused `gelu(x * scale + bias)` (reference: examples/05_fused_gelu.py:17-36)."""

import numpy as np

import enceladus
import enceladus.language as tl


@enceladus.jit
def fused_gelu_kernel(x_ptr, bias_ptr, out_ptr, n, n_cols, scale, BLOCK: tl.constexpr):
    pid = tl.program_id(0)
    offs = pid * BLOCK + tl.arange(0, BLOCK)
    mask = offs < n
    x = tl.load(x_ptr + offs, mask=mask).to(tl.float32)
    b = tl.load(bias_ptr + offs % n_cols, mask=mask).to(tl.float32)
    y = x * scale + b
    tl.store(out_ptr + offs, 0.5 * y * (1.0 + tl.erf(y * 0.7071067811865476)), mask=mask)


def fused_gelu(x, bias, scale: float, block: int = 1024):
    out = enceladus.new_empty(x)
    n = int(np.prod(x.shape))
    fused_gelu_kernel[(enceladus.cdiv(n, block),)](x, bias, out, n, x.shape[-1], scale,
                                                   BLOCK=block)
    return out
