"""Vector add `out = x + y` (reference: examples/01_vector_add.py:15-30)."""

import numpy as np

import enceladus
import enceladus.language as tl


@enceladus.jit
def add_kernel(x_ptr, y_ptr, out_ptr, n, BLOCK: tl.constexpr):
    pid = tl.program_id(0)
    offs = pid * BLOCK + tl.arange(0, BLOCK)
    mask = offs < n
    x = tl.load(x_ptr + offs, mask=mask)
    y = tl.load(y_ptr + offs, mask=mask)
    tl.store(out_ptr + offs, x + y, mask=mask)


def add(x, y, out=None, block: int = 1024, num_warps: int = 4):
    out = enceladus.new_empty(x) if out is None else out
    n = int(np.prod(x.shape))
    add_kernel[(enceladus.cdiv(n, block),)](x, y, out, n, BLOCK=block, num_warps=num_warps)
    return out
