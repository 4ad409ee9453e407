"""Row-wise cumulative sum with `tl.cumsum` (reference: examples/10_cumsum.py:17-42)."""

import numpy as np

import enceladus
import enceladus.language as tl


@enceladus.jit
def cumsum_kernel(out_ptr, in_ptr, n_rows, n_cols, stride_in, stride_out,
                  REVERSE: tl.constexpr, BLOCK_M: tl.constexpr, BLOCK_N: tl.constexpr):
    rows = tl.program_id(0) * BLOCK_M + tl.arange(0, BLOCK_M)
    cols = tl.arange(0, BLOCK_N)
    mask = (rows[:, None] < n_rows) & (cols[None, :] < n_cols)
    x = tl.load(in_ptr + rows[:, None] * stride_in + cols[None, :], mask=mask)
    y = tl.cumsum(x, axis=1, reverse=REVERSE)
    tl.store(out_ptr + rows[:, None] * stride_out + cols[None, :], y, mask=mask)


def cumsum(x, reverse: bool = False, out=None, num_warps: int = 4):
    m, n = x.shape
    dt = enceladus.element_dtype(x)
    if out is None:
        out = enceladus.new_empty(x, dtype=np.int32 if dt.kind in "iub" and dt.itemsize < 4
                                  else dt)
    block_n = enceladus.next_power_of_2(n)
    block_m = max(1, min(16, 4096 // block_n))
    cumsum_kernel[(enceladus.cdiv(m, block_m),)](
        out, x, m, n, enceladus.element_strides(x)[0], enceladus.element_strides(out)[0],
        REVERSE=reverse, BLOCK_M=block_m, BLOCK_N=block_n, num_warps=num_warps)
    return out
