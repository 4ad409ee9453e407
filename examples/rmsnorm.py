"""RMSNorm forward, one program per row (reference: examples/06_rmsnorm.py:15-37)."""

import enceladus
import enceladus.language as tl


@enceladus.jit
def rmsnorm_kernel(x_ptr, w_ptr, out_ptr, stride_x, stride_out, n_cols, eps,
                   BLOCK: tl.constexpr):
    row = tl.program_id(0)
    cols = tl.arange(0, BLOCK)
    mask = cols < n_cols
    x = tl.load(x_ptr + row * stride_x + cols, mask=mask, other=0.0).to(tl.float32)
    rstd = tl.rsqrt(tl.sum(x * x, axis=0) / n_cols + eps)
    w = tl.load(w_ptr + cols, mask=mask, other=0.0).to(tl.float32)
    tl.store(out_ptr + row * stride_out + cols, x * rstd * w, mask=mask)


def rmsnorm(x, w, eps: float = 1e-6, out=None, num_warps: int = 4):
    m, n = x.shape
    out = enceladus.new_empty(x) if out is None else out
    rmsnorm_kernel[(m,)](x, w, out, enceladus.element_strides(x)[0],
                         enceladus.element_strides(out)[0], n, eps,
                         BLOCK=enceladus.next_power_of_2(n), num_warps=num_warps)
    return out
