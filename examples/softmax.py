"""Row softmax, one program per row (reference: examples/02_softmax.py:15-38)."""

import enceladus
import enceladus.language as tl


@enceladus.jit
def softmax_kernel(out_ptr, in_ptr, stride_in, stride_out, n_cols, BLOCK: tl.constexpr):
    row = tl.program_id(0)
    cols = tl.arange(0, BLOCK)
    mask = cols < n_cols
    x = tl.load(in_ptr + row * stride_in + cols, mask=mask, other=-float("inf"))
    x = x.to(tl.float32)
    x = x - tl.max(x, axis=0)
    num = tl.exp(x)
    tl.store(out_ptr + row * stride_out + cols, num / tl.sum(num, axis=0), mask=mask)


def softmax(x, out=None, num_warps: int = 4):
    m, n = x.shape
    out = enceladus.new_empty(x) if out is None else out
    softmax_kernel[(m,)](out, x, enceladus.element_strides(x)[0],
                         enceladus.element_strides(out)[0], n,
                         BLOCK=enceladus.next_power_of_2(n), num_warps=num_warps)
    return out
