"""Histogram with `tl.atomic_add` (reference: examples/09_histogram.py:17-34)."""

import numpy as np

import enceladus
import enceladus.language as tl


@enceladus.jit
def histogram_kernel(x_ptr, hist_ptr, n, lo, inv_width, NUM_BINS: tl.constexpr,
                     BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    x = tl.load(x_ptr + offs, mask=offs < n, other=0.0).to(tl.float32)
    b = tl.floor((x - lo) * inv_width).to(tl.int32)
    ok = (offs < n) & (b >= 0) & (b < NUM_BINS)
    tl.atomic_add(hist_ptr + b, 1, mask=ok)


def histogram(x, num_bins: int, lo: float, hi: float, block: int = 1024, hist=None):
    if hist is None:
        hist = enceladus.new_zeros(x, (num_bins,), np.int32)
    n = int(np.prod(x.shape))
    histogram_kernel[(enceladus.cdiv(n, block),)](x, hist, n, float(lo), num_bins / (hi - lo),
                                                  NUM_BINS=num_bins, BLOCK=block)
    return hist
