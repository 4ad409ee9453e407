"""The launch that allocates nothing (`ek_launch_flush_noalloc`, include/enceladus_hip.h):
a privatised histogram with its partial rows in the library's static scratch array gives
the same bins as the allocating launch (`kernel[grid](...)`, partial rows in a buffer the
library allocates), bit for bit, on two calls in a row with the second one smaller, and a
launch that needs more scratch than the array holds is refused before anything runs."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _launch_both(n, bins, seed):
    import torch
    from enceladus_amd.runtime import device as D
    from examples.histogram import histogram_kernel
    print(f"[case] no-alloc histogram n={n} bins={bins}", flush=True)
    x = torch.from_numpy(np.random.default_rng(seed).integers(0, bins, n, dtype=np.int32))
    xd = x.cuda()
    grid = ((n + 1023) // 1024,)
    ref = torch.zeros(bins, dtype=torch.int32, device="cuda")
    histogram_kernel[grid](xd, ref, n, 0.0, 1.0, NUM_BINS=bins, BLOCK=1024)
    ck = histogram_kernel.warmup(xd, ref, n, 0.0, 1.0, NUM_BINS=bins, BLOCK=1024)
    assert ck.gen.flush is not None
    got = torch.zeros(bins, dtype=torch.int32, device="cuda")
    ck.launch_noalloc(grid, ck.pack([xd.data_ptr(), got.data_ptr(), n, 0.0, 1.0]),
                      D.current_stream())
    torch.cuda.synchronize()
    want = np.bincount(x.numpy(), minlength=bins).astype(np.int32)
    return got.cpu().numpy(), ref.cpu().numpy(), want, ck


def test_noalloc_launch_matches_allocating_launch():
    # the full-size config first, then a smaller ragged one over the same scratch array
    for n, seed in ((1 << 26, 0), (100_003, 1)):
        got, ref, want, ck = _launch_both(n, 1024, seed)
        assert np.array_equal(ref, want)
        assert np.array_equal(got, ref)


def test_noalloc_launch_refuses_oversized_scratch():
    import torch
    from enceladus_amd.compiler.errors import HipError
    from enceladus_amd.runtime import device as D
    from enceladus_amd.runtime import hip
    from examples.histogram import histogram_kernel
    bins, n = 16384, 1 << 24
    print(f"[case] no-alloc histogram refused: n={n} bins={bins}", flush=True)
    xd = torch.zeros(n, dtype=torch.int32, device="cuda")
    got = torch.zeros(bins, dtype=torch.int32, device="cuda")
    ck = histogram_kernel.warmup(xd, got, n, 0.0, 1.0, NUM_BINS=bins, BLOCK=1024)
    grid = ((n + 1023) // 1024,)
    assert ck.gen.flush is not None
    (gx, _, _), _ = ck.launch_grid(grid)
    assert gx * ck.gen.flush["total"] * 4 > hip.SCRATCH_BYTES
    with pytest.raises(HipError, match="static buffer"):
        ck.launch_noalloc(grid, ck.pack([xd.data_ptr(), got.data_ptr(), n, 0.0, 1.0]),
                          D.current_stream())
    torch.cuda.synchronize()
    assert int(got.sum()) == 0          # nothing ran
