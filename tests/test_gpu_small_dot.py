"""GPU parity for `tl.dot` on tiles below the MFMA minimums (8-row or 8-column tiles,
K = 8 with 16-bit operands), which the reference allows (language/ops.py:1258-1262: K a
multiple of 8, strips a multiple of 8). They run as fp32 multiply-adds from LDS; checked
against float64 NumPy products of the same rounded operands."""

import numpy as np
import pytest

import enceladus
import enceladus.language as tl

pytestmark = pytest.mark.gpu


@enceladus.jit
def _float_matmul(a_ptr, b_ptr, c_ptr, K, BM: tl.constexpr, BN: tl.constexpr,
                  BK: tl.constexpr, OUT16: tl.constexpr):
    rm, rn, rk = tl.arange(0, BM), tl.arange(0, BN), tl.arange(0, BK)
    if OUT16:
        acc = tl.zeros((BM, BN), tl.float16)
    else:
        acc = tl.zeros((BM, BN), tl.float32)
    for k in range(0, K, BK):
        a = tl.load(a_ptr + rm[:, None] * K + (k + rk)[None, :])
        b = tl.load(b_ptr + (k + rk)[:, None] * BN + rn[None, :])
        acc = tl.dot(a, b, acc)
    tl.store(c_ptr + rm[:, None] * BN + rn[None, :], acc.to(tl.float32))


CASES = [(8, 8, 8, 1), (8, 32, 8, 4), (16, 16, 8, 1), (32, 16, 8, 2), (64, 8, 16, 4)]


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("bm,bn,bk,nw", CASES)
def test_small_tile_dot(dtype, bm, bn, bk, nw):
    import torch
    print(f"[case] small dot {dtype} {bm}x{bn}x{bk} warps={nw}", flush=True)
    k = 4 * bk
    g = torch.Generator().manual_seed(8)
    tdt = getattr(torch, dtype)
    a = torch.randn((bm, k), generator=g).to(tdt)
    b = torch.randn((k, bn), generator=g).to(tdt)
    c = torch.zeros((bm, bn), dtype=torch.float32)
    ad, bd, cd = a.cuda(), b.cuda(), c.cuda()
    _float_matmul[(1,)](ad, bd, cd, k, BM=bm, BN=bn, BK=bk, OUT16=False, num_warps=nw)
    want = a.double().numpy() @ b.double().numpy()
    np.testing.assert_allclose(cd.cpu().numpy(), want, rtol=1e-5, atol=1e-4)


def test_small_tile_dot_fp16_accumulator():
    import torch
    print("[case] small dot fp16 accumulator", flush=True)
    g = torch.Generator().manual_seed(9)
    a = torch.randn((8, 16), generator=g).to(torch.float16)
    b = torch.randn((16, 8), generator=g).to(torch.float16)
    cd = torch.zeros((8, 8), dtype=torch.float32, device="cuda")
    _float_matmul[(1,)](a.cuda(), b.cuda(), cd, 16, BM=8, BN=8, BK=8, OUT16=True, num_warps=1)
    want = a.double().numpy() @ b.double().numpy()
    np.testing.assert_allclose(cd.cpu().numpy(), want, rtol=2e-3, atol=2e-3)
