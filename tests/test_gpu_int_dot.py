"""GPU parity for integer `tl.dot` against exact NumPy products (int64, wrapped to int32):
int8 on the i8 MFMAs (32x32x32, 32x32x16, 16x16x64, 16x16x32 shapes), uint8, int16 and
int32 on the multiply-add path, accumulators passed in and carried through a K loop, and
32-bit wraparound (reference: language/ops.py:1244-1270, integer operands accumulate in
int32 and wrap)."""

import numpy as np
import pytest

import enceladus
import enceladus.language as tl

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)


@enceladus.jit
def _int_matmul(a_ptr, b_ptr, c_ptr, K, BM: tl.constexpr, BN: tl.constexpr,
                BK: tl.constexpr, ACC: tl.constexpr):
    rm, rn, rk = tl.arange(0, BM), tl.arange(0, BN), tl.arange(0, BK)
    if ACC:
        acc = tl.load(c_ptr + rm[:, None] * BN + rn[None, :])
    else:
        acc = tl.zeros((BM, BN), tl.int32)
    for k in range(0, K, BK):
        a = tl.load(a_ptr + rm[:, None] * K + (k + rk)[None, :])
        b = tl.load(b_ptr + (k + rk)[:, None] * BN + rn[None, :])
        acc = tl.dot(a, b, acc)
    tl.store(c_ptr + rm[:, None] * BN + rn[None, :], acc)


def _wrap32(x):
    return ((x.astype(np.int64) + 2**31) % 2**32 - 2**31).astype(np.int32)


@pytest.mark.parametrize("dtype,bm,bn,bk,k,nw,acc", [
    (np.int8, 64, 64, 64, 128, 4, False),    # 32x32x32 MFMA
    (np.int8, 64, 64, 16, 48, 4, True),      # 32x32x16 MFMA
    (np.int8, 16, 16, 64, 64, 1, False),     # 16x16x64 MFMA
    (np.int8, 16, 32, 32, 96, 1, True),      # 16x16x32 MFMA
    (np.int8, 32, 32, 8, 16, 4, False),      # K step 8: multiply-add path
    (np.uint8, 32, 64, 32, 64, 4, False),
    (np.int16, 32, 32, 16, 32, 4, True),
    (np.int32, 16, 32, 8, 24, 2, False),
])
def test_integer_dot(dtype, bm, bn, bk, k, nw, acc):
    _say(f"int dot {np.dtype(dtype).name} {bm}x{bn}x{bk} K={k} warps={nw} acc={acc}")
    rng = np.random.default_rng(5)
    info = np.iinfo(dtype)
    lo, hi = (info.min, info.max + 1) if info.bits <= 8 else (-3000, 3000)
    a = rng.integers(lo, hi, (bm, k)).astype(dtype)
    b = rng.integers(lo, hi, (k, bn)).astype(dtype)
    c0 = rng.integers(-1000, 1000, (bm, bn)).astype(np.int32)
    c = c0.copy() if acc else np.zeros((bm, bn), np.int32)
    _int_matmul[(1,)](a, b, c, k, BM=bm, BN=bn, BK=bk, ACC=acc, num_warps=nw)
    want = a.astype(np.int64) @ b.astype(np.int64) + (c0 if acc else 0)
    np.testing.assert_array_equal(c, _wrap32(want))


def test_integer_dot_wraps_modulo_2_32():
    _say("int dot wraparound int32")
    rng = np.random.default_rng(6)
    a = rng.integers(-2**31, 2**31, (16, 16)).astype(np.int32)
    b = rng.integers(-2**31, 2**31, (16, 16)).astype(np.int32)
    c = np.zeros((16, 16), np.int32)
    _int_matmul[(1,)](a, b, c, 16, BM=16, BN=16, BK=16, ACC=False, num_warps=1)
    prods = (a.astype(object) @ b.astype(object))
    want = np.array([[int(v) % 2**32 for v in row] for row in prods], np.uint64)
    np.testing.assert_array_equal(c.view(np.uint32).astype(np.uint64), want)
