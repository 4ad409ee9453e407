"""Program versioning on the GPU: the guarded branch-free copy of a straight-line masked
program and the general copy give the same results as the per-access edge paths, for
interior, edge and partial-tile programs."""

import numpy as np
import pytest

import enceladus
import enceladus.language as tl

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)


@enceladus.jit
def _masked_add(x_ptr, y_ptr, o_ptr, n, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    tl.store(o_ptr + offs, tl.load(x_ptr + offs, mask=m) + tl.load(y_ptr + offs, mask=m), mask=m)


@enceladus.jit
def _masked_rows(x_ptr, o_ptr, n_rows, n_cols, stride, BM: tl.constexpr, BN: tl.constexpr):
    r = tl.program_id(0) * BM + tl.arange(0, BM)
    c = tl.program_id(1) * BN + tl.arange(0, BN)
    m = (r[:, None] < n_rows) & (c[None, :] < n_cols)
    x = tl.load(x_ptr + r[:, None] * stride + c[None, :], mask=m, other=-1.0)
    y = tl.where(c[None, :] < n_cols, x * 2.0 + 1.0, 0.0)
    tl.store(o_ptr + r[:, None] * stride + c[None, :], y, mask=m)


@pytest.mark.parametrize("mode", ["", "no_program_versioning", "no_serial_streams"])
@pytest.mark.parametrize("n", [1, 1023, 1024, 1025, (1 << 20) + 5])
def test_versioned_vector_kernel(n, mode, monkeypatch):
    _say(f"versioned add n={n} mode={mode!r}")
    monkeypatch.setenv("ENCELADUS_CODEGEN", mode)
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    y = rng.standard_normal(n).astype(np.float32)
    o = np.full(n + 7, 7.0, np.float32)
    _masked_add[(enceladus.cdiv(n, 1024),)](x, y, o, n, BLOCK=1024)
    assert np.array_equal(o[:n], x + y)
    assert np.all(o[n:] == 7.0)


@pytest.mark.parametrize("mode", ["", "no_program_versioning"])
@pytest.mark.parametrize("shape", [(64, 256), (67, 300), (1, 5), (130, 256)])
def test_versioned_2d_kernel(shape, mode, monkeypatch):
    _say(f"versioned rows shape={shape} mode={mode!r}")
    monkeypatch.setenv("ENCELADUS_CODEGEN", mode)
    rows, cols = shape
    stride = cols + 3
    x = np.random.default_rng(rows * cols).standard_normal((rows, stride)).astype(np.float32)
    o = np.full((rows, stride), 5.0, np.float32)
    grid = (enceladus.cdiv(rows, 16), enceladus.cdiv(cols, 128))
    _masked_rows[grid](x, o, rows, cols, stride, BM=16, BN=128)
    want = o.copy()
    want[:, :cols] = x[:, :cols] * np.float32(2.0) + np.float32(1.0)
    assert np.array_equal(o, want)
