"""GPU parity for the example kernels in every dtype and edge case the reference's own
example tests use (reference: tests/test_interpreter.py:37-112 and
tests/test_atomics_scans.py:200-227):

- vector add in fp32/fp16/bf16 at n = 1, 1000, 2^16 + 3;
- softmax in fp32/fp16 on (4, 128), (37, 1000) and (3, 20) (a 32-wide block on more lanes
  than elements, so whole lanes see only `other=-inf`), inputs scaled by 4;
- layernorm in fp32/fp16, block 256 on rows of 256 and 1000;
- matmul + bias + GELU on the ragged 200 x 96 x 130 in fp32/fp16;
- fused GELU in fp32/fp16/bf16; RMSNorm in fp32/fp16 with N(0,1) weights;
- cumsum in fp32/fp16/bf16/int8/int64, forward and reverse, on (5, 1000), (64, 32), (3, 7)
  and (3, 3000) (rows scanned in segments);
- the histogram example on float N(0,1) input over [-3, 3) in 48 bins, out-of-range values
  masked (bins of negative and fractional values through `floor`).

Each case is compared with the oracle interpreter on the same inputs and with the
example's NumPy closed form, at the reference's tolerances by output dtype (fp32 1e-5,
fp16 atol 1e-3 / rtol 2e-3, bf16 atol 1e-2 / rtol 1.6e-2; integers exact), with the
reference's overrides: atol 1e-4 for fp32 layernorm and the fp32 fused epilogue, 1e-4
for fp32 cumsum (sums associate differently).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import interpreter as O
from oracle import reference_np as R

pytestmark = pytest.mark.gpu

TOL = {"float32": (1e-5, 1e-5), "float16": (1e-3, 2e-3), "bfloat16": (1e-2, 1.6e-2)}


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _randn(rng, shape):
    return rng.standard_normal(shape).astype(np.float32)


def _round(a32: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values rounded to `dtype` and returned as float32 (bf16 by torch's RNE)."""
    if dtype == "bfloat16":
        import torch
        return torch.from_numpy(np.ascontiguousarray(a32, np.float32)).bfloat16().float().numpy()
    return np.asarray(a32).astype(dtype).astype(np.float32)


def _dev(a32: np.ndarray, dtype: str):
    """A kernel argument holding `a32` in `dtype`: NumPy for fp32/fp16/ints, a torch GPU
    tensor for bf16 (NumPy has no bfloat16)."""
    if dtype == "bfloat16":
        import torch
        return torch.from_numpy(np.ascontiguousarray(a32, np.float32)).bfloat16().cuda()
    return np.ascontiguousarray(a32).astype(dtype)


def _host(x):
    """A kernel argument as an oracle argument (torch bf16 on the CPU, NumPy otherwise)."""
    if hasattr(x, "detach"):
        return x.detach().cpu()
    return x


def _f32(x) -> np.ndarray:
    if hasattr(x, "detach"):
        return x.detach().float().cpu().numpy()
    return np.asarray(x).astype(np.float32) if np.asarray(x).dtype.kind == "f" else np.asarray(x)


def _close(got, want, dtype, atol=None, rtol=None, what=""):
    ta, tr = TOL.get(dtype, (0, 0))
    np.testing.assert_allclose(_f32(got).astype(np.float64), _f32(want).astype(np.float64),
                               atol=ta if atol is None else atol,
                               rtol=tr if rtol is None else rtol, err_msg=what)


def _out_like(x):
    import enceladus
    o = enceladus.new_zeros(x)
    return _host(o) if hasattr(o, "detach") else o


DT3 = ["float32", "float16", "bfloat16"]


@pytest.mark.parametrize("n", [1, 1000, (1 << 16) + 3])
@pytest.mark.parametrize("dtype", DT3)
def test_vector_add_dtypes(dtype, n):
    from examples.vector_add import add, add_kernel
    _say(f"vector add {dtype} n={n}")
    rng = np.random.default_rng(0)
    x32, y32 = _round(_randn(rng, n), dtype), _round(_randn(rng, n), dtype)
    x, y = _dev(x32, dtype), _dev(y32, dtype)
    got = add(x, y)
    want = _out_like(x)
    O.run_grid(add_kernel, ((n + 1023) // 1024,), _host(x), _host(y), want, n, BLOCK=1024)
    # fp32 adds of two rounded values, rounded once to the dtype: the same bits both ways
    assert np.array_equal(_f32(got), _f32(want))
    _close(got, _round(x32 + y32, dtype), dtype, what="vs closed form")


@pytest.mark.parametrize("shape", [(4, 128), (37, 1000), (3, 20)])
@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_softmax_dtypes(dtype, shape):
    from examples.softmax import softmax, softmax_kernel
    _say(f"softmax {dtype} {shape}")
    x32 = _round(_randn(np.random.default_rng(0), shape) * 4, dtype)
    x = _dev(x32, dtype)
    got = softmax(x)
    m, n = shape
    want = _out_like(x)
    O.run_grid(softmax_kernel, (m,), want, _host(x), n, n, n, BLOCK=1 << (n - 1).bit_length())
    _close(got, want, dtype, what="vs oracle")
    _close(got, _round(R.softmax(x32), dtype), dtype, what="vs closed form")


@pytest.mark.parametrize("shape,block", [((8, 256), 256), ((5, 1000), 256)])
@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_layernorm_dtypes(dtype, shape, block):
    from examples.layernorm import layernorm, layernorm_kernel
    _say(f"layernorm {dtype} {shape} block {block}")
    rng = np.random.default_rng(0)
    x32 = _round(_randn(rng, shape) * 2 + 1, dtype)
    w32, b32 = _round(_randn(rng, shape[1]), dtype), _round(_randn(rng, shape[1]), dtype)
    x, w, b = _dev(x32, dtype), _dev(w32, dtype), _dev(b32, dtype)
    y, mean, rstd = layernorm(x, w, b, block=block)
    m, n = shape
    oy, om, orr = _out_like(x), np.zeros(m, np.float32), np.zeros(m, np.float32)
    O.run_grid(layernorm_kernel, (m,), _host(x), oy, _host(w), _host(b), om, orr, n, n, n,
               1e-5, BLOCK=block)
    atol = 1e-4 if dtype == "float32" else None
    _close(y, oy, dtype, atol=atol, what="y vs oracle")
    _close(mean, om, "float32", what="mean vs oracle")
    _close(rstd, orr, "float32", what="rstd vs oracle")
    ry, rm, rr = R.layernorm(x32, w32, b32)
    _close(y, _round(ry, dtype), dtype, atol=atol, what="y vs closed form")
    _close(mean, rm, "float32", atol=1e-4, what="mean vs closed form")
    _close(rstd, rr, "float32", atol=1e-4, what="rstd vs closed form")


@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_matmul_fused_epilogue_ragged(dtype):
    from examples.matmul_fused import matmul_bias_gelu, matmul_bias_gelu_kernel
    _say(f"matmul + bias + GELU {dtype} 200x96x130")
    rng = np.random.default_rng(0)
    a32, b32 = _round(_randn(rng, (200, 96)), dtype), _round(_randn(rng, (96, 130)), dtype)
    bias32 = _round(_randn(rng, 130), dtype)
    a, b, bias = _dev(a32, dtype), _dev(b32, dtype), _dev(bias32, dtype)
    got = matmul_bias_gelu(a, b, bias)
    want = np.zeros((200, 130), dtype)
    O.run_grid(matmul_bias_gelu_kernel, (2, 2), a, b, bias, want, 200, 130, 96, 96, 130, 130,
               BM=128, BN=128, BK=64)
    atol = 1e-4 if dtype == "float32" else None
    _close(got, want, dtype, atol=atol, what="vs oracle")
    _close(got, _round(R.matmul_bias_gelu(a32, b32, bias32), dtype), dtype, atol=atol,
           what="vs closed form")


@pytest.mark.parametrize("shape", [(4, 256), (7, 300)])
@pytest.mark.parametrize("dtype", DT3)
def test_fused_gelu_dtypes(dtype, shape):
    from examples.fused_gelu import fused_gelu, fused_gelu_kernel
    _say(f"fused GELU {dtype} {shape}")
    rng = np.random.default_rng(0)
    x32, b32 = _round(_randn(rng, shape), dtype), _round(_randn(rng, shape[1]), dtype)
    x, bias = _dev(x32, dtype), _dev(b32, dtype)
    got = fused_gelu(x, bias, 0.75)
    n = shape[0] * shape[1]
    want = _out_like(x)
    O.run_grid(fused_gelu_kernel, ((n + 1023) // 1024,), _host(x), _host(bias), want, n,
               shape[1], 0.75, BLOCK=1024)
    _close(got, want, dtype, what="vs oracle")
    _close(got, _round(R.fused_gelu(x32, b32, 0.75), dtype), dtype, what="vs closed form")


@pytest.mark.parametrize("shape", [(4, 128), (9, 1000)])
@pytest.mark.parametrize("dtype", ["float32", "float16"])
def test_rmsnorm_dtypes(dtype, shape):
    from examples.rmsnorm import rmsnorm, rmsnorm_kernel
    _say(f"rmsnorm {dtype} {shape}")
    rng = np.random.default_rng(0)
    x32, w32 = _round(_randn(rng, shape), dtype), _round(_randn(rng, shape[1]), dtype)
    x, w = _dev(x32, dtype), _dev(w32, dtype)
    got = rmsnorm(x, w)
    m, n = shape
    want = _out_like(x)
    O.run_grid(rmsnorm_kernel, (m,), _host(x), _host(w), want, n, n, n, 1e-6,
               BLOCK=1 << (n - 1).bit_length())
    _close(got, want, dtype, what="vs oracle")
    _close(got, _round(R.rmsnorm(x32, w32), dtype), dtype, what="vs closed form")


@pytest.mark.parametrize("reverse", [False, True])
@pytest.mark.parametrize("shape", [(5, 1000), (64, 32), (3, 7), (3, 3000)])
@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16", "int8", "int64"])
def test_cumsum_dtypes(dtype, shape, reverse):
    import enceladus
    from examples.cumsum import cumsum, cumsum_kernel
    _say(f"cumsum {dtype} {shape} reverse={reverse}")
    rng = np.random.default_rng(shape[1])
    if dtype.startswith("int"):
        x = rng.integers(-100, 100, shape).astype(dtype)
        x32 = x
    else:
        x32 = _round((rng.standard_normal(shape) * 4).astype(np.float32), dtype)
        x = _dev(x32, dtype)
    got = cumsum(x, reverse)
    m, n = shape
    bn = 1 << (n - 1).bit_length()
    bm = max(1, min(16, 4096 // bn))
    want = _host(enceladus.new_zeros(got))
    O.run_grid(cumsum_kernel, ((m + bm - 1) // bm,), want, _host(x), m, n, n, n,
               REVERSE=reverse, BLOCK_M=bm, BLOCK_N=bn)
    if dtype.startswith("int"):
        assert np.asarray(got).dtype == (np.int32 if dtype == "int8" else np.int64)
        assert np.array_equal(got, want)
        assert np.array_equal(got, R.cumsum(x, reverse))
        return
    tol = 1e-4 if dtype == "float32" else None
    _close(got, want, dtype, atol=tol, rtol=tol, what="vs oracle")
    _close(got, _round(R.cumsum(x32, reverse), dtype), dtype, atol=tol, rtol=tol,
           what="vs closed form")


def test_histogram_float_example():
    """The reference's histogram example: 100,003 float32 N(0,1) values into 48 bins over
    [-3, 3); values outside fall in bins < 0 or >= 48 and are masked."""
    from examples.histogram import histogram, histogram_kernel
    _say("histogram float32 N(0,1) 100003 -> 48 bins over [-3, 3)")
    x = np.random.default_rng(5).standard_normal(100_003).astype(np.float32)
    got = histogram(x, 48, -3.0, 3.0)
    assert np.array_equal(got, R.histogram(x, 48, -3.0, 3.0))
    want = np.zeros(48, np.int32)
    n = x.size
    O.run_grid(histogram_kernel, ((n + 1023) // 1024,), x, want, n, -3.0, 48 / 6.0,
               NUM_BINS=48, BLOCK=1024)
    assert np.array_equal(got, want)
    assert 0 < int(got.sum()) < n      # some values fall outside [-3, 3)
