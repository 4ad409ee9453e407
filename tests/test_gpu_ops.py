"""GPU parity of the elementwise language: unary math, float and integer binary operators,
and conversions, each compiled kernel against the CPU oracle on the same seeded inputs
(reference test strategy: tests/test_interpreter.py test_unary_ops, test_binary_ops,
test_int_ops, test_int_to_half_casts, test_float_to_int_casts_match_metal,
test_integer_division_truncates).

Bars: integer results and conversions bit-exact; float32 exact for the correctly rounded
operations (add, sub, mul, div, sqrt, floor, ceil, abs, neg, max, min, comparisons) and
within rtol 1e-5 / atol 1e-6 for the transcendental functions (the device uses the
hardware exp2/log2 and polynomial approximations, the oracle NumPy); float16 results
within one float16 ulp (both sides compute in float32 and round once).
"""

import numpy as np
import pytest

import enceladus
import enceladus.language as tl
from oracle import interpreter as O

pytestmark = pytest.mark.gpu

N = 1000


def _say(msg):
    print(f"[case] {msg}", flush=True)


@enceladus.jit
def _unary_kernel(x_ptr, out_ptr, n, OP: tl.constexpr, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    x = tl.load(x_ptr + offs, mask=m, other=1.0)
    if OP == "exp":
        y = tl.exp(x)
    elif OP == "exp2":
        y = tl.exp2(x)
    elif OP == "log":
        y = tl.log(x)
    elif OP == "log2":
        y = tl.log2(x)
    elif OP == "sqrt":
        y = tl.sqrt(x)
    elif OP == "rsqrt":
        y = tl.rsqrt(x)
    elif OP == "sin":
        y = tl.sin(x)
    elif OP == "cos":
        y = tl.cos(x)
    elif OP == "tanh":
        y = tl.tanh(x)
    elif OP == "erf":
        y = tl.erf(x)
    elif OP == "sigmoid":
        y = tl.sigmoid(x)
    elif OP == "floor":
        y = tl.floor(x)
    elif OP == "ceil":
        y = tl.ceil(x)
    elif OP == "abs":
        y = tl.abs(x)
    else:
        y = -x
    tl.store(out_ptr + offs, y, mask=m)


EXACT = {"sqrt", "floor", "ceil", "abs", "neg"}
POSITIVE = {"log", "log2", "sqrt", "rsqrt"}


def _run_both(kernel, grid, ins, out_dtype, **consts):
    got = np.zeros(N, out_dtype)
    want = np.zeros(N, out_dtype)
    kernel[grid](*ins, got, N, **consts)
    O.run_grid(kernel, grid, *ins, want, N, **consts)
    return got, want


def _check_float(got, want, exact, dtype):
    if dtype == np.float16:
        np.testing.assert_allclose(got.astype(np.float32), want.astype(np.float32),
                                   rtol=1e-3, atol=1e-3)
    elif exact:
        np.testing.assert_array_equal(got, want)
    else:
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("op", ["exp", "exp2", "log", "log2", "sqrt", "rsqrt", "sin", "cos",
                                "tanh", "erf", "sigmoid", "floor", "ceil", "abs", "neg"])
def test_unary_ops(op, dtype):
    _say(f"unary {op} {np.dtype(dtype).name}")
    rng = np.random.default_rng(7)
    x = rng.standard_normal(N).astype(np.float32) * 3
    if op in POSITIVE:
        x = np.abs(x) + 0.05
    x = x.astype(dtype)
    got, want = _run_both(_unary_kernel, (4,), (x,), dtype, OP=op, BLOCK=256)
    _check_float(got, want, op in EXACT, dtype)


@enceladus.jit
def _binary_kernel(x_ptr, y_ptr, out_ptr, n, OP: tl.constexpr, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    x = tl.load(x_ptr + offs, mask=m, other=1)
    y = tl.load(y_ptr + offs, mask=m, other=1)
    if OP == "add":
        z = x + y
    elif OP == "sub":
        z = x - y
    elif OP == "mul":
        z = x * y
    elif OP == "div":
        z = x / y
    elif OP == "floordiv":
        z = x // y
    elif OP == "mod":
        z = x % y
    elif OP == "max":
        z = tl.maximum(x, y)
    elif OP == "min":
        z = tl.minimum(x, y)
    elif OP == "and":
        z = x & y
    elif OP == "or":
        z = x | y
    elif OP == "xor":
        z = x ^ y
    elif OP == "shl":
        z = x << y
    elif OP == "shr":
        z = x >> y
    elif OP == "lt":
        z = tl.where(x < y, x, y)
    else:
        z = tl.where(x == y, x, -y)
    tl.store(out_ptr + offs, z, mask=m)


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("op", ["add", "sub", "mul", "div", "mod", "max", "min", "lt", "eq"])
def test_float_binary_ops(op, dtype):
    _say(f"binary {op} {np.dtype(dtype).name}")
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(N) * 4).astype(dtype)
    y = (rng.standard_normal(N) * 2).astype(dtype)
    y[np.abs(y.astype(np.float32)) < 0.05] = 0.5
    y[::17] = x[::17]                       # some equal pairs for == and %
    got, want = _run_both(_binary_kernel, (4,), (x, y), dtype, OP=op, BLOCK=256)
    _check_float(got, want, op != "mod", dtype)


INT_OPS = ["add", "sub", "mul", "floordiv", "mod", "max", "min", "and", "or", "xor", "shl",
           "shr", "lt", "eq"]


@pytest.mark.parametrize("dtype", [np.int8, np.int32, np.int64, np.uint32])
@pytest.mark.parametrize("op", INT_OPS)
def test_int_ops(op, dtype):
    _say(f"int {op} {np.dtype(dtype).name}")
    rng = np.random.default_rng(9)
    info = np.iinfo(dtype)
    x = rng.integers(info.min, info.max, N, endpoint=True, dtype=dtype)
    y = rng.integers(info.min, info.max, N, endpoint=True, dtype=dtype)
    if op in ("floordiv", "mod"):
        y[y == 0] = 3
        if info.min < 0:
            y[(x == info.min) & (y == -1)] = 7          # the one overflowing quotient
        y[::5] = rng.integers(1, 9, len(y[::5])).astype(dtype)    # small divisors too
        x[::7] = -np.abs(x[::7].astype(np.int64)).astype(dtype) if info.min < 0 else x[::7]
    if op in ("shl", "shr"):
        y = rng.integers(0, info.bits, N).astype(dtype)
    y[::13] = x[::13]
    got, want = _run_both(_binary_kernel, (4,), (x, y), dtype, OP=op, BLOCK=256)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("dtype", [np.int8, np.int16, np.int32, np.int64, np.uint8, np.uint32])
@pytest.mark.parametrize("op", ["shl", "shr"])
def test_shift_counts_out_of_range(op, dtype):
    """Counts that are negative or at least the bit width follow NumPy's shift rules, as
    the reference interpreter's `np.left_shift`/`np.right_shift` do (reference
    interpreter/interp.py:622-623): a left shift gives 0, a right shift the sign fill.
    Checked against NumPy itself as well as the oracle; counts into the sign bit wrap."""
    _say(f"shift {op} out of range {np.dtype(dtype).name}")
    rng = np.random.default_rng(11)
    info = np.iinfo(dtype)
    x = rng.integers(info.min, info.max, N, endpoint=True, dtype=dtype)
    counts = np.concatenate([np.arange(-70, 140), [info.bits - 1, info.bits, info.bits + 1,
                                                     2 * info.bits, 255, 256, 257]])
    y = np.resize(counts, N).astype(np.int64).astype(dtype)     # wraps as the cast does
    got, want = _run_both(_binary_kernel, (4,), (x, y), dtype, OP=op, BLOCK=256)
    np.testing.assert_array_equal(got, want)
    ref = np.left_shift(x, y) if op == "shl" else np.right_shift(x, y)
    np.testing.assert_array_equal(got, ref)


@enceladus.jit
def _cast_kernel(x_ptr, out_ptr, n, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    x = tl.load(x_ptr + offs, mask=m)
    tl.store(out_ptr + offs, x.to(out_ptr.dtype.element_ty), mask=m)


def _float_edges(rng):
    x = (rng.standard_normal(N) * 1e3).astype(np.float32)
    x[:12] = [np.nan, np.inf, -np.inf, 3e9, -3e9, 1e20, -1e20, 2.5, -2.5, 255.9, -0.7, 65504.5]
    x[12::50] = rng.uniform(-5e4, 5e4, len(x[12::50])).astype(np.float32)
    return x


@pytest.mark.parametrize("dst", [np.int8, np.int16, np.int32, np.int64, np.uint8, np.uint32,
                                 np.float16])
def test_float32_conversions(dst):
    # truncation toward zero, saturation, NaN -> 0 for integers; RNE with overflow to inf
    # for float16
    _say(f"cast float32 -> {np.dtype(dst).name}")
    x = _float_edges(np.random.default_rng(10))
    got, want = _run_both(_cast_kernel, (4,), (x,), dst, BLOCK=256)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("src,dst", [(np.int32, np.float16), (np.int64, np.int32),
                                     (np.int32, np.uint8), (np.uint32, np.float32),
                                     (np.int64, np.float32), (np.int8, np.uint32)])
def test_integer_conversions(src, dst):
    _say(f"cast {np.dtype(src).name} -> {np.dtype(dst).name}")
    info = np.iinfo(src)
    x = np.random.default_rng(11).integers(info.min, info.max, N, endpoint=True, dtype=src)
    got, want = _run_both(_cast_kernel, (4,), (x,), dst, BLOCK=256)
    np.testing.assert_array_equal(got, want)


def test_bfloat16_conversion_rounds_to_nearest_even():
    import torch
    _say("cast float32 -> bfloat16")
    x = _float_edges(np.random.default_rng(12))
    x = x[np.isfinite(x)][:N // 2]
    xs = torch.from_numpy(x).cuda()
    out = torch.zeros(len(x), dtype=torch.bfloat16, device="cuda")
    _cast_kernel[(enceladus.cdiv(len(x), 256),)](xs, out, len(x), BLOCK=256)
    torch.cuda.synchronize()
    want = torch.from_numpy(x).to(torch.bfloat16)          # RNE, as the oracle's table
    assert torch.equal(out.cpu().view(torch.int16), want.view(torch.int16))
