"""GPU parity of the language's reductions and Python semantics: built-in reductions in
every width (NaN included), tuple reductions, loop-carried values, Python `range` over
64-bit and unsigned bounds, `and`/`or` returning operands, negative literals in unsigned
types, argument names that look like generated ones, and `tl.debug_barrier` (reference
test strategy: tests/test_interpreter.py test_shape_and_reduce_ops, test_reductions,
test_loop_carried_values_read_the_previous_iteration, test_64_bit_loops_follow_python_range,
test_uint64_loops_follow_python_range, test_bool_ops_return_operands,
test_welford_tuple_reduce, test_negative_literals_wrap_in_unsigned_types,
test_argmax_ignores_nan_like_max, test_argument_names_dont_clash_with_generated_code,
test_debug_barrier_orders_stores_before_loads_by_other_threads).

Reductions are checked against the CPU oracle on the same inputs: integer results, max,
min, argmax and argmin bit-exact, float sums within rtol 1e-5 (the device adds in a tree,
the oracle pairwise). The rest against Python's own closed forms.
"""

import numpy as np
import pytest

import enceladus
import enceladus.language as tl
from oracle import interpreter as O

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)


@enceladus.jit
def _reduce_kernel(x_ptr, out_ptr, OP: tl.constexpr, AXIS: tl.constexpr, M: tl.constexpr,
                   N: tl.constexpr):
    rm = tl.arange(0, M)
    rn = tl.arange(0, N)
    x = tl.load(x_ptr + rm[:, None] * N + rn[None, :])
    if OP == "sum":
        r = tl.sum(x, AXIS)
    elif OP == "max":
        r = tl.max(x, AXIS)
    elif OP == "min":
        r = tl.min(x, AXIS)
    elif OP == "argmax":
        r = tl.argmax(x, AXIS)
    else:
        r = tl.argmin(x, AXIS)
    if AXIS == 0:
        tl.store(out_ptr + rn, r)
    else:
        tl.store(out_ptr + rm, r)


@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.int8, np.int32, np.uint32])
@pytest.mark.parametrize("op", ["sum", "max", "min", "argmax", "argmin"])
def test_reductions(op, dtype, axis):
    _say(f"reduce {op} {np.dtype(dtype).name} axis={axis}")
    M, N = 32, 128
    rng = np.random.default_rng(21)
    if np.issubdtype(dtype, np.floating):
        x = (rng.standard_normal((M, N)) * 4).astype(dtype)
        x[3, 7] = x[3, 9]                         # ties: the first index wins
    else:
        info = np.iinfo(dtype)
        lo, hi = (max(info.min, -100), min(info.max, 100)) if op == "sum" else \
            (info.min, info.max)
        x = rng.integers(lo, hi, (M, N), endpoint=True).astype(dtype)
        x[5, :] = x[5, 0]
    out_dt = np.int32 if op.startswith("arg") else \
        (np.float32 if np.issubdtype(dtype, np.floating) else np.int64)
    n_out = N if axis == 0 else M
    got, want = np.zeros(n_out, out_dt), np.zeros(n_out, out_dt)
    _reduce_kernel[(1,)](x, got, OP=op, AXIS=axis, M=M, N=N)
    O.run_grid(_reduce_kernel, (1,), x, want, OP=op, AXIS=axis, M=M, N=N)
    if op == "sum" and np.issubdtype(dtype, np.floating):
        tol = 1e-3 if dtype == np.float16 else 1e-5
        np.testing.assert_allclose(got, want, rtol=tol, atol=tol)
    else:
        np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("op", ["max", "argmax", "min", "argmin"])
def test_nan_is_ignored_like_fmax(op):
    _say(f"NaN {op}")
    x = np.random.default_rng(22).standard_normal((32, 128)).astype(np.float32)
    x[:, 0] = np.nan
    x[4, :] = np.nan                               # an all-NaN row
    out_dt = np.int32 if op.startswith("arg") else np.float32
    got, want = np.zeros(32, out_dt), np.zeros(32, out_dt)
    _reduce_kernel[(1,)](x, got, OP=op, AXIS=1, M=32, N=128)
    O.run_grid(_reduce_kernel, (1,), x, want, OP=op, AXIS=1, M=32, N=128)
    np.testing.assert_array_equal(got, want)


@enceladus.jit
def _welford_combine(mean_a, m2_a, n_a, mean_b, m2_b, n_b):
    n = n_a + n_b
    delta = mean_b - mean_a
    frac = tl.where(n == 0, 0.0, n_b / n)
    return mean_a + delta * frac, m2_a + m2_b + delta * delta * n_a * frac, n


@enceladus.jit
def _welford_kernel(x_ptr, mean_ptr, var_ptr, n_cols, BLOCK: tl.constexpr):
    row = tl.program_id(0)
    cols = tl.arange(0, BLOCK)
    mask = cols < n_cols
    x = tl.load(x_ptr + row * n_cols + cols, mask=mask, other=0.0)
    count = mask.to(tl.float32)
    mean, m2, n = tl.reduce((x, tl.zeros_like(x), count), 0, _welford_combine)
    tl.store(mean_ptr + row, mean)
    tl.store(var_ptr + row, m2 / n)


def test_welford_tuple_reduce():
    _say("welford tuple reduce")
    x = (np.random.default_rng(23).standard_normal((6, 100)) * 3 + 1).astype(np.float32)
    mean, var = np.zeros(6, np.float32), np.zeros(6, np.float32)
    _welford_kernel[(6,)](x, mean, var, 100, BLOCK=128)
    np.testing.assert_allclose(mean, x.mean(1, dtype=np.float64), atol=1e-4)
    np.testing.assert_allclose(var, x.var(1, dtype=np.float64), atol=1e-4)


@enceladus.jit
def _carried_kernel(out_ptr, n, B: tl.constexpr):
    s = 0
    t = tl.zeros((B,), tl.int32)
    p, q = 1, 2
    for _ in range(n):
        t_new = tl.full((B,), s, tl.int32)     # a uniform tile that reads `s` before its update
        s = s + 1
        t = t_new
        p, q = q, p + q
    tl.store(out_ptr + tl.arange(0, B), t + p * 1000 + q * 100000)


@pytest.mark.parametrize("n", [0, 1, 3])
def test_loop_carried_values_read_the_previous_iteration(n):
    _say(f"carried n={n}")
    t, s, p, q = 0, 0, 1, 2
    for _ in range(n):
        t, s, p, q = s, s + 1, q, p + q
    out = np.empty(16, np.int32)
    _carried_kernel[(1,)](out, n, B=16)
    np.testing.assert_array_equal(out, t + p * 1000 + q * 100000)


@enceladus.jit
def _range64_kernel(out_ptr, base, lo, hi, step, STEP: tl.constexpr):
    acc = 0
    count = 0
    for i in range(base + lo, base + hi, step if STEP == 0 else STEP):
        acc += (i - base).to(tl.int32) * 1000
        count += 1
    tl.store(out_ptr, acc + count)


_range_u64_kernel = enceladus.jit(_range64_kernel.fn)


@pytest.mark.parametrize("lo,hi,step", [(0, 30, 1), (3, 30, 7), (30, 0, -1), (29, 0, -4),
                                        (0, 0, 1), (5, 0, 2), (0, 5, -1)])
@pytest.mark.parametrize("const_step", [False, True])
def test_64_bit_loops_follow_python_range(lo, hi, step, const_step):
    _say(f"range64 {lo},{hi},{step} const={const_step}")
    base = 5_000_000_000
    out = np.zeros(1, np.int32)
    _range64_kernel[(1,)](out, base, lo, hi, step, STEP=step if const_step else 0)
    r = range(lo, hi, step)
    assert out[0] == sum(r) * 1000 + len(r)


@pytest.mark.parametrize("lo,hi,step", [(0, 30, 1), (3, 30, 7), (5, 0, 2)])
@pytest.mark.parametrize("const_step", [False, True])
def test_uint64_loops_follow_python_range(lo, hi, step, const_step):
    _say(f"range u64 {lo},{hi},{step} const={const_step}")
    base = (1 << 63) + 5_000_000_000
    out = np.zeros(1, np.int32)
    _range_u64_kernel[(1,)](out, base, np.uint64(lo), np.uint64(hi), np.uint64(step),
                            STEP=step if const_step else 0)
    r = range(lo, hi, step)
    assert out[0] == sum(r) * 1000 + len(r)


BOOL_OPS = {
    "and": lambda n, m, f, x: n and m, "or": lambda n, m, f, x: n or m,
    "and_const": lambda n, m, f, x: n and 5, "or_const": lambda n, m, f, x: n or 5,
    "const_left": lambda n, m, f, x: 0 or n, "chain": lambda n, m, f, x: n and m and 9,
    "mixed": lambda n, m, f, x: n and (m + 1) * 2 or 11,
    "lazy_load": lambda n, m, f, x: n or x,
    "if_test": lambda n, m, f, x: 5 if (n and f) or not m else 6,
}


@enceladus.jit(do_not_specialize=["n", "m"])
def _bool_op_kernel(out_ptr, x_ptr, n, m, f, OP: tl.constexpr):
    if OP == "and":
        r = n and m
    elif OP == "or":
        r = n or m
    elif OP == "and_const":
        r = n and 5
    elif OP == "or_const":
        r = n or 5
    elif OP == "const_left":
        r = 0 or n
    elif OP == "chain":
        r = n and m and 9
    elif OP == "mixed":
        r = n and (m + 1) * 2 or 11
    elif OP == "lazy_load":
        r = n or tl.load(x_ptr)
    else:
        r = 5 if (n and f) or not m else 6
    tl.store(out_ptr, r)


@pytest.mark.parametrize("op", list(BOOL_OPS))
def test_bool_ops_return_operands(op):
    _say(f"bool op {op}")
    x = np.array([42], np.int32)
    got = []
    for n, m in [(3, 7), (0, 7), (2, 0), (0, 0)]:
        out = np.zeros(1, np.int32)
        _bool_op_kernel[(1,)](out, x, n, m, n / 2, OP=op)
        got.append(int(out[0]))
    assert got == [BOOL_OPS[op](n, m, n / 2, 42) for n, m in [(3, 7), (0, 7), (2, 0), (0, 0)]]


@enceladus.jit
def _unsigned_literal_kernel(x_ptr, out_ptr, n, OP: tl.constexpr, BLOCK: tl.constexpr):
    offs = tl.arange(0, BLOCK)
    if OP == "add":
        y = tl.load(x_ptr + offs) + -1
    elif OP == "other":
        y = tl.load(x_ptr + offs, mask=offs < n, other=-1)
    else:
        y = tl.full((BLOCK,), -1, x_ptr.dtype)
    tl.store(out_ptr + offs, y)


@pytest.mark.parametrize("dtype", [np.uint8, np.uint32])
@pytest.mark.parametrize("op", ["add", "other", "full"])
def test_negative_literals_wrap_in_unsigned_types(op, dtype):
    _say(f"unsigned literal {op} {np.dtype(dtype).name}")
    x = np.arange(16, dtype=dtype)
    out = np.empty_like(x)
    _unsigned_literal_kernel[(1,)](x, out, 5, OP=op, BLOCK=16)
    top = np.iinfo(dtype).max
    want = {"add": x - dtype(1), "other": np.where(np.arange(16) < 5, x, top).astype(dtype),
            "full": np.full(16, top, dtype)}[op]
    np.testing.assert_array_equal(out, want)


@enceladus.jit
def _clash_kernel(r, tc0, ek_lane, s1, a0, BLOCK: tl.constexpr):
    # argument names that look like the emitter's own identifiers
    offs = tl.arange(0, BLOCK)
    v = tl.load(r + offs) * tc0 + ek_lane
    tl.store(s1 + offs, v + a0)


def test_argument_names_dont_clash_with_generated_code():
    _say("argument names")
    x = np.arange(64, dtype=np.float32)
    out = np.zeros(64, np.float32)
    _clash_kernel[(1,)](x, 3.0, 2.0, out, 1.0, BLOCK=64)
    np.testing.assert_array_equal(out, x * 3 + 3)


@enceladus.jit
def _barrier_kernel(buf_ptr, out_ptr, BLOCK: tl.constexpr):
    offs = tl.arange(0, BLOCK)
    tl.store(buf_ptr + offs, offs * 3)
    tl.debug_barrier()
    # each thread reads elements another thread stored
    tl.store(out_ptr + offs, tl.load(buf_ptr + (BLOCK - 1 - offs)))


@pytest.mark.parametrize("num_warps", [1, 4])
def test_debug_barrier_orders_stores_before_loads_by_other_threads(num_warps):
    _say(f"debug_barrier warps={num_warps}")
    buf = np.zeros(1024, np.int32)
    out = np.zeros(1024, np.int32)
    _barrier_kernel[(1,)](buf, out, BLOCK=1024, num_warps=num_warps)
    np.testing.assert_array_equal(out, (1023 - np.arange(1024)) * 3)


# -- scans over every layout kind (reference: tests/test_atomics_scans.py:228-339) ----

@enceladus.jit
def _max_op(a, b):
    return tl.maximum(a, b)


@enceladus.jit
def _affine_op(a0, a1, b0, b1):
    # composes h -> a0 * h + a1, then h -> b0 * h + b1: associative, not commutative
    return a0 * b0, b0 * a1 + b1


@enceladus.jit
def _scan2d_kernel(a_ptr, b_ptr, x_ptr, y_ptr, M: tl.constexpr, N: tl.constexpr,
                   AXIS: tl.constexpr, REVERSE: tl.constexpr):
    offs = tl.arange(0, M)[:, None] * N + tl.arange(0, N)[None, :]
    a, b = tl.load(a_ptr + offs), tl.load(b_ptr + offs)
    h0, h1 = tl.associative_scan((a, b), AXIS, _affine_op, reverse=REVERSE)
    tl.store(a_ptr + offs, h0)
    tl.store(b_ptr + offs, h1)
    x = tl.load(x_ptr + offs)
    tl.store(y_ptr + offs, tl.associative_scan(x, AXIS, _max_op, reverse=REVERSE))


def _affine_ref(a, b, axis, reverse):
    a, b = np.moveaxis(a, axis, 0).copy(), np.moveaxis(b, axis, 0).copy()
    order = range(a.shape[0] - 2, -1, -1) if reverse else range(1, a.shape[0])
    prev = a.shape[0] - 1 if reverse else 0
    for i in order:
        a[i], b[i] = a[prev] * a[i], a[i] * b[prev] + b[i]
        prev = i
    return np.moveaxis(a, 0, axis), np.moveaxis(b, 0, axis)


@pytest.mark.parametrize("m,n", [(16, 64), (64, 16), (8, 2)])
@pytest.mark.parametrize("axis", [0, 1])
@pytest.mark.parametrize("reverse", [False, True])
def test_associative_scan_along_either_axis_of_a_2d_tile(m, n, axis, reverse):
    _say(f"scan2d {m}x{n} axis={axis} reverse={reverse}")
    rng = np.random.default_rng(m * n + axis)
    a = rng.integers(-3, 4, (m, n)).astype(np.int32)        # int32 wraps exactly in any order
    b = rng.integers(-100, 100, (m, n)).astype(np.int32)
    x = rng.standard_normal((m, n)).astype(np.float32)
    ga, gb, y = a.copy(), b.copy(), np.empty_like(x)
    _scan2d_kernel[(1,)](ga, gb, x, y, M=m, N=n, AXIS=axis, REVERSE=reverse)
    with np.errstate(over="ignore"):
        wa, wb = _affine_ref(a, b, axis, reverse)
    f = np.flip if reverse else (lambda z, axis: z)
    np.testing.assert_array_equal(ga, wa)
    np.testing.assert_array_equal(gb, wb)
    np.testing.assert_array_equal(y, f(np.maximum.accumulate(f(x, axis=axis), axis=axis),
                                       axis=axis))


@enceladus.jit
def _dot_cumsum_kernel(a_ptr, b_ptr, out_ptr, M: tl.constexpr, N: tl.constexpr,
                       K: tl.constexpr, AXIS: tl.constexpr):
    rm, rn, rk = tl.arange(0, M), tl.arange(0, N), tl.arange(0, K)
    a = tl.load(a_ptr + rm[:, None] * K + rk[None, :])
    b = tl.load(b_ptr + rk[:, None] * N + rn[None, :])
    c = tl.cumsum(tl.dot(a, b), axis=AXIS)
    tl.store(out_ptr + rm[:, None] * N + rn[None, :], c)


@pytest.mark.parametrize("axis", [0, 1])
def test_cumsum_of_a_dot_accumulator(axis):
    # the MFMA accumulator layout interleaves register and lane bits along both axes
    _say(f"cumsum of dot axis={axis}")
    rng = np.random.default_rng(axis)
    a = rng.integers(-2, 3, (64, 16)).astype(np.float32)
    b = rng.integers(-2, 3, (16, 32)).astype(np.float32)
    out = np.empty((64, 32), np.float32)
    _dot_cumsum_kernel[(1,)](a, b, out, M=64, N=32, K=16, AXIS=axis)
    np.testing.assert_array_equal(out, np.cumsum(a @ b, axis=axis))


@enceladus.jit
def _view_scan_kernel(a_ptr, b_ptr, out_a, out_b, REVERSE: tl.constexpr):
    offs = tl.arange(0, 2)[:, None] * 256 + tl.arange(0, 256)[None, :]
    a = tl.reshape(tl.trans(tl.load(a_ptr + offs)), (512,))
    b = tl.reshape(tl.trans(tl.load(b_ptr + offs)), (512,))
    h0, h1 = tl.associative_scan((a, b), 0, _affine_op, reverse=REVERSE)
    tl.store(out_a + tl.arange(0, 512), h0)
    tl.store(out_b + tl.arange(0, 512), h1)


@pytest.mark.parametrize("reverse", [False, True])
def test_scan_of_an_interleaved_view(reverse):
    _say(f"scan of a transposed view reverse={reverse}")
    rng = np.random.default_rng(7)
    a = rng.integers(-3, 4, (2, 256)).astype(np.int32)
    b = rng.integers(-100, 100, (2, 256)).astype(np.int32)
    oa, ob = np.empty(512, np.int32), np.empty(512, np.int32)
    _view_scan_kernel[(1,)](a, b, oa, ob, REVERSE=reverse)
    with np.errstate(over="ignore"):
        wa, wb = _affine_ref(a.T.reshape(-1), b.T.reshape(-1), 0, reverse)
    np.testing.assert_array_equal(oa, wa)
    np.testing.assert_array_equal(ob, wb)


_XOR_LANES = '''
#include "enceladus_cdna4.h"
template <int M> __device__ void one(uint32_t* o32, unsigned long long* o64, uint16_t* o16, int slot) {
  const int t = threadIdx.x, n = blockDim.x;
  const uint32_t v = 0x9E3779B9u * (uint32_t)(t + 1);
  o32[slot * n + t] = ek::shfl_xor<M>(v);
  o64[slot * n + t] = ek::shfl_xor<M>(((unsigned long long)v << 32) | (uint32_t)~t);
  o16[slot * n + t] = ek::shfl_xor<M>((uint16_t)(v >> 7));
}
extern "C" __global__ void xor_lanes(uint32_t* o32, unsigned long long* o64, uint16_t* o16) {
  one<1>(o32, o64, o16, 0); one<2>(o32, o64, o16, 1); one<4>(o32, o64, o16, 2);
  one<8>(o32, o64, o16, 3); one<16>(o32, o64, o16, 4); one<32>(o32, o64, o16, 5);
}
'''


def test_lane_exchanges_match_lane_xor():
    """`ek::shfl_xor<m>`, the lane butterfly of every reduction, returns lane ^ m's value
    for m = 1..32 and 16-, 32- and 64-bit values (DPP permutes, row mirrors and the gfx950
    permlane swaps), in every wave of a 4-wave workgroup."""
    _say("lane exchanges")
    k = enceladus.hip_kernel(_XOR_LANES, "xor_lanes")
    n = 256
    o32 = np.zeros((6, n), np.uint32)
    o64 = np.zeros((6, n), np.uint64)
    o16 = np.zeros((6, n), np.uint16)
    k[1, n](o32, o64, o16)
    t = np.arange(n, dtype=np.uint64)
    v = (np.uint64(0x9E3779B9) * (t + np.uint64(1))) & np.uint64(0xFFFFFFFF)
    v64 = (v << np.uint64(32)) | (~t & np.uint64(0xFFFFFFFF))
    for i in range(6):
        src = (np.arange(n) ^ (1 << i))
        np.testing.assert_array_equal(o32[i], v[src].astype(np.uint32), err_msg=f"xor {1 << i}")
        np.testing.assert_array_equal(o64[i], v64[src], err_msg=f"xor {1 << i}")
        np.testing.assert_array_equal(o16[i], ((v[src] >> np.uint64(7)) & np.uint64(0xFFFF)).astype(np.uint16),
                                      err_msg=f"xor {1 << i}")
