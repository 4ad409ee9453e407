"""Pins the CPU oracle (oracle/interpreter.py) against things other than its own formulas:
the examples' NumPy closed forms, brute force on tiny inputs, invariants, torch's bf16 RNE
cast, and hand-picked conversion edge cases. CPU only."""

import math

import numpy as np
import pytest

from oracle import interpreter as O
from oracle import reference_np as R


def test_vector_add_closed_form():
    from examples.vector_add import add_kernel
    n = 5000
    x = np.random.default_rng(0).standard_normal(n, dtype=np.float32)
    y = np.ones_like(x)
    out = np.empty_like(x)
    O.run_grid(add_kernel, (5,), x, y, out, n, BLOCK=1024)
    assert np.array_equal(out, x + y)


def test_softmax_and_rmsnorm_closed_form():
    from examples.rmsnorm import rmsnorm_kernel
    from examples.softmax import softmax_kernel
    x = np.random.default_rng(0).standard_normal((4, 300), dtype=np.float32)
    out = np.empty_like(x)
    O.run_grid(softmax_kernel, (4,), out, x, 300, 300, 300, BLOCK=512)
    np.testing.assert_allclose(out, R.softmax(x), rtol=1e-5, atol=1e-8)
    assert np.allclose(out.sum(1), 1.0, atol=1e-5)
    w = np.random.default_rng(1).uniform(0.5, 1.5, 300).astype(np.float32)
    O.run_grid(rmsnorm_kernel, (4,), x, w, out, 300, 300, 300, 1e-6, BLOCK=512)
    np.testing.assert_allclose(out, R.rmsnorm(x, w), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("reverse", [False, True])
def test_cumsum_exact_and_invariant(reverse):
    from examples.cumsum import cumsum_kernel
    x = np.random.default_rng(0).integers(-100, 100, (6, 70), dtype=np.int32)
    out = np.empty_like(x)
    O.run_grid(cumsum_kernel, (6,), out, x, 6, 70, 70, 70, REVERSE=reverse, BLOCK_M=1,
               BLOCK_N=128)
    assert np.array_equal(out, R.cumsum(x, reverse))
    # invariant: first differences recover the input
    d = np.diff(out, axis=1, prepend=0) if not reverse else \
        -np.diff(out, axis=1, append=0)
    assert np.array_equal(d, x)


def test_histogram_exact_and_counts():
    from examples.histogram import histogram_kernel
    x = np.random.default_rng(0).integers(0, 100, 3000, dtype=np.int32)
    h = np.zeros(64, np.int32)
    O.run_grid(histogram_kernel, (3,), x, h, 3000, 0.0, 1.0, NUM_BINS=64, BLOCK=1024)
    assert np.array_equal(h, R.histogram(x, 64, 0.0, 64.0))
    assert int(h.sum()) == int((x < 64).sum())   # out-of-range values are skipped


def test_dot_brute_force():
    import examples.matmul as mm
    rng = np.random.default_rng(3)
    a = rng.integers(-3, 4, (32, 48)).astype(np.float16)
    b = rng.integers(-3, 4, (48, 32)).astype(np.float16)
    c = np.empty((32, 32), np.float16)
    O.run_grid(mm.matmul_desc_kernel, (1, 1), a, b, c, 32, 32, 48, 48, 32, 32, BM=32, BN=32,
               BK=16)
    brute = np.zeros((32, 32))
    for i in range(32):
        for j in range(32):
            brute[i, j] = sum(float(a[i, k]) * float(b[k, j]) for k in range(48))
    assert np.array_equal(c.astype(np.float64), brute)   # small integers: exact


def test_descriptor_zero_padding():
    import examples.matmul as mm
    rng = np.random.default_rng(0)
    a = rng.standard_normal((40, 20)).astype(np.float32)
    b = rng.standard_normal((20, 24)).astype(np.float32)
    c = np.full((40, 24), 7.0, np.float32)
    O.run_grid(mm.matmul_desc_kernel, (1, 2), a, b, c, 40, 24, 20, 20, 24, 24, BM=32, BN=32,
               BK=16)
    np.testing.assert_allclose(c, a @ b, rtol=1e-5, atol=1e-5)


def test_attention_closed_form():
    from examples.flash_attention import attention_kernel
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal((1, 2, 64, 32), dtype=np.float32) for _ in range(3))
    for causal in (False, True):
        o = np.empty_like(q)
        O.run_grid(attention_kernel, (2, 2), q, k, v, o, 32 ** -0.5, 64, 64 * 32, 32,
                   HEAD_DIM=32, BLOCK_M=32, BLOCK_N=16, CAUSAL=causal)
        np.testing.assert_allclose(o, R.attention(q, k, v, causal), rtol=1e-4, atol=1e-5)


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    vals = np.concatenate([np.random.default_rng(0).standard_normal(10000, dtype=np.float32),
                           np.array([1.00390625, 1.01171875, -3.0078125, 65504.0, 1e-40,
                                     np.inf, -np.inf], np.float32)])
    mine = O.bf16_round(vals)
    ref = torch.from_numpy(vals).to(torch.bfloat16).float().numpy()
    assert np.array_equal(mine, ref)


def test_float_to_int_edges():
    f = np.array([np.nan, np.inf, -np.inf, 3.9, -3.9, 3e9, -3e9, 2147483520.0], np.float32)
    assert O.float_to_int(f, O.int32).tolist() == [0, 2147483647, -2147483648, 3, -3,
                                                   2147483647, -2147483648, 2147483520]
    assert O.float_to_int(np.array([300.0, -5.0], np.float32), O.uint8).tolist() == [255, 0]
    assert O.float_to_int(np.array([np.inf, 2.0 ** 64], np.float32), O.int64).tolist() == [0, 0]


def test_promotion_rules_known_answers():
    c = O.compute_dtype
    assert c("add", O.float16, O.bfloat16) is O.float32
    assert c("add", O.int32, 1.5) is O.float32
    assert c("add", O.float16, 2) is O.float16
    assert c("div", O.int32, O.int32) is O.float32
    assert c("add", O.int32, O.uint32) is O.uint32
    assert c("add", O.int64, O.uint32) is O.int64
    assert c("add", O.int1, O.int1) is O.int32
    with pytest.raises(TypeError):
        c("floordiv", O.float32, 2)


def test_c_division_truncates():
    a = O.to_tile(np.array([-7, 7, -7, 7], np.int32))
    b = O.to_tile(np.array([2, -2, -2, 0], np.int32))
    assert O.binary("floordiv", a, b).data.tolist() == [-3, -3, 3, 7]
    assert O.binary("mod", a, b).data.tolist() == [-1, 1, -1, 0]


def test_colliding_atomics_return_old_values_in_row_major_order():
    buf = np.zeros(2, np.int32)
    p = O._pointer(buf, O.int32)
    old = O.atomic_add(p + O.to_tile(np.array([0, 1, 0, 0], np.int32)), 1)
    assert buf.tolist() == [3, 1]
    assert old.data.tolist() == [0, 0, 1, 2]


def test_layernorm_closed_form():
    from examples.layernorm import layernorm_kernel
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 300), dtype=np.float32)
    w, b = (rng.standard_normal(300, dtype=np.float32) for _ in range(2))
    y = np.empty_like(x)
    mean, rstd = np.empty(3, np.float32), np.empty(3, np.float32)
    O.run_grid(layernorm_kernel, (3,), x, y, w, b, mean, rstd, 300, 300, 300, 1e-5, BLOCK=128)
    ry, rm, rr = R.layernorm(x, w, b)
    np.testing.assert_allclose(y, ry, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(mean, rm, rtol=1e-5, atol=1e-6)


def test_gelu_closed_form():
    from examples.fused_gelu import fused_gelu_kernel
    rng = np.random.default_rng(0)
    x = rng.standard_normal((8, 30), dtype=np.float32)
    bias = rng.standard_normal(30, dtype=np.float32)
    out = np.empty_like(x)
    O.run_grid(fused_gelu_kernel, (1,), x, bias, out, 240, 30, 0.5, BLOCK=256)
    np.testing.assert_allclose(out, R.fused_gelu(x, bias, 0.5), rtol=1e-5, atol=1e-6)
    assert math.isclose(float(R.gelu64(np.array([1.0]))[0]), 0.8413447460685429, rel_tol=1e-12)


# -- math functions at points the mathematics fixes -----------------------------------
# Each value is exact in float32 (or the function's correctly rounded result is), so a
# swapped function (sin for cos, log for log2, tanh for sigmoid), a dropped sign or a
# wrong base fails here.

def _un(op, vals):
    return O.unary(op, O.to_tile(np.array(vals, np.float32))).data.tolist()


def test_math_functions_at_exact_points():
    inf, nan = math.inf, math.nan
    assert _un("sin", [0.0, -0.0]) == [0.0, -0.0]
    assert math.copysign(1, _un("sin", [-0.0])[0]) == -1
    assert _un("sin", [np.float32(math.pi / 2)]) == [1.0]
    assert _un("sin", [np.float32(-math.pi / 2)]) == [-1.0]
    assert _un("cos", [0.0, -0.0]) == [1.0, 1.0]
    assert abs(_un("cos", [np.float32(math.pi)])[0] + 1.0) < 1e-7
    assert _un("tanh", [0.0, inf, -inf, 20.0, -20.0]) == [0.0, 1.0, -1.0, 1.0, -1.0]
    assert _un("sigmoid", [0.0, inf, -inf, 100.0]) == [0.5, 1.0, 0.0, 1.0]
    assert _un("log", [1.0, 0.0, inf]) == [0.0, -inf, inf]
    assert math.isnan(_un("log", [-1.0])[0])
    assert _un("log2", [1.0, 2.0, 8.0, 0.5, 2.0 ** -20, 2.0 ** 100, 0.0]) == \
        [0.0, 1.0, 3.0, -1.0, -20.0, 100.0, -inf]
    assert math.isnan(_un("log2", [-2.0])[0]) and math.isnan(_un("sin", [inf])[0])
    assert _un("exp2", [0.0, 3.0, -2.0, 10.0]) == [1.0, 8.0, 0.25, 1024.0]
    assert _un("exp", [0.0, -inf]) == [1.0, 0.0]
    assert _un("sqrt", [4.0, 0.25, 0.0]) == [2.0, 0.5, 0.0]
    assert _un("rsqrt", [4.0, 0.25]) == [0.5, 2.0]
    assert _un("floor", [-2.5, 2.5, -0.0]) == [-3.0, 2.0, -0.0]
    assert _un("ceil", [-2.5, 2.5]) == [-2.0, 3.0]
    assert _un("erf", [0.0, inf, -inf]) == [0.0, 1.0, -1.0]


def test_math_functions_satisfy_identities():
    """Identities between functions on random float32 inputs, to float32 tolerance:
    sin² + cos² = 1, tanh(x) = 2·sigmoid(2x) − 1, log2(x) = log(x) / ln 2,
    exp(log x) = x, sin(−x) = −sin(x), cos(−x) = cos(x)."""
    x = np.random.default_rng(3).uniform(-6, 6, 4096).astype(np.float32)
    p = np.abs(x) + np.float32(0.01)
    s, c = np.array(_un("sin", x)), np.array(_un("cos", x))
    np.testing.assert_allclose(s * s + c * c, 1.0, atol=1e-6)
    np.testing.assert_allclose(_un("tanh", x), 2 * np.array(_un("sigmoid", 2 * x)) - 1,
                               atol=2e-6)
    np.testing.assert_allclose(_un("log2", p), np.array(_un("log", p)) / math.log(2),
                               rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(_un("exp", _un("log", p)), p, rtol=2e-6)
    assert _un("sin", -x) == [-v for v in _un("sin", x)]
    assert _un("cos", -x) == _un("cos", x)


# -- argmax / argmin: first index of the NaN-ignoring extreme ----------------------------

def _brute_arg(row, kind):
    """Pure-Python restatement of the rule (reference language/ops.py:962-968): the first
    index whose value equals the NaN-ignoring max (min); an all-NaN row gives 0."""
    vals = [v for v in row if not (isinstance(v, float) and math.isnan(v))]
    if not vals:
        return 0
    best = max(vals) if kind == "argmax" else min(vals)
    return next(i for i, v in enumerate(row) if v == best)


def test_argmax_argmin_ties_and_nans():
    nan = math.nan
    rows = [[3.0, 1.0, 3.0, 2.0], [nan, 2.0, 5.0, nan], [nan, nan, nan, nan],
            [1.0, nan, 1.0, 0.5], [-0.0, 0.0, -1.0, -1.0], [-math.inf, -math.inf, nan, 7.0],
            [2.0, 2.0, 2.0, 2.0], [nan, -3.0, -3.0, 4.0]]
    a = np.array(rows, np.float32)
    for kind, fn in (("argmax", O.argmax), ("argmin", O.argmin)):
        got = fn(O.to_tile(a), 1).data.tolist()
        want = [_brute_arg([float(v) for v in r], kind) for r in a]
        assert got == want, kind
        col = fn(O.to_tile(a.T.copy()), 0).data.tolist()
        assert col == want
    # the value tl.max returns and the argmax index agree, NaNs ignored
    mx = O.max(O.to_tile(a), 1).data
    idx = O.argmax(O.to_tile(a), 1).data
    for r, m, i in zip(a, mx, idx):
        if not np.all(np.isnan(r)):
            assert r[i] == m
    ints = np.array([[5, 9, 9, 1], [-4, -4, -9, -9]], np.int32)
    assert O.argmax(O.to_tile(ints), 1).data.tolist() == [1, 0]
    assert O.argmin(O.to_tile(ints), 1).data.tolist() == [3, 2]


# -- shifts: NumPy's rules, which the reference interpreter inherits ------------------------

@pytest.mark.parametrize("dt", ["int8", "int16", "int32", "int64", "uint8", "uint16",
                                "uint32", "uint64"])
def test_shift_counts_follow_numpy(dt):
    """The reference shifts with `np.left_shift`/`np.right_shift` on counts cast to the
    value's dtype (interpreter/interp.py:622-623). For every count in [-70, 300) (cast as
    the compute dtype casts it), the oracle equals NumPy, and the out-of-range rule is the
    closed form: left shifts give 0, right shifts the sign fill."""
    npdt = np.dtype(dt)
    info = np.iinfo(npdt)
    x = np.array([info.min, info.max, 0, 1, 5, info.min + 3, info.max // 3], npdt)
    for c in range(-70, 300):
        y = np.full(x.shape, c, np.int64).astype(npdt)
        ot = O.to_tile(x)
        oc = O.to_tile(y)
        sl = O.binary("shl", ot, oc).data
        sr = O.binary("shr", ot, oc).data
        assert np.array_equal(sl, np.left_shift(x, y)), (dt, c)
        assert np.array_equal(sr, np.right_shift(x, y)), (dt, c)
        cnt = int(y[0])
        if cnt < 0 or cnt >= info.bits:
            assert np.all(sl == 0)
            fill = np.where(x < 0, -1, 0).astype(npdt) if info.min < 0 else np.zeros_like(x)
            assert np.array_equal(sr, fill)
