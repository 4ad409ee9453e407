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
