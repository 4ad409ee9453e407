"""GPU parity: each workload kernel on the HIP path against the CPU oracle and the
closed forms, on identical seeded inputs (reference test strategy: tests/conftest.py:102-145,
test_interpreter.py:37-112, test_attention.py:20-49, test_atomics_scans.py:200-227).

Integer kernels (cumsum, histogram) must match bit for bit; vector add is bit-exact (IEEE
add on both sides); float kernels use the tolerances stated in each test.
"""

import numpy as np
import pytest

import enceladus

from oracle import interpreter as O
from oracle import reference_np as R

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)


@pytest.mark.parametrize("n", [1, 1000, 65539, 100_000])
def test_vector_add(n):
    from examples.vector_add import add, add_kernel
    _say(f"vector_add n={n}")
    x = np.random.default_rng(0).standard_normal(n, dtype=np.float32)
    y = np.ones_like(x)
    got = add(x, y)
    want = np.empty_like(x)
    O.run_grid(add_kernel, ((n + 1023) // 1024,), x, y, want, n, BLOCK=1024)
    assert np.array_equal(got, want)
    assert np.array_equal(got, x + y)


@pytest.mark.parametrize("shape", [(64, 1000), (16, 8192), (3, 33)])
def test_softmax(shape):
    from examples.softmax import softmax, softmax_kernel
    _say(f"softmax {shape}")
    x = np.random.default_rng(0).standard_normal(shape, dtype=np.float32)
    got = softmax(x)
    want = np.empty_like(x)
    O.run_grid(softmax_kernel, (shape[0],), want, x, shape[1], shape[1], shape[1],
               BLOCK=1 << (shape[1] - 1).bit_length())
    # outputs are ~1/n: relative 1e-5 with a small absolute floor
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-8)
    np.testing.assert_allclose(got, R.softmax(x), rtol=1e-5, atol=1e-8)


@pytest.mark.parametrize("shape", [(32, 1000), (8, 8192)])
def test_rmsnorm(shape):
    from examples.rmsnorm import rmsnorm
    _say(f"rmsnorm {shape}")
    rng = np.random.default_rng(0)
    x = rng.standard_normal(shape, dtype=np.float32)
    w = np.random.default_rng(1).uniform(0.5, 1.5, shape[1]).astype(np.float32)
    got = rmsnorm(x, w)
    np.testing.assert_allclose(got, R.rmsnorm(x, w), rtol=1e-5, atol=1e-5)


def test_layernorm():
    from examples.layernorm import layernorm
    _say("layernorm 32x1000 block 256")
    rng = np.random.default_rng(0)
    x = rng.standard_normal((32, 1000), dtype=np.float32)
    w = rng.standard_normal(1000, dtype=np.float32)
    b = rng.standard_normal(1000, dtype=np.float32)
    y, mean, rstd = layernorm(x, w, b, block=256)
    ry, rm, rr = R.layernorm(x, w, b)
    np.testing.assert_allclose(y, ry, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(mean, rm, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(rstd, rr, rtol=1e-5, atol=1e-5)


def test_fused_gelu():
    from examples.fused_gelu import fused_gelu
    _say("fused_gelu 64x300")
    rng = np.random.default_rng(0)
    x = rng.standard_normal((64, 300), dtype=np.float32)
    bias = rng.standard_normal(300, dtype=np.float32)
    got = fused_gelu(x, bias, 0.5)
    np.testing.assert_allclose(got, R.fused_gelu(x, bias, 0.5), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("shape,reverse", [((8, 4096), False), ((300, 1000), False),
                                           ((37, 50), True), ((5, 4096), True),
                                           ((64, 256), False)])
def test_cumsum_int32(shape, reverse):
    from examples.cumsum import cumsum, cumsum_kernel
    _say(f"cumsum {shape} reverse={reverse}")
    x = np.random.default_rng(0).integers(-100, 100, shape, dtype=np.int32)
    got = cumsum(x, reverse)
    m, n = shape
    bn = 1 << (n - 1).bit_length()
    bm = max(1, min(16, 4096 // bn))
    want = np.empty_like(x)
    O.run_grid(cumsum_kernel, ((m + bm - 1) // bm,), want, x, m, n, n, n, REVERSE=reverse,
               BLOCK_M=bm, BLOCK_N=bn)
    assert np.array_equal(got, want)
    assert np.array_equal(got, R.cumsum(x, reverse))


@pytest.mark.parametrize("num_warps", [1, 2, 8])
@pytest.mark.parametrize("reverse", [False, True])
def test_cumsum_segmented_rows(num_warps, reverse):
    """Rows longer than one pass of the workgroup's 16-byte vectors are scanned in segments
    joined by carries: 8 segments in one wave (carries through lane shuffles), 4 over two
    waves and 1 over eight (through LDS), two rows per program, both directions."""
    from examples.cumsum import cumsum, cumsum_kernel
    _say(f"cumsum segmented (6, 2000) num_warps={num_warps} reverse={reverse}")
    x = np.random.default_rng(3).integers(-100, 100, (6, 2000), dtype=np.int32)
    got = cumsum(x, reverse, num_warps=num_warps)
    want = np.empty_like(x)
    O.run_grid(cumsum_kernel, (3,), want, x, 6, 2000, 2000, 2000, REVERSE=reverse,
               BLOCK_M=2, BLOCK_N=2048)
    assert np.array_equal(got, want)
    assert np.array_equal(got, R.cumsum(x, reverse))


@pytest.mark.parametrize("n,bins", [(1 << 20, 1024), (100_003, 64), (5000, 4096),
                                    (70_001, 100), (70_001, 6)])
@pytest.mark.parametrize("flush", ["two_level", "atomic"])
def test_histogram(n, bins, flush, monkeypatch):
    from examples.histogram import histogram
    _say(f"histogram n={n} bins={bins} flush={flush}")
    if flush == "atomic":
        monkeypatch.setenv("ENCELADUS_CODEGEN", "priv_flush=atomic")
    x = np.random.default_rng(0).integers(0, bins, n, dtype=np.int32)
    got = histogram(x, bins, 0.0, float(bins))
    assert np.array_equal(got, R.histogram(x, bins, 0.0, float(bins)))
    assert int(got.sum()) == n
    # the launch ran the flush this case names: one level of global atomics, or two
    from examples.histogram import histogram_kernel
    ck = histogram_kernel.warmup(x, got, n, 0.0, 1.0, NUM_BINS=bins, BLOCK=1024)
    assert (ck.gen.flush is None) == (flush == "atomic")


@enceladus.jit
def _two_histograms(x_ptr, h1_ptr, h2_ptr, n, B1: enceladus.language.constexpr,
                    B2: enceladus.language.constexpr, BLOCK: enceladus.language.constexpr):
    tl = enceladus.language
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    x = tl.load(x_ptr + offs, mask=offs < n, other=0)
    a = x % B1
    b = x // 7
    tl.atomic_add(h1_ptr + a, 1, mask=(offs < n) & (a >= 0) & (a < B1))
    tl.atomic_add(h2_ptr + b, 2, mask=(offs < n) & (b >= 0) & (b < B2))


def test_two_privatised_histograms_keep_separate_bins():
    """Two LDS-privatised atomics in one kernel: each has its own bins and its own flush
    (bit-exact against NumPy bincount)."""
    n, b1, b2 = 70_001, 256, 128
    _say(f"two histograms n={n} bins={b1},{b2}")
    x = np.random.default_rng(3).integers(0, 1000, n, dtype=np.int32)
    h1, h2 = np.zeros(b1, np.int32), np.zeros(b2, np.int32)
    _two_histograms[(enceladus.cdiv(n, 1024),)](x, h1, h2, n, B1=b1, B2=b2, BLOCK=1024)
    assert np.array_equal(h1, np.bincount(x % b1, minlength=b1).astype(np.int32))
    want2 = np.bincount(x // 7, minlength=1000)[:b2].astype(np.int32) * 2
    assert np.array_equal(h2, want2)


def _half(shape, seed, scale=1 / 64):
    return (np.random.default_rng(seed).standard_normal(shape, dtype=np.float32) * scale
            ).astype(np.float16)


@pytest.mark.parametrize("m,n,k,bm,bn,bk,nw", [(128, 128, 128, 128, 128, 64, 4),
                                                (256, 256, 256, 128, 128, 64, 4),
                                                (100, 90, 70, 64, 64, 32, 4),
                                                (64, 64, 64, 64, 64, 32, 4),
                                                (256, 128, 512, 64, 128, 64, 4)])
def test_matmul_desc(m, n, k, bm, bn, bk, nw):
    from examples.matmul import matmul_desc
    _say(f"matmul_desc {m}x{n}x{k} tile {bm}x{bn}x{bk}")
    a, b = _half((m, k), 0, 1 / 8), _half((k, n), 1, 1 / 8)
    got = matmul_desc(a, b, bm=bm, bn=bn, bk=bk, num_warps=nw).astype(np.float32)
    want = R.matmul(a, b).astype(np.float32)
    np.testing.assert_allclose(got, want, rtol=2e-3, atol=1e-3)


def test_matmul_pointer_tiles():
    from examples.matmul import matmul
    _say("matmul pointer tiles 100x90x70")
    a, b = _half((100, 70), 0, 1 / 8), _half((70, 90), 1, 1 / 8)
    got = matmul(a, b).astype(np.float32)
    np.testing.assert_allclose(got, R.matmul(a, b).astype(np.float32), rtol=2e-3, atol=1e-3)


def test_matmul_bias_gelu():
    from examples.matmul_fused import matmul_bias_gelu
    _say("matmul_bias_gelu 256x256x128")
    a, b = _half((256, 128), 0, 1 / 8), _half((128, 256), 1, 1 / 8)
    bias = np.random.default_rng(2).standard_normal(256, dtype=np.float32).astype(np.float16)
    got = matmul_bias_gelu(a, b, bias).astype(np.float32)
    want = R.matmul_bias_gelu(a, b, bias).astype(np.float32)
    np.testing.assert_allclose(got, want, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("causal,n,d,bm,bn", [(True, 256, 128, 128, 64), (False, 256, 128, 128, 64),
                                              (True, 200, 64, 64, 32), (False, 128, 32, 64, 32)])
def test_flash_attention_fp16(causal, n, d, bm, bn):
    from examples.flash_attention import attention
    _say(f"flash attention fp16 causal={causal} n={n} d={d}")
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal((1, 2, n, d), dtype=np.float32).astype(np.float16)
               for _ in range(3))
    got = attention(q, k, v, causal, block_m=bm, block_n=bn).astype(np.float64)
    want = R.attention(q, k, v, causal)
    np.testing.assert_allclose(got, want, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("scale", [-0.07, 0.3])
def test_flash_attention_scale_sign(scale):
    """A negative scale compiles the kernel without the max/scale fold (the launch's
    `positive` fact is absent); both signs match the float64 reference."""
    from examples.flash_attention import attention
    _say(f"flash attention fp16 scale={scale}")
    rng = np.random.default_rng(1)
    q, k, v = (rng.standard_normal((1, 2, 256, 64), dtype=np.float32).astype(np.float16)
               for _ in range(3))
    got = attention(q, k, v, True, sm_scale=scale, block_m=64, block_n=32).astype(np.float64)
    want = R.attention(q, k, v, True, sm_scale=scale)
    np.testing.assert_allclose(got, want, rtol=2e-3, atol=2e-3)


@pytest.mark.parametrize("m,n,k,bm,bn,bk,nw", [(512, 512, 256, 256, 256, 64, 4),
                                                (256, 512, 128, 128, 256, 32, 4),
                                                (512, 256, 192, 256, 128, 64, 4),
                                                (512, 512, 128, 256, 256, 64, 8),
                                                (320, 272, 200, 128, 128, 64, 4)])
def test_matmul_gemm_template(m, n, k, bm, bn, bk, nw):
    """The descriptor dot loop on the hand-written MFMA main loop, including ragged edges
    (zero-filled A/B tiles) and K not a multiple of BK."""
    from examples.matmul import matmul_desc
    _say(f"matmul template {m}x{n}x{k} tile {bm}x{bn}x{bk} warps {nw}")
    a, b = _half((m, k), 0, 1 / 8), _half((k, n), 1, 1 / 8)
    got = matmul_desc(a, b, bm=bm, bn=bn, bk=bk, num_warps=nw).astype(np.float32)
    want = R.matmul(a, b).astype(np.float32)
    np.testing.assert_allclose(got, want, rtol=2e-3, atol=1e-3)


@pytest.mark.parametrize("kind", ["template", "pointer"])
def test_matmul_without_transposed_accumulator(kind, monkeypatch):
    """ENCELADUS_CODEGEN=no_acc_transpose (the MFMA's own accumulator orientation) on the
    template main loop and on the generic dot lowering, ragged edges included."""
    from examples.matmul import matmul, matmul_desc
    _say(f"matmul {kind} 320x272x200 no_acc_transpose")
    monkeypatch.setenv("ENCELADUS_CODEGEN", "no_acc_transpose")
    a, b = _half((320, 200), 0, 1 / 8), _half((200, 272), 1, 1 / 8)
    if kind == "template":
        got = matmul_desc(a, b, bm=128, bn=128, bk=64, num_warps=4)
    else:
        got = matmul(a, b)
    want = R.matmul(a, b).astype(np.float32)
    np.testing.assert_allclose(got.astype(np.float32), want, rtol=2e-3, atol=1e-3)


def test_matmul_template_row_tails():
    """Row strides that are multiples of 16 elements around K and N that are not multiples of
    8: the last partial 16-byte chunk of each row is read, not dropped."""
    from examples.matmul import matmul_desc_kernel
    m, n, k, kp, np_ = 256, 250, 100, 112, 256
    _say(f"matmul template row tails {m}x{n}x{k} (row strides {kp}, {np_})")
    a, b = _half((m, kp), 0, 1 / 8), _half((k, np_), 1, 1 / 8)
    c = np.zeros((m, n), np.float16)
    matmul_desc_kernel[(enceladus.cdiv(n, 128), enceladus.cdiv(m, 128))](
        a, b, c, m, n, k, kp, np_, n, BM=128, BN=128, BK=64, num_warps=4)
    want = R.matmul(np.ascontiguousarray(a[:, :k]), np.ascontiguousarray(b[:, :n]))
    np.testing.assert_allclose(c.astype(np.float32), want.astype(np.float32), rtol=2e-3,
                               atol=1e-3)


def test_matmul_template_bf16_torch():
    import torch
    from examples.matmul import matmul_desc
    _say("matmul template bf16 512^3")
    g = torch.Generator().manual_seed(0)
    a = (torch.randn(512, 512, generator=g) / 8).bfloat16()
    b = (torch.randn(512, 512, generator=g) / 8).bfloat16()
    c = matmul_desc(a.cuda(), b.cuda(), bm=256, bn=256, bk=64).float().cpu()
    want = (a.float() @ b.float()).bfloat16().float()
    np.testing.assert_allclose(c.numpy(), want.numpy(), rtol=1.6e-2, atol=1e-2)


# -- Python semantics in compiled kernels (reference: tests/test_frontend.py:112-193) -----

import enceladus.language as tl  # noqa: E402


@enceladus.jit
def _loop_var_after_loop(out_ptr, n):
    i = 100
    for i in range(n):  # noqa: B007 - `i` is read after the loop
        pass
    tl.store(out_ptr, i)


@enceladus.jit
def _negate_mask(out_ptr, x_ptr, BLOCK: tl.constexpr):
    offs = tl.arange(0, BLOCK)
    m = tl.load(x_ptr + offs) > 0
    tl.store(out_ptr + offs, -m + 10 * ~m)


@enceladus.jit
def _unsigned_loop_bound(out_ptr, n_ptr):
    n = tl.load(n_ptr)
    count = 0
    for _ in range(0, n, 1_000_000_000):
        count += 1
    tl.store(out_ptr, count)


@enceladus.jit
def _chained_compare(out_ptr, x_ptr, a, b):
    tl.store(out_ptr, (a < b <= tl.load(x_ptr)).to(tl.int32))


@enceladus.jit
def _where_pointers(out_ptr, x_ptr, BLOCK: tl.constexpr):
    offs = tl.arange(0, BLOCK)
    tl.store(out_ptr + offs, tl.load(tl.where(offs % 2 == 0, x_ptr + offs, x_ptr + 50 + offs)))


@enceladus.jit
def _scalar_or(out_ptr, a, b):
    tl.store(out_ptr, a or b)
    tl.store(out_ptr + 1, a and b)


_VALS = np.arange(-32, 96, dtype=np.int32)


@pytest.mark.parametrize("case", ["loop_after", "loop_empty", "negate_mask", "uint_bound",
                                  "chained", "chained_short", "where_ptrs", "or_and",
                                  "or_and_zero"])
def test_python_semantics(case):
    _say(f"semantics {case}")
    i32 = np.zeros(2, np.int32)
    if case == "loop_after":
        _loop_var_after_loop[(1,)](i32, 5)
        assert i32[0] == 4
    elif case == "loop_empty":
        _loop_var_after_loop[(1,)](i32, 0)
        assert i32[0] == 100
    elif case == "negate_mask":
        out = np.zeros(64, np.int32)
        _negate_mask[(1,)](out, _VALS, BLOCK=64)
        assert np.array_equal(out, np.where(_VALS[:64] > 0, -1, 10))
    elif case == "uint_bound":
        _unsigned_loop_bound[(1,)](i32, np.array([3_000_000_000], np.uint32))
        assert i32[0] == 3
    elif case in ("chained", "chained_short"):
        a, b = (1, 2) if case == "chained" else (3, 2)
        _chained_compare[(1,)](i32, _VALS[40:], a, b)
        assert i32[0] == (1 if case == "chained" else 0)
    elif case == "where_ptrs":
        out = np.zeros(64, np.int32)
        _where_pointers[(1,)](out, _VALS, BLOCK=64)
        assert np.array_equal(out, np.where(np.arange(64) % 2 == 0, _VALS[:64], _VALS[50:114]))
    else:
        a = 0 if case == "or_and_zero" else 6
        _scalar_or[(1,)](i32, a, 9)
        assert list(i32) == [a or 9, a and 9]
