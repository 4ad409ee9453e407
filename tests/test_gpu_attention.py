"""Flash attention across the reference's shape cases, and the `tl.dot` paths attention
relies on: an accumulator that feeds a second dot, and row reductions of a dot result
(reference test strategy: tests/test_attention.py:14-160).

Inputs are ragged (37, 100 rows), head dims 32-128, causal and not, fp16/fp32/bf16, and
tile configs from one wave to eight. The bar is the reference's: fp16 atol 2e-3 (P is
rounded to the input type before the second dot), fp32 1e-5 scaled for the TF32-free fp32
path, bf16 2e-2, against the float64 closed form.
"""

import numpy as np
import pytest

import enceladus
import enceladus.language as tl
from oracle import reference_np as R

pytestmark = pytest.mark.gpu

# (dtype, seq_len, head_dim, causal, (BLOCK_M, BLOCK_N, num_warps))
CASES = [
    ("float16", 64, 64, False, (32, 32, 1)),
    ("float16", 64, 64, True, (32, 32, 1)),
    ("float16", 100, 64, False, (64, 32, 2)),
    ("float16", 100, 64, True, (64, 32, 2)),
    ("float16", 100, 128, False, (64, 32, 2)),
    ("float16", 100, 128, True, (32, 16, 1)),
    ("float16", 100, 64, True, (64, 16, 2)),
    ("float16", 37, 32, False, (32, 32, 1)),
    ("float16", 300, 128, True, (256, 128, 8)),
    ("float32", 100, 128, True, (32, 32, 1)),
    ("bfloat16", 100, 64, False, (32, 16, 1)),
    ("bfloat16", 300, 128, True, (128, 64, 4)),
    # one LDS stage each for K and V, the exponentials behind the mid barrier (split stages)
    ("bfloat16", 300, 128, True, (128, 128, 4)),
    ("float16", 300, 128, False, (128, 128, 4)),
]


@pytest.mark.parametrize("dtype,n,d,causal,cfg", CASES, ids=str)
def test_flash_attention(dtype, n, d, causal, cfg):
    import torch
    from examples.flash_attention import attention
    print(f"[case] attention {dtype} n={n} d={d} causal={causal} cfg={cfg}", flush=True)
    rng = np.random.default_rng(n + d)
    q32, k32, v32 = (rng.standard_normal((2, 2, n, d)).astype(np.float32) for _ in range(3))
    td = getattr(torch, dtype)
    q, k, v = (torch.from_numpy(x).to(td).cuda() for x in (q32, k32, v32))
    bm, bn, nw = cfg
    scale = 0.3 if causal else None
    o = attention(q, k, v, causal, scale, block_m=bm, block_n=bn, num_warps=nw)
    torch.cuda.synchronize()
    qf, kf, vf = (x.cpu().float().numpy() for x in (q, k, v))
    want = R.attention(qf, kf, vf, causal, scale)
    got = o.cpu().float().numpy()
    err = np.abs(got - want)
    print(f"[case] max abs error {err.max():.3g}, max relative {(err / np.abs(want)).max():.3g}",
          flush=True)
    atol = {"float16": 2e-3, "float32": 1e-5, "bfloat16": 2e-2}[dtype]
    np.testing.assert_allclose(got, want, atol=atol, rtol=atol)


@pytest.mark.parametrize("mode", ["no_split_sink", "no_split_stages", "no_acc_transpose"])
@pytest.mark.parametrize("causal", [True, False])
def test_flash_attention_emitter_switches(mode, causal, monkeypatch):
    """The orders and layouts the emitter switches restore stay correct (ragged length,
    the split-stage tile)."""
    import torch
    from examples.flash_attention import attention
    print(f"[case] attention bf16 n=300 d=128 causal={causal} 128x128/4 mode={mode}", flush=True)
    monkeypatch.setenv("ENCELADUS_CODEGEN", mode)
    rng = np.random.default_rng(300)
    q32, k32, v32 = (rng.standard_normal((1, 2, 300, 128)).astype(np.float32) for _ in range(3))
    q, k, v = (torch.from_numpy(x).to(torch.bfloat16).cuda() for x in (q32, k32, v32))
    o = attention(q, k, v, causal, 0.3, block_m=128, block_n=128, num_warps=4)
    torch.cuda.synchronize()
    qf, kf, vf = (x.cpu().float().numpy() for x in (q, k, v))
    want = R.attention(qf, kf, vf, causal, 0.3)
    np.testing.assert_allclose(o.cpu().float().numpy(), want, atol=2e-2, rtol=2e-2)


@enceladus.jit
def _two_dots(a_ptr, b_ptr, c_ptr, o_ptr, M, K, N1, N2, BM: tl.constexpr, BK: tl.constexpr,
              BN1: tl.constexpr, BN2: tl.constexpr):
    a_d = tl.make_tensor_descriptor(a_ptr, [M, K], [K, 1], [BM, BK])
    b_d = tl.make_tensor_descriptor(b_ptr, [K, N1], [N1, 1], [BK, BN1])
    c_d = tl.make_tensor_descriptor(c_ptr, [N1, N2], [N2, 1], [BN1, BN2])
    o_d = tl.make_tensor_descriptor(o_ptr, [M, N2], [N2, 1], [BM, BN2])
    a = a_d.load([0, 0])
    acc = tl.zeros((BM, BN2), tl.float32)
    for n in range(0, N1, BN1):
        p = tl.dot(a, b_d.load([0, n]))
        acc = tl.dot(p.to(tl.float16), c_d.load([n, 0]), acc)
    o_d.store([0, 0], acc)


@pytest.mark.parametrize("dot_warps", [(4, 1), (2, 2)])
def test_accumulator_feeds_a_second_dot(dot_warps):
    print(f"[case] two dots {dot_warps}", flush=True)
    rng = np.random.default_rng(1)
    m, k, n1, n2 = 50, 20, 70, 45            # ragged everywhere; three steps over N1
    a, b, c = (rng.standard_normal(s).astype(np.float16) for s in ((m, k), (k, n1), (n1, n2)))
    o = np.empty((m, n2), np.float32)
    _two_dots[(1,)](a, b, c, o, m, k, n1, n2, BM=64, BK=32, BN1=32, BN2=64,
                    dot_warps=dot_warps)
    p = (a.astype(np.float32) @ b.astype(np.float32)).astype(np.float16)
    np.testing.assert_allclose(o, p.astype(np.float32) @ c.astype(np.float32), atol=2e-2,
                               rtol=2e-3)


@enceladus.jit
def _dot_row_max(a_ptr, b_ptr, out_ptr, M, N, K, BM: tl.constexpr, BN: tl.constexpr,
                 BK: tl.constexpr):
    a_d = tl.make_tensor_descriptor(a_ptr, [M, K], [K, 1], [BM, BK])
    b_d = tl.make_tensor_descriptor(b_ptr, [K, N], [N, 1], [BK, BN])
    s = tl.dot(a_d.load([0, 0]), b_d.load([0, 0]))
    cols = tl.arange(0, BN)
    s = tl.where(cols[None, :] < N, s, float("-inf"))
    rows = tl.arange(0, BM)
    tl.store(out_ptr + rows, tl.max(s, 1), mask=rows < M)


@pytest.mark.parametrize("dot_warps", [(4, 1), (2, 2)])
def test_accumulator_row_reduction(dot_warps):
    print(f"[case] dot row max {dot_warps}", flush=True)
    rng = np.random.default_rng(2)
    m, n, k = 60, 30, 16
    a = rng.standard_normal((m, k)).astype(np.float16)
    b = rng.standard_normal((k, n)).astype(np.float16)
    out = np.empty(m, np.float32)
    _dot_row_max[(1,)](a, b, out, m, n, k, BM=64, BN=32, BK=16, dot_warps=dot_warps)
    np.testing.assert_allclose(out, (a.astype(np.float32) @ b.astype(np.float32)).max(1),
                               atol=1e-4)


# -- matmul shapes (reference: tests/test_interpreter.py:73-88, 730-770) ------------------

SHAPES = [(64, 64, 64), (513, 513, 513), (1000, 300, 777), (2048, 2048, 2048)]


@pytest.mark.parametrize("variant", ["desc", "pointer"])
@pytest.mark.parametrize("mkn", SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_matmul_shapes(dtype, mkn, variant):
    import torch
    from examples.matmul import matmul, matmul_desc
    print(f"[case] matmul {variant} {mkn} {dtype}", flush=True)
    m, k, n = mkn
    g = torch.Generator().manual_seed(m + k + n)
    td = getattr(torch, dtype)
    a = torch.randn(m, k, generator=g).to(td).cuda()
    b = torch.randn(k, n, generator=g).to(td).cuda()
    c = (matmul_desc if variant == "desc" else matmul)(a, b)
    torch.cuda.synchronize()
    want = a.double().cpu() @ b.double().cpu()
    # fp32 operands go through MFMA in fp32; half outputs round once to their type
    tol = {"float32": 1e-4 * k ** 0.5, "float16": 2e-3 * k ** 0.5 / 8,
           "bfloat16": 1.6e-2 * k ** 0.5 / 8}[dtype]
    torch.testing.assert_close(c.double().cpu(), want, atol=tol, rtol=tol)
