"""Matmul with a fused bias + GELU epilogue (reference: examples/07_matmul_fused.py:17-48)."""

import enceladus
import enceladus.language as tl
from enceladus_amd.configs import matmul_configs


@enceladus.jit
def matmul_bias_gelu_kernel(a_ptr, b_ptr, bias_ptr, c_ptr, M, N, K, stride_am, stride_bk,
                            stride_cm, BM: tl.constexpr, BN: tl.constexpr,
                            BK: tl.constexpr):
    pid_n, pid_m = tl.program_id(0), tl.program_id(1)
    a = tl.make_tensor_descriptor(a_ptr, [M, K], [stride_am, 1], [BM, BK])
    b = tl.make_tensor_descriptor(b_ptr, [K, N], [stride_bk, 1], [BK, BN])
    c = tl.make_tensor_descriptor(c_ptr, [M, N], [stride_cm, 1], [BM, BN])
    acc = tl.zeros((BM, BN), dtype=tl.float32)
    for k in range(0, K, BK):
        acc = tl.dot(a.load([pid_m * BM, k]), b.load([k, pid_n * BN]), acc)
    cols = pid_n * BN + tl.arange(0, BN)
    bias = tl.load(bias_ptr + cols, mask=cols < N, other=0.0).to(tl.float32)
    y = acc + bias[None, :]
    y = 0.5 * y * (1.0 + tl.erf(y * 0.7071067811865476))
    c.store([pid_m * BM, pid_n * BN], y.to(c.dtype))


def matmul_bias_gelu(a, b, bias, c=None, bm: int = 128, bn: int = 128, bk: int = 64,
                     num_warps: int = 4):
    (m, k), (_, n) = a.shape, b.shape
    if c is None:
        c = enceladus.new_empty(a, (m, n))
    grid = (enceladus.cdiv(n, bn), enceladus.cdiv(m, bm))
    matmul_bias_gelu_kernel[grid](a, b, bias, c, m, n, k, k, n, n, BM=bm, BN=bn, BK=bk,
                                  num_warps=num_warps)
    return c


def _configs_for_dtype(configs, named):
    allowed = matmul_configs(named["a_ptr"].dtype)
    return [c for c in configs if c in allowed]


# Not in the reference's example: the fused kernel under the matmul candidates, so the
# BASELINE's fused variant is tuned over the same BM/BN/BK sweep as the plain matmul.
matmul_bias_gelu_tuned = enceladus.autotune(
    configs=matmul_configs("float16") + matmul_configs("float32"),
    key=["M", "N", "K"],
    prune_configs_by={"early_config_prune": _configs_for_dtype},
)(matmul_bias_gelu_kernel)


def matmul_bias_gelu_autotuned(a, b, bias, c=None):
    """`matmul_bias_gelu` with the tile the autotuner measures fastest for this shape."""
    (m, k), (_, n) = a.shape, b.shape
    if c is None:
        c = enceladus.new_empty(a, (m, n))
    grid = lambda meta: (enceladus.cdiv(n, meta["BN"]), enceladus.cdiv(m, meta["BM"]))  # noqa: E731
    matmul_bias_gelu_tuned[grid](a, b, bias, c, m, n, k, k, n, n)
    return c
