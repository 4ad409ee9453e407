"""Flash-attention forward with online softmax (reference: examples/08_flash_attention.py:30-127)."""

import math

import enceladus
import enceladus.language as tl
from enceladus_amd.configs import attention_configs


@enceladus.jit
def attention_kernel(q_ptr, k_ptr, v_ptr, o_ptr, sm_scale, N_CTX, stride_h, stride_m,
                     HEAD_DIM: tl.constexpr, BLOCK_M: tl.constexpr, BLOCK_N: tl.constexpr,
                     CAUSAL: tl.constexpr):
    start_m = tl.program_id(0)
    base = tl.program_id(1) * stride_h
    q_desc = tl.make_tensor_descriptor(q_ptr + base, [N_CTX, HEAD_DIM], [stride_m, 1],
                                       [BLOCK_M, HEAD_DIM])
    k_desc = tl.make_tensor_descriptor(k_ptr + base, [N_CTX, HEAD_DIM], [stride_m, 1],
                                       [BLOCK_N, HEAD_DIM])
    v_desc = tl.make_tensor_descriptor(v_ptr + base, [N_CTX, HEAD_DIM], [stride_m, 1],
                                       [BLOCK_N, HEAD_DIM])
    o_desc = tl.make_tensor_descriptor(o_ptr + base, [N_CTX, HEAD_DIM], [stride_m, 1],
                                       [BLOCK_M, HEAD_DIM])
    offs_m = start_m * BLOCK_M + tl.arange(0, BLOCK_M)
    offs_n = tl.arange(0, BLOCK_N)
    m_i = tl.full([BLOCK_M], float("-inf"), tl.float32)
    l_i = tl.zeros([BLOCK_M], tl.float32)
    acc = tl.zeros([BLOCK_M, HEAD_DIM], tl.float32)
    qk_scale = sm_scale * 1.4426950408889634
    q = q_desc.load([start_m * BLOCK_M, 0])
    hi = N_CTX
    if CAUSAL:
        hi = tl.minimum((start_m + 1) * BLOCK_M, N_CTX)
    for start_n in range(0, hi, BLOCK_N):
        qk = tl.dot(q, tl.trans(k_desc.load([start_n, 0]))) * qk_scale
        cols = start_n + offs_n
        mask = cols[None, :] < N_CTX
        if CAUSAL:
            mask = mask & (offs_m[:, None] >= cols[None, :])
        qk = tl.where(mask, qk, float("-inf"))
        m_ij = tl.maximum(m_i, tl.max(qk, 1))
        p = tl.exp2(qk - m_ij[:, None])
        alpha = tl.exp2(m_i - m_ij)
        l_i = l_i * alpha + tl.sum(p, 1)
        acc = acc * alpha[:, None]
        acc = tl.dot(p.to(q_desc.dtype), v_desc.load([start_n, 0]), acc)
        m_i = m_ij
    acc = acc / l_i[:, None]
    o_desc.store([start_m * BLOCK_M, 0], acc.to(o_desc.dtype))


def _check(q, k, v):
    if not (tuple(q.shape) == tuple(k.shape) == tuple(v.shape)) or len(q.shape) != 4:
        raise ValueError("q, k, and v must all have shape (batch, heads, seq_len, head_dim)")
    if q.shape[-1] not in (16, 32, 64, 128):
        raise ValueError(f"head_dim must be 16, 32, 64, or 128, not {q.shape[-1]}")


def attention(q, k, v, causal: bool = False, sm_scale=None, o=None, block_m: int = 128,
              block_n: int = 64, num_warps: int = 4):
    _check(q, k, v)
    z, h, n, d = q.shape
    o = enceladus.new_empty(q) if o is None else o
    scale = 1.0 / math.sqrt(d) if sm_scale is None else sm_scale
    grid = (enceladus.cdiv(n, block_m), z * h)
    attention_kernel[grid](q, k, v, o, scale, n, n * d, d, HEAD_DIM=d, BLOCK_M=block_m,
                           BLOCK_N=block_n, CAUSAL=causal, num_warps=num_warps,
                           dot_warps=(num_warps, 1))
    return o


def _prune(configs, named):
    """The candidates `attention_configs` lists for this launch's dtype and head dimension."""
    allowed = attention_configs(named["q_ptr"].dtype, named["HEAD_DIM"])
    return [c for c in configs if c in allowed]


attention_tuned_kernel = enceladus.autotune(
    configs=attention_configs("float16", 128) + attention_configs("float32", 128),
    key=["N_CTX", "HEAD_DIM", "CAUSAL"],
    prune_configs_by={"early_config_prune": _prune},
)(attention_kernel)


def attention_tuned(q, k, v, causal: bool = False, sm_scale=None, o=None):
    """`attention` with the tile the autotuner measures fastest for this shape."""
    _check(q, k, v)
    z, h, n, d = q.shape
    o = enceladus.new_empty(q) if o is None else o
    scale = 1.0 / math.sqrt(d) if sm_scale is None else sm_scale
    grid = lambda meta: (enceladus.cdiv(n, meta["BLOCK_M"]), z * h)  # noqa: E731
    attention_tuned_kernel[grid](q, k, v, o, scale, n, n * d, d, HEAD_DIM=d, CAUSAL=causal)
    return o
