"""NumPy closed forms of the workloads (TEST INFRASTRUCTURE; see oracle/__init__.py).

Each restates the `reference()` function of the matching reference example
(reference: examples/01_vector_add.py:33, 02_softmax.py:41-44, 03_layernorm.py:64-71,
04_matmul.py:107-108, 05_fused_gelu.py:39-42, 06_rmsnorm.py:40-43,
07_matmul_fused.py:51-56, 08_flash_attention.py:130-140, 09_histogram.py:37-41,
10_cumsum.py:45-51).
"""

from __future__ import annotations

import math

import numpy as np


def vector_add(x, y):
    return x + y


def softmax(x):
    z = x.astype(np.float64)
    z = np.exp(z - z.max(axis=1, keepdims=True))
    return (z / z.sum(axis=1, keepdims=True)).astype(x.dtype)


def rmsnorm(x, w, eps=1e-6):
    z = x.astype(np.float64)
    rstd = 1 / np.sqrt((z * z).mean(axis=1, keepdims=True) + eps)
    return (z * rstd * w.astype(np.float64)).astype(x.dtype)


def layernorm(x, w, b, eps=1e-5):
    z = x.astype(np.float64)
    mean = z.mean(axis=1)
    var = z.var(axis=1)
    rstd = 1 / np.sqrt(var + eps)
    y = (z - mean[:, None]) * rstd[:, None] * w.astype(np.float64) + b.astype(np.float64)
    return y.astype(x.dtype), mean.astype(np.float32), rstd.astype(np.float32)


def matmul(a, b):
    return (a.astype(np.float32) @ b.astype(np.float32)).astype(a.dtype)


_erf = np.vectorize(math.erf, otypes=[np.float64])


def gelu64(y):
    return 0.5 * y * (1 + _erf(y / math.sqrt(2)))


def matmul_bias_gelu(a, b, bias):
    y = a.astype(np.float64) @ b.astype(np.float64) + bias.astype(np.float64)
    return gelu64(y).astype(a.dtype)


def fused_gelu(x, bias, scale):
    y = x.astype(np.float64) * np.float32(scale) + bias.astype(np.float64)
    return gelu64(y).astype(x.dtype)


def attention(q, k, v, causal=False, sm_scale=None):
    """q, k, v as float arrays (any float dtype); returns float64."""
    d = q.shape[-1]
    scale = 1.0 / math.sqrt(d) if sm_scale is None else sm_scale
    s = np.einsum("zhmd,zhnd->zhmn", q.astype(np.float64), k.astype(np.float64)) * scale
    if causal:
        n = q.shape[2]
        s = np.where(np.tril(np.ones((n, n), bool)), s, -np.inf)
    s = np.exp(s - s.max(-1, keepdims=True))
    p = s / s.sum(-1, keepdims=True)
    return np.einsum("zhmn,zhnd->zhmd", p, v.astype(np.float64))


def histogram(x, num_bins, lo, hi):
    xs = x.astype(np.float32)
    b = np.floor((xs - np.float32(lo)) * np.float32(num_bins / (hi - lo))).astype(np.int64)
    b = b[(b >= 0) & (b < num_bins)]
    return np.bincount(b, minlength=num_bins).astype(np.int32)


def cumsum(x, reverse=False):
    out_dtype = np.int32 if x.dtype.kind in "iub" and x.dtype.itemsize < 4 else x.dtype
    acc = out_dtype if x.dtype.kind in "iub" else np.float32
    z = x.astype(acc)
    if reverse:
        return np.flip(np.cumsum(np.flip(z, 1), axis=1, dtype=acc), 1).astype(out_dtype)
    return np.cumsum(z, axis=1, dtype=acc).astype(out_dtype)
