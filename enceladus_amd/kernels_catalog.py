"""The workload specializations that `__graft_entry__.build()` pre-compiles.

Compiling here (no GPU needed: hiprtc cross-compiles gfx950) fills the code-object cache so
GPU runs start without compile latency; it is also the compile-only coverage check.
"""

from __future__ import annotations

import numpy as np


def specs():
    import torch
    from examples import (cumsum, flash_attention, fused_gelu, histogram, layernorm, matmul,
                          matmul_fused, rmsnorm, softmax, vector_add)
    f32 = np.zeros(16, np.float32)
    i32 = np.zeros(16, np.int32)
    f16 = np.zeros(16, np.float16)
    bf = torch.zeros(16, dtype=torch.bfloat16)
    n28 = 1 << 28
    return [
        (vector_add.add_kernel, (f32, f32, f32, 100000), dict(BLOCK=1024)),
        (vector_add.add_kernel, (f32, f32, f32, n28), dict(BLOCK=1024)),
        (softmax.softmax_kernel, (f32, f32, 8192, 8192, 8192), dict(BLOCK=8192)),
        (rmsnorm.rmsnorm_kernel, (f32, f32, f32, 8192, 8192, 8192, 1e-6), dict(BLOCK=8192)),
        (layernorm.layernorm_kernel, (f32,) * 6 + (1000, 1000, 1000, 1e-5), dict(BLOCK=256)),
        (fused_gelu.fused_gelu_kernel, (f32, f32, f32, 1000, 100, 0.5), dict(BLOCK=1024)),
        (cumsum.cumsum_kernel, (i32, i32, 8192, 4096, 4096, 4096),
         dict(REVERSE=False, BLOCK_M=1, BLOCK_N=4096)),
        (histogram.histogram_kernel, (i32, i32, 1 << 26, 0.0, 1.0),
         dict(NUM_BINS=1024, BLOCK=1024)),
        (matmul.matmul_desc_kernel, (f16, f16, f16) + (4096,) * 6, dict(BM=128, BN=128, BK=64)),
        (matmul_fused.matmul_bias_gelu_kernel, (f16,) * 4 + (4096,) * 6,
         dict(BM=128, BN=128, BK=64)),
        (flash_attention.attention_kernel, (bf, bf, bf, bf, 0.088, 4096, 4096 * 128, 128),
         dict(HEAD_DIM=128, BLOCK_M=128, BLOCK_N=64, CAUSAL=True, dot_warps=(4, 1))),
        (flash_attention.attention_kernel, (bf, bf, bf, bf, 0.088, 1024, 1024 * 128, 128),
         dict(HEAD_DIM=128, BLOCK_M=128, BLOCK_N=64, CAUSAL=False, dot_warps=(4, 1))),
    ]


def compile_all(verbose: bool = False) -> int:
    from enceladus_amd.compiler import codegen_hip
    from enceladus_amd.runtime import compile as C
    n = 0
    for kern, args, kw in specs():
        kw = dict(kw)
        dw = kw.pop("dot_warps", None)
        nw = kw.pop("num_warps", 4)
        fn = kern.ir_for(*args, num_warps=nw, dot_warps=dw, **kw)
        gen = codegen_hip.generate(fn, {"dot_warps": dw})
        C.compile_code(gen.source, gen.name)
        n += 1
        if verbose:
            print(f"  compiled {gen.name} (lds {gen.lds_bytes} B)", flush=True)
    return n
