"""The workload specializations that `__graft_entry__.build()` pre-compiles.

Compiling here (no GPU needed: hiprtc cross-compiles gfx950) fills the code-object cache so
GPU runs start without compile latency; it is also the compile-only coverage check. The
list is every variant of the benchmark's workload table (`examples/workloads.py`, with
torch "meta" tensors standing in for the full-size buffers: same shapes, dtypes and
argument facts, no memory) plus the example wrappers' own default launches.
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


def table_specs():
    """(kernel, args, options) of every variant in the benchmark's workload table."""
    import torch
    from examples import workloads as W
    out = []
    for wl in W.table().values():
        bufs = {}
        host_shapes = _input_shapes(wl)
        for k, (shape, dt) in host_shapes.items():
            bufs[k] = torch.empty(shape, dtype=getattr(torch, dt), device="meta")
        for k, (shape, dt) in wl.outputs.items():
            bufs[k] = torch.empty(shape, dtype=getattr(torch, dt), device="meta")
        for v in wl.variants:
            _, args = wl.args(bufs, v)
            out.append((wl.kernel(), args, v.options()))
    return out


def _input_shapes(wl) -> dict:
    """Input names -> (shape, torch dtype name) of a workload, without generating data."""
    from examples import workloads as W
    if wl.name == "vector_add":
        return {"x": ((W.VADD_N,), "float32"), "y": ((W.VADD_N,), "float32")}
    if wl.name in ("softmax", "copy_rows"):
        return {"x": ((W.ROWS, W.COLS), "float32")}
    if wl.name in ("copy_flat", "read_flat"):
        return {"x": ((W.ROWS * W.COLS,), "float32")}
    if wl.name == "fill_flat":
        return {}
    if wl.name == "rmsnorm":
        return {"x": ((W.ROWS, W.COLS), "float32"), "w": ((W.COLS,), "float32")}
    if wl.name.startswith("matmul"):
        d = {"a": ((W.MM, W.MM), "float16"), "b": ((W.MM, W.MM), "float16")}
        if wl.name == "matmul_gelu":
            d["bias"] = ((W.MM,), "float16")
        return d
    if wl.name.startswith("attention"):
        n = wl.outputs["o"][0][2]
        return {k: ((W.ATT_B, W.ATT_H, n, W.ATT_D), "bfloat16") for k in "qkv"}
    if wl.name == "histogram":
        return {"x": ((W.HIST_N,), "int32")}
    if wl.name == "cumsum":
        return {"x": ((W.SCAN_ROWS, W.SCAN_COLS), "int32")}
    raise KeyError(wl.name)


def compile_all(verbose: bool = False) -> int:
    """Generates and hiprtc-compiles every listed specialization (hiprtc runs on a thread
    pool: each program is its own hiprtc object, and ctypes releases the GIL)."""
    from concurrent.futures import ThreadPoolExecutor

    jobs = []
    seen = set()
    for kern, args, kw in specs() + table_specs():
        kw = dict(kw)
        dw = kw.pop("dot_warps", None)
        nw = kw.pop("num_warps", 4)
        vals = kern._bind(args, kw)
        types, facts, consts = kern.specialize(vals)
        key = kern._key(types, facts, consts, nw, dw)
        if (kern, key) in seen:
            continue
        seen.add((kern, key))
        jobs.append((kern, types, facts, consts, nw, dw))

    def one(job):
        # the launch path's own compile: also records the specialization-cache entry
        kern, types, facts, consts, nw, dw = job
        return kern._compile_for(types, facts, consts, nw, dw).ck

    with ThreadPoolExecutor(max_workers=8) as ex:
        for ck in ex.map(one, jobs):
            if verbose:
                print(f"  compiled {ck.name} (lds {ck.lds_bytes} B)", flush=True)
    return len(jobs)
