"""Benchmark of the north-star workloads on one MI355X.

Prints one JSON line (the driver's contract). The headline workload is BASELINE config 2
(`configs[1]`): row softmax over fp32 [4096, 8192]; `value` is its whole-job GB/s with
inputs resident in HBM. The same run measures every other config (vector add 2^28,
RMSNorm, fp16 4096^3 matmul and + bias + GELU, bf16 flash attention causal 4096 and
non-causal 1024, int32 histogram and cumsum) and reports them under "workloads", each with
its roofline fraction. Kernel times come from HIP events recorded on the launch stream
around the timed launches; inputs rotate over several buffer sets totalling > 512 MB so
the 256 MB Infinity Cache can't serve them.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME[,NAME]]
                       [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
os.environ.setdefault("ENCELADUS_CACHE_DIR", os.path.join(ROOT, ".ek_cache"))

HBM_PEAK = 8.0e12          # bytes/s (MI355X HBM3E)
MFMA_PEAK_F16 = 2.5e15     # dense fp16/bf16 FLOP/s
GIB = 1 << 30


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Timer:
    """HIP-event timing on torch's current stream (the stream kernels launch on)."""

    def __init__(self, torch):
        self.torch = torch

    def run(self, launches, steps, warmup):
        torch = self.torch
        for i in range(warmup):
            launches[i % len(launches)]()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for i in range(steps):
            launches[i % len(launches)]()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / steps  # ms per launch


def make_launch(jfn, grid, args, num_warps=4, dot_warps=None, **constexprs):
    import ctypes
    from enceladus_amd.runtime import hip
    vals = jfn._bind(args, constexprs)
    lc = jfn._lookup(vals, num_warps, dot_warps)
    packed = []
    for n in lc.runtime_names:
        v = vals[n]
        packed.append(v.data_ptr() if hasattr(v, "data_ptr") else v)
    import torch
    sid = int(torch.cuda.current_stream().cuda_stream)
    # the kernel's dispatches (a privatised histogram adds its second flush level)
    disp = lc.ck.prepare(grid, lc.ck.pack(packed), sid)
    lib = hip.load_library()
    err = ctypes.create_string_buffer(256)
    stream = ctypes.c_void_p(sid or None)

    def launch():
        for fn, g, blk, buf, n in disp:
            rc = lib.ek_launch(stream, fn, g[0], g[1], g[2], blk, 1, 1, 0, buf, n, err, 256)
            if rc:
                raise RuntimeError(err.value.decode())
    launch.ck = lc.ck
    return launch


# (BM, BN, BK, num_warps) swept for the matmul rows: the autotuner's MI355X candidates
MATMUL_CONFIGS = [(256, 256, 64, 4), (256, 256, 32, 4), (256, 128, 64, 4), (128, 256, 64, 4),
                  (128, 128, 64, 4), (256, 256, 64, 8), (256, 256, 32, 8)]


# (BLOCK_M, BLOCK_N, num_warps) swept for the attention rows (dot_warps = (num_warps, 1))
ATTN_CONFIGS = [(128, 64, 4), (128, 128, 4), (128, 32, 4), (256, 64, 8), (256, 128, 8)]


# num_warps swept for the HBM-bound row kernels (a launch option, as the autotuner would)
HBM_WARPS = (4, 8, 16)


def best_of(timer, steps, warmup, options, build):
    best = None
    for o in options:
        ls = build(o)
        ms = timer.run(ls, steps, warmup)
        log(f"    num_warps={o}: {ms * 1e3:.1f} us")
        if best is None or ms < best[0]:
            best = (ms, ls, o)
    return best


def sets_for(bytes_per_set):
    return max(2, math.ceil(600e6 / bytes_per_set))


# ------------------------------------------------------------------------- workloads

def w_softmax(torch, timer, steps, warmup):
    from examples.softmax import softmax_kernel
    M, N = 4096, 8192
    nbytes = M * N * 4 * 2
    k = sets_for(nbytes)
    xs = [torch.randn(M, N, device="cuda", generator=None) for _ in range(k)]
    outs = [torch.empty_like(x) for x in xs]
    ms, launches, nw = best_of(timer, steps, warmup, HBM_WARPS, lambda nw: [
        make_launch(softmax_kernel, (M,), (o, x, N, N, N), BLOCK=8192, num_warps=nw)
        for x, o in zip(xs, outs)])
    return {"name": "softmax", "config": f"fp32 [4096, 8192] num_warps={nw}", "ms": ms,
            "bytes": nbytes, "gbps": nbytes / ms / 1e6, "dtype": "fp32", "bound": "hbm",
            "kernel": launches[0].ck.name}


def w_rmsnorm(torch, timer, steps, warmup):
    from examples.rmsnorm import rmsnorm_kernel
    M, N = 4096, 8192
    nbytes = M * N * 4 * 2 + N * 4
    k = sets_for(nbytes)
    g = torch.Generator(device="cpu").manual_seed(1)
    w = (torch.rand(N, generator=g) + 0.5).cuda()
    xs = [torch.randn(M, N, device="cuda") for _ in range(k)]
    outs = [torch.empty_like(x) for x in xs]
    ms, launches, nw = best_of(timer, steps, warmup, HBM_WARPS, lambda nw: [
        make_launch(rmsnorm_kernel, (M,), (x, w, o, N, N, N, 1e-6), BLOCK=8192, num_warps=nw)
        for x, o in zip(xs, outs)])
    return {"name": "rmsnorm", "config": f"fp32 [4096, 8192] eps 1e-6 num_warps={nw}", "ms": ms,
            "bytes": nbytes, "gbps": nbytes / ms / 1e6, "dtype": "fp32", "bound": "hbm",
            "kernel": launches[0].ck.name}


def w_vector_add(torch, timer, steps, warmup):
    from examples.vector_add import add_kernel
    n = 1 << 28
    nbytes = 12 * n
    xs = [torch.randn(n, device="cuda") for _ in range(2)]
    y = torch.ones(n, device="cuda")
    out = torch.empty(n, device="cuda")
    launches = [make_launch(add_kernel, (n // 1024,), (x, y, out, n), BLOCK=1024) for x in xs]
    ms = timer.run(launches, max(4, steps // 4), max(2, warmup // 4))
    return {"name": "vector_add", "config": "fp32 n=2^28 BLOCK 1024", "ms": ms,
            "bytes": nbytes, "gbps": nbytes / ms / 1e6, "dtype": "fp32", "bound": "hbm",
            "kernel": launches[0].ck.name}


def w_matmul(torch, timer, steps, warmup, fused=False):
    from examples.matmul import matmul_desc_kernel
    from examples.matmul_fused import matmul_bias_gelu_kernel
    M = N = K = 4096
    g = torch.Generator(device="cpu").manual_seed(0)
    a = (torch.randn(M, K, generator=g) / 64).half().cuda()
    b = (torch.randn(K, N, generator=g) / 64).half().cuda()
    bias = torch.randn(N, generator=g).half().cuda()
    c = torch.empty(M, N, dtype=torch.float16, device="cuda")
    best = None
    for bm, bn, bk, nw in MATMUL_CONFIGS:
        cfg = dict(BM=bm, BN=bn, BK=bk, num_warps=nw)
        grid = (N // bn, M // bm)
        if fused:
            l = make_launch(matmul_bias_gelu_kernel, grid, (a, b, bias, c, M, N, K, K, N, N), **cfg)
        else:
            l = make_launch(matmul_desc_kernel, grid, (a, b, c, M, N, K, K, N, N), **cfg)
        ms = timer.run([l], max(5, steps // 2), max(2, warmup // 2))
        log(f"    BM={bm} BN={bn} BK={bk} warps={nw}: {ms * 1e3:.1f} us")
        if best is None or ms < best[0]:
            best = (ms, l, cfg)
    ms, l, cfg = best
    flop = 2 * M * N * K
    return {"name": "matmul_gelu" if fused else "matmul", "config": "fp16 4096^3 fp32 acc"
            + (" + bias + GELU" if fused else "") + f" {cfg}", "ms": ms, "flop": flop,
            "tflops": flop / ms / 1e9, "dtype": "fp16", "bound": "mfma", "kernel": l.ck.name}


def w_attention(torch, timer, steps, warmup, causal=True, n=4096):
    from examples.flash_attention import attention_kernel
    B, H, D = 4, 32, 128
    g = torch.Generator(device="cpu").manual_seed(0)
    q, k, v = (torch.randn(B, H, n, D, generator=g).bfloat16().cuda() for _ in range(3))
    o = torch.empty_like(q)
    best = None
    for bm, bn, nw in ATTN_CONFIGS:
        l = make_launch(attention_kernel, (n // bm, B * H), (q, k, v, o, D ** -0.5, n, n * D, D),
                        HEAD_DIM=D, BLOCK_M=bm, BLOCK_N=bn, CAUSAL=causal, num_warps=nw,
                        dot_warps=(nw, 1))
        ms = timer.run([l], max(3, steps // 4), max(1, warmup // 4))
        log(f"    BLOCK_M={bm} BLOCK_N={bn} warps={nw}: {ms * 1e3:.1f} us")
        if best is None or ms < best[0]:
            best = (ms, l, (bm, bn, nw))
    ms, l, cfg = best
    flop = 4 * B * H * n * n * D // (2 if causal else 1)
    return {"name": f"attention_{'causal' if causal else 'noncausal'}_{n}",
            "config": f"bf16 [4,32,{n},128] {'causal' if causal else 'non-causal'} "
                      f"BLOCK_M/N/warps={cfg}", "ms": ms,
            "flop": flop, "tflops": flop / ms / 1e9, "dtype": "bf16", "bound": "mfma", "kernel": l.ck.name}


def w_histogram(torch, timer, steps, warmup):
    from examples.histogram import histogram_kernel
    n = 1 << 26
    g = torch.Generator(device="cpu").manual_seed(0)
    xs = [torch.randint(0, 1024, (n,), generator=g, dtype=torch.int32).cuda() for _ in range(3)]
    h = torch.zeros(1024, dtype=torch.int32, device="cuda")
    ms, launches, nw = best_of(timer, max(4, steps // 4), 2, (4, 8), lambda nw: [
        make_launch(histogram_kernel, (n // 1024,), (x, h, n, 0.0, 1.0), NUM_BINS=1024,
                    BLOCK=1024, num_warps=nw) for x in xs])
    nbytes = 4 * n
    return {"name": "histogram", "config": f"int32 2^26 -> 1024 bins num_warps={nw}", "ms": ms,
            "bytes": nbytes,
            "gbps": nbytes / ms / 1e6, "dtype": "int32", "bound": "hbm", "kernel": launches[0].ck.name}


def w_cumsum(torch, timer, steps, warmup):
    from examples.cumsum import cumsum_kernel
    M, N = 8192, 4096
    nbytes = M * N * 4 * 2
    g = torch.Generator(device="cpu").manual_seed(0)
    xs = [torch.randint(-100, 100, (M, N), generator=g, dtype=torch.int32).cuda()
          for _ in range(sets_for(nbytes))]
    outs = [torch.empty_like(x) for x in xs]
    ms, launches, nw = best_of(timer, steps, warmup, HBM_WARPS, lambda nw: [
        make_launch(cumsum_kernel, (M,), (o, x, M, N, N, N), REVERSE=False, BLOCK_M=1,
                    BLOCK_N=4096, num_warps=nw) for x, o in zip(xs, outs)])
    return {"name": "cumsum", "config": f"int32 [8192, 4096] rows num_warps={nw}", "ms": ms,
            "bytes": nbytes,
            "gbps": nbytes / ms / 1e6, "dtype": "int32", "bound": "hbm", "kernel": launches[0].ck.name}


def w_torch_matmul(torch, timer, steps, warmup):
    """Calibration only: torch.matmul (hipBLASLt) on the same fp16 4096^3 problem."""
    M = N = K = 4096
    a = (torch.randn(M, K, device="cuda") / 64).half()
    b = (torch.randn(K, N, device="cuda") / 64).half()
    c = torch.empty(M, N, dtype=torch.float16, device="cuda")
    ms = timer.run([lambda: torch.matmul(a, b, out=c)], max(5, steps // 2), 3)
    flop = 2 * M * N * K
    return {"name": "torch_matmul", "config": "hipBLASLt fp16 4096^3 (calibration, not ours)",
            "ms": ms, "flop": flop, "tflops": flop / ms / 1e9, "dtype": "fp16", "bound": "mfma",
            "kernel": "torch.matmul"}


def w_torch_attention(torch, timer, steps, warmup, causal=True, n=4096):
    """Calibration only: torch's scaled_dot_product_attention (its ROCm flash kernel) on
    the same bf16 [4, 32, n, 128] problem."""
    import torch.nn.functional as F
    B, H, D = 4, 32, 128
    q, k, v = (torch.randn(B, H, n, D, device="cuda").bfloat16() for _ in range(3))
    ms = timer.run([lambda: F.scaled_dot_product_attention(q, k, v, is_causal=causal)],
                   max(3, steps // 4), 2)
    flop = 4 * B * H * n * n * D // (2 if causal else 1)
    return {"name": "torch_attention", "config": f"torch SDPA bf16 [4,32,{n},128] "
            f"{'causal' if causal else 'non-causal'} (calibration, not ours)", "ms": ms,
            "flop": flop, "tflops": flop / ms / 1e9, "dtype": "bf16", "bound": "mfma",
            "kernel": "torch.sdpa"}


def w_copy_calib(torch, timer, steps, warmup):
    """Calibration for HBM counters: a plain 256 MiB device-to-device copy."""
    n = 64 << 20
    x = torch.randn(n, device="cuda")
    y = torch.empty_like(x)
    ms = timer.run([lambda: y.copy_(x)], max(4, steps // 4), 2)
    nbytes = 8 * n
    return {"name": "copy_calib", "config": "torch copy 256 MiB -> 256 MiB", "ms": ms,
            "bytes": nbytes, "gbps": nbytes / ms / 1e6, "dtype": "fp32", "bound": "hbm", "kernel": "copy"}


WORKLOADS = {
    "softmax": w_softmax, "rmsnorm": w_rmsnorm, "vector_add": w_vector_add,
    "matmul": lambda t, tm, s, w: w_matmul(t, tm, s, w, False),
    "matmul_gelu": lambda t, tm, s, w: w_matmul(t, tm, s, w, True),
    "attention_causal": lambda t, tm, s, w: w_attention(t, tm, s, w, True, 4096),
    "attention_noncausal": lambda t, tm, s, w: w_attention(t, tm, s, w, False, 1024),
    "histogram": w_histogram, "cumsum": w_cumsum,
    "torch_matmul": w_torch_matmul,
    "torch_attention": w_torch_attention,
    "copy_calib": w_copy_calib,
}
DEFAULT = [k for k in WORKLOADS if k not in ("torch_matmul", "torch_attention", "copy_calib")]


def measured_traffic(kernel: str):
    """HBM bytes per launch for `kernel` from the committed rocprofv3 counter summary."""
    import glob
    for path in glob.glob(os.path.join(ROOT, "profiles", "*_hbm_counters.txt")):
        text = open(path).read()
        if kernel in text:
            for line in text.splitlines():
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":")[1])
    return None


def cpu_baseline(budget_s=12.0):
    """The oracle interpreter (1 core) on a bounded sample of softmax rows."""
    import numpy as np
    from examples.softmax import softmax_kernel
    from oracle import interpreter as O
    M, N = 4096, 8192
    x = np.random.default_rng(0).standard_normal((M, N), dtype=np.float32)
    out = np.empty_like(x)
    rows = 0
    t0 = time.perf_counter()
    order = np.random.default_rng(1).permutation(M)
    while time.perf_counter() - t0 < budget_s and rows < M:
        O.run_grid(softmax_kernel, (M,), out, x, N, N, N, BLOCK=8192,
                   programs=[(int(order[rows]),)])
        rows += 1
    dt = time.perf_counter() - t0
    gbps = rows * N * 4 * 2 / dt / 1e9
    return {"value": gbps, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{rows} random rows of the fp32 [4096, 8192] softmax through the "
                      f"oracle interpreter in {dt:.1f} s (programs are independent)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default="")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--mm", default="", help="only this matmul config: BM,BN,BK,num_warps")
    ap.add_argument("--attn", default="", help="only this attention config: BM,BN,num_warps")
    args = ap.parse_args()
    global MATMUL_CONFIGS, ATTN_CONFIGS
    if args.mm:
        MATMUL_CONFIGS = [tuple(int(x) for x in args.mm.split(","))]
    if args.attn:
        ATTN_CONFIGS = [tuple(int(x) for x in args.attn.split(","))]
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; multi-GPU runs are out "
                          "of scope (every config shards with no exchange between GPUs)"}))
        sys.exit(2)
    import torch
    torch.cuda.init()
    from enceladus_amd.runtime import hip
    info = hip.device_info(0)
    log(f"device: {info.name.decode()} {info.arch.decode()} CUs={info.compute_units}")
    timer = Timer(torch)
    names = args.only.split(",") if args.only else DEFAULT
    results = {}
    for n in names:
        log(f"[bench] {n} ...")
        r = WORKLOADS[n](torch, timer, args.steps, args.warmup)
        if r["bound"] == "hbm":
            r["roofline_frac"] = r["gbps"] * 1e9 / HBM_PEAK
        else:
            r["roofline_frac"] = r["tflops"] * 1e12 / MFMA_PEAK_F16
        results[n] = r
        log(f"[bench] {n}: {r['ms'] * 1e3:.1f} us  " +
            (f"{r['gbps']:.0f} GB/s" if "gbps" in r else f"{r['tflops']:.1f} TFLOP/s") +
            f"  ({100 * r['roofline_frac']:.1f}% of roofline)")
    head = results.get("softmax") or next(iter(results.values()))
    line = {
        "metric": "matmul/flash-attn TFLOP/s, softmax GB/s, % of MI355X roofline",
        "value": round(head.get("gbps", head.get("tflops", 0.0)), 2),
        "unit": "GB/s" if "gbps" in head else "TFLOP/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": head.get("dtype", "fp32"), "data": "synthetic",
        "config": {"workload": f"{head['name']} {head['config']}",
                   "device": info.name.decode(), "arch": info.arch.decode(),
                   "cus": info.compute_units},
        "roofline": ({"bound": "hbm", "achieved": round(head["gbps"], 1),
                      "peak": HBM_PEAK / 1e9, "unit": "GB/s"} if head["bound"] == "hbm" else
                     {"bound": "mfma", "achieved": round(head["tflops"], 1),
                      "peak": MFMA_PEAK_F16 / 1e12, "unit": "TFLOP/s"}) | {
                     "frac": round(head["roofline_frac"], 4),
                     "traffic": measured_traffic(head["kernel"])},
        "workloads": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                          for kk, vv in v.items()} for k, v in results.items()},
    }
    if not args.no_cpu_baseline:
        log("[bench] cpu baseline (oracle interpreter, bounded sample) ...")
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
