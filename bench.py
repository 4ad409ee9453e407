"""Benchmark of the north-star workloads on one MI355X.

Prints one JSON line (the driver's contract). The headline workload is BASELINE config 2
(`configs[1]`): row softmax over fp32 [4096, 8192]; `value` is its whole-job GB/s with
inputs resident in HBM. The same run measures every other config (vector add 2^28,
RMSNorm, fp16 4096^3 matmul and + bias + GELU, bf16 flash attention causal 4096 and
non-causal 1024, int32 histogram and cumsum) and reports each under "workloads" with its
roofline fraction.

Every launch timed here comes from `examples/workloads.py`, the table that
`tests/test_gpu_bench_configs.py` checks variant by variant at the same full sizes against
the CPU oracle. Matmul and attention take the variant the library's autotuner picks
(`matmul_desc_tuned`, `matmul_bias_gelu_tuned`, `attention_tuned_kernel` over
`enceladus.configs`); the HBM-bound rows time each listed `num_warps` and report the
fastest. Kernel times come from HIP events recorded on the launch stream (torch's current
stream) around K pre-packed launches after W warm-ups and at least 50 ms of GPU time spent
warming up (as the reference's do_bench); inputs of the HBM-bound rows rotate
over buffer sets totalling > 600 MB so the 256 MB Infinity Cache cannot serve them.

The CPU baseline (`cpu_baseline`, and `cpu` under each workload) times the oracle
interpreter (a restatement of the reference's `ENCELADUS_INTERPRET=1` interpreter, one
core) on a random sample of each grid's programs, and NumPy's closed form (the examples'
`reference()` functions) on a bounded slice, both extrapolated to the full workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME[,NAME]]
                       [--no-cpu-baseline]
                       [--pin NAME=INDEX[,...]]
NAME is a workload of examples/workloads.py (the BASELINE configs, and copy_rows /
copy_flat: plain copies of the same bytes by this backend, the HBM ceiling the row kernels
are read against), copy_calib (torch's device copy, the counter calibration),
torch_matmul / torch_sdpa_causal / torch_sdpa_noncausal (the vendor libraries on the same
inputs; part of the default run) or launch_overhead (host cost of warm launches; part of
the default run).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
os.environ.setdefault("ENCELADUS_CACHE_DIR", os.path.join(ROOT, ".ek_cache"))

HBM_PEAK = 8.0e12          # bytes/s (MI355X HBM3E)
MFMA_PEAK_F16 = 2.5e15     # dense fp16/bf16 FLOP/s
WARMUP_MS = 50.0           # GPU time spent warming up before each timed region
METRIC = "matmul/flash-attn TFLOP/s, softmax GB/s, % of MI355X roofline"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Timer:
    """HIP-event timing on torch's current stream (the stream kernels launch on)."""

    def __init__(self, torch):
        self.torch = torch

    def run(self, launches, steps, warmup, warmup_ms=WARMUP_MS):
        """ms per launch over `steps` launches, after `warmup` launches and then more
        until the GPU has been busy for `warmup_ms` (the reference's do_bench warms up by
        GPU time the same way, testing.py:14-63: the clock is low after idle, and a
        kernel's first launches after an idle spell run up to 20% slower)."""
        torch = self.torch
        for i in range(warmup):
            launches[i % len(launches)]()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        spent, batch, i = 0.0, 1, warmup
        while spent < warmup_ms:
            s.record()
            for _ in range(batch):
                launches[i % len(launches)]()
                i += 1
            e.record()
            torch.cuda.synchronize()
            spent += s.elapsed_time(e)
            batch = min(2 * batch, 64)
        s.record()
        for i in range(steps):
            launches[i % len(launches)]()
        e.record()
        torch.cuda.synchronize()
        return s.elapsed_time(e) / steps  # ms per launch


def make_launch(jfn, grid, args, options):
    """A pre-packed launch of `jfn[grid](*args, **options)` on torch's current stream: the
    same specialization lookup as the Python front door, with no Python in the timed loop
    beyond one ctypes call per dispatch."""
    import ctypes

    import torch

    from enceladus_amd.runtime import hip
    options = dict(options)
    nw = options.pop("num_warps", 4)
    dw = options.pop("dot_warps", None)
    vals = jfn._bind(args, options)
    lc = jfn._lookup(vals, nw, dw)
    packed = []
    for n in lc.runtime_names:
        v = vals[n]
        packed.append(v.data_ptr() if hasattr(v, "data_ptr") else v)
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
    launch.shapes = [[list(g), blk] for _, g, blk, _, _ in disp]
    return launch


def rotation_sets(torch, wl, base):
    """Extra input sets (rolled copies of the seeded inputs) so that the sets together
    exceed 600 MB: consecutive launches then read HBM, not the Infinity Cache."""
    sets = [base]
    n = max(2, math.ceil(600e6 / wl.work)) if wl.bound == "hbm" else 1
    for i in range(1, n):
        s = {}
        for k, t in base.items():
            s[k] = torch.empty_like(t) if k in wl.outputs else torch.roll(t, i, 0)
        sets.append(s)
    return sets


def measure(torch, timer, wl, steps, warmup, pin=None):
    """Times workload `wl`: the autotuner's pick, the fastest listed variant, or, with
    `pin`, the variant at that index of the workload's table (for profiling runs)."""
    from examples import workloads as W
    host = wl.inputs()
    base = W.device_buffers(wl, host)
    sets = rotation_sets(torch, wl, base)
    r = {"name": wl.name, "bound": wl.bound, "dtype": wl.dtype, "tested_by":
         "tests/test_gpu_bench_configs.py"}
    if pin is not None:
        r["selected_by"] = "pinned (--pin)"
        choices = [wl.variants[pin]]
    elif wl.tuned is not None:
        # the library's autotuner picks the variant (on the seeded inputs)
        tuned = wl.tuned()
        _, args = wl.args(base, wl.variants[0])

        def grid(meta):
            return wl.args(base, W.Variant(tuple(meta.items())))[0]
        t0 = time.perf_counter()
        tuned[grid](*args, **wl.fixed)
        torch.cuda.synchronize()
        cfg = tuned.config_for(*args, **wl.fixed)
        v = wl.variant_of(cfg)
        key = tuned._key(tuned_named(tuned, args, wl.fixed))
        for c, ms in sorted(tuned.timings.get(key, {}).items(), key=lambda x: x[1]):
            log(f"    autotune {c}: {ms * 1e3:.1f} us")
        log(f"    autotuner picked {v.label} ({time.perf_counter() - t0:.1f} s)")
        assert v in wl.variants, f"autotuner pick {v} is not in the tested table"
        r["selected_by"] = "autotuner"
        choices = [v]
    else:
        r["selected_by"] = "fastest listed variant"
        choices = wl.variants
    best = None
    for v in choices:
        launches = [make_launch(wl.kernel(), *wl.args(s, v), v.options()) for s in sets]
        # at least 20 timed launches per row (vector add and attention each take about
        # 0.5 ms a launch, so 20 of them are 10-12 ms of GPU time)
        k = max(20, steps)
        ms = timer.run(launches, k, max(2, warmup // 2))
        log(f"    {v.label}: {ms * 1e3:.1f} us")
        if best is None or ms < best[0]:
            best = (ms, v, launches[0].ck, launches[0].shapes, launches)
    ms, v, ck, shapes, launches = best
    # The same launches one at a time with the GPU idle between them (HIP events around
    # each, the median of 20): how the library's do_bench and the autotuner sample. The
    # MFMA rows run faster this way than back to back, where they hold the clock down.
    from enceladus_amd import testing
    ms_iso = testing.do_bench(launches[0], warmup_ms=0.0, rep=20)
    # LDS bytes and registers tell the reported variant's dispatches apart from other
    # variants of the same grid in a kernel trace
    r.update({"config": f"{wl.describe} {v.label}", "variant": v.label, "ms": ms,
              "ms_isolated": ms_iso, "kernel": ck.name, "dispatches": shapes, "lds_bytes": ck.attrs["shared_bytes"],
              "vgprs": ck.attrs["num_regs"]})
    if wl.bound == "hbm":
        r["bytes"] = wl.work
        r["gbps"] = wl.work / ms / 1e6
        r["roofline_frac"] = r["gbps"] * 1e9 / HBM_PEAK
    else:
        r["flop"] = wl.work
        r["tflops"] = wl.work / ms / 1e9
        r["roofline_frac"] = r["tflops"] * 1e12 / MFMA_PEAK_F16
    r["traffic"] = measured_traffic(wl.name)
    del sets, base
    return r, host


def copy_calibration(torch, timer, steps):
    """A plain 256 MiB device-to-device copy (torch's copy kernel): the known-size kernel
    that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes. Run only when named
    in --only."""
    n = 64 << 20
    x = torch.randn(n, device="cuda")
    y = torch.empty_like(x)
    ms = timer.run([lambda: y.copy_(x)], max(4, steps // 4), 2)
    return {"name": "copy_calib", "config": "torch copy 256 MiB -> 256 MiB", "ms": ms,
            "bytes": 8 * n, "gbps": 8 * n / ms / 1e6, "bound": "hbm", "dtype": "fp32",
            "kernel": "copy", "roofline_frac": 8 * n / ms / 1e6 * 1e9 / HBM_PEAK}


TORCH_ROWS = ("torch_matmul", "torch_sdpa_causal", "torch_sdpa_noncausal")


def torch_reference(torch, timer, name, steps):
    """The vendor-library figure for an MFMA workload, on the same inputs and clock
    conditions: torch.matmul (hipBLASLt) for the fp16 4096^3 product, and torch's
    scaled_dot_product_attention restricted to its flash backend (an error, never the
    math fallback, when that backend is missing) for the two attention configs."""
    from examples import workloads as W
    if name == "torch_matmul":
        wl = W.table()["matmul"]
        b = W.device_buffers(wl)
        a, bb, c = b["a"], b["b"], b["c"]
        fn = lambda: torch.matmul(a, bb, out=c)  # noqa: E731
        cfg, work = "torch.matmul fp16 4096^3 (hipBLASLt)", wl.work
    else:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        causal = name.endswith("_causal")
        wl = W.table()["attention_causal" if causal else "attention_noncausal"]
        b = W.device_buffers(wl)
        q, k, v = b["q"], b["k"], b["v"]

        def fn():
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
                torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal)
        cfg, work = f"torch SDPA flash backend {wl.describe}", wl.work
    fn()
    torch.cuda.synchronize()
    ms = timer.run([fn], max(5, steps // 2), 3)
    return {"name": name, "config": cfg, "ms": ms, "flop": work, "bound": "mfma",
            "tflops": work / ms / 1e9, "roofline_frac": work / ms / 1e9 * 1e12 / MFMA_PEAK_F16,
            "dtype": wl.dtype, "kernel": "vendor library"}


def launch_overhead(torch, reps=5, n_launch=10_000):
    """Host cost of a warm launch (reference: benchmarks/bench_dispatch.py): µs per launch
    for back-to-back `@jit` launches of a 1024-element vector add through the Python front
    door (`kernel[grid](...)`, torch-ROCm tensors), the same kernel through a pre-packed
    `ek_launch` (the native floor), `torch.add(out=)`, and a launch + synchronize round
    trip. Medians over `reps` runs."""
    import statistics

    from examples.vector_add import add_kernel
    n = 1024
    x, y, o = (torch.randn(n, device="cuda") for _ in range(3))

    def jit_launch():
        add_kernel[(1,)](x, y, o, n, BLOCK=1024)

    native = make_launch(add_kernel, (1,), (x, y, o, n), {"BLOCK": 1024})

    def sustained(fn, count=n_launch):
        out = []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(count):
                fn()
            torch.cuda.synchronize()
            out.append((time.perf_counter() - t0) / count * 1e6)
        return statistics.median(out)

    def round_trip(fn, count=300):
        out = []
        for _ in range(count):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            out.append((time.perf_counter() - t0) * 1e6)
        return statistics.median(out)

    jit_launch()
    sustained(jit_launch, 2000)                  # warm the clocks and caches
    return {"jit_sustained_us": round(sustained(jit_launch), 2),
            "native_ek_launch_sustained_us": round(sustained(native), 2),
            "torch_add_sustained_us": round(sustained(lambda: torch.add(x, y, out=o)), 2),
            "jit_round_trip_us": round(round_trip(jit_launch), 2),
            "workload": "vector add n=1024, grid (1,), BLOCK 1024, torch-ROCm tensors"}


def tuned_named(tuned, args, fixed):
    from enceladus_amd.runtime.autotuner import _named
    return _named(tuned.fn, args, fixed)


def source_stamp() -> str:
    """A hash of everything that decides the generated kernels: the package's Python
    sources and device headers, and the example kernels and workload table. A counter
    summary records the stamp of the tree it measured."""
    import hashlib
    from pathlib import Path

    from enceladus_amd.runtime import speccache
    h = speccache.tree_hash(Path(ROOT) / "enceladus_amd")
    for p in sorted((Path(ROOT) / "examples").glob("*.py")):
        h.update(p.name.encode())
        h.update(p.read_bytes())
    return h.hexdigest()[:16]


def measured_traffic(name: str):
    """HBM bytes per launch of workload `name` from the committed rocprofv3 counter
    summaries (`traffic_bytes_per_launch[name]: N` lines), or None when no summary has
    the row or the summary measured other sources than this tree's (its
    `source_stamp: ...` line differs from `source_stamp()`): a stale figure is not
    reported."""
    import glob
    tag = f"traffic_bytes_per_launch[{name}]:"
    here = source_stamp()
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*counters*.txt"))):
        lines = open(path).read().splitlines()
        stamp = next((ln.split(":", 1)[1].strip() for ln in lines
                      if ln.startswith("source_stamp:")), None)
        for line in lines:
            if line.startswith(tag):
                return int(line.split(":")[1]) if stamp == here else None
    return None


# ------------------------------------------------------------------------- CPU baseline

def host_info():
    model = platform.processor() or ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count()
    blas = None
    try:
        from threadpoolctl import threadpool_info
        blas = [{"api": d.get("internal_api"), "threads": d.get("num_threads")}
                for d in threadpool_info()]
    except Exception:  # noqa: BLE001
        pass
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "affinity": aff,
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS"),
            "OPENBLAS_NUM_THREADS": os.environ.get("OPENBLAS_NUM_THREADS"), "blas": blas}


def _sample_programs(grid, budget_s, run_one, seed=1, stratify=None):
    """Runs a random sample of program ids through `run_one(pid)` for about `budget_s`;
    returns (programs run, seconds). `stratify(pid)` orders causal programs so that the
    sample covers every row of blocks evenly."""
    import numpy as np
    total = 1
    for g in grid:
        total *= g
    order = np.random.default_rng(seed).permutation(total)
    if stratify is not None:
        order = sorted(order.tolist(), key=stratify)
    done = 0
    t0 = time.perf_counter()
    while done < total and (done == 0 or time.perf_counter() - t0 < budget_s):
        i = int(order[done])
        pid = (i % grid[0], (i // grid[0]) % (grid[1] if len(grid) > 1 else 1))
        run_one(pid)
        done += 1
    return done, time.perf_counter() - t0, total


def cpu_workload(wl, host, v, budget_s=1.5):
    """The oracle interpreter on sampled programs and NumPy's closed form on a slice of
    workload `wl` (inputs `host`, variant `v`), both scaled to the full workload."""
    import numpy as np

    from examples import workloads as W
    from oracle import interpreter as O
    from oracle import reference_np as R
    c = dict(v.constexprs)
    out = {}
    if wl.name in ("softmax", "rmsnorm", "cumsum"):
        x = host["x"]
        m, n = x.shape
        y = np.zeros_like(x)
        if wl.name == "softmax":
            def one(pid):
                O.run_grid(wl.kernel(), (m,), y, x, n, n, n, **c, programs=[pid])
        elif wl.name == "rmsnorm":
            def one(pid):
                O.run_grid(wl.kernel(), (m,), x, host["w"], y, n, n, n, 1e-6, **c,
                           programs=[pid])
        else:
            def one(pid):
                O.run_grid(wl.kernel(), (m,), y, x, m, n, n, n, **c, programs=[pid])
        grid = (m,)
        rows = 512
        t0 = time.perf_counter()
        if wl.name == "softmax":
            R.softmax(x[:rows])
        elif wl.name == "rmsnorm":
            R.rmsnorm(x[:rows], host["w"])
        else:
            R.cumsum(x[:rows])
        np_s = (time.perf_counter() - t0) * m / rows
        np_sample = f"closed form on {rows} of {m} rows"
    elif wl.name == "vector_add":
        x, yv = host["x"], host["y"]
        n = x.size
        o = np.zeros(n, np.float32)

        def one(pid):
            O.run_grid(wl.kernel(), (n // 1024,), x, yv, o, n, BLOCK=1024, programs=[pid])
        grid = (n // 1024,)
        k = 1 << 24
        t0 = time.perf_counter()
        R.vector_add(x[:k], yv[:k])
        np_s = (time.perf_counter() - t0) * n / k
        np_sample = f"closed form on 2^24 of {n} elements"
    elif wl.name == "histogram":
        x = host["x"]
        n = x.size
        hist = np.zeros(W.HIST_BINS, np.int32)

        def one(pid):
            O.run_grid(wl.kernel(), (n // 1024,), x, hist, n, 0.0, 1.0, **c, programs=[pid])
        grid = (n // 1024,)
        t0 = time.perf_counter()
        R.histogram(x, W.HIST_BINS, 0.0, 1024.0)
        np_s = time.perf_counter() - t0
        np_sample = "closed form (np.bincount) on all elements"
    elif wl.name.startswith("matmul"):
        a, b = host["a"], host["b"]
        mm = a.shape[0]
        cc = np.zeros((mm, mm), np.float16)
        grid = (mm // c["BN"], mm // c["BM"])
        if wl.name == "matmul":
            def one(pid):
                O.run_grid(wl.kernel(), grid, a, b, cc, mm, mm, mm, mm, mm, mm, **c,
                           programs=[pid])
        else:
            def one(pid):
                O.run_grid(wl.kernel(), grid, a, b, host["bias"], cc, mm, mm, mm, mm, mm, mm,
                           **c, programs=[pid])
        rows = 256
        t0 = time.perf_counter()
        if wl.name == "matmul":
            R.matmul(a[:rows], b)
        else:
            R.matmul_bias_gelu(a[:rows], b, host["bias"])
        np_s = (time.perf_counter() - t0) * mm / rows
        np_sample = f"closed form on {rows} of {mm} rows of A"
    else:   # attention
        import torch
        q, k, vv = host["q"], host["k"], host["v"]
        z, h, n, d = q.shape
        ob = torch.zeros_like(q)
        bm = c["BLOCK_M"]
        grid = (n // bm, z * h)

        def one(pid):
            O.run_grid(wl.kernel(), grid, q, k, vv, ob, d ** -0.5, n, n * d, d, **c,
                       programs=[pid])
        t0 = time.perf_counter()
        R.attention(q[:1, :1].float().numpy(), k[:1, :1].float().numpy(),
                    vv[:1, :1].float().numpy(), c["CAUSAL"])
        np_s = (time.perf_counter() - t0) * z * h
        np_sample = f"float64 closed form on 1 of {z * h} (batch, head) slices"
    strat = None
    if wl.name == "attention_causal":
        def strat(i):   # interleave start_m blocks so a short sample spans all of them
            return (i // grid[0], i % grid[0])
    done, secs, total = _sample_programs(grid, budget_s, one, stratify=strat)
    interp_s = secs * total / done
    unit = "GB/s" if wl.bound == "hbm" else "TFLOP/s"
    scale = 1e9 if wl.bound == "hbm" else 1e12
    out["interpreter"] = {"value": wl.work / interp_s / scale, "unit": unit, "cores": 1,
                          "kind": "port", "full_run_s_est": interp_s,
                          "sample": f"{done} of {total} programs in {secs:.2f} s"}
    out["numpy"] = {"value": wl.work / np_s / scale, "unit": unit, "kind": "numpy",
                    "full_run_s_est": np_s, "sample": np_sample}
    return out


# ------------------------------------------------------------------ profile summaries
# `python bench.py --summarize-profiles DIR` tabulates the rocprofv3 output of the passes
# below (run on the GPU box from the repository root, each writing under DIR) into
# profiles/*.txt. Every summary records the source stamp of the tree the passes measured
# (from the trace pass's bench JSON), and the bench reads traffic from a summary only while
# that stamp is the current tree's.

PROFILE_ROWS = ("vector_add,softmax,rmsnorm,matmul,matmul_gelu,attention_causal,"
                "attention_noncausal,histogram,cumsum,copy_rows,copy_flat,read_flat,fill_flat,"
                "copy_calib,torch_matmul,torch_sdpa_causal,torch_sdpa_noncausal")
SQ_COUNTERS = ("SQ_BUSY_CYCLES SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_MFMA SQ_INSTS_VALU "
               "SQ_INSTS_LDS SQ_LDS_BANK_CONFLICT SQ_LDS_IDX_ACTIVE SQ_VALU_MFMA_COEXEC_CYCLES")
_KERNELS = {"vector_add": ["ek_add_kernel"], "softmax": ["ek_softmax_kernel"],
            "rmsnorm": ["ek_rmsnorm_kernel"], "matmul": ["ek_matmul_desc_kernel"],
            "matmul_gelu": ["ek_matmul_bias_gelu_kernel"],
            "attention_causal": ["ek_attention_kernel"],
            "attention_noncausal": ["ek_attention_kernel"],
            "histogram": ["ek_histogram_kernel", "ek_histogram_kernel_flush"],
            "cumsum": ["ek_cumsum_kernel"], "copy_rows": ["ek_copy_rows_kernel"],
            "copy_flat": ["ek_copy_flat_kernel"], "read_flat": ["ek_read_flat_kernel"],
            "fill_flat": ["ek_fill_flat_kernel"]}


def profile_commands(pins: str) -> list[str]:
    """The rocprofv3 passes the summaries come from, as run on the GPU box after
    `R=<repository root>; D=<output directory>; cd /tmp && export TMPDIR=/tmp`; the pins
    come from `python3 $R/bench.py --print-pins $D/trace_bench.json`."""
    return [
        "rocprofv3 --kernel-trace --stats -d $D/trace -o run --output-format csv -- "
        f"python3 $R/bench.py --only {PROFILE_ROWS} --no-cpu-baseline > $D/trace_bench.json",
        "rocprofv3 --pmc FETCH_SIZE -d $D/FETCH_SIZE -o run --output-format csv -- "
        f"python3 $R/bench.py --only {PROFILE_ROWS} --pin {pins} --steps 4 --warmup 1 "
        "--no-cpu-baseline > $D/FETCH_SIZE_bench.json",
        "rocprofv3 --pmc WRITE_SIZE -d $D/WRITE_SIZE (the same bench.py arguments) > "
        "$D/WRITE_SIZE_bench.json",
        f"rocprofv3 --pmc {SQ_COUNTERS} -d $D/sq -o run --output-format csv -- python3 "
        "$R/bench.py --only matmul,matmul_gelu,attention_causal,attention_noncausal "
        f"--pin {pins} --steps 3 --warmup 1 --no-cpu-baseline > $D/sq_bench.json"]


def profile_pins(trace_json: dict) -> str:
    """--pin arguments fixing each row to the variant the trace pass's bench reported."""
    from examples import workloads as W
    table = W.table()
    out = []
    for n, r in trace_json["workloads"].items():
        if n in table and "variant" in r:
            labels = [v.label for v in table[n].variants]
            out.append(f"{n}={labels.index(r['variant'])}")
    return ",".join(out)


def _bench_json(path):
    return json.loads([ln for ln in open(path) if ln.startswith("{")][-1])


def _row_of(kname, grid, block):
    """The bench row a dispatch of ours belongs to (the two attention configs share a
    kernel: causal grids have 4096 / BLOCK_M programs on x, non-causal 1024 / BLOCK_M)."""
    if kname == "ek_attention_kernel":
        bm = {512: 256, 256: 128, 128: 64}.get(block)
        if bm is None:
            return None
        return {4096: "attention_causal", 1024: "attention_noncausal"}.get(grid[0] * bm)
    for w, ks in _KERNELS.items():
        if kname in ks:
            return w
    return None


def summarize_profiles(d: str) -> None:
    import collections
    import csv
    import statistics
    import subprocess
    tj = _bench_json(f"{d}/trace_bench.json")
    stamp = tj.get("source_stamp")
    if stamp != source_stamp():
        raise SystemExit(f"the profiles measured sources {stamp}, this tree is "
                         f"{source_stamp()}: profile this tree again")
    try:
        commit = subprocess.run(["git", "-C", ROOT, "rev-parse", "--short=12", "HEAD"],
                                capture_output=True, text=True, check=True).stdout.strip()
        dirty = subprocess.run(["git", "-C", ROOT, "status", "--porcelain", "--",
                                "enceladus_amd", "examples"], capture_output=True,
                               text=True).stdout.strip()
        commit += " (with uncommitted changes)" if dirty else ""
    except (OSError, subprocess.CalledProcessError):
        commit = "unknown"
    pins = profile_pins(tj)
    cmds = profile_commands(pins)
    head = ["MI355X (gfx950, 256 CUs), one GPU, ROCm 7.2 rocprofv3; numbers from one GPU box",
            f"source_stamp: {stamp}",
            f"commit: {commit}",
            "(bench.py --print-stamp gives a tree's stamp; bench.py reports traffic from this "
            "file only while the stamps agree)", ""]
    W_ = tj["workloads"]
    m = statistics.median

    # -- kernel trace -------------------------------------------------------------------
    rows = list(csv.DictReader(open(f"{d}/trace/run_kernel_trace.csv")))
    groups, vendor = collections.defaultdict(list), collections.defaultdict(list)
    for r in rows:
        name = r["Kernel_Name"]
        blk = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * \
            int(r["Workgroup_Size_Z"])
        grid = tuple(int(r[f"Grid_Size_{a}"]) // int(r[f"Workgroup_Size_{a}"]) for a in "XYZ")
        dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        key = (name, grid, blk, int(r["LDS_Block_Size"]), int(r["VGPR_Count"]),
               int(r["Accum_VGPR_Count"]))
        w = _row_of(name, grid, blk)
        if w is not None:
            groups[(w,) + key].append(dur)
        elif name.startswith("Cijk_") or name == "attn_fwd":
            vendor[key].append(dur)
    out = ["rocprofv3 kernel trace of every bench.py workload (BASELINE configs, the copy, "
           "read and write ceilings) and the vendor libraries"] + head + [
        "command (on the GPU box; R = repository root, D = the output directory, run in /tmp "
        "with TMPDIR=/tmp):",
        "  " + cmds[0],
        "tabulated with: python bench.py --summarize-profiles $D", "",
        "Per workload: the bench's HIP-event time, then the per-dispatch durations from",
        "run_kernel_trace.csv grouped by (kernel, grid in workgroups, workgroup size, LDS,",
        "registers). '*' marks the dispatches of the variant the bench reports, told apart from",
        "other variants of the same grid by its LDS bytes and registers (a privatised histogram",
        "launch is two dispatches: the kernel and its _flush); the other rows are the variants",
        "the bench swept or the autotuner timed. Trace averages include the warm-up, tuning and",
        "sweep dispatches of the same shape.", ""]
    hdr = (f"    {'kernel':<30} {'grid (workgroups)':>18} {'wg':>5} {'LDS(B)':>7} {'VGPR':>4} "
           f"{'AGPR':>4} {'calls':>6} {'avg_us':>8} {'min_us':>8} {'max_us':>8}")
    for w in _KERNELS:
        if w not in W_:
            continue
        r = W_[w]
        rep = {(tuple(g), b) for g, b in r["dispatches"]}
        out += [f"{w}: {r['config']}  ({r['selected_by']})",
                f"  bench.py HIP events: {r['ms'] * 1e3:.1f} us per launch", hdr]
        items = sorted(((k, v) for k, v in groups.items() if k[0] == w),
                       key=lambda kv: -len(kv[1]))

        def reported(k):
            _, name, grid, blk, lds, vg, _ag = k
            if (grid, blk) not in rep:
                return False
            if name != r["kernel"]:
                return True                     # the histogram's flush dispatch
            # the trace rounds LDS up to 512-byte granules and counts registers in pairs
            return r["lds_bytes"] <= lds < r["lds_bytes"] + 512 and \
                abs(2 * vg - r["vgprs"]) < 16
        items.sort(key=lambda kv: not reported(kv[0]))
        for k, v in items:
            _, name, grid, blk, lds, vg, ag = k
            g = "x".join(str(x) for x in grid)
            out.append(f"  {'*' if reported(k) else ' '} {name:<30} {g:>18} {blk:>5} {lds:>7} "
                       f"{vg:>4} {ag:>4} {len(v):>6} {statistics.fmean(v):>8.2f} "
                       f"{min(v):>8.2f} {max(v):>8.2f}")
        out.append("")
    out.append("vendor libraries on the same inputs (bench.py torch_* rows):")
    for t in TORCH_ROWS:
        if t in W_:
            out.append(f"  {t}: {W_[t]['config']}: {W_[t]['ms'] * 1e3:.1f} us, "
                       f"{W_[t]['tflops']:.1f} TFLOP/s")
    out.append(hdr)
    for k, v in sorted(vendor.items(), key=lambda kv: kv[0][0]):
        name, grid, blk, lds, vg, ag = k
        nm = "Cijk_... (hipBLASLt)" if name.startswith("Cijk_") else "attn_fwd (torch SDPA)"
        g = "x".join(str(x) for x in grid)
        out.append(f"    {nm:<30} {g:>18} {blk:>5} {lds:>7} {vg:>4} {ag:>4} {len(v):>6} "
                   f"{statistics.fmean(v):>8.2f} {min(v):>8.2f} {max(v):>8.2f}")
    open(os.path.join(ROOT, "profiles", "workloads_kernel_trace.txt"), "w").write(
        "\n".join(out) + "\n")

    # -- HBM counters -------------------------------------------------------------------
    def counters(name):
        per, calib = collections.defaultdict(list), []
        for r in csv.DictReader(open(f"{d}/{name}/run_counter_collection.csv")):
            v = float(r["Counter_Value"])
            if r["Kernel_Name"] == "__amd_rocclr_copyBuffer" and int(r["Grid_Size"]) == 131072:
                calib.append(v)
                continue
            per[(r["Kernel_Name"], int(r["Grid_Size"]), int(r["Workgroup_Size"]))].append(v)
        return per, calib
    fetch, fcal = counters("FETCH_SIZE")
    write, wcal = counters("WRITE_SIZE")
    jf = _bench_json(f"{d}/FETCH_SIZE_bench.json")["workloads"]
    ff, wf = 262144 / m(fcal), 262144 / m(wcal)
    out = ["rocprofv3 HBM counters (FETCH_SIZE, WRITE_SIZE) of every bench.py workload"] + \
        head + [
        "commands (on the GPU box, as for the kernel trace), one counter per run, each workload",
        "pinned to the variant the trace pass's bench reported:",
        "  " + cmds[1], "  " + cmds[2],
        "tabulated with: python bench.py --summarize-profiles $D", "",
        "calibration (copy_calib: a 256 MiB torch device copy, 262144 KiB read and 262144 KiB "
        "written):",
        f"  FETCH_SIZE per dispatch: {m(fcal):.0f} KiB -> factor {ff:.3f}",
        f"  WRITE_SIZE per dispatch: {m(wcal):.0f} KiB -> factor {wf:.3f}", "",
        "FETCH_SIZE counts the L2's fetches from memory (HBM, or the Infinity Cache behind the",
        "L2), so for the MFMA kernels it is L2-miss traffic, an upper bound on HBM bytes.",
        "Mean per dispatch:", ""]
    traffic = {}
    for w in _KERNELS:
        if w not in jf:
            continue
        r = jf[w]
        out.append(f"{w}: {r['config']}")
        rd = wr = 0.0
        for (gx, gy, gz), b in r["dispatches"]:
            for kname in _KERNELS[w]:
                k = (kname, gx * gy * gz * b, b)
                if k in fetch:
                    fv, wv = statistics.fmean(fetch[k]), statistics.fmean(write[k])
                    out.append(f"  {kname} ({gx * gy * gz} workgroups x {b}): FETCH_SIZE "
                               f"{fv:.0f} KiB, WRITE_SIZE {wv:.0f} KiB")
                    rd += fv * ff
                    wr += wv * wf
        tot = round((rd + wr) * 1024)
        traffic[w] = tot
        if r["bound"] == "hbm":
            alg, what = r["bytes"], "algorithmic bytes (the bench's byte count)"
        elif w.startswith("matmul"):
            alg = 3 * 4096 * 4096 * 2 + (4096 * 2 if w == "matmul_gelu" else 0)
            what = "A + B read once, C written once (fp16)"
        else:
            n = 4096 if w == "attention_causal" else 1024
            alg = 4 * 4 * 32 * n * 128 * 2
            what = "Q, K, V read once, O written once (bf16)"
        out.append(f"  read {rd:.0f} KiB + written {wr:.0f} KiB = {tot} B per launch; {what}: "
                   f"{alg} B; measured / algorithmic {tot / alg:.4f}")
    out += ["", "bench.py reads the lines below into each workload's \"traffic\" (and the "
            "headline's roofline.traffic):"]
    out += [f"traffic_bytes_per_launch[{w}]: {t}" for w, t in traffic.items()]
    open(os.path.join(ROOT, "profiles", "workloads_hbm_counters.txt"), "w").write(
        "\n".join(out) + "\n")

    # -- SQ counters of the MFMA rows ----------------------------------------------------
    disp = collections.defaultdict(dict)
    for r in csv.DictReader(open(f"{d}/sq/run_counter_collection.csv")):
        e = disp[r["Dispatch_Id"]]
        e.update(name=r["Kernel_Name"], thr=int(r["Grid_Size"]), wg=int(r["Workgroup_Size"]),
                 dur=int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
        e[r["Counter_Name"]] = float(r["Counter_Value"])
    js = _bench_json(f"{d}/sq_bench.json")["workloads"]
    out = ["rocprofv3 SQ counters of the MFMA workloads (the variants the bench reports)"] + \
        head + ["command (on the GPU box, as for the kernel trace):",
                "  " + cmds[3],
                "tabulated with: python bench.py --summarize-profiles $D", "",
                "Counters are summed over the chip; per SIMD = / 1024 (256 CUs x 4 SIMDs). One",
                "v_mfma_f32_32x32x16 is 32768 FLOP and occupies its SIMD's MFMA unit for 32",
                "cycles. No clock is derived from these counters: the counters' window is longer",
                "than the dispatch (a GRBM_GUI_ACTIVE-based clock read above the 2.4 GHz maximum",
                "on short dispatches). 'MFMA busy at 2.4 GHz' is the MFMA cycles per SIMD over",
                "the dispatch's duration times the maximum clock: a lower bound on the busy",
                "fraction, exact only if the kernel ran at 2.4 GHz.", ""]
    for w in ("matmul", "matmul_gelu", "attention_causal", "attention_noncausal"):
        if w not in js:
            continue
        r = js[w]
        ((gx, gy, gz), b), = r["dispatches"]
        ds = [e for e in disp.values() if e["name"] == r["kernel"] and
              e["thr"] == gx * gy * gz * b and e["wg"] == b and "SQ_INSTS_MFMA" in e]
        mf = m([e["SQ_INSTS_MFMA"] for e in ds])
        va = m([e["SQ_INSTS_VALU"] for e in ds])
        busy = m([e["SQ_VALU_MFMA_BUSY_CYCLES"] for e in ds]) / 1024
        co = m([e["SQ_VALU_MFMA_COEXEC_CYCLES"] for e in ds]) / 1024
        lds = m([e["SQ_INSTS_LDS"] for e in ds])
        bc = m([e["SQ_LDS_BANK_CONFLICT"] for e in ds])
        dur = m([e["dur"] for e in ds])
        out += [f"{w}: {r['config']}",
                f"  {len(ds)} dispatches, median duration {dur / 1e3:.1f} us",
                f"  MFMA busy per SIMD {busy:.0f} cycles = {100 * busy / (dur * 2.4):.1f}% of the "
                f"dispatch at 2.4 GHz; MFMA/VALU co-issue {co:.0f} cycles per SIMD",
                f"  SQ_INSTS_MFMA {mf:.0f} (x 32768 FLOP = {mf * 32768 / r['flop']:.4f} x the "
                f"algorithmic FLOP), SQ_INSTS_VALU {va:.0f} ({va / mf:.2f} per MFMA)",
                f"  SQ_INSTS_LDS {lds:.0f}, SQ_LDS_BANK_CONFLICT {bc:.0f} "
                f"({bc / lds:.3f} per LDS instruction)", ""]
    open(os.path.join(ROOT, "profiles", "matmul_attention_sq_counters.txt"), "w").write(
        "\n".join(out) + "\n")
    print(f"wrote profiles/ from {d} (source_stamp {stamp}, commit {commit}, pins {pins})")


# ----------------------------------------------------------------------------- main

def main():
    from examples import workloads as W
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=40)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--only", default="")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--pin", default="", help="NAME=INDEX[,NAME=INDEX]: time only that "
                    "variant of the workload's table (profiling runs)")
    ap.add_argument("--print-stamp", action="store_true", help="print the source stamp "
                    "that counter summaries record, and exit")
    ap.add_argument("--print-pins", metavar="BENCH_JSON", help="print the --pin arguments "
                    "that fix every row to the variant a bench run reported, and exit")
    ap.add_argument("--summarize-profiles", metavar="DIR", help="tabulate the rocprofv3 "
                    "passes under DIR into profiles/*.txt, and exit (no GPU needed)")
    args = ap.parse_args()
    if args.print_stamp:
        print(source_stamp())
        return
    if args.print_pins:
        print(profile_pins(_bench_json(args.print_pins)))
        return
    if args.summarize_profiles:
        summarize_profiles(args.summarize_profiles)
        return
    pins = {k: int(v) for k, v in (p.split("=") for p in args.pin.split(",") if p)}
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
    table = W.table()
    names = args.only.split(",") if args.only else list(table) + list(TORCH_ROWS)
    results = {}
    cpu = {}
    for n in names:
        log(f"[bench] {n} ...")
        if n == "launch_overhead":
            continue
        if n == "copy_calib":
            results[n] = copy_calibration(torch, timer, args.steps)
            log(f"[bench] copy_calib: {results[n]['gbps']:.0f} GB/s")
            continue
        if n in TORCH_ROWS:
            try:
                results[n] = torch_reference(torch, timer, n, args.steps)
            except RuntimeError as e:     # a vendor backend this torch build lacks
                log(f"[bench] {n}: skipped ({e})")
                continue
            log(f"[bench] {n}: {results[n]['ms'] * 1e3:.1f} us  "
                f"{results[n]['tflops']:.1f} TFLOP/s")
            continue
        r, host = measure(torch, timer, table[n], args.steps, args.warmup, pins.get(n))
        if table[n].ceiling:
            r["ceiling"] = True
        results[n] = r
        log(f"[bench] {n}: {r['ms'] * 1e3:.1f} us  " +
            (f"{r['gbps']:.0f} GB/s" if "gbps" in r else f"{r['tflops']:.1f} TFLOP/s") +
            f"  ({100 * r['roofline_frac']:.1f}% of roofline; isolated launches "
            f"{r['ms_isolated'] * 1e3:.1f} us)")
        if not args.no_cpu_baseline and not table[n].ceiling:
            v = next(x for x in table[n].variants if x.label == r["variant"])
            cpu[n] = cpu_workload(table[n], host, v)
            r["cpu"] = cpu[n]
            log(f"    cpu: interpreter {cpu[n]['interpreter']['value']:.4g} "
                f"{cpu[n]['interpreter']['unit']} ({cpu[n]['interpreter']['sample']}), "
                f"numpy {cpu[n]['numpy']['value']:.4g}")
        del host
        torch.cuda.empty_cache()
    if not results:         # only the launch-overhead rows were asked for
        print(json.dumps({"metric": "warm launch overhead (us per launch)",
                          "launch_overhead": launch_overhead(torch)}), flush=True)
        return
    real = {k: r for k, r in results.items()
            if k != "copy_calib" and k not in TORCH_ROWS and not r.get("ceiling")} or results
    head = real.get("softmax") or next(iter(real.values()))
    line = {
        "metric": METRIC,
        "value": round(head.get("gbps", head.get("tflops", 0.0)), 2),
        "unit": "GB/s" if "gbps" in head else "TFLOP/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(head["ms"], 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": head.get("dtype", "fp32"), "data": "synthetic",
        "config": {"workload": f"{head['name']} {head['config']}",
                   "device": info.name.decode(), "arch": info.arch.decode(),
                   "cus": info.compute_units, "max_clock_mhz": info.clock_khz // 1000,
                   "mem_clock_mhz": info.mem_clock_khz // 1000,
                   "mem_bus_bits": info.mem_bus_width, "lds_per_block": info.lds_per_block,
                   "l2_bytes": info.l2_bytes, "hbm_bytes": info.total_mem},
        "roofline": ({"bound": "hbm", "achieved": round(head["gbps"], 1),
                      "peak": HBM_PEAK / 1e9, "unit": "GB/s"} if head["bound"] == "hbm" else
                     {"bound": "mfma", "achieved": round(head["tflops"], 1),
                      "peak": MFMA_PEAK_F16 / 1e12, "unit": "TFLOP/s"}) | {
                     "frac": round(head["roofline_frac"], 4),
                     "traffic": head.get("traffic")},
        "source_stamp": source_stamp(),
        "workloads": {k: {kk: (round(vv, 4) if isinstance(vv, float) else vv)
                          for kk, vv in v.items()} for k, v in results.items()},
    }
    if not args.only or "launch_overhead" in names:
        log("[bench] launch overhead ...")
        line["launch_overhead"] = launch_overhead(torch)
        log(f"    {line['launch_overhead']}")
    if cpu:
        hc = cpu.get(head["name"]) or next(iter(cpu.values()))
        ib = hc["interpreter"]
        line["cpu_baseline"] = {"value": ib["value"], "unit": ib["unit"], "cores": 1,
                                "kind": "port", "sample": f"{head['name']}: oracle "
                                f"interpreter, {ib['sample']}, scaled to the full workload",
                                "host": host_info()}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
