"""The BASELINE workloads at full size, and every specialization the benchmark may time.

One table with two users: `bench.py` times these launches (picking the fastest variant of
a workload, or the autotuner's pick where the workload is autotuned), and
`tests/test_gpu_bench_configs.py` runs every variant on the same inputs and checks it
against the CPU oracle. A number the benchmark reports therefore always comes from a
specialization (kernel, dtypes, constexprs, `num_warps`, `dot_warps`, argument facts) that
a GPU parity test ran at the same size.

Inputs follow the BASELINE configs: one `np.random.default_rng(seed)` per array (seed 0
for the first array, 1 for the second, ...), float32 draws cast to the working dtype; bf16
through torch's round-to-nearest-even cast.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Callable

import numpy as np

import enceladus
import enceladus.language as tl


@dataclass(frozen=True)
class Variant:
    """The launch options of one specialization: constexprs, waves, dot wave grid."""

    constexprs: tuple
    num_warps: int = 4
    dot_warps: tuple | None = None

    def options(self) -> dict:
        out = dict(self.constexprs)
        out["num_warps"] = self.num_warps
        if self.dot_warps:
            out["dot_warps"] = tuple(self.dot_warps)
        return out

    @property
    def label(self) -> str:
        parts = [f"{k}={v}" for k, v in self.constexprs]
        parts.append(f"num_warps={self.num_warps}")
        if self.dot_warps:
            parts.append(f"dot_warps={tuple(self.dot_warps)}")
        return " ".join(parts)

    @staticmethod
    def of(config) -> "Variant":
        """The variant of an autotuner `Config`."""
        return Variant(tuple(sorted(config.kwargs.items())), config.num_warps,
                       tuple(config.dot_warps) if config.dot_warps else None)


@dataclass
class Workload:
    """One BASELINE config: its kernel, inputs, launch and the variants it may run."""

    name: str
    describe: str
    kernel: Callable[[], object]          # returns the @jit kernel
    bound: str                            # "hbm" or "mfma"
    work: int                             # algorithmic bytes (hbm) or FLOP (mfma)
    dtype: str                            # the dtype the path computes in
    inputs: Callable[[], dict]            # host arrays (NumPy, or torch for bf16)
    outputs: dict                         # output name -> (shape, dtype name)
    args: Callable[[dict, Variant], tuple]  # (grid, positional args) from buffers
    variants: list = field(default_factory=list)
    tuned: Callable[[], object] | None = None  # the autotuned kernel, when autotuned
    fixed: dict = field(default_factory=dict)  # constexprs the autotuned launch passes
    ceiling: bool = False                 # a copy kernel that calibrates the HBM rows

    def variant_of(self, config) -> Variant:
        """The variant an autotuner `Config` selects for this workload."""
        kw = dict(config.kwargs, **self.fixed)
        return Variant(tuple(sorted(kw.items())), config.num_warps,
                       tuple(config.dot_warps) if config.dot_warps else None)


def _f32(seed, shape):
    return np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)


def _bf16(a: np.ndarray):
    import torch
    return torch.from_numpy(a).to(torch.bfloat16)


# -- config 1: vector add --------------------------------------------------------------

VADD_N = 1 << 28


def _vadd_inputs(n=VADD_N):
    x = _f32(0, n)
    return {"x": x, "y": np.ones_like(x)}


def _vadd_args(b, v):
    n = b["x"].numel()
    block = dict(v.constexprs)["BLOCK"]
    return ((n + block - 1) // block,), (b["x"], b["y"], b["out"], n)


# -- config 2: softmax and RMSNorm ------------------------------------------------------

ROWS, COLS = 4096, 8192
HBM_WARPS = (4, 8, 16)


def _row_inputs():
    return {"x": _f32(0, (ROWS, COLS))}


def _rms_inputs():
    return {"x": _f32(0, (ROWS, COLS)),
            "w": np.random.default_rng(1).uniform(0.5, 1.5, COLS).astype(np.float32)}


def _softmax_args(b, v):
    m, n = b["x"].shape
    return (m,), (b["out"], b["x"], n, n, n)


def _rms_args(b, v):
    m, n = b["x"].shape
    return (m,), (b["x"], b["w"], b["out"], n, n, n, 1e-6)


# -- config 3: matmul and matmul + bias + GELU -----------------------------------------

MM = 4096


def _mm_inputs():
    a = (_f32(0, (MM, MM)) / 64).astype(np.float16)
    b = (_f32(1, (MM, MM)) / 64).astype(np.float16)
    return {"a": a, "b": b}


def _mm_gelu_inputs():
    d = _mm_inputs()
    d["bias"] = _f32(2, MM).astype(np.float16)
    return d


def _mm_grid(b, v):
    c = dict(v.constexprs)
    m, k = b["a"].shape
    n = b["b"].shape[1]
    return (-(-n // c["BN"]), -(-m // c["BM"])), (m, n, k)


def _mm_args(b, v):
    grid, (m, n, k) = _mm_grid(b, v)
    return grid, (b["a"], b["b"], b["c"], m, n, k, k, n, n)


def _mm_gelu_args(b, v):
    grid, (m, n, k) = _mm_grid(b, v)
    return grid, (b["a"], b["b"], b["bias"], b["c"], m, n, k, k, n, n)


def _matmul_variants():
    from enceladus_amd.configs import matmul_configs
    return [Variant.of(c) for c in matmul_configs("float16")]


# -- config 4: flash attention ----------------------------------------------------------

ATT_B, ATT_H, ATT_D = 4, 32, 128


def _att_inputs(n):
    return {k: _bf16(_f32(i, (ATT_B, ATT_H, n, ATT_D))) for i, k in enumerate("qkv")}


def _att_args(b, v):
    c = dict(v.constexprs)
    z, h, n, d = b["q"].shape
    return ((n + c["BLOCK_M"] - 1) // c["BLOCK_M"], z * h), \
        (b["q"], b["k"], b["v"], b["o"], d ** -0.5, n, n * d, d)


def _attention_variants(causal):
    from enceladus_amd.configs import attention_configs
    out = []
    for c in attention_configs("bfloat16", ATT_D):
        kw = dict(c.kwargs, HEAD_DIM=ATT_D, CAUSAL=causal)
        out.append(Variant(tuple(sorted(kw.items())), c.num_warps,
                           tuple(c.dot_warps) if c.dot_warps else None))
    return out


def attention_flop(n, causal):
    """4 B H N^2 D, halved for causal (reference: benchmarks/bench_attention.py:9-10)."""
    return 4 * ATT_B * ATT_H * n * n * ATT_D // (2 if causal else 1)


# -- config 5: histogram and cumsum ----------------------------------------------------

HIST_N, HIST_BINS = 1 << 26, 1024
SCAN_ROWS, SCAN_COLS = 8192, 4096


def hist_inputs(n=HIST_N):
    return {"x": np.random.default_rng(0).integers(0, HIST_BINS, n, dtype=np.int32)}


def _hist_args(b, v):
    n = b["x"].numel()
    # the wrapper's lo = 0.0, hi = 1024.0 -> inv_width = NUM_BINS / (hi - lo) = 1.0
    return ((n + 1023) // 1024,), (b["x"], b["hist"], n, 0.0, 1.0)


def _scan_inputs():
    return {"x": np.random.default_rng(0).integers(-100, 100, (SCAN_ROWS, SCAN_COLS),
                                                   dtype=np.int32)}


def _scan_args(b, v):
    m, n = b["x"].shape
    return (m,), (b["out"], b["x"], m, n, n, n)


# -- copy ceilings ----------------------------------------------------------------------
# Plain copies compiled by this backend, in the row kernels' shape (one program per 32 KB
# row) and flat (small tiles, many programs): the HBM rate a kernel with the same access
# pattern and no arithmetic reaches on the same box. Not BASELINE configs.

@enceladus.jit
def copy_rows_kernel(out_ptr, in_ptr, stride, n_cols, BLOCK: tl.constexpr):
    row = tl.program_id(0)
    cols = tl.arange(0, BLOCK)
    mask = cols < n_cols
    x = tl.load(in_ptr + row * stride + cols, mask=mask)
    tl.store(out_ptr + row * stride + cols, x, mask=mask)


@enceladus.jit
def copy_flat_kernel(out_ptr, in_ptr, n, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    mask = offs < n
    tl.store(out_ptr + offs, tl.load(in_ptr + offs, mask=mask), mask=mask)


@enceladus.jit
def read_flat_kernel(out_ptr, in_ptr, n, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    x = tl.load(in_ptr + offs, mask=offs < n, other=0.0)
    tl.store(out_ptr + tl.program_id(0), tl.max(x, axis=0))


@enceladus.jit
def fill_flat_kernel(out_ptr, value, n, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    tl.store(out_ptr + offs, tl.full([BLOCK], value, tl.float32), mask=offs < n)


def _read_flat_args(b, v):
    n = b["x"].numel()
    block = dict(v.constexprs)["BLOCK"]
    return ((n + block - 1) // block,), (b["out"], b["x"], n)


def _fill_flat_args(b, v):
    n = b["out"].numel()
    block = dict(v.constexprs)["BLOCK"]
    return ((n + block - 1) // block,), (b["out"], 1.5, n)


def _copy_rows_args(b, v):
    m, n = b["x"].shape
    return (m,), (b["out"], b["x"], n, n)


def _copy_flat_args(b, v):
    n = b["x"].numel()
    block = dict(v.constexprs)["BLOCK"]
    return ((n + block - 1) // block,), (b["out"], b["x"], n)


def _k(module, name):
    def get():
        import importlib
        return getattr(importlib.import_module(f"examples.{module}"), name)
    return get


def table() -> dict[str, Workload]:
    """Every BASELINE workload by name."""
    w = {}
    w["vector_add"] = Workload(
        "vector_add", "fp32 n=2^28 BLOCK 1024", _k("vector_add", "add_kernel"), "hbm",
        12 * VADD_N, "fp32", _vadd_inputs, {"out": ((VADD_N,), "float32")}, _vadd_args,
        [Variant((("BLOCK", 1024),), nw) for nw in (4, 2)])
    w["softmax"] = Workload(
        "softmax", "fp32 [4096, 8192]", _k("softmax", "softmax_kernel"), "hbm",
        ROWS * COLS * 8, "fp32", _row_inputs, {"out": ((ROWS, COLS), "float32")},
        _softmax_args, [Variant((("BLOCK", 8192),), nw) for nw in HBM_WARPS])
    w["rmsnorm"] = Workload(
        "rmsnorm", "fp32 [4096, 8192] eps 1e-6", _k("rmsnorm", "rmsnorm_kernel"), "hbm",
        ROWS * COLS * 8 + COLS * 4, "fp32", _rms_inputs, {"out": ((ROWS, COLS), "float32")},
        _rms_args, [Variant((("BLOCK", 8192),), nw) for nw in HBM_WARPS])
    w["matmul"] = Workload(
        "matmul", "fp16 4096^3 fp32 acc", _k("matmul", "matmul_desc_kernel"), "mfma",
        2 * MM ** 3, "fp16", _mm_inputs, {"c": ((MM, MM), "float16")}, _mm_args,
        _matmul_variants(), _k("matmul", "matmul_desc_tuned"))
    w["matmul_gelu"] = Workload(
        "matmul_gelu", "fp16 4096^3 fp32 acc + bias + GELU",
        _k("matmul_fused", "matmul_bias_gelu_kernel"), "mfma", 2 * MM ** 3, "fp16",
        _mm_gelu_inputs, {"c": ((MM, MM), "float16")}, _mm_gelu_args, _matmul_variants(),
        _k("matmul_fused", "matmul_bias_gelu_tuned"))
    for causal, n in ((True, 4096), (False, 1024)):
        name = f"attention_{'causal' if causal else 'noncausal'}"
        w[name] = Workload(
            name, f"bf16 [4,32,{n},128] {'causal' if causal else 'non-causal'}",
            _k("flash_attention", "attention_kernel"), "mfma", attention_flop(n, causal),
            "bf16", (lambda n=n: _att_inputs(n)),
            {"o": ((ATT_B, ATT_H, n, ATT_D), "bfloat16")}, _att_args,
            _attention_variants(causal), _k("flash_attention", "attention_tuned_kernel"),
            {"HEAD_DIM": ATT_D, "CAUSAL": causal})
    w["histogram"] = Workload(
        "histogram", "int32 2^26 -> 1024 bins", _k("histogram", "histogram_kernel"), "hbm",
        4 * HIST_N, "int32", hist_inputs, {"hist": ((HIST_BINS,), "int32")}, _hist_args,
        # one variant: at BLOCK=1024 an 8-wave program holds 2 elements per thread (8-byte
        # loads, half the bytes per load of the 4-wave program) and its walk, bound by the
        # loads each wave has in flight, measured 60.0 us against 47.5 us; the 8-wave
        # program is parity-tested in tests/test_gpu_bench_configs.py but not timed
        [Variant((("BLOCK", 1024), ("NUM_BINS", HIST_BINS)), 4)])
    w["cumsum"] = Workload(
        "cumsum", "int32 [8192, 4096] rows", _k("cumsum", "cumsum_kernel"), "hbm",
        SCAN_ROWS * SCAN_COLS * 8, "int32", _scan_inputs,
        {"out": ((SCAN_ROWS, SCAN_COLS), "int32")}, _scan_args,
        [Variant((("BLOCK_M", 1), ("BLOCK_N", SCAN_COLS), ("REVERSE", False)), nw)
         for nw in HBM_WARPS])
    w["copy_rows"] = Workload(
        "copy_rows", "fp32 [4096, 8192] one row per program", lambda: copy_rows_kernel,
        "hbm", ROWS * COLS * 8, "fp32", _row_inputs, {"out": ((ROWS, COLS), "float32")},
        _copy_rows_args, [Variant((("BLOCK", 8192),), nw) for nw in HBM_WARPS],
        ceiling=True)
    w["copy_flat"] = Workload(
        "copy_flat", "fp32 2^25 elements", lambda: copy_flat_kernel, "hbm",
        ROWS * COLS * 8, "fp32", lambda: {"x": _f32(0, ROWS * COLS)},
        {"out": ((ROWS * COLS,), "float32")}, _copy_flat_args,
        [Variant((("BLOCK", b),), 4) for b in (1024, 2048, 4096)], ceiling=True)
    # One direction only, over the same 2^25 fp32 elements: the read and write rates
    # whose mix bounds every row above (a max per tile, whose 4-byte results are not
    # counted; a constant fill).
    w["read_flat"] = Workload(
        "read_flat", "fp32 2^25 elements read, max per tile", lambda: read_flat_kernel,
        "hbm", ROWS * COLS * 4, "fp32",
        lambda: {"x": _f32(0, ROWS * COLS)}, {"out": ((ROWS * COLS // 1024,), "float32")},
        _read_flat_args, [Variant((("BLOCK", b),), 4) for b in (1024, 2048, 4096)],
        ceiling=True)
    w["fill_flat"] = Workload(
        "fill_flat", "fp32 2^25 elements written", lambda: fill_flat_kernel, "hbm",
        ROWS * COLS * 4, "fp32", lambda: {}, {"out": ((ROWS * COLS,), "float32")},
        _fill_flat_args, [Variant((("BLOCK", b),), 4) for b in (1024, 2048, 4096)],
        ceiling=True)
    return w


def device_buffers(wl: Workload, host: dict | None = None) -> dict:
    """The workload's inputs as torch device tensors plus zeroed outputs."""
    import torch
    host = wl.inputs() if host is None else host
    out = {}
    for k, a in host.items():
        t = a if isinstance(a, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(a))
        out[k] = t.cuda()
    for k, (shape, dt) in wl.outputs.items():
        out[k] = torch.zeros(shape, dtype=getattr(torch, dt), device="cuda")
    return out


def launch(wl: Workload, bufs: dict, v: Variant):
    """Launches variant `v` of `wl` on `bufs` through the kernel's `kernel[grid](...)`."""
    grid, args = wl.args(bufs, v)
    return wl.kernel()[grid](*args, **v.options())

