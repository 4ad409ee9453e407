"""`kernel.explain` reports the compiler's decisions by source line (reference test
strategy: tests/test_debug.py:122-135). Compile-only: runs without a GPU."""

import numpy as np

import enceladus
import enceladus.language as tl


@enceladus.jit
def _transposed_sum(a_ptr, b_ptr, out_ptr, N: tl.constexpr):
    r = tl.arange(0, N)
    a = tl.load(a_ptr + r[:, None] * N + r[None, :])
    bt = tl.trans(tl.load(b_ptr + r[:, None] * N + r[None, :]))
    s = tl.sum(a + bt, axis=0)  # the exchange line
    tl.store(out_ptr + r, s)


def test_explain_reports_conversions_and_lds_by_line():
    a = np.zeros((64, 64), np.float32)
    out = np.zeros(64, np.float32)
    text = _transposed_sum.explain(a, a, out, grid=(1,), N=64)
    conv = [ln for ln in text.splitlines() if "LDS exchange" in ln]
    assert len(conv) == 1 and "test_explain.py:" in conv[0]
    assert "s = tl.sum(a + bt, axis=0)" in conv[0]
    reduce = [ln for ln in text.splitlines() if " reduce: " in ln]
    assert reduce and int(reduce[0].split("reduce:")[1].split()[0]) > 0
    ck = _transposed_sum.warmup(a, a, out, N=64)
    assert f"LDS: {ck.lds_bytes} bytes" in text
    assert "dot backend: none" in text


def test_explain_names_the_mfma_plan_of_each_dot():
    import torch
    from examples.flash_attention import attention_kernel
    bf = torch.zeros(16, dtype=torch.bfloat16)
    text = attention_kernel.explain(bf, bf, bf, bf, 0.088, 4096, 4096 * 128, 128,
                                    HEAD_DIM=128, BLOCK_M=256, BLOCK_N=128, CAUSAL=True,
                                    num_warps=8, dot_warps=(8, 1))
    dots = [ln for ln in text.splitlines() if "(MxNxK)" in ln]
    assert len(dots) == 2 and all("wave grid 8x1" in d and "MFMA 32x32x16" in d for d in dots)
    assert all("staged through LDS" in d for d in dots)


def test_explain_on_a_cache_hit_reports_the_kernel_that_was_loaded(monkeypatch, tmp_path):
    """A specialization loaded from the persistent cache has no emitter report; explain
    regenerates it with the options the kernel was compiled with (the ENCELADUS_CODEGEN
    switches included), so it describes the loaded kernel."""
    from enceladus_amd.runtime.jit import JITFunction
    from examples.matmul import matmul_desc_kernel
    monkeypatch.setenv("ENCELADUS_CACHE_DIR", str(tmp_path))
    monkeypatch.setenv("ENCELADUS_CODEGEN", "no_gemm_template")
    a = np.zeros((256, 256), np.float16)
    args = (a, a, a, 256, 256, 256, 256, 256, 256)
    kw = dict(BM=128, BN=128, BK=64, num_warps=4)
    first = JITFunction(matmul_desc_kernel.fn).warmup(*args, **kw)
    assert first.gen.report is not None and "GemmDma" not in first.hip
    fresh = JITFunction(matmul_desc_kernel.fn)          # empty in-memory cache: a disk hit
    ck = fresh.warmup(*args, **kw)
    assert ck.gen.report is None and ck.hip == first.hip
    text = fresh.explain(*args, **kw)
    assert "GEMM template" not in text and "MFMA 32x32x16" in text
