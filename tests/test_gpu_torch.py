"""GPU parity through torch-ROCm tensors (device pointers, no copies) and bf16 paths."""

import numpy as np
import pytest

from oracle import interpreter as O
from oracle import reference_np as R

pytestmark = pytest.mark.gpu


def test_torch_vector_add_device_pointers():
    import torch
    from examples.vector_add import add
    print("[case] torch vector add 2^20", flush=True)
    x = torch.randn(1 << 20, device="cuda")
    y = torch.ones_like(x)
    out = add(x, y)
    torch.cuda.synchronize()
    assert torch.equal(out, x + y)


@pytest.mark.parametrize("causal,n", [(True, 256), (False, 128)])
def test_flash_attention_bf16_torch(causal, n):
    import torch
    from examples.flash_attention import attention, attention_kernel
    print(f"[case] flash attention bf16 causal={causal} n={n}", flush=True)
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn((1, 2, n, 128), generator=g).to(torch.bfloat16) for _ in range(3))
    o = attention(q.cuda(), k.cuda(), v.cuda(), causal).float().cpu().numpy()
    want = R.attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), causal)
    np.testing.assert_allclose(o, want, rtol=1.6e-2, atol=1e-2)
    # against the oracle's bf16 semantics (P rounded to bf16 before the PV dot)
    ob = torch.empty_like(q)
    O.run_grid(attention_kernel, (n // 128, 2), q, k, v, ob, 128 ** -0.5, n, n * 128, 128,
               HEAD_DIM=128, BLOCK_M=128, BLOCK_N=64, CAUSAL=causal)
    np.testing.assert_allclose(o, ob.float().numpy(), rtol=1.6e-2, atol=1e-2)


def test_dlpack_export_to_torch():
    """enceladus.Tensor -> torch via DLPack (kDLROCM): shared HBM, no copy, and the
    exporting tensor stays alive until torch releases it."""
    import gc
    import numpy as np
    import torch
    import enceladus
    from enceladus_amd.runtime import dlpack
    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    t = enceladus.from_numpy(x)
    y = torch.from_dlpack(t)
    assert y.device.type == "cuda" and tuple(y.shape) == (3, 4) and y.dtype == torch.float32
    assert y.data_ptr() == t.data_ptr()
    np.testing.assert_array_equal(y.cpu().numpy(), x)
    y.mul_(2)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(t.numpy(), 2 * x)
    del t
    gc.collect()
    np.testing.assert_array_equal(y.cpu().numpy(), 2 * x)   # torch still holds the memory
    del y
    gc.collect()
    assert dlpack.live_exports() == 0


_SAXPY = '''
#include "enceladus_cdna4.h"
extern "C" __global__ void saxpy(float* out, const float* x, const float* y, float a, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = a * x[i] + y[i];
}
'''


def test_hip_kernel_escape_hatch():
    """Hand-written HIP through enceladus.hip_kernel, with NumPy (copied, written back) and
    torch-ROCm (device pointer) arguments. hipcc contracts a * x + y into one FMA, so the
    expected value is the singly rounded a * x + y (exact in float64, then rounded)."""
    import numpy as np
    import torch
    import enceladus
    k = enceladus.hip_kernel(_SAXPY, "saxpy")
    n = 10_000
    rng = np.random.default_rng(5)
    x, y = rng.standard_normal(n, dtype=np.float32), rng.standard_normal(n, dtype=np.float32)
    out = np.zeros(n, np.float32)
    k[(enceladus.cdiv(n, 256),), (256,)](out, x, y, 2.5, n)
    want = (np.float64(2.5) * x.astype(np.float64) + y).astype(np.float32)
    np.testing.assert_array_equal(out, want)
    xt, yt = torch.from_numpy(x).cuda(), torch.from_numpy(y).cuda()
    ot = torch.zeros(n, device="cuda")
    k[enceladus.cdiv(n, 128), 128](ot, xt, yt, 2.5, n)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(ot.cpu().numpy(), want)


def test_device_assert_reports_the_failing_program(monkeypatch):
    """ENCELADUS_DEBUG=1: a failing tl.device_assert raises DeviceAssertionError naming the
    first failing program and the assert's message and line; a passing one doesn't."""
    import numpy as np
    import pytest as _pt
    import enceladus
    from tests.test_compile_env import _debug_kernel
    monkeypatch.setenv("ENCELADUS_DEBUG", "1")
    k = _debug_kernel()
    x = np.zeros(1000, np.float32)
    k[(enceladus.cdiv(1000, 64),)](x, 1000, BLOCK=64)          # all below 100: no error
    x[700] = 500.0                                             # program 700 // 64 = 10
    with _pt.raises(enceladus.DeviceAssertionError) as e:
        k[(enceladus.cdiv(1000, 64),)](x, 1000, BLOCK=64)
    assert e.value.program_id == (10, 0, 0)
    assert "x must stay below 100" in str(e.value) and e.value.loc[1] > 0


def test_device_print_lines(capfd):
    """tl.device_print: one printf line per owned element, prefixed with the program id."""
    import numpy as np
    import enceladus
    from tests.test_compile_env import _debug_kernel
    k = _debug_kernel()
    x = np.arange(8, dtype=np.float32)
    k[(1,)](x, 8, BLOCK=64)
    enceladus.synchronize()
    out = capfd.readouterr().out
    lines = [ln for ln in out.splitlines() if ln.startswith("pid (0, 0, 0) idx")]
    assert len(lines) == 64
    assert "pid (0, 0, 0) idx (3) x: 3.000000" in lines


def test_tensor_factories():
    import enceladus
    print("[case] tensor factories", flush=True)
    assert np.array_equal(enceladus.ones((2, 3)).numpy(), np.ones((2, 3), np.float32))
    assert np.array_equal(enceladus.full(4, 7, "int32").numpy(), np.full(4, 7, np.int32))
    assert np.array_equal(enceladus.arange(5).numpy(), np.arange(5, dtype=np.int32))
    assert np.array_equal(enceladus.arange(2, 10, 3, dtype="int64").numpy(),
                          np.arange(2, 10, 3, dtype=np.int64))
    r = enceladus.rand(64, 32, seed=3).numpy()
    assert r.shape == (64, 32) and r.min() >= 0 and r.max() < 1
    assert np.array_equal(r, np.random.default_rng(3).random((64, 32), dtype=np.float32))
    z = enceladus.zeros_like(enceladus.ones((8,), "float16"))
    assert z.dtype.name == "fp16" and np.array_equal(z.numpy(), np.zeros(8, np.float16))
    assert enceladus.empty_like(np.zeros((3, 5), np.int8)).shape == (3, 5)


def test_async_numpy_chains_launches_and_copies_back_on_synchronize():
    import enceladus
    import enceladus.language as tl
    from examples.vector_add import add_kernel
    print("[case] async_numpy", flush=True)
    n = 10_000
    x = np.arange(n, dtype=np.float32)
    y = np.ones(n, np.float32)
    out = np.zeros(n, np.float32)
    enceladus.async_numpy(True)
    try:
        grid = (enceladus.cdiv(n, 1024),)
        add_kernel[grid](x, y, out, n, BLOCK=1024)      # out = x + 1
        add_kernel[grid](out, y, out, n, BLOCK=1024)    # reads the pending device copy
        enceladus.synchronize()
        assert np.array_equal(out, x + 2)
    finally:
        enceladus.async_numpy(False)
    add_kernel[grid](x, y, out, n, BLOCK=1024)          # synchronous again
    assert np.array_equal(out, x + 1)


def test_capture_writes_a_dispatch_trace(tmp_path):
    import json

    import torch

    import enceladus
    from examples.vector_add import add_kernel
    print("[case] capture", flush=True)
    x = torch.randn(1 << 20, device="cuda")
    out = torch.empty_like(x)
    path = tmp_path / "add.trace.json"
    with enceladus.capture(path) as p:
        for _ in range(3):
            add_kernel[(1024,)](x, x, out, x.numel(), BLOCK=1024)
    ev = json.loads(open(p).read())["traceEvents"]
    assert len(ev) == 3 and all(e["name"] == "ek_add_kernel" for e in ev)
    assert all(e["dur"] > 0 and e["args"]["grid"][0] == 1024 for e in ev)
    assert ev[0]["ts"] <= ev[1]["ts"] <= ev[2]["ts"]
    torch.testing.assert_close(out, 2 * x)


def test_writes_to_read_only_numpy_arrays_are_refused():
    """A kernel may read a read-only array but must not write one (reference:
    tests/test_runtime.py:333-355)."""
    from examples.vector_add import add_kernel
    print("[case] read-only numpy", flush=True)
    ro = np.frombuffer(bytes(32), np.float32)
    host = np.zeros(8, np.float32)
    add_kernel[(1,)](ro, ro, host, 8, BLOCK=8)
    np.testing.assert_array_equal(host, 0.0)
    with pytest.raises(ValueError, match="read-only NumPy array"):
        add_kernel[(1,)](host, host, ro, 8, BLOCK=8)
    with pytest.raises(ValueError, match="read-only NumPy array"):
        add_kernel[(1,)](host, host, np.broadcast_to(np.zeros(1, np.float32), (8,)), 8, BLOCK=8)
    assert not np.frombuffer(ro.tobytes(), np.float32).any()


@pytest.mark.gpu
@pytest.mark.parametrize("example", ["softmax", "rmsnorm", "vector_add"])
def test_math_is_bit_identical_across_launch_paths(example):
    # NumPy (copied in and out), torch-ROCm and enceladus.Tensor arguments select the same
    # specialization, so the results agree bit for bit (reference test strategy:
    # tests/test_interop.py test_math_is_bit_identical_across_launch_paths)
    import torch
    import enceladus
    print(f"[case] launch paths {example}", flush=True)
    rng = np.random.default_rng(40)
    if example == "vector_add":
        from examples.vector_add import add_kernel
        x, y = (rng.standard_normal(5000).astype(np.float32) for _ in range(2))
        run = lambda a, b, o: add_kernel[(5,)](a, b, o, 5000, BLOCK=1024)  # noqa: E731
        shape = (5000,)
    elif example == "softmax":
        from examples.softmax import softmax_kernel
        x, y = rng.standard_normal((16, 1000)).astype(np.float32), None
        run = lambda a, b, o: softmax_kernel[(16,)](o, a, 1000, 1000, 1000,  # noqa: E731
                                                     BLOCK=1024)
        shape = (16, 1000)
    else:
        from examples.rmsnorm import rmsnorm_kernel
        x = rng.standard_normal((16, 1000)).astype(np.float32)
        y = rng.uniform(0.5, 1.5, 1000).astype(np.float32)
        run = lambda a, b, o: rmsnorm_kernel[(16,)](a, b, o, 1000, 1000, 1000, 1e-6,  # noqa: E731
                                                     BLOCK=1024)
        shape = (16, 1000)
    outs = []
    o = np.zeros(shape, np.float32)
    run(x, y, o)
    outs.append(o)
    tx = torch.from_numpy(x).cuda()
    ty = torch.from_numpy(y).cuda() if y is not None else None
    to = torch.zeros(shape, dtype=torch.float32, device="cuda")
    run(tx, ty, to)
    torch.cuda.synchronize()
    outs.append(to.cpu().numpy())
    ex = enceladus.from_numpy(x)
    ey = enceladus.from_numpy(y) if y is not None else None
    eo = enceladus.zeros(shape)
    run(ex, ey, eo)
    outs.append(eo.numpy())
    assert outs[0].view(np.uint32).tolist() == outs[1].view(np.uint32).tolist()
    assert outs[0].view(np.uint32).tolist() == outs[2].view(np.uint32).tolist()


@pytest.mark.gpu
@pytest.mark.parametrize("pad", [0, 3, 64])
@pytest.mark.parametrize("case", ["softmax", "rmsnorm"])
def test_examples_on_padded_framework_arrays(case, pad):
    # row views into wider allocations: the row stride is the allocation's, not the width
    # (reference test strategy: tests/test_interop.py test_examples_on_framework_arrays)
    import torch
    print(f"[case] padded {case} pad={pad}", flush=True)
    m, n = 24, 1000
    g = torch.Generator().manual_seed(pad)
    base = torch.randn(m, n + pad, generator=g).cuda()
    x = base[:, :n]
    if case == "softmax":
        from examples.softmax import softmax
        got = softmax(x)
        want = R.softmax(x.cpu().numpy())
    else:
        from examples.rmsnorm import rmsnorm
        w = (torch.rand(n, generator=g) + 0.5).cuda()
        got = rmsnorm(x, w)
        want = R.rmsnorm(x.cpu().numpy(), w.cpu().numpy())
    torch.cuda.synchronize()
    np.testing.assert_allclose(got.cpu().numpy(), want, rtol=1e-5, atol=1e-6)
