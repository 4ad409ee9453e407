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
