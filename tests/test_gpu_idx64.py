"""GPU parity for 64-bit index math: an array of more than 2^31 elements (2 GiB of uint8
on one MI355X) processed by a kernel whose `pid * BLOCK + arange` would wrap in 32 bits
(reference: runtime/launcher.py:42-48, compiler/passes/widen_index.py)."""

import pytest

import enceladus
import enceladus.language as tl
from enceladus_amd.compiler import ir

pytestmark = pytest.mark.gpu


@enceladus.jit
def _add_u8(x_ptr, y_ptr, out_ptr, n, BLOCK: tl.constexpr):
    pid = tl.program_id(0)
    offs = pid * BLOCK + tl.arange(0, BLOCK)
    mask = offs < n
    x = tl.load(x_ptr + offs, mask=mask)
    y = tl.load(y_ptr + offs, mask=mask)
    tl.store(out_ptr + offs, x + y, mask=mask)


def test_add_past_2_31_elements():
    import torch
    n = (1 << 31) + 3000
    print(f"[case] idx64 uint8 add n={n}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(7)
    x = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda", generator=g)
    y = torch.randint(0, 256, (n,), dtype=torch.uint8, device="cuda", generator=g)
    out = torch.zeros(n, dtype=torch.uint8, device="cuda")
    block = 4096
    # the launch must compile the widened variant: check the IR before running it
    f = _add_u8.ir_for(x, y, out, n, BLOCK=block)
    offs = [op.operands[1].type.dtype.name for op in ir.walk(f.body) if op.name == "ptr_add"]
    assert offs and all(d == "i64" for d in offs), offs
    _add_u8[((n + block - 1) // block,)](x, y, out, n, BLOCK=block)
    torch.cuda.synchronize()
    want = x + y
    assert torch.equal(out[-(1 << 20):], want[-(1 << 20):])
    assert torch.equal(out, want)
