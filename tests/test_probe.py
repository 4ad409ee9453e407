"""The once-per-process MFMA lane-map probe (reference: runtime/device.py:108-145).

CPU: the probe's verdict logic against an emulated device, once with the lane maps the
emitter assumes (passes) and once with the accumulator transposed (raises
CompilationError). GPU: the real probe passes on the MI355X and runs before the first
MFMA kernel loads.
"""

import numpy as np
import pytest

from enceladus_amd.compiler import layout as L
from enceladus_amd.runtime import probe


class _EmulatedKernel:
    """Stands in for the compiled probe: builds A and B from the lanes' fragments with the
    operand maps, multiplies, and returns each lane's registers through `acc_map`."""

    def __init__(self, m, acc_map):
        self.m, self.acc_map = m, acc_map

    def __getitem__(self, launch):
        def run(a_in, b_in, out):
            plan = L.plan_dot(self.m, self.m, 16 if self.m == 32 else 32, 1, "fp16")
            i = plan.inst
            A = np.zeros((i.m, i.k), np.float32)
            B = np.zeros((i.k, i.n), np.float32)
            a_in, b_in = a_in.reshape(64, 8), b_in.reshape(64, 8)
            for (lane, r), (x, y) in probe._coords(L.mfma_operand(plan, "a")).items():
                A[x, y] = a_in[lane, r]
            for (lane, r), (x, y) in probe._coords(L.mfma_operand(plan, "b")).items():
                B[x, y] = b_in[lane, r]
            C = A @ B
            o = out.reshape(64, 16)
            for (lane, r), (x, y) in probe._coords(L.mfma_acc(plan)).items():
                x, y = self.acc_map(x, y)
                o[lane, r] = C[x, y]
        return run


@pytest.mark.parametrize("m", [32, 16])
def test_probe_accepts_the_emitters_maps_and_rejects_others(monkeypatch, m):
    import enceladus_amd.runtime.raw as raw
    monkeypatch.setattr(raw, "hip_kernel", lambda src, name: _EmulatedKernel(m, lambda x, y: (x, y)))
    assert probe._probe_shape(m)
    monkeypatch.setattr(raw, "hip_kernel", lambda src, name: _EmulatedKernel(m, lambda x, y: (y, x)))
    assert not probe._probe_shape(m)


def test_a_failed_probe_raises_compilation_error(monkeypatch):
    import enceladus
    monkeypatch.setattr(probe, "_ok", None)
    monkeypatch.setattr(probe, "_probe_shape", lambda m: False)

    class _Caps:
        name, architecture = "emulated", "gfx950"

    class _Dev:
        caps = _Caps()
    import enceladus_amd.runtime.device as D
    monkeypatch.setattr(D, "get_device", lambda: _Dev())
    with pytest.raises(enceladus.CompilationError, match="MFMA register layout"):
        probe.check_mfma_layout()


@pytest.mark.gpu
def test_probe_passes_on_this_gpu_before_the_first_mfma_kernel():
    import torch

    from examples.matmul import matmul
    print("[case] MFMA lane-map probe", flush=True)
    assert probe._probe_shape(32) and probe._probe_shape(16)
    a = torch.randn(64, 64, dtype=torch.float16, device="cuda")
    c = matmul(a, a)
    torch.cuda.synchronize()
    assert probe._ok is True
    torch.testing.assert_close(c.float(), a.float() @ a.float(), rtol=2e-3, atol=2e-2)
