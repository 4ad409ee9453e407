"""A once-per-process check of the MFMA lane maps that `tl.dot` codegen assumes.

The reference probes its `simdgroup_matrix` fragment layout on first use, because Metal
leaves it unspecified (reference: runtime/device.py:108-145, called from
runtime/compile.py:159-160 when a kernel uses simdgroup matrices). AMD documents the MFMA
register layouts, and the emitter's lane maps (`compiler/layout.py`: `mfma_operand`,
`mfma_acc`) are pinned by the GPU parity suite, but a code object that runs on a device with
other maps would compute wrong products silently. So before the first kernel with an MFMA
loads, one hand-written probe per instruction shape multiplies two small integer matrices
whose fragments are placed exactly where the layouts say, and every lane's accumulator
registers are compared with the product at the coordinates `mfma_acc` assigns them.
"""

from __future__ import annotations

import threading

import numpy as np

_SRC = r"""
#include "enceladus_cdna4.h"
extern "C" __global__ void ek_mfma_probe(const _Float16* a, const _Float16* b, float* out) {
  const int lane = threadIdx.x & 63;
  _Float16 fa[8], fb[8];
  for (int j = 0; j < 8; ++j) { fa[j] = a[lane * 8 + j]; fb[j] = b[lane * 8 + j]; }
  float acc[16];
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
  if (SHAPE == 32) ek::mfma_32x32x16(acc, fa, fb);
  else ek::mfma_16x16x32(acc, fa, fb);
  for (int r = 0; r < NREG; ++r) out[lane * 16 + r] = acc[r];
}
"""

_lock = threading.Lock()
_ok: bool | None = None


def _coords(lay):
    """{(lane, reg): tile coordinate} of a one-wave layout."""
    out = {}
    for lane in range(64):
        t = lay.thread_coord(lane, 0)
        for r in range(lay.nregs):
            c = lay.reg_coord(r)
            out[(lane, r)] = tuple(x + y for x, y in zip(t, c))
    return out


def _probe_shape(m: int) -> bool:
    from enceladus_amd.compiler import layout as L
    from enceladus_amd.runtime.raw import hip_kernel
    # the emitter's own plan for one wave and one instruction of this shape
    plan = L.plan_dot(m, m, 16 if m == 32 else 32, 1, "fp16")
    inst = plan.inst
    assert (inst.m, inst.kpl) == (m, 8), inst
    rng = np.random.default_rng(2024)
    A = rng.integers(-4, 5, (inst.m, inst.k)).astype(np.float16)
    B = rng.integers(-4, 5, (inst.k, inst.n)).astype(np.float16)
    want = A.astype(np.float32) @ B.astype(np.float32)          # exact: small integers
    a_in = np.zeros((64, 8), np.float16)
    b_in = np.zeros((64, 8), np.float16)
    for (lane, r), (i, k) in _coords(L.mfma_operand(plan, "a")).items():
        a_in[lane, r] = A[i, k]
    for (lane, r), (k, j) in _coords(L.mfma_operand(plan, "b")).items():
        b_in[lane, r] = B[k, j]
    acc = L.mfma_acc(plan)
    nreg = acc.nregs
    src = _SRC.replace("SHAPE", str(m)).replace("NREG", str(nreg))
    k = hip_kernel(src, "ek_mfma_probe")
    out = np.zeros((64, 16), np.float32)
    k[(1,), (64,)](a_in.ravel(), b_in.ravel(), out.ravel())
    got = out.reshape(64, 16)
    return all(got[lane, r] == want[i, j] for (lane, r), (i, j) in _coords(acc).items())


def check_mfma_layout() -> None:
    """Runs the probes once per process (the first MFMA kernel to load calls this).

    Raises:
        enceladus.CompilationError: the device's MFMA lane maps differ from the emitter's.
    """
    global _ok
    if _ok is None:
        with _lock:
            if _ok is None:
                _ok = _probe_shape(32) and _probe_shape(16)
    if not _ok:
        from enceladus_amd.compiler.errors import CompilationError
        from enceladus_amd.runtime.device import get_device
        raise CompilationError(
            "this GPU's MFMA register layout differs from the one the tl.dot lowering "
            "assumes, so tl.dot can't run here. Report this to the maintainers with the "
            f"device name, {get_device().caps.name} ({get_device().caps.architecture}).")
