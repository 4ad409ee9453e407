"""Builds libenceladus_hip.so in-tree with hipcc (host code only; kernels come from hiprtc).

Run `python -m enceladus_amd.csrc.build`. The library links against the HIP runtime and
hiprtc by soname; at load time the Python side decides which copies satisfy them.
"""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
LIB = HERE / "libenceladus_hip.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def build(verbose: bool = False) -> Path:
    src = HERE / "enceladus_hip.cpp"
    tmp = LIB.with_suffix(".so.tmp")
    # Host-only code: g++ against the HIP headers, no device pass.
    cmd = ["g++", "-O2", "-fPIC", "-shared", "-std=c++17", "-D__HIP_PLATFORM_AMD__",
           f"-I{ROCM / 'include'}", f"-I{ROOT / 'include'}", str(src), "-o", str(tmp),
           f"-L{ROCM / 'lib'}", f"-Wl,-rpath,{ROCM / 'lib'}", "-lhiprtc", "-lamdhip64"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB)
