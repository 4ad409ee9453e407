"""Builds libenceladus_hip.so in-tree: the host shim with g++ against the HIP headers, the
static scratch array of the no-allocation launch with hipcc (kernels come from hiprtc).

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
    obj = HERE / "enceladus_scratch.o"
    # The static scratch array of ek_launch_flush_noalloc is device memory: hipcc, gfx950.
    hip_cmd = ["hipcc", "-c", "-fPIC", "-O2", "-std=c++17", "--offload-arch=gfx950",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
               f"-I{ROOT / 'include'}", str(HERE / "enceladus_scratch.hip"), "-o", str(obj)]
    # The rest is host-only code: g++ against the HIP headers, no device pass.
    cmd = ["g++", "-O2", "-fPIC", "-shared", "-std=c++17", "-D__HIP_PLATFORM_AMD__",
           f"-I{ROCM / 'include'}", f"-I{ROOT / 'include'}", str(src), str(obj), "-o",
           str(tmp), f"-L{ROCM / 'lib'}", f"-Wl,-rpath,{ROCM / 'lib'}", "-lhiprtc",
           "-lamdhip64"]
    for c in (hip_cmd, cmd):
        if verbose:
            print(" ".join(c), flush=True)
        subprocess.run(c, check=True)
    os.replace(tmp, LIB)
    obj.unlink(missing_ok=True)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print(LIB)
