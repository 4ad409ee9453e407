"""`compile_module` at the reference's module path (reference: compiler/pipeline.py:14-38).

`kernel.ir(...)` returns a kernel's IR after the pass pipeline (`runtime.compile.build_module`:
simplify, 64-bit index widening, the attention scale rewrite, DCE, each verified under
ENCELADUS_VERIFY=1); `compile_module` lowers such a module to HIP C++ for gfx950 with the
compile options the module was built with and returns the generated kernel (`.source`,
`.name`, `.lds_bytes`, `.num_warps`), without compiling or launching it.
"""

from __future__ import annotations

from enceladus_amd.compiler import codegen_hip, ir
from enceladus_amd.compiler.errors import CompilationError

LDS_BYTES = 163840      # per workgroup on gfx950


def compile_module(module: ir.Func,
                   max_threadgroup_memory: int = LDS_BYTES) -> codegen_hip.GeneratedKernel:
    """Lowers a module from `kernel.ir(...)` to HIP C++.

    Raises:
        CompilationError: the kernel needs more LDS than `max_threadgroup_memory`, or uses
            something the emitter can't lower.
    """
    gen = codegen_hip.generate(module, dict(module.attrs))
    if gen.lds_bytes > max_threadgroup_memory:
        raise CompilationError(f"{module.name} needs {gen.lds_bytes} bytes of LDS, more than "
                               f"the {max_threadgroup_memory} available")
    return gen
