"""Writes `api_signatures.json`: the reference's public signatures, parsed from its source.

Run in a container that has the reference tree (default `/root/reference`):

    python tests/golden/make_api_signatures.py [REFERENCE_ROOT]

The reference is read as text with `ast`; nothing of it is imported or executed. Each
entry records the public name as drop-in code reaches it, the reference file:line of the
definition, and every parameter (name, kind, default as source text). Builtins of the tile
language drop their leading compiler-context parameter, which user code never passes.
`tests/test_api_conformance.py` compares this table with `inspect.signature` of the
MI355X package.
"""

from __future__ import annotations

import ast
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PKG = "src/enceladus"

# (public name, reference file under src/enceladus, qualified definition, drop first param)
# A dataclass definition yields its generated __init__ (fields in order, self first).
ENTRIES = [
    ("enceladus.jit", "runtime/jit.py", "jit", False),
    ("enceladus.cdiv", "runtime/jit.py", "cdiv", False),
    ("enceladus.next_power_of_2", "runtime/jit.py", "next_power_of_2", False),
    ("enceladus.JITFunction.__init__", "runtime/jit.py", "JITFunction.__init__", False),
    ("enceladus.JITFunction.__getitem__", "runtime/jit.py", "JITFunction.__getitem__", False),
    ("enceladus.JITFunction.bind", "runtime/jit.py", "JITFunction.bind", False),
    ("enceladus.JITFunction.specialize", "runtime/jit.py", "JITFunction.specialize", False),
    ("enceladus.JITFunction.ir", "runtime/jit.py", "JITFunction.ir", False),
    ("enceladus.JITFunction.run", "runtime/jit.py", "JITFunction.run", False),
    ("enceladus.JITFunction.warmup", "runtime/jit.py", "JITFunction.warmup", False),
    ("enceladus.JITFunction.explain", "runtime/jit.py", "JITFunction.explain", False),
    ("enceladus.autotune", "runtime/autotuner.py", "autotune", False),
    ("enceladus.heuristics", "runtime/autotuner.py", "heuristics", False),
    ("enceladus.Config", "runtime/autotuner.py", "Config", False),
    ("enceladus.Config.launch_options", "runtime/autotuner.py", "Config.launch_options", False),
    ("enceladus.Config.to_json", "runtime/autotuner.py", "Config.to_json", False),
    ("enceladus.Config.from_json", "runtime/autotuner.py", "Config.from_json", True),
    ("enceladus.get_device", "runtime/device.py", "get_device", False),
    ("enceladus.Capabilities", "runtime/device.py", "Capabilities", False),
    ("enceladus.synchronize", "runtime/stream.py", "synchronize", False),
    ("enceladus.capture", "runtime/debug.py", "capture", False),
    ("enceladus.lazy_mlx", "runtime/mlx_lazy.py", "lazy_mlx", False),
    ("enceladus.async_numpy", "runtime/interop.py", "async_numpy", False),
    ("enceladus.element_strides", "runtime/interop.py", "element_strides", False),
    ("enceladus.element_dtype", "runtime/interop.py", "element_dtype", False),
    ("enceladus.new_empty", "runtime/interop.py", "new_empty", False),
    ("enceladus.new_zeros", "runtime/interop.py", "new_zeros", False),
    ("enceladus.empty", "runtime/tensor.py", "empty", False),
    ("enceladus.full", "runtime/tensor.py", "full", False),
    ("enceladus.zeros", "runtime/tensor.py", "zeros", False),
    ("enceladus.ones", "runtime/tensor.py", "ones", False),
    ("enceladus.randn", "runtime/tensor.py", "randn", False),
    ("enceladus.rand", "runtime/tensor.py", "rand", False),
    ("enceladus.arange", "runtime/tensor.py", "arange", False),
    ("enceladus.empty_like", "runtime/tensor.py", "empty_like", False),
    ("enceladus.zeros_like", "runtime/tensor.py", "zeros_like", False),
    ("enceladus.from_numpy", "runtime/tensor.py", "from_numpy", False),
    ("enceladus.Tensor.numpy", "runtime/tensor.py", "Tensor.numpy", False),
    ("enceladus.Tensor.tolist", "runtime/tensor.py", "Tensor.tolist", False),
    ("enceladus.Tensor.copy_", "runtime/tensor.py", "Tensor.copy_", False),
    ("enceladus.Tensor.stride", "runtime/tensor.py", "Tensor.stride", False),
    ("enceladus.Tensor.size", "runtime/tensor.py", "Tensor.size", False),
    ("enceladus.Tensor.is_contiguous", "runtime/tensor.py", "Tensor.is_contiguous", False),
    ("enceladus.testing.do_bench", "testing.py", "do_bench", False),
    ("enceladus.testing.default_tolerance", "testing.py", "default_tolerance", False),
    ("enceladus.testing.assert_close", "testing.py", "assert_close", False),
    ("enceladus.configs.matmul_configs", "configs.py", "matmul_configs", False),
    ("enceladus.configs.attention_configs", "configs.py", "attention_configs", False),
]

# tl builtins: (tl name, file, definition). The definition is the compiler-side function
# (first parameter: the compiler context), or the function a factory wraps.
TL_OPS = "language/ops.py"
TL = [(n, TL_OPS, n) for n in (
    "program_id", "num_programs", "arange", "full", "zeros", "zeros_like", "full_like",
    "load", "store", "make_tensor_descriptor", "where", "maximum", "minimum", "fma", "cdiv",
    "clamp", "broadcast_to", "expand_dims", "reshape", "trans", "permute", "join", "split",
    "reduce", "dot", "static_assert", "static_print", "device_print", "device_assert",
    "debug_barrier", "multiple_of", "max_contiguous", "atomic_cas", "cumsum",
    "associative_scan")] + [
    ("abs", TL_OPS, "abs_"), ("sum", TL_OPS, "sum_"), ("max", TL_OPS, "max_"),
    ("min", TL_OPS, "min_"), ("cast", TL_OPS, "_to"),
    # factories: the inner `frontend` of _argminmax / _make_atomic, the math `_make`
    ("argmax", TL_OPS, "_argminmax.frontend"), ("argmin", TL_OPS, "_argminmax.frontend"),
] + [(f"atomic_{k}", TL_OPS, "_make_atomic.frontend")
     for k in ("add", "max", "min", "xchg", "and", "or", "xor")] + [
    (m, "language/math.py", "_make.frontend")
    for m in ("exp", "exp2", "log", "log2", "sqrt", "rsqrt", "sin", "cos", "tanh", "sigmoid",
              "erf", "floor", "ceil")]
# loop ranges: the loop-only frontend takes (*args, **kwargs); the signature user code
# sees is the one its bounds are normalised by (no context parameter)
TL_RANGES = [("range", TL_OPS, "range_bounds"), ("static_range", TL_OPS, "_i_static_range")]

def _find(tree: ast.Module, qual: str):
    node = tree
    for part in qual.split("."):
        body = node.body
        hit = None
        for n in body:
            if isinstance(n, (ast.FunctionDef, ast.ClassDef)) and n.name == part:
                hit = n
        if hit is None:
            raise KeyError(qual)
        node = hit
    return node


def _params(fn: ast.FunctionDef) -> list[list]:
    a = fn.args
    out = []
    pos = a.posonlyargs + a.args
    defaults = [None] * (len(pos) - len(a.defaults)) + list(a.defaults)
    for i, p in enumerate(pos):
        kind = "POSITIONAL_ONLY" if i < len(a.posonlyargs) else "POSITIONAL_OR_KEYWORD"
        d = defaults[i]
        out.append([p.arg, kind, None if d is None else ast.unparse(d)])
    if a.vararg:
        out.append([a.vararg.arg, "VAR_POSITIONAL", None])
    for p, d in zip(a.kwonlyargs, a.kw_defaults):
        out.append([p.arg, "KEYWORD_ONLY", None if d is None else ast.unparse(d)])
    if a.kwarg:
        out.append([a.kwarg.arg, "VAR_KEYWORD", None])
    return out


def _dataclass_init(cls: ast.ClassDef) -> list[list]:
    out = [["self", "POSITIONAL_OR_KEYWORD", None]]
    for n in cls.body:
        if isinstance(n, ast.AnnAssign) and isinstance(n.target, ast.Name):
            d = n.value
            if isinstance(d, ast.Call) and getattr(d.func, "id", "") == "field":
                kw = {k.arg: k.value for k in d.keywords}
                d = kw.get("default")
            out.append([n.target.id, "POSITIONAL_OR_KEYWORD",
                        None if d is None else ast.unparse(d)])
    return out


def main(root: str) -> None:
    src = Path(root) / PKG
    trees: dict[str, ast.Module] = {}

    def tree(f: str) -> ast.Module:
        if f not in trees:
            trees[f] = ast.parse((src / f).read_text())
        return trees[f]

    table = []

    def add(name, f, qual, drop, group):
        node = _find(tree(f), qual)
        if isinstance(node, ast.ClassDef):
            params = _dataclass_init(node)
        else:
            params = _params(node)
        if drop:
            params = params[1:]
        table.append({"name": name, "group": group, "ref": f"{PKG}/{f}:{node.lineno}",
                      "params": params})

    for name, f, qual, drop in ENTRIES:
        add(name, f, qual, drop, "api")
    for name, f, qual in TL:
        add(f"enceladus.language.{name}", f, qual, True, "tl")
    for name, f, qual in TL_RANGES:
        add(f"enceladus.language.{name}", f, qual, False, "tl")
    out = HERE / "api_signatures.json"
    out.write_text("[\n" + ",\n".join(json.dumps(e) for e in table) + "\n]\n")
    print(f"wrote {len(table)} signatures to {out}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
