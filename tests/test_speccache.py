"""The persistent specialization cache (CPU: hiprtc compiles without a GPU).

A second process that compiles the same specialization must not run the frontend or the
code generator; changing a global the kernel reads, the kernel's source, or the
specialization must compile again (reference: runtime/compile.py:38-47, cache.py:97-144)."""

import os
import subprocess
import sys
import textwrap

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

KERNEL = '''
import enceladus
import enceladus.language as tl

SCALE = {scale}


@enceladus.jit
def scaled_copy(x_ptr, out_ptr, n, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    tl.store(out_ptr + offs, tl.load(x_ptr + offs, mask=m) * SCALE, mask=m)
'''

PROBE = '''
import sys
sys.path.insert(0, {root!r}); sys.path.insert(0, {tmp!r})
import numpy as np
from enceladus_amd.runtime import compile as C
calls = []
real = C.build_module
def counting(*a, **k):
    calls.append(1)
    return real(*a, **k)
C.build_module = counting
import kmod
x = np.zeros({n}, np.float32)
ck = kmod.scaled_copy.warmup(x, x, {n}, BLOCK=256)
print("BUILDS", len(calls), "NAME", ck.name, "ARGS", [a.name for a in ck.args])
'''


def _run(tmp, scale, n=1000):
    with open(os.path.join(tmp, "kmod.py"), "w") as f:
        f.write(KERNEL.format(scale=scale))
    env = dict(os.environ, ENCELADUS_CACHE_DIR=os.path.join(tmp, "cache"),
               PYTHONDONTWRITEBYTECODE="1")
    env.pop("ENCELADUS_ALWAYS_COMPILE", None)
    out = subprocess.run([sys.executable, "-c", textwrap.dedent(PROBE.format(
        root=ROOT, tmp=tmp, n=n))], env=env, capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    line = [ln for ln in out.stdout.splitlines() if ln.startswith("BUILDS")][0]
    return int(line.split()[1]), line


def test_second_process_skips_the_frontend(tmp_path):
    tmp = str(tmp_path)
    builds, first = _run(tmp, 2.0)
    assert builds == 1
    builds, second = _run(tmp, 2.0)
    assert builds == 0, "a cached specialization ran the frontend again"
    assert first.split("NAME")[1] == second.split("NAME")[1]


def test_changed_global_or_specialization_compiles_again(tmp_path):
    tmp = str(tmp_path)
    assert _run(tmp, 2.0)[0] == 1
    assert _run(tmp, 3.0)[0] == 1          # SCALE changed: the fingerprint differs
    assert _run(tmp, 3.0)[0] == 0
    assert _run(tmp, 3.0, n=1024)[0] == 1  # n divisible by 16: another specialization


def test_compiler_hash_covers_the_runtime_sources(tmp_path):
    """The pass pipeline (runtime/compile.py) and the argument facts (runtime/jit.py) decide
    generated code too: editing either changes the hash every persistent key includes."""
    import shutil
    from pathlib import Path

    from enceladus_amd.runtime import speccache
    pkg = Path(speccache.__file__).resolve().parent.parent
    names = {p.relative_to(pkg).as_posix() for p in speccache.hashed_sources(pkg)}
    for must in ("runtime/compile.py", "runtime/jit.py", "compiler/codegen_hip.py",
                 "language/ops.py", "csrc/include/enceladus_cdna4.h"):
        assert must in names
    copy = tmp_path / "pkg"
    shutil.copytree(pkg, copy, ignore=shutil.ignore_patterns("__pycache__", "*.so"))
    before = speccache.tree_hash(copy).hexdigest()
    for rel in ("runtime/jit.py", "runtime/compile.py"):
        f = copy / rel
        f.write_text(f.read_text() + "\n# edited\n")
        after = speccache.tree_hash(copy).hexdigest()
        assert after != before
        before = after


def test_source_hash_is_not_inherited_by_a_new_function():
    """The source-hash memo holds its functions weakly and checks the code object, so a
    function created after another was collected never reuses the other's hash."""
    import gc

    from enceladus_amd.runtime import speccache
    ns = {}
    exec("def f():\n    return 1\n", ns)
    f = ns["f"]
    assert speccache._source_hash(f) is None        # no source file: nothing cached
    h = speccache._source_hash(test_source_hash_is_not_inherited_by_a_new_function)
    assert h == speccache._source_hash(test_source_hash_is_not_inherited_by_a_new_function)
    del f, ns
    gc.collect()
    assert all(k is not None for k in speccache._src_hash.keys())
