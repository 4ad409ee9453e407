"""The Python operator API against the reference's signatures, name by name (CPU).

`tests/golden/api_signatures.json` holds the reference's public signatures, parsed (not
imported) from its source by `tests/golden/make_api_signatures.py`; each row cites the
reference file:line of its definition. Drop-in code written for the reference must bind
the same way here, so for every row:

- the positional parameters match in order, name, kind and default (a parameter the
  reference requires may have a default here: that only accepts more calls);
- every keyword-only parameter of the reference exists here with the same default;
- `**kwargs` is present exactly when the reference has it;
- extra parameters are allowed only as keyword-only ones with defaults (they cannot
  change how a reference-valid call binds).

Module identity is checked as well: `enceladus.X` and `enceladus_amd.X` are one module
object, so an `except` on a class imported through either path catches the other's.
"""

from __future__ import annotations

import ast
import importlib
import inspect
import json
import os

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
TABLE = json.load(open(os.path.join(HERE, "golden", "api_signatures.json")))

_POSITIONAL = (inspect.Parameter.POSITIONAL_ONLY, inspect.Parameter.POSITIONAL_OR_KEYWORD,
               inspect.Parameter.VAR_POSITIONAL)


def _resolve(path: str):
    import enceladus  # noqa: F401  (installs the alias)
    parts = path.split(".")
    obj = importlib.import_module(parts[0])
    for p in parts[1:]:
        obj = getattr(obj, p)
    return obj


def _signature(obj):
    if inspect.isclass(obj):
        return inspect.signature(obj.__init__)
    return inspect.signature(obj)


def _default_matches(ref_text, ours) -> bool:
    if ref_text is None:
        return True         # required there: a default here only accepts more calls
    if ours is inspect.Parameter.empty:
        return False
    want = ast.literal_eval(ref_text)
    return type(want) is type(ours) and want == ours


@pytest.mark.parametrize("row", TABLE, ids=[r["name"] for r in TABLE])
def test_signature_matches_reference(row):
    obj = _resolve(row["name"])
    sig = _signature(obj)
    ours = list(sig.parameters.values())
    ref = row["params"]
    where = f"{row['name']} (reference {row['ref']})"

    ref_pos = [p for p in ref if p[1] in {k.name for k in _POSITIONAL}]
    our_pos = [p for p in ours if p.kind in _POSITIONAL]
    assert [(p.name, p.kind.name) for p in our_pos] == [(n, k) for n, k, _ in ref_pos], \
        f"{where}: positional parameters {[(p.name, p.kind.name) for p in our_pos]}"
    for (n, _, d), p in zip(ref_pos, our_pos):
        assert _default_matches(d, p.default), f"{where}: default of `{n}` is {p.default!r}, " \
                                               f"reference {d}"

    by_name = {p.name: p for p in ours}
    ref_names = {n for n, _, _ in ref}
    for n, k, d in ref:
        if k == "KEYWORD_ONLY":
            assert n in by_name and by_name[n].kind == inspect.Parameter.KEYWORD_ONLY, \
                f"{where}: keyword-only `{n}` missing"
            assert _default_matches(d, by_name[n].default), \
                f"{where}: default of `{n}` is {by_name[n].default!r}, reference {d}"
    ref_kw = any(k == "VAR_KEYWORD" for _, k, _ in ref)
    our_kw = any(p.kind == inspect.Parameter.VAR_KEYWORD for p in ours)
    assert ref_kw == our_kw, f"{where}: **kwargs present here: {our_kw}, reference: {ref_kw}"
    for p in ours:
        if p.name not in ref_names and p.kind != inspect.Parameter.VAR_KEYWORD:
            assert p.kind == inspect.Parameter.KEYWORD_ONLY and \
                p.default is not inspect.Parameter.empty, \
                f"{where}: extra parameter `{p.name}` ({p.kind.name}) changes how calls bind"


def test_table_covers_the_tl_namespace():
    """Every public `tl` name that is callable has a row (reference
    src/enceladus/language/__init__.py:86-97 `__all__`)."""
    import enceladus.language as tl
    rows = {r["name"].rsplit(".", 1)[1] for r in TABLE if r["group"] == "tl"}
    not_ops = {"bfloat16", "float16", "float32", "int1", "int8", "int16", "int32", "int64",
               "uint8", "uint16", "uint32", "uint64", "constexpr", "dtype", "math"}
    ref_all = (
        "abs arange argmax argmin bfloat16 broadcast_to cast cdiv ceil clamp constexpr cos dot "
        "dtype erf exp exp2 expand_dims float16 float32 floor fma full full_like int1 int8 "
        "int16 int32 int64 join load log log2 make_tensor_descriptor math max maximum min "
        "minimum num_programs permute program_id range reduce reshape rsqrt sigmoid sin split "
        "sqrt static_assert static_print static_range store sum tanh trans uint8 uint16 uint32 "
        "uint64 where zeros zeros_like associative_scan atomic_add atomic_and atomic_cas "
        "atomic_max atomic_min atomic_or atomic_xchg atomic_xor cumsum debug_barrier "
        "device_assert device_print max_contiguous multiple_of").split()
    for n in ref_all:
        assert hasattr(tl, n), f"tl.{n} missing"
    assert set(ref_all) - not_ops == rows


def test_missing_tl_name_is_a_compilation_error():
    """reference language/__init__.py:100-115: a missing name raises an error that is a
    CompilationError and an AttributeError (so `hasattr` still works)."""
    import enceladus
    import enceladus.language as tl
    assert not hasattr(tl, "no_such_op")
    with pytest.raises(enceladus.CompilationError):
        tl.no_such_op  # noqa: B018
    with pytest.raises(AttributeError, match="float64"):
        tl.float64  # noqa: B018


SUBMODULES = [
    "compiler", "compiler.errors", "compiler.ir", "compiler.frontend", "compiler.semantic",
    "compiler.layout", "compiler.explain", "compiler.pipeline", "runtime", "runtime.autotuner", "runtime.jit",
    "runtime.device", "runtime.tensor", "runtime.debug", "runtime.raw", "language",
    "language.core", "language.ops", "language.math", "configs", "testing",
]


@pytest.mark.parametrize("name", SUBMODULES)
def test_submodule_identity(name):
    import enceladus  # noqa: F401
    a = importlib.import_module(f"enceladus.{name}")
    b = importlib.import_module(f"enceladus_amd.{name}")
    assert a is b


def test_compilation_error_is_one_class():
    """reference tests/test_axis_info.py:10-12 and tests/test_autotune.py:12 import these
    through their submodules."""
    import enceladus
    from enceladus.compiler.errors import CompilationError, DeviceAssertionError
    from enceladus.runtime.autotuner import Config
    assert enceladus.compiler.errors.CompilationError is enceladus.CompilationError
    assert CompilationError is enceladus.CompilationError
    assert DeviceAssertionError is enceladus.DeviceAssertionError
    assert Config is enceladus.Config
    import enceladus_amd
    assert enceladus.testing is enceladus_amd.testing
    assert enceladus.configs is enceladus_amd.configs


def test_config_matches_reference_dataclass():
    """reference runtime/autotuner.py:54-103: positional order, dot_backend check, JSON."""
    import enceladus
    c = enceladus.Config({"BM": 64}, 8, (4, 2))
    assert c.num_warps == 8 and c.dot_warps == (4, 2) and c.dot_backend == "auto"
    assert c.launch_options() == {"num_warps": 8, "dot_warps": (4, 2)}
    with pytest.raises(ValueError, match="dot_backend"):
        enceladus.Config({}, dot_backend="bogus")
    assert enceladus.Config.from_json(c.to_json()) == c
    assert str(c) == "enceladus.Config({'BM': 64}, num_warps=8, dot_warps=(4, 2))"
    m = enceladus.Config({"BM": 64}, dot_backend="mpp")
    assert m.launch_options() == {"num_warps": 4, "dot_backend": "mpp"}


def test_default_tolerance_matches_reference():
    """reference testing.py:66-75."""
    import numpy as np

    import enceladus
    from enceladus.language import core
    t = enceladus.testing.default_tolerance
    assert t(np.float32) == (1e-5, 1e-5)
    assert t(np.float16) == (2e-3, 2e-3)
    assert t(core.bfloat16) == (2e-2, 2e-2)
    assert t(np.int32) == (0.0, 0.0)


def test_cdiv():
    import enceladus
    assert enceladus.cdiv(x=10, div=4) == 3
    assert enceladus.cdiv(8, 4) == 2


def test_warmup_and_explain_accept_dot_backend(capsys):
    """reference runtime/jit.py:527-570: `dot_backend` is accepted by warmup and explain
    ("mpp" and "simdgroup" lower to MFMA here) and an unknown name raises ValueError."""
    import numpy as np

    from tests.test_explain import _transposed_sum
    a = np.zeros((64, 64), np.float32)
    out = np.zeros(64, np.float32)
    ck = _transposed_sum.warmup(a, a, out, N=64, dot_backend="mpp")
    assert ck is _transposed_sum.warmup(a, a, out, N=64)
    text = _transposed_sum.explain(a, a, out, grid=(1,), N=64, dot_backend="simdgroup")
    assert text in capsys.readouterr().out          # printed and returned, as there
    for call in (lambda: _transposed_sum.warmup(a, a, out, N=64, dot_backend="bogus"),
                 lambda: _transposed_sum.explain(a, a, out, N=64, dot_backend="bogus"),
                 lambda: _transposed_sum[(1,)](a, a, out, N=64, dot_backend="bogus")):
        with pytest.raises(ValueError, match="dot_backend"):
            call()
    f = _transposed_sum.ir(a, a, out, N=64)
    assert f.name


def _scalar_kernel_src():
    import enceladus
    import enceladus.language as tl

    @enceladus.jit
    def k(x, C: tl.constexpr):
        tl.static_assert(True)
    return k


def test_warm_key_keeps_tuple_constexpr_types_apart():
    """(1,), (1.0,) and (True,) (and (0.0,) against (-0.0,)) are different constexprs:
    the warm-launch key keeps them apart as the general key does."""
    k = _scalar_kernel_src()
    keys = [k._fast_key((3,), {"C": c}, 4, None)[0]
            for c in ((1,), (1.0,), (True,), (0.0,), (-0.0,), [1])]
    assert len(set(keys)) == len(keys)
    assert k._fast_key((3,), {"C": (1,)}, 4, None)[0] == \
        k._fast_key((3,), {"C": (1,)}, 4, None)[0]


def test_warm_key_refuses_extra_positional_arguments():
    """A call with more positional arguments than parameters takes the general path, which
    raises TypeError, instead of launching and ignoring the extras."""
    k = _scalar_kernel_src()
    assert k._fast_key((3, 4, 5), {}, 4, None) is None
    assert k._make_binder(3, (), (3, 4, 5), {})((3, 4, 5), {}, 4, None) is None
    with pytest.raises(TypeError):
        k.bind((3, 4, 5), {})


def test_compile_module_at_the_reference_path():
    """reference tests/test_codegen.py:85-87 compile a kernel's IR through
    `enceladus.compiler.pipeline.compile_module` and compare sources."""
    import numpy as np

    from enceladus.compiler.pipeline import compile_module
    from tests.test_explain import _transposed_sum
    a = np.zeros((64, 64), np.float32)
    out = np.zeros(64, np.float32)
    first = compile_module(_transposed_sum.ir(a, a, out, N=64))
    second = compile_module(_transposed_sum.ir(a, a, out, N=64))
    assert first.source == second.source and "ek__transposed_sum" in first.source
    with pytest.raises(Exception, match="LDS"):
        compile_module(_transposed_sum.ir(a, a, out, N=64), max_threadgroup_memory=16)
