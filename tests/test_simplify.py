"""The simplifier, the constant folder and the IR verifier (reference test strategy:
tests/test_simplify.py, folding equals the interpreter; compiler/ir.py:788-851 verifier).

CPU: every binary, unary and conversion op the folder evaluates is compared bit for bit
with the oracle interpreter on edge values of every dtype (the folder is the product's own
restatement; the oracle is the checker); kernels of constant expressions fold to constants;
loop-invariant scalars leave their loop; identical pure ops merge; malformed IR is refused
with the stage and op named. GPU: a folded kernel stores the interpreter's values.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

import enceladus
import enceladus.language as tl
from enceladus_amd.compiler import fold, frontend, ir, simplify, verify
from enceladus_amd.compiler.errors import CompilationError
from enceladus_amd.language import core
from oracle import interpreter as O

INTS = [core.int8, core.int16, core.int32, core.int64, core.uint8, core.uint16,
        core.uint32, core.uint64]
FLOATS = [core.float16, core.bfloat16, core.float32]


def _edges(dt):
    if dt.is_floating():
        vals = [0.0, -0.0, 1.0, -1.0, 0.5, 3.0, -2.75, 1e-3, 65504.0, 1e30, -1e30,
                float("inf"), float("-inf"), float("nan"), 1.0 / 3.0, 7.25]
        return [fold.scalar(v, dt) for v in vals]
    lo, hi = O.int_range(O.as_dtype(dt.long_name))
    vals = {0, 1, 2, 3, 7, hi, lo, hi - 1, (hi + 1) // 2, 100 % (hi + 1)}
    if lo < 0:
        vals |= {-1, -2, -7, lo + 1, -100 % (hi + 1) - (hi + 1)}
    return [fold.scalar(v, dt) for v in sorted(vals)]


def _oracle_tile(x, dt):
    odt = O.as_dtype(dt.long_name)
    if dt.is_floating():
        return O.OTile(np.asarray(np.float32(x)), odt)
    return O.OTile(np.asarray(x, odt.np), odt)


def _same(got, want, dt) -> bool:
    if dt.is_floating() or isinstance(want, (np.floating, float)):
        g = np.array([got], np.float32).view(np.uint32)[0]
        w = np.array([want], np.float32).view(np.uint32)[0]
        if math.isnan(float(got)) and math.isnan(float(want)):
            return True
        return g == w
    return int(got) == int(want)


BIN = ["add", "sub", "mul", "div", "floordiv", "mod", "and", "or", "xor", "shl", "shr",
       "min", "max", "eq", "ne", "lt", "le", "gt", "ge"]


@pytest.mark.parametrize("dt", INTS + FLOATS, ids=lambda d: d.name)
def test_binary_folding_matches_the_interpreter(dt):
    vals = _edges(dt)
    checked = 0
    for op in BIN:
        for a in vals:
            for b in vals:
                got = fold.binary(op, a, b, dt)
                if got is None:
                    continue
                want = O.binary(op, _oracle_tile(a, dt), _oracle_tile(b, dt)).data
                assert _same(got, want.item(), dt), (op, dt.name, a, b, got, want)
                checked += 1
    assert checked > 100


UN = ["neg", "abs", "not", "exp", "exp2", "log", "log2", "sqrt", "rsqrt", "sin", "cos",
      "tanh", "sigmoid", "erf", "floor", "ceil"]


@pytest.mark.parametrize("dt", INTS + FLOATS, ids=lambda d: d.name)
def test_unary_folding_matches_the_interpreter(dt):
    checked = 0
    for op in UN:
        for a in _edges(dt):
            got = fold.unary(op, a, dt)
            if got is None:
                continue
            want = O.unary(op, _oracle_tile(a, dt)).data
            assert _same(got, want.item(), dt), (op, dt.name, a, got, want)
            checked += 1
    assert checked > 10


@pytest.mark.parametrize("src", INTS + FLOATS + [core.int1], ids=lambda d: d.name)
def test_conversion_folding_matches_the_interpreter(src):
    vals = _edges(src) if src is not core.int1 else [np.bool_(False), np.bool_(True)]
    for dst in INTS + FLOATS + [core.int1]:
        for a in vals:
            got = fold.cast(a, src, dst)
            if got is None:
                continue
            t = _oracle_tile(a, src) if src is not core.int1 else O.OTile(np.asarray(a),
                                                                           O.int1)
            want = t.to(O.as_dtype(dst.long_name)).data
            assert _same(got, want.item(), dst), (src.name, dst.name, a, got, want)


def test_undefined_cases_stay_unfolded():
    assert fold.binary("floordiv", np.int32(5), np.int32(0), core.int32) is None
    assert fold.binary("mod", np.int32(-2 ** 31), np.int32(-1), core.int32) is None
    assert fold.binary("shl", np.int32(1), np.int32(32), core.int32) is None
    assert fold.binary("shr", np.int32(1), np.int32(-1), core.int32) is None
    assert fold.unary("neg", np.int32(-2 ** 31), core.int32) is None
    assert fold.cast(np.float32("nan"), core.float32, core.int32) is None
    assert fold.cast(np.float32(3e9), core.float32, core.int32) is None
    # and a plausible mistake fails: C division truncates toward zero, not down
    assert int(fold.binary("floordiv", np.int32(-7), np.int32(2), core.int32)) == -3
    assert int(fold.binary("mod", np.int32(-7), np.int32(2), core.int32)) == -1


def _ir(kernel, types, consts, facts=None):
    facts = facts or {k: {} for k in types}
    return frontend.build_ir(kernel.fn, types, facts, consts)


@enceladus.jit
def _all_constant(out_ptr, n, B: tl.constexpr):
    r = tl.arange(0, B)
    c = tl.full((B,), 7, tl.int32)
    v = ((c * 3 - 1) // 4).to(tl.float32) + 0.5
    if (n * 0 + 2) * 1 > 1:
        tl.store(out_ptr + r, tl.where(v > 5.0, v, -v))
    else:
        tl.store(out_ptr + r, v)


_F32P = ir.TType((), core.float32, ptr=True)
_I32 = ir.TType((), core.int32)


def test_constant_expressions_fold_away():
    fn = _ir(_all_constant, {"out_ptr": _F32P, "n": _I32}, {"B": 64})
    before = {op.name for op in ir.walk(fn.body)}
    assert {"binary", "cast", "if"} <= before
    simplify.simplify(fn)
    verify.verify(fn, "test")
    names = [op.name for op in ir.walk(fn.body)]
    assert not {"binary", "cast", "select", "if"} & set(names), names
    consts = [op.attrs["value"] for op in ir.walk(fn.body) if op.name == "const"
              and op.result.type.dtype is core.float32]
    assert 5.5 in consts


@enceladus.jit
def _loop_invariant(out_ptr, x_ptr, n, scale, BLOCK: tl.constexpr):
    offs = tl.arange(0, BLOCK)
    acc = tl.zeros([BLOCK], tl.float32)
    for i in range(0, n):
        s = scale * 2.0 + 1.0          # loop-invariant scalar work
        t = scale * 2.0 + 1.0          # the same again
        acc += tl.load(x_ptr + i * BLOCK + offs) * s + t
    tl.store(out_ptr + offs, acc)


def test_invariants_leave_the_loop_and_duplicates_merge():
    types = {"out_ptr": _F32P, "x_ptr": _F32P, "n": _I32,
             "scale": ir.TType((), core.float32)}
    fn = _ir(_loop_invariant, types, {"BLOCK": 64})
    simplify.simplify(fn)
    verify.verify(fn, "test")
    loop = next(op for op in fn.body.ops if op.name == "for")
    body = [op for op in loop.regions[0].ops]
    scale = fn.args[3]
    muls = [op for op in ir.walk(fn.body) if op.name == "binary" and op.attrs["op"] == "mul"
            and scale in op.operands]
    # `scale * 2.0` once, in front of the loop, and its `+ 1.0` with it
    assert len(muls) == 1 and muls[0] in fn.body.ops
    adds = [op for op in fn.body.ops if op.name == "binary" and op.attrs["op"] == "add"
            and muls[0].result in op.operands]
    assert len(adds) == 1
    assert not any(op.name == "binary" and not op.result.type.shape and
                   op.result.type.dtype is core.float32 for op in body)


def test_identities_hold_for_every_value():
    @enceladus.jit
    def k(out_ptr, x_ptr, f_ptr, BLOCK: tl.constexpr):
        o = tl.arange(0, BLOCK)
        x = tl.load(x_ptr + o)
        f = tl.load(f_ptr + o)
        tl.store(out_ptr + o, ((x + 0) * 1 - 0) // 1 | 0)
        tl.store(f_ptr + o, f * 1.0 / 1.0 - 0.0 + (f * 0.0))
    i32p = ir.TType((), core.int32, ptr=True)
    fn = _ir(k, {"out_ptr": i32p, "x_ptr": i32p, "f_ptr": _F32P}, {"BLOCK": 64})
    simplify.simplify(fn)
    ops = [op.attrs.get("op") for op in ir.walk(fn.body) if op.name == "binary"]
    # integer chain gone; the float `f * 0.0` (not an identity: -0.0, NaN, inf) and the
    # `+` that adds it stay
    assert sorted(ops) == ["add", "mul"], ops


def test_verifier_refuses_malformed_ir():
    fn = _ir(_loop_invariant, {"out_ptr": _F32P, "x_ptr": _F32P, "n": _I32,
                               "scale": ir.TType((), core.float32)}, {"BLOCK": 64})
    verify.verify(fn, "the frontend")
    # a use before its definition
    ops = fn.body.ops
    i = next(k for k, op in enumerate(ops) if op.name == "for")
    bad = list(ops)
    bad.insert(0, bad.pop(i))
    fn.body.ops = bad
    with pytest.raises(CompilationError, match="before its definition"):
        verify.verify(fn, "a test")
    fn.body.ops = ops
    # a binary op whose operand dtypes differ
    b = next(op for op in ir.walk(fn.body) if op.name == "binary")
    saved = b.operands[1]
    b.operands[1] = fn.args[2]            # the int32 `n`
    if b.operands[0].type.dtype is core.int32:
        b.operands[1] = fn.args[3]        # the float32 `scale`
    with pytest.raises(CompilationError, match="after a test.*binary"):
        verify.verify(fn, "a test")
    b.operands[1] = saved
    # a loop body that does not end with yield
    loop = next(op for op in fn.body.ops if op.name == "for")
    y = loop.regions[0].ops.pop()
    with pytest.raises(CompilationError, match="yield"):
        verify.verify(fn, "a test")
    loop.regions[0].ops.append(y)
    verify.verify(fn, "a test")


@pytest.mark.gpu
def test_folded_kernel_matches_the_interpreter():
    out = np.zeros(64, np.float32)
    _all_constant[(1,)](out, 3, B=64)
    want = np.zeros(64, np.float32)
    O.run_grid(_all_constant, (1,), want, 3, B=64)
    np.testing.assert_array_equal(out, want)
    np.testing.assert_array_equal(out, np.full(64, 5.5, np.float32))
