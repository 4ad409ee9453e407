"""Frontend and JIT behaviour on the CPU: IR shape, compile-time folding, error messages,
specialization keys, and the interpreter-mode boundary."""

import numpy as np
import pytest

import enceladus
import enceladus.language as tl
from enceladus_amd.compiler import ir
from enceladus_amd.compiler.errors import CompilationError


@enceladus.jit
def _loop_kernel(x_ptr, n, BLOCK: tl.constexpr):
    acc = tl.zeros([BLOCK], dtype=tl.float32)
    for i in range(0, n, BLOCK):
        acc += tl.load(x_ptr + i + tl.arange(0, BLOCK), mask=i + tl.arange(0, BLOCK) < n)
    tl.store(x_ptr + tl.arange(0, BLOCK), acc)


def test_runtime_loop_carries_accumulator():
    f = _loop_kernel.ir_for(np.zeros(4, np.float32), 100, BLOCK=64)
    fors = [op for op in ir.walk(f.body) if op.name == "for"]
    assert len(fors) == 1 and len(fors[0].results) == 1
    assert fors[0].results[0].type == ir.TType((64,), enceladus.language.float32)


@enceladus.jit
def _bad_shape(x_ptr, n):
    tl.store(x_ptr + tl.arange(0, 100), 1.0)


def test_non_power_of_two_arange_is_rejected():
    with pytest.raises(CompilationError, match="power-of-two"):
        _bad_shape.ir_for(np.zeros(4, np.float32), 3)


@enceladus.jit
def _while_kernel(x_ptr, n):
    while n > 0:
        n = n - 1


def test_while_is_rejected_with_location():
    with pytest.raises(CompilationError) as e:
        _while_kernel.ir_for(np.zeros(4, np.float32), 3)
    assert "while" in str(e.value) and "test_frontend.py" in str(e.value)


@enceladus.jit
def _dot_bad(a_ptr, BLOCK: tl.constexpr):
    a = tl.load(a_ptr + tl.arange(0, BLOCK)[:, None] * BLOCK + tl.arange(0, BLOCK)[None, :])
    b = tl.load(a_ptr + tl.arange(0, 2 * BLOCK)[:, None] + tl.arange(0, BLOCK)[None, :])
    tl.dot(a, b)


def test_dot_shape_mismatch():
    with pytest.raises(CompilationError, match="inner dimensions"):
        _dot_bad.ir_for(np.zeros(4, np.float16), BLOCK=16)


def test_constexpr_branches_fold():
    @enceladus.jit
    def k(x_ptr, FLAG: tl.constexpr):
        if FLAG:
            tl.store(x_ptr, 1.0)
        else:
            tl.store(x_ptr, 2.0)
    f = k.ir_for(np.zeros(1, np.float32), FLAG=True)
    assert not any(op.name == "if" for op in ir.walk(f.body))


def test_specialization_facts():
    from enceladus_amd.runtime.jit import arg_facts, arg_type
    assert arg_facts(32) == {"divisibility": 16}
    assert arg_facts(1) == {"equal_to_1": True}
    assert arg_type(1 << 40).dtype is tl.int64
    assert arg_type(2.5).dtype is tl.float32


def test_interpreter_mode_is_not_a_product_fallback(monkeypatch):
    monkeypatch.setenv("ENCELADUS_INTERPRET", "1")
    from examples.vector_add import add
    with pytest.raises(RuntimeError, match="oracle"):
        add(np.zeros(4, np.float32), np.zeros(4, np.float32))


def test_calling_kernel_directly_raises():
    with pytest.raises(RuntimeError, match=r"\[grid\]"):
        _loop_kernel(1, 2)


def test_tl_names_outside_kernels_raise():
    with pytest.raises(RuntimeError):
        tl.program_id(0)


# -- join / split / reduce / associative_scan -----------------------------------------

@enceladus.jit
def _join_kernel(x_ptr, y_ptr, CASE: tl.constexpr):
    r = tl.arange(0, 16)
    x = tl.load(x_ptr + r)
    if CASE == "dtype":
        tl.join(x, tl.load(y_ptr + r))
    elif CASE == "literal":
        tl.store(x_ptr + tl.arange(0, 32), tl.reshape(tl.join(x, 3), (32,)))
    elif CASE == "split_shape":
        tl.split(x)
    elif CASE == "pointer":
        tl.join(x_ptr + r, x_ptr + r)
    elif CASE == "plain_combine":
        tl.reduce(x, 0, _plain_add)
    elif CASE == "arity":
        tl.reduce((x, x), 0, _one_of_two)
    elif CASE == "scan_axis":
        tl.associative_scan(x, None, _one_of_two)


def _plain_add(a, b):
    return a + b


@enceladus.jit
def _one_of_two(a0, a1, b0, b1):
    return a0 + b0


def _jk(case, ydt=np.float32):
    return _join_kernel.ir_for(np.zeros(4, np.float32), np.zeros(4, ydt), CASE=case)


def test_join_split_errors():
    with pytest.raises(CompilationError, match="one dtype"):
        _jk("dtype", np.float16)
    f = _jk("literal")
    j = [op for op in ir.walk(f.body) if op.name == "join"][0]
    assert j.result.type == ir.TType((16, 2), tl.float32)
    with pytest.raises(CompilationError, match="last dimension is 2"):
        _jk("split_shape")
    with pytest.raises(CompilationError, match="pointers"):
        _jk("pointer")


def test_combine_function_errors():
    with pytest.raises(CompilationError, match="@enceladus.jit"):
        _jk("plain_combine")
    with pytest.raises(CompilationError, match="returns 1 values for 2 inputs"):
        _jk("arity")
    with pytest.raises(CompilationError, match="needs an `axis`"):
        _jk("scan_axis")


def test_capture_and_lazy_mlx_arguments():
    with pytest.raises(ValueError, match=".json"):
        with enceladus.capture("trace.gputrace"):
            pass
    enceladus.lazy_mlx(False)
    with pytest.raises(NotImplementedError, match="MLX"):
        enceladus.lazy_mlx(True)


@enceladus.jit
def _methods_kernel(x_ptr, out_ptr):
    r = tl.arange(0, 16)
    x = tl.load(x_ptr + r[:, None] * 8 + tl.arange(0, 8)[None, :])
    a = x.permute(1, 0).abs().cast(tl.float16)
    v, i = x.max(axis=1, return_indices=True)
    s = x.sum(axis=0, keep_dims=True)
    tl.store(out_ptr + r, v + i.to(tl.float32) + tl.sum(a.to(tl.float32), 0) * 0.0 +
             tl.sum(s) * 0.0 + x.argmin(1).to(tl.float32))


def test_reference_tile_methods():
    f = _methods_kernel.ir_for(np.zeros(4, np.float32), np.zeros(4, np.float32))
    names = {op.name for op in ir.walk(f.body)}
    assert {"trans", "unary", "cast", "reduce"} <= names


# -- source-located errors (reference strategy: tests/test_frontend.py:24-109) -----------

@enceladus.jit
def _e_loop_type(x_ptr, n, BLOCK: tl.constexpr):
    acc = tl.zeros((BLOCK,), dtype=tl.float32)
    for _ in range(n):  # error
        acc = (acc + 1.0).to(tl.float16)
    tl.store(x_ptr + tl.arange(0, BLOCK), acc)


@enceladus.jit
def _e_or_types(x_ptr, n):
    tl.store(x_ptr, n or 2.5)  # error


@enceladus.jit
def _e_returns(x_ptr):
    return tl.load(x_ptr)  # error


@enceladus.jit
def _e_rec(x):
    return _e_rec(x)  # error


@enceladus.jit
def _e_calls_rec(x_ptr):
    tl.store(x_ptr, _e_rec(1.0))


@enceladus.jit
def _e_if_tile(x_ptr, BLOCK: tl.constexpr):
    x = tl.load(x_ptr + tl.arange(0, BLOCK))
    if x > 0:  # error
        x = -x
    tl.store(x_ptr + tl.arange(0, BLOCK), x)


@pytest.mark.parametrize("kernel,args,kw,phrase", [
    (_e_loop_type, (64,), {"BLOCK": 64}, "loop-carried variable `acc`"),
    (_e_or_types, (64,), {}, "both need the same type"),
    (_e_returns, (), {}, "can't return values"),
    (_e_calls_rec, (), {}, "recursion isn't supported"),
    (_e_if_tile, (), {"BLOCK": 64}, "tl.where"),
])
def test_errors_point_at_the_marked_line(kernel, args, kw, phrase):
    import inspect
    with pytest.raises(CompilationError) as e:
        kernel.ir_for(np.zeros(64, np.float32), *args, **kw)
    msg = str(e.value)
    assert phrase in msg
    fn = _e_rec.fn if kernel is _e_calls_rec else kernel.fn
    lines, start = inspect.getsourcelines(fn)
    off = next(i for i, t in enumerate(lines) if t.rstrip().endswith("# error"))
    assert f"{__file__}:{start + off}:" in msg
    assert lines[off].rstrip() in msg.splitlines()
    assert msg.splitlines()[-1].strip() == "^"


@enceladus.jit
def _h_constexpr(x_ptr, BLOCK):
    tl.store(x_ptr + tl.arange(0, BLOCK), 1.0)  # error


@enceladus.jit
def _h_and_tiles(x_ptr, BLOCK: tl.constexpr):
    x = tl.load(x_ptr + tl.arange(0, BLOCK))
    tl.store(x_ptr + tl.arange(0, BLOCK), x, mask=(x > 0) and (x < 1))  # error


@enceladus.jit
def _h_pow(x_ptr, BLOCK: tl.constexpr):
    x = tl.load(x_ptr + tl.arange(0, BLOCK))
    tl.store(x_ptr + tl.arange(0, BLOCK), x**2)  # error


@enceladus.jit
def _h_print(x_ptr, BLOCK: tl.constexpr):
    x = tl.load(x_ptr + tl.arange(0, BLOCK))
    print(x)  # error


@enceladus.jit
def _h_loopvar(x_ptr, n):
    i = 0.5
    for i in range(n):  # noqa: B007
        pass
    tl.store(x_ptr, i)  # error


@enceladus.jit
def _h_chained(x_ptr, BLOCK: tl.constexpr):
    x = tl.load(x_ptr + tl.arange(0, BLOCK))
    tl.store(x_ptr + tl.arange(0, BLOCK), x, mask=0 < x < 1)  # error


@enceladus.jit
def _h_dict(x_ptr):
    scale = {"a": 2.0}  # error
    tl.store(x_ptr, scale["a"])


@enceladus.jit
def _h_full_range(x_ptr, BLOCK: tl.constexpr):
    tl.store(x_ptr + tl.arange(0, BLOCK), tl.full((BLOCK,), 1e10, tl.int32))  # error


@pytest.mark.parametrize("kernel,args,kw,phrase", [
    (_h_constexpr, (16,), {}, "`BLOCK: tl.constexpr`"),
    (_h_and_tiles, (), {"BLOCK": 16}, "use `&`"),
    (_h_pow, (), {"BLOCK": 16}, "Multiply explicitly"),
    (_h_print, (), {"BLOCK": 16}, "Use tl.device_print"),
    (_h_loopvar, (3,), {}, "Give the loop variable a different name"),
    (_h_chained, (), {"BLOCK": 16}, "`(a < b) & (b < c)`"),
    (_h_dict, (), {}, "Use a compile-time tuple"),
    (_h_full_range, (), {"BLOCK": 16}, "Use a value in that range"),
])
def test_errors_say_what_to_do(kernel, args, kw, phrase):
    """Each error names the marked line and the fix (reference: tests/test_errors.py:24-271)."""
    import inspect
    x = np.zeros(64, np.int32 if kernel is _h_full_range else np.float32)
    with pytest.raises(CompilationError) as e:
        kernel.ir_for(x, *args, **kw)
    msg = str(e.value)
    assert phrase in msg
    lines, start = inspect.getsourcelines(kernel.fn)
    off = next(i for i, t in enumerate(lines) if t.rstrip().endswith("# error"))
    assert f"{__file__}:{start + off}:" in msg


@enceladus.jit
def _down_loop(out_ptr, n, f, STEP: tl.constexpr):
    acc = 0
    for i in range(n, 0, STEP):
        acc += i
    if (n and f) or not acc:      # truth values only: operand types may differ
        acc += 1
    tl.store(out_ptr, acc)


def test_negative_steps_and_truth_contexts_lower():
    import numpy as np
    from enceladus_amd.compiler import codegen_hip
    out = np.zeros(1, np.int32)
    src = codegen_hip.generate(_down_loop.ir_for(out, 10, 0.5, STEP=-3)).source
    assert "_n = " in src and "uint64_t" in src       # the trip-count loop form
    with pytest.raises(enceladus.CompilationError, match="must not be zero"):
        _down_loop.ir_for(out, 10, 0.5, STEP=0)


@enceladus.jit
def _fill(x_ptr, BLOCK: tl.constexpr):
    tl.store(x_ptr + tl.arange(0, 16), 1.0)


@pytest.mark.parametrize("args,kwargs,phrases", [
    (lambda: (np.zeros(64),), {"BLOCK": 16}, ["argument `x_ptr`", "astype(np.float32)"]),
    (lambda: (np.zeros(64, np.float32),), {}, ["missing a required argument: 'BLOCK'"]),
    (lambda: (np.zeros(64, np.float32),), {"BLOCK": {16: 16}}, ["parameter `BLOCK`", "a tuple"]),
])
def test_bad_arguments_name_the_kernel_and_argument(args, kwargs, phrases):
    with pytest.raises(TypeError) as e:
        _fill.warmup(*args(), **kwargs)
    msg = str(e.value)
    assert msg.startswith("_fill: ")
    for p in phrases:
        assert p in msg


def test_generated_binder_matches_the_generic_key():
    """The per-call-shape binder of the warm launch path computes exactly the key and
    runtime values of the generic key function, and declines (None) when an argument's type
    differs from the shape's first call (reference: runtime/jit.py:422-461). Scalar
    arguments only: the device-pointer case is checked on the GPU."""
    import enceladus
    import enceladus.language as tl

    @enceladus.jit
    def s(n, a, flag, BLOCK: tl.constexpr, S: tl.constexpr, NAME: tl.constexpr = "x"):
        pass

    cases = [((16, 2.0, True), {"BLOCK": 64, "S": 0.5}),
             ((17, -2.0, False), {"BLOCK": 64, "S": -0.0, "NAME": "y"}),
             ((1, 0.0, True), {"S": 1.5, "BLOCK": 128}),
             ((1 << 40, 3.0, False), {"BLOCK": 64, "S": 0.5})]
    for args, kw in cases:
        b = s._make_binder(len(args), tuple(kw), args, kw)
        for nw, dw in ((4, None), (8, (8, 1))):
            assert b(args, kw, nw, dw) == s._fast_key(args, kw, nw, dw)
        # another type in the same call shape: the binder declines, the generic key answers
        other = (float(args[0]),) + args[1:]
        assert b(other, kw, 4, None) is None
        assert s._fast_key(other, kw, 4, None) is not None
    # an unknown keyword: no binder key
    assert s._make_binder(0, ("nope",), (), {"nope": 1})((), {"nope": 1}, 4, None) is None
