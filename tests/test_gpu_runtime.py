"""Runtime behaviour around launches (reference test strategy: tests/test_runtime.py):
views of device tensors, C conversion of float scalars, grid limits, 64-bit variants for
arrays past 2^31 elements, and launches and synchronisations from several threads.
CPU cases need no GPU; the rest are marked `gpu`."""

import subprocess
import sys

import numpy as np
import pytest

import enceladus
import enceladus.language as tl
from enceladus_amd.runtime.tensor import Tensor

ROOT = __file__.rsplit("/tests/", 1)[0]


class _BigBuffer:
    """Stands in for a 16 GB allocation: only its metadata is read."""
    ptr, nbytes = 1 << 20, 1 << 34


def test_views_share_the_allocation_and_stay_inside_it():
    t = Tensor(_BigBuffer(), (4, 6), "float32")
    v = t[1:, ::2]
    assert v.shape == (3, 3) and v.strides == (6, 2) and v.buffer is t.buffer
    assert v.ptr == t.ptr + 6 * 4 and v.data_ptr == v.data_ptr() == v.ptr
    assert not v.is_contiguous() and v.stride(1) == 2 and v.size(0) == 3 and len(v) == 3
    for key in (slice(4, None), slice(2, 2)):
        e = t[key]
        assert e.numel == 0 and e.buffer is t.buffer
        assert 0 <= e.byte_offset <= t.buffer.nbytes
    with pytest.raises(TypeError):
        t[1, 2]
    with pytest.raises(ValueError, match="negative strides"):
        t[:, ::-1]


@enceladus.jit
def _masked_tail(x_ptr, y_ptr, n, STEP: tl.constexpr, BLOCK: tl.constexpr):
    pid = tl.program_id(0)
    offs = pid * STEP + tl.arange(0, BLOCK)
    local = offs - pid * STEP
    tl.store(y_ptr + pid * BLOCK + local, tl.load(x_ptr + local) + 1.0, mask=offs < n)


def test_arrays_past_2_31_elements_compile_a_64_bit_variant():
    x = np.arange(16, dtype=np.float32)
    n = (1 << 31) + 3
    from enceladus_amd.compiler import widen
    huge = Tensor(_BigBuffer(), ((1 << 31) + 1,), "float32")
    assert not widen.needs_idx64(_masked_tail.ir_for(x, x, n, STEP=1 << 30, BLOCK=16))
    assert widen.needs_idx64(_masked_tail.ir_for(huge, x, n, STEP=1 << 30, BLOCK=16))
    big = _masked_tail.warmup(huge, x, n, STEP=1 << 30, BLOCK=16)
    assert "(a0 + ((int64_t)" in big.hip            # 64-bit element offsets into x_ptr


@enceladus.jit
def _add_one(x_ptr, out_ptr, n, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    tl.store(out_ptr + offs, tl.load(x_ptr + offs, mask=m) + 1.0, mask=m)


@pytest.mark.gpu
def test_grids_past_the_hip_limits_are_refused():
    x = np.ones(8, np.float32)
    with pytest.raises(ValueError, match="exceeds the HIP limits"):
        _add_one[(1 << 31,)](x, x, 8, BLOCK=8)
    with pytest.raises(ValueError, match="exceeds the HIP limits"):
        _add_one[(1, 70000)](x, x, 8, BLOCK=8)


@pytest.mark.gpu
def test_kernels_read_and_write_views():
    print("[case] views", flush=True)
    base = enceladus.zeros((8, 16))
    host = np.arange(128, dtype=np.float32).reshape(8, 16)
    base.copy_(host)
    src = base[2:6]                                   # contiguous rows
    out = enceladus.zeros((4, 16))
    _add_one[(1,)](src, out, 64, BLOCK=64)
    np.testing.assert_array_equal(out.numpy(), host[2:6] + 1)
    col = base[:, 3:4]                                # a strided view reads back its elements
    np.testing.assert_array_equal(col.numpy(), host[:, 3:4])
    col.copy_(np.full((8, 1), -1.0, np.float32))      # and writes only them
    want = host.copy()
    want[:, 3] = -1
    np.testing.assert_array_equal(base.numpy(), want)


@enceladus.jit
def _scale(out_ptr, a):
    tl.store(out_ptr + tl.arange(0, 4), tl.full((4,), 1.0, tl.float32) * a)


@pytest.mark.gpu
@pytest.mark.parametrize("value", [1e40, -1e40, np.float64(1e39), 2.5])
def test_float_scalars_convert_like_c(value):
    print(f"[case] float scalar {value}", flush=True)
    out = np.zeros(4, np.float32)
    _scale[(1,)](out, value)
    want = np.float32(value) if abs(value) < 3.4e38 else np.copysign(np.inf, value)
    np.testing.assert_array_equal(out, want)


_THREADS = """
import sys, threading
sys.path.insert(0, {root!r})
import numpy as np
import enceladus
import enceladus.language as tl

@enceladus.jit
def inc(x_ptr, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    tl.store(x_ptr + offs, tl.load(x_ptr + offs) + 1)

ts = [enceladus.zeros(1024, dtype="int32") for _ in range(2)]
inc[(4,)](ts[0], BLOCK=256)                  # compile once before the threads start
enceladus.synchronize()
ts[0].copy_(np.zeros(1024, np.int32))
stop = threading.Event()
def syncer():
    while not stop.is_set():
        enceladus.synchronize()
def launch(t):
    for _ in range({n}):
        inc[(4,)](t, BLOCK=256)
syncers = [threading.Thread(target=syncer) for _ in range(2)]
launchers = [threading.Thread(target=launch, args=(t,)) for t in ts]
for th in syncers + launchers:
    th.start()
for th in launchers:
    th.join()
stop.set()
for th in syncers:
    th.join()
enceladus.synchronize()
for t in ts:
    np.testing.assert_array_equal(t.numpy(), {n})
print("ok", flush=True)
"""


@pytest.mark.gpu
def test_concurrent_launches_and_syncs(tmp_path):
    # its own process, so that a failure ends only this test (a file: the kernel's source
    # must be readable)
    print("[case] threads", flush=True)
    script = tmp_path / "threads.py"
    script.write_text(_THREADS.format(root=ROOT, n=5000))
    r = subprocess.run([sys.executable, str(script)], capture_output=True, timeout=100)
    assert r.returncode == 0, r.stderr.decode()[-2000:]
    assert b"ok" in r.stdout


# -- the launch cache and what a kernel read at compile time --------------------------

SCALE = 2.0
TUP = (2.0, 3.0)
ZERO = 0.0
FACTOR = 4.0


def _python_factor():
    return FACTOR


@enceladus.jit
def _helper(x):
    return x * SCALE


@enceladus.jit
def _scale_by_globals(x_ptr, out_ptr):
    offs = tl.arange(0, 16)
    x = tl.load(x_ptr + offs)
    tl.store(out_ptr + offs, _helper(x) + TUP[1] + _python_factor() + 1.0 / (x * 0.0 + ZERO))


def _globals_reference(x):
    with np.errstate(divide="ignore"):
        return x * SCALE + TUP[1] + FACTOR + 1.0 / (x * 0.0 + ZERO)


@pytest.mark.parametrize("name,value", [("SCALE", 5.0), ("TUP", (2.0, 7.0)), ("FACTOR", 9.0),
                                        ("ZERO", -0.0)])
def test_changed_globals_recompile(name, value, monkeypatch):
    x = np.arange(1, 17, dtype=np.float32)
    first = _scale_by_globals.warmup(x, x)
    assert first is _scale_by_globals.warmup(x, x)          # warm: the same kernel
    monkeypatch.setitem(globals(), name, value)
    assert _scale_by_globals.warmup(x, x) is not first      # the read value changed


@pytest.mark.gpu
@pytest.mark.parametrize("name,value", [("SCALE", 5.0), ("TUP", (2.0, 7.0)), ("FACTOR", 9.0),
                                        ("ZERO", -0.0)])
def test_changed_globals_give_new_results(name, value, monkeypatch):
    print(f"[case] global {name}", flush=True)
    x = np.arange(1, 17, dtype=np.float32)
    out = np.empty(16, np.float32)
    _scale_by_globals[(1,)](x, out)
    np.testing.assert_array_equal(out, _globals_reference(x))
    monkeypatch.setitem(globals(), name, value)
    _scale_by_globals[(1,)](x, out)
    np.testing.assert_array_equal(out, _globals_reference(x))


@enceladus.jit
def _reciprocal(out_ptr, C: tl.constexpr):
    offs = tl.arange(0, 16)
    tl.store(out_ptr + offs, 1.0 / (tl.full((16,), 1.0, tl.float32) * C))


@pytest.mark.gpu
def test_float_constexprs_are_keyed_by_bit_pattern():
    print("[case] float constexpr keys", flush=True)
    out = np.empty(16, np.float32)
    got, sizes = [], []
    for c in (0.0, -0.0, float("nan"), float("nan")):
        _reciprocal[(1,)](out, C=c)
        got.append(out[0])
        sizes.append(len(_reciprocal._cache))
    np.testing.assert_array_equal(got, [np.inf, -np.inf, np.nan, np.nan])
    assert sizes[3] == sizes[2]


@enceladus.jit
def _scaled(out_ptr, S: tl.constexpr):
    offs = tl.arange(0, 16)
    tl.store(out_ptr + offs, (offs + 2147483647) * S)


@pytest.mark.gpu
def test_constexprs_that_compare_equal_compile_separately():
    # 2 == 2.0 and 1 == True, but int32 math wraps and float math doesn't
    from oracle import interpreter as O
    print("[case] equal constexprs", flush=True)
    for s in (2, 2.0, 1, True):
        got, want = np.zeros(16, np.float32), np.zeros(16, np.float32)
        _scaled[(1,)](got, S=s)
        O.run_grid(_scaled, (1,), want, S=s)
        np.testing.assert_array_equal(got, want)


@pytest.mark.gpu
def test_warm_path_respecializes_on_argument_classes():
    """The warm launch path keys on argument classes: a size that is (or is not) a multiple
    of 16, a scale of either sign, an unaligned view and an int64 size each select their
    own specialization, and every launch is right."""
    import torch
    print("[case] warm-path specialization classes", flush=True)

    @enceladus.jit
    def axpy(x_ptr, out_ptr, n, a, BLOCK: tl.constexpr):
        offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
        m = offs < n
        tl.store(out_ptr + offs, tl.load(x_ptr + offs, mask=m) * a + 1.0, mask=m)

    base = torch.randn(5000, device="cuda")
    for n, a, off in [(4096, 2.0, 0), (4004, 2.0, 0), (4096, -3.0, 0), (4096, 2.0, 1),
                      (4001, 0.5, 3), (4096, 2.0, 0), (4004, 2.0, 0)]:
        x = base[off:off + n]
        out = torch.zeros(n, device="cuda")
        for _ in range(2):          # the second launch takes the warm path
            axpy[(enceladus.cdiv(n, 256),)](x, out, n, a, BLOCK=256)
        torch.cuda.synchronize()
        torch.testing.assert_close(out, x * a + 1.0)
    keys = list(axpy._fast)
    assert len(keys) >= 5


@pytest.mark.gpu
def test_binder_keys_match_the_generic_key_on_device_tensors():
    """With torch device tensors (contiguous, strided views, offset views, other dtypes) the
    generated binder gives the generic key function's key and pointers."""
    import torch
    from examples.vector_add import add_kernel
    print("[case] binder keys on device tensors", flush=True)
    base = torch.randn(4096, device="cuda")
    views = [base, base[1:1001], base[::2], base.view(64, 64)[:, :32],
             torch.zeros(100, dtype=torch.float16, device="cuda")]
    for x in views:
        args = (x, x, x, int(x.numel()))
        kw = {"BLOCK": 1024}
        b = add_kernel._make_binder(4, ("BLOCK",), args, kw)
        assert b(args, kw, 4, None) == add_kernel._fast_key(args, kw, 4, None)


WARM_SCALE = 2.0


@pytest.mark.gpu
def test_warm_path_follows_a_changed_global():
    """A global the kernel reads changes between warm launches: the next launch recompiles,
    and the warm entry then follows the new code (reference: runtime/jit.py:1037-1234)."""
    import torch
    global WARM_SCALE
    print("[case] warm path after a global changes", flush=True)

    @enceladus.jit
    def scale(x_ptr, out_ptr, n, BLOCK: tl.constexpr):
        offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
        m = offs < n
        tl.store(out_ptr + offs, tl.load(x_ptr + offs, mask=m) * WARM_SCALE, mask=m)

    x = torch.randn(1000, device="cuda")
    out = torch.zeros_like(x)
    try:
        for want in (2.0, 5.0, -1.5):
            WARM_SCALE = want
            for _ in range(3):      # the general path once, then warm launches
                out.zero_()
                scale[(4,)](x, out, 1000, BLOCK=256)
                torch.cuda.synchronize()
                torch.testing.assert_close(out, x * want)
            (ent,) = scale._fast.values()
            assert ent.lc.current()
    finally:
        WARM_SCALE = 2.0


@pytest.mark.gpu
def test_interleaved_host_views_written_by_one_launch():
    """Two written NumPy views of one array whose byte spans overlap (a[::2], a[1::2]) share
    one device copy: neither copy-back undoes the other's results."""
    print("[case] interleaved host views", flush=True)

    @enceladus.jit
    def two_writes(x_ptr, e_ptr, o_ptr, n, BLOCK: tl.constexpr):
        offs = tl.arange(0, BLOCK)
        m = offs < n
        x = tl.load(x_ptr + offs, mask=m)
        tl.store(e_ptr + offs * 2, x + 1.0, mask=m)
        tl.store(o_ptr + offs * 2, x + 2.0, mask=m)

    x = np.arange(100, dtype=np.float32)
    a = np.full(200, -5.0, np.float32)
    two_writes[(1,)](x, a[::2], a[1::2], 100, BLOCK=128)
    np.testing.assert_array_equal(a[::2], x + 1.0)
    np.testing.assert_array_equal(a[1::2], x + 2.0)
