"""Atomics (`tl.atomic_*`): every kind on native 32-bit paths, compare-and-swap loops and
8/16-bit elements packed next to elements other threads update, old values returned to
every thread that holds a copy of a replicated element, and scalar tickets (reference test
strategy: tests/test_atomics_scans.py:17-170).

Compile-only cases run on the CPU; the `gpu` cases compare the device against the closed
form of each update with one atomic per address (old values and memory bit-exact), and
against order-free properties where addresses collide.
"""

import numpy as np
import pytest

import enceladus
import enceladus.language as tl
from enceladus_amd.runtime import compile as C


@enceladus.jit
def _atomic_kernel(mem_ptr, idx_ptr, cmp_ptr, val_ptr, old_ptr, n, KIND: tl.constexpr,
                   BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    # atomic_cas has no mask: masked lanes address a spare slot at the end
    p = mem_ptr + tl.load(idx_ptr + offs, mask=m, other=n)
    v = tl.load(val_ptr + offs, mask=m)
    if KIND == "add":
        old = tl.atomic_add(p, v, mask=m)
    elif KIND == "max":
        old = tl.atomic_max(p, v, mask=m)
    elif KIND == "min":
        old = tl.atomic_min(p, v, mask=m)
    elif KIND == "xchg":
        old = tl.atomic_xchg(p, v, mask=m)
    elif KIND == "and":
        old = tl.atomic_and(p, v, mask=m)
    elif KIND == "or":
        old = tl.atomic_or(p, v, mask=m)
    elif KIND == "xor":
        old = tl.atomic_xor(p, v, mask=m)
    else:
        old = tl.atomic_cas(p, tl.load(cmp_ptr + offs, mask=m), v)
    tl.store(old_ptr + offs, old, mask=m)


# native paths, CAS loops on 32-bit words, and 8/16-bit elements inside shared words
CASES = [
    ("add", "int32"), ("add", "float32"), ("add", "int16"), ("add", "uint8"),
    ("max", "int32"), ("max", "uint32"), ("max", "float32"), ("max", "bfloat16"),
    ("min", "float16"), ("min", "int8"), ("xchg", "float32"), ("xchg", "int16"),
    ("and", "uint32"), ("or", "int16"), ("xor", "int32"),
    ("cas", "int32"), ("cas", "float32"), ("cas", "uint16"),
]


def _torch_dtype(name):
    import torch
    return getattr(torch, name)


def _values(rng, n, name):
    if name in ("float32", "float16", "bfloat16"):
        return (rng.standard_normal(n) * 8).astype(np.float32)
    info = np.iinfo(np.dtype(name))
    return rng.integers(info.min, info.max, n, endpoint=True).astype(np.dtype(name))


@pytest.mark.parametrize("kind,name", CASES)
def test_every_atomic_kind_compiles_for_gfx950(kind, name):
    import torch
    t = torch.zeros(8, dtype=_torch_dtype(name))
    i = torch.zeros(8, dtype=torch.int32)
    fn = _atomic_kernel.ir_for(t, i, t, t, t, 8, KIND=kind, BLOCK=256)
    ck = C.compile_ir(fn, {})
    assert ck.name == "ek__atomic_kernel"


def _expected(kind, mem, idx, cmp, val):
    """Memory and old values after one atomic per address (closed form of each update)."""
    mem = mem.copy()
    old = mem[idx].copy()
    new = {
        "add": lambda o, v: o + v, "max": np.maximum, "min": np.minimum,
        "xchg": lambda o, v: v, "and": np.bitwise_and, "or": np.bitwise_or,
        "xor": np.bitwise_xor, "cas": lambda o, v: np.where(o == cmp, v, o),
    }[kind](old, val)
    mem[idx] = new
    return mem, old


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1024, 1000])
@pytest.mark.parametrize("kind,name", CASES)
def test_atomics_return_old_values_and_update_memory(kind, name, n):
    print(f"[case] atomic_{kind} {name} n={n}", flush=True)
    rng = np.random.default_rng(len(kind) * n)
    idx = rng.permutation(n).astype(np.int32)          # one atomic per address
    mem = _values(rng, n + 1, name)
    val = _values(rng, n, name)
    cmp = np.where(rng.random(n) < 0.5, mem[idx], _values(rng, n, name))
    if name == "bfloat16":
        # NumPy has no bfloat16: torch device tensors, expected values from the rounded
        # inputs in float32 (max of two bf16 values is one of them, so exact)
        import torch
        to = lambda a: torch.from_numpy(a).to(torch.bfloat16)  # noqa: E731
        mem_t, val_t, cmp_t = to(mem), to(val), to(cmp)
        want_mem, want_old = _expected(kind, mem_t.float().numpy(), idx,
                                       cmp_t.float().numpy(), val_t.float().numpy())
        mem_d, val_d, cmp_d = mem_t.cuda(), val_t.cuda(), cmp_t.cuda()
        old_d = torch.zeros(n, dtype=torch.bfloat16, device="cuda")
        _atomic_kernel[(4,)](mem_d, torch.from_numpy(idx).cuda(), cmp_d, val_d, old_d, n,
                             KIND=kind, BLOCK=256)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(mem_d.float().cpu().numpy(), want_mem)
        np.testing.assert_array_equal(old_d.float().cpu().numpy(), want_old)
        return
    dt = np.dtype(name)
    mem, val, cmp = mem.astype(dt), val.astype(dt), cmp.astype(dt)
    want_mem, want_old = _expected(kind, mem, idx, cmp, val)
    old = np.zeros(n, dt)
    got = mem.copy()
    with np.errstate(over="ignore"):
        _atomic_kernel[(4,)](got, idx, cmp, val, old, n, KIND=kind, BLOCK=256)
    np.testing.assert_array_equal(old, want_old)
    np.testing.assert_array_equal(got, want_mem.astype(dt))


@enceladus.jit
def _count_kernel(cnt_ptr, old_ptr, cs_ptr, BLOCK: tl.constexpr):
    offs = tl.arange(0, BLOCK)
    old = tl.atomic_add(cnt_ptr + offs, 1)
    row = tl.program_id(0) * BLOCK + offs
    tl.store(old_ptr + row, old)
    # the scan reads the copies in every thread that holds an element, not only the owner's
    tl.store(cs_ptr + row, tl.cumsum(old, 0))


@pytest.mark.gpu
@pytest.mark.parametrize("block,num_warps", [(16, 1), (16, 4), (64, 4)])
def test_atomics_on_broadcast_layouts_run_once_per_element(block, num_warps):
    print(f"[case] replicated atomic block={block} warps={num_warps}", flush=True)
    progs = 3
    cnt = np.zeros(block, np.int32)
    old = np.full((progs, block), -1, np.int32)
    cs = np.zeros_like(old)
    _count_kernel[(progs,)](cnt, old, cs, BLOCK=block, num_warps=num_warps)
    np.testing.assert_array_equal(cnt, progs)
    np.testing.assert_array_equal(np.sort(old, axis=0), np.arange(progs)[:, None] + 0 * old)
    np.testing.assert_array_equal(cs, np.cumsum(old, axis=1))


@enceladus.jit
def _scalar_counter_kernel(cnt_ptr, fmax_ptr, out_ptr, vals_ptr):
    pid = tl.program_id(0)
    tl.store(out_ptr + pid, tl.atomic_add(cnt_ptr, 1))
    tl.atomic_max(fmax_ptr, tl.load(vals_ptr + pid))


@pytest.mark.gpu
def test_scalar_atomics_hand_out_unique_tickets():
    print("[case] scalar tickets", flush=True)
    progs = 40
    vals = np.random.default_rng(3).standard_normal(progs).astype(np.float32)
    cnt, fmax = np.zeros(1, np.int32), np.full(1, -np.inf, np.float32)
    out = np.full(progs, -1, np.int32)
    _scalar_counter_kernel[(progs,)](cnt, fmax, out, vals)
    assert cnt[0] == progs and fmax[0] == vals.max()
    np.testing.assert_array_equal(np.sort(out), np.arange(progs))


@enceladus.jit
def _u64_minmax_kernel(mem_ptr, idx_ptr, val_ptr, n, KIND: tl.constexpr, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    p = mem_ptr + tl.load(idx_ptr + offs, mask=m)
    v = tl.load(val_ptr + offs, mask=m)
    if KIND == "max":
        tl.atomic_max(p, v, mask=m)
    else:
        tl.atomic_min(p, v, mask=m)


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["max", "min"])
def test_uint64_max_and_min_with_colliding_addresses(kind):
    print(f"[case] uint64 atomic_{kind}", flush=True)
    rng = np.random.default_rng(4)
    n, slots = 3000, 37
    idx = rng.integers(0, slots, n).astype(np.int32)
    val = rng.integers(0, 2**64 - 1, n, dtype=np.uint64, endpoint=True)
    init = np.uint64(0) if kind == "max" else np.uint64(2**64 - 1)
    mem = np.full(slots, init, np.uint64)
    _u64_minmax_kernel[(enceladus.cdiv(n, 512),)](mem, idx, val, n, KIND=kind, BLOCK=512)
    want = np.full(slots, init, np.uint64)
    (np.maximum if kind == "max" else np.minimum).at(want, idx, val)
    np.testing.assert_array_equal(mem, want)


@enceladus.jit
def _collide_kernel(mem_ptr, val_ptr, n, SLOTS: tl.constexpr, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    tl.atomic_add(mem_ptr + offs % SLOTS, tl.load(val_ptr + offs, mask=m), mask=m)


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["int16", "uint8", "int32"])
def test_sub_word_adds_collide_with_their_neighbours(name):
    # 8/16-bit counters share 32-bit words: every update must land despite the neighbours'
    print(f"[case] colliding {name} adds", flush=True)
    rng = np.random.default_rng(5)
    n, slots = 20000, 7
    val = rng.integers(0, 3, n).astype(np.dtype(name))
    mem = np.zeros(slots + 1, np.dtype(name))
    _collide_kernel[(enceladus.cdiv(n, 256),)](mem, val, n, SLOTS=slots, BLOCK=256)
    want = np.zeros(slots + 1, np.int64)
    np.add.at(want, np.arange(n) % slots, val.astype(np.int64))
    np.testing.assert_array_equal(mem, want.astype(np.dtype(name)))
