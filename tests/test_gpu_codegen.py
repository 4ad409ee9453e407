"""Emitter behaviours that only a device run shows (reference test strategy:
tests/test_codegen.py:158-380): descriptor accesses past any edge of the tensor (negative
offsets included) are masked, dot loops whose K offsets start negative, end ragged or step
by less than a block give exact sums, a dot reads its operands before later writes to the
same memory, and float comparisons follow IEEE NaN rules.

Out-of-bounds cases run on views into the middle of one larger device allocation filled
with a guard value, so an access past the tensor stays inside the allocation and shows up
as a changed guard or a guard value read. Inputs are small integers in float32, so every
expected value is exact.
"""

import numpy as np
import pytest

import enceladus
import enceladus.language as tl

pytestmark = pytest.mark.gpu

GUARD = -7.0


def _guarded(t: np.ndarray):
    """(allocation, view): `t` in the middle third of a device buffer of guard values."""
    import torch
    n = t.size
    buf = torch.full((3 * n,), GUARD, dtype=torch.float32, device="cuda")
    buf[n:2 * n] = torch.from_numpy(np.ascontiguousarray(t, np.float32).ravel()).cuda()
    return buf, buf[n:2 * n]


@enceladus.jit
def _desc_load_at(x_ptr, out_ptr, M, N, o0, o1, B: tl.constexpr):
    d = tl.make_tensor_descriptor(x_ptr, [M, N], [N, 1], [B, B])
    r = tl.arange(0, B)
    tl.store(out_ptr + r[:, None] * B + r[None, :], d.load([o0, o1]))


@enceladus.jit
def _desc_store_at(x_ptr, out_ptr, M, N, o0, o1, B: tl.constexpr):
    d = tl.make_tensor_descriptor(out_ptr, [M, N], [N, 1], [B, B])
    r = tl.arange(0, B)
    d.store([o0, o1], tl.load(x_ptr + r[:, None] * B + r[None, :]))


@enceladus.jit
def _desc_dot_at(x_ptr, out_ptr, M, N, o0, o1, B: tl.constexpr):
    d = tl.make_tensor_descriptor(x_ptr, [M, N], [N, 1], [B, B])
    acc = tl.dot(d.load([o0, o1]), tl.trans(d.load([o1, o0])))
    r = tl.arange(0, B)
    tl.store(out_ptr + r[:, None] * B + r[None, :], acc)


def _block(x, o0, o1, r, c):
    """The r x c block of `x` at (o0, o1), zero outside `x`."""
    out = np.zeros((r, c), x.dtype)
    rows, cols = np.arange(o0, o0 + r), np.arange(o1, o1 + c)
    rm, cm = (rows >= 0) & (rows < x.shape[0]), (cols >= 0) & (cols < x.shape[1])
    out[np.ix_(rm, cm)] = x[np.ix_(rows[rm], cols[cm])]
    return out


@pytest.mark.parametrize("offsets", [(-3, -5), (-16, 0), (10, 12), (2, 4)])
@pytest.mark.parametrize("kind", ["load", "store", "dot"])
def test_descriptor_accesses_outside_the_tensor_are_masked(kind, offsets):
    import torch
    print(f"[case] descriptor {kind} at {offsets}", flush=True)
    m, n, b = 20, 24, 16
    o0, o1 = offsets
    rng = np.random.default_rng(30)
    x = rng.integers(-2, 3, (m, n)).astype(np.float32)
    src = rng.integers(-2, 3, (b, b)).astype(np.float32)
    if kind == "store":
        buf, view = _guarded(np.full((m, n), GUARD, np.float32))
        _desc_store_at[(1,)](torch.from_numpy(src).cuda(), view, m, n, o0, o1, B=b)
        torch.cuda.synchronize()
        t = np.full((m + 2 * b, n + 2 * b), GUARD, np.float32)
        t[b + o0:2 * b + o0, b + o1:2 * b + o1] = src
        want = np.full(3 * m * n, GUARD, np.float32)
        want[m * n:2 * m * n] = t[b:b + m, b:b + n].ravel()
        np.testing.assert_array_equal(buf.cpu().numpy(), want)
        return
    buf, view = _guarded(x)
    out = torch.empty((b, b), dtype=torch.float32, device="cuda")
    (_desc_load_at if kind == "load" else _desc_dot_at)[(1,)](view, out, m, n, o0, o1, B=b)
    torch.cuda.synchronize()
    want = _block(x, o0, o1, b, b) if kind == "load" else \
        _block(x, o0, o1, b, b) @ _block(x, o1, o0, b, b).T
    np.testing.assert_array_equal(out.cpu().numpy(), want)


@enceladus.jit
def _versioned_dot(a_ptr, b_ptr, out_ptr, M, N, K, lo, hi, koff, STEP: tl.constexpr,
                   TRANS_B: tl.constexpr, BM: tl.constexpr, BN: tl.constexpr,
                   BK: tl.constexpr):
    pid_n, pid_m = tl.program_id(0), tl.program_id(1)
    da = tl.make_tensor_descriptor(a_ptr, [M, K], [K, 1], [BM, BK])
    do = tl.make_tensor_descriptor(out_ptr, [M, N], [N, 1], [BM, BN])
    acc = tl.zeros((BM, BN), tl.float32)
    if TRANS_B:
        db = tl.make_tensor_descriptor(b_ptr, [N, K], [K, 1], [BN, BK])
        for k in range(lo, hi, STEP):
            acc = tl.dot(da.load([pid_m * BM, k + koff]), tl.trans(db.load([pid_n * BN, k])),
                         acc)
    else:
        db = tl.make_tensor_descriptor(b_ptr, [K, N], [N, 1], [BK, BN])
        for k in range(lo, hi, STEP):
            acc = tl.dot(da.load([pid_m * BM, koff + k]), db.load([k, pid_n * BN]), acc)
    do.store([pid_m * BM, pid_n * BN], acc)


# (M, N, K, lo, hi, koff, STEP, TRANS_B): aligned; ragged M, N and K; a shifted K offset
# that makes the last block ragged; negative offsets in early iterations; a step smaller
# than the block; K smaller than one block
VERSIONED = [
    (64, 64, 64, 0, 64, 0, 16, False), (40, 48, 47, 0, 47, 0, 16, True),
    (64, 32, 64, 0, 64, 1, 16, False), (32, 64, 40, -16, 40, 3, 16, True),
    (32, 32, 48, 0, 48, 0, 8, True), (40, 32, 5, 0, 5, 0, 16, False),
]


@pytest.mark.parametrize("case", VERSIONED, ids=str)
def test_edge_versioned_dot_loops(case):
    import torch
    print(f"[case] versioned dot {case}", flush=True)
    m, n, k, lo, hi, koff, step, trans_b = case
    bm, bn, bk = 32, 32, 16
    rng = np.random.default_rng(31)
    a = rng.integers(-3, 4, (m, k)).astype(np.float32)
    b = rng.integers(-3, 4, (n, k) if trans_b else (k, n)).astype(np.float32)
    grid = (-(-n // bn), -(-m // bm))
    _, a_v = _guarded(a)
    _, b_v = _guarded(b)
    out_buf, out_v = _guarded(np.zeros((m, n), np.float32))
    _versioned_dot[grid](a_v, b_v, out_v, m, n, k, lo, hi, koff, STEP=step, TRANS_B=trans_b,
                         BM=bm, BN=bn, BK=bk)
    torch.cuda.synchronize()
    want = np.zeros((grid[1] * bm, grid[0] * bn), np.float32)
    bt = b.T if trans_b else b
    for pm in range(grid[1]):
        for pn in range(grid[0]):
            for kk in range(lo, hi, step):
                want[pm * bm:(pm + 1) * bm, pn * bn:(pn + 1) * bn] += \
                    _block(a, pm * bm, kk + koff, bm, bk) @ _block(bt, kk, pn * bn, bk, bn)
    got = out_buf.cpu().numpy()
    np.testing.assert_array_equal(got[m * n:2 * m * n].reshape(m, n), want[:m, :n])
    assert (got[:m * n] == GUARD).all() and (got[2 * m * n:] == GUARD).all()


@enceladus.jit
def _dot_after_write(a_ptr, b_ptr, out_ptr, iters, N: tl.constexpr, CASE: tl.constexpr):
    da = tl.make_tensor_descriptor(a_ptr, [N, N], [N, 1], [N, N])
    db = tl.make_tensor_descriptor(b_ptr, [N, N], [N, 1], [N, N])
    do = tl.make_tensor_descriptor(out_ptr, [N, N], [N, 1], [N, N])
    r = tl.arange(0, N)
    a_ptrs = a_ptr + r[:, None] * N + r[None, :]
    b_ptrs = b_ptr + r[:, None] * N + r[None, :]
    b = db.load([0, 0])
    acc = tl.zeros((N, N), tl.float32)
    for _ in range(iters):
        # each case adds 1 to A or B in memory after loading it, which the dot must not see
        a = da.load([0, 0])
        if CASE == "desc_store":
            da.store([0, 0], tl.load(a_ptrs) + 1.0)
        elif CASE == "store":
            tl.store(a_ptrs, tl.load(a_ptrs) + 1.0)
        elif CASE == "atomic":
            tl.atomic_add(a_ptrs, 1.0)
        elif CASE == "if":
            if iters > 0:
                tl.store(a_ptrs, tl.load(a_ptrs) + 1.0)
        if CASE == "loop":
            acc = tl.dot(a, b, acc)
            tl.store(b_ptrs, tl.load(b_ptrs) + 1.0)
        else:
            acc = tl.dot(a, db.load([0, 0]), acc)
    do.store([0, 0], acc)


@pytest.mark.parametrize("case", ["desc_store", "store", "atomic", "if", "loop"])
def test_dot_reads_its_operands_before_later_writes(case):
    print(f"[case] dot after write {case}", flush=True)
    rng = np.random.default_rng(32)
    a = rng.integers(-2, 3, (32, 32)).astype(np.float32)
    b = rng.integers(-2, 3, (32, 32)).astype(np.float32)
    iters = 3 if case == "loop" else 1
    out = np.empty_like(a)
    _dot_after_write[(1,)](a.copy(), b.copy(), out, iters, N=32, CASE=case)
    np.testing.assert_array_equal(out, iters * (a @ b))


@enceladus.jit
def _nan_compare(x_ptr, y_ptr, bits_ptr, sel_ptr, N: tl.constexpr):
    r = tl.arange(0, N)
    x = tl.load(x_ptr + r)
    y = tl.load(y_ptr + r)
    bits = ((x == y).to(tl.int32) | (x != y).to(tl.int32) << 1 | (x < y).to(tl.int32) << 2
            | (x <= y).to(tl.int32) << 3 | (x > y).to(tl.int32) << 4
            | (x >= y).to(tl.int32) << 5 | (x != x).to(tl.int32) << 6)
    s = tl.load(x_ptr + 3)
    tl.store(bits_ptr + r, bits)
    tl.store(bits_ptr + N, (s != s).to(tl.int32) + (s == s).to(tl.int32) * 2)
    tl.store(sel_ptr + r, tl.where(x == x, x, -1.0))


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
def test_float_comparisons_follow_ieee_nan_rules(dtype):
    print(f"[case] NaN compares {np.dtype(dtype).name}", flush=True)
    n = 64
    rng = np.random.default_rng(33)
    x = rng.integers(-3, 4, n).astype(dtype)
    y = rng.integers(-3, 4, n).astype(dtype)
    x[[3, 20, 41]] = np.nan
    y[[20, 30]] = np.nan
    x[[7, 8]], y[[7, 9]] = np.inf, -np.inf
    bits, sel = np.empty(n + 1, np.int32), np.empty(n, dtype)
    _nan_compare[(1,)](x, y, bits, sel, N=n)
    with np.errstate(invalid="ignore"):
        preds = [x == y, x != y, x < y, x <= y, x > y, x >= y, x != x]
    want = sum(p.astype(np.int32) << i for i, p in enumerate(preds))
    np.testing.assert_array_equal(bits, np.append(want, 1).astype(np.int32))
    np.testing.assert_array_equal(sel, np.where(x == x, x, -1).astype(dtype))


@enceladus.jit
def _scale_rows(x_ptr, y_ptr, M, N, sx, sy, BM: tl.constexpr, BN: tl.constexpr):
    rm = tl.program_id(0) * BM + tl.arange(0, BM)
    rn = tl.arange(0, BN)
    mask = (rm[:, None] < M) & (rn[None, :] < N)
    x = tl.load(x_ptr + rm[:, None] * sx + rn[None, :], mask=mask, other=3)
    tl.store(y_ptr + rm[:, None] * sy + rn[None, :], x * 2 + 1, mask=mask)


# (case, M, N, x row stride, x offset into its allocation): aligned rows; rows that start
# at unaligned addresses; a view one element into its allocation; a mask that changes
# inside a vector
ROWS = [("aligned", 20, 64, 64, 0), ("odd_stride", 20, 64, 65, 0),
        ("offset_view", 20, 64, 64, 1), ("ragged_cols", 20, 50, 64, 0)]


@pytest.mark.parametrize("dtype", ["float32", "float16", "int8", "int64"])
@pytest.mark.parametrize("case,m,n,sx,off", ROWS, ids=[r[0] for r in ROWS])
def test_vector_accesses_match_scalar_ones(dtype, case, m, n, sx, off):
    # device views, so that unaligned rows and offsets reach the kernel as they are
    import torch
    print(f"[case] vector accesses {case} {dtype}", flush=True)
    td = getattr(torch, dtype)
    rng = np.random.default_rng(34)
    base = torch.from_numpy(rng.integers(-50, 50, off + m * sx + 8)).to(td).cuda()
    x = base[off:off + m * sx].view(m, sx)
    y = torch.zeros((m, 64), dtype=td, device="cuda")
    _scale_rows[(enceladus.cdiv(m, 8),)](x, y, m, n, sx, 64, BM=8, BN=64)
    torch.cuda.synchronize()
    want = torch.zeros((m, 64), dtype=td)
    want[:, :n] = x.cpu()[:, :n] * 2 + 1
    assert torch.equal(y.cpu(), want)


@pytest.mark.parametrize("mode", ["relaxed", "fast"])
def test_math_mode_divisions_stay_within_their_bound(mode):
    """A tile divided by its row sums (broadcast) and by a scalar: IEEE division where the
    mode keeps it (bit-exact against NumPy's float32 quotient), a reciprocal multiply where
    it does not (within 1.5 ulp of the quotient; reference math modes: runtime/jit.py:56)."""
    print(f"[case] math_mode={mode} divisions", flush=True)

    @enceladus.jit(math_mode=mode)
    def div(x_ptr, r_ptr, s_ptr, d, BLOCK: tl.constexpr):
        rows = tl.arange(0, BLOCK)[:, None]
        cols = tl.arange(0, BLOCK)[None, :]
        x = tl.load(x_ptr + rows * BLOCK + cols)
        tl.store(r_ptr + rows * BLOCK + cols, x / tl.sum(x, 1)[:, None])
        tl.store(s_ptr + rows * BLOCK + cols, x / d)

    rng = np.random.default_rng(3)
    x = rng.uniform(0.5, 2.0, (32, 32)).astype(np.float32)
    r = np.zeros_like(x)
    s = np.zeros_like(x)
    d = np.float32(3.7)
    div[(1,)](x, r, s, float(d), BLOCK=32)
    rowsum = x.astype(np.float64).sum(1, keepdims=True)
    q_row = (x / rowsum).astype(np.float32)
    ulp = np.spacing(np.abs(q_row))
    # the device's fp32 row sum may differ from float64's by its own rounding
    assert np.all(np.abs(r - q_row) <= 1.5 * ulp + 2e-6 * np.abs(q_row))
    q_s = x / d
    if mode == "relaxed":
        np.testing.assert_array_equal(s, q_s)
    else:
        assert np.all(np.abs(s - q_s) <= 1.5 * np.spacing(np.abs(q_s)))


def test_staged_loop_with_a_dot_under_a_branch():
    """A loop whose K tiles are staged through LDS by DMA but whose dot runs only on some
    iterations: the copies of the next stage must still go out on every iteration (they
    are issued from a dot only when the loop body always runs that dot)."""
    print("[case] staged loop, dot under a branch", flush=True)
    import torch

    @enceladus.jit
    def k(q_ptr, k_ptr, o_ptr, N, BM: tl.constexpr, BN: tl.constexpr, D: tl.constexpr):
        q_desc = tl.make_tensor_descriptor(q_ptr, [BM, D], [D, 1], [BM, D])
        k_desc = tl.make_tensor_descriptor(k_ptr, [N, D], [D, 1], [BN, D])
        q = q_desc.load([0, 0])
        acc = tl.zeros([BM, BN], tl.float32)
        for n0 in range(0, N, BN):
            kt = k_desc.load([n0, 0])
            if (n0 // BN) % 3 == 0:
                acc = tl.dot(q, tl.trans(kt), acc)
        rm = tl.arange(0, BM)[:, None]
        rn = tl.arange(0, BN)[None, :]
        tl.store(o_ptr + rm * BN + rn, acc)

    BM, BN, D, N = 64, 64, 64, 512
    rng = np.random.default_rng(5)
    q = rng.integers(-3, 4, (BM, D)).astype(np.float16)
    kk = rng.integers(-3, 4, (N, D)).astype(np.float16)
    o = torch.zeros((BM, BN), dtype=torch.float32, device="cuda")
    k[(1,)](torch.from_numpy(q).cuda(), torch.from_numpy(kk).cuda(), o, N, BM=BM, BN=BN, D=D)
    want = np.zeros((BM, BN), np.float64)
    for n0 in range(0, N, BN):
        if (n0 // BN) % 3 == 0:
            want += q.astype(np.float64) @ kk[n0:n0 + BN].astype(np.float64).T
    np.testing.assert_array_equal(o.cpu().numpy(), want)
