"""GPU parity for the tile-shape ops: `tl.join`, `tl.split`, `tl.reshape`, and the
combine-function forms `tl.reduce` and `tl.associative_scan`, against NumPy on the same
seeded inputs (reference test strategy: tests/test_join_split.py, test_atomics_scans.py).

Join, split and reshape only move data, so every dtype must match bit for bit. `tl.reduce`
and `tl.associative_scan` combine in the reference interpreter's order (halving tree;
Hillis-Steele), restated in NumPy below, so integer results are exact and float32 sums
are exact too; combine functions with a multiply-add use a stated tolerance because the
device may contract them to one fused multiply-add.
"""

import numpy as np
import pytest

import enceladus
import enceladus.language as tl

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _gen(rng, shape, dtype):
    if np.issubdtype(dtype, np.integer):
        return rng.integers(-50, 50, shape).astype(dtype)
    return rng.standard_normal(shape).astype(dtype)


# -- join / split ------------------------------------------------------------------

@enceladus.jit
def _shapes_kernel(x_ptr, y_ptr, out_ptr, CASE: tl.constexpr, M: tl.constexpr,
                   N: tl.constexpr):
    rm = tl.arange(0, M)
    rn = tl.arange(0, N)
    tile = rm[:, None] * N + rn[None, :]
    if CASE == "interleave":
        a = tl.load(x_ptr + tile)
        b = tl.load(y_ptr + tile)
        wide = tl.arange(0, 2 * N)
        tl.store(out_ptr + rm[:, None] * (2 * N) + wide[None, :],
                 tl.reshape(tl.join(a, b), (M, 2 * N)))
    elif CASE == "deinterleave":
        wide = tl.arange(0, 2 * N)
        v = tl.load(x_ptr + rm[:, None] * (2 * N) + wide[None, :])
        even, odd = tl.split(tl.reshape(v, (M, N, 2)))
        tl.store(out_ptr + tile, odd)
        tl.store(out_ptr + M * N + tile, even)
    elif CASE == "transposed":
        # rows of a (2, M) tile: after the transpose the split bit is a lane bit
        v = tl.load(x_ptr + tl.arange(0, 2)[:, None] * M + rm[None, :])
        first, second = v.T.split()
        tl.store(out_ptr + rm, second)
        tl.store(out_ptr + M + rm, first)
    elif CASE == "tiny":
        v = tl.load(x_ptr + rm[:, None] * 2 + tl.arange(0, 2)[None, :])
        first, second = tl.split(v)
        tl.store(out_ptr + rm, first + second)
        tl.store(out_ptr + M + rm, second)
    elif CASE == "reductions":
        v = tl.load(x_ptr + tile)
        pair = tl.join(tl.max(v, axis=1), tl.min(v, axis=1))
        tl.store(out_ptr + rm[:, None] * 2 + tl.arange(0, 2)[None, :], pair)
        hi, lo = tl.split(pair)
        tl.store(out_ptr + 2 * M + rm, hi - lo)
    elif CASE == "loop":
        v = tl.load(x_ptr + tile)
        acc = tl.zeros((M, N, 2), v.dtype)
        for i in range(4):
            acc = acc + tl.join(v * i, v)
        p, q = tl.split(acc)
        tl.store(out_ptr + tile, p)
        tl.store(out_ptr + M * N + tile, q)
    elif CASE == "computed":
        r32 = tl.arange(0, 32)
        c2 = tl.arange(0, 2)[None, :]
        tl.store(out_ptr + r32[:, None] * 2 + c2, tl.join(r32 * 2 + 1, r32 - 3).to(x_ptr.dtype))
        even, odd = tl.split(tl.reshape(tl.arange(0, 2 * N), (N, 2)))
        tl.store(out_ptr + 64 + rn, (odd * 3 - even).to(x_ptr.dtype))
    else:  # "scalar"
        s = tl.load(x_ptr)
        tl.store(out_ptr + tl.arange(0, 2), tl.join(7, s))
        u, w = tl.split(tl.load(x_ptr + 1 + tl.arange(0, 2)))
        tl.store(out_ptr + 2, w)
        tl.store(out_ptr + 3, u)


def _shapes_expected(case, x, y, m, n):
    if case == "interleave":
        return np.stack([x, y], -1).reshape(m, 2 * n)
    if case == "deinterleave":
        v = x.reshape(m, n, 2)
        return np.concatenate([v[..., 1].ravel(), v[..., 0].ravel()])
    if case == "transposed":
        return np.concatenate([x[1], x[0]])
    if case == "tiny":
        return np.concatenate([x[:, 0] + x[:, 1], x[:, 1]])
    if case == "reductions":
        hi, lo = x.max(1), x.min(1)
        return np.concatenate([np.stack([hi, lo], -1).ravel(), hi - lo])
    if case == "loop":
        return np.concatenate([(x * 6).ravel(), (x * 4).ravel()])
    if case == "computed":
        r32, r = np.arange(32), np.arange(2 * n)
        return np.concatenate([np.stack([2 * r32 + 1, r32 - 3], -1).ravel(),
                               r[1::2] * 3 - r[0::2]]).astype(x.dtype)
    return np.array([7, x[0], x[2], x[1]]).astype(x.dtype)


# case: (x shape, M, N, num_warps)
SHAPE_CASES = {
    "interleave": ((8, 64), 8, 64, 4),
    "deinterleave": ((16, 64), 16, 32, 4),
    "transposed": ((2, 64), 64, 1, 1),
    "tiny": ((16, 2), 16, 1, 4),
    "reductions": ((16, 32), 16, 32, 4),
    "loop": ((4, 32), 4, 32, 2),
    "computed": ((1,), 1, 8, 4),
    "scalar": ((3,), 1, 1, 1),
}


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.int32])
@pytest.mark.parametrize("case", list(SHAPE_CASES))
def test_join_split(case, dtype):
    _say(f"join/split {case} {np.dtype(dtype).name}")
    xs, m, n, nw = SHAPE_CASES[case]
    rng = np.random.default_rng(1)
    x = _gen(rng, xs, dtype)
    y = _gen(rng, xs, dtype)
    want = _shapes_expected(case, x, y, m, n).astype(dtype)
    out = np.zeros(want.size, dtype)
    _shapes_kernel[(1,)](x, y, out, CASE=case, M=m, N=n, num_warps=nw)
    np.testing.assert_array_equal(out, want.ravel())


@enceladus.jit
def _dot_pairs(a_ptr, b_ptr, out_ptr, M: tl.constexpr, N: tl.constexpr, K: tl.constexpr):
    rm, rn, rk = tl.arange(0, M), tl.arange(0, N), tl.arange(0, K)
    a = tl.load(a_ptr + rm[:, None] * K + rk[None, :])
    b = tl.load(b_ptr + rk[:, None] * N + rn[None, :])
    c = tl.dot(a, b)
    even, odd = tl.split(tl.reshape(c, (M, N // 2, 2)))
    tl.store(out_ptr + rm[:, None] * N + rn[None, :],
             tl.reshape(tl.join(odd * 2, even), (M, N)))
    flat = (rm[:, None] * N + rn[None, :])[:, :, None] * 2 + tl.arange(0, 2)[None, None, :]
    tl.store(out_ptr + M * N + flat, tl.join(c - 1, c))


@pytest.mark.parametrize("dtype", [np.float16, "bfloat16"])
@pytest.mark.parametrize("num_warps", [1, 4])
def test_join_split_of_dot_results(dtype, num_warps):
    import torch
    _say(f"dot join/split {dtype} warps={num_warps}")
    m, n, k = 64, 64, 32
    g = torch.Generator().manual_seed(2)
    tdt = torch.float16 if dtype is np.float16 else torch.bfloat16
    a = torch.randn((m, k), generator=g).to(tdt)
    b = torch.randn((k, n), generator=g).to(tdt)
    out = torch.zeros(3 * m * n, dtype=torch.float32)
    ad, bd, od = a.cuda(), b.cuda(), out.cuda()
    _dot_pairs[(1,)](ad, bd, od, M=m, N=n, K=k, num_warps=num_warps)
    got = od.cpu().numpy()
    c = a.double().numpy() @ b.double().numpy()
    s = c.reshape(m, n // 2, 2)
    swapped = np.stack([2 * s[..., 1], s[..., 0]], -1).reshape(m, n)
    want = np.concatenate([swapped.ravel(), np.stack([c - 1, c], -1).ravel()])
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-3)


# -- tl.reduce with a combine function -------------------------------------------------

@enceladus.jit
def _add(a, b):
    return a + b


@enceladus.jit
def _mul(a, b):
    return a * b


@enceladus.jit
def _argmax_pair(v0, i0, v1, i1):
    # larger value wins; on ties the smaller index
    take = (v1 > v0) | ((v1 == v0) & (i1 < i0))
    return tl.where(take, v1, v0), tl.where(take, i1, i0)


@enceladus.jit
def _reduce_kernel(x_ptr, out_ptr, M: tl.constexpr, N: tl.constexpr, CASE: tl.constexpr):
    rm, rn = tl.arange(0, M), tl.arange(0, N)
    x = tl.load(x_ptr + rm[:, None] * N + rn[None, :])
    if CASE == "rows":
        tl.store(out_ptr + rm, tl.reduce(x, 1, _add))
    elif CASE == "cols":
        tl.store(out_ptr + rn, tl.reduce(x, 0, _add))
    elif CASE == "all":
        tl.store(out_ptr, tl.reduce(x, None, _add))
    elif CASE == "keep":
        r = tl.reduce(x, 1, _add, keep_dims=True)
        tl.store(out_ptr + rm[:, None] + tl.zeros((M, 1), tl.int32), r)
    elif CASE == "prod":
        tl.store(out_ptr + rm, tl.reduce(x, 1, _mul))
    else:  # "argmax": a tuple reduction
        idx = rn[None, :] + tl.zeros((M, N), tl.int32)
        v, i = tl.reduce((x, idx), 1, _argmax_pair)
        tl.store(out_ptr + rm, v)
        tl.store(out_ptr + M + rm, i.to(x.dtype))


def _tree(x, axis, fn):
    """The reference interpreter's order: combine(x[:h], x[h:]) until one is left."""
    x = np.moveaxis(x, axis, -1)
    while x.shape[-1] > 1:
        h = x.shape[-1] // 2
        x = fn(x[..., :h], x[..., h:])
    return x[..., 0]


@pytest.mark.parametrize("case,dtype,m,n,nw", [
    ("rows", np.float32, 16, 256, 4),
    ("rows", np.int32, 8, 1024, 4),
    ("cols", np.float32, 64, 32, 4),
    ("cols", np.int32, 128, 16, 8),
    ("all", np.float32, 32, 64, 4),
    ("keep", np.int32, 16, 64, 2),
    ("prod", np.int32, 4, 16, 1),
    ("argmax", np.float32, 32, 128, 4),
    ("argmax", np.int32, 16, 64, 4),
])
def test_reduce_with_combine_function(case, dtype, m, n, nw):
    _say(f"reduce {case} {np.dtype(dtype).name} {m}x{n} warps={nw}")
    rng = np.random.default_rng(3)
    x = _gen(rng, (m, n), dtype)
    if case == "prod":
        x = rng.integers(-2, 3, (m, n)).astype(dtype)
    if case == "argmax" and dtype is np.int32:
        x = rng.integers(0, 6, (m, n)).astype(dtype)   # many ties
    add = lambda a, b: (a + b).astype(dtype)  # noqa: E731
    if case == "rows":
        want = _tree(x, 1, add)
    elif case == "cols":
        want = _tree(x, 0, add)
    elif case == "all":
        want = _tree(x.ravel(), 0, add).reshape(1)
    elif case == "keep":
        want = _tree(x, 1, add)
    elif case == "prod":
        want = _tree(x, 1, lambda a, b: (a * b).astype(dtype))
    else:
        want = np.concatenate([x.max(1), x.argmax(1).astype(dtype)])
    out = np.zeros(want.size, dtype)
    _reduce_kernel[(1,)](x, out, M=m, N=n, CASE=case, num_warps=nw)
    np.testing.assert_array_equal(out, np.asarray(want).ravel())


# -- tl.associative_scan ---------------------------------------------------------------

@enceladus.jit
def _compose(a0, a1, b0, b1):
    # affine maps t -> a0 * t + a1, applied earlier-first: not commutative
    return a0 * b0, a1 * b0 + b1


@enceladus.jit
def _max(a, b):
    return tl.maximum(a, b)


@enceladus.jit
def _scan_kernel(x_ptr, y_ptr, out_ptr, M: tl.constexpr, N: tl.constexpr, AX: tl.constexpr,
                 CASE: tl.constexpr, REV: tl.constexpr):
    rm, rn = tl.arange(0, M), tl.arange(0, N)
    tile = rm[:, None] * N + rn[None, :]
    x = tl.load(x_ptr + tile)
    if CASE == "add":
        tl.store(out_ptr + tile, tl.associative_scan(x, AX, _add, reverse=REV))
    elif CASE == "max":
        tl.store(out_ptr + tile, x.associative_scan(AX, _max, reverse=REV))
    else:  # "affine"
        y = tl.load(y_ptr + tile)
        p, q = tl.associative_scan((x, y), AX, _compose, reverse=REV)
        tl.store(out_ptr + tile, p)
        tl.store(out_ptr + M * N + tile, q)


def _hillis_steele(xs, axis, fn, reverse):
    xs = [np.moveaxis(x, axis, -1) for x in xs]
    if reverse:
        xs = [x[..., ::-1] for x in xs]
    n, s = xs[0].shape[-1], 1
    while s < n:
        res = fn(*[x[..., :n - s] for x in xs], *[x[..., s:] for x in xs])
        res = res if isinstance(res, tuple) else (res,)
        xs = [np.concatenate([x[..., :s], r], -1) for x, r in zip(xs, res)]
        s *= 2
    if reverse:
        xs = [x[..., ::-1] for x in xs]
    return [np.moveaxis(x, -1, axis) for x in xs]


@pytest.mark.parametrize("case,dtype,m,n,ax,rev,nw", [
    ("add", np.int32, 4, 256, 1, False, 4),
    ("add", np.int32, 4, 256, 1, True, 4),
    ("add", np.int32, 128, 8, 0, False, 4),
    ("add", np.float32, 8, 64, 1, False, 2),
    ("max", np.float32, 16, 128, 1, True, 4),
    ("max", np.int32, 64, 4, 0, True, 1),
    ("affine", np.int32, 2, 512, 1, False, 4),
    ("affine", np.int32, 2, 512, 1, True, 4),
    ("affine", np.float32, 32, 16, 0, False, 4),
])
def test_associative_scan(case, dtype, m, n, ax, rev, nw):
    _say(f"associative_scan {case} {np.dtype(dtype).name} {m}x{n} axis={ax} rev={rev}")
    rng = np.random.default_rng(4)
    x = _gen(rng, (m, n), dtype)
    y = _gen(rng, (m, n), dtype)
    if case == "affine" and dtype is np.int32:
        x = rng.choice(np.array([-1, 1], dtype), (m, n))
        y = rng.integers(-3, 4, (m, n)).astype(dtype)
    if case == "affine" and dtype is np.float32:
        x = (0.5 + rng.random((m, n))).astype(dtype)
    fns = {"add": lambda a, b: (a + b).astype(dtype),
           "max": lambda a, b: np.maximum(a, b),
           "affine": lambda a0, a1, b0, b1: ((a0 * b0).astype(dtype),
                                             (a1 * b0 + b1).astype(dtype))}
    ins = [x, y] if case == "affine" else [x]
    want = np.concatenate([w.ravel() for w in _hillis_steele(ins, ax, fns[case], rev)])
    out = np.zeros(want.size, dtype)
    _scan_kernel[(1,)](x, y, out, M=m, N=n, AX=ax, CASE=case, REV=rev, num_warps=nw)
    if dtype is np.float32 and case == "affine":
        np.testing.assert_allclose(out, want, rtol=1e-5, atol=1e-5)
    else:
        np.testing.assert_array_equal(out, want)
    if case == "add" and dtype is np.int32:
        ref = np.flip(np.cumsum(np.flip(x, ax), axis=ax), ax) if rev else np.cumsum(x, axis=ax)
        np.testing.assert_array_equal(out.reshape(m, n), ref.astype(dtype))
