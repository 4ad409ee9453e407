"""GPU parity for exactly what `bench.py` times, at the BASELINE configs' full sizes.

Every variant in `examples.workloads.table()` (the table the benchmark draws its launches
from: kernel, dtypes, constexprs, `num_warps`, `dot_warps`, and the autotuner's candidate
lists for matmul and attention) runs here on the full-size seeded inputs and is checked
against the CPU oracle (reference protocol: tests/conftest.py:102-145):

- softmax, RMSNorm [4096, 8192] and cumsum [8192, 4096]: the oracle runs every program;
- vector add 2^28: bit-exact against the closed form on every element, plus the oracle on
  a random sample of 2,048 programs;
- histogram 2^26 -> 1024 bins, and a ragged 2^26 + 3*1024 + 5: bit-exact against the
  closed form (np.bincount, pinned against the oracle in test_oracle.py); the launch is
  asserted to coarsen programs (several programs per workgroup, unrolled walk and tail);
- matmul and matmul + bias + GELU 4096^3: every element against an fp32 product (the
  oracle's `dot` arithmetic) at the fp16 tolerance, plus the oracle itself on sampled
  programs;
- flash attention bf16 [4,32,4096,128] causal and [4,32,1024,128]: every output element
  against an fp32 reference computed on the GPU, the oracle on a sample of
  (start_m, batch*head) programs stratified over start_m (first, middle, last blocks) and
  the float64 closed form on the same rows;
- the two copy kernels the benchmark reports as HBM ceilings: bit-exact; the read-only
  (max per tile) and write-only (fill) ceilings: exact.

Tolerances: the reference's by output dtype (tests/conftest.py:75-79): fp32 (1e-5, 1e-5)
with atol 1e-8 for softmax outputs of ~1/8192; fp16 (atol 1e-3, rtol 2e-3); bf16
(atol 1e-2, rtol 1.6e-2), 2e-2 against float64. Integer results must match exactly.
"""

from __future__ import annotations

import functools

import numpy as np
import pytest

from examples import workloads as W
from oracle import interpreter as O
from oracle import reference_np as R

pytestmark = pytest.mark.gpu

TABLE = W.table()


def _say(msg):
    print(f"[case] {msg}", flush=True)


def _params(name):
    return [pytest.param(v, id=_id(v)) for v in TABLE[name].variants]


def _id(v):
    return v.label.replace(", ", "/").replace(" ", ",")


@functools.lru_cache(maxsize=None)
def _host(name):
    return TABLE[name].inputs()


_BUFS: dict = {}


def _bufs(name):
    """Device buffers of one workload (kept while its tests run; the previous workload's
    are dropped to bound device memory)."""
    if name not in _BUFS:
        _BUFS.clear()
        _BUFS[name] = W.device_buffers(TABLE[name], _host(name))
    return _BUFS[name]


def _run(name, v):
    import torch
    b = _bufs(name)
    for k in TABLE[name].outputs:
        b[k].zero_()
    ck = W.launch(TABLE[name], b, v)
    torch.cuda.synchronize()
    return b, ck


# -- HBM-bound rows ----------------------------------------------------------------

@functools.lru_cache(maxsize=None)
def _oracle_rows(name):
    h = _host(name)
    wl = TABLE[name]
    v = wl.variants[0]
    x = h["x"]
    out = np.zeros(wl.outputs[next(iter(wl.outputs))][0], np.float32 if x.dtype.kind == "f"
                   else np.int32)
    m, n = x.shape
    c = dict(v.constexprs)
    if name == "softmax":
        O.run_grid(wl.kernel(), (m,), out, x, n, n, n, **c)
    elif name == "rmsnorm":
        O.run_grid(wl.kernel(), (m,), x, h["w"], out, n, n, n, 1e-6, **c)
    else:
        O.run_grid(wl.kernel(), (m,), out, x, m, n, n, n, **c)
    return out


@pytest.mark.parametrize("v", _params("softmax"))
def test_softmax_full(v):
    _say(f"softmax [4096, 8192] {v.label}")
    b, _ = _run("softmax", v)
    got = b["out"].cpu().numpy()
    np.testing.assert_allclose(got, _oracle_rows("softmax"), rtol=1e-5, atol=1e-8)
    np.testing.assert_allclose(got[::97], R.softmax(_host("softmax")["x"][::97]), rtol=1e-5,
                               atol=1e-8)


@pytest.mark.parametrize("v", _params("rmsnorm"))
def test_rmsnorm_full(v):
    _say(f"rmsnorm [4096, 8192] {v.label}")
    b, _ = _run("rmsnorm", v)
    got = b["out"].cpu().numpy()
    np.testing.assert_allclose(got, _oracle_rows("rmsnorm"), rtol=1e-5, atol=1e-5)
    h = _host("rmsnorm")
    np.testing.assert_allclose(got[::97], R.rmsnorm(h["x"][::97], h["w"]), rtol=1e-5,
                               atol=1e-5)


@pytest.mark.parametrize("v", _params("cumsum"))
def test_cumsum_full(v):
    _say(f"cumsum int32 [8192, 4096] {v.label}")
    b, _ = _run("cumsum", v)
    got = b["out"].cpu().numpy()
    assert np.array_equal(got, _oracle_rows("cumsum"))
    assert np.array_equal(got, R.cumsum(_host("cumsum")["x"]))


@pytest.mark.parametrize("v", _params("vector_add"))
def test_vector_add_full(v):
    _say(f"vector add fp32 2^28 {v.label}")
    b, _ = _run("vector_add", v)
    got = b["out"].cpu().numpy()
    h = _host("vector_add")
    assert np.array_equal(got, h["x"] + h["y"])
    # the oracle on 2,048 random programs and the last one (programs are independent)
    n = W.VADD_N
    nprog = n // 1024
    pids = np.random.default_rng(7).choice(nprog, 2048, replace=False).tolist() + [nprog - 1]
    want = np.zeros(n, np.float32)
    O.run_grid(TABLE["vector_add"].kernel(), (nprog,), h["x"], h["y"], want, n, BLOCK=1024,
               programs=[(p,) for p in pids])
    for p in pids:
        s = slice(p * 1024, (p + 1) * 1024)
        assert np.array_equal(got[s], want[s]), f"program {p}"


@pytest.mark.parametrize("name,v", [pytest.param(nm, v, id=f"{nm}-" + _id(v))
                                    for nm in ("copy_rows", "copy_flat")
                                    for v in TABLE[nm].variants])
def test_copy_ceilings_full(name, v):
    """The copy kernels the bench reports as HBM ceilings move every byte unchanged."""
    _say(f"{name} {v.label}")
    b, _ = _run(name, v)
    assert np.array_equal(b["out"].cpu().numpy(), _host(name)["x"])


@pytest.mark.parametrize("v", _params("read_flat"))
def test_read_ceiling_full(v):
    """The read-only ceiling kernel: each program's max matches the closed form exactly
    (a max is exact in any order)."""
    _say(f"read_flat {v.label}")
    b, _ = _run("read_flat", v)
    x = _host("read_flat")["x"]
    block = dict(v.constexprs)["BLOCK"]
    want = x.reshape(-1, block).max(axis=1)
    got = b["out"].cpu().numpy()[:want.size]
    assert np.array_equal(got, want)


@pytest.mark.parametrize("v", _params("fill_flat"))
def test_fill_ceiling_full(v):
    """The write-only ceiling kernel stores the constant into every element."""
    _say(f"fill_flat {v.label}")
    b, _ = _run("fill_flat", v)
    assert np.all(b["out"].cpu().numpy() == np.float32(1.5))


HIST_SIZES = [W.HIST_N, W.HIST_N + 3 * 1024 + 5]


@functools.lru_cache(maxsize=None)
def _hist_host(n):
    return W.hist_inputs(n)["x"]


# the timed variant, and the 8-wave program the table leaves out (it runs slower, not wrong)
_HIST_EXTRA = [W.Variant((("BLOCK", 1024), ("NUM_BINS", W.HIST_BINS)), 8)]


@pytest.mark.parametrize("n", HIST_SIZES, ids=["2^26", "2^26+3077"])
@pytest.mark.parametrize("v", _params("histogram") +
                         [pytest.param(v, id=_id(v)) for v in _HIST_EXTRA])
def test_histogram_full(v, n):
    import torch
    _say(f"histogram int32 n={n} -> 1024 bins {v.label}")
    wl = TABLE["histogram"]
    x = _hist_host(n)
    bufs = {"x": torch.from_numpy(x).cuda(),
            "hist": torch.zeros(W.HIST_BINS, dtype=torch.int32, device="cuda")}
    grid, args = wl.args(bufs, v)
    ck = W.launch(wl, bufs, v)
    torch.cuda.synchronize()
    got = bufs["hist"].cpu().numpy()
    assert np.array_equal(got, R.histogram(x, W.HIST_BINS, 0.0, 1024.0))
    assert int(got.sum()) == n
    # the coarsened walk ran: fewer workgroups than programs, each walking several
    (gx, _, _), _ = ck.launch_grid(grid)
    assert ck.gen.coarsen and gx < grid[0], (gx, grid)
    assert ck.gen.flush is not None          # the two-level flush of the timed config


# -- MFMA-bound rows ------------------------------------------------------------------

@functools.lru_cache(maxsize=None)
def _mm_f32():
    h = _host("matmul")
    return h["a"].astype(np.float32) @ h["b"].astype(np.float32)


def _mm_programs(v):
    c = dict(v.constexprs)
    gx, gy = W.MM // c["BN"], W.MM // c["BM"]
    return [(0, 0), (gx - 1, gy - 1), (gx // 2, 1 % gy)]


def _check_tiles(got, want, v, atol, rtol):
    c = dict(v.constexprs)
    for pn, pm in _mm_programs(v):
        rs = slice(pm * c["BM"], (pm + 1) * c["BM"])
        cs = slice(pn * c["BN"], (pn + 1) * c["BN"])
        np.testing.assert_allclose(got[rs, cs].astype(np.float32),
                                   want[rs, cs].astype(np.float32), atol=atol, rtol=rtol,
                                   err_msg=f"program ({pn}, {pm})")


@pytest.mark.parametrize("v", _params("matmul"))
def test_matmul_full(v):
    _say(f"matmul fp16 4096^3 {v.label}")
    b, _ = _run("matmul", v)
    got = b["c"].cpu().numpy()
    want = _mm_f32().astype(np.float16)
    np.testing.assert_allclose(got.astype(np.float32), want.astype(np.float32), atol=1e-3,
                               rtol=2e-3)
    h = _host("matmul")
    ora = np.zeros((W.MM, W.MM), np.float16)
    O.run_grid(TABLE["matmul"].kernel(), (1, 1), h["a"], h["b"], ora, W.MM, W.MM, W.MM,
               W.MM, W.MM, W.MM, **dict(v.constexprs), programs=_mm_programs(v))
    _check_tiles(got, ora, v, 1e-3, 2e-3)


@functools.lru_cache(maxsize=None)
def _gelu_ref():
    from scipy.special import erf
    h = _host("matmul_gelu")
    y = _mm_f32().astype(np.float64) + h["bias"].astype(np.float64)
    return (0.5 * y * (1.0 + erf(y / np.sqrt(2.0)))).astype(np.float16)


@pytest.mark.parametrize("v", _params("matmul_gelu"))
def test_matmul_gelu_full(v):
    _say(f"matmul + bias + GELU fp16 4096^3 {v.label}")
    b, _ = _run("matmul_gelu", v)
    got = b["c"].cpu().numpy()
    np.testing.assert_allclose(got.astype(np.float32), _gelu_ref().astype(np.float32),
                               atol=1e-3, rtol=2e-3)
    h = _host("matmul_gelu")
    ora = np.zeros((W.MM, W.MM), np.float16)
    O.run_grid(TABLE["matmul_gelu"].kernel(), (1, 1), h["a"], h["b"], h["bias"], ora, W.MM,
               W.MM, W.MM, W.MM, W.MM, W.MM, **dict(v.constexprs), programs=_mm_programs(v))
    _check_tiles(got, ora, v, 1e-3, 2e-3)


def _att_programs(n, bm):
    nblk = n // bm
    starts = sorted({0, nblk // 2, nblk - 1})
    heads = [5, 77]                     # (batch, head) = (0, 5) and (2, 13)
    return [(s, h) for s in starts for h in heads]


@functools.lru_cache(maxsize=2)
def _attention_fp32(name):
    """softmax(q k^T / sqrt(d)) v of the whole workload in float32 on the GPU, computed per
    (batch, group of 8 heads) to bound memory: the reference every output element of the
    timed kernels is compared with. fp32 matmuls on contiguous operands only."""
    import torch
    b = _bufs(name)
    q, k, v = (b[x] for x in "qkv")
    z, h, n, d = q.shape
    causal = name == "attention_causal"
    out = torch.empty((z, h, n, d), dtype=torch.float32, device=q.device)
    keep = torch.ones(n, n, dtype=torch.bool, device=q.device).tril() if causal else None
    for zi in range(z):
        for h0 in range(0, h, 8):
            qf = q[zi, h0:h0 + 8].float().contiguous()
            kt = k[zi, h0:h0 + 8].float().transpose(1, 2).contiguous()
            vf = v[zi, h0:h0 + 8].float().contiguous()
            sc = torch.matmul(qf, kt) * (d ** -0.5)
            if causal:
                sc = sc.masked_fill(~keep, float("-inf"))
            out[zi, h0:h0 + 8] = torch.matmul(torch.softmax(sc, dim=-1), vf)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("name,v", [pytest.param(nm, v, id=f"{nm}-" + _id(v))
                                    for nm in ("attention_causal", "attention_noncausal")
                                    for v in TABLE[nm].variants])
def test_attention_full(name, v):
    """Every output element of every timed variant against an fp32 reference computed on
    the GPU (atol 1e-2, rtol 1.6e-2: the bf16 tolerance), plus the oracle and the float64
    closed form on a stratified sample of programs."""
    import torch
    c = dict(v.constexprs)
    causal = c["CAUSAL"]
    _say(f"{name} bf16 {TABLE[name].describe} {v.label}")
    b, _ = _run(name, v)
    ref = _attention_fp32(name)
    err = (b["o"].float() - ref).abs()
    bound = 1e-2 + 1.6e-2 * ref.abs()
    bad = int((err > bound).sum())
    assert bad == 0, f"{bad} of {ref.numel()} output elements outside atol 1e-2 rtol 1.6e-2 " \
                     f"(max abs error {float(err.max()):.3g})"
    assert bool(torch.isfinite(b["o"].float()).all())
    got = b["o"].float().cpu().numpy()
    h = _host(name)
    n = h["q"].shape[2]
    ora = torch.zeros_like(h["q"])
    progs = _att_programs(n, c["BLOCK_M"])
    O.run_grid(TABLE[name].kernel(), (1, 1), h["q"], h["k"], h["v"], ora, W.ATT_D ** -0.5, n,
               n * W.ATT_D, W.ATT_D, **c, programs=progs)
    ora = ora.float().numpy()
    qf, kf, vf = (h[x].float().numpy() for x in "qkv")
    bm = c["BLOCK_M"]
    for s, bh in progs:
        z, hh = divmod(bh, W.ATT_H)
        rows = slice(s * bm, (s + 1) * bm)
        np.testing.assert_allclose(got[z, hh, rows], ora[z, hh, rows], rtol=1.6e-2, atol=1e-2,
                                   err_msg=f"program (start_m={s}, bh={bh}) vs oracle")
        # float64 closed form for the same query rows
        sc = (qf[z, hh, rows].astype(np.float64) @ kf[z, hh].astype(np.float64).T) \
            * W.ATT_D ** -0.5
        if causal:
            r = np.arange(s * bm, (s + 1) * bm)[:, None]
            sc = np.where(np.arange(n)[None, :] <= r, sc, -np.inf)
        p = np.exp(sc - sc.max(-1, keepdims=True))
        want = (p / p.sum(-1, keepdims=True)) @ vf[z, hh].astype(np.float64)
        np.testing.assert_allclose(got[z, hh, rows], want, rtol=2e-2, atol=2e-2,
                                   err_msg=f"program (start_m={s}, bh={bh}) vs float64")
