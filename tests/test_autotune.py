"""The autotuner: keys, persistence and state handling on the CPU; tuning on the GPU
(reference test strategy: tests/test_autotune.py)."""

import json
import os
import subprocess
import sys

import numpy as np
import pytest

import enceladus
import enceladus.language as tl
from enceladus_amd.runtime import autotuner as A

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@enceladus.jit
def _scale(x_ptr, out_ptr, n, factor, BLOCK: tl.constexpr, MODE: tl.constexpr = 0):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    tl.store(out_ptr + offs, tl.load(x_ptr + offs, mask=m) * factor, mask=m)


@enceladus.jit
def _accumulate(x_ptr, out_ptr, n, BLOCK: tl.constexpr):
    # adds into out: benchmarking it repeatedly would accumulate without reset_to_zero
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    tl.atomic_add(out_ptr + offs, tl.load(x_ptr + offs, mask=m), mask=m)


CONFIGS = [A.Config({"BLOCK": 128}), A.Config({"BLOCK": 256}, num_warps=8),
           A.Config({"BLOCK": 1024})]


def test_keys_normalise_scalars_dtypes_and_defaults():
    t = A.autotune(CONFIGS, key=["n", "MODE"])(_scale)
    x = np.zeros(10, np.float32)
    named = A._named(t.fn, (x, x, 10, 2.0), {})
    assert named["MODE"] == 0                     # the signature default fills the key
    k1 = t._key(named)
    k2 = t._key(A._named(t.fn, (x, x, np.int64(10), 2.0), {"MODE": 0}))
    assert k1 == k2                               # NumPy scalar == Python number
    k3 = t._key(A._named(t.fn, (x.astype(np.float16), x.astype(np.float16), 10, 2.0), {}))
    assert k3 != k1                               # element dtypes are part of the key
    assert A._key_value(tl.float16) == A._key_value(np.float16) == A._key_value("float16")


def test_logged_winner_must_still_be_a_candidate(tmp_path, monkeypatch):
    monkeypatch.setenv("ENCELADUS_CACHE_DIR", str(tmp_path))
    t = A.autotune(CONFIGS, key=["n"])(_scale)
    x = np.zeros(10, np.float32)
    named = A._named(t.fn, (x, x, 10, 2.0), {})
    key = t._key(named)
    t.tune_log.put(key, CONFIGS[1], {"Config(BLOCK=256)": 0.01})
    lines = t.log_path().read_text().splitlines()
    rec = json.loads(lines[-1])
    assert rec["key"] == key and rec["config"]["kwargs"] == {"BLOCK": 256}
    assert rec["config"]["num_warps"] == 8 and rec["timings_ms"]
    fresh = A.autotune(CONFIGS, key=["n"])(_scale)
    assert fresh._resolve(named, None) == CONFIGS[1]          # from the log, untuned
    pruned = A.autotune(CONFIGS[:1], key=["n"])(_scale)       # the winner is gone
    assert pruned._resolve(named, lambda k: "tuned") == "tuned"
    # a later line supersedes an earlier one; a torn line is skipped
    t.tune_log.put(key, CONFIGS[2], {})
    with open(t.log_path(), "a") as f:
        f.write('{"key": "torn", "conf')
    again = A.autotune(CONFIGS, key=["n"])(_scale)
    assert again._resolve(named, None) == CONFIGS[2]


def test_results_file_depends_on_the_compiler(tmp_path, monkeypatch):
    monkeypatch.setenv("ENCELADUS_CACHE_DIR", str(tmp_path))
    t = A.autotune(CONFIGS, key=["n"])(_scale)
    p1 = t.log_path()
    monkeypatch.setattr(A, "_compiler_hash", lambda: "different")
    assert t.log_path() != p1


def test_concurrent_appends_keep_every_result(tmp_path, monkeypatch):
    monkeypatch.setenv("ENCELADUS_CACHE_DIR", str(tmp_path))
    script = f"""
import sys; sys.path.insert(0, {ROOT!r}); sys.path.insert(0, {os.path.join(ROOT, 'tests')!r})
import os
os.environ["ENCELADUS_CACHE_DIR"] = {str(tmp_path)!r}
from test_autotune import CONFIGS, _scale
from enceladus_amd.runtime import autotuner as A
i = int(sys.argv[1])
t = A.autotune(CONFIGS, key=["n"])(_scale)
for j in range(20):
    t.tune_log.put(f"key{{i}}-{{j}}", CONFIGS[j % 3], {{"x" * 300: 1.0}})
"""
    procs = [subprocess.Popen([sys.executable, "-c", script, str(i)]) for i in range(4)]
    assert all(p.wait(timeout=120) == 0 for p in procs)
    t = A.autotune(CONFIGS, key=["n"])(_scale)
    assert len(t.tune_log.entries()) == 80
    assert all(json.loads(ln) for ln in t.log_path().read_text().splitlines())


def test_state_helpers_restore_and_zero():
    a = np.arange(5, dtype=np.float32)
    snap = A._snapshot(a)
    a += 3
    A._restore(a, snap)
    assert np.array_equal(a, np.arange(5, dtype=np.float32))
    A._zero(a)
    assert not a.any()


def test_heuristics_compute_constexprs():
    h = A.heuristics({"BLOCK": lambda a: 1 << (a["n"] - 1).bit_length()})(_scale)
    x = np.zeros(4, np.float32)
    assert h.resolve((x, x, 100, 1.0), {})["BLOCK"] == 128
    assert h.arg_names == _scale.arg_names


# -- on the GPU ------------------------------------------------------------------------

@pytest.mark.gpu
def test_tuning_skips_failing_configs_and_resets_state(tmp_path, monkeypatch):
    monkeypatch.setenv("ENCELADUS_CACHE_DIR", str(tmp_path))
    print("[case] autotune reset_to_zero", flush=True)
    bad = A.Config({"BLOCK": 100})                      # not a power of two: fails
    t = A.autotune([bad] + CONFIGS, key=["n"], reset_to_zero=["out_ptr"], rep=3,
                   warmup_ms=1)(_accumulate)
    n = 5000
    x = np.ones(n, np.float32)
    out = np.zeros(n, np.float32)
    with pytest.warns(UserWarning, match="skipping"):
        t[lambda m: (enceladus.cdiv(n, m["BLOCK"]),)](x, out, n)
    # tuning ran the kernel many times; the reset leaves exactly one launch's sum
    np.testing.assert_array_equal(out, 1.0)
    assert t.config_for(x, out, n) in CONFIGS
    ck = t.warmup(x, out, n)
    assert ck.name == "ek__accumulate"


@pytest.mark.gpu
def test_restore_value_and_persistence(tmp_path, monkeypatch):
    monkeypatch.setenv("ENCELADUS_CACHE_DIR", str(tmp_path))
    print("[case] autotune restore_value + persistence", flush=True)
    t = A.autotune(CONFIGS, key=["n"], restore_value=["out_ptr"], rep=3,
                   warmup_ms=1)(_accumulate)
    n = 3000
    x = np.full(n, 2.0, np.float32)
    out = np.full(n, 5.0, np.float32)
    t[lambda m: (enceladus.cdiv(n, m["BLOCK"]),)](x, out, n)
    np.testing.assert_array_equal(out, 7.0)
    win = t.config_for(x, out, n)
    again = A.autotune(CONFIGS, key=["n"], restore_value=["out_ptr"])(_accumulate)
    out2 = np.zeros(n, np.float32)
    again[lambda m: (enceladus.cdiv(n, m["BLOCK"]),)](x, out2, n)   # no tuning: saved winner
    np.testing.assert_array_equal(out2, 2.0)
    assert again.config_for(x, out2, n) == win and not again.timings


@pytest.mark.gpu
def test_tuned_matmul_example_matches_torch(tmp_path, monkeypatch):
    import warnings
    import torch
    sys.path.insert(0, os.path.join(ROOT, "examples"))
    from matmul import matmul_tuned
    monkeypatch.setenv("ENCELADUS_CACHE_DIR", str(tmp_path))
    print("[case] autotuned matmul 512x384x256 fp16", flush=True)
    g = torch.Generator().manual_seed(3)
    a = torch.randn(512, 256, generator=g).half().cuda()
    b = torch.randn(256, 384, generator=g).half().cuda()
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        c = matmul_tuned(a, b)
    torch.cuda.synchronize()
    ref = a.float() @ b.float()
    torch.testing.assert_close(c.float(), ref, rtol=1e-2, atol=1e-2)


@pytest.mark.gpu
def test_attention_tuned_example_matches_float64(tmp_path, monkeypatch):
    """attention_tuned (reference: examples/08_flash_attention.py:106-127) tunes over every
    attention_configs candidate for the dtype and head dimension and returns the same
    result as `attention`."""
    import warnings
    import torch
    from examples.flash_attention import attention, attention_tuned
    from oracle import reference_np as R
    monkeypatch.setenv("ENCELADUS_CACHE_DIR", str(tmp_path))
    print("[case] attention_tuned bf16 [1, 2, 256, 128] causal", flush=True)
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(1, 2, 256, 128, generator=g).bfloat16().cuda() for _ in range(3))
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        o = attention_tuned(q, k, v, causal=True)
    torch.cuda.synchronize()
    want = R.attention(*(x.float().cpu().numpy() for x in (q, k, v)), True)
    np.testing.assert_allclose(o.float().cpu().numpy(), want, rtol=2e-2, atol=2e-2)
    ref = attention(q, k, v, True)
    torch.testing.assert_close(o.float(), ref.float(), rtol=2e-2, atol=2e-2)
    with pytest.raises(ValueError, match="head_dim"):
        attention_tuned(q[..., :96], k[..., :96], v[..., :96])


@pytest.mark.gpu
def test_do_bench_times_dispatches_not_host_latency():
    """do_bench's samples are the GPU time of the dispatches: a launch preceded by a host
    sleep of 2 ms still times as the kernel alone."""
    import time
    import torch
    from enceladus_amd.testing import do_bench
    print("[case] do_bench dispatch timing", flush=True)
    n = 1 << 20
    x = torch.randn(n, device="cuda")
    out = torch.empty_like(x)

    def slow_host():
        time.sleep(0.002)
        _scale[(n // 1024,)](x, out, n, 2.0, BLOCK=1024)
    ms = do_bench(slow_host, warmup_ms=1, rep=5)
    assert ms < 1.0, ms                 # a 4 MB scale takes microseconds, not the 2 ms sleep
    torch.testing.assert_close(out, x * 2.0)
