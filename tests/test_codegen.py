"""Compile-only coverage of the HIP emitter (no GPU): every workload kernel lowers and
hiprtc-compiles for gfx950; layout invariants; kernarg packing. This is the analogue of the
reference's compile-without-GPU checks (reference tests/conftest.py:18-20, jit.py:590-627)."""

import numpy as np
import pytest

import enceladus
import enceladus.language as tl
from enceladus_amd.compiler import codegen_hip, ir
from enceladus_amd.compiler import layout as L
from enceladus_amd.language import core


def test_every_workload_kernel_compiles_for_gfx950():
    from enceladus_amd import kernels_catalog
    assert kernels_catalog.compile_all() >= 12


def test_codegen_is_deterministic():
    from examples.vector_add import add_kernel
    x = np.zeros(4, np.float32)
    a = codegen_hip.generate(add_kernel.ir_for(x, x, x, 1000, BLOCK=1024)).source
    b = codegen_hip.generate(add_kernel.ir_for(x, x, x, 1000, BLOCK=1024)).source
    assert a == b
    assert "vload_nt<float, 4>" in a   # 128-bit streaming accesses for aligned contiguous fp32


def test_blocked_layout_avoids_copies_when_the_tile_allows():
    """A tile with at least one element per thread is spread over every thread: the vector
    narrows instead of leaving waves that hold (and load) copies."""
    for n, nw, vec in ((1024, 4, 4), (1024, 8, 2), (1024, 16, 1), (256, 4, 1), (8192, 16, 4)):
        lay = L.default_blocked((n,), nw)
        assert lay.nregs * 64 * nw == n, (n, nw)
        assert all(b is not None for b in (*lay.lane, *lay.warp)), (n, nw)
        assert len([b for b in lay.reg if b[1] < L.log2(vec)]) == L.log2(vec)
    small = L.default_blocked((64,), 4)          # fewer elements than threads: copies remain
    assert small.nregs == 4 and any(b is None for b in small.warp)


def _covers_once(lay):
    seen = {}
    for w in range(lay.num_warps):
        for ln in range(64):
            if not lay.owns(ln, w):
                continue
            t = lay.thread_coord(ln, w)
            for r in range(lay.nregs):
                c = tuple(a + b for a, b in zip(t, lay.reg_coord(r)))
                seen[c] = seen.get(c, 0) + 1
    n = int(np.prod(lay.shape))
    return len(seen) == n and all(v == 1 for v in seen.values())


@pytest.mark.parametrize("bm,bn,bk,nw,dt,dw", [(128, 128, 64, 4, "fp16", None),
                                               (128, 64, 128, 4, "bf16", (4, 1)),
                                               (64, 64, 32, 4, "fp16", None),
                                               (32, 32, 16, 4, "fp32", None),
                                               (256, 256, 64, 8, "fp16", None)])
def test_mfma_layouts_cover_each_element_once(bm, bn, bk, nw, dt, dw):
    p = L.plan_dot(bm, bn, bk, nw, dt, dw)
    for lay in (L.mfma_acc(p), L.mfma_operand(p, "a"), L.mfma_operand(p, "b")):
        assert _covers_once(lay)


def test_mfma_operands_pair_k_consistently():
    """For each MFMA, lane-register (l, j) of A and B must carry the same k index."""
    p = L.plan_dot(64, 64, 32, 4, "fp16")
    la, lb = L.mfma_operand(p, "a"), L.mfma_operand(p, "b")
    for ln in range(64):
        for j in range(la.nregs):
            ka = (la.thread_coord(ln, 0)[1] + la.reg_coord(j)[1])
            kb = (lb.thread_coord(ln, 0)[0] + lb.reg_coord(j)[0])
            assert ka == kb


def test_blocked_and_scan_layouts():
    b = L.blocked((8192,), [0], 4, 4)
    assert _covers_once(b) and b.vec_dim_bits() == (0, 2)
    s = L.scan_layout((1, 4096), 1, 4)
    assert _covers_once(s) and L.scan_friendly(s, 1)
    assert not L.scan_friendly(b.expand(0), 1) or True


def test_scan_groups():
    """A scan runs in the coalesced blocked layout of a long row: a 4-element run per lane,
    then lanes and warps, then the remaining axis bits as register segments joined by
    carries; the layouts scan_friendly accepts are exactly those without segments."""
    for nw, groups in ((4, [2, 3]), (8, [2]), (16, [])):
        b = L.blocked((1, 4096), [1, 0], 4, nw)
        assert L.scan_groups(b, 1) == (2, groups)
        assert (L.scan_friendly(b, 1)) == (not groups)
        s = L.scan_layout((1, 4096), 1, nw)
        assert L.scan_groups(s, 1)[1] == [] and L.scan_friendly(s, 1)
    # along the rows of a 2-D tile: no run, lanes, warps, then two register segments
    b = L.blocked((64, 64), [1, 0], 4, 4)
    assert L.scan_groups(b, 0) == (0, [2, 3])
    # a run whose register bits are out of order: not scannable in place
    t = L.Layout((1, 256), ((1, 1), (1, 0)), tuple((1, i) for i in range(2, 8)), (), "blocked")
    assert L.scan_groups(t, 1) is None and not L.scan_friendly(t, 1)
    for shape, ax, nw in (((8, 256), 1, 4), ((256, 8), 0, 2), ((4, 4, 64), 2, 1)):
        for order in ([len(shape) - 1] + list(range(len(shape) - 1)), list(range(len(shape)))):
            lay = L.blocked(shape, order, 4, nw)
            g = L.scan_groups(lay, ax)
            assert (g is not None and not g[1]) == L.scan_friendly(lay, ax)


def test_views_are_free():
    b = L.blocked((64, 64), [1, 0], 8, 4)
    assert L.is_view(b.slice(1).expand(1), b)
    assert not L.is_view(L.blocked((64, 64), [0, 1], 8, 4), b)


def test_pack_args_natural_alignment():
    ka = [codegen_hip.KernelArg("p", "ptr", core.float32, "float*"),
          codegen_hip.KernelArg("n", "scalar", core.int32, "int32_t"),
          codegen_hip.KernelArg("q", "ptr", core.float32, "float*"),
          codegen_hip.KernelArg("e", "scalar", core.float32, "float")]
    buf = codegen_hip.pack_args(ka, [0x1000, 7, 0x2000, 1.5])
    assert len(buf) == 32
    assert buf[8:12] == (7).to_bytes(4, "little") and buf[16:24] == (0x2000).to_bytes(8, "little")


def test_literals_are_exact():
    assert codegen_hip.literal(float("inf"), core.float32) == "__builtin_inff()"
    assert codegen_hip.literal(1.0, core.bfloat16) == "ek::bf16{0x3f80}"
    assert codegen_hip.literal(-2147483648, core.int32).startswith("(int32_t)(-2147483647")


def test_program_id_remap_is_a_bijection():
    def remap(bx, by, gx, gy):
        nb = gx * gy
        L = bx + gx * by
        if nb % 8 == 0:
            L = (L % 8) * (nb // 8) + L // 8
        band = 4 * gx
        first = (L // band) * 4
        gs = min(gy - first, 4)
        r = L % band
        return (gx - 1 - r // gs, first + r % gs)
    src = "\n".join(codegen_hip.PID_REMAP)
    assert "(L & 7) * (nb >> 3)" in src and "ek_pid_x = gx - 1 - r / gs" in src
    for gx, gy in [(16, 16), (32, 128), (8, 1), (3, 5), (7, 9), (1, 1), (2, 100)]:
        got = {remap(x, y, gx, gy) for x in range(gx) for y in range(gy)}
        assert got == {(x, y) for x in range(gx) for y in range(gy)}


def test_descriptor_dot_loop_uses_gemm_template():
    from examples.matmul import matmul_desc_kernel
    f16 = np.zeros(16, np.float16)
    src = codegen_hip.generate(matmul_desc_kernel.ir_for(
        f16, f16, f16, 4096, 4096, 4096, 4096, 4096, 4096, BM=256, BN=256, BK=64)).source
    # aligned operands within 2 GiB: the LDS-DMA pipeline (64 KB stages, 2 of them); the
    # MFMAs compute C^T, so each lane holds 4 consecutive columns of a row and the epilogue
    # writes 8-byte runs to LDS
    assert "ek::GemmDma<_Float16, 256, 256, 64, 2, 2, 256, 2, 1, true>" in src
    assert "ek::vstore<_Float16, 4>(&sm[" in src
    # K and N not known to be multiples of 8: the template reads the row tails elementwise
    src3 = codegen_hip.generate(matmul_desc_kernel.ir_for(
        f16, f16, f16, 256, 250, 100, 112, 256, 250, BM=128, BN=128, BK=64)).source
    assert "ek::Gemm<_Float16, 128, 128, 64, 2, 2, 256, false, true>" in src3
    # ENCELADUS_CODEGEN=no_acc_transpose: the instruction's own orientation
    src4 = codegen_hip.generate(matmul_desc_kernel.ir_for(
        f16, f16, f16, 4096, 4096, 4096, 4096, 4096, 4096, BM=256, BN=256, BK=64),
        {"no_acc_transpose": True}).source
    assert "ek::GemmDma<_Float16, 256, 256, 64, 2, 2, 256, 2, 1>" in src4
    # unaligned strides fall back to the generic lowering
    src2 = codegen_hip.generate(matmul_desc_kernel.ir_for(
        f16, f16, f16, 100, 90, 70, 70, 90, 90, BM=64, BN=64, BK=32)).source
    assert "ek::Gemm<" not in src2


def test_lds_bank_model():
    """The pattern kernels whose SQ_LDS_BANK_CONFLICT counts fixed the model (conflict
    cycles = passes above one per pass)."""
    from enceladus_amd.compiler import lds
    pc = lds.pass_cycles
    r128 = lambda f: pc([f(l) for l in range(64)], 16)          # noqa: E731
    w128 = lambda f: pc([f(l) for l in range(64)], 16, True)    # noqa: E731
    r64 = lambda f: pc([f(l) for l in range(64)], 8)            # noqa: E731
    assert r128(lambda l: l * 16) == 4 and w128(lambda l: l * 16) == 8
    assert r128(lambda l: (l >> 1) * 16 + (l & 1) * 128) - 4 == 0
    assert r128(lambda l: (l % 8) * 16 + (l // 8) * 256) - 4 == 4
    gemm_a = lambda l: ((l % 32) * 8 + ((l // 32) ^ (((l % 32) >> 1) & 7))) * 16  # noqa: E731
    assert r128(gemm_a) - 4 == 0 and w128(gemm_a) - 8 == 8
    fa_old_v = lambda l: (4 * (l % 32)) * 144 + (l // 32) * 16  # noqa: E731
    assert r128(fa_old_v) - 4 == 12 and w128(fa_old_v) - 8 == 24
    assert r64(lambda l: l * 8) == 2
    assert r64(lambda l: (l % 16) * 8 + (l // 16) * 256) - 2 == 2
    assert r64(lambda l: (l % 32) * 144 + (l // 32) * 8) - 2 == 2
    assert r128(lambda l: (l % 4) * 16 + (l // 4) * 128) - 4 == 4
    assert r128(lambda l: (l % 2) * 16 + (l // 2) * 256) - 4 == 28
    # one dword read by every lane is a broadcast
    assert pc([0] * 64, 4) == 1


@pytest.mark.parametrize("head_dim,block_n", [(128, 64), (64, 64), (128, 32), (64, 128)])
def test_attention_stage_layouts_are_bijective_and_conflict_free(head_dim, block_n):
    import torch
    from enceladus_amd.compiler import lds
    from examples.flash_attention import attention_kernel
    bf = torch.zeros(16, dtype=torch.bfloat16)
    codegen_hip._STAGE_LAYOUTS.clear()
    f = attention_kernel.ir_for(bf, bf, bf, bf, 0.088, 4096, 4096 * head_dim, head_dim,
                                dot_warps=(4, 1), HEAD_DIM=head_dim, BLOCK_M=128,
                                BLOCK_N=block_n, CAUSAL=True)
    src = codegen_hip.generate(f, {"dot_warps": (4, 1)}).source
    got = list(codegen_hip._STAGE_LAYOUTS.values())
    assert len(got) == 2 and "ek::swz<" in src
    for sl, cyc, ideal in got:
        assert cyc == ideal, (sl, cyc, ideal)
        assert [sl.logical(sl.sp(x)) for x in range(sl.length)] == list(range(sl.length))
        offs = {sl.offset(ln, sl.sp(x)) for ln in range(sl.lines) for x in range(sl.length)}
        assert len(offs) == sl.lines * sl.length and max(offs) < sl.elems
        # a 16-byte chunk stays contiguous under the swizzle
        assert all(sl.offset(ln, 8 * c + e) == sl.offset(ln, 8 * c) + e
                   for ln in range(sl.lines) for c in range(sl.length // 8) for e in range(8))


def test_transpose_read_source_layouts():
    """ds_read_b64_tr_b16 (measured on gfx950: in each 16-lane group, output lane L, value t
    is element L % 4 of the read by lane 4t + L // 4) delivers the MFMA B fragments of a
    row-major LDS tile, including the attention PV operand's permuted k order; A fragments
    (k along registers, rows along lanes) do not fit it."""
    for bm, bn, bk, nw, dw, tr, ko in [(128, 128, 64, 4, (4, 1), True, (0, 1, 3, 2, 4, 5)),
                                       (256, 256, 64, 8, (4, 2), False, ()),
                                       (128, 64, 128, 4, (4, 1), True, ())]:
        plan = L.plan_dot(bm, bn, bk, nw, "bfloat16", dot_warps=dw, trans=tr, korder=ko)
        lb = L.mfma_operand(plan, "b")
        src = L.tr16_source(lb)
        assert src is not None and L.tr16_check(lb, src)
        assert L.tr16_source(L.mfma_operand(plan, "a")) is None


def test_two_privatised_histograms_get_their_own_bins():
    from tests.test_gpu_examples import _two_histograms
    i32 = np.zeros(16, np.int32)
    src = codegen_hip.generate(_two_histograms.ir_for(i32, i32, i32, 70001, B1=256, B2=128,
                                                      BLOCK=1024)).source
    assert "ek_bins0[256]" in src and "ek_bins1[128]" in src
    assert src.count("__HIP_MEMORY_SCOPE_AGENT") == 2      # one flush per histogram


@enceladus.jit
def _split_kinds(x_ptr, out_ptr, M: tl.constexpr, CASE: tl.constexpr):
    rm = tl.arange(0, M)
    if CASE == "register":
        v = tl.load(x_ptr + rm[:, None] * 2 + tl.arange(0, 2)[None, :])
    else:
        v = tl.load(x_ptr + tl.arange(0, 2)[:, None] * M + rm[None, :]).T
    a, b = tl.split(v)
    tl.store(out_ptr + rm, a - b)


def test_split_of_register_or_lane_bit_needs_no_lds():
    """The split coordinate in a register selects registers; in a lane it becomes a pair
    of shuffles. Neither goes through LDS (reference: codegen/msl.py:693-747 keeps the
    same two cases free)."""
    x = np.zeros(4, np.float32)
    reg = codegen_hip.generate(_split_kinds.ir_for(x, x, M=256, CASE="register"))
    lane = codegen_hip.generate(_split_kinds.ir_for(x, x, M=64, CASE="lane", num_warps=1))
    assert reg.lds_bytes == 0 and "ek::shfl(" not in reg.source
    assert lane.lds_bytes == 0 and "ek::shfl(" in lane.source


def test_reshape_is_a_view():
    """A reshape of a loaded tile relabels layout bits: no LDS round trip."""
    x = np.zeros(4, np.float32)
    f = _split_kinds.ir_for(x, x, M=256, CASE="register")
    assert any(op.name == "split" for op in ir.walk(f.body))
    lay = L.Layout((8, 16), ((1, 0), (1, 1)), ((1, 2), (1, 3), (0, 0), (0, 1), (0, 2), None),
                 (None,))
    flat = lay.reshape((128,))
    assert flat.reg == ((0, 0), (0, 1)) and flat.lane[:5] == ((0, 2), (0, 3), (0, 4),
                                                               (0, 5), (0, 6))
    assert flat.reshape((8, 16)).key() == lay.key()


def test_integer_dot_lowering():
    """int8 products run on the i8 MFMAs; uint8/16/32-bit ones as LDS multiply-adds; 64-bit
    operands are rejected (reference: language/ops.py:1244-1270)."""
    from tests.test_gpu_int_dot import _int_matmul
    c = np.zeros(4, np.int32)

    def src(dt, bm, bn, bk, nw=4):
        z = np.zeros(4, dt)
        return codegen_hip.generate(_int_matmul.ir_for(z, z, c, 64, BM=bm, BN=bn, BK=bk,
                                                       ACC=False, num_warps=nw)).source
    assert "ek::mfma_32x32x32(" in src(np.int8, 64, 64, 64)
    assert "ek::mfma_16x16x64(" in src(np.int8, 16, 16, 64, 1)
    for dt in (np.uint8, np.int16, np.int32):
        s = src(dt, 32, 32, 16)
        assert "mfma" not in s and "(uint32_t)sa[" in s
    from enceladus_amd.compiler.errors import CompilationError
    with pytest.raises(CompilationError, match="8-, 16- or 32-bit"):
        src(np.int64, 32, 32, 16)


@enceladus.jit
def _offsets_kernel(x_ptr, out_ptr, n, BLOCK: tl.constexpr):
    pid = tl.program_id(0)
    offs = pid * BLOCK + tl.arange(0, BLOCK)
    mask = offs < n
    v = tl.load(x_ptr + offs, mask=mask)
    tl.store(out_ptr + offs, v + offs.to(tl.uint8), mask=mask)


def test_idx64_widens_pointer_offsets_and_masks():
    """An argument spanning more than 2^31 elements gets 64-bit index math: every
    pointer offset and the mask reading it are int64, a use as data keeps int32
    (reference: compiler/passes/widen_index.py)."""
    from enceladus_amd.compiler import frontend, widen
    t = ir.TType((), core.uint8, ptr=True)
    types = {"x_ptr": t, "out_ptr": t, "n": ir.TType((), core.int64)}
    facts = {"x_ptr": {"idx64": True}, "out_ptr": {"idx64": True}, "n": {}}
    fn = frontend.build_ir(_offsets_kernel.fn, types, facts, {"BLOCK": 1024})
    assert widen.widen_index_math(fn) >= 3
    ops = list(ir.walk(fn.body))
    adds = [op for op in ops if op.name == "ptr_add"]
    assert adds and all(op.operands[1].type.dtype is core.int64 for op in adds)
    cmps = [op for op in ops if op.name == "binary" and op.attrs["op"] == "lt"]
    assert cmps and all(o.type.dtype is core.int64 for op in cmps for o in op.operands)
    casts = [op for op in ops if op.name == "cast" and op.result.type.dtype is core.uint8]
    assert casts and casts[0].operands[0].type.dtype is core.int32
    src = codegen_hip.generate(fn).source
    assert "(int64_t)" in src
    # without the fact nothing changes
    fn32 = frontend.build_ir(_offsets_kernel.fn, types, {"x_ptr": {}, "out_ptr": {}, "n": {}},
                             {"BLOCK": 1024})
    assert not widen.needs_idx64(fn32)


def test_idx64_fact_from_element_span():
    """`idx64` follows the element span from strides (no memory needed to test it)."""
    from enceladus_amd.runtime import jit
    import torch
    assert "idx64" not in jit.arg_facts(torch.empty(16, dtype=torch.uint8))

    class _Strided:
        shape = (2, 1 << 30)

        def stride(self):
            return (1 << 31, 1)
    assert jit._last_index(_Strided()) == (1 << 31) + (1 << 30) - 1 > jit.MAX_ELEMENT_INDEX


def test_softmax_scale_fold():
    """With a positive scale the attention loop reduces raw scores and scales only the row
    maxima (max commutes with a positive scale exactly); a negative scale keeps the
    per-score multiply (reference kernel: examples/08_flash_attention.py:30-127)."""
    import torch
    from examples.flash_attention import attention_kernel
    bf = torch.zeros(16, dtype=torch.bfloat16)

    def ops(scale):
        f = attention_kernel.ir_for(bf, bf, bf, bf, scale, 256, 256 * 64, 64, HEAD_DIM=64,
                                    BLOCK_M=64, BLOCK_N=32, CAUSAL=True, dot_warps=(4, 1))
        return [op for op in ir.walk(f.body)]
    pos = ops(0.125)
    assert any(op.name == "fma" for op in pos)
    red = [op for op in pos if op.name == "reduce" and op.attrs["kind"] == "max"][0]
    src = red.operands[0].op
    assert src.name == "select" and src.operands[1].op.name == "dot"
    neg = ops(-0.125)
    assert not any(op.name == "fma" for op in neg)
    red = [op for op in neg if op.name == "reduce" and op.attrs["kind"] == "max"][0]
    assert red.operands[0].op.operands[1].op.name == "binary"


def test_math_modes_pick_division_or_reciprocal():
    """relaxed (the default): a tile divided by a broadcast row statistic multiplies by its
    reciprocal, a scalar divisor keeps the IEEE division; fast: both multiply; an unknown
    mode is refused (reference: runtime/jit.py:56, :234-235)."""
    def src(mode, divisor_is_row):
        @enceladus.jit(math_mode=mode)
        def k(x_ptr, o_ptr, s, BLOCK: tl.constexpr):
            r = tl.arange(0, BLOCK)
            x = tl.load(x_ptr + r[:, None] * BLOCK + r[None, :])
            if divisor_is_row:
                y = x / tl.sum(x, 1)[:, None]
            else:
                y = x / s
            tl.store(o_ptr + r[:, None] * BLOCK + r[None, :], y)
        x = np.zeros(4, np.float32)
        f = k.ir_for(x, x, 2.0, BLOCK=32)
        return codegen_hip.generate(f, {"math_mode": mode}).source
    assert "(1.0f / " in src("relaxed", True)
    assert "(1.0f / " not in src("relaxed", False)
    assert "(1.0f / " in src("fast", False)
    with pytest.raises(ValueError, match="math_mode"):
        enceladus.jit(math_mode="precise")(lambda x: x)


@enceladus.jit
def _masked_add(x_ptr, y_ptr, o_ptr, n, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    m = offs < n
    tl.store(o_ptr + offs, tl.load(x_ptr + offs, mask=m) + tl.load(y_ptr + offs, mask=m), mask=m)


@enceladus.jit
def _store_then_load(x_ptr, o_ptr, n, BLOCK: tl.constexpr):
    offs = tl.program_id(0) * BLOCK + tl.arange(0, BLOCK)
    tl.store(o_ptr + offs, tl.load(x_ptr + offs, mask=offs < n), mask=offs < n)
    tl.store(o_ptr + n + offs, tl.load(x_ptr + n + offs, mask=offs < 2 * n), mask=offs < 2 * n)


def test_program_versioning():
    """A straight-line masked program gets one guarded copy without mask tests, which
    returns, ahead of the general copy; the general copy keeps only the masked paths; its
    streaming loads wait for the previous one. A guard that would follow a store is not
    taken (the general copy must start before any store), and the switch turns it off."""
    x = np.zeros(4, np.float32)
    f = _masked_add.ir_for(x, x, x, 1 << 20, BLOCK=1024)
    src = codegen_hip.generate(f).source
    fast, general = src.split("return;")
    assert fast.count("__builtin_expect(") == 1
    assert "vload_nt" in fast and " ? *" not in fast and fast.count("vstore_nt") == 1
    assert fast.count("__builtin_amdgcn_s_waitcnt(0x0F70)") == 1
    assert "__builtin_expect(" not in general and " ? *" in general
    off = codegen_hip.generate(f, {"no_program_versioning": True}).source
    assert "return;" not in off and "__builtin_expect(" not in off
    serial = codegen_hip.generate(f, {"no_serial_streams": True}).source
    assert "__builtin_amdgcn_s_waitcnt(0x0F70)" not in serial
    two = codegen_hip.generate(_store_then_load.ir_for(x, x, 1 << 20, BLOCK=1024)).source
    assert "__builtin_expect(" not in two


def _attention_source(bm, bn, nw, monkeypatch=None, **env):
    import torch

    from examples.flash_attention import attention_kernel
    bf = torch.zeros(16, dtype=torch.bfloat16)
    ck = attention_kernel.warmup(bf, bf, bf, bf, 0.088, 4096, 4096 * 128, 128, HEAD_DIM=128,
                                 BLOCK_M=bm, BLOCK_N=bn, CAUSAL=True, num_warps=nw,
                                 dot_warps=(nw, 1))
    return ck


def test_split_stages_for_a_four_wave_attention_tile(monkeypatch):
    """128x128 over 4 waves: one LDS stage each for K and V (64 KB, so two workgroups share a
    CU); V is copied under QK^T, the next K under PV, with a barrier between the dots.
    256x128 over 8 waves keeps two stages each (registers already limit it to one workgroup
    per CU), and ENCELADUS_CODEGEN=no_split_stages restores them."""
    ck = _attention_source(128, 128, 4)
    src = ck.hip
    assert ck.lds_bytes == 65536
    loop = src[src.index("for (int32_t iv"):src.index("++ek_it")]
    assert loop.count("s_barrier") == 2
    first, second = loop.split("s_barrier")[1], loop.split("s_barrier")[2]
    # the V tile of this iteration goes out under the first dot (descriptor a2 = v_ptr),
    # the K tile of the next iteration under the second (a1 = k_ptr)
    assert "rsrc_words(s8" in first and "_r0 = iv" in first
    assert "rsrc_words(s7" in second and "+ s5)" in second
    # the barrier between the dots sits after the row max and the rescale of the
    # accumulator (its skip branch is the ballot) and before the exponentials of the scores,
    # their row sum and their cast, which share one basic block with PV's MFMAs
    ex = "ek::exp2_fast(__builtin_fmaf("
    assert "ek::Max::op" in first and "__builtin_amdgcn_ballot_w64" in first
    assert ex not in first and ex in second
    assert second.index(ex) < second.index("ek::Sum::op") < second.index("ek::cvt<ek::bf16>") \
        < second.index("ek::mfma_32x32x16")
    monkeypatch.setenv("ENCELADUS_CODEGEN", "no_split_sink")
    late = _attention_source(128, 128, 4).hip
    late = late[late.index("for (int32_t iv"):late.index("++ek_it")].split("s_barrier")
    assert ex in late[1] and "ek::cvt<ek::bf16>" in late[1]
    monkeypatch.delenv("ENCELADUS_CODEGEN")
    assert _attention_source(256, 128, 8).lds_bytes == 131072
    monkeypatch.setenv("ENCELADUS_CODEGEN", "no_split_stages")
    assert _attention_source(128, 128, 4).lds_bytes == 131072


@enceladus.jit
def _attention_with_row_stats(q_ptr, k_ptr, v_ptr, o_ptr, m_ptr, sm_scale, N_CTX, stride_m,
                              HEAD_DIM: tl.constexpr, BLOCK_M: tl.constexpr,
                              BLOCK_N: tl.constexpr):
    """The attention body with a store of the running row max inside the loop."""
    start_m = tl.program_id(0)
    q_desc = tl.make_tensor_descriptor(q_ptr, [N_CTX, HEAD_DIM], [stride_m, 1],
                                       [BLOCK_M, HEAD_DIM])
    k_desc = tl.make_tensor_descriptor(k_ptr, [N_CTX, HEAD_DIM], [stride_m, 1],
                                       [BLOCK_N, HEAD_DIM])
    v_desc = tl.make_tensor_descriptor(v_ptr, [N_CTX, HEAD_DIM], [stride_m, 1],
                                       [BLOCK_N, HEAD_DIM])
    o_desc = tl.make_tensor_descriptor(o_ptr, [N_CTX, HEAD_DIM], [stride_m, 1],
                                       [BLOCK_M, HEAD_DIM])
    offs_m = start_m * BLOCK_M + tl.arange(0, BLOCK_M)
    m_i = tl.full([BLOCK_M], float("-inf"), tl.float32)
    l_i = tl.zeros([BLOCK_M], tl.float32)
    acc = tl.zeros([BLOCK_M, HEAD_DIM], tl.float32)
    q = q_desc.load([start_m * BLOCK_M, 0])
    for start_n in range(0, N_CTX, BLOCK_N):
        qk = tl.dot(q, tl.trans(k_desc.load([start_n, 0]))) * sm_scale
        m_ij = tl.maximum(m_i, tl.max(qk, 1))
        tl.store(m_ptr + offs_m, m_ij)
        p = tl.exp2(qk - m_ij[:, None])
        alpha = tl.exp2(m_i - m_ij)
        l_i = l_i * alpha + tl.sum(p, 1)
        acc = acc * alpha[:, None]
        acc = tl.dot(p.to(q_desc.dtype), v_desc.load([start_n, 0]), acc)
        m_i = m_ij
    o_desc.store([start_m * BLOCK_M, 0], (acc / l_i[:, None]).to(o_desc.dtype))


def test_split_sink_keeps_source_order_around_a_store():
    """An op with a side effect between the two dots (here a store of the row max) leaves
    the split-stage loop in source order: the exponentials stay before the barrier."""
    import torch
    bf = torch.zeros(16, dtype=torch.bfloat16)
    f32 = np.zeros(16, np.float32)
    src = codegen_hip.generate(_attention_with_row_stats.ir_for(
        bf, bf, bf, bf, f32, 0.088, 4096, 128, HEAD_DIM=128, BLOCK_M=128, BLOCK_N=128,
        num_warps=4, dot_warps=(4, 1))).source
    loop = src[src.index("for (int32_t iv"):src.index("++ek_it")]
    parts = loop.split("s_barrier")
    assert len(parts) == 3, "expected the split-stage loop (two barriers)"
    assert "ek::exp2_fast(__builtin_fmaf(" in parts[1] and "ek::cvt<ek::bf16>" in parts[1]
    assert "ek::exp2_fast(" not in parts[2]
