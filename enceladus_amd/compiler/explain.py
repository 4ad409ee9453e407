"""`kernel.explain`: a readable report of the compiler's decisions for one specialization
(reference: compiler/explain.py:88-172): the MFMA plan of every `tl.dot`, the layout of the
tiles the emitter anchors, every layout conversion through LDS with its source line and
size, the LDS each operation uses, and the registers of the built code object."""

from __future__ import annotations

import linecache
import os

from enceladus_amd.compiler import ir
from enceladus_amd.compiler import layout as LY


def describe_layout(lay: LY.Layout) -> str:
    """How a layout spreads a tile, per dimension: `regs 1x4, lanes 4x16, waves 4x1` means
    each thread holds 4 elements along dim 1, a wave's 64 lanes cover a 4 x 16 block of
    those, and 4 waves stack along dim 0."""
    rank = len(lay.shape)

    def split(bits):
        counts, zeros = [1] * rank, 0
        for b in bits:
            if b is None:
                zeros += 1
            else:
                counts[b[0]] *= 2
        return counts, zeros

    x = lambda c: "x".join(map(str, c)) if c else "1"  # noqa: E731
    reg, _ = split(lay.reg)
    lane, lz = split(lay.lane)
    warp, wz = split(lay.warp)
    kind = "MFMA fragments" if lay.kind != "blocked" else "blocked"
    out = f"{kind}: regs {x(reg)}, lanes {x(lane)}, waves {x(warp)}"
    if lz or wz:
        out += f", each element held by {1 << (lz + wz)} threads"
    return out


def _where(loc) -> str:
    return f"{os.path.basename(loc[0])}:{loc[1]}" if loc else "?"


def _source(loc) -> str:
    if not loc:
        return ""
    text = linecache.getline(loc[0], loc[1]).strip()
    return f"  `{text}`" if text else ""


def _type(v: ir.Value) -> str:
    t = v.type
    name = f"*{t.dtype.name}" if t.ptr else t.dtype.name
    return f"{name}[{', '.join(map(str, t.shape))}]" if t.shape else name


def explain(ck, grid=None) -> str:
    """The report for compiled kernel `ck` (a `CompiledKernel`)."""
    gen = ck.gen
    rep = gen.report or {}
    out = []
    add = out.append
    head = f"Kernel `{gen.name}`: num_warps={gen.num_warps} ({gen.num_warps * 64} threads " \
           "per program, wave64)"
    if grid is not None:
        head += f", grid {tuple(grid)}"
    add(head)
    extras = []
    if gen.asserts:
        extras.append(f"{len(gen.asserts)} device asserts")
    if gen.coarsen:
        extras.append(f"coarsened to {gen.coarsen} workgroups per CU")
    if gen.flush:
        extras.append(f"privatised bins flushed by `{gen.flush['name']}`")
    add("gfx950 (CDNA4), hiprtc" + (f" ({', '.join(extras)})" if extras else ""))
    try:
        a = ck.attrs
        add(f"Registers: {a['num_regs']} per thread, {a['local_bytes']} bytes of spills")
    except Exception:  # noqa: BLE001 - the attributes need a loaded code object (a GPU)
        pass

    dots = rep.get("dots", [])
    if not dots and not rep.get("gemm_template"):
        add("dot backend: none (the kernel has no tl.dot)")
    else:
        add("dot backend: CDNA4 MFMA")
        if rep.get("gemm_template"):
            loc = rep["gemm_template"]
            add(f"  {_where(loc)}  the K loop runs as the GEMM template (LDS DMA stages, "
                f"double-buffered){_source(loc)}")
        for d in dots:
            p = d["plan"]
            staged = f", {' and '.join(d['staged'])} staged through LDS" if d["staged"] else ""
            add(f"  {_where(d['loc'])}  {p.bm}x{p.bn}x{p.bk} (MxNxK), wave grid {p.wm}x{p.wn}, "
                f"MFMA {p.inst.m}x{p.inst.n}x{p.inst.k} (ek::{p.inst.fn}){staged}{_source(d['loc'])}")

    add("")
    add("Layout conversions:")
    convs = rep.get("conversions", [])
    if not convs:
        add("  (none)")
    for c in convs:
        v = c["value"]
        name = f" `{v.name_hint}`" if getattr(v, "name_hint", None) else ""
        add(f"  {_where(c['loc'])}  {_type(v)}{name}: LDS exchange, {c['bytes']} bytes, "
            f"2 barriers{_source(c['loc'])}")
        add(f"      from {describe_layout(c['src'])}")
        add(f"      to   {describe_layout(c['dst'])}")

    add("")
    add(f"LDS: {gen.lds_bytes} bytes of 163840 (one arena that each operation reuses; LDS "
        "stages and privatised bins have their own)")
    seen = set()
    for u in rep.get("lds", []):
        key = (u["loc"], u["op"], u["bytes"])
        if key in seen:
            continue
        seen.add(key)
        add(f"  {_where(u['loc'])}  {u['op']}: {u['bytes']} bytes{_source(u['loc'])}")
    return "\n".join(out)
