"""Specialization → code object, with an in-memory and on-disk cache.

`compile_specialization` builds IR, runs the HIP emitter, compiles with hiprtc for gfx950
and caches the code object under `$ENCELADUS_CACHE_DIR` (default
`~/.cache/enceladus_amd`), keyed by the generated source, the compile options, the device
header and the shim and HIP runtime versions. Reference: src/enceladus/runtime/compile.py:38-164 and cache.py:26-144
(disk cache of compiled kernels, corrupt entries recompiled).

Environment variables (reference: src/enceladus/runtime/compile.py:6-10):
    ENCELADUS_ALWAYS_COMPILE=1: ignore the disk cache.
    ENCELADUS_DUMP=1: write the IR and HIP source of each new specialization next to the
        cache and print their paths.
    ENCELADUS_OVERRIDE_DIR: compile `<dir>/<kernel_name>.hip` instead of the generated
        source when that file exists (it must define the same `ek_<kernel_name>` symbol
        and take the same arguments).
"""

from __future__ import annotations

import ctypes
import hashlib
import logging
import os
import sys
import threading
from pathlib import Path

from enceladus_amd.compiler import codegen_hip, frontend, ir, rewrite, simplify, verify, widen
from enceladus_amd.runtime import hip

log = logging.getLogger("enceladus")

ARCH = os.environ.get("ENCELADUS_ARCH", "gfx950")
BASE_OPTIONS = ["-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
                "-packed-fp32-ops", "-fno-gpu-rdc", "-mcumode"]

_mem_cache: dict[str, bytes] = {}
_lock = threading.Lock()


def cache_dir() -> Path:
    d = os.environ.get("ENCELADUS_CACHE_DIR")
    return Path(d) if d else Path.home() / ".cache" / "enceladus_amd"


def _header_hash() -> str:
    """The device header, the shim's version and the HIP runtime's (hiprtc ships with it):
    a code object compiled under another of them is not reused."""
    h = hashlib.sha256()
    h.update((hip.INCLUDE_DIR / "enceladus_cdna4.h").read_bytes())
    try:
        lib = hip.load_library()
        v = ctypes.c_int(0)
        lib.ek_runtime_version(ctypes.byref(v))
        h.update(f"{lib.ek_version().decode()}|{v.value}".encode())
    except Exception:  # noqa: BLE001 - the shim is missing: compiling fails loudly later
        pass
    return h.hexdigest()[:16]


_HDR = None


def compile_options(extra=()) -> list[str]:
    return [f"--offload-arch={ARCH}", *BASE_OPTIONS, f"-I{hip.INCLUDE_DIR}", *extra]


def compile_code(src: str, name: str, extra=()) -> bytes:
    """hiprtc-compiles `src` (cached by source hash)."""
    global _HDR
    if _HDR is None:
        _HDR = _header_hash()
    opts = compile_options(extra)
    key = hashlib.sha256("\0".join([src, name, _HDR, *opts]).encode()).hexdigest()
    with _lock:
        hit = _mem_cache.get(key)
    if hit is not None:
        return hit
    always = os.environ.get("ENCELADUS_ALWAYS_COMPILE") == "1"
    path = cache_dir() / key[:2] / f"{key}.hsaco"
    if not always and path.exists():
        data = path.read_bytes()
        if data[:4] == b"\x7fELF":
            with _lock:
                _mem_cache[key] = data
            return data
        log.debug("corrupt cache entry %s; recompiling", path)
    data, text = hip.compile_source(src, f"{name}.hip", opts)
    if text.strip():
        log.debug("hiprtc log for %s:\n%s", name, text)
    try:
        path.parent.mkdir(parents=True, exist_ok=True)
        tmp = path.with_suffix(f".tmp{os.getpid()}")
        tmp.write_bytes(data)
        os.replace(tmp, path)
    except OSError:
        pass
    with _lock:
        _mem_cache[key] = data
    return data


class CompiledKernel:
    """A compiled specialization: source, IR text, code object and (lazily) its function."""

    def __init__(self, gen: codegen_hip.GeneratedKernel, ir_text: str, code: bytes):
        self.gen = gen
        self.name = gen.name
        self.hip = gen.source
        self.msl = gen.source        # the reference's attribute name, kept for drop-in code
        self.ir = ir_text
        self.code = code
        self.num_warps = gen.num_warps
        self.threadgroup_memory_bytes = gen.lds_bytes
        self.lds_bytes = gen.lds_bytes
        self.args = gen.args
        self._module = None
        self._function = None
        self._attrs = None

    def function(self):
        if self._function is None:
            if "ek::mfma_" in self.hip or "ek::Gemm" in self.hip:
                # before the first MFMA kernel of the process runs: the device's MFMA lane
                # maps are the ones the emitter assumes (reference: compile.py:159-160)
                from enceladus_amd.runtime.probe import check_mfma_layout
                check_mfma_layout()
            m = ctypes.c_void_p()
            buf = ctypes.create_string_buffer(self.code, len(self.code))
            hip.call("ek_module_load", buf, len(self.code), ctypes.byref(m))
            f = ctypes.c_void_p()
            hip.call("ek_module_function", m, self.name.encode(), ctypes.byref(f))
            self._module, self._function = m, f
        return self._function

    @property
    def attrs(self) -> dict:
        if self._attrs is None:
            a = hip.FunctionAttrs()
            hip.call("ek_function_get_attrs", self.function(), ctypes.byref(a))
            self._attrs = {"num_regs": a.num_regs, "shared_bytes": a.shared_bytes,
                           "local_bytes": a.local_bytes, "max_threads": a.max_threads}
        return self._attrs

    def pack(self, values) -> bytes:
        values = list(values)
        if self.gen.flush:
            values.append(0)      # the partial-bin buffer, set per stream at launch
        b = codegen_hip.pack_args(self.args, values, pad8=not self.gen.coarsen)
        self.packed_size = len(b)
        return b

    def _flush_function(self):
        if getattr(self, "_flush_fn", None) is None:
            self.function()
            f = ctypes.c_void_p()
            hip.call("ek_module_function", self._module, self.gen.flush["name"].encode(),
                     ctypes.byref(f))
            self._flush_fn = f
        return self._flush_fn

    def _partials(self, stream: int, nwg: int) -> int:
        """The partial-bin buffer for launches on `stream` (kept for the kernel's life;
        launches of one specialization on one stream run in order, so they can share it)."""
        bufs = self.__dict__.setdefault("_part_bufs", {})
        need = max(16, nwg * self.gen.flush["total"] * 4)
        cur = bufs.get(stream)
        if cur is None or cur[1] < need:
            from enceladus_amd.runtime import tensor as T
            from enceladus_amd.language import core as _core
            t = T.Tensor((need,), _core.uint8)
            bufs[stream] = (t, need)
            cur = bufs[stream]
        return cur[0].ptr

    def prepare(self, grid, kernarg: bytes, stream: int = 0) -> list:
        """The dispatches of one logical launch: [(function, (gx, gy, gz), block, kernarg
        buffer, size)]: the kernel itself, then the second flush level when it has one."""
        gx, gy, gz = (tuple(grid) + (1, 1, 1))[:3]
        if gx == 0 or gy == 0 or gz == 0:
            return []
        (gx, gy, gz), extra = self.launch_grid(grid)
        if extra:
            kernarg = kernarg[:self.packed_size] + extra
            kernarg += b"\0" * ((-len(kernarg)) % 8)
        out = []
        fl = self.gen.flush
        if fl:
            import struct
            offs = codegen_hip.arg_offsets(self.args)
            part = self._partials(stream, gx)
            kb = bytearray(kernarg)
            struct.pack_into("<Q", kb, offs[-1], part)
            kernarg = bytes(kb)
            bases = [struct.unpack_from("<Q", kernarg, offs[i])[0] for i in fl["bases"]]
            fargs = [codegen_hip.KernelArg("p", "ptr", None, "int32_t*"),
                     codegen_hip.KernelArg("n", "scalar", None, "int32_t")] + \
                [codegen_hip.KernelArg("h", "ptr", None, "int32_t*") for _ in bases]
            fk = codegen_hip.pack_args(fargs, [part, gx, *bases])
        buf = ctypes.create_string_buffer(kernarg, len(kernarg))
        out.append((self.function(), (gx, gy, gz), self.gen.block, buf, len(kernarg)))
        if fl:
            fbuf = ctypes.create_string_buffer(fk, len(fk))
            out.append((self._flush_function(), (fl["chunks"], (gx + fl["rb"] - 1) // fl["rb"], 1), 256,
                        fbuf, len(fk)))
        return out

    def launch_noalloc(self, grid, kernarg: bytes, stream: int = 0):
        """One logical launch of a kernel with a two-level flush through
        `ek_launch_flush_noalloc`: the partial rows live in the library's static scratch
        array, so nothing is allocated (for callers that cannot allocate). Raises HipError
        when the launch needs more scratch than the array holds."""
        import struct
        fl = self.gen.flush
        if not fl:
            raise ValueError(f"{self.name} has no scratch buffer; launch it normally")
        gx, gy, gz = (tuple(grid) + (1, 1, 1))[:3]
        if gx == 0 or gy == 0 or gz == 0:
            return
        (gx, gy, gz), extra = self.launch_grid(grid)
        if extra:
            kernarg = kernarg[:self.packed_size] + extra
            kernarg += b"\0" * ((-len(kernarg)) % 8)
        offs = codegen_hip.arg_offsets(self.args)
        bases = [struct.unpack_from("<Q", kernarg, offs[i])[0] for i in fl["bases"]]
        fargs = [codegen_hip.KernelArg("p", "ptr", None, "int32_t*"),
                 codegen_hip.KernelArg("n", "scalar", None, "int32_t")] + \
            [codegen_hip.KernelArg("h", "ptr", None, "int32_t*") for _ in bases]
        fk = codegen_hip.pack_args(fargs, [0, gx, *bases])
        kb = ctypes.create_string_buffer(kernarg, len(kernarg))
        fb = ctypes.create_string_buffer(fk, len(fk))
        hip.call("ek_launch_flush_noalloc", ctypes.c_void_p(stream or None), self.function(),
                 gx, gy, gz, self.gen.block, kb, len(kernarg), offs[-1],
                 self._flush_function(), fl["chunks"], (gx + fl["rb"] - 1) // fl["rb"], 256,
                 fb, len(fk), 0, gx * fl["total"] * 4)

    def launch_grid(self, grid):
        """(launch grid, extra kernarg bytes) for a logical program grid."""
        gx, gy, gz = (tuple(grid) + (1, 1, 1))[:3]
        if not self.gen.coarsen:
            return (gx, gy, gz), b""
        total = gx * gy * gz
        cap = max(1, coarsen_cap() * self.gen.coarsen)
        import struct
        return (min(total, cap), 1, 1), struct.pack("<iii", gx, gy, gz)

    def launch_raw(self, grid, kernarg: bytes, stream: int = 0):
        from enceladus_amd.runtime import debug, timing
        timer = timing.current()
        for fn_, g_, blk, buf, n in self.prepare(grid, kernarg, stream):
            t0 = debug.before_launch(stream) if debug._active is not None else None
            if timer is not None:
                timer.launch(stream, fn_, g_, blk, buf, n)
            else:
                hip.call("ek_launch", ctypes.c_void_p(stream or None), fn_, g_[0], g_[1],
                         g_[2], blk, 1, 1, 0, buf, n)
            if t0 is not None:
                nm = self.name if fn_ is self._function else self.gen.flush["name"]
                debug.after_launch(t0, stream, nm, g_, blk,
                                   self.gen.lds_bytes if fn_ is self._function else 0)


_CAP = None


def coarsen_cap() -> int:
    """Compute units of GPU 0: a coarsened kernel launches `gen.coarsen` workgroups per CU."""
    global _CAP
    if _CAP is None:
        try:
            _CAP = hip.device_info(0).compute_units
        except Exception:  # noqa: BLE001
            _CAP = 256
    return _CAP


def compile_ir(fn: ir.Func, options: dict | None = None) -> CompiledKernel:
    gen = codegen_hip.generate(fn, options)
    ir_text = ir.print_func(fn)
    override = os.environ.get("ENCELADUS_OVERRIDE_DIR")
    if override:
        p = Path(override) / f"{fn.name}.hip"
        if p.exists():
            gen.source = p.read_text()
            log.warning("enceladus: %s: compiling %s instead of the generated source", fn.name, p)
    if os.environ.get("ENCELADUS_DUMP", "0") not in ("", "0"):
        tag = hashlib.sha256(gen.source.encode()).hexdigest()[:12]
        d = cache_dir() / "dump"
        d.mkdir(parents=True, exist_ok=True)
        (d / f"{fn.name}-{tag}.hip").write_text(gen.source)
        (d / f"{fn.name}-{tag}.ir").write_text(ir_text)
        print(f"enceladus: {fn.name}: IR and HIP source in {d}/{fn.name}-{tag}.{{ir,hip}}",
              file=sys.stderr)
    code = compile_code(gen.source, gen.name)
    return CompiledKernel(gen, ir_text, code)


def build_module(jfn, arg_types, arg_facts, constexprs, num_warps, options) -> ir.Func:
    """Frontend, then the IR passes in order (reference: compiler/pipeline.py:14-38); with
    ENCELADUS_VERIFY=1 the IR is verified after each stage."""
    fn = frontend.build_ir(jfn.fn, arg_types, arg_facts, constexprs, num_warps, options)
    verify.maybe_verify(fn, "the frontend")
    if not (options or {}).get("no_simplify"):
        simplify.simplify(fn)
        verify.maybe_verify(fn, "the simplifier")
    if widen.needs_idx64(fn):
        widen.widen_index_math(fn)
        verify.maybe_verify(fn, "64-bit index widening")
    if not (options or {}).get("no_scale_fold"):
        rewrite.fold_softmax_scale(fn)
        verify.maybe_verify(fn, "the attention scale rewrite")
    ir.dce(fn)
    verify.maybe_verify(fn, "dead-code elimination")
    return fn
