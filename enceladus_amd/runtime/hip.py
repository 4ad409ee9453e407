"""ctypes binding of the C-ABI shim `libenceladus_hip.so` (declared in include/enceladus_hip.h).

Loading order matters: PyTorch-ROCm ships its own HIP runtime with the same soname as the
system one. So that device pointers from torch tensors and from this runtime live in one
HIP runtime, the shim's `libamdhip64.so.7` dependency is satisfied by torch's copy when
torch is installed (loaded first, by path, with RTLD_GLOBAL; a later `import torch`
reuses the same file). hiprtc is the system ROCm one (a self-contained compiler).

There is no CPU fallback: if the shim or a GPU is missing, every entry point raises.
Reference: the nanobind module over the Metal C ABI, src/enceladus/_C/bindings.mm:340-649.
"""

from __future__ import annotations

import ctypes
import importlib.util
import os
import threading
from pathlib import Path

from enceladus_amd.compiler.errors import HipError

_HERE = Path(__file__).resolve().parent.parent / "csrc"
LIB_PATH = _HERE / "libenceladus_hip.so"
INCLUDE_DIR = _HERE / "include"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ERR_LEN = 65536

_lock = threading.Lock()
_lib = None


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64),
                ("compute_units", ctypes.c_int32), ("warp_size", ctypes.c_int32),
                ("max_threads_per_block", ctypes.c_int32), ("lds_per_block", ctypes.c_int64),
                ("total_mem", ctypes.c_int64), ("clock_khz", ctypes.c_int32),
                ("mem_clock_khz", ctypes.c_int32), ("mem_bus_width", ctypes.c_int32),
                ("l2_bytes", ctypes.c_int32)]


class FunctionAttrs(ctypes.Structure):
    _fields_ = [("num_regs", ctypes.c_int32), ("shared_bytes", ctypes.c_int32),
                ("local_bytes", ctypes.c_int32), ("max_threads", ctypes.c_int32)]


def _torch_lib_dir() -> Path | None:
    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.origin:
        return None
    d = Path(spec.origin).parent / "lib"
    return d if (d / "libamdhip64.so").exists() else None


def runtime_library() -> Path:
    """The libamdhip64 this process uses: torch's bundled copy if present, else ROCm's."""
    d = _torch_lib_dir()
    if d is not None:
        return d / "libamdhip64.so"
    return ROCM / "lib" / "libamdhip64.so"


_SIGS = {
    "ek_device_count": [ctypes.POINTER(ctypes.c_int)],
    "ek_device_get_info": [ctypes.c_int, ctypes.POINTER(DeviceInfo)],
    "ek_set_device": [ctypes.c_int],
    "ek_module_load": [ctypes.c_void_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_void_p)],
    "ek_module_unload": [ctypes.c_void_p],
    "ek_module_function": [ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p)],
    "ek_function_get_attrs": [ctypes.c_void_p, ctypes.POINTER(FunctionAttrs)],
    "ek_launch": [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_uint32] * 7 +
                 [ctypes.c_void_p, ctypes.c_size_t],
    "ek_stream_new": [ctypes.POINTER(ctypes.c_void_p)],
    "ek_stream_free": [ctypes.c_void_p],
    "ek_stream_sync": [ctypes.c_void_p],
    "ek_device_sync": [],
    "ek_malloc": [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t],
    "ek_free": [ctypes.c_void_p],
    "ek_memcpy_h2d": [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
    "ek_memcpy_d2h": [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
    "ek_memcpy_d2d": [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p],
    "ek_memset": [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p],
    "ek_event_new": [ctypes.POINTER(ctypes.c_void_p)],
    "ek_event_free": [ctypes.c_void_p],
    "ek_event_record": [ctypes.c_void_p, ctypes.c_void_p],
    "ek_event_elapsed_ms": [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_float)],
    "ek_timed_launch": [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_uint32] * 7 +
                       [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                        ctypes.POINTER(ctypes.c_float)],
    "ek_launch_timed_events": [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_uint32] * 7 +
                              [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                               ctypes.c_void_p],
    "ek_launch_flush_noalloc": [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_uint32] * 4 +
                               [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
                                ctypes.c_void_p] + [ctypes.c_uint32] * 3 +
                               [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
                                ctypes.c_size_t],
}

# The size of the no-allocation launch's static scratch array (EK_SCRATCH_BYTES).
SCRATCH_BYTES = 16 << 20

EXPORTED = sorted([*_SIGS, "ek_compile", "ek_buffer_free", "ek_version", "ek_runtime_version"])


def load_library():
    """Loads the shim (once). Raises HipError if it isn't built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise HipError(f"{LIB_PATH} is not built; run `python -m enceladus_amd.csrc.build` "
                           "(or __graft_entry__.build())")
        mode = ctypes.RTLD_GLOBAL
        ctypes.CDLL(str(runtime_library()), mode=mode)
        ctypes.CDLL(str(ROCM / "lib" / "libhiprtc.so.7"), mode=mode)
        lib = ctypes.CDLL(str(LIB_PATH), mode=mode)
        for name, args in _SIGS.items():
            f = getattr(lib, name)
            f.argtypes = [*args, ctypes.c_char_p, ctypes.c_size_t]
            f.restype = ctypes.c_int
        lib.ek_compile.argtypes = [ctypes.c_char_p, ctypes.c_char_p,
                                   ctypes.POINTER(ctypes.c_char_p), ctypes.c_int,
                                   ctypes.POINTER(ctypes.c_void_p),
                                   ctypes.POINTER(ctypes.c_size_t), ctypes.c_char_p,
                                   ctypes.c_size_t]
        lib.ek_compile.restype = ctypes.c_int
        lib.ek_buffer_free.argtypes = [ctypes.c_void_p]
        lib.ek_buffer_free.restype = None
        lib.ek_version.restype = ctypes.c_char_p
        lib.ek_runtime_version.argtypes = [ctypes.POINTER(ctypes.c_int)]
        _lib = lib
        return lib


def call(name: str, *args):
    """Calls shim function `name`, raising HipError with the shim's message on failure."""
    lib = load_library()
    err = ctypes.create_string_buffer(1024)
    rc = getattr(lib, name)(*args, err, 1024)
    if rc != 0:
        raise HipError(f"{name}: {err.value.decode(errors='replace')}")


def compile_source(src: str, name: str, options: list[str]) -> tuple[bytes, str]:
    """Compiles HIP C++ `src` with hiprtc; returns (code object bytes, compiler log)."""
    lib = load_library()
    opts = (ctypes.c_char_p * len(options))(*[o.encode() for o in options])
    code = ctypes.c_void_p()
    size = ctypes.c_size_t()
    log = ctypes.create_string_buffer(ERR_LEN)
    rc = lib.ek_compile(src.encode(), name.encode(), opts, len(options), ctypes.byref(code),
                        ctypes.byref(size), log, ERR_LEN)
    text = log.value.decode(errors="replace")
    if rc != 0:
        raise HipError(f"hiprtc failed to compile {name}:\n{text}")
    try:
        data = ctypes.string_at(code, size.value)
    finally:
        lib.ek_buffer_free(code)
    return data, text


def device_count() -> int:
    n = ctypes.c_int(0)
    try:
        call("ek_device_count", ctypes.byref(n))
    except HipError:
        return 0
    return n.value


def device_info(dev: int = 0) -> DeviceInfo:
    info = DeviceInfo()
    call("ek_device_get_info", dev, ctypes.byref(info))
    return info
