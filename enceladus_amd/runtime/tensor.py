"""Device tensors in HBM and array interop (NumPy, torch-ROCm, and our own `Tensor`).

Reference: `Tensor` and the array adapters (src/enceladus/runtime/tensor.py:65-363,
runtime/interop.py:38-62, 161, 323-420, 577). On MI355X a NumPy argument is copied into
HBM for the launch and copied back afterwards if the kernel writes it; a torch tensor on
the GPU or a `Tensor` is passed by device pointer with no copy.
"""

from __future__ import annotations

import ctypes
import sys
from typing import Any

import numpy as np

from enceladus_amd.language import core
from enceladus_amd.runtime import hip


class _Allocation:
    """One device allocation in HBM; freed when the last tensor viewing it goes away."""

    def __init__(self, nbytes: int):
        p = ctypes.c_void_p()
        hip.call("ek_malloc", ctypes.byref(p), max(int(nbytes), 16))
        self.ptr = p.value or 0
        self.nbytes = int(nbytes)

    def __del__(self):
        if getattr(self, "ptr", 0):
            try:
                hip.call("ek_free", ctypes.c_void_p(self.ptr))
            except Exception:  # noqa: BLE001
                pass
            self.ptr = 0


class _Ptr(int):
    """An address that reads both ways: `t.data_ptr` (the reference's property) and
    `t.data_ptr()` (torch's method)."""

    def __call__(self) -> int:
        return int(self)


def _contiguous(shape) -> tuple:
    st, s = [], 1
    for d in reversed(shape):
        st.append(s)
        s *= d
    return tuple(reversed(st))


class Tensor:
    """A device array in HBM: an allocation plus shape, element strides and an element
    offset, so that basic slicing gives views that share the allocation (reference:
    runtime/tensor.py:65-233). Host access copies: `numpy()` reads the elements back,
    `copy_()` writes them."""

    def __init__(self, shape, dtype: core.dtype, strides=None, offset: int = 0,
                 buffer: _Allocation | None = None):
        if hasattr(shape, "ptr") and hasattr(shape, "nbytes"):
            # the reference's order: Tensor(buffer, shape, dtype, strides=None, offset=0)
            shape, dtype, strides, offset, buffer = dtype, strides, offset or None, \
                buffer or 0, shape
        self.shape = tuple(int(s) for s in shape)
        self.dtype = _as_dtype(dtype)
        self.strides = tuple(int(x) for x in strides) if strides is not None else \
            _contiguous(self.shape)
        self.offset = int(offset)
        self.buffer = buffer if buffer is not None else \
            _Allocation(self.numel * self.dtype.itemsize)

    # ---- metadata ----
    @property
    def ndim(self) -> int:
        return len(self.shape)

    @property
    def numel(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    @property
    def itemsize(self) -> int:
        return self.dtype.itemsize

    @property
    def nbytes(self) -> int:
        return self.numel * self.itemsize

    @property
    def byte_offset(self) -> int:
        return self.offset * self.itemsize

    @property
    def ptr(self) -> int:
        """The device address of the first element."""
        return self.buffer.ptr + self.byte_offset

    @property
    def data_ptr(self) -> _Ptr:
        return _Ptr(self.ptr)

    def stride(self, dim: int | None = None):
        """The stride of dimension `dim` in elements (all strides when `dim` is None)."""
        return self.strides if dim is None else self.strides[dim]

    def size(self, dim: int | None = None):
        return self.shape if dim is None else self.shape[dim]

    def is_contiguous(self) -> bool:
        return self.strides == _contiguous(self.shape)

    def __len__(self) -> int:
        return self.shape[0]

    # ---- host access ----
    def _span(self) -> int:
        """Elements from the first to one past the last (strides are non-negative)."""
        if self.numel == 0:
            return 0
        return 1 + sum((n - 1) * st for n, st in zip(self.shape, self.strides))

    def _host_window(self, span: int) -> np.ndarray:
        w = np.empty(span, self.dtype.to_numpy())
        if span:
            from enceladus_amd.runtime import device
            device.synchronize()
            hip.call("ek_memcpy_d2h", w.ctypes.data_as(ctypes.c_void_p),
                     ctypes.c_void_p(self.ptr), span * self.itemsize, None)
        return w

    def _as_view(self, w: np.ndarray) -> np.ndarray:
        return np.lib.stride_tricks.as_strided(
            w, self.shape, [st * self.itemsize for st in self.strides])

    def numpy(self) -> np.ndarray:
        """Finishes pending GPU work and returns a host copy of the elements."""
        if self.is_contiguous():
            return self._host_window(self.numel).reshape(self.shape)
        return np.array(self._as_view(self._host_window(self._span())))

    def __array__(self, dtype=None, copy=None):
        a = self.numpy()
        return a.astype(dtype, copy=False) if dtype is not None else a

    def tolist(self) -> list:
        return self.numpy().tolist()

    def copy_from_numpy(self, a: np.ndarray) -> "Tensor":
        a = np.asarray(a, self.dtype.to_numpy())
        if a.shape != self.shape and a.size != self.numel:
            raise ValueError(f"size mismatch: {a.shape} into {self.shape}")
        if not self.numel:
            return self
        if self.is_contiguous():
            a = np.ascontiguousarray(a).reshape(-1)
            hip.call("ek_memcpy_h2d", ctypes.c_void_p(self.ptr),
                     a.ctypes.data_as(ctypes.c_void_p), self.nbytes, None)
            hip.call("ek_device_sync")
            return self
        # a strided view: read its window, write the elements, write the window back
        w = self._host_window(self._span())
        self._as_view(w)[...] = a.reshape(self.shape)
        hip.call("ek_memcpy_h2d", ctypes.c_void_p(self.ptr), w.ctypes.data_as(ctypes.c_void_p),
                 w.nbytes, None)
        hip.call("ek_device_sync")
        return self

    def copy_(self, src: Any) -> "Tensor":
        """Copies `src` (array-like, broadcast to this shape) into the tensor."""
        return self.copy_from_numpy(np.broadcast_to(
            np.asarray(src, self.dtype.to_numpy()), self.shape))

    def __getitem__(self, key) -> "Tensor":
        """A view sharing this tensor's allocation; basic slicing with positive steps."""
        es = self.itemsize
        probe = np.lib.stride_tricks.as_strided(
            np.zeros(1, self.dtype.to_numpy()), self.shape, [st * es for st in self.strides],
            writeable=False)
        v = probe[key]
        if not isinstance(v, np.ndarray) or (v.base is None and v.size):
            raise TypeError("Tensor indexing supports only slices that give a view; use "
                            ".numpy() to read single elements")
        if v.size == 0:
            return Tensor(v.shape, self.dtype, None, self.offset, self.buffer)
        if any(x < 0 for x in v.strides):
            raise ValueError("Tensor indexing doesn't support negative strides; index with "
                             "a positive step")
        off = (v.__array_interface__["data"][0] - probe.__array_interface__["data"][0]) // es
        return Tensor(v.shape, self.dtype, tuple(x // es for x in v.strides),
                      self.offset + off, self.buffer)

    def __repr__(self):
        return f"Tensor(shape={self.shape}, dtype={self.dtype})"

    # ---- DLPack (reference: runtime/tensor.py:159-194, kDLMetal there) ----

    def __dlpack_device__(self) -> tuple[int, int]:
        """`(kDLROCM, 0)`: the tensor lives in HBM of GPU 0."""
        from enceladus_amd.runtime.dlpack import K_DL_ROCM
        return (K_DL_ROCM, 0)

    def __dlpack__(self, *, stream: Any = None, max_version: tuple[int, int] | None = None,
                   dl_device: tuple[int, int] | None = None, copy: bool | None = None):
        """Exports the tensor as a kDLROCM DLPack capsule without copying. Pending GPU
        work is finished first (the consumer's `stream` is then free to read it).

        Raises:
            BufferError: the consumer asked for a copy or for another device.
        """
        from enceladus_amd.runtime import dlpack
        del stream
        if copy:
            raise BufferError("enceladus.Tensor exports without copying; copy=True isn't supported")
        if dl_device is not None and tuple(dl_device) != (dlpack.K_DL_ROCM, 0):
            raise BufferError(f"enceladus.Tensor lives on (kDLROCM, 0), not {tuple(dl_device)}")
        hip.call("ek_device_sync")
        versioned = max_version is not None and max_version[0] >= 1
        return dlpack.export(self, self.ptr, self.shape, self.strides, self.dtype.name,
                             versioned=versioned)


def _shape_arg(shape) -> tuple:
    if len(shape) == 1 and not isinstance(shape[0], (int, np.integer)):
        shape = tuple(shape[0])
    return tuple(int(s) for s in shape)


def empty(shape, dtype="float32") -> Tensor:
    if isinstance(shape, int):
        shape = (shape,)
    return Tensor(shape, _as_dtype(dtype))


def full(shape, value, dtype="float32") -> Tensor:
    """A tensor filled with `value` (reference: runtime/tensor.py:290-302)."""
    if isinstance(shape, int):
        shape = (shape,)
    dt = _as_dtype(dtype)
    return from_numpy(np.full(tuple(shape), value, dt.to_numpy()), dtype=dt)


def ones(shape, dtype="float32") -> Tensor:
    return full(shape, 1, dtype)


def rand(*shape, dtype="float32", seed: int | None = None) -> Tensor:
    """Samples from the uniform distribution on [0, 1) (reference: tensor.py:316-321)."""
    shape = _shape_arg(shape)
    v = np.random.default_rng(seed).random(shape, dtype=np.float32)
    return from_numpy(v.astype(_as_dtype(dtype).to_numpy()), dtype=dtype)


def arange(start: int, end: int | None = None, step: int = 1, dtype="int32") -> Tensor:
    if end is None:
        start, end = 0, start
    dt = _as_dtype(dtype)
    return from_numpy(np.arange(start, end, step).astype(dt.to_numpy()), dtype=dt)


def empty_like(t: Any, dtype=None) -> Tensor:
    return empty(tuple(t.shape), dtype if dtype is not None else elem_dtype(t))


def zeros_like(t: Any, dtype=None) -> Tensor:
    return zeros(tuple(t.shape), dtype if dtype is not None else elem_dtype(t))


def zeros(shape, dtype="float32") -> Tensor:
    t = empty(shape, dtype)
    if t.nbytes:
        hip.call("ek_memset", ctypes.c_void_p(t.ptr), 0, t.nbytes, None)
        hip.call("ek_device_sync")
    return t


def from_numpy(a: np.ndarray, *, dtype=None) -> Tensor:
    """A device tensor holding a copy of `a` (HBM is not host-visible, so it never aliases
    `a`); `dtype` reinterprets the elements' storage, e.g. uint16 data as bfloat16."""
    dt = _as_dtype(dtype) if dtype is not None else core.dtype_from_numpy(a.dtype)
    t = Tensor(a.shape, dt)
    return t.copy_from_numpy(a)


def randn(*shape, dtype="float32", seed: int | None = None) -> Tensor:
    """Samples from the standard normal distribution (reference: tensor.py:308-313)."""
    rng = np.random.default_rng(seed)
    return from_numpy(rng.standard_normal(_shape_arg(shape), dtype=np.float32).astype(
        _as_dtype(dtype).to_numpy()), dtype=dtype)


def _as_dtype(dt) -> core.dtype:
    if isinstance(dt, core.dtype):
        return dt
    if isinstance(dt, str):
        return core.dtype_from_name(dt)
    return core.dtype_from_numpy(dt)


# ---------------------------------------------------------------------------------------
# Interop helpers used by examples (reference: runtime/interop.py:323-420)
# ---------------------------------------------------------------------------------------

def _is_torch(x: Any) -> bool:
    t = sys.modules.get("torch")
    return t is not None and isinstance(x, t.Tensor)


def element_dtype(obj: Any) -> np.dtype:
    """The NumPy dtype of `obj`'s elements; bfloat16 reports `core.BF16_TAG` (kind "V")."""
    if isinstance(obj, Tensor):
        dt = obj.dtype
    elif _is_torch(obj):
        dt = core.dtype_from_torch(obj.dtype)
    else:
        return np.asarray(obj).dtype
    return core.BF16_TAG if dt is core.bfloat16 else dt.to_numpy()


def elem_dtype(x: Any) -> core.dtype:
    if isinstance(x, Tensor):
        return x.dtype
    if _is_torch(x):
        return core.dtype_from_torch(x.dtype)
    return core.dtype_from_numpy(np.asarray(x).dtype)


def element_strides(obj: Any) -> tuple[int, ...]:
    """The strides of any supported array, in elements."""
    if isinstance(obj, Tensor):
        return obj.strides
    if _is_torch(obj):
        return tuple(obj.stride())
    a = np.asarray(obj)
    return tuple(s // a.itemsize for s in a.strides)


def new_empty(like: Any, shape=None, dtype=None):
    """An uninitialised array of `like`'s kind (NumPy, torch, Tensor) and device."""
    shape = tuple(like.shape) if shape is None else tuple(shape)
    if _is_torch(like):
        import torch
        tdt = like.dtype if dtype is None else _torch_dtype(dtype)
        return torch.empty(shape, dtype=tdt, device=like.device)
    if isinstance(like, Tensor):
        return empty(shape, like.dtype if dtype is None else _as_dtype(dtype))
    return np.empty(shape, _numpy_storage(np.asarray(like).dtype if dtype is None else dtype))


def new_zeros(like: Any, shape=None, dtype=None):
    """A zero-filled array of `like`'s kind (NumPy, torch, Tensor) and device."""
    shape = tuple(like.shape) if shape is None else tuple(shape)
    if _is_torch(like):
        import torch
        tdt = like.dtype if dtype is None else _torch_dtype(dtype)
        return torch.zeros(shape, dtype=tdt, device=like.device)
    if isinstance(like, Tensor):
        return zeros(shape, like.dtype if dtype is None else _as_dtype(dtype))
    return np.zeros(shape, _numpy_storage(np.asarray(like).dtype if dtype is None else dtype))


def _numpy_storage(dt) -> np.dtype:
    """The NumPy storage dtype of element type `dt` (uint16 bit patterns for bfloat16)."""
    if isinstance(dt, core.dtype):
        return dt.to_numpy()
    d = np.dtype(dt)
    return core.bfloat16.to_numpy() if d.kind == "V" else d


def _torch_dtype(dt):
    import torch
    if not isinstance(dt, core.dtype) and not isinstance(dt, str):
        dt = core.dtype_from_numpy(dt)
    if isinstance(dt, core.dtype):
        name = dt.long_name
    else:
        name = np.dtype(dt).name
    return getattr(torch, {"int1": "bool"}.get(name, name))


def is_array_like(x: Any) -> bool:
    return isinstance(x, (np.ndarray, Tensor)) or _is_torch(x)


class Binding:
    """One array argument bound for a launch: its device pointer, plus a copy-back."""

    __slots__ = ("ptr", "host", "dev", "writeback", "keep", "key")

    def __init__(self, ptr, host=None, dev=None, keep=None, key=None):
        self.ptr = ptr
        self.host = host
        self.dev = dev
        self.writeback = False
        self.keep = keep
        self.key = key


# -- asynchronous host arrays (reference: runtime/interop.py:495-503) --------------------
# By default a launch that takes a NumPy (or CPU torch) array copies it to HBM, waits for
# the kernel and copies it back. With `async_numpy(True)` the launch returns at once; the
# device copy stays live and later launches on the same array use it (so chained kernels
# see each other's writes), and `enceladus.synchronize()` copies every written array back.
_async = False
_pending: dict[tuple[int, int], Binding] = {}


def async_numpy(enabled: bool = True) -> None:
    """Sets whether launches that touch host arrays return before the GPU finishes.
    With it on, call `enceladus.synchronize()` before reading or writing those arrays on
    the host. Turning it off synchronizes first."""
    global _async
    if not enabled and _async:
        flush_pending()
    _async = bool(enabled)


def flush_pending() -> None:
    """Waits for the device and copies back every host array a pending launch wrote."""
    if not _pending:
        return
    hip.call("ek_device_sync")
    items = list(_pending.values())
    _pending.clear()
    for b in items:
        finish_binding(b)


def complete_bindings(bindings: list) -> None:
    """After a launch: copy written host arrays back now, or leave them pending."""
    hosts = [b for b in bindings if b.host is not None]
    if not hosts:
        return
    if _async and all(b.key is not None for b in hosts):
        for b in hosts:
            p = _pending.get(b.key)
            if p is None:
                _pending[b.key] = b
            else:
                p.writeback = p.writeback or b.writeback
        return
    hip.call("ek_device_sync")
    for b in hosts:
        finish_binding(b)


def _bind_host(a: np.ndarray, n: int) -> Binding:
    start = a.__array_interface__["data"][0] if a.size else 0
    key = (start, n)
    if _pending:
        p = _pending.get(key)
        if p is not None:
            return Binding(p.dev.ptr, host=a, dev=p.dev, key=key)
        if any(s < start + n and start < s + m for s, m in _pending):
            flush_pending()       # another view of pending memory: settle it first
    dev = Tensor((max(n, 1),), core.uint8)
    if n:
        hip.call("ek_memcpy_h2d", ctypes.c_void_p(dev.ptr), ctypes.c_void_p(start), n, None)
    return Binding(dev.ptr, host=a, dev=dev, key=key)


def _host_array(x: Any):
    """The host ndarray behind a NumPy or CPU-torch argument, or None."""
    if isinstance(x, np.ndarray):
        return x
    if _is_torch(x) and x.device.type != "cuda":
        return x.detach().numpy()
    return None


def bind_arrays(values: list, writes: set) -> tuple[list, list]:
    """Binds the array arguments of one launch: (device pointer per array argument in
    order, bindings). Host arrays whose byte spans overlap (views of one buffer, such as
    `a[::2]` and `a[1::2]`) share one device copy of the union of their spans, so the
    kernel sees one memory as the host does and the copy back writes each byte once; other
    host arrays are copied alone, device arrays pass their pointers."""
    spans = []
    for i, v in enumerate(values):
        a = _host_array(v)
        if a is not None:
            n = _span_bytes(a)
            if n:
                spans.append((a.__array_interface__["data"][0], n, i, a))
    groups: dict[int, tuple[int, int]] = {}
    if len(spans) > 1:
        spans.sort(key=lambda t: t[0])
        lo, hi, members = spans[0][0], spans[0][0] + spans[0][1], [spans[0][2]]
        for start, n, i, _ in spans[1:]:
            if start < hi:
                hi = max(hi, start + n)
                members.append(i)
            else:
                if len(members) > 1:
                    for m in members:
                        groups[m] = (lo, hi)
                lo, hi, members = start, start + n, [i]
        if len(members) > 1:
            for m in members:
                groups[m] = (lo, hi)
    ptrs, bindings = [], []
    shared: dict[tuple[int, int], Binding] = {}
    for i, v in enumerate(values):
        if i in groups:
            lo, hi = groups[i]
            b = shared.get((lo, hi))
            if b is None:
                flush_pending()
                region = np.ctypeslib.as_array((ctypes.c_uint8 * (hi - lo)).from_address(lo))
                b = _bind_host(region, hi - lo)
                b.key = None                 # settled at the launch, never left pending
                shared[(lo, hi)] = b
                bindings.append(b)
            b.writeback = b.writeback or i in writes
            a = _host_array(v)
            ptrs.append(b.ptr + (a.__array_interface__["data"][0] - lo))
            continue
        b = bind_array(v)
        b.writeback = i in writes
        bindings.append(b)
        ptrs.append(b.ptr)
    return ptrs, bindings


def bind_array(x: Any) -> Binding:
    if isinstance(x, Tensor):
        return Binding(x.ptr, keep=x)
    if _is_torch(x):
        if x.device.type == "cuda":
            return Binding(int(x.data_ptr()), keep=x)
        a = x.detach().numpy()
        return _bind_host(a, _span_bytes(a))
    a = x if isinstance(x, np.ndarray) else np.asarray(x)
    return _bind_host(a, _span_bytes(a))


def _span_bytes(a: np.ndarray) -> int:
    if a.size == 0:
        return 0
    if any(s < 0 for s in a.strides):
        raise ValueError("arrays with negative strides can't be kernel arguments")
    return a.itemsize * (1 + sum((n - 1) * (s // a.itemsize) for n, s in zip(a.shape, a.strides)))


def finish_binding(b: Binding) -> None:
    if b.host is None or not b.writeback:
        return
    a = b.host
    n = _span_bytes(a)
    if n:
        start = a.__array_interface__["data"][0]
        hip.call("ek_memcpy_d2h", ctypes.c_void_p(start), ctypes.c_void_p(b.dev.ptr), n, None)
