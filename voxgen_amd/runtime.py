"""Python handles over the C ABI: device context, buffers and the model region.

Mirrors the reference's VulkanContext / GpuBuffer surface (src/vulkan.rs:79-955):
Context ~ VulkanContext::new, Buffer ~ GpuBuffer, Model ~ the uploaded GGUF data
region with its tensor table.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Iterable, Sequence

import weakref

import numpy as np

from . import abi

_DTYPE_NAMES = {abi.DTYPE_F32: "F32", abi.DTYPE_F16: "F16", abi.DTYPE_Q8_0: "Q8_0"}


@dataclass
class TensorDesc:
    """One tensor of a GGUF data region (TensorInfo, gguf.rs:51-59)."""
    name: str
    ggml_type: int
    dims: tuple          # GGUF order: dims[0] is the contiguous axis
    offset: int          # byte offset into the data region
    nbytes: int = 0

    def __post_init__(self):
        if not self.nbytes:
            self.nbytes = storage_bytes(self.ggml_type, self.dims)

    @property
    def type_name(self) -> str:
        return _DTYPE_NAMES.get(self.ggml_type, f"GGML_TYPE_{self.ggml_type}")

    def to_c(self) -> abi.TensorInfo:
        t = abi.TensorInfo()
        t.name = self.name.encode()
        t.ggml_type = self.ggml_type
        t.n_dims = len(self.dims)
        for i, d in enumerate(self.dims):
            t.dims[i] = d
        t.offset = self.offset
        t.bytes = self.nbytes
        return t

    @staticmethod
    def from_c(t: abi.TensorInfo) -> "TensorDesc":
        return TensorDesc(t.name.decode(), t.ggml_type, tuple(t.dims[i] for i in range(t.n_dims)),
                          t.offset, t.bytes)


def storage_bytes(ggml_type: int, dims: Sequence[int]) -> int:
    """GgmlType::storage_bytes (gguf.rs:37-48)."""
    n = int(np.prod(dims, dtype=np.uint64)) if len(dims) else 1
    if ggml_type == abi.DTYPE_F32:
        return n * 4
    if ggml_type == abi.DTYPE_F16:
        return n * 2
    if ggml_type == abi.DTYPE_Q8_0:
        if n % 32:
            raise ValueError(f"Q8_0 tensor has {n} elements, not divisible by 32")
        return n // 32 * 34
    raise ValueError(f"unsupported GGML tensor type {ggml_type}")


class Buffer:
    """Device memory owned by the caller (GpuBuffer)."""

    def __init__(self, ctx: "Context", handle: int, nbytes: int, owned: bool = True):
        self.ctx, self.handle, self.nbytes, self.owned = ctx, handle, nbytes, owned

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def free(self) -> None:
        if self.owned and self.handle and self.ctx.handle:
            abi.load().vx_free(self.ctx.handle, self.handle)
        self.handle = None

    @property
    def device_ptr(self) -> int:
        return abi.load().vx_buf_device_ptr(self.handle) or 0

    def upload(self, arr, offset: int = 0) -> "Buffer":
        a = np.ascontiguousarray(arr)
        abi.call("vx_upload", self.ctx.handle, self.handle, offset, a.ctypes.data_as(C.c_void_p),
                 a.nbytes)
        return self

    def download(self, dtype=np.float32, count: int | None = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dt.itemsize
        out = np.empty(count, dtype=dt)
        abi.call("vx_download", self.ctx.handle, self.handle, offset,
                 out.ctypes.data_as(C.c_void_p), out.nbytes)
        return out

    def fill_u32(self, value: int, count: int | None = None, offset: int = 0) -> None:
        if count is None:
            count = (self.nbytes - offset) // 4
        abi.call("vx_fill_u32", self.ctx.handle, self.handle, offset, value, count)


class Context:
    """One HIP device + one in-order stream (VulkanContext::new, vulkan.rs:284)."""

    def __init__(self, device: int = 0):
        self.handle = None
        # Engines created on this context (BaseLmEngine, LocDit): closed before the
        # context itself, whatever order the interpreter finalises objects in.
        self._engines = weakref.WeakSet()
        h = abi.CTX()
        abi.call("vx_init", device, C.byref(h))
        self.handle = h.value
        self.device = device

    def register(self, engine) -> None:
        self._engines.add(engine)

    def close(self) -> None:
        if self.handle:
            for e in list(self._engines):
                e.close()
            abi.load().vx_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self) -> dict:
        d = abi.DeviceInfo()
        abi.call("vx_device_info_get", self.handle, C.byref(d))
        return {k: (getattr(d, k).decode() if isinstance(getattr(d, k), bytes) else getattr(d, k))
                for k, _ in d._fields_}

    def alloc(self, nbytes: int) -> Buffer:
        h = abi.BUFP()
        abi.call("vx_alloc", self.handle, int(nbytes), C.byref(h))
        return Buffer(self, h.value, int(nbytes))

    def array(self, arr) -> Buffer:
        """Allocate a buffer holding a copy of `arr`."""
        a = np.ascontiguousarray(arr)
        return self.alloc(max(a.nbytes, 4)).upload(a)

    def zeros(self, nbytes: int) -> Buffer:
        b = self.alloc(nbytes)
        b.fill_u32(0, nbytes // 4)
        return b

    def sync(self) -> None:
        abi.call("vx_sync", self.handle)

    def set_cancelled(self, cancelled: bool) -> None:
        """Set or clear this context's cancellation word (the AtomicBool of
        synthesize_cancelable, runtime.rs:745-808): while it is set, every engine
        step on the context fails with VX_ERR_CANCELLED before it is enqueued.
        The word lives in this object and is registered on first use."""
        if getattr(self, "_cancel", None) is None:
            self._cancel = C.c_uint32(0)
            abi.call("vx_set_cancel_flag", self.handle, C.byref(self._cancel))
        self._cancel.value = 1 if cancelled else 0

    # graphs
    def graph_begin(self) -> None:
        abi.call("vx_graph_begin", self.handle)

    def graph_end(self) -> int:
        g = abi.GRAPH()
        abi.call("vx_graph_end", self.handle, C.byref(g))
        return g.value

    def graph_launch(self, g: int) -> None:
        abi.call("vx_graph_launch", self.handle, g)

    def graph_free(self, g: int) -> None:
        abi.call("vx_graph_free", self.handle, g)

    # profiling (gpu_profile_* vulkan.rs:587-635)
    def prof_enable(self, on: bool = True) -> None:
        abi.call("vx_prof_enable", self.handle, 1 if on else 0)

    def prof_reset(self) -> None:
        abi.call("vx_prof_reset", self.handle)

    def prof_snapshot(self) -> dict:
        n = C.c_uint32()
        abi.call("vx_prof_snapshot", self.handle, None, 0, C.byref(n))
        arr = (abi.ProfEntry * max(n.value, 1))()
        abi.call("vx_prof_snapshot", self.handle, arr, n.value, C.byref(n))
        return {arr[i].name.decode(): dict(total_ms=arr[i].total_ms, calls=arr[i].calls,
                                           avg_ms=arr[i].avg_ms) for i in range(n.value)}


class Model:
    """The GGUF data region on the device plus its tensor table."""

    def __init__(self, ctx: Context, data, tensors: Iterable[TensorDesc]):
        self.ctx = ctx
        self.handle = None
        buf = np.ascontiguousarray(np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray)) else data)
        tl = list(tensors)
        arr = (abi.TensorInfo * max(len(tl), 1))(*[t.to_c() for t in tl])
        h = abi.MODEL()
        abi.call("vx_model_upload", ctx.handle, buf.ctypes.data_as(C.c_void_p), buf.nbytes, arr,
                 len(tl), C.byref(h))
        self.handle = h.value
        self.tensors = {t.name: t for t in tl}

    @classmethod
    def from_gguf(cls, ctx: Context, gguf) -> "Model":
        self = cls.__new__(cls)
        self.ctx = ctx
        h = abi.MODEL()
        abi.call("vx_model_upload_gguf", ctx.handle, gguf.handle, C.byref(h))
        self.handle = h.value
        self.tensors = {t.name: t for t in gguf.tensors()}
        return self

    def free(self) -> None:
        if self.handle and self.ctx.handle:
            abi.load().vx_model_free(self.ctx.handle, self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    @property
    def device_bytes(self) -> int:
        return abi.load().vx_model_device_bytes(self.handle)

    def find(self, name: str) -> TensorDesc:
        t = abi.TensorInfo()
        abi.call("vx_model_find", self.handle, name.encode(), C.byref(t))
        return TensorDesc.from_c(t)

    def offset(self, name: str) -> int:
        return self.tensors[name].offset
