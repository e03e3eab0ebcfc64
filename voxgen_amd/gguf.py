"""GGUF v3 writer for synthetic models, and a reader handle over the C parser.

The writer produces the layout gguf.rs:222-286 parses: magic, version, counts,
metadata (key, type, value), tensor infos (name, rank, dims, type, offset), then
the data region at the next `general.alignment` boundary.
"""
from __future__ import annotations

import ctypes as C
import struct
from pathlib import Path

import numpy as np

from . import abi
from .runtime import TensorDesc

MAGIC = 0x46554747
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<B", 10: "<Q",
           11: "<q", 12: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(ty: int, v) -> bytes:
    if ty == 8:
        return _str(v)
    if ty == 9:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_value(et, x) for x in items)
    return struct.pack(_SCALAR[ty], int(v) if ty not in (6, 12) else float(v))


def header_bytes(metadata: dict, tensors, version: int = 3, alignment: int = 32) -> bytes:
    out = bytearray(struct.pack("<IIQQ", MAGIC, version, len(tensors), len(metadata)))
    for k, (ty, v) in metadata.items():
        out += _str(k) + struct.pack("<I", ty) + _value(ty, v)
    for t in tensors:
        out += _str(t.name) + struct.pack("<I", len(t.dims))
        out += b"".join(struct.pack("<Q", d) for d in t.dims)
        out += struct.pack("<IQ", t.ggml_type, t.offset)
    pad = (-len(out)) % alignment
    return bytes(out) + b"\0" * pad


def write(path, metadata: dict, tensors, data: np.ndarray | None, data_bytes: int | None = None,
          version: int = 3) -> Path:
    """Write a GGUF file. With data=None the data region is left sparse (zeros)."""
    path = Path(path)
    align = metadata.get("general.alignment", (4, 32))[1]
    hdr = header_bytes(metadata, tensors, version, align)
    with open(path, "wb") as f:
        f.write(hdr)
        if data is not None:
            f.write(memoryview(np.ascontiguousarray(data, dtype=np.uint8)))
        else:
            f.truncate(len(hdr) + int(data_bytes))
    return path


class Gguf:
    """Parsed GGUF (load_summary, gguf.rs:222-286) through the C ABI."""

    def __init__(self, path):
        self.handle = None
        h = abi.GGUF()
        abi.call("vx_gguf_open", str(path).encode(), C.byref(h))
        self.handle = h.value
        self.path = str(path)

    def close(self) -> None:
        if self.handle:
            abi.load().vx_gguf_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def summary(self) -> dict:
        s = abi.GgufSummary()
        abi.call("vx_gguf_summary_get", self.handle, C.byref(s))
        return {k: getattr(s, k) for k, _ in s._fields_}

    def tensors(self) -> list:
        n = self.summary()["tensor_count"]
        out = []
        for i in range(n):
            t = abi.TensorInfo()
            abi.call("vx_gguf_tensor_at", self.handle, i, C.byref(t))
            out.append(TensorDesc.from_c(t))
        return out

    def meta(self, key: str) -> str:
        buf = C.create_string_buffer(1024)
        abi.call("vx_gguf_meta", self.handle, key.encode(), buf, 1024)
        return buf.value.decode()

    def primary_format(self) -> int:
        v = C.c_uint32()
        abi.call("vx_gguf_primary_format", self.handle, C.byref(v))
        return v.value

    def baselm_config(self, active_context: int) -> dict:
        c = abi.BaseLmConfig()
        abi.call("vx_baselm_config_from_gguf", self.handle, active_context, C.byref(c))
        return {k: getattr(c, k) for k, _ in c._fields_}

    def acoustic_config(self, base_config: dict, active_context: int) -> dict:
        """AcousticConfig::from_gguf (acoustic.rs:59-125) against the BaseLM config."""
        b = abi.BaseLmConfig()
        for k, _ in b._fields_:
            setattr(b, k, base_config[k])
        c = abi.AcousticConfig()
        abi.call("vx_acoustic_config_from_gguf", self.handle, C.byref(b), active_context, C.byref(c))
        return {k: getattr(c, k) for k, _ in c._fields_}

    def audiovae_config(self) -> dict:
        """AudioVaeConfig::from_gguf (audiovae.rs:49-128)."""
        c = abi.AudioVaeConfig()
        abi.call("vx_audiovae_config_from_gguf", self.handle, C.byref(c))
        out = {}
        for k, _ in c._fields_:
            v = getattr(c, k)
            out[k] = list(v) if hasattr(v, "__len__") else v
        return out
