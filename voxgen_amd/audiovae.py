"""AudioVaeEngine over the C ABI: the decoder half of src/audiovae.rs
(AudioVaeEngine::decode_latents, audiovae.rs:330-372), with the reference's
argument checks; failures raise abi.VxError."""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import abi
from .runtime import Buffer, Context, Model


def config_struct(cfg: dict) -> abi.AudioVaeConfig:
    c = abi.AudioVaeConfig()
    for k, _ in c._fields_:
        v = cfg[k]
        if isinstance(v, (list, tuple)):
            arr = getattr(c, k)
            for i, x in enumerate(v):
                arr[i] = x
        else:
            setattr(c, k, v)
    return c


@dataclass
class AudioDecodeStats:
    """AudioDecodeStats (audiovae.rs:179-191)."""
    latent_frames: int
    latent_patches: int
    output_samples: int
    output_sample_rate: int
    duration_seconds: float
    checksum: float
    l2: float
    peak: float
    decode_ms: float
    scratch_bytes: int


class AudioVaeEngine:
    def __init__(self, ctx: Context, model: Model, config: dict, strict_geometry: bool = True):
        self.ctx, self.model, self.config = ctx, model, dict(config)
        self.handle = None
        h = abi.AUDIOVAE()
        abi.call("vx_audiovae_create", ctx.handle, model.handle, C.byref(config_struct(config)),
                 1 if strict_geometry else 0, C.byref(h))
        self.handle = h.value
        ctx.register(self)

    def close(self) -> None:
        if self.handle and self.ctx.handle:
            abi.load().vx_audiovae_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def scratch_bytes(self) -> int:
        return abi.load().vx_audiovae_scratch_bytes(self.handle)

    def decode_latents(self, frame_major) -> tuple[AudioDecodeStats, np.ndarray]:
        """decode_latents: frame-major latents [frames][latent_dim] -> (stats, wave)."""
        x = np.ascontiguousarray(frame_major, dtype=np.float32).ravel()
        ld, hop = self.config["latent_dim"], self.config["decoder_hop"]
        wave = np.zeros(max(1, (x.size // max(ld, 1)) * hop), np.float32)
        st = abi.AudioDecodeStats()
        abi.call("vx_audiovae_decode_latents", self.handle, x.ctypes.data_as(C.POINTER(C.c_float)), x.size,
                 wave.ctypes.data_as(C.POINTER(C.c_float)), wave.size, C.byref(st))
        return AudioDecodeStats(*(getattr(st, k) for k, _ in st._fields_)), wave

    def decode_latents_gpu(self, latents: Buffer, frames: int, wave: Buffer) -> None:
        """The same decode between device buffers (enqueue only)."""
        abi.call("vx_audiovae_decode_latents_gpu", self.handle, latents.handle, frames, wave.handle)
