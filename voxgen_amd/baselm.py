"""BaseLmEngine over the C ABI: the Python mirror of src/baselm.rs's engine API.

Method names and behaviour follow BaseLmEngine (baselm.rs:451-880): the same
entry points, position bookkeeping, context guard and error conditions (raised
as abi.VxError with the matching status).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import abi
from .runtime import Buffer, Context, Model

EXEC_MODES = {"graph": abi.EXEC_GRAPH, "fused": abi.EXEC_FUSED, "reference": abi.EXEC_REFERENCE,
              "persistent": abi.EXEC_PERSISTENT}
# Workgroup schedule of the batched prefill's gate/up projection (VX_PREFILL_*).
PREFILL_SCHEDULES = {"auto": abi.PREFILL_AUTO, "tiles": abi.PREFILL_TILES,
                     "streamk_tail_first": abi.PREFILL_STREAMK_TAIL_FIRST}


def config_struct(cfg: dict) -> abi.BaseLmConfig:
    c = abi.BaseLmConfig()
    for k, _ in c._fields_:
        setattr(c, k, cfg[k])
    return c


def rope_scaling_factor(cfg: dict) -> float:
    """BaseLmConfig::rope_scaling_factor (baselm.rs:194-205)."""
    return abi.load().vx_baselm_rope_scaling_factor(C.byref(config_struct(cfg)))


def kv_cache_bytes(cfg: dict) -> int:
    """BaseLmConfig::kv_cache_bytes (baselm.rs:182-188)."""
    return abi.load().vx_baselm_kv_cache_bytes(C.byref(config_struct(cfg)))


def effective_scale(v: float) -> float:
    """effective_scale (baselm.rs:1262-1264)."""
    return 1.0 if v == 0.0 else v


@dataclass
class StepResult:
    """BaseLmStepResult (baselm.rs:404-411)."""
    position: int
    elapsed_ms: float
    final_hidden_checksum: float
    final_hidden_l2: float
    top_logits: list


class BaseLmEngine:
    def __init__(self, ctx: Context, model: Model, config: dict, exec_mode: str = "graph",
                 strict_geometry: bool = True, attn_splits: int = 0, prefill_schedule: str = "auto"):
        self.ctx, self.model, self.config = ctx, model, dict(config)
        self.handle = None
        opt = abi.BaseLmOptions(EXEC_MODES[exec_mode], 1 if strict_geometry else 0, attn_splits,
                                PREFILL_SCHEDULES[prefill_schedule])
        h = abi.ENGINE()
        abi.call("vx_baselm_create", ctx.handle, model.handle, C.byref(config_struct(config)),
                 C.byref(opt), C.byref(h))
        self.handle = h.value
        ctx.register(self)

    def close(self) -> None:
        if self.handle and self.ctx.handle:   # a closed context already released the device
            abi.load().vx_baselm_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # --- state -----------------------------------------------------------
    @property
    def position(self) -> int:
        return abi.load().vx_baselm_position(self.handle)

    def set_position(self, p: int) -> None:
        abi.call("vx_baselm_set_position", self.handle, p)

    def reset(self) -> None:
        abi.call("vx_baselm_reset", self.handle)

    def buffer(self, name: str) -> Buffer:
        h = abi.load().vx_baselm_buffer(self.handle, abi.BUF[name.upper()])
        return Buffer(self.ctx, h, abi.load().vx_buf_size(h), owned=False)

    def output(self) -> np.ndarray:
        """output_buffer(): the normalised final hidden state (baselm.rs:608-612)."""
        return self.buffer("norm").download(np.float32, self.config["embedding_length"])

    # --- decode entry points -------------------------------------------
    def _result(self, r: abi.StepResult, top) -> StepResult:
        tl = [(top[i].token_id, top[i].logit) for i in range(r.n_top)] if top is not None else []
        return StepResult(r.position, r.elapsed_ms, r.final_hidden_checksum, r.final_hidden_l2, tl)

    def decode_token(self, token_id: int, top_k: int = 0) -> StepResult:
        r = abi.StepResult()
        top = (abi.TopLogit * max(top_k, 1))()
        abi.call("vx_baselm_decode_token", self.handle, token_id, top_k, C.byref(r), top)
        return self._result(r, top)

    def decode_embedding(self, embedding, top_k: int = 0) -> StepResult:
        e = np.ascontiguousarray(embedding, dtype=np.float32)
        r = abi.StepResult()
        top = (abi.TopLogit * max(top_k, 1))()
        abi.call("vx_baselm_decode_embedding", self.handle,
                 e.ctypes.data_as(C.POINTER(C.c_float)), e.size, top_k, C.byref(r), top)
        return self._result(r, top)

    def decode_token_gpu_only(self, token_id: int) -> int:
        p = C.c_uint32()
        abi.call("vx_baselm_decode_token_gpu_only", self.handle, token_id, C.byref(p))
        return p.value

    def decode_embedding_gpu_only(self, embedding) -> int:
        e = np.ascontiguousarray(embedding, dtype=np.float32)
        p = C.c_uint32()
        abi.call("vx_baselm_decode_embedding_gpu_only", self.handle,
                 e.ctypes.data_as(C.POINTER(C.c_float)), e.size, C.byref(p))
        return p.value

    def decode_embedding_from_gpu_only(self, source: Buffer) -> int:
        p = C.c_uint32()
        abi.call("vx_baselm_decode_embedding_from_gpu_only", self.handle, source.handle, C.byref(p))
        return p.value

    def decode_tokens_gpu_only(self, tokens) -> None:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        abi.call("vx_baselm_decode_tokens_gpu_only", self.handle,
                 t.ctypes.data_as(C.POINTER(C.c_uint32)), t.size)

    def prefill_tokens(self, tokens, top_k_last: int = 0) -> StepResult:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        r = abi.StepResult()
        top = (abi.TopLogit * max(top_k_last, 1))()
        abi.call("vx_baselm_prefill_tokens", self.handle, t.ctypes.data_as(C.POINTER(C.c_uint32)),
                 t.size, top_k_last, C.byref(r), top)
        return self._result(r, top)

    def prefill_tokens_batched(self, tokens, top_k_last: int = 0) -> StepResult:
        """prefill_tokens with all tokens through the layer stack at once (MFMA
        projections, causal attention over the cache)."""
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        r = abi.StepResult()
        top = (abi.TopLogit * max(top_k_last, 1))()
        abi.call("vx_baselm_prefill_tokens_batched", self.handle, t.ctypes.data_as(C.POINTER(C.c_uint32)),
                 t.size, top_k_last, C.byref(r), top)
        return self._result(r, top)

    def prefill_tokens_batched_gpu_only(self, tokens) -> None:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        abi.call("vx_baselm_prefill_tokens_batched_gpu_only", self.handle,
                 t.ctypes.data_as(C.POINTER(C.c_uint32)), t.size)

    def benchmark(self, token_id: int, warmup: int, iterations: int) -> dict:
        b = abi.BenchmarkResult()
        abi.call("vx_baselm_benchmark", self.handle, token_id, warmup, iterations, C.byref(b))
        return {k: getattr(b, k) for k, _ in b._fields_}

    LAYER_KERNELS = ("qkv", "attention", "attn_out", "swiglu", "down")

    def time_layer_kernel(self, name: str, reps: int = 4) -> float:
        """Average cost (ms) of one fused layer kernel inside a graph chain over all
        layers, each pass after a MALL-evicting read (every launch reads HBM), from
        HIP events on the engine stream."""
        out = C.c_double()
        abi.call("vx_baselm_time_layer_kernel", self.handle, self.LAYER_KERNELS.index(name), reps,
                 C.byref(out))
        return out.value

    def profile_steps(self, tokens) -> dict:
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        n = C.c_uint32()
        arr = (abi.ProfEntry * 64)()
        abi.call("vx_baselm_profile_steps", self.handle, t.ctypes.data_as(C.POINTER(C.c_uint32)),
                 t.size, arr, 64, C.byref(n))
        return {arr[i].name.decode(): dict(total_ms=arr[i].total_ms, calls=arr[i].calls,
                                           avg_ms=arr[i].avg_ms) for i in range(min(n.value, 64))}
