"""ResidualFsqEngine over the C ABI: the Python mirror of src/acoustic.rs's
ResidualLM + FSQ + fusion + stop-predictor engine (acoustic.rs:400-1035).

Method names, arguments and error conditions follow the reference; failures
raise abi.VxError with the matching status.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import abi
from .runtime import Buffer, Context, Model

EXEC_MODES = {"graph": abi.EXEC_GRAPH, "fused": abi.EXEC_FUSED, "reference": abi.EXEC_REFERENCE}


def config_struct(cfg: dict) -> abi.AcousticConfig:
    c = abi.AcousticConfig()
    for k, _ in c._fields_:
        setattr(c, k, cfg[k])
    return c


def kv_cache_bytes(cfg: dict) -> int:
    """AcousticConfig::kv_cache_bytes (acoustic.rs:176-182)."""
    return abi.load().vx_acoustic_kv_cache_bytes(C.byref(config_struct(cfg)))


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _fp(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_float))


@dataclass
class FsqResult:
    """FsqResult (acoustic.rs:359-366)."""
    elapsed_ms: float
    output_checksum: float
    output_l2: float
    latent_checksum: float
    latent_l2: float


@dataclass
class ResidualStepResult:
    """ResidualStepResult (acoustic.rs:368-379); fsq_* are None without FSQ."""
    position: int
    elapsed_ms: float
    fsq_applied: bool
    fsq_checksum: float | None
    fsq_l2: float | None
    fused_input_checksum: float
    fused_input_l2: float
    residual_hidden_checksum: float
    residual_hidden_l2: float


@dataclass
class ResidualGpuStep:
    """ResidualGpuStep (acoustic.rs:381)."""
    position: int
    elapsed_ms: float
    fsq_applied: bool


@dataclass
class StopPrediction:
    """StopPrediction (acoustic.rs:393-398)."""
    stop: bool
    continue_logit: float
    stop_logit: float
    elapsed_ms: float


class ResidualFsqEngine:
    def __init__(self, ctx: Context, model: Model, config: dict, exec_mode: str = "graph",
                 strict_geometry: bool = True):
        self.ctx, self.model, self.config = ctx, model, dict(config)
        self.handle = None
        opt = abi.ResidualOptions(EXEC_MODES[exec_mode], 1 if strict_geometry else 0)
        h = abi.RESIDUAL()
        abi.call("vx_residual_create", ctx.handle, model.handle, C.byref(config_struct(config)),
                 C.byref(opt), C.byref(h))
        self.handle = h.value
        ctx.register(self)

    def close(self) -> None:
        if self.handle and self.ctx.handle:
            abi.load().vx_residual_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # --- state (acoustic.rs:585-615) --------------------------------------
    @property
    def position(self) -> int:
        return abi.load().vx_residual_position(self.handle)

    def reset(self) -> None:
        abi.call("vx_residual_reset", self.handle)

    def allocated_bytes(self) -> int:
        return abi.load().vx_residual_allocated_bytes(self.handle)

    def buffer(self, name: str) -> Buffer:
        h = abi.load().vx_residual_buffer(self.handle, abi.RESIDUAL_BUF[name.upper()])
        return Buffer(self.ctx, h, abi.load().vx_buf_size(h), owned=False)

    def output_buffer(self) -> Buffer:
        return self.buffer("output")

    def current_lm_buffer(self) -> Buffer:
        return self.buffer("current_lm")

    def output(self) -> np.ndarray:
        return self.output_buffer().download(np.float32, self.config["embedding_length"])

    # --- entry points -------------------------------------------------------
    @staticmethod
    def _step(r: abi.ResidualStepResult) -> ResidualStepResult:
        fsq = bool(r.fsq_applied)
        return ResidualStepResult(r.position, r.elapsed_ms, fsq, r.fsq_checksum if fsq else None,
                                  r.fsq_l2 if fsq else None, r.fused_input_checksum, r.fused_input_l2,
                                  r.residual_hidden_checksum, r.residual_hidden_l2)

    @staticmethod
    def _gpu_step(r: abi.ResidualGpuStep) -> ResidualGpuStep:
        return ResidualGpuStep(r.position, r.elapsed_ms, bool(r.fsq_applied))

    def fsq_only(self, base_hidden) -> FsqResult:
        b = _f32(base_hidden)
        r = abi.FsqResult()
        abi.call("vx_residual_fsq_only", self.handle, _fp(b), b.size, C.byref(r))
        return FsqResult(r.elapsed_ms, r.output_checksum, r.output_l2, r.latent_checksum, r.latent_l2)

    def step(self, base_hidden, current_embedding) -> ResidualStepResult:
        b, e = _f32(base_hidden), _f32(current_embedding)
        if b.size != e.size:
            raise abi.VxError(abi.STATUS_CODE["VX_ERR_SHAPE"],
                              f"current embedding has {e.size} floats; expected {b.size}", "step")
        r = abi.ResidualStepResult()
        abi.call("vx_residual_step", self.handle, _fp(b), _fp(e), b.size, C.byref(r))
        return self._step(r)

    def step_from_gpu_base(self, base_hidden_gpu: Buffer, current_embedding) -> ResidualStepResult:
        e = _f32(current_embedding)
        r = abi.ResidualStepResult()
        abi.call("vx_residual_step_from_gpu_base", self.handle, base_hidden_gpu.handle, _fp(e), e.size,
                 C.byref(r))
        return self._step(r)

    def step_from_gpu_base_and_embedding(self, base_hidden_gpu: Buffer,
                                         current_embedding_gpu: Buffer) -> ResidualStepResult:
        r = abi.ResidualStepResult()
        abi.call("vx_residual_step_from_gpu_base_and_embedding", self.handle, base_hidden_gpu.handle,
                 current_embedding_gpu.handle, C.byref(r))
        return self._step(r)

    def step_from_gpu_base_and_embedding_gpu_only(self, base_hidden_gpu: Buffer,
                                                  current_embedding_gpu: Buffer) -> ResidualGpuStep:
        r = abi.ResidualGpuStep()
        abi.call("vx_residual_step_from_gpu_base_and_embedding_gpu_only", self.handle, base_hidden_gpu.handle,
                 current_embedding_gpu.handle, C.byref(r))
        return self._gpu_step(r)

    def step_text_prefix_from_gpu_base(self, base_hidden_gpu: Buffer) -> ResidualStepResult:
        r = abi.ResidualStepResult()
        abi.call("vx_residual_step_text_prefix_from_gpu_base", self.handle, base_hidden_gpu.handle, C.byref(r))
        return self._step(r)

    def step_text_prefix_from_gpu_base_gpu_only(self, base_hidden_gpu: Buffer) -> ResidualGpuStep:
        r = abi.ResidualGpuStep()
        abi.call("vx_residual_step_text_prefix_from_gpu_base_gpu_only", self.handle, base_hidden_gpu.handle,
                 C.byref(r))
        return self._gpu_step(r)

    def benchmark(self, base_hidden, current_embedding, warmup: int, iterations: int) -> dict:
        b, e = _f32(base_hidden), _f32(current_embedding)
        r = abi.ResidualBenchmark()
        abi.call("vx_residual_benchmark", self.handle, _fp(b), _fp(e), b.size, warmup, iterations, C.byref(r))
        return {k: getattr(r, k) for k, _ in r._fields_}

    @staticmethod
    def _stop(r: abi.StopPrediction) -> StopPrediction:
        return StopPrediction(bool(r.stop), r.continue_logit, r.stop_logit, r.elapsed_ms)

    def predict_stop_from_gpu_base(self, base_hidden_gpu: Buffer) -> StopPrediction:
        r = abi.StopPrediction()
        abi.call("vx_residual_predict_stop_from_gpu_base", self.handle, base_hidden_gpu.handle, C.byref(r))
        return self._stop(r)

    def predict_stop_from_current_lm(self) -> StopPrediction:
        r = abi.StopPrediction()
        abi.call("vx_residual_predict_stop_from_current_lm", self.handle, C.byref(r))
        return self._stop(r)

    def prefill_text_from_gpu_rows(self, rows: Buffer, n: int) -> None:
        """n text-prefix positions from n BaseLM output rows at once (enqueue only)."""
        abi.call("vx_residual_prefill_text_from_gpu_rows", self.handle, rows.handle, n)


def prefill_text_cross_engine(base, residual: ResidualFsqEngine, tokens) -> None:
    """The text runs of prefill_conditioning_plan (runtime.rs:483-566): BaseLM then
    ResidualLM text prefix for every token, batched per engine (enqueue only)."""
    t = np.ascontiguousarray(tokens, dtype=np.uint32)
    abi.call("vx_prefill_text_cross_engine", base.handle, residual.handle,
             t.ctypes.data_as(C.POINTER(C.c_uint32)), t.size)
