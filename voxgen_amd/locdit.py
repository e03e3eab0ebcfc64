"""LocDiT estimator and UnifiedCFM solve over the C ABI: the Python mirror of the
LocDiT half of LocalEngine (local.rs:264-537).

Method names follow LocalEngine: estimate() is locdit_from_cpu_mu
(local.rs:352-355) and cfm_solve() is cfm_from_cpu_mu (local.rs:359-363). Errors
raise abi.VxError with the status of the reference's bail.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import abi
from .runtime import Context, Model


@dataclass
class CfmOptions:
    """CfmOptions (local.rs:244-252); defaults are the CLI's (main.rs:239-257)."""
    n_timesteps: int = 10
    cfg_value: float = 2.0
    temperature: float = 1.0
    sway_sampling_coef: float = 1.0
    seed: int = 42
    use_cfg_zero_star: bool = True

    def to_c(self) -> abi.CfmOptions:
        return abi.CfmOptions(self.n_timesteps, self.cfg_value, self.temperature, self.sway_sampling_coef,
                              self.seed & 0xFFFFFFFFFFFFFFFF, 1 if self.use_cfg_zero_star else 0)


def _f32p(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_float))


class LocDit:
    def __init__(self, ctx: Context, model: Model, config: dict, rope_model: Model | None = None,
                 rope_factor_offset: int | None = None, strict_geometry: bool = True):
        self.ctx, self.model, self.config = ctx, model, dict(config)
        self.handle = None
        rm = rope_model or model
        if rope_factor_offset is None:
            rope_factor_offset = rm.offset("rope_factors_short.weight")
        c = abi.LocDitConfig()
        for k, _ in c._fields_:
            setattr(c, k, config[k])
        h = abi.LOCDIT()
        abi.call("vx_locdit_create", ctx.handle, model.handle, rm.handle, rope_factor_offset, C.byref(c),
                 1 if strict_geometry else 0, C.byref(h))
        self.handle = h.value
        self._keep = (model, rm)
        ctx.register(self)

    def close(self) -> None:
        if self.handle and self.ctx.handle:   # a closed context already released the device
            abi.load().vx_locdit_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def patch_floats(self) -> int:
        return self.config["patch"] * self.config["feat_dim"]

    def _inputs(self, cond, mu):
        cond = np.ascontiguousarray(cond, np.float32)
        mu = np.ascontiguousarray(mu if mu is not None else np.zeros(1, np.float32), np.float32)
        return cond, mu

    def estimate(self, x, cond, mu, t: float, dt: float = 0.0) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        cond, mu = self._inputs(cond, mu)
        out = np.empty(self.patch_floats, np.float32)
        abi.call("vx_locdit_estimate", self.handle, _f32p(x), _f32p(cond), _f32p(mu), t, dt, _f32p(out))
        return out

    def cfm_solve(self, cond, mu, options: CfmOptions | None = None, initial_x=None):
        options = options or CfmOptions()
        cond, mu = self._inputs(cond, mu)
        out = np.empty(self.patch_floats, np.float32)
        res = abi.CfmResult()
        ix = None
        if initial_x is not None:
            ix = np.ascontiguousarray(initial_x, np.float32)
        abi.call("vx_locdit_cfm_solve", self.handle, _f32p(cond), _f32p(mu), C.byref(options.to_c()),
                 _f32p(ix) if ix is not None else None, _f32p(out), C.byref(res))
        return out, {k: getattr(res, k) for k, _ in res._fields_}

    def cfm_from_model_hiddens(self, current_lm, residual_output, cond, options: CfmOptions | None = None,
                               initial_x=None):
        """cfm_from_model_hiddens (local.rs:379-381): mu projected on the device from
        the ResidualLM engine's current_lm and output buffers (runtime.Buffer)."""
        options = options or CfmOptions()
        cond = np.ascontiguousarray(cond, np.float32)
        out = np.empty(self.patch_floats, np.float32)
        res = abi.CfmResult()
        ix = None if initial_x is None else np.ascontiguousarray(initial_x, np.float32)
        abi.call("vx_locdit_cfm_solve_from_model_hiddens", self.handle, current_lm.handle, residual_output.handle,
                 _f32p(cond), C.byref(options.to_c()), _f32p(ix) if ix is not None else None, _f32p(out),
                 C.byref(res))
        return out, {k: getattr(res, k) for k, _ in res._fields_}
