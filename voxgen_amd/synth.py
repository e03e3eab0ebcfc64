"""Synthetic VoxCPM2 BaseLM models and inputs (no checkpoints are available).

The generator (csrc/synth.c, libvoxsynth.so) is counter-based, so every value is a
function of (seed, index) and the same model is produced wherever it runs.
Distributions follow the benchmark workloads:
  Q8_0 matrices  d = f16(|N(0,1)| * 0.01), q ~ U{-127..127}
  F16 matrices   N(0, 0.02)
  token_embd     F16 N(0, 0.02)
  norm gains     F32 N(1, 0.02)
  rope factors   F32 ones (LongRoPE with ext == 1)
Tensor names, dims and dtypes are those BaseLmConfig::from_gguf validates
(baselm.rs:60-180, 227-262).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

from . import abi
from .runtime import TensorDesc, storage_bytes

LIB_PATH = Path(__file__).resolve().parent / "libvoxsynth.so"
ALIGN = 32  # GGUF default general.alignment (gguf.rs:7)

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is missing: run `python voxgen_amd/build.py`")
        L = C.CDLL(str(LIB_PATH))
        u64, f32, vp = C.c_uint64, C.c_float, C.c_void_p
        L.vs_u64.restype = u64
        L.vs_u64.argtypes = [u64, u64]
        L.vs_normal.restype = C.c_double
        L.vs_normal.argtypes = [u64, u64]
        L.vs_fill_u64.argtypes = [vp, u64, u64, u64]
        L.vs_fill_normal_f32.argtypes = [vp, u64, u64, f32, f32]
        L.vs_fill_normal_f16.argtypes = [vp, u64, u64, f32, f32]
        L.vs_fill_uniform_u32.argtypes = [vp, u64, u64, C.c_uint32]
        L.vs_fill_q8_0.argtypes = [vp, u64, u64, f32]
        _lib = L
    return _lib


def _ptr(a: np.ndarray, byte_offset: int = 0) -> C.c_void_p:
    return C.c_void_p(a.ctypes.data + byte_offset)


def derive_seed(seed: int, k: int) -> int:
    return int(lib().vs_u64(seed & 0xFFFFFFFFFFFFFFFF, k))


def normal_f32(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().vs_fill_normal_f32(_ptr(out), n, seed, mean, std)
    return out


def normal_f16(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.uint16)
    lib().vs_fill_normal_f16(_ptr(out), n, seed, mean, std)
    return out.view(np.float16)


def uniform_u32(n: int, seed: int, bound: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().vs_fill_uniform_u32(_ptr(out), n, seed, bound)
    return out


def q8_0_blocks(n_blocks: int, seed: int, scale_sigma: float = 0.01) -> np.ndarray:
    out = np.empty(n_blocks * 34, np.uint8)
    lib().vs_fill_q8_0(_ptr(out), n_blocks, seed, scale_sigma)
    return out


@dataclass
class Region:
    """A GGUF-style data region under construction."""
    tensors: list = field(default_factory=list)
    size: int = 0

    def add(self, name: str, ggml_type: int, dims: tuple) -> TensorDesc:
        off = (self.size + ALIGN - 1) // ALIGN * ALIGN
        t = TensorDesc(name, ggml_type, tuple(int(d) for d in dims), off)
        self.tensors.append(t)
        self.size = off + t.nbytes
        return t


@dataclass
class SynthModel:
    data: np.ndarray               # uint8 data region
    tensors: list                  # TensorDesc list
    config: dict                   # vx_baselm_config fields
    metadata: dict                 # GGUF metadata (key -> (gguf type, value))

    def tensor(self, name: str) -> TensorDesc:
        for t in self.tensors:
            if t.name == name:
                return t
        raise KeyError(name)

    def offset(self, name: str) -> int:
        return self.tensor(name).offset


def baselm_config(layers=28, hidden=2048, ffn=6144, vocab=73448, q_heads=16, kv_heads=2,
                  head_dim=128, context_length=32768, active_context=None, eps=1e-6,
                  theta=10000.0, original_context=None, embedding_scale=0.0,
                  residual_scale=0.0, logit_scale=0.0, tied=True) -> dict:
    """vx_baselm_config fields. Defaults give rope scaling 1 (context == original)."""
    if original_context is None:
        original_context = context_length
    return dict(context_length=context_length,
                active_context_length=active_context or min(context_length, 8192),
                embedding_length=hidden, block_count=layers, feed_forward_length=ffn,
                vocab_size=vocab, head_count=q_heads, head_count_kv=kv_heads, head_dim=head_dim,
                kv_dim=kv_heads * head_dim, rms_epsilon=eps, rope_theta=theta,
                rope_dimension_count=head_dim, rope_original_context_length=original_context,
                rope_longrope=1, embedding_scale=embedding_scale, residual_scale=residual_scale,
                logit_scale=logit_scale, tied_output=1 if tied else 0)


def build_baselm(config: dict | None = None, seed: int = 0x5EED0002, weight_type: str = "q8_0",
                 embd_type: str = "f16", q8_scale_sigma: float = 0.01, f16_std: float = 0.02,
                 with_data: bool = True, **kw) -> SynthModel:
    """Synthetic MiniCPM4 BaseLM data region with the reference tensor table."""
    cfg = dict(config or baselm_config(**kw))
    H, F, V = cfg["embedding_length"], cfg["feed_forward_length"], cfg["vocab_size"]
    KV, L, hd = cfg["kv_dim"], cfg["block_count"], cfg["head_dim"]
    wt = abi.DTYPE_Q8_0 if weight_type == "q8_0" else abi.DTYPE_F16
    et = abi.DTYPE_Q8_0 if embd_type == "q8_0" else abi.DTYPE_F16
    reg = Region()
    reg.add("token_embd.weight", et, (H, V))
    reg.add("output_norm.weight", abi.DTYPE_F32, (H,))
    reg.add("rope_factors_short.weight", abi.DTYPE_F32, (hd // 2,))
    reg.add("rope_factors_long.weight", abi.DTYPE_F32, (hd // 2,))
    if not cfg.get("tied_output", 1):
        reg.add("output.weight", et, (H, V))
    for l in range(L):
        p = f"blk.{l}."
        reg.add(p + "attn_norm.weight", abi.DTYPE_F32, (H,))
        reg.add(p + "attn_q.weight", wt, (H, H))
        reg.add(p + "attn_k.weight", wt, (H, KV))
        reg.add(p + "attn_v.weight", wt, (H, KV))
        reg.add(p + "attn_output.weight", wt, (H, H))
        reg.add(p + "ffn_norm.weight", abi.DTYPE_F32, (H,))
        reg.add(p + "ffn_gate.weight", wt, (H, F))
        reg.add(p + "ffn_up.weight", wt, (H, F))
        reg.add(p + "ffn_down.weight", wt, (F, H))
    size = (reg.size + 255) // 256 * 256
    data = np.zeros(size if with_data else 0, np.uint8)
    if with_data:
        for i, t in enumerate(reg.tensors):
            s = derive_seed(seed, i)
            n = int(np.prod(t.dims))
            if t.ggml_type == abi.DTYPE_Q8_0:
                lib().vs_fill_q8_0(_ptr(data, t.offset), n // 32, s, q8_scale_sigma)
            elif t.name.startswith("rope_factors"):
                data[t.offset:t.offset + t.nbytes].view(np.float32)[:] = 1.0
            elif t.ggml_type == abi.DTYPE_F32:
                lib().vs_fill_normal_f32(_ptr(data, t.offset), n, s, 1.0, 0.02)
            else:
                std = 0.02 if t.name in ("token_embd.weight", "output.weight") else f16_std
                lib().vs_fill_normal_f16(_ptr(data, t.offset), n, s, 0.0, std)
    meta = gguf_metadata(cfg)
    return SynthModel(data, reg.tensors, cfg, meta)


def gguf_metadata(cfg: dict) -> dict:
    """Metadata BaseLmConfig::from_gguf reads (baselm.rs:60-99), as (gguf type, value)."""
    U32, F32, STR = 4, 6, 8
    m = {
        "general.architecture": (STR, "minicpm4"),
        "general.alignment": (U32, ALIGN),
        "minicpm4.context_length": (U32, cfg["context_length"]),
        "minicpm4.embedding_length": (U32, cfg["embedding_length"]),
        "minicpm4.block_count": (U32, cfg["block_count"]),
        "minicpm4.feed_forward_length": (U32, cfg["feed_forward_length"]),
        "minicpm4.attention.head_count": (U32, cfg["head_count"]),
        "minicpm4.attention.head_count_kv": (U32, cfg["head_count_kv"]),
        "minicpm4.attention.key_length": (U32, cfg["head_dim"]),
        "minicpm4.rope.dimension_count": (U32, cfg["rope_dimension_count"]),
        "minicpm4.attention.layer_norm_rms_epsilon": (F32, cfg["rms_epsilon"]),
        "minicpm4.rope.freq_base": (F32, cfg["rope_theta"]),
        "minicpm4.rope.scaling.type": (STR, "longrope" if cfg["rope_longrope"] else "none"),
        "minicpm4.rope.scaling.original_context_length": (U32, cfg["rope_original_context_length"]),
    }
    for k in ("embedding_scale", "residual_scale", "logit_scale"):
        if cfg.get(k):
            m["minicpm4." + k] = (F32, cfg[k])
    return m


def kv_cache_fill(layers: int, context: int, kv_dim: int, filled: int, seed: int) -> np.ndarray:
    """Packed f16 cache [layer][context][kv_dim] with N(0,1) in positions < filled."""
    c = np.zeros((layers, context, kv_dim), np.float16)
    if filled:
        v = normal_f16(layers * filled * kv_dim, seed).reshape(layers, filled, kv_dim)
        c[:, :filled, :] = v
    return c


def locdit_config(layers=12, hidden=1024, q_heads=16, kv_heads=2, head_dim=128, ffn=4096, feat_dim=64,
                  patch=4, n_mu=2, n_cond=None, cond_raw=0, uncond_zero_cond=0, eps=1e-6, theta=10000.0,
                  rope_scaling=1.0) -> dict:
    """vx_locdit_config fields. Defaults are the VoxCPM2 LocDiT contract
    (LocalConfig::from_gguf, local.rs:85-92): 12 x 1024, 16/2 x 128, ffn 4096,
    patch 4 x 64, mu1 + mu2 + time + 4 condition + 4 latent tokens."""
    return dict(hidden=hidden, layers=layers, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, ffn=ffn,
                feat_dim=feat_dim, patch=patch, n_mu=n_mu, n_cond=patch if n_cond is None else n_cond,
                cond_raw=cond_raw, uncond_zero_cond=uncond_zero_cond, rms_epsilon=eps, rope_theta=theta,
                rope_scaling=rope_scaling)


def build_locdit(cfg: dict, seed: int = 0x5EED0040, std: float = 0.02, with_mu_proj: bool = True) -> SynthModel:
    """Synthetic LocDiT tensors with the names and shapes validate_tensors checks
    (local.rs:127-168): F16 matrices N(0, std), F32 biases N(0, std), F32 norm
    gains N(1, 0.02), plus rope_factors_short.weight (ones) so the same region
    can serve as the RoPE-factor model."""
    H, F, hd = cfg["hidden"], cfg["ffn"], cfg["head_dim"]
    QD, KD, FD = cfg["q_heads"] * hd, cfg["kv_heads"] * hd, cfg["feat_dim"]
    reg = Region()
    reg.add("rope_factors_short.weight", abi.DTYPE_F32, (hd // 2,))

    def lin(name, cols, rows):
        reg.add(name + ".weight", abi.DTYPE_F16, (cols, rows))
        reg.add(name + ".bias", abi.DTYPE_F32, (rows,))

    lin("locdit.in_proj", FD, H)
    if not cfg["cond_raw"]:
        lin("locdit.cond_proj", FD, H)
    lin("locdit.out_proj", H, FD)
    reg.add("locdit.norm.weight", abi.DTYPE_F32, (H,))
    for p in ("locdit.time_mlp", "locdit.delta_time_mlp"):
        lin(p + ".linear_1", H, H)
        lin(p + ".linear_2", H, H)
    for l in range(cfg["layers"]):
        p = f"locdit.blk.{l}."
        reg.add(p + "attn_norm.weight", abi.DTYPE_F32, (H,))
        reg.add(p + "attn_q.weight", abi.DTYPE_F16, (H, QD))
        reg.add(p + "attn_k.weight", abi.DTYPE_F16, (H, KD))
        reg.add(p + "attn_v.weight", abi.DTYPE_F16, (H, KD))
        reg.add(p + "attn_output.weight", abi.DTYPE_F16, (QD, H))
        reg.add(p + "ffn_norm.weight", abi.DTYPE_F32, (H,))
        reg.add(p + "ffn_gate.weight", abi.DTYPE_F16, (H, F))
        reg.add(p + "ffn_up.weight", abi.DTYPE_F16, (H, F))
        reg.add(p + "ffn_down.weight", abi.DTYPE_F16, (F, H))
    # The mu projections from the ResidualLM engine's buffers (local.rs:141-144),
    # appended so that the tensors above keep their seeds.
    if with_mu_proj:
        lin("projections.lm_to_dit_proj", cfg.get("lm_hidden", 2048), H)
        lin("projections.res_to_dit_proj", cfg.get("lm_hidden", 2048), H)
    data = np.zeros((reg.size + 255) // 256 * 256, np.uint8)
    for i, t in enumerate(reg.tensors):
        s = derive_seed(seed, i)
        n = int(np.prod(t.dims))
        if t.name.startswith("rope_factors"):
            data[t.offset:t.offset + t.nbytes].view(np.float32)[:] = 1.0
        elif t.ggml_type == abi.DTYPE_F16:
            lib().vs_fill_normal_f16(_ptr(data, t.offset), n, s, 0.0, std)
        elif t.name.endswith("norm.weight"):
            lib().vs_fill_normal_f32(_ptr(data, t.offset), n, s, 1.0, 0.02)
        else:
            lib().vs_fill_normal_f32(_ptr(data, t.offset), n, s, 0.0, std)
    return SynthModel(data, reg.tensors, dict(cfg), {})


def acoustic_config(layers=8, hidden=2048, ffn=6144, q_heads=16, kv_heads=2, head_dim=128, latent=512,
                    fsq_scale=9.0, active_context=512, eps=1e-6, residual_scale=1.0) -> dict:
    """vx_acoustic_config fields. Defaults are the VoxCPM2 contract
    (AcousticConfig::from_gguf, acoustic.rs:83-103): 8 residual layers over the
    2048/6144/16/2/128 BaseLM geometry, FSQ latent 512, no RoPE."""
    return dict(model_version=2.0, residual_block_count=layers, embedding_length=hidden, feed_forward_length=ffn,
                head_count=q_heads, head_count_kv=kv_heads, head_dim=head_dim, kv_dim=kv_heads * head_dim,
                no_rope=1, active_context_length=active_context, rms_epsilon=eps, residual_scale=residual_scale,
                fsq_latent_dim=latent, fsq_scale=fsq_scale, fusion_input_dim=2 * hidden)


def build_acoustic(cfg: dict, seed: int = 0x5EED0060, std: float = 0.02, bias_f32_stop: bool = True,
                   with_data: bool = True) -> SynthModel:
    """Synthetic ResidualLM / FSQ / fusion / stop-predictor tensors with the names,
    shapes and dtypes validate_tensors checks (acoustic.rs:127-174): F16 matrices
    N(0, std), F16 biases N(0, std) (the stop predictor's linear1 bias F32 when
    bias_f32_stop), F32 norm gains N(1, 0.02)."""
    H, F, L = cfg["embedding_length"], cfg["feed_forward_length"], cfg["fsq_latent_dim"]
    KV = cfg["kv_dim"]
    reg = Region()
    f16, f32 = abi.DTYPE_F16, abi.DTYPE_F32
    reg.add("fsq.in_proj.weight", f16, (H, L))
    reg.add("fsq.in_proj.bias", f16, (L,))
    reg.add("fsq.out_proj.weight", f16, (L, H))
    reg.add("fsq.out_proj.bias", f16, (H,))
    reg.add("projections.res_fusion_proj.weight", f16, (2 * H, H))
    reg.add("projections.res_fusion_proj.bias", f16, (H,))
    reg.add("residual_lm.output_norm.weight", f32, (H,))
    for l in range(cfg["residual_block_count"]):
        p = f"residual_lm.blk.{l}."
        reg.add(p + "attn_norm.weight", f32, (H,))
        reg.add(p + "attn_q.weight", f16, (H, H))
        reg.add(p + "attn_k.weight", f16, (H, KV))
        reg.add(p + "attn_v.weight", f16, (H, KV))
        reg.add(p + "attn_output.weight", f16, (H, H))
        reg.add(p + "ffn_norm.weight", f32, (H,))
        reg.add(p + "ffn_gate.weight", f16, (H, F))
        reg.add(p + "ffn_up.weight", f16, (H, F))
        reg.add(p + "ffn_down.weight", f16, (F, H))
    reg.add("stop_predictor.linear1.weight", f16, (H, H))
    reg.add("stop_predictor.linear1.bias", f32 if bias_f32_stop else f16, (H,))
    reg.add("stop_predictor.linear2.weight", f16, (H, 2))
    data = np.zeros((reg.size + 255) // 256 * 256 if with_data else 0, np.uint8)
    if with_data:
        for i, t in enumerate(reg.tensors):
            s = derive_seed(seed, i)
            n = int(np.prod(t.dims))
            if t.name.endswith("norm.weight"):
                lib().vs_fill_normal_f32(_ptr(data, t.offset), n, s, 1.0, 0.02)
            elif t.ggml_type == f16:
                lib().vs_fill_normal_f16(_ptr(data, t.offset), n, s, 0.0, std)
            else:
                lib().vs_fill_normal_f32(_ptr(data, t.offset), n, s, 0.0, std)
    return SynthModel(data, reg.tensors, dict(cfg), acoustic_metadata(cfg))


def acoustic_metadata(cfg: dict) -> dict:
    """Metadata AcousticConfig::from_gguf reads (acoustic.rs:64-82)."""
    U32, F32, STR, BOOL = 4, 6, 8, 7
    return {
        "general.architecture": (STR, "voxcpm-acoustic"),
        "general.alignment": (U32, ALIGN),
        "voxcpm.model_version": (F32, cfg["model_version"]),
        "voxcpm.residual_lm.n_layer": (U32, cfg["residual_block_count"]),
        "voxcpm.residual_lm.n_embd": (U32, cfg["embedding_length"]),
        "voxcpm.residual_lm.no_rope": (BOOL, bool(cfg["no_rope"])),
        "voxcpm.fsq.latent_dim": (U32, cfg["fsq_latent_dim"]),
        "voxcpm.fsq.scale": (F32, cfg["fsq_scale"]),
    }


def audiovae_config(decoder_dim=2048, latent=64, encoder_dim=128, bucket=3) -> dict:
    """vx_audiovae_config fields. Defaults are the VoxCPM2 AudioVAE V2 contract
    (AudioVaeConfig::from_gguf, audiovae.rs:49-79)."""
    enc, dec = [2, 5, 8, 8], [8, 6, 5, 2, 2, 2]
    return dict(encoder_dim=encoder_dim, latent_dim=latent, decoder_dim=decoder_dim, sample_rate=16000,
                out_sample_rate=48000, encoder_rates=enc, decoder_rates=dec, encoder_hop=640, decoder_hop=1920,
                patch_size=4, input_samples_per_patch=2560, output_samples_per_patch=7680,
                sr_bin_boundaries=[20000, 30000, 40000], decoder_sr_bucket=bucket, depthwise=1)


def build_audiovae(cfg: dict, seed: int = 0x5EED0080, encoder: bool = False, with_data: bool = True) -> SynthModel:
    """Synthetic AudioVAE tensors with the names, shapes and F16 dtype that
    validate_tensors checks (audiovae.rs:81-128); the encoder's only with
    `encoder`. Conv weights N(0, 1/sqrt(fan-in)) (x0.3 for the residual units'
    1x1 convolutions, x0.1 for the output convolution, so the decoder's
    activations stay O(1) and tanh unsaturated), biases N(0, 0.02), snake alphas
    N(1, 0.1), sample-rate scale N(1, 0.05) and bias N(0, 0.02)."""
    f16 = abi.DTYPE_F16
    reg = Region()
    std = {}

    def conv(base, in_c, out_c, k, groups, transpose=False, gain=1.0):
        dims = (k, out_c // groups, in_c) if transpose else (k, in_c // groups, out_c)
        reg.add(base, f16, dims)
        std[base] = (0.0, gain / np.sqrt(2.0 * in_c if transpose else (in_c // groups) * k))
        reg.add(base + ".bias", f16, (out_c,))
        std[base + ".bias"] = (0.0, 0.02)

    def alpha(name, c):
        reg.add(name, f16, (1, c, 1))
        std[name] = (1.0, 0.1)

    if encoder:
        conv("audio_vae.encoder.block.0", 1, cfg["encoder_dim"], 7, 1)
        c = cfg["encoder_dim"]
        for stage, s in enumerate(cfg["encoder_rates"]):
            b = f"audio_vae.encoder.block.{stage + 1}"
            for ri in range(3):
                p = f"{b}.block.{ri}.block"
                alpha(p + ".0.alpha", c)
                conv(p + ".1", c, c, 7, c)
                alpha(p + ".2.alpha", c)
                conv(p + ".3", c, c, 1, 1)
            alpha(b + ".block.3.alpha", c)
            conv(b + ".block.4", c, 2 * c, 2 * s, 1)
            c *= 2
        conv("audio_vae.encoder.fc_mu", c, cfg["latent_dim"], 3, 1)
        conv("audio_vae.encoder.fc_logvar", c, cfg["latent_dim"], 3, 1)
    L = cfg["latent_dim"]
    conv("audio_vae.decoder.model.0", L, L, 7, L)
    conv("audio_vae.decoder.model.1", L, cfg["decoder_dim"], 1, 1)
    din = cfg["decoder_dim"]
    for i, s in enumerate(cfg["decoder_rates"]):
        mi, dout = i + 2, din // 2
        for kind, ms in (("scale_embed", (1.0, 0.05)), ("bias_embed", (0.0, 0.02))):
            name = f"audio_vae.decoder.sr_cond_model.{mi}.{kind}"
            reg.add(name, f16, (din, 4))
            std[name] = ms
        p = f"audio_vae.decoder.model.{mi}"
        alpha(p + ".block.0.alpha", din)
        conv(p + ".block.1", din, dout, 2 * s, 1, transpose=True)
        for rj in range(3):
            q = f"{p}.block.{rj + 2}.block"
            alpha(q + ".0.alpha", dout)
            conv(q + ".1", dout, dout, 7, dout)
            alpha(q + ".2.alpha", dout)
            conv(q + ".3", dout, dout, 1, 1, gain=0.3)
        din = dout
    alpha("audio_vae.decoder.model.8.alpha", din)
    conv("audio_vae.decoder.model.9", din, 1, 7, 1, gain=0.1)
    data = np.zeros((reg.size + 255) // 256 * 256 if with_data else 0, np.uint8)
    if with_data:
        for i, t in enumerate(reg.tensors):
            mean, sd = std[t.name]
            lib().vs_fill_normal_f16(_ptr(data, t.offset), int(np.prod(t.dims)), derive_seed(seed, i), mean, sd)
    meta = {
        "general.architecture": (8, "voxcpm-acoustic"),
        "general.alignment": (4, ALIGN),
        "voxcpm.model_version": (6, 2.0),
        "voxcpm.patch_size": (4, cfg["patch_size"]),
        "voxcpm.audiovae.encoder_dim": (4, cfg["encoder_dim"]),
        "voxcpm.audiovae.latent_dim": (4, cfg["latent_dim"]),
        "voxcpm.audiovae.decoder_dim": (4, cfg["decoder_dim"]),
        "voxcpm.audiovae.sample_rate": (4, cfg["sample_rate"]),
        "voxcpm.audiovae.out_sample_rate": (4, cfg["out_sample_rate"]),
        "voxcpm.audiovae.cond_type": (8, "scale_bias"),
    }
    return SynthModel(data, reg.tensors, dict(cfg), meta)
