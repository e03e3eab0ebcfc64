"""ctypes wrapper of liboracle.so, the CPU oracle (voxref.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker or the timed CPU baseline. It is
never a product path.
"""
from __future__ import annotations

import ctypes as C
import subprocess
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
from voxgen_amd import abi  # noqa: E402  (push struct layouts)

LIB_PATH = HERE / "liboracle.so"
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        vp, u32, f32 = C.c_void_p, C.c_uint32, C.c_float
        P = C.POINTER
        L.vr_f16_to_f32.restype = f32
        L.vr_f16_to_f32.argtypes = [C.c_uint16]
        L.vr_f32_to_f16.restype = C.c_uint16
        L.vr_f32_to_f16.argtypes = [f32]
        L.vr_f16_to_f32_n.argtypes = [vp, vp, C.c_uint64]
        L.vr_f32_to_f16_n.argtypes = [vp, vp, C.c_uint64]
        L.vr_dequant.argtypes = [vp, u32, u32, u32, u32, vp]
        L.vr_embedding.argtypes = [vp, vp, P(abi.EmbeddingPush)]
        L.vr_rmsnorm.argtypes = [vp, vp, vp, P(abi.RmsPush)]
        L.vr_residual_rmsnorm.argtypes = [vp, vp, vp, vp, P(abi.ResidualRmsPush)]
        L.vr_matvec.argtypes = [vp, vp, vp, P(abi.MatvecPush)]
        L.vr_qkv_matvec.argtypes = [vp, vp, vp, vp, vp, P(abi.QkvPush)]
        L.vr_matvec_swiglu.argtypes = [vp, vp, vp, P(abi.SwigluPush)]
        L.vr_rope.argtypes = [vp, vp, vp, P(abi.RopePush)]
        L.vr_store_kv.argtypes = [vp, vp, vp, vp, P(abi.StoreKvPush)]
        L.vr_attn_scores.argtypes = [vp, vp, vp, u32, P(abi.AttentionPush)]
        L.vr_softmax.argtypes = [vp, u32, P(abi.SoftmaxPush)]
        L.vr_attn_values.argtypes = [vp, vp, vp, u32, P(abi.AttentionPush)]
        L.vr_linear_bias.argtypes = [vp, vp, vp, P(abi.LinearBiasPush)]
        L.vr_fusion_linear.argtypes = [vp, vp, vp, vp, vp, P(abi.FusionPush)]
        L.vr_baselm_record.argtypes = [vp, vp, vp, u32, C.c_int]
        L.vr_baselm_decode_token.argtypes = [vp, vp, vp, u32, u32, C.c_int]
        L.vr_rope_scaling_factor.restype = f32
        L.vr_rope_scaling_factor.argtypes = [P(abi.BaseLmConfig)]
        L.vr_effective_scale.restype = f32
        L.vr_effective_scale.argtypes = [f32]
        L.vr_mix32.restype = u32
        L.vr_mix32.argtypes = [u32]
        L.vr_cfm_noise.argtypes = [vp, P(abi.CfmNoisePush)]
        L.vr_cfm_cfg_euler.argtypes = [vp, vp, vp, P(abi.CfmEulerPush)]
        L.vr_time_sinusoidal.argtypes = [vp, P(abi.TimePush)]
        L.vr_pack_locdit.argtypes = [vp, vp, vp, vp, vp, vp, P(abi.PackLocDitPush)]
        L.vr_cfm_time_span.restype = C.c_int
        L.vr_cfm_time_span.argtypes = [u32, f32, vp]
        L.vr_residual_lm_record.argtypes = [vp, vp, vp, u32]
        L.vr_fsq_quantize.argtypes = [vp, u32, f32]
        L.vr_silu_inplace.argtypes = [vp, u32]
        L.vr_vae_conv1d.argtypes = [vp, vp, vp, P(abi.VaeConvPush)]
        L.vr_vae_convt1d.argtypes = [vp, vp, vp, P(abi.VaeConvTPush)]
        L.vr_vae_snake.argtypes = [vp, vp, vp, P(abi.VaeSnakePush)]
        L.vr_vae_scale_bias.argtypes = [vp, vp, P(abi.VaeScalePush)]
        L.vr_vae_add.argtypes = [vp, vp, P(abi.VaeGridPush)]
        L.vr_vae_tanh.argtypes = [vp, u32]
        L.vr_set_threads.argtypes = [C.c_int]
        L.vr_get_threads.restype = C.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray) -> C.c_void_p:
    assert a.flags.c_contiguous
    return C.c_void_p(a.ctypes.data)


def f32(n) -> np.ndarray:
    return np.zeros(n, np.float32)


def set_threads(n: int) -> None:
    lib().vr_set_threads(n)


def threads() -> int:
    return lib().vr_get_threads()


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.size, np.float32)
    lib().vr_f16_to_f32_n(_p(b), _p(out), b.size)
    return out


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(a.size, np.uint16)
    lib().vr_f32_to_f16_n(_p(a), _p(out), a.size)
    return out


def dequant(blob: np.ndarray, offset: int, dtype: int, rows: int, cols: int) -> np.ndarray:
    out = np.empty(rows * cols, np.float32)
    lib().vr_dequant(_p(blob), offset, dtype, rows, cols, _p(out))
    return out.reshape(rows, cols)


def embedding(blob, push: abi.EmbeddingPush) -> np.ndarray:
    h = f32(push.cols)
    lib().vr_embedding(_p(blob), _p(h), C.byref(push))
    return h


def rmsnorm(blob, x, push: abi.RmsPush) -> np.ndarray:
    y = f32(push.n)
    x_c = np.ascontiguousarray(x, np.float32)  # held across the call
    lib().vr_rmsnorm(_p(blob), _p(x_c), _p(y), C.byref(push))
    return y


def residual_rmsnorm(blob, hidden, branch, push: abi.ResidualRmsPush):
    h = np.array(hidden, np.float32, copy=True)
    y = f32(push.n)
    branch_c = np.ascontiguousarray(branch, np.float32)  # held across the call
    lib().vr_residual_rmsnorm(_p(blob), _p(h), _p(branch_c), _p(y),
                              C.byref(push))
    return h, y


def matvec(blob, x, push: abi.MatvecPush, y=None) -> np.ndarray:
    y = f32(push.rows) if y is None else y
    x_c = np.ascontiguousarray(x, np.float32)  # held across the call
    lib().vr_matvec(_p(blob), _p(x_c), _p(y), C.byref(push))
    return y


def qkv_matvec(blob, x, push: abi.QkvPush):
    q, k, v = f32(push.q_rows), f32(push.kv_rows), f32(push.kv_rows)
    x_c = np.ascontiguousarray(x, np.float32)  # held across the call
    lib().vr_qkv_matvec(_p(blob), _p(x_c), _p(q), _p(k), _p(v),
                        C.byref(push))
    return q, k, v


def matvec_swiglu(blob, x, push: abi.SwigluPush) -> np.ndarray:
    y = f32(push.rows)
    x_c = np.ascontiguousarray(x, np.float32)  # held across the call
    lib().vr_matvec_swiglu(_p(blob), _p(x_c), _p(y), C.byref(push))
    return y


def rope(blob, q, k, push: abi.RopePush):
    q2 = np.array(q, np.float32, copy=True)
    k2 = np.array(k, np.float32, copy=True)
    lib().vr_rope(_p(blob), _p(q2), _p(k2), C.byref(push))
    return q2, k2


def store_kv(k, v, k_cache: np.ndarray, v_cache: np.ndarray, push: abi.StoreKvPush) -> None:
    """k_cache/v_cache: uint16 (f16 bits) arrays updated in place."""
    k_c = np.ascontiguousarray(k, np.float32)  # held across the call
    v_c = np.ascontiguousarray(v, np.float32)  # held across the call
    lib().vr_store_kv(_p(k_c), _p(v_c),
                      _p(k_cache), _p(v_cache), C.byref(push))


def attn_scores(q, k_cache, q_heads: int, push: abi.AttentionPush) -> np.ndarray:
    s = f32(q_heads * push.context)
    q_c = np.ascontiguousarray(q, np.float32)  # held across the call
    lib().vr_attn_scores(_p(q_c), _p(k_cache), _p(s), q_heads, C.byref(push))
    return s


def softmax(scores, heads: int, push: abi.SoftmaxPush) -> np.ndarray:
    s = np.array(scores, np.float32, copy=True)
    lib().vr_softmax(_p(s), heads, C.byref(push))
    return s


def attn_values(scores, v_cache, q_heads: int, push: abi.AttentionPush) -> np.ndarray:
    o = f32(q_heads * push.head_dim)
    scores_c = np.ascontiguousarray(scores, np.float32)  # held across the call
    lib().vr_attn_values(_p(scores_c), _p(v_cache), _p(o), q_heads,
                         C.byref(push))
    return o


def linear_bias(blob, x, push: abi.LinearBiasPush) -> np.ndarray:
    y = f32(push.rows)
    x_c = np.ascontiguousarray(x, np.float32)  # held across the call
    lib().vr_linear_bias(_p(blob), _p(x_c), _p(y), C.byref(push))
    return y


def fusion_linear(blob, left, right, push: abi.FusionPush):
    y, s = f32(push.rows), f32(push.rows)
    r = np.ascontiguousarray(right if right is not None else np.zeros(1), np.float32)
    left_c = np.ascontiguousarray(left, np.float32)  # held across the call
    lib().vr_fusion_linear(_p(blob), _p(left_c), _p(r), _p(y), _p(s),
                           C.byref(push))
    return y, s


def rope_scaling_factor(cfg: dict) -> float:
    from voxgen_amd.baselm import config_struct
    return lib().vr_rope_scaling_factor(C.byref(config_struct(cfg)))


def effective_scale(v: float) -> float:
    return lib().vr_effective_scale(v)


# ------------------------------------------------------------- whole model
class _Layer(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in (
        "attn_norm", "ffn_norm", "q", "k", "v", "o", "gate", "up", "down",
        "q_dtype", "k_dtype", "v_dtype", "o_dtype", "gate_dtype", "up_dtype", "down_dtype")]


class _BaseLm(C.Structure):
    _fields_ = [("cfg", abi.BaseLmConfig), ("token_embd", C.c_uint32), ("token_embd_dtype", C.c_uint32),
                ("output", C.c_uint32), ("output_dtype", C.c_uint32), ("output_norm", C.c_uint32),
                ("rope_factors", C.c_uint32), ("layers", C.POINTER(_Layer))]


class _State(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("hidden", "norm", "q", "k", "v", "attention", "gate",
                                          "branch", "logits", "scores", "kv_k", "kv_v")]


class BaseLm:
    """record_transformer on the CPU over a SynthModel-like (data, tensors, config)."""

    def __init__(self, data: np.ndarray, tensors: dict, cfg: dict):
        from voxgen_amd.baselm import config_struct
        self.blob = np.ascontiguousarray(data, dtype=np.uint8)
        if self.blob.size % 4:
            self.blob = np.concatenate([self.blob, np.zeros(4 - self.blob.size % 4, np.uint8)])
        self.cfg = dict(cfg)
        t = tensors
        L = cfg["block_count"]
        self._layers = (_Layer * L)()
        for l in range(L):
            p = f"blk.{l}."
            ly = self._layers[l]
            for fld, name in (("attn_norm", "attn_norm"), ("ffn_norm", "ffn_norm"), ("q", "attn_q"),
                              ("k", "attn_k"), ("v", "attn_v"), ("o", "attn_output"),
                              ("gate", "ffn_gate"), ("up", "ffn_up"), ("down", "ffn_down")):
                tt = t[p + name + ".weight"]
                setattr(ly, fld, tt.offset)
                if fld not in ("attn_norm", "ffn_norm"):
                    setattr(ly, fld + "_dtype", tt.ggml_type)
        m = _BaseLm()
        m.cfg = config_struct(cfg)
        emb = t["token_embd.weight"]
        out = t.get("output.weight", emb)
        m.token_embd, m.token_embd_dtype = emb.offset, emb.ggml_type
        m.output, m.output_dtype = out.offset, out.ggml_type
        m.output_norm = t["output_norm.weight"].offset
        long = cfg["context_length"] > cfg["rope_original_context_length"]
        m.rope_factors = t["rope_factors_long.weight" if long else "rope_factors_short.weight"].offset
        m.layers = C.cast(self._layers, C.POINTER(_Layer))
        self._m = m
        H, KV, F, V = cfg["embedding_length"], cfg["kv_dim"], cfg["feed_forward_length"], cfg["vocab_size"]
        ctx = cfg["active_context_length"]
        self.hidden, self.norm, self.q = f32(H), f32(H), f32(H)
        self.k, self.v, self.attention = f32(KV), f32(KV), f32(H)
        self.gate, self.branch, self.logits = f32(F), f32(H), f32(V)
        self.scores = f32(cfg["head_count"] * ctx)
        self.kv_k = np.zeros(L * ctx * KV, np.uint16)
        self.kv_v = np.zeros(L * ctx * KV, np.uint16)
        s = _State()
        for n, _ in _State._fields_:
            setattr(s, n, _p(getattr(self, n)))
        self._s = s

    def decode_token(self, token: int, position: int, logits: bool = False) -> np.ndarray:
        lib().vr_baselm_decode_token(_p(self.blob), C.byref(self._m), C.byref(self._s), token, position,
                                     1 if logits else 0)
        return self.norm.copy()

    def record(self, position: int, logits: bool = False) -> np.ndarray:
        """record_transformer from the current hidden state."""
        lib().vr_baselm_record(_p(self.blob), C.byref(self._m), C.byref(self._s), position,
                               1 if logits else 0)
        return self.norm.copy()


def fsq_quantize(x, scale: float) -> np.ndarray:
    """fsq_quantize.comp."""
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().vr_fsq_quantize(_p(y), y.size, scale)
    return y


def silu_inplace(x) -> np.ndarray:
    """silu_inplace.comp."""
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().vr_silu_inplace(_p(y), y.size)
    return y


class ResidualFsq:
    """ResidualFsqEngine (acoustic.rs:400-1035) on the CPU over a SynthModel-like
    (data, tensors, acoustic config): FSQ, fusion, record_residual_lm and the stop
    predictor from the per-op functions, with its own f16 KV cache."""

    def __init__(self, data: np.ndarray, tensors: dict, acfg: dict):
        self.blob = np.ascontiguousarray(data, dtype=np.uint8)
        if self.blob.size % 4:
            self.blob = np.concatenate([self.blob, np.zeros(4 - self.blob.size % 4, np.uint8)])
        self.cfg, self.t = dict(acfg), tensors
        L, H = acfg["residual_block_count"], acfg["embedding_length"]
        KV, F, ctx = acfg["kv_dim"], acfg["feed_forward_length"], acfg["active_context_length"]
        self._layers = (_Layer * L)()
        for l in range(L):
            p = f"residual_lm.blk.{l}."
            ly = self._layers[l]
            for fld, name in (("attn_norm", "attn_norm"), ("ffn_norm", "ffn_norm"), ("q", "attn_q"),
                              ("k", "attn_k"), ("v", "attn_v"), ("o", "attn_output"),
                              ("gate", "ffn_gate"), ("up", "ffn_up"), ("down", "ffn_down")):
                tt = tensors[p + name + ".weight"]
                setattr(ly, fld, tt.offset)
                if fld not in ("attn_norm", "ffn_norm"):
                    setattr(ly, fld + "_dtype", tt.ggml_type)
        m = _BaseLm()
        c = m.cfg
        c.context_length = c.active_context_length = ctx
        c.embedding_length, c.block_count, c.feed_forward_length = H, L, F
        c.head_count, c.head_count_kv = acfg["head_count"], acfg["head_count_kv"]
        c.head_dim, c.kv_dim = acfg["head_dim"], KV
        c.rms_epsilon, c.residual_scale = acfg["rms_epsilon"], acfg["residual_scale"]
        m.output_norm = tensors["residual_lm.output_norm.weight"].offset
        m.layers = C.cast(self._layers, C.POINTER(_Layer))
        self._m = m
        self.hidden, self.norm, self.q = f32(H), f32(H), f32(H)
        self.k, self.v, self.attention = f32(KV), f32(KV), f32(H)
        self.gate, self.branch, self.logits = f32(F), f32(H), f32(1)
        self.scores = f32(acfg["head_count"] * ctx)
        self.kv_k = np.zeros(L * ctx * KV, np.uint16)
        self.kv_v = np.zeros(L * ctx * KV, np.uint16)
        st = _State()
        for n, _ in _State._fields_:
            setattr(st, n, _p(getattr(self, n)))
        self._s = st
        self.current_lm = f32(H)

    def _lin(self, prefix, x, rows, cols):
        w, b = self.t[prefix + ".weight"], self.t[prefix + ".bias"]
        return linear_bias(self.blob, x, abi.LinearBiasPush(w.offset, b.offset, rows, cols, w.ggml_type,
                                                            b.ggml_type, 0, 1.0))

    def fsq(self, base):
        """record_fsq (acoustic.rs:909-939): (quantized latent, output)."""
        H, Ld = self.cfg["embedding_length"], self.cfg["fsq_latent_dim"]
        latent = fsq_quantize(self._lin("fsq.in_proj", base, Ld, H), self.cfg["fsq_scale"])
        return latent, self._lin("fsq.out_proj", latent, H, Ld)

    def step(self, base, embedding, position: int, fsq: bool = True) -> dict:
        """step_record_submit (acoustic.rs:847-893): FSQ (or the raw text-prefix
        state), current_lm, fusion, record_residual_lm at `position`."""
        H = self.cfg["embedding_length"]
        base = np.ascontiguousarray(base, dtype=np.float32)
        out = {}
        if fsq:
            out["latent"], left = self.fsq(base)
            out["fsq"] = left
            right = np.ascontiguousarray(embedding, dtype=np.float32)
        else:
            left, right = base, np.zeros(H, np.float32)
        self.current_lm = left.copy()
        w, b = self.t["projections.res_fusion_proj.weight"], self.t["projections.res_fusion_proj.bias"]
        fused, _ = fusion_linear(self.blob, left, right, abi.FusionPush(w.offset, b.offset, H, H, H, w.ggml_type,
                                                                     b.ggml_type, 0))
        out["fused"] = fused.copy()
        self.hidden[:] = fused
        lib().vr_residual_lm_record(_p(self.blob), C.byref(self._m), C.byref(self._s), position)
        out["norm"] = self.norm.copy()
        return out

    def stop(self, x):
        """predict_stop_* (acoustic.rs:619-652): the two logits (continue, stop)."""
        H = self.cfg["embedding_length"]
        h = silu_inplace(self._lin("stop_predictor.linear1", x, H, H))
        w = self.t["stop_predictor.linear2.weight"]
        return matvec(self.blob, h, abi.MatvecPush(w.offset, 2, H, w.ggml_type, 0, 1.0))


def _dt(t) -> int:
    return 1 if t.ggml_type == abi.DTYPE_F16 else 0


def vae_conv1d(blob, x, push: abi.VaeConvPush) -> np.ndarray:
    xc = np.ascontiguousarray(x, np.float32)
    y = f32(push.out_channels * push.out_length)
    lib().vr_vae_conv1d(_p(blob), _p(xc), _p(y), C.byref(push))
    return y


def vae_convt1d(blob, x, push: abi.VaeConvTPush) -> np.ndarray:
    xc = np.ascontiguousarray(x, np.float32)
    y = f32(push.out_channels * push.out_length)
    lib().vr_vae_convt1d(_p(blob), _p(xc), _p(y), C.byref(push))
    return y


def vae_snake(blob, x, push: abi.VaeSnakePush) -> np.ndarray:
    xc = np.ascontiguousarray(x, np.float32)
    y = f32(xc.size)
    lib().vr_vae_snake(_p(blob), _p(xc), _p(y), C.byref(push))
    return y


def vae_scale_bias(blob, x, push: abi.VaeScalePush) -> np.ndarray:
    y = np.ascontiguousarray(x, np.float32).copy()
    lib().vr_vae_scale_bias(_p(blob), _p(y), C.byref(push))
    return y


def vae_tanh(x) -> np.ndarray:
    y = np.ascontiguousarray(x, np.float32).copy()
    lib().vr_vae_tanh(_p(y), y.size)
    return y


class AudioVae:
    """AudioVaeEngine::decode_latents (audiovae.rs:330-372) on the CPU: the
    record_* sequence over channel-major buffers, with the reference's
    snapshot/residual order (record_residual, audiovae.rs:400-407)."""

    def __init__(self, data: np.ndarray, tensors: dict, cfg: dict):
        self.blob = np.ascontiguousarray(data, dtype=np.uint8)
        if self.blob.size % 4:
            self.blob = np.concatenate([self.blob, np.zeros(4 - self.blob.size % 4, np.uint8)])
        self.t, self.cfg = tensors, dict(cfg)

    def _conv(self, x, base, in_c, out_c, in_len, out_len, k, stride, dil, groups, pad):
        w, b = self.t[base], self.t[base + ".bias"]
        return vae_conv1d(self.blob, x, abi.VaeConvPush(w.offset, b.offset, in_c, out_c, in_len, out_len, k, stride,
                                                         dil, groups, pad, _dt(w), _dt(b), 1))

    def _snake(self, x, name, c, n):
        a = self.t[name]
        return vae_snake(self.blob, x, abi.VaeSnakePush(a.offset, c, n, _dt(a)))

    def decode(self, frame_major) -> np.ndarray:
        cfg = self.cfg
        ld = cfg["latent_dim"]
        fm = np.asarray(frame_major, np.float32).reshape(-1, ld)
        frames = fm.shape[0]
        x = np.ascontiguousarray(fm.T).ravel()             # frame_to_channel_major
        n, c = frames, ld
        x = self._conv(x, "audio_vae.decoder.model.0", c, c, n, n, 7, 1, 1, c, 6)
        x = self._conv(x, "audio_vae.decoder.model.1", c, cfg["decoder_dim"], n, n, 1, 1, 1, 1, 0)
        c = cfg["decoder_dim"]
        for i, s in enumerate(cfg["decoder_rates"]):
            mi, co = i + 2, c // 2
            sw = self.t[f"audio_vae.decoder.sr_cond_model.{mi}.scale_embed"]
            bw = self.t[f"audio_vae.decoder.sr_cond_model.{mi}.bias_embed"]
            x = vae_scale_bias(self.blob, x, abi.VaeScalePush(sw.offset, bw.offset, c, n, cfg["decoder_sr_bucket"],
                                                               4, _dt(sw), _dt(bw)))
            y = self._snake(x, f"audio_vae.decoder.model.{mi}.block.0.alpha", c, n)
            w, b = self.t[f"audio_vae.decoder.model.{mi}.block.1"], self.t[f"audio_vae.decoder.model.{mi}.block.1.bias"]
            x = vae_convt1d(self.blob, y, abi.VaeConvTPush(w.offset, b.offset, c, co, n, n * s, 2 * s, s, 1, _dt(w),
                                                            _dt(b), 1))
            c, n = co, n * s
            for rj, dil in enumerate((1, 3, 9)):
                p = f"audio_vae.decoder.model.{mi}.block.{rj + 2}.block"
                snap = x.copy()
                y = self._snake(x, p + ".0.alpha", c, n)
                x = self._conv(y, p + ".1", c, c, n, n, 7, 1, dil, c, 6 * dil)
                y = self._snake(x, p + ".2.alpha", c, n)
                x = self._conv(y, p + ".3", c, c, n, n, 1, 1, 1, 1, 0)
                lib().vr_vae_add(_p(x), _p(snap), C.byref(abi.VaeGridPush(c, n)))
        y = self._snake(x, "audio_vae.decoder.model.8.alpha", c, n)
        x = self._conv(y, "audio_vae.decoder.model.9", c, 1, n, n, 7, 1, 1, 1, 6)
        return vae_tanh(x)


def stats(v) -> tuple:
    """stats (acoustic.rs:1248-1257): position-weighted checksum and L2."""
    x = np.asarray(v, dtype=np.float64)
    return float(np.sum(x * (np.arange(x.size) % 251 + 1))), float(np.sqrt(np.sum(x * x)))


# ------------------------------------------------------------- CFM pieces
def mix32(v: int) -> int:
    return lib().vr_mix32(v & 0xFFFFFFFF)


def cfm_noise(push: abi.CfmNoisePush) -> np.ndarray:
    x = f32(push.n)
    lib().vr_cfm_noise(_p(x), C.byref(push))
    return x


def cfm_cfg_euler(x, pos, neg, push: abi.CfmEulerPush) -> np.ndarray:
    y = np.array(x, np.float32, copy=True)
    pos_c = np.ascontiguousarray(pos, np.float32)  # held across the call
    neg_c = np.ascontiguousarray(neg, np.float32)  # held across the call
    lib().vr_cfm_cfg_euler(_p(y), _p(pos_c), _p(neg_c),
                           C.byref(push))
    return y


def time_sinusoidal(push: abi.TimePush) -> np.ndarray:
    y = f32(push.dim)
    lib().vr_time_sinusoidal(_p(y), C.byref(push))
    return y


def pack_locdit(mu1, mu2, time, cond, x, push: abi.PackLocDitPush) -> np.ndarray:
    h = f32((3 + 2 * push.patch_tokens) * push.hidden)
    a = [np.ascontiguousarray(v, np.float32) for v in (mu1, mu2, time, cond, x)]
    lib().vr_pack_locdit(*[_p(v) for v in a], _p(h), C.byref(push))
    return h


def cfm_time_span(n: int, sway: float):
    out = f32(n + 1)
    st = lib().vr_cfm_time_span(n, sway, _p(out))
    return out if st == 0 else None


class LocDit:
    """LocDiT estimator and UnifiedCFM solve (local.rs:383-537) in float64 numpy:
    record_locdit_common + record_locdit_body (local.rs:445-468), record_time
    (470-480), record_transformer (482-527) with the seq_* / dense_* shader
    semantics, and cfm_solve (383-430). The token layout, mu zeroing of the
    unconditional pass and the condition modes follow vx_locdit_config."""

    def __init__(self, data: np.ndarray, tensors: dict, cfg: dict, rope_factors=None):
        self.blob = np.ascontiguousarray(data, dtype=np.uint8)
        self.c = dict(cfg)
        self.t = tensors
        c = self.c
        self.H, self.QD, self.KD = c["hidden"], c["q_heads"] * c["head_dim"], c["kv_heads"] * c["head_dim"]
        self.S = c["n_mu"] + 1 + c["n_cond"] + c["patch"]
        if rope_factors is None:
            rf = tensors["rope_factors_short.weight"]
            rope_factors = self.blob[rf.offset:rf.offset + rf.nbytes].view(np.float32)
        self.rope_factors = np.asarray(rope_factors, np.float64)
        self._cache = {}

    def _mat(self, name):
        w = self._cache.get(name)
        if w is None:
            t = self.t[name]
            cols, rows = t.dims[0], t.dims[1]
            w = self._cache[name] = dequant(self.blob, t.offset, t.ggml_type, rows, cols).astype(np.float64)
        return w

    def _vec(self, name):
        t = self.t[name]
        n = int(np.prod(t.dims))
        raw = self.blob[t.offset:t.offset + t.nbytes]
        return (raw.view(np.float32) if t.ggml_type == abi.DTYPE_F32 else raw.view(np.float16)).astype(np.float64)[:n]

    def _lin(self, prefix, x):
        return x @ self._mat(prefix + ".weight").T + self._vec(prefix + ".bias")

    def _rms(self, x, w):
        return x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + self.c["rms_epsilon"]) * w

    @staticmethod
    def _silu(x):
        return x / (1.0 + np.exp(-x))

    def time_embed(self, t, dt):
        """record_time: time_mlp(sin(t)) + delta_time_mlp(sin(dt)) (f64 sinusoid)."""
        H = self.H
        half = H // 2
        j = np.arange(H) % half
        freq = np.exp(j * (-np.log(10000.0) / max(half - 1, 1)))

        def sinus(v):
            a = 1000.0 * v * freq
            return np.where(np.arange(H) < half, np.sin(a), np.cos(a))

        tv = self._lin("locdit.time_mlp.linear_2", self._silu(self._lin("locdit.time_mlp.linear_1", sinus(t))))
        dv = self._lin("locdit.delta_time_mlp.linear_2",
                       self._silu(self._lin("locdit.delta_time_mlp.linear_1", sinus(dt))))
        return tv + dv

    def _rope(self, x, heads):
        c = self.c
        hd, half = c["head_dim"], c["head_dim"] // 2
        S = x.shape[0]
        pos = np.arange(S, dtype=np.float64)[:, None]
        i = np.arange(half, dtype=np.float64)
        ang = pos / (c["rope_theta"] ** (2.0 * i / hd) * self.rope_factors[:half])
        cs, sn = np.cos(ang) * c["rope_scaling"], np.sin(ang) * c["rope_scaling"]
        y = x.reshape(S, heads, hd).copy()
        a, b = y[..., :half].copy(), y[..., half:].copy()
        y[..., :half] = a * cs[:, None, :] - b * sn[:, None, :]
        y[..., half:] = b * cs[:, None, :] + a * sn[:, None, :]
        return y.reshape(S, heads * hd)

    def transformer(self, h):
        """record_transformer over one sequence h [S][H]; returns the final norm."""
        c = self.c
        L, hd, qh, kh = c["layers"], c["head_dim"], c["q_heads"], c["kv_heads"]
        S = h.shape[0]
        h = h.copy()
        norm = self._rms(h, self._vec("locdit.blk.0.attn_norm.weight"))
        for l in range(L):
            p = f"locdit.blk.{l}."
            q = self._rope(norm @ self._mat(p + "attn_q.weight").T, qh)
            k = self._rope(norm @ self._mat(p + "attn_k.weight").T, kh)
            v = norm @ self._mat(p + "attn_v.weight").T
            Q = q.reshape(S, qh, hd)
            K = k.reshape(S, kh, hd)[:, np.arange(qh) // (qh // kh), :]
            V = v.reshape(S, kh, hd)[:, np.arange(qh) // (qh // kh), :]
            sc = np.einsum("thd,shd->hts", Q, K) / np.sqrt(hd)
            pr = np.exp(sc - sc.max(axis=2, keepdims=True))
            pr /= pr.sum(axis=2, keepdims=True)
            att = np.einsum("hts,shd->thd", pr, V).reshape(S, qh * hd)
            h = h + att @ self._mat(p + "attn_output.weight").T
            norm = self._rms(h, self._vec(p + "ffn_norm.weight"))
            act = self._silu(norm @ self._mat(p + "ffn_gate.weight").T) * (norm @ self._mat(p + "ffn_up.weight").T)
            h = h + act @ self._mat(p + "ffn_down.weight").T
            nxt = f"locdit.blk.{l + 1}.attn_norm.weight" if l + 1 < L else "locdit.norm.weight"
            norm = self._rms(h, self._vec(nxt))
        return norm

    def estimate(self, x, cond, mu, t, dt, zero_mu=False):
        """One estimator pass: out [patch][feat] (flattened)."""
        c = self.c
        H, P, FD = self.H, c["patch"], c["feat_dim"]
        xt = self._lin("locdit.in_proj", np.asarray(x, np.float64).reshape(P, FD))
        if c["cond_raw"]:
            ct = np.asarray(cond, np.float64).reshape(c["n_cond"], H)
        else:
            ct = self._lin("locdit.cond_proj", np.asarray(cond, np.float64).reshape(P, FD))
        if zero_mu and c["uncond_zero_cond"]:
            ct = np.zeros_like(ct)
        rows = []
        if c["n_mu"]:
            m = np.asarray(mu, np.float64).reshape(c["n_mu"], H)
            rows.append(np.zeros_like(m) if zero_mu else m)
        rows += [self.time_embed(t, dt)[None, :], ct, xt]
        norm = self.transformer(np.concatenate(rows, axis=0))
        return self._lin("locdit.out_proj", norm[self.S - P:]).reshape(-1)

    def project_mu(self, current_lm, residual_output):
        """record_project_mu (local.rs:459-462): seq_linear_bias with one token,
        mu1 = lm_to_dit_proj . current_lm + b, mu2 = res_to_dit_proj . residual + b."""
        out = []
        for name, x in (("projections.lm_to_dit_proj", current_lm), ("projections.res_to_dit_proj", residual_output)):
            out.append(self._mat(name + ".weight") @ np.asarray(x, np.float64) + self._vec(name + ".bias"))
        return np.concatenate(out)

    def cfm_solve(self, cond, mu, n_timesteps=10, cfg_value=2.0, temperature=1.0, sway=1.0, seed=42,
                  zero_star=True, initial_x=None):
        c = self.c
        n = c["patch"] * c["feat_dim"]
        if initial_x is None:
            x = cfm_noise(abi.CfmNoisePush(n, seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF, temperature))
            x = x.astype(np.float64)
        else:
            x = np.asarray(initial_x, np.float64).copy()
        span = cfm_time_span(n_timesteps, sway).astype(np.float64)
        zi = max(1, int(np.floor(len(span) * 0.04))) if zero_star else 0
        for step in range(1, len(span)):
            if step <= zi:
                continue
            t, dt = float(np.float32(span[step - 1])), float(np.float32(span[step - 1]) - np.float32(span[step]))
            pos = self.estimate(x, cond, mu, t, 0.0)
            neg = self.estimate(x, cond, mu, t, 0.0, zero_mu=True)
            s = (pos @ neg) / (neg @ neg + 1e-8) if zero_star else 1.0
            x = x - dt * (neg * s + cfg_value * (pos - neg * s))
        return x
