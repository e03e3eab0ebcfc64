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
    lib().vr_rmsnorm(_p(blob), _p(np.ascontiguousarray(x, np.float32)), _p(y), C.byref(push))
    return y


def residual_rmsnorm(blob, hidden, branch, push: abi.ResidualRmsPush):
    h = np.array(hidden, np.float32, copy=True)
    y = f32(push.n)
    lib().vr_residual_rmsnorm(_p(blob), _p(h), _p(np.ascontiguousarray(branch, np.float32)), _p(y),
                              C.byref(push))
    return h, y


def matvec(blob, x, push: abi.MatvecPush, y=None) -> np.ndarray:
    y = f32(push.rows) if y is None else y
    lib().vr_matvec(_p(blob), _p(np.ascontiguousarray(x, np.float32)), _p(y), C.byref(push))
    return y


def qkv_matvec(blob, x, push: abi.QkvPush):
    q, k, v = f32(push.q_rows), f32(push.kv_rows), f32(push.kv_rows)
    lib().vr_qkv_matvec(_p(blob), _p(np.ascontiguousarray(x, np.float32)), _p(q), _p(k), _p(v),
                        C.byref(push))
    return q, k, v


def matvec_swiglu(blob, x, push: abi.SwigluPush) -> np.ndarray:
    y = f32(push.rows)
    lib().vr_matvec_swiglu(_p(blob), _p(np.ascontiguousarray(x, np.float32)), _p(y), C.byref(push))
    return y


def rope(blob, q, k, push: abi.RopePush):
    q2 = np.array(q, np.float32, copy=True)
    k2 = np.array(k, np.float32, copy=True)
    lib().vr_rope(_p(blob), _p(q2), _p(k2), C.byref(push))
    return q2, k2


def store_kv(k, v, k_cache: np.ndarray, v_cache: np.ndarray, push: abi.StoreKvPush) -> None:
    """k_cache/v_cache: uint16 (f16 bits) arrays updated in place."""
    lib().vr_store_kv(_p(np.ascontiguousarray(k, np.float32)), _p(np.ascontiguousarray(v, np.float32)),
                      _p(k_cache), _p(v_cache), C.byref(push))


def attn_scores(q, k_cache, q_heads: int, push: abi.AttentionPush) -> np.ndarray:
    s = f32(q_heads * push.context)
    lib().vr_attn_scores(_p(np.ascontiguousarray(q, np.float32)), _p(k_cache), _p(s), q_heads, C.byref(push))
    return s


def softmax(scores, heads: int, push: abi.SoftmaxPush) -> np.ndarray:
    s = np.array(scores, np.float32, copy=True)
    lib().vr_softmax(_p(s), heads, C.byref(push))
    return s


def attn_values(scores, v_cache, q_heads: int, push: abi.AttentionPush) -> np.ndarray:
    o = f32(q_heads * push.head_dim)
    lib().vr_attn_values(_p(np.ascontiguousarray(scores, np.float32)), _p(v_cache), _p(o), q_heads,
                         C.byref(push))
    return o


def linear_bias(blob, x, push: abi.LinearBiasPush) -> np.ndarray:
    y = f32(push.rows)
    lib().vr_linear_bias(_p(blob), _p(np.ascontiguousarray(x, np.float32)), _p(y), C.byref(push))
    return y


def fusion_linear(blob, left, right, push: abi.FusionPush):
    y, s = f32(push.rows), f32(push.rows)
    r = np.ascontiguousarray(right if right is not None else np.zeros(1), np.float32)
    lib().vr_fusion_linear(_p(blob), _p(np.ascontiguousarray(left, np.float32)), _p(r), _p(y), _p(s),
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
