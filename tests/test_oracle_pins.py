"""Pins the CPU oracle (oracle/voxref.c) against checks that do not reuse its code.

Each test derives the expected value a different way: numpy's IEEE half
conversion, a numpy decode of the GGUF Q8_0 block bytes, float64 linear algebra,
complex-number rotation, closed forms and invariants. A plausible slip in the
oracle (a dropped term, a transposed index, a wrong sign) fails one of them.
"""
import numpy as np
import pytest

import voxref
from conftest import rel_l2
from voxgen_amd import abi, synth
from voxgen_amd.synth import Region

RNG = np.random.default_rng(1234)


# ------------------------------------------------------------------ halves
def test_f16_to_f32_all_halves_match_numpy():
    bits = np.arange(65536, dtype=np.uint16)
    got = voxref.f16_bits_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_rne_matches_numpy():
    halves = np.arange(0, 0x7C00, dtype=np.uint16)
    lo = halves[:-1].view(np.float16).astype(np.float64)
    hi = halves[1:].view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32)              # exact ties (f32 holds them)
    rand = RNG.standard_normal(200000).astype(np.float32) * np.float32(300.0)
    tiny = (RNG.standard_normal(20000) * 1e-6).astype(np.float32)   # subnormal halves
    big = np.array([65504, 65519.99, 65520, 1e6, -1e6, np.inf, -np.inf, 0.0, -0.0], np.float32)
    for x in (mids, -mids, rand, tiny, big):
        got = voxref.f32_to_f16_bits(x)
        with np.errstate(over="ignore"):
            want = x.astype(np.float16).view(np.uint16)
        assert np.array_equal(got, want)
    nan = voxref.f32_to_f16_bits(np.array([np.nan], np.float32))
    assert np.isnan(nan.view(np.float16)[0])


# ---------------------------------------------------------------- helpers
def numpy_q8_decode(blob: np.ndarray, offset: int, rows: int, cols: int) -> np.ndarray:
    """GGUF Q8_0 (gguf.rs:41-45): per 34-byte block an f16 scale then 32 int8."""
    nb = rows * cols // 32
    blocks = blob[offset:offset + nb * 34].reshape(nb, 34)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float32)
    q = blocks[:, 2:].copy().view(np.int8).astype(np.float32)
    return (d * q).reshape(rows, cols)


def numpy_f16_decode(blob, offset, rows, cols):
    return blob[offset:offset + rows * cols * 2].copy().view(np.float16).astype(np.float32).reshape(rows, cols)


@pytest.fixture(scope="module")
def region():
    """A small data region with the matrix shapes the ops read."""
    reg = Region()
    specs = {
        "q8_a": (abi.DTYPE_Q8_0, (256, 64)),      # dims: [cols, rows]
        "q8_b": (abi.DTYPE_Q8_0, (256, 64)),
        "q8_k": (abi.DTYPE_Q8_0, (256, 32)),
        "q8_v": (abi.DTYPE_Q8_0, (256, 32)),
        "f16_a": (abi.DTYPE_F16, (256, 48)),
        "f32_a": (abi.DTYPE_F32, (64, 16)),
        "f16_fus": (abi.DTYPE_F16, (96, 40)),
        "norm": (abi.DTYPE_F32, (256,)),
        "bias32": (abi.DTYPE_F32, (64,)),
        "bias16": (abi.DTYPE_F16, (64,)),
        "factors": (abi.DTYPE_F32, (64,)),
    }
    ts = {k: reg.add(k, *v) for k, v in specs.items()}
    data = np.zeros((reg.size + 255) // 256 * 256, np.uint8)
    for i, (k, t) in enumerate(ts.items()):
        n = int(np.prod(t.dims))
        s = 1000 + i
        if t.ggml_type == abi.DTYPE_Q8_0:
            data[t.offset:t.offset + t.nbytes] = synth.q8_0_blocks(n // 32, s)
        elif t.ggml_type == abi.DTYPE_F16:
            data[t.offset:t.offset + t.nbytes] = synth.normal_f16(n, s, 0.0, 0.5).view(np.uint8)
        else:
            data[t.offset:t.offset + t.nbytes] = synth.normal_f32(n, s, 1.0, 0.3).view(np.uint8)
    data[ts["factors"].offset:ts["factors"].offset + 256].view(np.float32)[:] = \
        1.0 + np.arange(64, dtype=np.float32) / 32
    return data, ts


# ------------------------------------------------------------ dequant
def test_q8_dequant_matches_numpy_block_decode(region):
    data, ts = region
    t = ts["q8_a"]
    got = voxref.dequant(data, t.offset, abi.DTYPE_Q8_0, 64, 256)
    want = numpy_q8_decode(data, t.offset, 64, 256)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q8_dequant_special_values():
    blocks = np.zeros((6, 34), np.uint8)
    scales = np.array([0.0, -0.0, 6e-8, 65504.0, -1.5, 0.01], np.float16)
    blocks[:, :2] = scales.view(np.uint8).reshape(6, 2)
    q = np.tile(np.array([-128, 127, -1, 0, 1, -127, 64, -64], np.int8), 4)
    blocks[:, 2:] = q.view(np.uint8)
    blob = np.concatenate([blocks.ravel(), np.zeros(4, np.uint8)])
    got = voxref.dequant(blob, 0, abi.DTYPE_Q8_0, 6, 32)
    want = scales.astype(np.float32)[:, None] * q.astype(np.float32)[None, :]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_f16_dequant_is_widening(region):
    data, ts = region
    t = ts["f16_a"]
    got = voxref.dequant(data, t.offset, abi.DTYPE_F16, 48, 256)
    assert np.array_equal(got, numpy_f16_decode(data, t.offset, 48, 256))


def test_embedding_gather_bit_exact(region):
    data, ts = region
    for name, dt in (("q8_a", abi.DTYPE_Q8_0), ("f16_a", abi.DTYPE_F16)):
        t = ts[name]
        rows = t.dims[1]
        W = numpy_q8_decode(data, t.offset, rows, 256) if dt == abi.DTYPE_Q8_0 else \
            numpy_f16_decode(data, t.offset, rows, 256)
        for tok, alpha in ((0, 1.0), (rows - 1, 1.0), (7, 0.5)):
            h = voxref.embedding(data, abi.EmbeddingPush(t.offset, 256, tok, dt, alpha))
            assert np.array_equal(h, W[tok] * np.float32(alpha))


# ------------------------------------------------------------- matvecs
def test_matvec_matches_f64(region):
    data, ts = region
    x = RNG.standard_normal(256).astype(np.float32)
    for name, dt, rows in (("q8_a", 8, 64), ("f16_a", 1, 48)):
        t = ts[name]
        W = voxref.dequant(data, t.offset, dt, rows, 256).astype(np.float64)
        y = voxref.matvec(data, x, abi.MatvecPush(t.offset, rows, 256, dt, 0, 0.75))
        assert rel_l2(y, 0.75 * (W @ x.astype(np.float64))) < 1e-6


def test_matvec_one_hot_recovers_column_and_is_linear(region):
    data, ts = region
    t = ts["q8_a"]
    W = numpy_q8_decode(data, t.offset, 64, 256)
    e = np.zeros(256, np.float32)
    e[77] = 1.0
    y = voxref.matvec(data, e, abi.MatvecPush(t.offset, 64, 256, 8, 0, 1.0))
    assert np.array_equal(y, W[:, 77])
    a, b = RNG.standard_normal((2, 256)).astype(np.float32)
    p = abi.MatvecPush(t.offset, 64, 256, 8, 0, 1.0)
    lhs = voxref.matvec(data, 2 * a + b, p)
    rhs = 2 * voxref.matvec(data, a, p) + voxref.matvec(data, b, p)
    assert rel_l2(lhs, rhs) < 1e-5


def test_matvec_row_base_skips_rows(region):
    data, ts = region
    t = ts["q8_a"]
    x = RNG.standard_normal(256).astype(np.float32)
    y = np.full(64, 7.0, np.float32)
    voxref.matvec(data, x, abi.MatvecPush(t.offset, 64, 256, 8, 40, 1.0), y=y)
    full = voxref.matvec(data, x, abi.MatvecPush(t.offset, 64, 256, 8, 0, 1.0))
    assert np.all(y[:40] == 7.0) and np.array_equal(y[40:], full[40:])


def test_qkv_matvec_targets(region):
    data, ts = region
    x = RNG.standard_normal(256).astype(np.float32)
    p = abi.QkvPush(ts["q8_a"].offset, ts["q8_k"].offset, ts["q8_v"].offset, 64, 32, 256, 8, 8, 8, 0)
    q, k, v = voxref.qkv_matvec(data, x, p)
    for out, name, rows in ((q, "q8_a", 64), (k, "q8_k", 32), (v, "q8_v", 32)):
        W = numpy_q8_decode(data, ts[name].offset, rows, 256).astype(np.float64)
        assert rel_l2(out, W @ x) < 1e-6


def test_swiglu_closed_form(region):
    data, ts = region
    x = RNG.standard_normal(256).astype(np.float32) * 0.05
    Wg = numpy_q8_decode(data, ts["q8_a"].offset, 64, 256).astype(np.float64)
    Wu = numpy_q8_decode(data, ts["q8_b"].offset, 64, 256).astype(np.float64)
    y = voxref.matvec_swiglu(data, x, abi.SwigluPush(ts["q8_a"].offset, ts["q8_b"].offset, 64, 256, 8, 0))
    g, u = Wg @ x, Wu @ x
    assert rel_l2(y, g / (1 + np.exp(-g)) * u) < 1e-5
    y0 = voxref.matvec_swiglu(data, np.zeros(256, np.float32),
                              abi.SwigluPush(ts["q8_a"].offset, ts["q8_b"].offset, 64, 256, 8, 0))
    assert np.all(y0 == 0)


# ----------------------------------------------------------- norms
def test_rmsnorm_closed_form_and_scale_invariance(region):
    data, ts = region
    w = data[ts["norm"].offset:ts["norm"].offset + 1024].view(np.float32).astype(np.float64)
    x = RNG.standard_normal(256).astype(np.float32) * 3
    p = abi.RmsPush(ts["norm"].offset, 256, 1e-6)
    y = voxref.rmsnorm(data, x, p)
    xd = x.astype(np.float64)
    assert rel_l2(y, xd / np.sqrt(np.mean(xd ** 2) + 1e-6) * w) < 1e-6
    assert rel_l2(voxref.rmsnorm(data, x * 37.0, abi.RmsPush(ts["norm"].offset, 256, 0.0)),
                  voxref.rmsnorm(data, x, abi.RmsPush(ts["norm"].offset, 256, 0.0))) < 1e-6


def test_residual_rmsnorm_closed_form(region):
    data, ts = region
    w = data[ts["norm"].offset:ts["norm"].offset + 1024].view(np.float32).astype(np.float64)
    h = RNG.standard_normal(256).astype(np.float32)
    b = RNG.standard_normal(256).astype(np.float32)
    h2, y = voxref.residual_rmsnorm(data, h, b, abi.ResidualRmsPush(ts["norm"].offset, 256, 1e-6, 0.5))
    hv = h.astype(np.float64) + 0.5 * b
    assert rel_l2(h2, hv) < 1e-7
    assert rel_l2(y, hv / np.sqrt(np.mean(hv ** 2) + 1e-6) * w) < 1e-6


# ------------------------------------------------------------------ rope
def test_rope_is_complex_rotation(region):
    data, ts = region
    f = data[ts["factors"].offset:ts["factors"].offset + 256].view(np.float32).astype(np.float64)
    hd, qh, kh, pos, theta, sc = 128, 3, 2, 977, 10000.0, 1.25
    q = RNG.standard_normal(qh * hd).astype(np.float32)
    k = RNG.standard_normal(kh * hd).astype(np.float32)
    q2, k2 = voxref.rope(data, q, k, abi.RopePush(ts["factors"].offset, pos, qh, kh, hd, theta, sc))
    i = np.arange(hd // 2)
    ang = pos * theta ** (-2.0 * i / hd) / f
    rot = np.exp(1j * ang) * sc
    for src, got, heads in ((q, q2, qh), (k, k2, kh)):
        s = src.astype(np.float64).reshape(heads, hd)
        z = (s[:, :hd // 2] + 1j * s[:, hd // 2:]) * rot
        want = np.concatenate([z.real, z.imag], axis=1)
        np.testing.assert_allclose(got.reshape(heads, hd), want, rtol=0, atol=2e-4)
    q0, _ = voxref.rope(data, q, k, abi.RopePush(ts["factors"].offset, 0, qh, kh, hd, theta, 1.0))
    assert np.array_equal(q0, q)
    qn, _ = voxref.rope(data, q, k, abi.RopePush(ts["factors"].offset, 123, qh, kh, hd, theta, 1.0))
    pairs = lambda a: np.hypot(a.reshape(qh, hd)[:, :64], a.reshape(qh, hd)[:, 64:])
    np.testing.assert_allclose(pairs(qn), pairs(q), rtol=1e-5)


# ------------------------------------------------------------- kv cache
def test_store_kv_placement_and_rounding():
    L, ctx, kv = 3, 8, 256
    kc = np.zeros(L * ctx * kv, np.uint16)
    vc = np.zeros(L * ctx * kv, np.uint16)
    k = RNG.standard_normal(kv).astype(np.float32) * 100
    v = RNG.standard_normal(kv).astype(np.float32)
    voxref.store_kv(k, v, kc, vc, abi.StoreKvPush(2, 5, ctx, kv))
    ek = np.zeros((L, ctx, kv), np.uint16)
    ek[2, 5] = k.astype(np.float16).view(np.uint16)
    ev = np.zeros((L, ctx, kv), np.uint16)
    ev[2, 5] = v.astype(np.float16).view(np.uint16)
    assert np.array_equal(kc, ek.ravel()) and np.array_equal(vc, ev.ravel())


# ------------------------------------------------------------- attention
def numpy_attention(q, kc, vc, layer, ctx, pos, hd, qpk, kvh):
    Kc = kc.view(np.float16).astype(np.float64).reshape(-1, ctx, kvh * hd)[layer, :pos + 1]
    Vc = vc.view(np.float16).astype(np.float64).reshape(-1, ctx, kvh * hd)[layer, :pos + 1]
    out = []
    for h in range(qpk * kvh):
        g = h // qpk
        s = Kc[:, g * hd:(g + 1) * hd] @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        out.append(p @ Vc[:, g * hd:(g + 1) * hd])
    return np.concatenate(out)


@pytest.mark.parametrize("pos", [0, 1, 300])
def test_attention_three_ops_match_f64_softmax(pos):
    L, ctx, hd, qpk, kvh = 2, 320, 128, 4, 2
    kc = synth.normal_f16(L * ctx * kvh * hd, 77).view(np.uint16).copy()
    vc = synth.normal_f16(L * ctx * kvh * hd, 78).view(np.uint16).copy()
    q = RNG.standard_normal(qpk * kvh * hd).astype(np.float32) * 0.3
    ap = abi.AttentionPush(1, ctx, pos, hd, qpk, kvh)
    s = voxref.attn_scores(q, kc, qpk * kvh, ap)
    p = voxref.softmax(s, qpk * kvh, abi.SoftmaxPush(ctx, pos))
    sums = p.reshape(qpk * kvh, ctx)[:, :pos + 1].sum(axis=1)
    np.testing.assert_allclose(sums, 1.0, rtol=1e-5)
    o = voxref.attn_values(p, vc, qpk * kvh, ap)
    assert rel_l2(o, numpy_attention(q, kc, vc, 1, ctx, pos, hd, qpk, kvh)) < 1e-5
    if pos == 0:
        V0 = vc.view(np.float16).astype(np.float32).reshape(L, ctx, kvh * hd)[1, 0]
        want = np.concatenate([V0[(h // qpk) * hd:(h // qpk + 1) * hd] for h in range(qpk * kvh)])
        assert np.array_equal(o, want)


def test_softmax_shift_invariant():
    s = (RNG.standard_normal(2 * 64) * 5).astype(np.float32)
    a = voxref.softmax(s, 2, abi.SoftmaxPush(64, 40))
    b = voxref.softmax(s + np.float32(100.0), 2, abi.SoftmaxPush(64, 40))
    # Only t <= position is normalised; later slots are left untouched.
    np.testing.assert_allclose(a.reshape(2, 64)[:, :41], b.reshape(2, 64)[:, :41], atol=1e-6)
    assert np.array_equal(b.reshape(2, 64)[:, 41:], (s + np.float32(100.0)).reshape(2, 64)[:, 41:])


# ------------------------------------------------- linear_bias / fusion
def test_linear_bias_all_dtypes(region):
    data, ts = region
    x = RNG.standard_normal(64).astype(np.float32)
    t = ts["f32_a"]
    W = data[t.offset:t.offset + t.nbytes].view(np.float32).astype(np.float64).reshape(16, 64)
    b32 = data[ts["bias32"].offset:][:64 * 4].view(np.float32).astype(np.float64)
    b16 = data[ts["bias16"].offset:][:64 * 2].view(np.float16).astype(np.float64)
    for bo, bd, bias in ((ts["bias32"].offset, 0, b32), (ts["bias16"].offset, 1, b16), (0, 7, 0 * b32)):
        y = voxref.linear_bias(data, x, abi.LinearBiasPush(t.offset, bo, 16, 64, 0, bd, 0, 0.5))
        assert rel_l2(y, 0.5 * (W @ x + bias[:16])) < 1e-6
    xq = RNG.standard_normal(256).astype(np.float32)
    Wq = numpy_q8_decode(data, ts["q8_a"].offset, 64, 256).astype(np.float64)
    y = voxref.linear_bias(data, xq, abi.LinearBiasPush(ts["q8_a"].offset, ts["bias32"].offset, 64, 256, 8, 0, 0, 1.0))
    assert rel_l2(y, Wq @ xq + b32) < 1e-6


def test_fusion_linear_concat_and_snapshot(region):
    data, ts = region
    t = ts["f16_fus"]
    W = numpy_f16_decode(data, t.offset, 40, 96).astype(np.float64)
    left = RNG.standard_normal(64).astype(np.float32)
    right = RNG.standard_normal(32).astype(np.float32)
    b = data[ts["bias16"].offset:][:128].view(np.float16).astype(np.float64)
    y, s = voxref.fusion_linear(data, left, right, abi.FusionPush(t.offset, ts["bias16"].offset, 40, 64, 32, 1, 1, 0))
    assert np.array_equal(y, s)
    assert rel_l2(y, W @ np.concatenate([left, right]) + b[:40]) < 1e-6


# --------------------------------------------------------- full layer
def numpy_layer_stack(model, tokens_pos, cfg):
    """float64 MiniCPM4 decode written from the closed forms (not the oracle)."""
    data, T = model.data, {t.name: t for t in model.tensors}
    H, KV, F, hd = cfg["embedding_length"], cfg["kv_dim"], cfg["feed_forward_length"], cfg["head_dim"]
    qh, kvh, L, eps = cfg["head_count"], cfg["head_count_kv"], cfg["block_count"], cfg["rms_epsilon"]

    def W(name, rows, cols):
        t = T[name]
        return (numpy_q8_decode(data, t.offset, rows, cols) if t.ggml_type == 8
                else numpy_f16_decode(data, t.offset, rows, cols)).astype(np.float64)

    def vec(name):
        t = T[name]
        return data[t.offset:t.offset + t.nbytes].view(np.float32).astype(np.float64)

    def rms(x, w):
        return x / np.sqrt(np.mean(x * x) + eps) * w

    E = W("token_embd.weight", cfg["vocab_size"], H)
    Kc = [np.zeros((0, KV)) for _ in range(L)]
    Vc = [np.zeros((0, KV)) for _ in range(L)]
    outs = []
    i = np.arange(hd // 2)
    for tok, pos in tokens_pos:
        h = E[tok].copy()
        for l in range(L):
            p = f"blk.{l}."
            x = rms(h, vec(p + "attn_norm.weight"))
            q, k, v = W(p + "attn_q.weight", H, H) @ x, W(p + "attn_k.weight", KV, H) @ x, W(p + "attn_v.weight", KV, H) @ x
            rot = np.exp(1j * pos * cfg["rope_theta"] ** (-2.0 * i / hd))
            def apply(a, n):
                a = a.reshape(n, hd)
                z = (a[:, :hd // 2] + 1j * a[:, hd // 2:]) * rot
                return np.concatenate([z.real, z.imag], axis=1).ravel()
            q, k = apply(q, qh), apply(k, kvh)
            Kc[l] = np.vstack([Kc[l], k.astype(np.float16).astype(np.float64)])
            Vc[l] = np.vstack([Vc[l], v.astype(np.float16).astype(np.float64)])
            att = []
            for hh in range(qh):
                g = hh // (qh // kvh)
                s = Kc[l][:, g * hd:(g + 1) * hd] @ q[hh * hd:(hh + 1) * hd] / np.sqrt(hd)
                pr = np.exp(s - s.max())
                att.append((pr / pr.sum()) @ Vc[l][:, g * hd:(g + 1) * hd])
            h = h + W(p + "attn_output.weight", H, H) @ np.concatenate(att)
            x = rms(h, vec(p + "ffn_norm.weight"))
            g_, u_ = W(p + "ffn_gate.weight", F, H) @ x, W(p + "ffn_up.weight", F, H) @ x
            h = h + W(p + "ffn_down.weight", H, F) @ (g_ / (1 + np.exp(-g_)) * u_)
        outs.append(rms(h, vec("output_norm.weight")))
    return outs


def test_record_transformer_matches_f64_stack():
    cfg = synth.baselm_config(layers=2, hidden=256, ffn=512, vocab=96, q_heads=2, kv_heads=1,
                              head_dim=128, context_length=64, active_context=16)
    # Small weights keep the softmax away from ties so f32 and f64 agree closely.
    m = synth.build_baselm(cfg, seed=99, q8_scale_sigma=0.001)
    o = voxref.BaseLm(m.data, {t.name: t for t in m.tensors}, cfg)
    seq = [(5, 0), (17, 1), (95, 2), (0, 3)]
    want = numpy_layer_stack(m, seq, cfg)
    for (tok, pos), w in zip(seq, want):
        got = o.decode_token(tok, pos)
        assert rel_l2(got, w) < 1e-4, (tok, pos)
    kv = o.kv_k.reshape(2, 16, 128)
    assert np.all(kv[:, 4:] == 0) and np.any(kv[:, :4] != 0)


# ------------------------------------------------- reference known answers
def test_effective_scale_reference_unit_test():
    # baselm.rs:1319-1323
    assert voxref.effective_scale(0.0) == 1.0
    assert voxref.effective_scale(0.125) == 0.125


def test_rope_scaling_factor_closed_form():
    cfg = synth.baselm_config(context_length=32768, original_context=4096)
    want = np.sqrt(1 + np.log(32768 / 4096) / np.log(4096))
    assert abs(voxref.rope_scaling_factor(cfg) - want) < 1e-6
    assert voxref.rope_scaling_factor(synth.baselm_config(context_length=32768)) == 1.0
