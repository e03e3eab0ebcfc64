"""Pins of the ResidualLM / FSQ / fusion / stop-predictor oracle (voxref.ResidualFsq,
vr_fsq_quantize, vr_silu_inplace, vr_residual_lm_record) against the reference's
known answer (acoustic.rs:1266-1271) and float64 numpy written from the closed
forms, independently of voxref.c's code. CPU only.
"""
import numpy as np
import pytest

import voxref
from conftest import rel_l2
from test_oracle_pins import numpy_f16_decode
from voxgen_amd import synth


def round_half_away(t):
    return np.sign(t) * np.floor(np.abs(t) + 0.5)


def test_fsq_reference_known_answer():
    # acoustic.rs:1266-1271: (tanh(0.42) * 9).round() / 9 == 0.44444445
    got = voxref.fsq_quantize(np.array([0.42], np.float32), 9.0)[0]
    assert abs(got - 0.44444445) < 1e-6


def test_fsq_matches_f64_on_the_grid_and_is_odd():
    x = synth.normal_f32(1 << 14, 0x5EED0301, 0.0, 2.0)
    for scale in (9.0, 4.0, 1.5):
        got = voxref.fsq_quantize(x, scale)
        t = np.tanh(x.astype(np.float64)) * scale
        k = round_half_away(t)
        near = np.abs(np.abs(t - np.trunc(t)) - 0.5) < 1e-5   # ties decided by f32 rounding
        assert np.all(got[~near] == (k / scale).astype(np.float32)[~near]), scale
        kg = got.astype(np.float64) * scale
        assert np.allclose(kg, np.round(kg), atol=1e-5) and np.all(np.abs(kg) <= scale + 1e-5)
        assert np.array_equal(voxref.fsq_quantize(-x, scale), -got)


def test_silu_closed_form():
    x = synth.normal_f32(4096, 0x5EED0302, 0.0, 4.0)
    got = voxref.silu_inplace(x)
    x64 = x.astype(np.float64)
    assert rel_l2(got, x64 / (1 + np.exp(-x64))) < 1e-6
    assert voxref.silu_inplace(np.zeros(3, np.float32)).tolist() == [0.0, 0.0, 0.0]


def numpy_residual(model, acfg, steps):
    """float64 FSQ + fusion + ResidualLM (no RoPE) + stop head from the closed forms."""
    data, T = model.data, {t.name: t for t in model.tensors}
    H, KV, F, hd = acfg["embedding_length"], acfg["kv_dim"], acfg["feed_forward_length"], acfg["head_dim"]
    qh, kvh, L, eps = acfg["head_count"], acfg["head_count_kv"], acfg["residual_block_count"], acfg["rms_epsilon"]
    Ld, s = acfg["fsq_latent_dim"], acfg["fsq_scale"]

    def W(name, rows, cols):
        return numpy_f16_decode(data, T[name].offset, rows, cols).astype(np.float64)

    def vec(name):
        t = T[name]
        dt = np.float32 if t.ggml_type == 0 else np.float16
        return data[t.offset:t.offset + t.nbytes].view(dt).astype(np.float64)

    def rms(x, w):
        return x / np.sqrt(np.mean(x * x) + eps) * w

    Kc = [np.zeros((0, KV)) for _ in range(L)]
    Vc = [np.zeros((0, KV)) for _ in range(L)]
    outs = []
    for base, emb, fsq in steps:
        base = base.astype(np.float64)
        o = {}
        if fsq:
            lat = W("fsq.in_proj.weight", Ld, H) @ base + vec("fsq.in_proj.bias")
            t = np.tanh(lat) * s
            o["margin"] = np.min(np.abs(np.abs(t - np.trunc(t)) - 0.5))
            o["latent"] = round_half_away(t) / s
            left = W("fsq.out_proj.weight", H, Ld) @ o["latent"] + vec("fsq.out_proj.bias")
            o["fsq"], right = left, emb.astype(np.float64)
        else:
            left, right = base, np.zeros(H)
        h = W("projections.res_fusion_proj.weight", H, 2 * H) @ np.concatenate([left, right]) + \
            vec("projections.res_fusion_proj.bias")
        o["fused"] = h.copy()
        for l in range(L):
            p = f"residual_lm.blk.{l}."
            x = rms(h, vec(p + "attn_norm.weight"))
            q, k, v = W(p + "attn_q.weight", H, H) @ x, W(p + "attn_k.weight", KV, H) @ x, W(p + "attn_v.weight", KV, H) @ x
            Kc[l] = np.vstack([Kc[l], k.astype(np.float16).astype(np.float64)])
            Vc[l] = np.vstack([Vc[l], v.astype(np.float16).astype(np.float64)])
            att = []
            for hh in range(qh):
                g = hh // (qh // kvh)
                sc = Kc[l][:, g * hd:(g + 1) * hd] @ q[hh * hd:(hh + 1) * hd] / np.sqrt(hd)
                pr = np.exp(sc - sc.max())
                att.append((pr / pr.sum()) @ Vc[l][:, g * hd:(g + 1) * hd])
            h = h + W(p + "attn_output.weight", H, H) @ np.concatenate(att)
            x = rms(h, vec(p + "ffn_norm.weight"))
            g_, u_ = W(p + "ffn_gate.weight", F, H) @ x, W(p + "ffn_up.weight", F, H) @ x
            h = h + W(p + "ffn_down.weight", H, F) @ (g_ / (1 + np.exp(-g_)) * u_)
        o["norm"] = rms(h, vec("residual_lm.output_norm.weight"))
        sh = W("stop_predictor.linear1.weight", H, H) @ left + vec("stop_predictor.linear1.bias")
        o["stop"] = W("stop_predictor.linear2.weight", 2, H) @ (sh / (1 + np.exp(-sh)))
        outs.append(o)
    return outs


def small_acoustic():
    return synth.acoustic_config(layers=2, hidden=256, ffn=512, q_heads=2, kv_heads=1, head_dim=128, latent=64,
                                 active_context=16)


def test_residual_step_matches_f64_stack():
    acfg = small_acoustic()
    m = synth.build_acoustic(acfg, seed=0x5EED0303)
    o = voxref.ResidualFsq(m.data, {t.name: t for t in m.tensors}, acfg)
    H = acfg["embedding_length"]
    steps = [(synth.normal_f32(H, 10 + i), synth.normal_f32(H, 20 + i), i != 1) for i in range(4)]
    want = numpy_residual(m, acfg, steps)
    for pos, ((base, emb, fsq), w) in enumerate(zip(steps, want)):
        got = o.step(base, emb, pos, fsq=fsq)
        if fsq:
            assert w["margin"] > 1e-4, "inputs sit on an FSQ rounding boundary"
            assert np.array_equal(got["latent"], w["latent"].astype(np.float32)), pos
            assert rel_l2(got["fsq"], w["fsq"]) < 1e-5, pos
        assert rel_l2(got["fused"], w["fused"]) < 1e-5, pos
        assert rel_l2(got["norm"], w["norm"]) < 1e-4, pos
        assert rel_l2(o.stop(o.current_lm), w["stop"]) < 1e-4, pos
    kv = o.kv_k.reshape(2, 16, 128)
    assert np.all(kv[:, 4:] == 0) and np.any(kv[:, :4] != 0)


def test_residual_record_equals_baselm_record_at_position_zero():
    """RoPE at position 0 is the identity, so the no-RoPE stack and
    record_transformer must agree bit for bit there (and differ later)."""
    acfg = small_acoustic()
    m = synth.build_acoustic(acfg, seed=0x5EED0304)
    o = voxref.ResidualFsq(m.data, {t.name: t for t in m.tensors}, acfg)
    h = synth.normal_f32(acfg["embedding_length"], 5)
    o.hidden[:] = h
    voxref.lib().vr_residual_lm_record(voxref._p(o.blob), voxref.C.byref(o._m), voxref.C.byref(o._s), 0)
    a = o.norm.copy()
    # RoPE factors from a positive f32 vector, theta 10000: every angle is 0.
    o._m.rope_factors = m.offset("residual_lm.output_norm.weight")
    o._m.cfg.rope_theta = 10000.0
    o.kv_k[:] = 0
    o.kv_v[:] = 0
    o.hidden[:] = h
    voxref.lib().vr_baselm_record(voxref._p(o.blob), voxref.C.byref(o._m), voxref.C.byref(o._s), 0, 0)
    assert np.array_equal(a, o.norm)


def test_stats_weighting():
    # acoustic.rs:1248-1257: weights (i % 251) + 1.
    v = np.ones(300, np.float32)
    c, l2 = voxref.stats(v)
    assert c == sum(i % 251 + 1 for i in range(300)) and abs(l2 - np.sqrt(300)) < 1e-12
