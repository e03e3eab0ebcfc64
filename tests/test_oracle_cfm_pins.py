"""Pins of the CFM / LocDiT oracle (voxref.c CFM functions, voxref.LocDit).

Each oracle function is checked against something that does not restate its
own code: an algebraically derived inverse of the hash, float64 closed forms,
statistics of the noise, and a loop-by-loop transformer on a tiny geometry.
"""
import numpy as np
import pytest

import voxref
from conftest import rel_l2
from voxgen_amd import abi, synth

M32 = 0xFFFFFFFF


def _unxorshift(y: int, s: int) -> int:
    """Inverse of y = x ^ (x >> s) on 32 bits, derived by repeated shifting."""
    x = y
    k = s
    while k < 32:
        x ^= y >> k
        k += s
    return x & M32


def _inverse_mix32(v: int) -> int:
    # mix32 = xs16 . mul(c2) . xs15 . mul(c1) . xs16; undo the steps in reverse
    # with the modular inverses of the odd multipliers.
    v = _unxorshift(v, 16)
    v = (v * pow(0x846CA68B, -1, 1 << 32)) & M32
    v = _unxorshift(v, 15)
    v = (v * pow(0x7FEB352D, -1, 1 << 32)) & M32
    return _unxorshift(v, 16)


def test_mix32_is_inverted_by_the_algebraic_inverse():
    rng = np.random.default_rng(5)
    vals = [0, 1, 0xFFFFFFFF, 0x80000000, 0x9E3779B9] + [int(v) for v in rng.integers(0, 1 << 32, 20000)]
    for v in vals:
        assert _inverse_mix32(voxref.mix32(v)) == v
    assert voxref.mix32(0) == 0
    outs = {voxref.mix32(v) for v in range(4096)}
    assert len(outs) == 4096   # injective on a range


def test_cfm_noise_box_muller_against_f64():
    n, seed, temp = 512, 0x0123456789ABCDEF, 0.7
    lo, hi = seed & M32, seed >> 32
    got = voxref.cfm_noise(abi.CfmNoisePush(n, lo, hi, temp)).astype(np.float64)
    want = np.empty(n)
    for i in range(n):
        a = voxref.mix32((i >> 1) ^ lo ^ 0x9E3779B9)
        b = voxref.mix32((i >> 1) ^ hi ^ 0x85EBCA6B)
        u1 = max((a + 0.5) / 2.0 ** 32, 1e-7)
        u2 = (b + 0.5) / 2.0 ** 32
        r = np.sqrt(-2.0 * np.log(u1))
        want[i] = temp * r * (np.cos(2 * np.pi * u2) if i % 2 == 0 else np.sin(2 * np.pi * u2))
    assert rel_l2(got, want) < 1e-5


def test_cfm_noise_statistics_and_determinism():
    x = voxref.cfm_noise(abi.CfmNoisePush(1 << 16, 42, 0, 1.0)).astype(np.float64)
    assert abs(x.mean()) < 0.02 and abs(x.std() - 1.0) < 0.02
    assert np.array_equal(x, voxref.cfm_noise(abi.CfmNoisePush(1 << 16, 42, 0, 1.0)))
    y = voxref.cfm_noise(abi.CfmNoisePush(1 << 16, 43, 0, 1.0))
    assert not np.array_equal(x, y)
    assert np.all(voxref.cfm_noise(abi.CfmNoisePush(64, 42, 0, 0.0)) == 0)


@pytest.mark.parametrize("zero_star", [0, 1])
def test_cfm_cfg_euler_closed_form(zero_star):
    n = 256
    x = synth.normal_f32(n, 1).astype(np.float64)
    p = synth.normal_f32(n, 2).astype(np.float64)
    q = (0.5 * p + synth.normal_f32(n, 3)).astype(np.float64)
    dt, cfg = 0.11, 2.0
    got = voxref.cfm_cfg_euler(x, p, q, abi.CfmEulerPush(n, dt, cfg, zero_star))
    s = p @ q / (q @ q + 1e-8) if zero_star else 1.0
    want = x - dt * (q * s + cfg * (p - q * s))
    assert rel_l2(got, want) < 1e-6
    # cfg = 1 is the plain positive estimate whatever the scale.
    got1 = voxref.cfm_cfg_euler(x, p, q, abi.CfmEulerPush(n, dt, 1.0, zero_star))
    assert rel_l2(got1, x - dt * p) < 1e-6


def test_time_sinusoidal_closed_form():
    for dim, t in ((1024, 0.37), (64, 1.0), (1024, 0.0)):
        got = voxref.time_sinusoidal(abi.TimePush(dim, t))
        half = dim // 2
        j = np.arange(dim) % half
        a = 1000.0 * t * np.exp(j * (-np.log(1e4) / (half - 1)))
        want = np.where(np.arange(dim) < half, np.sin(a), np.cos(a))
        assert np.max(np.abs(got - want)) < 1e-3   # |a| up to 1000: f32 argument rounding
        if t == 0.0:
            assert np.all(got[:half] == 0) and np.all(got[half:] == 1)


def test_pack_locdit_concatenation():
    H, P = 32, 4
    mu1, mu2, tv = synth.normal_f32(H, 1), synth.normal_f32(H, 2), synth.normal_f32(H, 3)
    cond, x = synth.normal_f32(P * H, 4), synth.normal_f32(P * H, 5)
    got = voxref.pack_locdit(mu1, mu2, tv, cond, x, abi.PackLocDitPush(H, P, 0)).reshape(-1, H)
    want = np.concatenate([mu1[None], mu2[None], tv[None], cond.reshape(P, H), x.reshape(P, H)])
    assert np.array_equal(got, want)
    z = voxref.pack_locdit(mu1, mu2, tv, cond, x, abi.PackLocDitPush(H, P, 1)).reshape(-1, H)
    assert np.all(z[:2] == 0) and np.array_equal(z[2:], want[2:])


def test_cfm_time_span_closed_form():
    for n, sway in ((10, 1.0), (4, 0.5), (7, 0.0)):
        got = voxref.cfm_time_span(n, sway).astype(np.float64)
        t = 1 - np.arange(n + 1) / n
        assert rel_l2(got, t + sway * (np.cos(np.pi * t / 2) - 1 + t)) < 1e-6
        assert got[0] == 1.0 and abs(got[-1]) < 1e-7 and np.all(np.diff(got) <= 1e-6)
    assert rel_l2(voxref.cfm_time_span(7, 0.0), 1 - np.arange(8) / 7) < 1e-7
    assert voxref.cfm_time_span(0, 1.0) is None
    assert voxref.cfm_time_span(4, -3.0) is None   # not descending: the reference bails


# ------------------------------------------------------------ LocDiT oracle
def naive_locdit(m, cfg, x, cond, mu, t, dt, zero_mu=False):
    """Loop-by-loop restatement of one LocDiT pass on a tiny geometry."""
    blob = m.data
    T = {d.name: d for d in m.tensors}

    def mat(name):
        d = T[name]
        return voxref.dequant(blob, d.offset, d.ggml_type, d.dims[1], d.dims[0]).astype(np.float64)

    def vec(name):
        d = T[name]
        return blob[d.offset:d.offset + d.nbytes].view(np.float32).astype(np.float64)

    def lin(pre, v):
        W, b = mat(pre + ".weight"), vec(pre + ".bias")
        return [sum(W[r, c] * v[c] for c in range(len(v))) + b[r] for r in range(W.shape[0])]

    def rms(v, w):
        s = sum(e * e for e in v) / len(v)
        return [e / np.sqrt(s + cfg["rms_epsilon"]) * w[i] for i, e in enumerate(v)]

    silu = lambda v: v / (1 + np.exp(-v))
    H, hd, nq, nk, P, FD = cfg["hidden"], cfg["head_dim"], cfg["q_heads"], cfg["kv_heads"], cfg["patch"], cfg["feat_dim"]
    half = H // 2

    def sinus(v):
        return [np.sin(1000 * v * np.exp((i % half) * -np.log(1e4) / (half - 1))) if i < half else
                np.cos(1000 * v * np.exp((i % half) * -np.log(1e4) / (half - 1))) for i in range(H)]

    tt = lin("locdit.time_mlp.linear_2", [silu(e) for e in lin("locdit.time_mlp.linear_1", sinus(t))])
    dd = lin("locdit.delta_time_mlp.linear_2", [silu(e) for e in lin("locdit.delta_time_mlp.linear_1", sinus(dt))])
    rows = [list(np.zeros(H) if zero_mu else mu[i * H:(i + 1) * H]) for i in range(cfg["n_mu"])]
    rows.append([a + b for a, b in zip(tt, dd)])
    rows += [lin("locdit.cond_proj", cond[i * FD:(i + 1) * FD]) for i in range(P)]
    rows += [lin("locdit.in_proj", x[i * FD:(i + 1) * FD]) for i in range(P)]
    S = len(rows)
    h = [list(r) for r in rows]
    norm = [rms(r, vec("locdit.blk.0.attn_norm.weight")) for r in h]
    for l in range(cfg["layers"]):
        p = f"locdit.blk.{l}."
        Wq, Wk, Wv, Wo = mat(p + "attn_q.weight"), mat(p + "attn_k.weight"), mat(p + "attn_v.weight"), mat(p + "attn_output.weight")
        q = [[sum(Wq[r, c] * n[c] for c in range(H)) for r in range(nq * hd)] for n in norm]
        k = [[sum(Wk[r, c] * n[c] for c in range(H)) for r in range(nk * hd)] for n in norm]
        v = [[sum(Wv[r, c] * n[c] for c in range(H)) for r in range(nk * hd)] for n in norm]
        for s_ in range(S):
            for vecs, nh in ((q, nq), (k, nk)):
                for hh in range(nh):
                    for i in range(hd // 2):
                        ang = s_ / (cfg["rope_theta"] ** (2 * i / hd))
                        a, b = vecs[s_][hh * hd + i], vecs[s_][hh * hd + i + hd // 2]
                        vecs[s_][hh * hd + i] = a * np.cos(ang) - b * np.sin(ang)
                        vecs[s_][hh * hd + i + hd // 2] = b * np.cos(ang) + a * np.sin(ang)
        att = [[0.0] * (nq * hd) for _ in range(S)]
        for s_ in range(S):
            for hh in range(nq):
                kvh = hh // (nq // nk)
                sc = [sum(q[s_][hh * hd + d] * k[j][kvh * hd + d] for d in range(hd)) / np.sqrt(hd) for j in range(S)]
                mx = max(sc)
                e = [np.exp(z - mx) for z in sc]
                z = sum(e)
                for d in range(hd):
                    att[s_][hh * hd + d] = sum(e[j] / z * v[j][kvh * hd + d] for j in range(S))
        for s_ in range(S):
            o = [sum(Wo[r, c] * att[s_][c] for c in range(nq * hd)) for r in range(H)]
            h[s_] = [a + b for a, b in zip(h[s_], o)]
        norm = [rms(r, vec(p + "ffn_norm.weight")) for r in h]
        Wg, Wu, Wd = mat(p + "ffn_gate.weight"), mat(p + "ffn_up.weight"), mat(p + "ffn_down.weight")
        for s_ in range(S):
            g = [silu(sum(Wg[r, c] * norm[s_][c] for c in range(H))) * sum(Wu[r, c] * norm[s_][c] for c in range(H))
                 for r in range(cfg["ffn"])]
            dn = [sum(Wd[r, c] * g[c] for c in range(cfg["ffn"])) for r in range(H)]
            h[s_] = [a + b for a, b in zip(h[s_], dn)]
        nxt = f"locdit.blk.{l + 1}.attn_norm.weight" if l + 1 < cfg["layers"] else "locdit.norm.weight"
        norm = [rms(r, vec(nxt)) for r in h]
    out = []
    for s_ in range(S - P, S):
        out += lin("locdit.out_proj", norm[s_])
    return np.array(out)


def test_locdit_oracle_matches_loop_restatement():
    cfg = synth.locdit_config(layers=1, hidden=16, q_heads=2, kv_heads=1, head_dim=8, ffn=24, feat_dim=4, patch=2)
    m = synth.build_locdit(cfg, seed=7, std=0.2)
    o = voxref.LocDit(m.data, {t.name: t for t in m.tensors}, cfg)
    x, cond, mu = synth.normal_f32(8, 1), synth.normal_f32(8, 2), synth.normal_f32(32, 3)
    for zero_mu in (False, True):
        got = o.estimate(x, cond, mu, 0.63, 0.0, zero_mu=zero_mu)
        want = naive_locdit(m, cfg, x.astype(np.float64), cond.astype(np.float64), mu.astype(np.float64), 0.63, 0.0,
                            zero_mu=zero_mu)
        assert rel_l2(got, want) < 1e-10, zero_mu


def test_project_mu_matches_the_linear_bias_restatement():
    """LocDit.project_mu (record_project_mu, local.rs:459-462) against the C
    restatement of linear_bias.comp on the same F16 projection tensors, and a
    one-hot input recovers a weight column plus the bias."""
    cfg = synth.locdit_config(layers=1)
    m = synth.build_locdit(cfg, seed=0x5EED0901)
    ts = {t.name: t for t in m.tensors}
    o = voxref.LocDit(m.data, ts, cfg)
    x1, x2 = synth.normal_f32(2048, 0x5EED0902), synth.normal_f32(2048, 0x5EED0903)
    got = o.project_mu(x1, x2)
    for i, (name, x) in enumerate((("projections.lm_to_dit_proj", x1), ("projections.res_to_dit_proj", x2))):
        w, b = ts[name + ".weight"], ts[name + ".bias"]
        push = abi.LinearBiasPush(w.offset, b.offset, cfg["hidden"], 2048, abi.DTYPE_F16, 0, 0, 1.0)
        want = voxref.linear_bias(m.data, x, push)
        assert rel_l2(got[i * cfg["hidden"]:(i + 1) * cfg["hidden"]], want) < 1e-6, name
    onehot = np.zeros(2048, np.float32)
    onehot[77] = 1.0
    w = ts["projections.lm_to_dit_proj.weight"]
    col = m.data[w.offset:w.offset + w.nbytes].view(np.float16).reshape(cfg["hidden"], 2048)[:, 77]
    bias = m.data[ts["projections.lm_to_dit_proj.bias"].offset:][:cfg["hidden"] * 4].view(np.float32)
    assert np.allclose(o.project_mu(onehot, onehot)[:cfg["hidden"]], col.astype(np.float64) + bias, rtol=0, atol=1e-7)
