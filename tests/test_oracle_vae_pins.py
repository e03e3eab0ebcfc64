"""Pins of the AudioVAE oracle (vr_vae_* and voxref.AudioVae.decode) against
float64 numpy written from the operators' definitions, independently of
voxref.c: convolution as a gather over shifted slices, the transposed convolution
in PyTorch's scatter form, snake / scale-bias / tanh closed forms, and the whole
decoder (audiovae.rs:330-372) on a narrow synthetic model. CPU only.
"""
import numpy as np
import pytest

import voxref
from conftest import rel_l2
from voxgen_amd import abi, synth
from voxgen_amd.synth import Region


def f16_region(arrays):
    """A data region of F16 tensors (name -> array) -> (blob, offsets)."""
    reg = Region()
    for name, a in arrays.items():
        reg.add(name, abi.DTYPE_F16, (a.size,))
    blob = np.zeros((reg.size + 255) // 256 * 256, np.uint8)
    offs = {}
    for t in reg.tensors:
        a = arrays[t.name].astype(np.float16)
        blob[t.offset:t.offset + a.nbytes] = a.view(np.uint8)
        offs[t.name] = t.offset
    return blob, offs


def np_conv1d(x, w, b, stride, dil, groups, pad, out_len):
    """x [Cin][L], w [Cout][Cin/g][K]: y[o][t] = b[o] + sum x[ic][t s + k d - pad] w[o][icg][k]."""
    cin, L = x.shape
    cout, ipg, K = w.shape
    opg = cout // groups
    xp = np.concatenate([np.zeros((cin, pad)), x, np.zeros((cin, out_len * stride + K * dil))], axis=1)
    y = np.tile(b[:, None], (1, out_len)).astype(np.float64)
    for o in range(cout):
        g = o // opg
        for icg in range(ipg):
            for k in range(K):
                y[o] += w[o, icg, k] * xp[g * ipg + icg, k * dil: k * dil + out_len * stride: stride][:out_len]
    return y


def np_convt1d(x, w, b, stride, out_len):
    """PyTorch ConvTranspose1d (groups 1) as a scatter, cropped to out_len:
    w [Cin][Cout][K], y[o][ti s + k] += x[ic][ti] w[ic][o][k]."""
    cin, L = x.shape
    _, cout, K = w.shape
    y = np.zeros((cout, (L - 1) * stride + K))
    for ti in range(L):
        for k in range(K):
            y[:, ti * stride + k] += x[:, ti] @ w[:, :, k]
    return y[:, :out_len] + b[:, None]


def snake64(x, a):
    return x + np.sin(a * x) ** 2 / (a + 1e-9)


@pytest.mark.parametrize("cin,cout,K,stride,dil,groups,pad,L", [
    (3, 4, 7, 1, 1, 1, 6, 20), (8, 8, 7, 1, 3, 8, 18, 33), (6, 4, 3, 2, 1, 2, 2, 17), (4, 6, 16, 8, 1, 1, 8, 64)])
def test_conv1d_matches_f64_gather(cin, cout, K, stride, dil, groups, pad, L):
    rng = np.random.default_rng(cin * 100 + K)
    w = rng.normal(0, 0.3, (cout, cin // groups, K)).astype(np.float16)
    b = rng.normal(0, 0.1, cout).astype(np.float16)
    x = rng.normal(0, 1, (cin, L)).astype(np.float32)
    blob, off = f16_region({"w": w.ravel(), "b": b})
    out_len = (L + pad - dil * (K - 1) - 1) // stride + 1 if stride > 1 else L
    got = voxref.vae_conv1d(blob, x.ravel(), abi.VaeConvPush(off["w"], off["b"], cin, cout, L, out_len, K, stride,
                                                             dil, groups, pad, 1, 1, 1))
    want = np_conv1d(x.astype(np.float64), w.astype(np.float64), b.astype(np.float64), stride, dil, groups, pad,
                     out_len)
    assert rel_l2(got, want) < 1e-6


@pytest.mark.parametrize("cin,cout,stride,L", [(4, 3, 2, 9), (8, 4, 5, 7), (6, 2, 8, 5)])
def test_convtranspose1d_matches_f64_scatter(cin, cout, stride, L):
    rng = np.random.default_rng(cin * 10 + stride)
    K = 2 * stride
    w = rng.normal(0, 0.3, (cin, cout, K)).astype(np.float16)
    b = rng.normal(0, 0.1, cout).astype(np.float16)
    x = rng.normal(0, 1, (cin, L)).astype(np.float32)
    blob, off = f16_region({"w": w.ravel(), "b": b})
    got = voxref.vae_convt1d(blob, x.ravel(), abi.VaeConvTPush(off["w"], off["b"], cin, cout, L, L * stride, K,
                                                                stride, 1, 1, 1, 1))
    want = np_convt1d(x.astype(np.float64), w.astype(np.float64), b.astype(np.float64), stride, L * stride)
    assert rel_l2(got, want) < 1e-6


def test_snake_scale_bias_tanh_closed_forms():
    rng = np.random.default_rng(7)
    C, L = 5, 40
    a = rng.uniform(0.5, 1.5, C).astype(np.float16)
    sc = rng.normal(1, 0.1, (4, C)).astype(np.float16)
    bi = rng.normal(0, 0.1, (4, C)).astype(np.float16)
    blob, off = f16_region({"a": a, "s": sc.ravel(), "b": bi.ravel()})
    x = rng.normal(0, 2, (C, L)).astype(np.float32)
    got = voxref.vae_snake(blob, x.ravel(), abi.VaeSnakePush(off["a"], C, L, 1))
    assert rel_l2(got, snake64(x.astype(np.float64), a.astype(np.float64)[:, None])) < 1e-6
    got = voxref.vae_scale_bias(blob, x.ravel(), abi.VaeScalePush(off["s"], off["b"], C, L, 2, 4, 1, 1))
    want = x * sc[2].astype(np.float64)[:, None] + bi[2].astype(np.float64)[:, None]
    assert rel_l2(got, want) < 1e-6
    assert rel_l2(voxref.vae_tanh(x.ravel()), np.tanh(x.astype(np.float64)).ravel()) < 1e-6


def np_decode(m, cfg, latents):
    """float64 AudioVAE decode written from the module structure (audiovae.rs:330-372)."""
    T = {t.name: t for t in m.tensors}

    def arr(name, shape):
        t = T[name]
        return m.data[t.offset:t.offset + t.nbytes].view(np.float16).astype(np.float64).reshape(shape)

    def conv(x, base, cin, cout, k, groups, dil=1):
        w = arr(base, (cout, cin // groups, k))
        return np_conv1d(x, w, arr(base + ".bias", (cout,)), 1, dil, groups, 6 * dil if k == 7 else 0, x.shape[1])

    def snake(x, name):
        return snake64(x, arr(name, (x.shape[0],))[:, None])

    x = np.asarray(latents, np.float64).reshape(-1, cfg["latent_dim"]).T
    L = cfg["latent_dim"]
    x = conv(x, "audio_vae.decoder.model.0", L, L, 7, L)
    x = conv(x, "audio_vae.decoder.model.1", L, cfg["decoder_dim"], 1, 1)
    c = cfg["decoder_dim"]
    bk = cfg["decoder_sr_bucket"]
    for i, s in enumerate(cfg["decoder_rates"]):
        mi, co = i + 2, c // 2
        sc = arr(f"audio_vae.decoder.sr_cond_model.{mi}.scale_embed", (4, c))[bk]
        bi = arr(f"audio_vae.decoder.sr_cond_model.{mi}.bias_embed", (4, c))[bk]
        x = snake(x * sc[:, None] + bi[:, None], f"audio_vae.decoder.model.{mi}.block.0.alpha")
        p = f"audio_vae.decoder.model.{mi}.block.1"
        x = np_convt1d(x, arr(p, (c, co, 2 * s)), arr(p + ".bias", (co,)), s, x.shape[1] * s)
        c = co
        for rj, dil in enumerate((1, 3, 9)):
            q = f"audio_vae.decoder.model.{mi}.block.{rj + 2}.block"
            y = conv(snake(x, q + ".0.alpha"), q + ".1", c, c, 7, c, dil)
            x = x + conv(snake(y, q + ".2.alpha"), q + ".3", c, c, 1, 1)
    x = conv(snake(x, "audio_vae.decoder.model.8.alpha"), "audio_vae.decoder.model.9", c, 1, 7, 1)
    return np.tanh(x).ravel()


def test_decode_matches_f64_module():
    cfg = synth.audiovae_config(decoder_dim=64)
    m = synth.build_audiovae(cfg, seed=0x5EED0501)
    lat = synth.normal_f32(4 * 64, 0x800)
    got = voxref.AudioVae(m.data, {t.name: t for t in m.tensors}, cfg).decode(lat)
    want = np_decode(m, cfg, lat)
    assert got.size == 4 * 1920
    assert rel_l2(got, want) < 1e-5
    assert 0.05 < np.std(got) and np.max(np.abs(got)) < 0.99   # tanh not saturated: the test sees every stage
