"""AudioVAE decoder (AudioVaeEngine::decode_latents, audiovae.rs:330-372) and the
vae_*.comp entry points on the GPU against the oracle (voxref.AudioVae, vr_vae_*),
through the C ABI. Per-op kernels rel-L2 <= 1e-5; the decoded wave rel-L2 <= 1e-3
(the engine runs the 1x1 and transposed convolutions as f16-weight GEMMs with the
f32 activations split hi/lo, in its own order)."""
import numpy as np
import pytest

import voxref
from conftest import rel_l2
from test_oracle_vae_pins import f16_region
from voxgen_amd import abi, synth
from voxgen_amd.audiovae import AudioVaeEngine
from voxgen_amd.runtime import Model

pytestmark = pytest.mark.gpu


def test_vae_shader_entry_points(ctx):
    rng = np.random.default_rng(11)
    C, L = 16, 300
    arrays = {"dw": rng.normal(0, 0.3, (C, 1, 7)), "dwb": rng.normal(0, 0.1, C),
              "pw": rng.normal(0, 0.2, (8, C, 1)), "pwb": rng.normal(0, 0.1, 8),
              "st": rng.normal(0, 0.3, (C, 12, 6)), "stb": rng.normal(0, 0.1, 12),
              "ct": rng.normal(0, 0.3, (C, 8, 10)), "ctb": rng.normal(0, 0.1, 8),
              "a": rng.uniform(0.5, 1.5, C), "s": rng.normal(1, 0.1, (4, C)), "b": rng.normal(0, 0.1, (4, C))}
    blob, off = f16_region({k: np.asarray(v, np.float16).ravel() for k, v in arrays.items()})
    from voxgen_amd.runtime import TensorDesc
    model = Model(ctx, blob, [TensorDesc("blob", abi.DTYPE_F32, (blob.size // 4,), 0)])
    x = rng.normal(0, 1, (C, L)).astype(np.float32)
    xb = ctx.array(x)
    y = ctx.alloc(C * L * 5 * 4)
    cases = [
        ("conv1d", abi.VaeConvPush(off["dw"], off["dwb"], C, C, L, L, 7, 1, 3, C, 18, 1, 1, 1), C * L),
        ("conv1d", abi.VaeConvPush(off["pw"], off["pwb"], C, 8, L, L, 1, 1, 1, 1, 0, 1, 1, 1), 8 * L),
        ("conv1d", abi.VaeConvPush(off["st"], off["stb"], C, 12, L, L // 3, 6, 3, 1, 1, 3, 1, 1, 1), 12 * (L // 3)),
        ("conv1d", abi.VaeConvPush(off["pw"], off["pwb"], C, 8, L, L, 1, 1, 1, 1, 0, 1, 1, 0), 8 * L),
        ("convt", abi.VaeConvTPush(off["ct"], off["ctb"], C, 8, L, 5 * L, 10, 5, 1, 1, 1, 1), 8 * 5 * L),
    ]
    for kind, push, n in cases:
        print(f"vae op {kind} {n}", flush=True)
        if kind == "conv1d":
            abi.call("vx_vae_conv1d", ctx.handle, model.handle, xb.handle, y.handle, push)
            want = voxref.vae_conv1d(model_blob(blob), x.ravel(), push)
        else:
            abi.call("vx_vae_convtranspose1d", ctx.handle, model.handle, xb.handle, y.handle, push)
            want = voxref.vae_convt1d(model_blob(blob), x.ravel(), push)
        assert rel_l2(y.download(np.float32, n), want) < 1e-5, kind
    push = abi.VaeSnakePush(off["a"], C, L, 1)
    abi.call("vx_vae_snake", ctx.handle, model.handle, xb.handle, y.handle, push)
    assert rel_l2(y.download(np.float32, C * L), voxref.vae_snake(blob, x.ravel(), push)) < 1e-5
    push = abi.VaeScalePush(off["s"], off["b"], C, L, 3, 4, 1, 1)
    z = ctx.array(x)
    abi.call("vx_vae_scale_bias", ctx.handle, model.handle, z.handle, push)
    assert rel_l2(z.download(np.float32, C * L), voxref.vae_scale_bias(blob, x.ravel(), push)) < 1e-6
    abi.call("vx_vae_add", ctx.handle, z.handle, xb.handle, abi.VaeGridPush(C, L))
    abi.call("vx_vae_tanh", ctx.handle, z.handle, C * L)
    want = voxref.vae_tanh(voxref.vae_scale_bias(blob, x.ravel(), push) + x.ravel())
    assert rel_l2(z.download(np.float32, C * L), want) < 1e-6
    small = ctx.alloc(16)   # held in a name: a temporary Buffer frees its handle when .handle is read
    bad = abi.VaeConvPush(off["dw"], off["dwb"], C, C, L, L, 7, 1, 3, C, 18, 1, 1, 1)
    with pytest.raises(abi.VxError) as e:
        abi.call("vx_vae_conv1d", ctx.handle, model.handle, xb.handle, small.handle, bad)
    assert e.value.name == "VX_ERR_BOUNDS"
    model.free()


def model_blob(blob):
    return blob


def engine_case(ctx, dd, frames, seed):
    cfg = synth.audiovae_config(decoder_dim=dd)
    m = synth.build_audiovae(cfg, seed=seed)
    model = Model(ctx, m.data, m.tensors)
    eng = AudioVaeEngine(ctx, model, cfg, strict_geometry=(dd == 2048))
    lat = synth.normal_f32(frames * 64, seed + 1)
    o = voxref.AudioVae(m.data, {t.name: t for t in m.tensors}, cfg)
    return cfg, model, eng, lat, o


@pytest.mark.parametrize("dd,frames", [(256, 8), (2048, 4)])
def test_decode_matches_oracle(ctx, dd, frames):
    print(f"vae decode decoder_dim {dd} frames {frames}", flush=True)
    cfg, model, eng, lat, o = engine_case(ctx, dd, frames, 0x5EED0510 + dd)
    st, wave = eng.decode_latents(lat)
    want = o.decode(lat)
    assert wave.size == frames * 1920 == st.output_samples
    assert rel_l2(wave, want) < 1e-3
    assert st.latent_frames == frames and st.latent_patches == frames // 4 and st.output_sample_rate == 48000
    assert st.checksum == pytest.approx(float(np.sum(wave.astype(np.float64))), abs=1e-6 * wave.size)
    assert st.l2 == pytest.approx(float(np.linalg.norm(wave.astype(np.float64))), rel=1e-9)
    assert st.peak == pytest.approx(float(np.max(np.abs(wave))))
    assert st.scratch_bytes == eng.scratch_bytes() > 0
    lb, wb = ctx.array(lat), ctx.alloc(wave.size * 4)
    eng.decode_latents_gpu(lb, frames, wb)
    # split-K GEMMs accumulate with atomic adds: runs agree to rounding, not bit for bit
    assert rel_l2(wb.download(np.float32, wave.size), wave) < 1e-5
    eng.close()
    model.free()


def test_decode_errors(ctx):
    cfg, model, eng, lat, o = engine_case(ctx, 256, 4, 0x5EED0520)
    for bad, code in ((lat[:63], "VX_ERR_SHAPE"), (lat[:128], "VX_ERR_SHAPE"),
                      (np.where(np.arange(lat.size) == 5, np.nan, lat).astype(np.float32), "VX_ERR_INVALID_ARG")):
        with pytest.raises(abi.VxError) as e:
            eng.decode_latents(bad)
        assert e.value.name == code
    with pytest.raises(abi.VxError) as e:
        eng.decode_latents_gpu(ctx.array(lat), 4, ctx.alloc(1024))
    assert e.value.name == "VX_ERR_BOUNDS"
    # A frame count whose activations pass the 32-bit index range is refused by
    # the device-buffer entry as by the host one, before any buffer check or launch.
    patch = cfg["patch_size"]
    with pytest.raises(abi.VxError) as e:
        eng.decode_latents_gpu(ctx.array(lat), (0xFFFFFFFF // patch) * patch, ctx.alloc(1024))
    assert e.value.name == "VX_ERR_UNSUPPORTED"
    with pytest.raises(abi.VxError) as e:
        AudioVaeEngine(ctx, model, cfg, strict_geometry=True)
    assert e.value.name == "VX_ERR_UNSUPPORTED"
    eng.close()
    model.free()
