"""ResidualLM + FSQ + fusion + stop head (ResidualFsqEngine, acoustic.rs:400-1035)
on the GPU against the oracle (voxref.ResidualFsq), through the C ABI.

Every entry point of the engine runs in a sequence with its positions checked
against the oracle's step at the same position: the FSQ latent bit-exact (it is a
grid index), FSQ output / fusion snapshot / current_lm rel-L2 <= 1e-4, the
normalised ResidualLM output rel-L2 <= 1e-3 per step, the stop logits <= 1e-3,
the f16 KV rows within one f16 ulp-scale tolerance. Error paths follow the
reference's bail! conditions.
"""
import numpy as np
import pytest

import voxref
from conftest import rel_l2
from voxgen_amd import abi, synth
from voxgen_amd.residual import ResidualFsqEngine
from voxgen_amd.runtime import Model

pytestmark = pytest.mark.gpu


def oracle_of(m, acfg):
    return voxref.ResidualFsq(m.data, {t.name: t for t in m.tensors}, acfg)


@pytest.fixture(scope="module")
def two_layers(ctx):
    """The real 2048/6144/16/2/128 shapes with 2 ResidualLM layers."""
    acfg = synth.acoustic_config(layers=2, active_context=64)
    m = synth.build_acoustic(acfg, seed=0x5EED0401)
    model = Model(ctx, m.data, m.tensors)
    yield acfg, m, model
    model.free()


@pytest.fixture(scope="module")
def small(ctx):
    """hidden 256 (the unmerged attention path), 2 layers, context 8."""
    acfg = synth.acoustic_config(layers=2, hidden=256, ffn=512, q_heads=2, kv_heads=1, head_dim=128, latent=64,
                                 active_context=8)
    m = synth.build_acoustic(acfg, seed=0x5EED0402, bias_f32_stop=False)
    model = Model(ctx, m.data, m.tensors)
    yield acfg, m, model
    model.free()


def check_step(eng, o, res, want, fsq):
    H = eng.config["embedding_length"]
    if fsq:
        assert np.array_equal(eng.buffer("fsq_latent").download(np.float32, eng.config["fsq_latent_dim"]),
                              want["latent"])
        got_fsq = eng.buffer("fsq_output").download(np.float32, H)
        assert rel_l2(got_fsq, want["fsq"]) < 1e-4
    lm = eng.current_lm_buffer().download(np.float32, H)
    assert rel_l2(lm, o.current_lm) < 1e-4
    fused = eng.buffer("fusion_snapshot").download(np.float32, H)
    assert rel_l2(fused, want["fused"]) < 1e-4
    out = eng.output()
    assert rel_l2(out, want["norm"]) < 1e-3
    if res is not None and hasattr(res, "residual_hidden_checksum"):
        c, l2 = voxref.stats(out)
        assert res.residual_hidden_checksum == pytest.approx(c, rel=1e-9, abs=1e-9)
        assert res.residual_hidden_l2 == pytest.approx(l2, rel=1e-9)
        c, l2 = voxref.stats(fused)
        assert res.fused_input_checksum == pytest.approx(c, rel=1e-9, abs=1e-9)
        assert res.fsq_applied == fsq and (res.fsq_checksum is None) == (not fsq)


@pytest.mark.parametrize("mode", ["graph", "fused", "reference"])
def test_entry_point_sequence_matches_oracle(ctx, two_layers, mode):
    acfg, m, model = two_layers
    H = acfg["embedding_length"]
    eng = ResidualFsqEngine(ctx, model, acfg, exec_mode=mode, strict_geometry=False)
    o = oracle_of(m, acfg)
    bases = [synth.normal_f32(H, 0x100 + i) for i in range(8)]
    embs = [synth.normal_f32(H, 0x200 + i) for i in range(8)]
    base_buf, emb_buf = ctx.array(bases[0]), ctx.array(embs[0])
    calls = ["text", "text_gpu_only", "host", "gpu_base", "gpu_both", "gpu_both_only", "host", "gpu_both"]
    for pos, call in enumerate(calls):
        print(f"residual {mode} pos {pos} {call}", flush=True)
        b, e = bases[pos], embs[pos]
        base_buf.upload(b)
        emb_buf.upload(e)
        fsq = not call.startswith("text")
        if call == "text":
            res = eng.step_text_prefix_from_gpu_base(base_buf)
        elif call == "text_gpu_only":
            res = eng.step_text_prefix_from_gpu_base_gpu_only(base_buf)
        elif call == "host":
            res = eng.step(b, e)
        elif call == "gpu_base":
            res = eng.step_from_gpu_base(base_buf, e)
        elif call == "gpu_both":
            res = eng.step_from_gpu_base_and_embedding(base_buf, emb_buf)
        else:
            res = eng.step_from_gpu_base_and_embedding_gpu_only(base_buf, emb_buf)
        assert res.position == pos and eng.position == pos + 1
        want = o.step(b, e, pos, fsq=fsq)
        check_step(eng, o, res, want, fsq)
        kv = eng.buffer("kv_k").download(np.float16, 2 * acfg["active_context_length"] * acfg["kv_dim"])
        kv = kv.reshape(2, acfg["active_context_length"], -1)[:, pos].astype(np.float32)
        ref = o.kv_k.view(np.float16).reshape(2, acfg["active_context_length"], -1)[:, pos].astype(np.float32)
        assert np.max(np.abs(kv - ref)) <= 2e-3 * max(1.0, float(np.max(np.abs(ref))))
    st = eng.predict_stop_from_current_lm()
    want = o.stop(o.current_lm)
    assert rel_l2([st.continue_logit, st.stop_logit], want) < 1e-3
    assert st.stop == (st.stop_logit > st.continue_logit)
    base_buf.upload(bases[0])
    st = eng.predict_stop_from_gpu_base(base_buf)
    assert rel_l2([st.continue_logit, st.stop_logit], o.stop(bases[0])) < 1e-3
    eng.close()


def test_fsq_only_and_op(ctx, two_layers):
    acfg, m, model = two_layers
    H, Ld = acfg["embedding_length"], acfg["fsq_latent_dim"]
    eng = ResidualFsqEngine(ctx, model, acfg, strict_geometry=False)
    o = oracle_of(m, acfg)
    b = synth.normal_f32(H, 0x301)
    r = eng.fsq_only(b)
    assert eng.position == 0
    lat, out = o.fsq(b)
    got_lat = eng.buffer("fsq_latent").download(np.float32, Ld)
    assert np.array_equal(got_lat, lat)
    assert rel_l2(eng.buffer("fsq_output").download(np.float32, H), out) < 1e-4
    c, l2 = voxref.stats(got_lat)
    assert r.latent_checksum == pytest.approx(c, rel=1e-9, abs=1e-9) and r.latent_l2 == pytest.approx(l2)
    eng.close()
    # fsq_quantize.comp per-op entry point vs the oracle, away from rounding ties.
    x = synth.normal_f32(1 << 16, 0x302, 0.0, 2.0)
    buf = ctx.array(x)
    abi.call("vx_fsq_quantize", ctx.handle, buf.handle, abi.FsqPush(x.size, 9.0))
    got = buf.download(np.float32, x.size)
    want = voxref.fsq_quantize(x, 9.0)
    t = np.tanh(x.astype(np.float64)) * 9.0
    far = np.abs(np.abs(t - np.trunc(t)) - 0.5) > 1e-5
    assert np.array_equal(got[far], want[far])
    assert np.mean(got == want) > 0.9999


def test_small_geometry_reset_and_graph_cache(ctx, small):
    """hidden 256 (attention merged in its own kernel), F16 stop bias; reset
    replays the same positions; more base buffers than cached graphs."""
    acfg, m, model = small
    H = acfg["embedding_length"]
    eng = ResidualFsqEngine(ctx, model, acfg, exec_mode="graph", strict_geometry=False)
    o = oracle_of(m, acfg)
    bufs = [ctx.array(synth.normal_f32(H, 0x400 + i)) for i in range(10)]
    outs = []
    for pos in range(8):
        b = bufs[pos].download(np.float32, H)
        eng.step_text_prefix_from_gpu_base(bufs[pos])
        want = o.step(b, None, pos, fsq=False)
        assert rel_l2(eng.output(), want["norm"]) < 1e-3, pos
        outs.append(eng.output())
    with pytest.raises(abi.VxError) as e:
        eng.step_text_prefix_from_gpu_base(bufs[8])
    assert e.value.name == "VX_ERR_CONTEXT_FULL"
    eng.reset()
    for pos in range(3):
        eng.step_text_prefix_from_gpu_base(bufs[pos])
        assert np.array_equal(eng.output(), outs[pos])
    eng.reset()
    o2 = oracle_of(m, acfg)
    for pos in range(8):   # 8 + 2 distinct buffers through the 8-entry graph cache
        bb = bufs[(pos + 2) % 10]
        eng.step_text_prefix_from_gpu_base(bb)
        want = o2.step(bb.download(np.float32, H), None, pos, fsq=False)
        assert rel_l2(eng.output(), want["norm"]) < 1e-3, pos
    eng.close()


def test_errors_and_benchmark(ctx, small):
    acfg, m, model = small
    H = acfg["embedding_length"]
    eng = ResidualFsqEngine(ctx, model, acfg, strict_geometry=False)
    with pytest.raises(abi.VxError) as e:
        eng.step(np.zeros(H + 1, np.float32), np.zeros(H + 1, np.float32))
    assert e.value.name == "VX_ERR_SHAPE"
    with pytest.raises(abi.VxError) as e:
        eng.fsq_only(np.zeros(H - 1, np.float32))
    assert e.value.name == "VX_ERR_SHAPE"
    tiny = ctx.zeros(16)
    for f in (lambda: eng.step_text_prefix_from_gpu_base(tiny),
              lambda: eng.step_from_gpu_base(tiny, np.zeros(H, np.float32)),
              lambda: eng.predict_stop_from_gpu_base(tiny)):
        with pytest.raises(abi.VxError) as e:
            f()
        assert e.value.name == "VX_ERR_BOUNDS"
    with pytest.raises(abi.VxError) as e:
        eng.benchmark(np.zeros(H, np.float32), np.zeros(H, np.float32), 0, 0)
    assert e.value.name == "VX_ERR_INVALID_ARG"
    with pytest.raises(abi.VxError) as e:
        eng.benchmark(np.zeros(H, np.float32), np.zeros(H, np.float32), 4, 5)
    assert e.value.name == "VX_ERR_CONTEXT_FULL"
    r = eng.benchmark(synth.normal_f32(H, 1), synth.normal_f32(H, 2), 2, 3)
    assert r["iterations"] == 3 and 0 < r["min_ms"] <= r["mean_ms"] <= r["max_ms"]
    assert eng.position == 5
    kv = 2 * 2 * acfg["active_context_length"] * acfg["kv_dim"] * 2
    assert eng.allocated_bytes() >= model.device_bytes + kv
    eng.close()
    with pytest.raises(abi.VxError) as e:
        ResidualFsqEngine(ctx, model, acfg, strict_geometry=True)
    assert e.value.name == "VX_ERR_UNSUPPORTED"
    bad = dict(acfg, no_rope=0)
    with pytest.raises(abi.VxError) as e:
        ResidualFsqEngine(ctx, model, bad, strict_geometry=False)
    assert e.value.name == "VX_ERR_UNSUPPORTED"


def test_full_contract_steps(ctx):
    """The VoxCPM2 contract (8 layers, strict geometry): FSQ step, text-prefix
    step, FSQ step, against the oracle."""
    acfg = synth.acoustic_config(active_context=32)
    m = synth.build_acoustic(acfg, seed=0x5EED0403)
    model = Model(ctx, m.data, m.tensors)
    H = acfg["embedding_length"]
    eng = ResidualFsqEngine(ctx, model, acfg, strict_geometry=True)
    o = oracle_of(m, acfg)
    buf = ctx.array(np.zeros(H, np.float32))
    for pos, fsq in enumerate((True, False, True)):
        print(f"residual full pos {pos} fsq {fsq}", flush=True)
        b, e = synth.normal_f32(H, 0x500 + pos), synth.normal_f32(H, 0x600 + pos)
        if fsq:
            res = eng.step(b, e)
        else:
            buf.upload(b)
            res = eng.step_text_prefix_from_gpu_base(buf)
        want = o.step(b, e, pos, fsq=fsq)
        check_step(eng, o, res, want, fsq)
    st = eng.predict_stop_from_current_lm()
    assert rel_l2([st.continue_logit, st.stop_logit], o.stop(o.current_lm)) < 1e-3
    eng.close()
    model.free()
