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


# ------------------------------------------------------- batched text prefix
def _kv(eng, acfg, which, n):
    L, ctxlen, kv = acfg["residual_block_count"], acfg["active_context_length"], acfg["kv_dim"]
    c = eng.buffer(which).download(np.float16, L * ctxlen * kv).reshape(L, ctxlen, kv)
    return c[:, :n].astype(np.float32)


def test_prefill_from_rows_matches_per_position_steps(ctx):
    """600 text-prefix positions from given rows (two chunks, a partial 128-row
    tile) against the per-position text-prefix step, which the tests above pin to
    the oracle; then one FSQ step on top of each cache."""
    acfg = synth.acoustic_config(layers=2, active_context=640)
    m = synth.build_acoustic(acfg, seed=0x5EED0405)
    model = Model(ctx, m.data, m.tensors)
    H, n = acfg["embedding_length"], 600
    rows = synth.normal_f32(n * H, 0x700).reshape(n, H)
    rbuf = ctx.array(rows)
    one = ctx.array(np.zeros(H, np.float32))
    seq = ResidualFsqEngine(ctx, model, acfg, exec_mode="graph", strict_geometry=False)
    for t in range(n):
        one.upload(rows[t])
        seq.step_text_prefix_from_gpu_base_gpu_only(one)
    bat = ResidualFsqEngine(ctx, model, acfg, exec_mode="fused", strict_geometry=False)
    bat.prefill_text_from_gpu_rows(rbuf, n)
    ctx.sync()
    assert bat.position == n
    for name in ("output", "hidden", "fusion_snapshot", "current_lm"):
        a, b = bat.buffer(name).download(np.float32, H), seq.buffer(name).download(np.float32, H)
        assert rel_l2(a, b) < 1e-3, name
    for which in ("kv_k", "kv_v"):
        a, b = _kv(bat, acfg, which, n), _kv(seq, acfg, which, n)
        for l in range(2):
            assert rel_l2(a[l], b[l]) < 1e-3, (which, l)
    base, emb = ctx.array(synth.normal_f32(H, 0x701)), ctx.array(synth.normal_f32(H, 0x702))
    seq.step_from_gpu_base_and_embedding(base, emb)
    bat.step_from_gpu_base_and_embedding(base, emb)
    assert rel_l2(bat.output(), seq.output()) < 1e-3
    with pytest.raises(abi.VxError) as e:
        bat.prefill_text_from_gpu_rows(rbuf, 40)
    assert e.value.name == "VX_ERR_CONTEXT_FULL"
    ref = ResidualFsqEngine(ctx, model, acfg, exec_mode="reference", strict_geometry=False)
    with pytest.raises(abi.VxError) as e:
        ref.prefill_text_from_gpu_rows(rbuf, 4)
    assert e.value.name == "VX_ERR_STATE"
    for x in (seq, bat, ref):
        x.close()
    model.free()


def test_cross_engine_text_prefill_matches_sequential_and_oracle(ctx):
    """BaseLM (2 Q8_0 layers) + ResidualLM (2 F16 layers) text prefix of 37
    tokens: batched per engine vs one decode + one text-prefix step per token, and
    the last ResidualLM output vs the oracles chained the same way."""
    from voxgen_amd.baselm import BaseLmEngine
    from voxgen_amd.residual import prefill_text_cross_engine
    bcfg = synth.baselm_config(layers=2, vocab=512, context_length=256, active_context=256)
    bm = synth.build_baselm(bcfg, seed=0x5EED0406)
    bmodel = Model(ctx, bm.data, bm.tensors)
    acfg = synth.acoustic_config(layers=2, active_context=256)
    am = synth.build_acoustic(acfg, seed=0x5EED0407)
    amodel = Model(ctx, am.data, am.tensors)
    tokens = synth.uniform_u32(37, 0x703, 512)
    H = acfg["embedding_length"]
    b1 = BaseLmEngine(ctx, bmodel, bcfg, strict_geometry=False)
    r1 = ResidualFsqEngine(ctx, amodel, acfg, strict_geometry=False)
    for t in tokens:
        b1.decode_token_gpu_only(int(t))
        r1.step_text_prefix_from_gpu_base_gpu_only(b1.buffer("norm"))
    b2 = BaseLmEngine(ctx, bmodel, bcfg, strict_geometry=False)
    r2 = ResidualFsqEngine(ctx, amodel, acfg, strict_geometry=False)
    prefill_text_cross_engine(b2, r2, tokens)
    ctx.sync()
    assert b2.position == 37 and r2.position == 37
    assert rel_l2(b2.output(), b1.output()) < 1e-3
    for name in ("output", "current_lm", "fusion_snapshot"):
        assert rel_l2(r2.buffer(name).download(np.float32, H), r1.buffer(name).download(np.float32, H)) < 1e-3, name
    for which in ("kv_k", "kv_v"):
        a, b = _kv(r2, acfg, which, 37), _kv(r1, acfg, which, 37)
        assert rel_l2(a, b) < 1e-3, which
    ob = voxref.BaseLm(bm.data, {t.name: t for t in bm.tensors}, bcfg)
    orr = oracle_of(am, acfg)
    for pos, t in enumerate(tokens):
        row = ob.decode_token(int(t), pos)
        want = orr.step(row, None, pos, fsq=False)
    assert rel_l2(r2.output(), want["norm"]) < 5e-3
    r3 = ResidualFsqEngine(ctx, amodel, dict(acfg, embedding_length=H), strict_geometry=False)
    small = synth.baselm_config(layers=1, hidden=256, ffn=512, vocab=64, q_heads=2, kv_heads=1, context_length=64,
                                active_context=64)
    sm = synth.build_baselm(small, seed=3)
    smodel = Model(ctx, sm.data, sm.tensors)
    b3 = BaseLmEngine(ctx, smodel, small, strict_geometry=False)
    with pytest.raises(abi.VxError) as e:
        prefill_text_cross_engine(b3, r3, tokens[:4])
    assert e.value.name == "VX_ERR_SHAPE"
    for x in (b1, r1, b2, r2, r3, b3):
        x.close()
    for x in (bmodel, amodel, smodel):
        x.free()
