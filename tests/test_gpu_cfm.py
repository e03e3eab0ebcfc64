"""LocDiT estimator, UnifiedCFM solve and the CFM shader entry points on the GPU
against the oracle (voxref.LocDit in float64, voxref CFM functions).

The solve batches each Euler step's conditional and unconditional passes into
one sequence batch of two and replays the whole solve as one hipGraph; the
oracle runs the reference's order (positive pass, negative pass, update).
"""
import ctypes as C

import numpy as np
import pytest

import voxref
from conftest import rel_l2
from voxgen_amd import abi, synth
from voxgen_amd.locdit import CfmOptions, LocDit
from voxgen_amd.runtime import Model

pytestmark = pytest.mark.gpu


def oracle_of(m, cfg):
    return voxref.LocDit(m.data, {t.name: t for t in m.tensors}, cfg)


@pytest.fixture(scope="module")
def ref_shape(ctx):
    """The VoxCPM2 LocDiT layout (mu1, mu2, time, 4 condition, 4 latent tokens;
    16/2 x 128, hidden 1024, ffn 4096) with 2 layers."""
    cfg = synth.locdit_config(layers=2)
    m = synth.build_locdit(cfg, seed=0x5EED0201)
    model = Model(ctx, m.data, m.tensors)
    yield cfg, m, model, oracle_of(m, cfg)
    model.free()


def inputs(cfg, seed):
    x = synth.normal_f32(cfg["patch"] * cfg["feat_dim"], seed)
    cond_n = cfg["n_cond"] * cfg["hidden"] if cfg["cond_raw"] else cfg["patch"] * cfg["feat_dim"]
    cond = synth.normal_f32(cond_n, seed + 1)
    mu = synth.normal_f32(max(cfg["n_mu"], 1) * cfg["hidden"], seed + 2)
    return x, cond, mu


def test_estimate_matches_oracle(ctx, ref_shape):
    cfg, m, model, o = ref_shape
    loc = LocDit(ctx, model, cfg, strict_geometry=False)
    x, cond, mu = inputs(cfg, 0x5EED0202)
    for t, dt in ((0.9, 0.0), (0.3, 0.05)):
        got = loc.estimate(x, cond, mu, t, dt)
        assert rel_l2(got, o.estimate(x, cond, mu, t, dt)) < 1e-4, (t, dt)
    loc.close()


@pytest.mark.parametrize("zero_star", [True, False])
def test_cfm_solve_matches_oracle(ctx, ref_shape, zero_star):
    cfg, m, model, o = ref_shape
    loc = LocDit(ctx, model, cfg, strict_geometry=False)
    _, cond, mu = inputs(cfg, 0x5EED0203)
    opt = CfmOptions(n_timesteps=4, cfg_value=2.0, temperature=1.0, sway_sampling_coef=1.0, seed=1234,
                     use_cfg_zero_star=zero_star)
    got, res = loc.cfm_solve(cond, mu, opt)
    want = o.cfm_solve(cond, mu, n_timesteps=4, cfg_value=2.0, temperature=1.0, sway=1.0, seed=1234,
                       zero_star=zero_star)
    assert rel_l2(got, want) < 1e-4
    assert res["estimator_calls"] == (6 if zero_star else 8)
    assert res["zero_init_steps"] == (1 if zero_star else 0)
    assert abs(res["output_checksum"] - float(np.sum(got, dtype=np.float64))) < 1e-3
    loc.close()


def test_cfm_solve_graph_replay_seeds_and_initial_x(ctx, ref_shape):
    cfg, m, model, o = ref_shape
    loc = LocDit(ctx, model, cfg, strict_geometry=False)
    _, cond, mu = inputs(cfg, 0x5EED0204)
    opt = CfmOptions(n_timesteps=3, seed=7)
    a1, _ = loc.cfm_solve(cond, mu, opt)
    b1, _ = loc.cfm_solve(cond, mu, CfmOptions(n_timesteps=3, seed=8))   # same graph, new seed
    a2, _ = loc.cfm_solve(cond, mu, opt)
    # Replays agree to float rounding (the general stack's split-K projections
    # accumulate with atomics; the short-batch stack replays bit for bit).
    assert rel_l2(a2, a1) < 1e-5 and rel_l2(b1, a1) > 0.1
    assert rel_l2(b1, o.cfm_solve(cond, mu, n_timesteps=3, seed=8)) < 1e-4
    x0 = synth.normal_f32(256, 99)
    c1, _ = loc.cfm_solve(cond, mu, opt, initial_x=x0)
    assert rel_l2(c1, o.cfm_solve(cond, mu, n_timesteps=3, initial_x=x0)) < 1e-4
    loc.close()


def test_cfm_solve_switching_options(ctx, ref_shape):
    """The time-embedding rows are computed outside the solve graph, once per
    option set: solves alternating between step counts, sway coefficients and
    CFG-Zero* on one engine each match the oracle, the profiled (eager) solve
    included."""
    cfg, m, model, o = ref_shape
    loc = LocDit(ctx, model, cfg, strict_geometry=False)
    _, cond, mu = inputs(cfg, 0x5EED020B)
    cases = [dict(n_timesteps=3, sway=1.0, zero_star=True), dict(n_timesteps=5, sway=0.5, zero_star=False),
             dict(n_timesteps=3, sway=1.0, zero_star=True), dict(n_timesteps=3, sway=0.0, zero_star=True)]
    for i, k in enumerate(cases):
        opt = CfmOptions(n_timesteps=k["n_timesteps"], sway_sampling_coef=k["sway"], use_cfg_zero_star=k["zero_star"],
                         seed=21 + i)
        if i == 3:
            ctx.prof_enable(True)
        got, _ = loc.cfm_solve(cond, mu, opt)
        if i == 3:
            ctx.prof_enable(False)
        want = o.cfm_solve(cond, mu, n_timesteps=k["n_timesteps"], sway=k["sway"], zero_star=k["zero_star"],
                           seed=21 + i)
        assert rel_l2(got, want) < 1e-4, (i, k)
    # The graph cached by case 2 replays after the profiled solve left other rows in temb.
    got, _ = loc.cfm_solve(cond, mu, CfmOptions(n_timesteps=3, sway_sampling_coef=1.0, use_cfg_zero_star=True,
                                                seed=30))
    assert rel_l2(got, o.cfm_solve(cond, mu, n_timesteps=3, sway=1.0, zero_star=True, seed=30)) < 1e-4
    loc.close()


def test_cfm_solve_8_layers_16x64_cond32(ctx):
    """The benchmark's LocDiT shape: 8 layers, 16 x 64 MHA, 32 given condition rows
    zeroed in the unconditional pass, no mu tokens; 10 timesteps, cfg 2.0."""
    cfg = synth.locdit_config(layers=8, q_heads=16, kv_heads=16, head_dim=64, n_mu=0, n_cond=32, cond_raw=1,
                              uncond_zero_cond=1)
    m = synth.build_locdit(cfg, seed=0x5EED0205)
    model = Model(ctx, m.data, m.tensors)
    o = oracle_of(m, cfg)
    loc = LocDit(ctx, model, cfg, strict_geometry=False)
    _, cond, _ = inputs(cfg, 0x5EED0206)
    got, res = loc.cfm_solve(cond, None, CfmOptions(seed=42))
    want = o.cfm_solve(cond, None, seed=42)
    assert res["estimator_calls"] == 18
    assert rel_l2(got, want) < 1e-4
    loc.close()
    model.free()


@pytest.mark.parametrize("n_mu,n_cond,q_heads,kv_heads,head_dim", [(0, 1, 16, 2, 128), (2, 9, 16, 2, 128),
                                                                    (2, 9, 16, 16, 64), (2, 10, 16, 2, 128)])
def test_cfm_solve_short_sequences(ctx, n_mu, n_cond, q_heads, kv_heads, head_dim):
    """Sequences of 6, 16 and 17 tokens (n_mu + time + n_cond + 4 latent rows): the
    fused attention's 16-token instantiation at both ends (scores and softmax in
    one pass, the projection over 512 workgroups, the residual-stream stack) and,
    at 17 tokens, the general one of the slab stack; 3 timesteps against the
    oracle."""
    cfg = synth.locdit_config(layers=2, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, n_mu=n_mu,
                              n_cond=n_cond, cond_raw=1, uncond_zero_cond=1)
    m = synth.build_locdit(cfg, seed=0x5EED0209 + n_cond)
    model = Model(ctx, m.data, m.tensors)
    o = oracle_of(m, cfg)
    loc = LocDit(ctx, model, cfg, strict_geometry=False)
    _, cond, mu = inputs(cfg, 0x5EED020A + n_cond)
    mu = mu if n_mu else None
    got, res = loc.cfm_solve(cond, mu, CfmOptions(n_timesteps=3, seed=11))
    want = o.cfm_solve(cond, mu, n_timesteps=3, seed=11)
    assert rel_l2(got, want) < 1e-4
    loc.close()
    model.free()


@pytest.mark.parametrize("hidden,patch,fused", [(2048, 8, False), (4096, 2, True)])
def test_cfm_solve_residual_stream_wide_rows(ctx, hidden, patch, fused):
    """Residual-stream stack at the out_proj + Euler launch's LDS limit: at hidden
    4096 and patch 2 its 4 stream rows fill the 64 KB exactly and the launch folds
    the final rmsnorm in; at hidden 2048 and patch 8 the 16 rows (128 KB) do not
    fit, so the final rmsnorm runs and that launch reads the normed rows; 3
    timesteps against the oracle."""
    cfg = synth.locdit_config(layers=2, hidden=hidden, q_heads=16, kv_heads=2, head_dim=128,
                              ffn=1024 if fused else 2048, patch=patch, n_mu=0, n_cond=1, cond_raw=1,
                              uncond_zero_cond=1)
    m = synth.build_locdit(cfg, seed=0x5EED020C + patch)
    model = Model(ctx, m.data, m.tensors)
    o = oracle_of(m, cfg)
    loc = LocDit(ctx, model, cfg, strict_geometry=False)
    _, cond, _ = inputs(cfg, 0x5EED020D + patch)
    want = o.cfm_solve(cond, None, n_timesteps=3, seed=5)
    got, _ = loc.cfm_solve(cond, None, CfmOptions(n_timesteps=3, seed=5))
    assert rel_l2(got, want) < 1e-4
    ctx.prof_reset()
    ctx.prof_enable(True)
    got, _ = loc.cfm_solve(cond, None, CfmOptions(n_timesteps=3, seed=5))
    ctx.prof_enable(False)
    spans = ctx.prof_snapshot()
    assert rel_l2(got, want) < 1e-4
    # The residual stream: no per-layer residual rmsnorm.
    assert "local.seq_residual_rmsnorm" not in spans
    if fused:   # one out_proj + Euler launch per step, the final norm folded in
        assert "local.seq_rmsnorm" not in spans and spans["local.out_cfg_euler"]["calls"] > 0
    else:   # the final rmsnorm once per step, then out_proj and the Euler update
        assert "local.out_cfg_euler" not in spans
        assert spans["local.seq_rmsnorm"]["calls"] == spans["local.cfm_cfg_euler"]["calls"] > 0
    loc.close()
    model.free()


def test_cfm_solve_general_stack_long_condition(ctx):
    """66 tokens per sequence (61 given condition rows): past the fused dense
    attention's 64 tokens, so the solve takes the general layer stack (k_gemm with
    split-K accumulators, the three-kernel dense attention) instead of the
    short-batch one; 3 timesteps against the oracle."""
    cfg = synth.locdit_config(layers=2, hidden=256, q_heads=4, kv_heads=2, head_dim=64, ffn=512, n_mu=0, n_cond=61,
                              cond_raw=1, uncond_zero_cond=1)
    m = synth.build_locdit(cfg, seed=0x5EED0207)
    model = Model(ctx, m.data, m.tensors)
    o = oracle_of(m, cfg)
    loc = LocDit(ctx, model, cfg, strict_geometry=False)
    _, cond, _ = inputs(cfg, 0x5EED0208)
    got, res = loc.cfm_solve(cond, None, CfmOptions(n_timesteps=3, seed=7))
    want = o.cfm_solve(cond, None, n_timesteps=3, seed=7)
    assert rel_l2(got, want) < 1e-4
    loc.close()
    model.free()


def test_strict_geometry_and_errors(ctx, ref_shape):
    cfg, m, model, o = ref_shape
    with pytest.raises(abi.VxError) as e:
        LocDit(ctx, model, cfg, strict_geometry=True)   # 2 layers != 12
    assert e.value.name == "VX_ERR_UNSUPPORTED"
    with pytest.raises(abi.VxError) as e:
        LocDit(ctx, model, dict(cfg, layers=3), strict_geometry=False)
    assert e.value.name == "VX_ERR_NOT_FOUND"
    loc = LocDit(ctx, model, cfg, strict_geometry=False)
    x, cond, mu = inputs(cfg, 5)
    bad = cond.copy()
    bad[3] = np.nan
    with pytest.raises(abi.VxError) as e:
        loc.cfm_solve(bad, mu)
    assert e.value.name == "VX_ERR_INVALID_ARG"
    with pytest.raises(abi.VxError) as e:
        loc.cfm_solve(cond, mu, CfmOptions(n_timesteps=0))
    assert e.value.name == "VX_ERR_INVALID_ARG"
    with pytest.raises(abi.VxError) as e:
        loc.cfm_solve(cond, mu, CfmOptions(temperature=-1.0))
    assert e.value.name == "VX_ERR_INVALID_ARG"
    with pytest.raises(abi.VxError) as e:
        loc.estimate(x, cond, mu, float("inf"), 0.0)
    assert e.value.name == "VX_ERR_INVALID_ARG"
    loc.close()


def test_cfm_shader_entry_points(ctx):
    n = 256
    xb = ctx.zeros(n * 4)
    push = abi.CfmNoisePush(n, 0x89ABCDEF, 0x01234567, 0.8)
    abi.call("vx_cfm_noise", ctx.handle, xb.handle, C.byref(push))
    assert rel_l2(xb.download(np.float32, n), voxref.cfm_noise(push)) < 1e-6
    x, p, q = synth.normal_f32(n, 1), synth.normal_f32(n, 2), synth.normal_f32(n, 3)
    xb2, pb, qb = ctx.array(x), ctx.array(p), ctx.array(q)
    ep = abi.CfmEulerPush(n, 0.1, 2.0, 1)
    abi.call("vx_cfm_cfg_euler", ctx.handle, xb2.handle, pb.handle, qb.handle, C.byref(ep))
    assert rel_l2(xb2.download(np.float32, n), voxref.cfm_cfg_euler(x, p, q, ep)) < 1e-6
    # The shader is one 256-lane workgroup: the entry point refuses a longer latent.
    big = ctx.zeros(257 * 4)
    with pytest.raises(abi.VxError) as e:
        abi.call("vx_cfm_cfg_euler", ctx.handle, big.handle, big.handle, big.handle,
                 C.byref(abi.CfmEulerPush(257, 0.1, 2.0, 1)))
    assert e.value.name == "VX_ERR_UNSUPPORTED"
    tb = ctx.zeros(1024 * 4)
    tp = abi.TimePush(1024, 0.42)
    abi.call("vx_time_sinusoidal", ctx.handle, tb.handle, C.byref(tp))
    assert np.max(np.abs(tb.download(np.float32, 1024) - voxref.time_sinusoidal(tp))) < 1e-3
    H, P = 1024, 4
    parts = [synth.normal_f32(k, s) for k, s in ((H, 11), (H, 12), (H, 13), (P * H, 14), (P * H, 15))]
    bufs = [ctx.array(v) for v in parts]
    hb = ctx.zeros((3 + 2 * P) * H * 4)
    for zero in (0, 1):
        pp = abi.PackLocDitPush(H, P, zero)
        abi.call("vx_pack_locdit", ctx.handle, *[b.handle for b in bufs], hb.handle, C.byref(pp))
        assert np.array_equal(hb.download(np.float32, (3 + 2 * P) * H), voxref.pack_locdit(*parts, pp))
    sb = ctx.array(p * 3)
    abi.call("vx_silu_inplace", ctx.handle, sb.handle, n)
    pd = p.astype(np.float64) * 3
    assert rel_l2(sb.download(np.float32, n), pd / (1 + np.exp(-pd))) < 1e-6
    ab = ctx.array(x)
    abi.call("vx_add_vectors", ctx.handle, ab.handle, pb.handle, n)
    assert np.array_equal(ab.download(np.float32, n), x + p)


def test_cfm_from_model_hiddens_matches_chained_oracles(ctx, ref_shape):
    """cfm_from_model_hiddens (local.rs:379-381): the mu tokens are projected on
    the device from the ResidualLM engine's current_lm and output buffers
    (runtime.rs:239-243) inside the solve's graph. BaseLM (2 Q8_0 layers) ->
    ResidualLM (2 F16 layers, an FSQ step after a text-prefix step) -> LocDiT
    (reference layout, 2 layers), against the oracles chained the same way."""
    from voxgen_amd.baselm import BaseLmEngine
    from voxgen_amd.residual import ResidualFsqEngine
    cfg, m, model, o = ref_shape
    bcfg = synth.baselm_config(layers=2, vocab=512, context_length=256, active_context=256)
    bm = synth.build_baselm(bcfg, seed=0x5EED0240)
    acfg = synth.acoustic_config(layers=2, active_context=64)
    am = synth.build_acoustic(acfg, seed=0x5EED0241)
    bmodel, amodel = Model(ctx, bm.data, bm.tensors), Model(ctx, am.data, am.tensors)
    base = BaseLmEngine(ctx, bmodel, bcfg, strict_geometry=False)
    res = ResidualFsqEngine(ctx, amodel, acfg, strict_geometry=False)
    ob = voxref.BaseLm(bm.data, {t.name: t for t in bm.tensors}, bcfg)
    orr = voxref.ResidualFsq(am.data, {t.name: t for t in am.tensors}, acfg)
    toks = [int(t) for t in synth.uniform_u32(2, 0x5EED0242, 512)]
    emb = synth.normal_f32(2048, 0x5EED0243)
    # The chain up to the LocDiT inputs: each engine against its oracle, the
    # ResidualLM oracle fed the GPU's BaseLM rows (FSQ is a rounding: identical
    # inputs keep the latent exact instead of letting a tie flip it).
    base.decode_token_gpu_only(toks[0])
    b0 = base.buffer("norm").download(np.float32, 2048)
    assert rel_l2(b0, ob.decode_token(toks[0], 0)) < 5e-3
    res.step_text_prefix_from_gpu_base_gpu_only(base.buffer("norm"))
    orr.step(b0, None, 0, fsq=False)
    base.decode_token_gpu_only(toks[1])
    b1 = base.buffer("norm").download(np.float32, 2048)
    assert rel_l2(b1, ob.decode_token(toks[1], 1)) < 5e-3
    res.step_from_gpu_base(base.buffer("norm"), emb)
    want_step = orr.step(b1, emb, 1, fsq=True)
    ctx.sync()
    lm = res.current_lm_buffer().download(np.float32, 2048)
    out = res.output_buffer().download(np.float32, 2048)
    assert rel_l2(lm, want_step["fsq"]) < 1e-4
    assert rel_l2(out, want_step["norm"]) < 1e-3
    loc = LocDit(ctx, model, cfg, strict_geometry=False)
    _, cond, _ = inputs(cfg, 0x5EED0244)
    opt = CfmOptions(n_timesteps=4, cfg_value=2.0, temperature=1.0, sway_sampling_coef=1.0, seed=77,
                     use_cfg_zero_star=True)
    got, info = loc.cfm_from_model_hiddens(res.current_lm_buffer(), res.output_buffer(), cond, opt)
    mu = o.project_mu(lm, out)                           # the projection of the same device vectors, f64
    want = o.cfm_solve(cond, mu, n_timesteps=4, cfg_value=2.0, temperature=1.0, sway=1.0, seed=77,
                       zero_star=True)
    assert rel_l2(got, want) < 1e-3
    assert info["estimator_calls"] == 6
    host, _ = loc.cfm_solve(cond, mu.astype(np.float32), opt)  # the host-mu entry on the same mu
    assert rel_l2(got, host) < 1e-4
    # A replay reads the buffers' current contents: another step changes mu and the result.
    base.decode_token_gpu_only(toks[0])
    res.step_from_gpu_base(base.buffer("norm"), emb)
    ctx.sync()
    got2, _ = loc.cfm_from_model_hiddens(res.current_lm_buffer(), res.output_buffer(), cond, opt)
    mu2 = o.project_mu(res.current_lm_buffer().download(np.float32, 2048), res.output_buffer().download(np.float32, 2048))
    want2 = o.cfm_solve(cond, mu2, n_timesteps=4, cfg_value=2.0, temperature=1.0, sway=1.0, seed=77, zero_star=True)
    assert rel_l2(got2, want2) < 1e-3 and rel_l2(got2, got) > 1e-3
    with pytest.raises(abi.VxError) as e:
        loc.cfm_from_model_hiddens(res.current_lm_buffer(), ctx.zeros(1024), cond, opt)
    assert e.value.name in ("VX_ERR_BOUNDS", "VX_ERR_SHAPE")
    for x in (loc, res, base):
        x.close()
    bmodel.free()
    amodel.free()


def test_cfm_from_model_hiddens_needs_the_projections(ctx):
    cfg = synth.locdit_config(layers=1)
    m = synth.build_locdit(cfg, seed=0x5EED0250, with_mu_proj=False)
    model = Model(ctx, m.data, m.tensors)
    loc = LocDit(ctx, model, cfg, strict_geometry=False)
    _, cond, _ = inputs(cfg, 0x5EED0251)
    with pytest.raises(abi.VxError) as e:
        loc.cfm_from_model_hiddens(ctx.zeros(8192), ctx.zeros(8192), cond)
    assert e.value.name == "VX_ERR_NOT_FOUND"
    loc.close()
    with pytest.raises(abi.VxError) as e:  # the reference's contract requires them (local.rs:141-144)
        LocDit(ctx, model, synth.locdit_config(layers=1), strict_geometry=True)
    assert e.value.name in ("VX_ERR_NOT_FOUND", "VX_ERR_UNSUPPORTED")
    model.free()


def test_cfm_solve_at_the_reference_contract_strict(ctx):
    """The reference's enforced LocDiT geometry (LocalConfig::from_gguf,
    local.rs:37-48,85-92): 12 layers x 1024, 16/2 x 128, ffn 4096, mu1 + mu2 +
    time + 4 condition + 4 latent tokens, strict geometry on, against the oracle
    (host mu and model-hidden mu)."""
    cfg = synth.locdit_config()
    m = synth.build_locdit(cfg, seed=0x5EED0260)
    model = Model(ctx, m.data, m.tensors)
    o = oracle_of(m, cfg)
    loc = LocDit(ctx, model, cfg, strict_geometry=True)
    _, cond, mu = inputs(cfg, 0x5EED0261)
    opt = CfmOptions(n_timesteps=4, cfg_value=2.0, temperature=1.0, sway_sampling_coef=1.0, seed=9,
                     use_cfg_zero_star=True)
    got, info = loc.cfm_solve(cond, mu, opt)
    want = o.cfm_solve(cond, mu, n_timesteps=4, cfg_value=2.0, temperature=1.0, sway=1.0, seed=9, zero_star=True)
    assert rel_l2(got, want) < 1e-3 and info["estimator_calls"] == 6
    h1, h2 = ctx.array(synth.normal_f32(2048, 0x5EED0262)), ctx.array(synth.normal_f32(2048, 0x5EED0263))
    got_h, _ = loc.cfm_from_model_hiddens(h1, h2, cond, opt)
    mu_h = o.project_mu(h1.download(np.float32, 2048), h2.download(np.float32, 2048))
    want_h = o.cfm_solve(cond, mu_h, n_timesteps=4, cfg_value=2.0, temperature=1.0, sway=1.0, seed=9, zero_star=True)
    assert rel_l2(got_h, want_h) < 1e-3
    loc.close()
    model.free()
