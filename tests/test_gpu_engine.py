"""BaseLM engine parity (graph, fused-eager and reference op order) against the
oracle.

One decoder layer at context 512 (the single-layer benchmark workload), short
multi-layer sequences from position 0 through every decode entry point, error
conditions, and the full 28-layer VoxCPM2 geometry.
"""
import numpy as np
import pytest

import voxref
from conftest import rel_l2
from voxgen_amd import abi, synth
from voxgen_amd.baselm import BaseLmEngine
from voxgen_amd.runtime import Model

pytestmark = pytest.mark.gpu
MODES = ["graph", "fused", "reference"]


def kv_bits(layers, ctxlen, filled, seed):
    k = synth.kv_cache_fill(layers, ctxlen, 256, filled, seed).view(np.uint16).ravel().copy()
    v = synth.kv_cache_fill(layers, ctxlen, 256, filled, seed + 1).view(np.uint16).ravel().copy()
    return k, v


@pytest.fixture(scope="module")
def one_layer(ctx):
    cfg = synth.baselm_config(layers=1, vocab=1024, context_length=32768, active_context=1024)
    m = synth.build_baselm(cfg, seed=0x5EED0001)
    model = Model(ctx, m.data, m.tensors)
    yield cfg, m, model
    model.free()


@pytest.mark.parametrize("mode", MODES)
def test_one_layer_decode_at_context_512(ctx, one_layer, mode):
    cfg, m, model = one_layer
    kk, vv = kv_bits(1, 1024, 512, 0x5EED0011)
    eng = BaseLmEngine(ctx, model, cfg, exec_mode=mode, strict_geometry=False)
    eng.buffer("kv_k").upload(kk)
    eng.buffer("kv_v").upload(vv)
    eng.set_position(512)
    r = eng.decode_token(321, top_k=5)
    o = voxref.BaseLm(m.data, {t.name: t for t in m.tensors}, cfg)
    o.kv_k[:] = kk
    o.kv_v[:] = vv
    want = o.decode_token(321, 512, logits=True)
    assert r.position == 512 and eng.position == 513
    for name, ref in (("q", o.q), ("k", o.k), ("v", o.v), ("attention", o.attention), ("hidden", o.hidden)):
        got = eng.buffer(name).download(np.float32, ref.size)
        assert rel_l2(got, ref) < 1e-3, name
    got = eng.output()
    assert rel_l2(got, want) < 1e-3
    assert abs(r.final_hidden_checksum - float(np.sum(got, dtype=np.float64))) < 1e-6 * max(1, abs(r.final_hidden_checksum))
    assert rel_l2(eng.buffer("logits").download(np.float32, 1024), o.logits) < 1e-3
    assert [t for t, _ in r.top_logits] == list(np.argsort(-o.logits, kind="stable")[:5])
    # Cache: every row except position 512 is untouched; row 512 matches the oracle.
    kg = eng.buffer("kv_k").download(np.uint16, kk.size).reshape(1024, 256)
    vg = eng.buffer("kv_v").download(np.uint16, vv.size).reshape(1024, 256)
    keep = np.arange(1024) != 512
    assert np.array_equal(kg[keep], kk.reshape(1024, 256)[keep])
    assert np.array_equal(vg[keep], vv.reshape(1024, 256)[keep])
    assert rel_l2(kg[512].view(np.float16), o.kv_k.reshape(1024, 256)[512].view(np.float16)) < 1e-3
    assert rel_l2(vg[512].view(np.float16), o.kv_v.reshape(1024, 256)[512].view(np.float16)) < 1e-3
    eng.close()


@pytest.fixture(scope="module")
def two_layers(ctx):
    cfg = synth.baselm_config(layers=2, vocab=2048, context_length=32768, active_context=64)
    m = synth.build_baselm(cfg, seed=0x5EED0003)
    model = Model(ctx, m.data, m.tensors)
    yield cfg, m, model
    model.free()


@pytest.mark.parametrize("mode", MODES)
def test_sequence_from_position_zero(ctx, two_layers, mode):
    cfg, m, model = two_layers
    eng = BaseLmEngine(ctx, model, cfg, exec_mode=mode, strict_geometry=False)
    o = voxref.BaseLm(m.data, {t.name: t for t in m.tensors}, cfg)
    toks = synth.uniform_u32(6, 0x5EED0004, 2048)
    for pos, t in enumerate(toks):
        r = eng.decode_token(int(t))
        assert r.position == pos
        assert rel_l2(eng.output(), o.decode_token(int(t), pos)) < 1e-3, pos
    kg = eng.buffer("kv_k").download(np.uint16, o.kv_k.size).reshape(2, 64, 256)
    kw = o.kv_k.reshape(2, 64, 256)
    assert rel_l2(kg[:, :6].view(np.float16), kw[:, :6].view(np.float16)) < 1e-3
    assert np.all(kg[:, 6:] == 0)
    eng.close()


def test_entry_points_match_oracle(ctx, two_layers):
    cfg, m, model = two_layers
    eng = BaseLmEngine(ctx, model, cfg, exec_mode="graph", strict_geometry=False)
    o = voxref.BaseLm(m.data, {t.name: t for t in m.tensors}, cfg)
    toks = [int(t) for t in synth.uniform_u32(12, 0x5EED0005, 2048)]
    # decode_tokens_gpu_only: several steps with no host wait.
    eng.decode_tokens_gpu_only(toks[:4])
    for p in range(4):
        o.decode_token(toks[p], p)
    assert eng.position == 4 and rel_l2(eng.output(), o.norm) < 1e-3
    # decode_token_gpu_only
    assert eng.decode_token_gpu_only(toks[4]) == 4
    assert rel_l2(eng.output(), o.decode_token(toks[4], 4)) < 1e-3
    # decode_embedding (host f32 input) and its gpu_only form
    emb = synth.normal_f32(2048, 77, 0.0, 0.5)
    r = eng.decode_embedding(emb, top_k=3)
    o.hidden[:] = emb
    want = o.record(5, logits=True)
    assert r.position == 5 and rel_l2(eng.output(), want) < 1e-3
    assert [t for t, _ in r.top_logits] == list(np.argsort(-o.logits, kind="stable")[:3])
    assert eng.decode_embedding_gpu_only(emb * 2) == 6
    o.hidden[:] = emb * 2
    assert rel_l2(eng.output(), o.record(6)) < 1e-3
    # decode_embedding_from_gpu_only
    src = ctx.array(emb * -1)
    assert eng.decode_embedding_from_gpu_only(src) == 7
    o.hidden[:] = -emb
    assert rel_l2(eng.output(), o.record(7)) < 1e-3
    # prefill_tokens: sequential decode, top_k of the last token
    r = eng.prefill_tokens(toks[8:12], top_k_last=4)
    for i, t in enumerate(toks[8:12]):
        o.decode_token(t, 8 + i, logits=(i == 3))
    assert r.position == 11 and eng.position == 12
    assert rel_l2(eng.output(), o.norm) < 1e-3
    assert [t for t, _ in r.top_logits] == list(np.argsort(-o.logits, kind="stable")[:4])
    eng.close()


def test_engine_errors(ctx, two_layers):
    cfg, m, model = two_layers
    small = dict(cfg, active_context_length=3)
    eng = BaseLmEngine(ctx, model, small, exec_mode="graph", strict_geometry=False)
    with pytest.raises(abi.VxError) as e:
        eng.decode_token(2048)
    assert e.value.name == "VX_ERR_TOKEN_RANGE"
    with pytest.raises(abi.VxError) as e:
        eng.decode_embedding(np.zeros(100, np.float32))
    assert e.value.name == "VX_ERR_SHAPE"
    for t in (1, 2, 3):
        eng.decode_token(t)
    with pytest.raises(abi.VxError) as e:
        eng.decode_token(4)
    assert e.value.name == "VX_ERR_CONTEXT_FULL"
    with pytest.raises(abi.VxError) as e:
        eng.decode_tokens_gpu_only([1])
    assert e.value.name == "VX_ERR_CONTEXT_FULL"
    with pytest.raises(abi.VxError) as e:
        eng.benchmark(1, 2, 2)
    assert e.value.name == "VX_ERR_CONTEXT_FULL"
    eng.reset()
    assert eng.position == 0
    eng.decode_token(5)
    eng.close()
    with pytest.raises(abi.VxError) as e:
        BaseLmEngine(ctx, model, cfg, strict_geometry=True)
    assert e.value.name == "VX_ERR_UNSUPPORTED"
    bad = dict(cfg, vocab_size=100)
    with pytest.raises(abi.VxError) as e:
        BaseLmEngine(ctx, model, bad, strict_geometry=False)
    assert e.value.name == "VX_ERR_SHAPE"


def test_benchmark_and_profile(ctx, two_layers):
    cfg, m, model = two_layers
    eng = BaseLmEngine(ctx, model, cfg, exec_mode="graph", strict_geometry=False)
    b = eng.benchmark(7, 2, 5)
    assert b["iterations"] == 5 and b["tokens_per_second"] > 0 and b["min_ms"] <= b["mean_ms"] <= b["max_ms"]
    assert eng.position == 7
    prof = eng.profile_steps([1, 2, 3])
    for name in ("baselm.embedding", "baselm.qkv", "baselm.attention", "baselm.attn_out", "baselm.swiglu",
                 "baselm.down", "baselm.output_norm"):
        assert name in prof and prof[name]["calls"] >= 3 and prof[name]["avg_ms"] > 0
    assert prof["baselm.qkv"]["calls"] == 6
    eng.close()


@pytest.fixture(scope="module")
def full_model(ctx):
    cfg = synth.baselm_config(active_context=512)
    m = synth.build_baselm(cfg, seed=0x5EED0002)
    model = Model(ctx, m.data, m.tensors)
    o = voxref.BaseLm(m.data, {t.name: t for t in m.tensors}, cfg)
    yield cfg, m, model, o
    model.free()


def test_full_stack_from_position_zero(ctx, full_model):
    cfg, m, model, o = full_model
    toks = [int(t) for t in synth.uniform_u32(3, 0x5EED0006, cfg["vocab_size"])]
    wants, tops = [], []
    for pos, t in enumerate(toks):
        wants.append(o.decode_token(t, pos, logits=True))
        tops.append(list(np.argsort(-o.logits, kind="stable")[:5]))
    for mode in ("graph",):
        eng = BaseLmEngine(ctx, model, cfg, exec_mode=mode, strict_geometry=True)
        for pos, t in enumerate(toks):
            r = eng.decode_token(t, top_k=5)
            assert rel_l2(eng.output(), wants[pos]) < 5e-3, (mode, pos)
            assert [t for t, _ in r.top_logits][:3] == tops[pos][:3], mode
        eng.close()


def test_full_stack_decode_at_position_256(ctx, full_model):
    """28 layers with a 256-token cache (the decode benchmark's first timed position)."""
    cfg, m, model, o = full_model
    kk, vv = kv_bits(28, 512, 256, 0x5EED0007)
    toks = [int(t) for t in synth.uniform_u32(2, 0x5EED0008, cfg["vocab_size"])]
    o.kv_k[:] = kk
    o.kv_v[:] = vv
    wants = [o.decode_token(t, 256 + i) for i, t in enumerate(toks)]
    for mode in ("graph", "reference"):
        eng = BaseLmEngine(ctx, model, cfg, exec_mode=mode, strict_geometry=True)
        eng.buffer("kv_k").upload(kk)
        eng.buffer("kv_v").upload(vv)
        eng.set_position(256)
        for t, w in zip(toks, wants):
            eng.decode_token_gpu_only(t)
            assert rel_l2(eng.output(), w) < 5e-3, mode
        eng.close()


def test_persistent_mode_is_refused(ctx, two_layers):
    """The one-kernel persistent step is not built (its in-kernel phase hand-offs
    cost more than kernel boundaries on MI355X): the mode is a clear error."""
    cfg, m, model = two_layers
    with pytest.raises(abi.VxError) as e:
        BaseLmEngine(ctx, model, cfg, exec_mode="persistent", strict_geometry=False)
    assert e.value.name == "VX_ERR_UNSUPPORTED" and "persistent" in str(e.value)


def test_timeline_entry_points_need_the_timeline_build(ctx):
    """The shipped library has no per-wave stamps in its kernels: the timeline
    diagnostics (a -DVX_STAMPS build's) are a clear error there."""
    import ctypes as C
    if abi.load().vx_diag_timeline_arm(ctx.handle, 1024) == 0:
        pytest.skip("this is the -DVX_STAMPS build")
    assert "VX_STAMPS" in abi.load().vx_last_error().decode()
    nl, nw = C.c_uint64(7), C.c_uint64(7)
    with pytest.raises(abi.VxError) as e:
        abi.call("vx_diag_timeline_read", ctx.handle, None, 0, None, 0, C.byref(nl), C.byref(nw))
    assert e.value.name == "VX_ERR_UNSUPPORTED" and nl.value == 0 and nw.value == 0


def test_gguf_file_through_the_loader_decodes_like_the_oracle(ctx, full_model, tmp_path):
    """The real load path: the 28-layer model written as a GGUF v3 file, parsed by
    vx_gguf_open (load_summary, gguf.rs:222-286), configured by
    vx_baselm_config_from_gguf (BaseLmConfig::from_gguf, baselm.rs:60-180),
    uploaded by vx_model_upload_gguf (data region + Q8_0 repack) and decoded."""
    from voxgen_amd import gguf
    from voxgen_amd.gguf import Gguf
    cfg, m, _, o = full_model
    p = gguf.write(tmp_path / "baselm.gguf", m.metadata, m.tensors, m.data)
    g = Gguf(p)
    fcfg = g.baselm_config(cfg["active_context_length"])
    for k in ("embedding_length", "block_count", "feed_forward_length", "head_count", "head_count_kv",
              "head_dim", "vocab_size", "context_length"):
        assert fcfg[k] == cfg[k], k
    model = Model.from_gguf(ctx, g)
    try:
        eng = BaseLmEngine(ctx, model, fcfg, exec_mode="graph", strict_geometry=True)
        toks = [int(t) for t in synth.uniform_u32(2, 0x5EED000A, cfg["vocab_size"])]
        for pos, t in enumerate(toks):
            want = o.decode_token(t, pos, logits=True)
            r = eng.decode_token(t, top_k=3)
            assert rel_l2(eng.output(), want) < 5e-3, pos
            assert [i for i, _ in r.top_logits][:3] == list(np.argsort(-o.logits, kind="stable")[:3])
        eng.close()
    finally:
        model.free()
        g.close()


def test_cancellation_flag_stops_steps_before_they_are_enqueued(ctx, two_layers):
    """synthesize_cancelable's flag (runtime.rs:745-808): set before a step, the
    step fails with VX_ERR_CANCELLED and the engine position does not move; the
    steps already taken stay, and clearing the flag resumes decoding where it
    stopped, matching the oracle."""
    cfg, m, model = two_layers
    eng = BaseLmEngine(ctx, model, cfg, exec_mode="graph", strict_geometry=False)
    o = voxref.BaseLm(m.data, {t.name: t for t in m.tensors}, cfg)
    toks = [int(t) for t in synth.uniform_u32(6, 0x5EED000B, 2048)]
    try:
        eng.decode_tokens_gpu_only(toks[:2])
        for p in range(2):
            o.decode_token(toks[p], p)
        ctx.set_cancelled(True)
        for call in (lambda: eng.decode_token(toks[2]), lambda: eng.decode_token_gpu_only(toks[2]),
                     lambda: eng.decode_tokens_gpu_only(toks[2:4]), lambda: eng.prefill_tokens(toks[2:4]),
                     lambda: eng.prefill_tokens_batched(toks[2:4]),
                     lambda: eng.decode_embedding(synth.normal_f32(2048, 5, 0.0, 0.5))):
            with pytest.raises(abi.VxError) as e:
                call()
            assert e.value.name == "VX_ERR_CANCELLED" and "cancelled" in str(e.value)
            assert eng.position == 2
        ctx.set_cancelled(False)
        for p in (2, 3):
            r = eng.decode_token(toks[p])
            assert r.position == p
            assert rel_l2(eng.output(), o.decode_token(toks[p], p)) < 1e-3, p
    finally:
        ctx.set_cancelled(False)
        eng.close()
