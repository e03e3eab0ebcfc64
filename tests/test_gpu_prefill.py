"""Token-batched BaseLM prefill and the seq_* / dense_* per-op entry points.

The batched prefill (MFMA projections with exact Q8_0 weights and f16 hi/lo
activations, causal attention over the cache) must leave the engine in the state
prefill_tokens (baselm.rs:823-839) leaves it in: the oracle's sequential decode
of the same tokens gives the reference KV-cache rows, final hidden state and
logits. The per-op entry points are checked token by token against the oracle's
per-token functions (seq_linear_bias.comp is linear_bias.comp per token, and so
on) and the dense attention against its f64 closed form.
"""
import ctypes as C

import numpy as np
import pytest

import voxref
from conftest import rel_l2
from voxgen_amd import abi, synth
from voxgen_amd.baselm import BaseLmEngine, config_struct
from voxgen_amd.runtime import Model

pytestmark = pytest.mark.gpu


def kv_rows(eng, name, layers, ctxlen, kv_dim=256):
    return eng.buffer(name).download(np.uint16, layers * ctxlen * kv_dim).reshape(layers, ctxlen, kv_dim)


def f16(bits):
    return np.asarray(bits).view(np.float16).astype(np.float64)


@pytest.fixture(scope="module")
def small(ctx):
    """Two layers of the full VoxCPM2 geometry (Q8_0), context 1024."""
    cfg = synth.baselm_config(layers=2, vocab=4096, context_length=32768, active_context=1024)
    m = synth.build_baselm(cfg, seed=0x5EED0101)
    model = Model(ctx, m.data, m.tensors)
    yield cfg, m, model
    model.free()


def oracle_of(m, cfg):
    return voxref.BaseLm(m.data, {t.name: t for t in m.tensors}, cfg)


# ---------------------------------------------------------------- engine
@pytest.mark.parametrize("n", [1, 37, 130])
def test_batched_prefill_matches_sequential_oracle(ctx, small, n):
    cfg, m, model = small
    o = oracle_of(m, cfg)
    toks = [int(t) for t in synth.uniform_u32(n, 0x5EED0102 + n, cfg["vocab_size"])]
    print(f"batched prefill n={n}", flush=True)
    eng = BaseLmEngine(ctx, model, cfg, exec_mode="graph", strict_geometry=False)
    r = eng.prefill_tokens_batched(toks, top_k_last=5)
    for p, t in enumerate(toks):
        o.decode_token(t, p, logits=(p == n - 1))
    assert r.position == n - 1 and eng.position == n
    assert rel_l2(eng.output(), o.norm) < 1e-3
    assert rel_l2(eng.buffer("hidden").download(np.float32, 2048), o.hidden) < 1e-3
    assert rel_l2(eng.buffer("logits").download(np.float32, cfg["vocab_size"]), o.logits) < 1e-3
    assert [t for t, _ in r.top_logits][:3] == list(np.argsort(-o.logits, kind="stable")[:3])
    for name, ref in (("kv_k", o.kv_k), ("kv_v", o.kv_v)):
        got = kv_rows(eng, name, 2, 1024)
        want = ref.reshape(2, 1024, 256)
        for l in range(2):
            assert rel_l2(f16(got[l, :n]), f16(want[l, :n])) < 1e-3, (name, l)
        assert np.all(got[:, n:] == 0)
    eng.close()


def test_batched_prefill_gate_up_schedules(ctx, small):
    """The gate/up projection's workgroup schedules over 300 tokens: 3 token tiles x
    96 tiles of 64 gate/up rows = 288 tiles, just above 256 CUs, so "auto" runs the
    stream-K kernel. "streamk_tail_first" runs its other hand-off path (the tail
    stores and counts, the head finishes) and must give the same bits; "tiles"
    (one tile per workgroup) sums each tile's blocks in one chain instead of two
    parts, so it differs by fp32 rounding only. All three against the oracle."""
    cfg, m, model = small
    n = 300
    toks = [int(t) for t in synth.uniform_u32(n, 0x5EED010A, cfg["vocab_size"])]
    o = oracle_of(m, cfg)
    for p, t in enumerate(toks):
        o.decode_token(t, p)
    got = {}
    for sched in ("auto", "streamk_tail_first", "tiles"):
        print(f"batched prefill n={n} schedule={sched}", flush=True)
        eng = BaseLmEngine(ctx, model, cfg, exec_mode="graph", strict_geometry=False, prefill_schedule=sched)
        eng.prefill_tokens_batched(toks)
        got[sched] = (eng.output(), kv_rows(eng, "kv_k", 2, 1024)[:, :n], kv_rows(eng, "kv_v", 2, 1024)[:, :n])
        eng.close()
        assert rel_l2(got[sched][0], o.norm) < 1e-3, sched
        for l in range(2):
            assert rel_l2(f16(got[sched][1][l]), f16(o.kv_k.reshape(2, 1024, 256)[l, :n])) < 1e-3, (sched, l)
            assert rel_l2(f16(got[sched][2][l]), f16(o.kv_v.reshape(2, 1024, 256)[l, :n])) < 1e-3, (sched, l)
    for x, y in zip(got["auto"], got["streamk_tail_first"]):
        assert np.array_equal(x, y)
    assert rel_l2(got["auto"][0], got["tiles"][0]) < 1e-4
    assert np.array_equal(got["auto"][1][0], got["tiles"][1][0])   # layer 0's K rows precede any gate/up
    assert rel_l2(f16(got["auto"][2][1]), f16(got["tiles"][2][1])) < 1e-3
    opt = abi.BaseLmOptions(abi.EXEC_GRAPH, 0, 0, 3)   # no such schedule
    h = abi.ENGINE()
    with pytest.raises(abi.VxError) as err:
        abi.call("vx_baselm_create", ctx.handle, model.handle, C.byref(config_struct(cfg)), C.byref(opt), C.byref(h))
    assert err.value.name == "VX_ERR_INVALID_ARG" and "prefill_schedule" in str(err.value)


def test_batched_prefill_gate_up_half_tiles(ctx, small):
    """512 tokens (a full prefill chunk): 4 token tiles x 96 = 384 gate/up tiles, 1.5
    per 256 CUs, so "auto" runs 256 whole tiles and 128 tiles as two K halves that
    hand over through the part slots. Against "tiles" (one tile per workgroup; fp32
    rounding only) and the oracle."""
    cfg, m, model = small
    n = 512
    toks = [int(t) for t in synth.uniform_u32(n, 0x5EED010B, cfg["vocab_size"])]
    o = oracle_of(m, cfg)
    for p, t in enumerate(toks):
        o.decode_token(t, p)
    got = {}
    for sched in ("auto", "tiles"):
        print(f"batched prefill n={n} schedule={sched}", flush=True)
        eng = BaseLmEngine(ctx, model, cfg, exec_mode="graph", strict_geometry=False, prefill_schedule=sched)
        eng.prefill_tokens_batched(toks)
        got[sched] = (eng.output(), kv_rows(eng, "kv_v", 2, 1024)[:, :n])
        eng.close()
        assert rel_l2(got[sched][0], o.norm) < 1e-3, sched
        for l in range(2):
            assert rel_l2(f16(got[sched][1][l]), f16(o.kv_v.reshape(2, 1024, 256)[l, :n])) < 1e-3, (sched, l)
    assert rel_l2(got["auto"][0], got["tiles"][0]) < 1e-4
    assert rel_l2(f16(got["auto"][1][1]), f16(got["tiles"][1][1])) < 1e-3


def test_batched_prefill_continues_a_decode_and_spans_chunks(ctx, small):
    """Prefill at a non-zero position, longer than one 512-token chunk, then decode on."""
    cfg, m, model = small
    o = oracle_of(m, cfg)
    toks = [int(t) for t in synth.uniform_u32(606, 0x5EED0103, cfg["vocab_size"])]
    eng = BaseLmEngine(ctx, model, cfg, exec_mode="graph", strict_geometry=False)
    for p in range(3):
        eng.decode_token(toks[p])
        o.decode_token(toks[p], p)
    print("batched prefill of 600 tokens at position 3", flush=True)
    eng.prefill_tokens_batched_gpu_only(toks[3:603])
    for p in range(3, 603):
        o.decode_token(toks[p], p)
    assert eng.position == 603
    assert rel_l2(eng.output(), o.norm) < 1e-3
    for p in range(603, 606):
        eng.decode_token(toks[p])
        assert rel_l2(eng.output(), o.decode_token(toks[p], p)) < 1e-3, p
    got = kv_rows(eng, "kv_k", 2, 1024)
    want = o.kv_k.reshape(2, 1024, 256)
    for l in range(2):
        assert rel_l2(f16(got[l, :606]), f16(want[l, :606])) < 1e-3, l
    eng.close()


def test_batched_prefill_f16_weights(ctx):
    cfg = synth.baselm_config(layers=2, vocab=2048, context_length=32768, active_context=256)
    m = synth.build_baselm(cfg, seed=0x5EED0104, weight_type="f16")
    model = Model(ctx, m.data, m.tensors)
    o = oracle_of(m, cfg)
    toks = [int(t) for t in synth.uniform_u32(70, 0x5EED0105, 2048)]
    eng = BaseLmEngine(ctx, model, cfg, exec_mode="graph", strict_geometry=False)
    eng.prefill_tokens_batched(toks)
    for p, t in enumerate(toks):
        o.decode_token(t, p)
    assert rel_l2(eng.output(), o.norm) < 1e-3
    got = kv_rows(eng, "kv_v", 2, 256)
    assert rel_l2(f16(got[:, :70]), f16(o.kv_v.reshape(2, 256, 256)[:, :70])) < 1e-3
    eng.close()
    model.free()


def test_batched_prefill_errors(ctx, small):
    cfg, m, model = small
    eng = BaseLmEngine(ctx, model, dict(cfg, active_context_length=64), exec_mode="graph", strict_geometry=False)
    with pytest.raises(abi.VxError) as e:
        eng.prefill_tokens_batched([1, 2, cfg["vocab_size"]])
    assert e.value.name == "VX_ERR_TOKEN_RANGE"
    with pytest.raises(abi.VxError) as e:
        eng.prefill_tokens_batched([])
    assert e.value.name == "VX_ERR_INVALID_ARG"
    eng.prefill_tokens_batched_gpu_only(list(range(60)))
    with pytest.raises(abi.VxError) as e:
        eng.prefill_tokens_batched(list(range(5)))
    assert e.value.name == "VX_ERR_CONTEXT_FULL"
    assert eng.position == 60
    eng.close()


@pytest.fixture(scope="module")
def full(ctx):
    cfg = synth.baselm_config(active_context=512)
    m = synth.build_baselm(cfg, seed=0x5EED0106)
    model = Model(ctx, m.data, m.tensors)
    yield cfg, m, model
    model.free()


def test_full_stack_prefill_32_tokens_against_oracle(ctx, full):
    cfg, m, model = full
    o = oracle_of(m, cfg)
    toks = [int(t) for t in synth.uniform_u32(32, 0x5EED0107, cfg["vocab_size"])]
    eng = BaseLmEngine(ctx, model, cfg, exec_mode="graph", strict_geometry=True)
    r = eng.prefill_tokens_batched(toks, top_k_last=5)
    for p, t in enumerate(toks):
        o.decode_token(t, p, logits=(p == 31))
    assert rel_l2(eng.output(), o.norm) < 5e-3
    assert [t for t, _ in r.top_logits][:3] == list(np.argsort(-o.logits, kind="stable")[:3])
    got = kv_rows(eng, "kv_k", 28, 512)
    want = o.kv_k.reshape(28, 512, 256)
    assert rel_l2(f16(got[:, :32]), f16(want[:, :32])) < 5e-3
    eng.close()


def test_full_stack_prefill_384_matches_sequential_decode(ctx, full):
    """The T = 384 prefill workload: batched prefill against the oracle's
    sequential decode of the same 384 tokens (prefill_tokens, baselm.rs:823-839:
    final hidden, every layer's K/V rows, the last token's top logits), and
    against the same engine's sequential decode."""
    cfg, m, model = full
    toks = [int(t) for t in synth.uniform_u32(384, 0x5EED0108, cfg["vocab_size"])]
    o = oracle_of(m, cfg)
    for p, t in enumerate(toks):
        o.decode_token(t, p, logits=(p == 383))
    okv_k = o.kv_k.reshape(28, 512, 256)[:, :384]
    okv_v = o.kv_v.reshape(28, 512, 256)[:, :384]
    seq = BaseLmEngine(ctx, model, cfg, exec_mode="graph", strict_geometry=True)
    seq.prefill_tokens(toks)
    want_out = seq.output()
    want_k = kv_rows(seq, "kv_k", 28, 512)[:, :384]
    want_v = kv_rows(seq, "kv_v", 28, 512)[:, :384]
    seq.close()
    eng = BaseLmEngine(ctx, model, cfg, exec_mode="graph", strict_geometry=True)
    r = eng.prefill_tokens_batched(toks, top_k_last=5)
    assert eng.position == 384
    # against the oracle
    assert rel_l2(eng.output(), o.norm) < 5e-3
    assert [t for t, _ in r.top_logits][:3] == list(np.argsort(-o.logits, kind="stable")[:3])
    gk, gv = kv_rows(eng, "kv_k", 28, 512)[:, :384], kv_rows(eng, "kv_v", 28, 512)[:, :384]
    for l in range(28):
        assert rel_l2(f16(gk[l]), f16(okv_k[l])) < 5e-3, l
        assert rel_l2(f16(gv[l]), f16(okv_v[l])) < 5e-3, l
    # and against the engine's own sequential decode
    assert rel_l2(eng.output(), want_out) < 5e-3
    got_k = kv_rows(eng, "kv_k", 28, 512)[:, :384]
    got_v = kv_rows(eng, "kv_v", 28, 512)[:, :384]
    assert rel_l2(f16(got_k[0]), f16(want_k[0])) < 1e-3  # layer 0 sees only the projections
    for l in range(28):
        assert rel_l2(f16(got_k[l]), f16(want_k[l])) < 5e-3, l
        assert rel_l2(f16(got_v[l]), f16(want_v[l])) < 5e-3, l
    eng.close()


# ---------------------------------------------------------------- per-op
def tokens_x(T, cols, stride, base, seed):
    x = np.zeros(base + (T - 1) * stride + cols, np.float32)
    for t in range(T):
        x[base + t * stride: base + t * stride + cols] = synth.normal_f32(cols, seed + t)
    return x


@pytest.mark.parametrize("T,base,stride", [(1, 0, 2048), (64, 0, 2048), (100, 8, 2056), (7, 1, 2049)])
def test_seq_linear_bias_q8(ctx, small, T, base, stride):
    cfg, m, model = small
    t = m.tensor("blk.0.attn_q.weight")
    b = m.tensor("blk.1.attn_norm.weight")
    x = tokens_x(T, 2048, stride, base, 0x5EED0110)
    for has_bias in (0, 1):
        push = abi.SeqLinearPush(t.offset, b.offset, 2048, 2048, abi.DTYPE_Q8_0, 0, T, stride, 2050, base, 3,
                                 has_bias, 0.5)
        xb = ctx.array(x)
        yb = ctx.zeros((3 + (T - 1) * 2050 + 2048) * 4)
        abi.call("vx_seq_linear_bias", ctx.handle, model.handle, xb.handle, yb.handle, C.byref(push))
        y = yb.download(np.float32, 3 + (T - 1) * 2050 + 2048)
        for tok in range(T):
            lp = abi.LinearBiasPush(t.offset, b.offset if has_bias else 0, 2048, 2048, abi.DTYPE_Q8_0, 0, 0, 0.5)
            want = voxref.linear_bias(m.data, x[base + tok * stride: base + tok * stride + 2048], lp) if has_bias \
                else 0.5 * voxref.matvec(m.data, x[base + tok * stride: base + tok * stride + 2048],
                                         abi.MatvecPush(t.offset, 2048, 2048, abi.DTYPE_Q8_0, 0, 1.0))
            got = y[3 + tok * 2050: 3 + tok * 2050 + 2048]
            assert rel_l2(got, want) < (1e-4 if base % 4 == 0 else 1e-5), (tok, has_bias)


def test_seq_linear_bias_f16_and_f32_weights(ctx, small):
    cfg, m, model = small
    emb = m.tensor("token_embd.weight")   # F16 [4096, 2048] used as a 300-row matrix
    x = tokens_x(40, 2048, 2048, 0, 0x5EED0111)
    xb = ctx.array(x)
    yb = ctx.zeros(40 * 300 * 4)
    push = abi.SeqLinearPush(emb.offset, 0, 300, 2048, abi.DTYPE_F16, 0, 40, 2048, 300, 0, 0, 0, 1.0)
    abi.call("vx_seq_linear_bias", ctx.handle, model.handle, xb.handle, yb.handle, C.byref(push))
    y = yb.download(np.float32, 40 * 300).reshape(40, 300)
    W = voxref.dequant(m.data, emb.offset, abi.DTYPE_F16, 300, 2048).astype(np.float64)
    assert rel_l2(y, x.reshape(40, 2048).astype(np.float64) @ W.T) < 1e-5
    # F32 weights (a 64-float vector as a one-row matrix) take the generic kernel.
    rf = m.tensor("rope_factors_short.weight")
    xs = synth.normal_f32(64 * 3, 5)
    push = abi.SeqLinearPush(rf.offset, 0, 1, 64, abi.DTYPE_F32, 0, 3, 64, 1, 0, 0, 0, 2.0)
    yb2 = ctx.zeros(16)
    xsb = ctx.array(xs)  # keep the buffer alive across the call (a temporary would be freed first)
    abi.call("vx_seq_linear_bias", ctx.handle, model.handle, xsb.handle, yb2.handle, C.byref(push))
    assert rel_l2(yb2.download(np.float32, 3), 2.0 * xs.reshape(3, 64).sum(axis=1)) < 1e-6


def test_seq_qkv_and_swiglu(ctx, small):
    cfg, m, model = small
    T = 72
    x = tokens_x(T, 2048, 2048, 0, 0x5EED0112)
    xb = ctx.array(x)
    q, k, v = ctx.zeros(T * 2048 * 4), ctx.zeros(T * 256 * 4), ctx.zeros(T * 256 * 4)
    o = {n: m.tensor(f"blk.1.{n}.weight").offset for n in ("attn_q", "attn_k", "attn_v", "ffn_gate", "ffn_up")}
    push = abi.SeqQkvPush(o["attn_q"], o["attn_k"], o["attn_v"], 2048, 256, 2048, T, 2048, 2048, 256, 0)
    abi.call("vx_seq_qkv", ctx.handle, model.handle, xb.handle, q.handle, k.handle, v.handle, C.byref(push))
    qg = q.download(np.float32, T * 2048).reshape(T, 2048)
    kg = k.download(np.float32, T * 256).reshape(T, 256)
    vg = v.download(np.float32, T * 256).reshape(T, 256)
    qp = abi.QkvPush(o["attn_q"], o["attn_k"], o["attn_v"], 2048, 256, 2048, 8, 8, 8, 0)
    for t in (0, 1, 33, T - 1):
        wq, wk, wv = voxref.qkv_matvec(m.data, x[t * 2048:(t + 1) * 2048], qp)
        assert rel_l2(qg[t], wq) < 1e-4 and rel_l2(kg[t], wk) < 1e-4 and rel_l2(vg[t], wv) < 1e-4, t
    y = ctx.zeros(T * 6144 * 4)
    sp = abi.SeqSwigluPush(o["ffn_gate"], o["ffn_up"], 6144, 2048, T, 2048, 6144, 0, 0)
    abi.call("vx_seq_swiglu", ctx.handle, model.handle, xb.handle, y.handle, C.byref(sp))
    yg = y.download(np.float32, T * 6144).reshape(T, 6144)
    wp = abi.SwigluPush(o["ffn_gate"], o["ffn_up"], 6144, 2048, 8, 0)
    for t in (0, 5, T - 1):
        assert rel_l2(yg[t], voxref.matvec_swiglu(m.data, x[t * 2048:(t + 1) * 2048], wp)) < 1e-4, t


def test_seq_norms_rope_and_silu(ctx, small):
    cfg, m, model = small
    T = 9
    w = m.tensor("blk.0.ffn_norm.weight").offset
    x = tokens_x(T, 2048, 2048, 0, 0x5EED0113) * 3.0
    br = tokens_x(T, 2048, 2048, 0, 0x5EED0114)
    xb, yb = ctx.array(x), ctx.zeros(T * 2048 * 4)
    abi.call("vx_seq_rmsnorm", ctx.handle, model.handle, xb.handle, yb.handle,
             C.byref(abi.SeqRmsPush(w, 2048, T, 2048, 2048, 0, 0, 1e-6)))
    y = yb.download(np.float32, T * 2048).reshape(T, 2048)
    for t in range(T):
        assert rel_l2(y[t], voxref.rmsnorm(m.data, x[t * 2048:(t + 1) * 2048], abi.RmsPush(w, 2048, 1e-6))) < 1e-6
    hb, bb = ctx.array(x), ctx.array(br)
    abi.call("vx_seq_residual_rmsnorm", ctx.handle, model.handle, hb.handle, bb.handle, yb.handle,
             C.byref(abi.SeqResidualRmsPush(w, 2048, T, 2048, 2048, 2048, 0, 0, 0, 1e-6, 0.7)))
    y = yb.download(np.float32, T * 2048).reshape(T, 2048)
    h = hb.download(np.float32, T * 2048).reshape(T, 2048)
    for t in range(T):
        wh, wy = voxref.residual_rmsnorm(m.data, x[t * 2048:(t + 1) * 2048], br[t * 2048:(t + 1) * 2048],
                                         abi.ResidualRmsPush(w, 2048, 1e-6, 0.7))
        assert rel_l2(h[t], wh) < 1e-6 and rel_l2(y[t], wy) < 1e-6
    # RoPE: seq_rope is token t at position t; seq_rope_at adds a base.
    rf = m.tensor("rope_factors_short.weight").offset
    q = tokens_x(T, 2048, 2048, 0, 0x5EED0115)
    k = tokens_x(T, 256, 256, 0, 0x5EED0116)
    for base in (0, 700):
        qb, kb = ctx.array(q), ctx.array(k)
        push = abi.SeqRopePush(rf, T, 16, 2, 128, 2048, 256, 10000.0, 1.0)
        if base:
            abi.call("vx_seq_rope_at", ctx.handle, model.handle, qb.handle, kb.handle, base, C.byref(push))
        else:
            abi.call("vx_seq_rope", ctx.handle, model.handle, qb.handle, kb.handle, C.byref(push))
        qg = qb.download(np.float32, T * 2048).reshape(T, 2048)
        kg = kb.download(np.float32, T * 256).reshape(T, 256)
        for t in range(T):
            wq, wk = voxref.rope(m.data, q[t * 2048:(t + 1) * 2048], k[t * 256:(t + 1) * 256],
                                 abi.RopePush(rf, base + t, 16, 2, 128, 10000.0, 1.0))
            assert rel_l2(qg[t], wq) < 1e-4 and rel_l2(kg[t], wk) < 1e-4, (base, t)
    g = synth.normal_f32(1000, 1) * 4
    u = synth.normal_f32(1000, 2)
    gb, ub = ctx.array(g), ctx.array(u)
    abi.call("vx_seq_silu_mul", ctx.handle, gb.handle, ub.handle, 1000)
    gd = g.astype(np.float64)
    assert rel_l2(gb.download(np.float32, 1000), gd / (1 + np.exp(-gd)) * u) < 1e-6


@pytest.mark.parametrize("T,qh,kvh,hd", [(11, 16, 2, 128), (36, 16, 16, 64), (1, 4, 1, 64)])
def test_dense_attention(ctx, T, qh, kvh, hd):
    stride_s = T + 3
    q = synth.normal_f32(T * qh * hd, 0x5EED0117 + T)
    k = synth.normal_f32(T * kvh * hd, 0x5EED0118 + T)
    v = synth.normal_f32(T * kvh * hd, 0x5EED0119 + T)
    qb, kb, vb = ctx.array(q), ctx.array(k), ctx.array(v)
    sb = ctx.zeros(T * qh * stride_s * 4)
    ob = ctx.zeros(T * qh * hd * 4)
    abi.call("vx_dense_attn_scores", ctx.handle, qb.handle, kb.handle, sb.handle,
             C.byref(abi.DenseScoresPush(T, qh, kvh, hd, qh * hd, kvh * hd, stride_s)))
    abi.call("vx_dense_softmax", ctx.handle, sb.handle, C.byref(abi.DenseSoftmaxPush(T, qh, stride_s)))
    abi.call("vx_dense_attn_values", ctx.handle, sb.handle, vb.handle, ob.handle,
             C.byref(abi.DenseValuesPush(T, qh, kvh, hd, qh * hd, kvh * hd, stride_s)))
    Q = q.reshape(T, qh, hd).astype(np.float64)
    K = k.reshape(T, kvh, hd).astype(np.float64)
    V = v.reshape(T, kvh, hd).astype(np.float64)
    kvmap = np.arange(qh) // (qh // kvh)
    S = np.einsum("thd,shd->ths", Q, K[:, kvmap, :]) / np.sqrt(hd)
    P = np.exp(S - S.max(axis=2, keepdims=True))
    P /= P.sum(axis=2, keepdims=True)
    O = np.einsum("ths,shd->thd", P, V[:, kvmap, :])
    got_p = sb.download(np.float32, T * qh * stride_s).reshape(T, qh, stride_s)[:, :, :T]
    assert rel_l2(got_p, P) < 1e-5
    assert rel_l2(ob.download(np.float32, T * qh * hd).reshape(T, qh, hd), O) < 1e-5
