"""vx_fused_attention_noalloc: the fused attention entry point that allocates nothing.

Its output must equal vx_fused_attention's (same kernels, the caller's workspace
replaced by the per-GPU scratch) on consecutive calls, the second one smaller, so
whatever the first call left in the scratch cannot leak into the second. It is
also captured into a HIP graph (where any allocation would break the capture) and
replayed with eager work in between, every replay checked against the eager
result.
"""
import ctypes as C

import numpy as np
import pytest

import voxref
from conftest import rel_l2
from voxgen_amd import abi, synth

pytestmark = pytest.mark.gpu


def _case(ctx, L, ctxlen, hd, kvh, qpk, pos, splits, seed):
    qh = kvh * qpk
    kc = synth.normal_f16(L * ctxlen * kvh * hd, seed).view(np.uint16).copy()
    vc = synth.normal_f16(L * ctxlen * kvh * hd, seed + 1).view(np.uint16).copy()
    q = (synth.normal_f32(qh * hd, seed + 2) * 0.5).astype(np.float32)
    a = abi.FusedAttnArgs(L - 1, ctxlen, hd, qh, kvh, splits)
    bufs = dict(q=ctx.array(q), kc=ctx.array(kc), vc=ctx.array(vc), pos=ctx.array(np.array([pos], np.uint32)),
                ref=ctx.zeros(qh * hd * 4), na=ctx.zeros(qh * hd * 4))
    ap = abi.AttentionPush(L - 1, ctxlen, pos, hd, qpk, kvh)
    s = voxref.attn_scores(q, kc, qh, ap)
    pr = voxref.softmax(s, qh, abi.SoftmaxPush(ctxlen, pos))
    want = voxref.attn_values(pr, vc, qh, ap)
    return a, bufs, want, qh * hd


def _with_workspace(ctx, a, b):
    ws = ctx.zeros(abi.load().vx_fused_attention_scratch_bytes(C.byref(a)))
    abi.call("vx_fused_attention", ctx.handle, b["q"].handle, b["kc"].handle, b["vc"].handle, b["ref"].handle,
             ws.handle, b["pos"].handle, C.byref(a))
    return ws


def _noalloc(ctx, a, b):
    abi.call("vx_fused_attention_noalloc", ctx.handle, b["q"].handle, b["kc"].handle, b["vc"].handle,
             b["na"].handle, b["pos"].handle, C.byref(a))


def test_noalloc_attention_matches_workspace_entry_on_two_calls(ctx):
    # First call: 16 heads x 64 splits at position 1500 (541 KB of partials);
    # second, smaller: 4 heads x 8 splits, head_dim 64, position 100.
    for (L, ctxlen, hd, kvh, qpk, pos, splits, seed) in ((2, 2048, 128, 2, 8, 1500, 64, 0x5EED0700),
                                                         (1, 512, 64, 1, 4, 100, 8, 0x5EED0710)):
        a, b, want, n = _case(ctx, L, ctxlen, hd, kvh, qpk, pos, splits, seed)
        assert abi.load().vx_fused_attention_scratch_bytes(C.byref(a)) <= abi.NOALLOC_SCRATCH_BYTES
        _with_workspace(ctx, a, b)
        _noalloc(ctx, a, b)
        ctx.sync()
        ref = b["ref"].download(np.float32, n)
        got = b["na"].download(np.float32, n)
        assert np.array_equal(got, ref), (pos, splits)      # same kernels, same inputs: bit for bit
        assert rel_l2(got, want) < 1e-3                      # and the oracle's attention


def test_noalloc_attention_replays_in_a_graph(ctx):
    a, b, want, n = _case(ctx, 2, 1024, 128, 2, 8, 700, 16, 0x5EED0720)
    _noalloc(ctx, a, b)
    ctx.sync()
    eager = b["na"].download(np.float32, n)
    ctx.graph_begin()
    _noalloc(ctx, a, b)
    g = ctx.graph_end()
    try:
        for r in range(3):
            b["na"].upload(np.full(n, np.nan, np.float32))
            # eager work on the same scratch between replays: a smaller call
            a2, b2, _, n2 = _case(ctx, 1, 256, 64, 1, 4, 37 + r, 4, 0x5EED0730 + r)
            _noalloc(ctx, a2, b2)
            ctx.graph_launch(g)
            ctx.sync()
            assert np.array_equal(b["na"].download(np.float32, n), eager), r
    finally:
        ctx.graph_free(g)
    assert rel_l2(eager, want) < 1e-3


def test_noalloc_attention_refuses_more_than_its_scratch(ctx):
    # 64 heads x 64 splits x 132 floats needs 2.06 MiB of partials, above the 2 MiB scratch.
    a, b, _, _ = _case(ctx, 1, 64, 128, 8, 8, 10, 64, 0x5EED0740)
    assert abi.load().vx_fused_attention_scratch_bytes(C.byref(a)) > abi.NOALLOC_SCRATCH_BYTES
    with pytest.raises(abi.VxError) as e:
        _noalloc(ctx, a, b)
    assert e.value.name == "VX_ERR_BOUNDS"
