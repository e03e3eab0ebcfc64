"""Benchmark: VoxCPM2 BaseLM Q8_0 decode at batch 1 on one MI355X.

Workload (the 28-layer decode benchmark): hidden 2048, 28 layers, 16/2 heads x
128, FFN 6144, vocab 73448, Q8_0 weights (d = f16(|N(0,1)|*0.01), q ~ U[-127,127]),
F16 tied embedding N(0,0.02). A 256-token prefill fills the KV cache, then K
decode steps at positions 256..256+K-1 with token ids uniform from the vocab;
each step is one hipGraph replay of the fused decode step (LM head off, the
*_gpu_only semantics). A "step" is one decoded token.

Prints one JSON line with:
  value        tok/s over the K timed graph replays (inputs resident in HBM)
  roofline     the dominant kernel (the gate/up SwiGLU matvec): algorithmic bytes
               per launch / its average duration, measured with two HIP events on
               the engine stream around back-to-back launches over all 28 layers;
               roofline.rocprof is the same kernel's average duration in the
               committed rocprofv3 trace (profiles/kernels_decode28_q8.json)
  per_kernel   the same measurement for every kernel of the decode layer
  c0           the single Q8_0 2048x2048 matvec (matvec.comp) over 64 distinct
               copies (285 MB, beyond the 256 MB MALL) and hot in cache
  achievable   the best plain streaming-read GB/s of this GPU (1 GiB read), the
               practical ceiling next to the 8 TB/s spec
  latency      the reference's own benchmark semantics (BaseLmEngine::benchmark,
               baselm.rs:841-880): decode_token with the tied LM head and a host
               wait per token
  cpu_baseline the CPU oracle's decode throughput on a bounded sample
  prefill      the token-batched prefill of 384 tokens through the 28 layers
               (MFMA projections, causal attention over the cache): wall time and
               each kernel's HIP-event span, with the projection GEMMs' algorithmic
               TFLOP/s against the 2.5 PFLOP/s dense f16 MFMA peak
  cfm          the LocDiT flow-matching solve (8 layers, hidden 1024, CFG batch
               2, 10 timesteps): solve time and weight-streaming GB/s; and the
               same solve at the reference's 12-layer, 11-token geometry
  residual     the ResidualLM step (FSQ + fusion + 8 F16 layers without RoPE,
               hidden 2048): steps/s and weight-streaming GB/s
  audiovae     the AudioVAE decode of 40 latent frames (1.6 s of 48 kHz audio):
               time, real-time factor and GEMM-form TFLOP/s

  long_context the decode at --max-context 8192, positions 512..8000: tok/s and
               the attention and attn_out cost per layer

`--copy-calibration` instead runs one plain copy kernel of known size (the
reference point for the FETCH_SIZE / WRITE_SIZE counters); `--timeline` the
graph-mode per-kernel timelines of a -DVX_STAMPS build (the decode step, and the
LocDiT CFM solve).
"""
from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402

HBM_PEAK_GBPS = 8000.0
METRIC = "Q8_0 BaseLM decode tok/s @ batch 1; matvec HBM GB/s (% of 8 TB/s peak)"

# Decode geometry.
H, KV, F, L, V = 2048, 256, 6144, 28, 73448


def q8(rows, cols):
    """GGUF Q8_0 bytes of a rows x cols matrix (34 B per 32 weights)."""
    return rows * cols // 32 * 34


# Algorithmic HBM bytes per launch of each layer kernel (weights, activations in
# and out, KV-cache traffic); attention depends on the position.
KERNEL_BYTES = {
    # Wq|Wk|Wv + hidden + attn_norm + q/k/v out + K/V cache row writes
    "qkv": q8(H + 2 * KV, H) + 2 * H * 4 + (H + 2 * KV) * 4 + 2 * KV * 2,
    # Wo + attention vector + hidden read and write
    "attn_out": q8(H, H) + H * 4 + 2 * H * 4,
    # Wgate|Wup + hidden + ffn_norm + gate out
    "swiglu": 2 * q8(F, H) + 2 * H * 4 + F * 4,
    # Wdown + gate vector + hidden read and write
    "down": q8(H, F) + F * 4 + 2 * H * 4,
}


def attention_bytes(pos):
    """K and V rows 0..pos of the layer (f16) + q in + attention vector out."""
    return 2 * (pos + 1) * KV * 2 + H * 4 * 2


def step_bytes(pos, lm_head=False):
    """Algorithmic HBM bytes of one decode step at position pos (28 layers)."""
    per_layer = sum(KERNEL_BYTES.values()) + attention_bytes(pos)
    b = L * per_layer + H * 2 + H * 4 * 2  # embedding row (f16) + output norm
    if lm_head:
        b += V * H * 2 + V * 4
    return b


C0_BYTES = q8(H, H) + 2 * H * 4   # W + x in + y out (the single-matvec workload)


def graph_time_ms(ctx, launch, n_graph_launches=5):
    """Average wall time (ms) of one replay of a graph captured from launch()."""
    ctx.graph_begin()
    launch()
    g = ctx.graph_end()
    try:
        ctx.graph_launch(g)
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(n_graph_launches):
            ctx.graph_launch(g)
        ctx.sync()
        return (time.perf_counter() - t0) * 1e3 / n_graph_launches
    finally:
        ctx.graph_free(g)


def c0_leg(ctx, copies=64, per_graph=256):
    """y = W.x with W a 2048x2048 Q8_0 matrix (matvec.comp:46-62, the vx_matvec
    entry point): `copies` distinct matrices (q ~ U[-127,127], d = |N(0,1)|*0.01,
    x ~ N(0,1)) rotated inside one graph, so every launch reads HBM; and one
    matrix repeated (hot in the MALL/L2). Per launch, including the launch gap
    between dependent kernels of a graph."""
    import ctypes as C
    from voxgen_amd import abi, synth
    from voxgen_amd.runtime import Model
    reg = synth.Region()
    ts = [reg.add(f"c0.w{i}", abi.DTYPE_Q8_0, (H, H)) for i in range(copies)]
    data = np.zeros((reg.size + 255) // 256 * 256, np.uint8)
    for i, t in enumerate(ts):
        data[t.offset:t.offset + t.nbytes] = synth.q8_0_blocks(H * H // 32, 0x5EED0C00 + i)
    model = Model(ctx, data, ts)
    xb = ctx.array(synth.normal_f32(H, 0x5EED0C99))
    yb = ctx.zeros(H * 4)
    pushes = [abi.MatvecPush(t.offset, H, H, abi.DTYPE_Q8_0, 0, 1.0) for t in ts]

    def run(seq):
        def launch():
            for i in seq:
                abi.call("vx_matvec", ctx.handle, model.handle, xb.handle, yb.handle, C.byref(pushes[i]))
        return launch

    cold = graph_time_ms(ctx, run([i % copies for i in range(per_graph)])) / per_graph
    hot = graph_time_ms(ctx, run([0] * per_graph)) / per_graph
    model.free()
    gb = lambda ms: round(C0_BYTES / (ms * 1e-3) / 1e9, 1)
    return {"workload": "q8_0_matvec_2048x2048", "bytes_per_launch": C0_BYTES,
            "hbm": {"avg_us": round(cold * 1e3, 3), "GBps": gb(cold), "frac": round(gb(cold) / HBM_PEAK_GBPS, 4),
                    "copies": copies, "resident_MB": round(copies * q8(H, H) / 1e6, 1)},
            "hot": {"avg_us": round(hot * 1e3, 3), "GBps": gb(hot)},
            "note": "per launch inside a graph of 256 dependent launches, including the launch gap"}


def achievable_leg(ctx):
    """Best streaming-read bandwidth of a plain read kernel over 1 GiB (grid and
    loads in flight swept): the practical HBM ceiling of this GPU."""
    from voxgen_amd import abi
    nbytes = 1 << 30
    src, sink = ctx.zeros(nbytes), ctx.zeros(16 * 16384)
    best = None
    for blocks in (2048, 4096, 8192):
        for unroll in (4, 8):
            def launch():
                for _ in range(4):
                    abi.call("vx_diag_stream_read", ctx.handle, src.handle, 0, nbytes, sink.handle, blocks, unroll)
            ms = graph_time_ms(ctx, launch) / 4
            gbps = nbytes / (ms * 1e-3) / 1e9
            if best is None or gbps > best["GBps"]:
                best = {"GBps": round(gbps, 1), "blocks": blocks, "unroll": unroll}
    best["frac_of_spec"] = round(best["GBps"] / HBM_PEAK_GBPS, 4)
    best["bytes"] = nbytes
    return best


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--prefill", type=int, default=256)
    ap.add_argument("--lm-head", action="store_true", help="include the tied F16 LM head per step")
    ap.add_argument("--kernel-reps", type=int, default=8, help="passes over the 28 layers per kernel timing")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="target length of the CPU oracle sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--mode", default="graph", choices=["graph", "fused", "reference"])
    ap.add_argument("--prefill-tokens", type=int, default=384,
                    help="tokens of the token-batched prefill leg (0 skips it)")
    ap.add_argument("--prefill-reps", type=int, default=5)
    ap.add_argument("--cfm-reps", type=int, default=5, help="CFM solves timed (0 skips the CFM leg)")
    ap.add_argument("--cfm-only", action="store_true", help="run only the LocDiT CFM leg (for profiling)")
    ap.add_argument("--long-context", type=int, default=1,
                    help="1: also time decode with --max-context 8192 at positions up to 8000")
    ap.add_argument("--residual-steps", type=int, default=64,
                    help="ResidualLM steps timed (0 skips the ResidualLM leg)")
    ap.add_argument("--residual-only", action="store_true", help="run only the ResidualLM leg (for profiling)")
    ap.add_argument("--vae-frames", type=int, default=40, help="latent frames of the AudioVAE leg (0 skips it)")
    ap.add_argument("--vae-only", action="store_true", help="run only the AudioVAE leg (for profiling)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the token-batched prefill leg (for profiling)")
    ap.add_argument("--decode-only", action="store_true",
                    help="run only the prefill, warmup and timed decode steps, no graph-timed legs (for profiling)")
    ap.add_argument("--timeline", action="store_true",
                    help="graph-mode per-kernel timeline (needs the -DVX_STAMPS library in VOXHIP_LIBRARY)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run one copy kernel of known size and exit (PMC calibration)")
    ap.add_argument("--vendor-gemm", action="store_true",
                    help="time the vendor library's plain f16 GEMMs (torch.matmul -> hipBLASLt) at the T=384 "
                         "projection shapes and exit: the library ceiling for these shapes")
    return ap.parse_args()


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def vendor_gemm(T=384, reps=50):
    """The vendor library's plain f16 GEMM (torch.matmul, which hipBLASLt serves) at
    the four projection shapes of one prefill layer, single f16 operands (no hi/lo
    split, no Q8_0 dequant): back-to-back launches timed with torch events. A
    reference point for the achievable MFMA fraction at this token count."""
    import torch
    dev = torch.device("cuda")
    out = {}
    total_us = total_fl = 0.0
    for name, N, K in (("qkv", H + 2 * KV, H), ("attn_out", H, H), ("swiglu", 2 * F, H), ("down", H, F)):
        a = torch.randn(T, K, device=dev, dtype=torch.float16)
        b = torch.randn(N, K, device=dev, dtype=torch.float16)
        for _ in range(5):
            c = a @ b.t()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            c = a @ b.t()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        fl = 2.0 * T * N * K
        out[name] = {"M": T, "N": N, "K": K, "us": round(us, 2), "tflops": round(fl / us / 1e6, 1),
                     "frac": round(fl / us / 1e6 / F16_MFMA_PEAK_TFLOPS, 4)}
        total_us += us
        total_fl += fl
        del c
    out["layer"] = {"us": round(total_us, 2), "frac": round(total_fl / total_us / 1e6 / F16_MFMA_PEAK_TFLOPS, 4),
                    "prefill_gemm_ms_28L": round(28 * total_us / 1e3, 3)}
    out["library"] = f"torch {torch.__version__} (hipBLASLt)"
    log(f"vendor f16 GEMMs, one layer at T={T}: {total_us:.1f} us -> {out['layer']['frac']:.3f} of the f16 peak")
    print(json.dumps({"vendor_gemm": out}), flush=True)


def copy_calibration():
    """One 256 MiB device-to-device copy through vx_diag_stream_copy: FETCH_SIZE
    and WRITE_SIZE of this dispatch should read 256 MiB each."""
    from voxgen_amd import abi
    from voxgen_amd.runtime import Context
    abi.load()
    nbytes = 256 << 20
    with Context(0) as ctx:
        src, dst = ctx.zeros(nbytes), ctx.zeros(nbytes)
        abi.call("vx_diag_stream_copy", ctx.handle, dst.handle, src.handle, nbytes, 4096)
        ctx.sync()
        src.free()
        dst.free()
    print(json.dumps({"copy_calibration_bytes": nbytes}), flush=True)


F16_MFMA_PEAK_TFLOPS = 2500.0


def prefill_flops(T):
    """Algorithmic FLOP of each projection GEMM of one layer at T tokens."""
    return {"prefill.qkv": 2 * T * (H + 2 * KV) * H, "prefill.attn_out": 2 * T * H * H,
            "prefill.swiglu": 2 * T * 2 * F * H, "prefill.down": 2 * T * H * F}


def prefill_leg(ctx, eng, cfg, T, reps):
    """Token-batched prefill of T tokens through the 28 layers (positions 0..T-1):
    whole-prefill wall time around the stream, then one run with a HIP-event span
    around every kernel for the per-kernel breakdown."""
    toks = synth_tokens(T, cfg)
    eng.reset()
    eng.prefill_tokens_batched_gpu_only(toks)   # warm (allocates the workspace)
    ctx.sync()
    times = []
    for _ in range(reps):
        eng.reset()
        ctx.sync()
        t0 = time.perf_counter()
        eng.prefill_tokens_batched_gpu_only(toks)
        ctx.sync()
        times.append(time.perf_counter() - t0)
    ms = float(np.median(times)) * 1e3
    ctx.prof_reset()
    ctx.prof_enable(True)
    eng.reset()
    eng.prefill_tokens_batched_gpu_only(toks)
    ctx.sync()
    prof = ctx.prof_snapshot()
    ctx.prof_enable(False)
    fl = prefill_flops(T)
    per = {}
    gemm_ms = gemm_fl = 0.0
    for name, v in prof.items():
        e = dict(avg_us=round(v["avg_ms"] * 1e3, 3), calls=v["calls"], total_ms=round(v["total_ms"], 4))
        if name in fl:
            tf = fl[name] / (v["avg_ms"] * 1e-3) / 1e12
            e.update(tflops=round(tf, 1), mfma_frac=round(tf / F16_MFMA_PEAK_TFLOPS, 4))
            gemm_ms += v["total_ms"]
            gemm_fl += fl[name] * v["calls"]
        per[name] = e
    gemm_tf = gemm_fl / (gemm_ms * 1e-3) / 1e12 if gemm_ms else 0.0
    log(f"prefill T={T}: {ms:.3f} ms ({T / ms * 1e3:.0f} tok/s); GEMMs {gemm_ms:.3f} ms at "
        f"{gemm_tf:.1f} TFLOP/s = {gemm_tf / F16_MFMA_PEAK_TFLOPS:.3f} of f16 MFMA peak")
    return {"workload": f"baselm_q8_0_prefill_28L_T{T}", "tokens": T, "ms": round(ms, 3),
            "tok_s": round(T / ms * 1e3, 1),
            "gemm": {"ms": round(gemm_ms, 3), "flop": int(gemm_fl), "achieved": round(gemm_tf, 1),
                     "peak": F16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(gemm_tf / F16_MFMA_PEAK_TFLOPS, 4),
                     "precision": "Q8_0 weights exact (int8 as f16, block scale in fp32), activations as "
                                  "f16 hi+lo (two MFMAs per k-step), fp32 accumulation"},
            "per_kernel": per}


def cfm_leg(ctx, reps):
    """The LocDiT flow-matching solve at the benchmark shape: hidden 1024, 8 layers,
    16 x 64 heads, FFN 4096, F16 weights N(0, 0.02); 32 condition rows N(0,1) +
    the time token + 4 latent rows of 64; CFG batch 2 (the unconditional pass
    zeroes the condition rows); 10 timesteps, cfg 2.0, CFG-Zero*, seeded noise.
    Each Euler step runs both passes as one batch, so the step streams the
    weights once."""
    from voxgen_amd import synth
    from voxgen_amd.locdit import CfmOptions, LocDit
    from voxgen_amd.runtime import Model
    cfg = synth.locdit_config(layers=8, q_heads=16, kv_heads=16, head_dim=64, n_mu=0, n_cond=32, cond_raw=1,
                              uncond_zero_cond=1)
    m = synth.build_locdit(cfg, seed=0x5EED0014)
    model = Model(ctx, m.data, m.tensors)
    loc = LocDit(ctx, model, cfg, strict_geometry=False)
    cond = synth.normal_f32(32 * 1024, 0x5EED0015)
    opt = CfmOptions(n_timesteps=10, cfg_value=2.0, temperature=1.0, sway_sampling_coef=1.0, seed=42,
                     use_cfg_zero_star=True)
    out, res = loc.cfm_solve(cond, None, opt)            # captures the graph
    times = []
    for i in range(reps):
        t0 = time.perf_counter()
        out, res = loc.cfm_solve(cond, None, CfmOptions(seed=42 + i))
        times.append(time.perf_counter() - t0)
    ms = float(np.median(times)) * 1e3
    ctx.prof_reset()
    ctx.prof_enable(True)
    loc.cfm_solve(cond, None, opt)
    prof = ctx.prof_snapshot()
    ctx.prof_enable(False)
    loc.close()
    model.free()
    steps = res["estimator_calls"] // 2
    per_layer = 4 * 1024 * 1024 * 2 + 3 * 1024 * 4096 * 2          # q,k,v,o + gate,up,down (F16)
    step_bytes = 8 * per_layer + 4 * 1024 * 1024 * 2 + 2 * 64 * 1024 * 2   # + time MLPs, in/out proj
    solve_bytes = steps * step_bytes
    gbps = solve_bytes / (ms * 1e-3) / 1e9
    log(f"cfm solve: {ms:.3f} ms for {steps} Euler steps x 2 passes; {solve_bytes / 1e9:.2f} GB of weights "
        f"-> {gbps:.0f} GB/s")
    per = {k: dict(avg_us=round(v["avg_ms"] * 1e3, 3), calls=v["calls"], total_ms=round(v["total_ms"], 4))
           for k, v in prof.items()}
    ref = cfm_reference_shape(ctx, reps)
    return {"workload": "locdit_f16_cfm_8L_h1024_16x64_cond32_cfg2_batch2_10steps", "ms": round(ms, 3),
            "euler_steps": steps, "estimator_calls": res["estimator_calls"],
            "weight_bytes_per_solve": int(solve_bytes), "achieved_GBps": round(gbps, 1),
            "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4), "per_kernel_eager": per, "reference_shape": ref}


def cfm_reference_shape(ctx, reps):
    """The same solve at the reference's enforced LocDiT geometry (LocalConfig::
    from_gguf, local.rs:37-48,85-92): 12 layers x 1024, 16/2 heads x 128, FFN 4096,
    mu1 + mu2 + time + 4 condition + 4 latent tokens (11 per sequence), strict
    geometry, 10 timesteps, CFG batch 2."""
    from voxgen_amd import synth
    from voxgen_amd.locdit import CfmOptions, LocDit
    from voxgen_amd.runtime import Model
    cfg = synth.locdit_config()
    m = synth.build_locdit(cfg, seed=0x5EED0016)
    model = Model(ctx, m.data, m.tensors)
    loc = LocDit(ctx, model, cfg, strict_geometry=True)
    cond = synth.normal_f32(cfg["patch"] * cfg["feat_dim"], 0x5EED0017)
    mu = synth.normal_f32(2 * cfg["hidden"], 0x5EED0018)
    opt = CfmOptions(n_timesteps=10, cfg_value=2.0, temperature=1.0, sway_sampling_coef=1.0, seed=42,
                     use_cfg_zero_star=True)
    out, res = loc.cfm_solve(cond, mu, opt)                # captures the graph
    times = []
    for i in range(max(reps, 1)):
        t0 = time.perf_counter()
        loc.cfm_solve(cond, mu, CfmOptions(seed=42 + i))
        times.append(time.perf_counter() - t0)
    ms = float(np.median(times)) * 1e3
    loc.close()
    model.free()
    H, F, QD, KD, FD = 1024, 4096, 16 * 128, 2 * 128, 64
    layer = 2 * (H * (QD + 2 * KD) + QD * H + 3 * F * H)
    step_bytes = 12 * layer + 2 * (4 * H * H + 2 * FD * H)   # + time MLPs, in/out proj
    steps = res["estimator_calls"] // 2
    solve_bytes = steps * step_bytes
    gbps = solve_bytes / (ms * 1e-3) / 1e9
    log(f"cfm solve at the reference geometry (12L, 11 tokens): {ms:.3f} ms; {solve_bytes / 1e9:.2f} GB of weights "
        f"-> {gbps:.0f} GB/s")
    return {"workload": "locdit_f16_cfm_12L_h1024_16q2kv_x128_11tok_cfg2_batch2_10steps", "ms": round(ms, 3),
            "euler_steps": steps, "weight_bytes_per_solve": int(solve_bytes), "achieved_GBps": round(gbps, 1),
            "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4)}


def residual_step_bytes(pos):
    """Algorithmic bytes of one FSQ ResidualLM step at position pos: F16 weights
    and biases of fsq.in/out, the fusion projection and 8 layers, the f32 norm
    gains, and the f16 K/V rows read by the attention (positions 0..pos)."""
    Hr, Lr, Fr, KVr, Lat = 2048, 8, 6144, 256, 512
    fsq = 2 * (Lat * Hr + Lat) + 2 * (Hr * Lat + Hr)
    fusion = 2 * (Hr * 2 * Hr + Hr)
    layer = 2 * (Hr * (Hr + 2 * KVr) + Hr * Hr + 3 * Fr * Hr) + 2 * Hr * 4 + 2 * (pos + 1) * KVr * 2
    return fsq + fusion + Lr * layer + Hr * 4


LONG_POSITIONS = (512, 1024, 2048, 4096, 8000)


def long_context_leg(ctx, model, cfg, steps=16, reps=4):
    """Decode with --max-context 8192 (the reference default, main.rs:97-99) at
    positions up to 8000: tok/s over `steps` graph steps from each position, and
    the per-layer cost of the attention (partials, plus the combine on the wide
    path) and of attn_out there, in graph chains with HBM-resident weights. The
    engine's own choice (the wide attention from 1024 keys on) is timed next to the
    folded path alone (attn_splits = 8), which it replaces there. The cache holds
    zeros: timing does not depend on its values."""
    from voxgen_amd.baselm import BaseLmEngine
    lcfg = dict(cfg, active_context_length=8192)
    toks = synth_tokens(steps, cfg)
    out = {}
    for label, splits in (("engine", 0), ("folded_8_splits", 8)):
        eng = BaseLmEngine(ctx, model, lcfg, exec_mode="graph", strict_geometry=True, attn_splits=splits)
        res = {}
        for p in LONG_POSITIONS:
            eng.set_position(p)
            eng.decode_tokens_gpu_only(toks)   # warm (captures the graph of this path)
            ctx.sync()
            eng.set_position(p)
            t0 = time.perf_counter()
            eng.decode_tokens_gpu_only(toks)
            ctx.sync()
            el = time.perf_counter() - t0
            # The kernels are timed at the device position the steps left: p + steps.
            att = eng.time_layer_kernel("attention", reps) * 1e3
            ao = eng.time_layer_kernel("attn_out", reps) * 1e3
            keys = p + steps + 1
            res[str(p)] = {"tok_s": round(steps / el, 1), "ms_per_step": round(el * 1e3 / steps, 4),
                           "attention_us": round(att, 3), "attn_out_us": round(ao, 3), "keys_timed": keys}
            log(f"context 8192 ({label}), position {p}: {steps / el:.1f} tok/s; attention {att:.2f} us, "
                f"attn_out {ao:.2f} us per layer at {keys} keys")
        eng.close()
        out[label] = res
    return out


TIMELINE_KINDS = {1: "qkv", 2: "attention", 3: "attention", 4: "attn_out", 5: "swiglu", 6: "down"}
TICK_US = 0.01   # s_memrealtime's nominal 100 MHz; timeline_leg measures the rate


def read_timeline(ctx):
    """Launch table and per-wave (start, end) ticks of a -DVX_STAMPS library."""
    import ctypes as C
    from voxgen_amd import abi
    nl, nw = C.c_uint64(), C.c_uint64()
    abi.call("vx_diag_timeline_read", ctx.handle, None, 0, None, 0, C.byref(nl), C.byref(nw))
    launches = np.zeros(3 * nl.value, np.uint64)
    ticks = np.zeros(2 * nw.value, np.uint64)
    abi.call("vx_diag_timeline_read", ctx.handle, launches.ctypes.data_as(C.POINTER(C.c_uint64)), nl.value,
             ticks.ctypes.data_as(C.POINTER(C.c_uint64)), nw.value, C.byref(nl), C.byref(nw))
    return launches.reshape(-1, 3), ticks.reshape(-1, 2).astype(np.int64)


def timeline_spans(launches, ticks, first, count):
    """Per launch (kind, start, end, mean wave life, waves) over launches
    [first, first + count), ticks relative to the first launch's start."""
    rows = []
    for kind, w0, nw in launches[first:first + count]:
        t = ticks[int(w0):int(w0 + nw)]
        rows.append((int(kind), int(t[:, 0].min()), int(t[:, 1].max()), float((t[:, 1] - t[:, 0]).mean()), int(nw)))
    base = rows[0][1]
    return [(k, s - base, e - base, life, nw) for k, s, e, life, nw in rows], base


def timeline_summary(rows_per_step, layers=28, per_layer=5, tick_us=TICK_US):
    """Mean over steps: per kernel of the layer its span (first wave start to last
    wave end), the gap before it (previous stamped kernel's last wave end to its
    first wave start) and the mean wave life; the layer period; the step span."""
    spans = np.array([[e - s for _, s, e, _, _ in rows] for rows in rows_per_step], float) * tick_us
    starts = np.array([[s for _, s, _, _, _ in rows] for rows in rows_per_step], float) * tick_us
    ends = np.array([[e for _, _, e, _, _ in rows] for rows in rows_per_step], float) * tick_us
    lives = np.array([[l for _, _, _, l, _ in rows] for rows in rows_per_step], float) * tick_us
    gaps = np.zeros_like(spans)
    gaps[:, 1:] = starts[:, 1:] - ends[:, :-1]
    kinds = [TIMELINE_KINDS[k] for k, *_ in rows_per_step[0]]
    out = {}
    for j in range(per_layer):
        idx = list(range(j, layers * per_layer, per_layer))
        g = gaps[:, idx]
        if j == 0:
            g = g[:, 1:]   # layer 0's qkv follows the unstamped embedding and RoPE-table kernels
        out[kinds[j]] = {"span_us": round(float(spans[:, idx].mean()), 3),
                         "gap_before_us": round(float(g.mean()), 3),
                         "wave_life_us": round(float(lives[:, idx].mean()), 3),
                         "waves": rows_per_step[0][j][4]}
    period = (ends[:, per_layer * layers - 1] - ends[:, per_layer - 1]) / (layers - 1)
    return {"kernels": out, "layer_period_us": round(float(period.mean()), 3),
            "stamped_span_us": round(float((ends[:, -1] - starts[:, 0]).mean()), 3)}


def timeline_leg(steps=12):
    """Graph-mode decode timeline from a library built with -DVX_STAMPS (python -m
    voxgen_amd.build --timeline; VOXHIP_LIBRARY=voxgen_amd/timeline/libvoxhip.so):
    the 28-layer step of the headline workload (context 512, positions 256..,
    k_attn_chunk) and with --max-context 8192 at position 8000 (16 streamed
    slices). Each step is one graph replay; a replay's waves' ticks are read back
    after it."""
    from voxgen_amd import abi, synth
    from voxgen_amd.baselm import BaseLmEngine
    from voxgen_amd.runtime import Context, Model
    cfg = synth.baselm_config(active_context=512)
    m = synth.build_baselm(cfg, seed=0x5EED0002)
    toks = synth.uniform_u32(256 + steps + 16, 0x5EED0012, cfg["vocab_size"]).astype(np.uint32)
    ctx = Context(0)
    model = Model(ctx, m.data, m.tensors)
    abi.call("vx_diag_timeline_arm", ctx.handle, 1 << 22)
    report = {}
    for label, ecfg, start in (("context_512_position_256", cfg, 256),
                               ("context_8192_position_8000", dict(cfg, active_context_length=8192), 8000)):
        eng = BaseLmEngine(ctx, model, ecfg, exec_mode="graph", strict_geometry=True)
        launches0, _ = read_timeline(ctx)
        eng.set_position(start)
        eng.decode_tokens_gpu_only(toks[:4])   # captures this position's graph
        ctx.sync()
        launches, _ = read_timeline(ctx)
        first, count = len(launches0), len(launches) - len(launches0)
        assert count == 5 * cfg["block_count"], count
        # Each sample is a burst of `burst` back-to-back replays (the GPU at its
        # running clocks) whose last replay leaves the timeline. The tick rate:
        # samples 20 ms apart, the last launch's end ticks fitted against the host
        # clock after the burst's sync (tens of microseconds of error over 0.3 s).
        rows, walls, host_t, dev_t = [], [], [], []
        burst = 16
        for i in range(steps):
            eng.set_position(start + 4 + i)
            time.sleep(0.02)
            t0 = time.perf_counter()
            eng.decode_tokens_gpu_only(toks[4 + i:4 + i + burst])
            ctx.sync()
            t1 = time.perf_counter()
            walls.append((t1 - t0) / burst)
            launches, ticks = read_timeline(ctx)
            r, base = timeline_spans(launches, ticks, first, count)
            rows.append(r)
            host_t.append(t1)
            dev_t.append(base + r[-1][2])
        hz = float(np.polyfit(np.array(host_t) - host_t[0], np.array(dev_t, float) - dev_t[0], 1)[0])
        summ = timeline_summary(rows, cfg["block_count"], tick_us=1e6 / hz)
        summ["tick_mhz"] = round(hz / 1e6, 3)
        summ["host_ms_per_step"] = round(float(np.median(walls)) * 1e3, 4)
        report[label] = summ
        log(f"timeline {label}: layer period {summ['layer_period_us']} us, stamped span "
            f"{summ['stamped_span_us']} us, host {summ['host_ms_per_step']} ms/step; " +
            ", ".join(f"{k} {v['span_us']} (+{v['gap_before_us']})" for k, v in summ["kernels"].items()))
        eng.close()
    model.free()
    report["cfm_locdit8"] = cfm_timeline(ctx, 1e6 / hz)
    report["cfm_reference_12L"] = cfm_timeline(ctx, 1e6 / hz, reference=True)
    ctx.close()
    return report


# Stamped kernels of a LocDiT layer (kinds: 7 k_gemm_sk, 8 k_dense_attn_fused with
# the O projection, 9 k_seq_rmsnorm4): the slab stack of 2 x 37 rows, and the
# residual-stream stack of 2 x 11 rows (the rmsnorms folded into the projections).
CFM_LAYER_KERNELS = ("qkv", "attention_oproj", "rmsnorm_ffn", "gate_up", "down", "rmsnorm_next")
CFM_LAYER_KINDS = (7, 8, 9, 7, 7, 9)
CFM_REF_LAYER_KERNELS = ("qkv", "attention_oproj", "gate_up", "down")
CFM_REF_LAYER_KINDS = (7, 8, 7, 7)


def cfm_timeline(ctx, tick_us, solves=8, reference=False):
    """The LocDiT CFM solve graph at cfm_leg's shape and options (reference=True:
    cfm_reference_shape's), from the same -DVX_STAMPS library: per stamped kernel
    of a layer, the mean over the solve's layer passes and `solves` samples (each
    the last of four back-to-back solves) of its span, the gap after the previous
    stamped kernel, and the mean wave life."""
    from voxgen_amd import synth
    from voxgen_amd.locdit import CfmOptions, LocDit
    from voxgen_amd.runtime import Model
    if reference:
        cfg = synth.locdit_config()
        m = synth.build_locdit(cfg, seed=0x5EED0016)
        cond = synth.normal_f32(cfg["patch"] * cfg["feat_dim"], 0x5EED0017)
        mu = synth.normal_f32(2 * cfg["hidden"], 0x5EED0018)
        names, kinds = CFM_REF_LAYER_KERNELS, CFM_REF_LAYER_KINDS
    else:
        cfg = synth.locdit_config(layers=8, q_heads=16, kv_heads=16, head_dim=64, n_mu=0, n_cond=32, cond_raw=1,
                                  uncond_zero_cond=1)
        m = synth.build_locdit(cfg, seed=0x5EED0014)
        cond = synth.normal_f32(32 * 1024, 0x5EED0015)
        mu = None
        names, kinds = CFM_LAYER_KERNELS, CFM_LAYER_KINDS
    model = Model(ctx, m.data, m.tensors)
    loc = LocDit(ctx, model, cfg, strict_geometry=reference)
    launches0, _ = read_timeline(ctx)
    loc.cfm_solve(cond, mu, CfmOptions(n_timesteps=10, cfg_value=2.0, temperature=1.0, sway_sampling_coef=1.0,
                                       seed=42, use_cfg_zero_star=True))   # captures the solve's graph
    launches, _ = read_timeline(ctx)
    first, count = len(launches0), len(launches) - len(launches0)
    acc = {k: [] for k in names}
    walls = []
    for i in range(solves):
        time.sleep(0.02)
        t0 = time.perf_counter()
        for j in range(4):
            loc.cfm_solve(cond, mu, CfmOptions(seed=43 + 4 * i + j))
        walls.append((time.perf_counter() - t0) / 4)
        launches, ticks = read_timeline(ctx)
        rows, _ = timeline_spans(launches, ticks, first, count)
        seq, prev_end = [], None
        for kind, st, en, life, nw in rows:
            seq.append((kind, en - st, st - prev_end if prev_end is not None else np.nan, life, nw))
            prev_end = en
        j = 0
        while j + len(kinds) <= len(seq):
            if tuple(r[0] for r in seq[j:j + len(kinds)]) == kinds:
                for q, name in enumerate(names):
                    acc[name].append(seq[j + q][1:])
                j += len(kinds)
            else:
                j += 1
    loc.close()
    model.free()
    out = {}
    for name, v in acc.items():
        v = np.array(v, float)
        out[name] = {"span_us": round(float(v[:, 0].mean()) * tick_us, 3),
                     "gap_before_us": round(float(np.nanmean(v[:, 1])) * tick_us, 3),
                     "wave_life_us": round(float(v[:, 2].mean()) * tick_us, 3), "waves": int(v[0, 3]),
                     "layer_passes": len(v)}
    period = sum(k["span_us"] + k["gap_before_us"] for k in out.values())
    summ = {"kernels": out, "layer_period_us": round(period, 3), "host_ms_per_solve": round(float(np.median(walls)) * 1e3, 4)}
    log(f"timeline cfm {'reference 12L' if reference else 'locdit8'}: layer period {summ['layer_period_us']} us, "
        f"host {summ['host_ms_per_solve']} ms/solve; " +
        ", ".join(f"{k} {v['span_us']} (+{v['gap_before_us']})" for k, v in out.items()))
    return summ


def residual_leg(ctx, steps, warmup=8, baselm=None, bcfg=None, prefix=384, cpu_steps=0):
    """The ResidualLM step of the VoxCPM2 acoustic model (acoustic.rs:830-1035):
    FSQ of the BaseLM hidden, fusion with the acoustic embedding, 8 F16 layers
    (hidden 2048, FFN 6144, 16/2 x 128, no RoPE), F16 weights N(0, 0.02); inputs
    resident in device buffers, one graph replay per step with the reference's
    wait per step (step_from_gpu_base_and_embedding_gpu_only)."""
    from voxgen_amd import synth
    from voxgen_amd.residual import ResidualFsqEngine
    from voxgen_amd.runtime import Model
    acfg = synth.acoustic_config(active_context=512)
    m = synth.build_acoustic(acfg, seed=0x5EED0016)
    model = Model(ctx, m.data, m.tensors)
    eng = ResidualFsqEngine(ctx, model, acfg, exec_mode="graph", strict_geometry=True)
    base = ctx.array(synth.normal_f32(2048, 0x5EED0017))
    emb = ctx.array(synth.normal_f32(2048, 0x5EED0018))
    for _ in range(warmup):
        eng.step_from_gpu_base_and_embedding_gpu_only(base, emb)
    ctx.sync()
    p0 = eng.position
    t0 = time.perf_counter()
    for _ in range(steps):
        eng.step_from_gpu_base_and_embedding_gpu_only(base, emb)
    ctx.sync()
    elapsed = time.perf_counter() - t0
    ms = elapsed * 1e3 / steps
    nbytes = float(np.mean([residual_step_bytes(p) for p in range(p0, p0 + steps)]))
    gbps = nbytes / (ms * 1e-3) / 1e9
    ctx.prof_reset()
    ctx.prof_enable(True)
    eng.step_from_gpu_base_and_embedding_gpu_only(base, emb)
    prof = ctx.prof_snapshot()
    ctx.prof_enable(False)
    log(f"residual step: {ms * 1e3:.1f} us ({1e3 / ms:.0f} steps/s); {nbytes / 1e6:.1f} MB -> {gbps:.0f} GB/s")
    text = None
    if baselm is not None and prefix:
        text = text_prefill(ctx, baselm, bcfg, model, acfg, prefix)
    eng.close()
    model.free()
    cpu = None
    if cpu_steps:
        sys.path.insert(0, str(ROOT / "oracle"))
        import voxref
        o = voxref.ResidualFsq(m.data, {t.name: t for t in m.tensors}, acfg)
        b, e = synth.normal_f32(2048, 0x5EED0017), synth.normal_f32(2048, 0x5EED0018)
        t0 = time.perf_counter()
        for p in range(cpu_steps):
            o.step(b, e, p, fsq=True)
        el = time.perf_counter() - t0
        cpu = {"value": round(cpu_steps / el, 3), "unit": "steps/s", "cores": voxref.threads(), "kind": "port",
               "sample": f"{cpu_steps} FSQ ResidualLM steps at positions 0..{cpu_steps - 1}, same model, C oracle "
                         f"(oracle/voxref.c) with OpenMP over rows"}
        log(f"cpu oracle residual: {cpu_steps} steps in {el:.2f}s")
    per = {k: dict(avg_us=round(v["avg_ms"] * 1e3, 3), calls=v["calls"]) for k, v in prof.items()}
    return {"workload": "residual_lm_f16_fsq_fusion_8L_h2048_ffn6144_16q2kv", "us_per_step": round(ms * 1e3, 2),
            "steps_per_second": round(1e3 / ms, 1), "positions": f"{p0}..{p0 + steps - 1}",
            "bytes_per_step": int(nbytes), "achieved_GBps": round(gbps, 1), "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
            "per_kernel_eager": per, "text_prefill": text, "cpu_baseline": cpu}


def text_prefill(ctx, base, bcfg, amodel, acfg, T, reps=3, seq_positions=32):
    """The text-prefix run of a conditioning prefill (runtime.rs:483-566): T text
    tokens through the 28-layer BaseLM and the 8-layer ResidualLM. Batched: one
    cross-engine call (enqueue) + sync per rep, fresh positions. Per position:
    BaseLM decode + ResidualLM text-prefix step per token, timed over
    seq_positions tokens and reported per token."""
    from voxgen_amd import synth
    from voxgen_amd.residual import ResidualFsqEngine, prefill_text_cross_engine
    res = ResidualFsqEngine(ctx, amodel, acfg, exec_mode="graph", strict_geometry=True)
    tokens = synth.uniform_u32(T, 0x5EED0019, bcfg["vocab_size"]).astype(np.uint32)
    times = []
    for _ in range(reps + 1):
        base.reset()
        res.reset()
        ctx.sync()
        t0 = time.perf_counter()
        prefill_text_cross_engine(base, res, tokens)
        ctx.sync()
        times.append(time.perf_counter() - t0)
    ms = float(np.median(times[1:])) * 1e3
    base.reset()
    res.reset()
    norm = base.buffer("norm")
    for t in tokens[:4]:                                   # captures both graphs
        base.decode_token_gpu_only(int(t))
        res.step_text_prefix_from_gpu_base_gpu_only(norm)
    ctx.sync()
    t0 = time.perf_counter()
    for t in tokens[4:4 + seq_positions]:
        base.decode_token_gpu_only(int(t))
        res.step_text_prefix_from_gpu_base_gpu_only(norm)
    ctx.sync()
    per_pos_ms = (time.perf_counter() - t0) * 1e3 / seq_positions
    res.close()
    base.reset()
    log(f"text prefill of {T} tokens (BaseLM + ResidualLM): batched {ms:.2f} ms; per position "
        f"{per_pos_ms:.3f} ms/token -> {per_pos_ms * T:.1f} ms")
    return {"tokens": T, "batched_ms": round(ms, 3), "batched_tok_s": round(T / ms * 1e3, 1),
            "per_position_ms_per_token": round(per_pos_ms, 4), "per_position_ms_est": round(per_pos_ms * T, 2),
            "speedup": round(per_pos_ms * T / ms, 1)}


def vae_flops(frames):
    """Multiply-adds x 2 of one AudioVAE decode of `frames` latent frames at the
    VoxCPM2 geometry (latent 64, decoder 2048, rates 8,6,5,2,2,2)."""
    L, c = frames, 2048
    f = 2 * (64 * 7 * L + 64 * 2048 * L)
    for s in (8, 6, 5, 2, 2, 2):
        co, lo = c // 2, L * s
        f += 2 * lo * co * c * 2                       # transposed conv: 2 taps per input channel
        f += 3 * 2 * (lo * co * 7 + lo * co * co)      # residual units: depthwise k=7 + 1x1
        c, L = co, lo
    return f + 2 * L * c * 7


def vae_leg(ctx, frames, reps=5, cpu_frames=0):
    """AudioVAE decode (audiovae.rs:330-372) of `frames` latent frames at the VoxCPM2
    geometry, F16 weights (synthetic, activations O(1)), latents N(0,1) resident
    on the device (decode_latents_gpu), timed with a sync per decode."""
    from voxgen_amd import synth
    from voxgen_amd.audiovae import AudioVaeEngine
    from voxgen_amd.runtime import Model
    cfg = synth.audiovae_config()
    m = synth.build_audiovae(cfg, seed=0x5EED001A)
    model = Model(ctx, m.data, m.tensors)
    vae = AudioVaeEngine(ctx, model, cfg, strict_geometry=True)
    lat = ctx.array(synth.normal_f32(frames * 64, 0x5EED001B))
    wave = ctx.alloc(frames * 1920 * 4)
    vae.decode_latents_gpu(lat, frames, wave)
    ctx.sync()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        vae.decode_latents_gpu(lat, frames, wave)
        ctx.sync()
        times.append(time.perf_counter() - t0)
    ms = float(np.median(times)) * 1e3
    ctx.prof_reset()
    ctx.prof_enable(True)
    vae.decode_latents_gpu(lat, frames, wave)
    prof = ctx.prof_snapshot()
    ctx.prof_enable(False)
    vae.close()
    model.free()
    cpu = None
    if cpu_frames:
        sys.path.insert(0, str(ROOT / "oracle"))
        import voxref
        o = voxref.AudioVae(m.data, {t.name: t for t in m.tensors}, cfg)
        lat_h = synth.normal_f32(cpu_frames * 64, 0x5EED001B)
        t0 = time.perf_counter()
        o.decode(lat_h)
        el = time.perf_counter() - t0
        cpu = {"value": round(cpu_frames * 1920 / 48000 / el, 3), "unit": "audio s per s", "cores": voxref.threads(),
               "kind": "port", "sample": f"one decode of {cpu_frames} latent frames, same model, C oracle of the "
                                         f"vae_*.comp shaders (channel-major, OpenMP over output channels)"}
        log(f"cpu oracle audiovae: {cpu_frames} frames in {el:.2f}s")
    flops = vae_flops(frames)
    audio_s = frames * 1920 / 48000
    log(f"audiovae decode of {frames} frames ({audio_s:.2f} s audio): {ms:.2f} ms -> {audio_s * 1e3 / ms:.0f}x "
        f"real time, {flops / ms / 1e9:.1f} TFLOP/s")
    per = {k: dict(avg_us=round(v["avg_ms"] * 1e3, 3), calls=v["calls"], total_ms=round(v["total_ms"], 4))
           for k, v in prof.items()}
    return {"workload": f"audiovae_v2_decode_{frames}frames_dec2048", "ms": round(ms, 3),
            "audio_seconds": audio_s, "realtime_factor": round(audio_s * 1e3 / ms, 1),
            "flops": int(flops), "TFLOPs": round(flops / ms / 1e9, 2),
            "mfma_frac": round(flops / ms / 1e9 / 2500.0, 4), "per_span_eager": per, "cpu_baseline": cpu}


def synth_tokens(n, cfg):
    from voxgen_amd import synth
    return synth.uniform_u32(n, 0x5EED0013, cfg["vocab_size"]).astype(np.uint32)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: the BaseLM decode path has no multi-GPU form "
              f"(got --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)
    if args.vendor_gemm:
        vendor_gemm(args.prefill_tokens)
        return
    if args.copy_calibration:
        copy_calibration()
        return
    if args.timeline:
        print(json.dumps({"timeline": timeline_leg()}), flush=True)
        return
    from voxgen_amd import abi, synth
    from voxgen_amd.baselm import BaseLmEngine
    from voxgen_amd.runtime import Context, Model

    abi.load()
    K, W, P = args.steps, args.warmup, args.prefill
    active = max(P + max(K, W), args.prefill_tokens)
    cfg = synth.baselm_config(active_context=max(active, 512))
    t0 = time.perf_counter()
    m = synth.build_baselm(cfg, seed=0x5EED0002)
    log(f"synthetic 28-layer Q8_0 model: {m.data.nbytes / 1e9:.2f} GB in {time.perf_counter() - t0:.1f}s")
    tokens = synth.uniform_u32(P + max(K, W), 0x5EED0012, cfg["vocab_size"]).astype(np.uint32)
    ctx = Context(0)
    info = ctx.info()
    model = Model(ctx, m.data, m.tensors)
    eng = BaseLmEngine(ctx, model, cfg, exec_mode=args.mode, strict_geometry=True)
    log(f"device {info['name']} {info['arch']} CUs={info['compute_units']}; model on device "
        f"{model.device_bytes / 1e9:.2f} GB")
    if args.vae_only:
        va = vae_leg(ctx, args.vae_frames)
        eng.close()
        model.free()
        ctx.close()
        print(json.dumps({"audiovae": va}), flush=True)
        return
    if args.residual_only:
        rs = residual_leg(ctx, args.residual_steps, baselm=eng, bcfg=cfg)
        eng.close()
        model.free()
        ctx.close()
        print(json.dumps({"residual": rs}), flush=True)
        return
    if args.cfm_only:
        cf = cfm_leg(ctx, args.cfm_reps)
        eng.close()
        model.free()
        ctx.close()
        print(json.dumps({"cfm": cf}), flush=True)
        return
    if args.prefill_only:
        pf = prefill_leg(ctx, eng, cfg, args.prefill_tokens, args.prefill_reps)
        eng.close()
        model.free()
        ctx.close()
        print(json.dumps({"prefill": pf}), flush=True)
        return

    def run_steps(start, toks):
        eng.set_position(start)
        if args.lm_head:
            for t in toks:
                eng.decode_token(int(t))
        else:
            eng.decode_tokens_gpu_only(toks)

    eng.decode_tokens_gpu_only(tokens[:P])              # prefill positions 0..P-1
    run_steps(P, tokens[P:P + W])                         # warmup (also captures the graph)
    ctx.sync()
    timed = tokens[P:P + K]
    t0 = time.perf_counter()
    run_steps(P, timed)
    ctx.sync()
    elapsed = time.perf_counter() - t0
    tok_s = K / elapsed
    log(f"timed {K} steps at positions {P}..{P + K - 1}: {elapsed * 1e3:.2f} ms -> {tok_s:.1f} tok/s")
    if args.decode_only:
        eng.close()
        model.free()
        ctx.close()
        print(json.dumps({"decode": {"tok_s": round(tok_s, 2), "ms_per_step": round(elapsed * 1e3 / K, 4),
                                     "exec": args.mode, "positions": f"{P}..{P + K - 1}"}}), flush=True)
        return

    # Per-kernel cost: one layer kernel over the 28 layers' weights as a graph
    # chain, each pass after a 384 MiB read that evicts the MALL (so every launch
    # reads HBM, as in the step), HIP events on the engine stream, the reads
    # alone subtracted. Includes the launch gap. The device position is then P+K,
    # one past the context, which the attention clamps to the last cached
    # position P+K-1 (the qkv kernel stores no KV row there).
    pos_k = P + K - 1
    per_kernel = {}
    fam_bytes = fam_ms = 0.0
    for name in eng.LAYER_KERNELS:
        ms = eng.time_layer_kernel(name, args.kernel_reps)
        nbytes = KERNEL_BYTES.get(name, attention_bytes(pos_k))
        gbps = nbytes / (ms * 1e-3) / 1e9
        per_kernel[name] = dict(avg_us=round(ms * 1e3, 3), bytes=nbytes, GBps=round(gbps, 1),
                                frac=round(gbps / HBM_PEAK_GBPS, 4))
        if name in KERNEL_BYTES:
            fam_bytes += nbytes
            fam_ms += ms
    fam_gbps = fam_bytes / (fam_ms * 1e-3) / 1e9
    dom = per_kernel["swiglu"]
    traffic = None
    tfile = ROOT / "profiles" / "traffic_k_swiglu_decode28.json"
    if tfile.exists():
        try:
            traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None
    # The same kernel's average duration from the committed rocprofv3 kernel trace
    # of the eager decode (kernel execution only, no launch gap).
    rocprof = None
    rfile = ROOT / "profiles" / "kernels_decode28_q8.json"
    if rfile.exists():
        try:
            r = json.loads(rfile.read_text())
            gbps = r["algorithmic_bytes_per_launch"] / (r["avg_us"] * 1e-6) / 1e9
            rocprof = {"kernel": r["kernel"], "avg_us": r["avg_us"], "achieved": round(gbps, 1),
                       "frac": round(gbps / HBM_PEAK_GBPS, 4), "source": "profiles/kernels_decode28_q8.json"}
        except (OSError, ValueError, KeyError):
            rocprof = None
    achievable = achievable_leg(ctx)
    log(f"achievable streaming read: {achievable['GBps']:.0f} GB/s ({achievable['frac_of_spec']:.3f} of 8 TB/s)")
    roofline = dict(bound="hbm", achieved=dom["GBps"], peak=HBM_PEAK_GBPS, unit="GB/s",
                    frac=dom["frac"], traffic=traffic, kernel="k_swiglu (rmsnorm + gate/up Q8_0 matvec + SiLU)",
                    bytes_per_launch=dom["bytes"], avg_us=dom["avg_us"],
                    achievable_GBps=achievable["GBps"], frac_of_achievable=round(dom["GBps"] / achievable["GBps"], 4),
                    rocprof=rocprof)
    mean_step_bytes = float(np.mean([step_bytes(p, args.lm_head) for p in range(P, P + K)]))
    c0 = c0_leg(ctx)
    log(f"c0 matvec 2048x2048 Q8_0: {c0['hbm']['avg_us']:.2f} us from HBM ({c0['hbm']['GBps']:.0f} GB/s), "
        f"{c0['hot']['avg_us']:.2f} us hot")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(cfg, m, eng, tokens, P, args)
    # The reference's own benchmark (baselm.rs:841-880): decode_token with the
    # tied LM head and a host fence per token, from position 0.
    lb = eng.benchmark(int(tokens[0]), 4, 32)
    latency = {"semantics": "BaseLmEngine::benchmark: decode_token with the tied LM head, host wait per token",
               "mean_ms": round(lb["mean_ms"], 4), "min_ms": round(lb["min_ms"], 4), "max_ms": round(lb["max_ms"], 4),
               "tok_s": round(lb["tokens_per_second"], 1), "positions": "4..35"}
    log(f"reference-semantics decode (LM head, sync per token): {lb['mean_ms']:.3f} ms -> "
        f"{lb['tokens_per_second']:.1f} tok/s")
    long_ctx = long_context_leg(ctx, model, cfg) if args.long_context else None
    prefill = None
    if args.prefill_tokens:
        prefill = prefill_leg(ctx, eng, cfg, args.prefill_tokens, args.prefill_reps)
    residual = (residual_leg(ctx, args.residual_steps, baselm=eng, bcfg=cfg, cpu_steps=0 if args.no_cpu else 128)
                if args.residual_steps else None)
    eng.close()
    model.free()
    cfm = cfm_leg(ctx, args.cfm_reps) if args.cfm_reps else None
    audiovae = vae_leg(ctx, args.vae_frames, cpu_frames=0 if args.no_cpu else args.vae_frames) if args.vae_frames else None
    ctx.close()

    line = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(elapsed * 1e3 / K, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 x f32",
        "data": "synthetic",
        "config": {"workload": "baselm_q8_0_decode_28L_batch1", "layers": L, "hidden": H, "ffn": F,
                   "heads": "16q/2kv x 128", "vocab": V, "prefill": P,
                   "positions": f"{P}..{P + K - 1}", "lm_head": bool(args.lm_head),
                   "exec": args.mode, "parallelism": "single GPU"},
        "roofline": roofline,
        "matvec_family": {"achieved": round(fam_gbps, 1), "unit": "GB/s",
                          "frac": round(fam_gbps / HBM_PEAK_GBPS, 4),
                          "frac_of_achievable": round(fam_gbps / achievable["GBps"], 4),
                          "kernels": ["qkv", "attn_out", "swiglu", "down"]},
        "achievable": achievable,
        "c0": c0,
        "latency": latency,
        "step": {"bytes_mean": int(mean_step_bytes),
                 "achieved_GBps": round(mean_step_bytes * tok_s / 1e9, 1),
                 "frac": round(mean_step_bytes * tok_s / 1e9 / HBM_PEAK_GBPS, 4)},
        "per_kernel": per_kernel,
        "cpu_baseline": cpu,
        "long_context": long_ctx,
        "prefill": prefill,
        "cfm": cfm,
        "residual": residual,
        "audiovae": audiovae,
        "device": f"{info['name']} ({info['arch']})",
    }
    print(json.dumps(line), flush=True)


def cpu_baseline(cfg, m, eng, tokens, P, args):
    """The oracle's 28-layer decode on the host cores, on a bounded sample."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import voxref
    o = voxref.BaseLm(m.data, {t.name: t for t in m.tensors}, cfg)
    # KV cache of the prefill (positions 0..P-1), from the GPU run.
    o.kv_k[:] = eng.buffer("kv_k").download(np.uint16, o.kv_k.size)
    o.kv_v[:] = eng.buffer("kv_v").download(np.uint16, o.kv_v.size)
    t0 = time.perf_counter()
    o.decode_token(int(tokens[P]), P, logits=args.lm_head)
    one = time.perf_counter() - t0
    n = int(max(2, min(256, args.cpu_seconds // max(one, 1e-3))))
    n = min(n, len(tokens) - P - 1)
    t0 = time.perf_counter()
    for i in range(n):
        o.decode_token(int(tokens[P + 1 + i]), P + 1 + i, logits=args.lm_head)
    el = time.perf_counter() - t0
    thr = voxref.threads()
    log(f"cpu oracle: {n} steps in {el:.2f}s on {thr} threads")
    return {"value": round(n / el, 3), "unit": "tok/s", "cores": thr, "kind": "port",
            "sample": f"{n} decode steps at positions {P + 1}..{P + n} of the same 28-layer Q8_0 model and "
                      f"tokens (KV cache of the GPU prefill), C oracle (oracle/voxref.c) with OpenMP over rows; "
                      f"the reference's own CPU path (Rust + GLSL on Mesa lavapipe) is not buildable here",
            "cpu": cpu_model()}


def cpu_model():
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    main()
