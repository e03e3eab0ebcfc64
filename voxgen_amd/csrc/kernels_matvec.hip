// Batch-1 matrix-vector kernels for gfx950 (the HBM-bound "matvec family").
//
// Design (one wave64 owns RPW whole rows):
//   * Columns are taken in 1024-column groups. In each group lane l owns 16
//     columns whose x values are float4 loads contiguous across the wave:
//       Q8_0: columns 1024g + 256k + 4l + j      (k, j < 4; fragment index 4k + j)
//       F16 : columns 1024g + 512h + 8l + j      (h < 2, j < 8; index 8h + j)
//     The workgroup stages x (with its rmsnorm where fused) in LDS once; each
//     lane reads its x values from there and keeps them in registers for every
//     row the wave streams.
//   * Q8_0 rows come from the lane-interleaved repack (model.cpp): per lane and
//     group one 16 B load of quants and one 8 B load of its four block scales,
//     so every weight load instruction of a wave reads contiguous bytes. Bytes
//     are flipped to q+128 and converted with v_cvt_f32_ubyteN; the bias is
//     removed with the per-chunk sum of x: d*(sum (q+128)x - 128 sum x).
//   * F16 rows: two 16 B loads per lane and group, straight from the GGUF layout.
//   * All weight loads of the wave's rows are issued before any arithmetic, right
//     after the x loads, so HBM latency is paid once per wave and the staging of
//     x overlaps the weight streaming.
//   * fp32 accumulation, DPP wave reduction, lane 0 runs the epilogue.
// No MFMA: at batch 1 the arithmetic intensity is ~1 FLOP/byte.
#include "decode_dev.h"

namespace vx {
namespace {

// ------------------------------------------------------------ plain matvec
struct MvArgs {
    WRef w;
    const float *xl, *xr;
    uint32_t left, rows, cols, row_base;
    float alpha;
    const void *bias;
    uint32_t bias_dtype;
    float *y, *y2;
    float scale;
    VX_STAMP_FIELD
};

// Epilogue variants are compile-time: each kernel instance has one
// straight-line epilogue, with no runtime branch on the bias dtype.
enum Ep : int {
    EP_STORE = 0,       // y = alpha * acc                      (matvec.comp:61; linear_bias without bias)
    EP_BIAS_F32,        // y = alpha * (acc + f32 bias)         (linear_bias.comp:78-81)
    EP_BIAS_F16,        // y = alpha * (acc + f16 bias)
    EP_FUSION_F32,      // y = snapshot = acc + f32 bias        (fusion_linear.comp:72-77)
    EP_FUSION_F16,      // y = snapshot = acc + f16 bias
    EP_RESIDUAL,        // hidden += scale * acc                (residual_rmsnorm.comp:27-28)
    EP_RESIDUAL_BRANCH  // branch = acc; hidden += scale * acc
};

// Epilogue operand of a row (old hidden value, or the bias), loaded at kernel
// start so that no global load sits between the reduction and the store.
template <int EP>
__device__ __forceinline__ float epilogue_operand(const MvArgs &a, uint32_t row) {
    if constexpr (EP == EP_BIAS_F32 || EP == EP_FUSION_F32) return static_cast<const float *>(a.bias)[row];
    else if constexpr (EP == EP_BIAS_F16 || EP == EP_FUSION_F16)
        return h2f(static_cast<const unsigned short *>(a.bias)[row]);
    else if constexpr (EP == EP_RESIDUAL || EP == EP_RESIDUAL_BRANCH) return a.y[row];
    else return 0.f;
}

template <int EP>
__device__ __forceinline__ void epilogue(const MvArgs &a, uint32_t row, float acc, float op) {
    if constexpr (EP == EP_STORE) {
        a.y[row] = acc * a.alpha;                        // matvec.comp:61
    } else if constexpr (EP == EP_BIAS_F32 || EP == EP_BIAS_F16) {
        a.y[row] = (acc + op) * a.alpha;                 // linear_bias.comp:78-81
    } else if constexpr (EP == EP_FUSION_F32 || EP == EP_FUSION_F16) {
        const float v = acc + op;                        // fusion_linear.comp:72-77
        a.y[row] = v;
        a.y2[row] = v;
    } else {
        if constexpr (EP == EP_RESIDUAL_BRANCH) a.y2[row] = acc;
        a.y[row] = op + acc * a.scale;                   // residual_rmsnorm.comp:27-28
    }
}

// Issue order: x (L2-resident) first, then the weight rows (HBM), then the
// epilogue operands, so that vmcnt's in-order accounting lets the LDS staging of
// x proceed while the weights are in flight. Rows past the end are clamped to a
// valid row and their results dropped (no early exit: the staging has barriers).
// WPB waves share one staging of x: the staging reads are per workgroup, and
// under a full weight stream they compete with it for the L2 and the CU's load
// path, so the large shapes use 8-wave workgroups (measured on MI355X: down
// 5.28 -> 4.90 us, attn_out-shaped 3.03 -> 2.74 us against 4-wave groups).
template <int WT, int NG, int RPW, int EP, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_matvec(MvArgs a) {
    VX_WAVE_STAMP(a.stamps);
    __shared__ __align__(16) float xs[NG * kGroupCols];
    __shared__ float red[kWavesPerBlock];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar row math
    const uint32_t row0 = a.row_base + (blockIdx.x * WPB + wave) * RPW;
    // Only fusion_linear reads a concatenated x (compile-time, so the plain path
    // keeps its float4 loads).
    constexpr bool CONCAT = EP == EP_FUSION_F32 || EP == EP_FUSION_F16;
    XStage<NG, false> st;
    if constexpr (CONCAT) {
#pragma unroll
        for (int j = 0; j < NG; ++j) st.v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (threadIdx.x < (unsigned)kBlock) stage_issue_concat<NG>(st, a.xl, a.xr, a.left, a.cols);
    } else {
        stage_issue_first256<NG, false>(st, a.xl, nullptr, a.cols);
    }
    __builtin_amdgcn_sched_barrier(0);
    RowT<WT, NG> r[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) load_row(r[i], a.w, min(row0 + i, a.rows - 1u), a.cols, lane);
    float op[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) op[i] = epilogue_operand<EP>(a, min(row0 + i, a.rows - 1u));
    __builtin_amdgcn_sched_barrier(0);
    stage_finish_first256<NG, false>(st, xs, red, a.cols, 0.f);
    Frag<NG> f;
    frag_from_lds<WT, NG>(f, xs, lane);
    FragSums<NG> sx;
    frag_sums(f, sx);
    float acc[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) acc[i] = wave_sum_dpp(row_dot(r[i], f, sx));
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < RPW; ++i)
            if (row0 + i < a.rows) epilogue<EP>(a, row0 + i, acc[i], op[i]);
    }
}

// attn_out with the attention merge folded in: hidden += scale * Wo . attn, where
// attn is merged from the k_attn_chunk partials of every query head. The wave's
// weight rows are requested first; the 256 threads then merge the partials into
// LDS (each thread 4*NG consecutive outputs of one head, every split's record
// loaded before any is used) while those rows stream in, and every wave reads
// its x fragment from LDS. cols == q_heads * HD == 1024 * NG.
struct AttnOutArgs {
    MvArgs mv;
    float *attn;             // nullable: workgroup 0 also stores the merged vector here
    const float *part;
    const uint32_t *position;
    uint32_t context, splits;
};

template <int WT, int NG, int RPW, int HD, bool BRANCH, int WPB, int FS>
__global__ __launch_bounds__(64 * WPB) void k_attn_out(AttnOutArgs a) {
    VX_WAVE_STAMP(a.mv.stamps);
    // The first MT threads merge E outputs each (float4 units): every one of the
    // workgroup's threads up to 1024*NG/4 of them.
    constexpr int MT = 64 * WPB < 256 * NG ? 64 * WPB : 256 * NG;
    constexpr int E = 1024 * NG / MT;
    static_assert(E >= 4 && E % 4 == 0, "merge works in float4 units");
    __shared__ __align__(16) float xs[NG * kGroupCols];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const MvArgs &m = a.mv;
    const uint32_t row0 = (blockIdx.x * WPB + wave) * RPW;  // no early exit: barrier below
    // Every split record of this thread's head is requested up front, whatever
    // the position (records past the active splits get weight 0 by a select), so
    // these loads do not wait for the position and go out ahead of the weights.
    const bool merger = tid < MT;
    const uint32_t o0 = (uint32_t)(E * (merger ? tid : 0)), hh = o0 / HD, d0 = o0 % HD;
    float2 ml[FS];
    float4 av[FS][E / 4];
#pragma unroll
    for (uint32_t s = 0; s < FS; ++s) {
        ml[s] = make_float2(0.f, 0.f);
#pragma unroll
        for (int e = 0; e < E / 4; ++e) av[s][e] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (merger) {  // wave-uniform: MT is a multiple of 64
#pragma unroll
        for (uint32_t s = 0; s < FS; ++s) {
            const float *rec = a.part + ((size_t)hh * a.splits + (s < a.splits ? s : 0u)) * (HD + 4);
            ml[s] = *reinterpret_cast<const float2 *>(rec);
#pragma unroll
            for (int e = 0; e < E / 4; ++e) av[s][e] = *reinterpret_cast<const float4 *>(rec + 4 + d0 + 4 * e);
        }
    }
    const SplitPlan plan = split_plan(a.position, a.context, a.splits);
    __builtin_amdgcn_sched_barrier(0);
    RowT<WT, NG> r[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) load_row(r[i], m.w, min(row0 + i, m.rows - 1u), m.cols, lane);
    float op[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) op[i] = m.y[min(row0 + i, m.rows - 1u)];
    __builtin_amdgcn_sched_barrier(0);
    // Merge of the partials (k_attn_combine's arithmetic).
    float mx = -3.402823466e+38f;
#pragma unroll
    for (uint32_t s = 0; s < FS; ++s)
        if (s < plan.active) mx = fmaxf(mx, ml[s].x);
    float l = 0.f, o[E];
#pragma unroll
    for (int e = 0; e < E; ++e) o[e] = 0.f;
#pragma unroll
    for (uint32_t s = 0; s < FS; ++s) {
        const bool on = s < plan.active;
        const float w = on ? expf(ml[s].x - mx) : 0.f;
        l = on ? fmaf(ml[s].y, w, l) : l;
#pragma unroll
        for (int e = 0; e < E / 4; ++e) {
            o[4 * e] = on ? fmaf(av[s][e].x, w, o[4 * e]) : o[4 * e];
            o[4 * e + 1] = on ? fmaf(av[s][e].y, w, o[4 * e + 1]) : o[4 * e + 1];
            o[4 * e + 2] = on ? fmaf(av[s][e].z, w, o[4 * e + 2]) : o[4 * e + 2];
            o[4 * e + 3] = on ? fmaf(av[s][e].w, w, o[4 * e + 3]) : o[4 * e + 3];
        }
    }
    const float inv_l = 1.0f / l;
#pragma unroll
    for (int e = 0; e < E; e += 4)
        if (merger) {
            const float4 v = make_float4(o[e] * inv_l, o[e + 1] * inv_l, o[e + 2] * inv_l, o[e + 3] * inv_l);
            *reinterpret_cast<float4 *>(&xs[o0 + e]) = v;
            if (a.attn && blockIdx.x == 0) *reinterpret_cast<float4 *>(a.attn + o0 + e) = v;
        }
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    Frag<NG> f;
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(&xs[frag_col<WT>(g, lane, i)]);
            f.v[g][i] = v.x;
            f.v[g][i + 1] = v.y;
            f.v[g][i + 2] = v.z;
            f.v[g][i + 3] = v.w;
        }
    FragSums<NG> sx;
    frag_sums(f, sx);
    float acc[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) acc[i] = wave_sum_dpp(row_dot(r[i], f, sx));
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < RPW; ++i)
            if (row0 + i < m.rows) {
                if constexpr (BRANCH) m.y2[row0 + i] = acc[i];
                m.y[row0 + i] = op[i] + acc[i] * m.scale;
            }
    }
}

// Reference-shaped fallback for any dtype/shape (matvec.comp / linear_bias.comp):
// one 256-thread block per row, reading the GGUF layout from the raw region.
__device__ __forceinline__ float raw_weight(const uint8_t *raw, uint32_t off, uint32_t dtype,
                                            uint32_t cols, uint32_t row, uint32_t col) {
    if (dtype == VX_DTYPE_F32) {
        float v;
        memcpy(&v, raw + off + ((size_t)row * cols + col) * 4u, 4);
        return v;
    }
    if (dtype == VX_DTYPE_F16)
        return h2f(*reinterpret_cast<const unsigned short *>(raw + off + ((size_t)row * cols + col) * 2u));
    const size_t block = (size_t)row * (cols / 32u) + col / 32u;
    const uint8_t *b = raw + off + block * 34u;
    const int q = (int)(int8_t)b[2 + (col & 31u)];
    return h2f((unsigned short)(b[0] | (b[1] << 8))) * (float)q;
}

__device__ __forceinline__ float block_sum(float v, float *red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += red[i];
    return t;
}

template <int EP>
__global__ __launch_bounds__(kBlock) void k_matvec_generic(MvArgs a) {
    __shared__ float red[kBlock / 64];
    const uint32_t row = a.row_base + blockIdx.x;
    if (row >= a.rows) return;
    float s = 0.f;
    for (uint32_t c = threadIdx.x; c < a.cols; c += kBlock) {
        const float x = c < a.left ? a.xl[c] : a.xr[c - a.left];
        s += raw_weight(a.w.raw, a.w.raw_offset, a.w.dtype, a.cols, row, c) * x;
    }
    s = block_sum(s, red);
    if (threadIdx.x == 0) epilogue<EP>(a, row, s, epilogue_operand<EP>(a, row));
}

// --------------------------------------------------------------- SwiGLU
struct SwArgs {
    WRef g, u;
    const float *x, *norm;
    float eps;
    uint32_t rows, cols, row_base;
    float *y;
    VX_STAMP_FIELD
};

__device__ __forceinline__ float silu_mul(float g, float u) {
    return (g / (1.0f + expf(-g))) * u;  // matvec_swiglu.comp:67
}

// With the rmsnorm fused (ffn_norm), x*w is staged and 1/rms scales the two
// reduced dot products: silu(g/rms) * (u/rms).
template <int WT, int NG, int RPW, bool NORM, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_swiglu(SwArgs a) {
    VX_WAVE_STAMP(a.stamps);
    __shared__ __align__(16) float xs[NG * kGroupCols];
    __shared__ float red[kWavesPerBlock];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar row math
    const uint32_t row0 = a.row_base + (blockIdx.x * WPB + wave) * RPW;
    XStage<NG, NORM> st;
    stage_issue_first256<NG, NORM>(st, a.x, a.norm, a.cols);
    __builtin_amdgcn_sched_barrier(0);
    RowT<WT, NG> rg[RPW], ru[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const uint32_t row = min(row0 + i, a.rows - 1u);
        load_row(rg[i], a.g, row, a.cols, lane);
        load_row(ru[i], a.u, row, a.cols, lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    const float inv = stage_finish_first256<NG, NORM>(st, xs, red, a.cols, a.eps);
    Frag<NG> f;
    frag_from_lds<WT, NG>(f, xs, lane);
    FragSums<NG> sx;
    frag_sums(f, sx);
    float gs[RPW], us[RPW];
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        gs[i] = wave_sum_dpp(row_dot(rg[i], f, sx)) * inv;
        us[i] = wave_sum_dpp(row_dot(ru[i], f, sx)) * inv;
    }
    if (lane == 0) {
#pragma unroll
        for (int i = 0; i < RPW; ++i)
            if (row0 + i < a.rows) a.y[row0 + i] = silu_mul(gs[i], us[i]);
    }
}

__global__ __launch_bounds__(kBlock) void k_swiglu_generic(SwArgs a) {
    __shared__ float red[kBlock / 64];
    __shared__ float inv_s;
    const uint32_t row = a.row_base + blockIdx.x;
    if (row >= a.rows) return;
    float inv_rms = 1.f;
    if (a.norm) {
        float ss = 0.f;
        for (uint32_t c = threadIdx.x; c < a.cols; c += kBlock) ss += a.x[c] * a.x[c];
        ss = block_sum(ss, red);
        if (threadIdx.x == 0) inv_s = 1.0f / sqrtf(ss / (float)a.cols + a.eps);
        __syncthreads();
        inv_rms = inv_s;
    }
    float gs = 0.f, us = 0.f;
    for (uint32_t c = threadIdx.x; c < a.cols; c += kBlock) {
        const float x = a.norm ? a.x[c] * inv_rms * a.norm[c] : a.x[c];
        gs += raw_weight(a.g.raw, a.g.raw_offset, a.g.dtype, a.cols, row, c) * x;
        us += raw_weight(a.u.raw, a.u.raw_offset, a.u.dtype, a.cols, row, c) * x;
    }
    gs = block_sum(gs, red);
    us = block_sum(us, red);
    if (threadIdx.x == 0) a.y[row] = silu_mul(gs, us);
}

// ------------------------------------------- fused rmsnorm+QKV+RoPE+KV store
struct QkvArgs {
    WRef q, k, v;
    const float *hidden, *norm;
    float eps;
    uint32_t q_rows, kv_rows, cols, head_dim;
    const float *factors;
    float theta, scaling;
    uint32_t layer, context;
    float *qo, *ko, *vo;
    __half *kc, *vc;
    const uint32_t *position;
    const float2 *rope_cs;
    uint32_t no_rope;
    VX_STAMP_FIELD
};

// One wave per rotary pair: Q/K rows (i, i + head_dim/2) of a head, or two
// adjacent V rows. RoPE (rope.comp:28-49) and the f16 cache store
// (store_kv.comp:21-23) run on the reduced pair in lane 0.
template <int WT, int NG, int WPB>
__global__ __launch_bounds__(64 * WPB) void k_qkv_fused(QkvArgs a) {
    VX_WAVE_STAMP(a.stamps);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar row math
    __shared__ __align__(16) float xs[NG * kGroupCols];
    __shared__ float red[kWavesPerBlock];
    const uint32_t half_dim = a.head_dim >> 1;
    const uint32_t pq = a.q_rows >> 1, pk = a.kv_rows >> 1;
    const uint32_t p_raw = blockIdx.x * WPB + wave;
    const bool live = p_raw < pq + 2u * pk;  // no early exit: the staging has barriers
    const uint32_t p = live ? p_raw : pq + 2u * pk - 1u;
    int seg;
    uint32_t r0, r1;
    if (p < pq + pk) {
        seg = p < pq ? 0 : 1;
        const uint32_t pp = seg == 0 ? p : p - pq;
        const uint32_t head = pp / half_dim, i = pp % half_dim;
        r0 = head * a.head_dim + i;
        r1 = r0 + half_dim;
    } else {
        seg = 2;
        r0 = 2u * (p - pq - pk);
        r1 = r0 + 1u;
    }
    // Scalar selects of the segment's matrix (p and seg are wave-uniform).
    WRef w;
    w.ptr = seg == 0 ? a.q.ptr : (seg == 1 ? a.k.ptr : a.v.ptr);
    w.d = seg == 0 ? a.q.d : (seg == 1 ? a.k.d : a.v.d);
    XStage<NG, true> st;
    stage_issue_first256<NG, true>(st, a.hidden, a.norm, a.cols);
    __builtin_amdgcn_sched_barrier(0);
    RowT<WT, NG> rr[2];
    load_row(rr[0], w, r0, a.cols, lane);
    load_row(rr[1], w, r1, a.cols, lane);
    const uint32_t pos = *a.position;
    const uint32_t pair = r0 % a.head_dim;
    const bool rotate = seg < 2 && !a.no_rope;   // q/k rotated unless the stack runs without RoPE
    const float ext = rotate && !a.rope_cs ? a.factors[pair] : 1.f;
    const float2 cs_tab = rotate && a.rope_cs ? a.rope_cs[pair] : make_float2(1.f, 0.f);
    __builtin_amdgcn_sched_barrier(0);
    const float inv = stage_finish_first256<NG, true>(st, xs, red, a.cols, a.eps);
    Frag<NG> f;
    frag_from_lds<WT, NG>(f, xs, lane);
    FragSums<NG> sx;
    frag_sums(f, sx);
    float v0 = wave_sum_dpp(row_dot(rr[0], f, sx)) * inv;
    float v1 = wave_sum_dpp(row_dot(rr[1], f, sx)) * inv;
    if (lane != 0 || !live) return;
    if (rotate) {
        float c = cs_tab.x, s = cs_tab.y;
        if (!a.rope_cs) {  // rope.comp:28-41 inline
            const float exponent = (float)(pair * 2u) / (float)a.head_dim;
            const float inv_freq = 1.0f / powf(a.theta, exponent);
            const float angle = (float)pos * inv_freq / ext;
            c = cosf(angle) * a.scaling;
            s = sinf(angle) * a.scaling;
        }
        const float n0 = v0 * c - v1 * s;
        const float n1 = v1 * c + v0 * s;
        v0 = n0;
        v1 = n1;
    }
    float *dst = seg == 0 ? a.qo : (seg == 1 ? a.ko : a.vo);
    dst[r0] = v0;
    dst[r1] = v1;
    if (seg > 0 && pos < a.context) {
        __half *cache = seg == 1 ? a.kc : a.vc;
        const size_t base = ((size_t)a.layer * a.context + pos) * a.kv_rows;
        cache[base + r0] = __float2half_rn(v0);
        cache[base + r1] = __float2half_rn(v1);
    }
}

// --------------------------------------------------------------- utility
__global__ void k_dequant(WRef w, uint32_t rows, uint32_t cols, float *out) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (size_t)rows * cols) return;
    const uint32_t row = (uint32_t)(idx / cols), col = (uint32_t)(idx % cols);
    float v;
    if (w.wt == WT_Q8 && w.ptr) {
        // Inverse of the repack: column c = 1024g + 256k + 4l + j.
        const uint32_t g = col >> 10, k = (col >> 8) & 3u, l = (col >> 2) & 63u, j = col & 3u;
        const int8_t q = static_cast<const int8_t *>(w.ptr)[(size_t)row * cols + 1024u * g + 16u * l + 4u * k + j];
        const uint32_t m = l >> 3;
        const unsigned short dbits =
            reinterpret_cast<const unsigned short *>(w.d)[(size_t)row * (cols >> 5) + 32u * g + 4u * m + k];
        v = h2f(dbits) * (float)q;
    } else {
        v = raw_weight(w.raw, w.raw_offset, w.dtype, cols, row, col);
    }
    out[idx] = v;
}

// One thread per (row, 1024-column group, lane): gathers the lane's 16 quants of
// the group from four GGUF blocks and, for lanes 8m, the group's four scales of
// lane group m. cols % 1024 == 0.
__global__ void k_repack_q8(const uint8_t *raw, uint32_t rows, uint32_t cols, int8_t *qs,
                            unsigned short *d) {
    const uint32_t nb = cols >> 5, ng = cols >> 10;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (size_t)rows * ng * 64u) return;
    const uint32_t lane = (uint32_t)(t & 63u);
    const uint32_t g = (uint32_t)((t >> 6) % ng);
    const uint32_t row = (uint32_t)((t >> 6) / ng);
    const uint32_t m = lane >> 3, within = 4u * (lane & 7u);
    uint32_t words[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint8_t *blk = raw + ((size_t)row * nb + 32u * g + 8u * k + m) * 34u;
        words[k] = (uint32_t)blk[2 + within] | ((uint32_t)blk[3 + within] << 8) |
                   ((uint32_t)blk[4 + within] << 16) | ((uint32_t)blk[5 + within] << 24);
        if ((lane & 7u) == 0u)
            d[(size_t)row * nb + 32u * g + 4u * m + k] = (unsigned short)(blk[0] | (blk[1] << 8));
    }
    *reinterpret_cast<uint4 *>(qs + (size_t)row * cols + 1024u * g + 16u * lane) =
        make_uint4(words[0], words[1], words[2], words[3]);
}

// Column-group counts (cols / 1024, rounded up) with compiled fast paths.
bool ng_supported(uint32_t ng) { return ng == 1u || ng == 2u || ng == 3u || ng == 4u || ng == 6u || ng == 8u; }

template <int WT, int EP>
int dispatch_matvec_ng(hipStream_t s, const MvArgs &a, uint32_t ng) {
    const uint32_t n = a.rows - a.row_base;
    const bool big = n > 8192u && ng <= 2u;
#define VX_MV(NGV, RPWV, WPBV)                                                                       \
    do {                                                                                             \
        const uint32_t per_block = (WPBV) * (RPWV);                                                  \
        const uint32_t grid = (n + per_block - 1) / per_block;                                       \
        MvArgs b = a;                                                                                \
        VX_SET_STAMPS(b, ST_MATVEC, (uint64_t)grid * (WPBV));                                        \
        k_matvec<WT, NGV, RPWV, EP, WPBV><<<grid, 64 * (WPBV), 0, s>>>(b);                           \
    } while (0)
    switch (ng) {
        case 1:
            if (big) VX_MV(1, 4, 4); else VX_MV(1, 2, 4);
            break;
        case 2:
            if (big) VX_MV(2, 4, 4); else VX_MV(2, 1, 8);   // 2048 rows: 256 workgroups of 8 waves
            break;
        case 3: VX_MV(3, 2, 4); break;
        case 4: VX_MV(4, 2, 4); break;
        case 6: VX_MV(6, 1, 8); break;   // one row per wave, 8 waves: 256 workgroups for 2048 rows
        default: VX_MV(8, 1, 4); break;
    }
#undef VX_MV
    VX_LAUNCHED("k_matvec");
    return VX_OK;
}

template <int EP>
int launch_matvec_ep(hipStream_t s, const MvArgs &a, const WRef &w, bool fast, uint32_t ng) {
    if (fast) {
        if (w.wt == WT_Q8) return dispatch_matvec_ng<WT_Q8, EP>(s, a, ng);
        return dispatch_matvec_ng<WT_F16, EP>(s, a, ng);
    }
    k_matvec_generic<EP><<<a.rows - a.row_base, kBlock, 0, s>>>(a);
    VX_LAUNCHED("k_matvec_generic");
    return VX_OK;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

// Fast (wave-per-row) path: Q8_0 in the repacked layout with cols % 1024 == 0,
// or F16 with cols % 8 == 0; and a compiled column-group count.
bool fast_weight_ok(const WRef &w, uint32_t cols) {
    if (!ng_supported((cols + kGroupCols - 1) / kGroupCols)) return false;
    if (w.wt == WT_Q8)
        return w.ptr && w.d && cols % kGroupCols == 0 && aligned16(w.ptr) && ((uintptr_t)w.d & 7u) == 0;
    if (w.wt == WT_F16) return cols % 8u == 0 && aligned16(w.ptr);
    return false;
}

}  // namespace

int launch_matvec(hipStream_t s, const MatvecLaunch &l) {
    if (l.rows <= l.row_base || l.cols == 0) return VX_OK;
    if (l.xr && l.epi != EPI_FUSION)
        return fail(VX_ERR_INVALID_ARG, "a concatenated x is only read by the fusion epilogue");
    MvArgs a{};
    a.w = l.w;
    a.xl = l.xl;
    a.xr = l.xr ? l.xr : l.xl;
    a.left = l.xr ? l.left_cols : l.cols;
    a.rows = l.rows;
    a.cols = l.cols;
    a.row_base = l.row_base;
    a.alpha = l.alpha;
    a.bias = l.bias;
    a.bias_dtype = l.bias_dtype;
    a.y = l.y;
    a.y2 = l.y2;
    a.scale = l.scale;
    const uint32_t ng = (l.cols + kGroupCols - 1) / kGroupCols;
    const bool fast = fast_weight_ok(l.w, l.cols) && aligned16(l.xl);
    const bool has_bias = l.bias != nullptr && l.bias_dtype <= 1u;
    switch (l.epi) {
        case EPI_STORE: return launch_matvec_ep<EP_STORE>(s, a, l.w, fast, ng);
        case EPI_BIAS:
            if (!has_bias) return launch_matvec_ep<EP_STORE>(s, a, l.w, fast, ng);
            if (l.bias_dtype == 0u) return launch_matvec_ep<EP_BIAS_F32>(s, a, l.w, fast, ng);
            return launch_matvec_ep<EP_BIAS_F16>(s, a, l.w, fast, ng);
        case EPI_FUSION:
            if (!l.bias || !l.y2) return fail(VX_ERR_INVALID_ARG, "fusion epilogue needs a bias and a snapshot");
            if (l.bias_dtype == 0u) return launch_matvec_ep<EP_FUSION_F32>(s, a, l.w, fast, ng);
            return launch_matvec_ep<EP_FUSION_F16>(s, a, l.w, fast, ng);
        case EPI_RESIDUAL:
            if (l.y2) return launch_matvec_ep<EP_RESIDUAL_BRANCH>(s, a, l.w, fast, ng);
            return launch_matvec_ep<EP_RESIDUAL>(s, a, l.w, fast, ng);
        default: return fail(VX_ERR_INVALID_ARG, "unknown matvec epilogue %d", l.epi);
    }
}

int launch_swiglu(hipStream_t s, const SwigluLaunch &l) {
    if (l.rows <= l.row_base || l.cols == 0) return VX_OK;
    SwArgs a{l.g, l.u, l.x, l.norm, l.eps, l.rows, l.cols, l.row_base, l.y};
    const uint32_t ng = (l.cols + kGroupCols - 1) / kGroupCols;
    const uint32_t n = l.rows - l.row_base;
    const bool fast = l.g.wt == l.u.wt && fast_weight_ok(l.g, l.cols) && fast_weight_ok(l.u, l.cols) &&
                      aligned16(l.x) && (!l.norm || aligned16(l.norm));
    if (!fast) {
        k_swiglu_generic<<<n, kBlock, 0, s>>>(a);
        VX_LAUNCHED("k_swiglu_generic");
        return VX_OK;
    }
#define VX_SW(WTV, NGV, RPWV, WPBV)                                                                     \
    do {                                                                                                \
        const uint32_t grid = (n + (WPBV) * (RPWV) - 1) / ((WPBV) * (RPWV));                           \
        VX_SET_STAMPS(a, ST_SWIGLU, (uint64_t)grid * (WPBV));                                           \
        if (l.norm)                                                                                     \
            k_swiglu<WTV, NGV, RPWV, true, WPBV><<<grid, 64 * (WPBV), 0, s>>>(a);                       \
        else                                                                                            \
            k_swiglu<WTV, NGV, RPWV, false, WPBV><<<grid, 64 * (WPBV), 0, s>>>(a);                      \
    } while (0)
#define VX_SW_NG(WTV)                             \
    switch (ng) {                                 \
        case 1: VX_SW(WTV, 1, 2, 4); break;       \
        case 2: VX_SW(WTV, 2, 1, 8); break;       \
        case 3: VX_SW(WTV, 3, 2, 4); break;       \
        case 4: VX_SW(WTV, 4, 2, 4); break;       \
        case 6: VX_SW(WTV, 6, 1, 4); break;       \
        default: VX_SW(WTV, 8, 1, 4); break;      \
    }
    if (l.g.wt == WT_Q8) {
        VX_SW_NG(WT_Q8)
    } else {
        VX_SW_NG(WT_F16)
    }
#undef VX_SW_NG
#undef VX_SW
    VX_LAUNCHED("k_swiglu");
    return VX_OK;
}

int launch_qkv_fused(hipStream_t s, const QkvFusedLaunch &l) {
    const uint32_t ng = (l.cols + kGroupCols - 1) / kGroupCols;
    if (!fast_weight_ok(l.q, l.cols) || !fast_weight_ok(l.k, l.cols) ||
        !fast_weight_ok(l.v, l.cols) || l.q.wt != l.k.wt || l.q.wt != l.v.wt ||
        !aligned16(l.hidden) || !aligned16(l.norm) || (l.q_rows & 1u) || (l.kv_rows & 1u) ||
        (l.head_dim & 1u) || l.head_dim == 0)
        return fail(VX_ERR_UNSUPPORTED,
                    "fused QKV needs Q8_0 (cols %% 1024 == 0) or F16 weights of one dtype, a compiled "
                    "column count and aligned buffers");
    QkvArgs a{l.q,      l.k,        l.v,       l.hidden,  l.norm,  l.eps,    l.q_rows, l.kv_rows,
              l.cols,   l.head_dim, l.factors, l.theta,   l.scaling, l.layer, l.context, l.qo,
              l.ko,     l.vo,       l.kc,      l.vc,      l.position, l.rope_cs, l.no_rope ? 1u : 0u};
    const uint32_t pairs = (l.q_rows + 2u * l.kv_rows) / 2u;
    // 8-wave workgroups (one staging of x per 8 rotary pairs).
    constexpr uint32_t WPB = 8;
    const uint32_t grid = (pairs + WPB - 1) / WPB;
    VX_SET_STAMPS(a, ST_QKV, (uint64_t)grid * WPB);
#define VX_QKV(WTV, NGV) k_qkv_fused<WTV, NGV, WPB><<<grid, 64 * WPB, 0, s>>>(a)
#define VX_QKV_NG(WTV)                      \
    switch (ng) {                           \
        case 1: VX_QKV(WTV, 1); break;      \
        case 2: VX_QKV(WTV, 2); break;      \
        case 3: VX_QKV(WTV, 3); break;      \
        case 4: VX_QKV(WTV, 4); break;      \
        case 6: VX_QKV(WTV, 6); break;      \
        default: VX_QKV(WTV, 8); break;     \
    }
    if (l.q.wt == WT_Q8) {
        VX_QKV_NG(WT_Q8)
    } else {
        VX_QKV_NG(WT_F16)
    }
#undef VX_QKV_NG
#undef VX_QKV
    VX_LAUNCHED("k_qkv_fused");
    return VX_OK;
}

int launch_attn_out(hipStream_t s, const AttnOutLaunch &l) {
    const uint32_t ng = l.mv.cols / kGroupCols;
    if (l.mv.cols != l.q_heads * l.head_dim || l.mv.cols % kGroupCols || (ng != 1u && ng != 2u) ||
        (l.head_dim != 64u && l.head_dim != 128u) || l.splits == 0 || l.splits > kMaxFoldedSplits ||
        !fast_weight_ok(l.mv.w, l.mv.cols) || l.mv.row_base != 0 || l.mv.epi != EPI_RESIDUAL)
        return fail(VX_ERR_UNSUPPORTED,
                    "attn_out merge needs cols = q_heads*head_dim in {1024, 2048}, head_dim 64/128, "
                    "<= %u splits and a fast-path weight", kMaxFoldedSplits);
    AttnOutArgs a{};
    a.mv.w = l.mv.w;
    a.mv.rows = l.mv.rows;
    a.mv.cols = l.mv.cols;
    a.mv.y = l.mv.y;
    a.mv.y2 = l.mv.y2;
    a.mv.scale = l.mv.scale;
    a.attn = l.attn_out;
    a.part = reinterpret_cast<const float *>(reinterpret_cast<const uint8_t *>(l.partials) + 256);
    a.position = l.position;
    a.context = l.context;
    a.splits = l.splits;
    // 2048 columns: 8 waves of one row (256 workgroups for 2048 rows; 16-wave groups,
    // half the merge traffic, measured slower: 4.98 against 4.52 us); 1024: 4 waves of two.
#define VX_AO_FS(WTV, NGV, HDV, RPWV, WPBV, FSV)                                                           \
    do {                                                                                                   \
        const uint32_t grid = (l.mv.rows + (WPBV) * (RPWV) - 1) / ((WPBV) * (RPWV));                      \
        VX_SET_STAMPS(a.mv, ST_ATTN_OUT, (uint64_t)grid * (WPBV));                                         \
        if (l.mv.y2)                                                                                       \
            k_attn_out<WTV, NGV, RPWV, HDV, true, WPBV, FSV><<<grid, 64 * (WPBV), 0, s>>>(a);            \
        else                                                                                               \
            k_attn_out<WTV, NGV, RPWV, HDV, false, WPBV, FSV><<<grid, 64 * (WPBV), 0, s>>>(a);           \
    } while (0)
    // The merge loads every record slot up to FS whatever the position: 8 slots
    // for the short contexts' splits, 16 for long ones.
#define VX_AO(WTV, NGV, HDV, RPWV, WPBV)                               \
    do {                                                               \
        if (l.splits <= kShortSplits) VX_AO_FS(WTV, NGV, HDV, RPWV, WPBV, 8);   \
        else VX_AO_FS(WTV, NGV, HDV, RPWV, WPBV, 16);                  \
    } while (0)
#define VX_AO_WT(WTV)                                                                \
    if (ng == 2u) {                                                                  \
        if (l.head_dim == 128u) VX_AO(WTV, 2, 128, 1, 8); else VX_AO(WTV, 2, 64, 1, 8); \
    } else {                                                                         \
        if (l.head_dim == 128u) VX_AO(WTV, 1, 128, 2, 4); else VX_AO(WTV, 1, 64, 2, 4); \
    }
    if (l.mv.w.wt == WT_Q8) {
        VX_AO_WT(WT_Q8)
    } else {
        VX_AO_WT(WT_F16)
    }
#undef VX_AO_WT
#undef VX_AO
#undef VX_AO_FS
    VX_LAUNCHED("k_attn_out");
    return VX_OK;
}

int launch_dequant(hipStream_t s, const WRef &w, uint32_t rows, uint32_t cols, float *out) {
    const size_t n = (size_t)rows * cols;
    k_dequant<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(w, rows, cols, out);
    VX_LAUNCHED("k_dequant");
    return VX_OK;
}

int launch_repack_q8(hipStream_t s, const uint8_t *raw_tensor, uint32_t rows, uint32_t cols,
                     int8_t *qs, __half *d) {
    if (cols % kGroupCols) return fail(VX_ERR_INVALID_ARG, "Q8_0 repack needs cols %% 1024 == 0");
    const size_t threads = (size_t)rows * (cols / kGroupCols) * 64u;
    if (!threads) return VX_OK;
    k_repack_q8<<<(unsigned)((threads + 255) / 256), 256, 0, s>>>(raw_tensor, rows, cols, qs,
                                                                  reinterpret_cast<unsigned short *>(d));
    VX_LAUNCHED("k_repack_q8");
    return VX_OK;
}

}  // namespace vx
