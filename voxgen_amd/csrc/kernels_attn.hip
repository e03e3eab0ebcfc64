// Single-query (decode) attention over the packed f16 KV cache.
//
// k_attn_chunk: grid = splits x q_heads. Each workgroup takes one query head and
// one contiguous slice of the context [0, position] and runs an online softmax
// over 64-key tiles of it: the 256 threads are 64 keys x 4 quarters of the head
// dimension for the scores (a quad reduction per key; lane r of a quad holds dims
// 8(r + 4i)..+7, so each load of the quad reads 64 contiguous bytes), then
// head_dim dims x 256/head_dim key groups for P.V out of LDS. It writes one
// (max, sum, acc) partial per (head, slice). Every load a tile needs (q, K and V rows) is issued
// before any of it is used. The GQA map is attn_scores.comp's kvh = qh / q_per_kv.
// k_attn_rows writes the same records for slices of many keys, each wave
// streaming its keys with whole-row loads (below). k_attn_combine merges the
// slices of each head; the engine's decode step folds
// that merge into the attn_out matvec instead (k_attn_out in kernels_matvec.hip).
// Mathematically this is attn_scores.comp -> softmax.comp -> attn_values.comp
// (baselm.rs:969-996).
//
// The reference-granular kernels below keep the exact three-dispatch shape.
#include <cfloat>

#include "vx_internal.h"

namespace vx {
namespace {

constexpr int kTile = 64;

__device__ __forceinline__ float2 h2f2(uint32_t bits) {
    const _Float16 lo = __builtin_bit_cast(_Float16, (unsigned short)(bits & 0xffffu));
    const _Float16 hi = __builtin_bit_cast(_Float16, (unsigned short)(bits >> 16));
    return make_float2((float)lo, (float)hi);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// DPP reductions (no LDS round trips): quad swaps, row mirrors, then
// row_bcast15/31 fold the four 16-lane rows into lane 63, read back as a
// wave-uniform value.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                                 0xf, false));
}
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_keep(float v) {  // lanes the control does not write keep v
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, v),
                                                                 __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                                 0xf, false));
}
__device__ __forceinline__ float uniform_lane63(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp<0xb1>(v);        // quad_perm [1,0,3,2]
    v += dpp<0x4e>(v);        // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);       // row_half_mirror
    v += dpp<0x140>(v);       // row_mirror
    v += dpp<0x142, 0xa>(v);  // row_bcast:15
    v += dpp<0x143, 0xc>(v);  // row_bcast:31
    return uniform_lane63(v);
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_keep<0xb1>(v));
    v = fmaxf(v, dpp_keep<0x4e>(v));
    v = fmaxf(v, dpp_keep<0x141>(v));
    v = fmaxf(v, dpp_keep<0x140>(v));
    v = fmaxf(v, dpp_keep<0x142, 0xa>(v));
    v = fmaxf(v, dpp_keep<0x143, 0xc>(v));
    return uniform_lane63(v);
}
// Sum over each aligned quad of lanes, result in all four lanes.
__device__ __forceinline__ float quad_sum(float v) {
    v += dpp<0xb1>(v);  // quad_perm [1,0,3,2]
    v += dpp<0x4e>(v);  // quad_perm [2,3,0,1]
    return v;
}

struct AttnArgs {
    const float *q;
    const __half *kc, *vc;
    float *out, *part;
    const uint32_t *position;
    uint32_t layer, context, q_heads, kv_heads, splits;
    VX_STAMP_FIELD
};

// Partial record of one (head, slice): m, l, 2 pad words, acc[HD] (16-byte aligned acc).
template <int HD>
__device__ __forceinline__ float *part_rec(const AttnArgs &a, uint32_t h, uint32_t s) {
    return a.part + ((size_t)h * a.splits + s) * (HD + 4);
}

// k_attn_chunk: see the file comment.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_chunk(AttnArgs a) {
    VX_WAVE_STAMP(a.stamps);
    constexpr int R = HD / 4;            // dims per quarter (scores)
    constexpr int KG = 256 / HD;         // key groups (P.V)
    constexpr int KPG = kTile / KG;      // keys per group
    __shared__ __align__(16) __half vs[kTile][HD];
    __shared__ float ps[kTile];
    __shared__ float red[2][4];
    __shared__ float accs[256];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t s = blockIdx.x, h = blockIdx.y;
    const uint32_t kvh = h / (a.q_heads / a.kv_heads);
    const uint32_t kv_dim = a.kv_heads * HD;
    const int j = tid >> 2, r = tid & 3;

    // q and, when the split's keys do not depend on the position
    // (attn_fixed_chunk), the K and V rows of its one tile are issued
    // before the position is read: the position is a scalar load issued after
    // them (a compiler barrier keeps that order), so waiting for it does not wait
    // for the vector loads.
    // q quarter: element 8k + e of quarter r is dimension 8(r + 4k) + e, so the
    // four lanes of a key read 64 contiguous bytes of its row per load.
    float qv[R];
#pragma unroll
    for (int i = 0; i < R; i += 4) {
        const float4 v = *reinterpret_cast<const float4 *>(a.q + (size_t)h * HD + 8 * (r + 4 * (i >> 3)) + (i & 7));
        qv[i] = v.x;
        qv[i + 1] = v.y;
        qv[i + 2] = v.z;
        qv[i + 3] = v.w;
    }
    const float inv_sqrt = 1.0f / sqrtf((float)HD);
    const size_t layer_base = (size_t)a.layer * a.context;
    const size_t head_off = (size_t)kvh * HD + (size_t)r * 8;
    const uint32_t fc = attn_fixed_chunk(a.context, a.splits);
    const bool fixed = fc <= kAttnFixedChunk;
    uint4 kpre[R / 8], vpre[R / 8];
    if (fixed) {
        const uint32_t key = min(s * fc + (uint32_t)j, a.context - 1u);
        const size_t row = (layer_base + key) * kv_dim + head_off;
#pragma unroll
        for (int i = 0; i < R / 8; ++i) {
            kpre[i] = *reinterpret_cast<const uint4 *>(a.kc + row + 32 * i);
            vpre[i] = *reinterpret_cast<const uint4 *>(a.vc + row + 32 * i);
        }
    }
    asm volatile("" ::: "memory");
    const uint32_t pos_raw = *a.position;
    const SplitPlan plan = split_plan_at(pos_raw, a.context, a.splits);
    if (s >= plan.active) return;
    const uint32_t t0 = s * plan.chunk;
    const uint32_t t1 = min(plan.n, t0 + plan.chunk);

    float m_run = -FLT_MAX, l_run = 0.f, acc = 0.f;
    auto tile = [&](uint32_t tb, const uint4 *kw, uint4 *vw) {
        const uint32_t key = tb + (uint32_t)j;
        const bool valid = key < t1;
        if (!valid) {   // a fetched row past the slice (or the position) enters with p = 0
#pragma unroll
            for (int i = 0; i < R / 8; ++i) vw[i] = make_uint4(0, 0, 0, 0);
        }
        // Score of key j: quarter dot product, then a quad reduction.
        float d0 = 0.f, d1 = 0.f;
#pragma unroll
        for (int i = 0; i < R / 8; ++i) {
            const uint32_t w4[4] = {kw[i].x, kw[i].y, kw[i].z, kw[i].w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float2 kf = h2f2(w4[t]);
                d0 = fmaf(qv[8 * i + 2 * t], kf.x, d0);
                d1 = fmaf(qv[8 * i + 2 * t + 1], kf.y, d1);
            }
        }
        float sc = quad_sum(d0 + d1);
        sc = valid ? sc * inv_sqrt : -FLT_MAX;
        // Tile max across the workgroup.
        const float wm = wave_max_dpp(sc);
        if (lane == 0) red[0][wave] = wm;
        __syncthreads();
        const float tmax = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
        const float m_new = fmaxf(m_run, tmax);
        const float p = valid ? expf(sc - m_new) : 0.f;
        // V rows of the tile and p to LDS; each key's p counted once (quarter 0).
#pragma unroll
        for (int i = 0; i < R / 8; ++i) lds_st16(&vs[j][8 * (r + 4 * i)], vw[i]);
        if (r == 0) ps[j] = p;
        const float ws = wave_sum_dpp(r == 0 ? p : 0.f);
        if (lane == 0) red[1][wave] = ws;
        __syncthreads();
        const float tsum = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
        const float corr = expf(m_run - m_new);
        l_run = l_run * corr + tsum;
        m_run = m_new;
        // P.V: thread = (key group, dim).
        const int d = tid % HD, kg = tid / HD;
        float v = 0.f;
#pragma unroll 8
        for (int jj = 0; jj < KPG; ++jj) {
            const int k = kg * KPG + jj;
            v = fmaf(ps[k], __half2float(vs[k][d]), v);
        }
        acc = acc * corr + v;
        __syncthreads();
    };
    if (fixed) {
        tile(t0, kpre, vpre);
    } else {
        // Slices of several tiles: the next tile's rows are requested before the
        // current tile is computed, so each tile after the first waits only for
        // what its predecessor's arithmetic did not cover.
        auto fetch = [&](uint32_t tb, uint4 *kw, uint4 *vw) {
            const uint32_t key = tb + (uint32_t)j;
            const size_t row = (layer_base + (key < t1 ? key : t0)) * kv_dim + head_off;
#pragma unroll
            for (int i = 0; i < R / 8; ++i) {
                kw[i] = *reinterpret_cast<const uint4 *>(a.kc + row + 32 * i);
                vw[i] = *reinterpret_cast<const uint4 *>(a.vc + row + 32 * i);
            }
        };
        uint4 kw[R / 8], vw[R / 8], kn[R / 8], vn[R / 8];
        fetch(t0, kw, vw);
        for (uint32_t tb = t0; tb < t1; tb += kTile) {
            const bool more = tb + kTile < t1;   // workgroup-uniform
            if (more) fetch(tb + kTile, kn, vn);
            tile(tb, kw, vw);
#pragma unroll
            for (int i = 0; i < R / 8; ++i) {
                kw[i] = kn[i];
                vw[i] = vn[i];
            }
        }
    }
    accs[tid] = acc;
    __syncthreads();
    float *rec = part_rec<HD>(a, h, s);
    if (tid < HD) {
        float t = 0.f;
#pragma unroll
        for (int kg = 0; kg < KG; ++kg) t += accs[kg * HD + tid];
        rec[4 + tid] = t;
    }
    if (tid == 0) {
        rec[0] = m_run;
        rec[1] = l_run;
    }
}

// Lane-group reductions for k_attn_rows. A group is CH = 8 or 16 aligned lanes.
template <int CH>
__device__ __forceinline__ float group_sum(float v) {   // result in every lane of the group
    v += dpp<0xb1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4e>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror: the other quad of the half-row
    if constexpr (CH == 16) v += dpp<0x140>(v);   // row_mirror: the other half-row
    return v;
}
// The two values of a row pair (v_permlane16_swap: rows 0/1, 2/3) or of a
// half-wave pair (v_permlane32_swap): element 0 holds the lower row's value and
// element 1 the upper row's, in every lane of both rows.
__device__ __forceinline__ float2 pair16(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return make_float2(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
__device__ __forceinline__ float2 pair32(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return make_float2(__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1]));
}
// Over the wave's groups, lane c of every group meeting lane c of the others
// (for CH = 8 the two groups of a row first, by a rotation of 8).
template <int CH>
__device__ __forceinline__ float groups_sum(float v) {
    if constexpr (CH == 8) v += dpp<0x128>(v);   // row_ror:8
    float2 t = pair16(v);
    v = t.x + t.y;
    t = pair32(v);
    return t.x + t.y;
}
template <int CH>
__device__ __forceinline__ float groups_max(float v) {
    if constexpr (CH == 8) v = fmaxf(v, dpp<0x128>(v));
    float2 t = pair16(v);
    v = fmaxf(t.x, t.y);
    t = pair32(v);
    return fmaxf(t.x, t.y);
}

// k_attn_rows: the same partial records for slices of many keys (long contexts,
// and short ones whose slices depend on the position). Each of the NW waves
// streams its own keys with no LDS or barrier inside the key loop. A lane is
// chunk c (8 dimensions) of key group g, CH = HD / 8 lanes per key, so one
// 16-byte load instruction of the wave reads KPI = 64 / CH consecutive keys'
// rows of the KV head whole (256 bytes each at head_dim 128). A wave step is NL
// load instructions of K and of V (16 keys at head_dim 128), key base + KPI i + g
// in load i; scores are reduced over the group's lanes (DPP) and kept in log2
// units (exp2 on the hardware's v_exp_f32), and the sum of p and the 8
// accumulators per lane follow the online softmax with a lazy reference max (it
// moves only when a step's max exceeds it by more than 8 in log2 units). Rows
// are addressed by 32-bit byte offsets from the layer's (uniform) KV base. When a slice holds at most one step of keys whatever the
// position (attn_fixed_chunk <= STEP), the rows are requested before the position
// is read, as in k_attn_chunk, and rows past the position enter with p = 0 and
// zeroed V. After the loop the groups' accumulators meet by lane swaps, and the
// NW waves meet once in LDS. DEPTH steps of rows are in flight per wave (3: five
// and seven measured slower at 4113 and 8017 keys, 6.8 / 8.8 and 6.8 / 9.5 us
// against 6.3 / 8.6). The record's max is stored in natural-log units, like
// k_attn_chunk's.
template <int HD, int NW, int DEPTH = 3>
__global__ __launch_bounds__(64 * NW) void k_attn_rows(AttnArgs a) {
    VX_WAVE_STAMP(a.stamps);
    constexpr int CH = HD / 8;             // lanes per key
    constexpr int KPI = 64 / CH;           // keys per load instruction
    constexpr int NL = 4;                  // load instructions per step (K and V each)
    constexpr uint32_t STEPW = KPI * NL;   // keys per wave step
    constexpr uint32_t STEP = STEPW * NW;  // keys per workgroup step
    __shared__ float osh[NW][HD];
    __shared__ float wm[NW], wl[NW];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane / CH, c = lane % CH;
    const uint32_t s = blockIdx.x, h = blockIdx.y;
    const uint32_t kvh = h / (a.q_heads / a.kv_heads);
    const uint32_t row_bytes = a.kv_heads * HD * 2u;   // < 2^24, as is every key index (launch checks)
    const size_t layer_off = ((size_t)a.layer * a.context * a.kv_heads + kvh) * HD;
    const char *kb = reinterpret_cast<const char *>(a.kc + layer_off);
    const char *vb = reinterpret_cast<const char *>(a.vc + layer_off);
    const uint32_t lane_bytes = 16u * (uint32_t)c;
    // A step whose keys all lie at or before `last` (the common case: wave-uniform)
    // steps one offset by KPI rows per load; a step across `last` clamps each key.
    const uint32_t load_stride = KPI * row_bytes;
    auto fetch = [&](uint32_t base, uint32_t last, uint4 *kw, uint4 *vw) {
        if (base + STEPW - 1u <= last) {
            uint32_t off = __umul24(base + g, row_bytes) + lane_bytes;
#pragma unroll
            for (int i = 0; i < NL; ++i, off += load_stride) {
                kw[i] = *reinterpret_cast<const uint4 *>(kb + off);
                vw[i] = *reinterpret_cast<const uint4 *>(vb + off);
            }
        } else {
#pragma unroll
            for (int i = 0; i < NL; ++i) {
                const uint32_t off = __umul24(min(base + KPI * i + g, last), row_bytes) + lane_bytes;
                kw[i] = *reinterpret_cast<const uint4 *>(kb + off);
                vw[i] = *reinterpret_cast<const uint4 *>(vb + off);
            }
        }
    };
    const uint32_t fc = attn_fixed_chunk(a.context, a.splits);
    const bool fixed = fc <= kAttnFixedChunk && fc <= STEP;   // one step per slice, position-independent
    uint4 kr[DEPTH][NL], vr[DEPTH][NL];   // ring of DEPTH steps of rows in flight
    if (fixed) fetch(s * fc + STEPW * (uint32_t)wave, a.context - 1u, kr[0], vr[0]);
    float qv[8];
    {
        const float4 q0 = *reinterpret_cast<const float4 *>(a.q + (size_t)h * HD + 8 * c);
        const float4 q1 = *reinterpret_cast<const float4 *>(a.q + (size_t)h * HD + 8 * c + 4);
        qv[0] = q0.x, qv[1] = q0.y, qv[2] = q0.z, qv[3] = q0.w;
        qv[4] = q1.x, qv[5] = q1.y, qv[6] = q1.z, qv[7] = q1.w;
    }
    asm volatile("" ::: "memory");   // the fixed rows are requested before the position
    const SplitPlan plan = split_plan(a.position, a.context, a.splits);
    if (s >= plan.active) return;
    const uint32_t t0 = s * plan.chunk;
    const uint32_t t1 = min(plan.n, t0 + plan.chunk);
    const float scale = 1.4426950408889634f / sqrtf((float)HD);   // log2(e) / sqrt(d)
    float m = -FLT_MAX, lp = 0.f, o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.f;
    auto step = [&](uint32_t base, const uint4 *kw, const uint4 *vw) {
        float sc[NL];
        bool valid[NL];
        float smax = -FLT_MAX;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const uint32_t w4[4] = {kw[i].x, kw[i].y, kw[i].z, kw[i].w};
            float d0 = 0.f, d1 = 0.f;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float2 kf = h2f2(w4[t]);
                d0 = fmaf(qv[2 * t], kf.x, d0);
                d1 = fmaf(qv[2 * t + 1], kf.y, d1);
            }
            const float d = group_sum<CH>(d0 + d1);
            valid[i] = base + KPI * i + g < t1;
            sc[i] = valid[i] ? d * scale : -FLT_MAX;
            smax = fmaxf(smax, sc[i]);
        }
        // Lazy reference max (the same in every lane): it moves, and rescales the
        // sums, only when a step's max exceeds it by more than 2^8 in p.
        const float smax_all = groups_max<CH>(smax);
        if (smax_all > m + 8.f) {
            const float corr = __builtin_amdgcn_exp2f(m - smax_all);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] *= corr;
            lp *= corr;
            m = smax_all;
        }
        float ps = 0.f;
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const float p = valid[i] ? __builtin_amdgcn_exp2f(sc[i] - m) : 0.f;
            ps += p;
            const uint32_t w4[4] = {vw[i].x, vw[i].y, vw[i].z, vw[i].w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const float2 vf = h2f2(w4[t]);
                o[2 * t] = fmaf(p, vf.x, o[2 * t]);
                o[2 * t + 1] = fmaf(p, vf.y, o[2 * t + 1]);
            }
        }
        lp += ps;
    };
    const uint32_t base0 = t0 + STEPW * (uint32_t)wave;   // wave-uniform
    if (fixed) {
        // Rows past the position may hold anything; 0 * inf would not be 0.
#pragma unroll
        for (int i = 0; i < NL; ++i)
            if (base0 + KPI * i + g >= t1) vr[0][i] = make_uint4(0u, 0u, 0u, 0u);
    } else {
        fetch(base0, t1 - 1u, kr[0], vr[0]);
    }
#pragma unroll
    for (int u = 1; u < DEPTH; ++u) {
#pragma unroll
        for (int i = 0; i < NL; ++i) kr[u][i] = vr[u][i] = make_uint4(0u, 0u, 0u, 0u);
        if (base0 + u * STEP < t1) fetch(base0 + u * STEP, t1 - 1u, kr[u], vr[u]);
    }
    for (uint32_t b = base0; b < t1; b += DEPTH * STEP) {
#pragma unroll
        for (int u = 0; u < DEPTH; ++u) {
            const uint32_t bu = b + u * STEP;
            if (bu >= t1) break;
            step(bu, kr[u], vr[u]);
            if (bu + DEPTH * STEP < t1) fetch(bu + DEPTH * STEP, t1 - 1u, kr[u], vr[u]);
        }
    }
    // A wave with no key keeps m = -FLT_MAX, lp = 0, o = 0. Every lane of a
    // group holds the group's sum of p; each group is counted once.
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = groups_sum<CH>(o[e]);
    const float lw = groups_sum<CH>(lp);
    if (g == 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) osh[wave][8 * c + e] = o[e];
    }
    if (lane == 0) {
        wm[wave] = m;
        wl[wave] = lw;
    }
    __syncthreads();
    float mm = wm[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) mm = fmaxf(mm, wm[w]);
    float sw[NW], ll = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        sw[w] = wl[w] > 0.f ? __builtin_amdgcn_exp2f(wm[w] - mm) : 0.f;
        ll = fmaf(wl[w], sw[w], ll);
    }
    float *rec = part_rec<HD>(a, h, s);
    if (tid < HD) {
        float acc = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) acc = fmaf(osh[w][tid], sw[w], acc);
        rec[4 + tid] = acc;
    }
    if (tid == 0) {
        rec[0] = mm * 0.6931471805599453f;   // natural-log units
        rec[1] = ll;
    }
}

// Merge the active slices of one query head (one block of 512 threads per head).
// The block is G = 512 / HD groups of HD threads; group g takes slices
// g, g + G, ... and every lane issues the loads of all its slices' (max, sum)
// and accumulator before using any, so the merge costs one round trip to memory
// whatever the slice count. The groups' partial merges meet in LDS.
constexpr uint32_t kCombineThreads = 512;
template <int HD>
__global__ __launch_bounds__(kCombineThreads) void k_attn_combine(AttnArgs a) {
    constexpr uint32_t G = kCombineThreads / HD;          // slice groups
    constexpr uint32_t U = kMaxAttnSplits / G;            // slices per group at most
    __shared__ float gm[G], gl[G];
    __shared__ float gv[G][HD];
    const uint32_t h = blockIdx.x, d = threadIdx.x % HD, g = threadIdx.x / HD;
    const SplitPlan plan = split_plan(a.position, a.context, a.splits);
    float2 ml[U];
    float av[U];
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
        const uint32_t sl = g + G * u;
        const float *rec = part_rec<HD>(a, h, sl < plan.active ? sl : 0u);
        ml[u] = *reinterpret_cast<const float2 *>(rec);
        av[u] = rec[4 + d];
    }
    float m = -FLT_MAX;
#pragma unroll
    for (uint32_t u = 0; u < U; ++u)
        if (g + G * u < plan.active) m = fmaxf(m, ml[u].x);
    float l = 0.f, v = 0.f;
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) {
        const bool on = g + G * u < plan.active;
        const float w = on ? expf(ml[u].x - m) : 0.f;
        l = fmaf(ml[u].y, w, l);
        v = fmaf(av[u], w, v);
    }
    if (d == 0) {
        gm[g] = m;
        gl[g] = l;
    }
    gv[g][d] = v;
    __syncthreads();
    if (g == 0) {
        float mm = gm[0];
#pragma unroll
        for (uint32_t i = 1; i < G; ++i) mm = fmaxf(mm, gm[i]);
        float ll = 0.f, vv = 0.f;
#pragma unroll
        for (uint32_t i = 0; i < G; ++i) {
            const float w = gl[i] > 0.f ? expf(gm[i] - mm) : 0.f;   // a group with no active slice adds nothing
            ll = fmaf(gl[i], w, ll);
            vv = fmaf(gv[i][d], w, vv);
        }
        a.out[(size_t)h * HD + d] = vv / ll;
    }
}

// ------------------------------------------------ reference-granular kernels
// Host positions are validated before launch; a device position is clamped to
// the context so it can never index past the cache.
__device__ __forceinline__ uint32_t eff_pos(uint32_t pos, const uint32_t *dev, uint32_t context) {
    const uint32_t p = dev ? *dev : pos;
    return p < context ? p : context - 1u;
}

// attn_scores.comp:27-44: one 128-lane block per (key t, query head).
__global__ __launch_bounds__(128) void k_attn_scores(const float *q, const __half *kc, float *scores,
                                                     uint32_t layer, uint32_t context, uint32_t pos_in,
                                                     const uint32_t *dev_pos, uint32_t head_dim,
                                                     uint32_t q_per_kv, uint32_t kv_heads) {
    __shared__ float red[2];
    const uint32_t lane = threadIdx.x, t = blockIdx.x, qh = blockIdx.y;
    const uint32_t pos = eff_pos(pos_in, dev_pos, context);
    if (t > pos) return;
    const uint32_t kvh = qh / q_per_kv;
    const uint32_t kv_dim = kv_heads * head_dim;
    float prod = 0.f;
    if (lane < head_dim)
        prod = q[qh * head_dim + lane] *
               __half2float(kc[((size_t)layer * context + t) * kv_dim + kvh * head_dim + lane]);
    prod = wave_sum(prod);
    if ((lane & 63u) == 0) red[lane >> 6] = prod;
    __syncthreads();
    if (lane == 0) scores[(size_t)qh * context + t] = (red[0] + red[1]) * (1.0f / sqrtf((float)head_dim));
}

// softmax.comp:15-47 over t <= position, one 256-thread block per head.
__global__ __launch_bounds__(256) void k_softmax(float *scores, uint32_t context, uint32_t pos_in,
                                                 const uint32_t *dev_pos) {
    __shared__ float red[4];
    __shared__ float bcast;
    const uint32_t lane = threadIdx.x, head = blockIdx.x;
    const uint32_t pos = eff_pos(pos_in, dev_pos, context);
    float *s = scores + (size_t)head * context;
    float m = -3.402823466e+38f;
    for (uint32_t t = lane; t <= pos; t += 256) m = fmaxf(m, s[t]);
    m = wave_max(m);
    if ((lane & 63u) == 0) red[lane >> 6] = m;
    __syncthreads();
    if (lane == 0) bcast = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    const float gmax = bcast;
    float sum = 0.f;
    for (uint32_t t = lane; t <= pos; t += 256) sum += expf(s[t] - gmax);
    sum = wave_sum(sum);
    __syncthreads();
    if ((lane & 63u) == 0) red[lane >> 6] = sum;
    __syncthreads();
    if (lane == 0) bcast = 1.0f / (red[0] + red[1] + red[2] + red[3]);
    __syncthreads();
    const float inv_sum = bcast;
    for (uint32_t t = lane; t <= pos; t += 256) s[t] = expf(s[t] - gmax) * inv_sum;
}

// attn_values.comp:25-37: one block per query head, one lane per dimension,
// serial over keys.
__global__ __launch_bounds__(128) void k_attn_values(const float *scores, const __half *vc, float *out,
                                                     uint32_t layer, uint32_t context, uint32_t pos_in,
                                                     const uint32_t *dev_pos, uint32_t head_dim,
                                                     uint32_t q_per_kv, uint32_t kv_heads) {
    const uint32_t d = threadIdx.x, qh = blockIdx.x;
    if (d >= head_dim) return;
    const uint32_t pos = eff_pos(pos_in, dev_pos, context);
    const uint32_t kvh = qh / q_per_kv;
    const uint32_t kv_dim = kv_heads * head_dim;
    float accv = 0.f;
    for (uint32_t t = 0; t <= pos; ++t)
        accv += scores[(size_t)qh * context + t] *
                __half2float(vc[((size_t)layer * context + t) * kv_dim + kvh * head_dim + d]);
    out[qh * head_dim + d] = accv;
}

}  // namespace

uint64_t attn_scratch_bytes(uint32_t head_dim, uint32_t q_heads, uint32_t kv_heads, uint32_t splits) {
    (void)kv_heads;
    return 256u + (uint64_t)q_heads * splits * (head_dim + 4u) * 4u;
}

namespace {
int attn_validate(const AttnLaunch &l) {
    if (l.kv_heads == 0 || l.q_heads % l.kv_heads)
        return fail(VX_ERR_UNSUPPORTED, "decode attention needs q_heads to be a multiple of kv_heads");
    if (l.splits == 0 || l.splits > kMaxAttnSplits)
        return fail(VX_ERR_INVALID_ARG, "splits must be 1..%u", kMaxAttnSplits);
    if (l.context == 0) return fail(VX_ERR_INVALID_ARG, "context is zero");
    if (l.head_dim != 128 && l.head_dim != 64)
        return fail(VX_ERR_UNSUPPORTED, "decode attention supports head_dim 64 or 128, got %u", l.head_dim);
    return VX_OK;
}
AttnArgs attn_args(const AttnLaunch &l) {
    return AttnArgs{l.q, l.kc, l.vc, l.out, reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(l.partials) + 256),
                    l.position, l.layer, l.context, l.q_heads, l.kv_heads, l.splits};
}
}  // namespace

int launch_attn_partials(hipStream_t s, const AttnLaunch &l) {
    VX_CHECK(attn_validate(l));
    AttnArgs a = attn_args(l);
    dim3 grid(l.splits, l.q_heads);
    VX_SET_STAMPS(a, ST_ATTN_CHUNK, (uint64_t)l.splits * l.q_heads * 4u);
    if (l.head_dim == 128)
        k_attn_chunk<128><<<grid, 256, 0, s>>>(a);
    else
        k_attn_chunk<64><<<grid, 256, 0, s>>>(a);
    VX_LAUNCHED("k_attn_chunk");
    return VX_OK;
}

int launch_attn_stream(hipStream_t s, const AttnLaunch &l, uint32_t waves) {
    VX_CHECK(attn_validate(l));
    if (waves != 4u && waves != 8u) return fail(VX_ERR_INVALID_ARG, "stream attention runs 4 or 8 waves");
    // k_attn_rows addresses a layer's rows by 32-bit byte offsets and 24-bit products.
    if (l.context >= (1u << 24) || (uint64_t)l.context * l.kv_heads * l.head_dim * 2u >= (1ull << 32))
        return fail(VX_ERR_UNSUPPORTED, "stream attention: a layer's K (or V) rows must span under 4 GiB");
    AttnArgs a = attn_args(l);
    dim3 grid(l.splits, l.q_heads);
    const bool eight = waves == 8u;
    VX_SET_STAMPS(a, ST_ATTN_STREAM, (uint64_t)l.splits * l.q_heads * waves);
    if (l.head_dim == 128) {
        if (eight) k_attn_rows<128, 8><<<grid, 512, 0, s>>>(a);
        else k_attn_rows<128, 4><<<grid, 256, 0, s>>>(a);
    } else {
        if (eight) k_attn_rows<64, 8><<<grid, 512, 0, s>>>(a);
        else k_attn_rows<64, 4><<<grid, 256, 0, s>>>(a);
    }
    VX_LAUNCHED("k_attn_rows");
    return VX_OK;
}

int launch_attn_combine(hipStream_t s, const AttnLaunch &l) {
    VX_CHECK(attn_validate(l));
    const AttnArgs a = attn_args(l);
    if (l.head_dim == 128)
        k_attn_combine<128><<<l.q_heads, kCombineThreads, 0, s>>>(a);
    else
        k_attn_combine<64><<<l.q_heads, kCombineThreads, 0, s>>>(a);
    VX_LAUNCHED("k_attn_combine");
    return VX_OK;
}

int launch_attn_decode(hipStream_t s, const AttnLaunch &l) {
    VX_CHECK(launch_attn_partials(s, l));
    return launch_attn_combine(s, l);
}

int launch_attn_scores(hipStream_t s, const float *q, const __half *kc, float *scores, uint32_t layer,
                       uint32_t context, uint32_t position, const uint32_t *dev_position,
                       uint32_t head_dim, uint32_t q_per_kv, uint32_t kv_heads, uint32_t q_heads) {
    if (head_dim == 0 || head_dim > 128) return fail(VX_ERR_UNSUPPORTED, "attn_scores: head_dim must be 1..128");
    const uint32_t keys = dev_position ? context : position + 1u;
    dim3 grid(keys, q_heads);
    k_attn_scores<<<grid, 128, 0, s>>>(q, kc, scores, layer, context, position, dev_position, head_dim,
                                       q_per_kv, kv_heads);
    VX_LAUNCHED("k_attn_scores");
    return VX_OK;
}

int launch_softmax(hipStream_t s, float *scores, uint32_t heads, uint32_t context, uint32_t position,
                   const uint32_t *dev_position) {
    k_softmax<<<heads, 256, 0, s>>>(scores, context, position, dev_position);
    VX_LAUNCHED("k_softmax");
    return VX_OK;
}

int launch_attn_values(hipStream_t s, const float *scores, const __half *vc, float *out, uint32_t layer,
                       uint32_t context, uint32_t position, const uint32_t *dev_position,
                       uint32_t head_dim, uint32_t q_per_kv, uint32_t kv_heads, uint32_t q_heads) {
    if (head_dim == 0 || head_dim > 128) return fail(VX_ERR_UNSUPPORTED, "attn_values: head_dim must be 1..128");
    k_attn_values<<<q_heads, 128, 0, s>>>(scores, vc, out, layer, context, position, dev_position,
                                          head_dim, q_per_kv, kv_heads);
    VX_LAUNCHED("k_attn_values");
    return VX_OK;
}

}  // namespace vx
