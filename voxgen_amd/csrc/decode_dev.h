// Device helpers of the batch-1 matrix-vector kernels of the decode step
// (kernels_matvec.hip): wave64 row fragments over the lane-interleaved Q8_0
// repack (or F16 rows), x staged through LDS with an optional fused rmsnorm,
// fp32 dot products and DPP wave reductions. Everything is inline and lives in
// an unnamed namespace of the including translation unit.
#pragma once

#include <type_traits>

#include "vx_internal.h"

namespace vx {
namespace {

constexpr int kWavesPerBlock = 4;
constexpr int kBlock = 256;
constexpr uint32_t kGroupCols = 1024;

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// DPP reduction of a wave64 (gfx9 row/broadcast controls): quad swaps, row
// mirrors, then row_bcast15/31 fold the four 16-lane rows into lane 63, which is
// read back as a wave-uniform value. No LDS traffic.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK,
                                                                 0xf, false));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp<0xb1>(v);         // quad_perm [1,0,3,2]
    v += dpp<0x4e>(v);         // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);        // row_half_mirror
    v += dpp<0x140>(v);        // row_mirror
    v += dpp<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
    v += dpp<0x143, 0xc>(v);   // row_bcast:31 into rows 2 and 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ float h2f(unsigned short bits) {
    return (float)__builtin_bit_cast(_Float16, bits);
}
__device__ __forceinline__ float2 h2f2(uint32_t bits) {
    return make_float2(h2f((unsigned short)(bits & 0xffffu)), h2f((unsigned short)(bits >> 16)));
}

template <int WT>
__device__ __forceinline__ uint32_t frag_col(int g, int lane, int i) {
    if constexpr (WT == WT_Q8)
        return kGroupCols * (uint32_t)g + 256u * (uint32_t)(i >> 2) + 4u * (uint32_t)lane + (uint32_t)(i & 3);
    else
        return kGroupCols * (uint32_t)g + 512u * (uint32_t)(i >> 3) + 8u * (uint32_t)lane + (uint32_t)(i & 7);
}

template <int NG>
struct Frag {
    float v[NG][16];
};

// Per-chunk sums of the x fragment (the Q8_0 bias correction): sx[g][k] is the
// sum of the four x values lane-chunk k of group g multiplies.
template <int NG>
struct FragSums {
    float s[NG][4];
};
template <int NG>
__device__ __forceinline__ void frag_sums(const Frag<NG> &f, FragSums<NG> &sx) {
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int k = 0; k < 4; ++k)
            sx.s[g][k] = (f.v[g][4 * k] + f.v[g][4 * k + 1]) + (f.v[g][4 * k + 2] + f.v[g][4 * k + 3]);
}

// ------------------------------------------------------- x staged in LDS
// The workgroup loads x once (thread t: float4 at 1024j + 4t, j < NG), optionally
// applies rmsnorm(x)*w (rmsnorm.comp:21-42) with a block reduction, and stores it
// to LDS; every wave then reads its fragment from there. stage_issue only issues
// the loads, so a kernel can put its weight loads right behind them and
// stage_finish (which waits for x alone) overlaps the weight streaming.
template <int NG, bool NORM>
struct XStage {
    float4 v[NG];
    float4 w[NORM ? NG : 1];
};

template <int NG, bool NORM>
__device__ __forceinline__ void stage_issue(XStage<NG, NORM> &st, const float *x, const float *w, uint32_t cols) {
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        const uint32_t c = kGroupCols * j + 4u * t;
        const uint32_t cc = c < cols ? c : 0u;
        st.v[j] = *reinterpret_cast<const float4 *>(x + cc);
        if constexpr (NORM) st.w[j] = *reinterpret_cast<const float4 *>(w + cc);
    }
}

// x = xl[0..left) ++ xr[0..cols-left) (fusion_linear.comp:63), element by element.
template <int NG>
__device__ __forceinline__ void stage_issue_concat(XStage<NG, false> &st, const float *xl, const float *xr,
                                                   uint32_t left, uint32_t cols) {
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        float e[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t c = kGroupCols * j + 4u * t + q;
            const bool ok = c < cols;
            const uint32_t cc = ok ? c : 0u;
            const float v = cc < left ? xl[cc] : xr[cc - left];
            e[q] = ok ? v : 0.f;
        }
        st.v[j] = make_float4(e[0], e[1], e[2], e[3]);
    }
}

template <int NG, bool NORM>
__device__ __forceinline__ void stage_finish(XStage<NG, NORM> &st, float *xs, float *red, uint32_t cols, float eps) {
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < NG; ++j)
        if (kGroupCols * j + 4u * t >= cols) st.v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (NORM) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            ss = fmaf(st.v[j].x, st.v[j].x, ss);
            ss = fmaf(st.v[j].y, st.v[j].y, ss);
            ss = fmaf(st.v[j].z, st.v[j].z, ss);
            ss = fmaf(st.v[j].w, st.v[j].w, ss);
        }
        ss = wave_sum_dpp(ss);
        if ((t & 63u) == 0u) red[t >> 6] = ss;
        __syncthreads();
        const float total = (red[0] + red[1]) + (red[2] + red[3]);
        const float inv_rms = 1.0f / sqrtf(total / (float)cols + eps);
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            st.v[j].x = st.v[j].x * inv_rms * st.w[j].x;
            st.v[j].y = st.v[j].y * inv_rms * st.w[j].y;
            st.v[j].z = st.v[j].z * inv_rms * st.w[j].z;
            st.v[j].w = st.v[j].w * inv_rms * st.w[j].w;
        }
    }
#pragma unroll
    for (int j = 0; j < NG; ++j) *reinterpret_cast<float4 *>(xs + kGroupCols * j + 4u * t) = st.v[j];
    __syncthreads();
}

// Staging for workgroups of any wave count: the first 256 threads load x (and
// the norm weight w), store x (or x*w) to LDS and their per-wave partial sums of
// x^2 to red[0..3]; one barrier; every wave then reads its fragment. With NORM
// the rmsnorm's scalar 1/rms is returned instead of being applied to x, so the
// caller multiplies its reduced dot products by it: rmsnorm(x)*w . W[r] =
// (1/rms) * ((x*w) . W[r]). A scheduling barrier ends the staging, so the
// compiler cannot hoist weight arithmetic (which waits for the weight loads)
// above the LDS stores that other waves are waiting for at the barrier.
template <int NG, bool NORM>
__device__ __forceinline__ void stage_issue_first256(XStage<NG, NORM> &st, const float *x, const float *w,
                                                     uint32_t cols) {
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        st.v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (NORM) st.w[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (t < (uint32_t)kBlock) stage_issue<NG, NORM>(st, x, w, cols);
}

template <int NG, bool NORM>
__device__ __forceinline__ float stage_finish_first256(XStage<NG, NORM> &st, float *xs, float *red, uint32_t cols,
                                                       float eps) {
    const uint32_t t = threadIdx.x;
    if (t < (uint32_t)kBlock) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NG; ++j) {
            float4 v = st.v[j];
            if (kGroupCols * j + 4u * t >= cols) v = make_float4(0.f, 0.f, 0.f, 0.f);
            if constexpr (NORM) {
                ss = fmaf(v.x, v.x, ss);
                ss = fmaf(v.y, v.y, ss);
                ss = fmaf(v.z, v.z, ss);
                ss = fmaf(v.w, v.w, ss);
                v = make_float4(v.x * st.w[j].x, v.y * st.w[j].y, v.z * st.w[j].z, v.w * st.w[j].w);
            }
            *reinterpret_cast<float4 *>(xs + kGroupCols * j + 4u * t) = v;
        }
        if constexpr (NORM) {
            ss = wave_sum_dpp(ss);
            if ((t & 63u) == 0u) red[t >> 6] = ss;
        }
    }
    __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NORM) {
        const float total = (red[0] + red[1]) + (red[2] + red[3]);
        return 1.0f / sqrtf(total / (float)cols + eps);  // rmsnorm.comp:36-38
    } else {
        return 1.f;
    }
}

template <int WT, int NG>
__device__ __forceinline__ void frag_from_lds(Frag<NG> &f, const float *xs, int lane) {
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int i = 0; i < 16; i += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(xs + frag_col<WT>(g, lane, i));
            f.v[g][i] = v.x;
            f.v[g][i + 1] = v.y;
            f.v[g][i + 2] = v.z;
            f.v[g][i + 3] = v.w;
        }
}

// ---------------------------------------------------------------- Q8_0 rows
template <int NG>
struct Q8Row {
    uint4 q[NG];
    uint2 d[NG];
};

// Weight streams are read with nontemporal loads: a decode step reads 1.4 GB of
// weights once, and with ordinary loads they evict the KV cache, the activation
// vectors and the attention partials (a few MB, reused within the step and from
// step to step) from the L2s and the MALL. Decode 1433 -> 1491 tok/s.
typedef uint32_t vx_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t vx_u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ld_w16(const void *p) {
    const vx_u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const vx_u32x4 *>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 ld_w8(const void *p) {
    const vx_u32x2 v = __builtin_nontemporal_load(reinterpret_cast<const vx_u32x2 *>(p));
    return make_uint2(v[0], v[1]);
}

template <int NG>
__device__ __forceinline__ void load_row(Q8Row<NG> &r, const WRef &w, uint32_t row, uint32_t cols,
                                         int lane) {
    const int8_t *qrow = static_cast<const int8_t *>(w.ptr) + (size_t)row * cols;
    const unsigned short *drow = reinterpret_cast<const unsigned short *>(w.d) + (size_t)row * (cols >> 5);
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        r.q[g] = ld_w16(qrow + kGroupCols * g + 16 * lane);
        r.d[g] = ld_w8(drow + 32 * g + 4 * (lane >> 3));
    }
}

template <int NG>
__device__ __forceinline__ float row_dot(const Q8Row<NG> &r, const Frag<NG> &f, const FragSums<NG> &sx) {
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const uint32_t qw[4] = {r.q[g].x ^ 0x80808080u, r.q[g].y ^ 0x80808080u, r.q[g].z ^ 0x80808080u,
                                r.q[g].w ^ 0x80808080u};
        const float dk[4] = {h2f((unsigned short)(r.d[g].x & 0xffffu)), h2f((unsigned short)(r.d[g].x >> 16)),
                             h2f((unsigned short)(r.d[g].y & 0xffffu)), h2f((unsigned short)(r.d[g].y >> 16))};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float *x = &f.v[g][4 * k];
            float t0 = (float)(qw[k] & 0xffu) * x[0];
            float t1 = (float)((qw[k] >> 8) & 0xffu) * x[1];
            t0 = fmaf((float)((qw[k] >> 16) & 0xffu), x[2], t0);
            t1 = fmaf((float)(qw[k] >> 24), x[3], t1);
            const float t = fmaf(-128.f, sx.s[g][k], t0 + t1);
            if (k & 1)
                acc1 = fmaf(dk[k], t, acc1);
            else
                acc0 = fmaf(dk[k], t, acc0);
        }
    }
    return acc0 + acc1;
}

// ----------------------------------------------------------------- F16 rows
template <int NG>
struct F16Row {
    uint4 c[NG][2];
};

template <int NG>
__device__ __forceinline__ void load_row(F16Row<NG> &r, const WRef &w, uint32_t row, uint32_t cols,
                                         int lane) {
    const __half *wrow = static_cast<const __half *>(w.ptr) + (size_t)row * cols;
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t col = kGroupCols * g + 512u * h + 8u * lane;
            const bool ok = col < cols;
            const uint4 v = ld_w16(wrow + (ok ? col : 0u));
            r.c[g][h] = ok ? v : make_uint4(0u, 0u, 0u, 0u);
        }
}

template <int NG>
__device__ __forceinline__ float row_dot(const F16Row<NG> &r, const Frag<NG> &f, const FragSums<NG> &) {
    float s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t u[4] = {r.c[g][h].x, r.c[g][h].y, r.c[g][h].z, r.c[g][h].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float2 wv = h2f2(u[i]);
                s0 = fmaf(wv.x, f.v[g][8 * h + 2 * i], s0);
                s1 = fmaf(wv.y, f.v[g][8 * h + 2 * i + 1], s1);
            }
        }
    return s0 + s1;
}

template <int WT, int NG>
using RowT = typename std::conditional<WT == WT_Q8, Q8Row<NG>, F16Row<NG>>::type;

}  // namespace
}  // namespace vx
