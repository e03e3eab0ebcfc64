// Token-batched ("seq") kernels for gfx950: the prefill projections as MFMA
// GEMMs, causal attention over the f16 KV cache on MFMA, and the per-token ops
// around them (rmsnorm, RoPE, KV store).
//
// Projection GEMM  C[t][n] = sum_k X[t][k] * W[n][k]  (t: token, n: weight row)
//   * v_mfma_f32_32x32x16_f16, fp32 accumulation. Workgroup tile 64 tokens x 128
//     rows, 4 waves of 32 tokens x 64 rows (two 32x32 MFMA tiles each), k-stages
//     of 128 columns staged through LDS, next stage prefetched into registers
//     while the current one is multiplied. __launch_bounds__(256, 2): two
//     workgroups per CU so one's MFMA chain overlaps the other's VALU work.
//   * Q8_0 weights are read from the lane-interleaved repack the decode matvecs
//     stream (model.cpp). Every 128-byte span of a repacked row holds four whole
//     32-column blocks (block 32g + 8kk + m, kk < 4, for span m of 1024-column
//     group g), so a k-stage is one span per row: its int8 quants are widened to
//     f16 exactly (|q| <= 127) into LDS and the block scales d are applied in fp32
//     after each block's MFMAs: acc += d[n][b] * (sum_{k in b} q*x). The weights
//     enter the product exactly, as d*q does in matvec.comp:32-44.
//   * Activations are carried as two f16 planes, hi = f16(x), lo = f16(x - hi),
//     and both are multiplied (two MFMAs per k-step), so x enters the product
//     with ~22 significant bits. Activations must stay inside the f16 range
//     (|x| < 65504); the producers of the planes are the seq kernels below.
//   * F16 weights (the LocEnc/LocDiT seq_* shaders) are staged as they are.
//   * Workgroups are numbered XCD-major: consecutive ids of one XCD cover all
//     token tiles of the same weight rows, so each weight tile is read from HBM
//     once and reused from that XCD's L2.
//   * Split-K over k-stages with fp32 atomic adds for the thin (N <= 2560)
//     projections, so that a T = 384 prefill still fills 256 CUs.
#include <cfloat>

#include "vx_internal.h"

namespace vx {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float acc16 __attribute__((ext_vector_type(16)));

constexpr int GM = 64;      // tokens per workgroup tile
constexpr int GN = 128;     // weight rows per workgroup tile
constexpr int GK = 128;     // columns per k-stage
constexpr int LROW = 136;   // f16 per LDS row: 128 + 8 pad (272 B; rows shift 4 banks)

__device__ __forceinline__ acc16 mfma(h8 a, h8 b, acc16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float h2f(unsigned short bits) {
    return (float)__builtin_bit_cast(_Float16, bits);
}

// Four signed int8 quants (one dword) -> four exact f16 values: (q ^ 0x80) is
// q + 128 in 0..255; the f16 with bits 0x6400 | u is 1024 + u, minus 1152 = q.
__device__ __forceinline__ uint2 q8x4_to_f16(uint32_t w) {
    const uint32_t u = w ^ 0x80808080u;
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const h2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const h2v a = __builtin_bit_cast(h2v, lo) - bias;
    const h2v b = __builtin_bit_cast(h2v, hi) - bias;
    return make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
}

// hi/lo f16 split of four floats.
__device__ __forceinline__ void split4(float4 v, uint2 &hi, uint2 &lo) {
    const h4 h = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
    const h4 l = {(_Float16)(v.x - (float)h[0]), (_Float16)(v.y - (float)h[1]), (_Float16)(v.z - (float)h[2]),
                  (_Float16)(v.w - (float)h[3])};
    hi = __builtin_bit_cast(uint2, h);
    lo = __builtin_bit_cast(uint2, l);
}

// Column of element c of stage block kk of k-stage s.
template <int WK>
__device__ __forceinline__ uint32_t stage_col(uint32_t s, uint32_t kk) {
    if constexpr (WK == WT_Q8)
        return 1024u * (s >> 3) + 256u * kk + 32u * (s & 7u);
    else
        return 128u * s + 32u * kk;
}

// Per-thread global row pointers of one workgroup tile, resolved once before
// the k-loop (segment selection stays in registers; the k-loop only adds the
// stage offset). Rows past a matrix and tokens past T are clamped to row 0 /
// token 0: they are loaded and multiplied like the others, and the epilogue
// never stores their results. Loads are therefore unconditional.
template <int WK, bool XF32>
struct TilePtrs {
    const uint8_t *w[WK == WT_Q8 ? 4 : 8];   // weight row starts
    const uint8_t *d;                         // Q8 scale row start
    const uint8_t *x[XF32 ? 8 : 4];           // input row starts (hi plane / f32)
};

// Weight row of LDS row rho of tile tn: which matrix (0: seg, 1: the up matrix
// of a SwiGLU tile) and its row index.
template <int EPI>
__device__ __forceinline__ void tile_row(uint32_t tn, uint32_t tile0, uint32_t rho, uint32_t &mat, uint32_t &row) {
    if constexpr (EPI == GEPI_SWIGLU) {
        mat = (rho >> 5) & 1u;
        row = 64u * tn + 32u * (rho >> 6) + (rho & 31u);
    } else {
        mat = 0;
        row = (tn - tile0) * GN + rho;
    }
}

template <int WK, bool XF32, int EPI>
__device__ __forceinline__ void tile_ptrs(const GemmSeg &s0, const GemmSeg &s1, const GemmArgs &a, uint32_t tn,
                                          uint32_t m0, TilePtrs<WK, XF32> &p) {
    const uint32_t tid = threadIdx.x;
    const size_t K = a.K;
    constexpr int NW = WK == WT_Q8 ? 4 : 8;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const uint32_t c = tid + 256u * i, rho = WK == WT_Q8 ? c >> 3 : c >> 4;
        uint32_t mat, row;
        tile_row<EPI>(tn, s0.tile0, rho, mat, row);
        const uint32_t rows = mat ? s1.rows : s0.rows;
        if (row >= rows) row = 0;
        const uint8_t *base = WK == WT_Q8 ? reinterpret_cast<const uint8_t *>(mat ? s1.qs : s0.qs)
                                          : reinterpret_cast<const uint8_t *>(mat ? s1.w : s0.w);
        p.w[i] = base + (size_t)row * K * (WK == WT_Q8 ? 1u : 2u);
    }
    if constexpr (WK == WT_Q8) {
        uint32_t mat, row;
        tile_row<EPI>(tn, s0.tile0, tid & (GN - 1u), mat, row);
        const uint32_t rows = mat ? s1.rows : s0.rows;
        if (row >= rows) row = 0;
        const uint8_t *base = reinterpret_cast<const uint8_t *>(mat ? s1.d : s0.d);
        p.d = base + (size_t)row * (K / 32u) * 2u;
    } else {
        p.d = nullptr;
    }
    constexpr int NX = XF32 ? 8 : 4;
#pragma unroll
    for (int i = 0; i < NX; ++i) {
        const uint32_t c = tid + 256u * i, t = XF32 ? c >> 5 : c >> 4;
        uint32_t tok = m0 + t;
        if (tok >= a.T) tok = 0;
        const uint8_t *base = XF32 ? reinterpret_cast<const uint8_t *>(a.xf) : reinterpret_cast<const uint8_t *>(a.xh);
        p.x[i] = base + (size_t)tok * a.ldx * (XF32 ? 4u : 2u);
    }
}

template <int WK, bool XF32>
struct StageRegs {
    uint4 w[WK == WT_Q8 ? 4 : 8];
    uint2 d;
    uint4 x[8];   // planes: 4 hi + 4 lo chunks; f32: 8 float4 chunks
};

template <int WK, bool XF32>
__device__ __forceinline__ void load_stage(const TilePtrs<WK, XF32> &p, ptrdiff_t lo_delta, uint32_t s,
                                           StageRegs<WK, XF32> &r) {
    const uint32_t tid = threadIdx.x;
    if constexpr (WK == WT_Q8) {
        const uint32_t so = 1024u * (s >> 3) + 128u * (s & 7u);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t pp = (tid + 256u * i) & 7u;
            r.w[i] = *reinterpret_cast<const uint4 *>(p.w[i] + so + 16u * pp);
        }
        r.d = *reinterpret_cast<const uint2 *>(p.d + 2u * (32u * (s >> 3) + 4u * (s & 7u)));
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t pp = (tid + 256u * i) & 15u;
            r.w[i] = *reinterpret_cast<const uint4 *>(p.w[i] + 2u * (128u * s + 8u * pp));
        }
    }
    if constexpr (XF32) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t c = tid + 256u * i, kk = (c >> 3) & 3u, q = c & 7u;
            r.x[i] = *reinterpret_cast<const uint4 *>(p.x[i] + 4u * (stage_col<WK>(s, kk) + 4u * q));
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t c = tid + 256u * i, kk = (c >> 2) & 3u, q = c & 3u;
            const uint8_t *src = p.x[i] + 2u * (stage_col<WK>(s, kk) + 8u * q);
            r.x[i] = *reinterpret_cast<const uint4 *>(src);
            r.x[4 + i] = *reinterpret_cast<const uint4 *>(src + lo_delta);
        }
    }
}

template <int WK, bool XF32>
__device__ __forceinline__ void store_stage(const StageRegs<WK, XF32> &r, _Float16 *Wl, _Float16 *Xh, _Float16 *Xl,
                                            float *Ds) {
    const uint32_t tid = threadIdx.x;
    if constexpr (WK == WT_Q8) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t c = tid + 256u * i, rho = c >> 3, p = c & 7u;
            _Float16 *dst = Wl + rho * LROW + 4u * p;
            const uint32_t words[4] = {r.w[i].x, r.w[i].y, r.w[i].z, r.w[i].w};
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) *reinterpret_cast<uint2 *>(dst + 32 * kk) = q8x4_to_f16(words[kk]);
        }
        if (tid < (uint32_t)GN) {
            Ds[0 * GN + tid] = h2f((unsigned short)(r.d.x & 0xffffu));
            Ds[1 * GN + tid] = h2f((unsigned short)(r.d.x >> 16));
            Ds[2 * GN + tid] = h2f((unsigned short)(r.d.y & 0xffffu));
            Ds[3 * GN + tid] = h2f((unsigned short)(r.d.y >> 16));
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t c = tid + 256u * i, rho = c >> 4, p = c & 15u;
            lds_st16(Wl + rho * LROW + 8u * p, r.w[i]);
        }
    }
    if constexpr (XF32) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t c = tid + 256u * i, t = c >> 5, kk = (c >> 3) & 3u, q = c & 7u;
            uint2 hi, lo;
            split4(__builtin_bit_cast(float4, r.x[i]), hi, lo);
            *reinterpret_cast<uint2 *>(Xh + t * LROW + 32u * kk + 4u * q) = hi;
            *reinterpret_cast<uint2 *>(Xl + t * LROW + 32u * kk + 4u * q) = lo;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t c = tid + 256u * i, t = c >> 4, kk = (c >> 2) & 3u, q = c & 3u;
            lds_st16(Xh + t * LROW + 32u * kk + 8u * q, r.x[i]);
            lds_st16(Xl + t * LROW + 32u * kk + 8u * q, r.x[4 + i]);
        }
    }
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

template <int WK, bool XF32, int EPI>
__global__ __launch_bounds__(256, 2) void k_gemm(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) _Float16 Wl[GN * LROW];
    __shared__ __attribute__((aligned(16))) _Float16 Xh[GM * LROW];
    __shared__ __attribute__((aligned(16))) _Float16 Xl[GM * LROW];
    __shared__ float Ds[WK == WT_Q8 ? 4 * GN : 1];

    // XCD-major tile order: workgroup b runs on XCD b % 8.
    const uint32_t b = blockIdx.x;
    const uint32_t id = (b & 7u) * (gridDim.x >> 3) + (b >> 3);
    const uint32_t per_split = a.ntn * a.ntm;
    if (id >= per_split * a.ksplit) return;
    const uint32_t ks = id / per_split, rem = id - ks * per_split;
    const uint32_t tn = rem / a.ntm, tm = rem - tn * a.ntm;
    const uint32_t m0 = tm * GM;
    uint32_t seg = 0;
    if constexpr (EPI != GEPI_SWIGLU) {
        while (seg + 1 < a.nseg && tn >= a.seg[seg + 1].tile0) ++seg;
    }
    const uint32_t S = a.K / GK;
    const uint32_t s0 = ks * S / a.ksplit, s1 = (ks + 1) * S / a.ksplit;

    const uint32_t tid = threadIdx.x, lane = tid & 63u, l32 = lane & 31u, hs = lane >> 5;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wv & 1u, wn = wv >> 1;

    const GemmSeg &sg0 = a.seg[seg];
    const GemmSeg &sg1 = a.seg[EPI == GEPI_SWIGLU ? 1u : seg];
    TilePtrs<WK, XF32> tp;
    tile_ptrs<WK, XF32, EPI>(sg0, sg1, a, tn, m0, tp);
    const ptrdiff_t lo_delta = XF32 ? 0 : reinterpret_cast<const uint8_t *>(a.xl) - reinterpret_cast<const uint8_t *>(a.xh);

    acc16 acc0 = {}, acc1 = {};
    StageRegs<WK, XF32> st;
    if (s0 < s1) load_stage<WK, XF32>(tp, lo_delta, s0, st);
    const _Float16 *xa = Xh + (32u * wm + l32) * LROW + 8u * hs;
    const _Float16 *xb = Xl + (32u * wm + l32) * LROW + 8u * hs;
    const _Float16 *wa = Wl + (64u * wn + l32) * LROW + 8u * hs;
    const _Float16 *wb = wa + 32 * LROW;
    for (uint32_t s = s0; s < s1; ++s) {
        __syncthreads();
        store_stage<WK, XF32>(st, Wl, Xh, Xl, Ds);
        __syncthreads();
        if (s + 1 < s1) load_stage<WK, XF32>(tp, lo_delta, s + 1, st);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            if constexpr (WK == WT_Q8) {
                acc16 p0 = {}, p1 = {};
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int off = 32 * kk + 16 * h;
                    const h8 ah = *reinterpret_cast<const h8 *>(xa + off);
                    const h8 al = *reinterpret_cast<const h8 *>(xb + off);
                    const h8 b0 = *reinterpret_cast<const h8 *>(wa + off);
                    const h8 b1 = *reinterpret_cast<const h8 *>(wb + off);
                    p0 = mfma(ah, b0, p0);
                    p1 = mfma(ah, b1, p1);
                    p0 = mfma(al, b0, p0);
                    p1 = mfma(al, b1, p1);
                }
                const float d0 = Ds[kk * GN + 64u * wn + l32];
                const float d1 = Ds[kk * GN + 64u * wn + 32u + l32];
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    acc0[r] = fmaf(d0, p0[r], acc0[r]);
                    acc1[r] = fmaf(d1, p1[r], acc1[r]);
                }
            } else {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int off = 32 * kk + 16 * h;
                    const h8 ah = *reinterpret_cast<const h8 *>(xa + off);
                    const h8 al = *reinterpret_cast<const h8 *>(xb + off);
                    const h8 b0 = *reinterpret_cast<const h8 *>(wa + off);
                    const h8 b1 = *reinterpret_cast<const h8 *>(wb + off);
                    acc0 = mfma(ah, b0, acc0);
                    acc1 = mfma(ah, b1, acc1);
                    acc0 = mfma(al, b0, acc0);
                    acc1 = mfma(al, b1, acc1);
                }
            }
        }
    }

    // Epilogue. Lane (l32, hs) holds weight row rho = 64wn + 32*tile + l32 and
    // tokens m0 + 32wm + 8(r/4) + 4hs + r%4 (r < 16) of each tile.
    const uint32_t tbase = m0 + 32u * wm + 4u * hs;
    if constexpr (EPI == GEPI_SWIGLU) {
        uint32_t mat, row;
        tile_row<EPI>(tn, 0, 64u * wn + l32, mat, row);
        if (row >= sg0.rows) return;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t tok = tbase + 8u * (r >> 2) + (r & 3);
            if (tok >= a.T) continue;
            const float v = silu_mul(acc0[r], acc1[r]);
            if (a.seg[0].out) a.seg[0].out[(size_t)tok * a.seg[0].ldo + row] = v;
            if (a.oh) {
                const size_t o = a.o_tiled ? tiled_plane_index(tok, row, a.ldp) : (size_t)tok * a.ldp + row;
                const _Float16 hv = (_Float16)v;
                a.oh[o] = __builtin_bit_cast(__half, hv);
                a.ol[o] = __builtin_bit_cast(__half, (_Float16)(v - (float)hv));
            }
        }
    } else {
        const GemmSeg &sg = sg0;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            uint32_t mat, row;
            tile_row<EPI>(tn, sg.tile0, 64u * wn + 32u * t + l32, mat, row);
            if (row >= sg.rows) continue;
            float bias = 0.f;
            if ((EPI == GEPI_STORE || EPI == GEPI_RESIDUAL) && sg.bias && ks == 0)
                bias = sg.bias_dtype == 0 ? static_cast<const float *>(sg.bias)[row]
                                          : h2f(static_cast<const unsigned short *>(sg.bias)[row]);
            // Take the bias now: used first inside the branchy loop below, its
            // wait would drain every store issued before it.
            asm volatile("" : "+v"(bias));
            const acc16 &acc = t == 0 ? acc0 : acc1;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const uint32_t tok = tbase + 8u * (r >> 2) + (r & 3);
                if (tok >= a.T) continue;
                float *dst = sg.out + (size_t)tok * sg.ldo + row;
                if constexpr (EPI == GEPI_STORE) {
                    const float v = (acc[r] + bias) * a.alpha;
                    if (a.ksplit > 1)
                        unsafeAtomicAdd(dst, v);
                    else
                        *dst = v;
                } else {  // GEPI_RESIDUAL: hidden += scale * (W . x), an atomic add (no load to wait for;
                          // with one contributor it is exactly h + v)
                    unsafeAtomicAdd(dst, (sg.bias ? acc[r] + bias : acc[r]) * a.scale);
                }
            }
        }
    }
}

// ------------------------------------------------------------------------
// Per-token (residual +) rmsnorm: seq_rmsnorm.comp:9 / seq_residual_rmsnorm.comp:10.
// One workgroup per token. If branch != nullptr, h += scale * branch first (and
// h is written back). y = h * (1/sqrt(mean(h^2) + eps)) * w is written as f32
// (y, nullable) and/or as hi/lo f16 planes (yh/yl, nullable). Optionally zeroes
// `zero_n` floats of row t of up to four buffers, and the branch rows after they
// are read (split-K accumulators of the next GEMMs).
__global__ __launch_bounds__(256) void k_seq_rmsnorm(SeqNormArgs a) {
    __shared__ float red[4];
    const uint32_t t = blockIdx.x;
    float *h = a.h + (size_t)t * a.ldh;
    const float *br = a.branch ? a.branch + (size_t)t * a.ldb : nullptr;
    float s = 0.f;
    for (uint32_t i = threadIdx.x; i < a.n; i += 256u) {
        float v = h[i];
        if (br) {
            float add = br[i];
            for (uint32_t b = 1; b < a.nbranch; ++b) add += br[(size_t)b * a.branch_stride + i];
            v = v + add * a.scale;
            h[i] = v;
            if (a.clear_branch)
                for (uint32_t b = 0; b < a.nbranch; ++b) const_cast<float *>(br)[(size_t)b * a.branch_stride + i] = 0.f;
        }
        s += v * v;
    }
    if (!a.w) return;   // residual update only
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, 64);
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    s = red[0] + red[1] + red[2] + red[3];
    const float inv_rms = 1.0f / sqrtf(s / (float)a.n + a.eps);
    for (uint32_t i = threadIdx.x; i < a.n; i += 256u) {
        const float v = h[i] * inv_rms * a.w[i];
        if (a.y) a.y[(size_t)t * a.ldy + i] = v;
        if (a.yh) {
            const size_t o = a.tiled == 1   ? tiled_plane_index(t, i, a.n)
                             : a.tiled == 2 ? frag16_index(t, i, a.n)
                                            : (size_t)t * a.ldp + i;
            const _Float16 hv = (_Float16)v;
            a.yh[o] = __builtin_bit_cast(__half, hv);
            a.yl[o] = __builtin_bit_cast(__half, (_Float16)(v - (float)hv));
        }
    }
    for (int z = 0; z < 4; ++z)
        if (a.zero[z])
            for (uint32_t i = threadIdx.x; i < a.zero_n[z]; i += 256u) a.zero[z][(size_t)t * a.zero_n[z] + i] = 0.f;
}

// Lane exchanges of the sequence rmsnorm and the fused softmax (gfx9 DPP
// controls); lanes of rows outside ROW_MASK get `old`.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float seq_dpp(float v, float old = 0.f) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                                 CTRL, ROW_MASK, 0xf, false));
}
// Max and sum over each 16-lane row: quad swaps, then the half-row and row mirrors.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, seq_dpp<0xb1>(v));    // quad_perm [1,0,3,2]
    v = fmaxf(v, seq_dpp<0x4e>(v));    // quad_perm [2,3,0,1]
    v = fmaxf(v, seq_dpp<0x141>(v));   // row_half_mirror
    return fmaxf(v, seq_dpp<0x140>(v));   // row_mirror
}
__device__ __forceinline__ float row16_sum(float v) {
    v += seq_dpp<0xb1>(v);
    v += seq_dpp<0x4e>(v);
    v += seq_dpp<0x141>(v);
    return v + seq_dpp<0x140>(v);
}
// Over the whole wave: the 16-lane rows' results, then row_bcast15/31 fold the
// four rows into lane 63, read back as a wave-uniform value.
__device__ __forceinline__ float wave64_max(float v) {
    v = row16_max(v);
    v = fmaxf(v, seq_dpp<0x142, 0xa>(v, v));   // row_bcast:15 into rows 1 and 3
    v = fmaxf(v, seq_dpp<0x143, 0xc>(v, v));   // row_bcast:31 into rows 2 and 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float wave64_sum(float v) {
    v = row16_sum(v);
    v += seq_dpp<0x142, 0xa>(v);
    v += seq_dpp<0x143, 0xc>(v);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// k_seq_rmsnorm for n = 1024 * NV: thread t holds the float4 chunks t + 256j of
// the token's row in registers across the reduction; the branch rows of a chunk
// are all requested before they are summed. Same arithmetic, summation order
// h + scale * (b0 + b1 + ...) as k_seq_rmsnorm.
template <int NV, int MAXB>   // MAXB: branches the registers hold (>= a.nbranch)
__global__ __launch_bounds__(256) void k_seq_rmsnorm4(SeqNormArgs a) {
    VX_WAVE_STAMP(a.stamps);
    __shared__ float red[4];
    const uint32_t t = blockIdx.x, tid = threadIdx.x;
    float *h = a.h + (size_t)t * a.ldh;
    // Four consecutive columns from a multiple of 4 stay contiguous in frag32 order.
    auto hat = [&](uint32_t c) { return a.h_frag ? a.h + frag32_index(t, c, a.n) : h + c; };
    float4 v[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) v[j] = *reinterpret_cast<const float4 *>(hat(4u * (tid + 256u * j)));
    if (a.branch) {
        const float *br = a.branch + (size_t)t * a.ldb;
        float4 bv[NV][MAXB];
#pragma unroll
        for (int b = 0; b < MAXB; ++b)
#pragma unroll
            for (int j = 0; j < NV; ++j)
                bv[j][b] = (uint32_t)b < a.nbranch
                               ? *reinterpret_cast<const float4 *>(br + (size_t)b * a.branch_stride + 4u * (tid + 256u * j))
                               : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            float4 add = bv[j][0];
#pragma unroll
            for (int b = 1; b < MAXB; ++b)
                if ((uint32_t)b < a.nbranch) {
                    add.x += bv[j][b].x;
                    add.y += bv[j][b].y;
                    add.z += bv[j][b].z;
                    add.w += bv[j][b].w;
                }
            v[j] = make_float4(v[j].x + add.x * a.scale, v[j].y + add.y * a.scale, v[j].z + add.z * a.scale,
                               v[j].w + add.w * a.scale);
            *reinterpret_cast<float4 *>(hat(4u * (tid + 256u * j))) = v[j];
        }
        if (a.clear_branch)
            for (uint32_t b = 0; b < a.nbranch; ++b)
#pragma unroll
                for (int j = 0; j < NV; ++j)
                    *reinterpret_cast<float4 *>(const_cast<float *>(br) + (size_t)b * a.branch_stride +
                                                4u * (tid + 256u * j)) = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (a.hf) {
#pragma unroll
        for (int j = 0; j < NV; ++j) *reinterpret_cast<float4 *>(a.hf + frag32_index(t, 4u * (tid + 256u * j), a.n)) = v[j];
    }
    if (!a.w) return;   // residual update only
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NV; ++j) ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
    ss = wave64_sum(ss);   // DPP, no LDS round trips (-0.03 ms over the 8-layer 2 x 37-token solve)
    if ((tid & 63u) == 0) red[tid >> 6] = ss;
    __syncthreads();
    ss = red[0] + red[1] + red[2] + red[3];
    const float inv_rms = 1.0f / sqrtf(ss / (float)a.n + a.eps);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t c = 4u * (tid + 256u * j);
        const float4 w = *reinterpret_cast<const float4 *>(a.w + c);
        const float o[4] = {v[j].x * inv_rms * w.x, v[j].y * inv_rms * w.y, v[j].z * inv_rms * w.z, v[j].w * inv_rms * w.w};
        if (a.y) *reinterpret_cast<float4 *>(a.y + (size_t)t * a.ldy + c) = make_float4(o[0], o[1], o[2], o[3]);
        if (a.yh) {
            // Four columns from a multiple of 4 stay inside one 8-column chunk.
            const size_t po = a.tiled == 1   ? tiled_plane_index(t, c, a.n)
                              : a.tiled == 2 ? frag16_index(t, c, a.n)
                                             : (size_t)t * a.ldp + c;
            uint2 hi, lo;
            split4(make_float4(o[0], o[1], o[2], o[3]), hi, lo);
            *reinterpret_cast<uint2 *>(a.yh + po) = hi;
            *reinterpret_cast<uint2 *>(a.yl + po) = lo;
        }
    }
    for (int z = 0; z < 4; ++z)
        if (a.zero[z])
            for (uint32_t i = tid; i < a.zero_n[z]; i += 256u) a.zero[z][(size_t)t * a.zero_n[z] + i] = 0.f;
}

// Per-token RoPE at position base + t (rope.comp:22-51 / seq_rope.comp:8 with a
// position base), then the f16 KV store of token t at that position
// (store_kv.comp:16-24), and q as hi/lo planes for the attention kernel.
// The angle is computed exactly as the decode step's per-step table.
__global__ __launch_bounds__(256) void k_seq_rope_store(SeqRopeArgs a) {
    __shared__ float2 cs[64];
    const uint32_t t = blockIdx.x;
    const uint32_t pos = a.pos_base + (a.pos_period ? t % a.pos_period : t);
    const uint32_t half_dim = a.head_dim / 2u;
    if (threadIdx.x < half_dim && !a.no_rope) {
        const uint32_t i = threadIdx.x;
        const float exponent = (float)(i * 2u) / (float)a.head_dim;
        const float inv_freq = 1.0f / powf(a.theta, exponent);
        const float angle = (float)pos * inv_freq / a.factors[i];
        cs[i] = make_float2(cosf(angle) * a.scaling, sinf(angle) * a.scaling);
    }
    __syncthreads();
    float *q = a.q + (size_t)t * a.ldq;
    float *k = a.k + (size_t)t * a.ldk;
    const uint32_t q_pairs = a.q_heads * half_dim, k_pairs = a.kv_heads * half_dim;
    const uint32_t ns = a.nsplit ? a.nsplit : 1u;
    for (uint32_t p = threadIdx.x; p < q_pairs + k_pairs; p += 256u) {
        const bool isq = p < q_pairs;
        const uint32_t pp = isq ? p : p - q_pairs;
        const uint32_t head = pp / half_dim, i = pp - head * half_dim;
        float *buf = isq ? q : k;
        const uint32_t base = head * a.head_dim;
        // split-K partials (at most kSeqRopeMaxSplit), all loads issued together,
        // summed in split order
        float p0[kSeqRopeMaxSplit], p1[kSeqRopeMaxSplit];
#pragma unroll
        for (uint32_t sp = 0; sp < kSeqRopeMaxSplit; ++sp) {
            const size_t o = (size_t)(sp < ns ? sp : 0u) * a.split_stride + base + i;
            p0[sp] = buf[o];
            p1[sp] = buf[o + half_dim];
        }
        float x0 = p0[0], x1 = p1[0];
#pragma unroll
        for (uint32_t sp = 1; sp < kSeqRopeMaxSplit; ++sp) {
            x0 += sp < ns ? p0[sp] : 0.f;
            x1 += sp < ns ? p1[sp] : 0.f;
        }
        float y0 = x0, y1 = x1;
        if (!a.no_rope) {
            const float c = cs[i].x, s = cs[i].y;
            y0 = x0 * c - x1 * s;
            y1 = x1 * c + x0 * s;
        }
        if (isq) {
            if (a.q_inplace) {
                buf[base + i] = y0;
                buf[base + i + half_dim] = y1;
            }
            if (a.qh) {
                const size_t o = (size_t)t * a.ldqp + base + i;
                const _Float16 h0 = (_Float16)y0, h1 = (_Float16)y1;
                a.qh[o] = __builtin_bit_cast(__half, h0);
                a.ql[o] = __builtin_bit_cast(__half, (_Float16)(y0 - (float)h0));
                a.qh[o + half_dim] = __builtin_bit_cast(__half, h1);
                a.ql[o + half_dim] = __builtin_bit_cast(__half, (_Float16)(y1 - (float)h1));
            }
        } else {
            buf[base + i] = y0;
            buf[base + i + half_dim] = y1;
        }
    }
    if (!a.kc) return;
    __syncthreads();  // roped k visible to the store below
    if (pos >= a.context) return;
    const float *v = a.v + (size_t)t * a.ldk;
    const uint32_t kv_dim = a.kv_heads * a.head_dim;
    const size_t dst = ((size_t)a.layer * a.context + pos) * kv_dim;
    for (uint32_t i = threadIdx.x; i < kv_dim; i += 256u) {
        float pv[kSeqRopeMaxSplit];
#pragma unroll
        for (uint32_t sp = 0; sp < kSeqRopeMaxSplit; ++sp) pv[sp] = v[(size_t)(sp < ns ? sp : 0u) * a.split_stride + i];
        float vv = pv[0];
#pragma unroll
        for (uint32_t sp = 1; sp < kSeqRopeMaxSplit; ++sp) vv += sp < ns ? pv[sp] : 0.f;
        a.kc[dst + i] = __float2half_rn(k[i]);
        a.vc[dst + i] = __float2half_rn(vv);
    }
}

// ------------------------------------------------------------------------
// Causal attention of a token block over the f16 KV cache on MFMA
// (attn_scores.comp + softmax.comp + attn_values.comp for every query token
// t at position pos_base + t over keys 0..pos_base + t, as the decode step would
// compute them one token at a time).
//
// Workgroup: one KV head g and TPB = 32 / QPK consecutive query tokens, i.e. 32
// query rows (token x the QPK query heads of g). Four waves split the key blocks
// (32 keys each) round-robin, each keeping an online-softmax state, and merge at
// the end through LDS.
//   S^T (keys x rows) = K . Q^T   A = K block from LDS, B = q (hi and lo planes)
//   O^T (dims x rows) += V^T . P^T A = V^T from LDS, B = p (hi/lo) from registers
// Lane (l32, hs) holds query row l32 in both, so the softmax of a row is one
// in-lane reduction and one exchange with lane ^ 32, and p feeds the second
// product from the lane's own registers: its register r (key 8(r/4)+4hs+r%4)
// is used in k-slot 8hs + r%8 of k-step r/8, and the V^T operand supplies the
// same keys for those slots.
// K and V are both staged row per key with 16-byte stores (rows of HD + 8
// halves), and the V^T operand is gathered from the V rows with 2-byte reads
// (lane l32 reads dim 32dt + l32 of eight keys): the 32 lanes of a half-wave
// read 64 contiguous bytes of one key row, and the two half-waves' rows (4 keys
// apart, 4 * (HD + 8) / 2 dwords) start 16 banks apart, so no read conflicts;
// transposing V in LDS instead took 2-byte stores that collided 16 ways.
typedef short h4s __attribute__((ext_vector_type(4)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
// ds_read_b64_tr_b16 (gfx950): eight bytes per lane from LDS, transposed within
// each group of 16 lanes as described at its use.
__device__ __forceinline__ h4s lds_read_tr16(const _Float16 *p) {
    typedef __attribute__((address_space(3))) h4s lds_h4s;
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_h4s *)(__attribute__((address_space(3))) _Float16 *)p);
}

template <int HD, int QPK>
__global__ __launch_bounds__(256) void k_prefill_attn(PrefillAttnArgs a) {
    constexpr int TPB = 32 / QPK;
    constexpr int KROW = HD + 8;   // K and V block row (f16)
    constexpr int ND = HD / 32;    // output tiles of 32 dims
    constexpr int KS = HD / 16;    // k-steps over the head dim
    constexpr int WAVE_LDS = 2 * 32 * KROW;   // f16 per wave
    __shared__ __attribute__((aligned(16))) _Float16 lds[4 * WAVE_LDS];
    static_assert(4 * WAVE_LDS * 2 >= 4 * (ND * 16 * 64 * 4 + 2 * 32 * 4), "merge area");

    const uint32_t tid = threadIdx.x, lane = tid & 63u, l32 = lane & 31u, hs = lane >> 5;
    const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t g = blockIdx.y;
    const uint32_t t0 = blockIdx.x * TPB;
    const uint32_t tq = t0 + l32 / QPK;
    const uint32_t head = g * QPK + l32 % QPK;
    const bool qvalid = tq < a.T;
    const uint32_t qpos = a.pos_base + (qvalid ? tq : a.T - 1u);
    const uint32_t tlast = min(t0 + (uint32_t)TPB, a.T) - 1u;
    const uint32_t kmax = a.pos_base + tlast;   // last key any row of the block needs
    const uint32_t nblocks = kmax / 32u + 1u;
    const float scale2 = 1.4426950408889634f / sqrtf((float)HD);   // log2(e) / sqrt(d)
    constexpr float kLazyMax = 8.0f;
    const uint32_t kv_dim = a.kv_heads * HD;

    h8 qh[KS], ql[KS];
    {
        const size_t qo = (size_t)(qvalid ? tq : 0u) * a.ldq + head * HD + 8u * hs;
#pragma unroll
        for (int ds = 0; ds < KS; ++ds) {
            qh[ds] = qvalid ? *reinterpret_cast<const h8 *>(a.qh + qo + 16 * ds) : h8{};
            ql[ds] = qvalid ? *reinterpret_cast<const h8 *>(a.ql + qo + 16 * ds) : h8{};
        }
    }
    _Float16 *Ks = lds + w * WAVE_LDS;
    _Float16 *Vs = Ks + 32 * KROW;

    float m = -INFINITY, l = 0.f;
    acc16 o[ND];
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) o[dt] = acc16{};

    // K and V rows of a key block, in registers one block ahead of the block
    // being multiplied (the wave's next block is fetched while it computes).
    constexpr int CH = 32 * HD / 8 / 64;   // 16-byte chunks per lane per block
    uint4 kreg[CH], vreg[CH];
    auto fetch = [&](uint32_t kb) {
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const uint32_t c = lane + 64u * i, key = c / (HD / 8), p = c % (HD / 8);
            const uint32_t kp = kb * 32u + key;
            kreg[i] = vreg[i] = make_uint4(0, 0, 0, 0);
            if (kb < nblocks && kp <= kmax && kp < a.context) {
                const size_t src = ((size_t)a.layer * a.context + kp) * kv_dim + g * HD + 8u * p;
                kreg[i] = *reinterpret_cast<const uint4 *>(a.kc + src);
                vreg[i] = *reinterpret_cast<const uint4 *>(a.vc + src);
            }
        }
    };
    fetch(w);
    for (uint32_t kb = w; kb < nblocks; kb += 4u) {
        const uint32_t key0 = kb * 32u;
        // Stage K and V (row per key) of keys key0..key0+31, then fetch the next block.
#pragma unroll
        for (int i = 0; i < CH; ++i) {
            const uint32_t c = lane + 64u * i, key = c / (HD / 8), p = c % (HD / 8);
            *reinterpret_cast<uint4 *>(Ks + key * KROW + 8u * p) = kreg[i];
            *reinterpret_cast<uint4 *>(Vs + key * KROW + 8u * p) = vreg[i];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        fetch(kb + 4u);

        acc16 sc = {};
#pragma unroll
        for (int ds = 0; ds < KS; ++ds) {
            const h8 kf = *reinterpret_cast<const h8 *>(Ks + l32 * KROW + 16 * ds + 8 * hs);
            sc = mfma(kf, qh[ds], sc);
            sc = mfma(kf, ql[ds], sc);
        }
        // Scores in log2 units (scale * log2(e) folded in), so p = 2^(s - m).
        float mloc = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t key = key0 + 8u * (r >> 2) + 4u * hs + (r & 3);
            sc[r] = key <= qpos ? sc[r] * scale2 : -INFINITY;
            mloc = fmaxf(mloc, sc[r]);
        }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        // The row's reference max moves only when the block max exceeds it by more
        // than kLazyMax (p then stays below 2^kLazyMax, well inside f16), so the
        // output accumulators are rescaled only on the blocks where some row's
        // reference moved.
        const float mnew = mloc > m + kLazyMax ? mloc : m;
        float lsum = 0.f;
        float p[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            p[r] = sc[r] == -INFINITY ? 0.f : exp2f(sc[r] - mnew);
            lsum += p[r];
        }
        lsum += __shfl_xor(lsum, 32, 64);
        const float alpha = m == -INFINITY ? 0.f : exp2f(m - mnew);
        l = l * alpha + lsum;
        const bool moved = mnew != m;
        m = mnew;
        if (__any(moved)) {
#pragma unroll
            for (int dt = 0; dt < ND; ++dt)
#pragma unroll
                for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
        }
        h8 ph[2], pl[2];
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float v = p[8 * kh + i];
                const _Float16 hv = (_Float16)v;
                ph[kh][i] = hv;
                pl[kh][i] = (_Float16)(v - (float)hv);
            }
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
            h8 vf[ND];
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) {
                // Slot i of k-step kh is key 16kh + 8(i/4) + 4hs + i%4, dimension
                // 32dt + l32. ds_read_b64_tr_b16 hands lane 16g + 4a + b element j =
                // column b of the 8-byte row read by lane 16g + a + 4j of its group,
                // so the lane of the group with (a, j) = (lane % 4, lane / 4 % 4)
                // reads dims 4a..4a+3 of key 4hs + j (the group's 16 dims start
                // at 32dt + 16(g % 2), hs = g / 2) and every lane receives keys
                // +0..3 of its own dimension: slots 0..3, then 4..7 from 8 keys on.
                const _Float16 *vr = Vs + (16u * kh + 4u * hs + ((lane >> 2) & 3u)) * KROW + 32u * dt +
                                     16u * ((lane >> 4) & 1u) + 4u * (lane & 3u);
                const h4s lo4 = lds_read_tr16(vr), hi4 = lds_read_tr16(vr + 8 * KROW);
                vf[dt] = __builtin_shufflevector(__builtin_bit_cast(h4, lo4), __builtin_bit_cast(h4, hi4), 0, 1, 2, 3,
                                                 4, 5, 6, 7);
            }
            // The ND accumulators in turn, so no MFMA waits on the one before it.
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) o[dt] = mfma(vf[dt], ph[kh], o[dt]);
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) o[dt] = mfma(vf[dt], pl[kh], o[dt]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // Merge the four waves' states: wave w finalises output dims 32w..32w+31.
    __syncthreads();
    float *mo = reinterpret_cast<float *>(lds);            // [4 waves][ND][16][64]
    float *ms = mo + 4 * ND * 16 * 64;                      // [4][32] max
    float *ls = ms + 4 * 32;                                // [4][32] sum
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mo[((w * ND + dt) * 16 + r) * 64 + lane] = o[dt][r];
    if (hs == 0) {
        ms[w * 32 + l32] = m;
        ls[w * 32 + l32] = l;
    }
    __syncthreads();
    for (uint32_t dt = w; dt < (uint32_t)ND; dt += 4u) {
        float mw[4], M = -INFINITY;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            mw[v] = ms[v * 32 + l32];
            M = fmaxf(M, mw[v]);
        }
        float wt[4], L = 0.f;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            wt[v] = mw[v] == -INFINITY ? 0.f : exp2f(mw[v] - M);
            L += wt[v] * ls[v * 32 + l32];
        }
        const float inv = 1.0f / L;
        if (!qvalid) continue;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
            float outv[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int r = 4 * r4 + j;
                float acc = 0.f;
#pragma unroll
                for (int v = 0; v < 4; ++v) acc += wt[v] * mo[((v * ND + dt) * 16 + r) * 64 + lane];
                outv[j] = acc * inv;
            }
            const uint32_t d = 32u * dt + 8u * r4 + 4u * hs;
            const size_t oo = (size_t)tq * a.ldo + head * HD + d;
            if (a.out) *reinterpret_cast<float4 *>(a.out + oo) = make_float4(outv[0], outv[1], outv[2], outv[3]);
            if (a.oh) {
                uint2 hi, lo;
                split4(make_float4(outv[0], outv[1], outv[2], outv[3]), hi, lo);
                // Four columns from a multiple of 4 stay inside one 8-column half.
                const size_t po = a.tiled ? tiled_plane_index(tq, head * HD + d, a.ldo) : oo;
                *reinterpret_cast<uint2 *>(a.oh + po) = hi;
                *reinterpret_cast<uint2 *>(a.ol + po) = lo;
            }
        }
    }
}

// Embedding rows of T tokens (embedding.comp:28-48 per token): rows of the raw
// GGUF table (F16 or Q8_0 blocks) widened to f32 and scaled, bit-exact. Ids
// >= vocab give NaN rows; the host rejects them before launching.
__global__ __launch_bounds__(256) void k_seq_embedding(const uint8_t *raw, uint32_t off, uint32_t dtype,
                                                      uint32_t cols, const uint32_t *tokens, uint32_t vocab,
                                                      float alpha, float *out, uint32_t ldo) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x, t = blockIdx.y;
    if (i >= cols) return;
    const uint32_t token = tokens[t];
    float *dst = out + (size_t)t * ldo + i;
    if (token >= vocab) {
        *dst = __int_as_float(0x7fc00000);
        return;
    }
    float w;
    if (dtype == VX_DTYPE_F16) {
        w = h2f(*reinterpret_cast<const unsigned short *>(raw + off + ((size_t)token * cols + i) * 2u));
    } else {
        const size_t block = (size_t)token * (cols / 32u) + i / 32u;
        const uint8_t *b = raw + off + block * 34u;
        w = h2f((unsigned short)(b[0] | (b[1] << 8))) * (float)(int)(int8_t)b[2 + (i & 31u)];
    }
    *dst = w * alpha;
}

// ------------------------------------------------------------------------
// Reference-granular token-batched kernels for shapes the MFMA GEMM does not
// take (F32 weights, Q8_0 rows not a multiple of 1024 wide, unaligned strides)
// and the LocEnc/LocDiT dense attention (non-causal, f32).

// Weight element (row r, column c) of a dtype 0/1/8 matrix in the raw GGUF
// region (seq_linear_bias.comp:16-21).
__device__ __forceinline__ float weight_at(const uint8_t *raw, uint32_t off, uint32_t dtype, uint32_t cols,
                                           uint32_t r, uint32_t c) {
    if (dtype == VX_DTYPE_F32) return reinterpret_cast<const float *>(raw + off)[(size_t)r * cols + c];
    if (dtype == VX_DTYPE_F16) return h2f(reinterpret_cast<const unsigned short *>(raw + off)[(size_t)r * cols + c]);
    const uint8_t *b = raw + off + ((size_t)r * (cols / 32u) + c / 32u) * 34u;
    return h2f((unsigned short)(b[0] | (b[1] << 8))) * (float)(int)(int8_t)b[2u + (c & 31u)];
}

// One wave per (row, token): seq_linear_bias.comp:22-30 (mode 0) and
// seq_swiglu.comp:9 (mode 1, gate at w_off, up at w2_off).
__global__ __launch_bounds__(256) void k_seq_linear_generic(SeqGenericArgs a) {
    const uint32_t idx = blockIdx.x * 4u + (threadIdx.x >> 6), lane = threadIdx.x & 63u;
    if (idx >= a.rows * a.tokens) return;
    const uint32_t row = idx % a.rows, tok = idx / a.rows;
    const float *x = a.x + a.in_base + (size_t)tok * a.in_stride;
    float s = 0.f, s2 = 0.f;
    for (uint32_t c = lane; c < a.cols; c += 64u) {
        const float xv = x[c];
        s += weight_at(a.raw, a.w_off, a.dtype, a.cols, row, c) * xv;
        if (a.swiglu) s2 += weight_at(a.raw, a.w2_off, a.dtype, a.cols, row, c) * xv;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        s += __shfl_xor(s, o, 64);
        s2 += __shfl_xor(s2, o, 64);
    }
    if (lane != 0) return;
    float v;
    if (a.swiglu) {
        v = s / (1.0f + expf(-s)) * s2;
    } else {
        float b = 0.f;
        if (a.bias)
            b = a.bias_dtype == 0u ? static_cast<const float *>(a.bias)[row]
                                   : h2f(static_cast<const unsigned short *>(a.bias)[row]);
        v = (s + b) * a.alpha;
    }
    a.y[a.out_base + (size_t)tok * a.out_stride + row] = v;
}

// seq_silu_mul.comp:6: g = silu(g) * u.
__global__ __launch_bounds__(256) void k_silu_mul(float *g, const float *u, uint32_t n) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const float x = g[i];
    g[i] = x / (1.0f + expf(-x)) * u[i];
}

// dense_attn_scores.comp:8: s[(t*q_heads + h)*score_stride + key] = q_t,h . k_key,kv / sqrt(d),
// for every key < tokens (no mask). Workgroup (query token, head), lane per key.
__global__ __launch_bounds__(64) void k_dense_scores(DenseAttnArgs a) {
    __shared__ float qs[256];
    const uint32_t t = blockIdx.x, h = blockIdx.y, bz = blockIdx.z;
    a.q += (size_t)bz * a.tokens * a.q_stride;
    a.k += (size_t)bz * a.tokens * a.k_stride;
    a.s += (size_t)bz * a.tokens * a.q_heads * a.score_stride;
    const uint32_t kv = h / (a.q_heads / a.kv_heads);
    const float *q = a.q + (size_t)t * a.q_stride + h * a.head_dim;
    for (uint32_t i = threadIdx.x; i < a.head_dim; i += 64u) qs[i] = q[i];
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)a.head_dim);
    for (uint32_t key = threadIdx.x; key < a.tokens; key += 64u) {
        const float *k = a.k + (size_t)key * a.k_stride + kv * a.head_dim;
        float s = 0.f;
        for (uint32_t i = 0; i < a.head_dim; ++i) s += qs[i] * k[i];
        a.s[((size_t)t * a.q_heads + h) * a.score_stride + key] = s * scale;
    }
}

// dense_softmax.comp:5: max-subtracted softmax of each (token, head) row.
__global__ __launch_bounds__(64) void k_dense_softmax(float *s, uint32_t tokens, uint32_t q_heads,
                                                      uint32_t score_stride) {
    const uint32_t h = blockIdx.x, t = blockIdx.y + blockIdx.z * tokens;
    float *row = s + ((size_t)t * q_heads + h) * score_stride;
    float m = -FLT_MAX;
    for (uint32_t i = threadIdx.x; i < tokens; i += 64u) m = fmaxf(m, row[i]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    float z = 0.f;
    for (uint32_t i = threadIdx.x; i < tokens; i += 64u) {
        const float e = expf(row[i] - m);
        row[i] = e;
        z += e;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) z += __shfl_xor(z, o, 64);
    for (uint32_t i = threadIdx.x; i < tokens; i += 64u) row[i] = row[i] / z;
}

// dense_attn_values.comp:7: o[t*out_stride + h*d + j] = sum_key s[...key] * v[key*v_stride + kv*d + j].
__global__ __launch_bounds__(256) void k_dense_values(DenseAttnArgs a) {
    const uint32_t j = threadIdx.x, h = blockIdx.x, t = blockIdx.y, bz = blockIdx.z;
    if (j >= a.head_dim) return;
    a.v += (size_t)bz * a.tokens * a.v_stride;
    a.out += (size_t)bz * a.tokens * a.out_stride;
    a.s += (size_t)bz * a.tokens * a.q_heads * a.score_stride;
    const uint32_t kv = h / (a.q_heads / a.kv_heads);
    const float *row = a.s + ((size_t)t * a.q_heads + h) * a.score_stride;
    float z = 0.f;
    for (uint32_t key = 0; key < a.tokens; ++key) z += row[key] * a.v[(size_t)key * a.v_stride + kv * a.head_dim + j];
    a.out[(size_t)t * a.out_stride + h * a.head_dim + j] = z;
}

// dense_attn_scores.comp -> dense_softmax.comp -> dense_attn_values.comp for
// kDenseFusedRows query tokens of one head of one sequence in a workgroup: their q
// rows, the head's k and v rows (each padded by one float) and the rows x tokens
// probabilities live in LDS. Scores are thread per (row, key), the softmax a wave
// per row (lane per key, its max and sum reduced by DPP), the values thread per
// (row, dim); each dot product and value sum runs in the order of the three-kernel
// path (with the O projection and fewer outputs than threads, lane pairs take the
// even and odd keys of a value sum). Sequences of at most 16 tokens (the MAXT = 16 instantiation) take scores
// and softmax in one pass instead: a half-wave per query row, its two 16-lane rows
// each half of the head's dims (four partial sums per lane), the halves met by a
// row swap and the row max and sum by DPP, with no LDS round trip and one barrier
// fewer.
constexpr uint32_t kDenseFusedRows = 8;
// The attention + O-projection variant: eight query tokens (rows 0-7 of an MFMA
// A fragment, the rest zero) per workgroup, and at most kOprojBlocks weight
// blocks per wave.
constexpr uint32_t kOprojRows = 8;
constexpr uint32_t kOprojBlocks = 16;

typedef _Float16 oh8 __attribute__((ext_vector_type(8)));
typedef float of4 __attribute__((ext_vector_type(4)));

// Rows 0 + 1 and 2 + 3 of the wave, lane by lane: v_permlane16_swap leaves the
// lower row's value in element 0 and the upper row's in element 1 in every lane
// of both rows, so both rows of a pair hold the same sum.
__device__ __forceinline__ float row_pair_sum(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
}

// NSLAB > 1 (float4 staging only): q, k and v are the sums of NSLAB partial
// slabs a.slab_stride floats apart (a split-K projection's plain-store output).
//
// OPROJ: the workgroup then multiplies its kOprojRows x head_dim output by the
// head's columns of the O projection (a.wo, fragment layout, q_heads * head_dim
// columns), for the hidden rows of its share (blockIdx.z / row groups of
// a.nsplit), and stores the product to the head's partial slab
// (a.oslab + h * a.oslab_stride, [batch * tokens][hidden]): out = sum over the
// heads' slabs, the split-K of the O projection along its heads. The output
// enters as hi/lo f16 planes against exact f16 weights, two
// v_mfma_f32_16x16x32_f16 per 32 columns, the arithmetic of the short-batch GEMM.
// The weight blocks are requested before the attention starts.
//
// RES (with OPROJ): the residual-stream form. q, k and v are products of the
// un-normalised rows, and the staging multiplies each row by its 1/rms (from the
// K slabs' sums of squares in a.ssq); the projection is added to a.hres (the
// residual stream, frag32_index order) with atomic adds instead of head slabs.
// MAXT: the most tokens a sequence may have, which sizes the staging's register
// arrays (16: sequences of at most 16 tokens, a quarter of the loads).
template <int HD, int NSLAB = 1, bool OPROJ = false, bool RES = false,
          uint32_t MAXT = kDenseFusedMaxTokens>   // HD: head_dim when known at compile time, 0: a.head_dim
__global__ __launch_bounds__(256) void k_dense_attn_fused(DenseAttnArgs a) {
    VX_WAVE_STAMP(a.stamps);
    extern __shared__ __align__(16) float sm[];
    constexpr uint32_t ROWS = OPROJ ? kOprojRows : kDenseFusedRows;
    // Rows of a compile-time head_dim are padded to a multiple of four floats
    // (float4 LDS access, a four-bank shift per row), others by one float.
    const uint32_t S = a.tokens, D = HD ? (uint32_t)HD : a.head_dim, DP = HD ? (uint32_t)HD + 4u : D + 1u;
    const uint32_t ngroups = (S + ROWS - 1u) / ROWS;
    const uint32_t h = blockIdx.x, bz = blockIdx.y, rg = blockIdx.z % ngroups, t0 = rg * ROWS;
    const uint32_t R = min(ROWS, S - t0);
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t kv = h / (a.q_heads / a.kv_heads);
    const float *q = a.q + ((size_t)bz * S + t0) * a.q_stride + (size_t)h * D;
    const float *k = a.k + (size_t)bz * S * a.k_stride + (size_t)kv * D;
    const float *v = a.v + (size_t)bz * S * a.v_stride + (size_t)kv * D;
    const size_t ob = ((size_t)bz * S + t0) * a.out_stride + (size_t)h * D;
    float *ks = sm, *vs = ks + S * DP, *qs = vs + S * DP, *ps = qs + ROWS * DP;

    // O projection: 16-row groups [g0, g1) of the hidden rows, wave w taking
    // g0 + w, g0 + w + 4, ...; every block load is unconditional (clamped). The
    // loads are issued after the attention's own (vector loads complete in
    // order, so a wait for the staged rows would otherwise wait for them too).
    constexpr uint32_t KB = OPROJ ? (uint32_t)HD / 32u : 1u;     // 32-column blocks of the head
    constexpr uint32_t GPW = OPROJ ? kOprojBlocks / KB : 1u;     // groups per wave
    uint4 wb[GPW][KB];
    uint32_t g0 = 0, g1 = 0;
    auto fetch_wo = [&]() {
        if constexpr (OPROJ) {
            const uint32_t ng = a.hidden >> 4, sp = blockIdx.z / ngroups;
            g0 = sp * ng / a.nsplit;
            g1 = (sp + 1u) * ng / a.nsplit;
            const uint32_t kblocks = (a.q_heads * (uint32_t)HD) >> 5;
#pragma unroll
            for (uint32_t i = 0; i < GPW; ++i) {
                const uint32_t g = min(g0 + wave + 4u * i, g1 - 1u);
                const __half *blk = a.wo + (((size_t)g * kblocks + h * KB) << 9) + 8u * lane;
#pragma unroll
                for (uint32_t kb = 0; kb < KB; ++kb)
                    wb[i][kb] = *reinterpret_cast<const uint4 *>(blk + ((size_t)kb << 9));
            }
        }
    };
    bool staged = false;
    if constexpr (HD > 0) {
        if (a.vec && a.rope) {
            // Every global load of the stage is issued before the first LDS store:
            // V rows as float4 chunks, and for K and the query rows the two float4
            // chunks of a rotated pair (d..d+3, d+D/2..d+D/2+3) with their (cos, sin),
            // each slab separately. The loads are unconditional (chunks past the
            // rows reload the last one and are not stored): a load under a branch
            // makes the compiler wait for every load in flight at the branch's end.
            constexpr uint32_t H2 = HD / 2, C4 = H2 / 4, V4 = HD / 4;
            constexpr uint32_t NV = (MAXT * V4 + 255u) / 256u;
            constexpr uint32_t NKQ = ((MAXT + ROWS) * C4 + 255u) / 256u;
            // Slab 0 into vv / x0 / x1, slab 1 (NSLAB == 2) into the *b arrays.
            constexpr uint32_t NVB = NSLAB > 1 ? NV : 1u, NKB = NSLAB > 1 ? NKQ : 1u;
            float4 vv[NV], x0[NKQ], x1[NKQ], c01[NKQ], c23[NKQ], vvb[NVB], x0b[NKB], x1b[NKB];
            // RES: each staged row's sums of squares (one per K slab).
            constexpr uint32_t NSV = RES ? NV : 1u, NSK = RES ? NKQ : 1u;
            float sv[NSV][NSLAB], sk[NSK][NSLAB];
#pragma unroll
            for (uint32_t j = 0; j < NV; ++j) {
                const uint32_t i = min(tid + 256u * j, S * V4 - 1u), t = i / V4, c = i - t * V4;
                const float *src = v + (size_t)t * a.v_stride + 4u * c;
                vv[j] = *reinterpret_cast<const float4 *>(src);
                if constexpr (NSLAB > 1) vvb[j] = *reinterpret_cast<const float4 *>(src + a.slab_stride);
                if constexpr (RES) {
#pragma unroll
                    for (int sl = 0; sl < NSLAB; ++sl) sv[j][sl] = a.ssq[sl * a.ssq_stride + (size_t)bz * S + t];
                }
            }
#pragma unroll
            for (uint32_t j = 0; j < NKQ; ++j) {
                const uint32_t i = min(tid + 256u * j, (S + R) * C4 - 1u), r = i / C4, c = i - r * C4;
                const bool isk = r < S;
                const uint32_t t = isk ? r : r - S, pos = isk ? t : t0 + t;
                const float *row = isk ? k + (size_t)t * a.k_stride : q + (size_t)t * a.q_stride;
                x0[j] = *reinterpret_cast<const float4 *>(row + 4u * c);
                x1[j] = *reinterpret_cast<const float4 *>(row + H2 + 4u * c);
                if constexpr (NSLAB > 1) {
                    x0b[j] = *reinterpret_cast<const float4 *>(row + a.slab_stride + 4u * c);
                    x1b[j] = *reinterpret_cast<const float4 *>(row + a.slab_stride + H2 + 4u * c);
                }
                const float4 *cs = reinterpret_cast<const float4 *>(a.rope + (size_t)pos * H2 + 4u * c);
                c01[j] = cs[0];
                c23[j] = cs[1];
                if constexpr (RES) {
#pragma unroll
                    for (int sl = 0; sl < NSLAB; ++sl) sk[j][sl] = a.ssq[sl * a.ssq_stride + (size_t)bz * S + pos];
                }
            }
            if constexpr (NSLAB > 1) {
#pragma unroll
                for (uint32_t j = 0; j < NV; ++j) vv[j] += vvb[j];
#pragma unroll
                for (uint32_t j = 0; j < NKQ; ++j) {
                    x0[j] += x0b[j];
                    x1[j] += x1b[j];
                }
            }
            if constexpr (RES) {   // rmsnorm.comp:36-38: 1/rms of the row, from its slabs' sums
                auto inv_rms = [&](const float (&p)[NSLAB]) {
                    float sum = p[0];
#pragma unroll
                    for (int sl = 1; sl < NSLAB; ++sl) sum += p[sl];
                    return 1.0f / sqrtf(sum / (float)a.norm_n + a.eps);
                };
#pragma unroll
                for (uint32_t j = 0; j < NV; ++j) {
                    const float f = inv_rms(sv[j]);
                    vv[j] = make_float4(vv[j].x * f, vv[j].y * f, vv[j].z * f, vv[j].w * f);
                }
#pragma unroll
                for (uint32_t j = 0; j < NKQ; ++j) {
                    const float f = inv_rms(sk[j]);
                    x0[j] = make_float4(x0[j].x * f, x0[j].y * f, x0[j].z * f, x0[j].w * f);
                    x1[j] = make_float4(x1[j].x * f, x1[j].y * f, x1[j].z * f, x1[j].w * f);
                }
            }
            if constexpr (OPROJ) {
                // The weight loads after the staged rows' (with one slab the
                // compiler keeps that order by itself, and a scheduling barrier
                // there makes it spill).
                if constexpr (NSLAB > 1) __builtin_amdgcn_sched_barrier(0);
                fetch_wo();
            }
#pragma unroll
            for (uint32_t j = 0; j < NV; ++j) {
                const uint32_t i = tid + 256u * j, t = i / V4, c = i - t * V4;
                if (i < S * V4) *reinterpret_cast<float4 *>(vs + t * DP + 4u * c) = vv[j];
            }
#pragma unroll
            for (uint32_t j = 0; j < NKQ; ++j) {
                const uint32_t i = tid + 256u * j, r = i / C4, c = i - r * C4;
                if (i < (S + R) * C4) {
                    const bool isk = r < S;
                    const uint32_t t = isk ? r : r - S;
                    float *dst = (isk ? ks : qs) + t * DP + 4u * c;
                    const float a0[4] = {x0[j].x, x0[j].y, x0[j].z, x0[j].w};
                    const float a1[4] = {x1[j].x, x1[j].y, x1[j].z, x1[j].w};
                    const float co[4] = {c01[j].x, c01[j].z, c23[j].x, c23[j].z};
                    const float si[4] = {c01[j].y, c01[j].w, c23[j].y, c23[j].w};
                    float lo4[4], hi4[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        lo4[e] = a0[e] * co[e] - a1[e] * si[e];
                        hi4[e] = a1[e] * co[e] + a0[e] * si[e];
                    }
                    *reinterpret_cast<float4 *>(dst) = make_float4(lo4[0], lo4[1], lo4[2], lo4[3]);
                    *reinterpret_cast<float4 *>(dst + H2) = make_float4(hi4[0], hi4[1], hi4[2], hi4[3]);
                }
            }
            staged = true;
        }
    }
    if (!staged) {
        fetch_wo();
        for (uint32_t i = tid; i < S * D; i += 256u) {
            const uint32_t t = i / D, d = i - t * D;
            vs[t * DP + d] = v[(size_t)t * a.v_stride + d];
            if (!a.rope) ks[t * DP + d] = k[(size_t)t * a.k_stride + d];
        }
        if (!a.rope) {
            for (uint32_t i = tid; i < R * D; i += 256u) {
                const uint32_t t = i / D, d = i - t * D;
                qs[t * DP + d] = q[(size_t)t * a.q_stride + d];
            }
        } else {
            // Rotated pairs (d, d + D/2) at the row's position within its sequence.
            const uint32_t half = D >> 1;
            for (uint32_t i = tid; i < (S + R) * half; i += 256u) {
                const uint32_t r = i / half, d = i - r * half;
                const bool isk = r < S;
                const uint32_t t = isk ? r : r - S, pos = isk ? t : t0 + t;
                const float *row = isk ? k + (size_t)t * a.k_stride : q + (size_t)t * a.q_stride;
                float *dst = (isk ? ks : qs) + t * DP;
                const float x0 = row[d], x1 = row[d + half];
                const float2 cs = a.rope[pos * half + d];
                dst[d] = x0 * cs.x - x1 * cs.y;
                dst[d + half] = x1 * cs.x + x0 * cs.y;
            }
        }
    }
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)D);
    if constexpr (HD > 0 && MAXT <= 16u) {
        static_assert(ROWS <= 8u, "a half-wave per query row");
        // Lane (t, part, key): query row t = 2 wave + lane / 32, dims
        // [part HD/2, (part + 1) HD/2) with part = lane / 16 % 2, key = lane % 16.
        // Rows and keys past R and S read the last valid one and are not stored.
        const uint32_t t = 2u * wave + (lane >> 5), part = (lane >> 4) & 1u, key = lane & 15u;
        const float4 *q4 = reinterpret_cast<const float4 *>(qs + min(t, R - 1u) * DP + part * (uint32_t)(HD / 2));
        const float4 *k4 = reinterpret_cast<const float4 *>(ks + min(key, S - 1u) * DP + part * (uint32_t)(HD / 2));
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (uint32_t d4 = 0; d4 < (uint32_t)HD / 8u; ++d4) {
            const float4 x = q4[d4], y = k4[d4];
            float &p = acc[d4 & 3u];
            p += x.x * y.x;
            p += x.y * y.y;
            p += x.z * y.z;
            p += x.w * y.w;
        }
        float sc = row_pair_sum((acc[0] + acc[1]) + (acc[2] + acc[3])) * scale;
        sc = key < S ? sc : -FLT_MAX;
        const float m = row16_max(sc);
        const float ex = key < S ? expf(sc - m) : 0.f;
        const float z = row16_sum(ex);
        if (part == 0u && t < R && key < S) ps[t * S + key] = ex / z;
    } else {
    for (uint32_t e = tid; e < R * S; e += 256u) {
        const uint32_t t = e / S, key = e - t * S;
        float s = 0.f;
        if constexpr (HD > 0) {
            const float4 *q4 = reinterpret_cast<const float4 *>(qs + t * DP);
            const float4 *k4 = reinterpret_cast<const float4 *>(ks + key * DP);
#pragma unroll
            for (uint32_t d4 = 0; d4 < (uint32_t)HD / 4u; ++d4) {
                const float4 x = q4[d4], y = k4[d4];
                s += x.x * y.x;
                s += x.y * y.y;
                s += x.z * y.z;
                s += x.w * y.w;
            }
        } else {
#pragma unroll 16
            for (uint32_t d = 0; d < D; ++d) s += qs[t * DP + d] * ks[key * DP + d];
        }
        ps[e] = s * scale;
    }
    __syncthreads();
    for (uint32_t t = wave; t < R; t += 4u) {
        const float x = lane < S ? ps[t * S + lane] : -FLT_MAX;
        const float m = wave64_max(x);
        const float ex = lane < S ? expf(x - m) : 0.f;
        const float z = wave64_sum(ex);
        if (lane < S) ps[t * S + lane] = ex / z;
    }
    }
    __syncthreads();
    if constexpr (OPROJ) {
        // The output rows into the q rows' LDS (free once the scores are done),
        // rows past R as zeros. With fewer outputs than threads, lane pairs split
        // the keys (even and odd) and meet by a DPP swap.
        constexpr uint32_t D4 = (uint32_t)HD / 4u;
        constexpr uint32_t KS = ROWS * D4 * 2u <= 256u ? 2u : 1u;
        for (uint32_t o = tid; o < ROWS * D4 * KS; o += 256u) {
            const uint32_t item = o / KS, half = o % KS, t = item / D4, d4 = item - t * D4;
            float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
            if (t < R) {
#pragma unroll 4
                for (uint32_t key = half; key < S; key += KS) {
                    const float p = ps[t * S + key];
                    const float4 w = *reinterpret_cast<const float4 *>(vs + key * DP + 4u * d4);
                    z.x += p * w.x;
                    z.y += p * w.y;
                    z.z += p * w.z;
                    z.w += p * w.w;
                }
            }
            if constexpr (KS == 2) {   // quad_perm [1,0,3,2]: the pair's other half
                z = make_float4(z.x + seq_dpp<0xb1>(z.x), z.y + seq_dpp<0xb1>(z.y), z.z + seq_dpp<0xb1>(z.z),
                                z.w + seq_dpp<0xb1>(z.w));
                if (half == 0u) *reinterpret_cast<float4 *>(qs + t * DP + 4u * d4) = z;
            } else {
                *reinterpret_cast<float4 *>(qs + t * DP + 4u * d4) = z;
            }
        }
        __syncthreads();
        // A fragments: lane l = r + 16 c holds columns 8c..8c+7 of block kb for row r.
        oh8 ah[KB], al[KB];
        const uint32_t r = lane & 15u, c8 = 8u * (lane >> 4);
#pragma unroll
        for (uint32_t kb = 0; kb < KB; ++kb) {
            float z8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            if (r < ROWS) {
                const float4 u0 = *reinterpret_cast<const float4 *>(qs + r * DP + 32u * kb + c8);
                const float4 u1 = *reinterpret_cast<const float4 *>(qs + r * DP + 32u * kb + c8 + 4u);
                z8[0] = u0.x; z8[1] = u0.y; z8[2] = u0.z; z8[3] = u0.w;
                z8[4] = u1.x; z8[5] = u1.y; z8[6] = u1.z; z8[7] = u1.w;
            }
#pragma unroll
            for (uint32_t e = 0; e < 8u; ++e) {
                const _Float16 hv = (_Float16)z8[e];
                ah[kb][e] = hv;
                al[kb][e] = (_Float16)(z8[e] - (float)hv);
            }
        }
        float *slab = RES ? nullptr : a.oslab + (size_t)h * a.oslab_stride + ((size_t)bz * S + t0) * a.hidden;
        // RES: the workgroup's [ROWS][W] product tile, past the attention's LDS.
        float *ot = ps + ROWS * S;
        const uint32_t W = (g1 - g0) * 16u;
        const uint32_t tq = 4u * (lane >> 4);
#pragma unroll
        for (uint32_t i = 0; i < GPW; ++i) {
            const uint32_t g = g0 + wave + 4u * i;
            if (g >= g1) break;
            of4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (uint32_t kb = 0; kb < KB; ++kb) {
                const oh8 b = __builtin_bit_cast(oh8, wb[i][kb]);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[kb], b, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[kb], b, acc, 0, 0, 0);
            }
            // Lane (j, c) holds tokens 4c..4c+3 for hidden row 16 g + j.
            const uint32_t n = 16u * g + r;
#pragma unroll
            for (uint32_t e = 0; e < 4u; ++e)
                if (tq + e < R) {
                    if constexpr (RES)
                        ot[(tq + e) * W + (n - 16u * g0)] = acc[e];
                    else
                        slab[(size_t)(tq + e) * a.hidden + n] = acc[e];
                }
        }
        if constexpr (RES) {
            // Atomic adds in the stream's order: column groups of four, then rows,
            // so consecutive threads add to consecutive addresses (a row step is
            // four floats in frag32 order).
            __syncthreads();
            const uint32_t row0 = bz * S + t0;
            for (uint32_t idx = tid; idx < W * ROWS; idx += 256u) {
                const uint32_t e = idx & 3u, t = (idx >> 2) % ROWS, c = 4u * (idx / (4u * ROWS)) + e;
                if (t < R) unsafeAtomicAdd(a.hres + frag32_index(row0 + t, 16u * g0 + c, a.hidden), ot[t * W + c]);
            }
        }
        return;
    }
    auto put = [&](uint32_t t, uint32_t d, float z) {
        const size_t po = a.o_frag ? frag16_index((bz * S + t0 + t), h * D + d, a.out_stride)
                                   : ob + (size_t)t * a.out_stride + d;
        if (a.oh) {
            const _Float16 hv = (_Float16)z;
            a.oh[po] = __builtin_bit_cast(__half, hv);
            a.ol[po] = __builtin_bit_cast(__half, (_Float16)(z - (float)hv));
        } else {
            a.out[po] = z;
        }
    };
    if constexpr (HD > 0) {
        constexpr uint32_t D4 = (uint32_t)HD / 4u;
        for (uint32_t o = tid; o < R * D4; o += 256u) {
            const uint32_t t = o / D4, d4 = o - t * D4;
            float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
            for (uint32_t key = 0; key < S; ++key) {
                const float p = ps[t * S + key];
                const float4 w = *reinterpret_cast<const float4 *>(vs + key * DP + 4u * d4);
                z.x += p * w.x;
                z.y += p * w.y;
                z.z += p * w.z;
                z.w += p * w.w;
            }
            put(t, 4u * d4, z.x);
            put(t, 4u * d4 + 1u, z.y);
            put(t, 4u * d4 + 2u, z.z);
            put(t, 4u * d4 + 3u, z.w);
        }
    } else {
        for (uint32_t o = tid; o < R * D; o += 256u) {
            const uint32_t t = o / D, d = o - t * D;
            float z = 0.f;
#pragma unroll 8
            for (uint32_t key = 0; key < S; ++key) z += ps[t * S + key] * vs[key * DP + d];
            put(t, d, z);
        }
    }
}

}  // namespace

// ------------------------------------------------------------------ launchers
uint32_t gemm_tile_tokens(const GemmArgs &a) { return gemm_q8p_eligible(a) ? gemm_q8p_tile_tokens() : (uint32_t)GM; }

int launch_gemm(hipStream_t s, const GemmArgs &in) {
    GemmArgs a = in;
    if (a.T == 0) return VX_OK;
    if (a.nseg == 0 || a.nseg > 3) return fail(VX_ERR_INVALID_ARG, "gemm: 1..3 weight segments");
    if (a.wk == WT_Q8 ? (a.K % 1024u) : (a.K % (uint32_t)GK))
        return fail(VX_ERR_UNSUPPORTED, "gemm: K=%u must be a multiple of %u for this weight type", a.K,
                    a.wk == WT_Q8 ? 1024u : (uint32_t)GK);
    if (a.frag && (a.xn || a.res_frag)) {   // the short-batch kernel's residual-stream forms
        if (!gemm_skinny_eligible(a))
            return fail(VX_ERR_UNSUPPORTED, "gemm: residual-stream operands need the short-batch kernel "
                                            "(F16, T <= 128, aligned rows, K %% 32 == 0)");
        for (uint32_t i = 0; i < a.nseg; ++i)
            if (!a.seg[i].w) return fail(VX_ERR_INVALID_ARG, "gemm: segment %u weight pointers missing", i);
        return launch_gemm_skinny(s, a);
    }
    if (a.xf32 ? (!a.xf || (a.ldx % 4u)) : (!a.xh || !a.xl || (a.ldx % 8u)))
        return fail(VX_ERR_INVALID_ARG, "gemm: input rows must be 16-byte aligned");
    uint32_t tiles = 0;
    if (a.epi == GEPI_SWIGLU) {
        if (a.nseg != 2 || a.seg[0].rows != a.seg[1].rows)
            return fail(VX_ERR_INVALID_ARG, "gemm swiglu: needs gate and up of equal rows");
        tiles = (a.seg[0].rows + 63u) / 64u;
        if (a.ksplit != 1) return fail(VX_ERR_INVALID_ARG, "gemm swiglu: no split-K");
        if (a.oh && (!a.ol || (!a.ldp && !a.frag)))
            return fail(VX_ERR_INVALID_ARG, "gemm swiglu: plane output incomplete");
    } else {
        for (uint32_t i = 0; i < a.nseg; ++i) {
            a.seg[i].tile0 = tiles;
            tiles += (a.seg[i].rows + GN - 1u) / GN;
            if (!a.seg[i].out) return fail(VX_ERR_INVALID_ARG, "gemm: segment %u has no output", i);
        }
    }
    for (uint32_t i = 0; i < a.nseg; ++i) {
        const GemmSeg &g = a.seg[i];
        if (a.wk == WT_Q8 ? (!g.qs || !g.d) : !g.w)
            return fail(VX_ERR_INVALID_ARG, "gemm: segment %u weight pointers missing", i);
    }
    if (gemm_q8p_eligible(a)) return launch_gemm_q8p(s, a);
    if (gemm_skinny_eligible(a)) return launch_gemm_skinny(s, a);
    if (a.frag)
        return fail(VX_ERR_UNSUPPORTED, "gemm: fragment-layout operands need the short-batch kernel (F16, T <= 128, "
                                        "16-byte aligned, K %% 32 == 0; got T=%u K=%u)", a.T, a.K);
    if (a.split_store && a.ksplit > 1)
        return fail(VX_ERR_INVALID_ARG, "gemm: split partial stores need the prefill-layout Q8_0 or the short-batch F16 kernel");
    const uint32_t stages = a.K / GK;
    if (a.ksplit == 0) a.ksplit = 1;
    if (a.ksplit > stages) a.ksplit = stages;
    a.ntn = tiles;
    a.ntm = (a.T + GM - 1u) / GM;
    const uint64_t total = (uint64_t)a.ntn * a.ntm * a.ksplit;
    if (total == 0) return VX_OK;
    const uint64_t grid = (total + 7u) / 8u * 8u;
    if (grid > 0x7fffffffull) return fail(VX_ERR_UNSUPPORTED, "gemm: grid too large");
    const dim3 g((unsigned)grid), blk(256);
#define VX_GEMM_CASE(WKV, XF, EP)                                                                  \
    if (a.wk == WKV && a.xf32 == XF && a.epi == EP) {                                              \
        k_gemm<WKV, XF, EP><<<g, blk, 0, s>>>(a);                                                   \
        VX_LAUNCHED("k_gemm");                                                                      \
        return VX_OK;                                                                               \
    }
    VX_GEMM_CASE(WT_Q8, false, GEPI_STORE)
    VX_GEMM_CASE(WT_Q8, false, GEPI_RESIDUAL)
    VX_GEMM_CASE(WT_Q8, false, GEPI_SWIGLU)
    VX_GEMM_CASE(WT_Q8, true, GEPI_STORE)
    VX_GEMM_CASE(WT_Q8, true, GEPI_SWIGLU)
    VX_GEMM_CASE(WT_F16, false, GEPI_STORE)
    VX_GEMM_CASE(WT_F16, false, GEPI_RESIDUAL)
    VX_GEMM_CASE(WT_F16, false, GEPI_SWIGLU)
    VX_GEMM_CASE(WT_F16, true, GEPI_STORE)
    VX_GEMM_CASE(WT_F16, true, GEPI_RESIDUAL)
    VX_GEMM_CASE(WT_F16, true, GEPI_SWIGLU)
#undef VX_GEMM_CASE
    return fail(VX_ERR_UNSUPPORTED, "gemm: no kernel for weight type %u, f32 input %d, epilogue %u", a.wk,
                (int)a.xf32, a.epi);
}

int launch_seq_rmsnorm(hipStream_t s, const SeqNormArgs &a, uint32_t tokens) {
    if (tokens == 0) return VX_OK;
    if (a.yh && !a.yl) return fail(VX_ERR_INVALID_ARG, "seq rmsnorm: plane output incomplete");
    if (a.yh && a.tiled && a.n % 32u) return fail(VX_ERR_INVALID_ARG, "seq rmsnorm: tiled planes need n %% 32");
    if (a.nbranch == 0 || a.nbranch > kSeqNormMaxBranch)
        return fail(VX_ERR_INVALID_ARG, "seq rmsnorm: 1..%u branches", kSeqNormMaxBranch);
    if ((a.h_frag || a.hf) && (a.n % 1024u || a.n > 4096u || (a.h_frag && a.branch)))
        return fail(VX_ERR_UNSUPPORTED, "seq rmsnorm: the frag32 residual stream needs n = 1024 * k <= 4096, no branch");
    const bool vec = a.n % 1024u == 0 && a.n <= 4096u && a.ldh % 4u == 0 && (!a.branch || (a.ldb % 4u == 0 && a.branch_stride % 4u == 0)) &&
                     (!a.y || a.ldy % 4u == 0) && (!a.yh || a.tiled || a.ldp % 4u == 0);
    if (vec) {
        const bool wide = a.branch && a.nbranch > 8u;
        SeqNormArgs b = a;
        VX_SET_STAMPS(b, ST_SEQ_NORM, (uint64_t)tokens * 4u);
        switch (a.n / 1024u) {
            case 1: wide ? k_seq_rmsnorm4<1, 16><<<tokens, 256, 0, s>>>(b) : k_seq_rmsnorm4<1, 8><<<tokens, 256, 0, s>>>(b); break;
            case 2: wide ? k_seq_rmsnorm4<2, 16><<<tokens, 256, 0, s>>>(b) : k_seq_rmsnorm4<2, 8><<<tokens, 256, 0, s>>>(b); break;
            case 3: wide ? k_seq_rmsnorm4<3, 16><<<tokens, 256, 0, s>>>(b) : k_seq_rmsnorm4<3, 8><<<tokens, 256, 0, s>>>(b); break;
            default: wide ? k_seq_rmsnorm4<4, 16><<<tokens, 256, 0, s>>>(b) : k_seq_rmsnorm4<4, 8><<<tokens, 256, 0, s>>>(b); break;
        }
        VX_LAUNCHED("k_seq_rmsnorm4");
        return VX_OK;
    }
    k_seq_rmsnorm<<<tokens, 256, 0, s>>>(a);
    VX_LAUNCHED("k_seq_rmsnorm");
    return VX_OK;
}

int launch_seq_rope_store(hipStream_t s, const SeqRopeArgs &a, uint32_t tokens) {
    if (tokens == 0) return VX_OK;
    if (a.nsplit > kSeqRopeMaxSplit)
        return fail(VX_ERR_INVALID_ARG, "seq rope: at most %u split partials", kSeqRopeMaxSplit);
    if (a.head_dim == 0 || a.head_dim > 128u || (a.head_dim & 1u))
        return fail(VX_ERR_UNSUPPORTED, "seq rope: head_dim must be even and <= 128");
    if (a.kc && (!a.vc || !a.v)) return fail(VX_ERR_INVALID_ARG, "seq rope: KV store needs v and both caches");
    k_seq_rope_store<<<tokens, 256, 0, s>>>(a);
    VX_LAUNCHED("k_seq_rope_store");
    return VX_OK;
}

int launch_seq_embedding(hipStream_t s, const uint8_t *raw, uint32_t weight_offset, uint32_t dtype,
                         uint32_t cols, const uint32_t *tokens, uint32_t n, uint32_t vocab, float alpha,
                         float *out, uint32_t ldo) {
    if (!n || !cols) return VX_OK;
    k_seq_embedding<<<dim3((cols + 255u) / 256u, n), 256, 0, s>>>(raw, weight_offset, dtype, cols, tokens, vocab,
                                                                  alpha, out, ldo);
    VX_LAUNCHED("k_seq_embedding");
    return VX_OK;
}

int launch_seq_linear_generic(hipStream_t s, const SeqGenericArgs &a) {
    const uint64_t waves = (uint64_t)a.rows * a.tokens;
    if (!waves) return VX_OK;
    if (waves > 0xffffffffull) return fail(VX_ERR_UNSUPPORTED, "seq linear: too many rows x tokens");
    k_seq_linear_generic<<<(unsigned)((waves + 3u) / 4u), 256, 0, s>>>(a);
    VX_LAUNCHED("k_seq_linear_generic");
    return VX_OK;
}

int launch_silu_mul(hipStream_t s, float *g, const float *u, uint32_t n) {
    if (!n) return VX_OK;
    k_silu_mul<<<(n + 255u) / 256u, 256, 0, s>>>(g, u, n);
    VX_LAUNCHED("k_silu_mul");
    return VX_OK;
}

int launch_dense_attn(hipStream_t s, const DenseAttnArgs &a, int which) {
    if (!a.tokens || !a.q_heads || !a.batch) return VX_OK;
    if (!a.kv_heads || a.q_heads % a.kv_heads) return fail(VX_ERR_SHAPE, "dense attention: head counts");
    if (which == 0) {
        if (a.head_dim > 256u) return fail(VX_ERR_UNSUPPORTED, "dense attention: head_dim > 256");
        k_dense_scores<<<dim3(a.tokens, a.q_heads, a.batch), 64, 0, s>>>(a);
        VX_LAUNCHED("k_dense_scores");
    } else if (which == 1) {
        k_dense_softmax<<<dim3(a.q_heads, a.tokens, a.batch), 64, 0, s>>>(a.s, a.tokens, a.q_heads, a.score_stride);
        VX_LAUNCHED("k_dense_softmax");
    } else {
        if (a.head_dim > 256u) return fail(VX_ERR_UNSUPPORTED, "dense attention: head_dim > 256");
        k_dense_values<<<dim3(a.q_heads, a.tokens, a.batch), 256, 0, s>>>(a);
        VX_LAUNCHED("k_dense_values");
    }
    return VX_OK;
}

namespace {
__global__ __launch_bounds__(256) void k_rope_pos_table(float2 *tab, const float *factors, uint32_t tokens,
                                                        uint32_t head_dim, float theta, float scaling) {
    const uint32_t half = head_dim / 2u, n = tokens * half;
    const uint32_t j = blockIdx.x * 256u + threadIdx.x;
    if (j >= n) return;
    const uint32_t pos = j / half, i = j - pos * half;
    const float exponent = (float)(i * 2u) / (float)head_dim;   // as k_seq_rope_store
    const float inv_freq = 1.0f / powf(theta, exponent);
    const float angle = (float)pos * inv_freq / factors[i];
    tab[j] = make_float2(cosf(angle) * scaling, sinf(angle) * scaling);
}
}  // namespace

int launch_rope_pos_table(hipStream_t s, float2 *table, const float *factors, uint32_t tokens, uint32_t head_dim,
                          float theta, float scaling) {
    const uint32_t n = tokens * (head_dim / 2u);
    if (!n) return VX_OK;
    k_rope_pos_table<<<(n + 255u) / 256u, 256, 0, s>>>(table, factors, tokens, head_dim, theta, scaling);
    VX_LAUNCHED("k_rope_pos_table");
    return VX_OK;
}

uint64_t dense_fused_lds_rows(uint32_t tokens, uint32_t head_dim, uint32_t rows) {
    const uint32_t pad = head_dim == 64u || head_dim == 128u ? 4u : 1u;   // DP of the kernel
    return ((2ull * tokens + rows) * (head_dim + pad) + (uint64_t)rows * tokens) * 4u;
}

uint64_t dense_fused_lds(uint32_t tokens, uint32_t head_dim) {
    return dense_fused_lds_rows(tokens, head_dim, kDenseFusedRows);
}

bool dense_attn_oproj_eligible(uint32_t tokens, uint32_t head_dim) {
    return tokens > 0 && tokens <= kDenseFusedMaxTokens && (head_dim == 64u || head_dim == 128u) &&
           dense_fused_lds_rows(tokens, head_dim, kOprojRows) <= 65536u;
}

int launch_dense_attn_oproj(hipStream_t s, const DenseAttnArgs &a) {
    if (!a.tokens || !a.q_heads || !a.batch) return VX_OK;
    if (!a.kv_heads || a.q_heads % a.kv_heads) return fail(VX_ERR_SHAPE, "attention + O projection: head counts");
    if (!dense_attn_oproj_eligible(a.tokens, a.head_dim))
        return fail(VX_ERR_UNSUPPORTED, "attention + O projection: %u tokens x head_dim %u", a.tokens, a.head_dim);
    auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    const bool res = a.hres != nullptr;
    if (res != (a.ssq != nullptr) || (res && (a.hidden % 32u || !a.norm_n)))
        return fail(VX_ERR_INVALID_ARG, "attention + O projection: the residual-stream form needs hres, ssq, "
                                        "norm_n and hidden %% 32 == 0");
    if (!a.wo || !al16(a.wo) || !a.hidden || a.hidden % 16u ||
        (!res && (!a.oslab || a.oslab_stride < (uint64_t)a.batch * a.tokens * a.hidden)))
        return fail(VX_ERR_INVALID_ARG, "attention + O projection: weights or slabs");
    if (!a.rope || a.q_stride % 4u || a.k_stride % 4u || a.v_stride % 4u || !al16(a.q) || !al16(a.k) || !al16(a.v) ||
        !al16(a.rope) || (a.nslab != 1 && a.nslab != 2) || (a.nslab == 2 && a.slab_stride % 4u))
        return fail(VX_ERR_UNSUPPORTED, "attention + O projection: needs float4 rows, RoPE and 1 or 2 input slabs");
    DenseAttnArgs b = a;
    b.vec = 1;
    b.oh = b.ol = nullptr;
    b.out = nullptr;
    // Split the hidden rows so that no wave holds more than kOprojBlocks weight
    // blocks, and so that the grid reaches about 128 workgroups (512 for
    // sequences of at most 16 tokens, whose workgroups are short: two per CU
    // overlap one's staging with the other's projection).
    const uint32_t ngroups = (a.tokens + kOprojRows - 1u) / kOprojRows, ng = a.hidden / 16u;
    const uint32_t per_wave = kOprojBlocks / (a.head_dim / 32u);
    uint32_t nsplit = (ng + 4u * per_wave - 1u) / (4u * per_wave);
    const uint32_t base = a.q_heads * a.batch * ngroups, target = a.tokens <= 16u ? 512u : 128u;
    while (base * nsplit < target && 2u * nsplit <= (ng + 3u) / 4u) nsplit *= 2u;
    b.nsplit = nsplit;
    uint64_t lds = dense_fused_lds_rows(a.tokens, a.head_dim, kOprojRows);
    if (res) {   // the product tile of the residual-stream form
        lds += (uint64_t)kOprojRows * ((ng + nsplit - 1u) / nsplit) * 16u * 4u;
        if (lds > 65536u) return fail(VX_ERR_UNSUPPORTED, "attention + O projection: residual tile exceeds LDS");
    }
    const dim3 grid(a.q_heads, a.batch, ngroups * nsplit);
    VX_SET_STAMPS(b, ST_DENSE_ATTN, (uint64_t)grid.x * grid.y * grid.z * 4u);
    const bool short_seq = a.tokens <= 16u;
#define VX_OPROJ(HDV, NS, RS)                                                               \
    do {                                                                                    \
        if (short_seq) k_dense_attn_fused<HDV, NS, true, RS, 16u><<<grid, 256, (size_t)lds, s>>>(b); \
        else k_dense_attn_fused<HDV, NS, true, RS><<<grid, 256, (size_t)lds, s>>>(b);       \
    } while (0)
    if (res) {
        if (a.head_dim == 64u && a.nslab == 2) VX_OPROJ(64, 2, true);
        else if (a.head_dim == 128u && a.nslab == 2) VX_OPROJ(128, 2, true);
        else if (a.head_dim == 64u) VX_OPROJ(64, 1, true);
        else VX_OPROJ(128, 1, true);
    } else {
        if (a.head_dim == 64u && a.nslab == 2) VX_OPROJ(64, 2, false);
        else if (a.head_dim == 128u && a.nslab == 2) VX_OPROJ(128, 2, false);
        else if (a.head_dim == 64u) VX_OPROJ(64, 1, false);
        else VX_OPROJ(128, 1, false);
    }
#undef VX_OPROJ
    VX_LAUNCHED("k_dense_attn_fused");
    return VX_OK;
}

int launch_dense_attn_fused(hipStream_t s, const DenseAttnArgs &a) {
    if (!a.tokens || !a.q_heads || !a.batch) return VX_OK;
    if (!a.kv_heads || a.q_heads % a.kv_heads) return fail(VX_ERR_SHAPE, "dense attention: head counts");
    const uint64_t lds = dense_fused_lds(a.tokens, a.head_dim);
    if (a.tokens > kDenseFusedMaxTokens || a.head_dim == 0 || lds > 65536u)
        return fail(VX_ERR_UNSUPPORTED, "fused dense attention: %u tokens x head_dim %u do not fit", a.tokens,
                    a.head_dim);
    if (a.oh && !a.ol) return fail(VX_ERR_INVALID_ARG, "fused dense attention: plane output incomplete");
    if (!a.oh && !a.out) return fail(VX_ERR_INVALID_ARG, "fused dense attention: no output");
    if (a.o_frag && (!a.oh || a.out_stride % 32u))
        return fail(VX_ERR_INVALID_ARG, "fused dense attention: fragment-layout planes need width %% 32");
    DenseAttnArgs b = a;
    auto al16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
    b.vec = a.q_stride % 4u == 0 && a.k_stride % 4u == 0 && a.v_stride % 4u == 0 && al16(a.q) && al16(a.k) &&
            al16(a.v) && al16(a.rope);
    if (a.nslab > 2 || (a.nslab == 2 && (!b.vec || !a.rope || (a.head_dim != 64u && a.head_dim != 128u) ||
                                          a.slab_stride % 4u)))
        return fail(VX_ERR_UNSUPPORTED, "fused dense attention: %u input slabs", a.nslab);
    const dim3 grid(a.q_heads, a.batch, (a.tokens + kDenseFusedRows - 1u) / kDenseFusedRows);
    const bool short_seq = a.tokens <= 16u;
    if (a.head_dim == 64u && a.nslab == 2 && short_seq)
        k_dense_attn_fused<64, 2, false, false, 16u><<<grid, 256, (size_t)lds, s>>>(b);
    else if (a.head_dim == 128u && a.nslab == 2 && short_seq)
        k_dense_attn_fused<128, 2, false, false, 16u><<<grid, 256, (size_t)lds, s>>>(b);
    else if (a.head_dim == 64u && a.nslab == 2)
        k_dense_attn_fused<64, 2><<<grid, 256, (size_t)lds, s>>>(b);
    else if (a.head_dim == 128u && a.nslab == 2)
        k_dense_attn_fused<128, 2><<<grid, 256, (size_t)lds, s>>>(b);
    else if (a.head_dim == 64u)
        k_dense_attn_fused<64><<<grid, 256, (size_t)lds, s>>>(b);
    else if (a.head_dim == 128u)
        k_dense_attn_fused<128><<<grid, 256, (size_t)lds, s>>>(b);
    else
        k_dense_attn_fused<0><<<grid, 256, (size_t)lds, s>>>(b);
    VX_LAUNCHED("k_dense_attn_fused");
    return VX_OK;
}

int launch_prefill_attn(hipStream_t s, const PrefillAttnArgs &a) {
    if (a.T == 0) return VX_OK;
    if (a.kv_heads == 0 || a.q_heads % a.kv_heads) return fail(VX_ERR_SHAPE, "prefill attention: head counts");
    const uint32_t qpk = a.q_heads / a.kv_heads;
    if ((uint64_t)a.pos_base + a.T > a.context)
        return fail(VX_ERR_CONTEXT_FULL, "prefill attention: positions beyond the context");
    if (a.oh && !a.ol) return fail(VX_ERR_INVALID_ARG, "prefill attention: plane output incomplete");
    if (a.ldq % 8u || a.ldo % 4u) return fail(VX_ERR_INVALID_ARG, "prefill attention: row strides");
    if (a.oh && a.tiled && a.ldo % 32u) return fail(VX_ERR_INVALID_ARG, "prefill attention: tiled planes need width %% 32");
#define VX_ATTN_CASE(HDV, QPKV)                                                                  \
    if (a.head_dim == HDV && qpk == QPKV) {                                                      \
        dim3 g((a.T + (32u / QPKV) - 1u) / (32u / QPKV), a.kv_heads);                            \
        k_prefill_attn<HDV, QPKV><<<g, 256, 0, s>>>(a);                                          \
        VX_LAUNCHED("k_prefill_attn");                                                           \
        return VX_OK;                                                                            \
    }
    VX_ATTN_CASE(128, 8)
    VX_ATTN_CASE(128, 4)
    VX_ATTN_CASE(128, 2)
    VX_ATTN_CASE(128, 1)
    VX_ATTN_CASE(64, 8)
    VX_ATTN_CASE(64, 4)
    VX_ATTN_CASE(64, 2)
    VX_ATTN_CASE(64, 1)
#undef VX_ATTN_CASE
    return fail(VX_ERR_UNSUPPORTED, "prefill attention: head_dim %u with %u query heads per KV head", a.head_dim,
                qpk);
}

}  // namespace vx
