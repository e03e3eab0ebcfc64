// Short-batch projection GEMM on gfx950: F16 weights, at most 128 tokens, X as
// hi/lo f16 planes. This is the shape of the LocDiT estimator, which projects the
// CFG batch of two sequences (2 x 37 rows at 32 condition tokens) through every
// weight matrix once per Euler step.
//
//   C[t][n] = sum_k X[t][k] * W[n][k],  X = hi + lo (two MFMAs per product),
//   W exact f16, fp32 accumulation: the arithmetic of k_gemm.
//
// At so few tokens every workgroup reads all of X, and the kernel is bound by
// how fast a CU pulls operands in. A wave64 load whose lanes touch 16 rows of
// 64 bytes each moves about 30 GB/s per workgroup on MI355X, one that reads 1 KB
// of contiguous bytes 75-85 GB/s. So both operands are stored in the fragment
// layout (frag16_index): the weights repacked once at model set-up, the planes
// written so by their producers (rmsnorm, attention, this kernel's SwiGLU
// epilogue). Then:
//   * a workgroup owns 32 weight rows (two 16-row B fragments) and every token
//     (MT 16-token A fragments), and its four waves take interleaved 32-column
//     k-steps of the workgroup's K range, so the waves share no operand and
//     every operand is one contiguous 1 KB block: global -> VGPR ->
//     v_mfma_f32_16x16x32_f16, with no LDS staging and no barrier in the k-loop;
//   * each wave keeps kSkDepth k-steps of operands in flight (a register ring,
//     fully unrolled so the ring indices are static);
//   * the four waves' partial tiles meet in LDS once, and each thread then
//     finishes whole outputs: stores, bias, the SwiGLU epilogue (silu(g) * u
//     with gate and up rows in the two fragments), or a split-K partial slab;
//   * split K across workgroups writes partial slabs with plain stores (slab s
//     at out + s * ws_stride); the consumer sums them. No atomics and no
//     cleared accumulators, so a captured graph replays it as is.
//   * with GemmArgs::xn (XN) X is the residual stream itself, f32 in the same
//     fragment order (frag32_index), and the rmsnorm in front of the projection
//     is folded in: each lane multiplies its eight values by the norm weights and
//     splits them to hi/lo f16 in registers, and accumulates their squares; the
//     row sums of squares meet in LDS, and 1/rms scales the row's products
//     (rmsnorm(x) w . W = (1/rms) ((x w) . W)), in the SwiGLU epilogue or, for a
//     split projection, in its consumer (the slabs' sums of squares are stored).
//   * with GemmArgs::res_frag the products are added to the residual stream with
//     atomic adds (every K slab), in place of partial slabs and a reduction pass.
#include <type_traits>

#include "vx_internal.h"

namespace vx {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kSkRows = 32;   // weight rows per workgroup (GEPI_STORE): two 16-row fragments
constexpr uint32_t kSkPairs = 16;  // gate/up row pairs per workgroup (GEPI_SWIGLU)
constexpr int kSkDepth = 3;        // k-steps in flight per wave (4 with at most two token fragments)
constexpr uint32_t kSkMaxTokens = 128;

// Weights are read once per launch: nontemporal loads keep them from evicting
// the activation planes and partial slabs the other kernels of the layer reuse.
__device__ __forceinline__ uint4 ld_nt16(const __half *p) {
    typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ f4 mfma16(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <int MT>
struct SkOps {
    uint4 w[2];
    uint4 xh[MT], xl[MT];
};
template <int MT>
struct SkOpsN {      // X from the f32 residual stream: 8 values per lane and token fragment
    uint4 w[2];
    float4 x[MT][2];
    float4 nw[2];    // the lane's 8 norm weights
};

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// Grid: a.ntn row tiles x a.ksplit k-slabs, 256 threads.
template <int MT, int EPI, bool XN = false>
__global__ __launch_bounds__(256) void k_gemm_sk(GemmArgs a) {
    VX_WAVE_STAMP(a.stamps);
    // Partial tiles of the four waves: [wave][mt][fragment][lane] x 4 floats.
    __shared__ f4 red[4][MT][2][64];
    __shared__ float ssl[XN ? 4 : 1][XN ? MT : 1][16];   // XN: each wave's row sums of squares
    const uint32_t tile = blockIdx.x % a.ntn, ks = blockIdx.x / a.ntn;
    const uint32_t tid = threadIdx.x, lane = tid & 63u;
    const uint32_t wv = __builtin_amdgcn_readfirstlane(tid >> 6);

    uint32_t seg = 0;
    if constexpr (EPI != GEPI_SWIGLU) {
        while (seg + 1 < a.nseg && tile >= a.seg[seg + 1].tile0) ++seg;
    }
    const GemmSeg &sg = a.seg[seg];
    const uint32_t S = a.K >> 5;
    // Row groups past a matrix are clamped to its last one. Token rows past T in
    // the last A block are multiplied like the others and never stored (each
    // output row of an MFMA depends only on its own A row). With at most two A
    // blocks, when T - 1 is among the last block's first eight rows, rows past it
    // read row T - 1 instead, so that rows 8-15 (the second 128 bytes of each
    // 256-byte column group) add no cache line of their own; otherwise they read
    // whatever the producer left there.
    const __half *wr[2];
#pragma unroll
    for (int f = 0; f < 2; ++f) {
        uint32_t rg, rows;
        const __half *base;
        if constexpr (EPI == GEPI_SWIGLU) {
            rg = tile;
            rows = a.seg[f].rows;
            base = a.seg[f].w;
        } else {
            rg = 2u * (tile - sg.tile0) + f;
            rows = sg.rows;
            base = sg.w;
        }
        const uint32_t last = (rows - 1u) >> 4;
        if (rg > last) rg = last;
        wr[f] = base + ((size_t)rg * S << 9) + 8u * lane;
    }
    uint32_t xlane[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const uint32_t last = a.T - 1u - min(a.T - 1u, 16u * (uint32_t)mt);
        xlane[mt] = MT <= 2 && last < 8u ? (lane & ~15u) | min(lane & 15u, last) : lane;
    }
    const __half *xr[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xr[mt] = a.xh + ((size_t)mt * S << 9) + 8u * xlane[mt];
    const ptrdiff_t lo = a.xl - a.xh;

    const uint32_t s0 = ks * S / a.ksplit, s1 = (ks + 1u) * S / a.ksplit;
    const int n_it = s0 + wv < s1 ? (int)((s1 - s0 - wv + 3u) >> 2) : 0;

    f4 acc[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt][0] = acc[mt][1] = f4{0.f, 0.f, 0.f, 0.f};
    float ss[MT];   // XN: the lane's sum of squares per token fragment
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) ss[mt] = 0.f;

    using Ops = typename std::conditional<XN, SkOpsN<MT>, SkOps<MT>>::type;
    // With at most two token fragments a k-step's operands are fewer registers, and
    // four steps in flight cover the whole K range of a wave in the QKV and
    // ffn_down launches of the 11-token contract (four k-steps each).
    constexpr int DEPTH = MT <= 2 ? 4 : kSkDepth;
    Ops ring[DEPTH];
    auto load = [&](Ops &o, int i) {
        const uint32_t step = s0 + wv + 4u * (uint32_t)i;
        const uint32_t c = step << 9;   // block offset of the k-step (halves of W; floats of xn)
        o.w[0] = ld_nt16(wr[0] + c);
        o.w[1] = ld_nt16(wr[1] + c);
        if constexpr (XN) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const float *p = a.xn + ((size_t)mt * S << 9) + c + 4u * xlane[mt];
                o.x[mt][0] = *reinterpret_cast<const float4 *>(p);
                o.x[mt][1] = *reinterpret_cast<const float4 *>(p + 256);
            }
            const float *nw = a.xn_w + (step << 5) + 8u * (lane >> 4);
            o.nw[0] = *reinterpret_cast<const float4 *>(nw);
            o.nw[1] = *reinterpret_cast<const float4 *>(nw + 4);
        } else {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                o.xh[mt] = *reinterpret_cast<const uint4 *>(xr[mt] + c);
                o.xl[mt] = *reinterpret_cast<const uint4 *>(xr[mt] + lo + c);
            }
        }
    };
    auto mma = [&](const Ops &o) {
        const h8 b0 = __builtin_bit_cast(h8, o.w[0]), b1 = __builtin_bit_cast(h8, o.w[1]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            h8 ah, al;
            if constexpr (XN) {
                const float xv[8] = {o.x[mt][0].x, o.x[mt][0].y, o.x[mt][0].z, o.x[mt][0].w,
                                     o.x[mt][1].x, o.x[mt][1].y, o.x[mt][1].z, o.x[mt][1].w};
                const float wv8[8] = {o.nw[0].x, o.nw[0].y, o.nw[0].z, o.nw[0].w,
                                      o.nw[1].x, o.nw[1].y, o.nw[1].z, o.nw[1].w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float y = xv[e] * wv8[e];
                    const _Float16 hv = (_Float16)y;
                    ah[e] = hv;
                    al[e] = (_Float16)(y - (float)hv);
                    ss[mt] = fmaf(xv[e], xv[e], ss[mt]);
                }
            } else {
                ah = __builtin_bit_cast(h8, o.xh[mt]);
                al = __builtin_bit_cast(h8, o.xl[mt]);
            }
            acc[mt][0] = mfma16(ah, b0, acc[mt][0]);
            acc[mt][1] = mfma16(ah, b1, acc[mt][1]);
            acc[mt][0] = mfma16(al, b0, acc[mt][0]);
            acc[mt][1] = mfma16(al, b1, acc[mt][1]);
        }
    };
    // The loads are unconditional (steps past the wave's last one reload its last
    // step): a load under a branch would make the compiler's wait counting assume
    // the branch not taken and wait for every load in flight before each MFMA.
    if (n_it > 0) {
#pragma unroll
        for (int u = 0; u < DEPTH - 1; ++u) load(ring[u], min(u, n_it - 1));
        for (int it = 0; it < n_it; it += DEPTH) {
#pragma unroll
            for (int u = 0; u < DEPTH; ++u) {
                const int i = it + u;
                load(ring[(u + DEPTH - 1) % DEPTH], min(i + DEPTH - 1, n_it - 1));
                if (i < n_it) mma(ring[u]);
            }
        }
    }

    // Lane (j, q) of a 16x16 accumulator holds tokens 4q..4q+3 of its A fragment
    // for weight row j of its B fragment.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        red[wv][mt][0][lane] = acc[mt][0];
        red[wv][mt][1][lane] = acc[mt][1];
    }
    if constexpr (XN) {
        // Lanes r, r + 16, r + 32, r + 48 hold row r's columns.
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            float v = ss[mt];
            v += __shfl_xor(v, 16, 64);
            v += __shfl_xor(v, 32, 64);
            if (lane < 16u) ssl[wv][mt][lane] = v;
        }
    }
    __syncthreads();
    // XN: the workgroup's sum of squares of token tok (over its K range).
    auto row_ss = [&](uint32_t tok) {
        if constexpr (XN) {
            const uint32_t mt = tok >> 4, r = tok & 15u;
            return (ssl[0][mt][r] + ssl[1][mt][r]) + (ssl[2][mt][r] + ssl[3][mt][r]);
        } else {
            return 0.f;
        }
    };
    auto part = [&](uint32_t mt, uint32_t f, uint32_t tl, uint32_t n) {
        const uint32_t ln = n + 16u * ((tl >> 2) & 3u), r = tl & 3u;
        return red[0][mt][f][ln][r] + red[1][mt][f][ln][r] + red[2][mt][f][ln][r] + red[3][mt][f][ln][r];
    };
    if constexpr (EPI == GEPI_SWIGLU) {
        for (uint32_t o = tid; o < 256u * MT; o += 256u) {
            const uint32_t n = o & 15u, tl = o >> 4, mt = tl >> 4;
            const uint32_t tok = tl, row = kSkPairs * tile + n;
            if (tok >= a.T || row >= a.seg[0].rows) continue;
            float g = part(mt, 0, tl & 15u, n), u = part(mt, 1, tl & 15u, n);
            if constexpr (XN) {   // rmsnorm.comp:36-38 over the full row (no split K here)
                const float inv = 1.0f / sqrtf(row_ss(tok) / (float)a.K + a.xn_eps);
                g *= inv;
                u *= inv;
            }
            const float v = silu_mul(g, u);
            if (a.seg[0].out) a.seg[0].out[(size_t)tok * a.seg[0].ldo + row] = v;
            if (a.oh) {
                const size_t po = frag16_index(tok, row, a.seg[0].rows);
                const _Float16 hv = (_Float16)v;
                a.oh[po] = __builtin_bit_cast(__half, hv);
                a.ol[po] = __builtin_bit_cast(__half, (_Float16)(v - (float)hv));
            }
        }
    } else {
        if constexpr (XN) {   // the K slab's sums of squares, once (the first row tile)
            if (a.xn_ss && tile == 0u && tid < 16u * MT && tid < a.T) a.xn_ss[(size_t)ks * a.xn_ss_stride + tid] = row_ss(tid);
        }
        if (a.res_frag) {
            // The tile's outputs are MT whole 2 KB blocks of the stream (32 columns
            // of its rows, 16 tokens each): thread order = block order, so every
            // wave's atomic adds cover 256 contiguous bytes.
            for (uint32_t o = tid; o < 512u * MT; o += 256u) {
                const uint32_t mt = o >> 9, w = o & 511u, li = (w >> 2) & 63u;
                const uint32_t r = li & 15u, nl = 8u * (li >> 4) + 4u * (w >> 8) + (w & 3u);
                const uint32_t tok = 16u * mt + r, row = kSkRows * (tile - sg.tile0) + nl;
                if (tok >= a.T || row >= sg.rows) continue;
                float v = part(mt, nl >> 4, r, nl & 15u);
                if (sg.bias && ks == 0)
                    v += sg.bias_dtype == 0 ? static_cast<const float *>(sg.bias)[row]
                                            : __half2float(static_cast<const __half *>(sg.bias)[row]);
                unsafeAtomicAdd(a.res_frag + frag32_index(tok, row, sg.rows), v * a.alpha);
            }
            return;
        }
        float *out = sg.out + (a.ksplit > 1 ? (size_t)ks * a.ws_stride : 0);
        for (uint32_t o = tid; o < 512u * MT; o += 256u) {
            const uint32_t nl = o & 31u, tl = o >> 5, mt = tl >> 4;
            const uint32_t tok = tl, row = kSkRows * (tile - sg.tile0) + nl;
            if (tok >= a.T || row >= sg.rows) continue;
            float v = part(mt, nl >> 4, tl & 15u, nl & 15u);
            if (sg.bias && ks == 0)
                v += sg.bias_dtype == 0 ? static_cast<const float *>(sg.bias)[row]
                                        : __half2float(static_cast<const __half *>(sg.bias)[row]);
            out[(size_t)tok * sg.ldo + row] = v * a.alpha;
        }
    }
}

template <int EPI, bool XN>
int launch_sk(hipStream_t s, const GemmArgs &a, uint32_t grid) {
    const uint32_t mt = (a.T + 15u) / 16u;
    switch (mt) {
#define VX_SK_CASE(M)                                  \
    case M:                                            \
        k_gemm_sk<M, EPI, XN><<<grid, 256, 0, s>>>(a); \
        break;
        VX_SK_CASE(1)
        VX_SK_CASE(2)
        VX_SK_CASE(3)
        VX_SK_CASE(4)
        VX_SK_CASE(5)
        VX_SK_CASE(6)
        VX_SK_CASE(7)
        VX_SK_CASE(8)
#undef VX_SK_CASE
        default: return fail(VX_ERR_UNSUPPORTED, "skinny gemm: %u tokens", a.T);
    }
    VX_LAUNCHED("k_gemm_sk");
    return VX_OK;
}

// One thread per 8-column chunk of the padded matrix.
__global__ __launch_bounds__(256) void k_repack_frag16(const __half *src, __half *dst, uint32_t rows, uint32_t K,
                                                       uint64_t total) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i >= total) return;
    const uint32_t per_row = K >> 3, r = (uint32_t)(i / per_row), c = (uint32_t)(i - (uint64_t)r * per_row) << 3;
    const uint4 v = r < rows ? *reinterpret_cast<const uint4 *>(src + (size_t)r * K + c) : make_uint4(0, 0, 0, 0);
    *reinterpret_cast<uint4 *>(dst + frag16_index(r, c, K)) = v;
}

}  // namespace

bool gemm_skinny_eligible(const GemmArgs &a) {
    if (!a.frag || a.wk != WT_F16 || a.xf32 || a.x_tiled || a.T == 0 || a.T > kSkMaxTokens || a.K % 32u) return false;
    if (a.xn) {
        if (!a.xn_w || ((reinterpret_cast<uintptr_t>(a.xn) | reinterpret_cast<uintptr_t>(a.xn_w)) & 15u)) return false;
    } else if (!a.xh || !a.xl || ((reinterpret_cast<uintptr_t>(a.xh) | reinterpret_cast<uintptr_t>(a.xl)) & 15u)) {
        return false;
    }
    if (a.res_frag && (a.epi != GEPI_STORE || a.nseg != 1 || a.seg[0].rows % 32u)) return false;
    for (uint32_t i = 0; i < a.nseg; ++i)
        if (!a.seg[i].w || (reinterpret_cast<uintptr_t>(a.seg[i].w) & 15u) || a.seg[i].rows == 0) return false;
    if (a.epi == GEPI_SWIGLU) return a.ksplit <= 1 && !a.o_tiled && a.nseg == 2 && a.seg[0].rows % 32u == 0;
    if (a.epi == GEPI_STORE) return a.ksplit <= 1 || a.split_store || a.res_frag;
    return false;
}

// Called by launch_gemm with validated, eligible arguments; sets the tiling fields.
int launch_gemm_skinny(hipStream_t s, GemmArgs a) {
    uint32_t tiles = 0;
    if (a.epi == GEPI_SWIGLU) {
        tiles = (a.seg[0].rows + kSkPairs - 1u) / kSkPairs;
    } else {
        for (uint32_t i = 0; i < a.nseg; ++i) {
            a.seg[i].tile0 = tiles;
            tiles += (a.seg[i].rows + kSkRows - 1u) / kSkRows;
        }
    }
    const uint32_t steps = a.K / 32u;
    if (a.ksplit == 0) a.ksplit = 1;
    if (a.ksplit > steps) a.ksplit = steps;
    a.ntn = tiles;
    a.ntm = 1;
    const uint64_t grid = (uint64_t)tiles * a.ksplit;
    if (grid == 0) return VX_OK;
    if (grid > 0x7fffffffull) return fail(VX_ERR_UNSUPPORTED, "skinny gemm: grid too large");
    VX_SET_STAMPS(a, ST_GEMM_SK, grid * 4u);
    if (a.xn)
        return a.epi == GEPI_SWIGLU ? launch_sk<GEPI_SWIGLU, true>(s, a, (uint32_t)grid)
                                    : launch_sk<GEPI_STORE, true>(s, a, (uint32_t)grid);
    return a.epi == GEPI_SWIGLU ? launch_sk<GEPI_SWIGLU, false>(s, a, (uint32_t)grid)
                                : launch_sk<GEPI_STORE, false>(s, a, (uint32_t)grid);
}

int launch_repack_frag16(hipStream_t s, const __half *src, __half *dst, uint32_t rows, uint32_t K) {
    if (!src || !dst || !rows || !K || K % 32u) return fail(VX_ERR_INVALID_ARG, "frag16 repack: bad matrix");
    if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u)
        return fail(VX_ERR_INVALID_ARG, "frag16 repack: 16-byte alignment");
    const uint64_t total = (uint64_t)((rows + 15u) & ~15u) * (K >> 3);
    k_repack_frag16<<<(unsigned)((total + 255u) / 256u), 256, 0, s>>>(src, dst, rows, K, total);
    VX_LAUNCHED("k_repack_frag16");
    return VX_OK;
}

}  // namespace vx
