// Prefill projection GEMM for Q8_0 weights on gfx950, token-batched (T >= 128):
//   C[t][n] = sum_k X[t][k] * W[n][k],   X as hi/lo f16 planes, W = d * q (Q8_0).
//
// Same arithmetic as k_gemm (kernels_seq.hip): the int8 quants enter the MFMA as
// exact f16, each 32-column block's partial product is scaled by its f32 block
// scale afterwards (acc += d[n][b] * sum_{k in b} q*x, matvec.comp:32-44), and X
// enters as hi + lo planes through two MFMAs. The kernel is organised around
// keeping the matrix cores fed at small token counts:
//   * workgroup tile 128 tokens x 128 weight rows, four waves of 64 x 64 (2 x 2
//     v_mfma_f32_32x32x16_f16 tiles per plane), two workgroups per CU, so each
//     SIMD holds two waves and one's VALU work (quant widening, scale FMAs)
//     runs under the other's MFMAs;
//   * both operands are stored for this kernel: the weights in the prefill
//     layout (PrefillMatrix, repacked once per model) and X in the tiled plane
//     layout (tiled_plane_index, written so by the producers). A k-stage is one
//     32-column Q8_0 block, and its operands are contiguous pieces: 8 KB per X
//     plane, 4 KB of quants, 512 B of scales. Each wave copies six pieces per
//     stage global -> LDS by the DMA path (global_load_lds: no registers, no
//     VALU, every fetched byte used) into a ring of kStages LDS slots,
//     kStages - 1 stages ahead of the one being multiplied;
//   * the quants stay 8-bit in LDS (stored as q + 128; a quarter of the f16
//     footprint, which is what fits two workgroups per CU) and are widened when
//     a wave reads its B fragment;
//   * both layouts carry a permutation so every fragment read from LDS is free
//     of bank conflicts (for 32 and for 64 banks) after a verbatim copy;
//   * the VALU work of a block (64 scale FMAs and the quant widening per lane)
//     is as long as its 16 MFMAs and a wave issues both in order, so the block
//     loop is unrolled over the ring slots (constant LDS offsets, no address
//     VALU), the DMA addresses are scalar, and the block is split by output
//     half so that scale FMAs and widening issue between MFMAs;
//   * the epilogue stages the results in the ring's LDS and writes them with
//     16-byte stores of contiguous runs (split-K partial slabs, plain outputs and
//     the tiled SwiGLU planes): per-workgroup timestamps on MI355X showed the
//     scattered 4-byte partial stores taking 3.8-6.1 us of a 12-58 us launch.
// Measured alternatives, slower on MI355X at T = 384: 16-column stages, one
// workgroup per CU with a deeper ring (up to 7 slots), f16 quants in LDS,
// weights as exact hi/lo f16 pairs of d*q (three MFMAs per k-step, no scale
// step), fragments prefetched a block ahead, double-buffered block products,
// split K to put two workgroups on every CU, a stream-K schedule of the
// SwiGLU tiles (equal block ranges over one or two workgroups per CU), and eight-wave
// workgroups of 64 x 32 wave tiles (two waves per SIMD from one tile, the
// gate/up rows exchanged through LDS): 5.0 ms of GEMMs per T = 384 prefill
// against 4.0 ms, the A fragments then being read from LDS by four waves each.
#include <type_traits>

#include "vx_internal.h"

namespace vx {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float acc16 __attribute__((ext_vector_type(16)));

constexpr int kBM = 128;                       // tokens per workgroup tile
constexpr int kBN = 128;                       // weight rows per workgroup tile
constexpr int kStages = 3;                     // LDS ring slots (61.5 KB: two workgroups per CU)
constexpr int kXBytes = kBM * 32 * 2;          // one plane of a stage: f16 [token][32]
constexpr int kWBytes = kBN * 32;              // int8 quants [row][32]
constexpr int kDBytes = kBN * 4;               // f32 scales [row]
constexpr int kXOff = 0, kWOff = 2 * kXBytes, kDOff = kWOff + kWBytes;
constexpr int kStageBytes = kDOff + kDBytes;   // 20992
constexpr int kOpsPerStage = 6;                // DMA instructions per wave per stage

// Chunk permutations of the stored layouts: X rows of 64 bytes in 16-byte
// chunks (tiled_plane_index), quant rows of 32 bytes in 8-byte chunks
// (PrefillMatrix); both conflict-free for 32 and for 64 LDS banks.
__device__ __forceinline__ uint32_t xperm(uint32_t t) { return ((t >> 1) ^ (t >> 3)) & 3u; }
__device__ __forceinline__ uint32_t wperm(uint32_t n) { return ((n >> 2) ^ (n >> 4)) & 3u; }

// Four stored quants u = q + 128 (one dword) -> four exact f16 values q: the f16
// with bits 0x6400 | u is 1024 + u, minus 1152 = q.
__device__ __forceinline__ uint2 q8x4_to_f16(uint32_t u) {
    const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);
    const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);
    const h2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    const h2v a = __builtin_bit_cast(h2v, lo) - bias;
    const h2v b = __builtin_bit_cast(h2v, hi) - bias;
    return make_uint2(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b));
}

__device__ __forceinline__ acc16 mfma(h8 a, h8 b, acc16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Weight row of tile row rho (as k_gemm's tile_row): SwiGLU tiles interleave 32
// gate rows and the same 32 up rows, so one lane holds g and u of one row.
template <int EPI>
__device__ __forceinline__ uint32_t tile_row(uint32_t tn, uint32_t tile0, uint32_t rho) {
    if constexpr (EPI == GEPI_SWIGLU)
        return 64u * tn + 32u * (rho >> 6) + (rho & 31u);
    else
        return (tn - tile0) * kBN + rho;
}

// s_waitcnt vmcnt(N) (expcnt at its maximum; lgkmcnt 0 when LGKM0, else at its
// maximum), gfx9 encoding.
template <int N, bool LGKM0 = false>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | ((LGKM0 ? 0 : 15) << 8));
}

// LDS DMA, issued from asm: the compiler then does not model these as LDS
// writes, so it adds no waits of its own before LDS reads (it cannot tell ring
// slots apart reliably and would drain every DMA in flight). The ring protocol
// orders them instead: a slot is read only after wait_vm<> has retired its DMA
// and a barrier, and refilled only after a barrier that follows its last read.
// `lds` is the LDS byte address of lane 0's destination (wave-uniform, in M0);
// lane i writes at lds + i * size.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
// The global address is a wave-uniform base in an SGPR pair plus a per-lane
// 32-bit offset, so advancing a stream by one block is scalar arithmetic. (An
// LDS DMA may not read M0 in the instruction right after the write: one wait
// state between them.)
__device__ __forceinline__ void dma16(const uint8_t *base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}
__device__ __forceinline__ void dma4(const uint8_t *base, uint32_t voff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}
// A pointer that is the same in every lane, made explicitly wave-uniform.
__device__ __forceinline__ const uint8_t *uniform_ptr(const void *p) {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const uint8_t *>(((uint64_t)hi << 32) | lo);
}

// Stage b (32-column block) of the tile: wave w copies X pieces 4w .. 4w + 3
// (1 KB each, plane = piece / 8), quant piece w (1 KB), and one 256 B half of
// the scales (waves 2 and 3 repeat what waves 0 and 1 copy). Bases are the
// wave's pieces at block 0; lane i adds 16 i (4 i for the scales).
struct Src {
    const uint8_t *x[4];   // X plane piece
    const uint8_t *w;      // quants + 1024 * wave
    const uint8_t *d;      // scales + 256 * (wave & 1)
};

__device__ __forceinline__ void issue_stage(const Src &src, uint32_t blk, uint32_t slot, uint32_t wave,
                                            uint32_t lane) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t u = 4u * wave + (uint32_t)j;
        dma16(src.x[j] + (size_t)blk * kXBytes, 16u * lane, slot + kXOff + (u >> 3) * kXBytes + (u & 7u) * 1024u);
    }
    dma16(src.w + (size_t)blk * kWBytes, 16u * lane, slot + kWOff + wave * 1024u);
    dma4(src.d + (size_t)blk * kDBytes, 4u * lane, slot + kDOff + (wave & 1u) * 256u);
}

// The LDS ring of the block loop; the epilogues stage their results in it too.
__device__ __forceinline__ uint8_t *gemm_ring() {
    __shared__ __attribute__((aligned(16))) uint8_t ring[kStages * kStageBytes];
    return ring;
}

// Blocks kb0 .. kb0 + nkb - 1 (nkb >= 1) of tile (tn, tm) of segment sg into acc
// (overwritten). Every DMA of the wave has landed when this returns; the ring is
// reused only after a barrier (other waves may still read their last block).
template <int EPI>
__device__ __forceinline__ void tile_blocks(const GemmArgs &a, const GemmSeg &sg, uint32_t tn, uint32_t tm,
                                            uint32_t kb0, uint32_t nkb, acc16 (&acc)[2][2]) {
    uint8_t *const ring = gemm_ring();
    const uint32_t ring_lds = lds_addr(ring);
    const uint32_t nblk = a.K / 32u;

    const uint32_t tid = threadIdx.x, lane = tid & 63u, l32 = lane & 31u, hs = lane >> 5;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave & 1u, wn = wave >> 1;

    // ---- DMA sources of this tile at block 0 (wave-uniform bases)
    Src src;
    {
        const uint32_t lt = EPI == GEPI_SWIGLU ? tn : tn - sg.tile0;   // tile within the matrix
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t u = 4u * wave + (uint32_t)j;
            const uint8_t *plane = reinterpret_cast<const uint8_t *>((u >> 3) ? a.xl : a.xh);
            src.x[j] = uniform_ptr(plane + ((size_t)tm * nblk) * kXBytes + (u & 7u) * 1024u);
        }
        src.w = uniform_ptr(reinterpret_cast<const uint8_t *>(sg.pq) + ((size_t)lt * nblk) * kWBytes + 1024u * wave);
        src.d = uniform_ptr(reinterpret_cast<const uint8_t *>(sg.pd) + ((size_t)lt * nblk) * kDBytes +
                            256u * (wave & 1u));
    }

    // ---- fragment addresses inside a stage slot: k-step e covers columns
    // 16e .. 16e + 15 of the block; this lane takes 8 of them, chunk 2e + hs.
    uint32_t xa[2][2];   // [mt][e] (plane hi; lo is + kXBytes)
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const uint32_t t = 64u * wm + 32u * (uint32_t)mt + l32;
#pragma unroll
        for (int e = 0; e < 2; ++e) xa[mt][e] = kXOff + t * 64u + (((2u * (uint32_t)e + hs) ^ xperm(t)) * 16u);
    }
    uint32_t wa[2][2], da[2];   // [nt][e] quant dword pair, [nt] scale
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const uint32_t n = 64u * wn + 32u * (uint32_t)nt + l32;
#pragma unroll
        for (int e = 0; e < 2; ++e) wa[nt][e] = kWOff + n * 32u + (((2u * (uint32_t)e + hs) ^ wperm(n)) * 8u);
        da[nt] = kDOff + n * 4u;
    }

    // ---- prologue: blocks 0 .. kStages-2 (indices clamped: always the same
    // number of DMA instructions per stage, which the vmcnt waits count on)
#pragma unroll
    for (int s = 0; s < kStages - 1; ++s)
        issue_stage(src, kb0 + ((uint32_t)s < nkb ? (uint32_t)s : nkb - 1u), ring_lds + (uint32_t)s * kStageBytes, wave,
                    lane);

    acc16 p[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = p[i][j] = acc16{};
    float dprev1 = 0.f;   // scale of the previous block's second output half

    // One block in ring slot SL (compile-time, so every LDS address is a base
    // register plus an immediate): wait for its DMA, refill the slot consumed
    // last, read the fragments, then
    //   widen the quants of output half 0;
    //   MFMAs of half 0, interleaved with the previous block's half-1 scale FMAs
    //   (acc += d * p) and the widening of half 1;
    //   MFMAs of half 1, interleaved with this block's half-0 scale FMAs.
    // A wave issues VALU and MFMA work in order, so this keeps its VALU work in
    // the gaps between matrix instructions; half 1's scale FMAs wait for the
    // next block (or the end of the loop).
    auto block = [&](uint32_t it, auto slot_c) {
        constexpr uint32_t SL = decltype(slot_c)::value;
        __builtin_amdgcn_sched_barrier(0);
        wait_vm<kOpsPerStage * (kStages - 2), true>();
        __builtin_amdgcn_s_barrier();
        const uint32_t nxt = it + kStages - 1u;
        issue_stage(src, kb0 + (nxt < nkb ? nxt : nkb - 1u), ring_lds + ((SL + kStages - 1u) % kStages) * kStageBytes,
                    wave, lane);
        const uint8_t *slot = ring + SL * kStageBytes;
        uint2 q[2][2];
        h8 ah[2][2], al[2][2], bf[2][2];   // [e][nt], [e][mt], [e][mt], [e][nt]
#pragma unroll
        for (int e = 0; e < 2; ++e) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) q[e][nt] = *reinterpret_cast<const uint2 *>(slot + wa[nt][e]);
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                ah[e][mt] = *reinterpret_cast<const h8 *>(slot + xa[mt][e]);
                al[e][mt] = *reinterpret_cast<const h8 *>(slot + xa[mt][e] + kXBytes);
            }
        }
        const float d0 = *reinterpret_cast<const float *>(slot + da[0]);
        const float d1 = *reinterpret_cast<const float *>(slot + da[1]);
        auto widen = [&](int nt) {
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const uint2 f0 = q8x4_to_f16(q[e][nt].x), f1 = q8x4_to_f16(q[e][nt].y);
                bf[e][nt] = __builtin_bit_cast(h8, make_uint4(f0.x, f0.y, f1.x, f1.y));
            }
        };
        auto mfmas = [&](int nt) {   // no two dependent MFMAs adjacent
#pragma unroll
            for (int e = 0; e < 2; ++e) {
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) p[mt][nt] = mfma(ah[e][mt], bf[e][nt], e == 0 ? acc16{} : p[mt][nt]);
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) p[mt][nt] = mfma(al[e][mt], bf[e][nt], p[mt][nt]);
            }
        };
        auto scale = [&](int nt, float d) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[mt][nt][r] = fmaf(d, p[mt][nt][r], acc[mt][nt][r]);
        };
        widen(0);
        __builtin_amdgcn_sched_barrier(0);
        scale(1, dprev1);   // reads p[.][1] before this block's half-1 MFMAs rewrite it
        widen(1);
        mfmas(0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);   // then six VALU
        }
        __builtin_amdgcn_sched_barrier(0);
        scale(0, d0);
        mfmas(1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);
        }
        dprev1 = d1;
    };
    static_assert(kStages == 3, "the block loop is unrolled over three ring slots");
    uint32_t it = 0;
    for (; it + 3u <= nkb; it += 3u) {
        block(it, std::integral_constant<uint32_t, 0>{});
        block(it + 1u, std::integral_constant<uint32_t, 1>{});
        block(it + 2u, std::integral_constant<uint32_t, 2>{});
    }
    if (it < nkb) block(it, std::integral_constant<uint32_t, 0>{});
    if (it + 1u < nkb) block(it + 1u, std::integral_constant<uint32_t, 1>{});
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[mt][1][r] = fmaf(dprev1, p[mt][1][r], acc[mt][1][r]);
    // Drain the DMA of the clamped trailing stages before the workgroup ends.
    wait_vm<0>();
}

// Accumulator layout: lane (l32, hs) of wave (wm, wn) holds, for tile (mt, nt),
// tile row rho = 64wn + 32nt + l32 and tokens m0 + 64wm + 32mt + 8(r/4) + 4hs + r%4.
// SwiGLU tiles interleave 32 gate rows (nt = 0) with the same 32 up rows (nt = 1),
// so output column 64tn + 32wn + l32 is silu(acc[.][0]) * acc[.][1].

// SwiGLU output to tiled planes: each 32-column group of the tile is one
// contiguous 8 KB block per plane in that layout, built in LDS and copied out
// whole with 16-byte stores. Token rows past T (the last tile's padding) get
// zeros. Every thread of the workgroup calls it (barriers inside).
__device__ __forceinline__ void swiglu_planes(const GemmArgs &a, uint32_t tn, uint32_t m0, const acc16 (&acc)[2][2]) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, l32 = lane & 31u, hs = lane >> 5;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave & 1u, wn = wave >> 1;
    _Float16 *const st = reinterpret_cast<_Float16 *>(gemm_ring());   // [plane][group][128][32]
    __syncthreads();   // ring idle: every wave has drained its DMA and read its last block
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t ti = 64u * wm + 32u * (uint32_t)mt + 8u * (uint32_t)(r >> 2) + 4u * hs + (uint32_t)(r & 3);
            const float g = acc[mt][0][r], u = acc[mt][1][r];
            const float v = m0 + ti < a.T ? g / (1.0f + expf(-g)) * u : 0.f;   // matvec_swiglu.comp:67
            const _Float16 hv = (_Float16)v;
            const uint32_t o =
                (wn * 128u + ti) * 32u + 8u * ((l32 >> 3) ^ (((ti >> 1) ^ (ti >> 3)) & 3u)) + (l32 & 7u);
            st[o] = hv;
            st[2u * 128u * 32u + o] = (_Float16)(v - (float)hv);
        }
    __syncthreads();
#pragma unroll
    for (uint32_t i = tid; i < 4u * 512u; i += 256u) {
        const uint32_t blk = i / 512u, j = i % 512u;   // block = (plane, group); 512 chunks of 16 bytes
        const uint32_t col0 = 64u * tn + 32u * (blk & 1u);
        if (col0 >= a.seg[0].rows) continue;
        __half *const dst = ((blk >> 1) ? a.ol : a.oh) + tiled_plane_index(m0, col0, a.ldp);
        *reinterpret_cast<uint4 *>(dst + 8u * j) = *reinterpret_cast<const uint4 *>(st + blk * 4096u + 8u * j);
    }
}

// SwiGLU output with per-element stores: the f32 output and/or row-major planes.
// Stores only (no loads): a load here would make every element wait for the
// stores before it.
__device__ __forceinline__ void swiglu_scalar(const GemmArgs &a, uint32_t tn, uint32_t m0, const acc16 (&acc)[2][2]) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, l32 = lane & 31u, hs = lane >> 5;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t wm = wave & 1u, wn = wave >> 1;
    float *const out0 = a.seg[0].out;
    const uint32_t ldo0 = a.seg[0].ldo;
    const uint32_t row = tile_row<GEPI_SWIGLU>(tn, 0, 64u * wn + l32);
    if (row >= a.seg[0].rows) return;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
        const uint32_t tbase = m0 + 64u * wm + 32u * (uint32_t)mt + 4u * hs;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const uint32_t tok = tbase + 8u * (uint32_t)(r >> 2) + (uint32_t)(r & 3);
            if (tok >= a.T) continue;
            const float g = acc[mt][0][r], u = acc[mt][1][r];
            const float v = g / (1.0f + expf(-g)) * u;   // matvec_swiglu.comp:67
            if (out0) out0[(size_t)tok * ldo0 + row] = v;
            if (a.oh) {
                const size_t o = a.o_tiled ? tiled_plane_index(tok, row, a.ldp) : (size_t)tok * a.ldp + row;
                const _Float16 hv = (_Float16)v;
                a.oh[o] = __builtin_bit_cast(__half, hv);
                a.ol[o] = __builtin_bit_cast(__half, (_Float16)(v - (float)hv));
            }
        }
    }
}

template <int EPI>
__global__ __launch_bounds__(256, 2) void k_gemm_q8p(GemmArgs a) {
    // XCD-major order: workgroup b runs on XCD b % 8; consecutive ids of one XCD
    // cover the token tiles of the same weight rows.
    const uint32_t b = blockIdx.x;
    const uint32_t id = (b & 7u) * (gridDim.x >> 3) + (b >> 3);
    const uint32_t per_split = a.ntn * a.ntm;
    if (id >= per_split * a.ksplit) return;
    const uint32_t ks = id / per_split, rem = id - ks * per_split;
    const uint32_t tn = rem / a.ntm, tm = rem - tn * a.ntm;
    const uint32_t m0 = tm * kBM;
    uint32_t seg = 0;
    if constexpr (EPI != GEPI_SWIGLU) {
        while (seg + 1 < a.nseg && tn >= a.seg[seg + 1].tile0) ++seg;
    }
    const GemmSeg &sg = a.seg[seg];
    const uint32_t nblk = a.K / 32u;
    const uint32_t kb0 = ks * nblk / a.ksplit, kb1 = (ks + 1u) * nblk / a.ksplit;
    if (kb1 == kb0) return;   // nothing to add (ksplit is clamped to the block count)

    acc16 acc[2][2];
    tile_blocks<EPI>(a, sg, tn, tm, kb0, kb1 - kb0, acc);

    if constexpr (EPI == GEPI_SWIGLU) {
        if (a.o_tiled && a.oh && !a.seg[0].out)
            swiglu_planes(a, tn, m0, acc);
        else
            swiglu_scalar(a, tn, m0, acc);
    } else {
        const uint32_t tid = threadIdx.x, lane = tid & 63u, l32 = lane & 31u, hs = lane >> 5;
        const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
        const uint32_t wm = wave & 1u, wn = wave >> 1;
        float *const out0 = sg.out;
        const uint32_t ldo0 = sg.ldo, rows0 = sg.rows;
        // Plain stores (a whole product, or one split's partial slab) go through
        // LDS (the ring is free once every wave has drained its DMA) in two passes
        // of 64 tokens and leave as 16-byte stores, 512 contiguous bytes per token
        // row, instead of 4-byte stores scattered over every lane's 64 results.
        const bool plain =
            EPI == GEPI_STORE ? (a.ksplit == 1u || a.split_store != 0u) : (a.ws != nullptr && a.ksplit > 1u);
        if (plain && a.wide) {
            float *const base = EPI == GEPI_STORE ? out0 + (a.ksplit > 1u ? ks * a.ws_stride : 0u)
                                                  : a.ws + ks * a.ws_stride;
            const float f = EPI == GEPI_STORE ? a.alpha : a.scale;
            float *const st = reinterpret_cast<float *>(gemm_ring());
            constexpr uint32_t kLd = kBN + 8;   // staging row: the two half-waves' tokens 32 banks apart
            const uint32_t row_base = tile_row<EPI>(tn, sg.tile0, 0);
#pragma unroll
            for (uint32_t pass = 0; pass < 2u; ++pass) {
                __syncthreads();   // ring (pass 0) or the previous pass's reads are done
                if (wm == pass) {
#pragma unroll
                    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                        for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                            for (int r = 0; r < 16; ++r)
                                st[(32u * mt + 8u * (uint32_t)(r >> 2) + 4u * hs + (uint32_t)(r & 3)) * kLd +
                                   64u * wn + 32u * nt + l32] = acc[mt][nt][r] * f;
                }
                __syncthreads();
#pragma unroll
                for (uint32_t i = tid; i < 64u * (kBN / 4u); i += 256u) {
                    const uint32_t tl = i / (kBN / 4u), c4 = i % (kBN / 4u);
                    const uint32_t tok = m0 + 64u * pass + tl, row = row_base + 4u * c4;
                    if (tok < a.T && row < rows0)
                        *reinterpret_cast<float4 *>(base + (size_t)tok * ldo0 + row) =
                            *reinterpret_cast<const float4 *>(st + tl * kLd + 4u * c4);
                }
            }
            return;
        }
        // Per-element epilogue: stores and atomics only (no loads). Residual adds
        // are atomic adds, which with one contributor (no split) give exactly
        // h + v; split residual products go to the partial workspace when one is
        // given.
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const uint32_t tbase = m0 + 64u * wm + 32u * (uint32_t)mt + 4u * hs;
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const uint32_t row = tile_row<EPI>(tn, sg.tile0, 64u * wn + 32u * (uint32_t)nt + l32);
                if (row >= rows0) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t tok = tbase + 8u * (uint32_t)(r >> 2) + (uint32_t)(r & 3);
                    if (tok >= a.T) continue;
                    float *dst = out0 + (size_t)tok * ldo0 + row;
                    if constexpr (EPI == GEPI_STORE) {
                        const float v = acc[mt][nt][r] * a.alpha;
                        if (a.ksplit == 1)
                            *dst = v;
                        else if (a.split_store)
                            dst[ks * a.ws_stride] = v;
                        else
                            unsafeAtomicAdd(dst, v);
                    } else if (a.ws && a.ksplit > 1) {
                        a.ws[ks * a.ws_stride + (size_t)tok * ldo0 + row] = acc[mt][nt][r] * a.scale;
                    } else {
                        unsafeAtomicAdd(dst, acc[mt][nt][r] * a.scale);
                    }
                }
            }
        }
    }
}

// A tile part in a slot: element (i, j, r) of thread t at float (32i + 16j + r) * 256 + t,
// so every store or load of a wave covers 256 contiguous bytes.
//
// How a part passes between workgroups, and the hardware property it rests on:
// the part is written with agent-scope relaxed atomic stores, the writer waits for
// their acknowledgements (s_waitcnt 0) before its counter atomic, and the reader,
// once it has seen the count, reads the part with agent-scope relaxed atomic loads.
// The HIP memory model gives relaxed atomics no ordering: a release on the count
// and an acquire on its read would. This code instead relies on how LLVM compiles
// agent-scope atomics for gfx942/gfx950 (AMDGPUUsage, "Memory Model GFX942"):
// loads and stores carry sc1, so they bypass the non-coherent per-XCD L2 and are
// performed at the device-coherent level, and a store's acknowledgement means it
// is visible there (checked in this build's ISA: global_store/global_load ... sc1).
// The release/acquire pair would add an L2 write-back (buffer_wbl2 sc1) and an L2
// invalidation (buffer_inv sc1); measured on MI355X inside a decode-size kernel
// the release alone cost about 5 us per hand-off against 1.3 us for this protocol.
// Keep every access to a part an agent-scope atomic: a plain store or load here
// would break the hand-off without any error. The bit-exact test of both hand-off
// orders (VX_PREFILL_STREAMK_TAIL_FIRST) is the guard.
__device__ __forceinline__ void sk_store(float *slot, const acc16 (&acc)[2][2]) {
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                __hip_atomic_store(slot + (size_t)(32 * i + 16 * j + r) * 256u + tid, acc[i][j][r], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0);   // every part store acknowledged before the count
    __syncthreads();
}
__device__ __forceinline__ void sk_add(const float *slot, acc16 (&acc)[2][2]) {
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                acc[i][j][r] += __hip_atomic_load(slot + (size_t)(32 * i + 16 * j + r) * 256u + tid, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
}

// Stream-K schedule of the SwiGLU tiles, for a tile count a little above the
// CU count (which would leave a few CUs a second whole tile): the sequence of
// (tile, block) pairs, tile major, is cut into gridDim.x equal ranges of
// a.sk_per > K/32 blocks, one workgroup (one CU) each, so a tile is shared by at
// most two neighbouring workgroups: its head ends the range of workgroup w and
// its tail starts that of w + 1. A workgroup first computes the head it holds and
// stores it to its slot (device-scope stores, past the XCD's L2), acknowledged
// before it counts itself on the counter of boundary w; then its whole tiles;
// last the tail it holds, by which time the previous workgroup's head is normally
// stored: the counter says so, and the tail adds that head (device-scope loads)
// and runs the epilogue. If the head is not there yet, the tail stores itself and
// counts, and whichever of the two counts second finishes the tile and clears the
// counter. Nothing waits on another workgroup, and fp32 addition of the two parts
// commutes, so the result does not depend on which finishes. TAIL_FIRST computes
// the tail first, so the store-and-count path runs every time (same result bits).
template <bool TAIL_FIRST>
__global__ __launch_bounds__(256, 2) void k_gemm_q8p_sk(GemmArgs a) {
    __shared__ uint32_t flag;
    const uint32_t b = blockIdx.x;
    const uint32_t id = (b & 7u) * (gridDim.x >> 3) + (b >> 3);   // XCD-major, as k_gemm_q8p
    const uint32_t nblk = a.K / 32u;
    const uint32_t total = a.ntn * a.ntm * nblk;
    const uint32_t g0 = min(id * a.sk_per, total), g1 = min(g0 + a.sk_per, total);
    if (g0 >= g1) return;
    const uint32_t tid = threadIdx.x;
    const uint32_t t_first = g0 / nblk, t_last = (g1 - 1u) / nblk;
    const uint32_t tail_kb = g0 % nblk, head_n = g1 % nblk;   // 0: the range starts / ends on a tile edge
    auto slot = [&](uint32_t w, uint32_t part) { return a.sk_ws + ((size_t)w * 2u + part) * kSkTileFloats; };
    const bool has_head = head_n != 0u, has_tail = tail_kb != 0u;
    bool first = true;
    auto run = [&](uint32_t tile, uint32_t kb, uint32_t n, acc16 (&acc)[2][2]) {
        if (!first) __syncthreads();   // the previous piece's ring and staging reads are done
        first = false;
        const uint32_t tn = tile / a.ntm, tm = tile - tn * a.ntm;
        tile_blocks<GEPI_SWIGLU>(a, a.seg[0], tn, tm, kb, n, acc);
    };
    auto finish = [&](uint32_t tile, const acc16 (&acc)[2][2]) {
        const uint32_t tn = tile / a.ntm;
        swiglu_planes(a, tn, (tile - tn * a.ntm) * kBM, acc);
    };
    auto head = [&]() {   // the head of tile t_last; its tail starts range id + 1
        acc16 acc[2][2];
        run(t_last, 0u, head_n, acc);
        sk_store(slot(id, 1u), acc);
        if (tid == 0) flag = atomicAdd(a.sk_cnt + id, 1u);
        __syncthreads();
        if (flag != 0u) {   // the tail is stored already: finish the tile here
            sk_add(slot(id + 1u, 0u), acc);
            if (tid == 0) __hip_atomic_store(a.sk_cnt + id, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            finish(t_last, acc);
        }
    };
    auto tail = [&]() {   // the tail of tile t_first; its head ends range id - 1
        acc16 acc[2][2];
        run(t_first, tail_kb, nblk - tail_kb, acc);
        const uint32_t bnd = id - 1u;
        if (tid == 0) flag = __hip_atomic_load(a.sk_cnt + bnd, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        bool done_here = flag != 0u;
        if (!done_here) {   // the head is still being computed: store, count, and see who is second
            sk_store(slot(id, 0u), acc);
            if (tid == 0) flag = atomicAdd(a.sk_cnt + bnd, 1u);
            __syncthreads();
            done_here = flag != 0u;
        }
        if (done_here) {
            sk_add(slot(bnd, 1u), acc);
            if (tid == 0) __hip_atomic_store(a.sk_cnt + bnd, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            finish(t_first, acc);
        }
    };
    auto whole = [&]() {
        const uint32_t full0 = has_tail ? t_first + 1u : t_first, full1 = has_head ? t_last : t_last + 1u;
        for (uint32_t tile = full0; tile < full1; ++tile) {
            acc16 acc[2][2];
            run(tile, 0u, nblk, acc);
            finish(tile, acc);
        }
    };
    if constexpr (TAIL_FIRST) {
        if (has_tail) tail();
        if (has_head) head();
        whole();
    } else {
        if (has_head) head();
        whole();
        if (has_tail) tail();
    }
}

// Gate/up tiles between 1.25 and 1.5 per CU (T = 385..512 for the 6144-row FFN
// on 256 CUs): the first a.sk_grid tiles run whole, one workgroup each, and every
// other tile runs as two K halves in two workgroups, which the dispatcher places
// in the second workgroup slot of the CUs (blocks are dispatched in order), so a
// CU runs a whole tile and at most one half side by side instead of up to two
// whole tiles. The halves of a tile (on one XCD) store their parts, count on the
// tile's counter, and the second to count adds the other part and runs the
// epilogue, then clears the counter; nothing waits, and the sum commutes.
__global__ __launch_bounds__(256, 2) void k_gemm_q8p_half(GemmArgs a) {
    __shared__ uint32_t flag;
    const uint32_t b = blockIdx.x, G = a.sk_grid, nblk = a.K / 32u;
    const uint32_t tid = threadIdx.x;
    uint32_t tile, kb0, nkb, hid = 0;
    const bool half = b >= G;
    if (!half) {
        tile = (b & 7u) * (G >> 3) + (b >> 3);   // XCD-major over the whole tiles
        kb0 = 0u;
        nkb = nblk;
    } else {
        const uint32_t h = b - G, H = gridDim.x - G;   // H % 16 == 0: a tile's halves on one XCD
        hid = (h & 7u) * (H >> 3) + (h >> 3);
        tile = G + (hid >> 1);
        kb0 = (hid & 1u) ? nblk / 2u : 0u;
        nkb = (hid & 1u) ? nblk - nblk / 2u : nblk / 2u;
    }
    const uint32_t tn = tile / a.ntm, tm = tile - tn * a.ntm;
    acc16 acc[2][2];
    tile_blocks<GEPI_SWIGLU>(a, a.seg[0], tn, tm, kb0, nkb, acc);
    if (half) {
        uint32_t *const cnt = a.sk_cnt + (hid >> 1);
        sk_store(a.sk_ws + (size_t)hid * kSkTileFloats, acc);
        if (tid == 0) flag = atomicAdd(cnt, 1u);
        __syncthreads();
        if (flag == 0u) return;   // the other half finishes the tile
        sk_add(a.sk_ws + (size_t)(hid ^ 1u) * kSkTileFloats, acc);
        if (tid == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    swiglu_planes(a, tn, tm * kBM, acc);
}

// One thread per 32-byte quant row piece (tile, block b, row n) of the output.
__global__ __launch_bounds__(256) void k_repack_prefill(const uint8_t *raw, uint32_t off0, uint32_t off1,
                                                        uint32_t rows, uint32_t K, int interleave, uint64_t total,
                                                        int8_t *q, float *d) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i >= total) return;
    const uint32_t nb = K / 32u;
    const uint32_t n = (uint32_t)(i & 127u), blk = (uint32_t)((i >> 7) % nb), tile = (uint32_t)((i >> 7) / nb);
    const uint32_t r_out = 128u * tile + n;
    uint32_t mat = 0, row = r_out;
    if (interleave) {
        mat = (r_out >> 5) & 1u;
        row = 32u * (r_out >> 6) + (r_out & 31u);
    }
    const bool live = row < rows;
    const uint8_t *b = raw + (mat ? off1 : off0) + ((size_t)(live ? row : 0u) * nb + blk) * 34u;
    const uint32_t g = wperm(n);
    uint32_t w[8];   // stored chunk sc holds source chunk sc ^ g, each byte q + 128
#pragma unroll
    for (int sc = 0; sc < 4; ++sc) {
        const uint32_t src = 2u + 8u * ((uint32_t)sc ^ g);
        const uint32_t lo = b[src] | (b[src + 1] << 8) | (b[src + 2] << 16) | ((uint32_t)b[src + 3] << 24);
        const uint32_t hi = b[src + 4] | (b[src + 5] << 8) | (b[src + 6] << 16) | ((uint32_t)b[src + 7] << 24);
        w[2 * sc] = (live ? lo : 0u) ^ 0x80808080u;
        w[2 * sc + 1] = (live ? hi : 0u) ^ 0x80808080u;
    }
    uint4 *dst = reinterpret_cast<uint4 *>(q + i * 32u);
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
    d[((size_t)tile * nb + blk) * 128u + n] =
        live ? (float)__builtin_bit_cast(_Float16, (unsigned short)(b[0] | (b[1] << 8))) : 0.f;
}

}  // namespace

uint32_t gemm_q8p_tile_tokens() { return kBM; }

bool gemm_q8p_eligible(const GemmArgs &a) {
    if (a.wk != WT_Q8 || a.xf32 || !a.x_tiled || a.T == 0 || a.K % 32u) return false;
    const uint32_t nseg = a.epi == GEPI_SWIGLU ? 1u : a.nseg;
    for (uint32_t i = 0; i < nseg; ++i)
        if (!a.seg[i].pq || !a.seg[i].pd || a.seg[i].bias) return false;   // no bias epilogue here
    return true;
}

uint64_t prefill_matrix_bytes(uint32_t rows_out, uint32_t K) {
    const uint64_t rp = (rows_out + 127u) / 128u * 128u;
    return rp * K + rp * (K / 32u) * 4u;
}

int launch_repack_prefill(hipStream_t s, const uint8_t *raw, uint32_t off0, uint32_t off1, uint32_t rows,
                          uint32_t K, int interleave, int8_t *q, float *d) {
    if (K % 32u || !raw || !q || !d) return fail(VX_ERR_INVALID_ARG, "prefill repack: K %% 32 and buffers");
    if (interleave && rows % 32u) return fail(VX_ERR_INVALID_ARG, "prefill repack: interleaved rows %% 32");
    const uint32_t rows_out = interleave ? 2u * rows : rows;
    const uint64_t rp = (rows_out + 127u) / 128u * 128u;
    const uint64_t total = rp * (K / 32u);
    k_repack_prefill<<<(unsigned)((total + 255u) / 256u), 256, 0, s>>>(raw, off0, off1, rows, K, interleave, total, q,
                                                                        d);
    VX_LAUNCHED("k_repack_prefill");
    return VX_OK;
}

// Called by launch_gemm with validated arguments; sets the tiling fields.
// For GEPI_SWIGLU, seg[0].pq/pd hold the interleaved gate/up matrix.
int launch_gemm_q8p(hipStream_t s, GemmArgs a) {
    uint32_t tiles = 0;
    if (a.epi == GEPI_SWIGLU) {
        tiles = (a.seg[0].rows + 63u) / 64u;
        if (a.oh && a.o_tiled && a.ldp % 32u) return fail(VX_ERR_INVALID_ARG, "gemm: tiled output width %% 32");
    } else {
        for (uint32_t i = 0; i < a.nseg; ++i) {
            a.seg[i].tile0 = tiles;
            tiles += (a.seg[i].rows + kBN - 1u) / kBN;
        }
    }
    const uint32_t nblk = a.K / 32u;
    if (a.ksplit == 0) a.ksplit = 1;
    if (a.ksplit > nblk) a.ksplit = nblk;
    a.ntn = tiles;
    a.ntm = (a.T + kBM - 1u) / kBM;
    const uint64_t total = (uint64_t)a.ntn * a.ntm * a.ksplit;
    if (total == 0) return VX_OK;
    const uint64_t grid = (total + 7u) / 8u * 8u;
    if (grid > 0x7fffffffull) return fail(VX_ERR_UNSUPPORTED, "gemm: grid too large");
    const uint64_t tiles_all = (uint64_t)a.ntn * a.ntm;
    if (a.epi == GEPI_SWIGLU && a.sk_ws && a.sk_cnt && a.sk_grid >= 8u && a.sk_grid % 8u == 0u && a.o_tiled &&
        a.oh && !a.seg[0].out && tiles_all > a.sk_grid && tiles_all * 4u <= (uint64_t)a.sk_grid * 5u &&
        tiles_all * nblk <= 0xffffffffull) {
        // Stream-K: more tiles than workgroups, so every range is longer than a
        // tile (at most two workgroups share one; a range that ends inside a tile
        // has a successor, one that starts inside one a predecessor), and at most
        // 1.25 tiles per CU, where the second-tile imbalance is worth removing
        // (from 1.5 up, two resident workgroups per CU do better).
        a.sk_per = (uint32_t)((tiles_all * nblk + a.sk_grid - 1u) / a.sk_grid);
        if (a.sk_tail_first)
            k_gemm_q8p_sk<true><<<a.sk_grid, 256, 0, s>>>(a);
        else
            k_gemm_q8p_sk<false><<<a.sk_grid, 256, 0, s>>>(a);
        VX_LAUNCHED("k_gemm_q8p_sk");
        return VX_OK;
    }
    if (a.epi == GEPI_SWIGLU && a.sk_ws && a.sk_cnt && a.sk_grid >= 8u && a.sk_grid % 8u == 0u && a.o_tiled &&
        a.oh && !a.seg[0].out && tiles_all * 4u > (uint64_t)a.sk_grid * 5u && tiles_all * 2u <= (uint64_t)a.sk_grid * 3u &&
        (tiles_all - a.sk_grid) % 8u == 0u && nblk >= 2u) {
        // Whole tiles for the first sk_grid, K halves for the rest: 2 (tiles - sk_grid)
        // <= sk_grid halves (a multiple of 16, so a tile's halves share an XCD), at
        // most one per CU beside its whole tile; a part slot per half, a counter per
        // split tile.
        const uint32_t halves = 2u * (uint32_t)(tiles_all - a.sk_grid);
        k_gemm_q8p_half<<<a.sk_grid + halves, 256, 0, s>>>(a);
        VX_LAUNCHED("k_gemm_q8p_half");
        return VX_OK;
    }
    // 16-byte epilogue stores need every output row start and slab 16-byte aligned.
    a.wide = (a.ws_stride % 4u == 0u && reinterpret_cast<uintptr_t>(a.ws) % 16u == 0u) ? 1u : 0u;
    if (a.epi != GEPI_SWIGLU)
        for (uint32_t i = 0; i < a.nseg; ++i)
            if (a.seg[i].rows % 4u || a.seg[i].ldo % 4u || reinterpret_cast<uintptr_t>(a.seg[i].out) % 16u) a.wide = 0;
    switch (a.epi) {
        case GEPI_STORE: k_gemm_q8p<GEPI_STORE><<<(unsigned)grid, 256, 0, s>>>(a); break;
        case GEPI_RESIDUAL: k_gemm_q8p<GEPI_RESIDUAL><<<(unsigned)grid, 256, 0, s>>>(a); break;
        case GEPI_SWIGLU: k_gemm_q8p<GEPI_SWIGLU><<<(unsigned)grid, 256, 0, s>>>(a); break;
        default: return fail(VX_ERR_UNSUPPORTED, "gemm: epilogue %u", a.epi);
    }
    VX_LAUNCHED("k_gemm_q8p");
    return VX_OK;
}

}  // namespace vx
