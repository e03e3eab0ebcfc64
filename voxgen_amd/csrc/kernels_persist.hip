// Persistent decode step: every layer of record_transformer (baselm.rs:922-1039)
// in ONE kernel, so that the weight streaming of a phase overlaps the work of the
// phase before it.
//
// Per layer, five phases (the five kernels of the per-kernel step):
//   A  rmsnorm(h)*attn_norm -> Q/K/V rows -> RoPE -> q, k, v and the f16 KV row
//   B  split-context attention partials; the last slice of a head to finish
//      merges that head's partials into the attention vector
//   C  h += scale * Wo . attention
//   D  act = silu(Wg . n) * (Wu . n), n = rmsnorm(h)*ffn_norm
//   E  h += scale * Wdown . act
// The grid is kPersistGroups groups of one workgroup per CU. Phases are numbered
// p = 5*layer + k and group p % kPersistGroups runs phase p. A workgroup first
// issues the loads of its weight rows for its next phase (they do not depend on
// anything computed in the step), then waits until the phase before is finished,
// then reads that phase's outputs and computes. With two groups the weights of
// phase p stream in while phase p-1 runs on the other group (each wave's load
// counter retires in order, so that overlap needs a second group); measured on
// MI355X this is slower than one group, because the streaming raises the latency
// of the coherent hand-offs between phases, so one group is compiled.
// Phase completion is counted on eight per-XCD counters (one cache line each)
// with device-scope atomic adds; no memory fence is issued: every value one
// workgroup hands to another inside the step (h, q/k/v, the KV row, partials,
// attention, act) is written with device-scope stores and read with device-scope
// loads, which the hardware keeps coherent across XCDs, and a workgroup waits
// for its own stores to complete before it counts itself done. Every wait is
// bounded: on timeout the kernel records an error word and all later waits fall
// through, so a fault of the protocol ends the step with an error instead of
// hanging the device. All workgroups must be resident at once (checked against
// the occupancy before the first launch).
#include <cfloat>

#include "decode_dev.h"

namespace vx {
namespace {

// ------------------------------------------------------- coherent accesses
__device__ __forceinline__ float ld_c(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_c(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float4 ld_c4(const float *p) {
    const uint64_t a = __hip_atomic_load(reinterpret_cast<const uint64_t *>(p), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t b = __hip_atomic_load(reinterpret_cast<const uint64_t *>(p) + 1, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    return make_float4(__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)),
                       __uint_as_float((uint32_t)b), __uint_as_float((uint32_t)(b >> 32)));
}
__device__ __forceinline__ void st_c16(__half *p, float v) {
    __hip_atomic_store(reinterpret_cast<unsigned short *>(p), __half_as_ushort(__float2half_rn(v)), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint4 ld_c16b(const void *p) {  // 16 bytes
    const uint64_t a = __hip_atomic_load(reinterpret_cast<const uint64_t *>(p), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    const uint64_t b = __hip_atomic_load(reinterpret_cast<const uint64_t *>(p) + 1, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
    return make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32));
}

// The layer table holds generic pointers; loads through them would be flat
// loads, which also count against the LDS wait counter and so stall every LDS
// access behind the weight stream. All of them point into global memory.
#define VX_GLOBAL __attribute__((address_space(1)))
typedef unsigned int gu32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int gu32x2 __attribute__((ext_vector_type(2)));
typedef float gf32x4 __attribute__((ext_vector_type(4)));
template <int NG>
__device__ __forceinline__ void load_row_g(Q8Row<NG> &r, const void *qs, const __half *d, uint32_t row,
                                           uint32_t cols, int lane) {
    const VX_GLOBAL int8_t *qrow = (const VX_GLOBAL int8_t *)qs + (size_t)row * cols;
    const VX_GLOBAL unsigned short *drow = (const VX_GLOBAL unsigned short *)d + (size_t)row * (cols >> 5);
#pragma unroll
    for (int g = 0; g < NG; ++g) {
        const gu32x4 q = *(const VX_GLOBAL gu32x4 *)(qrow + kGroupCols * g + 16 * lane);
        const gu32x2 d2 = *(const VX_GLOBAL gu32x2 *)(drow + 32 * g + 4 * (lane >> 3));
        r.q[g] = make_uint4(q.x, q.y, q.z, q.w);
        r.d[g] = make_uint2(d2.x, d2.y);
    }
}

// Weight rows are requested before a phase waits for the one before it. The
// compiler would sink those loads past the wait loop to their first use; an
// empty asm that takes the registers as operands keeps them ahead of it.
template <int NG>
__device__ __forceinline__ void pin(Q8Row<NG> &r) {
#pragma unroll
    for (int g = 0; g < NG; ++g)
        asm volatile("" : "+v"(r.q[g].x), "+v"(r.q[g].y), "+v"(r.q[g].z), "+v"(r.q[g].w), "+v"(r.d[g].x),
                     "+v"(r.d[g].y));
}
__device__ __forceinline__ void pin(float &v) { asm volatile("" : "+v"(v)); }

// ------------------------------------------------------------ phase counting
constexpr uint32_t kSpinLimit = 1u << 20;
constexpr uint32_t kPersistMaxSplits = 16;   // context slices per head (merged unrolled)

// This workgroup has finished phase `idx`: its stores have completed (the wait
// below), then one device-scope add on its XCD's counter.
__device__ __forceinline__ void phase_done(unsigned *cnt, uint32_t idx) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        __hip_atomic_fetch_add(&cnt[(size_t)idx * kPersistCntStride + (blockIdx.x & 7u) * 32u], 1u,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until all G workgroups have finished phase `idx` (the sum of the eight
// per-XCD counters reaches G), bounded.
__device__ __forceinline__ void phase_wait(unsigned *cnt, uint32_t idx, uint32_t G, unsigned *err) {
    if (threadIdx.x < 64) {
        const unsigned *c = cnt + (size_t)idx * kPersistCntStride;
        uint32_t spins = 0;
        while (true) {
            uint32_t v = threadIdx.x < 8 ? __hip_atomic_load(&c[threadIdx.x * 32u], __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_AGENT)
                                         : 0u;
            v += __shfl_xor(v, 4, 64);
            v += __shfl_xor(v, 2, 64);
            v += __shfl_xor(v, 1, 64);
            v = __shfl(v, 0, 64);
            if (v >= G) break;
            if (++spins > kSpinLimit || __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                if (threadIdx.x == 0) atomicOr(err, 1u);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

// x (length 1024*NG) staged in LDS from coherent loads, with rmsnorm(x)*w fused
// when w is set (stage_issue/stage_finish of the per-kernel step).
template <int NG, bool NORM>
__device__ __forceinline__ void stage_coherent(const float *x, const float *w, float *xs, float *red, uint32_t cols,
                                               float eps) {
    XStage<NG, NORM> st;
    const uint32_t t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        const uint32_t c = kGroupCols * j + 4u * t;
        const uint32_t cc = c < cols ? c : 0u;
        st.v[j] = ld_c4(x + cc);
        if constexpr (NORM) {
            const gf32x4 v = *(const VX_GLOBAL gf32x4 *)(w + cc);
            st.w[j] = make_float4(v.x, v.y, v.z, v.w);
        }
    }
    stage_finish<NG, NORM>(st, xs, red, cols, eps);
}

struct PStage {  // A workgroup's x fragment, read from LDS after staging
    template <int NG>
    __device__ __forceinline__ static void frag(Frag<NG> &f, FragSums<NG> &sx, const float *xs, int lane) {
        frag_from_lds<WT_Q8, NG>(f, xs, lane);
        frag_sums(f, sx);
    }
};

// ---------------------------------------------------------------- phase B
// Split-context attention of one (slice s, head h) unit (k_attn_chunk's
// arithmetic, kernels_attn.hip), with q and the KV rows read coherently, the
// partial record stored coherently, and the last slice of the head to finish
// merging all of the head's records into att[h*HD ..].
template <int HD>
__device__ void attn_unit(const PersistArgs &a, uint32_t layer, uint32_t s, uint32_t h, uint32_t pos,
                          const SplitPlan &plan, __half (*vs)[HD], float *ps, float (*red)[4], float *accs,
                          uint32_t *flag) {
    constexpr int R = HD / 4, KG = 256 / HD, KPG = 64 / KG;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t kvh = h / (a.q_heads / a.kv_heads);
    const uint32_t kv_dim = a.kv_heads * HD;
    const int j = tid >> 2, r = tid & 3;
    float qv[R];
#pragma unroll
    for (int i = 0; i < R; i += 4) {
        const float4 v = ld_c4(a.q + (size_t)h * HD + r * R + i);
        qv[i] = v.x;
        qv[i + 1] = v.y;
        qv[i + 2] = v.z;
        qv[i + 3] = v.w;
    }
    const uint32_t t0 = s * plan.chunk, t1 = min(plan.n, t0 + plan.chunk);
    const float inv_sqrt = 1.0f / sqrtf((float)HD);
    const size_t layer_base = (size_t)layer * a.context;
    float m_run = -FLT_MAX, l_run = 0.f, acc = 0.f;
    for (uint32_t tb = t0; tb < t1; tb += 64u) {
        const uint32_t key = tb + (uint32_t)j;
        const bool valid = key < t1;
        const uint32_t kk = valid ? key : t0;
        const size_t row = (layer_base + kk) * kv_dim + (size_t)kvh * HD + (size_t)r * R;
        uint4 kw[R / 8], vw[R / 8];
        if (kk == pos) {  // the row phase A wrote in this launch
#pragma unroll
            for (int i = 0; i < R / 8; ++i) {
                kw[i] = ld_c16b(a.kc + row + 8 * i);
                vw[i] = ld_c16b(a.vc + row + 8 * i);
            }
        } else {          // rows of earlier launches
#pragma unroll
            for (int i = 0; i < R / 8; ++i) {
                kw[i] = *reinterpret_cast<const uint4 *>(a.kc + row + 8 * i);
                vw[i] = *reinterpret_cast<const uint4 *>(a.vc + row + 8 * i);
            }
        }
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
        float sc = d0 + d1;
        sc += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sc), 0xb1, 0xf, 0xf, false));
        sc += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, sc), 0x4e, 0xf, 0xf, false));
        sc = valid ? sc * inv_sqrt : -FLT_MAX;
        float wm = sc;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) wm = fmaxf(wm, __shfl_xor(wm, o, 64));
        if (lane == 0) red[0][wave] = wm;
        __syncthreads();
        const float tmax = fmaxf(fmaxf(red[0][0], red[0][1]), fmaxf(red[0][2], red[0][3]));
        const float m_new = fmaxf(m_run, tmax);
        const float p = valid ? expf(sc - m_new) : 0.f;
#pragma unroll
        for (int i = 0; i < R / 8; ++i) *reinterpret_cast<uint4 *>(&vs[j][r * R + 8 * i]) = vw[i];
        if (r == 0) ps[j] = p;
        float ws = r == 0 ? p : 0.f;
        ws = wave_sum_dpp(ws);
        if (lane == 0) red[1][wave] = ws;
        __syncthreads();
        const float tsum = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
        const float corr = expf(m_run - m_new);
        l_run = l_run * corr + tsum;
        m_run = m_new;
        const int d = tid % HD, kg = tid / HD;
        float v = 0.f;
#pragma unroll 8
        for (int jj = 0; jj < KPG; ++jj) {
            const int k = kg * KPG + jj;
            v = fmaf(ps[k], __half2float(vs[k][d]), v);
        }
        acc = acc * corr + v;
        __syncthreads();
    }
    accs[tid] = acc;
    __syncthreads();
    float *rec = a.part + ((size_t)h * a.splits + s) * (HD + 4);
    if (tid < HD) {
        float t = 0.f;
#pragma unroll
        for (int kg = 0; kg < KG; ++kg) t += accs[kg * HD + tid];
        st_c(rec + 4 + tid, t);
    }
    if (tid == 0) {
        st_c(rec + 0, m_run);
        st_c(rec + 1, l_run);
    }
    // Arrival count of the head's slices; the last one merges.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const uint32_t old = __hip_atomic_fetch_add(&a.head_cnt[(size_t)layer * a.q_heads + h], 1u, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
        *flag = old + 1u == plan.active ? 1u : 0u;
    }
    __syncthreads();
    if (*flag == 0u) return;
    // Every record is requested before any is used (slots past the active
    // slices read slice 0 and get weight 0), as k_attn_combine's arithmetic.
    if (tid < HD) {
        float m[kPersistMaxSplits], lv[kPersistMaxSplits], ov[kPersistMaxSplits];
#pragma unroll
        for (uint32_t t = 0; t < kPersistMaxSplits; ++t) {
            const float *rr = a.part + ((size_t)h * a.splits + (t < plan.active ? t : 0u)) * (HD + 4);
            m[t] = ld_c(rr);
            lv[t] = ld_c(rr + 1);
            ov[t] = ld_c(rr + 4 + tid);
        }
        float mx = -FLT_MAX;
#pragma unroll
        for (uint32_t t = 0; t < kPersistMaxSplits; ++t)
            if (t < plan.active) mx = fmaxf(mx, m[t]);
        float l = 0.f, o = 0.f;
#pragma unroll
        for (uint32_t t = 0; t < kPersistMaxSplits; ++t) {
            const bool on = t < plan.active;
            const float w = on ? expf(m[t] - mx) : 0.f;
            l = on ? fmaf(lv[t], w, l) : l;
            o = on ? fmaf(ov[t], w, o) : o;
        }
        st_c(a.att + (size_t)h * HD + tid, o / l);
    }
}

// Profiling timeline (PersistArgs::trace): thread 0 of each workgroup stores the
// 100 MHz device clock; k = 0 phase start, 1 wait over, 2 completion counted.
__device__ __forceinline__ void mark(const PersistArgs &a, uint32_t idx, uint32_t k) {
    if (a.trace && threadIdx.x == 0)
        a.trace[((size_t)blockIdx.x * a.n_layers * kPersistPhases + idx) * 4u + k] =
            (unsigned long long)wall_clock64();
}

// ---------------------------------------------------------------- the kernel
template <int NGH, int NGF, int RPWC, int RPWD>
__global__ __launch_bounds__(256, kPersistGroups) void k_decode_persistent(PersistArgs a) {
    __shared__ __align__(16) float xs[(NGF > NGH ? NGF : NGH) * kGroupCols];
    __shared__ float red[kWavesPerBlock];
    __shared__ __align__(16) __half vs[64][128];
    __shared__ float ps[64];
    __shared__ float red2[2][4];
    __shared__ float accs[256];
    __shared__ uint32_t flag;
    const int tid = threadIdx.x, lane = tid & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // G workgroups per group; lb = index within the group.
    const uint32_t G = gridDim.x / kPersistGroups, grp = blockIdx.x / G, lb = blockIdx.x % G;
    const uint32_t gw = lb * kWavesPerBlock + wave, NW = G * kWavesPerBlock;
    const uint32_t H = a.H, F = a.F, KV = a.KV, HD = 128u, half_dim = 64u;
    const uint32_t pq = H / 2u, pk = KV / 2u, NP = pq + 2u * pk;
    const uint32_t pos = *a.position;
    const SplitPlan plan = split_plan(a.position, a.context, a.splits);
    const uint32_t nunits = a.q_heads * a.splits;
    float hkeep[RPWC];   // this wave's h rows after phase C, reused by phase E

    for (uint32_t l = 0; l < a.n_layers; ++l) {
        const PLayer &L = a.layers[l];
        // ------------------------------------------------ A: QKV + RoPE + KV row
        if ((l * 5u + 0u) % kPersistGroups == grp) {
            mark(a, l * 5u + 0u, 0);
            Q8Row<NGH> rr[2][2];
            uint32_t r0s[2], r1s[2];
            int segs[2];
            bool live[2];
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const uint32_t praw = gw + (uint32_t)k * NW;
                live[k] = praw < NP;
                const uint32_t p = live[k] ? praw : NP - 1u;
                int seg;
                uint32_t r0, r1;
                if (p < pq + pk) {
                    seg = p < pq ? 0 : 1;
                    const uint32_t pp = seg == 0 ? p : p - pq;
                    r0 = (pp / half_dim) * HD + pp % half_dim;
                    r1 = r0 + half_dim;
                } else {
                    seg = 2;
                    r0 = 2u * (p - pq - pk);
                    r1 = r0 + 1u;
                }
                const void *wq = seg == 0 ? L.q : (seg == 1 ? L.k : L.v);
                const __half *wd = seg == 0 ? L.qd : (seg == 1 ? L.kd : L.vd);
                load_row_g(rr[k][0], wq, wd, r0, H, lane);
                load_row_g(rr[k][1], wq, wd, r1, H, lane);
                r0s[k] = r0;
                r1s[k] = r1;
                segs[k] = seg;
            }
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                pin(rr[k][0]);
                pin(rr[k][1]);
            }
            if (l > 0) phase_wait(a.cnt, (l - 1u) * 5u + 4u, G, a.err);
            mark(a, l * 5u + 0u, 1);
            stage_coherent<NGH, true>(a.h, L.attn_norm, xs, red, H, a.eps);
            Frag<NGH> f;
            FragSums<NGH> sx;
            PStage::frag<NGH>(f, sx, xs, lane);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                float v0 = wave_sum_dpp(row_dot(rr[k][0], f, sx));
                float v1 = wave_sum_dpp(row_dot(rr[k][1], f, sx));
                if (lane == 0 && live[k]) {
                    const int seg = segs[k];
                    const uint32_t r0 = r0s[k], r1 = r1s[k];
                    if (seg < 2) {
                        const float2 cs = a.rope_cs[r0 % HD];
                        const float n0 = v0 * cs.x - v1 * cs.y;
                        const float n1 = v1 * cs.x + v0 * cs.y;
                        v0 = n0;
                        v1 = n1;
                    }
                    float *dst = seg == 0 ? a.q : (seg == 1 ? a.k : a.v);
                    st_c(dst + r0, v0);
                    st_c(dst + r1, v1);
                    if (seg > 0 && pos < a.context) {
                        __half *cache = seg == 1 ? a.kc : a.vc;
                        const size_t base = ((size_t)l * a.context + pos) * KV;
                        st_c16(cache + base + r0, v0);
                        st_c16(cache + base + r1, v1);
                    }
                }
            }
            phase_done(a.cnt, l * 5u + 0u);
            mark(a, l * 5u + 0u, 2);
        }
        // ------------------------------------------------ B: attention
        if ((l * 5u + 1u) % kPersistGroups == grp) {
            mark(a, l * 5u + 1u, 0);
            phase_wait(a.cnt, l * 5u + 0u, G, a.err);
            mark(a, l * 5u + 1u, 1);
            for (uint32_t u = lb; u < nunits; u += G) {
                const uint32_t s = u % a.splits, h = u / a.splits;
                if (s < plan.active) attn_unit<128>(a, l, s, h, pos, plan, vs, ps, red2, accs, &flag);
            }
            phase_done(a.cnt, l * 5u + 1u);
            mark(a, l * 5u + 1u, 2);
        }
        // ------------------------------------------------ C: attn_out + residual
        if ((l * 5u + 2u) % kPersistGroups == grp) {
            mark(a, l * 5u + 2u, 0);
            const uint32_t row0 = gw * RPWC;
            Q8Row<NGH> r[RPWC];
#pragma unroll
            for (int i = 0; i < RPWC; ++i) load_row_g(r[i], L.o, L.od, row0 + i, H, lane);
            float hold[RPWC];
#pragma unroll
            for (int i = 0; i < RPWC; ++i) hold[i] = ld_c(a.h + row0 + i);
#pragma unroll
            for (int i = 0; i < RPWC; ++i) {
                pin(r[i]);
                pin(hold[i]);
            }
            phase_wait(a.cnt, l * 5u + 1u, G, a.err);
            mark(a, l * 5u + 2u, 1);
            stage_coherent<NGH, false>(a.att, nullptr, xs, red, H, 0.f);
            Frag<NGH> f;
            FragSums<NGH> sx;
            PStage::frag<NGH>(f, sx, xs, lane);
#pragma unroll
            for (int i = 0; i < RPWC; ++i) {
                const float acc = wave_sum_dpp(row_dot(r[i], f, sx));
                hkeep[i] = hold[i] + acc * a.scale;
                if (lane == 0) st_c(a.h + row0 + i, hkeep[i]);
            }
            phase_done(a.cnt, l * 5u + 2u);
            mark(a, l * 5u + 2u, 2);
        }
        // ------------------------------------------------ D: rmsnorm + SwiGLU
        if ((l * 5u + 3u) % kPersistGroups == grp) {
            mark(a, l * 5u + 3u, 0);
            const uint32_t row0 = gw * RPWD;
            Q8Row<NGH> rg[RPWD], ru[RPWD];

#pragma unroll
            for (int i = 0; i < RPWD; ++i) {
                load_row_g(rg[i], L.g, L.gd, row0 + i, H, lane);
                load_row_g(ru[i], L.u, L.ud, row0 + i, H, lane);
            }
#pragma unroll
            for (int i = 0; i < RPWD; ++i) {
                pin(rg[i]);
                pin(ru[i]);
            }
            phase_wait(a.cnt, l * 5u + 2u, G, a.err);
            mark(a, l * 5u + 3u, 1);
            stage_coherent<NGH, true>(a.h, L.ffn_norm, xs, red, H, a.eps);
            Frag<NGH> f;
            FragSums<NGH> sx;
            PStage::frag<NGH>(f, sx, xs, lane);
#pragma unroll
            for (int i = 0; i < RPWD; ++i) {
                const float g = wave_sum_dpp(row_dot(rg[i], f, sx));
                const float uu = wave_sum_dpp(row_dot(ru[i], f, sx));
                if (lane == 0) st_c(a.act + row0 + i, (g / (1.0f + expf(-g))) * uu);
            }
            phase_done(a.cnt, l * 5u + 3u);
            mark(a, l * 5u + 3u, 2);
        }
        // ------------------------------------------------ E: down + residual
        if ((l * 5u + 4u) % kPersistGroups == grp) {
            mark(a, l * 5u + 4u, 0);
            const uint32_t row0 = gw * RPWC;
            Q8Row<NGF> r[RPWC];
#pragma unroll
            for (int i = 0; i < RPWC; ++i) load_row_g(r[i], L.dn, L.dnd, row0 + i, F, lane);
#pragma unroll
            for (int i = 0; i < RPWC; ++i) pin(r[i]);
            phase_wait(a.cnt, l * 5u + 3u, G, a.err);
            mark(a, l * 5u + 4u, 1);
            stage_coherent<NGF, false>(a.act, nullptr, xs, red, F, 0.f);
            Frag<NGF> f;
            FragSums<NGF> sx;
            PStage::frag<NGF>(f, sx, xs, lane);
#pragma unroll
            for (int i = 0; i < RPWC; ++i) {
                const float acc = wave_sum_dpp(row_dot(r[i], f, sx));
                if (lane == 0) st_c(a.h + row0 + i, hkeep[i] + acc * a.scale);
            }
            phase_done(a.cnt, l * 5u + 4u);
            mark(a, l * 5u + 4u, 2);
        }
    }
}

}  // namespace

uint64_t persist_counter_words(uint32_t n_layers, uint32_t q_heads) {
    return (uint64_t)n_layers * kPersistPhases * kPersistCntStride + (uint64_t)n_layers * q_heads;
}

// Compiled instance: H = 2048 (two 1024-column groups), F = 6144, head_dim 128,
// 2 rows per wave in attn_out/down (H = 2 * 4 * cus) and 6 gate/up row pairs
// per wave in SwiGLU (F = 6 * 4 * cus), at most two rotary pairs per wave in
// the QKV phase; `cus` workgroups per group.
bool persistent_supported(uint32_t H, uint32_t F, uint32_t KV, uint32_t q_heads, uint32_t head_dim, uint32_t cus) {
    const uint32_t waves = cus * kWavesPerBlock;
    return H == 2048u && F == 6144u && head_dim == 128u && q_heads * head_dim == H && KV % 2u == 0u &&
           H == 2u * waves && F == 6u * waves && H / 2u + KV <= 2u * waves;
}

int launch_decode_persistent(hipStream_t s, const PersistArgs &a, uint32_t cus) {
    if (!persistent_supported(a.H, a.F, a.KV, a.q_heads, a.H / (a.q_heads ? a.q_heads : 1u), cus) ||
        a.kv_heads == 0 || a.q_heads % a.kv_heads || a.KV != a.kv_heads * 128u || a.splits == 0 ||
        a.splits > kPersistMaxSplits)
        return fail(VX_ERR_UNSUPPORTED, "persistent decode step: geometry H=%u F=%u KV=%u on %u CUs not compiled",
                    a.H, a.F, a.KV, cus);
    k_decode_persistent<2, 6, 2, 6><<<kPersistGroups * cus, 256, 0, s>>>(a);
    VX_LAUNCHED("k_decode_persistent");
    return VX_OK;
}

int persistent_occupancy(int *blocks_per_cu) {
    const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
        blocks_per_cu, reinterpret_cast<const void *>(&k_decode_persistent<2, 6, 2, 6>), 256, 0);
    if (e != hipSuccess) return fail(VX_ERR_HIP, "occupancy query failed: %s", hipGetErrorString(e));
    return VX_OK;
}

}  // namespace vx
