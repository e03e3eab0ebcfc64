// Single-query (decode) attention over the packed f16 KV cache.
//
// k_attn_partial: grid = splits x kv_heads. Each workgroup takes one KV head and
// a contiguous slice of the context, stages 32-key tiles of K and V in LDS, and
// runs all q_per_kv query heads of that KV head against them (the GQA sharing of
// attn_scores.comp's kvh = qh / q_per_kv), with an online softmax, writing a
// (max, sum, acc) partial per head. k_attn_combine merges the partials of each
// query head. The kernel boundary orders the two, so no device-scope fence or
// atomic is needed. Mathematically this is attn_scores.comp -> softmax.comp ->
// attn_values.comp (baselm.rs:969-996).
//
// The reference-granular kernels below keep the exact three-dispatch shape.
#include <cfloat>

#include "vx_internal.h"

namespace vx {
namespace {

constexpr int kTile = 32;
constexpr int kMaxQpk = 16;

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

struct AttnArgs {
    const float *q;
    const __half *kc, *vc;
    float *out, *part;
    const uint32_t *position;
    uint32_t layer, context, q_heads, kv_heads, splits;
};

// Split of the context [0, pos] into `active` contiguous chunks, identical in
// the partial and the combine kernel.
struct SplitPlan {
    uint32_t n, active, chunk;
};
__device__ __forceinline__ SplitPlan split_plan(const AttnArgs &a) {
    uint32_t pos = *a.position;
    if (pos >= a.context) pos = a.context - 1u;
    SplitPlan p;
    p.n = pos + 1u;
    p.active = min(a.splits, (p.n + kTile - 1u) / kTile);
    p.chunk = (p.n + p.active - 1u) / p.active;
    return p;
}

// Partials: part layout [kv_heads][splits][qpk][HD + 2] floats = m, l, acc[HD].
template <int HD>
__global__ __launch_bounds__(256) void k_attn_partial(AttnArgs a) {
    constexpr int KSTRIDE = HD / 2 + 1;  // words per K row in LDS (+1 word: no bank conflicts)
    __shared__ __align__(16) float qs[kMaxQpk][HD];
    __shared__ __align__(16) uint32_t ks[kTile][KSTRIDE];
    __shared__ __align__(16) __half vs[kTile][HD];
    __shared__ float ps[kMaxQpk][kTile];
    __shared__ float m_s[kMaxQpk], l_s[kMaxQpk], corr_s[kMaxQpk];

    const int tid = threadIdx.x;
    const uint32_t split = blockIdx.x, kvh = blockIdx.y;
    const uint32_t qpk = a.q_heads / a.kv_heads;
    const uint32_t kv_dim = a.kv_heads * HD;
    const SplitPlan plan = split_plan(a);
    if (split >= plan.active) return;
    const uint32_t t_begin = split * plan.chunk;
    const uint32_t t_end = min(plan.n, t_begin + plan.chunk);
    const float inv_sqrt = 1.0f / sqrtf((float)HD);

    constexpr int OUT_PER_T = (kMaxQpk * HD) / 256;
    float acc[OUT_PER_T];
#pragma unroll
    for (int j = 0; j < OUT_PER_T; ++j) acc[j] = 0.f;

    for (uint32_t i = tid; i < qpk * HD; i += 256)
        qs[i / HD][i % HD] = a.q[(size_t)(kvh * qpk + i / HD) * HD + (i % HD)];
    if (tid < (int)qpk) {
        m_s[tid] = -FLT_MAX;
        l_s[tid] = 0.f;
    }
    for (uint32_t t0 = t_begin; t0 < t_end; t0 += kTile) {
        const uint32_t nt = min((uint32_t)kTile, t_end - t0);
        __syncthreads();
        // Stage K and V rows t0..t0+nt (HD halves each, 16 B per thread-load).
        constexpr int CHUNKS = HD / 8;
        for (int i = tid; i < kTile * CHUNKS; i += 256) {
            const int j = i / CHUNKS, c = i % CHUNKS;
            const bool ok = (uint32_t)j < nt;
            const size_t base = ((size_t)a.layer * a.context + t0 + (ok ? j : 0)) * kv_dim + kvh * HD + 8 * c;
            uint4 kv = *reinterpret_cast<const uint4 *>(a.kc + base);
            uint4 vv = *reinterpret_cast<const uint4 *>(a.vc + base);
            if (!ok) kv = vv = make_uint4(0u, 0u, 0u, 0u);
            ks[j][4 * c + 0] = kv.x;
            ks[j][4 * c + 1] = kv.y;
            ks[j][4 * c + 2] = kv.z;
            ks[j][4 * c + 3] = kv.w;
            *reinterpret_cast<uint4 *>(&vs[j][8 * c]) = vv;
        }
        __syncthreads();
        // Scores: a half-wave (32 lanes) holds one head's 32 keys; the per-head
        // tile max and exp-sum are half-wave shuffles.
        for (uint32_t idx = tid; idx < qpk * kTile; idx += 256) {
            const uint32_t h = idx / kTile, j = idx % kTile;
            float s = -FLT_MAX;
            if (j < nt) {
                float d0 = 0.f, d1 = 0.f;
#pragma unroll 8
                for (int w = 0; w < HD / 2; ++w) {
                    const float2 kf = h2f2(ks[j][w]);
                    d0 = fmaf(qs[h][2 * w], kf.x, d0);
                    d1 = fmaf(qs[h][2 * w + 1], kf.y, d1);
                }
                s = (d0 + d1) * inv_sqrt;
            }
            float tmax = s;
#pragma unroll
            for (int o = 16; o >= 1; o >>= 1) tmax = fmaxf(tmax, __shfl_xor(tmax, o, 32));
            const float m_old = m_s[h];
            const float m_new = fmaxf(m_old, tmax);
            const float p = j < nt ? expf(s - m_new) : 0.f;
            float psum = p;
#pragma unroll
            for (int o = 16; o >= 1; o >>= 1) psum += __shfl_xor(psum, o, 32);
            ps[h][j] = p;
            if (j == 0) {
                const float corr = expf(m_old - m_new);
                corr_s[h] = corr;
                l_s[h] = l_s[h] * corr + psum;
                m_s[h] = m_new;
            }
        }
        __syncthreads();
#pragma unroll
        for (int jj = 0; jj < OUT_PER_T; ++jj) {
            const uint32_t o = tid + 256u * jj;
            const uint32_t h = o / HD, d = o % HD;
            if (h < qpk) {
                float v = acc[jj] * corr_s[h];
                for (uint32_t j = 0; j < nt; ++j) v = fmaf(ps[h][j], __half2float(vs[j][d]), v);
                acc[jj] = v;
            }
        }
    }
    __syncthreads();
    float *part = a.part + ((size_t)(kvh * a.splits + split) * qpk) * (HD + 2);
#pragma unroll
    for (int jj = 0; jj < OUT_PER_T; ++jj) {
        const uint32_t o = tid + 256u * jj;
        const uint32_t h = o / HD, d = o % HD;
        if (h < qpk) part[h * (HD + 2) + 2 + d] = acc[jj];
    }
    if (tid < (int)qpk) {
        part[tid * (HD + 2)] = m_s[tid];
        part[tid * (HD + 2) + 1] = l_s[tid];
    }
}

// Merge the active splits of one query head: one block per head, one lane per dim.
template <int HD>
__global__ __launch_bounds__(HD) void k_attn_combine(AttnArgs a) {
    __shared__ float w_s[1024];
    __shared__ float inv_l_s;
    const uint32_t h = blockIdx.x, d = threadIdx.x;
    const uint32_t qpk = a.q_heads / a.kv_heads;
    const uint32_t kvh = h / qpk, hh = h % qpk;
    const SplitPlan plan = split_plan(a);
    const float *part0 = a.part + ((size_t)kvh * a.splits * qpk + hh) * (HD + 2);
    const size_t stride = (size_t)qpk * (HD + 2);
    float m = -FLT_MAX;
    for (uint32_t s = 0; s < plan.active; ++s) m = fmaxf(m, part0[s * stride]);
    for (uint32_t s = d; s < plan.active; s += HD) w_s[s] = expf(part0[s * stride] - m);
    __syncthreads();
    if (d == 0) {
        float l = 0.f;
        for (uint32_t s = 0; s < plan.active; ++s) l = fmaf(part0[s * stride + 1], w_s[s], l);
        inv_l_s = 1.0f / l;
    }
    __syncthreads();
    float v = 0.f;
    for (uint32_t s = 0; s < plan.active; ++s) v = fmaf(part0[s * stride + 2 + d], w_s[s], v);
    a.out[(size_t)h * HD + d] = v * inv_l_s;
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
    const uint64_t qpk = kv_heads ? q_heads / kv_heads : 0;
    return 256u + (uint64_t)kv_heads * splits * qpk * (head_dim + 2u) * 4u;
}

int launch_attn_decode(hipStream_t s, const AttnLaunch &l) {
    if (l.kv_heads == 0 || l.q_heads % l.kv_heads || l.q_heads / l.kv_heads > (uint32_t)kMaxQpk)
        return fail(VX_ERR_UNSUPPORTED, "decode attention needs q_heads/kv_heads <= %d", kMaxQpk);
    if (l.splits == 0 || l.splits > 1024u) return fail(VX_ERR_INVALID_ARG, "splits must be 1..1024");
    if (l.context == 0) return fail(VX_ERR_INVALID_ARG, "context is zero");
    AttnArgs a{l.q, l.kc, l.vc, l.out, reinterpret_cast<float *>(reinterpret_cast<uint8_t *>(l.partials) + 256),
               l.position, l.layer, l.context, l.q_heads, l.kv_heads, l.splits};
    dim3 grid(l.splits, l.kv_heads);
    if (l.head_dim == 128) {
        k_attn_partial<128><<<grid, 256, 0, s>>>(a);
        k_attn_combine<128><<<l.q_heads, 128, 0, s>>>(a);
    } else if (l.head_dim == 64) {
        k_attn_partial<64><<<grid, 256, 0, s>>>(a);
        k_attn_combine<64><<<l.q_heads, 64, 0, s>>>(a);
    } else {
        return fail(VX_ERR_UNSUPPORTED, "decode attention supports head_dim 64 or 128, got %u", l.head_dim);
    }
    VX_LAUNCHED("k_attn_partial/k_attn_combine");
    return VX_OK;
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
