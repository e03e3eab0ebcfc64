// Kernels of the LocDiT flow-matching solve (UnifiedCFM, local.rs:383-430):
// seeded Gaussian noise, the CFG-Zero* Euler update, the sinusoidal time
// embedding, LocDiT token packing, and small elementwise ops. All fp32; the
// noise hash is exact integer arithmetic.
#include "decode_dev.h"   // wave_sum_dpp

namespace vx {
namespace {

// Integer finaliser of cfm_noise.comp:11-18 (xorshift-multiply, two rounds).
__device__ __forceinline__ uint32_t mix32(uint32_t v) {
    v ^= v >> 16;
    v *= 0x7feb352du;
    v ^= v >> 15;
    v *= 0x846ca68bu;
    v ^= v >> 16;
    return v;
}

// cfm_noise.comp:25-37: x[i] = temperature * Box-Muller(u(a), u(b)) for the pair
// i/2, with a, b hashes of the pair index and the 64-bit seed. The seed is read
// from device memory (seed[0] = low word, seed[1] = high word) when `seed` is set,
// so that a captured solve replays with new seeds.
__global__ __launch_bounds__(256) void k_cfm_noise(float *x, uint32_t n, const uint32_t *seed, uint32_t seed_lo,
                                                   uint32_t seed_hi, float temperature) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const uint32_t lo = seed ? seed[0] : seed_lo, hi = seed ? seed[1] : seed_hi;
    const uint32_t pair = i >> 1;
    const uint32_t a = mix32(pair ^ lo ^ 0x9e3779b9u);
    const uint32_t b = mix32(pair ^ hi ^ 0x85ebca6bu);
    const float u1 = fmaxf(((float)a + 0.5f) * (1.0f / 4294967296.0f), 1.0e-7f);
    const float u2 = ((float)b + 0.5f) * (1.0f / 4294967296.0f);
    const float r = sqrtf(-2.0f * logf(u1));
    const float theta = 6.28318530717958647692f * u2;
    const float z = (i & 1u) == 0u ? r * cosf(theta) : r * sinf(theta);
    x[i] = z * temperature;
}

// cfm_cfg_euler.comp:15-36 with the conditional and unconditional estimates
// read from `pos` and `neg` (rows of the CFG batch): s = <p,n>/(|n|^2 + 1e-8)
// under CFG-Zero* (else 1); x -= dt * (n*s + cfg*(p - n*s)). One workgroup; the
// dot products are block reductions over n <= 1024 elements.
// One 256-thread workgroup: the CFG-Zero* guided velocity and the Euler update.
// COHERENT: pos and neg were written by other workgroups of the launch and are
// read with device-scope loads (past this workgroup's L2).
template <bool COHERENT = false>
__device__ __forceinline__ void cfg_euler_block(float *x, const float *pos, const float *neg, uint32_t n, float dt,
                                                float cfg, uint32_t zero_star) {
    auto ld = [](const float *p) {
        if constexpr (COHERENT) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else return *p;
    };
    __shared__ float red[2][4];
    // The first NR chunks of 256 stay in registers for the update (one round of
    // loads instead of two); the wave sums reduce by DPP.
    constexpr uint32_t NR = 4;
    float pr[NR], qr[NR];
    float pn = 0.f, nn = 0.f;
#pragma unroll
    for (uint32_t j = 0; j < NR; ++j) {
        const uint32_t i = threadIdx.x + 256u * j;
        pr[j] = i < n ? ld(pos + i) : 0.f;
        qr[j] = i < n ? ld(neg + i) : 0.f;
    }
#pragma unroll
    for (uint32_t j = 0; j < NR; ++j) {
        pn += pr[j] * qr[j];
        nn += qr[j] * qr[j];
    }
    for (uint32_t i = threadIdx.x + 256u * NR; i < n; i += 256u) {
        const float p = ld(pos + i), q = ld(neg + i);
        pn += p * q;
        nn += q * q;
    }
    pn = wave_sum_dpp(pn);
    nn = wave_sum_dpp(nn);
    if ((threadIdx.x & 63u) == 0) {
        red[0][threadIdx.x >> 6] = pn;
        red[1][threadIdx.x >> 6] = nn;
    }
    __syncthreads();
    pn = red[0][0] + red[0][1] + red[0][2] + red[0][3];
    nn = red[1][0] + red[1][1] + red[1][2] + red[1][3];
    const float scale = zero_star ? pn / (nn + 1.0e-8f) : 1.0f;
#pragma unroll
    for (uint32_t j = 0; j < NR; ++j) {
        const uint32_t i = threadIdx.x + 256u * j;
        if (i < n) x[i] -= dt * (qr[j] * scale + cfg * (pr[j] - qr[j] * scale));
    }
    for (uint32_t i = threadIdx.x + 256u * NR; i < n; i += 256u) {
        const float p = ld(pos + i), q = ld(neg + i);
        const float guided = q * scale + cfg * (p - q * scale);
        x[i] -= dt * guided;
    }
}

__global__ __launch_bounds__(256) void k_cfm_cfg_euler(float *x, const float *pos, const float *neg, uint32_t n,
                                                       float dt, float cfg, uint32_t zero_star) {
    cfg_euler_block(x, pos, neg, n, dt, cfg, zero_star);
}

// The estimator's out_proj for the x tokens of both sequences (seq_linear_bias,
// F16 weights: one wave per output feature, each lane a contiguous 1/64 of the
// row, then a wave reduction), and then the update above, run by the last
// workgroup to finish. Each workgroup stores its outputs with device-scope
// stores (written through to the device's coherence point), waits until every
// one is acknowledged, and counts itself in a.counter; the one that takes the
// count to gridDim.x reads all outputs with device-scope loads, applies
// cfg_euler_block and resets the counter for the next launch. No workgroup
// waits for another. (A device-scope fence here would write back and
// invalidate the whole L2 of every workgroup's XCD: tens of microseconds over a
// few hundred workgroups on MI355X.)
template <bool FRAG>   // a.rows_frag
__global__ __launch_bounds__(256) void k_cfm_out_euler(CfmOutEulerArgs a) {
    __shared__ uint32_t is_last;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t f = blockIdx.x * 4u + wave, R = 2u * a.patch, n = a.patch * a.feat;
    // FRAG: the x rows copied from the stream into LDS as f32 rows (16-byte pieces
    // of frag32 order, four columns each), so that the lanes' reads below are
    // contiguous; a lane's own columns of one row in frag32 order lie in another
    // 2 KB block each.
    extern __shared__ __align__(16) float xrows[];
    if constexpr (FRAG) {
        const uint32_t h4 = a.hidden >> 2;
        for (uint32_t i = threadIdx.x; i < R * h4; i += 256u) {
            const uint32_t r = i / h4, c = 4u * (i - r * h4);
            const uint32_t b = r / a.patch, p = r - b * a.patch, row = b * a.tokens + a.x0 + p;
            *reinterpret_cast<float4 *>(xrows + (size_t)r * a.hidden + c) =
                *reinterpret_cast<const float4 *>(a.rows + frag32_index(row, c, a.hidden));
        }
        __syncthreads();
    }
    if (f < a.feat) {
        const uint32_t ch = a.hidden >> 6;   // columns per lane, a multiple of 8
        float acc[kOutEulerMaxRows], ss[kOutEulerMaxRows];
#pragma unroll
        for (uint32_t r = 0; r < kOutEulerMaxRows; ++r) acc[r] = ss[r] = 0.f;
        const __half *wr = a.w + (size_t)f * a.hidden + lane * ch;
        for (uint32_t c = 0; c < ch; c += 8u) {
            const uint4 wv = *reinterpret_cast<const uint4 *>(wr + c);
            const uint32_t w4[4] = {wv.x, wv.y, wv.z, wv.w};
            float w8[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float2 t = __half22float2(*reinterpret_cast<const __half2 *>(&w4[e]));
                w8[2 * e] = t.x;
                w8[2 * e + 1] = t.y;
            }
            const uint32_t c0 = lane * ch + c;   // a multiple of 8
            if constexpr (FRAG) {   // the final norm's weights folded into the row of W
                const float4 n0 = *reinterpret_cast<const float4 *>(a.norm_w + c0);
                const float4 n1 = *reinterpret_cast<const float4 *>(a.norm_w + c0 + 4);
                w8[0] *= n0.x; w8[1] *= n0.y; w8[2] *= n0.z; w8[3] *= n0.w;
                w8[4] *= n1.x; w8[5] *= n1.y; w8[6] *= n1.z; w8[7] *= n1.w;
            }
#pragma unroll
            for (uint32_t r = 0; r < kOutEulerMaxRows; ++r) {
                if (r >= R) break;
                const uint32_t b = r / a.patch, p = r - b * a.patch, row = b * a.tokens + a.x0 + p;
                float4 u0, u1;
                if constexpr (FRAG) {   // the row's columns c0..c0+7 from LDS
                    (void)row;
                    const float *xr = xrows + (size_t)r * a.hidden + c0;
                    u0 = *reinterpret_cast<const float4 *>(xr);
                    u1 = *reinterpret_cast<const float4 *>(xr + 4);
                    ss[r] += u0.x * u0.x + u0.y * u0.y + u0.z * u0.z + u0.w * u0.w +
                             u1.x * u1.x + u1.y * u1.y + u1.z * u1.z + u1.w * u1.w;
                } else {
                    const float *xr = a.rows + (size_t)row * a.hidden + c0;
                    u0 = *reinterpret_cast<const float4 *>(xr);
                    u1 = *reinterpret_cast<const float4 *>(xr + 4);
                }
                acc[r] += w8[0] * u0.x;
                acc[r] += w8[1] * u0.y;
                acc[r] += w8[2] * u0.z;
                acc[r] += w8[3] * u0.w;
                acc[r] += w8[4] * u1.x;
                acc[r] += w8[5] * u1.y;
                acc[r] += w8[6] * u1.z;
                acc[r] += w8[7] * u1.w;
            }
        }
        const float bias = !a.bias ? 0.f
                           : a.bias_dtype == 0 ? static_cast<const float *>(a.bias)[f]
                                               : __half2float(static_cast<const __half *>(a.bias)[f]);
#pragma unroll
        for (uint32_t r = 0; r < kOutEulerMaxRows; ++r) {
            if (r >= R) break;
            float v = wave_sum_dpp(acc[r]);   // wave-uniform
            if constexpr (FRAG) v *= 1.0f / sqrtf(wave_sum_dpp(ss[r]) / (float)a.hidden + a.eps);   // rmsnorm.comp:36-38
            if (lane == r) {
                const uint32_t b = r / a.patch, p = r - b * a.patch;
                __hip_atomic_store(a.out + (size_t)b * n + (size_t)p * a.feat + f, v + bias, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    // Hand-off to the last workgroup: agent-scope relaxed atomic stores, their
    // acknowledgements awaited, then the counter; the last workgroup reads the rows
    // with agent-scope relaxed atomic loads (cfg_euler_block<true>). This rests on
    // gfx942/gfx950 compiling agent-scope atomics past the per-XCD L2 (sc1), not on
    // the HIP memory model; see the stream-K part hand-off in kernels_gemm.hip.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0);   // every output store acknowledged
    __syncthreads();
    if (threadIdx.x == 0) is_last = atomicAdd(a.counter, 1u) == gridDim.x - 1u;
    __syncthreads();
    if (!is_last) return;
    cfg_euler_block<true>(a.x, a.out, a.out + n, n, a.dt, a.cfg, a.zero_star);
    if (threadIdx.x == 0) *a.counter = 0u;
}

// time_sinusoidal.comp:5: out[i] = sin(a) for i < dim/2, cos(a) after, with
// a = 1000 t exp(-j ln(1e4)/(dim/2 - 1)), j = i mod dim/2. t from device memory
// (t_dev[t_index]) when t_dev is set, so a captured solve can step through t.
__global__ __launch_bounds__(256) void k_time_sinusoidal(float *out, uint32_t dim, float t_in, const float *t_dev,
                                                         uint32_t t_index) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= dim) return;
    const float t = t_dev ? t_dev[t_index + blockIdx.y] : t_in;   // row blockIdx.y of a batch
    out += (size_t)blockIdx.y * dim;
    const uint32_t half_dim = dim / 2u;
    const uint32_t j = i % half_dim;
    const float denom = (float)max(half_dim - 1u, 1u);
    const float freq = expf((float)j * (-logf(10000.0f) / denom));
    const float a = 1000.0f * t * freq;
    out[i] = i < half_dim ? sinf(a) : cosf(a);
}

// pack_locdit.comp:10 generalised to n_mu mu tokens, one time token, n_cond
// condition rows and n_x latent rows, for `batch` sequences laid out back to
// back; sequence b zeroes its mu tokens when bit b of zero_mu_mask is set and
// its condition rows when bit b of zero_cond_mask is set.
__global__ __launch_bounds__(256) void k_pack_locdit(PackLocditArgs a) {
    const uint32_t seq_tokens = a.n_mu + 1u + a.n_cond + a.n_x;
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    const uint32_t per = seq_tokens * a.hidden;
    if (i >= per * a.batch) return;
    const uint32_t b = i / per, r = i - b * per;
    const uint32_t tok = r / a.hidden, d = r - tok * a.hidden;
    float v;
    if (tok < a.n_mu) {
        v = (a.zero_mu_mask >> b) & 1u ? 0.f : a.mu[tok][d];
    } else if (tok == a.n_mu) {
        v = a.time[d];
    } else if (tok < a.n_mu + 1u + a.n_cond) {
        v = (a.zero_cond_mask >> b) & 1u ? 0.f : a.cond[(tok - a.n_mu - 1u) * a.hidden + d];
    } else if (a.in_w) {
        // seq_linear_bias.comp for one x token: bias + W[d] . x (fp32, f16 weights).
        const uint32_t tx = tok - a.n_mu - 1u - a.n_cond;
        const __half *w = a.in_w + (size_t)d * a.feat;
        const float *xp = a.xpatch + (size_t)tx * a.feat;
        float acc = 0.f;
        // Eight-column chunks: one 16-byte weight load each, all issued up front
        // (feat % 8 == 0 and 16-byte rows are checked at launch).
        constexpr uint32_t kMaxChunks = 16;   // feat <= 128
        uint4 wc[kMaxChunks];
#pragma unroll
        for (uint32_t c = 0; c < kMaxChunks; ++c)
            wc[c] = 8u * c < a.feat ? *reinterpret_cast<const uint4 *>(w + 8u * c) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (uint32_t c = 0; c < kMaxChunks; ++c) {
            if (8u * c >= a.feat) break;
            const uint32_t u[4] = {wc[c].x, wc[c].y, wc[c].z, wc[c].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const __half2 h = __builtin_bit_cast(__half2, u[k]);
                acc = fmaf(__low2float(h), xp[8u * c + 2u * k], acc);
                acc = fmaf(__high2float(h), xp[8u * c + 2u * k + 1u], acc);
            }
        }
        const float bias = !a.in_b ? 0.f
                           : a.in_bt == 0 ? static_cast<const float *>(a.in_b)[d]
                                          : __half2float(static_cast<const __half *>(a.in_b)[d]);
        v = acc + bias;
    } else {
        v = a.x[(tok - a.n_mu - 1u - a.n_cond) * a.hidden + d];
    }
    if (a.out_frag) a.out[frag32_index(b * seq_tokens + tok, d, a.hidden)] = v;
    else a.out[i] = v;
}

// silu_inplace.comp:5 and add_vectors.comp:6.
__global__ __launch_bounds__(256) void k_silu_inplace(float *x, uint32_t n) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const float v = x[i];
    x[i] = v / (1.0f + expf(-v));
}

// fsq_quantize.comp: the latent of the finite scalar quantizer, in place. Ties of
// v * scale round away from zero (f32::round of acoustic.rs:1266-1271).
__global__ __launch_bounds__(256) void k_fsq_quantize(float *x, uint32_t n, float scale) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const float v = tanhf(x[i]);
    x[i] = roundf(v * scale) / scale;
}

// a[r][i] += b[i] for each of gridDim.y rows r of n values.
__global__ __launch_bounds__(256) void k_add_vectors(float *a, const float *b, uint32_t n) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < n) a[(size_t)blockIdx.y * n + i] += b[i];
}

}  // namespace

int launch_cfm_noise(hipStream_t s, float *x, uint32_t n, const uint32_t *dev_seed, uint64_t seed, float temperature) {
    if (!n) return VX_OK;
    k_cfm_noise<<<(n + 255u) / 256u, 256, 0, s>>>(x, n, dev_seed, (uint32_t)seed, (uint32_t)(seed >> 32), temperature);
    VX_LAUNCHED("k_cfm_noise");
    return VX_OK;
}

int launch_cfm_cfg_euler(hipStream_t s, float *x, const float *pos, const float *neg, uint32_t n, float dt, float cfg,
                         uint32_t zero_star) {
    if (!n) return VX_OK;
    k_cfm_cfg_euler<<<1, 256, 0, s>>>(x, pos, neg, n, dt, cfg, zero_star);
    VX_LAUNCHED("k_cfm_cfg_euler");
    return VX_OK;
}

bool cfm_out_euler_eligible(uint32_t patch, uint32_t feat, uint32_t hidden, const void *w) {
    return patch > 0 && 2u * patch <= kOutEulerMaxRows && feat > 0 && hidden % 512u == 0 && w &&
           (reinterpret_cast<uintptr_t>(w) & 15u) == 0;
}

int launch_cfm_out_euler(hipStream_t s, const CfmOutEulerArgs &a) {
    if (!cfm_out_euler_eligible(a.patch, a.feat, a.hidden, a.w) || !a.rows || !a.out || !a.x || !a.counter ||
        (reinterpret_cast<uintptr_t>(a.rows) & 15u) ||
        (a.rows_frag && (!a.norm_w || (reinterpret_cast<uintptr_t>(a.norm_w) & 15u))))
        return fail(VX_ERR_UNSUPPORTED, "cfm out_proj + euler: patch %u, feat %u, hidden %u", a.patch, a.feat,
                    a.hidden);
    if (a.rows_frag) {
        const uint64_t lds = (uint64_t)2u * a.patch * a.hidden * 4u;
        if (lds > 65536u) return fail(VX_ERR_UNSUPPORTED, "cfm out_proj + euler: %u x rows of %u in LDS", 2u * a.patch,
                                      a.hidden);
        k_cfm_out_euler<true><<<(a.feat + 3u) / 4u, 256, (size_t)lds, s>>>(a);
    }
    else k_cfm_out_euler<false><<<(a.feat + 3u) / 4u, 256, 0, s>>>(a);
    VX_LAUNCHED("k_cfm_out_euler");
    return VX_OK;
}

int launch_time_sinusoidal(hipStream_t s, float *out, uint32_t dim, float t, const float *t_dev, uint32_t t_index,
                           uint32_t rows) {
    if (!dim || !rows) return VX_OK;
    if (rows > 1 && !t_dev) return fail(VX_ERR_INVALID_ARG, "time_sinusoidal: several rows need device t values");
    k_time_sinusoidal<<<dim3((dim + 255u) / 256u, rows), 256, 0, s>>>(out, dim, t, t_dev, t_index);
    VX_LAUNCHED("k_time_sinusoidal");
    return VX_OK;
}

int launch_pack_locdit(hipStream_t s, const PackLocditArgs &a) {
    const uint64_t n = (uint64_t)(a.n_mu + 1u + a.n_cond + a.n_x) * a.hidden * a.batch;
    if (!n) return VX_OK;
    if (a.in_w && (a.feat == 0 || a.feat > 128u || a.feat % 8u || !a.xpatch ||
                   (reinterpret_cast<uintptr_t>(a.in_w) & 15u)))
        return fail(VX_ERR_UNSUPPORTED, "pack_locdit: fused in_proj needs feat %% 8 == 0, <= 128, 16-byte rows");
    if (a.out_frag && a.hidden % 32u)
        return fail(VX_ERR_UNSUPPORTED, "pack_locdit: a frag32 stream needs hidden %% 32 == 0");
    k_pack_locdit<<<(unsigned)((n + 255u) / 256u), 256, 0, s>>>(a);
    VX_LAUNCHED("k_pack_locdit");
    return VX_OK;
}

int launch_silu_inplace(hipStream_t s, float *x, uint32_t n) {
    if (!n) return VX_OK;
    k_silu_inplace<<<(n + 255u) / 256u, 256, 0, s>>>(x, n);
    VX_LAUNCHED("k_silu_inplace");
    return VX_OK;
}

int launch_fsq_quantize(hipStream_t s, float *x, uint32_t n, float scale) {
    if (!n) return VX_OK;
    k_fsq_quantize<<<(n + 255u) / 256u, 256, 0, s>>>(x, n, scale);
    VX_LAUNCHED("k_fsq_quantize");
    return VX_OK;
}

int launch_add_vectors(hipStream_t s, float *a, const float *b, uint32_t n, uint32_t rows) {
    if (!n || !rows) return VX_OK;
    k_add_vectors<<<dim3((n + 255u) / 256u, rows), 256, 0, s>>>(a, b, n);
    VX_LAUNCHED("k_add_vectors");
    return VX_OK;
}

}  // namespace vx
