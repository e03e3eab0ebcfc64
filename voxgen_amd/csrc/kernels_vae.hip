// AudioVAE decoder kernels (vae_*.comp).
//
// Two families:
//  * channel-major [C][L] kernels with the reference shaders' semantics, behind
//    the per-op entry points (vae_conv1d.comp, vae_convtranspose1d.comp,
//    vae_snake.comp, vae_scale_bias.comp, vae_add.comp, vae_tanh.comp);
//  * frame-major [L][C] kernels of the decode engine, where the 1x1 convolutions
//    and the transposed convolutions are GEMMs on MFMA (k_gemm) and the
//    elementwise work (scale/bias, snake) is fused into the passes around them.
// Snake: x + sin(a x)^2 / (a + 1e-9) (vae_snake.comp:13-16).
#include "vx_internal.h"

namespace vx {
namespace {

__device__ __forceinline__ float hf(__half v) { return __half2float(v); }

// A model scalar of GGML dtype 1 (F16) or 0 (F32).
__device__ __forceinline__ float ldw(const void *p, uint32_t i, uint32_t dtype) {
    return dtype == 1u ? hf(static_cast<const __half *>(p)[i]) : static_cast<const float *>(p)[i];
}

__device__ __forceinline__ float snake(float x, float a) {
    const float s = sinf(a * x);
    return x + (s * s) / (a + 1e-9f);
}
// The decode engine's snake with the channel's 1 / (a + 1e-9) computed once.
__device__ __forceinline__ float snake_inv(float a) { return 1.0f / (a + 1e-9f); }
// (The native __sinf measured no faster here: 0.72 against 0.69 ms per decode.)
__device__ __forceinline__ float snake_fm(float x, float a, float inv) {
    const float s = sinf(a * x);
    return fmaf(s * s, inv, x);
}

// ------------------------------------------------------------ channel-major
__global__ __launch_bounds__(256) void k_vae_conv1d_cm(VaeConvArgs a) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x, oc = blockIdx.y;
    if (t >= a.out_length || oc >= a.out_channels) return;
    const uint32_t out_pg = a.out_channels / a.groups, in_pg = a.in_channels / a.groups;
    const uint32_t in_base = (oc / out_pg) * in_pg;
    float sum = a.bias ? ldw(a.bias, oc, a.bias_dtype) : 0.f;
    for (uint32_t icg = 0; icg < in_pg; ++icg) {
        const uint32_t ic = in_base + icg;
        for (uint32_t k = 0; k < a.kernel; ++k) {
            const int ti = (int)(t * a.stride + k * a.dilation) - (int)a.left_pad;
            if (ti < 0 || ti >= (int)a.in_length) continue;
            const float w = ldw(a.w, (oc * in_pg + icg) * a.kernel + k, a.w_dtype);
            sum += a.x[(size_t)ic * a.in_length + (uint32_t)ti] * w;
        }
    }
    a.y[(size_t)oc * a.out_length + t] = sum;
}

__global__ __launch_bounds__(256) void k_vae_convt1d_cm(VaeConvArgs a) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x, oc = blockIdx.y;
    if (t >= a.out_length || oc >= a.out_channels) return;
    const uint32_t out_pg = a.out_channels / a.groups, in_pg = a.in_channels / a.groups;
    const uint32_t group = oc / out_pg, ocg = oc - group * out_pg, in_base = group * in_pg;
    float sum = a.bias ? ldw(a.bias, oc, a.bias_dtype) : 0.f;
    const uint32_t first_k = t % a.stride;
    for (uint32_t icg = 0; icg < in_pg; ++icg) {
        const uint32_t ic = in_base + icg;
        for (uint32_t k = first_k; k < a.kernel; k += a.stride) {
            if (t < k) continue;
            const uint32_t ti = (t - k) / a.stride;
            if (ti >= a.in_length) continue;
            sum += a.x[(size_t)ic * a.in_length + ti] * ldw(a.w, (ic * out_pg + ocg) * a.kernel + k, a.w_dtype);
        }
    }
    a.y[(size_t)oc * a.out_length + t] = sum;
}

__global__ __launch_bounds__(256) void k_vae_snake_cm(const float *x, float *y, const void *alpha, uint32_t dtype,
                                                      uint32_t channels, uint32_t length) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x, c = blockIdx.y;
    if (t >= length || c >= channels) return;
    const size_t i = (size_t)c * length + t;
    y[i] = snake(x[i], ldw(alpha, c, dtype));
}

__global__ __launch_bounds__(256) void k_vae_scale_bias_cm(float *x, const void *scale, const void *bias,
                                                           uint32_t sdt, uint32_t bdt, uint32_t channels,
                                                           uint32_t length, uint32_t bucket) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x, c = blockIdx.y;
    if (t >= length || c >= channels) return;
    const size_t i = (size_t)c * length + t;
    const uint32_t idx = bucket * channels + c;
    x[i] = x[i] * ldw(scale, idx, sdt) + ldw(bias, idx, bdt);
}

__global__ __launch_bounds__(256) void k_vae_add_cm(float *a, const float *b, uint32_t channels, uint32_t length) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x, c = blockIdx.y;
    if (t >= length || c >= channels) return;
    const size_t i = (size_t)c * length + t;
    a[i] += b[i];
}

__global__ __launch_bounds__(256) void k_vae_tanh(float *x, uint32_t n) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < n) x[i] = tanhf(x[i]);
}

// -------------------------------------------------------------- frame-major
// Depthwise k-tap convolution over [L][C] rows, stride 1, dilation d, left pad
// (causal): y[t][c] = post(b[c] + sum_k w[c][k] pre(x[t + k d - pad][c])), where
// pre / post are the snake of alpha_in / alpha_out when given. One thread per
// (t, c), c fastest.
__global__ __launch_bounds__(256) void k_vae_dwconv_fm(VaeDwArgs a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (i >= (uint64_t)a.length * a.channels) return;
    const uint32_t t = (uint32_t)(i / a.channels), c = (uint32_t)(i - (uint64_t)t * a.channels);
    const float ain = a.alpha_in ? hf(a.alpha_in[c]) : 0.f;
    float sum = hf(a.b[c]);
    for (uint32_t k = 0; k < a.kernel; ++k) {
        const int ti = (int)(t + k * a.dilation) - (int)a.left_pad;
        if (ti < 0) continue;
        float v = a.x[(size_t)ti * a.channels + c];
        if (a.alpha_in) v = snake(v, ain);
        sum += v * hf(a.w[c * a.kernel + k]);
    }
    if (a.alpha_out) sum = snake(sum, hf(a.alpha_out[c]));
    a.y[i] = sum;
}

// The same convolution when left_pad = (kernel - 1) * dilation (the causal
// layers) and kernel <= KMAX, tiled: a workgroup covers TB = 2048 / CB rows of CB
// channels (CB a power of two <= 64, so each thread keeps one channel), stages
// pre(x) for its rows and their left halo in LDS once (pre(0) = 0, so the zero
// padding stays zero), then takes the taps from LDS with the channel's weights,
// bias and snake alphas in registers. Every staging load is issued before the
// first is used.
template <int KMAX>
__global__ __launch_bounds__(256) void k_vae_dwconv_tiled_fm(VaeDwArgs a, uint32_t cb_shift) {
    constexpr uint32_t kMaxHalo = 54u, NS = (2048u + 64u * kMaxHalo + 255u) / 256u;
    __shared__ float xs[2048 + 64 * kMaxHalo];
    const uint32_t CB = 1u << cb_shift, TB = 2048u >> cb_shift, halo = a.left_pad;
    const uint32_t t0 = blockIdx.x * TB, C = a.channels, tid = threadIdx.x;
    const uint32_t cc = tid & (CB - 1u), c = blockIdx.y * CB + cc;
    const bool cval = c < C;
    const uint32_t n_st = (TB + halo) << cb_shift;
    float xv[NS];
#pragma unroll
    for (uint32_t i = 0; i < NS; ++i) {
        const uint32_t idx = tid + 256u * i;
        const int ti = (int)(t0 + (idx >> cb_shift)) - (int)halo;
        xv[i] = idx < n_st && cval && ti >= 0 && (uint32_t)ti < a.length ? a.x[(size_t)ti * C + c] : 0.f;
    }
    const float ain = a.alpha_in && cval ? hf(a.alpha_in[c]) : 0.f;
    const float aout = a.alpha_out && cval ? hf(a.alpha_out[c]) : 0.f;
    const float iin = snake_inv(ain), iout = snake_inv(aout);
    const float bias = cval ? hf(a.b[c]) : 0.f;
    float wk[KMAX];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) wk[k] = cval && (uint32_t)k < a.kernel ? hf(a.w[c * a.kernel + k]) : 0.f;
#pragma unroll
    for (uint32_t i = 0; i < NS; ++i) {
        const uint32_t idx = tid + 256u * i;
        if (idx < n_st) xs[idx] = a.alpha_in ? snake_fm(xv[i], ain, iin) : xv[i];
    }
    __syncthreads();
#pragma unroll
    for (uint32_t i = 0; i < 8u; ++i) {   // TB * CB = 2048 outputs, 8 per thread
        const uint32_t r = (tid + 256u * i) >> cb_shift, t = t0 + r;
        if (t >= a.length || !cval) continue;
        float sum = bias;
#pragma unroll
        for (int k = 0; k < KMAX; ++k)
            if ((uint32_t)k < a.kernel) sum += xs[((r + k * a.dilation) << cb_shift) + cc] * wk[k];
        if (a.alpha_out) sum = snake_fm(sum, aout, iout);
        a.y[(size_t)t * C + c] = sum;
    }
}

// A residual unit of a narrow stage (C = 32 or 64 channels) in one pass: the
// workgroup stages snake_a1(x) for TB = 4096 / C rows and their causal halo
// (6 d rows) in LDS, computes the depthwise conv and snake_a2 into a second LDS
// tile, then the 1x1 conv with each thread's weight row in registers (the tile's
// row read as float4 broadcasts) plus bias and the residual x. Two launches and a
// round trip of the intermediate through HBM become one; every staging load is
// issued before the first is used. (At 128 channels the same pass, 93 KB of LDS
// and 128 FMAs per output on one workgroup per CU, took 79.5 us against 27.3 for
// the depthwise kernel plus the MFMA GEMM.)
template <int C>
__global__ __launch_bounds__(256) void k_vae_resunit_fm(VaeResUnitArgs a) {
    static_assert(C == 32 || C == 64, "narrow stages only");
    constexpr uint32_t TB = 4096u / C, kMaxHalo = 54u, K = 7u;
    constexpr uint32_t NS = ((TB + kMaxHalo) * C + 255u) / 256u;
    constexpr uint32_t G = 256u / C;   // row groups of the thread block
    __shared__ __align__(16) float xs[(TB + kMaxHalo) * C];
    __shared__ __align__(16) float hs[TB * C];
    const uint32_t tid = threadIdx.x, t0 = blockIdx.x * TB, halo = 6u * a.dilation;
    const uint32_t n_st = (TB + halo) * C;
    const uint32_t c = tid % C;   // n_st, C are multiples of 256 / C, so idx % C == c
    float xv[NS];
#pragma unroll
    for (uint32_t i = 0; i < NS; ++i) {
        const uint32_t idx = tid + 256u * i;
        const int ti = (int)(t0 + idx / C) - (int)halo;
        xv[i] = idx < n_st && ti >= 0 && (uint32_t)ti < a.length ? a.x[(size_t)ti * C + c] : 0.f;
    }
    const float a1 = hf(a.a1[c]), a2 = hf(a.a2[c]), db = hf(a.db[c]);
    const float i1 = snake_inv(a1), i2 = snake_inv(a2);
#pragma unroll
    for (uint32_t i = 0; i < NS; ++i) {
        const uint32_t idx = tid + 256u * i;
        if (idx < n_st) xs[idx] = snake_fm(xv[i], a1, i1);   // snake(0) = 0: the padding stays zero
    }
    float wk[K];
#pragma unroll
    for (uint32_t k = 0; k < K; ++k) wk[k] = hf(a.dw[c * K + k]);
    float pw[C];
#pragma unroll
    for (uint32_t j = 0; j < C; j += 8) {
        const uint4 u = *reinterpret_cast<const uint4 *>(a.pw + (size_t)c * C + j);
        const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const __half2 h = __builtin_bit_cast(__half2, uw[e]);
            pw[j + 2 * e] = __low2float(h);
            pw[j + 2 * e + 1] = __high2float(h);
        }
    }
    const float pb = hf(a.pb[c]);
    __syncthreads();
    for (uint32_t r = tid / C; r < TB; r += G) {
        float sum = db;
#pragma unroll
        for (uint32_t k = 0; k < K; ++k) sum += xs[(r + k * a.dilation) * C + c] * wk[k];
        hs[r * C + c] = snake_fm(sum, a2, i2);
    }
    __syncthreads();
    for (uint32_t r = tid / C; r < TB; r += G) {
        const uint32_t t = t0 + r;
        if (t >= a.length) break;
        const float4 *h4 = reinterpret_cast<const float4 *>(hs + r * C);
        float s0 = pb, s1 = 0.f;
#pragma unroll
        for (uint32_t j = 0; j < C / 4; ++j) {
            const float4 v = h4[j];
            s0 = fmaf(v.x, pw[4 * j], s0);
            s1 = fmaf(v.y, pw[4 * j + 1], s1);
            s0 = fmaf(v.z, pw[4 * j + 2], s0);
            s1 = fmaf(v.w, pw[4 * j + 3], s1);
        }
        a.y[(size_t)t * C + c] = a.x[(size_t)t * C + c] + (s0 + s1);
    }
}

// Input of a stride-s transposed convolution as a GEMM: row j of X2 is
// [pre(x[j]) | pre(x[j-1])] (zeros for j = 0), pre = snake(alpha)(x * scale + bias)
// with the per-channel scale/bias of the sample-rate bucket.
__global__ __launch_bounds__(256) void k_vae_convt_input_fm(VaeConvtInArgs a) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    const uint32_t C = a.channels;
    if (i >= (uint64_t)a.length * 2u * C) return;
    const uint32_t j = (uint32_t)(i / (2u * C)), r = (uint32_t)(i - (uint64_t)j * 2u * C);
    const uint32_t tap = r >= C ? 1u : 0u, c = r - tap * C;
    float v = 0.f;
    if (j >= tap) {
        const float x = a.x[(size_t)(j - tap) * C + c];
        const float pre = a.scale ? x * hf(a.scale[c]) + hf(a.bias[c]) : x;
        const float al = hf(a.alpha[c]);
        v = snake_fm(pre, al, snake_inv(al));
    }
    a.x2[i] = v;
}

// Repack of a ConvTranspose1d weight [Cin][Cout][2s] (kernel 2s, stride s) for
// the GEMM form: W'[(r Cout + oc)][tap Cin + ic] = W[ic][oc][r + tap s], and the
// bias tiled over the s phases, b'[r Cout + oc] = b[oc].
__global__ __launch_bounds__(256) void k_vae_repack_convt(const __half *w, const __half *b, uint32_t cin,
                                                          uint32_t cout, uint32_t s, __half *wp, float *bp) {
    const uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    const uint64_t n = (uint64_t)s * cout * 2u * cin;
    if (i < n) {
        const uint32_t row = (uint32_t)(i / (2u * cin)), col = (uint32_t)(i - (uint64_t)row * 2u * cin);
        const uint32_t r = row / cout, oc = row - r * cout, tap = col / cin, ic = col - tap * cin;
        wp[i] = w[((size_t)ic * cout + oc) * (2u * s) + r + tap * s];
    }
    if (i < (uint64_t)s * cout) bp[i] = hf(b[i % cout]);
}

// y[t][n] (+)= b[n] + sum_k x[t][k] W[n][k] for short K (the GEMM takes K % 128
// == 0): a workgroup covers NB = min(N, 256) outputs of RB rows, the rows staged
// in LDS; thread (g, n) computes rows g, g + G, ... (G = 256 / NB, at most
// kLinRows of them) together, reading W[n] once in 8-column chunks (K % 8 == 0).
constexpr uint32_t kLinRows = 8;
__global__ __launch_bounds__(256) void k_vae_linear_fm(VaeLinearArgs a, uint32_t NB, uint32_t RB) {
    extern __shared__ float xs[];
    const uint32_t tid = threadIdx.x, G = 256u / NB, n = blockIdx.x * NB + tid % NB, g = tid / NB;
    const uint32_t r0 = blockIdx.y * RB;
    for (uint32_t idx = tid; idx < RB * a.K; idx += 256u) {
        const uint32_t r = idx / a.K, k = idx - r * a.K;
        xs[idx] = r0 + r < a.T ? a.x[(size_t)(r0 + r) * a.ldx + k] : 0.f;
    }
    __syncthreads();
    if (n >= a.N || g >= G) return;
    const __half *w = a.w + (size_t)n * a.K;
    const float b = a.bias_f32 ? a.bias_f32[n] : (a.bias ? hf(a.bias[n]) : 0.f);
    float acc[kLinRows];
#pragma unroll
    for (uint32_t j = 0; j < kLinRows; ++j) acc[j] = 0.f;
    for (uint32_t k0 = 0; k0 < a.K; k0 += 8u) {
        const uint4 wc = *reinterpret_cast<const uint4 *>(w + k0);
        const uint32_t wu[4] = {wc.x, wc.y, wc.z, wc.w};
        float wf[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const __half2 h = __builtin_bit_cast(__half2, wu[e]);
            wf[2 * e] = __low2float(h);
            wf[2 * e + 1] = __high2float(h);
        }
#pragma unroll
        for (uint32_t j = 0; j < kLinRows; ++j) {
            const uint32_t r = g + G * j;
            if (r >= RB) break;
            const float *xr = xs + r * a.K + k0;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[j] += xr[e] * wf[e];
        }
    }
#pragma unroll
    for (uint32_t j = 0; j < kLinRows; ++j) {
        const uint32_t r = g + G * j;
        if (r >= RB || r0 + r >= a.T) break;
        const float v = acc[j] + b;
        float *dst = a.y + (size_t)(r0 + r) * a.ldy + n;
        *dst = a.residual ? *dst + v : v;
    }
}

// Any K and weight alignment: W[n][k] read element by element.
__global__ __launch_bounds__(256) void k_vae_linear_fm_any(VaeLinearArgs a, uint32_t NB, uint32_t RB) {
    extern __shared__ float xs[];
    const uint32_t tid = threadIdx.x, G = 256u / NB, n = blockIdx.x * NB + tid % NB, g = tid / NB;
    const uint32_t r0 = blockIdx.y * RB;
    for (uint32_t idx = tid; idx < RB * a.K; idx += 256u) {
        const uint32_t r = idx / a.K, k = idx - r * a.K;
        xs[idx] = r0 + r < a.T ? a.x[(size_t)(r0 + r) * a.ldx + k] : 0.f;
    }
    __syncthreads();
    if (n >= a.N || g >= G) return;
    const __half *w = a.w + (size_t)n * a.K;
    const float b = a.bias_f32 ? a.bias_f32[n] : (a.bias ? hf(a.bias[n]) : 0.f);
    for (uint32_t r = g; r < RB && r0 + r < a.T; r += G) {
        float sum = 0.f;
        for (uint32_t k = 0; k < a.K; ++k) sum += xs[r * a.K + k] * hf(w[k]);
        const float v = sum + b;
        float *dst = a.y + (size_t)(r0 + r) * a.ldy + n;
        *dst = a.residual ? *dst + v : v;
    }
}

// Decoder head: wave[t] = tanh(b + sum_c sum_k w[c][k] snake(x[t + k - pad][c])),
// one output channel (model.8 snake, model.9 conv, vae_tanh.comp).
__global__ __launch_bounds__(256) void k_vae_head_fm(VaeHeadArgs a) {
    const uint32_t t = blockIdx.x * 256u + threadIdx.x;
    if (t >= a.length) return;
    float sum = hf(a.b[0]);
    for (uint32_t c = 0; c < a.channels; ++c) {
        const float al = hf(a.alpha[c]);
        for (uint32_t k = 0; k < a.kernel; ++k) {
            const int ti = (int)(t + k) - (int)a.left_pad;
            if (ti < 0) continue;
            sum += snake(a.x[(size_t)ti * a.channels + c], al) * hf(a.w[c * a.kernel + k]);
        }
    }
    a.y[t] = tanhf(sum);
}

// The head tiled over 256 output rows: snake(x) of the rows and the left halo
// staged once in LDS (row stride C + 1), C <= 48, with the conv weights in LDS.
// For the decoder's 32 output channels (NC = 32) every staging load is issued
// before the first is used; NC = 0 takes any C with a plain staging loop.
template <uint32_t NC>
__global__ __launch_bounds__(256) void k_vae_head_tiled_fm(VaeHeadArgs a) {
    __shared__ float xs[(256 + 6) * 49];
    __shared__ float ws[48 * 7];
    const uint32_t C = NC ? NC : a.channels, S = C + 1u, t0 = blockIdx.x * 256u, halo = a.left_pad;
    const uint32_t n_st = (256u + halo) * C, tid = threadIdx.x;
    for (uint32_t i = tid; i < C * a.kernel; i += 256u) ws[i] = hf(a.w[i]);
    if constexpr (NC != 0) {
        constexpr uint32_t NS = ((256u + 6u) * NC + 255u) / 256u;
        float xv[NS];
#pragma unroll
        for (uint32_t i = 0; i < NS; ++i) {
            const uint32_t idx = tid + 256u * i, r = idx / NC, c = idx % NC;
            const int ti = (int)(t0 + r) - (int)halo;
            xv[i] = idx < n_st && ti >= 0 && (uint32_t)ti < a.length ? a.x[(size_t)ti * NC + c] : 0.f;
        }
        const uint32_t c = tid % NC;   // NC divides 256: each thread keeps one channel
        const float al = hf(a.alpha[c]), inv = snake_inv(al);
#pragma unroll
        for (uint32_t i = 0; i < NS; ++i) {
            const uint32_t idx = tid + 256u * i;
            if (idx < n_st) xs[(idx / NC) * S + c] = snake_fm(xv[i], al, inv);   // snake(0) = 0
        }
    } else {
        for (uint32_t idx = tid; idx < n_st; idx += 256u) {
            const uint32_t r = idx / C, c = idx - r * C;
            const int ti = (int)(t0 + r) - (int)halo;
            const float al = hf(a.alpha[c]);
            xs[r * S + c] = ti >= 0 && (uint32_t)ti < a.length ? snake_fm(a.x[(size_t)ti * C + c], al, snake_inv(al))
                                                               : 0.f;
        }
    }
    __syncthreads();
    const uint32_t t = t0 + tid;
    if (t >= a.length) return;
    float sum = hf(a.b[0]);
    for (uint32_t c = 0; c < C; ++c)
        for (uint32_t k = 0; k < a.kernel; ++k) sum += xs[(tid + k) * S + c] * ws[c * a.kernel + k];
    a.y[t] = tanhf(sum);
}

unsigned grid1(uint64_t n) { return (unsigned)((n + 255u) / 256u); }

}  // namespace

int launch_vae_conv1d_cm(hipStream_t s, const VaeConvArgs &a, bool transpose) {
    if (!a.out_length || !a.out_channels) return VX_OK;
    const dim3 g(grid1(a.out_length), a.out_channels);
    if (transpose) {
        k_vae_convt1d_cm<<<g, 256, 0, s>>>(a);
        VX_LAUNCHED("k_vae_convt1d_cm");
    } else {
        k_vae_conv1d_cm<<<g, 256, 0, s>>>(a);
        VX_LAUNCHED("k_vae_conv1d_cm");
    }
    return VX_OK;
}

int launch_vae_snake_cm(hipStream_t s, const float *x, float *y, const void *alpha, uint32_t dtype, uint32_t c,
                        uint32_t len) {
    if (!c || !len) return VX_OK;
    k_vae_snake_cm<<<dim3(grid1(len), c), 256, 0, s>>>(x, y, alpha, dtype, c, len);
    VX_LAUNCHED("k_vae_snake_cm");
    return VX_OK;
}

int launch_vae_scale_bias_cm(hipStream_t s, float *x, const void *scale, const void *bias, uint32_t sdt,
                             uint32_t bdt, uint32_t c, uint32_t len, uint32_t bucket) {
    if (!c || !len) return VX_OK;
    k_vae_scale_bias_cm<<<dim3(grid1(len), c), 256, 0, s>>>(x, scale, bias, sdt, bdt, c, len, bucket);
    VX_LAUNCHED("k_vae_scale_bias_cm");
    return VX_OK;
}

int launch_vae_add_cm(hipStream_t s, float *a, const float *b, uint32_t c, uint32_t len) {
    if (!c || !len) return VX_OK;
    k_vae_add_cm<<<dim3(grid1(len), c), 256, 0, s>>>(a, b, c, len);
    VX_LAUNCHED("k_vae_add_cm");
    return VX_OK;
}

int launch_vae_tanh(hipStream_t s, float *x, uint32_t n) {
    if (!n) return VX_OK;
    k_vae_tanh<<<grid1(n), 256, 0, s>>>(x, n);
    VX_LAUNCHED("k_vae_tanh");
    return VX_OK;
}

int launch_vae_dwconv_fm(hipStream_t s, const VaeDwArgs &a) {
    const uint64_t n = (uint64_t)a.length * a.channels;
    if (!n) return VX_OK;
    if (a.kernel >= 1u && a.kernel <= 8u && a.left_pad == (a.kernel - 1u) * a.dilation && a.left_pad <= 54u) {
        const uint32_t CB = a.channels < 64u ? a.channels : 64u;   // >= 1; 2048 / CB rows per workgroup
        if ((CB & (CB - 1u)) == 0) {
            const uint32_t sh = (uint32_t)__builtin_ctz(CB), cblocks = (a.channels + CB - 1u) / CB;
            const uint32_t tb = 2048u >> sh;
            k_vae_dwconv_tiled_fm<8><<<dim3((a.length + tb - 1u) / tb, cblocks), 256, 0, s>>>(a, sh);
            VX_LAUNCHED("k_vae_dwconv_tiled_fm");
            return VX_OK;
        }
    }
    k_vae_dwconv_fm<<<grid1(n), 256, 0, s>>>(a);
    VX_LAUNCHED("k_vae_dwconv_fm");
    return VX_OK;
}

bool vae_resunit_eligible(const VaeResUnitArgs &a) {
    const bool aligned = ((reinterpret_cast<uintptr_t>(a.pw) | reinterpret_cast<uintptr_t>(a.x) |
                           reinterpret_cast<uintptr_t>(a.y)) & 15u) == 0;
    return (a.channels == 32u || a.channels == 64u) && a.dilation >= 1u &&
           6u * a.dilation <= 54u && aligned && a.x != a.y;
}

int launch_vae_resunit_fm(hipStream_t s, const VaeResUnitArgs &a) {
    if (!a.length) return VX_OK;
    if (!vae_resunit_eligible(a)) return fail(VX_ERR_UNSUPPORTED, "vae residual unit: %u channels, dilation %u",
                                              a.channels, a.dilation);
    const uint32_t tb = 4096u / a.channels;
    const uint32_t grid = (a.length + tb - 1u) / tb;
    if (a.channels == 32u)
        k_vae_resunit_fm<32><<<grid, 256, 0, s>>>(a);
    else
        k_vae_resunit_fm<64><<<grid, 256, 0, s>>>(a);
    VX_LAUNCHED("k_vae_resunit_fm");
    return VX_OK;
}

int launch_vae_convt_input_fm(hipStream_t s, const VaeConvtInArgs &a) {
    const uint64_t n = (uint64_t)a.length * 2u * a.channels;
    if (!n) return VX_OK;
    k_vae_convt_input_fm<<<grid1(n), 256, 0, s>>>(a);
    VX_LAUNCHED("k_vae_convt_input_fm");
    return VX_OK;
}

int launch_vae_repack_convt(hipStream_t s, const __half *w, const __half *b, uint32_t cin, uint32_t cout,
                            uint32_t stride, __half *wp, float *bp) {
    const uint64_t n = (uint64_t)stride * cout * 2u * cin;
    k_vae_repack_convt<<<grid1(n), 256, 0, s>>>(w, b, cin, cout, stride, wp, bp);
    VX_LAUNCHED("k_vae_repack_convt");
    return VX_OK;
}

int launch_vae_linear_fm(hipStream_t s, const VaeLinearArgs &a) {
    if (!a.T || !a.N) return VX_OK;
    if (a.K > 4096u) return fail(VX_ERR_UNSUPPORTED, "vae linear: K %u > 4096", a.K);
    const bool chunks = a.K % 8u == 0 && (reinterpret_cast<uintptr_t>(a.w) & 15u) == 0;
    const uint32_t NB = a.N < 256u ? a.N : 256u, G = 256u / NB;
    uint32_t rpt = 8192u / (G * a.K);
    rpt = rpt < 1u ? 1u : (rpt > kLinRows ? kLinRows : rpt);
    const uint32_t RB = G * rpt;   // RB * K <= max(8192, G * K) floats
    if ((uint64_t)RB * a.K * 4u > 65536u)
        return fail(VX_ERR_UNSUPPORTED, "vae linear: %u rows x K %u exceed the LDS tile", RB, a.K);
    const dim3 grid((a.N + NB - 1u) / NB, (a.T + RB - 1u) / RB);
    if (chunks) {
        k_vae_linear_fm<<<grid, 256, (size_t)RB * a.K * 4u, s>>>(a, NB, RB);
        VX_LAUNCHED("k_vae_linear_fm");
    } else {
        k_vae_linear_fm_any<<<grid, 256, (size_t)RB * a.K * 4u, s>>>(a, NB, RB);
        VX_LAUNCHED("k_vae_linear_fm_any");
    }
    return VX_OK;
}

int launch_vae_head_fm(hipStream_t s, const VaeHeadArgs &a) {
    if (!a.length) return VX_OK;
    if (a.channels <= 48u && a.left_pad <= 6u && a.kernel == a.left_pad + 1u) {
        if (a.channels == 32u)
            k_vae_head_tiled_fm<32><<<grid1(a.length), 256, 0, s>>>(a);
        else
            k_vae_head_tiled_fm<0><<<grid1(a.length), 256, 0, s>>>(a);
        VX_LAUNCHED("k_vae_head_tiled_fm");
        return VX_OK;
    }
    k_vae_head_fm<<<grid1(a.length), 256, 0, s>>>(a);
    VX_LAUNCHED("k_vae_head_fm");
    return VX_OK;
}

}  // namespace vx
