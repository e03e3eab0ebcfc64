// Small single-workgroup and elementwise kernels of the decode step:
// rmsnorm, residual_rmsnorm, rope, store_kv, embedding gather, step bookkeeping.
#include "vx_internal.h"

namespace vx {
namespace {

__device__ __forceinline__ float h2f(unsigned short bits) {
    return (float)__builtin_bit_cast(_Float16, bits);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Sum over a 256-thread block; every thread receives the total.
__device__ __forceinline__ float block_sum256(float v, float *red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    const float t = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
    return t;
}

// rmsnorm.comp:21-42. When `advance` is set, thread 0 bumps the device decode
// position afterwards (the last kernel of an engine step).
__global__ __launch_bounds__(256) void k_rmsnorm(const float *x, float *y, const float *w, uint32_t n,
                                                 float eps, uint32_t *advance) {
    __shared__ float red[4];
    float s = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += 256) {
        const float v = x[i];
        s += v * v;
    }
    s = block_sum256(s, red);
    const float inv_rms = 1.0f / sqrtf(s / (float)n + eps);
    for (uint32_t i = threadIdx.x; i < n; i += 256) y[i] = x[i] * inv_rms * w[i];
    if (advance && threadIdx.x == 0) *advance = *advance + 1u;
}

// residual_rmsnorm.comp:23-42.
__global__ __launch_bounds__(256) void k_residual_rmsnorm(float *h, const float *branch, float *y,
                                                          const float *w, uint32_t n, float eps,
                                                          float scale) {
    __shared__ float red[4];
    float s = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += 256) {
        const float v = h[i] + branch[i] * scale;
        h[i] = v;
        s += v * v;
    }
    s = block_sum256(s, red);
    const float inv_rms = 1.0f / sqrtf(s / (float)n + eps);
    for (uint32_t i = threadIdx.x; i < n; i += 256) y[i] = h[i] * inv_rms * w[i];
}

// rope.comp:22-51: block = head (q heads then kv heads), lane = rotary pair.
__global__ __launch_bounds__(64) void k_rope(float *q, float *k, const float *factors, uint32_t pos_in,
                                             const uint32_t *dev_pos, uint32_t q_heads, uint32_t kv_heads,
                                             uint32_t head_dim, float theta, float scaling) {
    const uint32_t pair = threadIdx.x, head = blockIdx.x;
    const uint32_t half_dim = head_dim / 2u;
    if (pair >= half_dim) return;
    const uint32_t position = dev_pos ? *dev_pos : pos_in;
    const float ext = factors[pair];
    const float exponent = (float)(pair * 2u) / (float)head_dim;
    const float inv_freq = 1.0f / powf(theta, exponent);
    const float angle = (float)position * inv_freq / ext;
    const float c = cosf(angle) * scaling;
    const float s = sinf(angle) * scaling;
    float *buf;
    uint32_t base;
    if (head < q_heads) {
        buf = q;
        base = head * head_dim;
    } else {
        if (head - q_heads >= kv_heads) return;
        buf = k;
        base = (head - q_heads) * head_dim;
    }
    const float a = buf[base + pair];
    const float b = buf[base + pair + half_dim];
    buf[base + pair] = a * c - b * s;
    buf[base + pair + half_dim] = b * c + a * s;
}

// store_kv.comp:16-24: packed f16 pairs at word (layer*context+position)*kv_dim/2 + w.
__global__ __launch_bounds__(128) void k_store_kv(const float *k, const float *v, uint32_t *kc, uint32_t *vc,
                                                  uint32_t layer, uint32_t pos_in, const uint32_t *dev_pos,
                                                  uint32_t context, uint32_t kv_dim) {
    const uint32_t word_i = threadIdx.x;
    const uint32_t words_per_token = kv_dim / 2u;
    if (word_i >= words_per_token) return;
    const uint32_t position = dev_pos ? *dev_pos : pos_in;
    if (position >= context) return;
    const uint32_t d = word_i * 2u;
    const size_t dst = ((size_t)layer * context + position) * words_per_token + word_i;
    const __half k0 = __float2half_rn(k[d]), k1 = __float2half_rn(k[d + 1u]);
    const __half v0 = __float2half_rn(v[d]), v1 = __float2half_rn(v[d + 1u]);
    kc[dst] = (uint32_t)__half_as_ushort(k0) | ((uint32_t)__half_as_ushort(k1) << 16);
    vc[dst] = (uint32_t)__half_as_ushort(v0) | ((uint32_t)__half_as_ushort(v1) << 16);
}

// embedding.comp:28-48: hidden[i] = load_weight(token, i) * alpha from the raw
// GGUF region (F16 or Q8_0 blocks), so the gather is bit-exact.
__global__ __launch_bounds__(256) void k_embedding(const uint8_t *raw, uint32_t off, uint32_t dtype,
                                                   uint32_t cols, uint32_t token_in,
                                                   const uint32_t *dev_tokens, const uint32_t *dev_pos,
                                                   uint32_t tokens_len, uint32_t vocab, float alpha,
                                                   float *hidden) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= cols) return;
    uint32_t token = token_in;
    if (dev_tokens) {
        const uint32_t p = *dev_pos;
        token = p < tokens_len ? dev_tokens[p] : vocab;
    }
    if (token >= vocab) {
        hidden[i] = __int_as_float(0x7fc00000);
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
    hidden[i] = w * alpha;
}

// Per-step RoPE table: table[i] = (cos(angle)*scaling, sin(angle)*scaling) for
// rotary pair i at the device decode position, with rope.comp's angle
// pos * theta^(-2i/d) / ext[i] (rope.comp:28-41). Every layer's fused QKV kernel
// reads its pair from here, so the transcendentals run once per step.
__global__ __launch_bounds__(64) void k_rope_table(const float *factors, const uint32_t *position,
                                                   uint32_t head_dim, float theta, float scaling,
                                                   float2 *table) {
    const uint32_t i = threadIdx.x;
    if (i >= head_dim / 2u) return;
    const uint32_t pos = *position;
    const float exponent = (float)(i * 2u) / (float)head_dim;
    const float inv_freq = 1.0f / powf(theta, exponent);
    const float angle = (float)pos * inv_freq / factors[i];
    table[i] = make_float2(cosf(angle) * scaling, sinf(angle) * scaling);
}

__global__ void k_set_step(uint32_t *tokens, uint32_t *position, uint32_t pos, uint32_t token,
                           int write_token) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        position[0] = pos;
        if (write_token) tokens[pos] = token;
    }
}

__global__ void k_fill_u32(uint32_t *dst, uint32_t value, uint64_t count) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = value;
}

}  // namespace

int launch_rmsnorm(hipStream_t s, const float *x, float *y, const float *w, uint32_t n, float eps,
                   uint32_t *advance_position) {
    k_rmsnorm<<<1, 256, 0, s>>>(x, y, w, n, eps, advance_position);
    VX_LAUNCHED("k_rmsnorm");
    return VX_OK;
}

int launch_residual_rmsnorm(hipStream_t s, float *h, const float *branch, float *y, const float *w,
                            uint32_t n, float eps, float scale) {
    k_residual_rmsnorm<<<1, 256, 0, s>>>(h, branch, y, w, n, eps, scale);
    VX_LAUNCHED("k_residual_rmsnorm");
    return VX_OK;
}

int launch_rope(hipStream_t s, float *q, float *k, const float *factors, uint32_t position,
                const uint32_t *dev_position, uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim,
                float theta, float scaling) {
    if (q_heads + kv_heads == 0) return VX_OK;
    k_rope<<<q_heads + kv_heads, 64, 0, s>>>(q, k, factors, position, dev_position, q_heads, kv_heads,
                                              head_dim, theta, scaling);
    VX_LAUNCHED("k_rope");
    return VX_OK;
}

int launch_store_kv(hipStream_t s, const float *k, const float *v, __half *kc, __half *vc, uint32_t layer,
                    uint32_t position, const uint32_t *dev_position, uint32_t context, uint32_t kv_dim) {
    k_store_kv<<<1, 128, 0, s>>>(k, v, reinterpret_cast<uint32_t *>(kc), reinterpret_cast<uint32_t *>(vc),
                                 layer, position, dev_position, context, kv_dim);
    VX_LAUNCHED("k_store_kv");
    return VX_OK;
}

int launch_embedding(hipStream_t s, const uint8_t *raw, uint32_t weight_offset, uint32_t dtype,
                     uint32_t cols, uint32_t token, const uint32_t *dev_tokens,
                     const uint32_t *dev_position, uint32_t vocab, float alpha, float *hidden,
                     uint32_t tokens_len) {
    if (!cols) return VX_OK;
    k_embedding<<<(cols + 255u) / 256u, 256, 0, s>>>(raw, weight_offset, dtype, cols, token, dev_tokens,
                                                     dev_position, tokens_len, vocab, alpha, hidden);
    VX_LAUNCHED("k_embedding");
    return VX_OK;
}

int launch_rope_table(hipStream_t s, const float *factors, const uint32_t *position, uint32_t head_dim,
                      float theta, float scaling, float2 *table) {
    if (head_dim == 0 || head_dim > 128u || (head_dim & 1u))
        return fail(VX_ERR_UNSUPPORTED, "rope table: head_dim must be even and <= 128");
    k_rope_table<<<1, 64, 0, s>>>(factors, position, head_dim, theta, scaling, table);
    VX_LAUNCHED("k_rope_table");
    return VX_OK;
}

int launch_set_step(hipStream_t s, uint32_t *tokens, uint32_t *position, uint32_t pos, uint32_t token,
                    int write_token) {
    k_set_step<<<1, 64, 0, s>>>(tokens, position, pos, token, write_token);
    VX_LAUNCHED("k_set_step");
    return VX_OK;
}

int launch_fill_u32(hipStream_t s, uint32_t *dst, uint32_t value, uint64_t count) {
    uint64_t blocks = (count + 255u) / 256u;
    if (blocks > 4096u) blocks = 4096u;
    k_fill_u32<<<(unsigned)blocks, 256, 0, s>>>(dst, value, count);
    VX_LAUNCHED("k_fill_u32");
    return VX_OK;
}

}  // namespace vx
