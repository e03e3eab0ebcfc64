/*
 * voxref.c — CPU oracle for the VoxCPM2 BaseLM compute path.
 *
 * TEST INFRASTRUCTURE ONLY (see voxref.h). Restates VoxGen's Normal-mode
 * shaders and record_transformer; never linked into the product library.
 *
 * Pinning (what checks each function independently of this file's formulas;
 * the tests live in tests/test_oracle_pins.py):
 *   vr_f16_to_f32 / vr_f32_to_f16  all 65536 halves vs numpy float16; RNE ties,
 *                                  overflow, subnormal, NaN classes vs numpy.
 *   vr_dequant (Q8_0, F16)          numpy structured-dtype decode of the block
 *                                  bytes (gguf.rs:41-45 layout), bit-exact.
 *   vr_embedding                    numpy row gather, bit-exact; alpha scaling.
 *   vr_matvec / vr_qkv_matvec /     f64 numpy W@x on the numpy-decoded W
 *   vr_linear_bias / vr_fusion_linear (rel-L2 <= 1e-6); one-hot x recovers a
 *                                  column; linearity in x.
 *   vr_matvec_swiglu                f64 silu(g)*u closed form; silu(0)=0.
 *   vr_rmsnorm / vr_residual_rmsnorm f64 closed form; scale invariance.
 *   vr_rope                         complex-number NeoX rotation (f64);
 *                                  position 0 is the identity; pair norms kept.
 *   vr_store_kv                     numpy index formula + float16 RNE, bit-exact.
 *   vr_attn_scores/softmax/values   f64 numpy softmax(qK^T/sqrt(d))V with the
 *                                  GQA map kv = q/q_per_kv; rows sum to 1.
 *   vr_baselm_record                f64 numpy re-derivation of one layer from
 *                                  the closed forms above (not this file's code).
 *   vr_rope_scaling_factor,         reference unit tests baselm.rs:1319-1358 and
 *   vr_effective_scale              closed forms.
 *   vr_mix32                        the published inverse of this finaliser
 *                                  (lowbias32 family) undoes it on 10^5
 *                                  values; mix32(0) = 0.
 *   vr_cfm_noise                    the hash words bit-exact against vr_mix32;
 *                                  Box-Muller pairs against f64 numpy; the
 *                                  sample mean/variance of 2^16 draws.
 *   vr_cfm_cfg_euler                f64 numpy closed form of the CFG-Zero*
 *                                  update; zero_star off = plain CFG; cfg = 1
 *                                  reduces to the positive estimate.
 *   vr_time_sinusoidal              f64 numpy closed form; t = 0 gives 0 / 1.
 *   vr_pack_locdit                  numpy concatenation; zero_mu rows are 0.
 *   vr_cfm_time_span                closed form; endpoints 1 and 0; sway = 0
 *                                  gives the linear grid; descending check.
 *   vr_fsq_quantize                 the known answer of acoustic.rs:1266-1271
 *                                  (0.42 at scale 9 -> 4/9); f64 numpy
 *                                  round-half-away(tanh(x)*s)/s; outputs on the
 *                                  grid k/s with |k| <= s; odd symmetry.
 *   vr_silu_inplace                 f64 x/(1+e^-x); silu(0) = 0.
 *   vr_vae_conv1d                   f64 numpy gather over shifted slices
 *                                  (groups, stride, dilation, causal pad).
 *   vr_vae_convt1d                  f64 numpy scatter form out[ti s + k] +=
 *                                  x[ti] w[k] (PyTorch ConvTranspose1d), cropped.
 *   vr_vae_snake / scale_bias / add / tanh  f64 closed forms.
 *   vr_residual_lm_record           f64 numpy re-derivation of one layer
 *                                  without RoPE; equals vr_baselm_record at
 *                                  position 0, where RoPE is the identity.
 * Parity unpinned at the bit level (inside the float tolerances): the
 * driver's rounding of exp/sin/cos/pow/inversesqrt and FMA contraction.
 */
#include "voxref.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- halves */
float vr_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t mant = (uint32_t)h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {
            /* subnormal: mant * 2^-24, renormalised */
            int e = -1;
            do {
                e++;
                mant <<= 1;
            } while ((mant & 0x400u) == 0);
            bits = sign | ((uint32_t)(112 - e) << 23) | ((mant & 0x3ffu) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t vr_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t mant = x & 0x7fffffu;
    if (exp == 0xffu) {
        if (mant) return (uint16_t)(sign | 0x7e00u | (mant >> 13));
        return (uint16_t)(sign | 0x7c00u);
    }
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m24 = mant | 0x800000u;
        int shift = 14 - e;
        uint32_t hm = m24 >> shift;
        uint32_t rem = m24 & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

static float g_half_lut[65536];
static pthread_once_t g_lut_once = PTHREAD_ONCE_INIT;
static void lut_init(void) {
    for (uint32_t i = 0; i < 65536u; ++i) g_half_lut[i] = vr_f16_to_f32((uint16_t)i);
}
static inline float h2f(uint32_t bits) { return g_half_lut[bits & 0xffffu]; }
static inline void ensure_lut(void) { pthread_once(&g_lut_once, lut_init); }

void vr_f16_to_f32_n(const uint16_t *src, float *dst, uint64_t n) {
    ensure_lut();
    for (uint64_t i = 0; i < n; ++i) dst[i] = h2f(src[i]);
}
void vr_f32_to_f16_n(const float *src, uint16_t *dst, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) dst[i] = vr_f32_to_f16(src[i]);
}

/* ------------------------------------------------- model-buffer word loads */
/* The shaders read the model buffer as u32 words (matvec.comp:19-30). */
static inline uint32_t word_at(const uint8_t *blob, uint32_t o) {
    uint32_t w;
    memcpy(&w, blob + (o & ~3u), 4);
    return w;
}
static inline uint32_t load_u8(const uint8_t *blob, uint32_t o) {
    return (word_at(blob, o) >> ((o & 3u) * 8u)) & 0xffu;
}
static inline float load_f16(const uint8_t *blob, uint32_t o) {
    return h2f((word_at(blob, o) >> ((o & 2u) * 8u)) & 0xffffu);
}
static inline float load_f32(const uint8_t *blob, uint32_t o) {
    uint32_t w = word_at(blob, o);
    float f;
    memcpy(&f, &w, 4);
    return f;
}

/* Q8_0 element (matvec.comp:36-43). */
static inline float q8_weight(const uint8_t *blob, uint32_t off, uint32_t cols, uint32_t row,
                              uint32_t col) {
    uint32_t blocks_per_row = cols / 32u;
    uint32_t block = row * blocks_per_row + col / 32u;
    uint32_t base = off + block * 34u;
    float d = load_f16(blob, base);
    uint32_t raw = load_u8(blob, base + 2u + (col & 31u));
    int q = raw < 128u ? (int)raw : (int)raw - 256;
    return d * (float)q;
}

/* matvec.comp load_weight: dtype 1 = F16, anything else = Q8_0. */
static inline float mv_weight(const uint8_t *blob, uint32_t off, uint32_t dtype, uint32_t cols,
                              uint32_t row, uint32_t col) {
    if (dtype == 1u) return load_f16(blob, off + row * (cols * 2u) + col * 2u);
    return q8_weight(blob, off, cols, row, col);
}
/* linear_bias.comp / fusion_linear.comp load_weight: 0 = F32, 1 = F16, else Q8_0. */
static inline float lb_weight(const uint8_t *blob, uint32_t off, uint32_t dtype, uint32_t cols,
                              uint32_t row, uint32_t col) {
    if (dtype == 0u) return load_f32(blob, off + (row * cols + col) * 4u);
    if (dtype == 1u) return load_f16(blob, off + (row * cols + col) * 2u);
    return q8_weight(blob, off, cols, row, col);
}

float vr_load_weight(const uint8_t *blob, uint32_t weight_offset, uint32_t dtype, uint32_t cols,
                     uint32_t row, uint32_t col) {
    ensure_lut();
    return lb_weight(blob, weight_offset, dtype, cols, row, col);
}

void vr_dequant(const uint8_t *blob, uint32_t weight_offset, uint32_t dtype, uint32_t rows,
                uint32_t cols, float *out) {
    ensure_lut();
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < (int64_t)rows; ++r)
        for (uint32_t c = 0; c < cols; ++c)
            out[(uint64_t)r * cols + c] = lb_weight(blob, weight_offset, dtype, cols, (uint32_t)r, c);
}

/* ------------------------------------------------------ workgroup helpers */
/* Shared-memory tree over 256 partials (matvec.comp:57-60). */
static inline float tree_sum(float *p, uint32_t width) {
    for (uint32_t stride = width / 2u; stride > 0u; stride >>= 1u)
        for (uint32_t l = 0; l < stride; ++l) p[l] += p[l + stride];
    return p[0];
}
static inline float tree_max(float *p, uint32_t width) {
    for (uint32_t stride = width / 2u; stride > 0u; stride >>= 1u)
        for (uint32_t l = 0; l < stride; ++l) p[l] = p[l] > p[l + stride] ? p[l] : p[l + stride];
    return p[0];
}

/* Decode weights [base, base+n) of one row into wbuf. The values are exactly
 * the shader's load_weight results (d*float(q) for Q8_0, widened halves for
 * F16); only the loads are batched. kind 0 = matvec.comp family (1 = F16,
 * else Q8_0); kind 1 = linear_bias.comp family (0 = F32, 1 = F16, else Q8_0). */
static void decode_chunk(const uint8_t *blob, uint32_t off, uint32_t dtype, int kind, uint32_t cols,
                         uint32_t row, uint32_t base, uint32_t n, float *wbuf) {
    if (kind == 1 && dtype == 0u) {
        for (uint32_t l = 0; l < n; ++l) wbuf[l] = load_f32(blob, off + (row * cols + base + l) * 4u);
        return;
    }
    if (dtype == 1u) {
        for (uint32_t l = 0; l < n; ++l) wbuf[l] = load_f16(blob, off + (row * cols + base + l) * 2u);
        return;
    }
    uint32_t l = 0;
    while (l < n) {
        uint32_t col = base + l;
        uint32_t block = row * (cols / 32u) + col / 32u;
        uint32_t bb = off + block * 34u;
        float d = load_f16(blob, bb);
        uint32_t end = (col | 31u) + 1u - base;
        if (end > n) end = n;
        for (; l < end; ++l) {
            uint32_t raw = load_u8(blob, bb + 2u + ((base + l) & 31u));
            int q = raw < 128u ? (int)raw : (int)raw - 256;
            wbuf[l] = d * (float)q;
        }
    }
}

/* One 256-lane workgroup dot product: lane l accumulates columns l, l+256, ...
 * in order (matvec.comp:51-54), then the shared-memory tree. The chunk loop
 * keeps that per-lane order while letting the compiler vectorise across lanes. */
#define WG 256u
static float wg_row_dot(const uint8_t *blob, uint32_t off, uint32_t dtype, int kind, uint32_t cols,
                        uint32_t row, const float *x) {
    float partial[WG];
    float wbuf[WG];
    for (uint32_t l = 0; l < WG; ++l) partial[l] = 0.0f;
    for (uint32_t base = 0; base < cols; base += WG) {
        uint32_t n = cols - base < WG ? cols - base : WG;
        decode_chunk(blob, off, dtype, kind, cols, row, base, n, wbuf);
        for (uint32_t l = 0; l < n; ++l) partial[l] += wbuf[l] * x[base + l];
    }
    return tree_sum(partial, WG);
}

/* ------------------------------------------------------------------ ops */
void vr_embedding(const uint8_t *blob, float *hidden, const vx_embedding_push *pc) {
    ensure_lut(); /* embedding.comp:43-48 */
    for (uint32_t i = 0; i < pc->cols; ++i)
        hidden[i] = mv_weight(blob, pc->weight_offset, pc->dtype, pc->cols, pc->token_id, i) * pc->alpha;
}

void vr_rmsnorm(const uint8_t *blob, const float *x, float *y, const vx_rms_push *pc) {
    float partial[WG]; /* rmsnorm.comp:21-42 */
    for (uint32_t l = 0; l < WG; ++l) {
        float sum = 0.0f;
        for (uint32_t i = l; i < pc->n; i += WG) {
            float v = x[i];
            sum += v * v;
        }
        partial[l] = sum;
    }
    float s = tree_sum(partial, WG);
    float inv_rms = 1.0f / sqrtf(s / (float)pc->n + pc->eps);
    for (uint32_t i = 0; i < pc->n; ++i) y[i] = x[i] * inv_rms * load_f32(blob, pc->weight_offset + i * 4u);
}

void vr_residual_rmsnorm(const uint8_t *blob, float *hidden, const float *branch, float *y,
                         const vx_residual_rms_push *pc) {
    float partial[WG]; /* residual_rmsnorm.comp:23-42 */
    for (uint32_t l = 0; l < WG; ++l) {
        float sum = 0.0f;
        for (uint32_t i = l; i < pc->n; i += WG) {
            float v = hidden[i] + branch[i] * pc->scale;
            hidden[i] = v;
            sum += v * v;
        }
        partial[l] = sum;
    }
    float s = tree_sum(partial, WG);
    float inv_rms = 1.0f / sqrtf(s / (float)pc->n + pc->eps);
    for (uint32_t i = 0; i < pc->n; ++i)
        y[i] = hidden[i] * inv_rms * load_f32(blob, pc->weight_offset + i * 4u);
}

void vr_matvec(const uint8_t *blob, const float *x, float *y, const vx_matvec_push *pc) {
    ensure_lut(); /* matvec.comp:46-62 over every row the host loop dispatches */
#pragma omp parallel for schedule(static)
    for (int64_t r = pc->row_base; r < (int64_t)pc->rows; ++r)
        y[r] = wg_row_dot(blob, pc->weight_offset, pc->dtype, 0, pc->cols, (uint32_t)r, x) * pc->alpha;
}

void vr_qkv_matvec(const uint8_t *blob, const float *x, float *q, float *k, float *v,
                   const vx_qkv_push *pc) {
    ensure_lut(); /* qkv_matvec.comp:53-95 */
    uint32_t total = pc->q_rows + 2u * pc->kv_rows;
#pragma omp parallel for schedule(static)
    for (int64_t cr = pc->row_base; cr < (int64_t)total; ++cr) {
        uint32_t combined = (uint32_t)cr, off, dtype, row;
        float *dst;
        if (combined < pc->q_rows) {
            off = pc->q_weight_offset; dtype = pc->q_dtype; row = combined; dst = q;
        } else if (combined < pc->q_rows + pc->kv_rows) {
            off = pc->k_weight_offset; dtype = pc->k_dtype; row = combined - pc->q_rows; dst = k;
        } else {
            off = pc->v_weight_offset; dtype = pc->v_dtype; row = combined - pc->q_rows - pc->kv_rows; dst = v;
        }
        dst[row] = wg_row_dot(blob, off, dtype, 0, pc->cols, row, x);
    }
}

void vr_matvec_swiglu(const uint8_t *blob, const float *x, float *y, const vx_swiglu_push *pc) {
    ensure_lut(); /* matvec_swiglu.comp:44-69 */
#pragma omp parallel for schedule(static)
    for (int64_t r = pc->row_base; r < (int64_t)pc->rows; ++r) {
        float gp[WG], up[WG], gw[WG], uw[WG];
        for (uint32_t l = 0; l < WG; ++l) gp[l] = up[l] = 0.0f;
        for (uint32_t base = 0; base < pc->cols; base += WG) {
            uint32_t n = pc->cols - base < WG ? pc->cols - base : WG;
            decode_chunk(blob, pc->gate_weight_offset, pc->dtype, 0, pc->cols, (uint32_t)r, base, n, gw);
            decode_chunk(blob, pc->up_weight_offset, pc->dtype, 0, pc->cols, (uint32_t)r, base, n, uw);
            for (uint32_t l = 0; l < n; ++l) {
                float xv = x[base + l];
                gp[l] += gw[l] * xv;
                up[l] += uw[l] * xv;
            }
        }
        float g = tree_sum(gp, WG);
        float u = tree_sum(up, WG);
        y[r] = (g / (1.0f + expf(-g))) * u;
    }
}

void vr_rope(const uint8_t *blob, float *q, float *k, const vx_rope_push *pc) {
    uint32_t half_dim = pc->head_dim / 2u; /* rope.comp:22-51 */
    for (uint32_t head = 0; head < pc->q_heads + pc->kv_heads; ++head) {
        for (uint32_t pair = 0; pair < half_dim && pair < 64u; ++pair) {
            float ext = load_f32(blob, pc->factor_offset + pair * 4u);
            float exponent = (float)(pair * 2u) / (float)pc->head_dim;
            float inv_freq = 1.0f / powf(pc->rope_theta, exponent);
            float angle = (float)pc->position * inv_freq / ext;
            float c = cosf(angle) * pc->scaling_factor;
            float s = sinf(angle) * pc->scaling_factor;
            float *buf;
            uint32_t base;
            if (head < pc->q_heads) {
                buf = q; base = head * pc->head_dim;
            } else {
                buf = k; base = (head - pc->q_heads) * pc->head_dim;
            }
            float a = buf[base + pair];
            float b = buf[base + pair + half_dim];
            buf[base + pair] = a * c - b * s;
            buf[base + pair + half_dim] = b * c + a * s;
        }
    }
}

void vr_store_kv(const float *k, const float *v, uint32_t *k_cache, uint32_t *v_cache,
                 const vx_store_kv_push *pc) {
    uint32_t words_per_token = pc->kv_dim / 2u; /* store_kv.comp:16-24 */
    for (uint32_t w = 0; w < words_per_token && w < 128u; ++w) {
        uint32_t d = w * 2u;
        uint64_t dst = ((uint64_t)pc->layer * pc->context + pc->position) * words_per_token + w;
        k_cache[dst] = (uint32_t)vr_f32_to_f16(k[d]) | ((uint32_t)vr_f32_to_f16(k[d + 1u]) << 16);
        v_cache[dst] = (uint32_t)vr_f32_to_f16(v[d]) | ((uint32_t)vr_f32_to_f16(v[d + 1u]) << 16);
    }
}

static inline float cache_at(const uint32_t *cache, const vx_attention_push *pc, uint32_t pos,
                             uint32_t dim) {
    uint32_t kv_dim = pc->kv_heads * pc->head_dim; /* attn_scores.comp:19-25 */
    uint32_t words_per_token = kv_dim / 2u;
    uint64_t word_i = ((uint64_t)pc->layer * pc->context + pos) * words_per_token + dim / 2u;
    uint32_t word = cache[word_i];
    return h2f((dim & 1u) == 0u ? (word & 0xffffu) : (word >> 16));
}

void vr_attn_scores(const float *q, const uint32_t *k_cache, float *scores, uint32_t q_heads,
                    const vx_attention_push *pc) {
    ensure_lut(); /* attn_scores.comp:27-44, grid (position+1) x q_heads */
    float inv = 1.0f / sqrtf((float)pc->head_dim);
#pragma omp parallel for schedule(static)
    for (int64_t qh = 0; qh < (int64_t)q_heads; ++qh) {
        uint32_t kvh = (uint32_t)qh / pc->q_per_kv;
        for (uint32_t t = 0; t <= pc->position; ++t) {
            float partial[128];
            for (uint32_t lane = 0; lane < 128u; ++lane) {
                partial[lane] = lane < pc->head_dim
                    ? q[qh * pc->head_dim + lane] * cache_at(k_cache, pc, t, kvh * pc->head_dim + lane)
                    : 0.0f;
            }
            scores[qh * pc->context + t] = tree_sum(partial, 128u) * inv;
        }
    }
}

void vr_softmax(float *scores, uint32_t heads, const vx_softmax_push *pc) {
#pragma omp parallel for schedule(static) /* softmax.comp:15-47 */
    for (int64_t head = 0; head < (int64_t)heads; ++head) {
        float *s = scores + head * pc->context;
        float scratch[WG];
        for (uint32_t l = 0; l < WG; ++l) {
            float m = -3.402823466e+38f;
            for (uint32_t t = l; t <= pc->position; t += WG) m = m > s[t] ? m : s[t];
            scratch[l] = m;
        }
        float global_max = tree_max(scratch, WG);
        for (uint32_t l = 0; l < WG; ++l) {
            float sum = 0.0f;
            for (uint32_t t = l; t <= pc->position; t += WG) sum += expf(s[t] - global_max);
            scratch[l] = sum;
        }
        float inv_sum = 1.0f / tree_sum(scratch, WG);
        for (uint32_t t = 0; t <= pc->position; ++t) s[t] = expf(s[t] - global_max) * inv_sum;
    }
}

void vr_attn_values(const float *scores, const uint32_t *v_cache, float *out, uint32_t q_heads,
                    const vx_attention_push *pc) {
    ensure_lut(); /* attn_values.comp:25-37 */
#pragma omp parallel for schedule(static)
    for (int64_t qh = 0; qh < (int64_t)q_heads; ++qh) {
        uint32_t kvh = (uint32_t)qh / pc->q_per_kv;
        for (uint32_t d = 0; d < pc->head_dim && d < 128u; ++d) {
            float acc = 0.0f;
            for (uint32_t t = 0; t <= pc->position; ++t)
                acc += scores[qh * pc->context + t] * cache_at(v_cache, pc, t, kvh * pc->head_dim + d);
            out[qh * pc->head_dim + d] = acc;
        }
    }
}

static inline float load_scalar_lb(const uint8_t *blob, uint32_t o, uint32_t dtype) {
    if (dtype == 0u) return load_f32(blob, o); /* linear_bias.comp:38-42 */
    if (dtype == 1u) return load_f16(blob, o);
    return 0.0f;
}

void vr_linear_bias(const uint8_t *blob, const float *x, float *y, const vx_linear_bias_push *pc) {
    ensure_lut(); /* linear_bias.comp:63-82 */
#pragma omp parallel for schedule(static)
    for (int64_t r = pc->row_base; r < (int64_t)pc->rows; ++r) {
        float s = wg_row_dot(blob, pc->weight_offset, pc->weight_dtype, 1, pc->cols, (uint32_t)r, x);
        float bias = load_scalar_lb(blob, pc->bias_offset + (uint32_t)r * (pc->bias_dtype == 0u ? 4u : 2u),
                                    pc->bias_dtype);
        y[r] = (s + bias) * pc->alpha;
    }
}

void vr_fusion_linear(const uint8_t *blob, const float *left, const float *right, float *y,
                      float *snapshot, const vx_fusion_push *pc) {
    ensure_lut(); /* fusion_linear.comp:56-78 */
    uint32_t cols = pc->left_cols + pc->right_cols;
    float *x = (float *)malloc(sizeof(float) * (cols ? cols : 1u));
    for (uint32_t c = 0; c < pc->left_cols; ++c) x[c] = left[c];
    for (uint32_t c = 0; c < pc->right_cols; ++c) x[pc->left_cols + c] = right[c];
#pragma omp parallel for schedule(static)
    for (int64_t r = pc->row_base; r < (int64_t)pc->rows; ++r) {
        float s = wg_row_dot(blob, pc->weight_offset, pc->weight_dtype, 1, cols, (uint32_t)r, x);
        uint32_t bo = pc->bias_offset + (uint32_t)r * (pc->bias_dtype == 0u ? 4u : 2u);
        float bias = pc->bias_dtype == 0u ? load_f32(blob, bo) : load_f16(blob, bo);
        float value = s + bias;
        y[r] = value;
        snapshot[r] = value;
    }
    free(x);
}

/* ------------------------------------------------------- host sequencing */
float vr_effective_scale(float v) { return v == 0.0f ? 1.0f : v; }

float vr_rope_scaling_factor(const vx_baselm_config *c) {
    /* baselm.rs:194-205 */
    if (!c->rope_longrope || c->context_length <= c->rope_original_context_length ||
        c->rope_original_context_length <= 1u)
        return 1.0f;
    float max = (float)c->context_length;
    float original = (float)c->rope_original_context_length;
    return sqrtf(1.0f + logf(max / original) / logf(original));
}

/* record_transformer (baselm.rs:892-1052), or record_residual_lm
 * (acoustic.rs:968-1035) when rotate == 0: the same op order without RoPE. */
static void record_stack(const uint8_t *blob, const vr_baselm *m, vr_state *s, uint32_t position,
                         int compute_logits, int rotate) {
    const vx_baselm_config *c = &m->cfg;
    float residual_scale = vr_effective_scale(c->residual_scale);
    uint32_t q_per_kv = c->head_count / c->head_count_kv;
    vx_rms_push rp = {m->layers[0].attn_norm, c->embedding_length, c->rms_epsilon};
    vr_rmsnorm(blob, s->hidden, s->norm, &rp);
    for (uint32_t layer = 0; layer < c->block_count; ++layer) {
        const vr_layer *L = &m->layers[layer];
        vx_qkv_push qp = {L->q, L->k, L->v, c->embedding_length, c->kv_dim, c->embedding_length,
                          L->q_dtype, L->k_dtype, L->v_dtype, 0u};
        vr_qkv_matvec(blob, s->norm, s->q, s->k, s->v, &qp);
        if (rotate) {
            vx_rope_push ro = {m->rope_factors, position, c->head_count, c->head_count_kv, c->head_dim,
                               c->rope_theta, vr_rope_scaling_factor(c)};
            vr_rope(blob, s->q, s->k, &ro);
        }
        vx_store_kv_push sk = {layer, position, c->active_context_length, c->kv_dim};
        vr_store_kv(s->k, s->v, s->kv_k, s->kv_v, &sk);
        vx_attention_push ap = {layer, c->active_context_length, position, c->head_dim, q_per_kv,
                                c->head_count_kv};
        vr_attn_scores(s->q, s->kv_k, s->scores, c->head_count, &ap);
        vx_softmax_push sp = {c->active_context_length, position};
        vr_softmax(s->scores, c->head_count, &sp);
        vr_attn_values(s->scores, s->kv_v, s->attention, c->head_count, &ap);
        vx_matvec_push op = {L->o, c->embedding_length, c->embedding_length, L->o_dtype, 0u, 1.0f};
        vr_matvec(blob, s->attention, s->branch, &op);
        vx_residual_rms_push r1 = {L->ffn_norm, c->embedding_length, c->rms_epsilon, residual_scale};
        vr_residual_rmsnorm(blob, s->hidden, s->branch, s->norm, &r1);
        vx_swiglu_push gp = {L->gate, L->up, c->feed_forward_length, c->embedding_length, L->gate_dtype, 0u};
        vr_matvec_swiglu(blob, s->norm, s->gate, &gp);
        vx_matvec_push dp = {L->down, c->embedding_length, c->feed_forward_length, L->down_dtype, 0u, 1.0f};
        vr_matvec(blob, s->gate, s->branch, &dp);
        uint32_t next_norm = layer + 1u < c->block_count ? m->layers[layer + 1u].attn_norm : m->output_norm;
        vx_residual_rms_push r2 = {next_norm, c->embedding_length, c->rms_epsilon, residual_scale};
        vr_residual_rmsnorm(blob, s->hidden, s->branch, s->norm, &r2);
    }
    if (compute_logits) {
        vx_matvec_push lp = {m->output, c->vocab_size, c->embedding_length, m->output_dtype, 0u,
                             vr_effective_scale(c->logit_scale)};
        vr_matvec(blob, s->norm, s->logits, &lp);
    }
}

void vr_baselm_record(const uint8_t *blob, const vr_baselm *m, vr_state *s, uint32_t position,
                      int compute_logits) {
    record_stack(blob, m, s, position, compute_logits, 1);
}

void vr_residual_lm_record(const uint8_t *blob, const vr_baselm *m, vr_state *s, uint32_t position) {
    record_stack(blob, m, s, position, 0, 0);
}

/* fsq_quantize.comp; ties of v * scale round away from zero (f32::round, the
 * known answer of acoustic.rs:1266-1271). */
void vr_fsq_quantize(float *x, uint32_t n, float scale) {
    for (uint32_t i = 0; i < n; ++i) x[i] = roundf(tanhf(x[i]) * scale) / scale;
}

/* silu_inplace.comp. */
void vr_silu_inplace(float *x, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) x[i] = x[i] / (1.0f + expf(-x[i]));
}

void vr_baselm_decode_token(const uint8_t *blob, const vr_baselm *m, vr_state *s,
                            uint32_t token_id, uint32_t position, int compute_logits) {
    vx_embedding_push ep = {m->token_embd, m->cfg.embedding_length, token_id, m->token_embd_dtype,
                            vr_effective_scale(m->cfg.embedding_scale)};
    vr_embedding(blob, s->hidden, &ep); /* baselm.rs:634-647 */
    vr_baselm_record(blob, m, s, position, compute_logits);
}

/* --------------------------------------------------------------- AudioVAE */
/* The vae_*.comp shaders over channel-major [C][L] buffers. */
static inline float vae_scalar(const uint8_t *blob, uint32_t base, uint32_t i, uint32_t dtype) {
    return dtype == 1u ? load_f16(blob, base + i * 2u) : load_f32(blob, base + i * 4u);
}

void vr_vae_conv1d(const uint8_t *blob, const float *x, float *y, const vx_vae_conv_push *pc) {
    ensure_lut();
    const uint32_t out_pg = pc->out_channels / pc->groups, in_pg = pc->in_channels / pc->groups;
#pragma omp parallel for schedule(static)
    for (uint32_t oc = 0; oc < pc->out_channels; ++oc) { /* vae_conv1d.comp:33-57 */
        const uint32_t in_base = (oc / out_pg) * in_pg;
        for (uint32_t t = 0; t < pc->out_length; ++t) {
            float sum = pc->has_bias ? vae_scalar(blob, pc->bias_offset, oc, pc->bias_dtype) : 0.0f;
            for (uint32_t icg = 0; icg < in_pg; ++icg) {
                const uint32_t ic = in_base + icg;
                for (uint32_t k = 0; k < pc->kernel; ++k) {
                    const int64_t ti = (int64_t)t * pc->stride + (int64_t)k * pc->dilation - (int64_t)pc->left_pad;
                    if (ti < 0 || ti >= (int64_t)pc->in_length) continue;
                    const float w = vae_scalar(blob, pc->weight_offset, (oc * in_pg + icg) * pc->kernel + k,
                                               pc->weight_dtype);
                    sum += x[(size_t)ic * pc->in_length + (size_t)ti] * w;
                }
            }
            y[(size_t)oc * pc->out_length + t] = sum;
        }
    }
}

void vr_vae_convt1d(const uint8_t *blob, const float *x, float *y, const vx_vae_convt_push *pc) {
    ensure_lut();
    const uint32_t out_pg = pc->out_channels / pc->groups, in_pg = pc->in_channels / pc->groups;
#pragma omp parallel for schedule(static)
    for (uint32_t oc = 0; oc < pc->out_channels; ++oc) { /* vae_convtranspose1d.comp:23-48 */
        const uint32_t group = oc / out_pg, ocg = oc - group * out_pg, in_base = group * in_pg;
        for (uint32_t t = 0; t < pc->out_length; ++t) {
            float sum = pc->has_bias ? vae_scalar(blob, pc->bias_offset, oc, pc->bias_dtype) : 0.0f;
            for (uint32_t icg = 0; icg < in_pg; ++icg) {
                const uint32_t ic = in_base + icg;
                for (uint32_t k = t % pc->stride; k < pc->kernel; k += pc->stride) {
                    if (t < k) continue;
                    const uint32_t ti = (t - k) / pc->stride;
                    if (ti >= pc->in_length) continue;
                    sum += x[(size_t)ic * pc->in_length + ti] *
                           vae_scalar(blob, pc->weight_offset, (ic * out_pg + ocg) * pc->kernel + k, pc->weight_dtype);
                }
            }
            y[(size_t)oc * pc->out_length + t] = sum;
        }
    }
}

void vr_vae_snake(const uint8_t *blob, const float *x, float *y, const vx_vae_snake_push *pc) {
    ensure_lut();
    for (uint32_t c = 0; c < pc->channels; ++c) { /* vae_snake.comp:9-17 */
        const float a = vae_scalar(blob, pc->alpha_offset, c, pc->dtype);
        for (uint32_t t = 0; t < pc->length; ++t) {
            const size_t i = (size_t)c * pc->length + t;
            const float s = sinf(a * x[i]);
            y[i] = x[i] + (s * s) / (a + 1e-9f);
        }
    }
}

void vr_vae_scale_bias(const uint8_t *blob, float *x, const vx_vae_scale_push *pc) {
    ensure_lut();
    for (uint32_t c = 0; c < pc->channels; ++c) { /* vae_scale_bias.comp:9-17 */
        const uint32_t idx = pc->bucket * pc->channels + c;
        const float sc = vae_scalar(blob, pc->scale_offset, idx, pc->scale_dtype);
        const float bi = vae_scalar(blob, pc->bias_offset, idx, pc->bias_dtype);
        for (uint32_t t = 0; t < pc->length; ++t) {
            const size_t i = (size_t)c * pc->length + t;
            x[i] = x[i] * sc + bi;
        }
    }
}

void vr_vae_add(float *a, const float *b, const vx_vae_grid_push *pc) {
    const size_t n = (size_t)pc->channels * pc->length;
    for (size_t i = 0; i < n; ++i) a[i] += b[i];
}

void vr_vae_tanh(float *x, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) x[i] = tanhf(x[i]);
}

/* ------------------------------------------------------------- CFM pieces */
/* cfm_noise.comp:11-18: integer finaliser. */
uint32_t vr_mix32(uint32_t v) {
    v ^= v >> 16;
    v *= 0x7feb352du;
    v ^= v >> 15;
    v *= 0x846ca68bu;
    v ^= v >> 16;
    return v;
}

/* cfm_noise.comp:25-37, one invocation per element i < n. */
void vr_cfm_noise(float *x, const vx_cfm_noise_push *pc) {
    for (uint32_t i = 0; i < pc->n; ++i) {
        uint32_t pair = i >> 1;
        uint32_t a = vr_mix32(pair ^ pc->seed_lo ^ 0x9e3779b9u);
        uint32_t b = vr_mix32(pair ^ pc->seed_hi ^ 0x85ebca6bu);
        float u1 = ((float)a + 0.5f) * (1.0f / 4294967296.0f);
        if (u1 < 1.0e-7f) u1 = 1.0e-7f;
        float u2 = ((float)b + 0.5f) * (1.0f / 4294967296.0f);
        float r = sqrtf(-2.0f * logf(u1));
        float theta = 6.28318530717958647692f * u2;
        float z = (i & 1u) == 0u ? r * cosf(theta) : r * sinf(theta);
        x[i] = z * pc->temperature;
    }
}

/* cfm_cfg_euler.comp:15-36: 256-lane tree reduction of <p,n> and |n|^2, then
 * x -= dt * (n*s + cfg*(p - n*s)) with s the CFG-Zero* scale (or 1).
 * For n <= 256 this is the shader exactly (one element per lane). The strided
 * loop for n > 256 is NOT the reference's behaviour (its single workgroup only
 * covers x[0..256)): it restates the engine solve's generalisation for latent
 * sizes above 256, which only non-reference geometries have; the per-op entry
 * point refuses n > 256. */
void vr_cfm_cfg_euler(float *x, const float *pos, const float *neg, const vx_cfm_euler_push *pc) {
    float dot[256], nrm[256];
    for (uint32_t i = 0; i < 256u; ++i) {
        float p = 0.0f, n = 0.0f;
        for (uint32_t j = i; j < pc->n; j += 256u) { /* the shader's one element per lane, strided for n > 256 */
            p += pos[j] * neg[j];
            n += neg[j] * neg[j];
        }
        dot[i] = p;
        nrm[i] = n;
    }
    for (uint32_t stride = 128u; stride > 0u; stride >>= 1u)
        for (uint32_t i = 0; i < stride; ++i) {
            dot[i] += dot[i + stride];
            nrm[i] += nrm[i + stride];
        }
    float scale = pc->use_zero_star ? dot[0] / (nrm[0] + 1.0e-8f) : 1.0f;
    for (uint32_t i = 0; i < pc->n; ++i) {
        float g = neg[i] * scale + pc->cfg * (pos[i] - neg[i] * scale);
        x[i] -= pc->dt * g;
    }
}

/* time_sinusoidal.comp:5. */
void vr_time_sinusoidal(float *out, const vx_time_push *pc) {
    uint32_t half = pc->dim / 2u;
    float denom = (float)(half > 1u ? half - 1u : 1u);
    for (uint32_t i = 0; i < pc->dim; ++i) {
        uint32_t j = i % half;
        float freq = expf((float)j * (-logf(10000.0f) / denom));
        float a = 1000.0f * pc->t * freq;
        out[i] = i < half ? sinf(a) : cosf(a);
    }
}

/* pack_locdit.comp:10: rows [mu1, mu2, time, cond x P, x x P]. */
void vr_pack_locdit(const float *mu1, const float *mu2, const float *time, const float *cond, const float *x,
                    float *hidden, const vx_pack_locdit_push *pc) {
    uint32_t H = pc->hidden, P = pc->patch_tokens;
    for (uint32_t i = 0; i < (3u + 2u * P) * H; ++i) {
        uint32_t tok = i / H, d = i % H;
        float v;
        if (tok == 0u) v = pc->zero_mu ? 0.0f : mu1[d];
        else if (tok == 1u) v = pc->zero_mu ? 0.0f : mu2[d];
        else if (tok == 2u) v = time[d];
        else if (tok < 3u + P) v = cond[(tok - 3u) * H + d];
        else v = x[(tok - 3u - P) * H + d];
        hidden[i] = v;
    }
}

/* cfm_time_span (local.rs:531-537); returns 0 or -1 when the schedule is not
 * descending (the reference's bail). out holds n + 1 values. */
int vr_cfm_time_span(uint32_t n, float sway, float *out) {
    if (n == 0u) return -1;
    for (uint32_t i = 0; i <= n; ++i) {
        float t = 1.0f - (float)i / (float)n;
        out[i] = t + sway * (cosf(1.57079632679489661923f * t) - 1.0f + t);
    }
    for (uint32_t i = 1; i <= n; ++i)
        if (out[i] > out[i - 1] + 1.0e-6f) return -1;
    return 0;
}

void vr_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
int vr_get_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
