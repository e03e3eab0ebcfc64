/*
 * voxref.h — CPU oracle for the VoxCPM2 BaseLM compute path.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of VoxGen's Normal-mode
 * GLSL shaders and of the host op order in src/baselm.rs. Only tests/, the smoke
 * check and bench.py's cpu_baseline leg may load it, and only as the checker or
 * the timed CPU baseline — never as a product path.
 *
 * Each function follows one reference shader, including its per-workgroup
 * reduction order (256 lanes striding the columns, then a shared-memory tree),
 * so that the f32 results differ from the reference only by transcendental
 * rounding (exp/sin/cos/pow/inversesqrt) and FMA contraction, which the
 * reference leaves to the Vulkan driver. The library is built with
 * -ffp-contract=off.
 *
 * Pinning status of every function is listed in the header of voxref.c.
 */
#ifndef VOXREF_H
#define VOXREF_H
#include <stdint.h>
#include "../include/voxhip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* IEEE half <-> float (unpackHalf2x16 exact widening / packHalf2x16 RNE). */
float vr_f16_to_f32(uint16_t h);
uint16_t vr_f32_to_f16(float f);
void vr_f16_to_f32_n(const uint16_t *src, float *dst, uint64_t n);
void vr_f32_to_f16_n(const float *src, uint16_t *dst, uint64_t n);

/* matvec.comp:32-44 load_weight for one (row, col) of a dtype 0/1/8 matrix. */
float vr_load_weight(const uint8_t *blob, uint32_t weight_offset, uint32_t dtype, uint32_t cols,
                     uint32_t row, uint32_t col);
/* Dequantize rows x cols (row-major f32 out). */
void vr_dequant(const uint8_t *blob, uint32_t weight_offset, uint32_t dtype, uint32_t rows,
                uint32_t cols, float *out);

void vr_embedding(const uint8_t *blob, float *hidden, const vx_embedding_push *pc);
void vr_rmsnorm(const uint8_t *blob, const float *x, float *y, const vx_rms_push *pc);
void vr_residual_rmsnorm(const uint8_t *blob, float *hidden, const float *branch, float *y,
                         const vx_residual_rms_push *pc);
void vr_matvec(const uint8_t *blob, const float *x, float *y, const vx_matvec_push *pc);
void vr_qkv_matvec(const uint8_t *blob, const float *x, float *q, float *k, float *v,
                   const vx_qkv_push *pc);
void vr_matvec_swiglu(const uint8_t *blob, const float *x, float *y, const vx_swiglu_push *pc);
void vr_rope(const uint8_t *blob, float *q, float *k, const vx_rope_push *pc);
void vr_store_kv(const float *k, const float *v, uint32_t *k_cache, uint32_t *v_cache,
                 const vx_store_kv_push *pc);
void vr_attn_scores(const float *q, const uint32_t *k_cache, float *scores, uint32_t q_heads,
                    const vx_attention_push *pc);
void vr_softmax(float *scores, uint32_t heads, const vx_softmax_push *pc);
void vr_attn_values(const float *scores, const uint32_t *v_cache, float *out, uint32_t q_heads,
                    const vx_attention_push *pc);
void vr_linear_bias(const uint8_t *blob, const float *x, float *y, const vx_linear_bias_push *pc);
void vr_fusion_linear(const uint8_t *blob, const float *left, const float *right, float *y,
                      float *snapshot, const vx_fusion_push *pc);

/* BaseLM model description: tensor byte offsets into the data region. */
typedef struct vr_layer {
    uint32_t attn_norm, ffn_norm;
    uint32_t q, k, v, o, gate, up, down;
    uint32_t q_dtype, k_dtype, v_dtype, o_dtype, gate_dtype, up_dtype, down_dtype;
} vr_layer;
typedef struct vr_baselm {
    vx_baselm_config cfg;
    uint32_t token_embd, token_embd_dtype;
    uint32_t output, output_dtype;          /* tied: token_embd */
    uint32_t output_norm;
    uint32_t rope_factors;                  /* the factor set record_transformer picks */
    const vr_layer *layers;                 /* cfg.block_count entries */
} vr_baselm;
/* Activation and cache buffers of one engine (BaseLmEngine fields, baselm.rs:423-440). */
typedef struct vr_state {
    float *hidden, *norm, *q, *k, *v, *attention, *gate, *branch, *logits, *scores;
    uint32_t *kv_k, *kv_v;                  /* packed f16 pairs, [layer][ctx][kv_dim/2] words */
} vr_state;

/* record_transformer (baselm.rs:892-1052) at `position`. */
void vr_baselm_record(const uint8_t *blob, const vr_baselm *m, vr_state *s, uint32_t position,
                      int compute_logits);
/* record_residual_lm (acoustic.rs:968-1035): record_transformer's order without
 * RoPE and without logits; m->cfg carries the ResidualLM geometry. */
void vr_residual_lm_record(const uint8_t *blob, const vr_baselm *m, vr_state *s, uint32_t position);
/* fsq_quantize.comp (in place). */
void vr_fsq_quantize(float *x, uint32_t n, float scale);
/* silu_inplace.comp (in place). */
void vr_silu_inplace(float *x, uint32_t n);
/* vae_*.comp over channel-major [C][L] f32 buffers. */
void vr_vae_conv1d(const uint8_t *blob, const float *x, float *y, const vx_vae_conv_push *pc);
void vr_vae_convt1d(const uint8_t *blob, const float *x, float *y, const vx_vae_convt_push *pc);
void vr_vae_snake(const uint8_t *blob, const float *x, float *y, const vx_vae_snake_push *pc);
void vr_vae_scale_bias(const uint8_t *blob, float *x, const vx_vae_scale_push *pc);
void vr_vae_add(float *a, const float *b, const vx_vae_grid_push *pc);
void vr_vae_tanh(float *x, uint32_t n);
/* Embedding dispatch (baselm.rs:634-647) then record_transformer. */
void vr_baselm_decode_token(const uint8_t *blob, const vr_baselm *m, vr_state *s,
                            uint32_t token_id, uint32_t position, int compute_logits);
/* BaseLmConfig::rope_scaling_factor (baselm.rs:194-205). */
float vr_rope_scaling_factor(const vx_baselm_config *cfg);
/* effective_scale (baselm.rs:1262-1264). */
float vr_effective_scale(float v);

/* CFM pieces of the LocDiT solve (local.rs:383-430). */
uint32_t vr_mix32(uint32_t v);
void vr_cfm_noise(float *x, const vx_cfm_noise_push *pc);
void vr_cfm_cfg_euler(float *x, const float *pos, const float *neg, const vx_cfm_euler_push *pc);
void vr_time_sinusoidal(float *out, const vx_time_push *pc);
void vr_pack_locdit(const float *mu1, const float *mu2, const float *time, const float *cond, const float *x,
                    float *hidden, const vx_pack_locdit_push *pc);
int vr_cfm_time_span(uint32_t n, float sway, float *out);

/* Threads used by the OpenMP loops (0 = runtime default). */
void vr_set_threads(int n);
int vr_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
