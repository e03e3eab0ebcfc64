/*
 * voxhip.h — C ABI of the MI355X (gfx950) BaseLM compute library.
 *
 * This is the drop-in boundary that replaces VoxGen's Vulkan dispatch layer
 * (src/vulkan.rs) for the VoxCPM2 BaseLM path. Every per-op entry point takes
 * the same #[repr(C)] push struct the reference shaders consume (field order and
 * types identical), plus the buffers the reference binds to that pipeline.
 * Plain C types only: pointers, sizes, u32/f32 push structs. No torch types.
 *
 * Conventions
 *   - Every function returns vx_status (0 = OK, negative = error) unless noted.
 *     The message of the last failure on the calling thread is vx_last_error().
 *     The library never aborts the process.
 *   - One vx_ctx = one device + one in-order HIP stream. Calls on one context are
 *     serialised by the caller (the reference holds a per-engine Mutex,
 *     runtime.rs:168-188). Work is enqueued asynchronously; vx_sync() waits.
 *     Stream order replaces the reference's buffer barriers (vulkan.rs:691-802),
 *     which therefore have no counterpart here.
 *   - Weights live in a vx_model (the uploaded GGUF data region). Ops address a
 *     weight by its u32 byte offset into that region, exactly as the reference
 *     push structs do (baselm.rs:1257-1260). The offset must start a tensor of the
 *     model's table; Q8_0 matrices are repacked on upload for coalesced loads and
 *     resolved through that table.
 *   - Ownership: the caller owns every vx_buf / vx_model / vx_baselm it creates and
 *     frees it with the matching *_free / *_destroy call.
 */
#ifndef VOXHIP_H
#define VOXHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VX_ABI_VERSION 2   /* 2: vx_baselm_options.prefill_schedule */

/* ------------------------------------------------------------------------- */
/* Status codes. The conditions mirror the reference's anyhow bails.          */
/* ------------------------------------------------------------------------- */
typedef enum vx_status {
    VX_OK = 0,
    VX_ERR_INVALID_ARG = -1,   /* null handle, zero size, bad enum            */
    VX_ERR_HIP = -2,           /* HIP runtime error (message has the hipError) */
    VX_ERR_OOM = -3,           /* device allocation failed (runtime.rs:265-272) */
    VX_ERR_SHAPE = -4,         /* shape / dtype mismatch (baselm.rs:1083-1088,1124-1130,1163-1168) */
    VX_ERR_BOUNDS = -5,        /* a bound buffer is too small for the push extents */
    VX_ERR_UNSUPPORTED = -6,   /* dtype or geometry this build does not run     */
    VX_ERR_CONTEXT_FULL = -7,  /* KV cache full (baselm.rs:882-890)             */
    VX_ERR_TOKEN_RANGE = -8,   /* token id >= vocab (baselm.rs:629-631)         */
    VX_ERR_GGUF = -9,          /* GGUF magic/version/truncation (gguf.rs:226-228,281-284) */
    VX_ERR_NOT_FOUND = -10,    /* missing tensor or metadata key                */
    VX_ERR_OFFSET = -11,       /* data region >= 4 GiB (baselm.rs:468-470)      */
    VX_ERR_CANCELLED = -12,    /* cancel flag set before a step (runtime.rs:745-808) */
    VX_ERR_NO_DEVICE = -13,    /* no HIP device / index out of range            */
    VX_ERR_STATE = -14         /* call not valid in the current state           */
} vx_status;

/* GGML dtype codes carried in push structs: dtype_code (baselm.rs:1239-1245),
 * GgmlType::from_raw (gguf.rs:31-33). */
#define VX_DTYPE_F32 0u
#define VX_DTYPE_F16 1u
#define VX_DTYPE_Q8_0 8u

typedef struct vx_ctx vx_ctx;
typedef struct vx_buf vx_buf;
typedef struct vx_model vx_model;
typedef struct vx_graph vx_graph;
typedef struct vx_baselm vx_baselm;
typedef struct vx_gguf vx_gguf;
typedef struct vx_locdit vx_locdit;
typedef struct vx_residual vx_residual;
typedef struct vx_audiovae vx_audiovae;

/* ------------------------------------------------------------------------- */
/* Push structs: identical layout to the reference's #[repr(C)] structs.      */
/* ------------------------------------------------------------------------- */
typedef struct vx_embedding_push {  /* EmbeddingPush baselm.rs:287-295 */
    uint32_t weight_offset, cols, token_id, dtype;
    float alpha;
} vx_embedding_push;

typedef struct vx_rms_push {        /* RmsPush baselm.rs:296-302 */
    uint32_t weight_offset, n;
    float eps;
} vx_rms_push;

typedef struct vx_matvec_push {     /* MatvecPush baselm.rs:303-312 */
    uint32_t weight_offset, rows, cols, dtype, row_base;
    float alpha;
} vx_matvec_push;

typedef struct vx_rope_push {       /* RopePush baselm.rs:313-323 */
    uint32_t factor_offset, position, q_heads, kv_heads, head_dim;
    float rope_theta, scaling_factor;
} vx_rope_push;

typedef struct vx_store_kv_push {   /* StoreKvPush baselm.rs:324-331 */
    uint32_t layer, position, context, kv_dim;
} vx_store_kv_push;

typedef struct vx_attention_push {  /* AttentionPush baselm.rs:332-341 */
    uint32_t layer, context, position, head_dim, q_per_kv, kv_heads;
} vx_attention_push;

typedef struct vx_softmax_push {    /* SoftmaxPush baselm.rs:342-347 */
    uint32_t context, position;
} vx_softmax_push;

typedef struct vx_qkv_push {        /* QkvPush baselm.rs:348-361 */
    uint32_t q_weight_offset, k_weight_offset, v_weight_offset;
    uint32_t q_rows, kv_rows, cols;
    uint32_t q_dtype, k_dtype, v_dtype;
    uint32_t row_base;
} vx_qkv_push;

typedef struct vx_swiglu_push {     /* SwigluPush baselm.rs:363-372 */
    uint32_t gate_weight_offset, up_weight_offset, rows, cols, dtype, row_base;
} vx_swiglu_push;

typedef struct vx_residual_rms_push { /* ResidualRmsPush baselm.rs:373-380 */
    uint32_t weight_offset, n;
    float eps, scale;
} vx_residual_rms_push;

typedef struct vx_linear_bias_push {  /* LinearBiasPush acoustic.rs:237-247 */
    uint32_t weight_offset, bias_offset, rows, cols, weight_dtype, bias_dtype, row_base;
    float alpha;
} vx_linear_bias_push;

typedef struct vx_fusion_push {     /* FusionPush acoustic.rs:257-268 */
    uint32_t weight_offset, bias_offset, rows, left_cols, right_cols;
    uint32_t weight_dtype, bias_dtype, row_base;
} vx_fusion_push;

/* Token-batched ("seq") push structs of the LocEnc/LocDiT pipelines,
 * identical to local.rs:183-212. */
typedef struct vx_seq_linear_push {   /* SeqLinearPush local.rs:183-184 */
    uint32_t weight_offset, bias_offset, rows, cols, weight_dtype, bias_dtype, tokens;
    uint32_t input_stride, output_stride, input_base, output_base, has_bias;
    float alpha;
} vx_seq_linear_push;

typedef struct vx_seq_rms_push {      /* SeqRmsPush local.rs:185-186 */
    uint32_t weight_offset, n, tokens, input_stride, output_stride, input_base, output_base;
    float eps;
} vx_seq_rms_push;

typedef struct vx_seq_residual_rms_push { /* SeqResidualRmsPush local.rs:187-188 */
    uint32_t weight_offset, n, tokens, hidden_stride, branch_stride, output_stride;
    uint32_t hidden_base, branch_base, output_base;
    float eps, scale;
} vx_seq_residual_rms_push;

typedef struct vx_seq_qkv_push {      /* SeqQkvPush local.rs:189-190 */
    uint32_t q_weight_offset, k_weight_offset, v_weight_offset, q_rows, kv_rows, cols, tokens;
    uint32_t input_stride, q_stride, kv_stride, input_base;
} vx_seq_qkv_push;

typedef struct vx_seq_swiglu_push {   /* SeqSwigluPush local.rs:191-192 */
    uint32_t gate_weight_offset, up_weight_offset, rows, cols, tokens;
    uint32_t input_stride, output_stride, input_base, output_base;
} vx_seq_swiglu_push;

typedef struct vx_seq_rope_push {     /* SeqRopePush local.rs:193-194 */
    uint32_t factor_offset, tokens, q_heads, kv_heads, head_dim, q_stride, k_stride;
    float rope_theta, scaling_factor;
} vx_seq_rope_push;

typedef struct vx_dense_scores_push { /* DenseScoresPush local.rs:195-196 */
    uint32_t tokens, q_heads, kv_heads, head_dim, q_stride, k_stride, score_stride;
} vx_dense_scores_push;

typedef struct vx_dense_softmax_push { /* DenseSoftmaxPush local.rs:197-198 */
    uint32_t tokens, q_heads, score_stride;
} vx_dense_softmax_push;

typedef struct vx_dense_values_push { /* DenseValuesPush local.rs:199-200 */
    uint32_t tokens, q_heads, kv_heads, head_dim, out_stride, v_stride, score_stride;
} vx_dense_values_push;

/* CFM / LocDiT push structs, identical to local.rs:201-212. */
typedef struct vx_cfm_noise_push {     /* CfmNoisePush local.rs:209-210 */
    uint32_t n, seed_lo, seed_hi;
    float temperature;
} vx_cfm_noise_push;

typedef struct vx_cfm_euler_push {     /* CfmEulerPush local.rs:211-212 */
    uint32_t n;
    float dt, cfg;
    uint32_t use_zero_star;
} vx_cfm_euler_push;

typedef struct vx_time_push {          /* TimePush local.rs:207-208 */
    uint32_t dim;
    float t;
} vx_time_push;

typedef struct vx_pack_locdit_push {   /* PackLocDitPush local.rs:205-206 */
    uint32_t hidden, patch_tokens, zero_mu;
} vx_pack_locdit_push;

/* ------------------------------------------------------------------------- */
/* Context, buffers, streams (replaces VulkanContext, vulkan.rs:96-113).      */
/* ------------------------------------------------------------------------- */
int vx_abi_version(void);
/* Message of the last failed call on this thread ("" if none). */
const char *vx_last_error(void);

/* VulkanContext::new (vulkan.rs:284-466): select one device, one queue. */
int vx_init(int device_index, vx_ctx **out);
int vx_destroy(vx_ctx *ctx);
typedef struct vx_device_info {
    char name[256];
    char arch[64];            /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
    uint64_t total_global_mem;
    uint32_t compute_units;
    uint32_t wavefront_size;
    uint32_t l2_cache_bytes;
    uint32_t lds_bytes_per_block;
    uint32_t clock_khz;
    uint32_t memory_clock_khz;
    uint32_t memory_bus_width;
} vx_device_info;
int vx_device_info_get(vx_ctx *ctx, vx_device_info *out);

/* create_buffer (vulkan.rs:488-535) + GpuBuffer Drop (vulkan.rs:87-94). */
int vx_alloc(vx_ctx *ctx, uint64_t bytes, vx_buf **out);
int vx_free(vx_ctx *ctx, vx_buf *buf);
uint64_t vx_buf_size(const vx_buf *buf);
/* Raw device address, for interop (e.g. wrapping in a framework tensor). */
void *vx_buf_device_ptr(const vx_buf *buf);
/* upload_f32 / upload_device_local (vulkan.rs:804-866); synchronous w.r.t. src. */
int vx_upload(vx_ctx *ctx, vx_buf *dst, uint64_t dst_offset, const void *src, uint64_t bytes);
/* read_f32 (vulkan.rs:905-955); waits for queued work first. */
int vx_download(vx_ctx *ctx, const vx_buf *src, uint64_t src_offset, void *dst, uint64_t bytes);
/* cmd_copy_buffer (baselm.rs:804-813); enqueued on the context stream. */
int vx_copy(vx_ctx *ctx, vx_buf *dst, uint64_t dst_offset, const vx_buf *src,
            uint64_t src_offset, uint64_t bytes);
/* Fill `count` u32 words with `value` using a kernel (safe inside graph capture). */
int vx_fill_u32(vx_ctx *ctx, vx_buf *dst, uint64_t dst_offset, uint32_t value, uint64_t count);
/* submit_and_wait (vulkan.rs:637-657): block until the stream drains. */
int vx_sync(vx_ctx *ctx);
/* Cancellation (the AtomicBool of Runtime::synthesize_cancelable,
 * runtime.rs:745-808). The caller registers a word it may set from any thread
 * (null unregisters it). Every step-level entry point of the engines on this
 * context reads it before enqueuing a step (BaseLM decode, each token of a
 * multi-token call, each chunk of a batched prefill, a ResidualLM step or
 * prefix, a LocDiT estimate or CFM solve, an AudioVAE decode) and, while it is
 * nonzero, returns VX_ERR_CANCELLED ("speech synthesis cancelled") with that
 * step not enqueued. Work already enqueued runs to completion. */
int vx_set_cancel_flag(vx_ctx *ctx, const uint32_t *flag);

/* Graph capture of enqueued work (replaces recording one command buffer). */
int vx_graph_begin(vx_ctx *ctx);
int vx_graph_end(vx_ctx *ctx, vx_graph **out);
int vx_graph_launch(vx_ctx *ctx, vx_graph *graph);
int vx_graph_free(vx_ctx *ctx, vx_graph *graph);

/* GPU profiling: gpu_profile_begin/end/snapshot/reset (vulkan.rs:587-635).
 * When enabled, every op and engine kernel is bracketed by HIP events on the
 * context stream; totals are collected at vx_sync() and aggregated by name. */
typedef struct vx_prof_entry {
    char name[64];
    double total_ms;
    uint64_t calls;
    double avg_ms;
} vx_prof_entry;
int vx_prof_enable(vx_ctx *ctx, int enabled);
int vx_prof_reset(vx_ctx *ctx);
/* Copies up to `cap` entries; *count receives the number of distinct names. */
int vx_prof_snapshot(vx_ctx *ctx, vx_prof_entry *out, uint32_t cap, uint32_t *count);

/* ------------------------------------------------------------------------- */
/* Model data (upload_device_local of the GGUF data region, baselm.rs:472-477)*/
/* ------------------------------------------------------------------------- */
typedef struct vx_tensor_info {     /* TensorInfo gguf.rs:51-59 */
    char name[96];
    uint32_t ggml_type;             /* VX_DTYPE_* */
    uint32_t n_dims;
    uint64_t dims[4];               /* GGUF order: dims[0] is the contiguous axis; a GGUF
                                       tensor of rank 5..8 is listed with n_dims 4 and its
                                       dims 3.. folded into dims[3] */
    uint64_t offset;                /* byte offset into the data region */
    uint64_t bytes;
} vx_tensor_info;

/* Upload `bytes` of GGUF data region plus its tensor table. Rank-2 Q8_0 tensors
 * are additionally repacked on the device into the coalesced layout the matvec
 * and GEMM kernels read; the original bytes stay resident for bit-exact gathers.
 * Fails with VX_ERR_OFFSET if the region is >= 4 GiB (u32 push offsets). The
 * tensor table is validated first, with checked size arithmetic (element counts,
 * byte sizes and extents that overflow are VX_ERR_GGUF or VX_ERR_SHAPE), before
 * the context is used or any device memory is touched. */
int vx_model_upload(vx_ctx *ctx, const void *data, uint64_t bytes,
                    const vx_tensor_info *tensors, uint32_t n_tensors, vx_model **out);
int vx_model_free(vx_ctx *ctx, vx_model *model);
uint32_t vx_model_tensor_count(const vx_model *model);
int vx_model_tensor_at(const vx_model *model, uint32_t index, vx_tensor_info *out);
/* GgufSummary::tensor (gguf.rs:84-87). */
int vx_model_find(const vx_model *model, const char *name, vx_tensor_info *out);
/* Device bytes held by the model (raw region + repacked copies). */
uint64_t vx_model_device_bytes(const vx_model *model);
/* Dequantize rows [0,rows) of the weight at `weight_offset` into f32 `out`
 * (row-major rows x cols) from the same device layout the matvecs read. Pins the
 * Q8_0 repack: the result must equal d*float(q) (matvec.comp:32-44) bit for bit. */
int vx_dequant(vx_ctx *ctx, const vx_model *model, uint32_t weight_offset, uint32_t rows,
               uint32_t cols, uint32_t dtype, vx_buf *out);

/* ------------------------------------------------------------------------- */
/* Per-op entry points: one per reference pipeline. Each runs the whole       */
/* dispatch loop of the corresponding host helper (rows row_base..rows), and  */
/* checks bound buffer sizes against the push extents before launching.       */
/* ------------------------------------------------------------------------- */
/* embedding.comp:43-48, dispatch baselm.rs:634-647 */
int vx_embedding(vx_ctx *ctx, const vx_model *model, vx_buf *hidden, const vx_embedding_push *pc);
/* Same, token id read from device u32 tokens[position[0]] (graph replay). */
int vx_embedding_devtok(vx_ctx *ctx, const vx_model *model, vx_buf *hidden, const vx_buf *tokens,
                        const vx_buf *position, const vx_embedding_push *pc);
/* rmsnorm.comp:21-42, dispatch_rms baselm.rs:1054-1073 */
int vx_rmsnorm(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y, const vx_rms_push *pc);
/* residual_rmsnorm.comp:23-42, dispatch_residual_rms baselm.rs:1190-1202 */
int vx_residual_rmsnorm(vx_ctx *ctx, const vx_model *model, vx_buf *hidden, const vx_buf *branch,
                        vx_buf *y, const vx_residual_rms_push *pc);
/* matvec.comp:46-62, dispatch_matvec baselm.rs:1115-1153 */
int vx_matvec(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y, const vx_matvec_push *pc);
/* qkv_matvec.comp:53-95, dispatch_qkv baselm.rs:1075-1113 */
int vx_qkv_matvec(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *q, vx_buf *k,
                  vx_buf *v, const vx_qkv_push *pc);
/* matvec_swiglu.comp:44-69, dispatch_swiglu baselm.rs:1155-1188 */
int vx_matvec_swiglu(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y,
                     const vx_swiglu_push *pc);
/* rope.comp:22-51, dispatch baselm.rs:933-953 */
int vx_rope(vx_ctx *ctx, const vx_model *model, vx_buf *q, vx_buf *k, const vx_rope_push *pc);
/* Same, position read from device u32 position[0]; pc->position is ignored. */
int vx_rope_devpos(vx_ctx *ctx, const vx_model *model, vx_buf *q, vx_buf *k, const vx_buf *position,
                   const vx_rope_push *pc);
/* store_kv.comp:16-24, dispatch baselm.rs:956-967. k_cache/v_cache are the
 * packed f16 caches [layer][context][kv_dim]. */
int vx_store_kv(vx_ctx *ctx, const vx_buf *k, const vx_buf *v, vx_buf *k_cache, vx_buf *v_cache,
                const vx_store_kv_push *pc);
int vx_store_kv_devpos(vx_ctx *ctx, const vx_buf *k, const vx_buf *v, vx_buf *k_cache,
                       vx_buf *v_cache, const vx_buf *position, const vx_store_kv_push *pc);
/* attn_scores.comp:27-44, dispatch baselm.rs:969-980 (grid (position+1) x q_heads);
 * q_heads = q_per_kv * kv_heads. scores is f32 [q_heads][context]. */
int vx_attn_scores(vx_ctx *ctx, const vx_buf *q, const vx_buf *k_cache, vx_buf *scores,
                   const vx_attention_push *pc);
int vx_attn_scores_devpos(vx_ctx *ctx, const vx_buf *q, const vx_buf *k_cache, vx_buf *scores,
                          const vx_buf *position, const vx_attention_push *pc);
/* softmax.comp:15-47, dispatch baselm.rs:982-991 (grid = heads). */
int vx_softmax(vx_ctx *ctx, vx_buf *scores, uint32_t heads, const vx_softmax_push *pc);
int vx_softmax_devpos(vx_ctx *ctx, vx_buf *scores, uint32_t heads, const vx_buf *position,
                      const vx_softmax_push *pc);
/* attn_values.comp:25-37, dispatch baselm.rs:993-996 (grid = q heads). */
int vx_attn_values(vx_ctx *ctx, const vx_buf *scores, const vx_buf *v_cache, vx_buf *out,
                   const vx_attention_push *pc);
int vx_attn_values_devpos(vx_ctx *ctx, const vx_buf *scores, const vx_buf *v_cache, vx_buf *out,
                          const vx_buf *position, const vx_attention_push *pc);
/* linear_bias.comp:63-82, dispatch acoustic.rs:1130-1161 */
int vx_linear_bias(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y,
                   const vx_linear_bias_push *pc);
/* fusion_linear.comp:56-78, dispatch acoustic.rs:941-966 (two identical outputs). */
int vx_fusion_linear(vx_ctx *ctx, const vx_model *model, const vx_buf *left, const vx_buf *right,
                     vx_buf *y, vx_buf *snapshot, const vx_fusion_push *pc);

/* ------------------------------------------------------------------------- */
/* Token-batched per-op entry points (the seq_* / dense_* pipelines, dispatched */
/* by local.rs:482-560). Buffers are f32 [tokens][stride] with the push's base */
/* offsets (in floats). Projections run on MFMA (f16 hi/lo activations, exact  */
/* weights, fp32 accumulation) when the weights are Q8_0 rows a multiple of    */
/* 1024 wide or F16 rows a multiple of 128 and input rows are 16-byte aligned; */
/* other shapes and F32 weights take a one-wave-per-output kernel.             */
/* ------------------------------------------------------------------------- */
/* seq_linear_bias.comp:22-30, record_linear local.rs:549-556:
 * y[t][r] = alpha * (W[r] . x[t] + b[r]); weight dtype 0/1/8, bias 0/1. */
int vx_seq_linear_bias(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y,
                       const vx_seq_linear_push *pc);
/* seq_qkv.comp:17-28, record_qkv local.rs:539-546. The reference shader reads
 * F16 weights only; here each of q/k/v may be F16 or Q8_0 (from the tensor table). */
int vx_seq_qkv(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *q, vx_buf *k, vx_buf *v,
               const vx_seq_qkv_push *pc);
/* seq_swiglu.comp:9, record_swiglu local.rs:560: y = silu(Wg.x) * (Wu.x); F16 or Q8_0. */
int vx_seq_swiglu(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y, const vx_seq_swiglu_push *pc);
/* seq_silu_mul.comp:6: gate[i] = silu(gate[i]) * up[i], i < n. */
int vx_seq_silu_mul(vx_ctx *ctx, vx_buf *gate, const vx_buf *up, uint32_t n);
/* seq_rmsnorm.comp:9, record_rms local.rs:558. */
int vx_seq_rmsnorm(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y, const vx_seq_rms_push *pc);
/* seq_residual_rmsnorm.comp:10, record_residual_rms local.rs:559. */
int vx_seq_residual_rmsnorm(vx_ctx *ctx, const vx_model *model, vx_buf *hidden, const vx_buf *branch, vx_buf *y,
                            const vx_seq_residual_rms_push *pc);
/* seq_rope.comp:8 (position = token index, local.rs:498). */
int vx_seq_rope(vx_ctx *ctx, const vx_model *model, vx_buf *q, vx_buf *k, const vx_seq_rope_push *pc);
/* Same with token t at position position_base + t (the BaseLM prefill needs the
 * decode position; the reference's seq_rope always starts at 0). */
int vx_seq_rope_at(vx_ctx *ctx, const vx_model *model, vx_buf *q, vx_buf *k, uint32_t position_base,
                   const vx_seq_rope_push *pc);
/* dense_attn_scores.comp:8, dense_softmax.comp:5, dense_attn_values.comp:7
 * (local.rs:500-504): full tokens x tokens attention, no causal mask. scores is
 * f32 [tokens][q_heads][score_stride]. */
int vx_dense_attn_scores(vx_ctx *ctx, const vx_buf *q, const vx_buf *k, vx_buf *scores,
                         const vx_dense_scores_push *pc);
int vx_dense_softmax(vx_ctx *ctx, vx_buf *scores, const vx_dense_softmax_push *pc);
int vx_dense_attn_values(vx_ctx *ctx, const vx_buf *scores, const vx_buf *v, vx_buf *out,
                         const vx_dense_values_push *pc);

/* ------------------------------------------------------------------------- */
/* Fused decode kernels used by the engine's graph (no single reference       */
/* pipeline: each is the composition of the reference ops named).            */
/* All read the decode position from device u32 position[0].                  */
/* ------------------------------------------------------------------------- */
typedef struct vx_fused_qkv_args {
    uint32_t norm_offset;           /* attn_norm weight (f32), rmsnorm.comp */
    float eps;
    uint32_t q_weight_offset, k_weight_offset, v_weight_offset;
    uint32_t q_rows, kv_rows, cols; /* q_rows = q_heads*head_dim, kv_rows = kv_heads*head_dim */
    uint32_t dtype;                 /* shared by q/k/v: VX_DTYPE_Q8_0 or VX_DTYPE_F16 */
    uint32_t factor_offset;         /* LongRoPE ext factors (f32[head_dim/2]) */
    uint32_t head_dim;
    float rope_theta, scaling_factor;
    uint32_t layer, context;
} vx_fused_qkv_args;
/* rmsnorm(hidden)*w -> qkv_matvec -> rope -> store_kv, one launch.
 * (rmsnorm.comp + qkv_matvec.comp + rope.comp + store_kv.comp; baselm.rs:915-967) */
int vx_fused_qkv_rope_store(vx_ctx *ctx, const vx_model *model, const vx_buf *hidden, vx_buf *q,
                            vx_buf *k, vx_buf *v, vx_buf *k_cache, vx_buf *v_cache,
                            const vx_buf *position, const vx_fused_qkv_args *a);

typedef struct vx_fused_attn_args {
    uint32_t layer, context, head_dim, q_heads, kv_heads;
    uint32_t splits;                /* context splits per kv head (grid = splits x kv_heads) */
} vx_fused_attn_args;
/* Split-context single-query attention: a partials kernel (online softmax per
 * context slice, all q heads of a KV head together) and a combine kernel;
 * attn_scores.comp + softmax.comp + attn_values.comp (baselm.rs:969-996).
 * `scratch` must hold vx_fused_attention_scratch_bytes(a) bytes. */
uint64_t vx_fused_attention_scratch_bytes(const vx_fused_attn_args *a);
int vx_fused_attention(vx_ctx *ctx, const vx_buf *q, const vx_buf *k_cache, const vx_buf *v_cache,
                       vx_buf *out, vx_buf *scratch, const vx_buf *position,
                       const vx_fused_attn_args *a);

/* Bytes of device scratch each GPU holds (from vx_init until the process ends)
 * for the entry points that allocate nothing. */
#define VX_NOALLOC_SCRATCH_BYTES (2u * 1024u * 1024u)
/* vx_fused_attention without the scratch argument, for callers that cannot
 * allocate: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc. It has no counterpart in the reference. It calls no
 * hipMalloc, hipFree, hipMemset or other allocating routine: the partials go to
 * a fixed per-GPU scratch of VX_NOALLOC_SCRATCH_BYTES, so a call needing more
 * than that (vx_fused_attention_scratch_bytes(a)) fails with VX_ERR_BOUNDS.
 * Every call on one GPU shares that scratch: calls that overlap on one GPU (on
 * different streams or contexts) race; calls in one stream are ordered. */
int vx_fused_attention_noalloc(vx_ctx *ctx, const vx_buf *q, const vx_buf *k_cache,
                               const vx_buf *v_cache, vx_buf *out, const vx_buf *position,
                               const vx_fused_attn_args *a);

typedef struct vx_fused_residual_args {
    uint32_t weight_offset, rows, cols, dtype;
    float scale;                    /* residual_scale (effective) */
} vx_fused_residual_args;
/* hidden += scale * (W . x): matvec.comp then the residual half of
 * residual_rmsnorm.comp (baselm.rs:998-1011,1022-1037). `branch`, if not NULL,
 * receives W . x. */
int vx_fused_matvec_residual(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *hidden,
                             vx_buf *branch, const vx_fused_residual_args *a);

typedef struct vx_fused_swiglu_args {
    uint32_t norm_offset;           /* ffn_norm weight (f32) */
    float eps;
    uint32_t gate_weight_offset, up_weight_offset, rows, cols, dtype;
} vx_fused_swiglu_args;
/* rmsnorm(hidden)*w -> matvec_swiglu (rmsnorm half of residual_rmsnorm.comp +
 * matvec_swiglu.comp; baselm.rs:1007-1021). */
int vx_fused_rms_swiglu(vx_ctx *ctx, const vx_model *model, const vx_buf *hidden, vx_buf *y,
                        const vx_fused_swiglu_args *a);

/* ------------------------------------------------------------------------- */
/* Diagnostics (no reference counterpart): plain streaming kernels that       */
/* calibrate the HBM roofline and the PMC byte counters.                      */
/* ------------------------------------------------------------------------- */
/* Read `bytes` of src at `offset` (both multiples of 16) with `blocks` x 256
 * threads and `unroll` (1, 2, 4, 8) 16-byte loads in flight per thread; sink
 * receives one word per wave (blocks * 16 bytes). */
int vx_diag_stream_read(vx_ctx *ctx, const vx_buf *src, uint64_t offset, uint64_t bytes, vx_buf *sink,
                        uint32_t blocks, uint32_t unroll);
/* Copy `bytes` (multiple of 16) from src to dst with `blocks` x 256 threads. */
int vx_diag_stream_copy(vx_ctx *ctx, vx_buf *dst, const vx_buf *src, uint64_t bytes, uint32_t blocks);
/* Decode-kernel timeline, for a library built with -DVX_STAMPS (`python -m
 * voxgen_amd.build --timeline`); the shipped library returns VX_ERR_UNSUPPORTED.
 * vx_diag_timeline_arm reserves room for `waves` wave records on ctx's device
 * (cleared) and empties the launch table: every decode kernel enqueued or
 * captured into a graph afterwards (qkv, attention, attn_out, SwiGLU, matvec)
 * gets one record per wave, which each run of the kernel (each graph replay)
 * overwrites with its s_memrealtime ticks (100 MHz) at the wave's start and end.
 * Launches past the reserved room are not recorded. One timeline per process. */
int vx_diag_timeline_arm(vx_ctx *ctx, uint64_t waves);
/* After vx_sync: copies up to max_launches launch records, three u64 each
 * (kind: 1 qkv, 2 attention chunk, 3 attention stream, 4 attn_out, 5 SwiGLU,
 * 6 matvec; first wave record; wave count), and up to max_waves (start, end)
 * tick pairs; *n_launches and *n_waves receive the totals recorded. */
int vx_diag_timeline_read(vx_ctx *ctx, uint64_t *launches, uint64_t max_launches, uint64_t *ticks,
                          uint64_t max_waves, uint64_t *n_launches, uint64_t *n_waves);

/* ------------------------------------------------------------------------- */
/* GGUF (gguf.rs:222-286): host-side parse of a model file.                   */
/* ------------------------------------------------------------------------- */
int vx_gguf_open(const char *path, vx_gguf **out);
int vx_gguf_close(vx_gguf *g);
typedef struct vx_gguf_summary {    /* GgufSummary gguf.rs:61-81 (scalar part) */
    uint32_t version;
    uint64_t tensor_count, metadata_count, alignment, data_offset, file_bytes, tensor_bytes;
} vx_gguf_summary;
int vx_gguf_summary_get(const vx_gguf *g, vx_gguf_summary *out);
int vx_gguf_tensor_at(const vx_gguf *g, uint32_t index, vx_tensor_info *out);
int vx_gguf_find(const vx_gguf *g, const char *name, vx_tensor_info *out);
/* Metadata value rendered as text, as GgufSummary::metadata stores it. */
int vx_gguf_meta(const vx_gguf *g, const char *key, char *out, uint32_t cap);
/* GgufSummary::primary_base_format (gguf.rs:117-133): 8 = Q8_0, 1 = F16. */
int vx_gguf_primary_format(const vx_gguf *g, uint32_t *dtype_out);
/* Upload the file's data region and tensor table as a vx_model. */
int vx_model_upload_gguf(vx_ctx *ctx, const vx_gguf *g, vx_model **out);

/* ------------------------------------------------------------------------- */
/* BaseLM engine (BaseLmEngine, baselm.rs:423-890).                           */
/* ------------------------------------------------------------------------- */
typedef struct vx_baselm_config {   /* BaseLmConfig baselm.rs:34-56 */
    uint32_t context_length;
    uint32_t active_context_length;
    uint32_t embedding_length;
    uint32_t block_count;
    uint32_t feed_forward_length;
    uint32_t vocab_size;
    uint32_t head_count;
    uint32_t head_count_kv;
    uint32_t head_dim;
    uint32_t kv_dim;
    float rms_epsilon;
    float rope_theta;
    uint32_t rope_dimension_count;
    uint32_t rope_original_context_length;
    uint32_t rope_longrope;         /* 1: rope_scaling_type == "longrope", 0: "none" */
    float embedding_scale;
    float residual_scale;
    float logit_scale;
    uint32_t tied_output;
} vx_baselm_config;

/* BaseLmConfig::from_gguf (baselm.rs:60-180), including every geometry check. */
int vx_baselm_config_from_gguf(const vx_gguf *g, uint32_t active_context_length,
                               vx_baselm_config *out);
/* BaseLmConfig::rope_scaling_factor (baselm.rs:194-205). */
float vx_baselm_rope_scaling_factor(const vx_baselm_config *cfg);
/* BaseLmConfig::kv_cache_bytes / per_cache_bytes (baselm.rs:182-192). */
uint64_t vx_baselm_kv_cache_bytes(const vx_baselm_config *cfg);

/* Execution modes of the engine. */
#define VX_EXEC_GRAPH 0u     /* fused kernels, each step replayed as one hipGraph */
#define VX_EXEC_FUSED 1u     /* fused kernels launched eagerly                   */
#define VX_EXEC_REFERENCE 2u /* the reference's 11 per-op dispatches per layer   */
#define VX_EXEC_PERSISTENT 3u /* reserved: the one-kernel persistent step, measured
                                 slower than VX_EXEC_GRAPH on MI355X and removed;
                                 vx_baselm_create refuses it (VX_ERR_UNSUPPORTED) */

typedef struct vx_baselm_options {
    uint32_t exec_mode;          /* VX_EXEC_* */
    uint32_t strict_geometry;    /* 1: enforce the VoxCPM2 geometry (baselm.rs:102-113);
                                    0: allow other layer counts/sizes for harnesses */
    uint32_t attn_splits;        /* 0 = choose from active_context_length */
    uint32_t prefill_schedule;   /* VX_PREFILL_* (batched prefill, gate/up GEMM) */
} vx_baselm_options;
/* Workgroup schedule of the batched prefill's gate/up projection (no counterpart
 * in the reference, which has no batched MFMA prefill). */
#define VX_PREFILL_AUTO 0u       /* stream-K when the tiles just exceed the CUs,
                                    whole and half-K tiles side by side up to 1.5
                                    tiles per CU, else one tile per workgroup    */
#define VX_PREFILL_TILES 1u      /* one tile per workgroup                       */
#define VX_PREFILL_STREAMK_TAIL_FIRST 2u /* stream-K with each workgroup's tile
                                    tail computed before its head: the hand-off
                                    order AUTO meets only when a workgroup starts
                                    late; bit-identical results, slower          */

/* BaseLmEngine::new (baselm.rs:451-586). Validates every tensor of the model
 * against the config (validate_layer baselm.rs:227-262) and allocates the
 * activation buffers and the packed f16 KV caches. */
int vx_baselm_create(vx_ctx *ctx, const vx_model *model, const vx_baselm_config *cfg,
                     const vx_baselm_options *opt, vx_baselm **out);
int vx_baselm_destroy(vx_baselm *eng);
/* reset (baselm.rs:616-620): position := 0, cache contents left in place. */
int vx_baselm_reset(vx_baselm *eng);
uint32_t vx_baselm_position(const vx_baselm *eng);
/* Harness hook: set the next decode position (e.g. after filling the cache). */
int vx_baselm_set_position(vx_baselm *eng, uint32_t position);

typedef struct vx_top_logit {       /* TopLogit baselm.rs:398-402 */
    uint32_t token_id;
    float logit;
} vx_top_logit;
typedef struct vx_step_result {     /* BaseLmStepResult baselm.rs:404-411 */
    uint32_t position;
    double elapsed_ms;
    double final_hidden_checksum;
    double final_hidden_l2;
    uint32_t n_top;                 /* entries written to the caller's top array */
} vx_step_result;

/* top_k_logits (baselm.rs:1296-1311): finite logits sorted descending (ties by
 * ascending id), first min(k, finite count) written to out. Host-only. */
int vx_top_k_logits(const float *logits, uint32_t n, uint32_t k, vx_top_logit *out, uint32_t *n_out);

/* decode_token (baselm.rs:622-655): embedding + layers + LM head, then
 * readback of the final hidden state and the top_k logits into `top`
 * (caller array of top_k entries; may be NULL when top_k == 0). */
int vx_baselm_decode_token(vx_baselm *eng, uint32_t token_id, uint32_t top_k,
                           vx_step_result *res, vx_top_logit *top);
/* decode_embedding (baselm.rs:657-680): host f32[embedding_length] input. */
int vx_baselm_decode_embedding(vx_baselm *eng, const float *embedding, uint32_t n, uint32_t top_k,
                               vx_step_result *res, vx_top_logit *top);
/* decode_token_gpu_only (baselm.rs:689-721): no LM head, no readback. */
int vx_baselm_decode_token_gpu_only(vx_baselm *eng, uint32_t token_id, uint32_t *position_out);
/* decode_embedding_gpu_only (baselm.rs:764-791). */
int vx_baselm_decode_embedding_gpu_only(vx_baselm *eng, const float *embedding, uint32_t n,
                                        uint32_t *position_out);
/* decode_embedding_from_gpu_only (baselm.rs:793-821): device f32 source. */
int vx_baselm_decode_embedding_from_gpu_only(vx_baselm *eng, const vx_buf *source,
                                             uint32_t *position_out);
/* Token-only steps for n tokens enqueued back to back without host waits
 * (the batching record_token_gpu_only_in provides, baselm.rs:726-762). */
int vx_baselm_decode_tokens_gpu_only(vx_baselm *eng, const uint32_t *tokens, uint32_t n);
/* prefill_tokens (baselm.rs:823-839): sequential decode of every token. */
int vx_baselm_prefill_tokens(vx_baselm *eng, const uint32_t *tokens, uint32_t n, uint32_t top_k_last,
                             vx_step_result *res, vx_top_logit *top);
/* Token-batched prefill: prefill_tokens (baselm.rs:823-839) with the n tokens
 * run through the layer stack together -- MFMA projections over all tokens,
 * causal attention over the KV cache, KV rows stored at positions
 * position..position+n-1 -- instead of n sequential decode steps. Same engine
 * state afterwards (KV cache, position, hidden/norm of the last token, its
 * logits and top_k) to rounding. Needs Q8_0 row widths that are multiples of
 * 1024 (F16: of 128), head_dim 64/128 and 1/2/4/8 query heads per KV head. */
int vx_baselm_prefill_tokens_batched(vx_baselm *eng, const uint32_t *tokens, uint32_t n,
                                     uint32_t top_k_last, vx_step_result *res, vx_top_logit *top);
/* Same without the LM head, readback or host wait (the *_gpu_only semantics). */
int vx_baselm_prefill_tokens_batched_gpu_only(vx_baselm *eng, const uint32_t *tokens, uint32_t n);
typedef struct vx_baselm_benchmark_result { /* BaseLmBenchmark baselm.rs:413-421 */
    uint32_t iterations, token_id;
    double mean_ms, min_ms, max_ms, tokens_per_second;
} vx_baselm_benchmark_result;
/* benchmark (baselm.rs:841-880). */
int vx_baselm_benchmark(vx_baselm *eng, uint32_t token_id, uint32_t warmup, uint32_t iterations,
                        vx_baselm_benchmark_result *out);
/* Engine-owned buffers: output_buffer (norm, baselm.rs:608-612) and the rest. */
#define VX_BASELM_BUF_HIDDEN 0u
#define VX_BASELM_BUF_NORM 1u
#define VX_BASELM_BUF_Q 2u
#define VX_BASELM_BUF_K 3u
#define VX_BASELM_BUF_V 4u
#define VX_BASELM_BUF_ATTENTION 5u
#define VX_BASELM_BUF_GATE 6u
#define VX_BASELM_BUF_BRANCH 7u
#define VX_BASELM_BUF_LOGITS 8u
#define VX_BASELM_BUF_SCORES 9u
#define VX_BASELM_BUF_KV_K 10u
#define VX_BASELM_BUF_KV_V 11u
#define VX_BASELM_BUF_POSITION 12u
vx_buf *vx_baselm_buffer(vx_baselm *eng, uint32_t which);
/* Per-kernel timing of `n` token-only steps, each kernel bracketed by HIP events
 * on the engine stream (mirrors the reference's "baselm.*" profile spans).
 * Fills up to `cap` entries; *count receives the number of kernel names. */
int vx_baselm_profile_steps(vx_baselm *eng, const uint32_t *tokens, uint32_t n,
                            vx_prof_entry *out, uint32_t cap, uint32_t *count);

/* Average cost of one kernel of the fused decode layer inside a graph chain:
 * `reps` passes, each a 384 MiB streaming read that evicts the MALL and the L2s
 * followed by the kernel over every layer, captured as one graph and timed with
 * HIP events on the engine stream; a graph of the reads alone is subtracted. Each
 * launch therefore reads its weights from HBM, as in a decode step, and the
 * figure includes the launch gap between dependent kernels. Allocates 384 MiB for
 * the call. `which`: VX_LAYER_KERNEL_*. The kernels read the device position and
 * overwrite the engine's activations and the KV-cache row at that position. No
 * reference counterpart: it is the measurement the gpu_profile spans
 * (vulkan.rs:587-612) give per dispatch. */
#define VX_LAYER_KERNEL_QKV 0u
#define VX_LAYER_KERNEL_ATTENTION 1u
#define VX_LAYER_KERNEL_ATTN_OUT 2u
#define VX_LAYER_KERNEL_SWIGLU 3u
#define VX_LAYER_KERNEL_DOWN 4u
int vx_baselm_time_layer_kernel(vx_baselm *eng, uint32_t which, uint32_t reps, double *avg_ms);

/* ------------------------------------------------------------------------- */
/* CFM shader entry points (UnifiedCFM pieces, local.rs:383-430).             */
/* ------------------------------------------------------------------------- */
/* cfm_noise.comp:25-37: x[i] = temperature * N(0,1) from the integer hash of
 * (i/2, seed); dispatched at local.rs:404. */
int vx_cfm_noise(vx_ctx *ctx, vx_buf *x, const vx_cfm_noise_push *pc);
/* cfm_cfg_euler.comp:15-36 (CFG-Zero* scale, Euler step), local.rs:423. */
int vx_cfm_cfg_euler(vx_ctx *ctx, vx_buf *x, const vx_buf *positive, const vx_buf *negative,
                     const vx_cfm_euler_push *pc);
/* time_sinusoidal.comp:5, local.rs:471. */
int vx_time_sinusoidal(vx_ctx *ctx, vx_buf *out, const vx_time_push *pc);
/* pack_locdit.comp:10: [mu1, mu2, time, cond x patch, x x patch] rows, local.rs:465. */
int vx_pack_locdit(vx_ctx *ctx, const vx_buf *mu1, const vx_buf *mu2, const vx_buf *time, const vx_buf *cond,
                   const vx_buf *x, vx_buf *hidden, const vx_pack_locdit_push *pc);
/* silu_inplace.comp:5 and add_vectors.comp:6. */
int vx_silu_inplace(vx_ctx *ctx, vx_buf *x, uint32_t n);
typedef struct vx_fsq_push {        /* FsqPush acoustic.rs:249-255 */
    uint32_t n;
    float scale;
} vx_fsq_push;
/* fsq_quantize.comp: latent[i] = round(tanh(latent[i]) * scale) / scale, in place
 * (record_fsq, acoustic.rs:922-928). Ties round away from zero. */
int vx_fsq_quantize(vx_ctx *ctx, vx_buf *latent, const vx_fsq_push *pc);
int vx_add_vectors(vx_ctx *ctx, vx_buf *a, const vx_buf *b, uint32_t n);

/* ------------------------------------------------------------------------- */
/* LocDiT estimator + UnifiedCFM solve (LocalEngine, local.rs:264-537).       */
/* ------------------------------------------------------------------------- */
typedef struct vx_locdit_config {   /* LocalConfig local.rs:51-70, LocDiT part */
    uint32_t hidden, layers, q_heads, kv_heads, head_dim, ffn;
    uint32_t feat_dim, patch;       /* latent patch: patch tokens x feat_dim (4 x 64) */
    uint32_t n_mu;                  /* mu tokens ahead of the time token (VoxCPM2: 2) */
    uint32_t n_cond;                /* condition tokens after the time token */
    uint32_t cond_raw;              /* 0: condition = patch x feat_dim latent through locdit.cond_proj
                                       (n_cond == patch, the reference); 1: n_cond x hidden rows given */
    uint32_t uncond_zero_cond;      /* 1: the unconditional CFG pass also zeroes the condition rows
                                       (the reference zeroes only the mu tokens) */
    float rms_epsilon, rope_theta, rope_scaling;
} vx_locdit_config;

typedef struct vx_cfm_options {     /* CfmOptions local.rs:244-252 */
    uint32_t n_timesteps;
    float cfg_value, temperature, sway_sampling_coef;
    uint64_t seed;
    uint32_t use_cfg_zero_star;
} vx_cfm_options;

typedef struct vx_cfm_result {      /* CfmResult local.rs:253-261 (scalar part) */
    double elapsed_ms;
    uint32_t n_timesteps, estimator_calls, zero_init_steps;
    double output_checksum, output_l2;
    float output_min, output_max;
} vx_cfm_result;

/* LocalEngine::new (local.rs:276-339), LocDiT half: validates the locdit.*
 * tensors of `model` (F16 matrices, F32 norms; validate_tensors local.rs:127-168)
 * and allocates a CFG batch of two sequences. RoPE factors are the BaseLM's
 * (rope_model, rope_factor_offset; local.rs:336-337). strict_geometry enforces
 * the VoxCPM2 contract (12 x 1024, 16/2 x 128, ffn 4096, 4 x 64, two mu tokens). */
int vx_locdit_create(vx_ctx *ctx, const vx_model *model, const vx_model *rope_model, uint32_t rope_factor_offset,
                     const vx_locdit_config *cfg, uint32_t strict_geometry, vx_locdit **out);
int vx_locdit_destroy(vx_locdit *loc);
/* locdit_from_cpu_mu (local.rs:352-355): one estimator pass on host inputs
 * x [patch x feat_dim], cond (see cond_raw), mu [n_mu x hidden]; out [patch x feat_dim]. */
int vx_locdit_estimate(vx_locdit *loc, const float *x, const float *cond, const float *mu, float t, float dt,
                       float *out);
/* cfm_from_cpu_mu (local.rs:359-363, cfm_solve 383-430): noise (or initial_x),
 * then every Euler step's conditional and unconditional estimate as one batch
 * of two and the CFG-Zero* update; the whole solve is one hipGraph replay.
 * out_patch receives the final x [patch x feat_dim]. */
int vx_locdit_cfm_solve(vx_locdit *loc, const float *cond, const float *mu, const vx_cfm_options *opt,
                        const float *initial_x, float *out_patch, vx_cfm_result *res);
/* cfm_from_model_hiddens (local.rs:379-381; record_project_mu 459-462): the same
 * solve with the two mu tokens projected on the device, inside the solve's graph,
 * from the ResidualLM engine's buffers the reference binds to the local engine
 * (runtime.rs:239-243): mu1 = projections.lm_to_dit_proj . current_lm + b
 * (VX_RESIDUAL_BUF_CURRENT_LM), mu2 = projections.res_to_dit_proj . output + b
 * (VX_RESIDUAL_BUF_OUTPUT); each buffer holds the projections' input width
 * (2048) of f32. No host round trip. VX_ERR_NOT_FOUND if the model lacks the
 * projections (they are required only under strict geometry). */
int vx_locdit_cfm_solve_from_model_hiddens(vx_locdit *loc, const vx_buf *current_lm,
                                           const vx_buf *residual_output, const float *cond,
                                           const vx_cfm_options *opt, const float *initial_x,
                                           float *out_patch, vx_cfm_result *res);

/* ------------------------------------------------------------------------- */
/* ResidualLM + FSQ + fusion + stop head (ResidualFsqEngine, acoustic.rs:400-1035). */
/* ------------------------------------------------------------------------- */
typedef struct vx_acoustic_config { /* AcousticConfig acoustic.rs:39-56 (numeric part) */
    float model_version;
    uint32_t residual_block_count;
    uint32_t embedding_length;
    uint32_t feed_forward_length;
    uint32_t head_count;
    uint32_t head_count_kv;
    uint32_t head_dim;
    uint32_t kv_dim;
    uint32_t no_rope;
    uint32_t active_context_length;
    float rms_epsilon;
    float residual_scale;           /* already effective_scale()d, acoustic.rs:117 */
    uint32_t fsq_latent_dim;
    float fsq_scale;
    uint32_t fusion_input_dim;
} vx_acoustic_config;

/* AcousticConfig::from_gguf (acoustic.rs:59-125): architecture, version and the
 * 8/2048/512/no-RoPE contract, BaseLM geometry compatibility, every tensor
 * (validate_tensors acoustic.rs:127-174) and GgufSummary::validate_acoustic_f16
 * (gguf.rs:150-160). */
int vx_acoustic_config_from_gguf(const vx_gguf *g, const vx_baselm_config *base, uint32_t active_context_length,
                                 vx_acoustic_config *out);
/* AcousticConfig::kv_cache_bytes / per_cache_bytes (acoustic.rs:176-187). */
uint64_t vx_acoustic_kv_cache_bytes(const vx_acoustic_config *cfg);

typedef struct vx_residual_options {
    uint32_t exec_mode;             /* VX_EXEC_GRAPH, VX_EXEC_FUSED or VX_EXEC_REFERENCE */
    uint32_t strict_geometry;       /* 1: the VoxCPM2 contract; 0: other sizes for harnesses */
} vx_residual_options;

typedef struct vx_fsq_result {      /* FsqResult acoustic.rs:359-366 */
    double elapsed_ms;
    double output_checksum, output_l2;
    double latent_checksum, latent_l2;
} vx_fsq_result;

typedef struct vx_residual_step_result {   /* ResidualStepResult acoustic.rs:368-379 */
    uint32_t position;
    uint32_t fsq_applied;
    double elapsed_ms;
    double fsq_checksum, fsq_l2;    /* 0 when fsq_applied == 0 (None) */
    double fused_input_checksum, fused_input_l2;
    double residual_hidden_checksum, residual_hidden_l2;
} vx_residual_step_result;

typedef struct vx_residual_gpu_step {      /* ResidualGpuStep acoustic.rs:381 */
    uint32_t position;
    uint32_t fsq_applied;
    double elapsed_ms;
} vx_residual_gpu_step;

typedef struct vx_residual_benchmark {     /* ResidualBenchmark acoustic.rs:384-391 */
    uint32_t iterations;
    double mean_ms, min_ms, max_ms, steps_per_second;
} vx_residual_benchmark_result;

typedef struct vx_stop_prediction {        /* StopPrediction acoustic.rs:393-398 */
    uint32_t stop;                  /* stop_logit > continue_logit */
    float continue_logit, stop_logit;
    double elapsed_ms;
} vx_stop_prediction;

/* ResidualFsqEngine::new (acoustic.rs:432-583): resolves every tensor, allocates
 * the activations and the f16 ResidualLM KV caches. */
int vx_residual_create(vx_ctx *ctx, const vx_model *acoustic, const vx_acoustic_config *cfg,
                       const vx_residual_options *opt, vx_residual **out);
int vx_residual_destroy(vx_residual *eng);
uint32_t vx_residual_position(const vx_residual *eng);          /* acoustic.rs:585 */
int vx_residual_reset(vx_residual *eng);                        /* acoustic.rs:589 */
uint64_t vx_residual_allocated_bytes(const vx_residual *eng);   /* acoustic.rs:591-613 */

#define VX_RESIDUAL_BUF_OUTPUT 0u        /* norm: the normalised ResidualLM output (output_buffer) */
#define VX_RESIDUAL_BUF_CURRENT_LM 1u    /* current_lm_buffer (acoustic.rs:588) */
#define VX_RESIDUAL_BUF_FSQ_LATENT 2u
#define VX_RESIDUAL_BUF_FSQ_OUTPUT 3u
#define VX_RESIDUAL_BUF_FUSION_SNAPSHOT 4u
#define VX_RESIDUAL_BUF_HIDDEN 5u
#define VX_RESIDUAL_BUF_KV_K 6u
#define VX_RESIDUAL_BUF_KV_V 7u
#define VX_RESIDUAL_BUF_STOP_LOGITS 8u
vx_buf *vx_residual_buffer(vx_residual *eng, uint32_t which);

/* fsq_only (acoustic.rs:654-676): FSQ of a host hidden state; no position change. */
int vx_residual_fsq_only(vx_residual *eng, const float *base_hidden, uint32_t n, vx_fsq_result *out);
/* step (acoustic.rs:678-692): FSQ(base) -> current_lm, fusion with the current
 * acoustic embedding, one ResidualLM position. Host inputs of n floats each. */
int vx_residual_step(vx_residual *eng, const float *base_hidden, const float *current_embedding, uint32_t n,
                     vx_residual_step_result *out);
/* step_from_gpu_base (acoustic.rs:694-710). */
int vx_residual_step_from_gpu_base(vx_residual *eng, const vx_buf *base_hidden, const float *current_embedding,
                                   uint32_t n, vx_residual_step_result *out);
/* step_from_gpu_base_and_embedding (acoustic.rs:712-726). */
int vx_residual_step_from_gpu_base_and_embedding(vx_residual *eng, const vx_buf *base_hidden,
                                                 const vx_buf *current_embedding, vx_residual_step_result *out);
/* step_from_gpu_base_and_embedding_gpu_only (acoustic.rs:728-731): enqueue only. */
int vx_residual_step_from_gpu_base_and_embedding_gpu_only(vx_residual *eng, const vx_buf *base_hidden,
                                                          const vx_buf *current_embedding,
                                                          vx_residual_gpu_step *out);
/* step_text_prefix_from_gpu_base (acoustic.rs:740-757): no FSQ, raw BaseLM
 * hidden -> current_lm, zero acoustic half of the fusion input. */
int vx_residual_step_text_prefix_from_gpu_base(vx_residual *eng, const vx_buf *base_hidden,
                                               vx_residual_step_result *out);
/* step_text_prefix_from_gpu_base_gpu_only (acoustic.rs:733-736): enqueue only. */
int vx_residual_step_text_prefix_from_gpu_base_gpu_only(vx_residual *eng, const vx_buf *base_hidden,
                                                        vx_residual_gpu_step *out);
/* benchmark (acoustic.rs:759-793): reset, warmup + iterations host steps. */
int vx_residual_benchmark(vx_residual *eng, const float *base_hidden, const float *current_embedding, uint32_t n,
                          uint32_t warmup, uint32_t iterations, vx_residual_benchmark_result *out);
/* predict_stop_from_gpu_base (acoustic.rs:619-634): Linear+SiLU+Linear(->2). */
int vx_residual_predict_stop_from_gpu_base(vx_residual *eng, const vx_buf *base_hidden, vx_stop_prediction *out);
/* predict_stop_from_current_lm (acoustic.rs:638-652). */
int vx_residual_predict_stop_from_current_lm(vx_residual *eng, vx_stop_prediction *out);
/* n text-prefix positions (step_text_prefix_from_gpu_base_gpu_only each,
 * acoustic.rs:733-736) from n BaseLM output rows [n][hidden] f32 at once: one
 * batched fusion projection and a token-batched ResidualLM stack. Enqueue only;
 * graph or fused exec mode. */
int vx_residual_prefill_text_from_gpu_rows(vx_residual *eng, const vx_buf *rows, uint32_t n);
/* The text runs of prefill_conditioning_plan (runtime.rs:483-566): for each token,
 * a BaseLM decode then a ResidualLM text-prefix step from its output, computed as
 * a batched BaseLM prefill (every position's output row kept) followed by the
 * batched ResidualLM text prefix, in chunks of up to 512 positions. Both engines
 * advance by n and end in the state of the last position. Enqueue only. */
int vx_prefill_text_cross_engine(vx_baselm *base, vx_residual *eng, const uint32_t *tokens, uint32_t n);

/* ------------------------------------------------------------------------- */
/* AudioVAE decoder (AudioVaeEngine::decode_latents, audiovae.rs:330-372).     */
/* ------------------------------------------------------------------------- */
typedef struct vx_vae_conv_push {   /* ConvPush audiovae.rs:198-202 */
    uint32_t weight_offset, bias_offset, in_channels, out_channels, in_length, out_length;
    uint32_t kernel, stride, dilation, groups, left_pad, weight_dtype, bias_dtype, has_bias;
} vx_vae_conv_push;
typedef struct vx_vae_convt_push {  /* ConvTPush audiovae.rs:203-204 */
    uint32_t weight_offset, bias_offset, in_channels, out_channels, in_length, out_length;
    uint32_t kernel, stride, groups, weight_dtype, bias_dtype, has_bias;
} vx_vae_convt_push;
typedef struct vx_vae_snake_push {  /* SnakePush audiovae.rs:205-206 */
    uint32_t alpha_offset, channels, length, dtype;
} vx_vae_snake_push;
typedef struct vx_vae_scale_push {  /* ScalePush audiovae.rs:207-208 */
    uint32_t scale_offset, bias_offset, channels, length, bucket, buckets, scale_dtype, bias_dtype;
} vx_vae_scale_push;
typedef struct vx_vae_grid_push {   /* GridPush audiovae.rs:210 */
    uint32_t channels, length;
} vx_vae_grid_push;
/* The shaders over channel-major [C][L] f32 buffers, model scalars from the model
 * region: vae_conv1d.comp, vae_convtranspose1d.comp, vae_snake.comp (x -> y),
 * vae_scale_bias.comp (in place), vae_add.comp (a += b), vae_tanh.comp. */
int vx_vae_conv1d(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y, const vx_vae_conv_push *pc);
int vx_vae_convtranspose1d(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y,
                           const vx_vae_convt_push *pc);
int vx_vae_snake(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y, const vx_vae_snake_push *pc);
int vx_vae_scale_bias(vx_ctx *ctx, const vx_model *model, vx_buf *x, const vx_vae_scale_push *pc);
int vx_vae_add(vx_ctx *ctx, vx_buf *a, const vx_buf *b, const vx_vae_grid_push *pc);
int vx_vae_tanh(vx_ctx *ctx, vx_buf *x, uint32_t n);

typedef struct vx_audiovae_config { /* AudioVaeConfig audiovae.rs:29-47 (numeric part) */
    uint32_t encoder_dim, latent_dim, decoder_dim, sample_rate, out_sample_rate;
    uint32_t encoder_rates[4];
    uint32_t decoder_rates[6];
    uint32_t encoder_hop, decoder_hop, patch_size;
    uint32_t input_samples_per_patch, output_samples_per_patch;
    uint32_t sr_bin_boundaries[3];
    uint32_t decoder_sr_bucket;
    uint32_t depthwise;
} vx_audiovae_config;
/* AudioVaeConfig::from_gguf (audiovae.rs:49-79) with validate_tensors
 * (audiovae.rs:81-128): the V2 geometry, cond_type scale_bias, every encoder and
 * decoder tensor. */
int vx_audiovae_config_from_gguf(const vx_gguf *g, vx_audiovae_config *out);

typedef struct vx_audio_decode_stats {   /* AudioDecodeStats audiovae.rs:179-191 */
    uint32_t latent_frames, latent_patches, output_samples, output_sample_rate;
    double duration_seconds, checksum, l2;
    float peak;
    double decode_ms;
    uint64_t scratch_bytes;
} vx_audio_decode_stats;

/* AudioVaeEngine::new (audiovae.rs:256-260): resolves the decoder tensors and
 * repacks the transposed-convolution weights for the GEMM form. strict_geometry
 * 0 admits other decoder widths (harnesses). */
int vx_audiovae_create(vx_ctx *ctx, const vx_model *model, const vx_audiovae_config *cfg, uint32_t strict_geometry,
                       vx_audiovae **out);
int vx_audiovae_destroy(vx_audiovae *vae);
uint64_t vx_audiovae_scratch_bytes(const vx_audiovae *vae);   /* audiovae.rs:261 */
/* decode_latents (audiovae.rs:330-372): frame-major latents [frames][latent_dim]
 * (frames a multiple of patch_size) -> mono wave of frames * decoder_hop samples
 * at out_sample_rate into wave (wave_cap floats). */
int vx_audiovae_decode_latents(vx_audiovae *vae, const float *frame_major, uint64_t n_values, float *wave,
                               uint64_t wave_cap, vx_audio_decode_stats *out);
/* The same decode from and to device buffers, enqueue only (no checks of the
 * values; frames a multiple of patch_size). */
int vx_audiovae_decode_latents_gpu(vx_audiovae *vae, const vx_buf *frame_major, uint32_t frames, vx_buf *wave);

#ifdef __cplusplus
}
#endif
#endif /* VOXHIP_H */
