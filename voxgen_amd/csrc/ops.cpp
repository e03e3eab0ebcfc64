// Per-op C ABI: one entry point per reference pipeline. Each validates the push
// extents against the model's tensor table and the bound buffers (so no kernel
// is launched with an out-of-range operand), then enqueues the HIP kernel(s).
#include "vx_internal.h"

using namespace vx;

namespace {

inline float *F(vx_buf *b) { return static_cast<float *>(b->ptr); }
inline const float *CF(const vx_buf *b) { return static_cast<const float *>(b->ptr); }
inline const uint32_t *CU(const vx_buf *b) { return static_cast<const uint32_t *>(b->ptr); }

int need_ctx(vx_ctx *ctx, const void *pc, const char *what) {
    if (!ctx || !pc) return fail(VX_ERR_INVALID_ARG, "%s: null context or push struct", what);
    return VX_OK;
}

// matvec.comp family: dtype 1 is F16, 8 is Q8_0 (dtype_code, baselm.rs:1239-1245).
int check_mv_dtype(uint32_t dtype, const char *what) {
    if (dtype != VX_DTYPE_F16 && dtype != VX_DTYPE_Q8_0)
        return fail(VX_ERR_UNSUPPORTED, "%s: unsupported BaseLM matrix type %u", what, dtype);
    return VX_OK;
}

uint64_t cache_halves(uint32_t layer, uint32_t context, uint32_t position_plus1, uint32_t kv_dim) {
    return ((uint64_t)layer * context + position_plus1) * kv_dim;
}

}  // namespace

extern "C" {

int vx_embedding(vx_ctx *ctx, const vx_model *model, vx_buf *hidden, const vx_embedding_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_embedding"));
    const uint32_t dtype = pc->dtype == VX_DTYPE_F16 ? VX_DTYPE_F16 : VX_DTYPE_Q8_0;
    WRef w;
    VX_CHECK(resolve_matrix(model, pc->weight_offset, dtype, 1, pc->cols, &w, "vx_embedding"));
    if (pc->token_id >= w.rows)
        return fail(VX_ERR_TOKEN_RANGE, "token id %u is outside vocabulary 0..%u", pc->token_id, w.rows);
    VX_CHECK(need_buf(hidden, (uint64_t)pc->cols * 4u, "vx_embedding hidden"));
    ProfSpan span(ctx, "baselm.embedding");
    return launch_embedding(ctx->stream, model->raw, pc->weight_offset, dtype, pc->cols, pc->token_id,
                            nullptr, nullptr, w.rows, pc->alpha, F(hidden));
}

int vx_embedding_devtok(vx_ctx *ctx, const vx_model *model, vx_buf *hidden, const vx_buf *tokens,
                        const vx_buf *position, const vx_embedding_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_embedding_devtok"));
    const uint32_t dtype = pc->dtype == VX_DTYPE_F16 ? VX_DTYPE_F16 : VX_DTYPE_Q8_0;
    WRef w;
    VX_CHECK(resolve_matrix(model, pc->weight_offset, dtype, 1, pc->cols, &w, "vx_embedding_devtok"));
    VX_CHECK(need_buf(hidden, (uint64_t)pc->cols * 4u, "vx_embedding_devtok hidden"));
    VX_CHECK(need_buf(tokens, 4u, "vx_embedding_devtok tokens"));
    VX_CHECK(need_buf(position, 4u, "vx_embedding_devtok position"));
    ProfSpan span(ctx, "baselm.embedding");
    return launch_embedding(ctx->stream, model->raw, pc->weight_offset, dtype, pc->cols, 0, CU(tokens),
                            CU(position), w.rows, pc->alpha, F(hidden), (uint32_t)(tokens->bytes / 4u));
}

int vx_rmsnorm(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y, const vx_rms_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_rmsnorm"));
    const void *w = nullptr;
    VX_CHECK(resolve_vector(model, pc->weight_offset, VX_DTYPE_F32, pc->n, &w, "vx_rmsnorm weight"));
    VX_CHECK(need_buf(x, (uint64_t)pc->n * 4u, "vx_rmsnorm x"));
    VX_CHECK(need_buf(y, (uint64_t)pc->n * 4u, "vx_rmsnorm y"));
    ProfSpan span(ctx, "baselm.rmsnorm");
    return launch_rmsnorm(ctx->stream, CF(x), F(y), static_cast<const float *>(w), pc->n, pc->eps, nullptr);
}

int vx_residual_rmsnorm(vx_ctx *ctx, const vx_model *model, vx_buf *hidden, const vx_buf *branch, vx_buf *y,
                        const vx_residual_rms_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_residual_rmsnorm"));
    const void *w = nullptr;
    VX_CHECK(resolve_vector(model, pc->weight_offset, VX_DTYPE_F32, pc->n, &w, "vx_residual_rmsnorm weight"));
    VX_CHECK(need_buf(hidden, (uint64_t)pc->n * 4u, "vx_residual_rmsnorm hidden"));
    VX_CHECK(need_buf(branch, (uint64_t)pc->n * 4u, "vx_residual_rmsnorm branch"));
    VX_CHECK(need_buf(y, (uint64_t)pc->n * 4u, "vx_residual_rmsnorm y"));
    ProfSpan span(ctx, "baselm.residual_rmsnorm");
    return launch_residual_rmsnorm(ctx->stream, F(hidden), CF(branch), F(y), static_cast<const float *>(w),
                                   pc->n, pc->eps, pc->scale);
}

int vx_matvec(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y, const vx_matvec_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_matvec"));
    VX_CHECK(check_mv_dtype(pc->dtype, "vx_matvec"));
    WRef w;
    VX_CHECK(resolve_matrix(model, pc->weight_offset, pc->dtype, pc->rows, pc->cols, &w, "vx_matvec"));
    VX_CHECK(need_buf(x, (uint64_t)pc->cols * 4u, "vx_matvec x"));
    VX_CHECK(need_buf(y, (uint64_t)pc->rows * 4u, "vx_matvec y"));
    ProfSpan span(ctx, "baselm.matvec");
    MatvecLaunch l;
    l.w = w;
    l.xl = CF(x);
    l.rows = pc->rows;
    l.cols = pc->cols;
    l.row_base = pc->row_base;
    l.alpha = pc->alpha;
    l.epi = EPI_STORE;
    l.y = F(y);
    return launch_matvec(ctx->stream, l);
}

int vx_qkv_matvec(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *q, vx_buf *k, vx_buf *v,
                  const vx_qkv_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_qkv_matvec"));
    const uint32_t offs[3] = {pc->q_weight_offset, pc->k_weight_offset, pc->v_weight_offset};
    const uint32_t dts[3] = {pc->q_dtype, pc->k_dtype, pc->v_dtype};
    const uint32_t rows[3] = {pc->q_rows, pc->kv_rows, pc->kv_rows};
    vx_buf *outs[3] = {q, k, v};
    WRef w[3];
    static const char *names[3] = {"vx_qkv_matvec q", "vx_qkv_matvec k", "vx_qkv_matvec v"};
    for (int i = 0; i < 3; ++i) {
        VX_CHECK(check_mv_dtype(dts[i], names[i]));
        VX_CHECK(resolve_matrix(model, offs[i], dts[i], rows[i], pc->cols, &w[i], names[i]));
        VX_CHECK(need_buf(outs[i], (uint64_t)rows[i] * 4u, names[i]));
    }
    VX_CHECK(need_buf(x, (uint64_t)pc->cols * 4u, "vx_qkv_matvec x"));
    ProfSpan span(ctx, "baselm.qkv");
    // One combined row space q | k | v (qkv_matvec.comp:55-78); rows below
    // row_base are skipped exactly as the reference dispatch loop would.
    uint32_t seg_start = 0;
    for (int i = 0; i < 3; ++i) {
        const uint32_t seg_end = seg_start + rows[i];
        if (pc->row_base < seg_end) {
            MatvecLaunch l;
            l.w = w[i];
            l.xl = CF(x);
            l.rows = rows[i];
            l.cols = pc->cols;
            l.row_base = pc->row_base > seg_start ? pc->row_base - seg_start : 0u;
            l.alpha = 1.0f;
            l.epi = EPI_STORE;
            l.y = F(outs[i]);
            VX_CHECK(launch_matvec(ctx->stream, l));
        }
        seg_start = seg_end;
    }
    return VX_OK;
}

int vx_matvec_swiglu(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y, const vx_swiglu_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_matvec_swiglu"));
    VX_CHECK(check_mv_dtype(pc->dtype, "vx_matvec_swiglu"));
    SwigluLaunch l;
    VX_CHECK(resolve_matrix(model, pc->gate_weight_offset, pc->dtype, pc->rows, pc->cols, &l.g,
                            "vx_matvec_swiglu gate"));
    VX_CHECK(resolve_matrix(model, pc->up_weight_offset, pc->dtype, pc->rows, pc->cols, &l.u,
                            "vx_matvec_swiglu up"));
    VX_CHECK(need_buf(x, (uint64_t)pc->cols * 4u, "vx_matvec_swiglu x"));
    VX_CHECK(need_buf(y, (uint64_t)pc->rows * 4u, "vx_matvec_swiglu y"));
    ProfSpan span(ctx, "baselm.swiglu");
    l.x = CF(x);
    l.rows = pc->rows;
    l.cols = pc->cols;
    l.row_base = pc->row_base;
    l.y = F(y);
    return launch_swiglu(ctx->stream, l);
}

static int rope_common(vx_ctx *ctx, const vx_model *model, vx_buf *q, vx_buf *k, const vx_buf *position,
                       const vx_rope_push *pc, const char *what) {
    VX_CHECK(need_ctx(ctx, pc, what));
    const uint32_t half_dim = pc->head_dim / 2u;
    const uint32_t pairs = half_dim < 64u ? half_dim : 64u;
    const void *f = nullptr;
    VX_CHECK(resolve_vector(model, pc->factor_offset, VX_DTYPE_F32, pairs, &f, what));
    VX_CHECK(need_buf(q, (uint64_t)pc->q_heads * pc->head_dim * 4u, "rope q"));
    VX_CHECK(need_buf(k, (uint64_t)pc->kv_heads * pc->head_dim * 4u, "rope k"));
    if (position) VX_CHECK(need_buf(position, 4u, "rope position"));
    ProfSpan span(ctx, "baselm.rope");
    return launch_rope(ctx->stream, F(q), F(k), static_cast<const float *>(f), pc->position,
                       position ? CU(position) : nullptr, pc->q_heads, pc->kv_heads, pc->head_dim,
                       pc->rope_theta, pc->scaling_factor);
}

int vx_rope(vx_ctx *ctx, const vx_model *model, vx_buf *q, vx_buf *k, const vx_rope_push *pc) {
    return rope_common(ctx, model, q, k, nullptr, pc, "vx_rope");
}

int vx_rope_devpos(vx_ctx *ctx, const vx_model *model, vx_buf *q, vx_buf *k, const vx_buf *position,
                   const vx_rope_push *pc) {
    if (!position) return fail(VX_ERR_INVALID_ARG, "vx_rope_devpos: null position");
    return rope_common(ctx, model, q, k, position, pc, "vx_rope_devpos");
}

static int store_kv_common(vx_ctx *ctx, const vx_buf *k, const vx_buf *v, vx_buf *kc, vx_buf *vc,
                           const vx_buf *position, const vx_store_kv_push *pc, const char *what) {
    VX_CHECK(need_ctx(ctx, pc, what));
    if (pc->kv_dim % 2u) return fail(VX_ERR_SHAPE, "%s: kv_dim %u is odd", what, pc->kv_dim);
    const uint32_t words = pc->kv_dim / 2u < 128u ? pc->kv_dim / 2u : 128u;
    VX_CHECK(need_buf(k, (uint64_t)words * 8u, "store_kv k"));
    VX_CHECK(need_buf(v, (uint64_t)words * 8u, "store_kv v"));
    uint64_t need;
    if (position) {
        VX_CHECK(need_buf(position, 4u, "store_kv position"));
        need = cache_halves(pc->layer + 1u, pc->context, 0, pc->kv_dim) * 2u;
    } else {
        if (pc->position >= pc->context)
            return fail(VX_ERR_CONTEXT_FULL, "%s: position %u >= context %u", what, pc->position, pc->context);
        need = cache_halves(pc->layer, pc->context, pc->position + 1u, pc->kv_dim) * 2u;
    }
    VX_CHECK(need_buf(kc, need, "store_kv k_cache"));
    VX_CHECK(need_buf(vc, need, "store_kv v_cache"));
    ProfSpan span(ctx, "baselm.store_kv");
    return launch_store_kv(ctx->stream, CF(k), CF(v), static_cast<__half *>(kc->ptr),
                           static_cast<__half *>(vc->ptr), pc->layer, pc->position,
                           position ? CU(position) : nullptr, pc->context, pc->kv_dim);
}

int vx_store_kv(vx_ctx *ctx, const vx_buf *k, const vx_buf *v, vx_buf *k_cache, vx_buf *v_cache,
                const vx_store_kv_push *pc) {
    return store_kv_common(ctx, k, v, k_cache, v_cache, nullptr, pc, "vx_store_kv");
}

int vx_store_kv_devpos(vx_ctx *ctx, const vx_buf *k, const vx_buf *v, vx_buf *k_cache, vx_buf *v_cache,
                       const vx_buf *position, const vx_store_kv_push *pc) {
    if (!position) return fail(VX_ERR_INVALID_ARG, "vx_store_kv_devpos: null position");
    return store_kv_common(ctx, k, v, k_cache, v_cache, position, pc, "vx_store_kv_devpos");
}

static int attn_check(const vx_attention_push *pc, const vx_buf *position, const vx_buf *cache,
                      const char *what) {
    if (pc->head_dim == 0 || pc->head_dim > 128u || pc->q_per_kv == 0 || pc->kv_heads == 0)
        return fail(VX_ERR_UNSUPPORTED, "%s: head_dim 1..128 and nonzero head counts required", what);
    const uint32_t kv_dim = pc->kv_heads * pc->head_dim;
    uint64_t need;
    if (position) {
        VX_CHECK(need_buf(position, 4u, "attention position"));
        need = cache_halves(pc->layer + 1u, pc->context, 0, kv_dim) * 2u;
    } else {
        if (pc->position >= pc->context)
            return fail(VX_ERR_CONTEXT_FULL, "%s: position %u >= context %u", what, pc->position, pc->context);
        need = cache_halves(pc->layer, pc->context, pc->position + 1u, kv_dim) * 2u;
    }
    return need_buf(cache, need, "attention cache");
}

static int attn_scores_common(vx_ctx *ctx, const vx_buf *q, const vx_buf *kc, vx_buf *scores,
                              const vx_buf *position, const vx_attention_push *pc, const char *what) {
    VX_CHECK(need_ctx(ctx, pc, what));
    VX_CHECK(attn_check(pc, position, kc, what));
    const uint32_t q_heads = pc->q_per_kv * pc->kv_heads;
    VX_CHECK(need_buf(q, (uint64_t)q_heads * pc->head_dim * 4u, "attn_scores q"));
    VX_CHECK(need_buf(scores, (uint64_t)q_heads * pc->context * 4u, "attn_scores scores"));
    ProfSpan span(ctx, "baselm.attn_scores");
    return launch_attn_scores(ctx->stream, CF(q), static_cast<const __half *>(kc->ptr), F(scores), pc->layer,
                              pc->context, pc->position, position ? CU(position) : nullptr, pc->head_dim,
                              pc->q_per_kv, pc->kv_heads, q_heads);
}

int vx_attn_scores(vx_ctx *ctx, const vx_buf *q, const vx_buf *k_cache, vx_buf *scores,
                   const vx_attention_push *pc) {
    return attn_scores_common(ctx, q, k_cache, scores, nullptr, pc, "vx_attn_scores");
}

int vx_attn_scores_devpos(vx_ctx *ctx, const vx_buf *q, const vx_buf *k_cache, vx_buf *scores,
                          const vx_buf *position, const vx_attention_push *pc) {
    if (!position) return fail(VX_ERR_INVALID_ARG, "vx_attn_scores_devpos: null position");
    return attn_scores_common(ctx, q, k_cache, scores, position, pc, "vx_attn_scores_devpos");
}

static int softmax_common(vx_ctx *ctx, vx_buf *scores, uint32_t heads, const vx_buf *position,
                          const vx_softmax_push *pc, const char *what) {
    VX_CHECK(need_ctx(ctx, pc, what));
    if (position) {
        VX_CHECK(need_buf(position, 4u, "softmax position"));
    } else if (pc->position >= pc->context) {
        return fail(VX_ERR_CONTEXT_FULL, "%s: position %u >= context %u", what, pc->position, pc->context);
    }
    VX_CHECK(need_buf(scores, (uint64_t)heads * pc->context * 4u, "softmax scores"));
    ProfSpan span(ctx, "baselm.softmax");
    return launch_softmax(ctx->stream, F(scores), heads, pc->context, pc->position,
                          position ? CU(position) : nullptr);
}

int vx_softmax(vx_ctx *ctx, vx_buf *scores, uint32_t heads, const vx_softmax_push *pc) {
    return softmax_common(ctx, scores, heads, nullptr, pc, "vx_softmax");
}

int vx_softmax_devpos(vx_ctx *ctx, vx_buf *scores, uint32_t heads, const vx_buf *position,
                      const vx_softmax_push *pc) {
    if (!position) return fail(VX_ERR_INVALID_ARG, "vx_softmax_devpos: null position");
    return softmax_common(ctx, scores, heads, position, pc, "vx_softmax_devpos");
}

static int attn_values_common(vx_ctx *ctx, const vx_buf *scores, const vx_buf *vc, vx_buf *out,
                              const vx_buf *position, const vx_attention_push *pc, const char *what) {
    VX_CHECK(need_ctx(ctx, pc, what));
    VX_CHECK(attn_check(pc, position, vc, what));
    const uint32_t q_heads = pc->q_per_kv * pc->kv_heads;
    VX_CHECK(need_buf(scores, (uint64_t)q_heads * pc->context * 4u, "attn_values scores"));
    VX_CHECK(need_buf(out, (uint64_t)q_heads * pc->head_dim * 4u, "attn_values out"));
    ProfSpan span(ctx, "baselm.attn_values");
    return launch_attn_values(ctx->stream, CF(scores), static_cast<const __half *>(vc->ptr), F(out),
                              pc->layer, pc->context, pc->position, position ? CU(position) : nullptr,
                              pc->head_dim, pc->q_per_kv, pc->kv_heads, q_heads);
}

int vx_attn_values(vx_ctx *ctx, const vx_buf *scores, const vx_buf *v_cache, vx_buf *out,
                   const vx_attention_push *pc) {
    return attn_values_common(ctx, scores, v_cache, out, nullptr, pc, "vx_attn_values");
}

int vx_attn_values_devpos(vx_ctx *ctx, const vx_buf *scores, const vx_buf *v_cache, vx_buf *out,
                          const vx_buf *position, const vx_attention_push *pc) {
    if (!position) return fail(VX_ERR_INVALID_ARG, "vx_attn_values_devpos: null position");
    return attn_values_common(ctx, scores, v_cache, out, position, pc, "vx_attn_values_devpos");
}

int vx_linear_bias(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y,
                   const vx_linear_bias_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_linear_bias"));
    // linear_bias.comp:44-61: 0 = F32, 1 = F16, anything else = Q8_0.
    const uint32_t wd = pc->weight_dtype <= 1u ? pc->weight_dtype : VX_DTYPE_Q8_0;
    WRef w;
    VX_CHECK(resolve_matrix(model, pc->weight_offset, wd, pc->rows, pc->cols, &w, "vx_linear_bias"));
    const void *bias = nullptr;
    if (pc->bias_dtype <= 1u)
        VX_CHECK(resolve_vector(model, pc->bias_offset, pc->bias_dtype, pc->rows, &bias, "vx_linear_bias bias"));
    VX_CHECK(need_buf(x, (uint64_t)pc->cols * 4u, "vx_linear_bias x"));
    VX_CHECK(need_buf(y, (uint64_t)pc->rows * 4u, "vx_linear_bias y"));
    ProfSpan span(ctx, "acoustic.linear_bias");
    MatvecLaunch l;
    l.w = w;
    l.xl = CF(x);
    l.rows = pc->rows;
    l.cols = pc->cols;
    l.row_base = pc->row_base;
    l.alpha = pc->alpha;
    l.epi = EPI_BIAS;
    l.bias = bias;
    l.bias_dtype = pc->bias_dtype <= 1u ? pc->bias_dtype : 2u;
    l.y = F(y);
    return launch_matvec(ctx->stream, l);
}

int vx_fusion_linear(vx_ctx *ctx, const vx_model *model, const vx_buf *left, const vx_buf *right, vx_buf *y,
                     vx_buf *snapshot, const vx_fusion_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_fusion_linear"));
    const uint32_t cols = pc->left_cols + pc->right_cols;
    const uint32_t wd = pc->weight_dtype <= 1u ? pc->weight_dtype : VX_DTYPE_Q8_0;
    WRef w;
    VX_CHECK(resolve_matrix(model, pc->weight_offset, wd, pc->rows, cols, &w, "vx_fusion_linear"));
    // fusion_linear.comp:37-39: bias dtype 0 = F32, anything else = F16.
    const uint32_t bd = pc->bias_dtype == 0u ? VX_DTYPE_F32 : VX_DTYPE_F16;
    const void *bias = nullptr;
    VX_CHECK(resolve_vector(model, pc->bias_offset, bd, pc->rows, &bias, "vx_fusion_linear bias"));
    VX_CHECK(need_buf(left, (uint64_t)pc->left_cols * 4u, "vx_fusion_linear left"));
    if (pc->right_cols) VX_CHECK(need_buf(right, (uint64_t)pc->right_cols * 4u, "vx_fusion_linear right"));
    VX_CHECK(need_buf(y, (uint64_t)pc->rows * 4u, "vx_fusion_linear y"));
    VX_CHECK(need_buf(snapshot, (uint64_t)pc->rows * 4u, "vx_fusion_linear snapshot"));
    ProfSpan span(ctx, "acoustic.fusion_linear");
    MatvecLaunch l;
    l.w = w;
    l.xl = CF(left);
    l.xr = pc->right_cols ? CF(right) : nullptr;
    l.left_cols = pc->left_cols;
    l.rows = pc->rows;
    l.cols = cols;
    l.row_base = pc->row_base;
    l.epi = EPI_FUSION;
    l.bias = bias;
    l.bias_dtype = bd;
    l.y = F(y);
    l.y2 = F(snapshot);
    return launch_matvec(ctx->stream, l);
}

// ------------------------------------------------------------- fused ops
int vx_fused_qkv_rope_store(vx_ctx *ctx, const vx_model *model, const vx_buf *hidden, vx_buf *q, vx_buf *k,
                            vx_buf *v, vx_buf *k_cache, vx_buf *v_cache, const vx_buf *position,
                            const vx_fused_qkv_args *a) {
    VX_CHECK(need_ctx(ctx, a, "vx_fused_qkv_rope_store"));
    VX_CHECK(check_mv_dtype(a->dtype, "vx_fused_qkv_rope_store"));
    if (a->head_dim == 0 || a->q_rows % a->head_dim || a->kv_rows % a->head_dim)
        return fail(VX_ERR_SHAPE, "fused qkv: rows must be whole heads");
    QkvFusedLaunch l;
    VX_CHECK(resolve_matrix(model, a->q_weight_offset, a->dtype, a->q_rows, a->cols, &l.q, "fused qkv q"));
    VX_CHECK(resolve_matrix(model, a->k_weight_offset, a->dtype, a->kv_rows, a->cols, &l.k, "fused qkv k"));
    VX_CHECK(resolve_matrix(model, a->v_weight_offset, a->dtype, a->kv_rows, a->cols, &l.v, "fused qkv v"));
    const void *nw = nullptr, *fw = nullptr;
    VX_CHECK(resolve_vector(model, a->norm_offset, VX_DTYPE_F32, a->cols, &nw, "fused qkv norm"));
    VX_CHECK(resolve_vector(model, a->factor_offset, VX_DTYPE_F32, a->head_dim / 2u, &fw, "fused qkv factors"));
    VX_CHECK(need_buf(hidden, (uint64_t)a->cols * 4u, "fused qkv hidden"));
    VX_CHECK(need_buf(q, (uint64_t)a->q_rows * 4u, "fused qkv q out"));
    VX_CHECK(need_buf(k, (uint64_t)a->kv_rows * 4u, "fused qkv k out"));
    VX_CHECK(need_buf(v, (uint64_t)a->kv_rows * 4u, "fused qkv v out"));
    const uint64_t cache = cache_halves(a->layer + 1u, a->context, 0, a->kv_rows) * 2u;
    VX_CHECK(need_buf(k_cache, cache, "fused qkv k_cache"));
    VX_CHECK(need_buf(v_cache, cache, "fused qkv v_cache"));
    VX_CHECK(need_buf(position, 4u, "fused qkv position"));
    l.hidden = CF(hidden);
    l.norm = static_cast<const float *>(nw);
    l.eps = a->eps;
    l.q_rows = a->q_rows;
    l.kv_rows = a->kv_rows;
    l.cols = a->cols;
    l.head_dim = a->head_dim;
    l.factors = static_cast<const float *>(fw);
    l.theta = a->rope_theta;
    l.scaling = a->scaling_factor;
    l.layer = a->layer;
    l.context = a->context;
    l.qo = F(q);
    l.ko = F(k);
    l.vo = F(v);
    l.kc = static_cast<__half *>(k_cache->ptr);
    l.vc = static_cast<__half *>(v_cache->ptr);
    l.position = CU(position);
    ProfSpan span(ctx, "baselm.qkv_rope_store");
    return launch_qkv_fused(ctx->stream, l);
}

uint64_t vx_fused_attention_scratch_bytes(const vx_fused_attn_args *a) {
    if (!a) return 0;
    return attn_scratch_bytes(a->head_dim, a->q_heads, a->kv_heads, a->splits);
}

namespace {
// Checks and launch description shared by the two fused attention entry points;
// the caller supplies the partials buffer.
int fused_attention_launch(const vx_buf *q, const vx_buf *k_cache, const vx_buf *v_cache, vx_buf *out,
                           const vx_buf *position, const vx_fused_attn_args *a, AttnLaunch *l) {
    if (a->kv_heads == 0 || a->q_heads % a->kv_heads)
        return fail(VX_ERR_SHAPE, "fused attention: q_heads must be a multiple of kv_heads");
    const uint32_t kv_dim = a->kv_heads * a->head_dim;
    const uint64_t cache = cache_halves(a->layer + 1u, a->context, 0, kv_dim) * 2u;
    VX_CHECK(need_buf(q, (uint64_t)a->q_heads * a->head_dim * 4u, "fused attention q"));
    VX_CHECK(need_buf(k_cache, cache, "fused attention k_cache"));
    VX_CHECK(need_buf(v_cache, cache, "fused attention v_cache"));
    VX_CHECK(need_buf(out, (uint64_t)a->q_heads * a->head_dim * 4u, "fused attention out"));
    VX_CHECK(need_buf(position, 4u, "fused attention position"));
    l->q = CF(q);
    l->kc = static_cast<const __half *>(k_cache->ptr);
    l->vc = static_cast<const __half *>(v_cache->ptr);
    l->out = F(out);
    l->position = CU(position);
    l->layer = a->layer;
    l->context = a->context;
    l->head_dim = a->head_dim;
    l->q_heads = a->q_heads;
    l->kv_heads = a->kv_heads;
    l->splits = a->splits;
    return VX_OK;
}
}  // namespace

int vx_fused_attention(vx_ctx *ctx, const vx_buf *q, const vx_buf *k_cache, const vx_buf *v_cache, vx_buf *out,
                       vx_buf *scratch, const vx_buf *position, const vx_fused_attn_args *a) {
    VX_CHECK(need_ctx(ctx, a, "vx_fused_attention"));
    AttnLaunch l;
    VX_CHECK(fused_attention_launch(q, k_cache, v_cache, out, position, a, &l));
    VX_CHECK(need_buf(scratch, vx_fused_attention_scratch_bytes(a), "fused attention scratch"));
    l.partials = F(scratch);
    ProfSpan span(ctx, "baselm.attention");
    return launch_attn_decode(ctx->stream, l);
}

// The partials go to this GPU's no-allocation scratch (runtime.cpp), resolved at
// vx_init. Nothing here allocates, frees or clears memory: the split records are
// written by the partials kernel before the combine kernel reads them, so
// nothing in the scratch needs to start at zero.
int vx_fused_attention_noalloc(vx_ctx *ctx, const vx_buf *q, const vx_buf *k_cache, const vx_buf *v_cache,
                               vx_buf *out, const vx_buf *position, const vx_fused_attn_args *a) {
    VX_CHECK(need_ctx(ctx, a, "vx_fused_attention_noalloc"));
    AttnLaunch l;
    VX_CHECK(fused_attention_launch(q, k_cache, v_cache, out, position, a, &l));
    const uint64_t need = vx_fused_attention_scratch_bytes(a);
    if (need > VX_NOALLOC_SCRATCH_BYTES)
        return fail(VX_ERR_BOUNDS,
                    "vx_fused_attention_noalloc: %u heads x %u splits need %llu bytes of partials; the "
                    "no-allocation scratch holds %u",
                    a->q_heads, a->splits, (unsigned long long)need, (unsigned)VX_NOALLOC_SCRATCH_BYTES);
    if (!ctx->noalloc_scratch)
        return fail(VX_ERR_STATE, "vx_fused_attention_noalloc: the context has no scratch address");
    l.partials = static_cast<float *>(ctx->noalloc_scratch);
    return launch_attn_decode(ctx->stream, l);
}

int vx_fused_matvec_residual(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *hidden, vx_buf *branch,
                             const vx_fused_residual_args *a) {
    VX_CHECK(need_ctx(ctx, a, "vx_fused_matvec_residual"));
    VX_CHECK(check_mv_dtype(a->dtype, "vx_fused_matvec_residual"));
    MatvecLaunch l;
    VX_CHECK(resolve_matrix(model, a->weight_offset, a->dtype, a->rows, a->cols, &l.w, "fused residual"));
    VX_CHECK(need_buf(x, (uint64_t)a->cols * 4u, "fused residual x"));
    VX_CHECK(need_buf(hidden, (uint64_t)a->rows * 4u, "fused residual hidden"));
    if (branch) VX_CHECK(need_buf(branch, (uint64_t)a->rows * 4u, "fused residual branch"));
    l.xl = CF(x);
    l.rows = a->rows;
    l.cols = a->cols;
    l.epi = EPI_RESIDUAL;
    l.y = F(hidden);
    l.y2 = branch ? F(branch) : nullptr;
    l.scale = a->scale;
    ProfSpan span(ctx, "baselm.matvec_residual");
    return launch_matvec(ctx->stream, l);
}

int vx_fused_rms_swiglu(vx_ctx *ctx, const vx_model *model, const vx_buf *hidden, vx_buf *y,
                        const vx_fused_swiglu_args *a) {
    VX_CHECK(need_ctx(ctx, a, "vx_fused_rms_swiglu"));
    VX_CHECK(check_mv_dtype(a->dtype, "vx_fused_rms_swiglu"));
    SwigluLaunch l;
    VX_CHECK(resolve_matrix(model, a->gate_weight_offset, a->dtype, a->rows, a->cols, &l.g, "fused swiglu gate"));
    VX_CHECK(resolve_matrix(model, a->up_weight_offset, a->dtype, a->rows, a->cols, &l.u, "fused swiglu up"));
    const void *nw = nullptr;
    VX_CHECK(resolve_vector(model, a->norm_offset, VX_DTYPE_F32, a->cols, &nw, "fused swiglu norm"));
    VX_CHECK(need_buf(hidden, (uint64_t)a->cols * 4u, "fused swiglu hidden"));
    VX_CHECK(need_buf(y, (uint64_t)a->rows * 4u, "fused swiglu y"));
    l.x = CF(hidden);
    l.norm = static_cast<const float *>(nw);
    l.eps = a->eps;
    l.rows = a->rows;
    l.cols = a->cols;
    l.y = F(y);
    ProfSpan span(ctx, "baselm.rms_swiglu");
    return launch_swiglu(ctx->stream, l);
}

}  // extern "C"
