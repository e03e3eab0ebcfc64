// Token-batched per-op C ABI: one entry point per seq_* / dense_* pipeline of
// the reference (local.rs:183-212 push structs, local.rs:482-560 dispatches).
// Projections run on the MFMA GEMM (kernels_seq.hip) when the weight layout and
// strides allow it -- Q8_0 rows a multiple of 1024 wide (the repacked layout) or
// F16 rows a multiple of 128, 16-byte aligned input rows -- and on the generic
// one-wave-per-output kernel otherwise. Every entry point checks the push
// extents against the model's tensor table and the bound buffers first.
#include <algorithm>

#include "vx_internal.h"

using namespace vx;

namespace {

inline float *F(vx_buf *b) { return static_cast<float *>(b->ptr); }
inline const float *CF(const vx_buf *b) { return static_cast<const float *>(b->ptr); }

int need_ctx(vx_ctx *ctx, const void *pc, const char *what) {
    if (!ctx || !pc) return fail(VX_ERR_INVALID_ARG, "%s: null context or push struct", what);
    return VX_OK;
}

// Floats a [tokens][stride] region starting at `base` spans when each row reads `n`.
uint64_t span(uint32_t base, uint32_t tokens, uint32_t stride, uint32_t n) {
    return tokens ? (uint64_t)base + (uint64_t)(tokens - 1u) * stride + n : 0u;
}

// dtype of the tensor at `offset`, from the model's table.
int tensor_dtype(const vx_model *m, uint32_t offset, uint32_t *dtype, const char *what) {
    if (!m) return fail(VX_ERR_INVALID_ARG, "%s: null model", what);
    const vx_tensor_info *t;
    VX_CHECK(find_tensor_at(m, offset, &t));
    *dtype = t->ggml_type;
    return VX_OK;
}

bool gemm_ok(const WRef &w, uint32_t cols, uint32_t in_base, uint32_t in_stride, uint32_t tokens) {
    const bool layout = (w.wt == WT_Q8 && w.ptr && cols % 1024u == 0) || (w.wt == WT_F16 && cols % 128u == 0);
    const bool aligned = in_base % 4u == 0 && (tokens <= 1 || in_stride % 4u == 0);
    return layout && aligned;
}

// Compute units of the current device (cached per device).
uint32_t device_cus() {
    static uint32_t cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256u;
    if (!cus[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
        cus[dev] = (uint32_t)n;
    }
    return cus[dev];
}

// Split-K factor that brings a projection of `n_tiles` x ceil(T/64) tiles to
// about one workgroup per CU (k-stages of 128 columns; at most 8 splits).
uint32_t split_for(uint32_t n_tiles, uint32_t tokens, uint32_t K) {
    const uint32_t tiles = n_tiles * ((tokens + 63u) / 64u);
    const uint32_t cus = device_cus();
    if (tiles >= cus) return 1u;
    uint32_t ks = (cus + tiles - 1u) / tiles;
    ks = std::min<uint32_t>(ks, 8u);
    ks = std::min<uint32_t>(ks, std::max<uint32_t>(1u, K / 128u));
    return ks;
}

GemmSeg seg_of(const WRef &w, uint32_t rows, float *out, uint32_t ldo) {
    GemmSeg g;
    if (w.wt == WT_Q8) {
        g.qs = static_cast<const int8_t *>(w.ptr);
        g.d = w.d;
    } else {
        g.w = static_cast<const __half *>(w.ptr);
    }
    g.rows = rows;
    g.out = out;
    g.ldo = ldo;
    return g;
}

}  // namespace

namespace vx {

int enqueue_seq_linear(hipStream_t s, const WRef &w, const void *bias, uint32_t bias_dtype, uint32_t rows,
                       uint32_t cols, uint32_t tokens, const float *x, uint32_t in_base, uint32_t in_stride,
                       float *y, uint32_t out_base, uint32_t out_stride, float alpha, bool out_zeroed) {
    if (!tokens || !rows) return VX_OK;
    if (tokens == 1) {  // one token: the batch-1 matvec (matvec.comp / linear_bias.comp)
        MatvecLaunch m;
        m.w = w;
        m.xl = x + in_base;
        m.rows = rows;
        m.cols = cols;
        m.alpha = alpha;
        m.epi = bias ? EPI_BIAS : EPI_STORE;
        m.bias = bias;
        m.bias_dtype = bias_dtype;
        m.y = y + out_base;
        return launch_matvec(s, m);
    }
    if (gemm_ok(w, cols, in_base, in_stride, tokens)) {
        GemmArgs g;
        g.wk = w.wt;
        g.epi = GEPI_STORE;
        g.xf32 = 1;
        g.seg[0] = seg_of(w, rows, y + out_base, out_stride);
        g.seg[0].bias = bias;
        g.seg[0].bias_dtype = bias_dtype;
        g.K = cols;
        g.T = tokens;
        g.xf = x + in_base;
        g.ldx = in_stride;
        g.alpha = alpha;
        // Few tiles (a short token batch): split K and accumulate with atomics into a
        // zeroed output, when the output rows are dense so they can be cleared whole.
        if (out_stride == rows) g.ksplit = split_for((rows + 127u) / 128u, tokens, cols);
        if (g.ksplit > 1 && !out_zeroed)
            VX_CHECK(launch_fill_u32(s, reinterpret_cast<uint32_t *>(y + out_base), 0u, (uint64_t)tokens * rows));
        return launch_gemm(s, g);
    }
    SeqGenericArgs a;
    a.raw = w.raw;
    a.w_off = w.raw_offset;
    a.dtype = w.dtype;
    a.rows = rows;
    a.cols = cols;
    a.tokens = tokens;
    a.x = x;
    a.in_base = in_base;
    a.in_stride = in_stride;
    a.y = y;
    a.out_base = out_base;
    a.out_stride = out_stride;
    a.bias = bias;
    a.bias_dtype = bias_dtype;
    a.alpha = alpha;
    return launch_seq_linear_generic(s, a);
}

int enqueue_seq_qkv(hipStream_t s, const WRef w[3], const uint32_t rows[3], uint32_t cols, uint32_t tokens,
                    const float *x, uint32_t in_base, uint32_t in_stride, float *const out[3],
                    const uint32_t strides[3], bool out_zeroed) {
    if (!tokens) return VX_OK;
    bool all = tokens > 1 && w[0].wt == w[1].wt && w[0].wt == w[2].wt;
    for (int i = 0; i < 3; ++i) all = all && gemm_ok(w[i], cols, in_base, in_stride, tokens);
    if (all) {
        GemmArgs g;
        g.wk = w[0].wt;
        g.epi = GEPI_STORE;
        g.xf32 = 1;
        for (int i = 0; i < 3; ++i) g.seg[i] = seg_of(w[i], rows[i], out[i], strides[i]);
        g.nseg = 3;
        g.K = cols;
        g.T = tokens;
        g.xf = x + in_base;
        g.ldx = in_stride;
        if (strides[0] == rows[0] && strides[1] == rows[1] && strides[2] == rows[2]) {
            const uint32_t nt = (rows[0] + 127u) / 128u + (rows[1] + 127u) / 128u + (rows[2] + 127u) / 128u;
            g.ksplit = split_for(nt, tokens, cols);
        }
        if (g.ksplit > 1 && !out_zeroed)
            for (int i = 0; i < 3; ++i)
                VX_CHECK(launch_fill_u32(s, reinterpret_cast<uint32_t *>(out[i]), 0u, (uint64_t)tokens * rows[i]));
        return launch_gemm(s, g);
    }
    for (int i = 0; i < 3; ++i)
        VX_CHECK(enqueue_seq_linear(s, w[i], nullptr, 0, rows[i], cols, tokens, x, in_base, in_stride, out[i], 0,
                                    strides[i], 1.f, out_zeroed));
    return VX_OK;
}

int enqueue_seq_swiglu(hipStream_t s, const WRef &g, const WRef &u, uint32_t rows, uint32_t cols, uint32_t tokens,
                       const float *x, uint32_t in_base, uint32_t in_stride, float *y, uint32_t out_base,
                       uint32_t out_stride) {
    if (!tokens || !rows) return VX_OK;
    if (tokens == 1) {
        SwigluLaunch a;
        a.g = g;
        a.u = u;
        a.x = x + in_base;
        a.rows = rows;
        a.cols = cols;
        a.y = y + out_base;
        return launch_swiglu(s, a);
    }
    if (g.wt == u.wt && gemm_ok(g, cols, in_base, in_stride, tokens) && gemm_ok(u, cols, in_base, in_stride, tokens)) {
        GemmArgs a;
        a.wk = g.wt;
        a.epi = GEPI_SWIGLU;
        a.xf32 = 1;
        a.seg[0] = seg_of(g, rows, y + out_base, out_stride);
        a.seg[1] = seg_of(u, rows, nullptr, 0);
        a.nseg = 2;
        a.K = cols;
        a.T = tokens;
        a.xf = x + in_base;
        a.ldx = in_stride;
        return launch_gemm(s, a);
    }
    SeqGenericArgs a;
    a.raw = g.raw;
    a.w_off = g.raw_offset;
    a.w2_off = u.raw_offset;
    a.dtype = g.dtype;
    a.rows = rows;
    a.cols = cols;
    a.tokens = tokens;
    a.x = x;
    a.in_base = in_base;
    a.in_stride = in_stride;
    a.y = y;
    a.out_base = out_base;
    a.out_stride = out_stride;
    a.swiglu = 1;
    return launch_seq_linear_generic(s, a);
}

}  // namespace vx

extern "C" {

int vx_seq_linear_bias(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y,
                       const vx_seq_linear_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_seq_linear_bias"));
    WRef w;
    VX_CHECK(resolve_matrix(model, pc->weight_offset, pc->weight_dtype, pc->rows, pc->cols, &w,
                            "vx_seq_linear_bias weight"));
    const void *bias = nullptr;
    if (pc->has_bias) {
        if (pc->bias_dtype != VX_DTYPE_F32 && pc->bias_dtype != VX_DTYPE_F16)
            return fail(VX_ERR_UNSUPPORTED, "vx_seq_linear_bias: bias dtype %u", pc->bias_dtype);
        VX_CHECK(resolve_vector(model, pc->bias_offset, pc->bias_dtype, pc->rows, &bias, "vx_seq_linear_bias bias"));
    }
    VX_CHECK(need_buf(x, span(pc->input_base, pc->tokens, pc->input_stride, pc->cols) * 4u, "vx_seq_linear_bias x"));
    VX_CHECK(need_buf(y, span(pc->output_base, pc->tokens, pc->output_stride, pc->rows) * 4u, "vx_seq_linear_bias y"));
    ProfSpan sp(ctx, "local.seq_linear");
    return enqueue_seq_linear(ctx->stream, w, pc->has_bias ? bias : nullptr, pc->bias_dtype, pc->rows, pc->cols,
                              pc->tokens, CF(x), pc->input_base, pc->input_stride, F(y), pc->output_base,
                              pc->output_stride, pc->alpha);
}

int vx_seq_qkv(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *q, vx_buf *k, vx_buf *v,
               const vx_seq_qkv_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_seq_qkv"));
    const uint32_t offs[3] = {pc->q_weight_offset, pc->k_weight_offset, pc->v_weight_offset};
    const uint32_t rows[3] = {pc->q_rows, pc->kv_rows, pc->kv_rows};
    const uint32_t strides[3] = {pc->q_stride, pc->kv_stride, pc->kv_stride};
    vx_buf *outs[3] = {q, k, v};
    const char *names[3] = {"vx_seq_qkv q", "vx_seq_qkv k", "vx_seq_qkv v"};
    WRef w[3];
    for (int i = 0; i < 3; ++i) {
        uint32_t dt;
        VX_CHECK(tensor_dtype(model, offs[i], &dt, names[i]));
        if (dt != VX_DTYPE_F16 && dt != VX_DTYPE_Q8_0)
            return fail(VX_ERR_UNSUPPORTED, "%s: seq_qkv takes F16 or Q8_0 weights, got %u", names[i], dt);
        VX_CHECK(resolve_matrix(model, offs[i], dt, rows[i], pc->cols, &w[i], names[i]));
        VX_CHECK(need_buf(outs[i], span(0, pc->tokens, strides[i], rows[i]) * 4u, names[i]));
    }
    VX_CHECK(need_buf(x, span(pc->input_base, pc->tokens, pc->input_stride, pc->cols) * 4u, "vx_seq_qkv x"));
    ProfSpan sp(ctx, "local.seq_qkv");
    float *const o[3] = {F(q), F(k), F(v)};
    return enqueue_seq_qkv(ctx->stream, w, rows, pc->cols, pc->tokens, CF(x), pc->input_base, pc->input_stride, o,
                           strides);
}

int vx_seq_swiglu(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y, const vx_seq_swiglu_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_seq_swiglu"));
    uint32_t dg, du;
    VX_CHECK(tensor_dtype(model, pc->gate_weight_offset, &dg, "vx_seq_swiglu gate"));
    VX_CHECK(tensor_dtype(model, pc->up_weight_offset, &du, "vx_seq_swiglu up"));
    if (dg != du || (dg != VX_DTYPE_F16 && dg != VX_DTYPE_Q8_0))
        return fail(VX_ERR_UNSUPPORTED, "vx_seq_swiglu: gate/up must share an F16 or Q8_0 type (%u, %u)", dg, du);
    WRef wg, wu;
    VX_CHECK(resolve_matrix(model, pc->gate_weight_offset, dg, pc->rows, pc->cols, &wg, "vx_seq_swiglu gate"));
    VX_CHECK(resolve_matrix(model, pc->up_weight_offset, du, pc->rows, pc->cols, &wu, "vx_seq_swiglu up"));
    VX_CHECK(need_buf(x, span(pc->input_base, pc->tokens, pc->input_stride, pc->cols) * 4u, "vx_seq_swiglu x"));
    VX_CHECK(need_buf(y, span(pc->output_base, pc->tokens, pc->output_stride, pc->rows) * 4u, "vx_seq_swiglu y"));
    ProfSpan sp(ctx, "local.seq_swiglu");
    return enqueue_seq_swiglu(ctx->stream, wg, wu, pc->rows, pc->cols, pc->tokens, CF(x), pc->input_base,
                              pc->input_stride, F(y), pc->output_base, pc->output_stride);
}

int vx_seq_silu_mul(vx_ctx *ctx, vx_buf *gate, const vx_buf *up, uint32_t n) {
    if (!ctx) return fail(VX_ERR_INVALID_ARG, "vx_seq_silu_mul: null context");
    VX_CHECK(need_buf(gate, (uint64_t)n * 4u, "vx_seq_silu_mul gate"));
    VX_CHECK(need_buf(up, (uint64_t)n * 4u, "vx_seq_silu_mul up"));
    ProfSpan sp(ctx, "local.seq_silu_mul");
    return launch_silu_mul(ctx->stream, F(gate), CF(up), n);
}

int vx_seq_rmsnorm(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y, const vx_seq_rms_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_seq_rmsnorm"));
    const void *w = nullptr;
    VX_CHECK(resolve_vector(model, pc->weight_offset, VX_DTYPE_F32, pc->n, &w, "vx_seq_rmsnorm weight"));
    VX_CHECK(need_buf(x, span(pc->input_base, pc->tokens, pc->input_stride, pc->n) * 4u, "vx_seq_rmsnorm x"));
    VX_CHECK(need_buf(y, span(pc->output_base, pc->tokens, pc->output_stride, pc->n) * 4u, "vx_seq_rmsnorm y"));
    ProfSpan sp(ctx, "local.seq_rmsnorm");
    SeqNormArgs a;
    a.h = const_cast<float *>(CF(x)) + pc->input_base;  // read only: no branch
    a.ldh = pc->input_stride;
    a.w = static_cast<const float *>(w);
    a.n = pc->n;
    a.eps = pc->eps;
    a.y = F(y) + pc->output_base;
    a.ldy = pc->output_stride;
    return launch_seq_rmsnorm(ctx->stream, a, pc->tokens);
}

int vx_seq_residual_rmsnorm(vx_ctx *ctx, const vx_model *model, vx_buf *hidden, const vx_buf *branch, vx_buf *y,
                            const vx_seq_residual_rms_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_seq_residual_rmsnorm"));
    const void *w = nullptr;
    VX_CHECK(resolve_vector(model, pc->weight_offset, VX_DTYPE_F32, pc->n, &w, "vx_seq_residual_rmsnorm weight"));
    VX_CHECK(need_buf(hidden, span(pc->hidden_base, pc->tokens, pc->hidden_stride, pc->n) * 4u,
                      "vx_seq_residual_rmsnorm hidden"));
    VX_CHECK(need_buf(branch, span(pc->branch_base, pc->tokens, pc->branch_stride, pc->n) * 4u,
                      "vx_seq_residual_rmsnorm branch"));
    VX_CHECK(need_buf(y, span(pc->output_base, pc->tokens, pc->output_stride, pc->n) * 4u,
                      "vx_seq_residual_rmsnorm y"));
    ProfSpan sp(ctx, "local.seq_residual_rmsnorm");
    SeqNormArgs a;
    a.h = F(hidden) + pc->hidden_base;
    a.ldh = pc->hidden_stride;
    a.branch = CF(branch) + pc->branch_base;
    a.ldb = pc->branch_stride;
    a.scale = pc->scale;
    a.w = static_cast<const float *>(w);
    a.n = pc->n;
    a.eps = pc->eps;
    a.y = F(y) + pc->output_base;
    a.ldy = pc->output_stride;
    return launch_seq_rmsnorm(ctx->stream, a, pc->tokens);
}

int vx_seq_rope_at(vx_ctx *ctx, const vx_model *model, vx_buf *q, vx_buf *k, uint32_t position_base,
                   const vx_seq_rope_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_seq_rope"));
    if (pc->head_dim == 0 || (pc->head_dim & 1u) || pc->head_dim > 128u)
        return fail(VX_ERR_UNSUPPORTED, "vx_seq_rope: head_dim %u (even, <= 128)", pc->head_dim);
    const void *f = nullptr;
    VX_CHECK(resolve_vector(model, pc->factor_offset, VX_DTYPE_F32, pc->head_dim / 2u, &f, "vx_seq_rope factors"));
    VX_CHECK(need_buf(q, span(0, pc->tokens, pc->q_stride, pc->q_heads * pc->head_dim) * 4u, "vx_seq_rope q"));
    VX_CHECK(need_buf(k, span(0, pc->tokens, pc->k_stride, pc->kv_heads * pc->head_dim) * 4u, "vx_seq_rope k"));
    ProfSpan sp(ctx, "local.seq_rope");
    SeqRopeArgs a;
    a.q = F(q);
    a.k = F(k);
    a.ldq = pc->q_stride;
    a.ldk = pc->k_stride;
    a.factors = static_cast<const float *>(f);
    a.pos_base = position_base;
    a.q_heads = pc->q_heads;
    a.kv_heads = pc->kv_heads;
    a.head_dim = pc->head_dim;
    a.theta = pc->rope_theta;
    a.scaling = pc->scaling_factor;
    return launch_seq_rope_store(ctx->stream, a, pc->tokens);
}

int vx_seq_rope(vx_ctx *ctx, const vx_model *model, vx_buf *q, vx_buf *k, const vx_seq_rope_push *pc) {
    return vx_seq_rope_at(ctx, model, q, k, 0u, pc);
}

int vx_dense_attn_scores(vx_ctx *ctx, const vx_buf *q, const vx_buf *k, vx_buf *scores,
                         const vx_dense_scores_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_dense_attn_scores"));
    if (pc->kv_heads == 0 || pc->q_heads % pc->kv_heads)
        return fail(VX_ERR_SHAPE, "vx_dense_attn_scores: q_heads %u not a multiple of kv_heads %u", pc->q_heads,
                    pc->kv_heads);
    if (pc->tokens > pc->score_stride) return fail(VX_ERR_SHAPE, "vx_dense_attn_scores: tokens > score_stride");
    VX_CHECK(need_buf(q, span(0, pc->tokens, pc->q_stride, pc->q_heads * pc->head_dim) * 4u, "dense scores q"));
    VX_CHECK(need_buf(k, span(0, pc->tokens, pc->k_stride, pc->kv_heads * pc->head_dim) * 4u, "dense scores k"));
    VX_CHECK(need_buf(scores, (uint64_t)pc->tokens * pc->q_heads * pc->score_stride * 4u, "dense scores s"));
    ProfSpan sp(ctx, "local.attn_scores");
    DenseAttnArgs a;
    a.q = CF(q);
    a.k = CF(k);
    a.s = F(scores);
    a.tokens = pc->tokens;
    a.q_heads = pc->q_heads;
    a.kv_heads = pc->kv_heads;
    a.head_dim = pc->head_dim;
    a.q_stride = pc->q_stride;
    a.k_stride = pc->k_stride;
    a.score_stride = pc->score_stride;
    return launch_dense_attn(ctx->stream, a, 0);
}

int vx_dense_softmax(vx_ctx *ctx, vx_buf *scores, const vx_dense_softmax_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_dense_softmax"));
    if (pc->tokens > pc->score_stride) return fail(VX_ERR_SHAPE, "vx_dense_softmax: tokens > score_stride");
    VX_CHECK(need_buf(scores, (uint64_t)pc->tokens * pc->q_heads * pc->score_stride * 4u, "dense softmax s"));
    ProfSpan sp(ctx, "local.softmax");
    DenseAttnArgs a;
    a.s = F(scores);
    a.tokens = pc->tokens;
    a.q_heads = pc->q_heads;
    a.kv_heads = 1;
    a.score_stride = pc->score_stride;
    return launch_dense_attn(ctx->stream, a, 1);
}

int vx_dense_attn_values(vx_ctx *ctx, const vx_buf *scores, const vx_buf *v, vx_buf *out,
                         const vx_dense_values_push *pc) {
    VX_CHECK(need_ctx(ctx, pc, "vx_dense_attn_values"));
    if (pc->kv_heads == 0 || pc->q_heads % pc->kv_heads)
        return fail(VX_ERR_SHAPE, "vx_dense_attn_values: q_heads %u not a multiple of kv_heads %u", pc->q_heads,
                    pc->kv_heads);
    if (pc->tokens > pc->score_stride) return fail(VX_ERR_SHAPE, "vx_dense_attn_values: tokens > score_stride");
    VX_CHECK(need_buf(scores, (uint64_t)pc->tokens * pc->q_heads * pc->score_stride * 4u, "dense values s"));
    VX_CHECK(need_buf(v, span(0, pc->tokens, pc->v_stride, pc->kv_heads * pc->head_dim) * 4u, "dense values v"));
    VX_CHECK(need_buf(out, span(0, pc->tokens, pc->out_stride, pc->q_heads * pc->head_dim) * 4u, "dense values out"));
    ProfSpan sp(ctx, "local.attn_values");
    DenseAttnArgs a;
    a.s = F(const_cast<vx_buf *>(scores));
    a.v = CF(v);
    a.out = F(out);
    a.tokens = pc->tokens;
    a.q_heads = pc->q_heads;
    a.kv_heads = pc->kv_heads;
    a.head_dim = pc->head_dim;
    a.v_stride = pc->v_stride;
    a.out_stride = pc->out_stride;
    a.score_stride = pc->score_stride;
    return launch_dense_attn(ctx->stream, a, 2);
}

}  // extern "C"
