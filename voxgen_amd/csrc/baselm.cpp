// BaseLM engine: the host side of BaseLmEngine (baselm.rs:423-890) over HIP.
//
// Decode step in the default (graph) mode, all reading the decode position and
// the token id from device memory so one captured hipGraph is replayed per token:
//   embedding gather                                  embedding.comp
//   per layer:
//     k_qkv_fused      rmsnorm(h)*attn_norm -> Q/K/V -> RoPE -> f16 KV store
//     k_attn_decode    split-context single-query attention + combine
//     k_matvec (resid) h += Wo . attn
//     k_swiglu (norm)  gate = silu(Wg . n) * (Wu . n), n = rmsnorm(h)*ffn_norm
//     k_matvec (resid) h += Wdown . gate
//   k_rmsnorm          norm = rmsnorm(h)*output_norm, then position += 1
//   [LM head matvec]   logits = logit_scale * Wout . norm
// This is record_transformer's op order (baselm.rs:892-1052) with each
// residual_rmsnorm split between the producing matvec (residual add) and the
// consuming matvec (normalisation), which removes 2 launches per layer.
// VX_EXEC_REFERENCE instead issues the reference's 11 per-op dispatches.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>

#include "vx_internal.h"

using namespace vx;

namespace {

using Layer = StackLayer;

float effective_scale(float v) { return v == 0.0f ? 1.0f : v; }  // baselm.rs:1262-1264

}  // namespace

struct vx_baselm {
    vx_ctx *ctx = nullptr;
    const vx_model *model = nullptr;
    vx_baselm_config cfg{};
    vx_baselm_options opt{};
    vx_buf *hidden = nullptr, *norm = nullptr, *q = nullptr, *k = nullptr, *v = nullptr;
    vx_buf *attention = nullptr, *gate = nullptr, *branch = nullptr, *logits = nullptr;
    vx_buf *scores = nullptr, *kv_k = nullptr, *kv_v = nullptr, *position = nullptr;
    vx_buf *tokens = nullptr, *attn_scratch = nullptr, *rope_table = nullptr;
    std::vector<Layer> layers;
    uint32_t embd_offset = 0, embd_dtype = 1;
    WRef output;
    const float *output_norm = nullptr, *rope_factors = nullptr;
    float residual_scale = 1.f, embedding_alpha = 1.f, logit_alpha = 1.f, rope_scaling = 1.f;
    uint32_t splits = 8;
    bool fold_attn_merge = false;  // attention merge folded into the attn_out matvec
    // Attention tiers by the step's key count (attn_tier): tier 0 is the short
    // contexts' k_attn_chunk over `splits` slices; tiers 1 and 2 stream
    // tier_splits[t] slices of many keys through k_attn_rows (0: tier unused).
    // attn_out merges the slices of every tier.
    uint32_t tier_splits[3] = {0, 0, 0};
    uint32_t pos = 0;
    vx_graph *graphs[2][2][3] = {};   // [embedding input][LM head][attention tier]
    // Token-batched prefill workspace (allocated on first use): residual stream,
    // hi/lo f16 planes of the GEMM inputs, q/k/v, roped q planes, token ids.
    StackWork pf;
    vx_buf *pf_tok = nullptr;
    // Q8_0 weights in the prefill-GEMM layout (built by the first batched prefill
    // that can use them; empty when some projection is not Q8_0).
    std::vector<StackPrefillWeights> pw;
    vx_buf *pw_arena = nullptr;
    bool pw_tried = false;
};

namespace {

int find(const vx_model *m, const std::string &name, const vx_tensor_info **out) {
    auto it = m->by_name.find(name);
    if (it == m->by_name.end())
        return fail(VX_ERR_NOT_FOUND, "required GGUF tensor \"%s\" is missing", name.c_str());
    *out = &m->tensors[it->second];
    return VX_OK;
}

int require_dims(const vx_tensor_info *t, std::initializer_list<uint64_t> dims) {
    bool ok = t->n_dims == dims.size();
    uint32_t i = 0;
    for (uint64_t d : dims) {
        if (!ok) break;
        ok = t->dims[i++] == d;
    }
    if (!ok) {  // require_dims baselm.rs:264-269
        std::string want, got;
        for (uint64_t d : dims) want += std::to_string(d) + ",";
        for (uint32_t j = 0; j < t->n_dims; ++j) got += std::to_string(t->dims[j]) + ",";
        return fail(VX_ERR_SHAPE, "tensor %s has dimensions [%s], expected [%s]", t->name, got.c_str(),
                    want.c_str());
    }
    return VX_OK;
}

int require_f32(const vx_tensor_info *t) {
    if (t->ggml_type != VX_DTYPE_F32)
        return fail(VX_ERR_SHAPE, "tensor %s is type %u, expected F32", t->name, t->ggml_type);
    return VX_OK;
}

int require_matrix_type(const vx_tensor_info *t) {  // baselm.rs:276-284
    if (t->ggml_type != VX_DTYPE_F16 && t->ggml_type != VX_DTYPE_Q8_0)
        return fail(VX_ERR_SHAPE, "matrix %s uses unsupported type %u", t->name, t->ggml_type);
    if (t->ggml_type == VX_DTYPE_Q8_0 && t->dims[0] % 32u)
        return fail(VX_ERR_SHAPE, "Q8_0 matrix %s has row width %llu, not divisible by 32", t->name,
                    (unsigned long long)t->dims[0]);
    return VX_OK;
}

int matrix(const vx_model *m, const std::string &name, uint64_t cols, uint64_t rows, WRef *out) {
    const vx_tensor_info *t;
    VX_CHECK(find(m, name, &t));
    VX_CHECK(require_dims(t, {cols, rows}));
    VX_CHECK(require_matrix_type(t));
    return resolve_matrix(m, (uint32_t)t->offset, t->ggml_type, (uint32_t)rows, (uint32_t)cols, out,
                          name.c_str());
}

int vec_f32(const vx_model *m, const std::string &name, uint64_t n, const float **out, uint32_t *off = nullptr) {
    const vx_tensor_info *t;
    VX_CHECK(find(m, name, &t));
    VX_CHECK(require_dims(t, {n}));
    VX_CHECK(require_f32(t));
    const void *p;
    VX_CHECK(resolve_vector(m, (uint32_t)t->offset, VX_DTYPE_F32, (uint32_t)n, &p, name.c_str()));
    *out = static_cast<const float *>(p);
    if (off) *off = (uint32_t)t->offset;
    return VX_OK;
}

int validate_config(const vx_baselm_config &c, bool strict) {
    if (c.active_context_length == 0 || c.active_context_length > c.context_length)
        return fail(VX_ERR_INVALID_ARG, "--max-context must be in 1..=%u, got %u", c.context_length,
                    c.active_context_length);
    if (strict && (c.embedding_length != 2048 || c.block_count != 28 || c.feed_forward_length != 6144 ||
                   c.head_count != 16 || c.head_count_kv != 2 || c.head_dim != 128 ||
                   c.rope_dimension_count != 128))  // baselm.rs:102-113
        return fail(VX_ERR_UNSUPPORTED,
                    "unsupported MiniCPM4 BaseLM geometry: embd=%u, layers=%u, ffn=%u, heads=%u, "
                    "kv_heads=%u, head_dim=%u, rope_dim=%u",
                    c.embedding_length, c.block_count, c.feed_forward_length, c.head_count,
                    c.head_count_kv, c.head_dim, c.rope_dimension_count);
    if (c.head_count_kv == 0 || c.head_count % c.head_count_kv)
        return fail(VX_ERR_SHAPE, "head_count %u is not divisible by head_count_kv %u", c.head_count,
                    c.head_count_kv);
    if (c.rope_dimension_count != c.head_dim)
        return fail(VX_ERR_UNSUPPORTED, "partial RoPE is not implemented: rope_dimension_count=%u, head_dim=%u",
                    c.rope_dimension_count, c.head_dim);
    if (c.kv_dim != c.head_count_kv * c.head_dim)
        return fail(VX_ERR_SHAPE, "kv_dim %u != head_count_kv*head_dim", c.kv_dim);
    if (c.head_count * c.head_dim != c.embedding_length)
        return fail(VX_ERR_SHAPE, "head_count*head_dim must equal embedding_length");
    if (!c.rope_longrope)  // baselm.rs:902-912
        return fail(VX_ERR_UNSUPPORTED, "MiniCPM4 BaseLM without LongRoPE factors is not enabled");
    if (c.block_count == 0) return fail(VX_ERR_SHAPE, "block_count is zero");
    return VX_OK;
}

int alloc(vx_ctx *ctx, uint64_t bytes, vx_buf **out) { return vx_alloc(ctx, bytes, out); }

void free_all(vx_baselm *e) {
    for (auto &plane : e->graphs)
        for (auto &row : plane)
            for (auto &g : row)
                if (g) {
                    vx_graph_free(e->ctx, g);
                    g = nullptr;
                }
    vx_buf **bufs[] = {&e->hidden, &e->norm,   &e->q,      &e->k,        &e->v,
                       &e->attention, &e->gate, &e->branch, &e->logits, &e->scores,
                       &e->kv_k, &e->kv_v,     &e->position, &e->tokens, &e->attn_scratch, &e->rope_table,
                       &e->pf_tok, &e->pw_arena};
    for (vx_buf **b : bufs) {
        vx_free(e->ctx, *b);
        *b = nullptr;
    }
    prefill_stack_free(e->ctx, &e->pf);
    e->pw.clear();
    e->pw_tried = false;
}

inline float *F(vx_buf *b) { return static_cast<float *>(b->ptr); }
inline uint32_t *U(vx_buf *b) { return static_cast<uint32_t *>(b->ptr); }
inline __half *H(vx_buf *b) { return static_cast<__half *>(b->ptr); }

// Kernels of one layer of the fused decode step.
enum LayerKernel : uint32_t { LK_QKV = 0, LK_ATTENTION = 1, LK_ATTN_OUT = 2, LK_SWIGLU = 3, LK_DOWN = 4, LK_COUNT = 5 };
const char *const kLayerKernelNames[LK_COUNT] = {"baselm.qkv", "baselm.attention", "baselm.attn_out",
                                                 "baselm.swiglu", "baselm.down"};

// Attention tier of a step over `pos + 1` keys. Up to kTier1FromKeys keys the
// short contexts' kShortSplits slices: k_attn_chunk while the slices are
// position-independent (context <= 64 * splits: their keys are fetched before the
// position is known), else k_attn_rows with four waves; then kShortSplits slices
// of k_attn_rows with eight waves; from kTier2FromKeys keys kMaxFoldedSplits
// slices of four waves. With the first stream kernel (64-byte row pieces, expf),
// measured on MI355X per layer, attention + attn_out at 1041 / 2065 / 4113 / 8017
// keys: tier 0 11.5 / 15.3 / 23.1 / 36.8 us, tier 1 10.3 / 11.8 / 14.3 / 19.3 us,
// tier 2 10.9 / 11.9 / 13.6 / 16.1 us. k_attn_rows (whole-row loads, exp2, 32-bit
// row offsets: 892 against 1221 VALU instructions per kernel) took the attention at
// 2065 / 4113 / 8017 keys from 7.9 / 7.7 / 10.0 to 6.3 / 6.5 / 8.8 us, and at 513
// keys of an 8192 context (tier 0, position-dependent slices) from 5.4 (k_attn_chunk)
// to 4.3 us; wave counts 4 or 8 in tiers 1 and 2 measured alike.
constexpr uint32_t kTier1FromKeys = 1025;
constexpr uint32_t kTier2FromKeys = 2561;
uint32_t attn_tier(const vx_baselm *e, uint32_t pos) {
    const uint32_t n = pos + 1u;
    if (n >= kTier2FromKeys && e->tier_splits[2]) return 2;
    if (n >= kTier1FromKeys && e->tier_splits[1]) return 1;
    return 0;
}

// Enqueue one kernel of layer l (all read the decode position from device memory).
int enqueue_layer_kernel(vx_baselm *e, uint32_t which, uint32_t l, uint32_t tier) {
    hipStream_t s = e->ctx->stream;
    const vx_baselm_config &c = e->cfg;
    const Layer &L = e->layers[l];
    AttnLaunch at;
    at.q = F(e->q);
    at.kc = H(e->kv_k);
    at.vc = H(e->kv_v);
    at.out = F(e->attention);
    at.partials = F(e->attn_scratch);
    at.position = U(e->position);
    at.layer = l;
    at.context = c.active_context_length;
    at.head_dim = c.head_dim;
    at.q_heads = c.head_count;
    at.kv_heads = c.head_count_kv;
    at.splits = tier ? e->tier_splits[tier] : e->splits;
    const bool fold = e->fold_attn_merge;
    switch (which) {
        case LK_QKV: {
            QkvFusedLaunch a;
            a.rope_cs = reinterpret_cast<const float2 *>(e->rope_table->ptr);
            a.q = L.q;
            a.k = L.k;
            a.v = L.v;
            a.hidden = F(e->hidden);
            a.norm = L.attn_norm;
            a.eps = c.rms_epsilon;
            a.q_rows = c.embedding_length;
            a.kv_rows = c.kv_dim;
            a.cols = c.embedding_length;
            a.head_dim = c.head_dim;
            a.factors = e->rope_factors;
            a.theta = c.rope_theta;
            a.scaling = e->rope_scaling;
            a.layer = l;
            a.context = c.active_context_length;
            a.qo = F(e->q);
            a.ko = F(e->k);
            a.vo = F(e->v);
            a.kc = H(e->kv_k);
            a.vc = H(e->kv_v);
            a.position = U(e->position);
            return launch_qkv_fused(s, a);
        }
        case LK_ATTENTION:
            // Partials only when attn_out merges them; else partials + merge.
            if (tier) return launch_attn_stream(s, at, tier == 1 ? 8u : 4u);   // tiers 1 and 2 imply the fold
            // k_attn_chunk while its slices are position-independent (their rows are
            // requested before the position); otherwise the whole-row stream kernel.
            if (fold && attn_fixed_chunk(at.context, at.splits) > kAttnFixedChunk)
                return launch_attn_stream(s, at, 4u);
            return fold ? launch_attn_partials(s, at) : launch_attn_decode(s, at);
        case LK_ATTN_OUT: {
            MatvecLaunch ao;
            ao.w = L.o;
            ao.xl = F(e->attention);
            ao.rows = c.embedding_length;
            ao.cols = c.embedding_length;
            ao.epi = EPI_RESIDUAL;
            ao.y = F(e->hidden);
            ao.scale = e->residual_scale;
            if (!fold) return launch_matvec(s, ao);
            AttnOutLaunch a;
            a.mv = ao;
            a.partials = at.partials;
            a.attn_out = F(e->attention);
            a.position = at.position;
            a.context = at.context;
            a.splits = at.splits;
            a.q_heads = at.q_heads;
            a.head_dim = at.head_dim;
            return launch_attn_out(s, a);
        }
        case LK_SWIGLU: {
            SwigluLaunch a;
            a.g = L.gate;
            a.u = L.up;
            a.x = F(e->hidden);
            a.norm = L.ffn_norm;
            a.eps = c.rms_epsilon;
            a.rows = c.feed_forward_length;
            a.cols = c.embedding_length;
            a.y = F(e->gate);
            return launch_swiglu(s, a);
        }
        case LK_DOWN: {
            MatvecLaunch a;
            a.w = L.down;
            a.xl = F(e->gate);
            a.rows = c.embedding_length;
            a.cols = c.feed_forward_length;
            a.epi = EPI_RESIDUAL;
            a.y = F(e->hidden);
            a.scale = e->residual_scale;
            return launch_matvec(s, a);
        }
        default: return fail(VX_ERR_INVALID_ARG, "unknown layer kernel %u", which);
    }
}

// LM head on the final normalised hidden state (baselm.rs:1040-1050).
int enqueue_logits(vx_baselm *e) {
    ProfSpan sp(e->ctx, "baselm.logits");
    const vx_baselm_config &c = e->cfg;
    MatvecLaunch a;
    a.w = e->output;
    a.xl = F(e->norm);
    a.rows = c.vocab_size;
    a.cols = c.embedding_length;
    a.alpha = e->logit_alpha;
    a.epi = EPI_STORE;
    a.y = F(e->logits);
    return launch_matvec(e->ctx->stream, a);
}

// The fused decode step, enqueued on the context stream.
int enqueue_fused(vx_baselm *e, bool with_embedding, bool logits, uint32_t tier) {
    vx_ctx *ctx = e->ctx;
    hipStream_t s = ctx->stream;
    const vx_baselm_config &c = e->cfg;
    if (with_embedding) {
        ProfSpan sp(ctx, "baselm.embedding");
        VX_CHECK(launch_embedding(s, e->model->raw, e->embd_offset, e->embd_dtype, c.embedding_length, 0,
                                  U(e->tokens), U(e->position), c.vocab_size, e->embedding_alpha, F(e->hidden),
                                  c.active_context_length));
    }
    {
        ProfSpan sp(ctx, "baselm.rope_table");
        VX_CHECK(launch_rope_table(s, e->rope_factors, U(e->position), c.head_dim, c.rope_theta, e->rope_scaling,
                                   reinterpret_cast<float2 *>(e->rope_table->ptr)));
    }
    for (uint32_t l = 0; l < c.block_count; ++l)
        for (uint32_t k = 0; k < LK_COUNT; ++k) {
            ProfSpan sp(ctx, kLayerKernelNames[k]);
            VX_CHECK(enqueue_layer_kernel(e, k, l, tier));
        }
    {
        ProfSpan sp(ctx, "baselm.output_norm");
        VX_CHECK(launch_rmsnorm(s, F(e->hidden), F(e->norm), e->output_norm, c.embedding_length, c.rms_epsilon,
                                U(e->position)));
    }
    if (logits) VX_CHECK(enqueue_logits(e));
    return VX_OK;
}

// The reference's dispatch sequence (record_transformer) with a host position.
int enqueue_reference(vx_baselm *e, uint32_t position, bool with_embedding, uint32_t token, bool logits) {
    vx_ctx *ctx = e->ctx;
    hipStream_t s = ctx->stream;
    const vx_baselm_config &c = e->cfg;
    const uint32_t q_per_kv = c.head_count / c.head_count_kv;
    if (with_embedding) {
        ProfSpan sp(ctx, "baselm.embedding");
        VX_CHECK(launch_embedding(s, e->model->raw, e->embd_offset, e->embd_dtype, c.embedding_length, token,
                                  nullptr, nullptr, c.vocab_size, e->embedding_alpha, F(e->hidden)));
    }
    {
        ProfSpan sp(ctx, "baselm.rmsnorm");
        VX_CHECK(launch_rmsnorm(s, F(e->hidden), F(e->norm), e->layers[0].attn_norm, c.embedding_length,
                                c.rms_epsilon, nullptr));
    }
    auto mv = [&](const WRef &w, const float *x, float *y, uint32_t rows, uint32_t cols, float alpha) {
        MatvecLaunch a;
        a.w = w;
        a.xl = x;
        a.rows = rows;
        a.cols = cols;
        a.alpha = alpha;
        a.epi = EPI_STORE;
        a.y = y;
        return launch_matvec(s, a);
    };
    for (uint32_t l = 0; l < c.block_count; ++l) {
        const Layer &L = e->layers[l];
        {
            ProfSpan sp(ctx, "baselm.qkv");
            VX_CHECK(mv(L.q, F(e->norm), F(e->q), c.embedding_length, c.embedding_length, 1.f));
            VX_CHECK(mv(L.k, F(e->norm), F(e->k), c.kv_dim, c.embedding_length, 1.f));
            VX_CHECK(mv(L.v, F(e->norm), F(e->v), c.kv_dim, c.embedding_length, 1.f));
        }
        {
            ProfSpan sp(ctx, "baselm.rope");
            VX_CHECK(launch_rope(s, F(e->q), F(e->k), e->rope_factors, position, nullptr, c.head_count,
                                 c.head_count_kv, c.head_dim, c.rope_theta, e->rope_scaling));
        }
        {
            ProfSpan sp(ctx, "baselm.store_kv");
            VX_CHECK(launch_store_kv(s, F(e->k), F(e->v), H(e->kv_k), H(e->kv_v), l, position, nullptr,
                                     c.active_context_length, c.kv_dim));
        }
        {
            ProfSpan sp(ctx, "baselm.attn_scores");
            VX_CHECK(launch_attn_scores(s, F(e->q), H(e->kv_k), F(e->scores), l, c.active_context_length,
                                        position, nullptr, c.head_dim, q_per_kv, c.head_count_kv, c.head_count));
        }
        {
            ProfSpan sp(ctx, "baselm.softmax");
            VX_CHECK(launch_softmax(s, F(e->scores), c.head_count, c.active_context_length, position, nullptr));
        }
        {
            ProfSpan sp(ctx, "baselm.attn_values");
            VX_CHECK(launch_attn_values(s, F(e->scores), H(e->kv_v), F(e->attention), l, c.active_context_length,
                                        position, nullptr, c.head_dim, q_per_kv, c.head_count_kv, c.head_count));
        }
        {
            ProfSpan sp(ctx, "baselm.matvec");
            VX_CHECK(mv(L.o, F(e->attention), F(e->branch), c.embedding_length, c.embedding_length, 1.f));
        }
        {
            ProfSpan sp(ctx, "baselm.residual_rmsnorm");
            VX_CHECK(launch_residual_rmsnorm(s, F(e->hidden), F(e->branch), F(e->norm), L.ffn_norm,
                                             c.embedding_length, c.rms_epsilon, e->residual_scale));
        }
        {
            ProfSpan sp(ctx, "baselm.swiglu");
            SwigluLaunch a;
            a.g = L.gate;
            a.u = L.up;
            a.x = F(e->norm);
            a.rows = c.feed_forward_length;
            a.cols = c.embedding_length;
            a.y = F(e->gate);
            VX_CHECK(launch_swiglu(s, a));
        }
        {
            ProfSpan sp(ctx, "baselm.matvec");
            VX_CHECK(mv(L.down, F(e->gate), F(e->branch), c.embedding_length, c.feed_forward_length, 1.f));
        }
        {
            ProfSpan sp(ctx, "baselm.residual_rmsnorm");
            const float *next = l + 1 < c.block_count ? e->layers[l + 1].attn_norm : e->output_norm;
            VX_CHECK(launch_residual_rmsnorm(s, F(e->hidden), F(e->branch), F(e->norm), next, c.embedding_length,
                                             c.rms_epsilon, e->residual_scale));
        }
    }
    if (logits) {
        ProfSpan sp(ctx, "baselm.matvec");
        VX_CHECK(mv(e->output, F(e->norm), F(e->logits), c.vocab_size, c.embedding_length, e->logit_alpha));
    }
    // Keep the device position in step with the host (the fused path advances it).
    return launch_set_step(s, U(e->tokens), U(e->position), position + 1u, 0, 0);
}

// One step at host position e->pos. The device position buffer already holds it.
int run_step(vx_baselm *e, bool with_embedding, uint32_t token, bool logits) {
    if (e->opt.exec_mode == VX_EXEC_REFERENCE) return enqueue_reference(e, e->pos, with_embedding, token, logits);
    const uint32_t tier = attn_tier(e, e->pos);
    if (e->ctx->prof_enabled) return enqueue_fused(e, with_embedding, logits, tier);
    if (e->opt.exec_mode == VX_EXEC_FUSED) return enqueue_fused(e, with_embedding, logits, tier);
    vx_graph *&g = e->graphs[with_embedding ? 1 : 0][logits ? 1 : 0][tier];
    if (!g) {
        VX_CHECK(vx_graph_begin(e->ctx));
        int st = enqueue_fused(e, with_embedding, logits, tier);
        vx_graph *ng = nullptr;
        int st2 = vx_graph_end(e->ctx, &ng);
        if (st != VX_OK) {
            if (ng) vx_graph_free(e->ctx, ng);
            return st;
        }
        VX_CHECK(st2);
        g = ng;
    }
    return vx_graph_launch(e->ctx, g);
}

// ------------------------------------------------------------------ prefill
// Token-batched prefill (the seq_* op family of local.rs:482-527 applied to the
// BaseLM stack, with Q8_0 projections, a causal mask and a position base):
//   embedding rows -> per layer:
//     rmsnorm(h)*attn_norm -> f16 hi/lo planes        (k_seq_rmsnorm)
//     q|k|v = planes . Wq|Wk|Wv                       (k_gemm, split-K)
//     RoPE at pos0+t, K/V rows -> f16 cache, q planes  (k_seq_rope_store)
//     causal attention over cache keys 0..pos0+t       (k_prefill_attn)
//     h += scale * Wo . attn                           (k_gemm residual)
//     rmsnorm(h)*ffn_norm -> planes                    (k_seq_rmsnorm)
//     act = silu(Wg . n) * (Wu . n) -> planes          (k_gemm swiglu)
//     h += scale * Wdown . act                         (k_gemm residual)
//   then the last token's rmsnorm(h)*output_norm into the engine's norm buffer.
// This computes what prefill_tokens (baselm.rs:823-839) computes one token at a
// time: the same KV-cache rows and the same final state, to rounding.
int ensure_prefill_work(vx_baselm *e) {
    if (e->pf.cap) return VX_OK;
    const vx_baselm_config &c = e->cfg;
    const uint32_t cap = std::min<uint32_t>(kPrefillChunk, c.active_context_length);
    VX_CHECK(prefill_stack_alloc(e->ctx, cap, c.embedding_length, c.feed_forward_length, c.kv_dim, &e->pf));
    return alloc(e->ctx, (uint64_t)c.active_context_length * 4u, &e->pf_tok);
}

// The BaseLM layers as a token-batched stack (RoPE on, the engine's KV caches).
PrefillStack make_stack(vx_baselm *e) {
    const vx_baselm_config &c = e->cfg;
    PrefillStack p;
    p.ctx = e->ctx;
    p.nH = c.embedding_length;
    p.nF = c.feed_forward_length;
    p.nKV = c.kv_dim;
    p.q_heads = c.head_count;
    p.kv_heads = c.head_count_kv;
    p.head_dim = c.head_dim;
    p.context = c.active_context_length;
    p.n_layers = c.block_count;
    p.eps = c.rms_epsilon;
    p.residual_scale = e->residual_scale;
    p.layers = e->layers.data();
    p.pw = e->pw.empty() ? nullptr : e->pw.data();
    p.rope = true;
    p.rope_factors = e->rope_factors;
    p.theta = c.rope_theta;
    p.rope_scaling = e->rope_scaling;
    p.kc = H(e->kv_k);
    p.vc = H(e->kv_v);
    p.work = &e->pf;
    p.schedule = e->opt.prefill_schedule;
    return p;
}

// Split-K factor that brings a projection to about one workgroup per CU.
// Repack every layer's Q8_0 projections into the prefill-GEMM layout (once;
// about 53 MB per layer at the VoxCPM2 geometry). Left empty, so that prefill
// uses the general GEMM, when a projection is not Q8_0.
int ensure_prefill_weights(vx_baselm *e) {
    if (e->pw_tried) return VX_OK;
    e->pw_tried = true;
    const vx_baselm_config &c = e->cfg;
    const uint32_t nH = c.embedding_length, nF = c.feed_forward_length, nKV = c.kv_dim;
    for (const Layer &L : e->layers) {
        const WRef *m[7] = {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down};
        for (const WRef *w : m)
            if (w->dtype != VX_DTYPE_Q8_0 || !w->raw) return VX_OK;
    }
    if (nH % 32u || nF % 32u) return VX_OK;
    const uint64_t per_layer = prefill_matrix_bytes(nH, nH) + 2u * prefill_matrix_bytes(nKV, nH) +
                               prefill_matrix_bytes(nH, nH) + prefill_matrix_bytes(2u * nF, nH) +
                               prefill_matrix_bytes(nH, nF) + 6u * 256u;
    VX_CHECK(alloc(e->ctx, per_layer * c.block_count, &e->pw_arena));
    uint8_t *cur = static_cast<uint8_t *>(e->pw_arena->ptr);
    hipStream_t s = e->ctx->stream;
    auto place = [&](PrefillMatrix &pm, const WRef &w0, const WRef *w1, uint32_t rows, uint32_t K) {
        const uint32_t rows_out = w1 ? 2u * rows : rows;
        pm.rows_pad = (rows_out + 127u) / 128u * 128u;
        pm.q = reinterpret_cast<int8_t *>(cur);
        pm.d = reinterpret_cast<float *>(cur + (uint64_t)pm.rows_pad * K);
        cur += (prefill_matrix_bytes(rows_out, K) + 255u) / 256u * 256u;
        return launch_repack_prefill(s, w0.raw, w0.raw_offset, w1 ? w1->raw_offset : 0u, rows, K, w1 ? 1 : 0, pm.q,
                                     pm.d);
    };
    e->pw.resize(c.block_count);
    for (uint32_t l = 0; l < c.block_count; ++l) {
        const Layer &L = e->layers[l];
        StackPrefillWeights &P = e->pw[l];
        int st = VX_OK;
        if ((st = place(P.q, L.q, nullptr, nH, nH)) || (st = place(P.k, L.k, nullptr, nKV, nH)) ||
            (st = place(P.v, L.v, nullptr, nKV, nH)) || (st = place(P.o, L.o, nullptr, nH, nH)) ||
            (st = place(P.gu, L.gate, &L.up, nF, nH)) || (st = place(P.down, L.down, nullptr, nH, nF))) {
            e->pw.clear();
            return st;
        }
    }
    return VX_OK;
}

// One chunk of T tokens at positions pos0..pos0+T-1, token ids at tok (device).
int enqueue_prefill_chunk(vx_baselm *e, const uint32_t *tok, uint32_t pos0, uint32_t T, float *rows) {
    vx_ctx *ctx = e->ctx;
    hipStream_t s = ctx->stream;
    const vx_baselm_config &c = e->cfg;
    const uint32_t nH = c.embedding_length;
    {
        ProfSpan sp(ctx, "prefill.embedding");
        VX_CHECK(launch_seq_embedding(s, e->model->raw, e->embd_offset, e->embd_dtype, nH, tok, T, c.vocab_size,
                                      e->embedding_alpha, F(e->pf.h), nH));
    }
    VX_CHECK(enqueue_prefill_stack(make_stack(e), pos0, T));
    if (rows) {   // every token's output_buffer (rmsnorm(h)*output_norm), as the decode step leaves it
        ProfSpan sp(ctx, "prefill.output_rows");
        SeqNormArgs n;
        n.h = F(e->pf.h);
        n.ldh = nH;
        n.w = e->output_norm;
        n.n = nH;
        n.eps = c.rms_epsilon;
        n.y = rows;
        n.ldy = nH;
        VX_CHECK(launch_seq_rmsnorm(s, n, T));
    }
    // Engine state after the chunk: hidden = last token's residual stream, norm =
    // its rmsnorm(h)*output_norm (record_transformer's final residual_rmsnorm).
    ProfSpan sp(ctx, "prefill.output_norm");
    const float *last = F(e->pf.h) + (size_t)(T - 1u) * nH;
    VX_HIP(hipMemcpyAsync(e->hidden->ptr, last, (size_t)nH * 4u, hipMemcpyDeviceToDevice, s));
    return launch_rmsnorm(s, last, F(e->norm), e->output_norm, nH, c.rms_epsilon, nullptr);
}

// Prefill n tokens at the engine position: upload the ids, run the chunks, leave
// the device position at the next decode position.
int enqueue_prefill(vx_baselm *e, const uint32_t *tokens, uint32_t n, float *rows = nullptr) {
    VX_CHECK(prefill_stack_check(make_stack(e)));
    VX_CHECK(ensure_prefill_work(e));
    VX_CHECK(ensure_prefill_weights(e));
    hipStream_t s = e->ctx->stream;
    VX_HIP(hipMemcpyAsync(e->pf_tok->ptr, tokens, (size_t)n * 4u, hipMemcpyHostToDevice, s));
    uint32_t done = 0;
    int cancelled = VX_OK;
    while (done < n) {
        // A cancellation between chunks keeps the chunks already enqueued (their
        // K/V rows and position), as a host-side stop between decode steps does.
        if ((cancelled = check_cancel(e->ctx)) != VX_OK) break;
        const uint32_t T = std::min<uint32_t>(e->pf.cap, n - done);
        VX_CHECK(enqueue_prefill_chunk(e, U(e->pf_tok) + done, e->pos + done, T,
                                       rows ? rows + (size_t)done * e->cfg.embedding_length : nullptr));
        done += T;
    }
    VX_CHECK(launch_set_step(s, U(e->tokens), U(e->position), e->pos + done, 0, 0));
    e->pos += done;
    return cancelled;
}

int ensure_context(const vx_baselm *e, uint32_t steps) {  // baselm.rs:882-890
    if ((uint64_t)e->pos + steps > e->cfg.active_context_length)
        return fail(VX_ERR_CONTEXT_FULL, "BaseLM KV cache is full at %u tokens; reset or increase --max-context",
                    e->cfg.active_context_length);
    return VX_OK;
}

int check_token(const vx_baselm *e, uint32_t token) {  // baselm.rs:629-631
    if (token >= e->cfg.vocab_size)
        return fail(VX_ERR_TOKEN_RANGE, "token id %u is outside vocabulary 0..%u", token, e->cfg.vocab_size);
    return VX_OK;
}

double now_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// collect_result (baselm.rs:1204-1231).
int collect_result(vx_baselm *e, uint32_t position, double elapsed_ms, uint32_t top_k, vx_step_result *res,
                   vx_top_logit *top) {
    const uint32_t n = e->cfg.embedding_length;
    std::vector<float> h(n);
    VX_CHECK(vx_download(e->ctx, e->norm, 0, h.data(), (uint64_t)n * 4u));
    double sum = 0.0, sq = 0.0;
    for (float x : h) {
        sum += (double)x;
        sq += (double)x * (double)x;
    }
    uint32_t n_top = 0;
    if (top_k > 0 && top) {
        const uint32_t vocab = e->cfg.vocab_size;
        std::vector<float> lg(vocab);
        VX_CHECK(vx_download(e->ctx, e->logits, 0, lg.data(), (uint64_t)vocab * 4u));
        VX_CHECK(vx_top_k_logits(lg.data(), vocab, top_k, top, &n_top));
    }
    if (res) {
        res->position = position;
        res->elapsed_ms = elapsed_ms;
        res->final_hidden_checksum = sum;
        res->final_hidden_l2 = std::sqrt(sq);
        res->n_top = n_top;
    }
    return VX_OK;
}

int upload_embedding(vx_baselm *e, const float *emb, uint32_t n) {
    if (!emb) return fail(VX_ERR_INVALID_ARG, "external embedding is null");
    if (n != e->cfg.embedding_length)
        return fail(VX_ERR_SHAPE, "external embedding has %u floats; expected %u", n, e->cfg.embedding_length);
    VX_HIP(hipStreamSynchronize(e->ctx->stream));
    VX_HIP(hipMemcpyAsync(e->hidden->ptr, emb, (size_t)n * 4u, hipMemcpyHostToDevice, e->ctx->stream));
    VX_HIP(hipStreamSynchronize(e->ctx->stream));
    return VX_OK;
}

}  // namespace

namespace vx {

vx_ctx *baselm_context(const vx_baselm *e) { return e->ctx; }

uint32_t baselm_hidden_size(const vx_baselm *e) { return e->cfg.embedding_length; }

int baselm_prefill_rows(vx_baselm *e, const uint32_t *tokens, uint32_t n, float *rows) {
    if (!tokens || n == 0) return fail(VX_ERR_INVALID_ARG, "prefill token list is empty");
    for (uint32_t i = 0; i < n; ++i) VX_CHECK(check_token(e, tokens[i]));
    VX_CHECK(ensure_context(e, n));
    return enqueue_prefill(e, tokens, n, rows);
}

}  // namespace vx

extern "C" {

int vx_top_k_logits(const float *logits, uint32_t n, uint32_t k, vx_top_logit *out, uint32_t *n_out) {
    if ((!logits && n) || (!out && k)) return fail(VX_ERR_INVALID_ARG, "vx_top_k_logits: null argument");
    std::vector<uint32_t> idx;
    idx.reserve(n);
    for (uint32_t i = 0; i < n; ++i)
        if (std::isfinite(logits[i])) idx.push_back(i);
    const uint32_t m = std::min<uint32_t>(k, (uint32_t)idx.size());
    std::partial_sort(idx.begin(), idx.begin() + m, idx.end(), [&](uint32_t a, uint32_t b) {
        return logits[a] > logits[b] || (logits[a] == logits[b] && a < b);
    });
    for (uint32_t i = 0; i < m; ++i) out[i] = vx_top_logit{idx[i], logits[idx[i]]};
    if (n_out) *n_out = m;
    return VX_OK;
}

float vx_baselm_rope_scaling_factor(const vx_baselm_config *c) {
    if (!c) return 1.0f;
    if (!c->rope_longrope || c->context_length <= c->rope_original_context_length ||
        c->rope_original_context_length <= 1u)
        return 1.0f;
    const float max = (float)c->context_length;
    const float original = (float)c->rope_original_context_length;
    return std::sqrt(1.0f + std::log(max / original) / std::log(original));
}

uint64_t vx_baselm_kv_cache_bytes(const vx_baselm_config *c) {
    if (!c) return 0;
    return (uint64_t)c->block_count * c->active_context_length * c->kv_dim * 2u * 2u;
}

int vx_baselm_create(vx_ctx *ctx, const vx_model *model, const vx_baselm_config *cfg,
                     const vx_baselm_options *opt, vx_baselm **out) {
    if (!ctx || !model || !cfg || !out) return fail(VX_ERR_INVALID_ARG, "vx_baselm_create: null argument");
    *out = nullptr;
    vx_baselm_options o{};
    o.exec_mode = VX_EXEC_GRAPH;
    o.strict_geometry = 1;
    if (opt) o = *opt;
    if (o.exec_mode > VX_EXEC_PERSISTENT) return fail(VX_ERR_INVALID_ARG, "unknown exec_mode %u", o.exec_mode);
    if (o.exec_mode == VX_EXEC_PERSISTENT)
        return fail(VX_ERR_UNSUPPORTED, "the persistent decode step is not built: its in-kernel phase hand-offs "
                                        "cost more than kernel boundaries on this GPU; use VX_EXEC_GRAPH");
    VX_CHECK(validate_config(*cfg, o.strict_geometry != 0));
    const vx_baselm_config &c = *cfg;
    vx_baselm *e = new vx_baselm();
    e->ctx = ctx;
    e->model = model;
    e->cfg = c;
    e->opt = o;
    auto bail = [&](int st) {
        free_all(e);
        delete e;
        return st;
    };
    // Tensor validation (BaseLmConfig::from_gguf / validate_layer, baselm.rs:123-180, 227-262).
    const vx_tensor_info *embd;
    int st = find(model, "token_embd.weight", &embd);
    if (st) return bail(st);
    if (embd->n_dims != 2) return bail(fail(VX_ERR_SHAPE, "token_embd.weight must be rank 2"));
    if ((st = require_dims(embd, {c.embedding_length, c.vocab_size}))) return bail(st);
    if ((st = require_matrix_type(embd))) return bail(st);
    e->embd_offset = (uint32_t)embd->offset;
    e->embd_dtype = embd->ggml_type;
    if (model->by_name.count("output.weight")) {
        if ((st = matrix(model, "output.weight", c.embedding_length, c.vocab_size, &e->output))) return bail(st);
    } else {
        if ((st = matrix(model, "token_embd.weight", c.embedding_length, c.vocab_size, &e->output))) return bail(st);
    }
    if ((st = vec_f32(model, "output_norm.weight", c.embedding_length, &e->output_norm))) return bail(st);
    const char *factor_name = c.context_length > c.rope_original_context_length ? "rope_factors_long.weight"
                                                                                 : "rope_factors_short.weight";
    if ((st = vec_f32(model, "rope_factors_short.weight", c.head_dim / 2u, &e->rope_factors))) return bail(st);
    if ((st = vec_f32(model, "rope_factors_long.weight", c.head_dim / 2u, &e->rope_factors))) return bail(st);
    if ((st = vec_f32(model, factor_name, c.head_dim / 2u, &e->rope_factors))) return bail(st);
    e->layers.resize(c.block_count);
    for (uint32_t l = 0; l < c.block_count; ++l) {
        Layer &L = e->layers[l];
        const std::string p = "blk." + std::to_string(l) + ".";
        const uint64_t H = c.embedding_length, KV = c.kv_dim, FF = c.feed_forward_length;
        if ((st = vec_f32(model, p + "attn_norm.weight", H, &L.attn_norm))) return bail(st);
        if ((st = vec_f32(model, p + "ffn_norm.weight", H, &L.ffn_norm))) return bail(st);
        if ((st = matrix(model, p + "attn_q.weight", H, H, &L.q))) return bail(st);
        if ((st = matrix(model, p + "attn_k.weight", H, KV, &L.k))) return bail(st);
        if ((st = matrix(model, p + "attn_v.weight", H, KV, &L.v))) return bail(st);
        if ((st = matrix(model, p + "attn_output.weight", H, H, &L.o))) return bail(st);
        if ((st = matrix(model, p + "ffn_gate.weight", H, FF, &L.gate))) return bail(st);
        if ((st = matrix(model, p + "ffn_up.weight", H, FF, &L.up))) return bail(st);
        if ((st = matrix(model, p + "ffn_down.weight", FF, H, &L.down))) return bail(st);
        if (L.gate.dtype != L.up.dtype)  // dispatch_swiglu baselm.rs:1166-1168
            return bail(fail(VX_ERR_SHAPE, "SwiGLU gate/up dtypes differ in layer %u", l));
        if (o.exec_mode != VX_EXEC_REFERENCE && (L.q.dtype != L.k.dtype || L.q.dtype != L.v.dtype))
            return bail(fail(VX_ERR_UNSUPPORTED, "fused QKV needs one dtype for q/k/v (layer %u)", l));
    }
    if (c.head_count / c.head_count_kv > 16u || (c.head_dim != 64u && c.head_dim != 128u))
        if (o.exec_mode != VX_EXEC_REFERENCE)
            return bail(fail(VX_ERR_UNSUPPORTED, "fused attention needs head_dim 64/128 and q_per_kv <= 16"));
    e->residual_scale = effective_scale(c.residual_scale);
    e->embedding_alpha = effective_scale(c.embedding_scale);
    e->logit_alpha = effective_scale(c.logit_scale);
    e->rope_scaling = vx_baselm_rope_scaling_factor(&c);
    // Context splits of the decode attention: one per 64 positions of the active
    // context, at most kShortSplits (attn_out merges them itself).
    if (o.prefill_schedule > VX_PREFILL_STREAMK_TAIL_FIRST)
        return bail(fail(VX_ERR_INVALID_ARG, "unknown prefill_schedule %u", o.prefill_schedule));
    uint32_t splits = o.attn_splits;
    if (splits == 0)
        splits = std::min<uint32_t>(kShortSplits, std::max<uint32_t>(1u, (c.active_context_length + 63u) / 64u));
    if (splits > kMaxAttnSplits)
        return bail(fail(VX_ERR_INVALID_ARG, "attn_splits must be at most %u", kMaxAttnSplits));
    e->splits = splits;
    // The streamed attention tiers of long contexts (unless the caller fixed the
    // split count).
    const bool foldable = c.head_count * c.head_dim == c.embedding_length &&
                          (c.embedding_length == 1024u || c.embedding_length == 2048u) &&
                          (c.head_dim == 64u || c.head_dim == 128u);
    if (o.attn_splits == 0 && foldable && o.exec_mode != VX_EXEC_REFERENCE) {
        if (c.active_context_length >= kTier1FromKeys) e->tier_splits[1] = kShortSplits;
        if (c.active_context_length >= kTier2FromKeys) e->tier_splits[2] = kMaxFoldedSplits;
    }
    e->fold_attn_merge = splits <= kMaxFoldedSplits && foldable;
    // Buffers (BaseLmEngine::new, baselm.rs:479-506).
    const uint64_t f = 4;
    const uint64_t cache = vx_baselm_kv_cache_bytes(&c) / 2u;
    if ((st = alloc(ctx, c.embedding_length * f, &e->hidden)) || (st = alloc(ctx, c.embedding_length * f, &e->norm)) ||
        (st = alloc(ctx, c.embedding_length * f, &e->q)) || (st = alloc(ctx, c.kv_dim * f, &e->k)) ||
        (st = alloc(ctx, c.kv_dim * f, &e->v)) || (st = alloc(ctx, c.embedding_length * f, &e->attention)) ||
        (st = alloc(ctx, c.feed_forward_length * f, &e->gate)) ||
        (st = alloc(ctx, c.embedding_length * f, &e->branch)) || (st = alloc(ctx, c.vocab_size * f, &e->logits)) ||
        (st = alloc(ctx, (uint64_t)c.head_count * c.active_context_length * f, &e->scores)) ||
        (st = alloc(ctx, cache, &e->kv_k)) || (st = alloc(ctx, cache, &e->kv_v)) ||
        (st = alloc(ctx, 256, &e->position)) || (st = alloc(ctx, (uint64_t)c.active_context_length * 4u, &e->tokens)) ||
        (st = alloc(ctx, attn_scratch_bytes(c.head_dim, c.head_count, c.head_count_kv, std::max({splits, e->tier_splits[1], e->tier_splits[2]})),
                    &e->attn_scratch)) ||
        (st = alloc(ctx, (uint64_t)c.head_dim * 4u, &e->rope_table)))
        return bail(st);
    // Zero state once (outside any graph). Cache contents are otherwise only ever
    // overwritten, as in the reference (reset leaves stale KV, baselm.rs:616-620).
    vx_buf *zero[] = {e->hidden, e->norm, e->kv_k, e->kv_v, e->position, e->tokens, e->attn_scratch, e->logits};
    for (vx_buf *b : zero)
        if (hipMemsetAsync(b->ptr, 0, b->bytes, ctx->stream) != hipSuccess)
            return bail(fail(VX_ERR_HIP, "hipMemsetAsync of engine state failed"));
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return bail(fail(VX_ERR_HIP, "engine init sync failed"));
    *out = e;
    return VX_OK;
}

int vx_baselm_destroy(vx_baselm *e) {
    if (!e) return VX_OK;
    (void)hipStreamSynchronize(e->ctx->stream);
    free_all(e);
    delete e;
    return VX_OK;
}

int vx_baselm_reset(vx_baselm *e) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_baselm_reset: null engine");
    e->pos = 0;
    return VX_OK;
}

uint32_t vx_baselm_position(const vx_baselm *e) { return e ? e->pos : 0u; }

int vx_baselm_set_position(vx_baselm *e, uint32_t position) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_baselm_set_position: null engine");
    if (position > e->cfg.active_context_length)
        return fail(VX_ERR_CONTEXT_FULL, "position %u beyond context %u", position, e->cfg.active_context_length);
    e->pos = position;
    return VX_OK;
}

int vx_baselm_decode_token(vx_baselm *e, uint32_t token_id, uint32_t top_k, vx_step_result *res, vx_top_logit *top) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_baselm_decode_token: null engine");
    VX_CHECK(check_cancel(e->ctx));
    VX_CHECK(check_token(e, token_id));
    VX_CHECK(ensure_context(e, 1));
    const uint32_t position = e->pos;
    const double t0 = now_ms();
    VX_CHECK(launch_set_step(e->ctx->stream, U(e->tokens), U(e->position), position, token_id, 1));
    VX_CHECK(run_step(e, true, token_id, true));
    VX_CHECK(vx_sync(e->ctx));
    const double elapsed = now_ms() - t0;
    e->pos += 1;
    return collect_result(e, position, elapsed, top_k, res, top);
}

int vx_baselm_decode_embedding(vx_baselm *e, const float *embedding, uint32_t n, uint32_t top_k,
                               vx_step_result *res, vx_top_logit *top) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_baselm_decode_embedding: null engine");
    VX_CHECK(check_cancel(e->ctx));
    VX_CHECK(ensure_context(e, 1));
    VX_CHECK(upload_embedding(e, embedding, n));
    const uint32_t position = e->pos;
    const double t0 = now_ms();
    VX_CHECK(launch_set_step(e->ctx->stream, U(e->tokens), U(e->position), position, 0, 0));
    VX_CHECK(run_step(e, false, 0, true));
    VX_CHECK(vx_sync(e->ctx));
    const double elapsed = now_ms() - t0;
    e->pos += 1;
    return collect_result(e, position, elapsed, top_k, res, top);
}

int vx_baselm_decode_token_gpu_only(vx_baselm *e, uint32_t token_id, uint32_t *position_out) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_baselm_decode_token_gpu_only: null engine");
    VX_CHECK(check_cancel(e->ctx));
    VX_CHECK(check_token(e, token_id));
    VX_CHECK(ensure_context(e, 1));
    const uint32_t position = e->pos;
    VX_CHECK(launch_set_step(e->ctx->stream, U(e->tokens), U(e->position), position, token_id, 1));
    VX_CHECK(run_step(e, true, token_id, false));
    e->pos += 1;
    if (position_out) *position_out = position;
    return VX_OK;
}

int vx_baselm_decode_embedding_gpu_only(vx_baselm *e, const float *embedding, uint32_t n, uint32_t *position_out) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_baselm_decode_embedding_gpu_only: null engine");
    VX_CHECK(check_cancel(e->ctx));
    VX_CHECK(ensure_context(e, 1));
    VX_CHECK(upload_embedding(e, embedding, n));
    const uint32_t position = e->pos;
    VX_CHECK(launch_set_step(e->ctx->stream, U(e->tokens), U(e->position), position, 0, 0));
    VX_CHECK(run_step(e, false, 0, false));
    e->pos += 1;
    if (position_out) *position_out = position;
    return VX_OK;
}

int vx_baselm_decode_embedding_from_gpu_only(vx_baselm *e, const vx_buf *source, uint32_t *position_out) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_baselm_decode_embedding_from_gpu_only: null engine");
    VX_CHECK(check_cancel(e->ctx));
    if (!source || source->bytes < (uint64_t)e->cfg.embedding_length * 4u)  // baselm.rs:799-801
        return fail(VX_ERR_BOUNDS, "GPU embedding source is too small for BaseLM %u-float input",
                    e->cfg.embedding_length);
    VX_CHECK(ensure_context(e, 1));
    const uint32_t position = e->pos;
    VX_HIP(hipMemcpyAsync(e->hidden->ptr, source->ptr, (size_t)e->cfg.embedding_length * 4u,
                          hipMemcpyDeviceToDevice, e->ctx->stream));
    VX_CHECK(launch_set_step(e->ctx->stream, U(e->tokens), U(e->position), position, 0, 0));
    VX_CHECK(run_step(e, false, 0, false));
    e->pos += 1;
    if (position_out) *position_out = position;
    return VX_OK;
}

int vx_baselm_decode_tokens_gpu_only(vx_baselm *e, const uint32_t *tokens, uint32_t n) {
    if (!e || (!tokens && n)) return fail(VX_ERR_INVALID_ARG, "vx_baselm_decode_tokens_gpu_only: null argument");
    if (n == 0) return VX_OK;
    for (uint32_t i = 0; i < n; ++i) VX_CHECK(check_token(e, tokens[i]));
    VX_CHECK(ensure_context(e, n));
    VX_CHECK(check_cancel(e->ctx));
    VX_HIP(hipMemcpyAsync(U(e->tokens) + e->pos, tokens, (size_t)n * 4u, hipMemcpyHostToDevice, e->ctx->stream));
    VX_HIP(hipStreamSynchronize(e->ctx->stream));
    VX_CHECK(launch_set_step(e->ctx->stream, U(e->tokens), U(e->position), e->pos, 0, 0));
    for (uint32_t i = 0; i < n; ++i) {
        VX_CHECK(check_cancel(e->ctx));   // each token is a step: earlier ones stay done
        if (e->opt.exec_mode == VX_EXEC_REFERENCE) {
            VX_CHECK(enqueue_reference(e, e->pos, true, tokens[i], false));
        } else {
            VX_CHECK(run_step(e, true, tokens[i], false));
        }
        e->pos += 1;
    }
    return VX_OK;
}

int vx_baselm_prefill_tokens(vx_baselm *e, const uint32_t *tokens, uint32_t n, uint32_t top_k_last,
                             vx_step_result *res, vx_top_logit *top) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_baselm_prefill_tokens: null engine");
    if (!tokens || n == 0) return fail(VX_ERR_INVALID_ARG, "prefill token list is empty");
    for (uint32_t i = 0; i < n; ++i) VX_CHECK(check_token(e, tokens[i]));
    VX_CHECK(ensure_context(e, n));
    // Every token is a decode step (baselm.rs:823-839). Only the last step's
    // logits are observable, so earlier steps skip the LM head.
    if (n > 1) VX_CHECK(vx_baselm_decode_tokens_gpu_only(e, tokens, n - 1));
    return vx_baselm_decode_token(e, tokens[n - 1], top_k_last, res, top);
}

int vx_baselm_prefill_tokens_batched(vx_baselm *e, const uint32_t *tokens, uint32_t n, uint32_t top_k_last,
                                     vx_step_result *res, vx_top_logit *top) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_baselm_prefill_tokens_batched: null engine");
    if (!tokens || n == 0) return fail(VX_ERR_INVALID_ARG, "prefill token list is empty");
    for (uint32_t i = 0; i < n; ++i) VX_CHECK(check_token(e, tokens[i]));
    VX_CHECK(ensure_context(e, n));
    const double t0 = now_ms();
    VX_CHECK(enqueue_prefill(e, tokens, n));
    VX_CHECK(enqueue_logits(e));  // decode_token of the last token computes logits
    VX_CHECK(vx_sync(e->ctx));
    const double elapsed = now_ms() - t0;
    return collect_result(e, e->pos - 1u, elapsed, top_k_last, res, top);
}

int vx_baselm_prefill_tokens_batched_gpu_only(vx_baselm *e, const uint32_t *tokens, uint32_t n) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_baselm_prefill_tokens_batched_gpu_only: null engine");
    if (!tokens || n == 0) return fail(VX_ERR_INVALID_ARG, "prefill token list is empty");
    for (uint32_t i = 0; i < n; ++i) VX_CHECK(check_token(e, tokens[i]));
    VX_CHECK(ensure_context(e, n));
    return enqueue_prefill(e, tokens, n);
}

int vx_baselm_benchmark(vx_baselm *e, uint32_t token_id, uint32_t warmup, uint32_t iterations,
                        vx_baselm_benchmark_result *out) {
    if (!e || !out) return fail(VX_ERR_INVALID_ARG, "vx_baselm_benchmark: null argument");
    if (iterations == 0) return fail(VX_ERR_INVALID_ARG, "benchmark iterations must be > 0");
    const uint64_t needed = (uint64_t)warmup + iterations;
    if (needed > e->cfg.active_context_length)
        return fail(VX_ERR_CONTEXT_FULL, "benchmark needs %llu context positions but --max-context is %u",
                    (unsigned long long)needed, e->cfg.active_context_length);
    e->pos = 0;  // reset (baselm.rs:857)
    for (uint32_t i = 0; i < warmup; ++i) VX_CHECK(vx_baselm_decode_token(e, token_id, 0, nullptr, nullptr));
    double sum = 0.0, mn = INFINITY, mx = 0.0;
    for (uint32_t i = 0; i < iterations; ++i) {
        vx_step_result r;
        VX_CHECK(vx_baselm_decode_token(e, token_id, 0, &r, nullptr));
        sum += r.elapsed_ms;
        mn = std::min(mn, r.elapsed_ms);
        mx = std::max(mx, r.elapsed_ms);
    }
    out->iterations = iterations;
    out->token_id = token_id;
    out->mean_ms = sum / iterations;
    out->min_ms = mn;
    out->max_ms = mx;
    out->tokens_per_second = 1000.0 / out->mean_ms;
    return VX_OK;
}

vx_buf *vx_baselm_buffer(vx_baselm *e, uint32_t which) {
    if (!e) return nullptr;
    switch (which) {
        case VX_BASELM_BUF_HIDDEN: return e->hidden;
        case VX_BASELM_BUF_NORM: return e->norm;
        case VX_BASELM_BUF_Q: return e->q;
        case VX_BASELM_BUF_K: return e->k;
        case VX_BASELM_BUF_V: return e->v;
        case VX_BASELM_BUF_ATTENTION: return e->attention;
        case VX_BASELM_BUF_GATE: return e->gate;
        case VX_BASELM_BUF_BRANCH: return e->branch;
        case VX_BASELM_BUF_LOGITS: return e->logits;
        case VX_BASELM_BUF_SCORES: return e->scores;
        case VX_BASELM_BUF_KV_K: return e->kv_k;
        case VX_BASELM_BUF_KV_V: return e->kv_v;
        case VX_BASELM_BUF_POSITION: return e->position;
        default: return nullptr;
    }
}

int vx_baselm_profile_steps(vx_baselm *e, const uint32_t *tokens, uint32_t n, vx_prof_entry *out, uint32_t cap,
                            uint32_t *count) {
    if (!e || (!tokens && n)) return fail(VX_ERR_INVALID_ARG, "vx_baselm_profile_steps: null argument");
    for (uint32_t i = 0; i < n; ++i) VX_CHECK(check_token(e, tokens[i]));
    VX_CHECK(ensure_context(e, n));
    vx_ctx *ctx = e->ctx;
    VX_CHECK(vx_prof_reset(ctx));
    const bool was = ctx->prof_enabled;
    ctx->prof_enabled = true;
    int st = VX_OK;
    for (uint32_t i = 0; i < n && st == VX_OK; ++i) {
        st = launch_set_step(ctx->stream, U(e->tokens), U(e->position), e->pos, tokens[i], 1);
        if (st == VX_OK) {
            if (e->opt.exec_mode == VX_EXEC_REFERENCE)
                st = enqueue_reference(e, e->pos, true, tokens[i], false);
            else
                st = enqueue_fused(e, true, false, attn_tier(e, e->pos));
        }
        if (st == VX_OK) st = vx_sync(ctx);
        e->pos += 1;
    }
    ctx->prof_enabled = was;
    VX_CHECK(st);
    return vx_prof_snapshot(ctx, out, cap, count);
}

int vx_baselm_time_layer_kernel(vx_baselm *e, uint32_t which, uint32_t reps, double *avg_ms) {
    if (!e || !avg_ms) return fail(VX_ERR_INVALID_ARG, "vx_baselm_time_layer_kernel: null argument");
    if (which >= LK_COUNT) return fail(VX_ERR_INVALID_ARG, "unknown layer kernel %u", which);
    if (reps == 0) return fail(VX_ERR_INVALID_ARG, "reps must be > 0");
    if (e->opt.exec_mode == VX_EXEC_REFERENCE)
        return fail(VX_ERR_STATE, "kernel timing needs the fused decode kernels (graph or fused mode)");
    vx_ctx *ctx = e->ctx;
    // Each pass: a 384 MiB streaming read that evicts the 256 MiB MALL and the L2s,
    // then the kernel over the 28 layers' weights, as one graph; a second graph of
    // the reads alone is subtracted. So every launch reads its weights from HBM,
    // as in the decode step, and the figure is its cost inside a graph chain
    // (duration plus the launch gap between dependent kernels).
    constexpr uint64_t kEvict = 384ull << 20;
    constexpr uint32_t kEvictBlocks = 4096;
    vx_buf *ev = nullptr, *sink = nullptr;
    vx_graph *ga = nullptr, *gb = nullptr;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    int st = vx_alloc(ctx, kEvict, &ev);
    if (st == VX_OK) st = vx_alloc(ctx, (uint64_t)kEvictBlocks * 16u, &sink);
    auto capture = [&](bool with_kernel, vx_graph **out) {
        int s2 = vx_graph_begin(ctx);
        for (uint32_t r = 0; r < reps && s2 == VX_OK; ++r) {
            s2 = vx_diag_stream_read(ctx, ev, 0, kEvict, sink, kEvictBlocks, 4);
            for (uint32_t l = 0; with_kernel && l < e->cfg.block_count && s2 == VX_OK; ++l)
                s2 = enqueue_layer_kernel(e, which, l, attn_tier(e, e->pos));
        }
        const int s3 = vx_graph_end(ctx, out);
        return s2 != VX_OK ? s2 : s3;
    };
    if (st == VX_OK) st = capture(true, &ga);
    if (st == VX_OK) st = capture(false, &gb);
    if (st == VX_OK && (hipEventCreate(&t0) != hipSuccess || hipEventCreate(&t1) != hipSuccess))
        st = fail(VX_ERR_HIP, "hipEventCreate failed");
    double ms[2] = {0.0, 0.0};
    for (int k = 0; k < 2 && st == VX_OK; ++k) {
        vx_graph *g = k == 0 ? ga : gb;
        st = vx_graph_launch(ctx, g);  // warm
        if (st == VX_OK && hipEventRecord(t0, ctx->stream) != hipSuccess) st = fail(VX_ERR_HIP, "hipEventRecord failed");
        for (int rep = 0; rep < 3 && st == VX_OK; ++rep) st = vx_graph_launch(ctx, g);
        if (st == VX_OK && hipEventRecord(t1, ctx->stream) != hipSuccess) st = fail(VX_ERR_HIP, "hipEventRecord failed");
        float f = 0.f;
        if (st == VX_OK && hipEventSynchronize(t1) != hipSuccess) st = fail(VX_ERR_HIP, "hipEventSynchronize failed");
        if (st == VX_OK && hipEventElapsedTime(&f, t0, t1) != hipSuccess) st = fail(VX_ERR_HIP, "hipEventElapsedTime failed");
        ms[k] = (double)f / 3.0;
    }
    if (t0) (void)hipEventDestroy(t0);
    if (t1) (void)hipEventDestroy(t1);
    if (ga) vx_graph_free(ctx, ga);
    if (gb) vx_graph_free(ctx, gb);
    vx_free(ctx, ev);
    vx_free(ctx, sink);
    VX_CHECK(st);
    *avg_ms = (ms[0] - ms[1]) / ((double)reps * e->cfg.block_count);
    return VX_OK;
}

}  // extern "C"
