// ResidualLM + FSQ + fusion + stop head (ResidualFsqEngine, acoustic.rs:400-1035)
// over HIP.
//
// One step (step_record_submit, acoustic.rs:847-893) in the fused modes:
//   FSQ         latent = fsq.in_proj(base) + b                k_matvec (bias)
//               latent = round(tanh(latent) * s) / s          k_fsq_quantize
//               fsq    = fsq.out_proj(latent) + b             k_matvec (bias, second store = current_lm)
//   or (text prefix) current_lm = base                        device copy
//   fusion      hidden = res_fusion_proj([fsq | base, embedding | 0]) + b, snapshot   k_matvec (fusion)
//   8 ResidualLM layers, the BaseLM decode kernels with RoPE off:
//     k_qkv_fused      rmsnorm(h)*attn_norm -> Q/K/V -> f16 KV store
//     attention        split-context single-query attention
//     k_matvec (resid) h += Wo . attn
//     k_swiglu (norm)  gate = silu(Wg . n) * (Wu . n), n = rmsnorm(h)*ffn_norm
//     k_matvec (resid) h += Wdown . gate
//   k_rmsnorm          norm = rmsnorm(h)*output_norm, then position += 1
// That is record_residual_lm's op order (acoustic.rs:968-1035) with each
// residual_rmsnorm split between its producing and consuming kernel. In graph
// mode a step is one hipGraph, cached per (FSQ or text prefix, base buffer,
// embedding buffer). VX_EXEC_REFERENCE issues the reference's per-op dispatches.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <string>

#include "vx_internal.h"

using namespace vx;

namespace {

using RLayer = StackLayer;

struct Lin {
    WRef w;
    const void *b = nullptr;
    uint32_t bt = 0;   // 0 = f32 bias, 1 = f16 bias
};

struct CachedGraph {
    bool fsq = false;
    const void *base = nullptr, *emb = nullptr;
    vx_graph *g = nullptr;
};

constexpr size_t kMaxCachedGraphs = 8;

inline float *F(vx_buf *b) { return static_cast<float *>(b->ptr); }
inline const float *F(const vx_buf *b) { return static_cast<const float *>(b->ptr); }
inline uint32_t *U(vx_buf *b) { return static_cast<uint32_t *>(b->ptr); }
inline __half *H(vx_buf *b) { return static_cast<__half *>(b->ptr); }

}  // namespace

struct vx_residual {
    vx_ctx *ctx = nullptr;
    const vx_model *model = nullptr;
    vx_acoustic_config cfg{};
    vx_residual_options opt{};
    Lin fsq_in, fsq_out, fusion, stop1;
    WRef stop2;
    const float *output_norm = nullptr;
    std::vector<RLayer> layers;
    vx_buf *base_input = nullptr, *current_embed = nullptr, *zero_embed = nullptr, *fsq_latent = nullptr;
    vx_buf *fsq_output = nullptr, *current_lm = nullptr, *hidden = nullptr, *fusion_snapshot = nullptr;
    vx_buf *norm = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attention = nullptr, *gate = nullptr;
    vx_buf *branch = nullptr, *scores = nullptr, *kv_k = nullptr, *kv_v = nullptr, *stop_hidden = nullptr;
    vx_buf *stop_logits = nullptr, *position = nullptr, *attn_scratch = nullptr;
    uint32_t splits = 1;
    bool fold_attn_merge = false;
    uint32_t pos = 0;
    std::vector<CachedGraph> graphs;
    // Token-batched text prefix (allocated on first use): the layer stack's
    // activations, the fusion input [cap][2H] (right half kept zero) and the
    // BaseLM output rows of a cross-engine chunk [cap][H].
    StackWork pf;
    vx_buf *fuse_x = nullptr, *rows = nullptr;
};

namespace {

int find(const vx_model *m, const std::string &name, const vx_tensor_info **out) {
    auto it = m->by_name.find(name);
    if (it == m->by_name.end())
        return fail(VX_ERR_NOT_FOUND, "required GGUF tensor \"%s\" is missing", name.c_str());
    *out = &m->tensors[it->second];
    return VX_OK;
}

// require_matrix(.., require_f16 = true) (acoustic.rs:189-205): dims [cols, rows], F16.
int matrix(const vx_model *m, const std::string &name, uint32_t cols, uint32_t rows, WRef *w) {
    const vx_tensor_info *t;
    VX_CHECK(find(m, name, &t));
    if (t->n_dims != 2 || t->dims[0] != cols || t->dims[1] != rows)
        return fail(VX_ERR_SHAPE, "tensor %s has dimensions [%llu, %llu], expected [%u, %u]", name.c_str(),
                    (unsigned long long)t->dims[0], (unsigned long long)(t->n_dims > 1 ? t->dims[1] : 1), cols,
                    rows);
    if (t->ggml_type != VX_DTYPE_F16)
        return fail(VX_ERR_SHAPE, "tensor %s is type %u, expected F16 from VoxCPM2-Acoustic-F16.gguf", name.c_str(),
                    t->ggml_type);
    return resolve_matrix(m, (uint32_t)t->offset, VX_DTYPE_F16, rows, cols, w, name.c_str());
}

// require_vector (acoustic.rs:207-216); f32_only adds the F32 checks of the norms.
int vector(const vx_model *m, const std::string &name, uint32_t n, bool allow_f32, bool f32_only, const void **p,
           uint32_t *bt) {
    const vx_tensor_info *t;
    VX_CHECK(find(m, name, &t));
    if (t->n_dims != 1 || t->dims[0] != n)
        return fail(VX_ERR_SHAPE, "tensor %s has dimensions [%llu], expected [%u]", name.c_str(),
                    (unsigned long long)t->dims[0], n);
    const bool ok = t->ggml_type == VX_DTYPE_F16 || (allow_f32 && t->ggml_type == VX_DTYPE_F32);
    if (!ok || (f32_only && t->ggml_type != VX_DTYPE_F32))
        return fail(VX_ERR_SHAPE, "tensor %s uses unsupported vector type %u", name.c_str(), t->ggml_type);
    if (bt) *bt = t->ggml_type == VX_DTYPE_F32 ? 0u : 1u;
    return resolve_vector(m, (uint32_t)t->offset, t->ggml_type, n, p, name.c_str());
}

int norm_f32(const vx_model *m, const std::string &name, uint32_t n, const float **out) {
    const void *p = nullptr;
    VX_CHECK(vector(m, name, n, true, true, &p, nullptr));
    *out = static_cast<const float *>(p);
    return VX_OK;
}

int linear(const vx_model *m, const std::string &prefix, uint32_t cols, uint32_t rows, bool bias_f32, Lin *l) {
    VX_CHECK(matrix(m, prefix + ".weight", cols, rows, &l->w));
    return vector(m, prefix + ".bias", rows, bias_f32, false, &l->b, &l->bt);
}

int validate(const vx_acoustic_config &c, bool strict) {
    if (!c.residual_block_count || !c.embedding_length || !c.feed_forward_length || !c.head_count ||
        !c.head_count_kv || !c.head_dim || !c.fsq_latent_dim || !c.active_context_length)
        return fail(VX_ERR_INVALID_ARG, "acoustic config has a zero dimension");
    if (c.kv_dim != c.head_count_kv * c.head_dim || c.fusion_input_dim != 2u * c.embedding_length)
        return fail(VX_ERR_SHAPE, "acoustic config: kv_dim %u / fusion_input_dim %u inconsistent", c.kv_dim,
                    c.fusion_input_dim);
    if (c.head_count % c.head_count_kv)
        return fail(VX_ERR_SHAPE, "head_count %u is not divisible by head_count_kv %u", c.head_count, c.head_count_kv);
    if (c.head_count * c.head_dim != c.embedding_length)
        return fail(VX_ERR_SHAPE, "head_count x head_dim (%u) != embedding_length %u", c.head_count * c.head_dim,
                    c.embedding_length);
    if (!c.no_rope) return fail(VX_ERR_UNSUPPORTED, "VoxCPM2 ResidualLM must run with no_rope=true");
    if (!std::isfinite(c.fsq_scale) || c.fsq_scale <= 0.f)
        return fail(VX_ERR_INVALID_ARG, "invalid FSQ scale %g", c.fsq_scale);
    if (c.active_context_length > 8192u)
        return fail(VX_ERR_INVALID_ARG, "ResidualLM --max-context must be in 1..=8192; got %u", c.active_context_length);
    if (strict && (c.residual_block_count != 8 || c.embedding_length != 2048 || c.fsq_latent_dim != 512 ||
                   c.feed_forward_length != 6144 || c.head_count != 16 || c.head_count_kv != 2 || c.head_dim != 128))
        return fail(VX_ERR_UNSUPPORTED,
                    "unsupported VoxCPM2 acoustic contract: residual_layers=%u, embd=%u, fsq_latent=%u; expected "
                    "8/2048/512 over the 2048/6144/16/2/128 BaseLM geometry",
                    c.residual_block_count, c.embedding_length, c.fsq_latent_dim);
    return VX_OK;
}

void free_all(vx_residual *e) {
    for (CachedGraph &g : e->graphs)
        if (g.g) vx_graph_free(e->ctx, g.g);
    e->graphs.clear();
    prefill_stack_free(e->ctx, &e->pf);
    for (vx_buf **b : {&e->fuse_x, &e->rows})
        if (*b) {
            vx_free(e->ctx, *b);
            *b = nullptr;
        }
    vx_buf **bufs[] = {&e->base_input, &e->current_embed, &e->zero_embed, &e->fsq_latent, &e->fsq_output,
                       &e->current_lm, &e->hidden,        &e->fusion_snapshot, &e->norm,  &e->q,
                       &e->k,          &e->v,             &e->attention, &e->gate,        &e->branch,
                       &e->scores,     &e->kv_k,          &e->kv_v,      &e->stop_hidden, &e->stop_logits,
                       &e->position,   &e->attn_scratch};
    for (vx_buf **b : bufs)
        if (*b) {
            vx_free(e->ctx, *b);
            *b = nullptr;
        }
}

double now_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// stats (acoustic.rs:1248-1257): position-weighted checksum and L2 norm.
void stats(const std::vector<float> &v, double *checksum, double *l2) {
    double c = 0.0, sq = 0.0;
    for (size_t i = 0; i < v.size(); ++i) {
        const double x = (double)v[i];
        c += x * (double)(i % 251u + 1u);
        sq += x * x;
    }
    *checksum = c;
    *l2 = std::sqrt(sq);
}

int download_stats(vx_residual *e, const vx_buf *b, uint32_t n, double *checksum, double *l2) {
    std::vector<float> h(n);
    VX_CHECK(vx_download(e->ctx, b, 0, h.data(), (uint64_t)n * 4u));
    stats(h, checksum, l2);
    return VX_OK;
}

int linear_bias(hipStream_t s, const Lin &l, const float *x, float *y, uint32_t rows, uint32_t cols,
                float *y2 = nullptr) {
    MatvecLaunch a;
    a.w = l.w;
    a.xl = x;
    a.rows = rows;
    a.cols = cols;
    a.bias = l.b;
    a.bias_dtype = l.bt;
    a.y = y;
    // linear_bias.comp with alpha 1 stores (acc + b) * 1 = acc + b, which the
    // fusion epilogue stores to both outputs.
    a.epi = y2 ? EPI_FUSION : EPI_BIAS;
    a.y2 = y2;
    return launch_matvec(s, a);
}

// record_fsq (acoustic.rs:909-939); current_lm (nullable) receives a second copy
// of the FSQ output (record_current_lm_copy, acoustic.rs:895-907).
int enqueue_fsq(vx_residual *e, const float *base, float *current_lm) {
    vx_ctx *ctx = e->ctx;
    hipStream_t s = ctx->stream;
    const vx_acoustic_config &c = e->cfg;
    {
        ProfSpan sp(ctx, "residual.fsq_in");
        VX_CHECK(linear_bias(s, e->fsq_in, base, F(e->fsq_latent), c.fsq_latent_dim, c.embedding_length));
    }
    {
        ProfSpan sp(ctx, "residual.fsq_quantize");
        VX_CHECK(launch_fsq_quantize(s, F(e->fsq_latent), c.fsq_latent_dim, c.fsq_scale));
    }
    ProfSpan sp(ctx, "residual.fsq_out");
    return linear_bias(s, e->fsq_out, F(e->fsq_latent), F(e->fsq_output), c.embedding_length, c.fsq_latent_dim,
                       current_lm);
}

// record_fusion (acoustic.rs:941-966): hidden = W [left | right] + b, snapshot.
int enqueue_fusion(vx_residual *e, const float *left, const float *right) {
    ProfSpan sp(e->ctx, "residual.fusion");
    const vx_acoustic_config &c = e->cfg;
    MatvecLaunch a;
    a.w = e->fusion.w;
    a.xl = left;
    a.xr = right;
    a.left_cols = c.embedding_length;
    a.rows = c.embedding_length;
    a.cols = c.fusion_input_dim;
    a.epi = EPI_FUSION;
    a.bias = e->fusion.b;
    a.bias_dtype = e->fusion.bt;
    a.y = F(e->hidden);
    a.y2 = F(e->fusion_snapshot);
    return launch_matvec(e->ctx->stream, a);
}

// The ResidualLM stack with the fused decode kernels (device position).
int enqueue_layers_fused(vx_residual *e) {
    vx_ctx *ctx = e->ctx;
    hipStream_t s = ctx->stream;
    const vx_acoustic_config &c = e->cfg;
    AttnLaunch at;
    at.q = F(e->q);
    at.kc = H(e->kv_k);
    at.vc = H(e->kv_v);
    at.out = F(e->attention);
    at.partials = F(e->attn_scratch);
    at.position = U(e->position);
    at.context = c.active_context_length;
    at.head_dim = c.head_dim;
    at.q_heads = c.head_count;
    at.kv_heads = c.head_count_kv;
    at.splits = e->splits;
    for (uint32_t l = 0; l < c.residual_block_count; ++l) {
        const RLayer &L = e->layers[l];
        at.layer = l;
        {
            ProfSpan sp(ctx, "residual.qkv");
            QkvFusedLaunch a;
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
            a.no_rope = true;
            a.layer = l;
            a.context = c.active_context_length;
            a.qo = F(e->q);
            a.ko = F(e->k);
            a.vo = F(e->v);
            a.kc = H(e->kv_k);
            a.vc = H(e->kv_v);
            a.position = U(e->position);
            VX_CHECK(launch_qkv_fused(s, a));
        }
        {
            ProfSpan sp(ctx, "residual.attention");
            VX_CHECK(e->fold_attn_merge ? launch_attn_partials(s, at) : launch_attn_decode(s, at));
        }
        {
            ProfSpan sp(ctx, "residual.attn_out");
            MatvecLaunch ao;
            ao.w = L.o;
            ao.xl = F(e->attention);
            ao.rows = c.embedding_length;
            ao.cols = c.embedding_length;
            ao.epi = EPI_RESIDUAL;
            ao.y = F(e->hidden);
            ao.scale = c.residual_scale;
            if (e->fold_attn_merge) {
                AttnOutLaunch a;
                a.mv = ao;
                a.partials = at.partials;
                a.attn_out = F(e->attention);
                a.position = at.position;
                a.context = at.context;
                a.splits = at.splits;
                a.q_heads = at.q_heads;
                a.head_dim = at.head_dim;
                VX_CHECK(launch_attn_out(s, a));
            } else {
                VX_CHECK(launch_matvec(s, ao));
            }
        }
        {
            ProfSpan sp(ctx, "residual.swiglu");
            SwigluLaunch a;
            a.g = L.gate;
            a.u = L.up;
            a.x = F(e->hidden);
            a.norm = L.ffn_norm;
            a.eps = c.rms_epsilon;
            a.rows = c.feed_forward_length;
            a.cols = c.embedding_length;
            a.y = F(e->gate);
            VX_CHECK(launch_swiglu(s, a));
        }
        {
            ProfSpan sp(ctx, "residual.down");
            MatvecLaunch a;
            a.w = L.down;
            a.xl = F(e->gate);
            a.rows = c.embedding_length;
            a.cols = c.feed_forward_length;
            a.epi = EPI_RESIDUAL;
            a.y = F(e->hidden);
            a.scale = c.residual_scale;
            VX_CHECK(launch_matvec(s, a));
        }
    }
    ProfSpan sp(ctx, "residual.output_norm");
    return launch_rmsnorm(s, F(e->hidden), F(e->norm), e->output_norm, c.embedding_length, c.rms_epsilon,
                          U(e->position));
}

// record_residual_lm (acoustic.rs:968-1035) as the reference's per-op dispatches.
int enqueue_layers_reference(vx_residual *e, uint32_t position) {
    vx_ctx *ctx = e->ctx;
    hipStream_t s = ctx->stream;
    const vx_acoustic_config &c = e->cfg;
    const uint32_t q_per_kv = c.head_count / c.head_count_kv;
    auto mv = [&](const WRef &w, const float *x, float *y, uint32_t rows, uint32_t cols) {
        MatvecLaunch a;
        a.w = w;
        a.xl = x;
        a.rows = rows;
        a.cols = cols;
        a.epi = EPI_STORE;
        a.y = y;
        return launch_matvec(s, a);
    };
    {
        ProfSpan sp(ctx, "residual.rmsnorm");
        VX_CHECK(launch_rmsnorm(s, F(e->hidden), F(e->norm), e->layers[0].attn_norm, c.embedding_length,
                                c.rms_epsilon, nullptr));
    }
    for (uint32_t l = 0; l < c.residual_block_count; ++l) {
        const RLayer &L = e->layers[l];
        {
            ProfSpan sp(ctx, "residual.qkv");
            VX_CHECK(mv(L.q, F(e->norm), F(e->q), c.embedding_length, c.embedding_length));
            VX_CHECK(mv(L.k, F(e->norm), F(e->k), c.kv_dim, c.embedding_length));
            VX_CHECK(mv(L.v, F(e->norm), F(e->v), c.kv_dim, c.embedding_length));
        }
        {
            ProfSpan sp(ctx, "residual.store_kv");
            VX_CHECK(launch_store_kv(s, F(e->k), F(e->v), H(e->kv_k), H(e->kv_v), l, position, nullptr,
                                     c.active_context_length, c.kv_dim));
        }
        {
            ProfSpan sp(ctx, "residual.attention");
            VX_CHECK(launch_attn_scores(s, F(e->q), H(e->kv_k), F(e->scores), l, c.active_context_length, position,
                                        nullptr, c.head_dim, q_per_kv, c.head_count_kv, c.head_count));
            VX_CHECK(launch_softmax(s, F(e->scores), c.head_count, c.active_context_length, position, nullptr));
            VX_CHECK(launch_attn_values(s, F(e->scores), H(e->kv_v), F(e->attention), l, c.active_context_length,
                                        position, nullptr, c.head_dim, q_per_kv, c.head_count_kv, c.head_count));
        }
        {
            ProfSpan sp(ctx, "residual.matvec");
            VX_CHECK(mv(L.o, F(e->attention), F(e->branch), c.embedding_length, c.embedding_length));
        }
        {
            ProfSpan sp(ctx, "residual.residual_rmsnorm");
            VX_CHECK(launch_residual_rmsnorm(s, F(e->hidden), F(e->branch), F(e->norm), L.ffn_norm,
                                             c.embedding_length, c.rms_epsilon, c.residual_scale));
        }
        {
            ProfSpan sp(ctx, "residual.swiglu");
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
            ProfSpan sp(ctx, "residual.matvec");
            VX_CHECK(mv(L.down, F(e->gate), F(e->branch), c.embedding_length, c.feed_forward_length));
        }
        {
            ProfSpan sp(ctx, "residual.residual_rmsnorm");
            const float *next = l + 1 < c.residual_block_count ? e->layers[l + 1].attn_norm : e->output_norm;
            VX_CHECK(launch_residual_rmsnorm(s, F(e->hidden), F(e->branch), F(e->norm), next, c.embedding_length,
                                             c.rms_epsilon, c.residual_scale));
        }
    }
    return launch_set_step(s, nullptr, U(e->position), position + 1u, 0, 0);
}

// One step's work after the device position holds e->pos: FSQ (or the raw
// copy), fusion, the ResidualLM stack.
int enqueue_step(vx_residual *e, bool fsq, const float *base, const float *emb) {
    const vx_acoustic_config &c = e->cfg;
    if (fsq) {
        VX_CHECK(enqueue_fsq(e, base, F(e->current_lm)));
    } else {
        ProfSpan sp(e->ctx, "residual.current_lm_copy");
        VX_HIP(hipMemcpyAsync(e->current_lm->ptr, base, (size_t)c.embedding_length * 4u, hipMemcpyDeviceToDevice,
                              e->ctx->stream));
    }
    VX_CHECK(enqueue_fusion(e, fsq ? F(e->fsq_output) : base, fsq ? emb : F(e->zero_embed)));
    if (e->opt.exec_mode == VX_EXEC_REFERENCE) return enqueue_layers_reference(e, e->pos);
    return enqueue_layers_fused(e);
}

// Enqueue one step at e->pos (replaying or capturing its graph in graph mode).
int run_step(vx_residual *e, bool fsq, const float *base, const float *emb) {
    if (e->pos >= e->cfg.active_context_length)
        return fail(VX_ERR_CONTEXT_FULL, "ResidualLM KV cache is full at %u positions", e->cfg.active_context_length);
    vx_ctx *ctx = e->ctx;
    VX_CHECK(launch_set_step(ctx->stream, nullptr, U(e->position), e->pos, 0, 0));
    if (e->opt.exec_mode != VX_EXEC_GRAPH || ctx->prof_enabled) return enqueue_step(e, fsq, base, emb);
    for (const CachedGraph &g : e->graphs)
        if (g.fsq == fsq && g.base == base && g.emb == emb) return vx_graph_launch(ctx, g.g);
    VX_CHECK(vx_graph_begin(ctx));
    const int st = enqueue_step(e, fsq, base, emb);
    vx_graph *ng = nullptr;
    const int st2 = vx_graph_end(ctx, &ng);
    if (st != VX_OK) {
        if (ng) vx_graph_free(ctx, ng);
        return st;
    }
    VX_CHECK(st2);
    if (e->graphs.size() >= kMaxCachedGraphs) {
        vx_graph_free(ctx, e->graphs.front().g);
        e->graphs.erase(e->graphs.begin());
    }
    e->graphs.push_back(CachedGraph{fsq, base, emb, ng});
    return vx_graph_launch(ctx, ng);
}

// step_record_submit (acoustic.rs:847-893) after the inputs are in place.
int submit_step(vx_residual *e, bool fsq, const float *base, const float *emb, vx_residual_step_result *out) {
    VX_CHECK(check_cancel(e->ctx));
    const uint32_t position = e->pos;
    const double t0 = now_ms();
    VX_CHECK(run_step(e, fsq, base, emb));
    VX_CHECK(vx_sync(e->ctx));
    const double elapsed = now_ms() - t0;
    e->pos += 1;
    if (!out) return VX_OK;
    const uint32_t n = e->cfg.embedding_length;
    vx_residual_step_result r{};
    r.position = position;
    r.fsq_applied = fsq ? 1u : 0u;
    r.elapsed_ms = elapsed;
    if (fsq) VX_CHECK(download_stats(e, e->fsq_output, n, &r.fsq_checksum, &r.fsq_l2));
    VX_CHECK(download_stats(e, e->fusion_snapshot, n, &r.fused_input_checksum, &r.fused_input_l2));
    VX_CHECK(download_stats(e, e->norm, n, &r.residual_hidden_checksum, &r.residual_hidden_l2));
    *out = r;
    return VX_OK;
}

// step_record_submit_gpu_only (acoustic.rs:830-845): waits, reads nothing back.
int submit_step_gpu_only(vx_residual *e, bool fsq, const float *base, const float *emb, vx_residual_gpu_step *out) {
    VX_CHECK(check_cancel(e->ctx));
    const uint32_t position = e->pos;
    const double t0 = now_ms();
    VX_CHECK(run_step(e, fsq, base, emb));
    VX_CHECK(vx_sync(e->ctx));
    const double elapsed = now_ms() - t0;
    e->pos += 1;
    if (out) *out = vx_residual_gpu_step{position, fsq ? 1u : 0u, elapsed};
    return VX_OK;
}

int check_host(const vx_residual *e, const float *v, uint32_t n, const char *what) {  // acoustic.rs:1212-1217
    if (!v) return fail(VX_ERR_INVALID_ARG, "%s is null", what);
    if (n != e->cfg.embedding_length)
        return fail(VX_ERR_SHAPE, "%s has %u floats; expected %u", what, n, e->cfg.embedding_length);
    return VX_OK;
}

int check_gpu(const vx_residual *e, const vx_buf *b, const char *what) {
    if (!b || b->bytes < (uint64_t)e->cfg.embedding_length * 4u)
        return fail(VX_ERR_BOUNDS, "%s is too small for %u f32 values", what, e->cfg.embedding_length);
    return VX_OK;
}

int upload_host(vx_residual *e, vx_buf *dst, const float *src) {
    VX_HIP(hipStreamSynchronize(e->ctx->stream));
    VX_HIP(hipMemcpyAsync(dst->ptr, src, (size_t)e->cfg.embedding_length * 4u, hipMemcpyHostToDevice,
                          e->ctx->stream));
    VX_HIP(hipStreamSynchronize(e->ctx->stream));
    return VX_OK;
}

// Stop predictor (acoustic.rs:619-652): Linear(H->H)+b, SiLU, Linear(H->2).
int predict_stop(vx_residual *e, const float *x, vx_stop_prediction *out) {
    VX_CHECK(check_cancel(e->ctx));
    vx_ctx *ctx = e->ctx;
    hipStream_t s = ctx->stream;
    const vx_acoustic_config &c = e->cfg;
    const double t0 = now_ms();
    {
        ProfSpan sp(ctx, "residual.stop_linear1");
        VX_CHECK(linear_bias(s, e->stop1, x, F(e->stop_hidden), c.embedding_length, c.embedding_length));
    }
    {
        ProfSpan sp(ctx, "residual.stop_silu");
        VX_CHECK(launch_silu_inplace(s, F(e->stop_hidden), c.embedding_length));
    }
    {
        ProfSpan sp(ctx, "residual.stop_linear2");
        MatvecLaunch a;
        a.w = e->stop2;
        a.xl = F(e->stop_hidden);
        a.rows = 2;
        a.cols = c.embedding_length;
        a.epi = EPI_STORE;
        a.y = F(e->stop_logits);
        VX_CHECK(launch_matvec(s, a));
    }
    float logits[2];
    VX_CHECK(vx_download(ctx, e->stop_logits, 0, logits, sizeof(logits)));
    if (out) *out = vx_stop_prediction{logits[1] > logits[0] ? 1u : 0u, logits[0], logits[1], now_ms() - t0};
    return VX_OK;
}

// ------------------------------------------------------------- batched text prefix
// The text-prefix positions of a conditioning prefill (runtime.rs:483-566 runs
// them one BaseLM decode + one ResidualLM text-prefix step at a time) as one
// token batch per engine: the BaseLM batched prefill leaves every position's
// output row, the fusion projection takes [row | 0] for all rows at once, and the
// ResidualLM layers run as a token-batched stack without RoPE over its own cache.
// The engine state afterwards is the last position's, as after the per-position
// steps: hidden, norm (output), fusion snapshot and current_lm (the raw row).
int ensure_prefill_work(vx_residual *e) {
    if (e->pf.cap) return VX_OK;
    const vx_acoustic_config &c = e->cfg;
    const uint32_t cap = std::min<uint32_t>(kPrefillChunk, c.active_context_length);
    VX_CHECK(prefill_stack_alloc(e->ctx, cap, c.embedding_length, c.feed_forward_length, c.kv_dim, &e->pf));
    VX_CHECK(vx_alloc(e->ctx, (uint64_t)cap * c.fusion_input_dim * 4u, &e->fuse_x));
    VX_CHECK(vx_alloc(e->ctx, (uint64_t)cap * c.embedding_length * 4u, &e->rows));
    VX_HIP(hipMemsetAsync(e->fuse_x->ptr, 0, e->fuse_x->bytes, e->ctx->stream));
    return VX_OK;
}

PrefillStack make_stack(vx_residual *e) {
    const vx_acoustic_config &c = e->cfg;
    PrefillStack p;
    p.ctx = e->ctx;
    p.nH = c.embedding_length;
    p.nF = c.feed_forward_length;
    p.nKV = c.kv_dim;
    p.q_heads = c.head_count;
    p.kv_heads = c.head_count_kv;
    p.head_dim = c.head_dim;
    p.context = c.active_context_length;
    p.n_layers = c.residual_block_count;
    p.eps = c.rms_epsilon;
    p.residual_scale = c.residual_scale;
    p.layers = e->layers.data();
    p.rope = false;
    p.kc = H(e->kv_k);
    p.vc = H(e->kv_v);
    p.work = &e->pf;
    return p;
}

int check_prefill(vx_residual *e, uint32_t n) {
    if (n == 0) return fail(VX_ERR_INVALID_ARG, "text prefix of zero positions");
    if ((uint64_t)e->pos + n > e->cfg.active_context_length)
        return fail(VX_ERR_CONTEXT_FULL, "ResidualLM KV cache is full at %u positions", e->cfg.active_context_length);
    if (e->opt.exec_mode == VX_EXEC_REFERENCE)
        return fail(VX_ERR_STATE, "the batched text prefix needs the graph or fused exec mode");
    VX_CHECK(prefill_stack_check(make_stack(e)));
    return ensure_prefill_work(e);
}

// T <= cap text-prefix positions from BaseLM output rows [T][H] (device).
int enqueue_prefill_rows(vx_residual *e, const float *rows, uint32_t T) {
    vx_ctx *ctx = e->ctx;
    hipStream_t s = ctx->stream;
    const vx_acoustic_config &c = e->cfg;
    const uint32_t nH = c.embedding_length;
    {
        ProfSpan sp(ctx, "residual.prefix_fusion");
        VX_HIP(hipMemcpy2DAsync(e->fuse_x->ptr, (size_t)c.fusion_input_dim * 4u, rows, (size_t)nH * 4u,
                                (size_t)nH * 4u, T, hipMemcpyDeviceToDevice, s));
        VX_CHECK(enqueue_seq_linear(s, e->fusion.w, e->fusion.b, e->fusion.bt, nH, c.fusion_input_dim, T,
                                    F(e->fuse_x), 0, c.fusion_input_dim, F(e->pf.h), 0, nH, 1.f));
    }
    const float *last_fused = F(e->pf.h) + (size_t)(T - 1u) * nH;
    VX_HIP(hipMemcpyAsync(e->fusion_snapshot->ptr, last_fused, (size_t)nH * 4u, hipMemcpyDeviceToDevice, s));
    VX_HIP(hipMemcpyAsync(e->current_lm->ptr, rows + (size_t)(T - 1u) * nH, (size_t)nH * 4u,
                          hipMemcpyDeviceToDevice, s));
    VX_CHECK(enqueue_prefill_stack(make_stack(e), e->pos, T));
    ProfSpan sp(ctx, "residual.prefix_output_norm");
    const float *last = F(e->pf.h) + (size_t)(T - 1u) * nH;
    VX_HIP(hipMemcpyAsync(e->hidden->ptr, last, (size_t)nH * 4u, hipMemcpyDeviceToDevice, s));
    VX_CHECK(launch_rmsnorm(s, last, F(e->norm), e->output_norm, nH, c.rms_epsilon, nullptr));
    e->pos += T;
    return launch_set_step(s, nullptr, U(e->position), e->pos, 0, 0);
}

}  // namespace

extern "C" {

int vx_residual_prefill_text_from_gpu_rows(vx_residual *e, const vx_buf *rows, uint32_t n) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_residual_prefill_text_from_gpu_rows: null engine");
    VX_CHECK(check_cancel(e->ctx));
    if (!rows || rows->bytes < (uint64_t)n * e->cfg.embedding_length * 4u)
        return fail(VX_ERR_BOUNDS, "BaseLM output rows buffer is too small for %u x %u f32 values", n,
                    e->cfg.embedding_length);
    VX_CHECK(check_prefill(e, n));
    for (uint32_t done = 0; done < n;) {
        const uint32_t T = std::min<uint32_t>(e->pf.cap, n - done);
        VX_CHECK(enqueue_prefill_rows(e, F(rows) + (size_t)done * e->cfg.embedding_length, T));
        done += T;
    }
    return VX_OK;
}

int vx_prefill_text_cross_engine(vx_baselm *base, vx_residual *e, const uint32_t *tokens, uint32_t n) {
    if (!base || !e) return fail(VX_ERR_INVALID_ARG, "vx_prefill_text_cross_engine: null engine");
    VX_CHECK(check_cancel(e->ctx));
    if (baselm_context(base) != e->ctx)
        return fail(VX_ERR_INVALID_ARG, "the BaseLM and ResidualLM engines must share one context");
    if (baselm_hidden_size(base) != e->cfg.embedding_length)
        return fail(VX_ERR_SHAPE, "BaseLM hidden %u != ResidualLM hidden %u", baselm_hidden_size(base),
                    e->cfg.embedding_length);
    if (!tokens) return fail(VX_ERR_INVALID_ARG, "prefill token list is empty");
    VX_CHECK(check_prefill(e, n));
    for (uint32_t done = 0; done < n;) {
        const uint32_t T = std::min<uint32_t>(e->pf.cap, n - done);
        VX_CHECK(baselm_prefill_rows(base, tokens + done, T, F(e->rows)));
        VX_CHECK(enqueue_prefill_rows(e, F(e->rows), T));
        done += T;
    }
    return VX_OK;
}

uint64_t vx_acoustic_kv_cache_bytes(const vx_acoustic_config *c) {
    if (!c) return 0;
    return (uint64_t)c->residual_block_count * c->active_context_length * c->kv_dim * 2u * 2u;
}

int vx_residual_create(vx_ctx *ctx, const vx_model *model, const vx_acoustic_config *cfg,
                       const vx_residual_options *opt, vx_residual **out) {
    if (!ctx || !model || !cfg || !out) return fail(VX_ERR_INVALID_ARG, "vx_residual_create: null argument");
    *out = nullptr;
    vx_residual_options o{VX_EXEC_GRAPH, 1};
    if (opt) o = *opt;
    if (o.exec_mode != VX_EXEC_GRAPH && o.exec_mode != VX_EXEC_FUSED && o.exec_mode != VX_EXEC_REFERENCE)
        return fail(VX_ERR_INVALID_ARG, "ResidualLM exec_mode %u (graph, fused or reference)", o.exec_mode);
    VX_CHECK(validate(*cfg, o.strict_geometry != 0));
    const vx_acoustic_config &c = *cfg;
    if (o.exec_mode != VX_EXEC_REFERENCE && c.head_dim != 64u && c.head_dim != 128u)
        return fail(VX_ERR_UNSUPPORTED, "fused attention needs head_dim 64/128");
    vx_residual *e = new vx_residual();
    e->ctx = ctx;
    e->model = model;
    e->cfg = c;
    e->opt = o;
    auto bail = [&](int st) {
        free_all(e);
        delete e;
        return st;
    };
    const uint32_t Hd = c.embedding_length, L = c.fsq_latent_dim, KV = c.kv_dim, FF = c.feed_forward_length;
    int st;
    // validate_tensors (acoustic.rs:127-174).
    if ((st = linear(model, "fsq.in_proj", Hd, L, false, &e->fsq_in)) ||
        (st = linear(model, "fsq.out_proj", L, Hd, false, &e->fsq_out)) ||
        (st = linear(model, "projections.res_fusion_proj", c.fusion_input_dim, Hd, false, &e->fusion)) ||
        (st = norm_f32(model, "residual_lm.output_norm.weight", Hd, &e->output_norm)) ||
        (st = linear(model, "stop_predictor.linear1", Hd, Hd, true, &e->stop1)) ||
        (st = matrix(model, "stop_predictor.linear2.weight", Hd, 2, &e->stop2)))
        return bail(st);
    e->layers.resize(c.residual_block_count);
    for (uint32_t l = 0; l < c.residual_block_count; ++l) {
        RLayer &R = e->layers[l];
        const std::string p = "residual_lm.blk." + std::to_string(l) + ".";
        if ((st = norm_f32(model, p + "attn_norm.weight", Hd, &R.attn_norm)) ||
            (st = norm_f32(model, p + "ffn_norm.weight", Hd, &R.ffn_norm)) ||
            (st = matrix(model, p + "attn_q.weight", Hd, Hd, &R.q)) ||
            (st = matrix(model, p + "attn_k.weight", Hd, KV, &R.k)) ||
            (st = matrix(model, p + "attn_v.weight", Hd, KV, &R.v)) ||
            (st = matrix(model, p + "attn_output.weight", Hd, Hd, &R.o)) ||
            (st = matrix(model, p + "ffn_gate.weight", Hd, FF, &R.gate)) ||
            (st = matrix(model, p + "ffn_up.weight", Hd, FF, &R.up)) ||
            (st = matrix(model, p + "ffn_down.weight", FF, Hd, &R.down)))
            return bail(st);
    }
    // Attention splits as in the BaseLM engine: one per 64 positions of the
    // active context, at most the number attn_out merges itself.
    e->splits = std::min<uint32_t>(kShortSplits, std::max<uint32_t>(1u, (c.active_context_length + 63u) / 64u));
    e->fold_attn_merge = (Hd == 1024u || Hd == 2048u) && (c.head_dim == 64u || c.head_dim == 128u);
    // Buffers (ResidualFsqEngine::new, acoustic.rs:470-504) plus the device
    // position and the attention partials.
    const uint64_t f = 4, cache = vx_acoustic_kv_cache_bytes(&c) / 2u;
    if ((st = vx_alloc(ctx, Hd * f, &e->base_input)) || (st = vx_alloc(ctx, Hd * f, &e->current_embed)) ||
        (st = vx_alloc(ctx, Hd * f, &e->zero_embed)) || (st = vx_alloc(ctx, L * f, &e->fsq_latent)) ||
        (st = vx_alloc(ctx, Hd * f, &e->fsq_output)) || (st = vx_alloc(ctx, Hd * f, &e->current_lm)) ||
        (st = vx_alloc(ctx, Hd * f, &e->hidden)) || (st = vx_alloc(ctx, Hd * f, &e->fusion_snapshot)) ||
        (st = vx_alloc(ctx, Hd * f, &e->norm)) || (st = vx_alloc(ctx, Hd * f, &e->q)) ||
        (st = vx_alloc(ctx, KV * f, &e->k)) || (st = vx_alloc(ctx, KV * f, &e->v)) ||
        (st = vx_alloc(ctx, Hd * f, &e->attention)) || (st = vx_alloc(ctx, FF * f, &e->gate)) ||
        (st = vx_alloc(ctx, Hd * f, &e->branch)) ||
        (st = vx_alloc(ctx, (uint64_t)c.head_count * c.active_context_length * f, &e->scores)) ||
        (st = vx_alloc(ctx, cache, &e->kv_k)) || (st = vx_alloc(ctx, cache, &e->kv_v)) ||
        (st = vx_alloc(ctx, Hd * f, &e->stop_hidden)) || (st = vx_alloc(ctx, 2 * f, &e->stop_logits)) ||
        (st = vx_alloc(ctx, 256, &e->position)) ||
        (st = vx_alloc(ctx, attn_scratch_bytes(c.head_dim, c.head_count, c.head_count_kv, e->splits),
                       &e->attn_scratch)))
        return bail(st);
    // Zero state once, outside any graph (zero_embed is the text-prefix right half).
    vx_buf *zero[] = {e->zero_embed, e->hidden,   e->norm,     e->kv_k,         e->kv_v,
                      e->position,   e->current_lm, e->fsq_output, e->attn_scratch, e->stop_logits};
    for (vx_buf *b : zero)
        if (hipMemsetAsync(b->ptr, 0, b->bytes, ctx->stream) != hipSuccess)
            return bail(fail(VX_ERR_HIP, "hipMemsetAsync of engine state failed"));
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return bail(fail(VX_ERR_HIP, "engine init sync failed"));
    *out = e;
    return VX_OK;
}

int vx_residual_destroy(vx_residual *e) {
    if (!e) return VX_OK;
    (void)hipStreamSynchronize(e->ctx->stream);
    free_all(e);
    delete e;
    return VX_OK;
}

uint32_t vx_residual_position(const vx_residual *e) { return e ? e->pos : 0u; }

int vx_residual_reset(vx_residual *e) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_residual_reset: null engine");
    e->pos = 0;
    return VX_OK;
}

uint64_t vx_residual_allocated_bytes(const vx_residual *e) {
    if (!e) return 0;
    uint64_t total = vx_model_device_bytes(e->model);
    const vx_buf *bufs[] = {e->base_input, e->current_embed, e->zero_embed, e->fsq_latent, e->fsq_output,
                            e->current_lm, e->hidden,        e->fusion_snapshot, e->norm,  e->q,
                            e->k,          e->v,             e->attention, e->gate,        e->branch,
                            e->scores,     e->kv_k,          e->kv_v,      e->stop_hidden, e->stop_logits,
                            e->position,   e->attn_scratch};
    for (const vx_buf *b : bufs) total += b ? b->bytes : 0u;
    return total;
}

vx_buf *vx_residual_buffer(vx_residual *e, uint32_t which) {
    if (!e) return nullptr;
    switch (which) {
        case VX_RESIDUAL_BUF_OUTPUT: return e->norm;
        case VX_RESIDUAL_BUF_CURRENT_LM: return e->current_lm;
        case VX_RESIDUAL_BUF_FSQ_LATENT: return e->fsq_latent;
        case VX_RESIDUAL_BUF_FSQ_OUTPUT: return e->fsq_output;
        case VX_RESIDUAL_BUF_FUSION_SNAPSHOT: return e->fusion_snapshot;
        case VX_RESIDUAL_BUF_HIDDEN: return e->hidden;
        case VX_RESIDUAL_BUF_KV_K: return e->kv_k;
        case VX_RESIDUAL_BUF_KV_V: return e->kv_v;
        case VX_RESIDUAL_BUF_STOP_LOGITS: return e->stop_logits;
        default: return nullptr;
    }
}

int vx_residual_fsq_only(vx_residual *e, const float *base_hidden, uint32_t n, vx_fsq_result *out) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_residual_fsq_only: null engine");
    VX_CHECK(check_cancel(e->ctx));
    VX_CHECK(check_host(e, base_hidden, n, "FSQ input"));
    VX_CHECK(upload_host(e, e->base_input, base_hidden));
    const double t0 = now_ms();
    VX_CHECK(enqueue_fsq(e, F(e->base_input), nullptr));
    VX_CHECK(vx_sync(e->ctx));
    const double elapsed = now_ms() - t0;
    if (!out) return VX_OK;
    vx_fsq_result r{};
    r.elapsed_ms = elapsed;
    VX_CHECK(download_stats(e, e->fsq_latent, e->cfg.fsq_latent_dim, &r.latent_checksum, &r.latent_l2));
    VX_CHECK(download_stats(e, e->fsq_output, e->cfg.embedding_length, &r.output_checksum, &r.output_l2));
    *out = r;
    return VX_OK;
}

int vx_residual_step(vx_residual *e, const float *base_hidden, const float *current_embedding, uint32_t n,
                     vx_residual_step_result *out) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_residual_step: null engine");
    VX_CHECK(check_host(e, base_hidden, n, "ResidualLM base hidden"));
    VX_CHECK(check_host(e, current_embedding, n, "ResidualLM current embedding"));
    VX_CHECK(upload_host(e, e->base_input, base_hidden));
    VX_CHECK(upload_host(e, e->current_embed, current_embedding));
    return submit_step(e, true, F(e->base_input), F(e->current_embed), out);
}

int vx_residual_step_from_gpu_base(vx_residual *e, const vx_buf *base_hidden, const float *current_embedding,
                                   uint32_t n, vx_residual_step_result *out) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_residual_step_from_gpu_base: null engine");
    VX_CHECK(check_host(e, current_embedding, n, "ResidualLM current embedding"));
    VX_CHECK(check_gpu(e, base_hidden, "GPU BaseLM output buffer"));
    VX_CHECK(upload_host(e, e->current_embed, current_embedding));
    return submit_step(e, true, F(base_hidden), F(e->current_embed), out);
}

int vx_residual_step_from_gpu_base_and_embedding(vx_residual *e, const vx_buf *base_hidden,
                                                 const vx_buf *current_embedding, vx_residual_step_result *out) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_residual_step_from_gpu_base_and_embedding: null engine");
    VX_CHECK(check_gpu(e, base_hidden, "GPU BaseLM buffer"));
    VX_CHECK(check_gpu(e, current_embedding, "GPU current-embedding buffer"));
    return submit_step(e, true, F(base_hidden), F(current_embedding), out);
}

int vx_residual_step_from_gpu_base_and_embedding_gpu_only(vx_residual *e, const vx_buf *base_hidden,
                                                          const vx_buf *current_embedding,
                                                          vx_residual_gpu_step *out) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_residual_step_from_gpu_base_and_embedding_gpu_only: null engine");
    VX_CHECK(check_gpu(e, base_hidden, "GPU BaseLM buffer"));
    VX_CHECK(check_gpu(e, current_embedding, "GPU current-embedding buffer"));
    return submit_step_gpu_only(e, true, F(base_hidden), F(current_embedding), out);
}

int vx_residual_step_text_prefix_from_gpu_base(vx_residual *e, const vx_buf *base_hidden,
                                               vx_residual_step_result *out) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_residual_step_text_prefix_from_gpu_base: null engine");
    VX_CHECK(check_gpu(e, base_hidden, "GPU BaseLM output buffer"));
    return submit_step(e, false, F(base_hidden), F(e->zero_embed), out);
}

int vx_residual_step_text_prefix_from_gpu_base_gpu_only(vx_residual *e, const vx_buf *base_hidden,
                                                        vx_residual_gpu_step *out) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_residual_step_text_prefix_from_gpu_base_gpu_only: null engine");
    VX_CHECK(check_gpu(e, base_hidden, "GPU BaseLM output buffer"));
    return submit_step_gpu_only(e, false, F(base_hidden), F(e->zero_embed), out);
}

int vx_residual_benchmark(vx_residual *e, const float *base_hidden, const float *current_embedding, uint32_t n,
                          uint32_t warmup, uint32_t iterations, vx_residual_benchmark_result *out) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_residual_benchmark: null engine");
    if (iterations == 0) return fail(VX_ERR_INVALID_ARG, "benchmark iterations must be > 0");
    if ((uint64_t)warmup + iterations > e->cfg.active_context_length)
        return fail(VX_ERR_CONTEXT_FULL, "ResidualLM benchmark exceeds --max-context");
    e->pos = 0;
    vx_residual_step_result r{};
    for (uint32_t i = 0; i < warmup; ++i) VX_CHECK(vx_residual_step(e, base_hidden, current_embedding, n, &r));
    double sum = 0.0, mn = INFINITY, mx = 0.0;
    for (uint32_t i = 0; i < iterations; ++i) {
        VX_CHECK(vx_residual_step(e, base_hidden, current_embedding, n, &r));
        sum += r.elapsed_ms;
        mn = std::min(mn, r.elapsed_ms);
        mx = std::max(mx, r.elapsed_ms);
    }
    if (out) {
        out->iterations = iterations;
        out->mean_ms = sum / iterations;
        out->min_ms = mn;
        out->max_ms = mx;
        out->steps_per_second = 1000.0 / out->mean_ms;
    }
    return VX_OK;
}

int vx_residual_predict_stop_from_gpu_base(vx_residual *e, const vx_buf *base_hidden, vx_stop_prediction *out) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_residual_predict_stop_from_gpu_base: null engine");
    if (!base_hidden || base_hidden->bytes < (uint64_t)e->cfg.embedding_length * 4u)
        return fail(VX_ERR_BOUNDS, "GPU BaseLM hidden is too small for stop predictor");
    return predict_stop(e, F(base_hidden), out);
}

int vx_residual_predict_stop_from_current_lm(vx_residual *e, vx_stop_prediction *out) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_residual_predict_stop_from_current_lm: null engine");
    return predict_stop(e, F(e->current_lm), out);
}

int vx_fsq_quantize(vx_ctx *ctx, vx_buf *latent, const vx_fsq_push *pc) {
    if (!ctx || !pc) return fail(VX_ERR_INVALID_ARG, "vx_fsq_quantize: null argument");
    VX_CHECK(need_buf(latent, (uint64_t)pc->n * 4u, "vx_fsq_quantize latent"));
    ProfSpan sp(ctx, "residual.fsq_quantize");
    return launch_fsq_quantize(ctx->stream, F(latent), pc->n, pc->scale);
}

}  // extern "C"
