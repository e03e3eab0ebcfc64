// LocDiT estimator and the UnifiedCFM solve (LocalEngine, local.rs:264-537) over
// HIP, plus the per-op entry points of the CFM shaders.
//
// One estimator pass (record_locdit_common + record_locdit_body,
// local.rs:445-468):
//   x tokens    = in_proj(x patch) + b          [patch][hidden]
//   cond tokens = cond_proj(cond patch) + b     [patch][hidden] (or given rows)
//   time token  = time_mlp(sin(t)) + delta_time_mlp(sin(dt))
//   hidden      = [mu tokens | time | cond tokens | x tokens]   (pack_locdit)
//   transformer: rmsnorm, per layer q/k/v -> RoPE (position = token index) ->
//                dense attention -> attn_output -> residual rmsnorm -> SwiGLU ->
//                down -> residual rmsnorm (record_transformer, local.rs:482-527)
//   out         = out_proj(norm of the x tokens) + b  [patch][feat]
// The solve (cfm_solve, local.rs:383-430) runs the conditional and the
// unconditional pass of every Euler step as ONE batch of two sequences: the
// projections see 2 x tokens rows (each weight is streamed once per step, not
// twice), the attention stays per sequence, and the CFG-Zero* update reads both
// outputs. The whole solve is captured as one hipGraph and replayed while the
// options are unchanged; the noise seed is read from device memory.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <string>

#include "vx_internal.h"

using namespace vx;

namespace {

struct LocLayer {
    WRef q, k, v, o, gate, up, down;
    const float *attn_norm = nullptr, *ffn_norm = nullptr;
    // The same matrices in the fragment layout (frag16_index), for the short-batch
    // layer stack: q, k, v, o, gate, up, down.
    const __half *frag[7] = {};
};

struct Lin {
    WRef w;
    const void *b = nullptr;
    uint32_t bt = 0;
};

inline float *F(vx_buf *b) { return static_cast<float *>(b->ptr); }

}  // namespace

struct vx_locdit {
    vx_ctx *ctx = nullptr;
    const vx_model *model = nullptr;
    vx_locdit_config cfg{};
    uint32_t S = 0;   // tokens per sequence
    bool dense_fused = false;   // attention of a sequence fits the one-kernel path
    Lin in_proj, cond_proj, out_proj, t1, t2, d1, d2;
    // projections.lm_to_dit_proj / res_to_dit_proj (local.rs:141-144): the mu
    // tokens from the ResidualLM engine's current_lm and output buffers.
    Lin lm_to_dit, res_to_dit;
    bool has_mu_proj = false;
    uint32_t lm_hidden = 0;   // their input width (the BaseLM embedding length)
    const float *norm_w = nullptr, *rope_factors = nullptr;
    std::vector<LocLayer> layers;
    // State and activations (two sequences: conditional, unconditional).
    vx_buf *x = nullptr, *cond_in = nullptr, *mu = nullptr, *patch_proj = nullptr, *cond_proj_out = nullptr;
    vx_buf *tsin = nullptr, *ttmp = nullptr, *tvec = nullptr, *dsin = nullptr, *dtmp = nullptr, *dvec = nullptr;
    vx_buf *hidden = nullptr, *norm = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr;
    vx_buf *gate = nullptr, *branch = nullptr, *scores = nullptr, *out = nullptr, *seed = nullptr;
    vx_buf *rope_tab = nullptr;   // (cos, sin) per position of a sequence, for the fused attention
    // Short-batch layer stack (the CFG batch fits the short-batch GEMM): normed
    // activations, attention output and SwiGLU output as hi/lo f16 planes, and
    // the split-K partial slabs of attn_output and ffn_down, summed by the
    // residual rmsnorm that follows each.
    bool sk = false;
    // The attention kernel also applies the O projection (one partial slab per
    // query head) in place of a separate attn_output GEMM.
    bool attn_oproj = false;
    // A solve step's out_proj and CFG-Zero* Euler update run as one launch;
    // out_ctr is its completion counter (zero between launches).
    bool out_euler = false;
    vx_buf *out_ctr = nullptr;
    uint32_t ks_qkv = 1, ks_o = 1, ks_down = 1;
    vx_buf *qkvp = nullptr;   // q | k | v rows of each of ks_qkv partial slabs
    vx_buf *yh = nullptr, *yl = nullptr, *ah = nullptr, *al = nullptr, *acth = nullptr, *actl = nullptr;
    vx_buf *part = nullptr;
    vx_buf *wfrag = nullptr;   // every layer's matrices in the fragment layout
    // The residual stream as f32 in the fragment order (frag32_index), with both
    // rmsnorms of a layer folded into the projections that read it (QKV, gate/up)
    // and the attention/O and ffn_down products added to it atomically: four
    // launches per layer instead of six. ssq: the QKV K slabs' row sums of squares.
    bool fold_norm = false;
    vx_buf *hres = nullptr, *ssq = nullptr;
    // Time embeddings of every estimator call of a solve, computed as one batch:
    // t values, sinusoid rows, MLP hidden rows, embeddings ([steps][hidden]).
    vx_buf *tvals = nullptr, *trows = nullptr, *tmid = nullptr, *temb = nullptr;
    uint32_t trows_cap = 0;
    vx_graph *graph = nullptr;
    vx_cfm_options graph_opt{};
    // temb holds the time rows of these options (set by the last eager
    // computation); the cached graph reads them and does not recompute them.
    bool temb_ready = false;
    vx_cfm_options temb_opt{};
    int graph_initial_x = -1;
    const float *graph_mu_src[2] = {nullptr, nullptr};   // model-hidden sources the graph projects, or null
};

namespace {

int find(const vx_model *m, const std::string &name, const vx_tensor_info **out) {
    auto it = m->by_name.find(name);
    if (it == m->by_name.end())
        return fail(VX_ERR_NOT_FOUND, "required GGUF tensor \"%s\" is missing", name.c_str());
    *out = &m->tensors[it->second];
    return VX_OK;
}

// require_matrix (local.rs:170-174): dims [cols, rows], F16.
int matrix(const vx_model *m, const std::string &name, uint32_t cols, uint32_t rows, WRef *w) {
    const vx_tensor_info *t;
    VX_CHECK(find(m, name, &t));
    if (t->n_dims != 2 || t->dims[0] != cols || t->dims[1] != rows)
        return fail(VX_ERR_SHAPE, "%s has dimensions [%llu, %llu], expected [%u, %u]", name.c_str(),
                    (unsigned long long)t->dims[0], (unsigned long long)(t->n_dims > 1 ? t->dims[1] : 1), cols,
                    rows);
    if (t->ggml_type != VX_DTYPE_F16)
        return fail(VX_ERR_SHAPE, "%s is type %u, expected F16 acoustic weight", name.c_str(), t->ggml_type);
    return resolve_matrix(m, (uint32_t)t->offset, VX_DTYPE_F16, rows, cols, w, name.c_str());
}

// require_vector (local.rs:175-180).
int vector(const vx_model *m, const std::string &name, uint32_t n, bool f32_only, const void **p, uint32_t *dtype) {
    const vx_tensor_info *t;
    VX_CHECK(find(m, name, &t));
    if (t->n_dims != 1 || t->dims[0] != n)
        return fail(VX_ERR_SHAPE, "%s has dimensions [%llu], expected [%u]", name.c_str(),
                    (unsigned long long)t->dims[0], n);
    if (f32_only && t->ggml_type != VX_DTYPE_F32)
        return fail(VX_ERR_SHAPE, "%s is type %u, expected F32 norm", name.c_str(), t->ggml_type);
    if (t->ggml_type != VX_DTYPE_F32 && t->ggml_type != VX_DTYPE_F16)
        return fail(VX_ERR_SHAPE, "%s has unsupported type %u", name.c_str(), t->ggml_type);
    if (dtype) *dtype = t->ggml_type == VX_DTYPE_F32 ? 0u : 1u;
    return resolve_vector(m, (uint32_t)t->offset, t->ggml_type, n, p, name.c_str());
}

int linear(const vx_model *m, const std::string &prefix, uint32_t cols, uint32_t rows, Lin *l) {
    VX_CHECK(matrix(m, prefix + ".weight", cols, rows, &l->w));
    return vector(m, prefix + ".bias", rows, false, &l->b, &l->bt);
}

int validate(const vx_locdit_config &c, bool strict) {
    if (!c.hidden || !c.layers || !c.q_heads || !c.kv_heads || !c.head_dim || !c.ffn || !c.feat_dim || !c.patch)
        return fail(VX_ERR_INVALID_ARG, "LocDiT config has a zero dimension");
    if (c.n_mu > 2) return fail(VX_ERR_UNSUPPORTED, "LocDiT takes at most two mu tokens");
    if (!c.cond_raw && c.n_cond != c.patch)
        return fail(VX_ERR_SHAPE, "projected condition has patch=%u tokens, config says %u", c.patch, c.n_cond);
    if (c.q_heads % c.kv_heads) return fail(VX_ERR_SHAPE, "q_heads %u not a multiple of kv_heads %u", c.q_heads, c.kv_heads);
    if (c.head_dim > 128u || (c.head_dim & 1u)) return fail(VX_ERR_UNSUPPORTED, "head_dim %u (even, <= 128)", c.head_dim);
    if (strict && (c.hidden != 1024u || c.layers != 12u || c.q_heads != 16u || c.kv_heads != 2u || c.head_dim != 128u ||
                   c.ffn != 4096u || c.patch != 4u || c.feat_dim != 64u || c.n_mu != 2u || c.cond_raw))
        // LocalConfig::from_gguf (local.rs:85-92) and the 16q/2kv x 128 geometry check.
        return fail(VX_ERR_UNSUPPORTED,
                    "unsupported VoxCPM2 local contract: LocDiT=%ux%u, heads %u/%u x %u, ffn %u, patch %u x %u; "
                    "expected 12x1024, 16/2 x 128, 4096, 4 x 64",
                    c.layers, c.hidden, c.q_heads, c.kv_heads, c.head_dim, c.ffn, c.patch, c.feat_dim);
    const uint64_t S = (uint64_t)c.n_mu + 1u + c.n_cond + c.patch;
    if (S > 4096u) return fail(VX_ERR_UNSUPPORTED, "LocDiT sequence of %llu tokens", (unsigned long long)S);
    return VX_OK;
}

void free_all(vx_locdit *e) {
    if (e->graph) {
        vx_graph_free(e->ctx, e->graph);
        e->graph = nullptr;
    }
    vx_buf **bufs[] = {&e->x,      &e->cond_in, &e->mu,   &e->patch_proj, &e->cond_proj_out, &e->tsin,
                       &e->ttmp,   &e->tvec,    &e->dsin, &e->dtmp,       &e->dvec,          &e->hidden,
                       &e->norm,   &e->q,       &e->k,    &e->v,          &e->attn,          &e->gate,
                       &e->branch, &e->scores,  &e->out,  &e->seed,       &e->rope_tab,
                       &e->tvals,  &e->trows,   &e->tmid, &e->temb,       &e->yh,            &e->yl,
                       &e->ah,     &e->al,      &e->acth, &e->actl,       &e->part,          &e->wfrag,
                       &e->qkvp,   &e->out_ctr, &e->hres, &e->ssq};
    for (vx_buf **b : bufs) {
        vx_free(e->ctx, *b);
        *b = nullptr;
    }
}

// Time embedding (record_time, local.rs:470-480): tvec = time_mlp(sin(t)) +
// delta_time_mlp(sin(dt)), each MLP linear -> SiLU -> linear.
int enqueue_time(vx_locdit *e, float t, float dt) {
    hipStream_t s = e->ctx->stream;
    const uint32_t H = e->cfg.hidden;
    ProfSpan sp(e->ctx, "local.time");
    VX_CHECK(launch_time_sinusoidal(s, F(e->tsin), H, t, nullptr, 0));
    VX_CHECK(launch_time_sinusoidal(s, F(e->dsin), H, dt, nullptr, 0));
    VX_CHECK(enqueue_seq_linear(s, e->t1.w, e->t1.b, e->t1.bt, H, H, 1, F(e->tsin), 0, H, F(e->ttmp), 0, H, 1.f));
    VX_CHECK(enqueue_seq_linear(s, e->d1.w, e->d1.b, e->d1.bt, H, H, 1, F(e->dsin), 0, H, F(e->dtmp), 0, H, 1.f));
    VX_CHECK(launch_silu_inplace(s, F(e->ttmp), H));
    VX_CHECK(launch_silu_inplace(s, F(e->dtmp), H));
    VX_CHECK(enqueue_seq_linear(s, e->t2.w, e->t2.b, e->t2.bt, H, H, 1, F(e->ttmp), 0, H, F(e->tvec), 0, H, 1.f));
    VX_CHECK(enqueue_seq_linear(s, e->d2.w, e->d2.b, e->d2.bt, H, H, 1, F(e->dtmp), 0, H, F(e->dvec), 0, H, 1.f));
    return launch_add_vectors(s, F(e->tvec), F(e->dvec), H);
}

// record_time for the n estimator calls of a solve at once: row i of temb is
// time_mlp(sin(t_i)) + delta_time_mlp(sin(0)) (the solve's estimator dt is zero),
// t_i read from the device t values.
int enqueue_time_rows(vx_locdit *e, uint32_t n) {
    hipStream_t s = e->ctx->stream;
    const uint32_t H = e->cfg.hidden;
    ProfSpan sp(e->ctx, "local.time");
    VX_CHECK(launch_time_sinusoidal(s, F(e->trows), H, 0.0f, static_cast<const float *>(e->tvals->ptr), 0, n));
    VX_CHECK(enqueue_seq_linear(s, e->t1.w, e->t1.b, e->t1.bt, H, H, n, F(e->trows), 0, H, F(e->tmid), 0, H, 1.f));
    VX_CHECK(launch_silu_inplace(s, F(e->tmid), n * H));
    VX_CHECK(enqueue_seq_linear(s, e->t2.w, e->t2.b, e->t2.bt, H, H, n, F(e->tmid), 0, H, F(e->temb), 0, H, 1.f));
    VX_CHECK(launch_time_sinusoidal(s, F(e->dsin), H, 0.0f, nullptr, 0));
    VX_CHECK(enqueue_seq_linear(s, e->d1.w, e->d1.b, e->d1.bt, H, H, 1, F(e->dsin), 0, H, F(e->dtmp), 0, H, 1.f));
    VX_CHECK(launch_silu_inplace(s, F(e->dtmp), H));
    VX_CHECK(enqueue_seq_linear(s, e->d2.w, e->d2.b, e->d2.bt, H, H, 1, F(e->dtmp), 0, H, F(e->dvec), 0, H, 1.f));
    return launch_add_vectors(s, F(e->temb), F(e->dvec), H, n);
}

// in_proj / cond_proj (record_locdit_common, local.rs:445-449). The short-batch
// stack computes in_proj inside the pack instead (enqueue_body).
int enqueue_inputs(vx_locdit *e) {
    hipStream_t s = e->ctx->stream;
    const vx_locdit_config &c = e->cfg;
    ProfSpan sp(e->ctx, "local.locdit_in");
    if (!e->sk)
        VX_CHECK(enqueue_seq_linear(s, e->in_proj.w, e->in_proj.b, e->in_proj.bt, c.hidden, c.feat_dim, c.patch,
                                    F(e->x), 0, c.feat_dim, F(e->patch_proj), 0, c.hidden, 1.f));
    if (!c.cond_raw)
        VX_CHECK(enqueue_seq_linear(s, e->cond_proj.w, e->cond_proj.b, e->cond_proj.bt, c.hidden, c.feat_dim, c.patch,
                                    F(e->cond_in), 0, c.feat_dim, F(e->cond_proj_out), 0, c.hidden, 1.f));
    return VX_OK;
}

// record_transformer (local.rs:482-527) with the general kernels: k_gemm
// projections (split K by atomic adds into accumulators that the rmsnorm kernels
// clear), the fused or three-kernel dense attention, and separate residual
// rmsnorms.
int enqueue_layers_general(vx_locdit *e, uint32_t batch) {
    vx_ctx *ctx = e->ctx;
    hipStream_t s = ctx->stream;
    const vx_locdit_config &c = e->cfg;
    const uint32_t H = c.hidden, S = e->S, M = S * batch;
    const uint32_t QD = c.q_heads * c.head_dim, KD = c.kv_heads * c.head_dim;
    // Split-K projections add into outputs that the rmsnorm kernels clear on the
    // way: the first norm clears q, k, v and the branch; the residual norm after
    // attn_out clears the branch (the down projection's accumulator) once it has
    // read it, and the one after down clears the branch and the next layer's q, k, v.
    SeqNormArgs n;
    n.h = F(e->hidden);
    n.ldh = H;
    n.w = e->layers[0].attn_norm;
    n.n = H;
    n.eps = c.rms_epsilon;
    n.y = F(e->norm);
    n.ldy = H;
    n.zero[0] = F(e->q);
    n.zero_n[0] = QD;
    n.zero[1] = F(e->k);
    n.zero_n[1] = KD;
    n.zero[2] = F(e->v);
    n.zero_n[2] = KD;
    n.zero[3] = F(e->branch);
    n.zero_n[3] = H;
    {
        ProfSpan sp(ctx, "local.seq_rmsnorm");
        VX_CHECK(launch_seq_rmsnorm(s, n, M));
    }
    for (uint32_t l = 0; l < c.layers; ++l) {
        const LocLayer &L = e->layers[l];
        {
            ProfSpan sp(ctx, "local.seq_qkv");
            const WRef w[3] = {L.q, L.k, L.v};
            const uint32_t rows[3] = {QD, KD, KD}, strides[3] = {QD, KD, KD};
            float *const o[3] = {F(e->q), F(e->k), F(e->v)};
            VX_CHECK(enqueue_seq_qkv(s, w, rows, H, M, F(e->norm), 0, H, o, strides, true));
        }
        if (!e->dense_fused) {
            ProfSpan sp(ctx, "local.seq_rope");
            SeqRopeArgs r;
            r.q = F(e->q);
            r.k = F(e->k);
            r.ldq = QD;
            r.ldk = KD;
            r.factors = e->rope_factors;
            r.q_heads = c.q_heads;
            r.kv_heads = c.kv_heads;
            r.head_dim = c.head_dim;
            r.pos_period = S;   // seq_rope.comp:8: position = token index within the sequence
            r.theta = c.rope_theta;
            r.scaling = c.rope_scaling;
            VX_CHECK(launch_seq_rope_store(s, r, M));
        }
        {
            ProfSpan sp(ctx, "local.attention");
            DenseAttnArgs a;
            a.q = F(e->q);
            a.k = F(e->k);
            a.v = F(e->v);
            a.s = F(e->scores);
            a.out = F(e->attn);
            a.tokens = S;
            a.q_heads = c.q_heads;
            a.kv_heads = c.kv_heads;
            a.head_dim = c.head_dim;
            a.q_stride = QD;
            a.k_stride = KD;
            a.v_stride = KD;
            a.out_stride = QD;
            a.score_stride = S;
            a.batch = batch;
            if (e->dense_fused) {
                a.rope = reinterpret_cast<const float2 *>(e->rope_tab->ptr);   // RoPE applied while staging q, k
                VX_CHECK(launch_dense_attn_fused(s, a));
            } else {
                VX_CHECK(launch_dense_attn(s, a, 0));
                VX_CHECK(launch_dense_attn(s, a, 1));
                VX_CHECK(launch_dense_attn(s, a, 2));
            }
        }
        {
            ProfSpan sp(ctx, "local.seq_linear");
            VX_CHECK(
                enqueue_seq_linear(s, L.o, nullptr, 0, H, QD, M, F(e->attn), 0, QD, F(e->branch), 0, H, 1.f, true));
        }
        SeqNormArgs r;
        r.h = F(e->hidden);
        r.ldh = H;
        r.branch = F(e->branch);
        r.ldb = H;
        r.scale = 1.f;
        r.n = H;
        r.eps = c.rms_epsilon;
        r.y = F(e->norm);
        r.ldy = H;
        r.clear_branch = 1;
        {
            ProfSpan sp(ctx, "local.seq_residual_rmsnorm");
            r.w = L.ffn_norm;
            VX_CHECK(launch_seq_rmsnorm(s, r, M));
        }
        {
            ProfSpan sp(ctx, "local.seq_swiglu");
            VX_CHECK(enqueue_seq_swiglu(s, L.gate, L.up, c.ffn, H, M, F(e->norm), 0, H, F(e->gate), 0, c.ffn));
        }
        {
            ProfSpan sp(ctx, "local.seq_linear");
            VX_CHECK(enqueue_seq_linear(s, L.down, nullptr, 0, H, c.ffn, M, F(e->gate), 0, c.ffn, F(e->branch), 0, H,
                                        1.f, true));
        }
        {
            ProfSpan sp(ctx, "local.seq_residual_rmsnorm");
            r.w = l + 1 < c.layers ? e->layers[l + 1].attn_norm : e->norm_w;
            for (int z = 0; z < 3; ++z) {
                r.zero[z] = n.zero[z];
                r.zero_n[z] = n.zero_n[z];
            }
            VX_CHECK(launch_seq_rmsnorm(s, r, M));
            for (int z = 0; z < 3; ++z) r.zero[z] = nullptr;
        }
    }
    return VX_OK;
}

constexpr uint64_t kFoldNormMaxRows = 32;   // CFG batch rows up to which fold_norm is chosen

// record_transformer (local.rs:482-527) on the residual stream (fold_norm): four
// launches per layer, the rmsnorms folded into the projections that read h.
//   h (rows) -> the residual stream hres (frag32 order)        (once per pass)
//   per layer:
//     q|k|v slabs = (hres * attn_norm) . Wq|Wk|Wv, each K slab's row sums of
//       squares to ssq                                          (k_gemm_sk, XN)
//     attention over q, k, v scaled by 1/rms (RoPE while staging),
//       hres += O projection, atomic adds                      (k_dense_attn_fused, RES)
//     act = silu(g / rms) * (u / rms), g|u = (hres * ffn_norm) . Wg|Wu
//                                                              (k_gemm_sk, XN, SwiGLU)
//     hres += act . Wdown, atomic adds from every K slab       (k_gemm_sk, res_frag)
//   norm = rmsnorm(hres) * locdit.norm, f32 rows for out_proj   (once per pass)
// The fp32 atomic additions make the order of a residual row's sums vary from
// run to run (results agree to rounding, not bit for bit).
// The pack wrote the stream (hres) itself. final_norm false: the caller's
// out_proj + Euler launch folds the final rmsnorm in (CfmOutEulerArgs::rows_frag).
int enqueue_layers_residual(vx_locdit *e, uint32_t batch, bool final_norm) {
    vx_ctx *ctx = e->ctx;
    hipStream_t s = ctx->stream;
    const vx_locdit_config &c = e->cfg;
    const uint32_t H = c.hidden, S = e->S, M = S * batch;
    const uint32_t QD = c.q_heads * c.head_dim, KD = c.kv_heads * c.head_dim;
    const uint64_t R16 = ((uint64_t)2u * S + 15u) & ~15ull;   // rows of the stream, as allocated
    float *hres = F(e->hres), *ssq = F(e->ssq);
    __half *acth = static_cast<__half *>(e->acth->ptr), *actl = static_cast<__half *>(e->actl->ptr);
    auto wseg = [](const __half *w, uint32_t rows, float *out, uint32_t ldo) {
        GemmSeg g;
        g.w = w;
        g.rows = rows;
        g.out = out;
        g.ldo = ldo;
        return g;
    };
    auto gemm = [&](uint32_t K) {
        GemmArgs g;
        g.wk = WT_F16;
        g.epi = GEPI_STORE;
        g.ldx = K;
        g.K = K;
        g.T = M;
        g.frag = 1;
        return g;
    };
    for (uint32_t l = 0; l < c.layers; ++l) {
        const LocLayer &L = e->layers[l];
        float *qp = F(e->qkvp), *kp = qp + (size_t)M * QD, *vp = kp + (size_t)M * KD;
        const uint64_t qkv_slab = (uint64_t)M * (QD + 2u * KD);
        {
            ProfSpan sp(ctx, "local.seq_qkv");
            GemmArgs g = gemm(H);
            g.xn = hres;
            g.xn_w = L.attn_norm;
            g.xn_eps = c.rms_epsilon;
            g.xn_ss = ssq;
            g.xn_ss_stride = R16;
            g.seg[0] = wseg(L.frag[0], QD, qp, QD);
            g.seg[1] = wseg(L.frag[1], KD, kp, KD);
            g.seg[2] = wseg(L.frag[2], KD, vp, KD);
            g.nseg = 3;
            g.ksplit = e->ks_qkv;
            g.split_store = 1;
            g.ws_stride = qkv_slab;
            VX_CHECK(launch_gemm(s, g));
        }
        {
            ProfSpan sp(ctx, "local.attention_oproj");
            DenseAttnArgs a;
            a.q = qp;
            a.k = kp;
            a.v = vp;
            a.nslab = e->ks_qkv;
            a.slab_stride = qkv_slab;
            a.tokens = S;
            a.q_heads = c.q_heads;
            a.kv_heads = c.kv_heads;
            a.head_dim = c.head_dim;
            a.q_stride = QD;
            a.k_stride = KD;
            a.v_stride = KD;
            a.out_stride = QD;
            a.score_stride = S;
            a.batch = batch;
            a.rope = reinterpret_cast<const float2 *>(e->rope_tab->ptr);
            a.wo = L.frag[3];
            a.hidden = H;
            a.hres = hres;
            a.ssq = ssq;
            a.ssq_stride = R16;
            a.norm_n = H;
            a.eps = c.rms_epsilon;
            VX_CHECK(launch_dense_attn_oproj(s, a));
        }
        {
            ProfSpan sp(ctx, "local.seq_swiglu");
            GemmArgs g = gemm(H);
            g.epi = GEPI_SWIGLU;
            g.xn = hres;
            g.xn_w = L.ffn_norm;
            g.xn_eps = c.rms_epsilon;
            g.seg[0] = wseg(L.frag[4], c.ffn, nullptr, 0);
            g.seg[1] = wseg(L.frag[5], c.ffn, nullptr, 0);
            g.nseg = 2;
            g.oh = acth;
            g.ol = actl;
            VX_CHECK(launch_gemm(s, g));
        }
        {
            ProfSpan sp(ctx, "local.seq_linear");
            GemmArgs g = gemm(c.ffn);
            g.xh = acth;
            g.xl = actl;
            g.seg[0] = wseg(L.frag[6], H, nullptr, H);
            g.ksplit = e->ks_down;
            g.res_frag = hres;
            VX_CHECK(launch_gemm(s, g));
        }
    }
    if (!final_norm) return VX_OK;
    ProfSpan sp(ctx, "local.seq_rmsnorm");
    SeqNormArgs r;
    r.h = hres;
    r.h_frag = 1;
    r.ldh = H;
    r.n = H;
    r.eps = c.rms_epsilon;
    r.w = e->norm_w;
    r.y = F(e->norm);   // out_proj reads f32 rows
    r.ldy = H;
    return launch_seq_rmsnorm(s, r, M);
}

// record_transformer (local.rs:482-527) for a batch that fits the short-batch
// GEMM (kernels_skinny.hip), five kernels per sublayer pair and no cleared
// accumulators:
//   rmsnorm -> hi/lo planes y
//   q, k, v = y . Wq|Wk|Wv                       (one GEMM, plain stores)
//   fused dense attention (RoPE while staging)   -> hi/lo planes of the output
//   attn_output: K split into ks_o partial slabs (plain stores)
//   residual rmsnorm: h += sum of the slabs, y = norm(h) * ffn_norm -> planes
//   gate/up with the SwiGLU epilogue             -> hi/lo planes
//   ffn_down: K split into ks_down partial slabs
//   residual rmsnorm: h += sum of the slabs, y = norm(h) * next attn_norm -> planes
//     (after the last layer: * locdit.norm, f32 rows for out_proj)
int enqueue_layers_sk(vx_locdit *e, uint32_t batch) {
    vx_ctx *ctx = e->ctx;
    hipStream_t s = ctx->stream;
    const vx_locdit_config &c = e->cfg;
    const uint32_t H = c.hidden, S = e->S, M = S * batch;
    const uint32_t QD = c.q_heads * c.head_dim, KD = c.kv_heads * c.head_dim;
    __half *yh = static_cast<__half *>(e->yh->ptr), *yl = static_cast<__half *>(e->yl->ptr);
    __half *ah = static_cast<__half *>(e->ah->ptr), *al = static_cast<__half *>(e->al->ptr);
    __half *acth = static_cast<__half *>(e->acth->ptr), *actl = static_cast<__half *>(e->actl->ptr);
    float *part = F(e->part);
    auto wseg = [](const __half *w, uint32_t rows, float *out, uint32_t ldo) {
        GemmSeg g;
        g.w = w;
        g.rows = rows;
        g.out = out;
        g.ldo = ldo;
        return g;
    };
    auto gemm = [&](const __half *xh, const __half *xl, uint32_t K) {
        GemmArgs g;
        g.wk = WT_F16;
        g.epi = GEPI_STORE;
        g.xh = xh;
        g.xl = xl;
        g.ldx = K;
        g.K = K;
        g.T = M;
        g.frag = 1;
        return g;
    };
    SeqNormArgs n;
    n.h = F(e->hidden);
    n.ldh = H;
    n.w = e->layers[0].attn_norm;
    n.n = H;
    n.eps = c.rms_epsilon;
    n.yh = yh;
    n.yl = yl;
    n.tiled = 2;   // planes in the fragment layout
    {
        ProfSpan sp(ctx, "local.seq_rmsnorm");
        VX_CHECK(launch_seq_rmsnorm(s, n, M));
    }
    for (uint32_t l = 0; l < c.layers; ++l) {
        const LocLayer &L = e->layers[l];
        float *qp = F(e->qkvp), *kp = qp + (size_t)M * QD, *vp = kp + (size_t)M * KD;
        const uint64_t qkv_slab = (uint64_t)M * (QD + 2u * KD);
        {
            ProfSpan sp(ctx, "local.seq_qkv");
            GemmArgs g = gemm(yh, yl, H);
            g.seg[0] = wseg(L.frag[0], QD, qp, QD);
            g.seg[1] = wseg(L.frag[1], KD, kp, KD);
            g.seg[2] = wseg(L.frag[2], KD, vp, KD);
            g.nseg = 3;
            g.ksplit = e->ks_qkv;
            g.split_store = 1;
            g.ws_stride = qkv_slab;
            VX_CHECK(launch_gemm(s, g));
        }
        DenseAttnArgs a;
        a.q = qp;
        a.k = kp;
        a.v = vp;
        a.nslab = e->ks_qkv;
        a.slab_stride = qkv_slab;
        a.tokens = S;
        a.q_heads = c.q_heads;
        a.kv_heads = c.kv_heads;
        a.head_dim = c.head_dim;
        a.q_stride = QD;
        a.k_stride = KD;
        a.v_stride = KD;
        a.out_stride = QD;
        a.score_stride = S;
        a.batch = batch;
        a.rope = reinterpret_cast<const float2 *>(e->rope_tab->ptr);
        if (e->attn_oproj) {
            ProfSpan sp(ctx, "local.attention_oproj");
            a.wo = L.frag[3];
            a.hidden = H;
            a.oslab = part;
            a.oslab_stride = (uint64_t)M * H;
            VX_CHECK(launch_dense_attn_oproj(s, a));
        } else {
            {
                ProfSpan sp(ctx, "local.attention");
                a.out = F(e->attn);
                a.oh = ah;
                a.ol = al;
                a.o_frag = 1;
                VX_CHECK(launch_dense_attn_fused(s, a));
            }
            ProfSpan sp(ctx, "local.seq_linear");
            GemmArgs g = gemm(ah, al, QD);
            g.seg[0] = wseg(L.frag[3], H, part, H);
            g.ksplit = e->ks_o;
            g.split_store = 1;
            g.ws_stride = (uint64_t)M * H;
            VX_CHECK(launch_gemm(s, g));
        }
        SeqNormArgs r = n;
        r.branch = part;
        r.ldb = H;
        r.scale = 1.f;
        {
            ProfSpan sp(ctx, "local.seq_residual_rmsnorm");
            r.nbranch = e->attn_oproj ? c.q_heads : e->ks_o;
            r.branch_stride = (uint64_t)M * H;
            r.w = L.ffn_norm;
            VX_CHECK(launch_seq_rmsnorm(s, r, M));
        }
        {
            ProfSpan sp(ctx, "local.seq_swiglu");
            GemmArgs g = gemm(yh, yl, H);
            g.epi = GEPI_SWIGLU;
            g.seg[0] = wseg(L.frag[4], c.ffn, nullptr, 0);
            g.seg[1] = wseg(L.frag[5], c.ffn, nullptr, 0);
            g.nseg = 2;
            g.oh = acth;
            g.ol = actl;
            VX_CHECK(launch_gemm(s, g));
        }
        {
            ProfSpan sp(ctx, "local.seq_linear");
            GemmArgs g = gemm(acth, actl, c.ffn);
            g.seg[0] = wseg(L.frag[6], H, part, H);
            g.ksplit = e->ks_down;
            g.split_store = 1;
            g.ws_stride = (uint64_t)M * H;
            VX_CHECK(launch_gemm(s, g));
        }
        {
            ProfSpan sp(ctx, "local.seq_residual_rmsnorm");
            const bool last = l + 1 == c.layers;
            r.nbranch = e->ks_down;
            r.branch_stride = (uint64_t)M * H;
            r.w = last ? e->norm_w : e->layers[l + 1].attn_norm;
            if (last) {   // out_proj reads f32 rows
                r.y = F(e->norm);
                r.ldy = H;
                r.yh = r.yl = nullptr;
                r.tiled = 0;
            }
            VX_CHECK(launch_seq_rmsnorm(s, r, M));
        }
    }
    return VX_OK;
}

// pack_locdit + record_transformer + out_proj for `batch` sequences (1: the
// conditional pass; 2: conditional then unconditional).
int enqueue_body(vx_locdit *e, uint32_t batch, const float *time_row = nullptr, bool skip_out = false) {
    vx_ctx *ctx = e->ctx;
    hipStream_t s = ctx->stream;
    const vx_locdit_config &c = e->cfg;
    const uint32_t H = c.hidden, S = e->S;
    {
        ProfSpan sp(ctx, "local.pack_locdit");
        PackLocditArgs p;
        p.mu[0] = F(e->mu);
        p.mu[1] = F(e->mu) + H;
        p.time = time_row ? time_row : F(e->tvec);
        p.cond = c.cond_raw ? F(e->cond_in) : F(e->cond_proj_out);
        p.x = F(e->patch_proj);
        p.out = e->fold_norm ? F(e->hres) : F(e->hidden);
        p.out_frag = e->fold_norm ? 1u : 0u;   // the residual-stream stack's stream
        p.hidden = H;
        p.n_mu = c.n_mu;
        p.n_cond = c.n_cond;
        p.n_x = c.patch;
        p.batch = batch;
        p.zero_mu_mask = 0x2u;                               // the unconditional sequence (local.rs:413-421)
        p.zero_cond_mask = c.uncond_zero_cond ? 0x2u : 0u;
        if (e->sk) {   // x tokens = in_proj(x patch) + b, computed by the pack
            p.in_w = static_cast<const __half *>(e->in_proj.w.ptr);
            p.in_b = e->in_proj.b;
            p.in_bt = e->in_proj.bt;
            p.feat = c.feat_dim;
            p.xpatch = F(e->x);
        }
        VX_CHECK(launch_pack_locdit(s, p));
    }
    VX_CHECK(e->fold_norm ? enqueue_layers_residual(e, batch, !skip_out)
                          : e->sk ? enqueue_layers_sk(e, batch) : enqueue_layers_general(e, batch));
    if (skip_out) return VX_OK;   // the caller's launch applies out_proj
    ProfSpan sp(ctx, "local.locdit_out");
    const uint32_t x0 = c.n_mu + 1u + c.n_cond;   // first x token of a sequence
    for (uint32_t b = 0; b < batch; ++b)
        VX_CHECK(enqueue_seq_linear(s, e->out_proj.w, e->out_proj.b, e->out_proj.bt, c.feat_dim, H, c.patch,
                                    F(e->norm), (b * S + x0) * H, H, F(e->out), b * c.patch * c.feat_dim, c.feat_dim,
                                    1.f));
    return VX_OK;
}

// cfm_time_span (local.rs:531-537): t_i = 1 - i/n, w = t + sway (cos(pi t / 2) - 1 + t).
int time_span(uint32_t n, float sway, std::vector<float> &out) {
    if (n == 0) return fail(VX_ERR_INVALID_ARG, "CFM n_timesteps must be >= 1");
    out.clear();
    for (uint32_t i = 0; i <= n; ++i) {
        const float t = 1.0f - (float)i / (float)n;
        const float w = t + sway * (std::cos(1.57079632679489661923f * t) - 1.0f + t);
        if (!std::isfinite(w)) return fail(VX_ERR_INVALID_ARG, "non-finite CFM time grid at %u", i);
        out.push_back(w);
    }
    for (size_t i = 1; i < out.size(); ++i)
        if (out[i] > out[i - 1] + 1.0e-6f)
            return fail(VX_ERR_INVALID_ARG, "CFM sway schedule is not descending at %zu: %g -> %g", i, out[i - 1],
                        out[i]);
    return VX_OK;
}

int validate_options(const vx_cfm_options &o) {  // CfmOptions::validate (local.rs:262-268)
    if (o.n_timesteps == 0) return fail(VX_ERR_INVALID_ARG, "CFM n_timesteps must be >= 1");
    if (!std::isfinite(o.cfg_value) || !std::isfinite(o.temperature) || !std::isfinite(o.sway_sampling_coef))
        return fail(VX_ERR_INVALID_ARG, "CFM options must be finite");
    if (o.temperature < 0.0f) return fail(VX_ERR_INVALID_ARG, "CFM temperature must be >= 0");
    return VX_OK;
}

uint32_t zero_init_steps(const vx_cfm_options &o, size_t span_len) {
    return o.use_cfg_zero_star ? std::max<uint32_t>(1u, (uint32_t)std::floor((float)span_len * 0.04f)) : 0u;
}

// record_project_mu (local.rs:459-462): mu1 = lm_to_dit_proj . current_lm + b and
// mu2 = res_to_dit_proj . residual + b (seq_linear_bias with one token), written
// into the two mu tokens of the solve.
int enqueue_project_mu(vx_locdit *e, const float *current_lm, const float *residual) {
    hipStream_t s = e->ctx->stream;
    const uint32_t H = e->cfg.hidden;
    const Lin *proj[2] = {&e->lm_to_dit, &e->res_to_dit};
    const float *src[2] = {current_lm, residual};
    for (int i = 0; i < 2; ++i) {
        ProfSpan sp(e->ctx, "local.seq_linear");
        MatvecLaunch a;
        a.w = proj[i]->w;
        a.xl = src[i];
        a.rows = H;
        a.cols = e->lm_hidden;
        a.epi = EPI_BIAS;
        a.bias = proj[i]->b;
        a.bias_dtype = proj[i]->bt;
        a.alpha = 1.f;
        a.y = F(e->mu) + (size_t)i * H;
        VX_CHECK(launch_matvec(s, a));
    }
    return VX_OK;
}

// The solve after the inputs are in place (cfm_solve, local.rs:383-430). With
// mu_src set, the mu tokens are first projected from those device vectors
// (cfm_from_model_hiddens, local.rs:379-381,399-401).
int enqueue_solve(vx_locdit *e, const vx_cfm_options &o, bool initial_x, uint32_t *calls,
                  const float *const *mu_src = nullptr, bool time_rows = true) {
    hipStream_t s = e->ctx->stream;
    const vx_locdit_config &c = e->cfg;
    const uint32_t n = c.patch * c.feat_dim;
    if (mu_src) VX_CHECK(enqueue_project_mu(e, mu_src[0], mu_src[1]));
    std::vector<float> span;
    VX_CHECK(time_span(o.n_timesteps, o.sway_sampling_coef, span));
    if (!initial_x) {
        ProfSpan sp(e->ctx, "local.cfm_noise");
        VX_CHECK(launch_cfm_noise(s, F(e->x), n, static_cast<const uint32_t *>(e->seed->ptr), 0, o.temperature));
    }
    const uint32_t zi = zero_init_steps(o, span.size());
    uint32_t est = 0, k = 0;
    uint32_t active = 0;
    for (size_t step = 1; step < span.size(); ++step) active += step > zi ? 1u : 0u;
    if (active > e->trows_cap) return fail(VX_ERR_STATE, "CFM time rows were not prepared for %u steps", active);
    // mean_mode = false: estimator dt is zero. Without time_rows the caller has
    // already filled temb for these options.
    if (active && time_rows) VX_CHECK(enqueue_time_rows(e, active));
    for (size_t step = 1; step < span.size(); ++step) {
        if (step <= zi) continue;
        const float t = span[step - 1], dt = t - span[step];
        (void)t;
        VX_CHECK(enqueue_inputs(e));
        VX_CHECK(enqueue_body(e, 2, F(e->temb) + (size_t)k++ * e->cfg.hidden, e->out_euler));
        if (e->out_euler) {
            ProfSpan sp(e->ctx, "local.out_cfg_euler");
            CfmOutEulerArgs a;
            a.rows = F(e->norm);
            if (e->fold_norm) {   // the stream itself, the final norm folded in
                a.rows = F(e->hres);
                a.rows_frag = 1;
                a.norm_w = e->norm_w;
                a.eps = c.rms_epsilon;
            }
            a.tokens = e->S;
            a.x0 = c.n_mu + 1u + c.n_cond;
            a.patch = c.patch;
            a.feat = c.feat_dim;
            a.hidden = c.hidden;
            a.w = static_cast<const __half *>(e->out_proj.w.ptr);
            a.bias = e->out_proj.b;
            a.bias_dtype = e->out_proj.bt;
            a.out = F(e->out);
            a.x = F(e->x);
            a.dt = dt;
            a.cfg = o.cfg_value;
            a.zero_star = o.use_cfg_zero_star ? 1u : 0u;
            a.counter = static_cast<uint32_t *>(e->out_ctr->ptr);
            VX_CHECK(launch_cfm_out_euler(s, a));
        } else {
            ProfSpan sp(e->ctx, "local.cfm_cfg_euler");
            VX_CHECK(launch_cfm_cfg_euler(s, F(e->x), F(e->out), F(e->out) + n, n, dt, o.cfg_value,
                                          o.use_cfg_zero_star ? 1u : 0u));
        }
        est += 2;
    }
    if (calls) *calls = est;
    return VX_OK;
}

// The t values of the solve's estimator calls, on the device before the solve is
// enqueued (or captured); the row buffers grow with the step count, and a cached
// graph that addresses replaced buffers is dropped.
int prepare_time_rows(vx_locdit *e, const vx_cfm_options &o) {
    std::vector<float> span;
    VX_CHECK(time_span(o.n_timesteps, o.sway_sampling_coef, span));
    const uint32_t zi = zero_init_steps(o, span.size());
    std::vector<float> ts;
    for (size_t step = 1; step < span.size(); ++step)
        if (step > zi) ts.push_back(span[step - 1]);
    if (ts.empty()) return VX_OK;
    vx_ctx *ctx = e->ctx;
    const uint32_t n = (uint32_t)ts.size(), H = e->cfg.hidden;
    if (n > e->trows_cap) {
        VX_HIP(hipStreamSynchronize(ctx->stream));
        if (e->graph) {
            vx_graph_free(ctx, e->graph);
            e->graph = nullptr;
        }
        for (vx_buf **b : {&e->tvals, &e->trows, &e->tmid, &e->temb})
            if (*b) {
                vx_free(ctx, *b);
                *b = nullptr;
            }
        e->trows_cap = 0;
        e->temb_ready = false;
        VX_CHECK(vx_alloc(ctx, (uint64_t)n * 4u, &e->tvals));
        VX_CHECK(vx_alloc(ctx, (uint64_t)n * H * 4u, &e->trows));
        VX_CHECK(vx_alloc(ctx, (uint64_t)n * H * 4u, &e->tmid));
        VX_CHECK(vx_alloc(ctx, (uint64_t)n * H * 4u, &e->temb));
        e->trows_cap = n;
    }
    return vx_upload(ctx, e->tvals, 0, ts.data(), (uint64_t)n * 4u);
}

int check_finite(const float *v, uint64_t n, const char *what) {
    for (uint64_t i = 0; i < n; ++i)
        if (!std::isfinite(v[i]))
            return fail(VX_ERR_INVALID_ARG, "%s contains non-finite value at index %llu: %g", what,
                        (unsigned long long)i, v[i]);
    return VX_OK;
}

int upload_inputs(vx_locdit *e, const float *cond, const float *mu) {
    const vx_locdit_config &c = e->cfg;
    const uint64_t cn = c.cond_raw ? (uint64_t)c.n_cond * c.hidden : (uint64_t)c.patch * c.feat_dim;
    if (!cond) return fail(VX_ERR_INVALID_ARG, "LocDiT condition is null");
    VX_CHECK(check_finite(cond, cn, "CFM condition"));
    VX_CHECK(vx_upload(e->ctx, e->cond_in, 0, cond, cn * 4u));
    if (c.n_mu) {
        if (!mu) return fail(VX_ERR_INVALID_ARG, "LocDiT mu is null");
        VX_CHECK(check_finite(mu, (uint64_t)c.n_mu * c.hidden, "CFM mu"));
        VX_CHECK(vx_upload(e->ctx, e->mu, 0, mu, (uint64_t)c.n_mu * c.hidden * 4u));
    }
    return VX_OK;
}

double now_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

bool same_options(const vx_cfm_options &a, const vx_cfm_options &b) {
    return a.n_timesteps == b.n_timesteps && a.cfg_value == b.cfg_value && a.temperature == b.temperature &&
           a.sway_sampling_coef == b.sway_sampling_coef && a.use_cfg_zero_star == b.use_cfg_zero_star;
}

}  // namespace

extern "C" {

int vx_locdit_create(vx_ctx *ctx, const vx_model *model, const vx_model *rope_model, uint32_t rope_factor_offset,
                     const vx_locdit_config *cfg, uint32_t strict_geometry, vx_locdit **out) {
    if (!ctx || !model || !rope_model || !cfg || !out) return fail(VX_ERR_INVALID_ARG, "vx_locdit_create: null argument");
    *out = nullptr;
    VX_CHECK(validate(*cfg, strict_geometry != 0));
    vx_locdit *e = new vx_locdit();
    e->ctx = ctx;
    e->model = model;
    e->cfg = *cfg;
    const vx_locdit_config &c = e->cfg;
    e->S = c.n_mu + 1u + c.n_cond + c.patch;
    e->dense_fused = e->S <= kDenseFusedMaxTokens && dense_fused_lds(e->S, c.head_dim) <= 65536u;
    auto bail = [&](int st) {
        free_all(e);
        delete e;
        return st;
    };
    const uint32_t H = c.hidden, QD = c.q_heads * c.head_dim, KD = c.kv_heads * c.head_dim;
    // validate_tensors (local.rs:127-145) for the LocDiT half.
    int st;
    if ((st = linear(model, "locdit.in_proj", c.feat_dim, H, &e->in_proj))) return bail(st);
    if (!c.cond_raw && (st = linear(model, "locdit.cond_proj", c.feat_dim, H, &e->cond_proj))) return bail(st);
    if ((st = linear(model, "locdit.out_proj", H, c.feat_dim, &e->out_proj))) return bail(st);
    const void *p;
    if ((st = vector(model, "locdit.norm.weight", H, true, &p, nullptr))) return bail(st);
    e->norm_w = static_cast<const float *>(p);
    if ((st = linear(model, "locdit.time_mlp.linear_1", H, H, &e->t1)) ||
        (st = linear(model, "locdit.time_mlp.linear_2", H, H, &e->t2)) ||
        (st = linear(model, "locdit.delta_time_mlp.linear_1", H, H, &e->d1)) ||
        (st = linear(model, "locdit.delta_time_mlp.linear_2", H, H, &e->d2)))
        return bail(st);
    e->layers.resize(c.layers);
    for (uint32_t l = 0; l < c.layers; ++l) {  // validate_local_layers (local.rs:150-168)
        LocLayer &L = e->layers[l];
        const std::string pre = "locdit.blk." + std::to_string(l) + ".";
        if ((st = vector(model, pre + "attn_norm.weight", H, true, &p, nullptr))) return bail(st);
        L.attn_norm = static_cast<const float *>(p);
        if ((st = vector(model, pre + "ffn_norm.weight", H, true, &p, nullptr))) return bail(st);
        L.ffn_norm = static_cast<const float *>(p);
        if ((st = matrix(model, pre + "attn_q.weight", H, QD, &L.q)) || (st = matrix(model, pre + "attn_k.weight", H, KD, &L.k)) ||
            (st = matrix(model, pre + "attn_v.weight", H, KD, &L.v)) ||
            (st = matrix(model, pre + "attn_output.weight", QD, H, &L.o)) ||
            (st = matrix(model, pre + "ffn_gate.weight", H, c.ffn, &L.gate)) ||
            (st = matrix(model, pre + "ffn_up.weight", H, c.ffn, &L.up)) ||
            (st = matrix(model, pre + "ffn_down.weight", c.ffn, H, &L.down)))
            return bail(st);
    }
    // The mu projections are required by the reference's contract (local.rs:141-144);
    // outside it they are optional and only the model-hidden solve needs them.
    {
        const bool have = model->by_name.count("projections.lm_to_dit_proj.weight") != 0;
        if (have || strict_geometry) {
            const vx_tensor_info *t;
            if ((st = find(model, "projections.lm_to_dit_proj.weight", &t))) return bail(st);
            const uint32_t in = t->n_dims == 2 ? (uint32_t)t->dims[0] : 0u;
            if (strict_geometry && in != 2048u)
                return bail(fail(VX_ERR_SHAPE, "projections.lm_to_dit_proj.weight has %u columns, expected 2048", in));
            if ((st = linear(model, "projections.lm_to_dit_proj", in, H, &e->lm_to_dit)) ||
                (st = linear(model, "projections.res_to_dit_proj", in, H, &e->res_to_dit)))
                return bail(st);
            e->has_mu_proj = true;
            e->lm_hidden = in;
        }
    }
    if ((st = resolve_vector(rope_model, rope_factor_offset, VX_DTYPE_F32, c.head_dim / 2u, &p, "LocDiT rope factors")))
        return bail(st);
    e->rope_factors = static_cast<const float *>(p);
    // Buffers (LocalEngine::new, local.rs:285-297), sized for the CFG batch of two.
    const uint64_t f = 4, S2 = 2ull * e->S;
    const uint64_t cond_n = c.cond_raw ? (uint64_t)c.n_cond * H : (uint64_t)c.patch * c.feat_dim;
    struct {
        vx_buf **b;
        uint64_t n;
    } bufs[] = {{&e->x, (uint64_t)c.patch * c.feat_dim},
                {&e->cond_in, cond_n},
                {&e->mu, 2ull * H},
                {&e->patch_proj, (uint64_t)c.patch * H},
                {&e->cond_proj_out, (uint64_t)c.patch * H},
                {&e->tsin, H},
                {&e->ttmp, H},
                {&e->tvec, H},
                {&e->dsin, H},
                {&e->dtmp, H},
                {&e->dvec, H},
                {&e->hidden, S2 * H},
                {&e->norm, S2 * H},
                {&e->q, S2 * QD},
                {&e->k, S2 * KD},
                {&e->v, S2 * KD},
                {&e->attn, S2 * QD},
                {&e->gate, S2 * c.ffn},
                {&e->branch, S2 * H},
                {&e->scores, S2 * c.q_heads * e->S},
                {&e->out, 2ull * c.patch * c.feat_dim},
                {&e->seed, 2},
                {&e->rope_tab, (uint64_t)e->S * c.head_dim}};
    for (auto &b : bufs)
        if ((st = vx_alloc(ctx, std::max<uint64_t>(b.n * f, 16u), b.b))) return bail(st);
    for (auto &b : bufs)
        if (hipMemsetAsync((*b.b)->ptr, 0, (*b.b)->bytes, ctx->stream) != hipSuccess)
            return bail(fail(VX_ERR_HIP, "hipMemsetAsync of LocDiT state failed"));
    // The short-batch layer stack when the CFG batch and every projection fit the
    // short-batch GEMM (at most 128 rows, K and N multiples of 128, 16-byte
    // aligned F16 rows) and the attention runs fused.
    {
        auto al16 = [](const WRef &w) { return (reinterpret_cast<uintptr_t>(w.ptr) & 15u) == 0; };
        bool ok = e->dense_fused && S2 <= 128u && H % 128u == 0 && QD % 128u == 0 && KD % 32u == 0 &&
                  c.ffn % 128u == 0 && c.head_dim % 8u == 0 && c.feat_dim % 8u == 0 && c.feat_dim <= 128u &&
                  al16(e->in_proj.w);
        for (const LocLayer &L : e->layers)
            ok = ok && al16(L.q) && al16(L.k) && al16(L.v) && al16(L.o) && al16(L.gate) && al16(L.up) && al16(L.down);
        if (ok) {
            // K slabs of attn_output and ffn_down: about one workgroup per CU, at
            // least four 32-column k-steps per slab, at most the branches the
            // residual rmsnorm sums.
            const uint32_t cus = std::max(1, ctx->props.multiProcessorCount);
            auto slabs = [&](uint32_t rows, uint32_t K) {
                const uint32_t tiles = (rows + 31u) / 32u;
                uint32_t k = std::max(1u, cus / tiles);
                k = std::min(k, std::min(kSeqNormMaxBranch, K / 128u));
                return std::max(1u, k);
            };
            e->ks_qkv = std::min(2u, slabs(QD + 2u * KD, H));   // the attention sums at most two
            e->ks_o = slabs(H, QD);
            e->ks_down = slabs(H, c.ffn);
            e->attn_oproj = c.q_heads <= kSeqNormMaxBranch && H % 16u == 0 && dense_attn_oproj_eligible(e->S, c.head_dim);
            // The residual-stream stack when the CFG batch is at most two token
            // fragments: each of its GEMM workgroups splits the whole f32 stream
            // itself (what the rmsnorm did once), which at 2 x 11 tokens costs less
            // than the two rmsnorm launches it removes (the 12-layer, 11-token
            // solve 4.00 -> 3.63 ms) but at 2 x 37 tokens more (3.71 -> 3.81 ms).
            e->fold_norm = e->attn_oproj && H % 1024u == 0 && H <= 4096u && S2 <= kFoldNormMaxRows;
            const uint64_t ks = std::max({e->ks_o, e->ks_down, e->attn_oproj ? c.q_heads : 1u});
            const uint64_t R16 = (S2 + 15u) & ~15ull;   // plane rows, padded to whole fragments
            struct {
                vx_buf **b;
                uint64_t bytes;
            } sk[] = {{&e->yh, R16 * H * 2u},          {&e->yl, R16 * H * 2u},
                      {&e->ah, R16 * QD * 2u},         {&e->al, R16 * QD * 2u},
                      {&e->acth, R16 * c.ffn * 2u},    {&e->actl, R16 * c.ffn * 2u},
                      {&e->part, ks * S2 * H * 4u},
                      {&e->qkvp, (uint64_t)e->ks_qkv * S2 * (QD + 2u * KD) * 4u},
                      {&e->hres, R16 * H * 4u},
                      {&e->ssq, 2u * R16 * 4u}};
            for (auto &b : sk) {
                if ((st = vx_alloc(ctx, b.bytes, b.b))) return bail(st);
                if (hipMemsetAsync((*b.b)->ptr, 0, (*b.b)->bytes, ctx->stream) != hipSuccess)
                    return bail(fail(VX_ERR_HIP, "hipMemsetAsync of LocDiT state failed"));
            }
            // The layer matrices in the fragment layout (a second copy of the
            // LocDiT weights, streamed by the short-batch GEMM).
            auto pad16 = [](uint64_t r) { return (r + 15u) & ~15ull; };
            const uint64_t per_layer = (pad16(QD) + 2u * pad16(KD)) * H + pad16(H) * QD + 2u * pad16(c.ffn) * H +
                                       pad16(H) * c.ffn;
            if ((st = vx_alloc(ctx, per_layer * c.layers * 2u, &e->wfrag))) return bail(st);
            __half *dst = static_cast<__half *>(e->wfrag->ptr);
            for (LocLayer &L : e->layers) {
                const WRef *m[7] = {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down};
                const uint32_t rows[7] = {QD, KD, KD, H, c.ffn, c.ffn, H};
                const uint32_t cols[7] = {H, H, H, QD, H, H, c.ffn};
                for (int i = 0; i < 7; ++i) {
                    if ((st = launch_repack_frag16(ctx->stream, static_cast<const __half *>(m[i]->ptr), dst, rows[i],
                                                   cols[i])))
                        return bail(st);
                    L.frag[i] = dst;
                    dst += pad16(rows[i]) * cols[i];
                }
            }
            e->sk = true;
            // out_proj + Euler update in one launch (F16 out_proj, rows of the
            // normed hidden f32 and 16-byte aligned). On the residual stream it
            // stages the 2 x patch stream rows in LDS (at most 64 KB); past that
            // the final rmsnorm runs and the launch reads its rows instead.
            const bool rows_fit = !e->fold_norm || 2ull * c.patch * H * 4u <= 65536u;
            if (e->out_proj.w.wt == WT_F16 && e->out_proj.w.dtype == 1 && rows_fit &&
                cfm_out_euler_eligible(c.patch, c.feat_dim, H, e->out_proj.w.ptr)) {
                if ((st = vx_alloc(ctx, 256u, &e->out_ctr))) return bail(st);
                if (hipMemsetAsync(e->out_ctr->ptr, 0, 256u, ctx->stream) != hipSuccess)
                    return bail(fail(VX_ERR_HIP, "hipMemsetAsync of LocDiT state failed"));
                e->out_euler = true;
            }
        }
    }
    if (e->dense_fused && (st = launch_rope_pos_table(ctx->stream, reinterpret_cast<float2 *>(e->rope_tab->ptr),
                                                      e->rope_factors, e->S, c.head_dim, c.rope_theta,
                                                      c.rope_scaling)))
        return bail(st);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return bail(fail(VX_ERR_HIP, "LocDiT init sync failed"));
    *out = e;
    return VX_OK;
}

int vx_locdit_destroy(vx_locdit *e) {
    if (!e) return VX_OK;
    (void)hipStreamSynchronize(e->ctx->stream);
    free_all(e);
    delete e;
    return VX_OK;
}

int vx_locdit_estimate(vx_locdit *e, const float *x, const float *cond, const float *mu, float t, float dt,
                       float *out) {
    if (!e || !x || !out) return fail(VX_ERR_INVALID_ARG, "vx_locdit_estimate: null argument");
    VX_CHECK(check_cancel(e->ctx));
    const vx_locdit_config &c = e->cfg;
    const uint64_t n = (uint64_t)c.patch * c.feat_dim;
    if (!std::isfinite(t) || !std::isfinite(dt))  // check_time (local.rs:563)
        return fail(VX_ERR_INVALID_ARG, "LocDiT t/dt must be finite, got t=%g, dt=%g", t, dt);
    VX_CHECK(check_finite(x, n, "LocDiT x"));
    VX_CHECK(upload_inputs(e, cond, mu));
    VX_CHECK(vx_upload(e->ctx, e->x, 0, x, n * 4u));
    VX_CHECK(enqueue_inputs(e));
    VX_CHECK(enqueue_time(e, t, dt));
    VX_CHECK(enqueue_body(e, 1));
    return vx_download(e->ctx, e->out, 0, out, n * 4u);
}

}  // extern "C"

namespace {
// cfm_solve (local.rs:383-430) from host mu (mu_src null) or from model hiddens.
int solve(vx_locdit *e, const float *cond, const float *mu, const float *const *mu_src, const vx_cfm_options *opt,
          const float *initial_x, float *out_patch, vx_cfm_result *res) {
    VX_CHECK(validate_options(*opt));
    const vx_locdit_config &c = e->cfg;
    const uint64_t n = (uint64_t)c.patch * c.feat_dim;
    vx_ctx *ctx = e->ctx;
    const double t0 = now_ms();
    if (mu_src) {
        const uint64_t cn = c.cond_raw ? (uint64_t)c.n_cond * c.hidden : (uint64_t)c.patch * c.feat_dim;
        if (!cond) return fail(VX_ERR_INVALID_ARG, "LocDiT condition is null");
        VX_CHECK(check_finite(cond, cn, "CFM condition"));
        VX_CHECK(vx_upload(ctx, e->cond_in, 0, cond, cn * 4u));
    } else {
        VX_CHECK(upload_inputs(e, cond, mu));
    }
    if (initial_x) {
        VX_CHECK(check_finite(initial_x, n, "CFM initial x"));
        VX_CHECK(vx_upload(ctx, e->x, 0, initial_x, n * 4u));
    }
    const uint32_t seed[2] = {(uint32_t)opt->seed, (uint32_t)(opt->seed >> 32)};
    VX_CHECK(vx_upload(ctx, e->seed, 0, seed, 8u));
    VX_CHECK(prepare_time_rows(e, *opt));
    uint32_t calls = 0;
    if (ctx->prof_enabled) {
        e->temb_ready = false;
        VX_CHECK(enqueue_solve(e, *opt, initial_x != nullptr, &calls, mu_src));
        e->temb_opt = *opt;
        e->temb_ready = true;
    } else {
        // The time rows depend on the options only: computed eagerly when they
        // change, outside the graph that every replay of these options runs.
        if (!e->temb_ready || !same_options(e->temb_opt, *opt)) {
            std::vector<float> span;
            VX_CHECK(time_span(opt->n_timesteps, opt->sway_sampling_coef, span));
            const uint32_t zi = zero_init_steps(*opt, span.size());
            uint32_t active = 0;
            for (size_t step = 1; step < span.size(); ++step) active += step > zi ? 1u : 0u;
            e->temb_ready = false;
            if (active) VX_CHECK(enqueue_time_rows(e, active));
            e->temb_opt = *opt;
            e->temb_ready = true;
        }
        const int ix = initial_x ? 1 : 0;
        const float *src0 = mu_src ? mu_src[0] : nullptr, *src1 = mu_src ? mu_src[1] : nullptr;
        if (!e->graph || !same_options(e->graph_opt, *opt) || e->graph_initial_x != ix ||
            e->graph_mu_src[0] != src0 || e->graph_mu_src[1] != src1) {
            if (e->graph) {
                vx_graph_free(ctx, e->graph);
                e->graph = nullptr;
            }
            VX_CHECK(vx_graph_begin(ctx));
            const int st = enqueue_solve(e, *opt, initial_x != nullptr, &calls, mu_src, false);
            vx_graph *g = nullptr;
            const int st2 = vx_graph_end(ctx, &g);
            if (st != VX_OK) {
                if (g) vx_graph_free(ctx, g);
                return st;
            }
            VX_CHECK(st2);
            e->graph = g;
            e->graph_opt = *opt;
            e->graph_initial_x = ix;
            e->graph_mu_src[0] = src0;
            e->graph_mu_src[1] = src1;
        }
        std::vector<float> span;
        VX_CHECK(time_span(opt->n_timesteps, opt->sway_sampling_coef, span));
        calls = 2u * (uint32_t)(span.size() - 1u - std::min<size_t>(zero_init_steps(*opt, span.size()), span.size() - 1u));
        VX_CHECK(vx_graph_launch(ctx, e->graph));
    }
    VX_CHECK(vx_download(ctx, e->x, 0, out_patch, n * 4u));
    if (res) {
        std::vector<float> span;
        VX_CHECK(time_span(opt->n_timesteps, opt->sway_sampling_coef, span));
        double sum = 0, sq = 0;
        float mn = INFINITY, mx = -INFINITY;
        for (uint64_t i = 0; i < n; ++i) {
            sum += out_patch[i];
            sq += (double)out_patch[i] * out_patch[i];
            mn = std::min(mn, out_patch[i]);
            mx = std::max(mx, out_patch[i]);
        }
        res->elapsed_ms = now_ms() - t0;
        res->n_timesteps = opt->n_timesteps;
        res->estimator_calls = calls;
        res->zero_init_steps = zero_init_steps(*opt, span.size());
        res->output_checksum = sum;
        res->output_l2 = std::sqrt(sq);
        res->output_min = mn;
        res->output_max = mx;
    }
    return VX_OK;
}
}  // namespace

extern "C" {

int vx_locdit_cfm_solve(vx_locdit *e, const float *cond, const float *mu, const vx_cfm_options *opt,
                        const float *initial_x, float *out_patch, vx_cfm_result *res) {
    if (!e || !opt || !out_patch) return fail(VX_ERR_INVALID_ARG, "vx_locdit_cfm_solve: null argument");
    VX_CHECK(check_cancel(e->ctx));
    return solve(e, cond, mu, nullptr, opt, initial_x, out_patch, res);
}

int vx_locdit_cfm_solve_from_model_hiddens(vx_locdit *e, const vx_buf *current_lm, const vx_buf *residual_output,
                                           const float *cond, const vx_cfm_options *opt, const float *initial_x,
                                           float *out_patch, vx_cfm_result *res) {
    if (!e || !opt || !out_patch)
        return fail(VX_ERR_INVALID_ARG, "vx_locdit_cfm_solve_from_model_hiddens: null argument");
    VX_CHECK(check_cancel(e->ctx));
    if (!e->has_mu_proj)
        return fail(VX_ERR_NOT_FOUND, "required GGUF tensor \"projections.lm_to_dit_proj.weight\" is missing");
    if (e->cfg.n_mu != 2u)
        return fail(VX_ERR_UNSUPPORTED, "the model-hidden solve projects two mu tokens; the config has %u", e->cfg.n_mu);
    VX_CHECK(need_buf(current_lm, (uint64_t)e->lm_hidden * 4u, "CFM current_lm"));
    VX_CHECK(need_buf(residual_output, (uint64_t)e->lm_hidden * 4u, "CFM residual output"));
    const float *src[2] = {static_cast<const float *>(current_lm->ptr), static_cast<const float *>(residual_output->ptr)};
    return solve(e, cond, nullptr, src, opt, initial_x, out_patch, res);
}

// ------------------------------------------------------- CFM shader entry points
int vx_cfm_noise(vx_ctx *ctx, vx_buf *x, const vx_cfm_noise_push *pc) {
    if (!ctx || !pc) return fail(VX_ERR_INVALID_ARG, "vx_cfm_noise: null argument");
    VX_CHECK(need_buf(x, (uint64_t)pc->n * 4u, "vx_cfm_noise x"));
    ProfSpan sp(ctx, "local.cfm_noise");
    return launch_cfm_noise(ctx->stream, F(x), pc->n, nullptr, ((uint64_t)pc->seed_hi << 32) | pc->seed_lo,
                            pc->temperature);
}

int vx_cfm_cfg_euler(vx_ctx *ctx, vx_buf *x, const vx_buf *positive, const vx_buf *negative,
                     const vx_cfm_euler_push *pc) {
    if (!ctx || !pc) return fail(VX_ERR_INVALID_ARG, "vx_cfm_cfg_euler: null argument");
    // cfm_cfg_euler.comp runs one 256-lane workgroup: it reduces over and updates
    // x[0..256) only. Larger n would have another meaning here, so it is refused.
    if (pc->n > 256u)
        return fail(VX_ERR_UNSUPPORTED, "vx_cfm_cfg_euler: n = %u, but cfm_cfg_euler.comp covers at most 256 "
                    "elements (one 256-lane workgroup)", pc->n);
    VX_CHECK(need_buf(x, (uint64_t)pc->n * 4u, "vx_cfm_cfg_euler x"));
    VX_CHECK(need_buf(positive, (uint64_t)pc->n * 4u, "vx_cfm_cfg_euler positive"));
    VX_CHECK(need_buf(negative, (uint64_t)pc->n * 4u, "vx_cfm_cfg_euler negative"));
    ProfSpan sp(ctx, "local.cfm_cfg_euler");
    return launch_cfm_cfg_euler(ctx->stream, F(x), static_cast<const float *>(positive->ptr),
                                static_cast<const float *>(negative->ptr), pc->n, pc->dt, pc->cfg, pc->use_zero_star);
}

int vx_time_sinusoidal(vx_ctx *ctx, vx_buf *out, const vx_time_push *pc) {
    if (!ctx || !pc) return fail(VX_ERR_INVALID_ARG, "vx_time_sinusoidal: null argument");
    VX_CHECK(need_buf(out, (uint64_t)pc->dim * 4u, "vx_time_sinusoidal out"));
    ProfSpan sp(ctx, "local.time_sinusoidal");
    return launch_time_sinusoidal(ctx->stream, F(out), pc->dim, pc->t, nullptr, 0);
}

int vx_pack_locdit(vx_ctx *ctx, const vx_buf *mu1, const vx_buf *mu2, const vx_buf *time, const vx_buf *cond,
                   const vx_buf *x, vx_buf *hidden, const vx_pack_locdit_push *pc) {
    if (!ctx || !pc) return fail(VX_ERR_INVALID_ARG, "vx_pack_locdit: null argument");
    const uint64_t H = pc->hidden, P = pc->patch_tokens;
    VX_CHECK(need_buf(mu1, H * 4u, "vx_pack_locdit mu1"));
    VX_CHECK(need_buf(mu2, H * 4u, "vx_pack_locdit mu2"));
    VX_CHECK(need_buf(time, H * 4u, "vx_pack_locdit time"));
    VX_CHECK(need_buf(cond, P * H * 4u, "vx_pack_locdit cond"));
    VX_CHECK(need_buf(x, P * H * 4u, "vx_pack_locdit x"));
    VX_CHECK(need_buf(hidden, (3u + 2u * P) * H * 4u, "vx_pack_locdit hidden"));
    ProfSpan sp(ctx, "local.pack_locdit");
    PackLocditArgs a;
    a.mu[0] = static_cast<const float *>(mu1->ptr);
    a.mu[1] = static_cast<const float *>(mu2->ptr);
    a.time = static_cast<const float *>(time->ptr);
    a.cond = static_cast<const float *>(cond->ptr);
    a.x = static_cast<const float *>(x->ptr);
    a.out = F(hidden);
    a.hidden = pc->hidden;
    a.n_mu = 2;
    a.n_cond = pc->patch_tokens;
    a.n_x = pc->patch_tokens;
    a.zero_mu_mask = pc->zero_mu ? 1u : 0u;
    return launch_pack_locdit(ctx->stream, a);
}

int vx_silu_inplace(vx_ctx *ctx, vx_buf *x, uint32_t n) {
    if (!ctx) return fail(VX_ERR_INVALID_ARG, "vx_silu_inplace: null context");
    VX_CHECK(need_buf(x, (uint64_t)n * 4u, "vx_silu_inplace x"));
    return launch_silu_inplace(ctx->stream, F(x), n);
}

int vx_add_vectors(vx_ctx *ctx, vx_buf *a, const vx_buf *b, uint32_t n) {
    if (!ctx) return fail(VX_ERR_INVALID_ARG, "vx_add_vectors: null context");
    VX_CHECK(need_buf(a, (uint64_t)n * 4u, "vx_add_vectors a"));
    VX_CHECK(need_buf(b, (uint64_t)n * 4u, "vx_add_vectors b"));
    return launch_add_vectors(ctx->stream, F(a), static_cast<const float *>(b->ptr), n);
}

}  // extern "C"
