// Token-batched prefill of a layer stack (the seq_* op family of
// local.rs:482-527 applied to a MiniCPM4-style decoder stack, with a causal mask
// and a position base), shared by the BaseLM (with RoPE) and the ResidualLM
// (without RoPE):
//   per layer over the rows of the residual stream h:
//     rmsnorm(h)*attn_norm -> f16 hi/lo planes        (k_seq_rmsnorm)
//     q|k|v = planes . Wq|Wk|Wv                       (k_gemm, split-K)
//     RoPE at pos0+t (or none), K/V rows -> f16 cache, q planes  (k_seq_rope_store)
//     causal attention over cache keys 0..pos0+t       (k_prefill_attn)
//     h += scale * Wo . attn                           (k_gemm residual)
//     rmsnorm(h)*ffn_norm -> planes                    (k_seq_rmsnorm)
//     act = silu(Wg . n) * (Wu . n) -> planes          (k_gemm swiglu)
//     h += scale * Wdown . act                         (k_gemm residual)
// Row t computes what the decode step computes at position pos0 + t: the same
// KV-cache rows and the same residual stream, to rounding.
#include <algorithm>

#include "vx_internal.h"

namespace vx {

namespace {

inline float *F(vx_buf *b) { return static_cast<float *>(b->ptr); }
inline __half *H(vx_buf *b) { return static_cast<__half *>(b->ptr); }

// Split-K factor for a projection of n_tiles 128-row tiles and tt-token tiles:
// as many workgroups as fit one per CU (rounded down: a second workgroup on a CU
// runs at well under twice one's throughput, so the CUs that hold two would set
// the time; measured on MI355X, rounding up instead made the T = 384 prefill 5%
// slower, T = 256 and 512 2%), at least four 32-column blocks per split.
uint32_t pick_split(const vx_ctx *ctx, uint32_t tt, uint32_t n_tiles, uint32_t T, uint32_t K) {
    const uint32_t tiles = n_tiles * ((T + tt - 1u) / tt);
    const uint32_t cus = ctx->props.multiProcessorCount > 0 ? (uint32_t)ctx->props.multiProcessorCount : 256u;
    uint32_t ks = std::max<uint32_t>(1u, cus / tiles);
    ks = std::min<uint32_t>(ks, tt > 64u ? 8u : 4u);
    ks = std::min<uint32_t>(ks, std::max<uint32_t>(1u, K / 128u));
    return std::max<uint32_t>(ks, 1u);
}

GemmSeg gemm_seg(const WRef &w, uint32_t rows, float *out, uint32_t ldo) {
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

int prefill_stack_check(const PrefillStack &p) {
    for (uint32_t l = 0; l < p.n_layers; ++l) {
        const StackLayer &L = p.layers[l];
        const WRef *ws[] = {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down};
        for (const WRef *w : ws) {
            if (w->wt == WT_Q8 && !w->ptr)
                return fail(VX_ERR_UNSUPPORTED,
                            "batched prefill needs Q8_0 row widths that are multiples of 1024 (layer %u)", l);
            if (w->wt == WT_F16 && (w->cols % 128u))
                return fail(VX_ERR_UNSUPPORTED, "batched prefill needs F16 row widths that are multiples of 128");
            if (w->wt == WT_F32) return fail(VX_ERR_UNSUPPORTED, "batched prefill has no F32 projection path");
        }
    }
    if (p.head_dim != 64u && p.head_dim != 128u)
        return fail(VX_ERR_UNSUPPORTED, "batched prefill attention needs head_dim 64 or 128");
    const uint32_t qpk = p.q_heads / p.kv_heads;
    if (qpk != 1u && qpk != 2u && qpk != 4u && qpk != 8u)
        return fail(VX_ERR_UNSUPPORTED, "batched prefill attention needs 1, 2, 4 or 8 query heads per KV head");
    if (p.rope && !p.rope_factors) return fail(VX_ERR_INVALID_ARG, "batched prefill with RoPE needs its factors");
    return VX_OK;
}

int prefill_stack_alloc(vx_ctx *ctx, uint32_t cap, uint32_t nH, uint32_t nF, uint32_t nKV, StackWork *w) {
    if (w->cap) return VX_OK;
    const uint64_t H = nH, F = nF, KV = nKV, T = cap;
    const uint64_t Tp = (T + 127u) / 128u * 128u;   // GEMM input planes: whole 128-token tiles
    VX_CHECK(vx_alloc(ctx, T * H * 4u, &w->h));
    VX_CHECK(vx_alloc(ctx, Tp * H * 2u, &w->xh));
    VX_CHECK(vx_alloc(ctx, Tp * H * 2u, &w->xl));
    VX_CHECK(vx_alloc(ctx, Tp * F * 2u, &w->ah));
    VX_CHECK(vx_alloc(ctx, Tp * F * 2u, &w->al));
    VX_CHECK(vx_alloc(ctx, T * H * 2u, &w->qh));
    VX_CHECK(vx_alloc(ctx, T * H * 2u, &w->ql));
    VX_CHECK(vx_alloc(ctx, T * H * 4u, &w->q));
    VX_CHECK(vx_alloc(ctx, T * KV * 4u, &w->k));
    VX_CHECK(vx_alloc(ctx, T * KV * 4u, &w->v));
    // Split-K partials: of the residual projections ([split][T][H]) and of QKV
    // ([split][T][H + 2 KV]); the two uses never overlap in time.
    VX_CHECK(vx_alloc(ctx, (uint64_t)kPrefillMaxSplit * T * (H + 2u * KV) * 4u, &w->ws));
    // Stream-K SwiGLU: two tile parts per workgroup and a counter per workgroup
    // boundary, one workgroup per CU; the counters start at zero.
    const uint32_t cus = ctx->props.multiProcessorCount > 0 ? (uint32_t)ctx->props.multiProcessorCount : 256u;
    w->sk_grid = cus / 8u * 8u;
    if (w->sk_grid) {
        VX_CHECK(vx_alloc(ctx, (uint64_t)w->sk_grid * 2u * kSkTileFloats * 4u, &w->sk_ws));
        VX_CHECK(vx_alloc(ctx, (uint64_t)w->sk_grid * 4u, &w->sk_cnt));
        VX_HIP(hipMemsetAsync(w->sk_cnt->ptr, 0, w->sk_cnt->bytes, ctx->stream));
    }
    w->cap = cap;
    return VX_OK;
}

void prefill_stack_free(vx_ctx *ctx, StackWork *w) {
    vx_buf **bufs[] = {&w->h,  &w->xh, &w->xl, &w->ah, &w->al,    &w->qh,
                       &w->ql, &w->q,  &w->k,  &w->v,  &w->ws, &w->sk_ws, &w->sk_cnt};
    for (vx_buf **b : bufs) {
        if (*b) vx_free(ctx, *b);
        *b = nullptr;
    }
    w->cap = 0;
    w->sk_grid = 0;
}

int enqueue_prefill_stack(const PrefillStack &p, uint32_t pos0, uint32_t T) {
    vx_ctx *ctx = p.ctx;
    hipStream_t s = ctx->stream;
    const StackWork &w = *p.work;
    const uint32_t nH = p.nH, nF = p.nF, nKV = p.nKV;
    if (T == 0 || T > w.cap) return fail(VX_ERR_INVALID_ARG, "prefill chunk of %u rows (capacity %u)", T, w.cap);
    // The deep-pipelined GEMM takes the prefill-layout weights and tiled planes,
    // from one full 128-token tile up.
    const bool tiled = p.pw != nullptr && T >= gemm_q8p_tile_tokens();
    const uint32_t tt = tiled ? gemm_q8p_tile_tokens() : 64u;
    const uint32_t ks_qkv = pick_split(p.ctx, tt, (nH + 127u) / 128u + 2u * ((nKV + 127u) / 128u), T, nH);
    const uint32_t ks_o = pick_split(p.ctx, tt, (nH + 127u) / 128u, T, nH);
    const uint32_t ks_down = pick_split(p.ctx, tt, (nH + 127u) / 128u, T, nF);
    // Split residual projections on the tiled path leave their partials in
    // the workspace; the next rmsnorm adds them to h (no atomics in the GEMM epilogue).
    const uint64_t ws_stride = (uint64_t)w.cap * nH;
    const bool ws_o = tiled && ks_o > 1, ws_down = tiled && ks_down > 1;
    // Split QKV on the tiled path stores its partials to the workspace as well (q, k, v
    // regions of one split, ws_qkv floats per split); the RoPE kernel sums them.
    const bool ws_qkv = tiled && ks_qkv > 1;
    const uint64_t ws_qkv_stride = (uint64_t)w.cap * (nH + 2u * nKV);
    float *const wq = F(w.ws), *const wk = wq + (size_t)w.cap * nH, *const wv = wk + (size_t)w.cap * nKV;
    for (uint32_t l = 0; l < p.n_layers; ++l) {
        const StackLayer &L = p.layers[l];
        {
            ProfSpan sp(ctx, "prefill.norm");
            SeqNormArgs n;
            n.h = F(w.h);
            n.ldh = nH;
            n.w = L.attn_norm;
            if (l > 0 && ws_down) {
                n.branch = F(w.ws);
                n.ldb = nH;
                n.nbranch = ks_down;
                n.branch_stride = ws_stride;
            }
            n.n = nH;
            n.eps = p.eps;
            n.yh = H(w.xh);
            n.yl = H(w.xl);
            n.ldp = nH;
            n.tiled = tiled ? 1u : 0u;
            if (ks_qkv > 1 && !ws_qkv) {
                n.zero[0] = F(w.q);
                n.zero_n[0] = nH;
                n.zero[1] = F(w.k);
                n.zero_n[1] = nKV;
                n.zero[2] = F(w.v);
                n.zero_n[2] = nKV;
            }
            VX_CHECK(launch_seq_rmsnorm(s, n, T));
        }
        {
            ProfSpan sp(ctx, "prefill.qkv");
            GemmArgs g;
            g.wk = L.q.wt;
            g.epi = GEPI_STORE;
            g.seg[0] = gemm_seg(L.q, nH, F(w.q), nH);
            g.seg[1] = gemm_seg(L.k, nKV, F(w.k), nKV);
            g.seg[2] = gemm_seg(L.v, nKV, F(w.v), nKV);
            if (tiled) {
                const StackPrefillWeights &P = p.pw[l];
                g.seg[0].pq = P.q.q;
                g.seg[0].pd = P.q.d;
                g.seg[1].pq = P.k.q;
                g.seg[1].pd = P.k.d;
                g.seg[2].pq = P.v.q;
                g.seg[2].pd = P.v.d;
                g.x_tiled = 1;
            }
            g.nseg = 3;
            g.K = nH;
            g.T = T;
            g.xh = H(w.xh);
            g.xl = H(w.xl);
            g.ldx = nH;
            g.ksplit = ks_qkv;
            if (ws_qkv) {
                g.seg[0].out = wq;
                g.seg[1].out = wk;
                g.seg[2].out = wv;
                g.split_store = 1;
                g.ws_stride = ws_qkv_stride;
            }
            VX_CHECK(launch_gemm(s, g));
        }
        {
            ProfSpan sp(ctx, "prefill.rope_store");
            SeqRopeArgs r;
            r.q = ws_qkv ? wq : F(w.q);
            r.k = ws_qkv ? wk : F(w.k);
            r.v = ws_qkv ? wv : F(w.v);
            if (ws_qkv) {
                r.nsplit = ks_qkv;
                r.split_stride = ws_qkv_stride;
            }
            r.ldq = nH;
            r.ldk = nKV;
            r.factors = p.rope_factors;
            r.pos_base = pos0;
            r.q_heads = p.q_heads;
            r.kv_heads = p.kv_heads;
            r.head_dim = p.head_dim;
            r.theta = p.theta;
            r.scaling = p.rope_scaling;
            r.q_inplace = 0;
            r.qh = H(w.qh);
            r.ql = H(w.ql);
            r.ldqp = nH;
            r.kc = p.kc;
            r.vc = p.vc;
            r.no_rope = p.rope ? 0u : 1u;
            r.layer = l;
            r.context = p.context;
            VX_CHECK(launch_seq_rope_store(s, r, T));
        }
        {
            ProfSpan sp(ctx, "prefill.attention");
            PrefillAttnArgs a;
            a.qh = H(w.qh);
            a.ql = H(w.ql);
            a.ldq = nH;
            a.kc = p.kc;
            a.vc = p.vc;
            a.layer = l;
            a.context = p.context;
            a.pos_base = pos0;
            a.T = T;
            a.q_heads = p.q_heads;
            a.kv_heads = p.kv_heads;
            a.head_dim = p.head_dim;
            a.oh = H(w.xh);
            a.ol = H(w.xl);
            a.ldo = nH;
            a.tiled = tiled ? 1u : 0u;
            VX_CHECK(launch_prefill_attn(s, a));
        }
        {
            ProfSpan sp(ctx, "prefill.attn_out");
            GemmArgs g;
            g.wk = L.o.wt;
            g.epi = GEPI_RESIDUAL;
            g.seg[0] = gemm_seg(L.o, nH, F(w.h), nH);
            if (tiled) {
                g.seg[0].pq = p.pw[l].o.q;
                g.seg[0].pd = p.pw[l].o.d;
                g.x_tiled = 1;
            }
            g.K = nH;
            g.T = T;
            g.xh = H(w.xh);
            g.xl = H(w.xl);
            g.ldx = nH;
            g.scale = p.residual_scale;
            g.ksplit = ks_o;
            if (ws_o) {
                g.ws = F(w.ws);
                g.ws_stride = ws_stride;
            }
            VX_CHECK(launch_gemm(s, g));
        }
        {
            ProfSpan sp(ctx, "prefill.norm");
            SeqNormArgs n;
            n.h = F(w.h);
            n.ldh = nH;
            n.w = L.ffn_norm;
            if (ws_o) {
                n.branch = F(w.ws);
                n.ldb = nH;
                n.nbranch = ks_o;
                n.branch_stride = ws_stride;
            }
            n.n = nH;
            n.eps = p.eps;
            n.yh = H(w.xh);
            n.yl = H(w.xl);
            n.ldp = nH;
            n.tiled = tiled ? 1u : 0u;
            VX_CHECK(launch_seq_rmsnorm(s, n, T));
        }
        {
            ProfSpan sp(ctx, "prefill.swiglu");
            GemmArgs g;
            g.wk = L.gate.wt;
            g.epi = GEPI_SWIGLU;
            g.seg[0] = gemm_seg(L.gate, nF, nullptr, 0);
            g.seg[1] = gemm_seg(L.up, nF, nullptr, 0);
            if (tiled) {
                g.seg[0].pq = p.pw[l].gu.q;   // gate and up interleaved
                g.seg[0].pd = p.pw[l].gu.d;
                g.x_tiled = 1;
                g.o_tiled = 1;
            }
            g.nseg = 2;
            g.K = nH;
            g.T = T;
            g.xh = H(w.xh);
            g.xl = H(w.xl);
            g.ldx = nH;
            g.oh = H(w.ah);
            g.ol = H(w.al);
            g.ldp = nF;
            if (tiled && w.sk_grid && p.schedule != VX_PREFILL_TILES) {
                g.sk_ws = F(w.sk_ws);
                g.sk_cnt = static_cast<uint32_t *>(w.sk_cnt->ptr);
                g.sk_grid = w.sk_grid;
                g.sk_tail_first = p.schedule == VX_PREFILL_STREAMK_TAIL_FIRST ? 1u : 0u;
            }
            VX_CHECK(launch_gemm(s, g));
        }
        {
            ProfSpan sp(ctx, "prefill.down");
            GemmArgs g;
            g.wk = L.down.wt;
            g.epi = GEPI_RESIDUAL;
            g.seg[0] = gemm_seg(L.down, nH, F(w.h), nH);
            if (tiled) {
                g.seg[0].pq = p.pw[l].down.q;
                g.seg[0].pd = p.pw[l].down.d;
                g.x_tiled = 1;
            }
            g.K = nF;
            g.T = T;
            g.xh = H(w.ah);
            g.xl = H(w.al);
            g.ldx = nF;
            g.scale = p.residual_scale;
            g.ksplit = ks_down;
            if (ws_down) {
                g.ws = F(w.ws);
                g.ws_stride = ws_stride;
            }
            VX_CHECK(launch_gemm(s, g));
        }
    }
    if (ws_down) {   // the last layer's down partials
        ProfSpan sp(ctx, "prefill.norm");
        SeqNormArgs n;
        n.h = F(w.h);
        n.ldh = nH;
        n.n = nH;
        n.branch = F(w.ws);
        n.ldb = nH;
        n.nbranch = ks_down;
        n.branch_stride = ws_stride;
        VX_CHECK(launch_seq_rmsnorm(s, n, T));
    }
    return VX_OK;
}

}  // namespace vx
