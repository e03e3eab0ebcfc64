// AudioVAE decoder (AudioVaeEngine::decode_latents, audiovae.rs:330-372) over HIP,
// plus the per-op entry points of the vae_*.comp shaders.
//
// The engine keeps activations frame-major, [length][channels], so that the
// matrix-shaped parts run as GEMMs on MFMA:
//   model.0   depthwise k=7 causal conv                  k_vae_dwconv_fm
//   model.1   1x1 conv latent -> decoder_dim             k_vae_linear_fm (K = latent)
//   6 stages  scale/bias + snake + ConvTranspose1d(k=2s, stride s):
//               [pre(x[j]) | pre(x[j-1])] rows           k_vae_convt_input_fm
//               one GEMM, N = s * Cout, K = 2 Cin        k_gemm (repacked weights)
//             3 residual units (dilation 1, 3, 9):
//               snake -> depthwise k=7 dilated -> snake  k_vae_dwconv_fm
//               x += 1x1 conv + bias                     k_gemm residual (or k_vae_linear_fm)
//               (32 and 64 channels: both in one pass, k_vae_resunit_fm)
//   head      snake -> conv k=7 to one channel -> tanh   k_vae_head_fm
// Row j of the transposed convolution's output phases r = 0..s-1 is output time
// s j + r, so the GEMM's [L][s Cout] output is the frame-major [s L][Cout] output.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <string>

#include "vx_internal.h"

using namespace vx;

namespace {

constexpr uint32_t kStages = 6;
constexpr uint32_t kSrBuckets = 4;   // DECODER_SR_BUCKETS

struct Res {
    const __half *a1 = nullptr, *dw_w = nullptr, *dw_b = nullptr, *a2 = nullptr, *pw_w = nullptr, *pw_b = nullptr;
    uint32_t dilation = 1;
};
struct Stage {
    const __half *scale = nullptr, *bias = nullptr, *alpha = nullptr;   // scale/bias rows of the bucket
    __half *ct_w = nullptr;    // [s Cout][2 Cin]
    float *ct_b = nullptr;     // [s Cout]
    uint32_t stride = 1, cin = 0, cout = 0;
    Res res[3];
};

inline float *F(vx_buf *b) { return static_cast<float *>(b->ptr); }

}  // namespace

struct vx_audiovae {
    vx_ctx *ctx = nullptr;
    const vx_model *model = nullptr;
    vx_audiovae_config cfg{};
    const __half *m0_w = nullptr, *m0_b = nullptr, *m1_w = nullptr, *m1_b = nullptr;
    const __half *head_alpha = nullptr, *head_w = nullptr, *head_b = nullptr;
    Stage st[kStages];
    vx_buf *arena = nullptr;               // repacked transposed-conv weights and biases
    vx_buf *cur = nullptr, *tmp = nullptr, *x2 = nullptr, *io = nullptr, *wave = nullptr;
    uint64_t act_cap = 0, tmp_cap = 0, x2_cap = 0, io_cap = 0, wave_cap = 0;
};

namespace {

int find(const vx_model *m, const std::string &name, const vx_tensor_info **out) {
    auto it = m->by_name.find(name);
    if (it == m->by_name.end())
        return fail(VX_ERR_NOT_FOUND, "required GGUF tensor \"%s\" is missing", name.c_str());
    *out = &m->tensors[it->second];
    return VX_OK;
}

const __half *at(const vx_model *m, const vx_tensor_info *t) {
    return reinterpret_cast<const __half *>(m->raw + t->offset);
}

// require_alpha (audiovae.rs:134-138).
int alpha(const vx_model *m, const std::string &name, uint32_t c, const __half **out) {
    const vx_tensor_info *t;
    VX_CHECK(find(m, name, &t));
    uint64_t n = 1;
    for (uint32_t d = 0; d < t->n_dims; ++d) n *= t->dims[d];
    if (t->ggml_type != VX_DTYPE_F16) return fail(VX_ERR_SHAPE, "AudioVAE tensor %s is not F16", name.c_str());
    if (n != c) return fail(VX_ERR_SHAPE, "AudioVAE alpha %s has %llu values, expected %u", name.c_str(),
                            (unsigned long long)n, c);
    *out = at(m, t);
    return VX_OK;
}

// require_conv (audiovae.rs:139-150): weight dims [k, in/groups, out] (or
// [k, out/groups, in] transposed), F16; F16 bias of out values.
int conv(const vx_model *m, const std::string &base, uint32_t in_c, uint32_t out_c, uint32_t kernel,
         uint32_t groups, bool transpose, const __half **w, const __half **b) {
    const vx_tensor_info *t;
    VX_CHECK(find(m, base, &t));
    const uint64_t d1 = transpose ? out_c / groups : in_c / groups, d2 = transpose ? in_c : out_c;
    if (t->ggml_type != VX_DTYPE_F16) return fail(VX_ERR_SHAPE, "AudioVAE tensor %s is not F16", base.c_str());
    if (t->n_dims != 3 || t->dims[0] != kernel || t->dims[1] != d1 || t->dims[2] != d2)
        return fail(VX_ERR_SHAPE, "AudioVAE tensor %s dimensions, expected [%u, %llu, %llu]", base.c_str(), kernel,
                    (unsigned long long)d1, (unsigned long long)d2);
    if ((uintptr_t)at(m, t) & 15u) return fail(VX_ERR_SHAPE, "AudioVAE tensor %s is not 16-byte aligned", base.c_str());
    *w = at(m, t);
    return alpha(m, base + ".bias", out_c, b);
}

uint64_t decoder_max_elements(const vx_audiovae_config &c, uint64_t frames, uint64_t *x2_max) {
    uint64_t len = frames, ch = c.decoder_dim, mx = std::max<uint64_t>((uint64_t)c.latent_dim * frames, ch * len);
    *x2_max = 0;
    for (uint32_t i = 0; i < kStages; ++i) {
        *x2_max = std::max<uint64_t>(*x2_max, 2u * ch * len);
        len *= c.decoder_rates[i];
        ch /= 2u;
        mx = std::max<uint64_t>(mx, ch * len);
    }
    return std::max<uint64_t>(mx, len);
}

int grow(vx_ctx *ctx, vx_buf **b, uint64_t *cap, uint64_t floats) {
    if (*cap >= floats) return VX_OK;
    if (*b) {   // an earlier enqueued decode may still read or write it
        VX_HIP(hipStreamSynchronize(ctx->stream));
        vx_free(ctx, *b);
    }
    *b = nullptr;
    *cap = 0;
    VX_CHECK(vx_alloc(ctx, std::max<uint64_t>(floats, 64u) * 4u, b));
    *cap = floats;
    return VX_OK;
}

// y[t][n] (+)= b[n] + sum_k x[t][k] W[n][k]: the MFMA GEMM when K is a multiple
// of 128, else the short-K kernel. Few tiles: split K with atomic adds into a
// zeroed (store) or the residual (residual) output.
int linear(vx_ctx *ctx, const float *x, uint32_t ldx, const __half *w, const __half *b16, const float *b32,
           float *y, uint32_t ldy, uint32_t T, uint32_t N, uint32_t K, bool residual) {
    hipStream_t s = ctx->stream;
    if (K % 128u || (uintptr_t)w & 15u) {
        VaeLinearArgs a;
        a.x = x;
        a.ldx = ldx;
        a.w = w;
        a.bias = b16;
        a.bias_f32 = b32;
        a.y = y;
        a.ldy = ldy;
        a.T = T;
        a.N = N;
        a.K = K;
        a.residual = residual ? 1u : 0u;
        return launch_vae_linear_fm(s, a);
    }
    GemmArgs g;
    g.wk = WT_F16;
    g.epi = residual ? GEPI_RESIDUAL : GEPI_STORE;
    g.xf32 = 1;
    g.seg[0].w = w;
    g.seg[0].rows = N;
    g.seg[0].out = y;
    g.seg[0].ldo = ldy;
    g.seg[0].bias = b32 ? static_cast<const void *>(b32) : static_cast<const void *>(b16);
    g.seg[0].bias_dtype = b32 ? 0u : 1u;
    g.K = K;
    g.T = T;
    g.xf = x;
    g.ldx = ldx;
    const uint32_t tt = gemm_tile_tokens(g);
    const uint32_t tiles = ((N + 127u) / 128u) * ((T + tt - 1u) / tt);
    const uint32_t cus = ctx->props.multiProcessorCount > 0 ? (uint32_t)ctx->props.multiProcessorCount : 256u;
    uint32_t ks = (cus + tiles - 1u) / tiles;
    ks = std::min<uint32_t>(std::min<uint32_t>(ks, 8u), std::max<uint32_t>(1u, K / 256u));
    g.ksplit = std::max<uint32_t>(ks, 1u);
    if (g.ksplit > 1 && !residual) {
        if (ldy != N) g.ksplit = 1;   // the zero fill covers dense rows only
        else VX_CHECK(launch_fill_u32(s, reinterpret_cast<uint32_t *>(y), 0u, (uint64_t)T * N));
    }
    return launch_gemm(s, g);
}

// The decode of `frames` latent frames at in (frame-major) into wave.
int enqueue_decode(vx_audiovae *e, const float *in, uint32_t frames, float *wave) {
    vx_ctx *ctx = e->ctx;
    hipStream_t s = ctx->stream;
    const vx_audiovae_config &c = e->cfg;
    uint64_t x2_max = 0;
    const uint64_t act = decoder_max_elements(c, frames, &x2_max);
    // Every stage indexes its activations (and the output length) in 32 bits.
    if (act > 0xffffffffull || x2_max > 0xffffffffull)
        return fail(VX_ERR_UNSUPPORTED, "AudioVAE decoder activation exceeds the 32-bit index range");
    VX_CHECK(grow(ctx, &e->cur, &e->act_cap, act));
    VX_CHECK(grow(ctx, &e->tmp, &e->tmp_cap, act));
    VX_CHECK(grow(ctx, &e->x2, &e->x2_cap, x2_max));
    float *cur = F(e->cur), *tmp = F(e->tmp);
    uint32_t len = frames, ch = c.latent_dim;
    {
        ProfSpan sp(ctx, "audiovae.stem");
        VaeDwArgs d;   // model.0: depthwise k=7, left pad 6
        d.x = in;
        d.y = tmp;
        d.w = e->m0_w;
        d.b = e->m0_b;
        d.channels = ch;
        d.length = len;
        d.kernel = 7;
        d.dilation = 1;
        d.left_pad = 6;
        VX_CHECK(launch_vae_dwconv_fm(s, d));
        VX_CHECK(linear(ctx, tmp, ch, e->m1_w, e->m1_b, nullptr, cur, c.decoder_dim, len, c.decoder_dim, ch, false));
        ch = c.decoder_dim;
    }
    for (uint32_t i = 0; i < kStages; ++i) {
        const Stage &S = e->st[i];
        {
            ProfSpan sp(ctx, "audiovae.upsample");
            VaeConvtInArgs a;
            a.x = cur;
            a.x2 = F(e->x2);
            a.scale = S.scale;
            a.bias = S.bias;
            a.alpha = S.alpha;
            a.channels = ch;
            a.length = len;
            VX_CHECK(launch_vae_convt_input_fm(s, a));
            VX_CHECK(linear(ctx, F(e->x2), 2u * ch, S.ct_w, nullptr, S.ct_b, tmp, S.stride * S.cout, len,
                            S.stride * S.cout, 2u * ch, false));
        }
        std::swap(cur, tmp);
        len *= S.stride;
        ch = S.cout;
        for (const Res &R : S.res) {
            ProfSpan sp(ctx, "audiovae.residual");
            VaeResUnitArgs u;
            u.x = cur;
            u.y = tmp;
            u.a1 = R.a1;
            u.dw = R.dw_w;
            u.db = R.dw_b;
            u.a2 = R.a2;
            u.pw = R.pw_w;
            u.pb = R.pw_b;
            u.channels = ch;
            u.length = len;
            u.dilation = R.dilation;
            if (vae_resunit_eligible(u)) {
                VX_CHECK(launch_vae_resunit_fm(s, u));
                std::swap(cur, tmp);
                continue;
            }
            VaeDwArgs d;
            d.x = cur;
            d.y = tmp;
            d.w = R.dw_w;
            d.b = R.dw_b;
            d.alpha_in = R.a1;
            d.alpha_out = R.a2;
            d.channels = ch;
            d.length = len;
            d.kernel = 7;
            d.dilation = R.dilation;
            d.left_pad = 6u * R.dilation;
            VX_CHECK(launch_vae_dwconv_fm(s, d));
            VX_CHECK(linear(ctx, tmp, ch, R.pw_w, R.pw_b, nullptr, cur, ch, len, ch, ch, true));
        }
    }
    ProfSpan sp(ctx, "audiovae.head");
    VaeHeadArgs h;
    h.x = cur;
    h.y = wave;
    h.alpha = e->head_alpha;
    h.w = e->head_w;
    h.b = e->head_b;
    h.channels = ch;
    h.length = len;
    return launch_vae_head_fm(s, h);
}

int validate(const vx_audiovae_config &c, bool strict) {
    if (!c.latent_dim || !c.decoder_dim || !c.patch_size || c.decoder_dim % 64u)
        return fail(VX_ERR_INVALID_ARG, "AudioVAE config: latent %u, decoder %u (a multiple of 64), patch %u",
                    c.latent_dim, c.decoder_dim, c.patch_size);
    if (c.decoder_sr_bucket >= kSrBuckets) return fail(VX_ERR_INVALID_ARG, "sample-rate bucket %u", c.decoder_sr_bucket);
    static const uint32_t rates[kStages] = {8, 6, 5, 2, 2, 2};   // DECODER_RATES audiovae.rs:18
    for (uint32_t i = 0; i < kStages; ++i)
        if (c.decoder_rates[i] != rates[i]) return fail(VX_ERR_UNSUPPORTED, "AudioVAE decoder rates are 8,6,5,2,2,2");
    if (strict && (c.encoder_dim != 128 || c.latent_dim != 64 || c.decoder_dim != 2048 || c.sample_rate != 16000 ||
                   c.out_sample_rate != 48000 || c.patch_size != 4))
        return fail(VX_ERR_UNSUPPORTED, "unsupported VoxCPM2 AudioVAE geometry: enc=%u, latent=%u, dec=%u, sr=%u, "
                    "out_sr=%u, patch=%u", c.encoder_dim, c.latent_dim, c.decoder_dim, c.sample_rate,
                    c.out_sample_rate, c.patch_size);
    return VX_OK;
}

void free_all(vx_audiovae *e) {
    for (vx_buf **b : {&e->arena, &e->cur, &e->tmp, &e->x2, &e->io, &e->wave})
        if (*b) {
            vx_free(e->ctx, *b);
            *b = nullptr;
        }
}

double now_ms() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

const void *model_ptr(const vx_model *m, uint32_t offset) { return m->raw + offset; }

int check_span(const vx_model *m, uint32_t offset, uint64_t count, uint32_t dtype, const char *what) {
    const uint64_t bytes = count * (dtype == 1u ? 2u : 4u);
    if ((uint64_t)offset + bytes > m->raw_bytes)
        return fail(VX_ERR_BOUNDS, "%s reads past the model region", what);
    if (dtype > 1u) return fail(VX_ERR_UNSUPPORTED, "%s: AudioVAE scalars are F32 or F16", what);
    return VX_OK;
}

}  // namespace

extern "C" {

int vx_audiovae_create(vx_ctx *ctx, const vx_model *model, const vx_audiovae_config *cfg, uint32_t strict_geometry,
                       vx_audiovae **out) {
    if (!ctx || !model || !cfg || !out) return fail(VX_ERR_INVALID_ARG, "vx_audiovae_create: null argument");
    *out = nullptr;
    VX_CHECK(validate(*cfg, strict_geometry != 0));
    const vx_audiovae_config &c = *cfg;
    vx_audiovae *e = new vx_audiovae();
    e->ctx = ctx;
    e->model = model;
    e->cfg = c;
    auto bail = [&](int st) {
        free_all(e);
        delete e;
        return st;
    };
    int st;
    const uint32_t L = c.latent_dim;
    if ((st = conv(model, "audio_vae.decoder.model.0", L, L, 7, L, false, &e->m0_w, &e->m0_b)) ||
        (st = conv(model, "audio_vae.decoder.model.1", L, c.decoder_dim, 1, 1, false, &e->m1_w, &e->m1_b)))
        return bail(st);
    uint64_t arena = 0;
    uint32_t din = c.decoder_dim;
    for (uint32_t i = 0; i < kStages; ++i) {
        const uint32_t s = c.decoder_rates[i], dout = din / 2u;
        arena += ((uint64_t)s * dout * 2u * din * 2u + 255u) / 256u * 256u + ((uint64_t)s * dout * 4u + 255u) / 256u * 256u;
        din = dout;
    }
    if ((st = vx_alloc(ctx, arena, &e->arena))) return bail(st);
    uint8_t *cur = static_cast<uint8_t *>(e->arena->ptr);
    din = c.decoder_dim;
    for (uint32_t i = 0; i < kStages; ++i) {
        Stage &S = e->st[i];
        const uint32_t mi = i + 2, s = c.decoder_rates[i], dout = din / 2u;
        const std::string p = "audio_vae.decoder.model." + std::to_string(mi);
        S.stride = s;
        S.cin = din;
        S.cout = dout;
        // require_sr_embed (audiovae.rs:151-161): [channels, buckets] F16; the
        // bucket's row of each.
        for (int kind = 0; kind < 2; ++kind) {
            const std::string n = "audio_vae.decoder.sr_cond_model." + std::to_string(mi) +
                                  (kind ? ".bias_embed" : ".scale_embed");
            const vx_tensor_info *t;
            if ((st = find(model, n, &t))) return bail(st);
            if (t->ggml_type != VX_DTYPE_F16 || t->n_dims != 2 || t->dims[0] != din || t->dims[1] != kSrBuckets)
                return bail(fail(VX_ERR_SHAPE, "AudioVAE %s dimensions, expected [%u, %u] F16", n.c_str(), din,
                                 kSrBuckets));
            (kind ? S.bias : S.scale) = at(model, t) + (size_t)c.decoder_sr_bucket * din;
        }
        const __half *ctw, *ctb;
        if ((st = alpha(model, p + ".block.0.alpha", din, &S.alpha)) ||
            (st = conv(model, p + ".block.1", din, dout, 2u * s, 1, true, &ctw, &ctb)))
            return bail(st);
        S.ct_w = reinterpret_cast<__half *>(cur);
        cur += ((uint64_t)s * dout * 2u * din * 2u + 255u) / 256u * 256u;
        S.ct_b = reinterpret_cast<float *>(cur);
        cur += ((uint64_t)s * dout * 4u + 255u) / 256u * 256u;
        if ((st = launch_vae_repack_convt(ctx->stream, ctw, ctb, din, dout, s, S.ct_w, S.ct_b))) return bail(st);
        static const uint32_t dil[3] = {1, 3, 9};
        for (uint32_t r = 0; r < 3; ++r) {
            Res &R = S.res[r];
            const std::string q = p + ".block." + std::to_string(r + 2) + ".block";   // no NoiseBlock in VoxCPM2
            R.dilation = dil[r];
            if ((st = alpha(model, q + ".0.alpha", dout, &R.a1)) ||
                (st = conv(model, q + ".1", dout, dout, 7, dout, false, &R.dw_w, &R.dw_b)) ||
                (st = alpha(model, q + ".2.alpha", dout, &R.a2)) ||
                (st = conv(model, q + ".3", dout, dout, 1, 1, false, &R.pw_w, &R.pw_b)))
                return bail(st);
        }
        din = dout;
    }
    if ((st = alpha(model, "audio_vae.decoder.model.8.alpha", din, &e->head_alpha)) ||
        (st = conv(model, "audio_vae.decoder.model.9", din, 1, 7, 1, false, &e->head_w, &e->head_b)))
        return bail(st);
    if (hipStreamSynchronize(ctx->stream) != hipSuccess) return bail(fail(VX_ERR_HIP, "AudioVAE repack failed"));
    *out = e;
    return VX_OK;
}

int vx_audiovae_destroy(vx_audiovae *e) {
    if (!e) return VX_OK;
    (void)hipStreamSynchronize(e->ctx->stream);
    free_all(e);
    delete e;
    return VX_OK;
}

uint64_t vx_audiovae_scratch_bytes(const vx_audiovae *e) {
    if (!e) return 0;
    uint64_t n = 0;
    for (const vx_buf *b : {e->cur, e->tmp, e->x2, e->io, e->wave}) n += b ? b->bytes : 0u;
    return n;
}

int vx_audiovae_decode_latents_gpu(vx_audiovae *e, const vx_buf *frame_major, uint32_t frames, vx_buf *wave) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_audiovae_decode_latents_gpu: null engine");
    VX_CHECK(check_cancel(e->ctx));
    const vx_audiovae_config &c = e->cfg;
    if (frames == 0 || frames % c.patch_size)
        return fail(VX_ERR_SHAPE, "VoxCPM2 AudioVAE decode expects latent frames in groups of %u, got %u",
                    c.patch_size, frames);
    uint64_t x2_max = 0;
    if (decoder_max_elements(c, frames, &x2_max) > 0xffffffffull || x2_max > 0xffffffffull)
        return fail(VX_ERR_UNSUPPORTED, "AudioVAE decoder activation exceeds the 32-bit index range");
    VX_CHECK(need_buf(frame_major, (uint64_t)frames * c.latent_dim * 4u, "AudioVAE latents"));
    VX_CHECK(need_buf(wave, (uint64_t)frames * c.decoder_hop * 4u, "AudioVAE wave"));
    return enqueue_decode(e, static_cast<const float *>(frame_major->ptr), frames, F(wave));
}

int vx_audiovae_decode_latents(vx_audiovae *e, const float *frame_major, uint64_t n_values, float *wave,
                               uint64_t wave_cap, vx_audio_decode_stats *out) {
    if (!e) return fail(VX_ERR_INVALID_ARG, "vx_audiovae_decode_latents: null engine");
    VX_CHECK(check_cancel(e->ctx));
    const vx_audiovae_config &c = e->cfg;
    const uint64_t ld = c.latent_dim;
    if (!frame_major || n_values == 0 || n_values % ld)
        return fail(VX_ERR_SHAPE, "AudioVAE latent input must contain N*%u f32 values", c.latent_dim);
    for (uint64_t i = 0; i < n_values; ++i)
        if (!std::isfinite(frame_major[i])) return fail(VX_ERR_INVALID_ARG, "AudioVAE latent input contains NaN/inf");
    const uint64_t frames = n_values / ld;
    if (frames % c.patch_size)
        return fail(VX_ERR_SHAPE, "VoxCPM2 AudioVAE decode expects latent frames in groups of %u, got %llu",
                    c.patch_size, (unsigned long long)frames);
    uint64_t x2_max = 0;
    if (frames > 0xffffffffull || decoder_max_elements(c, frames, &x2_max) > 0xffffffffull ||
        x2_max > 0xffffffffull)
        return fail(VX_ERR_UNSUPPORTED, "AudioVAE decoder activation exceeds the 32-bit index range");
    const uint64_t samples = frames * c.decoder_hop;
    if (!wave || wave_cap < samples)
        return fail(VX_ERR_BOUNDS, "wave buffer holds %llu floats; the decode writes %llu",
                    (unsigned long long)wave_cap, (unsigned long long)samples);
    vx_ctx *ctx = e->ctx;
    VX_CHECK(grow(ctx, &e->io, &e->io_cap, n_values));
    VX_CHECK(grow(ctx, &e->wave, &e->wave_cap, samples));
    VX_HIP(hipStreamSynchronize(ctx->stream));
    const double t0 = now_ms();
    VX_HIP(hipMemcpyAsync(e->io->ptr, frame_major, n_values * 4u, hipMemcpyHostToDevice, ctx->stream));
    VX_CHECK(enqueue_decode(e, F(e->io), (uint32_t)frames, F(e->wave)));
    VX_CHECK(vx_download(ctx, e->wave, 0, wave, samples * 4u));
    const double ms = now_ms() - t0;
    double sum = 0, sq = 0;
    float peak = 0.f;
    for (uint64_t i = 0; i < samples; ++i) {
        if (!std::isfinite(wave[i])) return fail(VX_ERR_STATE, "AudioVAE decoder produced NaN/inf");
        sum += wave[i];
        sq += (double)wave[i] * wave[i];
        peak = std::max(peak, std::fabs(wave[i]));
    }
    if (out) {
        out->latent_frames = (uint32_t)frames;
        out->latent_patches = (uint32_t)(frames / c.patch_size);
        out->output_samples = (uint32_t)samples;
        out->output_sample_rate = c.out_sample_rate;
        out->duration_seconds = (double)samples / c.out_sample_rate;
        out->checksum = sum;
        out->l2 = std::sqrt(sq);
        out->peak = peak;
        out->decode_ms = ms;
        out->scratch_bytes = vx_audiovae_scratch_bytes(e);
    }
    return VX_OK;
}

// ------------------------------------------------------------ per-op entry points
int vx_vae_conv1d(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y, const vx_vae_conv_push *pc) {
    if (!ctx || !model || !pc) return fail(VX_ERR_INVALID_ARG, "vx_vae_conv1d: null argument");
    if (!pc->groups || pc->in_channels % pc->groups || pc->out_channels % pc->groups || !pc->stride || !pc->kernel)
        return fail(VX_ERR_INVALID_ARG, "vx_vae_conv1d: groups/stride/kernel");
    VX_CHECK(need_buf(x, (uint64_t)pc->in_channels * pc->in_length * 4u, "vx_vae_conv1d x"));
    VX_CHECK(need_buf(y, (uint64_t)pc->out_channels * pc->out_length * 4u, "vx_vae_conv1d y"));
    VX_CHECK(check_span(model, pc->weight_offset,
                        (uint64_t)pc->out_channels * (pc->in_channels / pc->groups) * pc->kernel, pc->weight_dtype,
                        "vx_vae_conv1d weight"));
    if (pc->has_bias) VX_CHECK(check_span(model, pc->bias_offset, pc->out_channels, pc->bias_dtype, "vx_vae_conv1d bias"));
    VaeConvArgs a;
    a.x = static_cast<const float *>(x->ptr);
    a.y = F(y);
    a.w = model_ptr(model, pc->weight_offset);
    a.bias = pc->has_bias ? model_ptr(model, pc->bias_offset) : nullptr;
    a.w_dtype = pc->weight_dtype;
    a.bias_dtype = pc->bias_dtype;
    a.in_channels = pc->in_channels;
    a.out_channels = pc->out_channels;
    a.in_length = pc->in_length;
    a.out_length = pc->out_length;
    a.kernel = pc->kernel;
    a.stride = pc->stride;
    a.dilation = pc->dilation;
    a.groups = pc->groups;
    a.left_pad = pc->left_pad;
    ProfSpan sp(ctx, "audiovae.conv1d");
    return launch_vae_conv1d_cm(ctx->stream, a, false);
}

int vx_vae_convtranspose1d(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y,
                           const vx_vae_convt_push *pc) {
    if (!ctx || !model || !pc) return fail(VX_ERR_INVALID_ARG, "vx_vae_convtranspose1d: null argument");
    if (!pc->groups || pc->in_channels % pc->groups || pc->out_channels % pc->groups || !pc->stride || !pc->kernel)
        return fail(VX_ERR_INVALID_ARG, "vx_vae_convtranspose1d: groups/stride/kernel");
    VX_CHECK(need_buf(x, (uint64_t)pc->in_channels * pc->in_length * 4u, "vx_vae_convtranspose1d x"));
    VX_CHECK(need_buf(y, (uint64_t)pc->out_channels * pc->out_length * 4u, "vx_vae_convtranspose1d y"));
    VX_CHECK(check_span(model, pc->weight_offset,
                        (uint64_t)pc->in_channels * (pc->out_channels / pc->groups) * pc->kernel, pc->weight_dtype,
                        "vx_vae_convtranspose1d weight"));
    if (pc->has_bias)
        VX_CHECK(check_span(model, pc->bias_offset, pc->out_channels, pc->bias_dtype, "vx_vae_convtranspose1d bias"));
    VaeConvArgs a;
    a.x = static_cast<const float *>(x->ptr);
    a.y = F(y);
    a.w = model_ptr(model, pc->weight_offset);
    a.bias = pc->has_bias ? model_ptr(model, pc->bias_offset) : nullptr;
    a.w_dtype = pc->weight_dtype;
    a.bias_dtype = pc->bias_dtype;
    a.in_channels = pc->in_channels;
    a.out_channels = pc->out_channels;
    a.in_length = pc->in_length;
    a.out_length = pc->out_length;
    a.kernel = pc->kernel;
    a.stride = pc->stride;
    a.groups = pc->groups;
    ProfSpan sp(ctx, "audiovae.convtranspose1d");
    return launch_vae_conv1d_cm(ctx->stream, a, true);
}

int vx_vae_snake(vx_ctx *ctx, const vx_model *model, const vx_buf *x, vx_buf *y, const vx_vae_snake_push *pc) {
    if (!ctx || !model || !pc) return fail(VX_ERR_INVALID_ARG, "vx_vae_snake: null argument");
    const uint64_t n = (uint64_t)pc->channels * pc->length;
    VX_CHECK(need_buf(x, n * 4u, "vx_vae_snake x"));
    VX_CHECK(need_buf(y, n * 4u, "vx_vae_snake y"));
    VX_CHECK(check_span(model, pc->alpha_offset, pc->channels, pc->dtype, "vx_vae_snake alpha"));
    ProfSpan sp(ctx, "audiovae.snake");
    return launch_vae_snake_cm(ctx->stream, static_cast<const float *>(x->ptr), F(y),
                               model_ptr(model, pc->alpha_offset), pc->dtype, pc->channels, pc->length);
}

int vx_vae_scale_bias(vx_ctx *ctx, const vx_model *model, vx_buf *x, const vx_vae_scale_push *pc) {
    if (!ctx || !model || !pc) return fail(VX_ERR_INVALID_ARG, "vx_vae_scale_bias: null argument");
    if (pc->bucket >= pc->buckets) return fail(VX_ERR_INVALID_ARG, "vx_vae_scale_bias: bucket %u of %u", pc->bucket,
                                               pc->buckets);
    VX_CHECK(need_buf(x, (uint64_t)pc->channels * pc->length * 4u, "vx_vae_scale_bias x"));
    const uint64_t rows = (uint64_t)pc->buckets * pc->channels;
    VX_CHECK(check_span(model, pc->scale_offset, rows, pc->scale_dtype, "vx_vae_scale_bias scale"));
    VX_CHECK(check_span(model, pc->bias_offset, rows, pc->bias_dtype, "vx_vae_scale_bias bias"));
    ProfSpan sp(ctx, "audiovae.scale_bias");
    return launch_vae_scale_bias_cm(ctx->stream, F(x), model_ptr(model, pc->scale_offset),
                                    model_ptr(model, pc->bias_offset), pc->scale_dtype, pc->bias_dtype, pc->channels,
                                    pc->length, pc->bucket);
}

int vx_vae_add(vx_ctx *ctx, vx_buf *a, const vx_buf *b, const vx_vae_grid_push *pc) {
    if (!ctx || !pc) return fail(VX_ERR_INVALID_ARG, "vx_vae_add: null argument");
    const uint64_t n = (uint64_t)pc->channels * pc->length;
    VX_CHECK(need_buf(a, n * 4u, "vx_vae_add a"));
    VX_CHECK(need_buf(b, n * 4u, "vx_vae_add b"));
    ProfSpan sp(ctx, "audiovae.add");
    return launch_vae_add_cm(ctx->stream, F(a), static_cast<const float *>(b->ptr), pc->channels, pc->length);
}

int vx_vae_tanh(vx_ctx *ctx, vx_buf *x, uint32_t n) {
    if (!ctx) return fail(VX_ERR_INVALID_ARG, "vx_vae_tanh: null context");
    VX_CHECK(need_buf(x, (uint64_t)n * 4u, "vx_vae_tanh x"));
    ProfSpan sp(ctx, "audiovae.tanh");
    return launch_vae_tanh(ctx->stream, F(x), n);
}

}  // extern "C"
