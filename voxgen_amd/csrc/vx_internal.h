// Internal declarations shared by the host runtime (.cpp) and kernel (.hip) files
// of libvoxhip.so. Nothing here is part of the public ABI (include/voxhip.h).
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/voxhip.h"

namespace vx {

// ------------------------------------------------------------------ errors
void set_error_v(const char *fmt, va_list ap);
int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

#define VX_HIP(call)                                                                      \
    do {                                                                                  \
        hipError_t e_ = (call);                                                           \
        if (e_ != hipSuccess)                                                             \
            return ::vx::fail(VX_ERR_HIP, "%s failed: %s (%s:%d)", #call,                 \
                              hipGetErrorString(e_), __FILE__, __LINE__);                 \
    } while (0)

#define VX_CHECK(expr)                        \
    do {                                      \
        int s_ = (expr);                      \
        if (s_ != VX_OK) return s_;           \
    } while (0)

// Launch-error check after a <<<>>> launch.
#define VX_LAUNCHED(name)                                                                 \
    do {                                                                                  \
        hipError_t e_ = hipGetLastError();                                                \
        if (e_ != hipSuccess)                                                             \
            return ::vx::fail(VX_ERR_HIP, "launch of %s failed: %s", name,                \
                              hipGetErrorString(e_));                                     \
    } while (0)

// ------------------------------------------------------- timeline build
// A library built with -DVX_STAMPS (never the shipped one) records a timeline of
// the decode kernels: each wave writes one (start, end) pair of s_memrealtime
// ticks into slots that stamp_slots hands out launch by launch when the launch
// is enqueued or captured, so every replay of a captured graph rewrites its own
// launches' slots (vx_diag_timeline_arm / _read).
#ifdef VX_STAMPS
enum StampKind : uint32_t {
    ST_QKV = 1, ST_ATTN_CHUNK = 2, ST_ATTN_STREAM = 3, ST_ATTN_OUT = 4, ST_SWIGLU = 5, ST_MATVEC = 6,
    ST_GEMM_SK = 7, ST_DENSE_ATTN = 8, ST_SEQ_NORM = 9,   // the LocDiT short-batch stack
};
// Slots for `waves` waves, or nullptr when no timeline is armed or it is full.
uint64_t *stamp_slots(uint32_t kind, uint64_t waves);
struct WaveStamp {
    uint64_t *slot;
    uint64_t t0 = 0;
    __device__ explicit WaveStamp(uint64_t *base) : slot(base) {
        if (slot) {
            const uint64_t wg = blockIdx.x + (uint64_t)gridDim.x * (blockIdx.y + (uint64_t)gridDim.y * blockIdx.z);
            slot += 2 * (wg * (blockDim.x >> 6) + (threadIdx.x >> 6));
            t0 = __builtin_amdgcn_s_memrealtime();
        }
    }
    __device__ ~WaveStamp() {
        if (slot && (threadIdx.x & 63) == 0) {
            const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
            slot[0] = t0;
            slot[1] = t1;
        }
    }
};
#define VX_STAMP_FIELD uint64_t *stamps = nullptr;
#define VX_WAVE_STAMP(p) ::vx::WaveStamp vx_wave_stamp_(p)
#define VX_SET_STAMPS(args, kind, waves) ((args).stamps = ::vx::stamp_slots((kind), (waves)))
#else
#define VX_STAMP_FIELD
#define VX_WAVE_STAMP(p) ((void)0)
#define VX_SET_STAMPS(args, kind, waves) ((void)0)
#endif

// ------------------------------------------------------- weight references
enum WeightType : uint32_t { WT_Q8 = 0, WT_F16 = 1, WT_F32 = 2 };

// A matrix the kernels can stream. Q8_0 matrices with cols % 1024 == 0 are
// referenced in the repacked layout (model.cpp), built for wave64 loads in which
// lane l owns columns 1024g + 256k + 4l + j (k, j < 4) of every 1024-column
// group g of a row:
//   qs: int8 [rows][cols]; byte 1024g + 16l + 4k + j of a row holds the quant of
//       column 1024g + 256k + 4l + j, so lane l reads its 16 quants of group g
//       with one 16-byte load and a wave reads 1 KB of contiguous bytes;
//   d:  f16 [rows][cols/32]; element 32g + 4m + k of a row is the scale of block
//       32g + 8k + m (the block of lane 8m..8m+7's chunk k), so lane l reads its
//       four scales of group g with one 8-byte load.
// The x values a lane needs, x[1024g + 256k + 4l .. +3], are then float4 loads
// that are contiguous across the wave. Other Q8_0 matrices have ptr == nullptr
// and are read from the raw GGUF region. F16/F32 matrices use the GGUF layout.
struct WRef {
    uint32_t wt = WT_F16;        // WeightType of the fast path
    uint32_t dtype = 1;          // GGML dtype code
    const void *ptr = nullptr;   // qs (Q8) or element data (F16/F32)
    const __half *d = nullptr;   // Q8 scales
    uint32_t rows = 0, cols = 0; // matrix extent available
    const uint8_t *raw = nullptr;   // raw data region on the device
    uint32_t raw_offset = 0;        // byte offset of the tensor in the region
};

// ------------------------------------------------------------- profiling
struct ProfPending {
    std::string name;
    hipEvent_t start, end;
};
struct ProfTotal {
    double total_ms = 0.0;
    uint64_t calls = 0;
};

}  // namespace vx

struct vx_buf {
    void *ptr = nullptr;
    uint64_t bytes = 0;
    bool owned = true;
};

struct vx_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    bool capturing = false;
    bool prof_enabled = false;
    std::vector<vx::ProfPending> prof_pending;
    std::vector<hipEvent_t> event_pool;
    std::unordered_map<std::string, vx::ProfTotal> prof_totals;
    std::vector<std::string> prof_order;
    hipDeviceProp_t props{};
    void *noalloc_scratch = nullptr;  // device address of this GPU's no-allocation scratch
    const uint32_t *cancel = nullptr; // caller's cancellation word (vx_set_cancel_flag), nullable
};

struct vx_model {
    vx_ctx *ctx = nullptr;
    uint8_t *raw = nullptr;       // device copy of the data region
    uint64_t raw_bytes = 0;
    uint8_t *packed = nullptr;    // device arena of repacked Q8_0 matrices
    uint64_t packed_bytes = 0;
    std::vector<vx_tensor_info> tensors;
    std::vector<uint64_t> packed_qs;   // per tensor: offset of qs in arena (or UINT64_MAX)
    std::vector<uint64_t> packed_d;    // per tensor: offset of d in arena
    std::unordered_map<uint64_t, uint32_t> by_offset;
    std::unordered_map<std::string, uint32_t> by_name;
};

struct vx_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

namespace vx {

// ------------------------------------------------------------ runtime glue
// Profiling span around enqueued work (no-op unless ctx->prof_enabled and not
// capturing). Mirrors gpu_profile_begin/end (vulkan.rs:587-612).
class ProfSpan {
  public:
    ProfSpan(vx_ctx *ctx, const char *name);
    ~ProfSpan();
    ProfSpan(const ProfSpan &) = delete;
    ProfSpan &operator=(const ProfSpan &) = delete;

  private:
    vx_ctx *ctx_;
    hipEvent_t start_ = nullptr;
    std::string name_;
};
int collect_profile(vx_ctx *ctx);

// Model lookups.
int find_tensor_at(const vx_model *m, uint32_t offset, const vx_tensor_info **out);
// Resolve a weight matrix at `offset` whose GGUF dims are [cols, >=rows].
int resolve_matrix(const vx_model *m, uint32_t offset, uint32_t dtype, uint32_t rows, uint32_t cols,
                   WRef *out, const char *what);
// Resolve a vector of n elements of `dtype` (0 = F32, 1 = F16) at `offset`.
int resolve_vector(const vx_model *m, uint32_t offset, uint32_t dtype, uint32_t n,
                   const void **out, const char *what);

// Buffer validation.
int need_buf(const vx_buf *b, uint64_t bytes, const char *what);
// VX_ERR_CANCELLED when the context's cancellation word is set (acquire load).
int check_cancel(const vx_ctx *ctx);

// ------------------------------------------------------------ launchers
// Epilogues of the matvec kernel.
enum Epilogue : int { EPI_STORE = 0, EPI_BIAS = 1, EPI_FUSION = 2, EPI_RESIDUAL = 3 };

struct MatvecLaunch {
    WRef w;
    const float *xl = nullptr;    // x = xl[0..left_cols) ++ xr
    const float *xr = nullptr;
    uint32_t left_cols = 0;
    uint32_t rows = 0, cols = 0, row_base = 0;
    float alpha = 1.0f;
    int epi = EPI_STORE;
    const void *bias = nullptr;
    uint32_t bias_dtype = 0;
    float *y = nullptr;           // STORE/BIAS/FUSION output; RESIDUAL: hidden (in/out)
    float *y2 = nullptr;          // FUSION snapshot; RESIDUAL: branch (nullable)
    float scale = 1.0f;           // RESIDUAL scale
};
int launch_matvec(hipStream_t s, const MatvecLaunch &a);

struct SwigluLaunch {
    WRef g, u;
    const float *x = nullptr;     // plain input, or hidden when norm != nullptr
    const float *norm = nullptr;  // fused rmsnorm weight (f32), nullable
    float eps = 0.0f;
    uint32_t rows = 0, cols = 0, row_base = 0;
    float *y = nullptr;
};
int launch_swiglu(hipStream_t s, const SwigluLaunch &a);

struct QkvFusedLaunch {
    WRef q, k, v;
    const float *hidden = nullptr;
    const float *norm = nullptr;
    float eps = 0.0f;
    uint32_t q_rows = 0, kv_rows = 0, cols = 0, head_dim = 0;
    const float *factors = nullptr;
    float theta = 10000.0f, scaling = 1.0f;
    uint32_t layer = 0, context = 0;
    float *qo = nullptr, *ko = nullptr, *vo = nullptr;
    __half *kc = nullptr, *vc = nullptr;
    const uint32_t *position = nullptr;
    const float2 *rope_cs = nullptr;   // nullable: per-step (cos, sin) table from launch_rope_table
    bool no_rope = false;              // q/k stored unrotated (a stack without RoPE)
};
int launch_qkv_fused(hipStream_t s, const QkvFusedLaunch &a);

// 16-byte store to LDS written as four dwords (the compiler still emits one
// ds_write_b128). Assigning a HIP uint4 through a reinterpret_cast pointer into an
// f16 LDS array kept the source registers in scratch memory.
__device__ __forceinline__ void lds_st16(void *p, const uint4 &v) {
    uint32_t *d = static_cast<uint32_t *>(p);
    d[0] = v.x;
    d[1] = v.y;
    d[2] = v.z;
    d[3] = v.w;
}

struct AttnLaunch {
    const float *q = nullptr;
    const __half *kc = nullptr, *vc = nullptr;
    float *out = nullptr;
    float *partials = nullptr;
    const uint32_t *position = nullptr;
    uint32_t layer = 0, context = 0, head_dim = 0, q_heads = 0, kv_heads = 0, splits = 0;
};
// Partials: 256 bytes of header, then per (q head, split) a record of head_dim+4
// floats: max, sum, 2 pad words, acc[head_dim].
uint64_t attn_scratch_bytes(uint32_t head_dim, uint32_t q_heads, uint32_t kv_heads, uint32_t splits);
constexpr uint32_t kMaxAttnSplits = 64;     // splits of a standalone attention call
constexpr uint32_t kMaxFoldedSplits = 16;   // splits the attn_out prologue merges
constexpr uint32_t kShortSplits = 8;        // splits of a short context (at most 64 keys each at 512)
constexpr uint32_t kAttnMinChunk = 32;      // fewest keys per active split
// Split of the context [0, position] into `active` contiguous chunks, identical
// in every kernel that reads the partials.
struct SplitPlan {
    uint32_t n, active, chunk;
};
// Keys of a split when they do not depend on the position: ceil(context /
// splits), used whenever it is at most kAttnFixedChunk, so that the attention
// workgroups can fetch their keys before the position arrives.
constexpr uint32_t kAttnFixedChunk = 64;   // one key tile of k_attn_chunk
__host__ __device__ __forceinline__ uint32_t attn_fixed_chunk(uint32_t context, uint32_t splits) {
    return (context + splits - 1u) / splits;
}
// The splits of positions 0..pos: slice s is keys [s * chunk, min(n, (s + 1) * chunk)),
// for s < active. Every kernel that writes or merges the slices computes it the
// same way from the same position.
__device__ __forceinline__ SplitPlan split_plan_at(uint32_t pos, uint32_t context, uint32_t splits) {
    if (pos >= context) pos = context - 1u;
    SplitPlan p;
    p.n = pos + 1u;
    const uint32_t fc = attn_fixed_chunk(context, splits);
    if (fc <= kAttnFixedChunk) {
        p.chunk = fc;
        p.active = (p.n + fc - 1u) / fc;
    } else {
        p.active = min(splits, (p.n + kAttnMinChunk - 1u) / kAttnMinChunk);
        p.chunk = (p.n + p.active - 1u) / p.active;
    }
    return p;
}
__device__ __forceinline__ SplitPlan split_plan(const uint32_t *position, uint32_t context, uint32_t splits) {
    return split_plan_at(*position, context, splits);
}
// attn_out matvec (EPI_RESIDUAL) whose x is merged from the attention partials.
struct AttnOutLaunch {
    MatvecLaunch mv;
    const float *partials = nullptr;   // the AttnLaunch scratch (header + records)
    float *attn_out = nullptr;         // nullable: also store the merged attention vector
    const uint32_t *position = nullptr;
    uint32_t context = 0, splits = 0, q_heads = 0, head_dim = 0;
};
int launch_attn_out(hipStream_t s, const AttnOutLaunch &a);
// Partials only (k_attn_chunk), and partials + per-head merge (k_attn_combine).
int launch_attn_partials(hipStream_t s, const AttnLaunch &a);
// The same partials from k_attn_rows (4 or 8 waves per slice): every wave
// streams its own keys with no barrier inside the key loop.
int launch_attn_stream(hipStream_t s, const AttnLaunch &a, uint32_t waves);
int launch_attn_decode(hipStream_t s, const AttnLaunch &a);
// The per-head merge of the partial records alone (k_attn_combine) into a.out.
int launch_attn_combine(hipStream_t s, const AttnLaunch &a);

// Reference-granular kernels.
int launch_rmsnorm(hipStream_t s, const float *x, float *y, const float *w, uint32_t n, float eps,
                   uint32_t *advance_position);
int launch_residual_rmsnorm(hipStream_t s, float *h, const float *branch, float *y, const float *w,
                            uint32_t n, float eps, float scale);
int launch_rope(hipStream_t s, float *q, float *k, const float *factors, uint32_t position,
                const uint32_t *dev_position, uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim,
                float theta, float scaling);
int launch_store_kv(hipStream_t s, const float *k, const float *v, __half *kc, __half *vc,
                    uint32_t layer, uint32_t position, const uint32_t *dev_position,
                    uint32_t context, uint32_t kv_dim);
int launch_attn_scores(hipStream_t s, const float *q, const __half *kc, float *scores,
                       uint32_t layer, uint32_t context, uint32_t position,
                       const uint32_t *dev_position, uint32_t head_dim, uint32_t q_per_kv,
                       uint32_t kv_heads, uint32_t q_heads);
int launch_softmax(hipStream_t s, float *scores, uint32_t heads, uint32_t context,
                   uint32_t position, const uint32_t *dev_position);
int launch_attn_values(hipStream_t s, const float *scores, const __half *vc, float *out,
                       uint32_t layer, uint32_t context, uint32_t position,
                       const uint32_t *dev_position, uint32_t head_dim, uint32_t q_per_kv,
                       uint32_t kv_heads, uint32_t q_heads);
// Token id from `token`, or dev_tokens[dev_position[0]] when dev_tokens is set
// (tokens_len entries). Ids >= vocab produce NaN rows instead of reading out of range.
int launch_embedding(hipStream_t s, const uint8_t *raw, uint32_t weight_offset, uint32_t dtype,
                     uint32_t cols, uint32_t token, const uint32_t *dev_tokens,
                     const uint32_t *dev_position, uint32_t vocab, float alpha, float *hidden,
                     uint32_t tokens_len = 0);
// table[i] = (cos, sin)(angle_i) * scaling at the device position (i < head_dim/2).
int launch_rope_table(hipStream_t s, const float *factors, const uint32_t *position, uint32_t head_dim,
                      float theta, float scaling, float2 *table);
int launch_set_step(hipStream_t s, uint32_t *tokens, uint32_t *position, uint32_t pos,
                    uint32_t token, int write_token);
int launch_fill_u32(hipStream_t s, uint32_t *dst, uint32_t value, uint64_t count);
int launch_dequant(hipStream_t s, const WRef &w, uint32_t rows, uint32_t cols, float *out);

// ------------------------------------------------- token-batched (seq) kernels
// Projection GEMM C[t][n] = sum_k X[t][k] W[n][k] on MFMA (kernels_seq.hip).
enum GemmEpilogue : uint32_t {
    GEPI_STORE = 0,     // out[t][n] = alpha * (acc + bias[n])   (atomic add when split)
    GEPI_RESIDUAL = 1,  // out[t][n] += scale * (acc [+ bias[n]]) (atomic add when split)
    GEPI_SWIGLU = 2     // seg 0 = gate, seg 1 = up: silu(g) * u -> seg[0].out and/or planes
};
struct GemmSeg {                    // one weight matrix covering part of N
    const int8_t *qs = nullptr;     // Q8_0: repacked quants (WRef::ptr) ...
    const __half *d = nullptr;      // ... and scales (WRef::d)
    const int8_t *pq = nullptr;     // Q8_0 in the prefill-GEMM layout (PrefillMatrix), nullable ...
    const float *pd = nullptr;      // ... and its f32 scales
    const __half *w = nullptr;      // F16: [rows][K]
    uint32_t rows = 0;
    uint32_t tile0 = 0;             // set by launch_gemm
    float *out = nullptr;           // [T][ldo] f32
    uint32_t ldo = 0;
    const void *bias = nullptr;     // GEPI_STORE: f32 (bias_dtype 0) or f16 (1), nullable
    uint32_t bias_dtype = 0;
};
struct GemmArgs {
    uint32_t wk = WT_Q8;            // WT_Q8 (repacked, K % 1024 == 0) or WT_F16 (K % 128 == 0)
    uint32_t epi = GEPI_STORE;
    uint32_t xf32 = 0;              // 1: X is f32 (xf), split to hi/lo in the kernel
    GemmSeg seg[3];
    uint32_t nseg = 1;
    uint32_t K = 0, T = 0;
    const __half *xh = nullptr, *xl = nullptr;  // X as hi/lo f16 planes [T][ldx]
    const float *xf = nullptr;                  // X as f32 [T][ldx]
    uint32_t ldx = 0;
    float alpha = 1.f, scale = 1.f;
    __half *oh = nullptr, *ol = nullptr;        // GEPI_SWIGLU plane output [T][ldp]
    uint32_t ldp = 0;
    uint32_t ksplit = 1;
    uint32_t ntn = 0, ntm = 0;                  // set by launch_gemm
    uint32_t x_tiled = 0;           // 1: xh/xl are in the tiled plane layout (tiled_plane_index)
    uint32_t o_tiled = 0;           // 1: GEPI_SWIGLU writes oh/ol in the tiled plane layout
    // GEPI_RESIDUAL with ksplit > 1 on the prefill-layout kernel: when set, split
    // s stores scale * (its partial product) to ws + s * ws_stride ([T][ldo]) with
    // plain stores instead of adding to out; the consumer adds the partials.
    float *ws = nullptr;
    uint64_t ws_stride = 0;
    // GEPI_STORE with ksplit > 1 on the prefill-layout kernel: when set, split s
    // stores alpha * (its partial product) to out + s * ws_stride (each segment's
    // [T][ldo]) with plain stores instead of atomic adds; the consumer sums them.
    uint32_t split_store = 0;
    uint32_t wide = 0;              // set by launch_gemm: plain-store epilogues may use 16-byte stores
    VX_STAMP_FIELD
    // GEPI_SWIGLU on the prefill-layout kernel with tiled plane output: with
    // sk_grid set (a multiple of 8, normally the CU count) and a little more than
    // sk_grid tiles, the tiles' blocks are cut into sk_grid equal ranges, one
    // workgroup each (stream-K). sk_ws holds 2 * sk_grid tile parts of
    // kSkTileFloats floats, sk_cnt sk_grid counters, zero before a launch and
    // zero again after it.
    float *sk_ws = nullptr;
    uint32_t *sk_cnt = nullptr;
    uint32_t sk_grid = 0;
    uint32_t sk_per = 0;            // blocks per workgroup, set by launch_gemm
    uint32_t sk_tail_first = 0;     // 1: each workgroup computes its tile tail before its head
    // 1: the short-batch F16 kernel's operand layout: the weights (seg[i].w) and
    // the X planes are in the fragment layout (frag16_index), and GEPI_SWIGLU
    // writes oh/ol in it (width seg[0].rows).
    uint32_t frag = 0;
    // Short-batch kernel only. xn (nullable): X is rmsnorm(xn) * xn_w with xn an
    // f32 [T][K] matrix in frag32_index order; the kernel multiplies by xn_w and
    // splits to hi/lo in registers, and 1/rms of each row (from the sum of squares
    // of its xn values, eps xn_eps) scales the products: GEPI_SWIGLU applies it
    // before the SiLU; GEPI_STORE leaves the products unscaled and the workgroups
    // of the first row tile store each K slab's sums of squares to xn_ss +
    // slab * xn_ss_stride ([T]), for the consumer to finish the norm.
    const float *xn = nullptr, *xn_w = nullptr;
    float xn_eps = 0.f;
    float *xn_ss = nullptr;
    uint64_t xn_ss_stride = 0;
    // Short-batch GEPI_STORE only, nullable: add alpha * the product (every K slab)
    // to res_frag, an f32 [T][seg[0].rows] matrix in frag32_index order, with
    // atomic adds (a residual update; no slabs).
    float *res_frag = nullptr;
};
int launch_gemm(hipStream_t s, const GemmArgs &a);
// Short-batch F16 kernel (kernels_skinny.hip): operands in the fragment layout
// (GemmArgs::frag), T <= 128, GEPI_STORE (split K only as partial slabs,
// split_store) or GEPI_SWIGLU. launch_gemm takes every call with frag set.
bool gemm_skinny_eligible(const GemmArgs &a);
int launch_gemm_skinny(hipStream_t s, GemmArgs a);
// Fragment layout of a matrix with K columns (K % 32 == 0) and rows padded to a
// multiple of 16: one contiguous 1 KB block per 16 rows x 32 columns, blocks of a
// 16-row group consecutive along K; inside a block, lane l = r + 16 g (r = row
// % 16, g = column % 32 / 8) holds columns 8g..8g+7 of row r, eight halves. A
// wave64 16-byte load of one block is then exactly the A or B operand of
// v_mfma_f32_16x16x32_f16 (rows along M or N, the block's 32 columns along K),
// and every operand load is 1 KB of contiguous bytes.
__host__ __device__ __forceinline__ size_t frag16_index(uint32_t r, uint32_t c, uint32_t K) {
    return (((size_t)(r >> 4) * (K >> 5) + (c >> 5)) << 9) + ((((c >> 3) & 3u) << 4) + (r & 15u)) * 8u + (c & 7u);
}
// The same fragment order for an f32 matrix (the LocDiT residual stream): one 2 KB
// block per 16 rows x 32 columns, in two 1 KB halves, half h holding for every
// lane l = r + 16 g the four columns 8g + 4h .. 8g + 4h + 3 of row r. A wave's two
// 16-byte loads of a block give each lane the eight values of its f16 fragment,
// each load 1 KB of contiguous bytes.
__host__ __device__ __forceinline__ size_t frag32_index(uint32_t r, uint32_t c, uint32_t K) {
    return (((size_t)(r >> 4) * (K >> 5) + (c >> 5)) << 9) + (((c >> 2) & 1u) << 8) +
           ((((c >> 3) & 3u) << 4) + (r & 15u)) * 4u + (c & 3u);
}
// Rewrites an F16 [rows][K] row-major matrix in the fragment layout (rows padded
// to a multiple of 16 with zeros): dst holds ceil(rows/16)*16*K halves.
int launch_repack_frag16(hipStream_t s, const __half *src, __half *dst, uint32_t rows, uint32_t K);
// Tiled hi/lo plane layout read by the prefill GEMM (kernels_gemm.hip):
// f16 [T/128][K/32][128][32], i.e. one contiguous 8 KB piece per (128-token
// tile, 32-column block); the four 8-column chunks of a token's 32 values are
// permuted by the token's index in the tile (chunk c stored at c ^ f(t),
// f(t) = ((t >> 1) ^ (t >> 3)) & 3), which makes the GEMM's fragment reads
// conflict-free once the piece is copied to LDS. T is padded to a multiple of 128.
__host__ __device__ __forceinline__ size_t tiled_plane_index(uint32_t t, uint32_t c, uint32_t K) {
    const uint32_t ti = t & 127u, f = ((ti >> 1) ^ (ti >> 3)) & 3u;
    return ((((size_t)(t >> 7) * (K >> 5) + (c >> 5)) << 7) + ti) * 32u + 8u * (((c >> 3) & 3u) ^ f) + (c & 7u);
}
// Q8_0 matrix in the prefill-GEMM layout: quants stored as q + 128 (uint8, the
// sign bit flipped) [rows_pad/128][K/32][128][32]
// (one contiguous 4 KB piece per 128-row tile and 32-column block; the four
// 8-byte chunks of a row permuted as chunk c at c ^ g(n), g(n) = ((n >> 2) ^
// (n >> 4)) & 3 for row n of the tile), scales f32 [rows_pad/128][K/32][128].
// With interleave, rows come from two matrices (gate, up) as 32 of the first,
// the same 32 of the second, and so on, the row order of a SwiGLU tile.
// Padding rows hold q = 0 (byte 0x80) with scale 0.
struct PrefillMatrix {
    int8_t *q = nullptr;
    float *d = nullptr;
    uint32_t rows_pad = 0;
};
uint64_t prefill_matrix_bytes(uint32_t rows_out, uint32_t K);   // q + d, rows padded to 128
int launch_repack_prefill(hipStream_t s, const uint8_t *raw, uint32_t off0, uint32_t off1, uint32_t rows,
                          uint32_t K, int interleave, int8_t *q, float *d);
// The deep-pipelined Q8_0 x hi/lo-plane GEMM (kernels_gemm.hip), which
// launch_gemm picks when the weights have the prefill layout and X is tiled.
bool gemm_q8p_eligible(const GemmArgs &a);
uint32_t gemm_q8p_tile_tokens();
int launch_gemm_q8p(hipStream_t s, GemmArgs a);
// Tokens per workgroup tile of the kernel launch_gemm picks for these arguments.
uint32_t gemm_tile_tokens(const GemmArgs &a);

struct SeqNormArgs {
    float *h = nullptr;             // [T][ldh] input (and residual stream when branch is set)
    uint32_t ldh = 0;
    const float *branch = nullptr;  // nullable: h += scale * branch first
    uint32_t ldb = 0;
    float scale = 1.f;
    uint32_t nbranch = 1;           // branches added (at branch + i * branch_stride), when branch is set
    uint64_t branch_stride = 0;
    const float *w = nullptr;       // f32 gains [n], nullable: only the residual update
    uint32_t n = 0;
    float eps = 0.f;
    float *y = nullptr;             // nullable f32 output [T][ldy]
    uint32_t ldy = 0;
    __half *yh = nullptr, *yl = nullptr;   // nullable hi/lo planes [T][ldp]
    uint32_t ldp = 0;
    uint32_t tiled = 0;             // 1: planes in the tiled layout of width n, 2: in the fragment
                                    // layout of width n (frag16_index); ldp unused for both
    float *zero[4] = {nullptr, nullptr, nullptr, nullptr};   // rows of split-K accumulators to clear
    uint32_t zero_n[4] = {0, 0, 0, 0};
    // 1: zero the branch rows (every split) after reading them, so the buffer is the
    // cleared accumulator of the next split-K GEMM; the branch memory must be writable.
    uint32_t clear_branch = 0;
    // k_seq_rmsnorm4 only: h_frag = 1 reads h in frag32_index order (width n, ldh
    // unused; no branch); hf (nullable) receives h, after any residual update, in
    // frag32_index order of width n.
    uint32_t h_frag = 0;
    float *hf = nullptr;
    VX_STAMP_FIELD
};
constexpr uint32_t kSeqNormMaxBranch = 16;
int launch_seq_rmsnorm(hipStream_t s, const SeqNormArgs &a, uint32_t tokens);

struct SeqRopeArgs {
    float *q = nullptr, *k = nullptr;   // [T][ldq], [T][ldk]
    const float *v = nullptr;           // [T][ldk] (KV store)
    uint32_t ldq = 0, ldk = 0;
    const float *factors = nullptr;
    uint32_t pos_base = 0, q_heads = 0, kv_heads = 0, head_dim = 0;
    uint32_t pos_period = 0;            // nonzero: row t is at position pos_base + t % pos_period
    float theta = 10000.f, scaling = 1.f;
    int q_inplace = 1;                  // write roped q back to q
    __half *qh = nullptr, *ql = nullptr;   // nullable roped q planes [T][ldqp]
    uint32_t ldqp = 0;
    __half *kc = nullptr, *vc = nullptr;   // nullable: store K/V rows [layer][context][kv_dim]
    uint32_t layer = 0, context = 0;
    // q, k and v hold nsplit partial products split_stride floats apart (split-K
    // GEMM output); the kernel reads their sums and writes roped k to split 0.
    uint32_t nsplit = 1;
    uint64_t split_stride = 0;
    uint32_t no_rope = 0;               // 1: q/k pass through unrotated (factors unused)
};
constexpr uint32_t kSeqRopeMaxSplit = 8;
int launch_seq_rope_store(hipStream_t s, const SeqRopeArgs &a, uint32_t tokens);

// ------------------------------------------- token-batched decoder stack (prefill)
struct StackLayer {
    WRef q, k, v, o, gate, up, down;
    const float *attn_norm = nullptr, *ffn_norm = nullptr;
};
struct StackPrefillWeights {        // Q8_0 projections in the prefill-GEMM layout
    PrefillMatrix q, k, v, o, gu, down;
};
struct StackWork {                  // activations of one chunk of rows (cap rows)
    uint32_t cap = 0;
    vx_buf *h = nullptr;            // residual stream [cap][nH] f32: the input rows, then the output
    vx_buf *xh = nullptr, *xl = nullptr, *ah = nullptr, *al = nullptr, *qh = nullptr, *ql = nullptr;
    vx_buf *q = nullptr, *k = nullptr, *v = nullptr, *ws = nullptr;
    vx_buf *sk_ws = nullptr, *sk_cnt = nullptr;   // stream-K SwiGLU tile parts and counters
    uint32_t sk_grid = 0;                         // its workgroups: the CU count rounded down to 8
};
constexpr uint32_t kPrefillChunk = 512;     // rows per chunk
constexpr uint32_t kPrefillMaxSplit = 8;    // split-K factor bound
constexpr uint32_t kSkTileFloats = 128u * 128u;   // accumulators of one 128 x 128 prefill GEMM tile
struct PrefillStack {
    vx_ctx *ctx = nullptr;
    uint32_t nH = 0, nF = 0, nKV = 0, q_heads = 0, kv_heads = 0, head_dim = 0, context = 0, n_layers = 0;
    float eps = 0.f, residual_scale = 1.f;
    const StackLayer *layers = nullptr;
    const StackPrefillWeights *pw = nullptr;   // nullable: per-layer prefill-layout Q8_0 weights
    bool rope = true;
    const float *rope_factors = nullptr;
    float theta = 10000.f, rope_scaling = 1.f;
    __half *kc = nullptr, *vc = nullptr;       // f16 caches [layer][context][nKV]
    const StackWork *work = nullptr;
    uint32_t schedule = VX_PREFILL_AUTO;       // gate/up GEMM schedule (VX_PREFILL_*)
};
int prefill_stack_check(const PrefillStack &p);
int prefill_stack_alloc(vx_ctx *ctx, uint32_t cap, uint32_t nH, uint32_t nF, uint32_t nKV, StackWork *w);
void prefill_stack_free(vx_ctx *ctx, StackWork *w);
// The layers over rows 0..T-1 of work->h at positions pos0..pos0+T-1 (K/V rows
// stored at those positions); work->h then holds every row's residual stream.
int enqueue_prefill_stack(const PrefillStack &p, uint32_t pos0, uint32_t T);

// ------------------------------------------------------------ AudioVAE (kernels_vae.hip)
struct VaeConvArgs {                // vae_conv1d.comp / vae_convtranspose1d.comp, channel-major
    const float *x = nullptr;
    float *y = nullptr;
    const void *w = nullptr, *bias = nullptr;   // model scalars (dtype 0 = f32, 1 = f16); bias nullable
    uint32_t w_dtype = 1, bias_dtype = 1;
    uint32_t in_channels = 0, out_channels = 0, in_length = 0, out_length = 0;
    uint32_t kernel = 1, stride = 1, dilation = 1, groups = 1, left_pad = 0;
};
int launch_vae_conv1d_cm(hipStream_t s, const VaeConvArgs &a, bool transpose);
int launch_vae_snake_cm(hipStream_t s, const float *x, float *y, const void *alpha, uint32_t dtype, uint32_t c,
                        uint32_t len);
int launch_vae_scale_bias_cm(hipStream_t s, float *x, const void *scale, const void *bias, uint32_t sdt,
                             uint32_t bdt, uint32_t c, uint32_t len, uint32_t bucket);
int launch_vae_add_cm(hipStream_t s, float *a, const float *b, uint32_t c, uint32_t len);
int launch_vae_tanh(hipStream_t s, float *x, uint32_t n);
struct VaeDwArgs {                  // depthwise conv over frame-major rows
    const float *x = nullptr;
    float *y = nullptr;
    const __half *w = nullptr, *b = nullptr;            // [C][kernel], [C]
    const __half *alpha_in = nullptr, *alpha_out = nullptr;   // nullable snakes
    uint32_t channels = 0, length = 0, kernel = 7, dilation = 1, left_pad = 0;
};
int launch_vae_dwconv_fm(hipStream_t s, const VaeDwArgs &a);
// A decoder residual unit in one pass for 32 or 64 channels:
//   y[t][n] = x[t][n] + pb[n] + sum_c pw[n][c] snake_a2(db[c] + sum_k dw[c][k] snake_a1(x[t + k d - 6d][c]))
// (the depthwise conv, kernel 7, causal, and the 1x1 conv). y must not alias x.
struct VaeResUnitArgs {
    const float *x = nullptr;
    float *y = nullptr;
    const __half *a1 = nullptr, *dw = nullptr, *db = nullptr, *a2 = nullptr, *pw = nullptr, *pb = nullptr;
    uint32_t channels = 0, length = 0, dilation = 1;
};
bool vae_resunit_eligible(const VaeResUnitArgs &a);
int launch_vae_resunit_fm(hipStream_t s, const VaeResUnitArgs &a);
struct VaeConvtInArgs {             // [pre(x[j]) | pre(x[j-1])] rows for the transposed-conv GEMM
    const float *x = nullptr;
    float *x2 = nullptr;
    const __half *scale = nullptr, *bias = nullptr;     // nullable: the sample-rate bucket's rows
    const __half *alpha = nullptr;
    uint32_t channels = 0, length = 0;
};
int launch_vae_convt_input_fm(hipStream_t s, const VaeConvtInArgs &a);
int launch_vae_repack_convt(hipStream_t s, const __half *w, const __half *b, uint32_t cin, uint32_t cout,
                            uint32_t stride, __half *wp, float *bp);
struct VaeLinearArgs {              // y[t][n] (+)= b[n] + x[t] . W[n], short K
    const float *x = nullptr;
    uint32_t ldx = 0;
    const __half *w = nullptr;      // [N][K]
    const __half *bias = nullptr;
    const float *bias_f32 = nullptr;
    float *y = nullptr;
    uint32_t ldy = 0;
    uint32_t T = 0, N = 0, K = 0;
    uint32_t residual = 0;
};
int launch_vae_linear_fm(hipStream_t s, const VaeLinearArgs &a);
struct VaeHeadArgs {                // snake -> k-tap conv to one channel -> tanh
    const float *x = nullptr;
    float *y = nullptr;
    const __half *alpha = nullptr, *w = nullptr, *b = nullptr;
    uint32_t channels = 0, length = 0, kernel = 7, left_pad = 6;
};
int launch_vae_head_fm(hipStream_t s, const VaeHeadArgs &a);

// Engine hooks of the cross-engine text prefill (baselm.cpp). baselm_prefill_rows
// runs the batched prefill of n tokens at the engine position and, when rows is
// set, stores every token's rmsnorm(h)*output_norm there ([n][hidden] f32).
vx_ctx *baselm_context(const vx_baselm *e);
uint32_t baselm_hidden_size(const vx_baselm *e);
int baselm_prefill_rows(vx_baselm *e, const uint32_t *tokens, uint32_t n, float *rows);

struct PrefillAttnArgs {
    const __half *qh = nullptr, *ql = nullptr;  // roped q planes [T][ldq]
    uint32_t ldq = 0;
    const __half *kc = nullptr, *vc = nullptr;  // f16 caches [layer][context][kv_heads*head_dim]
    uint32_t layer = 0, context = 0, pos_base = 0, T = 0;
    uint32_t q_heads = 0, kv_heads = 0, head_dim = 0;
    float *out = nullptr;                       // nullable f32 [T][ldo]
    __half *oh = nullptr, *ol = nullptr;        // nullable planes [T][ldo]
    uint32_t ldo = 0;
    uint32_t tiled = 0;                         // 1: planes in the tiled layout of width ldo
};
int launch_prefill_attn(hipStream_t s, const PrefillAttnArgs &a);
// seq_linear_bias.comp / seq_swiglu.comp for any shape and dtype, one wave per
// (row, token), reading the raw GGUF region.
struct SeqGenericArgs {
    const uint8_t *raw = nullptr;
    uint32_t w_off = 0, w2_off = 0, dtype = 0, rows = 0, cols = 0, tokens = 0;
    const float *x = nullptr;
    uint32_t in_base = 0, in_stride = 0;
    float *y = nullptr;
    uint32_t out_base = 0, out_stride = 0;
    const void *bias = nullptr;     // device pointer, nullable; f32 (bias_dtype 0) or f16 (1)
    uint32_t bias_dtype = 0;
    float alpha = 1.f;
    int swiglu = 0;
};
int launch_seq_linear_generic(hipStream_t s, const SeqGenericArgs &a);

// Token-batched projections (seq_ops.cpp) over resolved weights, choosing the
// MFMA GEMM (f32 input split to hi/lo in the kernel), the decode matvec for a
// single token, or the generic kernel. Strides and bases are in floats.
// When a split-K GEMM adds into its output, the output is cleared first unless
// out_zeroed says the caller already left it zero (e.g. cleared by the rmsnorm
// kernel that runs before).
// y[t][r] = alpha * (W[r] . x[t] + b[r])                     seq_linear_bias.comp
int enqueue_seq_linear(hipStream_t s, const WRef &w, const void *bias, uint32_t bias_dtype, uint32_t rows,
                       uint32_t cols, uint32_t tokens, const float *x, uint32_t in_base, uint32_t in_stride,
                       float *y, uint32_t out_base, uint32_t out_stride, float alpha, bool out_zeroed = false);
// q|k|v[t] = Wq|Wk|Wv . x[t]                                  seq_qkv.comp
int enqueue_seq_qkv(hipStream_t s, const WRef w[3], const uint32_t rows[3], uint32_t cols, uint32_t tokens,
                    const float *x, uint32_t in_base, uint32_t in_stride, float *const out[3],
                    const uint32_t strides[3], bool out_zeroed = false);
// y[t][r] = silu(Wg[r] . x[t]) * (Wu[r] . x[t])                 seq_swiglu.comp
int enqueue_seq_swiglu(hipStream_t s, const WRef &g, const WRef &u, uint32_t rows, uint32_t cols, uint32_t tokens,
                       const float *x, uint32_t in_base, uint32_t in_stride, float *y, uint32_t out_base,
                       uint32_t out_stride);
int launch_silu_mul(hipStream_t s, float *g, const float *u, uint32_t n);
// dense_attn_scores / dense_softmax / dense_attn_values (which = 0 / 1 / 2).
struct DenseAttnArgs {
    const float *q = nullptr, *k = nullptr, *v = nullptr;
    float *s = nullptr, *out = nullptr;
    uint32_t tokens = 0, q_heads = 0, kv_heads = 0, head_dim = 0;
    uint32_t q_stride = 0, k_stride = 0, v_stride = 0, out_stride = 0, score_stride = 0;
    // Independent sequences of `tokens` rows each (the CFG batch): sequence b
    // starts b*tokens rows into q/k/v/out and b*tokens*q_heads score rows in.
    uint32_t batch = 1;
    // Fused kernel only, nullable: (cos, sin) [tokens][head_dim / 2] of each token's
    // position within its sequence; q and k rows are then rotated (NeoX pairs d,
    // d + head_dim / 2) as they are staged, in place of a separate RoPE pass.
    const float2 *rope = nullptr;
    // Fused kernel only, nullable: the output as hi/lo f16 planes (indexed as out)
    // in place of the f32 out.
    __half *oh = nullptr, *ol = nullptr;
    uint32_t o_frag = 0;   // 1: the planes in the fragment layout of width out_stride
    // Fused kernel only: q, k, v as the sums of nslab (1 or 2) partial slabs,
    // slab_stride floats apart (float4-aligned rows and RoPE required for 2).
    uint32_t nslab = 1;
    uint64_t slab_stride = 0;
    uint32_t vec = 0;      // set by launch_dense_attn_fused: 16-byte rows, float4 staging
    // launch_dense_attn_oproj only: the O projection [hidden][q_heads * head_dim]
    // in the fragment layout, and the per-head partial slabs it writes (head h at
    // oslab + h * oslab_stride, [batch * tokens][hidden]; their sum is the
    // projection). nsplit is set by the launcher.
    const __half *wo = nullptr;
    uint32_t hidden = 0;
    float *oslab = nullptr;
    uint64_t oslab_stride = 0;
    uint32_t nsplit = 1;
    // launch_dense_attn_oproj only. hres (nullable): add the projection to hres,
    // the residual stream [batch * tokens][hidden] in frag32_index order, with
    // atomic adds, instead of writing the head slabs. ssq (nullable): q, k and v
    // are products of the un-normalised rows, and ssq + s * ssq_stride (s < nslab)
    // hold the K slabs' sums of squares of each row: the staging scales every q,
    // k and v row by 1 / sqrt(sum / norm_n + eps).
    float *hres = nullptr;
    const float *ssq = nullptr;
    uint64_t ssq_stride = 0;
    uint32_t norm_n = 0;
    float eps = 0.f;
    VX_STAMP_FIELD
};
int launch_dense_attn(hipStream_t s, const DenseAttnArgs &a, int which);
// table[p][i] = (cos, sin)(p * theta^(-2i/head_dim) / factors[i]) * scaling for
// positions p < tokens (the angle of k_seq_rope_store).
int launch_rope_pos_table(hipStream_t s, float2 *table, const float *factors, uint32_t tokens, uint32_t head_dim,
                          float theta, float scaling);
// The three phases in one kernel (one workgroup per head, sequence and eight query
// tokens, everything in LDS) for sequences of at most kDenseFusedMaxTokens tokens whose q, k, v and
// scores fit 64 KB of LDS; VX_ERR_UNSUPPORTED otherwise. The scores are not stored.
constexpr uint32_t kDenseFusedMaxTokens = 64;
uint64_t dense_fused_lds(uint32_t tokens, uint32_t head_dim);   // bytes of LDS the fused kernel needs
int launch_dense_attn_fused(hipStream_t s, const DenseAttnArgs &a);
// The fused attention followed by the head's share of the O projection (16 query
// tokens per workgroup): one partial slab per query head, summed by the consumer.
// head_dim 64 or 128, float4-aligned q/k/v rows with RoPE, hidden % 16 == 0,
// 16-byte aligned weights; VX_ERR_UNSUPPORTED otherwise.
bool dense_attn_oproj_eligible(uint32_t tokens, uint32_t head_dim);
int launch_dense_attn_oproj(hipStream_t s, const DenseAttnArgs &a);
// ---------------------------------------------- CFM / LocDiT (kernels_cfm.hip)
// Noise seed from dev_seed[0..1] (low, high word) when set, else from `seed`.
int launch_cfm_noise(hipStream_t s, float *x, uint32_t n, const uint32_t *dev_seed, uint64_t seed, float temperature);
int launch_cfm_cfg_euler(hipStream_t s, float *x, const float *pos, const float *neg, uint32_t n, float dt, float cfg,
                         uint32_t zero_star);
// The estimator's out_proj (F16 weights) for the x tokens of both CFG sequences,
// then the CFG-Zero* Euler update, in one launch (the update by the last
// workgroup to finish). counter: a device word that is zero between launches.
constexpr uint32_t kOutEulerMaxRows = 16;   // 2 * patch
struct CfmOutEulerArgs {
    const float *rows = nullptr;     // normed hidden rows [2 * tokens][hidden], 16-byte aligned
    uint32_t tokens = 0, x0 = 0, patch = 0, feat = 0, hidden = 0;   // x tokens: rows x0 .. x0 + patch - 1
    const __half *w = nullptr;       // out_proj [feat][hidden]
    const void *bias = nullptr;      // nullable, [feat], f32 (bias_dtype 0) or f16
    uint32_t bias_dtype = 0;
    float *out = nullptr;            // [2][patch * feat]: conditional, unconditional
    float *x = nullptr;              // [patch * feat], updated in place
    float dt = 0.f, cfg = 0.f;
    uint32_t zero_star = 0;
    uint32_t *counter = nullptr;
    // 1: rows is the un-normalised residual stream in frag32_index order, and the
    // final rmsnorm (weights norm_w, eps over hidden) is folded in: each x row's
    // 1/rms scales its products with (w . norm_w).
    uint32_t rows_frag = 0;
    const float *norm_w = nullptr;
    float eps = 0.f;
};
bool cfm_out_euler_eligible(uint32_t patch, uint32_t feat, uint32_t hidden, const void *w);
int launch_cfm_out_euler(hipStream_t s, const CfmOutEulerArgs &a);
// t from t_dev[t_index] when t_dev is set.
// rows > 1: row r from t_dev[t_index + r] into out + r * dim.
int launch_time_sinusoidal(hipStream_t s, float *out, uint32_t dim, float t, const float *t_dev, uint32_t t_index,
                           uint32_t rows = 1);
struct PackLocditArgs {
    const float *mu[2] = {nullptr, nullptr};   // mu tokens (n_mu <= 2), [hidden] each
    const float *time = nullptr;    // [hidden]
    const float *cond = nullptr;    // [n_cond][hidden]
    const float *x = nullptr;       // [n_x][hidden]
    float *out = nullptr;           // [batch][n_mu + 1 + n_cond + n_x][hidden]
    uint32_t hidden = 0, n_mu = 0, n_cond = 0, n_x = 0, batch = 1;
    uint32_t zero_mu_mask = 0, zero_cond_mask = 0;
    // Nullable: the x tokens computed here as in_proj(x patch) + b (seq_linear_bias
    // with F16 weights [hidden][feat], bias f32 (in_bt 0) or f16 (1)) from
    // xpatch [n_x][feat], in place of the rows at x.
    const __half *in_w = nullptr;
    const void *in_b = nullptr;
    uint32_t in_bt = 0, feat = 0;
    const float *xpatch = nullptr;
    // 1: out is a residual stream in frag32_index order (rows batch * tokens,
    // hidden % 32 == 0) instead of f32 rows.
    uint32_t out_frag = 0;
};
int launch_pack_locdit(hipStream_t s, const PackLocditArgs &a);
int launch_silu_inplace(hipStream_t s, float *x, uint32_t n);
// x[i] = round(tanh(x[i]) * scale) / scale (fsq_quantize.comp), i < n.
int launch_fsq_quantize(hipStream_t s, float *x, uint32_t n, float scale);
// a[r][i] += b[i] for rows r < rows of n values.
int launch_add_vectors(hipStream_t s, float *a, const float *b, uint32_t n, uint32_t rows = 1);
// Embedding rows of n device token ids into out[t][ldo] (bit-exact gather).
int launch_seq_embedding(hipStream_t s, const uint8_t *raw, uint32_t weight_offset, uint32_t dtype,
                         uint32_t cols, const uint32_t *tokens, uint32_t n, uint32_t vocab, float alpha,
                         float *out, uint32_t ldo);
int launch_repack_q8(hipStream_t s, const uint8_t *raw_tensor, uint32_t rows, uint32_t cols,
                     int8_t *qs, __half *d);


}  // namespace vx
