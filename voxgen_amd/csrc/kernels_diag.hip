// Streaming diagnostics: a plain HBM read and a plain copy. They calibrate the
// roofline (achievable read bandwidth next to the 8 TB/s spec) and the PMC byte
// counters (FETCH_SIZE/WRITE_SIZE of a copy of known size).
#include <algorithm>

#include "vx_internal.h"

namespace vx {
namespace {

// Grid-stride read of n16 16-byte words, U loads in flight per thread per trip.
// Each wave folds what it read into one word of `sink` so nothing is elided.
template <int U>
__global__ __launch_bounds__(256) void k_stream_read(const uint4 *src, uint64_t n16, uint32_t *sink) {
    uint32_t acc = 0;
    const uint64_t stride = (uint64_t)gridDim.x * 256u * U;
    for (uint64_t base = (uint64_t)blockIdx.x * 256u * U + threadIdx.x; base < n16; base += stride) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint64_t i = base + (uint64_t)u * 256u;
            const uint4 t = src[i < n16 ? i : 0];
            v[u] = i < n16 ? t : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o, 64);
    if ((threadIdx.x & 63u) == 0) sink[blockIdx.x * 4u + (threadIdx.x >> 6)] = acc;
}

__global__ __launch_bounds__(256) void k_stream_copy(uint4 *dst, const uint4 *src, uint64_t n16) {
    const uint64_t stride = (uint64_t)gridDim.x * 256u;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

}  // namespace

#ifdef VX_STAMPS
namespace {
struct Timeline {
    uint64_t *ticks = nullptr;   // device: (start, end) per wave record
    uint64_t cap = 0, used = 0;  // wave records
    int device = -1;
    std::vector<uint64_t> launches;   // (kind, first record, waves) per launch
};
Timeline g_timeline;
}  // namespace

uint64_t *stamp_slots(uint32_t kind, uint64_t waves) {
    Timeline &t = g_timeline;
    if (!t.ticks || waves > t.cap - t.used) return nullptr;
    uint64_t *p = t.ticks + 2u * t.used;
    t.launches.insert(t.launches.end(), {(uint64_t)kind, t.used, waves});
    t.used += waves;
    return p;
}
#endif
}  // namespace vx

using namespace vx;

extern "C" {

int vx_diag_stream_read(vx_ctx *ctx, const vx_buf *src, uint64_t offset, uint64_t bytes, vx_buf *sink,
                        uint32_t blocks, uint32_t unroll) {
    if (!ctx || !src || !sink) return fail(VX_ERR_INVALID_ARG, "vx_diag_stream_read: null argument");
    if (offset % 16u || bytes % 16u || bytes == 0)
        return fail(VX_ERR_INVALID_ARG, "vx_diag_stream_read: offset and bytes must be multiples of 16");
    if (blocks == 0 || blocks > (1u << 20)) return fail(VX_ERR_INVALID_ARG, "vx_diag_stream_read: blocks 1..2^20");
    if (offset > src->bytes || bytes > src->bytes - offset)
        return fail(VX_ERR_BOUNDS, "vx_diag_stream_read: range exceeds source buffer");
    VX_CHECK(need_buf(sink, (uint64_t)blocks * 16u, "vx_diag_stream_read sink"));
    const uint4 *p = reinterpret_cast<const uint4 *>(static_cast<const uint8_t *>(src->ptr) + offset);
    uint32_t *k = static_cast<uint32_t *>(sink->ptr);
    ProfSpan span(ctx, "diag.stream_read");
    switch (unroll) {
        case 1: k_stream_read<1><<<blocks, 256, 0, ctx->stream>>>(p, bytes / 16u, k); break;
        case 2: k_stream_read<2><<<blocks, 256, 0, ctx->stream>>>(p, bytes / 16u, k); break;
        case 4: k_stream_read<4><<<blocks, 256, 0, ctx->stream>>>(p, bytes / 16u, k); break;
        case 8: k_stream_read<8><<<blocks, 256, 0, ctx->stream>>>(p, bytes / 16u, k); break;
        default: return fail(VX_ERR_INVALID_ARG, "vx_diag_stream_read: unroll must be 1, 2, 4 or 8");
    }
    VX_LAUNCHED("k_stream_read");
    return VX_OK;
}

int vx_diag_stream_copy(vx_ctx *ctx, vx_buf *dst, const vx_buf *src, uint64_t bytes, uint32_t blocks) {
    if (!ctx || !src || !dst) return fail(VX_ERR_INVALID_ARG, "vx_diag_stream_copy: null argument");
    if (bytes % 16u || bytes == 0) return fail(VX_ERR_INVALID_ARG, "vx_diag_stream_copy: bytes must be a multiple of 16");
    if (blocks == 0 || blocks > (1u << 20)) return fail(VX_ERR_INVALID_ARG, "vx_diag_stream_copy: blocks 1..2^20");
    VX_CHECK(need_buf(src, bytes, "vx_diag_stream_copy src"));
    VX_CHECK(need_buf(dst, bytes, "vx_diag_stream_copy dst"));
    ProfSpan span(ctx, "diag.stream_copy");
    k_stream_copy<<<blocks, 256, 0, ctx->stream>>>(static_cast<uint4 *>(dst->ptr),
                                                    static_cast<const uint4 *>(src->ptr), bytes / 16u);
    VX_LAUNCHED("k_stream_copy");
    return VX_OK;
}

#ifdef VX_STAMPS
int vx_diag_timeline_arm(vx_ctx *ctx, uint64_t waves) {
    if (!ctx || waves == 0 || waves > (1ull << 26))
        return fail(VX_ERR_INVALID_ARG, "vx_diag_timeline_arm: null context or waves outside 1..2^26");
    Timeline &t = g_timeline;
    VX_HIP(hipSetDevice(ctx->device));
    // A graph captured under an earlier arm keeps writing the old records, so
    // those stay allocated until the process ends.
    t = Timeline{};
    void *p = nullptr;
    if (hipMalloc(&p, waves * 16u) != hipSuccess) return fail(VX_ERR_OOM, "vx_diag_timeline_arm: %llu records",
                                                              (unsigned long long)waves);
    VX_HIP(hipMemset(p, 0, waves * 16u));
    VX_HIP(hipDeviceSynchronize());
    t.ticks = static_cast<uint64_t *>(p);
    t.cap = waves;
    t.device = ctx->device;
    return VX_OK;
}

int vx_diag_timeline_read(vx_ctx *ctx, uint64_t *launches, uint64_t max_launches, uint64_t *ticks,
                          uint64_t max_waves, uint64_t *n_launches, uint64_t *n_waves) {
    if (!ctx || !n_launches || !n_waves || (max_launches && !launches) || (max_waves && !ticks))
        return fail(VX_ERR_INVALID_ARG, "vx_diag_timeline_read: null argument");
    const Timeline &t = g_timeline;
    if (!t.ticks || t.device != ctx->device) return fail(VX_ERR_STATE, "vx_diag_timeline_read: no timeline armed");
    *n_launches = t.launches.size() / 3u;
    *n_waves = t.used;
    const uint64_t nl = std::min<uint64_t>(max_launches, *n_launches);
    std::copy(t.launches.begin(), t.launches.begin() + 3u * nl, launches);
    const uint64_t nw = std::min<uint64_t>(max_waves, t.used);
    if (nw) {
        VX_HIP(hipSetDevice(ctx->device));
        VX_HIP(hipMemcpy(ticks, t.ticks, nw * 16u, hipMemcpyDeviceToHost));
    }
    return VX_OK;
}
#else
int vx_diag_timeline_arm(vx_ctx *ctx, uint64_t waves) {
    (void)ctx;
    (void)waves;
    return fail(VX_ERR_UNSUPPORTED, "vx_diag_timeline_arm: this library was built without -DVX_STAMPS");
}

int vx_diag_timeline_read(vx_ctx *ctx, uint64_t *launches, uint64_t max_launches, uint64_t *ticks,
                          uint64_t max_waves, uint64_t *n_launches, uint64_t *n_waves) {
    (void)ctx, (void)launches, (void)max_launches, (void)ticks, (void)max_waves;
    if (n_launches) *n_launches = 0;
    if (n_waves) *n_waves = 0;
    return fail(VX_ERR_UNSUPPORTED, "vx_diag_timeline_read: this library was built without -DVX_STAMPS");
}
#endif

}  // extern "C"
