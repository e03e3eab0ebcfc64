// Device context, buffers, stream, graph capture and profiling spans.
// Replaces VulkanContext (vulkan.rs:96-113, 284-955) with one HIP device and one
// in-order stream per context.
#include <cstdio>
#include <cstring>
#include <mutex>

#include "vx_internal.h"

namespace vx {

static thread_local std::string g_last_error;

void set_error_v(const char *fmt, va_list ap) {
    char buf[1024];
    vsnprintf(buf, sizeof(buf), fmt, ap);
    g_last_error = buf;
}

int fail(int code, const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    set_error_v(fmt, ap);
    va_end(ap);
    return code;
}

void clear_error() { g_last_error.clear(); }

int check_cancel(const vx_ctx *ctx) {
    if (ctx && ctx->cancel && __atomic_load_n(ctx->cancel, __ATOMIC_ACQUIRE) != 0u)
        return fail(VX_ERR_CANCELLED, "speech synthesis cancelled");  // runtime.rs:746-808
    return VX_OK;
}

int need_buf(const vx_buf *b, uint64_t bytes, const char *what) {
    if (!b || !b->ptr) return fail(VX_ERR_INVALID_ARG, "%s: null buffer", what);
    if (b->bytes < bytes)
        return fail(VX_ERR_BOUNDS, "%s: buffer holds %llu bytes, op needs %llu", what,
                    (unsigned long long)b->bytes, (unsigned long long)bytes);
    return VX_OK;
}

static hipEvent_t take_event(vx_ctx *ctx) {
    if (!ctx->event_pool.empty()) {
        hipEvent_t e = ctx->event_pool.back();
        ctx->event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

ProfSpan::ProfSpan(vx_ctx *ctx, const char *name) : ctx_(ctx) {
    if (!ctx_ || !ctx_->prof_enabled || ctx_->capturing) {
        ctx_ = nullptr;
        return;
    }
    start_ = take_event(ctx_);
    if (!start_ || hipEventRecord(start_, ctx_->stream) != hipSuccess) {
        ctx_ = nullptr;
        return;
    }
    name_ = name;
}

ProfSpan::~ProfSpan() {
    if (!ctx_) return;
    hipEvent_t end = take_event(ctx_);
    if (!end || hipEventRecord(end, ctx_->stream) != hipSuccess) return;
    ctx_->prof_pending.push_back({name_, start_, end});
}

int collect_profile(vx_ctx *ctx) {
    for (auto &p : ctx->prof_pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, p.start, p.end) == hipSuccess) {
            auto it = ctx->prof_totals.find(p.name);
            if (it == ctx->prof_totals.end()) {
                ctx->prof_order.push_back(p.name);
                it = ctx->prof_totals.emplace(p.name, ProfTotal{}).first;
            }
            it->second.total_ms += ms;
            it->second.calls += 1;
        }
        ctx->event_pool.push_back(p.start);
        ctx->event_pool.push_back(p.end);
    }
    ctx->prof_pending.clear();
    return VX_OK;
}

}  // namespace vx

using namespace vx;

// Device scratch of the entry points that allocate nothing
// (vx_fused_attention_noalloc): VX_NOALLOC_SCRATCH_BYTES per GPU, held until the
// process ends. Host code never passes this array's name to a kernel or a copy:
// vx_init resolves the device address of this GPU's copy once (with the device
// current) and keeps it in the context.
static __device__ __align__(256) uint8_t scratch[VX_NOALLOC_SCRATCH_BYTES];

extern "C" {

int vx_abi_version(void) { return VX_ABI_VERSION; }

const char *vx_last_error(void) { return g_last_error.c_str(); }

int vx_init(int device_index, vx_ctx **out) {
    if (!out) return fail(VX_ERR_INVALID_ARG, "vx_init: out is null");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0)
        return fail(VX_ERR_NO_DEVICE, "no HIP device available (%s)", hipGetErrorString(e));
    if (device_index < 0 || device_index >= count)
        return fail(VX_ERR_NO_DEVICE, "device index %d outside 0..%d", device_index, count - 1);
    VX_HIP(hipSetDevice(device_index));
    vx_ctx *ctx = new vx_ctx();
    ctx->device = device_index;
    if (hipGetDeviceProperties(&ctx->props, device_index) != hipSuccess) {
        delete ctx;
        return fail(VX_ERR_HIP, "hipGetDeviceProperties failed");
    }
    // Default priority: every stream of this library runs at normal priority.
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return fail(VX_ERR_HIP, "hipStreamCreate failed");
    }
    void *sp = nullptr;
    e = hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !sp) {
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return fail(VX_ERR_HIP, "hipGetSymbolAddress of the no-allocation scratch failed: %s",
                    hipGetErrorString(e));
    }
    ctx->noalloc_scratch = sp;
    *out = ctx;
    return VX_OK;
}

int vx_destroy(vx_ctx *ctx) {
    if (!ctx) return VX_OK;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    collect_profile(ctx);
    for (hipEvent_t ev : ctx->event_pool) hipEventDestroy(ev);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return VX_OK;
}

int vx_device_info_get(vx_ctx *ctx, vx_device_info *out) {
    if (!ctx || !out) return fail(VX_ERR_INVALID_ARG, "vx_device_info_get: null argument");
    memset(out, 0, sizeof(*out));
    const hipDeviceProp_t &p = ctx->props;
    snprintf(out->name, sizeof(out->name), "%s", p.name);
    snprintf(out->arch, sizeof(out->arch), "%s", p.gcnArchName);
    out->total_global_mem = p.totalGlobalMem;
    out->compute_units = (uint32_t)p.multiProcessorCount;
    out->wavefront_size = (uint32_t)p.warpSize;
    out->l2_cache_bytes = (uint32_t)p.l2CacheSize;
    out->lds_bytes_per_block = (uint32_t)p.sharedMemPerBlock;
    out->clock_khz = (uint32_t)p.clockRate;
    out->memory_clock_khz = (uint32_t)p.memoryClockRate;
    out->memory_bus_width = (uint32_t)p.memoryBusWidth;
    return VX_OK;
}

int vx_alloc(vx_ctx *ctx, uint64_t bytes, vx_buf **out) {
    if (!ctx || !out) return fail(VX_ERR_INVALID_ARG, "vx_alloc: null argument");
    if (bytes == 0) return fail(VX_ERR_INVALID_ARG, "vx_alloc: zero-byte buffer");
    *out = nullptr;
    VX_HIP(hipSetDevice(ctx->device));
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess)
        return fail(VX_ERR_OOM, "hipMalloc(%llu) failed: %s", (unsigned long long)bytes,
                    hipGetErrorString(e));
    vx_buf *b = new vx_buf();
    b->ptr = p;
    b->bytes = bytes;
    *out = b;
    return VX_OK;
}

int vx_free(vx_ctx *ctx, vx_buf *buf) {
    if (!buf) return VX_OK;
    if (ctx) (void)hipSetDevice(ctx->device);
    if (buf->owned && buf->ptr) (void)hipFree(buf->ptr);
    delete buf;
    return VX_OK;
}

uint64_t vx_buf_size(const vx_buf *buf) { return buf ? buf->bytes : 0; }
void *vx_buf_device_ptr(const vx_buf *buf) { return buf ? buf->ptr : nullptr; }

int vx_upload(vx_ctx *ctx, vx_buf *dst, uint64_t dst_offset, const void *src, uint64_t bytes) {
    if (!ctx || !dst || (!src && bytes)) return fail(VX_ERR_INVALID_ARG, "vx_upload: null argument");
    if (dst_offset > dst->bytes || bytes > dst->bytes - dst_offset)
        return fail(VX_ERR_BOUNDS, "vx_upload: %llu bytes at %llu exceed buffer of %llu",
                    (unsigned long long)bytes, (unsigned long long)dst_offset,
                    (unsigned long long)dst->bytes);
    if (!bytes) return VX_OK;
    VX_HIP(hipSetDevice(ctx->device));
    VX_HIP(hipMemcpyAsync((uint8_t *)dst->ptr + dst_offset, src, bytes, hipMemcpyHostToDevice,
                          ctx->stream));
    VX_HIP(hipStreamSynchronize(ctx->stream));
    return VX_OK;
}

int vx_download(vx_ctx *ctx, const vx_buf *src, uint64_t src_offset, void *dst, uint64_t bytes) {
    if (!ctx || !src || (!dst && bytes)) return fail(VX_ERR_INVALID_ARG, "vx_download: null argument");
    if (src_offset > src->bytes || bytes > src->bytes - src_offset)
        return fail(VX_ERR_BOUNDS, "vx_download: %llu bytes at %llu exceed buffer of %llu",
                    (unsigned long long)bytes, (unsigned long long)src_offset,
                    (unsigned long long)src->bytes);
    if (!bytes) return VX_OK;
    VX_HIP(hipSetDevice(ctx->device));
    VX_HIP(hipMemcpyAsync(dst, (const uint8_t *)src->ptr + src_offset, bytes, hipMemcpyDeviceToHost,
                          ctx->stream));
    VX_HIP(hipStreamSynchronize(ctx->stream));
    collect_profile(ctx);
    return VX_OK;
}

int vx_copy(vx_ctx *ctx, vx_buf *dst, uint64_t dst_offset, const vx_buf *src, uint64_t src_offset,
            uint64_t bytes) {
    if (!ctx || !dst || !src) return fail(VX_ERR_INVALID_ARG, "vx_copy: null argument");
    if (dst_offset > dst->bytes || bytes > dst->bytes - dst_offset || src_offset > src->bytes ||
        bytes > src->bytes - src_offset)
        return fail(VX_ERR_BOUNDS, "vx_copy: range exceeds a buffer");
    if (!bytes) return VX_OK;
    VX_HIP(hipMemcpyAsync((uint8_t *)dst->ptr + dst_offset, (const uint8_t *)src->ptr + src_offset,
                          bytes, hipMemcpyDeviceToDevice, ctx->stream));
    return VX_OK;
}

int vx_fill_u32(vx_ctx *ctx, vx_buf *dst, uint64_t dst_offset, uint32_t value, uint64_t count) {
    if (!ctx || !dst) return fail(VX_ERR_INVALID_ARG, "vx_fill_u32: null argument");
    if (dst_offset % 4 != 0) return fail(VX_ERR_INVALID_ARG, "vx_fill_u32: offset not word aligned");
    if (dst_offset > dst->bytes || count > (dst->bytes - dst_offset) / 4)
        return fail(VX_ERR_BOUNDS, "vx_fill_u32: range exceeds buffer");
    if (!count) return VX_OK;
    return launch_fill_u32(ctx->stream, (uint32_t *)((uint8_t *)dst->ptr + dst_offset), value, count);
}

int vx_set_cancel_flag(vx_ctx *ctx, const uint32_t *flag) {
    if (!ctx) return fail(VX_ERR_INVALID_ARG, "vx_set_cancel_flag: null context");
    ctx->cancel = flag;
    return VX_OK;
}

int vx_sync(vx_ctx *ctx) {
    if (!ctx) return fail(VX_ERR_INVALID_ARG, "vx_sync: null context");
    VX_HIP(hipStreamSynchronize(ctx->stream));
    collect_profile(ctx);
    return VX_OK;
}

int vx_graph_begin(vx_ctx *ctx) {
    if (!ctx) return fail(VX_ERR_INVALID_ARG, "vx_graph_begin: null context");
    if (ctx->capturing) return fail(VX_ERR_STATE, "vx_graph_begin: already capturing");
    VX_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
    return VX_OK;
}

int vx_graph_end(vx_ctx *ctx, vx_graph **out) {
    if (!ctx || !out) return fail(VX_ERR_INVALID_ARG, "vx_graph_end: null argument");
    if (!ctx->capturing) return fail(VX_ERR_STATE, "vx_graph_end: not capturing");
    ctx->capturing = false;
    hipGraph_t g = nullptr;
    VX_HIP(hipStreamEndCapture(ctx->stream, &g));
    hipGraphExec_t ex = nullptr;
    hipError_t e = hipGraphInstantiate(&ex, g, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g);
        return fail(VX_ERR_HIP, "hipGraphInstantiate failed: %s", hipGetErrorString(e));
    }
    vx_graph *vg = new vx_graph();
    vg->graph = g;
    vg->exec = ex;
    *out = vg;
    return VX_OK;
}

int vx_graph_launch(vx_ctx *ctx, vx_graph *graph) {
    if (!ctx || !graph) return fail(VX_ERR_INVALID_ARG, "vx_graph_launch: null argument");
    VX_HIP(hipGraphLaunch(graph->exec, ctx->stream));
    return VX_OK;
}

int vx_graph_free(vx_ctx *ctx, vx_graph *graph) {
    (void)ctx;
    if (!graph) return VX_OK;
    if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
    if (graph->graph) (void)hipGraphDestroy(graph->graph);
    delete graph;
    return VX_OK;
}

int vx_prof_enable(vx_ctx *ctx, int enabled) {
    if (!ctx) return fail(VX_ERR_INVALID_ARG, "vx_prof_enable: null context");
    ctx->prof_enabled = enabled != 0;
    return VX_OK;
}

int vx_prof_reset(vx_ctx *ctx) {
    if (!ctx) return fail(VX_ERR_INVALID_ARG, "vx_prof_reset: null context");
    VX_HIP(hipStreamSynchronize(ctx->stream));
    collect_profile(ctx);
    ctx->prof_totals.clear();
    ctx->prof_order.clear();
    return VX_OK;
}

int vx_prof_snapshot(vx_ctx *ctx, vx_prof_entry *out, uint32_t cap, uint32_t *count) {
    if (!ctx) return fail(VX_ERR_INVALID_ARG, "vx_prof_snapshot: null context");
    VX_HIP(hipStreamSynchronize(ctx->stream));
    collect_profile(ctx);
    uint32_t n = 0;
    for (const std::string &name : ctx->prof_order) {
        const ProfTotal &t = ctx->prof_totals[name];
        if (out && n < cap) {
            vx_prof_entry &e = out[n];
            memset(&e, 0, sizeof(e));
            snprintf(e.name, sizeof(e.name), "%s", name.c_str());
            e.total_ms = t.total_ms;
            e.calls = t.calls;
            e.avg_ms = t.calls ? t.total_ms / (double)t.calls : 0.0;
        }
        ++n;
    }
    if (count) *count = n;
    return VX_OK;
}

}  // extern "C"
