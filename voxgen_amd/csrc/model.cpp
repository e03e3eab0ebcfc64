// Model data region on the device (upload_device_local, baselm.rs:472-477) and
// the tensor table the per-op entry points resolve u32 weight offsets through.
//
// Rank-2 Q8_0 tensors whose row width is a multiple of 1024 are repacked once on
// upload into the lane-interleaved layout the matvec kernels stream with 128-bit
// loads (see WRef in vx_internal.h). Quants and scales are moved, never
// re-rounded, so dequantised values are bit-identical to the GGUF blocks
// (gguf.rs:41-45, matvec.comp:36-43). Other Q8_0 tensors stay in the GGUF
// layout and are read from the raw region.
#include <cstring>

#include "vx_internal.h"

namespace vx {

// GgmlType::storage_bytes (gguf.rs:37-48), checked: *ok is false for an unknown
// type, a Q8_0 count not divisible by 32, or a size that does not fit 64 bits.
static uint64_t ggml_bytes(uint32_t type, uint64_t elements, bool *ok) {
    *ok = true;
    uint64_t units = elements, per = 0;
    switch (type) {
        case VX_DTYPE_F32: per = 4u; break;
        case VX_DTYPE_F16: per = 2u; break;
        case VX_DTYPE_Q8_0:
            if (elements % 32u) { *ok = false; return 0; }
            units = elements / 32u;
            per = 34u;
            break;
        default: *ok = false; return 0;
    }
    if (units > UINT64_MAX / per) { *ok = false; return 0; }
    return units * per;
}

// Element count of a tensor's dims, false on overflow.
static bool element_count(const vx_tensor_info &t, uint64_t *out) {
    uint64_t elems = 1;
    for (uint32_t k = 0; k < t.n_dims; ++k) {
        if (t.dims[k] && elems > UINT64_MAX / t.dims[k]) return false;
        elems *= t.dims[k];
    }
    *out = elems;
    return true;
}

int find_tensor_at(const vx_model *m, uint32_t offset, const vx_tensor_info **out) {
    auto it = m->by_offset.find(offset);
    if (it == m->by_offset.end())
        return fail(VX_ERR_NOT_FOUND, "no tensor of the model starts at byte offset %u", offset);
    *out = &m->tensors[it->second];
    return VX_OK;
}

int resolve_matrix(const vx_model *m, uint32_t offset, uint32_t dtype, uint32_t rows, uint32_t cols,
                   WRef *out, const char *what) {
    if (!m) return fail(VX_ERR_INVALID_ARG, "%s: null model", what);
    auto it = m->by_offset.find(offset);
    if (it == m->by_offset.end())
        return fail(VX_ERR_NOT_FOUND, "%s: no tensor starts at weight offset %u", what, offset);
    uint32_t idx = it->second;
    const vx_tensor_info &t = m->tensors[idx];
    if (t.ggml_type != dtype)
        return fail(VX_ERR_SHAPE, "%s: tensor %s is dtype %u, push says %u", what, t.name,
                    t.ggml_type, dtype);
    uint64_t tcols = t.dims[0];
    uint64_t trows = t.n_dims >= 2 ? t.dims[1] : 1;
    for (uint32_t i = 2; i < t.n_dims; ++i) trows *= t.dims[i];
    if (tcols != cols || trows < rows)
        return fail(VX_ERR_SHAPE, "%s: tensor %s is [%llu, %llu], op needs [%u, >=%u]", what, t.name,
                    (unsigned long long)tcols, (unsigned long long)trows, cols, rows);
    WRef w;
    w.dtype = dtype;
    w.rows = (uint32_t)trows;
    w.cols = cols;
    w.raw = m->raw;
    w.raw_offset = offset;
    if (dtype == VX_DTYPE_Q8_0) {
        w.wt = WT_Q8;
        if (m->packed_qs[idx] != UINT64_MAX) {  // else: raw GGUF blocks only
            w.ptr = m->packed + m->packed_qs[idx];
            w.d = (const __half *)(m->packed + m->packed_d[idx]);
        }
    } else if (dtype == VX_DTYPE_F16) {
        w.wt = WT_F16;
        w.ptr = m->raw + offset;
    } else if (dtype == VX_DTYPE_F32) {
        w.wt = WT_F32;
        w.ptr = m->raw + offset;
    } else {
        return fail(VX_ERR_UNSUPPORTED, "%s: dtype %u unsupported", what, dtype);
    }
    *out = w;
    return VX_OK;
}

int resolve_vector(const vx_model *m, uint32_t offset, uint32_t dtype, uint32_t n, const void **out,
                   const char *what) {
    if (!m) return fail(VX_ERR_INVALID_ARG, "%s: null model", what);
    auto it = m->by_offset.find(offset);
    if (it == m->by_offset.end())
        return fail(VX_ERR_NOT_FOUND, "%s: no tensor starts at offset %u", what, offset);
    const vx_tensor_info &t = m->tensors[it->second];
    if (t.ggml_type != dtype)
        return fail(VX_ERR_SHAPE, "%s: tensor %s is dtype %u, expected %u", what, t.name, t.ggml_type,
                    dtype);
    uint64_t elems = 1;
    for (uint32_t i = 0; i < t.n_dims; ++i) elems *= t.dims[i];
    if (elems < n)
        return fail(VX_ERR_SHAPE, "%s: tensor %s has %llu elements, op reads %u", what, t.name,
                    (unsigned long long)elems, n);
    *out = m->raw + offset;
    return VX_OK;
}

}  // namespace vx

using namespace vx;

extern "C" {

// The tensor table is validated before the context is used, so a bad table is
// refused without any device work (and is reported even without a context).
int vx_model_upload(vx_ctx *ctx, const void *data, uint64_t bytes, const vx_tensor_info *tensors,
                    uint32_t n_tensors, vx_model **out) {
    if (!data || !out || (!tensors && n_tensors))
        return fail(VX_ERR_INVALID_ARG, "vx_model_upload: null argument");
    *out = nullptr;
    if (bytes == 0) return fail(VX_ERR_INVALID_ARG, "vx_model_upload: empty data region");
    if (bytes > 0xffffffffull)  // baselm.rs:468-470
        return fail(VX_ERR_OFFSET,
                    "data region exceeds 4 GiB; push structs carry 32-bit byte offsets");
    // Validate the table before touching the device.
    uint64_t packed_total = 0;
    std::vector<uint64_t> pq(n_tensors, UINT64_MAX), pd(n_tensors, UINT64_MAX);
    for (uint32_t i = 0; i < n_tensors; ++i) {
        const vx_tensor_info &t = tensors[i];
        if (t.n_dims == 0 || t.n_dims > 4)
            return fail(VX_ERR_GGUF, "tensor %u has rank %u", i, t.n_dims);
        uint64_t elems = 1;
        if (!element_count(t, &elems)) return fail(VX_ERR_GGUF, "tensor %.96s: element-count overflow", t.name);
        bool ok = true;
        uint64_t tb = ggml_bytes(t.ggml_type, elems, &ok);
        if (!ok) {
            if (t.ggml_type == VX_DTYPE_F32 || t.ggml_type == VX_DTYPE_F16 ||
                (t.ggml_type == VX_DTYPE_Q8_0 && elems % 32u == 0))
                return fail(VX_ERR_GGUF, "tensor %.96s: tensor size overflow", t.name);
            return fail(VX_ERR_UNSUPPORTED, "tensor %.96s: unsupported type %u or size", t.name,
                        t.ggml_type);
        }
        if (t.offset > bytes || tb > bytes - t.offset)
            return fail(VX_ERR_GGUF, "tensor %.96s extends beyond the data region", t.name);
        if (t.ggml_type == VX_DTYPE_Q8_0 && t.n_dims == 2) {
            uint64_t rows = t.dims[1], cols = t.dims[0];
            if (rows > UINT32_MAX || cols > UINT32_MAX)  // the repack kernel takes 32-bit extents
                return fail(VX_ERR_SHAPE, "Q8_0 matrix %.96s is [%llu, %llu], beyond 32-bit extents", t.name,
                            (unsigned long long)cols, (unsigned long long)rows);
            if (cols % 32u)
                return fail(VX_ERR_SHAPE, "Q8_0 matrix %.96s has row width %llu, not divisible by 32",
                            t.name, (unsigned long long)cols);
            if (t.offset % 2u)
                return fail(VX_ERR_UNSUPPORTED, "Q8_0 matrix %.96s at odd offset", t.name);
            if (cols % 1024u) continue;  // read in place from the raw region
            pq[i] = packed_total;
            packed_total += (rows * cols + 255u) & ~255ull;
            pd[i] = packed_total;
            packed_total += (rows * (cols / 32u) * 2u + 255u) & ~255ull;
        }
    }
    if (!ctx) return fail(VX_ERR_INVALID_ARG, "vx_model_upload: null context");
    VX_HIP(hipSetDevice(ctx->device));
    vx_model *m = new vx_model();
    m->ctx = ctx;
    m->raw_bytes = (bytes + 255u) & ~255ull;
    hipError_t e = hipMalloc(&m->raw, m->raw_bytes);
    if (e != hipSuccess) {
        delete m;
        return fail(VX_ERR_OOM, "hipMalloc of %llu-byte model region failed: %s",
                    (unsigned long long)bytes, hipGetErrorString(e));
    }
    if (packed_total) {
        e = hipMalloc(&m->packed, packed_total);
        if (e != hipSuccess) {
            (void)hipFree(m->raw);
            delete m;
            return fail(VX_ERR_OOM, "hipMalloc of %llu-byte repack arena failed: %s",
                        (unsigned long long)packed_total, hipGetErrorString(e));
        }
        m->packed_bytes = packed_total;
    }
    e = hipMemsetAsync(m->raw + bytes, 0, m->raw_bytes - bytes, ctx->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(m->raw, data, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        vx_model_free(ctx, m);
        return fail(VX_ERR_HIP, "model upload failed: %s", hipGetErrorString(e));
    }
    m->tensors.assign(tensors, tensors + n_tensors);
    m->packed_qs = pq;
    m->packed_d = pd;
    for (uint32_t i = 0; i < n_tensors; ++i) {
        m->tensors[i].name[sizeof(m->tensors[i].name) - 1] = '\0';
        uint64_t elems = 1;
        (void)element_count(m->tensors[i], &elems);  // validated above
        bool ok = true;
        m->tensors[i].bytes = ggml_bytes(m->tensors[i].ggml_type, elems, &ok);
        m->by_offset.emplace(m->tensors[i].offset, i);  // first tensor at an offset wins
        m->by_name.emplace(std::string(m->tensors[i].name), i);
        if (pq[i] != UINT64_MAX) {
            const vx_tensor_info &t = m->tensors[i];
            int s = launch_repack_q8(ctx->stream, m->raw + t.offset, (uint32_t)t.dims[1],
                                     (uint32_t)t.dims[0], (int8_t *)(m->packed + pq[i]),
                                     (__half *)(m->packed + pd[i]));
            if (s != VX_OK) {
                vx_model_free(ctx, m);
                return s;
            }
        }
    }
    e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        vx_model_free(ctx, m);
        return fail(VX_ERR_HIP, "model repack failed: %s", hipGetErrorString(e));
    }
    *out = m;
    return VX_OK;
}

int vx_model_free(vx_ctx *ctx, vx_model *model) {
    if (!model) return VX_OK;
    if (ctx) (void)hipSetDevice(ctx->device);
    if (model->raw) (void)hipFree(model->raw);
    if (model->packed) (void)hipFree(model->packed);
    delete model;
    return VX_OK;
}

uint32_t vx_model_tensor_count(const vx_model *model) {
    return model ? (uint32_t)model->tensors.size() : 0u;
}

int vx_model_tensor_at(const vx_model *model, uint32_t index, vx_tensor_info *out) {
    if (!model || !out) return fail(VX_ERR_INVALID_ARG, "vx_model_tensor_at: null argument");
    if (index >= model->tensors.size())
        return fail(VX_ERR_INVALID_ARG, "vx_model_tensor_at: index %u out of range", index);
    *out = model->tensors[index];
    return VX_OK;
}

int vx_model_find(const vx_model *model, const char *name, vx_tensor_info *out) {
    if (!model || !name) return fail(VX_ERR_INVALID_ARG, "vx_model_find: null argument");
    auto it = model->by_name.find(name);
    if (it == model->by_name.end())
        return fail(VX_ERR_NOT_FOUND, "required GGUF tensor \"%s\" is missing", name);
    if (out) *out = model->tensors[it->second];
    return VX_OK;
}

uint64_t vx_model_device_bytes(const vx_model *model) {
    return model ? model->raw_bytes + model->packed_bytes : 0u;
}

int vx_dequant(vx_ctx *ctx, const vx_model *model, uint32_t weight_offset, uint32_t rows,
               uint32_t cols, uint32_t dtype, vx_buf *out) {
    if (!ctx || !model) return fail(VX_ERR_INVALID_ARG, "vx_dequant: null argument");
    WRef w;
    VX_CHECK(resolve_matrix(model, weight_offset, dtype, rows, cols, &w, "vx_dequant"));
    VX_CHECK(need_buf(out, (uint64_t)rows * cols * 4u, "vx_dequant out"));
    if (rows == 0 || cols == 0) return VX_OK;
    ProfSpan span(ctx, "dequant");
    return launch_dequant(ctx->stream, w, rows, cols, (float *)out->ptr);
}

}  // extern "C"
