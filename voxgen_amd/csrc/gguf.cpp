// GGUF v2/v3 reader (gguf.rs:163-286) and BaseLmConfig::from_gguf
// (baselm.rs:60-180). Host-only; the file is memory-mapped read-only and only
// the header pages are touched until the data region is uploaded.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>

#include "vx_internal.h"

using namespace vx;

namespace {

constexpr uint32_t kGgufMagic = 0x46554747u;  // "GGUF" little-endian (gguf.rs:6)
constexpr uint64_t kDefaultAlignment = 32;     // gguf.rs:7

enum MetaKind { META_INT, META_UINT, META_FLOAT, META_BOOL, META_STRING, META_OTHER };

struct MetaValue {
    MetaKind kind = META_OTHER;
    int64_t i = 0;
    uint64_t u = 0;
    double f = 0.0;
    bool b = false;
    std::string s;
};

struct Reader {
    const uint8_t *p;
    uint64_t n, pos = 0;
    bool ok = true;
    std::string err;
    const uint8_t *take(uint64_t k) {
        if (!ok) return nullptr;
        if (k > n - pos) {  // gguf.rs:166-170
            ok = false;
            err = "unexpected EOF while reading GGUF at byte " + std::to_string(pos);
            return nullptr;
        }
        const uint8_t *r = p + pos;
        pos += k;
        return r;
    }
    template <typename T>
    T get() {
        T v{};
        const uint8_t *b = take(sizeof(T));
        if (b) memcpy(&v, b, sizeof(T));
        return v;
    }
    std::string str() {
        const uint64_t len = get<uint64_t>();
        const uint8_t *b = take(len);
        if (!b) return std::string();
        if (!valid_utf8(b, len)) {  // gguf.rs:182 (std::str::from_utf8)
            ok = false;
            err = "invalid UTF-8 in GGUF string";
            return std::string();
        }
        return std::string(reinterpret_cast<const char *>(b), len);
    }
    // Well-formed UTF-8 as Rust's from_utf8 checks it: no overlong forms, no
    // surrogates, nothing above U+10FFFF.
    static bool valid_utf8(const uint8_t *s, uint64_t n) {
        uint64_t i = 0;
        while (i < n) {
            const uint8_t c = s[i];
            if (c < 0x80) { ++i; continue; }
            uint32_t need, cp;
            if (c >= 0xC2 && c <= 0xDF) { need = 1; cp = c & 0x1Fu; }
            else if (c >= 0xE0 && c <= 0xEF) { need = 2; cp = c & 0x0Fu; }
            else if (c >= 0xF0 && c <= 0xF4) { need = 3; cp = c & 0x07u; }
            else return false;
            if (need > n - i - 1) return false;
            for (uint32_t k = 1; k <= need; ++k) {
                const uint8_t d = s[i + k];
                if ((d & 0xC0u) != 0x80u) return false;
                cp = (cp << 6) | (d & 0x3Fu);
            }
            if ((need == 2 && (cp < 0x800 || (cp >= 0xD800 && cp <= 0xDFFF))) ||
                (need == 3 && (cp < 0x10000 || cp > 0x10FFFF)))
                return false;
            i += need + 1;
        }
        return true;
    }
};

bool read_value(Reader &r, uint32_t ty, int depth, MetaValue &out, std::vector<std::string> *strings) {
    if (depth > 8) {
        r.ok = false;
        r.err = "GGUF metadata nesting too deep";
        return false;
    }
    switch (ty) {  // read_meta_value gguf.rs:190-220
        case 0: out.kind = META_UINT; out.u = r.get<uint8_t>(); break;
        case 1: out.kind = META_INT; out.i = r.get<int8_t>(); break;
        case 2: out.kind = META_UINT; out.u = r.get<uint16_t>(); break;
        case 3: out.kind = META_INT; out.i = r.get<int16_t>(); break;
        case 4: out.kind = META_UINT; out.u = r.get<uint32_t>(); break;
        case 5: out.kind = META_INT; out.i = r.get<int32_t>(); break;
        case 6: out.kind = META_FLOAT; out.f = r.get<float>(); break;
        case 7: out.kind = META_BOOL; out.b = r.get<uint8_t>() != 0; break;
        case 8: out.kind = META_STRING; out.s = r.str(); break;
        case 9: {
            const uint32_t et = r.get<uint32_t>();
            const uint64_t cnt = r.get<uint64_t>();
            out.kind = META_OTHER;
            for (uint64_t i = 0; i < cnt && r.ok; ++i) {
                MetaValue tmp;
                if (!read_value(r, et, depth + 1, tmp, nullptr)) return false;
                if (strings && et == 8) strings->push_back(std::move(tmp.s));
            }
            break;
        }
        case 10: out.kind = META_UINT; out.u = r.get<uint64_t>(); break;
        case 11: out.kind = META_INT; out.i = r.get<int64_t>(); break;
        case 12: out.kind = META_FLOAT; out.f = r.get<double>(); break;
        default:
            r.ok = false;
            r.err = "unknown GGUF metadata value type " + std::to_string(ty);
            return false;
    }
    return r.ok;
}

// Byte size of a tensor, with the multiplications checked (gguf.rs:37-48 uses
// checked_mul and fails on overflow).
bool storage_bytes(uint32_t type, uint64_t elements, uint64_t *out, std::string *err) {
    uint64_t units = elements, per = 0;
    switch (type) {  // GgmlType::storage_bytes gguf.rs:37-48
        case 0: per = 4u; break;
        case 1: per = 2u; break;
        case 8:
            if (elements % 32u) {
                *err = "Q8_0 tensor has " + std::to_string(elements) + " elements, not divisible by 32";
                return false;
            }
            units = elements / 32u;
            per = 34u;
            break;
        default: *err = "unsupported GGML tensor type " + std::to_string(type); return false;
    }
    if (units > UINT64_MAX / per) {
        *err = "tensor size overflow";
        return false;
    }
    *out = units * per;
    return true;
}

}  // namespace

struct vx_gguf {
    std::string path;
    int fd = -1;
    const uint8_t *map = nullptr;
    uint64_t file_bytes = 0;
    vx_gguf_summary summary{};
    std::map<std::string, MetaValue> metadata;
    std::vector<vx_tensor_info> tensors;
    std::vector<std::string> tokens, merges;
};

namespace {

// meta_u32 (baselm.rs:282-287): the first key whose value reads as a u32.
bool meta_u32(const vx_gguf *g, std::initializer_list<const char *> keys, uint32_t *out) {
    for (const char *k : keys) {
        auto it = g->metadata.find(k);
        if (it == g->metadata.end()) continue;
        const MetaValue &v = it->second;
        if (v.kind == META_UINT && v.u <= 0xffffffffull) { *out = (uint32_t)v.u; return true; }
        if (v.kind == META_INT && v.i >= 0 && v.i <= 0xffffffffll) { *out = (uint32_t)v.i; return true; }
        if (v.kind == META_FLOAT && v.f >= 0 && v.f <= 4294967295.0 && std::floor(v.f) == v.f) {
            *out = (uint32_t)v.f;
            return true;
        }
        if (v.kind == META_STRING) {
            // str::parse::<u32> (baselm.rs:275): an optional '+', then decimal
            // digits only; no whitespace, no other sign, no base prefix.
            const std::string &t = v.s;
            size_t i = !t.empty() && t[0] == '+' ? 1u : 0u;
            if (i < t.size()) {
                uint64_t x = 0;
                bool good = true;
                for (; i < t.size() && good; ++i) {
                    if (t[i] < '0' || t[i] > '9') good = false;
                    else x = x * 10u + (uint64_t)(t[i] - '0');
                    if (x > 0xffffffffull) good = false;
                }
                if (good) {
                    *out = (uint32_t)x;
                    return true;
                }
            }
        }
    }
    return false;
}

// meta_f32 (baselm.rs:288-293).
bool meta_f32(const vx_gguf *g, std::initializer_list<const char *> keys, float *out) {
    for (const char *k : keys) {
        auto it = g->metadata.find(k);
        if (it == g->metadata.end()) continue;
        const MetaValue &v = it->second;
        if (v.kind == META_UINT) { *out = (float)v.u; return true; }
        if (v.kind == META_INT) { *out = (float)v.i; return true; }
        if (v.kind == META_FLOAT) { *out = (float)v.f; return true; }
        if (v.kind == META_STRING && !v.s.empty()) {
            // str::parse::<f32> (baselm.rs:281): decimal or exponent forms and
            // inf/infinity/nan, no surrounding whitespace, no hexadecimal forms,
            // which strtof would also take.
            const std::string &t = v.s;
            const bool plain = t.find_first_of(" \t\n\r\v\fxXpP()") == std::string::npos;
            char *end = nullptr;
            const float x = plain ? strtof(t.c_str(), &end) : 0.f;
            if (plain && end && *end == '\0') { *out = x; return true; }
        }
    }
    return false;
}

bool meta_string(const vx_gguf *g, const char *key, std::string *out) {
    auto it = g->metadata.find(key);
    if (it == g->metadata.end()) return false;
    const MetaValue &v = it->second;
    switch (v.kind) {
        case META_STRING: *out = v.s; return true;
        case META_UINT: *out = std::to_string(v.u); return true;
        case META_INT: *out = std::to_string(v.i); return true;
        case META_BOOL: *out = v.b ? "true" : "false"; return true;
        case META_FLOAT: {
            char buf[64];
            snprintf(buf, sizeof(buf), "%.9g", v.f);
            *out = buf;
            return true;
        }
        default: return false;
    }
}

const vx_tensor_info *tensor(const vx_gguf *g, const char *name) {
    for (const vx_tensor_info &t : g->tensors)
        if (strcmp(t.name, name) == 0) return &t;
    return nullptr;
}

int need_tensor(const vx_gguf *g, const std::string &name, const vx_tensor_info **out) {
    *out = tensor(g, name.c_str());
    if (!*out)
        return fail(VX_ERR_NOT_FOUND, "required GGUF tensor \"%s\" is missing from %s", name.c_str(),
                    g->path.c_str());
    return VX_OK;
}

int dims_eq(const vx_tensor_info *t, std::initializer_list<uint64_t> d) {
    bool ok = t->n_dims == d.size();
    uint32_t i = 0;
    for (uint64_t x : d) {
        if (!ok) break;
        ok = t->dims[i++] == x;
    }
    if (!ok) return fail(VX_ERR_SHAPE, "tensor %s has unexpected dimensions", t->name);
    return VX_OK;
}

int is_f32(const vx_tensor_info *t) {
    if (t->ggml_type != 0) return fail(VX_ERR_SHAPE, "tensor %s is not F32", t->name);
    return VX_OK;
}

int is_matrix(const vx_tensor_info *t) {
    if (t->ggml_type != 1 && t->ggml_type != 8)
        return fail(VX_ERR_SHAPE, "matrix %s uses unsupported type %u", t->name, t->ggml_type);
    if (t->ggml_type == 8 && t->dims[0] % 32u)
        return fail(VX_ERR_SHAPE, "Q8_0 matrix %s has row width %llu, not divisible by 32", t->name,
                    (unsigned long long)t->dims[0]);
    return VX_OK;
}

}  // namespace

extern "C" {

int vx_gguf_open(const char *path, vx_gguf **out) {
    if (!path || !out) return fail(VX_ERR_INVALID_ARG, "vx_gguf_open: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(VX_ERR_GGUF, "open %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return fail(VX_ERR_GGUF, "stat %s failed", path);
    }
    const uint64_t size = (uint64_t)st.st_size;
    if (size == 0) {
        close(fd);
        return fail(VX_ERR_GGUF, "unexpected EOF while reading GGUF at byte 0");
    }
    void *m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
        close(fd);
        return fail(VX_ERR_GGUF, "mmap %s failed", path);
    }
    vx_gguf *g = new vx_gguf();
    g->path = path;
    g->fd = fd;
    g->map = static_cast<const uint8_t *>(m);
    g->file_bytes = size;
    auto bail = [&](int code, const std::string &msg) {
        vx_gguf_close(g);
        return fail(code, "%s", msg.c_str());
    };
    Reader r{g->map, size};
    if (r.get<uint32_t>() != kGgufMagic || !r.ok) return bail(VX_ERR_GGUF, std::string(path) + " is not a GGUF file");
    const uint32_t version = r.get<uint32_t>();
    if (!r.ok) return bail(VX_ERR_GGUF, r.err);
    if (version < 2 || version > 3)
        return bail(VX_ERR_GGUF, "unsupported GGUF version " + std::to_string(version) + "; expected v2/v3");
    const uint64_t tensor_count = r.get<uint64_t>();
    const uint64_t metadata_count = r.get<uint64_t>();
    uint64_t alignment = kDefaultAlignment;
    for (uint64_t i = 0; i < metadata_count && r.ok; ++i) {
        std::string key = r.str();
        const uint32_t ty = r.get<uint32_t>();
        MetaValue v;
        std::vector<std::string> strings;
        if (!read_value(r, ty, 0, v, &strings)) break;
        if (ty == 9) {
            if (key == "tokenizer.ggml.tokens") g->tokens = std::move(strings);
            if (key == "tokenizer.ggml.merges") g->merges = std::move(strings);
            continue;
        }
        if (v.kind == META_UINT && (ty == 4 || ty == 10)) {
            if (key == "general.alignment") alignment = v.u ? v.u : 1;  // gguf.rs:242
            g->metadata[key] = v;
        } else if (key.size() <= 128 && (v.kind != META_STRING || v.s.size() <= 512)) {
            g->metadata[key] = v;  // gguf.rs:240
        }
    }
    if (!r.ok) return bail(VX_ERR_GGUF, r.err);
    for (uint64_t i = 0; i < tensor_count && r.ok; ++i) {
        vx_tensor_info t{};
        const std::string name = r.str();
        const uint32_t n_dims = r.get<uint32_t>();
        if (!r.ok) break;
        if (n_dims == 0 || n_dims > 8)
            return bail(VX_ERR_GGUF, "invalid tensor rank " + std::to_string(n_dims) + " for " + name);
        uint64_t elements = 1;
        uint64_t dims[8];
        for (uint32_t d = 0; d < n_dims; ++d) {
            dims[d] = r.get<uint64_t>();
            if (dims[d] && elements > UINT64_MAX / dims[d])
                return bail(VX_ERR_GGUF, "element-count overflow for " + name);
            elements *= dims[d];
        }
        t.ggml_type = r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        if (!r.ok) break;
        if (name.size() >= sizeof(t.name)) return bail(VX_ERR_UNSUPPORTED, "tensor name too long: " + name);
        snprintf(t.name, sizeof(t.name), "%s", name.c_str());
        // Ranks up to 8 are read as gguf.rs:253-256 reads them. The table keeps four
        // dims: a rank 5..8 tensor is listed with its dims 3.. folded into dims[3]
        // (same element count and memory order). No engine reads such a tensor.
        t.n_dims = n_dims < 4u ? n_dims : 4u;
        for (uint32_t d = 0; d < t.n_dims; ++d) t.dims[d] = dims[d];
        for (uint32_t d = 4; d < n_dims; ++d) {
            if (dims[d] && t.dims[3] > UINT64_MAX / dims[d]) {
                // gguf.rs's checked product is 0 once any dim is 0, so a tensor with
                // no elements is accepted whatever its other dims: list it with a
                // folded dim of 0 instead of failing on the fold.
                if (elements == 0) {
                    t.dims[3] = 0;
                    break;
                }
                return bail(VX_ERR_GGUF, "element-count overflow for " + name);
            }
            t.dims[3] *= dims[d];
        }
        std::string err;
        if (!storage_bytes(t.ggml_type, elements, &t.bytes, &err)) return bail(VX_ERR_GGUF, "tensor " + name + ": " + err);
        g->summary.tensor_bytes += t.bytes;
        g->tensors.push_back(t);
    }
    if (!r.ok) return bail(VX_ERR_GGUF, r.err);
    const uint64_t data_offset = (r.pos + alignment - 1) / alignment * alignment;  // gguf.rs:278-279
    for (const vx_tensor_info &t : g->tensors) {
        // data_offset + offset + bytes <= size, without wrapping (gguf.rs:281 checked_add).
        if (data_offset > size || t.offset > size - data_offset || t.bytes > size - data_offset - t.offset)
            return bail(VX_ERR_GGUF, std::string("tensor ") + t.name + " extends beyond end of " + path);
    }
    g->summary.version = version;
    g->summary.tensor_count = tensor_count;
    g->summary.metadata_count = metadata_count;
    g->summary.alignment = alignment;
    g->summary.data_offset = data_offset;
    g->summary.file_bytes = size;
    *out = g;
    return VX_OK;
}

int vx_gguf_close(vx_gguf *g) {
    if (!g) return VX_OK;
    if (g->map) munmap(const_cast<uint8_t *>(g->map), g->file_bytes);
    if (g->fd >= 0) close(g->fd);
    delete g;
    return VX_OK;
}

int vx_gguf_summary_get(const vx_gguf *g, vx_gguf_summary *out) {
    if (!g || !out) return fail(VX_ERR_INVALID_ARG, "vx_gguf_summary_get: null argument");
    *out = g->summary;
    return VX_OK;
}

int vx_gguf_tensor_at(const vx_gguf *g, uint32_t index, vx_tensor_info *out) {
    if (!g || !out) return fail(VX_ERR_INVALID_ARG, "vx_gguf_tensor_at: null argument");
    if (index >= g->tensors.size()) return fail(VX_ERR_INVALID_ARG, "tensor index %u out of range", index);
    *out = g->tensors[index];
    return VX_OK;
}

int vx_gguf_find(const vx_gguf *g, const char *name, vx_tensor_info *out) {
    if (!g || !name) return fail(VX_ERR_INVALID_ARG, "vx_gguf_find: null argument");
    const vx_tensor_info *t = tensor(g, name);
    if (!t) return fail(VX_ERR_NOT_FOUND, "required GGUF tensor \"%s\" is missing from %s", name, g->path.c_str());
    if (out) *out = *t;
    return VX_OK;
}

int vx_gguf_meta(const vx_gguf *g, const char *key, char *out, uint32_t cap) {
    if (!g || !key) return fail(VX_ERR_INVALID_ARG, "vx_gguf_meta: null argument");
    std::string s;
    if (!meta_string(g, key, &s))
        return fail(VX_ERR_NOT_FOUND, "required GGUF metadata key \"%s\" is missing from %s", key, g->path.c_str());
    if (out && cap) snprintf(out, cap, "%s", s.c_str());
    return VX_OK;
}

int vx_gguf_primary_format(const vx_gguf *g, uint32_t *dtype_out) {
    if (!g || !dtype_out) return fail(VX_ERR_INVALID_ARG, "vx_gguf_primary_format: null argument");
    uint64_t q8 = 0, f16 = 0;  // gguf.rs:117-133
    for (const vx_tensor_info &t : g->tensors) {
        uint64_t elements = 1;
        for (uint32_t d = 0; d < t.n_dims; ++d) elements *= t.dims[d];
        if (t.n_dims < 2 || elements < 4096) continue;
        if (t.ggml_type == 8) q8 += t.bytes;
        if (t.ggml_type == 1) f16 += t.bytes;
    }
    if (q8 > 0 && q8 >= f16) { *dtype_out = VX_DTYPE_Q8_0; return VX_OK; }
    if (f16 > 0) { *dtype_out = VX_DTYPE_F16; return VX_OK; }
    return fail(VX_ERR_GGUF, "could not identify BaseLM as Q8_0 or F16 from the tensor table");
}

int vx_model_upload_gguf(vx_ctx *ctx, const vx_gguf *g, vx_model **out) {
    if (!ctx || !g || !out) return fail(VX_ERR_INVALID_ARG, "vx_model_upload_gguf: null argument");
    const uint64_t bytes = g->file_bytes - g->summary.data_offset;
    if (bytes == 0) return fail(VX_ERR_GGUF, "GGUF has an empty data region");
    return vx_model_upload(ctx, g->map + g->summary.data_offset, bytes, g->tensors.data(),
                           (uint32_t)g->tensors.size(), out);
}

int vx_baselm_config_from_gguf(const vx_gguf *g, uint32_t active_context_length, vx_baselm_config *out) {
    if (!g || !out) return fail(VX_ERR_INVALID_ARG, "vx_baselm_config_from_gguf: null argument");
    vx_baselm_config c{};
    std::string arch;
    if (!meta_string(g, "general.architecture", &arch))
        return fail(VX_ERR_NOT_FOUND, "required GGUF metadata key \"general.architecture\" is missing");
    if (arch != "minicpm4")
        return fail(VX_ERR_UNSUPPORTED, "VoxGen BaseLM expects general.architecture=minicpm4, got \"%s\"", arch.c_str());
#define REQ_U32(field, ...)                                                                       \
    if (!meta_u32(g, {__VA_ARGS__}, &c.field))                                                    \
        return fail(VX_ERR_NOT_FOUND, "missing required metadata: %s", #__VA_ARGS__);
#define REQ_F32(field, ...)                                                                       \
    if (!meta_f32(g, {__VA_ARGS__}, &c.field))                                                    \
        return fail(VX_ERR_NOT_FOUND, "missing required metadata: %s", #__VA_ARGS__);
    REQ_U32(context_length, "minicpm4.context_length");
    if (active_context_length == 0 || active_context_length > c.context_length)
        return fail(VX_ERR_INVALID_ARG, "--max-context must be in 1..=%u, got %u", c.context_length,
                    active_context_length);
    c.active_context_length = active_context_length;
    REQ_U32(embedding_length, "minicpm4.embedding_length");
    REQ_U32(block_count, "minicpm4.block_count");
    REQ_U32(feed_forward_length, "minicpm4.feed_forward_length");
    REQ_U32(head_count, "minicpm4.attention.head_count");
    REQ_U32(head_count_kv, "minicpm4.attention.head_count_kv");
    REQ_U32(head_dim, "minicpm4.attention.key_length", "minicpm4.rope.dimension_count");
    REQ_U32(rope_dimension_count, "minicpm4.rope.dimension_count");
    REQ_F32(rms_epsilon, "minicpm4.attention.layer_norm_rms_epsilon");
    REQ_F32(rope_theta, "minicpm4.rope.freq_base");
#undef REQ_U32
#undef REQ_F32
    std::string scaling = "none";
    meta_string(g, "minicpm4.rope.scaling.type", &scaling);
    if (!meta_u32(g, {"minicpm4.rope.scaling.original_context_length", "minicpm4.rope.scaling.original_context_len"},
                  &c.rope_original_context_length))
        c.rope_original_context_length = c.context_length;
    if (!meta_f32(g, {"minicpm4.embedding_scale"}, &c.embedding_scale)) c.embedding_scale = 0.f;
    if (!meta_f32(g, {"minicpm4.residual_scale"}, &c.residual_scale)) c.residual_scale = 0.f;
    if (!meta_f32(g, {"minicpm4.logit_scale"}, &c.logit_scale)) c.logit_scale = 0.f;
    if (c.embedding_length != 2048 || c.block_count != 28 || c.feed_forward_length != 6144 || c.head_count != 16 ||
        c.head_count_kv != 2 || c.head_dim != 128 || c.rope_dimension_count != 128)
        return fail(VX_ERR_UNSUPPORTED,
                    "unsupported MiniCPM4 BaseLM geometry: embd=%u, layers=%u, ffn=%u, heads=%u, kv_heads=%u, "
                    "head_dim=%u, rope_dim=%u",
                    c.embedding_length, c.block_count, c.feed_forward_length, c.head_count, c.head_count_kv,
                    c.head_dim, c.rope_dimension_count);
    if (c.head_count % c.head_count_kv)
        return fail(VX_ERR_SHAPE, "head_count %u is not divisible by head_count_kv %u", c.head_count, c.head_count_kv);
    if (c.rope_dimension_count != c.head_dim)
        return fail(VX_ERR_UNSUPPORTED, "partial RoPE is not implemented");
    if (scaling != "longrope" && scaling != "none")
        return fail(VX_ERR_UNSUPPORTED, "unsupported RoPE scaling type \"%s\"; expected longrope", scaling.c_str());
    c.rope_longrope = scaling == "longrope";
    c.kv_dim = c.head_count_kv * c.head_dim;
    const uint64_t H = c.embedding_length;
    const vx_tensor_info *t;
    VX_CHECK(need_tensor(g, "token_embd.weight", &t));
    if (t->n_dims != 2) return fail(VX_ERR_SHAPE, "token_embd.weight must be rank 2");
    if (t->dims[1] > 0xffffffffull) return fail(VX_ERR_SHAPE, "vocabulary size exceeds u32");
    c.vocab_size = (uint32_t)t->dims[1];
    VX_CHECK(dims_eq(t, {H, c.vocab_size}));
    VX_CHECK(is_matrix(t));
    const vx_tensor_info *o = tensor(g, "output.weight");
    if (o) {
        VX_CHECK(dims_eq(o, {H, c.vocab_size}));
        VX_CHECK(is_matrix(o));
    }
    c.tied_output = o ? 0u : 1u;
    VX_CHECK(need_tensor(g, "output_norm.weight", &t));
    VX_CHECK(dims_eq(t, {H}));
    if (c.rope_longrope) {
        for (const char *n : {"rope_factors_short.weight", "rope_factors_long.weight"}) {
            VX_CHECK(need_tensor(g, n, &t));
            VX_CHECK(dims_eq(t, {(uint64_t)c.head_dim / 2u}));
            VX_CHECK(is_f32(t));
        }
    }
    const uint64_t KV = c.kv_dim, FF = c.feed_forward_length;
    for (uint32_t l = 0; l < c.block_count; ++l) {  // validate_layer baselm.rs:227-262
        const std::string p = "blk." + std::to_string(l) + ".";
        for (const char *n : {"attn_norm.weight", "ffn_norm.weight"}) {
            VX_CHECK(need_tensor(g, p + n, &t));
            VX_CHECK(dims_eq(t, {H}));
            VX_CHECK(is_f32(t));
        }
        const struct {
            const char *n;
            uint64_t a, b;
        } mats[] = {{"attn_q.weight", H, H},       {"attn_k.weight", H, KV},   {"attn_v.weight", H, KV},
                    {"attn_output.weight", H, H},  {"ffn_gate.weight", H, FF}, {"ffn_up.weight", H, FF},
                    {"ffn_down.weight", FF, H}};
        for (const auto &m : mats) {
            VX_CHECK(need_tensor(g, p + m.n, &t));
            VX_CHECK(dims_eq(t, {m.a, m.b}));
            VX_CHECK(is_matrix(t));
        }
    }
    VX_CHECK(need_tensor(g, "output_norm.weight", &t));
    VX_CHECK(is_f32(t));
    *out = c;
    return VX_OK;
}

// AcousticConfig::from_gguf (acoustic.rs:59-125) with GgufSummary::validate_acoustic_f16
// (gguf.rs:150-160) and validate_tensors (acoustic.rs:127-174).
int vx_acoustic_config_from_gguf(const vx_gguf *g, const vx_baselm_config *base, uint32_t active_context_length,
                                 vx_acoustic_config *out) {
    if (!g || !base || !out) return fail(VX_ERR_INVALID_ARG, "vx_acoustic_config_from_gguf: null argument");
    bool any_f16 = false;
    for (const vx_tensor_info &t : g->tensors) {
        if (t.ggml_type != 0 && t.ggml_type != 1)
            return fail(VX_ERR_UNSUPPORTED, "Unsupported acoustic tensor type %u in %s; the F16 acoustic GGUF is required",
                        t.ggml_type, t.name);
        uint64_t elements = 1;
        for (uint32_t d = 0; d < t.n_dims; ++d) elements *= t.dims[d];
        if (t.ggml_type == 1 && elements >= 4096) any_f16 = true;
    }
    if (!any_f16) return fail(VX_ERR_GGUF, "acoustic GGUF does not contain expected F16 weight tensors");
    std::string arch, no_rope;
    if (!meta_string(g, "general.architecture", &arch))
        return fail(VX_ERR_NOT_FOUND, "required GGUF metadata key \"general.architecture\" is missing");
    if (arch != "voxcpm-acoustic")
        return fail(VX_ERR_UNSUPPORTED, "expected general.architecture=voxcpm-acoustic for the acoustic GGUF, got \"%s\"",
                    arch.c_str());
    vx_acoustic_config c{};
    if (!meta_f32(g, {"voxcpm.model_version"}, &c.model_version))
        return fail(VX_ERR_NOT_FOUND, "missing required metadata: voxcpm.model_version");
    if (std::fabs(c.model_version - 2.0f) > 0.01f)
        return fail(VX_ERR_UNSUPPORTED, "specialized for VoxCPM2 acoustic v2.0, got model_version=%g", c.model_version);
    if (active_context_length == 0 || active_context_length > 8192u)  // VOXCPM2_MAX_GENERATION_CONTEXT
        return fail(VX_ERR_INVALID_ARG, "ResidualLM --max-context must be in 1..=8192; got %u", active_context_length);
    if (!meta_u32(g, {"voxcpm.residual_lm.n_layer"}, &c.residual_block_count) ||
        !meta_u32(g, {"voxcpm.residual_lm.n_embd"}, &c.embedding_length) ||
        !meta_u32(g, {"voxcpm.fsq.latent_dim"}, &c.fsq_latent_dim) || !meta_f32(g, {"voxcpm.fsq.scale"}, &c.fsq_scale) ||
        !meta_string(g, "voxcpm.residual_lm.no_rope", &no_rope))
        return fail(VX_ERR_NOT_FOUND, "missing required voxcpm.residual_lm / voxcpm.fsq metadata");
    if (no_rope == "true" || no_rope == "1")  // metadata_bool gguf.rs:104-110
        c.no_rope = 1;
    else if (no_rope == "false" || no_rope == "0")
        c.no_rope = 0;
    else
        return fail(VX_ERR_GGUF, "GGUF metadata \"voxcpm.residual_lm.no_rope\" is not a bool");
    if (c.residual_block_count != 8 || c.embedding_length != 2048 || c.fsq_latent_dim != 512 || !c.no_rope)
        return fail(VX_ERR_UNSUPPORTED,
                    "unsupported VoxCPM2 acoustic contract: residual_layers=%u, embd=%u, fsq_latent=%u, no_rope=%u; "
                    "expected 8/2048/512/true",
                    c.residual_block_count, c.embedding_length, c.fsq_latent_dim, c.no_rope);
    if (base->embedding_length != c.embedding_length || base->feed_forward_length != 6144 || base->head_count != 16 ||
        base->head_count_kv != 2 || base->head_dim != 128)
        return fail(VX_ERR_UNSUPPORTED, "BaseLM geometry is incompatible with VoxCPM2 ResidualLM");
    if (!std::isfinite(c.fsq_scale) || c.fsq_scale <= 0.f)
        return fail(VX_ERR_INVALID_ARG, "invalid FSQ scale %g", c.fsq_scale);
    c.feed_forward_length = base->feed_forward_length;
    c.head_count = base->head_count;
    c.head_count_kv = base->head_count_kv;
    c.head_dim = base->head_dim;
    c.kv_dim = base->kv_dim;
    c.active_context_length = active_context_length;
    c.rms_epsilon = base->rms_epsilon;
    c.residual_scale = base->residual_scale == 0.f ? 1.f : base->residual_scale;
    c.fusion_input_dim = c.embedding_length * 2u;
    const uint64_t H = c.embedding_length, L = c.fsq_latent_dim, KV = c.kv_dim, FF = c.feed_forward_length;
    const vx_tensor_info *t;
    auto f16_matrix = [&](const std::string &name, uint64_t cols, uint64_t rows) -> int {  // require_matrix(.., true)
        VX_CHECK(need_tensor(g, name, &t));
        VX_CHECK(dims_eq(t, {cols, rows}));
        if (t->ggml_type != 1)
            return fail(VX_ERR_SHAPE, "tensor %s is type %u, expected F16 from VoxCPM2-Acoustic-F16.gguf", t->name,
                        t->ggml_type);
        return VX_OK;
    };
    auto vector = [&](const std::string &name, uint64_t n, bool allow_f32) -> int {  // require_vector
        VX_CHECK(need_tensor(g, name, &t));
        VX_CHECK(dims_eq(t, {n}));
        if (!(t->ggml_type == 1 || (allow_f32 && t->ggml_type == 0)))
            return fail(VX_ERR_SHAPE, "tensor %s uses unsupported vector type %u", t->name, t->ggml_type);
        return VX_OK;
    };
    VX_CHECK(f16_matrix("fsq.in_proj.weight", H, L));
    VX_CHECK(vector("fsq.in_proj.bias", L, false));
    VX_CHECK(f16_matrix("fsq.out_proj.weight", L, H));
    VX_CHECK(vector("fsq.out_proj.bias", H, false));
    VX_CHECK(f16_matrix("projections.res_fusion_proj.weight", c.fusion_input_dim, H));
    VX_CHECK(vector("projections.res_fusion_proj.bias", H, false));
    VX_CHECK(vector("residual_lm.output_norm.weight", H, true));
    VX_CHECK(is_f32(t));
    for (uint32_t l = 0; l < c.residual_block_count; ++l) {
        const std::string p = "residual_lm.blk." + std::to_string(l) + ".";
        for (const char *n : {"attn_norm.weight", "ffn_norm.weight"}) {
            VX_CHECK(vector(p + n, H, true));
            VX_CHECK(is_f32(t));
        }
        const struct {
            const char *n;
            uint64_t cols, rows;
        } mats[] = {{"attn_q.weight", H, H},       {"attn_k.weight", H, KV},   {"attn_v.weight", H, KV},
                    {"attn_output.weight", H, H},  {"ffn_gate.weight", H, FF}, {"ffn_up.weight", H, FF},
                    {"ffn_down.weight", FF, H}};
        for (const auto &m : mats) VX_CHECK(f16_matrix(p + m.n, m.cols, m.rows));
    }
    VX_CHECK(f16_matrix("stop_predictor.linear1.weight", H, H));
    VX_CHECK(vector("stop_predictor.linear1.bias", H, true));
    VX_CHECK(f16_matrix("stop_predictor.linear2.weight", H, 2));
    *out = c;
    return VX_OK;
}

// AudioVaeConfig::from_gguf (audiovae.rs:49-79) and validate_tensors
// (audiovae.rs:81-128).
int vx_audiovae_config_from_gguf(const vx_gguf *g, vx_audiovae_config *out) {
    if (!g || !out) return fail(VX_ERR_INVALID_ARG, "vx_audiovae_config_from_gguf: null argument");
    vx_audiovae_config c{};
    float version = 0.f;
    if (!meta_f32(g, {"voxcpm.model_version"}, &version))
        return fail(VX_ERR_NOT_FOUND, "missing required metadata: voxcpm.model_version");
    if (std::fabs(version - 2.0f) > 0.01f)
        return fail(VX_ERR_UNSUPPORTED, "AudioVAE V2 requires VoxCPM2 acoustic model_version=2.0, got %g", version);
    std::string cond;
    if (!meta_u32(g, {"voxcpm.audiovae.encoder_dim"}, &c.encoder_dim) ||
        !meta_u32(g, {"voxcpm.audiovae.latent_dim"}, &c.latent_dim) ||
        !meta_u32(g, {"voxcpm.audiovae.decoder_dim"}, &c.decoder_dim) ||
        !meta_u32(g, {"voxcpm.audiovae.sample_rate"}, &c.sample_rate) ||
        !meta_u32(g, {"voxcpm.audiovae.out_sample_rate"}, &c.out_sample_rate) ||
        !meta_string(g, "voxcpm.audiovae.cond_type", &cond) || !meta_u32(g, {"voxcpm.patch_size"}, &c.patch_size))
        return fail(VX_ERR_NOT_FOUND, "missing required voxcpm.audiovae / voxcpm.patch_size metadata");
    if (c.encoder_dim != 128 || c.latent_dim != 64 || c.decoder_dim != 2048 || c.sample_rate != 16000 ||
        c.out_sample_rate != 48000 || c.patch_size != 4)
        return fail(VX_ERR_UNSUPPORTED, "unsupported VoxCPM2 AudioVAE geometry: enc=%u, latent=%u, dec=%u, sr=%u, "
                    "out_sr=%u, patch=%u", c.encoder_dim, c.latent_dim, c.decoder_dim, c.sample_rate,
                    c.out_sample_rate, c.patch_size);
    if (cond != "scale_bias")
        return fail(VX_ERR_UNSUPPORTED, "AudioVAE cond_type must be scale_bias, got \"%s\"", cond.c_str());
    static const uint32_t enc[4] = {2, 5, 8, 8}, dec[6] = {8, 6, 5, 2, 2, 2}, bins[3] = {20000, 30000, 40000};
    c.encoder_hop = c.decoder_hop = 1;
    for (uint32_t i = 0; i < 4; ++i) c.encoder_hop *= (c.encoder_rates[i] = enc[i]);
    for (uint32_t i = 0; i < 6; ++i) c.decoder_hop *= (c.decoder_rates[i] = dec[i]);
    c.input_samples_per_patch = c.encoder_hop * c.patch_size;
    c.output_samples_per_patch = c.decoder_hop * c.patch_size;
    for (uint32_t i = 0; i < 3; ++i) {
        c.sr_bin_boundaries[i] = bins[i];
        if (c.out_sample_rate > bins[i] && c.decoder_sr_bucket == i) c.decoder_sr_bucket = i + 1;
    }
    c.depthwise = 1;
    const vx_tensor_info *t;
    auto f16 = [&](const std::string &name) -> int {   // require_f16
        VX_CHECK(need_tensor(g, name, &t));
        if (t->ggml_type != 1) return fail(VX_ERR_SHAPE, "AudioVAE tensor %s is type %u, expected F16", t->name,
                                           t->ggml_type);
        return VX_OK;
    };
    auto elements = [&]() {
        uint64_t n = 1;
        for (uint32_t d = 0; d < t->n_dims; ++d) n *= t->dims[d];
        return n;
    };
    auto alpha = [&](const std::string &name, uint64_t ch) -> int {   // require_alpha
        VX_CHECK(f16(name));
        if (elements() != ch) return fail(VX_ERR_SHAPE, "AudioVAE alpha %s has %llu values, expected %llu", t->name,
                                          (unsigned long long)elements(), (unsigned long long)ch);
        return VX_OK;
    };
    auto conv = [&](const std::string &base, uint64_t in_c, uint64_t out_c, uint64_t k, uint64_t groups,
                    bool transpose) -> int {   // require_conv
        VX_CHECK(f16(base));
        VX_CHECK(dims_eq(t, {k, transpose ? out_c / groups : in_c / groups, transpose ? in_c : out_c}));
        VX_CHECK(f16(base + ".bias"));
        if (elements() != out_c) return fail(VX_ERR_SHAPE, "AudioVAE bias %s has %llu values, expected %llu", t->name,
                                             (unsigned long long)elements(), (unsigned long long)out_c);
        return VX_OK;
    };
    VX_CHECK(conv("audio_vae.encoder.block.0", 1, 128, 7, 1, false));
    uint64_t ch = c.encoder_dim;
    for (uint32_t stage = 0; stage < 4; ++stage) {
        const std::string b = "audio_vae.encoder.block." + std::to_string(stage + 1);
        for (uint32_t ri = 0; ri < 3; ++ri) {
            const std::string p = b + ".block." + std::to_string(ri) + ".block";
            VX_CHECK(alpha(p + ".0.alpha", ch));
            VX_CHECK(conv(p + ".1", ch, ch, 7, ch, false));
            VX_CHECK(alpha(p + ".2.alpha", ch));
            VX_CHECK(conv(p + ".3", ch, ch, 1, 1, false));
        }
        VX_CHECK(alpha(b + ".block.3.alpha", ch));
        VX_CHECK(conv(b + ".block.4", ch, ch * 2, enc[stage] * 2u, 1, false));
        ch *= 2;
    }
    VX_CHECK(conv("audio_vae.encoder.fc_mu", ch, c.latent_dim, 3, 1, false));
    VX_CHECK(conv("audio_vae.encoder.fc_logvar", ch, c.latent_dim, 3, 1, false));
    VX_CHECK(conv("audio_vae.decoder.model.0", c.latent_dim, c.latent_dim, 7, c.latent_dim, false));
    VX_CHECK(conv("audio_vae.decoder.model.1", c.latent_dim, c.decoder_dim, 1, 1, false));
    uint64_t din = c.decoder_dim;
    for (uint32_t i = 0; i < 6; ++i) {
        const std::string mi = std::to_string(i + 2), p = "audio_vae.decoder.model." + mi;
        const uint64_t dout = din / 2;
        for (const char *kind : {"scale_embed", "bias_embed"}) {   // require_sr_embed
            VX_CHECK(f16("audio_vae.decoder.sr_cond_model." + mi + "." + kind));
            VX_CHECK(dims_eq(t, {din, 4}));
        }
        VX_CHECK(alpha(p + ".block.0.alpha", din));
        VX_CHECK(conv(p + ".block.1", din, dout, dec[i] * 2u, 1, true));
        for (uint32_t rj = 0; rj < 3; ++rj) {
            const std::string q = p + ".block." + std::to_string(rj + 2) + ".block";
            VX_CHECK(alpha(q + ".0.alpha", dout));
            VX_CHECK(conv(q + ".1", dout, dout, 7, dout, false));
            VX_CHECK(alpha(q + ".2.alpha", dout));
            VX_CHECK(conv(q + ".3", dout, dout, 1, 1, false));
        }
        din = dout;
    }
    VX_CHECK(alpha("audio_vae.decoder.model.8.alpha", din));
    VX_CHECK(conv("audio_vae.decoder.model.9", din, 1, 7, 1, false));
    *out = c;
    return VX_OK;
}

}  // extern "C"
