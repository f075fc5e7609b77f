// GGUF v2/v3 reader and the BitNet model loader that fills the device
// registry from it.
//
// Reference: GgufFile::parse (src/gguf/reader.rs:120-415, helpers :417-800),
// TensorView and the I2_S trailing scale block (src/gguf/tensor.rs:21-54,
// :86-105, :278-309), ModelConfig::from_gguf_metadata_with_prefix
// (src/model/config.rs:61-160), the BitNet architecture strings and roles
// (src/model/architecture/bitnet.rs, mod.rs:40-80) and ModelGraph::from_gguf
// (src/model/graph.rs:79-237, validate_layer_tensor :368-420).
//
// The file is read in place: a parsed wm_gguf keeps pointers into the
// caller's buffer (wm_gguf_parse) or into its own read-only mapping
// (wm_gguf_open); tensor bytes are only read when they are uploaded.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <array>
#include <initializer_list>
#include <map>
#include <string>
#include <vector>

#include "wm_internal.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" read as a little-endian u32
constexpr uint64_t kDefaultAlignment = 32;
constexpr uint64_t kMaxTensors = 1000000, kMaxKv = 1000000, kMaxArray = 1000000;
constexpr uint32_t kMaxDims = 4;
constexpr int kMaxArrayDepth = 16;
constexpr uint64_t kMaxString = 1048576;
constexpr uint64_t kI2sScaleBlock = 32;

enum vtype : uint32_t {
    V_U8 = 0, V_I8, V_U16, V_I16, V_U32, V_I32, V_F32, V_BOOL, V_STR, V_ARR, V_U64, V_I64, V_F64
};

struct gg_value {
    uint32_t type = 0;
    uint64_t u = 0;  // unsigned integers and bool
    int64_t i = 0;   // signed integers
    double f = 0.0;  // floats
    std::string s;
    std::vector<gg_value> arr;
    // GgufValue::as_u64 (reader.rs:48-59): unsigned types, and signed ones >= 0
    bool as_u64(uint64_t *out) const {
        switch (type) {
            case V_U8: case V_U16: case V_U32: case V_U64: *out = u; return true;
            case V_I32: case V_I64: if (i >= 0) { *out = (uint64_t)i; return true; } return false;
            default: return false;
        }
    }
    // GgufValue::as_f32 (reader.rs:70-76)
    bool as_f32(float *out) const {
        if (type == V_F32) { *out = (float)f; return true; }
        if (type == V_F64) { *out = (float)f; return true; }
        return false;
    }
};

struct gg_tensor {
    std::string name;
    std::vector<uint64_t> shape;
    uint32_t type = 0;
    uint64_t offset = 0, len = 0;  // absolute file offset and data bytes
    bool has_scale = false;        // I2_S: the 32-byte block after the data
};

// the parse error and the status it maps onto
struct gg_error {
    wm_status st = WM_OK;
    std::string msg;
};

struct cursor {
    const uint8_t *p;
    uint64_t len, pos = 0;
    bool take(void *dst, uint64_t n) {
        if (n > len - pos) return false;
        std::memcpy(dst, p + pos, n);
        pos += n;
        return true;
    }
    template <typename T>
    bool get(T *v) { return take(v, sizeof(T)); }
};

wm_status fail(gg_error *e, wm_status st, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    e->st = st;
    e->msg = buf;
    return st;
}

// UTF-8 validation with the position and length rules of Rust's
// core::str::from_utf8 (the reference decodes every string with
// String::from_utf8, reader.rs:465): on failure `why` is that error's text,
// "invalid utf-8 sequence of N bytes from index I" or "incomplete utf-8
// byte sequence from index I".
bool valid_utf8(const std::string &s, std::string *why) {
    const size_t n = s.size();
    size_t i = 0;
    const auto b = [&](size_t k) { return (uint8_t)s[k]; };
    const auto bad = [&](size_t start, int len) {
        *why = len ? "invalid utf-8 sequence of " + std::to_string(len) + " bytes from index " + std::to_string(start)
                   : "incomplete utf-8 byte sequence from index " + std::to_string(start);
        return false;
    };
    while (i < n) {
        const uint8_t c = b(i);
        if (c < 0x80) { i++; continue; }
        int width = c >= 0xC2 && c <= 0xDF ? 2 : c >= 0xE0 && c <= 0xEF ? 3 : c >= 0xF0 && c <= 0xF4 ? 4 : 0;
        if (!width) return bad(i, 1);
        // the second byte's range depends on the first (no overlongs, no
        // surrogates, nothing past U+10FFFF)
        uint8_t lo = 0x80, hi = 0xBF;
        if (c == 0xE0) lo = 0xA0;
        else if (c == 0xED) hi = 0x9F;
        else if (c == 0xF0) lo = 0x90;
        else if (c == 0xF4) hi = 0x8F;
        if (i + 1 >= n) return bad(i, 0);
        if (b(i + 1) < lo || b(i + 1) > hi) return bad(i, 1);
        for (int k = 2; k < width; k++) {
            if (i + k >= n) return bad(i, 0);
            if ((b(i + k) & 0xC0) != 0x80) return bad(i, k);
        }
        i += (size_t)width;
    }
    return true;
}

// read_gguf_string (reader.rs:452-466): u64 length, at most 1 MiB, UTF-8
bool read_string(cursor &c, std::string *out, std::string *why) {
    uint64_t n;
    if (!c.get(&n)) { *why = "string length: unexpected end of data"; return false; }
    if (n > kMaxString) {
        *why = "string length " + std::to_string(n) + " exceeds 1 MiB safety limit";
        return false;
    }
    out->assign(n, '\0');
    if (!c.take(&(*out)[0], n)) { *why = "string body: unexpected end of data"; return false; }
    std::string u;
    if (!valid_utf8(*out, &u)) { *why = "invalid UTF-8: " + u; return false; }
    return true;
}

// the smallest encoding of a value of each type, for the count checks
// (reader.rs validate_array)
uint64_t min_size(uint32_t t) {
    switch (t) {
        case V_U8: case V_I8: case V_BOOL: return 1;
        case V_U16: case V_I16: return 2;
        case V_U32: case V_I32: case V_F32: return 4;
        case V_U64: case V_I64: case V_F64: case V_STR: return 8;
        case V_ARR: return 12;
        default: return 1;
    }
}

bool read_value(cursor &c, uint32_t t, gg_value *v, int depth, std::string *why) {
    v->type = t;
    switch (t) {
        case V_U8: { uint8_t x; if (!c.get(&x)) break; v->u = x; return true; }
        case V_I8: { int8_t x; if (!c.get(&x)) break; v->i = x; return true; }
        case V_U16: { uint16_t x; if (!c.get(&x)) break; v->u = x; return true; }
        case V_I16: { int16_t x; if (!c.get(&x)) break; v->i = x; return true; }
        case V_U32: { uint32_t x; if (!c.get(&x)) break; v->u = x; return true; }
        case V_I32: { int32_t x; if (!c.get(&x)) break; v->i = x; return true; }
        case V_F32: { float x; if (!c.get(&x)) break; v->f = x; return true; }
        case V_BOOL: { uint8_t x; if (!c.get(&x)) break; v->u = x != 0; return true; }
        case V_U64: { uint64_t x; if (!c.get(&x)) break; v->u = x; return true; }
        case V_I64: { int64_t x; if (!c.get(&x)) break; v->i = x; return true; }
        case V_F64: { double x; if (!c.get(&x)) break; v->f = x; return true; }
        case V_STR: return read_string(c, &v->s, why);
        case V_ARR: {
            uint32_t et;
            uint64_t n;
            if (!c.get(&et)) { *why = "array element type: unexpected end of data"; return false; }
            if (!c.get(&n)) { *why = "array count: unexpected end of data"; return false; }
            // validate_array (reader.rs:633-681)
            if (depth + 1 > kMaxArrayDepth) {
                *why = "metadata array nesting depth " + std::to_string(depth + 1) + " exceeds 16";
                return false;
            }
            if (n > kMaxArray) {
                *why = "array count " + std::to_string(n) + " exceeds safety limit " + std::to_string(kMaxArray);
                return false;
            }
            if (et > V_F64) { *why = "unknown type tag " + std::to_string(et) + " in array element"; return false; }
            if (n * min_size(et) > c.len - c.pos) {
                *why = "array of " + std::to_string(n) + " elements cannot fit in " +
                       std::to_string(c.len - c.pos) + " remaining bytes";
                return false;
            }
            v->arr.resize(n);
            for (uint64_t k = 0; k < n; k++)
                if (!read_value(c, et, &v->arr[k], depth + 1, why)) {
                    *why = "array[" + std::to_string(k) + "]: " + *why;
                    return false;
                }
            return true;
        }
        default:
            *why = "unknown value type " + std::to_string(t);
            return false;
    }
    *why = "value: unexpected end of data";
    return false;
}

// compute_tensor_byte_len (reader.rs:688-760, tensor.rs:104-200): bytes of
// a tensor of this type and shape; false when the type's size is unknown
// (the tensor is then rejected).  The row-blocked types need whole blocks
// per row.
bool tensor_bytes(const std::vector<uint64_t> &shape, uint32_t type, uint64_t *out, std::string *why) {
    struct row_type { uint32_t id; uint64_t block, bytes; const char *name; };
    static const row_type kRows[] = {{2, 32, 18, "Q4_0"}, {14, 256, 210, "Q6_K"},
                                     {12, 256, 144, "Q4_K"}, {8, 32, 34, "Q8_0"}};
    for (const auto &rt : kRows) {
        if (rt.id != type) continue;
        if (shape.empty()) { *why = std::string(rt.name) + " tensor has no dimensions"; return false; }
        if (shape[0] == 0) { *out = 0; return true; }
        if (shape[0] % rt.block) {
            *why = std::string(rt.name) + " row length " + std::to_string(shape[0]) +
                   " is not a multiple of " + std::to_string(rt.block);
            return false;
        }
        unsigned __int128 v = (unsigned __int128)(shape[0] / rt.block) * rt.bytes;
        for (size_t d = 1; d < shape.size(); d++) {
            v *= shape[d];
            if (v >> 64) break;  // stays above 2^64 from here on: each factor fits 64 bits
        }
        if (v >> 64) { *why = std::string(rt.name) + " tensor size overflow"; return false; }
        *out = (uint64_t)v;
        return true;
    }
    unsigned __int128 n = 1;
    for (uint64_t d : shape) {
        n *= d;
        if (n >> 64) { *why = "shape product overflow"; return false; }
    }
    if (n == 0) { *out = 0; return true; }
    uint64_t block = 0, bytes = 0;
    switch (type) {
        case 0: block = 1; bytes = 4; break;                      // F32
        case 1: case 30: block = 1; bytes = 2; break;             // F16, BF16
        case 28: case 27: block = 1; bytes = 8; break;            // F64, I64
        case 24: case 37: block = 1; bytes = 1; break;            // I8, I8_S
        case 25: block = 1; bytes = 2; break;                     // I16
        case 26: block = 1; bytes = 4; break;                     // I32
        case 3: block = 32; bytes = 20; break;                    // Q4_1
        case 6: block = 32; bytes = 22; break;                    // Q5_0
        case 7: block = 32; bytes = 24; break;                    // Q5_1
        case 9: block = 32; bytes = 40; break;                    // Q8_1
        case 10: block = 256; bytes = 84; break;                  // Q2_K
        case 11: block = 256; bytes = 110; break;                 // Q3_K
        case 13: block = 256; bytes = 176; break;                 // Q5_K
        case 15: block = 256; bytes = 292; break;                 // Q8_K
        case WM_TYPE_I2S: block = 128; bytes = 32; break;         // 2 bits per value
        default:
            *why = "has unsupported type " + std::to_string(type) + "; byte length is unknown";
            return false;
    }
    if ((uint64_t)n % block) {
        *why = "element count " + std::to_string((uint64_t)n) + " is not divisible by block size " +
               std::to_string(block) + " for type " + std::to_string(type);
        return false;
    }
    const unsigned __int128 b = (n / block) * bytes;
    if (b >> 64) { *why = "byte length overflow"; return false; }
    *out = (uint64_t)b;
    return true;
}

}  // namespace

struct wm_gguf {
    const uint8_t *data = nullptr;
    uint64_t len = 0;
    void *map = nullptr;  // the mapping owned by wm_gguf_open
    size_t map_len = 0;
    uint32_t version = 0;
    uint64_t alignment = kDefaultAlignment, data_start = 0;
    std::map<std::string, gg_value> meta;
    std::vector<gg_tensor> tensors;
};

namespace {

// validate_count (reader.rs:428-451): a safety limit, then a lower bound on
// the bytes the entries need
wm_status count_check(gg_error *e, const char *what, uint64_t count, uint64_t limit, uint64_t remaining,
                      uint64_t min_entry) {
    if (count > limit)
        return fail(e, WM_E_PARSE, "%s %llu exceeds safety limit %llu", what, (unsigned long long)count,
                    (unsigned long long)limit);
    if (count * min_entry > remaining)  // count <= 1e6: no overflow
        return fail(e, WM_E_PARSE, "%s %llu cannot fit in %llu remaining bytes", what, (unsigned long long)count,
                    (unsigned long long)remaining);
    return WM_OK;
}

wm_status parse(const uint8_t *data, uint64_t len, wm_gguf *g, gg_error *e) {
    cursor c{data, len};
    uint32_t magic, version;
    if (!c.get(&magic)) return fail(e, WM_E_PARSE, "reading magic: unexpected end of data");
    if (magic != kMagic) return fail(e, WM_E_MAGIC, "Invalid GGUF magic (expected 0x46554747, got 0x%08X)", magic);
    if (!c.get(&version)) return fail(e, WM_E_PARSE, "reading version: unexpected end of data");
    if (version != 2 && version != 3)
        return fail(e, WM_E_VERSION, "Unsupported GGUF version: %u (supported: 2, 3)", version);
    uint64_t n_tensors, n_kv;
    if (!c.get(&n_tensors)) return fail(e, WM_E_PARSE, "reading tensor_count: unexpected end of data");
    if (!c.get(&n_kv)) return fail(e, WM_E_PARSE, "reading metadata_kv_count: unexpected end of data");
    if (count_check(e, "tensor_count", n_tensors, kMaxTensors, len - c.pos, 24) ||
        count_check(e, "metadata_kv_count", n_kv, kMaxKv, len - c.pos, 13))
        return e->st;
    g->version = version;
    std::string why;
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key;
        if (!read_string(c, &key, &why))
            return fail(e, WM_E_PARSE, "metadata[%llu] key: %s", (unsigned long long)i, why.c_str());
        uint32_t t;
        gg_value v;
        if (!c.get(&t)) return fail(e, WM_E_PARSE, "metadata[%llu] (key=\"%s\") value: type tag: unexpected end of data", (unsigned long long)i, key.c_str());
        if (!read_value(c, t, &v, 0, &why))
            return fail(e, WM_E_PARSE, "metadata[%llu] (key=\"%s\") value: %s", (unsigned long long)i, key.c_str(), why.c_str());
        g->meta[key] = std::move(v);
    }
    // general.alignment (reader.rs:182-193)
    const auto al = g->meta.find("general.alignment");
    uint64_t a = kDefaultAlignment;
    if (al != g->meta.end() && !al->second.as_u64(&a)) a = kDefaultAlignment;
    if (a == 0 || (a & (a - 1))) return fail(e, WM_E_PARSE, "invalid alignment value: %llu", (unsigned long long)a);
    g->alignment = a;
    if (count_check(e, "tensor_count", n_tensors, kMaxTensors, len - c.pos, 24)) return e->st;
    struct raw { std::string name; std::vector<uint64_t> shape; uint32_t type; uint64_t rel; };
    std::vector<raw> infos(n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        raw &r = infos[i];
        if (!read_string(c, &r.name, &why))
            return fail(e, WM_E_PARSE, "tensor[%llu] name: %s", (unsigned long long)i, why.c_str());
        uint32_t nd;
        if (!c.get(&nd)) return fail(e, WM_E_PARSE, "tensor[%llu] n_dims: unexpected end of data", (unsigned long long)i);
        if (nd > kMaxDims) return fail(e, WM_E_PARSE, "tensor[%llu] n_dims %u exceeds %u", (unsigned long long)i, nd, kMaxDims);
        r.shape.resize(nd);
        for (uint32_t d = 0; d < nd; d++)
            if (!c.get(&r.shape[d]))
                return fail(e, WM_E_PARSE, "tensor[%llu] shape[%u]: unexpected end of data", (unsigned long long)i, d);
        if (!c.get(&r.type)) return fail(e, WM_E_PARSE, "tensor[%llu] ggml_type: unexpected end of data", (unsigned long long)i);
        if (!c.get(&r.rel)) return fail(e, WM_E_PARSE, "tensor[%llu] offset: unexpected end of data", (unsigned long long)i);
    }
    // the data section starts at the next alignment boundary (reader.rs:244-256)
    const uint64_t rem = c.pos % a;
    g->data_start = rem ? c.pos + (a - rem) : c.pos;
    if (!infos.empty() && g->data_start > len)
        return fail(e, WM_E_PARSE, "tensor data section starts beyond EOF: %llu > %llu",
                    (unsigned long long)g->data_start, (unsigned long long)len);
    g->tensors.resize(n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        const raw &r = infos[i];
        gg_tensor &t = g->tensors[i];
        t.name = r.name;
        t.shape = r.shape;
        t.type = r.type;
        if (r.rel > UINT64_MAX - g->data_start)
            return fail(e, WM_E_PARSE, "tensor \"%s\" offset overflow", r.name.c_str());
        t.offset = g->data_start + r.rel;
        uint64_t next = UINT64_MAX;  // the nearest other tensor's start
        for (uint64_t j = 0; j < n_tensors; j++) {
            if (j == i) continue;
            if (infos[j].rel == r.rel)
                return fail(e, WM_E_PARSE, "tensor \"%s\" shares data offset %llu with another tensor",
                            r.name.c_str(), (unsigned long long)r.rel);
            if (infos[j].rel > r.rel && infos[j].rel < next) next = infos[j].rel;
        }
        const uint64_t next_abs = next == UINT64_MAX ? UINT64_MAX : g->data_start + next;
        if (!tensor_bytes(r.shape, r.type, &t.len, &why))
            return fail(e, WM_E_PARSE, why.compare(0, 15, "has unsupported") == 0 ? "tensor \"%s\" %s" : "tensor \"%s\": %s",
                        r.name.c_str(), why.c_str());
        if (t.len > UINT64_MAX - t.offset)
            return fail(e, WM_E_PARSE, "tensor \"%s\" end offset overflow", r.name.c_str());
        const uint64_t end = t.offset + t.len;
        if (end > len)
            return fail(e, WM_E_BOUNDS, "Tensor data out of bounds: tensor \"%s\" requires bytes [%llu..%llu), file size = %llu",
                        r.name.c_str(), (unsigned long long)t.offset, (unsigned long long)end, (unsigned long long)len);
        if (end > next_abs)
            return fail(e, WM_E_PARSE, "tensor \"%s\" range %llu..%llu overlaps next tensor at %llu", r.name.c_str(),
                        (unsigned long long)t.offset, (unsigned long long)end, (unsigned long long)next_abs);
        // I2_S: a 32-byte block after the codes, its first 4 bytes the
        // per-tensor f32 scale (reader.rs:359-392, tensor.rs:278-309)
        if (r.type == WM_TYPE_I2S) {
            const uint64_t scale_end = end + kI2sScaleBlock;
            if (scale_end > len)
                return fail(e, WM_E_BOUNDS, "Tensor data out of bounds: tensor \"%s (scale block)\" requires bytes [%llu..%llu), file size = %llu",
                            r.name.c_str(), (unsigned long long)end, (unsigned long long)scale_end, (unsigned long long)len);
            if (scale_end > next_abs)
                return fail(e, WM_E_PARSE, "I2_S tensor \"%s\" scale block ends at %llu, overlapping next tensor at %llu",
                            r.name.c_str(), (unsigned long long)scale_end, (unsigned long long)next_abs);
            t.has_scale = true;
        }
    }
    return WM_OK;
}

void copy_error(const gg_error &e, char *err, size_t err_len) {
    if (err && err_len) {
        std::snprintf(err, err_len, "%s", e.msg.c_str());
    }
}

const gg_value *meta(const wm_gguf *g, const std::string &key) {
    const auto it = g->meta.find(key);
    return it == g->meta.end() ? nullptr : &it->second;
}

// required_u32 / required_f32 (config.rs:265-309): a missing key, or one of
// another type, is missing metadata; a value past u32 is a parse error
wm_status required_u32(const wm_gguf *g, const std::string &key, uint32_t *out, gg_error *e) {
    const gg_value *v = meta(g, key);
    uint64_t x;
    if (!v || !v->as_u64(&x)) return fail(e, WM_E_METADATA, "Missing required metadata key(s): %s (u32/u64)", key.c_str());
    if (x > UINT32_MAX)
        return fail(e, WM_E_PARSE, "metadata key %s value %llu does not fit in u32", key.c_str(), (unsigned long long)x);
    *out = (uint32_t)x;
    return WM_OK;
}

wm_status required_f32(const wm_gguf *g, const std::string &key, float *out, gg_error *e) {
    const gg_value *v = meta(g, key);
    if (!v || !v->as_f32(out)) return fail(e, WM_E_METADATA, "Missing required metadata key(s): %s (f32)", key.c_str());
    return WM_OK;
}

// ModelConfig::from_gguf_metadata for the BitNet family (config.rs:61-160):
// general.architecture is one of the BitNet strings (bitnet.rs:29-43) and is
// also the prefix of every other key; keys are read, and rejected, in the
// reference's order
wm_status bitnet_config(const wm_gguf *g, wm_model_config *cfg, gg_error *e) {
    const gg_value *arch = meta(g, "general.architecture");
    if (!arch || arch->type != V_STR)
        return fail(e, WM_E_METADATA, "Missing required metadata key(s): general.architecture (string)");
    const std::string &a = arch->s;
    if (a != "bitnet-b1.58" && a != "bitnet-25" && a != "bitnet")
        return fail(e, WM_E_ARCH, "Unsupported architecture: \"%s\"", a.c_str());
    const auto k = [&](const char *suffix) { return a + "." + suffix; };
    uint32_t n_layers, n_embd, n_ff, ctx_len, heads, kv_heads, n_rot, vocab;
    float eps, base;
    if (required_u32(g, k("block_count"), &n_layers, e) || required_u32(g, k("embedding_length"), &n_embd, e) ||
        required_u32(g, k("feed_forward_length"), &n_ff, e) || required_u32(g, k("context_length"), &ctx_len, e) ||
        required_u32(g, k("attention.head_count"), &heads, e) ||
        required_u32(g, k("attention.head_count_kv"), &kv_heads, e) ||
        required_f32(g, k("attention.layer_norm_rms_epsilon"), &eps, e) ||
        required_u32(g, k("rope.dimension_count"), &n_rot, e) || required_f32(g, k("rope.freq_base"), &base, e) ||
        required_u32(g, k("vocab_size"), &vocab, e))
        return e->st;
    if (heads == 0) return fail(e, WM_E_PARSE, "head_count must be > 0");
    if (n_embd % heads) return fail(e, WM_E_PARSE, "embedding_length %u not divisible by head_count %u", n_embd, heads);
    const uint32_t head_dim = n_embd / heads;
    if (kv_heads == 0) return fail(e, WM_E_PARSE, "head_count_kv must be > 0");
    if (heads % kv_heads)
        return fail(e, WM_E_PARSE, "head_count %u not divisible by head_count_kv %u (GQA ratio must be integer)", heads, kv_heads);
    if ((uint64_t)head_dim * kv_heads > UINT32_MAX) return fail(e, WM_E_PARSE, "head_dim * head_count_kv overflow");
    if (n_rot != head_dim) return fail(e, WM_E_PARSE, "rope.dimension_count (%u) must equal head_dim (%u)", n_rot, head_dim);
    if (n_layers == 0) return fail(e, WM_E_PARSE, "block_count must be > 0");
    if (vocab == 0) return fail(e, WM_E_PARSE, "vocab_size must be > 0");
    *cfg = wm_model_config{n_layers, n_embd, n_ff, heads, kv_heads, head_dim, n_rot, vocab, ctx_len, eps, base};
    return WM_OK;
}

const char *type_name(uint32_t t) {
    switch (t) {
        case 0: return "F32";
        case 1: return "F16";
        case 14: return "Q6_K";
        case WM_TYPE_I2S: return "I2_S";
        default: return "other";
    }
}

// check_dtype / check_shape (graph.rs:464-503)
wm_status check_tensor(const gg_tensor *t, uint32_t type, std::initializer_list<uint64_t> shape, gg_error *e) {
    if (t->type != type)
        return fail(e, WM_E_PARSE, "tensor \"%s\": expected dtype %s (%u), got %s (%u)", t->name.c_str(),
                    type_name(type), type, type_name(t->type), t->type);
    if (t->shape != std::vector<uint64_t>(shape)) {
        const auto fmt = [](const std::vector<uint64_t> &v) {
            std::string s = "[";
            for (size_t i = 0; i < v.size(); i++) s += (i ? ", " : "") + std::to_string(v[i]);
            return s + "]";
        };
        return fail(e, WM_E_SHAPE, "tensor \"%s\": expected shape %s, got %s", t->name.c_str(),
                    fmt(std::vector<uint64_t>(shape)).c_str(), fmt(t->shape).c_str());
    }
    return WM_OK;
}

// the tensors of a BitNet model, found and checked before anything is
// uploaded
struct plan {
    const gg_tensor *embd = nullptr, *onorm = nullptr;
    std::vector<std::array<const gg_tensor *, 7>> lin;   // q k v o gate up down
    std::vector<std::array<const gg_tensor *, 4>> norm;  // attn, attn_sub, ffn, ffn_sub
};

// ModelGraph::from_gguf (graph.rs:79-237) for the BitNet sub-norm variant, in
// its order: unique names, no bias tensors, token_embd, output_norm, an
// optional output.weight (checked, then unused: BitNet ties the lm-head to
// token_embd), then every layer's roles in the architecture's order
// (bitnet.rs:58-75) with validate_layer_tensor's dtypes and shapes
// (graph.rs:368-420).  token_embd may be F16 in the reference; this
// library's embedding and lm-head kernels read Q6_K only.
wm_status plan_model(const wm_gguf *g, const wm_model_config &cfg, plan *p, gg_error *e) {
    std::map<std::string, const gg_tensor *> by_name;
    for (const auto &t : g->tensors) by_name.emplace(t.name, &t);
    if (by_name.size() != g->tensors.size())
        return fail(e, WM_E_PARSE, "duplicate tensor names in GGUF tensor directory");
    for (const auto &t : g->tensors)
        if (t.name.size() >= 5 && t.name.compare(t.name.size() - 5, 5, ".bias") == 0)
            return fail(e, WM_E_NOT_IMPLEMENTED, "bias tensor \"%s\" is not supported for BitNet", t.name.c_str());
    const auto need = [&](const std::string &name, const gg_tensor **t) -> wm_status {
        const auto it = by_name.find(name);
        if (it == by_name.end()) return fail(e, WM_E_METADATA, "Missing required metadata key(s): tensor %s", name.c_str());
        *t = it->second;
        return WM_OK;
    };
    const uint64_t E = cfg.n_embd, F = cfg.n_ff, KV = (uint64_t)cfg.n_kv_heads * cfg.head_dim, V = cfg.vocab_size;
    if (need("token_embd.weight", &p->embd)) return e->st;
    if (p->embd->type != WM_TYPE_Q6K) {
        if (p->embd->type == 1)
            return fail(e, WM_E_UNSUPPORTED_TYPE, "tensor \"token_embd.weight\": F16 embeddings are not supported by this library (Q6_K only)");
        return fail(e, WM_E_PARSE, "tensor \"token_embd.weight\": expected dtype F16 or Q6_K, got %s (%u)",
                    type_name(p->embd->type), p->embd->type);
    }
    if (check_tensor(p->embd, WM_TYPE_Q6K, {E, V}, e)) return e->st;
    if (need("output_norm.weight", &p->onorm) || check_tensor(p->onorm, 0, {E}, e)) return e->st;
    const auto outw = by_name.find("output.weight");
    if (outw != by_name.end()) {
        const gg_tensor *t = outw->second;
        if (t->type != 1 && t->type != WM_TYPE_Q6K)
            return fail(e, WM_E_PARSE, "tensor \"output.weight\": expected dtype F16 or Q6_K, got %s (%u)",
                        type_name(t->type), t->type);
        if (check_tensor(t, t->type, {E, V}, e)) return e->st;
    }
    // role order: attn_norm, attn_sub_norm, q, k, v, o, ffn_norm, ffn_sub_norm, gate, up, down
    struct role { const char *name; bool linear; int slot; uint64_t a, b; };
    const role roles[11] = {{"attn_norm", false, 0, E, 0},   {"attn_sub_norm", false, 1, E, 0},
                            {"attn_q", true, 0, E, E},       {"attn_k", true, 1, E, KV},
                            {"attn_v", true, 2, E, KV},      {"attn_output", true, 3, E, E},
                            {"ffn_norm", false, 2, E, 0},    {"ffn_sub_norm", false, 3, F, 0},
                            {"ffn_gate", true, 4, E, F},     {"ffn_up", true, 5, E, F},
                            {"ffn_down", true, 6, F, E}};
    p->lin.resize(cfg.n_layers);
    p->norm.resize(cfg.n_layers);
    for (uint32_t l = 0; l < cfg.n_layers; l++)
        for (const role &r : roles) {
            const gg_tensor *t;
            if (need("blk." + std::to_string(l) + "." + r.name + ".weight", &t)) return e->st;
            if (r.linear) {
                if (check_tensor(t, WM_TYPE_I2S, {r.a, r.b}, e)) return e->st;
                p->lin[l][r.slot] = t;
            } else {
                if (check_tensor(t, 0, {r.a}, e)) return e->st;
                p->norm[l][r.slot] = t;
            }
        }
    return WM_OK;
}

}  // namespace

extern "C" {

wm_status wm_gguf_parse(const uint8_t *data, size_t len, wm_gguf **out, char *err, size_t err_len) {
    if (!out || (!data && len)) return WM_E_ARG;
    *out = nullptr;
    wm_gguf *g = new wm_gguf();
    g->data = data;
    g->len = len;
    gg_error e;
    if (parse(data, len, g, &e) != WM_OK) {
        copy_error(e, err, err_len);
        delete g;
        return e.st;
    }
    *out = g;
    return WM_OK;
}

wm_status wm_gguf_open(const char *path, wm_gguf **out, char *err, size_t err_len) {
    if (!path || !out) return WM_E_ARG;
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    gg_error e;
    if (fd < 0) {
        fail(&e, WM_E_IO, "Invalid model file: %s", path);
        copy_error(e, err, err_len);
        return e.st;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        close(fd);
        fail(&e, WM_E_IO, "Invalid model file: %s", path);
        copy_error(e, err, err_len);
        return e.st;
    }
    if (st.st_size == 0) {  // nothing to map: the parse reports the missing magic
        close(fd);
        return wm_gguf_parse(nullptr, 0, out, err, err_len);
    }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) {
        fail(&e, WM_E_IO, "mmap of %s failed", path);
        copy_error(e, err, err_len);
        return e.st;
    }
    wm_gguf *g = new wm_gguf();
    g->data = static_cast<const uint8_t *>(m);
    g->len = (uint64_t)st.st_size;
    g->map = m;
    g->map_len = (size_t)st.st_size;
    if (parse(g->data, g->len, g, &e) != WM_OK) {
        copy_error(e, err, err_len);
        munmap(m, g->map_len);
        delete g;
        return e.st;
    }
    *out = g;
    return WM_OK;
}

void wm_gguf_close(wm_gguf *g) {
    if (!g) return;
    if (g->map) munmap(g->map, g->map_len);
    delete g;
}

uint32_t wm_gguf_version(const wm_gguf *g) { return g ? g->version : 0; }
uint64_t wm_gguf_alignment(const wm_gguf *g) { return g ? g->alignment : 0; }
uint64_t wm_gguf_tensor_count(const wm_gguf *g) { return g ? (uint64_t)g->tensors.size() : 0; }
uint64_t wm_gguf_data_offset(const wm_gguf *g) { return g ? g->data_start : 0; }

int64_t wm_gguf_find_tensor(const wm_gguf *g, const char *name) {
    if (!g || !name) return -1;
    for (size_t i = 0; i < g->tensors.size(); i++)
        if (g->tensors[i].name == name) return (int64_t)i;
    return -1;
}

wm_status wm_gguf_tensor_info(const wm_gguf *g, uint64_t index, const char **name, uint32_t *type,
                              uint32_t *n_dims, uint64_t shape[4], uint64_t *offset, uint64_t *bytes,
                              const uint8_t **data, const uint8_t **scale_block) {
    if (!g || index >= g->tensors.size()) return WM_E_ARG;
    const gg_tensor &t = g->tensors[index];
    if (name) *name = t.name.c_str();
    if (type) *type = t.type;
    if (n_dims) *n_dims = (uint32_t)t.shape.size();
    if (shape)
        for (size_t d = 0; d < 4; d++) shape[d] = d < t.shape.size() ? t.shape[d] : 0;
    if (offset) *offset = t.offset;
    if (bytes) *bytes = t.len;
    if (data) *data = g->data + t.offset;
    if (scale_block) *scale_block = t.has_scale ? g->data + t.offset + t.len : nullptr;
    return WM_OK;
}

wm_status wm_gguf_meta_u64(const wm_gguf *g, const char *key, uint64_t *out) {
    if (!g || !key || !out) return WM_E_ARG;
    const gg_value *v = meta(g, key);
    if (!v) return WM_E_METADATA;
    return v->as_u64(out) ? WM_OK : WM_E_METADATA;
}

wm_status wm_gguf_meta_f32(const wm_gguf *g, const char *key, float *out) {
    if (!g || !key || !out) return WM_E_ARG;
    const gg_value *v = meta(g, key);
    if (!v) return WM_E_METADATA;
    return v->as_f32(out) ? WM_OK : WM_E_METADATA;
}

wm_status wm_gguf_meta_str(const wm_gguf *g, const char *key, const char **out) {
    if (!g || !key || !out) return WM_E_ARG;
    const gg_value *v = meta(g, key);
    if (!v || v->type != V_STR) return WM_E_METADATA;
    *out = v->s.c_str();
    return WM_OK;
}

wm_status wm_gguf_bitnet_config(const wm_gguf *g, wm_model_config *cfg, char *err, size_t err_len) {
    if (!g || !cfg) return WM_E_ARG;
    gg_error e;
    if (bitnet_config(g, cfg, &e) != WM_OK) {
        copy_error(e, err, err_len);
        return e.st;
    }
    return WM_OK;
}

wm_status wm_gguf_bitnet_check(const wm_gguf *g, char *err, size_t err_len) {
    if (!g) return WM_E_ARG;
    wm_model_config cfg;
    plan p;
    gg_error e;
    if (bitnet_config(g, &cfg, &e) != WM_OK || plan_model(g, cfg, &p, &e) != WM_OK) {
        copy_error(e, err, err_len);
        return e.st;
    }
    return WM_OK;
}

wm_status wm_model_from_gguf(wm_ctx *ctx, const wm_gguf *g, uint32_t max_context, wm_model **out) {
    if (!ctx || !g || !out) return WM_E_ARG;
    *out = nullptr;
    wm_model_config cfg;
    plan p;
    gg_error e;
    if (bitnet_config(g, &cfg, &e) != WM_OK || plan_model(g, cfg, &p, &e) != WM_OK)
        return wm_set_error(ctx, e.st, "%s", e.msg.c_str());
    // KV caches for this model are at most max_context long (0: the file's
    // context_length)
    if (max_context && max_context < cfg.context_length) cfg.context_length = max_context;
    const uint64_t E = cfg.n_embd, F = cfg.n_ff, KV = (uint64_t)cfg.n_kv_heads * cfg.head_dim;
    const uint64_t lin_in[7] = {E, E, E, E, E, E, F}, lin_out[7] = {E, KV, KV, E, F, F, E};
    const auto floats = [&](const gg_tensor *t) {  // f32 little-endian, copied out aligned
        std::vector<float> v(t->len / 4);
        std::memcpy(v.data(), g->data + t->offset, v.size() * 4);
        return v;
    };
    wm_model *m = nullptr;
    wm_status st = wm_model_create(ctx, &cfg, &m);
    if (st) return st;
    for (uint32_t l = 0; l < cfg.n_layers && !st; l++) {
        wm_tensor *ts[7] = {};
        for (int r = 0; r < 7 && !st; r++) {
            const gg_tensor *t = p.lin[l][r];
            st = wm_tensor_upload_i2s(ctx, g->data + t->offset, t->len, g->data + t->offset + t->len,
                                      kI2sScaleBlock, lin_in[r], lin_out[r], &ts[r]);
        }
        if (!st) {
            const std::vector<float> an = floats(p.norm[l][0]), asn = floats(p.norm[l][1]),
                                     fn = floats(p.norm[l][2]), fsn = floats(p.norm[l][3]);
            st = wm_model_set_layer(m, l, ts[0], ts[1], ts[2], ts[3], ts[4], ts[5], ts[6], an.data(),
                                    asn.data(), fn.data(), fsn.data());
        }
        for (wm_tensor *t : ts) wm_tensor_destroy(t);
    }
    if (!st) {
        wm_tensor *te = nullptr;
        st = wm_tensor_upload_q6k(ctx, g->data + p.embd->offset, p.embd->len, E, cfg.vocab_size, &te);
        if (!st) {
            const std::vector<float> on = floats(p.onorm);
            st = wm_model_set_output(m, te, on.data());
        }
        wm_tensor_destroy(te);
    }
    if (st) {
        wm_model_destroy(m);
        return st;
    }
    *out = m;
    return WM_OK;
}

}  // extern "C"
