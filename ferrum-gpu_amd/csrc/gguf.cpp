// GGUF v3 container reader (ferrum_gguf/src/io/reader.rs:1-322) and the device uploads of its
// tensors.
//
// The parser walks the header with a bounds-checked cursor; sizes use checked 64-bit arithmetic,
// and every count read from the header is proven to fit in the file before anything is sized from
// it. Metadata and tensor names are not copied: entries keep offsets into the file's bytes, which
// the handle owns (a heap copy, or a read-only mapping from fh_gguf_open), so a tokenizer table of
// 150k strings costs one offset pair per string. Quantized tensors go to the device as their
// stored bytes (fh_gguf_upload_qweight), never through an f32 round trip.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

#include "internal.hpp"

using namespace fh;

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" little-endian (ferrum_gguf/src/lib.rs:20)
constexpr uint64_t kDefaultAlignment = 32;

enum : uint32_t {
    T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7,
    T_STR = 8, T_ARR = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12
};

struct Span {
    uint64_t off = 0, len = 0;
};

struct Kv {
    Span key;
    uint32_t type = 0;
    Span payload;               // scalar bytes, string bytes, or the packed array elements
    uint32_t elem_type = 0;     // arrays
    uint64_t count = 0;         // arrays
    std::vector<Span> strings;  // string arrays: each element's bytes
};

struct Tensor {
    Span name;
    uint32_t nd = 0;
    uint64_t dims[4] = {0, 0, 0, 0};
    uint32_t type = 0;
    uint64_t offset = 0, elements = 0, nbytes = 0;
};

// Bytes per block and elements per block of the block formats (ferrum_gguf/src/codec/blocks.rs:34-48
// and quant.rs:32-33): Q4_0 18, Q4_1 20, Q5_0 22, Q5_1 24, Q8_0 34, Q8_1 36, MXFP4 17 per 32; the
// k-quants Q2_K 84, Q3_K 110, Q4_K 144, Q5_K 176, Q6_K 210 per 256.
bool block_layout(uint32_t ty, uint64_t *bytes, uint64_t *elems) {
    switch (ty) {
    case FH_GGML_Q4_0: *bytes = 18; *elems = 32; return true;
    case FH_GGML_Q4_1: *bytes = 20; *elems = 32; return true;
    case FH_GGML_Q5_0: *bytes = 22; *elems = 32; return true;
    case FH_GGML_Q5_1: *bytes = 24; *elems = 32; return true;
    case FH_GGML_Q8_0: *bytes = 34; *elems = 32; return true;
    case FH_GGML_Q8_1: *bytes = 36; *elems = 32; return true;
    case FH_GGML_MXFP4: *bytes = 17; *elems = 32; return true;
    case FH_GGML_Q2_K: *bytes = 84; *elems = 256; return true;
    case FH_GGML_Q3_K: *bytes = 110; *elems = 256; return true;
    case FH_GGML_Q4_K: *bytes = 144; *elems = 256; return true;
    case FH_GGML_Q5_K: *bytes = 176; *elems = 256; return true;
    case FH_GGML_Q6_K: *bytes = 210; *elems = 256; return true;
    default: return false;
    }
}

bool mul_ok(uint64_t a, uint64_t b, uint64_t *out) { return !__builtin_mul_overflow(a, b, out); }

// quant::nbytes (quant.rs:17-47), with the same messages.
fh_status nbytes_of(uint32_t ty, uint64_t n, uint64_t *out) {
    uint64_t per = 0;
    switch (ty) {
    case FH_GGML_F32:
    case FH_GGML_I32: per = 4; break;
    case FH_GGML_F16:
    case FH_GGML_I16: per = 2; break;
    default: break;
    }
    if (per) {
        if (!mul_ok(n, per, out)) return fail(FH_ERR_INVALID, "gguf: tensor size overflows");
        return FH_OK;
    }
    uint64_t bytes = 0, elems = 0;
    if (!block_layout(ty, &bytes, &elems)) return fail(FH_ERR_UNSUPPORTED, "gguf: unsupported ggml tensor type %u", ty);
    if (n % elems)
        return fail(FH_ERR_INVALID, "gguf: %llu elements is not a multiple of the block size %llu",
                    (unsigned long long)n, (unsigned long long)elems);
    if (!mul_ok(n / elems, bytes, out)) return fail(FH_ERR_INVALID, "gguf: tensor size overflows");
    return FH_OK;
}

// Strict UTF-8 (what Rust's String::from_utf8 accepts): no overlong forms, no surrogates, nothing
// above U+10FFFF, no truncated sequences.
bool valid_utf8(const uint8_t *s, uint64_t n) {
    uint64_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            i++;
            continue;
        }
        int len;
        uint8_t lo = 0x80, hi = 0xbf;  // range of the second byte
        if (c >= 0xc2 && c <= 0xdf) len = 2;
        else if (c == 0xe0) len = 3, lo = 0xa0;
        else if ((c >= 0xe1 && c <= 0xec) || c == 0xee || c == 0xef) len = 3;
        else if (c == 0xed) len = 3, hi = 0x9f;
        else if (c == 0xf0) len = 4, lo = 0x90;
        else if (c >= 0xf1 && c <= 0xf3) len = 4;
        else if (c == 0xf4) len = 4, hi = 0x8f;
        else return false;
        if (n - i < (uint64_t)len) return false;
        if (s[i + 1] < lo || s[i + 1] > hi) return false;
        for (int j = 2; j < len; j++)
            if ((s[i + j] & 0xc0) != 0x80) return false;
        i += len;
    }
    return true;
}

// Bounds-checked reader over the loaded bytes (reader.rs:103-158).
struct Cursor {
    const uint8_t *b;
    uint64_t len, p = 0;

    fh_status take(uint64_t n, uint64_t *at) {
        uint64_t end;
        if (__builtin_add_overflow(p, n, &end) || end > len) return fail(FH_ERR_INVALID, "gguf: unexpected end of file");
        *at = p;
        p = end;
        return FH_OK;
    }
    template <class T>
    fh_status scalar(T *v) {
        uint64_t at;
        fh_status st = take(sizeof(T), &at);
        if (st) return st;
        std::memcpy(v, b + at, sizeof(T));  // the format is little-endian, as is the host
        return FH_OK;
    }
    fh_status string(Span *s) {
        uint64_t n, at;
        fh_status st = scalar(&n);
        if (st || (st = take(n, &at))) return st;
        if (!valid_utf8(b + at, n)) return fail(FH_ERR_INVALID, "gguf: string is not valid UTF-8");
        *s = {at, n};
        return FH_OK;
    }
    // One value of tag `ty` (reader.rs:125-157). Nested arrays are refused, and an array count
    // beyond the remaining bytes is hostile (every element needs at least one byte).
    fh_status value(uint32_t ty, Kv *kv, bool in_array) {
        uint64_t at;
        switch (ty) {
        case T_U8: case T_I8: case T_BOOL: return take(1, &at);
        case T_U16: case T_I16: return take(2, &at);
        case T_U32: case T_I32: case T_F32: return take(4, &at);
        case T_U64: case T_I64: case T_F64: return take(8, &at);
        case T_STR: {
            Span s;
            fh_status st = string(&s);
            if (st) return st;
            if (in_array) kv->strings.push_back(s);
            else kv->payload = s;
            return FH_OK;
        }
        case T_ARR: {
            if (in_array) return fail(FH_ERR_INVALID, "gguf: nested arrays are not supported");
            uint32_t et;
            uint64_t n;
            fh_status st = scalar(&et);
            if (st || (st = scalar(&n))) return st;
            if (n > len - p) return fail(FH_ERR_INVALID, "gguf: array length exceeds the file");
            kv->elem_type = et;
            kv->count = n;
            if (et == T_STR) kv->strings.reserve(n);  // n <= remaining bytes: bounded by the file
            const uint64_t start = p;
            // as in the reference, the element tag is only checked by reading elements, so an
            // empty array of any tag is accepted
            for (uint64_t i = 0; i < n; i++)
                if ((st = value(et, kv, true))) return st;
            kv->payload = {start, p - start};
            return FH_OK;
        }
        default: return fail(FH_ERR_INVALID, "gguf: unknown metadata value type %u", ty);
        }
    }
};

}  // namespace

struct fh_gguf {
    const uint8_t *bytes = nullptr;  // the loaded bytes (a prefix of the file for parse_prefix)
    uint64_t len = 0;
    uint64_t total = 0;              // the file length extents were checked against
    std::vector<uint8_t> owned;
    void *map = nullptr;
    size_t map_len = 0;
    std::vector<Kv> kv;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string_view, size_t> index;
    uint64_t data_start = 0;

    ~fh_gguf() {
        if (map) munmap(map, map_len);
    }
    std::string_view view(Span s) const { return {(const char *)bytes + s.off, (size_t)s.len}; }
};

namespace {

// Gguf::parse_prefix (reader.rs:172-247) over g->bytes / g->len with extents against g->total.
fh_status parse(fh_gguf *g) {
    Cursor c{g->bytes, g->len};
    uint32_t magic, version;
    fh_status st = c.scalar(&magic);
    if (st) return st;
    if (magic != kMagic) return fail(FH_ERR_INVALID, "gguf: bad magic: not a GGUF file");
    if ((st = c.scalar(&version))) return st;
    if (version != 3) return fail(FH_ERR_INVALID, "gguf: unsupported GGUF version %u (need 3)", version);
    uint64_t n_tensors, n_kv;
    if ((st = c.scalar(&n_tensors)) || (st = c.scalar(&n_kv))) return st;
    // each entry takes at least 8 bytes, which bounds what the counts may claim
    if (n_kv > g->len / 8 || n_tensors > g->len / 8)
        return fail(FH_ERR_INVALID, "gguf: header counts exceed the file size");
    g->kv.resize(n_kv);
    for (auto &kv : g->kv) {
        if ((st = c.string(&kv.key)) || (st = c.scalar(&kv.type))) return st;
        const uint64_t start = c.p;
        if ((st = c.value(kv.type, &kv, false))) return st;
        if (kv.type != T_STR && kv.type != T_ARR) kv.payload = {start, c.p - start};
    }
    g->tensors.resize(n_tensors);
    for (auto &t : g->tensors) {
        if ((st = c.string(&t.name)) || (st = c.scalar(&t.nd))) return st;
        if (t.nd == 0 || t.nd > 4) {
            const std::string_view nm = g->view(t.name);
            return fail(FH_ERR_INVALID, "gguf: tensor '%.*s' has %u dims (1 to 4 supported)", (int)nm.size(),
                        nm.data(), t.nd);
        }
        for (uint32_t d = 0; d < t.nd; d++)
            if ((st = c.scalar(&t.dims[d]))) return st;
        if ((st = c.scalar(&t.type)) || (st = c.scalar(&t.offset))) return st;
    }
    // general.alignment: the first entry of that key decides (Gguf::get finds the first)
    uint64_t alignment = kDefaultAlignment;
    for (const auto &kv : g->kv) {
        if (g->view(kv.key) != "general.alignment") continue;
        uint32_t a = 0;
        if (kv.type == T_U32) std::memcpy(&a, g->bytes + kv.payload.off, 4);
        if (kv.type != T_U32 || a == 0) return fail(FH_ERR_INVALID, "gguf: general.alignment must be a positive u32");
        alignment = a;
        break;
    }
    g->data_start = (c.p + alignment - 1) / alignment * alignment;  // c.p < 2^63: no overflow
    if (g->data_start > g->total) return fail(FH_ERR_INVALID, "gguf: file ends before the tensor data");
    g->index.reserve(n_tensors);
    for (size_t i = 0; i < g->tensors.size(); i++) {
        Tensor &t = g->tensors[i];
        const std::string_view nm = g->view(t.name);
        uint64_t n = 1;
        for (uint32_t d = 0; d < t.nd; d++)
            if (!mul_ok(n, t.dims[d], &n)) return fail(FH_ERR_INVALID, "gguf: tensor element count overflows");
        t.elements = n;
        if ((st = nbytes_of(t.type, n, &t.nbytes))) return st;
        uint64_t start, end;
        if (__builtin_add_overflow(t.offset, g->data_start, &start) || __builtin_add_overflow(start, t.nbytes, &end) ||
            end > g->total)
            return fail(FH_ERR_INVALID, "gguf: tensor '%.*s' extends past the end of the file", (int)nm.size(),
                        nm.data());
        if (!g->index.emplace(nm, i).second)
            return fail(FH_ERR_INVALID, "gguf: duplicate tensor name '%.*s'", (int)nm.size(), nm.data());
    }
    return FH_OK;
}

fh_status finish(fh_gguf *g, fh_gguf **out) {
    fh_status st = parse(g);
    if (st) {
        delete g;
        return st;
    }
    *out = g;
    return FH_OK;
}

const Kv *find_kv(const fh_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    const std::string_view k(key);
    for (const auto &kv : g->kv)
        if (g->view(kv.key) == k) return &kv;
    return nullptr;
}

fh_status lookup(const fh_gguf *g, const char *name, const Tensor **out) {
    if (!g || !name) return fail(FH_ERR_INVALID, "gguf: no file or name");
    auto it = g->index.find(std::string_view(name));
    if (it == g->index.end()) return fail(FH_ERR_INVALID, "gguf: missing tensor '%s'", name);
    *out = &g->tensors[it->second];
    return FH_OK;
}

fh_status span_of(const fh_gguf *g, const char *name, const Tensor *t, const uint8_t **data, size_t *len) {
    const uint64_t start = g->data_start + t->offset;  // inside the file, proven by the parse
    if (start + t->nbytes > g->len)
        return fail(FH_ERR_INVALID, "gguf: tensor '%s' data was not loaded (header-only parse)", name);
    *data = g->bytes + start;
    *len = (size_t)t->nbytes;
    return FH_OK;
}

}  // namespace

extern "C" {

fh_status fh_ggml_nbytes(uint32_t ggml_type, uint64_t n, uint64_t *out) {
    if (!out) return fail(FH_ERR_INVALID, "gguf: no output");
    return nbytes_of(ggml_type, n, out);
}

fh_status fh_gguf_parse_prefix(const uint8_t *bytes, size_t len, uint64_t total, fh_gguf **out) {
    if (!out || (!bytes && len)) return fail(FH_ERR_INVALID, "gguf: no bytes or output");
    *out = nullptr;
    if (total < len) return fail(FH_ERR_INVALID, "gguf: the prefix is longer than the file");
    fh_gguf *g = new (std::nothrow) fh_gguf;
    if (!g) return fail(FH_ERR_OOM, "host out of memory");
    try {
        g->owned.assign(bytes, bytes + len);
    } catch (const std::bad_alloc &) {
        delete g;
        return fail(FH_ERR_OOM, "host out of memory");
    }
    g->bytes = g->owned.data();
    g->len = len;
    g->total = total;
    try {
        return finish(g, out);
    } catch (const std::bad_alloc &) {
        return fail(FH_ERR_OOM, "host out of memory");
    }
}

fh_status fh_gguf_parse(const uint8_t *bytes, size_t len, fh_gguf **out) {
    return fh_gguf_parse_prefix(bytes, len, len, out);
}

fh_status fh_gguf_open(const char *path, fh_gguf **out) {
    if (!out || !path) return fail(FH_ERR_INVALID, "gguf: no path or output");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(FH_ERR_INVALID, "gguf: cannot open '%s': %s", path, strerror(errno));
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        const int e = errno;
        close(fd);
        return fail(FH_ERR_INVALID, "gguf: cannot stat '%s': %s", path, strerror(e));
    }
    fh_gguf *g = new (std::nothrow) fh_gguf;
    if (!g) {
        close(fd);
        return fail(FH_ERR_OOM, "host out of memory");
    }
    if (sb.st_size > 0) {
        void *m = mmap(nullptr, (size_t)sb.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            const int e = errno;
            close(fd);
            delete g;
            return fail(FH_ERR_INVALID, "gguf: cannot map '%s': %s", path, strerror(e));
        }
        g->map = m;
        g->map_len = (size_t)sb.st_size;
        g->bytes = (const uint8_t *)m;
    }
    close(fd);  // the mapping keeps the file
    g->len = g->total = (uint64_t)sb.st_size;
    try {
        return finish(g, out);
    } catch (const std::bad_alloc &) {
        return fail(FH_ERR_OOM, "host out of memory");
    }
}

void fh_gguf_close(fh_gguf *g) { delete g; }

size_t fh_gguf_describe(const fh_gguf *g, char *buf, size_t cap) {
    if (!g) return 0;
    const int n = snprintf(buf, buf ? cap : 0, "Gguf { %zu keys, %zu tensors, %llu bytes }", g->kv.size(),
                           g->tensors.size(), (unsigned long long)g->len);
    return n < 0 ? 0 : (size_t)n;
}

size_t fh_gguf_kv_count(const fh_gguf *g) { return g ? g->kv.size() : 0; }

fh_status fh_gguf_kv_key(const fh_gguf *g, size_t i, const char **key, size_t *len) {
    if (!g || i >= g->kv.size() || !key || !len) return fail(FH_ERR_INVALID, "gguf: no metadata entry %zu", i);
    *key = (const char *)g->bytes + g->kv[i].key.off;
    *len = (size_t)g->kv[i].key.len;
    return FH_OK;
}

fh_status fh_gguf_kv_value(const fh_gguf *g, size_t i, uint32_t *type, const uint8_t **data, size_t *nbytes) {
    if (!g || i >= g->kv.size() || !type || !data || !nbytes)
        return fail(FH_ERR_INVALID, "gguf: no metadata entry %zu", i);
    const Kv &kv = g->kv[i];
    *type = kv.type;
    *data = g->bytes + kv.payload.off;
    *nbytes = (size_t)kv.payload.len;
    return FH_OK;
}

fh_status fh_gguf_kv_array(const fh_gguf *g, size_t i, uint32_t *elem_type, uint64_t *count) {
    if (!g || i >= g->kv.size() || !elem_type || !count) return fail(FH_ERR_INVALID, "gguf: no metadata entry %zu", i);
    if (g->kv[i].type != T_ARR) return fail(FH_ERR_INVALID, "gguf: metadata entry %zu is not an array", i);
    *elem_type = g->kv[i].elem_type;
    *count = g->kv[i].count;
    return FH_OK;
}

fh_status fh_gguf_kv_array_string(const fh_gguf *g, size_t i, uint64_t j, const char **s, size_t *len) {
    if (!g || i >= g->kv.size() || !s || !len) return fail(FH_ERR_INVALID, "gguf: no metadata entry %zu", i);
    const Kv &kv = g->kv[i];
    if (kv.type != T_ARR || kv.elem_type != T_STR)
        return fail(FH_ERR_INVALID, "gguf: metadata entry %zu is not a string array", i);
    if (j >= kv.strings.size()) return fail(FH_ERR_INVALID, "gguf: element %llu is out of range", (unsigned long long)j);
    *s = (const char *)g->bytes + kv.strings[j].off;
    *len = (size_t)kv.strings[j].len;
    return FH_OK;
}

fh_status fh_gguf_find_key(const fh_gguf *g, const char *key, size_t *index) {
    const Kv *kv = find_kv(g, key);
    if (!kv || !index) return fail(FH_ERR_INVALID, "gguf: missing key '%s'", key ? key : "");
    *index = (size_t)(kv - g->kv.data());
    return FH_OK;
}

// Gguf::uint (reader.rs:254-268): any integer width, non-negative.
fh_status fh_gguf_get_uint(const fh_gguf *g, const char *key, uint64_t *out) {
    const Kv *kv = find_kv(g, key);
    if (!kv) return fail(FH_ERR_INVALID, "gguf: missing key '%s'", key ? key : "");
    if (!out) return fail(FH_ERR_INVALID, "gguf: no output");
    const uint8_t *p = g->bytes + kv->payload.off;
    switch (kv->type) {
    case T_U8: *out = p[0]; return FH_OK;
    case T_U16: { uint16_t v; std::memcpy(&v, p, 2); *out = v; return FH_OK; }
    case T_U32: { uint32_t v; std::memcpy(&v, p, 4); *out = v; return FH_OK; }
    case T_U64: { uint64_t v; std::memcpy(&v, p, 8); *out = v; return FH_OK; }
    case T_I32: { int32_t v; std::memcpy(&v, p, 4); if (v >= 0) { *out = (uint64_t)v; return FH_OK; } break; }
    case T_I64: { int64_t v; std::memcpy(&v, p, 8); if (v >= 0) { *out = (uint64_t)v; return FH_OK; } break; }
    default: break;
    }
    return fail(FH_ERR_INVALID, "gguf: '%s' is not a non-negative integer", key);
}

fh_status fh_gguf_get_float(const fh_gguf *g, const char *key, float *out) {
    const Kv *kv = find_kv(g, key);
    if (!kv) return fail(FH_ERR_INVALID, "gguf: missing key '%s'", key ? key : "");
    if (kv->type != T_F32) return fail(FH_ERR_INVALID, "gguf: '%s' is not an f32", key);
    if (!out) return fail(FH_ERR_INVALID, "gguf: no output");
    std::memcpy(out, g->bytes + kv->payload.off, 4);
    return FH_OK;
}

fh_status fh_gguf_get_string(const fh_gguf *g, const char *key, const char **s, size_t *len) {
    const Kv *kv = find_kv(g, key);
    if (!kv) return fail(FH_ERR_INVALID, "gguf: missing key '%s'", key ? key : "");
    if (kv->type != T_STR) return fail(FH_ERR_INVALID, "gguf: '%s' is not a string", key);
    if (!s || !len) return fail(FH_ERR_INVALID, "gguf: no output");
    *s = (const char *)g->bytes + kv->payload.off;
    *len = (size_t)kv->payload.len;
    return FH_OK;
}

size_t fh_gguf_tensor_count(const fh_gguf *g) { return g ? g->tensors.size() : 0; }

fh_status fh_gguf_tensor_info(const fh_gguf *g, size_t i, fh_gguf_tensor *out) {
    if (!g || i >= g->tensors.size() || !out) return fail(FH_ERR_INVALID, "gguf: no tensor %zu", i);
    const Tensor &t = g->tensors[i];
    out->name = (const char *)g->bytes + t.name.off;
    out->name_len = (size_t)t.name.len;
    out->n_dims = t.nd;
    for (int d = 0; d < 4; d++) out->dims[d] = t.dims[d];
    out->ggml_type = t.type;
    out->offset = t.offset;
    out->elements = t.elements;
    out->nbytes = t.nbytes;
    return FH_OK;
}

fh_status fh_gguf_find_tensor(const fh_gguf *g, const char *name, size_t *index) {
    const Tensor *t;
    fh_status st = lookup(g, name, &t);
    if (st) return st;
    if (!index) return fail(FH_ERR_INVALID, "gguf: no output");
    *index = (size_t)(t - g->tensors.data());
    return FH_OK;
}

fh_status fh_gguf_tensor_bytes(const fh_gguf *g, const char *name, const uint8_t **data, size_t *len) {
    const Tensor *t;
    fh_status st = lookup(g, name, &t);
    if (st) return st;
    if (!data || !len) return fail(FH_ERR_INVALID, "gguf: no output");
    return span_of(g, name, t, data, len);
}

uint64_t fh_gguf_data_offset(const fh_gguf *g) { return g ? g->data_start : 0; }

fh_status fh_gguf_upload_qweight(fh_device *dev, const fh_gguf *g, const char *name, fh_qweight **out) {
    const Tensor *t;
    fh_status st = lookup(g, name, &t);
    if (st) return st;
    if (!out) return fail(FH_ERR_INVALID, "gguf: no output");
    if (t->type != FH_GGML_Q8_0 && t->type != FH_GGML_Q4_0 && !ext_kind((int)t->type))
        return fail(FH_ERR_UNSUPPORTED,
                    "gguf: tensor '%s' has ggml type %u, not a weight format (Q8_0, Q4_0, F16, MXFP4, Q2_K)", name,
                    t->type);
    uint64_t n = 1;
    for (uint32_t d = 1; d < t->nd; d++) n *= t->dims[d];  // no overflow: the parse bounded the product
    const uint8_t *data;
    size_t len;
    if ((st = span_of(g, name, t, &data, &len))) return st;
    return fh_qweight_upload_gguf(dev, (fh_kind)t->type, data, len, (size_t)t->dims[0], (size_t)n, out);
}

fh_status fh_gguf_upload_f32(fh_device *dev, const fh_gguf *g, const char *name, fh_buffer **out) {
    const Tensor *t;
    fh_status st = lookup(g, name, &t);
    if (st) return st;
    if (!out) return fail(FH_ERR_INVALID, "gguf: no output");
    *out = nullptr;
    const uint8_t *data;
    size_t len;
    if ((st = span_of(g, name, t, &data, &len))) return st;
    const size_t n = (size_t)t->elements;
    switch (t->type) {
    case FH_GGML_F32: return fh_buffer_upload(dev, (const float *)data, n, out);
    case FH_GGML_F16:
    case FH_GGML_Q8_0:
    case FH_GGML_Q4_0: break;
    case FH_GGML_Q4_1:
    case FH_GGML_Q5_0:
    case FH_GGML_Q5_1:
    case FH_GGML_Q8_1:
    case FH_GGML_Q2_K:
    case FH_GGML_Q3_K:
    case FH_GGML_Q4_K:
    case FH_GGML_Q5_K:
    case FH_GGML_Q6_K:
    case FH_GGML_MXFP4: break;  // fh_decode's block decoders (formats.hip)
    case FH_GGML_I16:
    case FH_GGML_I32:
        return fail(FH_ERR_INVALID, "gguf: integer tensors have no f32 form; read them with tensor_bytes");
    default:
        return fail(FH_ERR_UNSUPPORTED, "gguf: tensor '%s' of ggml type %u has no device decode", name, t->type);
    }
    fh_buffer *stage = nullptr, *dst = nullptr;
    if ((st = fh_bytes_upload(dev, data, len, &stage))) return st;
    if ((st = fh_buffer_zeros(dev, n, &dst)) == FH_OK) {
        if (t->type == FH_GGML_F16) {
            if ((st = begin_command(dev, "tensor_f32")) == FH_OK) {
                if (n) (void)launch_decode_f16(dev->stream, (const uint16_t *)stage->ptr, (float *)dst->ptr, n);
                st = end_command(dev, "tensor_f32");
            }
        } else {
            st = fh_decode(dev, (fh_kind)t->type, stage, n, dst);
        }
    }
    if (st == FH_OK) st = fh_device_sync(dev);  // the staging buffer is freed next
    fh_buffer_free(stage);
    if (st) {
        fh_buffer_free(dst);
        return st;
    }
    *out = dst;
    return FH_OK;
}

}  // extern "C"

// ---- model-loading helpers shared by the GPT-2 and Llama loaders ----
namespace fh {

std::string tensor_name(const char *base, size_t layer, const char *suffix) {
    return std::string(base) + std::to_string(layer) + "." + suffix;
}

fh_status cfg_uint(const fh_gguf *g, const char *key, size_t *out) {
    uint64_t v;
    fh_status st = fh_gguf_get_uint(g, key, &v);
    if (st) return st;
    *out = (size_t)v;
    return FH_OK;
}

fh_status host_vec(const fh_gguf *g, const char *who, const std::string &name, size_t len, std::vector<float> *out) {
    const Tensor *t;
    fh_status st = lookup(g, name.c_str(), &t);
    if (st) return st;
    if (t->elements != len || t->type != FH_GGML_F32)
        return fail(FH_ERR_INVALID, "%s: tensor '%s' must be %zu F32 values (has %llu of ggml type %u)", who,
                    name.c_str(), len, (unsigned long long)t->elements, t->type);
    const uint8_t *data;
    size_t n;
    if ((st = span_of(g, name.c_str(), t, &data, &n))) return st;
    try {
        out->resize(len);
    } catch (const std::bad_alloc &) {
        return fail(FH_ERR_OOM, "host out of memory");
    }
    if (len) memcpy(out->data(), data, len * 4);  // the file's alignment may leave it unaligned
    return FH_OK;
}

fh_status load_vec(fh_device *dev, const fh_gguf *g, const char *who, const std::string &name, size_t len,
                   fh_buffer **out) {
    std::vector<float> v;
    fh_status st = host_vec(g, who, name, len, &v);
    if (st) return st;
    return fh_buffer_upload(dev, v.data(), len, out);
}

// The stored rows of a Q8_0/Q4_0 matrix of k inputs and n outputs (GGML dims [k, n]), checked
// against the model's one block format.
static fh_status mat_rows(const fh_gguf *g, const char *who, const std::string &name, size_t k, size_t n,
                          fh_kind *kind, const uint8_t **data, size_t *len) {
    const Tensor *t;
    fh_status st = lookup(g, name.c_str(), &t);
    if (st) return st;
    if (t->nd != 2 || t->dims[0] != k || t->dims[1] != n)
        return fail(FH_ERR_INVALID, "%s: tensor '%s' must have dims [%zu, %zu]", who, name.c_str(), k, n);
    if (t->type != FH_GGML_Q8_0 && t->type != FH_GGML_Q4_0)
        return fail(FH_ERR_UNSUPPORTED, "%s: tensor '%s' has ggml type %u; the model's matrices must be Q8_0 or Q4_0",
                    who, name.c_str(), t->type);
    if (*kind == (fh_kind)0) *kind = (fh_kind)t->type;
    if ((fh_kind)t->type != *kind)
        return fail(FH_ERR_UNSUPPORTED, "%s: tensor '%s' mixes block formats (the model's matrices must share one)",
                    who, name.c_str());
    return span_of(g, name.c_str(), t, data, len);
}

fh_status load_mat(fh_device *dev, const fh_gguf *g, const char *who, const std::string &name, size_t k, size_t n,
                   fh_kind *kind, fh_qweight **out) {
    const uint8_t *data;
    size_t len;
    fh_status st = mat_rows(g, who, name, k, n, kind, &data, &len);
    if (st) return st;
    return fh_qweight_upload_gguf(dev, *kind, data, len, k, n, out);
}

fh_status load_mat_rows(fh_device *dev, const fh_gguf *g, const char *who, const std::string *names,
                        const size_t *ns, size_t count, size_t k, fh_kind *kind, fh_qweight **out, bool interleave) {
    if (interleave && (count != 2 || ns[0] != ns[1] || ns[0] % 32))
        return fail(FH_ERR_INVALID, "%s: interleaving needs two parts of equal rows, a multiple of 32", who);
    std::vector<std::pair<const uint8_t *, size_t>> parts(count);
    size_t total = 0, rows = 0;
    for (size_t i = 0; i < count; i++) {
        fh_status st = mat_rows(g, who, names[i], k, ns[i], kind, &parts[i].first, &parts[i].second);
        if (st) return st;
        total += parts[i].second;
        rows += ns[i];
    }
    std::vector<uint8_t> joined;
    try {
        joined.resize(total);
    } catch (const std::bad_alloc &) {
        return fail(FH_ERR_OOM, "host out of memory");
    }
    size_t at = 0;
    if (interleave) {  // 32 rows of part 0, 32 of part 1, ... (rows are whole blocks of k)
        const size_t run = parts[0].second / (ns[0] / 32);
        for (size_t c = 0; c < ns[0] / 32; c++)
            for (auto &p : parts) {
                memcpy(joined.data() + at, p.first + c * run, run);
                at += run;
            }
    } else {
        for (auto &p : parts) {
            memcpy(joined.data() + at, p.first, p.second);
            at += p.second;
        }
    }
    return fh_qweight_upload_gguf(dev, *kind, joined.data(), total, k, rows, out);
}

}  // namespace fh
