// q8_gguf.cpp -- the read-only GGUF reader of include/q8gguf.h.
//
// Follows the reference's GgufFile (apps/engine/src/gguf.rs): the file is
// mapped read-only (memmap2 there, mmap(2) here), the header, metadata and
// tensor table are parsed with a bounds-checked cursor, metadata arrays are
// recorded as (element type, length, file offset) and decoded only when asked
// for, and every tensor is checked to lie inside the file.  Tensor data is
// handed out as pointers into the map, so the device residency cache keys a
// weight by its place in the file exactly as the reference's
// Weight::identity() does (apps/engine/src/tensor.rs:40-42).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/q8gguf.h"
#include "q8_internal.h"

namespace {

using q8i::set_error;

constexpr uint32_t kMagic = 0x46554747u;   // "GGUF" little-endian (gguf.rs:15)
constexpr uint64_t kDefaultAlignment = 32;  // gguf.rs:16
// Arrays of arrays recurse (gguf.rs:444-468); bound the depth so a hostile
// file cannot exhaust the stack.
constexpr int kMaxArrayDepth = 64;

int format_error(const char *msg) { return set_error(Q8_ERR_FORMAT, "malformed gguf: %s", msg); }

// Rust's str::from_utf8 acceptance: shortest forms only, no surrogates,
// nothing above U+10FFFF.
bool valid_utf8(const uint8_t *p, uint64_t n) {
    uint64_t i = 0;
    while (i < n) {
        const uint8_t c = p[i];
        if (c < 0x80) {
            i++;
            continue;
        }
        int extra;
        uint8_t lo = 0x80, hi = 0xbf;
        if (c >= 0xc2 && c <= 0xdf) {
            extra = 1;
        } else if (c >= 0xe0 && c <= 0xef) {
            extra = 2;
            if (c == 0xe0) lo = 0xa0;
            if (c == 0xed) hi = 0x9f;
        } else if (c >= 0xf0 && c <= 0xf4) {
            extra = 3;
            if (c == 0xf0) lo = 0x90;
            if (c == 0xf4) hi = 0x8f;
        } else {
            return false;
        }
        if (n - i <= (uint64_t)extra) return false;
        if (p[i + 1] < lo || p[i + 1] > hi) return false;
        for (int j = 2; j <= extra; j++)
            if ((p[i + j] & 0xc0) != 0x80) return false;
        i += extra + 1;
    }
    return true;
}

// The reference's Reader (gguf.rs:313-402): little-endian fields from a
// cursor that never leaves the map.
struct Reader {
    const uint8_t *data;
    uint64_t size;
    uint64_t pos;

    int take(uint64_t len, const uint8_t **out) {
        if (len > size - pos) return format_error("unexpected end of file");
        *out = data + pos;
        pos += len;
        return Q8_OK;
    }
    template <typename T>
    int get(T *v) {
        const uint8_t *p = nullptr;
        if (int rc = take(sizeof(T), &p)) return rc;
        std::memcpy(v, p, sizeof(T));  // x86-64 and the file are both little-endian
        return Q8_OK;
    }
    // gguf.rs:382-388: u64 length, then UTF-8 bytes.
    int str(const uint8_t **p, uint64_t *len) {
        if (int rc = get(len)) return rc;
        if (int rc = take(*len, p)) return rc;
        if (!valid_utf8(*p, *len)) return format_error("invalid utf-8 in string");
        return Q8_OK;
    }
    int str(std::string *s) {
        const uint8_t *p = nullptr;
        uint64_t len;
        if (int rc = str(&p, &len)) return rc;
        s->assign(reinterpret_cast<const char *>(p), len);
        return Q8_OK;
    }
};

enum class Kind { UInt, Int, Float, Bool, Text, Array };

// MetaValue (gguf.rs:73-86).
struct Meta {
    Kind kind = Kind::UInt;
    uint32_t type = 0;  // the file's value type id
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0;
    bool b = false;
    std::string text;
    uint32_t elem_type = 0;
    uint64_t len = 0;
    uint64_t data_offset = 0;  // absolute offset of an array's first element
};

// skip_array (gguf.rs:444-468).
int skip_array(Reader &r, uint32_t elem_type, uint64_t len, int depth) {
    if (depth > kMaxArrayDepth) return format_error("arrays nested too deeply");
    uint64_t size = 0;
    switch (elem_type) {
        case 0: case 1: case 7: size = 1; break;
        case 2: case 3: size = 2; break;
        case 4: case 5: case 6: size = 4; break;
        case 10: case 11: case 12: size = 8; break;
        case 8: case 9: size = 0; break;
        default: return set_error(Q8_ERR_FORMAT, "malformed gguf: unknown array element type %u", elem_type);
    }
    if (size) {
        if (len > (r.size - r.pos) / size) return format_error("unexpected end of file");
        r.pos += size * len;
        return Q8_OK;
    }
    for (uint64_t i = 0; i < len; i++) {
        if (elem_type == 8) {
            const uint8_t *p = nullptr;
            uint64_t n;
            if (int rc = r.str(&p, &n)) return rc;
        } else {
            uint32_t nested_type;
            uint64_t nested_len;
            if (int rc = r.get(&nested_type)) return rc;
            if (int rc = r.get(&nested_len)) return rc;
            if (int rc = skip_array(r, nested_type, nested_len, depth + 1)) return rc;
        }
    }
    return Q8_OK;
}

// read_typed_value (gguf.rs:404-442).
int read_value(Reader &r, uint32_t type, Meta *m) {
    m->type = type;
    switch (type) {
        case 0: { uint8_t v; if (int rc = r.get(&v)) return rc; m->kind = Kind::UInt; m->u = v; return Q8_OK; }
        case 1: { int8_t v; if (int rc = r.get(&v)) return rc; m->kind = Kind::Int; m->i = v; return Q8_OK; }
        case 2: { uint16_t v; if (int rc = r.get(&v)) return rc; m->kind = Kind::UInt; m->u = v; return Q8_OK; }
        case 3: { int16_t v; if (int rc = r.get(&v)) return rc; m->kind = Kind::Int; m->i = v; return Q8_OK; }
        case 4: { uint32_t v; if (int rc = r.get(&v)) return rc; m->kind = Kind::UInt; m->u = v; return Q8_OK; }
        case 5: { int32_t v; if (int rc = r.get(&v)) return rc; m->kind = Kind::Int; m->i = v; return Q8_OK; }
        case 6: { float v; if (int rc = r.get(&v)) return rc; m->kind = Kind::Float; m->f = v; return Q8_OK; }
        case 7: { uint8_t v; if (int rc = r.get(&v)) return rc; m->kind = Kind::Bool; m->b = v != 0; return Q8_OK; }
        case 8: m->kind = Kind::Text; return r.str(&m->text);
        case 9: {
            m->kind = Kind::Array;
            if (int rc = r.get(&m->elem_type)) return rc;
            if (int rc = r.get(&m->len)) return rc;
            m->data_offset = r.pos;
            return skip_array(r, m->elem_type, m->len, 1);
        }
        case 10: { uint64_t v; if (int rc = r.get(&v)) return rc; m->kind = Kind::UInt; m->u = v; return Q8_OK; }
        case 11: { int64_t v; if (int rc = r.get(&v)) return rc; m->kind = Kind::Int; m->i = v; return Q8_OK; }
        case 12: { double v; if (int rc = r.get(&v)) return rc; m->kind = Kind::Float; m->f = v; return Q8_OK; }
        default: return set_error(Q8_ERR_FORMAT, "malformed gguf: unknown metadata value type %u", type);
    }
}

// DType (gguf.rs:19-56): elements and bytes per block.
bool dtype_block(uint32_t id, uint64_t *elems, uint64_t *bytes) {
    switch (id) {
        case Q8_GGUF_F32: *elems = 1; *bytes = 4; return true;
        case Q8_GGUF_F16: *elems = 1; *bytes = 2; return true;
        case Q8_GGUF_Q8_0: *elems = 32; *bytes = 34; return true;
        default: return false;
    }
}

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t dtype;
    uint64_t offset, byte_len, elements;
};

}  // namespace

struct q8_gguf {
    const uint8_t *map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = kDefaultAlignment;
    uint64_t data_start = 0;
    std::unordered_map<std::string, Meta> meta;
    std::vector<std::string> keys;  // first-definition order
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> first;  // name -> first tensor of that name

    ~q8_gguf() {
        if (map) munmap(const_cast<uint8_t *>(map), size);
    }
};

namespace {

int parse(q8_gguf *g) {
    Reader r{g->map, g->size, 0};
    uint32_t magic, version;
    if (int rc = r.get(&magic)) return rc;
    if (magic != kMagic) return set_error(Q8_ERR_FORMAT, "malformed gguf: bad magic %#010x", magic);
    if (int rc = r.get(&version)) return rc;
    if (version < 2 || version > 3) return set_error(Q8_ERR_FORMAT, "malformed gguf: unsupported version %u", version);
    g->version = version;
    uint64_t tensor_count, kv_count;
    if (int rc = r.get(&tensor_count)) return rc;
    if (int rc = r.get(&kv_count)) return rc;

    for (uint64_t i = 0; i < kv_count; i++) {
        std::string key;
        if (int rc = r.str(&key)) return rc;
        uint32_t type;
        if (int rc = r.get(&type)) return rc;
        Meta m;
        if (int rc = read_value(r, type, &m)) return rc;
        auto it = g->meta.find(key);
        if (it == g->meta.end()) {
            g->keys.push_back(key);
            g->meta.emplace(std::move(key), std::move(m));
        } else {
            it->second = std::move(m);  // HashMap::insert: the last value wins
        }
    }

    for (uint64_t i = 0; i < tensor_count; i++) {
        Tensor t;
        if (int rc = r.str(&t.name)) return rc;
        uint32_t n_dims;
        if (int rc = r.get(&n_dims)) return rc;
        uint64_t elements = 1;
        bool overflow = false;
        for (uint32_t d = 0; d < n_dims; d++) {
            uint64_t dim;
            if (int rc = r.get(&dim)) return rc;
            t.dims.push_back(dim);
            if (dim && elements > UINT64_MAX / dim) overflow = true;
            elements *= dim;
        }
        if (int rc = r.get(&t.dtype)) return rc;
        uint64_t be, bb;
        if (!dtype_block(t.dtype, &be, &bb)) return set_error(Q8_ERR_UNSUPPORTED, "unsupported: tensor type id %u", t.dtype);
        if (int rc = r.get(&t.offset)) return rc;
        if (overflow)
            return set_error(Q8_ERR_FORMAT, "malformed gguf: tensor %s: element count overflows", t.name.c_str());
        if (elements % be)
            return set_error(Q8_ERR_FORMAT,
                             "malformed gguf: tensor %s: %llu elements is not a multiple of the %llu block size",
                             t.name.c_str(), (unsigned long long)elements, (unsigned long long)be);
        if (elements / be > UINT64_MAX / bb)
            return set_error(Q8_ERR_FORMAT, "malformed gguf: tensor %s: byte length overflows", t.name.c_str());
        t.elements = elements;
        t.byte_len = elements / be * bb;
        g->first.emplace(t.name, g->tensors.size());  // keeps the first of a repeated name
        g->tensors.push_back(std::move(t));
    }

    auto al = g->meta.find("general.alignment");
    g->alignment = (al != g->meta.end() && al->second.kind == Kind::UInt) ? al->second.u : kDefaultAlignment;
    if (g->alignment == 0) return set_error(Q8_ERR_FORMAT, "malformed gguf: general.alignment is 0");
    const uint64_t pos = r.pos;
    const uint64_t rounded = pos / g->alignment + (pos % g->alignment != 0);
    if (rounded > UINT64_MAX / g->alignment || rounded * g->alignment > g->size)
        return set_error(Q8_ERR_FORMAT, "malformed gguf: tensor data starts past end of file");
    g->data_start = rounded * g->alignment;
    for (const Tensor &t : g->tensors) {
        const uint64_t room = g->size - g->data_start;
        if (t.offset > room || t.byte_len > room - t.offset)
            return set_error(Q8_ERR_FORMAT, "malformed gguf: tensor %s runs past end of file", t.name.c_str());
    }
    return Q8_OK;
}

void fill(const q8_gguf *g, const Tensor &t, q8_gguf_tensor_info *out) {
    out->name = t.name.c_str();
    out->name_len = t.name.size();
    out->n_dims = (uint32_t)t.dims.size();
    out->dims = t.dims.data();
    out->dtype = t.dtype;
    out->offset = t.offset;
    out->byte_len = t.byte_len;
    out->elements = t.elements;
    out->data = g->map ? g->map + g->data_start + t.offset : nullptr;
}

int find_meta(const q8_gguf *g, const char *key, const Meta **m) {
    if (!g || !key) return set_error(Q8_ERR_INVALID, "gguf: null argument");
    auto it = g->meta.find(key);
    if (it == g->meta.end()) return set_error(Q8_ERR_MISSING, "missing metadata key: %s", key);
    *m = &it->second;
    return Q8_OK;
}

// The array behind `key` when its element type is one of `accepted`
// (gguf.rs:250-311 match arms).
int find_array(const q8_gguf *g, const char *key, std::initializer_list<uint32_t> accepted, const char *what,
               const Meta **m) {
    if (int rc = find_meta(g, key, m)) return rc;
    if ((*m)->kind != Kind::Array) return set_error(Q8_ERR_FORMAT, "malformed gguf: %s is not an array", key);
    for (uint32_t a : accepted)
        if ((*m)->elem_type == a) return Q8_OK;
    return set_error(Q8_ERR_FORMAT, "malformed gguf: %s is not %s", key, what);
}

}  // namespace

extern "C" {

int q8_gguf_open(const char *path, q8_gguf **out) {
    if (!path || !out) return set_error(Q8_ERR_INVALID, "q8_gguf_open: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return set_error(Q8_ERR_IO, "io error: %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        const int err = errno;
        close(fd);
        return set_error(Q8_ERR_IO, "io error: %s: %s", path, strerror(err));
    }
    q8_gguf *g = new q8_gguf;
    g->size = (uint64_t)st.st_size;
    if (g->size) {
        void *p = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) {
            const int err = errno;
            close(fd);
            delete g;
            return set_error(Q8_ERR_IO, "io error: mmap %s: %s", path, strerror(err));
        }
        g->map = static_cast<const uint8_t *>(p);
    }
    close(fd);  // the mapping stays valid without the descriptor
    const int rc = parse(g);
    if (rc != Q8_OK) {
        delete g;
        return rc;
    }
    *out = g;
    return Q8_OK;
}

void q8_gguf_close(q8_gguf *g) { delete g; }

int q8_gguf_layout(const q8_gguf *g, uint32_t *version, uint64_t *alignment, uint64_t *data_start,
                   uint64_t *file_bytes) {
    if (!g) return set_error(Q8_ERR_INVALID, "gguf: null handle");
    if (version) *version = g->version;
    if (alignment) *alignment = g->alignment;
    if (data_start) *data_start = g->data_start;
    if (file_bytes) *file_bytes = g->size;
    return Q8_OK;
}

int q8_gguf_tensor_count(const q8_gguf *g, uint64_t *count) {
    if (!g || !count) return set_error(Q8_ERR_INVALID, "gguf: null argument");
    *count = g->tensors.size();
    return Q8_OK;
}

int q8_gguf_tensor_at(const q8_gguf *g, uint64_t index, q8_gguf_tensor_info *out) {
    if (!g || !out) return set_error(Q8_ERR_INVALID, "gguf: null argument");
    if (index >= g->tensors.size())
        return set_error(Q8_ERR_INVALID, "tensor index %llu of %zu", (unsigned long long)index, g->tensors.size());
    fill(g, g->tensors[index], out);
    return Q8_OK;
}

int q8_gguf_tensor(const q8_gguf *g, const char *name, q8_gguf_tensor_info *out) {
    if (!g || !name || !out) return set_error(Q8_ERR_INVALID, "gguf: null argument");
    auto it = g->first.find(name);
    if (it == g->first.end()) return set_error(Q8_ERR_MISSING, "missing tensor: %s", name);
    fill(g, g->tensors[it->second], out);
    return Q8_OK;
}

int q8_gguf_meta_count(const q8_gguf *g, uint64_t *count) {
    if (!g || !count) return set_error(Q8_ERR_INVALID, "gguf: null argument");
    *count = g->keys.size();
    return Q8_OK;
}

int q8_gguf_meta_key_at(const q8_gguf *g, uint64_t index, const char **key) {
    if (!g || !key) return set_error(Q8_ERR_INVALID, "gguf: null argument");
    if (index >= g->keys.size())
        return set_error(Q8_ERR_INVALID, "metadata index %llu of %zu", (unsigned long long)index, g->keys.size());
    *key = g->keys[index].c_str();
    return Q8_OK;
}

int q8_gguf_meta_type(const q8_gguf *g, const char *key, uint32_t *type, uint32_t *elem_type, uint64_t *len) {
    const Meta *m;
    if (int rc = find_meta(g, key, &m)) return rc;
    const bool array = m->kind == Kind::Array;
    if (type) *type = m->type;
    if (elem_type) *elem_type = array ? m->elem_type : 0;
    if (len) *len = array ? m->len : 0;
    return Q8_OK;
}

// gguf.rs:193-202
int q8_gguf_meta_u64(const q8_gguf *g, const char *key, uint64_t *out) {
    const Meta *m;
    if (int rc = find_meta(g, key, &m)) return rc;
    if (!out) return set_error(Q8_ERR_INVALID, "gguf: null argument");
    if (m->kind == Kind::UInt) {
        *out = m->u;
        return Q8_OK;
    }
    if (m->kind == Kind::Int && m->i >= 0) {
        *out = (uint64_t)m->i;
        return Q8_OK;
    }
    return set_error(Q8_ERR_FORMAT, "malformed gguf: %s is not an unsigned integer", key);
}

// gguf.rs:204-210: f32 and f64 values, the latter rounded to f32.
int q8_gguf_meta_f32(const q8_gguf *g, const char *key, float *out) {
    const Meta *m;
    if (int rc = find_meta(g, key, &m)) return rc;
    if (!out) return set_error(Q8_ERR_INVALID, "gguf: null argument");
    if (m->kind != Kind::Float) return set_error(Q8_ERR_FORMAT, "malformed gguf: %s is not a float", key);
    *out = (float)m->f;
    return Q8_OK;
}

// gguf.rs:212-218
int q8_gguf_meta_bool(const q8_gguf *g, const char *key, int *out) {
    const Meta *m;
    if (int rc = find_meta(g, key, &m)) return rc;
    if (!out) return set_error(Q8_ERR_INVALID, "gguf: null argument");
    if (m->kind != Kind::Bool) return set_error(Q8_ERR_FORMAT, "malformed gguf: %s is not a bool", key);
    *out = m->b ? 1 : 0;
    return Q8_OK;
}

// gguf.rs:242-248
int q8_gguf_meta_str(const q8_gguf *g, const char *key, const char **str, uint64_t *len) {
    const Meta *m;
    if (int rc = find_meta(g, key, &m)) return rc;
    if (!str) return set_error(Q8_ERR_INVALID, "gguf: null argument");
    if (m->kind != Kind::Text) return set_error(Q8_ERR_FORMAT, "malformed gguf: %s is not a string", key);
    *str = m->text.c_str();
    if (len) *len = m->text.size();
    return Q8_OK;
}

// gguf.rs:238-240
int q8_gguf_has_key_prefix(const q8_gguf *g, const char *prefix) {
    if (!g || !prefix) return 0;
    const size_t n = strlen(prefix);
    for (const std::string &k : g->keys)
        if (k.size() >= n && k.compare(0, n, prefix) == 0) return 1;
    return 0;
}

// gguf.rs:250-278: I32 (5) or U32 (4) elements, read as 32 bits.
int q8_gguf_meta_i32_array(const q8_gguf *g, const char *key, int32_t *out, uint64_t cap, uint64_t *len) {
    const Meta *m;
    if (int rc = find_array(g, key, {4, 5}, "an integer array", &m)) return rc;
    if (len) *len = m->len;
    const uint64_t n = m->len < cap ? m->len : cap;
    if (n && !out) return set_error(Q8_ERR_INVALID, "gguf: null output");
    if (n) std::memcpy(out, g->map + m->data_offset, n * 4);
    return Q8_OK;
}

// gguf.rs:281-296: F32 elements.
int q8_gguf_meta_f32_array(const q8_gguf *g, const char *key, float *out, uint64_t cap, uint64_t *len) {
    const Meta *m;
    if (int rc = find_array(g, key, {6}, "a float array", &m)) return rc;
    if (len) *len = m->len;
    const uint64_t n = m->len < cap ? m->len : cap;
    if (n && !out) return set_error(Q8_ERR_INVALID, "gguf: null output");
    if (n) std::memcpy(out, g->map + m->data_offset, n * 4);
    return Q8_OK;
}

// gguf.rs:299-311: STRING elements, as pointers into the map.
int q8_gguf_meta_str_array(const q8_gguf *g, const char *key, const char **ptrs, uint64_t *lens, uint64_t cap,
                           uint64_t *len) {
    const Meta *m;
    if (int rc = find_array(g, key, {8}, "a string array", &m)) return rc;
    if (len) *len = m->len;
    const uint64_t n = m->len < cap ? m->len : cap;
    if (n && (!ptrs || !lens)) return set_error(Q8_ERR_INVALID, "gguf: null output");
    Reader r{g->map, g->size, m->data_offset};
    for (uint64_t i = 0; i < n; i++) {
        const uint8_t *p = nullptr;
        uint64_t l;
        if (int rc = r.str(&p, &l)) return rc;  // validated at open; kept checked
        ptrs[i] = reinterpret_cast<const char *>(p);
        lens[i] = l;
    }
    return Q8_OK;
}

// model.rs:1670-1684 (shape check) + Gpu::quantized (cuda/mod.rs:1769-1790).
int q8_gguf_weight(q8_ctx *c, const q8_gguf *g, const char *name, int k, int out, const q8_weight **weight) {
    if (!c || !g || !name || !weight) return set_error(Q8_ERR_INVALID, "q8_gguf_weight: null argument");
    q8_gguf_tensor_info t;
    if (int rc = q8_gguf_tensor(g, name, &t)) return rc;
    if (k < 0 || out < 0 || t.n_dims != 2 || t.dims[0] != (uint64_t)k || t.dims[1] != (uint64_t)out) {
        std::string shape = "[";
        for (uint32_t d = 0; d < t.n_dims; d++) shape += (d ? ", " : "") + std::to_string(t.dims[d]);
        shape += "]";
        return set_error(Q8_ERR_FORMAT, "malformed gguf: %s has shape %s, expected [%d, %d]", name, shape.c_str(), k,
                         out);
    }
    if (t.dtype != Q8_GGUF_Q8_0)
        return set_error(Q8_ERR_UNSUPPORTED, "unsupported: %s is tensor type %u, the device path takes Q8_0", name,
                         t.dtype);
    return q8_weight_resident(c, t.data, t.byte_len, k, out, weight);
}

}  // extern "C"
