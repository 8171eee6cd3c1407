// gguf.cpp — GGUF v2/v3 reader for the C ABI (rt_gguf_*).
//
// Restates the reference's crates/gguf parser (parser.rs:22-57 parse order,
// types.rs:142-198 block tables, error.rs variants) and the engine's loader
// (crates/engine/src/loader.rs:124-218: parse, then mmap the whole file and
// address each tensor at data_offset + tensor offset).  The file is mapped
// read-only; tensor bytes are handed out as host pointers into the mapping or
// copied to device memory with rt_gguf_upload.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/runit_hip.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" (types.rs:4)
constexpr uint64_t kDefaultAlignment = 32;  // types.rs:9

// GgufDtype → (elements per block, bytes per block) (types.rs:142-198);
// {0, 0} for ids the reference does not know.
struct BlockInfo { uint32_t el, bytes; };
BlockInfo block_info(uint32_t t) {
    switch (t) {
        case 0: return {1, 4};      // F32
        case 1: return {1, 2};      // F16
        case 2: return {32, 18};    // Q4_0
        case 3: return {32, 20};    // Q4_1
        case 6: return {32, 22};    // Q5_0
        case 7: return {32, 24};    // Q5_1
        case 8: return {32, 34};    // Q8_0
        case 9: return {32, 40};    // Q8_1
        case 10: return {256, 84};  // Q2_K
        case 11: return {256, 110}; // Q3_K
        case 12: return {256, 144}; // Q4_K
        case 13: return {256, 176}; // Q5_K
        case 14: return {256, 210}; // Q6_K
        case 15: return {256, 292}; // Q8_K
        case 16: return {256, 66};  // IQ2_XXS
        case 17: return {256, 74};  // IQ2_XS
        case 18: return {256, 98};  // IQ3_XXS
        case 19: return {256, 50};  // IQ1_S
        case 20: return {32, 18};   // IQ4_NL
        case 21: return {256, 110}; // IQ3_S
        case 22: return {256, 82};  // IQ2_S
        case 23: return {32, 36};   // IQ4_XS (as the reference's table has it)
        case 24: return {1, 1};     // I8
        case 25: return {1, 2};     // I16
        case 26: return {1, 4};     // I32
        case 27: return {1, 8};     // I64
        case 28: return {1, 8};     // F64
        case 29: return {256, 56};  // IQ1_M
        case 30: return {1, 2};     // BF16
        default: return {0, 0};
    }
}

// Metadata value types (GgufMetadataValueType): 0 u8, 1 i8, 2 u16, 3 i16,
// 4 u32, 5 i32, 6 f32, 7 bool, 8 string, 9 array, 10 u64, 11 i64, 12 f64.
uint32_t scalar_size(uint32_t t) {
    switch (t) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        default: return 0;
    }
}

struct Meta {
    std::string key;
    uint32_t type = 0;
    uint64_t u = 0;  // integer / bool value (as u64 bit pattern)
    double f = 0.0;  // float value
    std::string s;   // string value
    uint32_t elem_type = 0;  // arrays
    uint64_t count = 0;
    uint64_t arr_off = 0;    // file offset of the first element
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t dtype = 0;
    uint64_t offset = 0;  // relative to the data region
    uint64_t bytes = 0;
};

thread_local char g_err[512];

}  // namespace

struct rt_gguf {
    int fd = -1;
    const uint8_t* map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = kDefaultAlignment;
    uint64_t data_offset = 0;
    std::vector<Meta> meta;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int64_t> meta_idx, tensor_idx;
};

namespace {

int gfail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    return code;
}

// Bounds-checked little-endian reader over the mapping.
struct Reader {
    const uint8_t* p;
    uint64_t size, pos = 0;
    int err = RT_OK;
    bool need(uint64_t n) {
        if (err != RT_OK) return false;
        if (pos + n > size || pos + n < pos) {
            err = gfail(RT_ERR_GGUF_EOF,
                        "unexpected end of file at offset %llu (need %llu bytes, have %llu)",
                        (unsigned long long)pos, (unsigned long long)n,
                        (unsigned long long)(size - pos));
            return false;
        }
        return true;
    }
    template <typename T>
    T get() {
        T v{};
        if (!need(sizeof(T))) return v;
        memcpy(&v, p + pos, sizeof(T));
        pos += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!need(n)) return {};
        std::string s((const char*)p + pos, n);
        pos += n;
        return s;
    }
    void skip(uint64_t n) {
        if (need(n)) pos += n;
    }
};

// Minimal UTF-8 validity check (the reference rejects invalid strings,
// parser.rs read_string → GgufError::InvalidUtf8).
bool utf8_ok(const std::string& s) {
    const size_t n = s.size();
    size_t i = 0;
    while (i < n) {
        const unsigned char c = (unsigned char)s[i];
        const size_t len = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 0;
        if (len == 0 || i + len > n) return false;
        for (size_t k = 1; k < len; ++k)
            if ((((unsigned char)s[i + k]) & 0xC0) != 0x80) return false;
        i += len;
    }
    return true;
}

// Reads one value of type t (parser.rs read_typed_value); arrays are
// recorded by position and skipped.
void read_value(Reader& r, uint32_t t, Meta& m) {
    m.type = t;
    switch (t) {
        case 0: m.u = r.get<uint8_t>(); break;
        case 1: m.u = (uint64_t)(int64_t)r.get<int8_t>(); break;
        case 2: m.u = r.get<uint16_t>(); break;
        case 3: m.u = (uint64_t)(int64_t)r.get<int16_t>(); break;
        case 4: m.u = r.get<uint32_t>(); break;
        case 5: m.u = (uint64_t)(int64_t)r.get<int32_t>(); break;
        case 6: m.f = r.get<float>(); break;
        case 7: m.u = r.get<uint8_t>() != 0; break;
        case 8: {
            const uint64_t at = r.pos;
            m.s = r.str();
            if (r.err == RT_OK && !utf8_ok(m.s))
                r.err = gfail(RT_ERR_GGUF_UTF8, "invalid UTF-8 string in metadata at offset %llu",
                              (unsigned long long)at);
            break;
        }
        case 10: m.u = r.get<uint64_t>(); break;
        case 11: m.u = (uint64_t)r.get<int64_t>(); break;
        case 12: m.f = r.get<double>(); break;
        case 9: {
            m.elem_type = r.get<uint32_t>();
            m.count = r.get<uint64_t>();
            if (r.err != RT_OK) return;
            m.arr_off = r.pos;
            if (m.elem_type == 8) {
                for (uint64_t i = 0; i < m.count && r.err == RT_OK; ++i) r.str();
            } else if (m.elem_type == 9 || scalar_size(m.elem_type) == 0) {
                // nested arrays are legal GGUF; walk them element by element
                for (uint64_t i = 0; i < m.count && r.err == RT_OK; ++i) {
                    Meta sub;
                    if (m.elem_type != 9 && scalar_size(m.elem_type) == 0) {
                        r.err = gfail(RT_ERR_GGUF_METADATA_TYPE, "unknown metadata value type: %u",
                                      m.elem_type);
                        return;
                    }
                    read_value(r, m.elem_type, sub);
                }
            } else {
                r.skip(m.count * scalar_size(m.elem_type));
            }
            break;
        }
        default:
            r.err = gfail(RT_ERR_GGUF_METADATA_TYPE, "unknown metadata value type: %u", t);
    }
}

}  // namespace

extern "C" {

const char* rt_gguf_last_error(void) { return g_err; }

int rt_gguf_open(const char* path, rt_gguf** out) {
    if (!out || !path) return gfail(RT_ERR_GGUF_IO, "I/O error: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return gfail(RT_ERR_GGUF_IO, "I/O error: cannot open '%s'", path);
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return gfail(RT_ERR_GGUF_IO, "I/O error: cannot stat '%s'", path);
    }
    auto* g = new rt_gguf();
    g->fd = fd;
    g->size = (uint64_t)st.st_size;
    if (g->size > 0) {
        void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            rt_gguf_close(g);
            return gfail(RT_ERR_GGUF_IO, "I/O error: cannot map '%s'", path);
        }
        g->map = (const uint8_t*)m;
    }
    Reader r{g->map, g->size};
    // header (parser.rs read_header)
    const uint32_t magic = r.get<uint32_t>();
    if (r.err == RT_OK && magic != kMagic) {
        rt_gguf_close(g);
        return gfail(RT_ERR_GGUF_MAGIC,
                     "invalid GGUF magic: expected 0x46554747 (\"GGUF\"), got 0x%08X", magic);
    }
    g->version = r.get<uint32_t>();
    if (r.err == RT_OK && g->version != 2 && g->version != 3) {
        const uint32_t v = g->version;
        rt_gguf_close(g);
        return gfail(RT_ERR_GGUF_VERSION, "unsupported GGUF version: %u (expected 2 or 3)", v);
    }
    const uint64_t n_tensors = r.get<uint64_t>();
    const uint64_t n_kv = r.get<uint64_t>();
    // metadata (a key seen twice keeps the last value, as HashMap::insert does)
    for (uint64_t i = 0; i < n_kv && r.err == RT_OK; ++i) {
        Meta m;
        m.key = r.str();
        const uint32_t t = r.get<uint32_t>();
        if (r.err != RT_OK) break;
        read_value(r, t, m);
        if (r.err != RT_OK) break;
        auto it = g->meta_idx.find(m.key);
        if (it != g->meta_idx.end()) {
            g->meta[it->second] = m;
        } else {
            g->meta_idx[m.key] = (int64_t)g->meta.size();
            g->meta.push_back(m);
        }
    }
    if (r.err == RT_OK) {
        // general.alignment: a u32 value (Metadata::as_u32), default 32
        auto it = g->meta_idx.find("general.alignment");
        if (it != g->meta_idx.end() && g->meta[it->second].type == 4 && g->meta[it->second].u)
            g->alignment = g->meta[it->second].u;
    }
    // tensor infos (parser.rs read_tensor_info)
    for (uint64_t i = 0; i < n_tensors && r.err == RT_OK; ++i) {
        Tensor t;
        t.name = r.str();
        const uint32_t nd = r.get<uint32_t>();
        for (uint32_t d = 0; d < nd && r.err == RT_OK; ++d) t.dims.push_back(r.get<uint64_t>());
        t.dtype = r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        if (r.err != RT_OK) break;
        const BlockInfo bi = block_info(t.dtype);
        if (bi.el == 0) {
            const uint32_t dt = t.dtype;
            rt_gguf_close(g);
            return gfail(RT_ERR_GGUF_DTYPE, "unknown tensor dtype: %u", dt);
        }
        uint64_t n = 1;
        for (uint64_t d : t.dims) n *= d;
        if (n == 0) n = 1;  // num_elements() is at least 1 (types.rs)
        // tensor_data_size: whole blocks (types.rs)
        t.bytes = (n + bi.el - 1) / bi.el * bi.bytes;
        g->tensor_idx[t.name] = (int64_t)g->tensors.size();
        g->tensors.push_back(t);
    }
    if (r.err != RT_OK) {
        const int e = r.err;
        rt_gguf_close(g);
        return e;
    }
    g->data_offset = (r.pos + g->alignment - 1) / g->alignment * g->alignment;
    for (const Tensor& t : g->tensors)
        if (g->data_offset + t.offset + t.bytes > g->size) {
            rt_gguf_close(g);
            return gfail(RT_ERR_GGUF_DATA_OVERFLOW, "tensor data region exceeds file size");
        }
    *out = g;
    return RT_OK;
}

void rt_gguf_close(rt_gguf* g) {
    if (!g) return;
    if (g->map) munmap((void*)g->map, g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

uint32_t rt_gguf_version(const rt_gguf* g) { return g ? g->version : 0; }
uint64_t rt_gguf_alignment(const rt_gguf* g) { return g ? g->alignment : 0; }
uint64_t rt_gguf_data_offset(const rt_gguf* g) { return g ? g->data_offset : 0; }
uint64_t rt_gguf_tensor_count(const rt_gguf* g) { return g ? g->tensors.size() : 0; }
uint64_t rt_gguf_meta_count(const rt_gguf* g) { return g ? g->meta.size() : 0; }

int64_t rt_gguf_find_tensor(const rt_gguf* g, const char* name) {
    if (!g || !name) return -1;
    auto it = g->tensor_idx.find(name);
    return it == g->tensor_idx.end() ? -1 : it->second;
}

int rt_gguf_tensor_info(const rt_gguf* g, uint64_t i, const char** name, uint32_t* n_dims,
                        uint64_t dims[8], uint32_t* dtype, uint64_t* offset, uint64_t* bytes) {
    if (!g || i >= g->tensors.size()) return gfail(RT_ERR_GGUF_IO, "tensor index out of range");
    const Tensor& t = g->tensors[i];
    if (name) *name = t.name.c_str();
    if (n_dims) *n_dims = (uint32_t)t.dims.size();
    if (dims)
        for (size_t d = 0; d < t.dims.size() && d < 8; ++d) dims[d] = t.dims[d];
    if (dtype) *dtype = t.dtype;
    if (offset) *offset = t.offset;
    if (bytes) *bytes = t.bytes;
    return RT_OK;
}

const void* rt_gguf_tensor_data(const rt_gguf* g, uint64_t i) {
    if (!g || i >= g->tensors.size()) return nullptr;
    return g->map + g->data_offset + g->tensors[i].offset;
}

int rt_gguf_upload(rt_ctx* ctx, const rt_gguf* g, uint64_t i, void* dst_dev) {
    if (!g || i >= g->tensors.size() || !dst_dev)
        return gfail(RT_ERR_GGUF_IO, "upload: bad tensor index or null destination");
    const Tensor& t = g->tensors[i];
    return rt_upload(ctx, dst_dev, g->map + g->data_offset + t.offset, t.bytes);
}

int64_t rt_gguf_find_meta(const rt_gguf* g, const char* key) {
    if (!g || !key) return -1;
    auto it = g->meta_idx.find(key);
    return it == g->meta_idx.end() ? -1 : it->second;
}

int rt_gguf_meta_info(const rt_gguf* g, uint64_t i, const char** key, uint32_t* type,
                      uint32_t* elem_type, uint64_t* count) {
    if (!g || i >= g->meta.size()) return gfail(RT_ERR_GGUF_IO, "metadata index out of range");
    const Meta& m = g->meta[i];
    if (key) *key = m.key.c_str();
    if (type) *type = m.type;
    if (elem_type) *elem_type = m.elem_type;
    if (count) *count = m.count;
    return RT_OK;
}

// Integer value (types 0-5, 7, 10, 11) as a signed 64-bit number.
int rt_gguf_meta_int(const rt_gguf* g, uint64_t i, int64_t* out) {
    if (!g || i >= g->meta.size() || !out) return gfail(RT_ERR_GGUF_IO, "metadata index out of range");
    const Meta& m = g->meta[i];
    switch (m.type) {
        case 0: case 1: case 2: case 3: case 4: case 5: case 7: case 10: case 11:
            *out = (int64_t)m.u;
            return RT_OK;
        default:
            return gfail(RT_ERR_GGUF_METADATA_TYPE, "metadata '%s' is not an integer", m.key.c_str());
    }
}

int rt_gguf_meta_float(const rt_gguf* g, uint64_t i, double* out) {
    if (!g || i >= g->meta.size() || !out) return gfail(RT_ERR_GGUF_IO, "metadata index out of range");
    const Meta& m = g->meta[i];
    if (m.type != 6 && m.type != 12)
        return gfail(RT_ERR_GGUF_METADATA_TYPE, "metadata '%s' is not a float", m.key.c_str());
    *out = m.f;
    return RT_OK;
}

const char* rt_gguf_meta_string(const rt_gguf* g, uint64_t i) {
    if (!g || i >= g->meta.size() || g->meta[i].type != 8) return nullptr;
    return g->meta[i].s.c_str();
}

// Copies up to `max` scalar array elements (converted to double) into out.
int rt_gguf_meta_array_numbers(const rt_gguf* g, uint64_t i, double* out, uint64_t max) {
    if (!g || i >= g->meta.size()) return gfail(RT_ERR_GGUF_IO, "metadata index out of range");
    const Meta& m = g->meta[i];
    const uint32_t es = scalar_size(m.elem_type);
    if (m.type != 9 || es == 0)
        return gfail(RT_ERR_GGUF_METADATA_TYPE, "metadata '%s' is not a numeric array",
                     m.key.c_str());
    const uint8_t* p = g->map + m.arr_off;
    for (uint64_t k = 0; k < m.count && k < max; ++k, p += es) {
        double v = 0;
        switch (m.elem_type) {
            case 0: v = *(const uint8_t*)p; break;
            case 1: v = *(const int8_t*)p; break;
            case 2: { uint16_t x; memcpy(&x, p, 2); v = x; break; }
            case 3: { int16_t x; memcpy(&x, p, 2); v = x; break; }
            case 4: { uint32_t x; memcpy(&x, p, 4); v = x; break; }
            case 5: { int32_t x; memcpy(&x, p, 4); v = x; break; }
            case 6: { float x; memcpy(&x, p, 4); v = x; break; }
            case 7: v = *p != 0; break;
            case 10: { uint64_t x; memcpy(&x, p, 8); v = (double)x; break; }
            case 11: { int64_t x; memcpy(&x, p, 8); v = (double)x; break; }
            case 12: { double x; memcpy(&x, p, 8); v = x; break; }
        }
        out[k] = v;
    }
    return RT_OK;
}

// String element k of a string array (a pointer into the mapping and its
// length; not NUL-terminated).
int rt_gguf_meta_array_string(const rt_gguf* g, uint64_t i, uint64_t k, const char** s,
                              uint64_t* len) {
    if (!g || i >= g->meta.size()) return gfail(RT_ERR_GGUF_IO, "metadata index out of range");
    const Meta& m = g->meta[i];
    if (m.type != 9 || m.elem_type != 8 || k >= m.count)
        return gfail(RT_ERR_GGUF_METADATA_TYPE, "metadata '%s' has no string element %llu",
                     m.key.c_str(), (unsigned long long)k);
    uint64_t off = m.arr_off;
    for (uint64_t j = 0; j < k; ++j) {
        uint64_t n;
        memcpy(&n, g->map + off, 8);
        off += 8 + n;
    }
    uint64_t n;
    memcpy(&n, g->map + off, 8);
    if (s) *s = (const char*)g->map + off + 8;
    if (len) *len = n;
    return RT_OK;
}

}  // extern "C"
