// Packed GGUF loader and device weight cache.
//
// The reader follows GgufReader::open (barq_core/src/gguf.rs:250-337): magic
// "GGUF", version <= 3, u64 tensor and KV counts, KV pairs of the 13 value
// types (arrays nest), `general.alignment` when it is a u32 (default 32),
// tensor infos (name, dims, type id, offset), data section at the aligned
// position after the infos.  The file is memory-mapped and a tensor is its
// packed bytes at data_offset + offset (the position load_tensor seeks to,
// :428-431); nothing is dequantized at load.
//
// The cache replaces WeightCache's dequantize-and-transpose entries
// (models/src/weight_cache.rs:172-210) with one device allocation holding
// every tensor's packed bytes, 256-byte aligned, in file order.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "api_internal.hpp"

using barq_api::DeviceGuard;
using barq_api::fail;
using barq_api::ok;

namespace {

constexpr uint32_t GGUF_MAX_VERSION = 3;        // gguf.rs:30
constexpr uint32_t GGUF_DEFAULT_ALIGNMENT = 32;  // gguf.rs:33

// value types (GgufType, gguf.rs:38-52)
enum : uint32_t {
    V_U8 = 0, V_I8 = 1, V_U16 = 2, V_I16 = 3, V_U32 = 4, V_I32 = 5, V_F32 = 6, V_BOOL = 7,
    V_STRING = 8, V_ARRAY = 9, V_U64 = 10, V_I64 = 11, V_F64 = 12
};

size_t scalar_size(uint32_t t) {
    switch (t) {
    case V_U8: case V_I8: case V_BOOL: return 1;
    case V_U16: case V_I16: return 2;
    case V_U32: case V_I32: case V_F32: return 4;
    case V_U64: case V_I64: case V_F64: return 8;
    default: return 0;
    }
}

// Tensor type ids GgufTensorType::from_u32 accepts (gguf.rs:141-166), with the
// block geometry of those whose layout is known here (0 bytes: accepted but
// not sized, like the reference's IQ types, which it cannot load either).
bool tensor_type_geometry(uint32_t t, size_t* elems, size_t* bytes) {
    switch (t) {
    case 0: *elems = 1; *bytes = 4; return true;       // F32
    case 1: *elems = 1; *bytes = 2; return true;       // F16
    case 2: *elems = 32; *bytes = 18; return true;     // Q4_0 (GGUF block_q4_0)
    case 3: *elems = 32; *bytes = 20; return true;     // Q4_1
    case 6: *elems = 32; *bytes = 22; return true;     // Q5_0
    case 7: *elems = 32; *bytes = 24; return true;     // Q5_1
    case 8: *elems = 32; *bytes = 34; return true;     // Q8_0
    case 9: *elems = 32; *bytes = 36; return true;     // Q8_1
    case 10: *elems = 256; *bytes = 84; return true;   // Q2_K
    case 11: *elems = 256; *bytes = 110; return true;  // Q3_K
    case 12: *elems = 256; *bytes = 144; return true;  // Q4_K
    case 13: *elems = 256; *bytes = 176; return true;  // Q5_K
    case 14: *elems = 256; *bytes = 210; return true;  // Q6_K
    case 15: *elems = 256; *bytes = 292; return true;  // Q8_K
    case 16: case 18: case 19: case 30000: *elems = 256; *bytes = 0; return true;   // IQ4_KS, IQ2_KS, IQ3_KS, Q4_K_R4
    default: return false;
    }
}

bool valid_utf8(const uint8_t* p, size_t n) {
    size_t i = 0;
    while (i < n) {
        const uint8_t c = p[i];
        size_t len;
        uint32_t cp;
        if (c < 0x80) { i++; continue; }
        if ((c & 0xE0) == 0xC0) { len = 2; cp = c & 0x1F; }
        else if ((c & 0xF0) == 0xE0) { len = 3; cp = c & 0x0F; }
        else if ((c & 0xF8) == 0xF0) { len = 4; cp = c & 0x07; }
        else return false;
        if (i + len > n) return false;
        for (size_t j = 1; j < len; j++) {
            if ((p[i + j] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (p[i + j] & 0x3F);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && (cp < 0x10000 || cp > 0x10FFFF)) ||
            (cp >= 0xD800 && cp <= 0xDFFF))
            return false;   // overlong, out of range or a surrogate: rejected like String::from_utf8
        i += len;
    }
    return true;
}

struct Cursor {
    const uint8_t* base;
    size_t size, pos;
    bool take(size_t n) {
        if (n > size - pos) return false;
        pos += n;
        return true;
    }
    template <class T>
    bool read(T* v) {
        if (sizeof(T) > size - pos) return false;
        memcpy(v, base + pos, sizeof(T));
        pos += sizeof(T);
        return true;
    }
};

}  // namespace

struct barq_rocm_gguf {
    int fd = -1;
    const uint8_t* map = nullptr;
    size_t size = 0;
    uint32_t version = 0, alignment = GGUF_DEFAULT_ALIGNMENT;
    uint64_t n_tensors = 0, n_kv = 0, data_offset = 0;
    struct KV {
        uint32_t type = 0, arr_type = 0;
        uint64_t arr_len = 0;
        size_t value_pos = 0;   // file position of the value (after the type id)
    };
    std::unordered_map<std::string, KV> kv;   // a repeated key keeps the last value (HashMap::insert)
    struct Tensor {
        std::string name;
        uint32_t n_dims = 0, type = 0;
        uint64_t dims[4] = {1, 1, 1, 1};
        uint64_t offset = 0, nbytes = 0;
    };
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> by_name;   // first tensor of a name (iter().find)
};

namespace {

int gguf_err(const char* what, size_t pos) { return fail(BARQ_E_GGUF, "invalid GGUF: %s at byte %zu", what, pos); }

int read_string(Cursor& c, std::string* out) {
    uint64_t len;
    if (!c.read(&len)) return fail(BARQ_E_IO, "GGUF: file ends inside a string length at byte %zu", c.pos);
    if (len > c.size - c.pos) return fail(BARQ_E_IO, "GGUF: string of %llu bytes past the end of the file at byte %zu",
                                          (unsigned long long)len, c.pos);
    if (!valid_utf8(c.base + c.pos, (size_t)len)) return gguf_err("string is not UTF-8", c.pos);
    if (out) out->assign(reinterpret_cast<const char*>(c.base + c.pos), (size_t)len);
    c.pos += (size_t)len;
    return ok();
}

// Skips one value of type t (GgufReader::read_value, gguf.rs:348-373).
int skip_value(Cursor& c, uint32_t t, int depth) {
    if (depth > 64) return gguf_err("arrays nested too deeply", c.pos);
    if (t == V_STRING) return read_string(c, nullptr);
    if (t == V_ARRAY) {
        uint32_t et;
        uint64_t n;
        if (!c.read(&et) || !c.read(&n)) return fail(BARQ_E_IO, "GGUF: file ends inside an array header at byte %zu", c.pos);
        if (et > V_F64) return fail(BARQ_E_GGUF, "invalid GGUF: Unknown type: %u", et);
        const size_t es = scalar_size(et);
        if (es) {
            if (n > (c.size - c.pos) / es) return fail(BARQ_E_IO, "GGUF: array past the end of the file at byte %zu", c.pos);
            c.pos += (size_t)(n * es);
            return ok();
        }
        for (uint64_t i = 0; i < n; i++) {
            const int rc = skip_value(c, et, depth + 1);
            if (rc != BARQ_OK) return rc;
        }
        return ok();
    }
    const size_t s = scalar_size(t);
    if (!s) return fail(BARQ_E_GGUF, "invalid GGUF: Unknown type: %u", t);
    if (!c.take(s)) return fail(BARQ_E_IO, "GGUF: file ends inside a value at byte %zu", c.pos);
    return ok();
}

int parse(barq_rocm_gguf* g) {
    Cursor c{g->map, g->size, 0};
    uint8_t magic[4];
    if (!c.read(&magic)) return fail(BARQ_E_IO, "GGUF: file shorter than the magic");
    if (memcmp(magic, "GGUF", 4) != 0) return fail(BARQ_E_GGUF, "invalid GGUF: Invalid magic, expected \"GGUF\"");
    if (!c.read(&g->version)) return fail(BARQ_E_IO, "GGUF: file ends inside the version");
    if (g->version > GGUF_MAX_VERSION)
        return fail(BARQ_E_GGUF, "invalid GGUF: Unsupported version: %u, maximum supported: %u", g->version, GGUF_MAX_VERSION);
    if (!c.read(&g->n_tensors) || !c.read(&g->n_kv)) return fail(BARQ_E_IO, "GGUF: file ends inside the header");
    for (uint64_t i = 0; i < g->n_kv; i++) {
        std::string key;
        int rc = read_string(c, &key);
        if (rc != BARQ_OK) return rc;
        barq_rocm_gguf::KV v;
        if (!c.read(&v.type)) return fail(BARQ_E_IO, "GGUF: file ends inside a value type at byte %zu", c.pos);
        if (v.type > V_F64) return fail(BARQ_E_GGUF, "invalid GGUF: Unknown type: %u", v.type);
        v.value_pos = c.pos;
        if (v.type == V_ARRAY) {
            Cursor h = c;
            if (!h.read(&v.arr_type) || !h.read(&v.arr_len))
                return fail(BARQ_E_IO, "GGUF: file ends inside an array header at byte %zu", c.pos);
        }
        rc = skip_value(c, v.type, 0);
        if (rc != BARQ_OK) return rc;
        g->kv[key] = v;
    }
    // general.alignment when stored as a u32 (gguf.rs:279-282)
    auto al = g->kv.find("general.alignment");
    if (al != g->kv.end() && al->second.type == V_U32) memcpy(&g->alignment, g->map + al->second.value_pos, 4);
    if (g->alignment == 0 || (g->alignment & (g->alignment - 1)))
        return fail(BARQ_E_GGUF, "invalid GGUF: general.alignment %u is not a power of two", g->alignment);
    g->tensors.reserve((size_t)(g->n_tensors < g->size / 24 ? g->n_tensors : g->size / 24));
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        barq_rocm_gguf::Tensor t;
        int rc = read_string(c, &t.name);
        if (rc != BARQ_OK) return rc;
        if (!c.read(&t.n_dims)) return fail(BARQ_E_IO, "GGUF: file ends inside a tensor info at byte %zu", c.pos);
        uint64_t elements = 1;
        for (uint32_t d = 0; d < t.n_dims; d++) {
            uint64_t v;
            if (!c.read(&v)) return fail(BARQ_E_IO, "GGUF: file ends inside tensor dims at byte %zu", c.pos);
            if (d < 4) t.dims[d] = v;
            else t.dims[3] *= v;   // more than four dims fold into the outermost
            elements *= v;
        }
        if (!c.read(&t.type) || !c.read(&t.offset))
            return fail(BARQ_E_IO, "GGUF: file ends inside a tensor info at byte %zu", c.pos);
        size_t be = 0, bb = 0;
        if (!tensor_type_geometry(t.type, &be, &bb)) return fail(BARQ_E_GGUF, "invalid GGUF: Unknown GGUF tensor type: %u", t.type);
        t.nbytes = (bb && t.dims[0] % be == 0) ? elements / be * bb : 0;
        g->by_name.emplace(t.name, g->tensors.size());
        g->tensors.push_back(std::move(t));
    }
    const uint64_t a = g->alignment;
    g->data_offset = (c.pos + a - 1) & ~(a - 1);
    return ok();
}

}  // namespace

extern "C" {

int barq_rocm_gguf_open(const char* path, barq_rocm_gguf** out) {
    if (!path || !out) return fail(BARQ_E_INVALID, "gguf_open: null argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(BARQ_E_IO, "GGUF: cannot open %s: %s", path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return fail(BARQ_E_IO, "GGUF: cannot stat %s", path);
    }
    auto* g = new barq_rocm_gguf();
    g->fd = fd;
    g->size = (size_t)st.st_size;
    if (g->size) {
        void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            close(fd);
            delete g;
            return fail(BARQ_E_IO, "GGUF: cannot map %s", path);
        }
        g->map = static_cast<const uint8_t*>(m);
    }
    const int rc = parse(g);
    if (rc != BARQ_OK) {
        barq_rocm_gguf_close(g);
        return rc;
    }
    *out = g;
    return ok();
}

int barq_rocm_gguf_close(barq_rocm_gguf* g) {
    if (!g) return ok();
    if (g->map) munmap(const_cast<uint8_t*>(g->map), g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
    return ok();
}

int barq_rocm_gguf_info(const barq_rocm_gguf* g, uint32_t* version, uint64_t* n_tensors, uint64_t* n_kv,
                        uint32_t* alignment, uint64_t* data_offset) {
    if (!g) return fail(BARQ_E_INVALID, "gguf_info: null file");
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = g->n_tensors;
    if (n_kv) *n_kv = g->n_kv;
    if (alignment) *alignment = g->alignment;
    if (data_offset) *data_offset = g->data_offset;
    return ok();
}

int barq_rocm_gguf_tensor(const barq_rocm_gguf* g, uint64_t index, const char** name, int* type, uint32_t* n_dims,
                          uint64_t* dims, uint64_t* offset, uint64_t* nbytes, const void** data) {
    if (!g) return fail(BARQ_E_INVALID, "gguf_tensor: null file");
    if (index >= g->tensors.size()) return fail(BARQ_E_INVALID, "gguf_tensor: index %llu of %zu", (unsigned long long)index,
                                                g->tensors.size());
    const auto& t = g->tensors[(size_t)index];
    if (name) *name = t.name.c_str();
    if (type) *type = (int)t.type;
    if (n_dims) *n_dims = t.n_dims;
    if (dims) memcpy(dims, t.dims, sizeof t.dims);
    if (offset) *offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    if (data) {
        *data = nullptr;
        if (t.nbytes) {
            // load_tensor's read_exact fails with Error::Io past the end of the file
            const uint64_t start = g->data_offset + t.offset;
            if (start < g->data_offset || start > g->size || t.nbytes > g->size - start)
                return fail(BARQ_E_IO, "GGUF: tensor %s (%llu bytes at %llu) extends past the end of the file (%zu bytes)",
                            t.name.c_str(), (unsigned long long)t.nbytes, (unsigned long long)start, g->size);
            *data = g->map + start;
        }
    }
    return ok();
}

int barq_rocm_gguf_find_tensor(const barq_rocm_gguf* g, const char* name, uint64_t* index) {
    if (!g || !name || !index) return fail(BARQ_E_INVALID, "gguf_find_tensor: null argument");
    auto it = g->by_name.find(name);
    if (it == g->by_name.end()) return fail(BARQ_E_INVALID, "Tensor not found: %s", name);   // load_tensor, gguf.rs:416-418
    *index = it->second;
    return ok();
}

int barq_rocm_gguf_kv_type(const barq_rocm_gguf* g, const char* key, int* type, int* array_type, uint64_t* array_len) {
    if (!g || !key) return fail(BARQ_E_INVALID, "gguf_kv_type: null argument");
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return fail(BARQ_E_INVALID, "GGUF key not found: %s", key);
    if (type) *type = (int)it->second.type;
    if (array_type) *array_type = it->second.type == V_ARRAY ? (int)it->second.arr_type : -1;
    if (array_len) *array_len = it->second.type == V_ARRAY ? it->second.arr_len : 0;
    return ok();
}

int barq_rocm_gguf_kv_int(const barq_rocm_gguf* g, const char* key, int64_t* value) {
    if (!g || !key || !value) return fail(BARQ_E_INVALID, "gguf_kv_int: null argument");
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return fail(BARQ_E_INVALID, "GGUF key not found: %s", key);
    const uint8_t* p = g->map + it->second.value_pos;
    switch (it->second.type) {
    case V_U8: *value = p[0]; return ok();
    case V_I8: *value = (int8_t)p[0]; return ok();
    case V_BOOL: *value = p[0] != 0; return ok();
    case V_U16: { uint16_t v; memcpy(&v, p, 2); *value = v; return ok(); }
    case V_I16: { int16_t v; memcpy(&v, p, 2); *value = v; return ok(); }
    case V_U32: { uint32_t v; memcpy(&v, p, 4); *value = v; return ok(); }
    case V_I32: { int32_t v; memcpy(&v, p, 4); *value = v; return ok(); }
    case V_I64: { int64_t v; memcpy(&v, p, 8); *value = v; return ok(); }
    case V_U64: {
        uint64_t v;
        memcpy(&v, p, 8);
        if (v > (uint64_t)INT64_MAX) return fail(BARQ_E_DIM, "GGUF key %s: %llu does not fit int64", key, (unsigned long long)v);
        *value = (int64_t)v;
        return ok();
    }
    default: return fail(BARQ_E_UNSUPPORTED, "GGUF key %s is not an integer (type %u)", key, it->second.type);
    }
}

int barq_rocm_gguf_kv_number(const barq_rocm_gguf* g, const char* key, double* value) {
    if (!g || !key || !value) return fail(BARQ_E_INVALID, "gguf_kv_number: null argument");
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return fail(BARQ_E_INVALID, "GGUF key not found: %s", key);
    const uint8_t* p = g->map + it->second.value_pos;
    if (it->second.type == V_F32) { float v; memcpy(&v, p, 4); *value = v; return ok(); }
    if (it->second.type == V_F64) { double v; memcpy(&v, p, 8); *value = v; return ok(); }
    if (it->second.type == V_U64) { uint64_t v; memcpy(&v, p, 8); *value = (double)v; return ok(); }
    int64_t iv;
    const int rc = barq_rocm_gguf_kv_int(g, key, &iv);
    if (rc != BARQ_OK) return fail(BARQ_E_UNSUPPORTED, "GGUF key %s is not a number (type %u)", key, it->second.type);
    *value = (double)iv;
    return ok();
}

int barq_rocm_gguf_kv_string(const barq_rocm_gguf* g, const char* key, const char** ptr, uint64_t* len) {
    if (!g || !key || !ptr || !len) return fail(BARQ_E_INVALID, "gguf_kv_string: null argument");
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return fail(BARQ_E_INVALID, "GGUF key not found: %s", key);
    if (it->second.type != V_STRING) return fail(BARQ_E_UNSUPPORTED, "GGUF key %s is not a string (type %u)", key, it->second.type);
    uint64_t n;
    memcpy(&n, g->map + it->second.value_pos, 8);
    *ptr = reinterpret_cast<const char*>(g->map + it->second.value_pos + 8);
    *len = n;
    return ok();
}

}  // extern "C"

// ---- device weight cache ------------------------------------------------------

struct barq_rocm_cache {
    int device = 0;
    void* base = nullptr;
    uint64_t bytes = 0;
    struct Entry {
        int type = 0;
        uint64_t n_rows = 0, k = 0, offset = 0, nbytes = 0;
    };
    std::unordered_map<std::string, Entry> entries;
};

extern "C" {

int barq_rocm_cache_create(barq_rocm_handle* h, const barq_rocm_gguf* g, barq_rocm_cache** out) {
    if (!h || !g || !out) return fail(BARQ_E_INVALID, "cache_create: null argument");
    *out = nullptr;
    DeviceGuard dg(h);
    auto* c = new barq_rocm_cache();
    c->device = h->device;
    uint64_t total = 0;
    for (size_t i = 0; i < g->tensors.size(); i++) {
        const auto& t = g->tensors[i];
        if (!t.nbytes || g->by_name.at(t.name) != i) continue;   // unsized types are not cached; first of a name wins
        const void* src;
        const int rc = barq_rocm_gguf_tensor(g, i, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, &src);
        if (rc != BARQ_OK) {
            delete c;
            return rc;
        }
        barq_rocm_cache::Entry e;
        e.type = (int)t.type;
        e.k = t.dims[0];
        e.n_rows = t.dims[1] * t.dims[2] * t.dims[3];
        e.offset = total;
        e.nbytes = t.nbytes;
        total += (t.nbytes + 255) / 256 * 256;
        c->entries.emplace(t.name, e);
    }
    if (total) {
        const hipError_t e = hipMalloc(&c->base, total);
        if (e != hipSuccess) {
            delete c;
            return fail(BARQ_E_ALLOC, "cache_create: %llu device bytes: %s", (unsigned long long)total, hipGetErrorString(e));
        }
    }
    c->bytes = total;
    for (size_t i = 0; i < g->tensors.size(); i++) {
        const auto& t = g->tensors[i];
        if (!t.nbytes || g->by_name.at(t.name) != i) continue;
        auto it = c->entries.find(t.name);
        const hipError_t e = hipMemcpyAsync(static_cast<uint8_t*>(c->base) + it->second.offset,
                                            g->map + g->data_offset + t.offset, t.nbytes, hipMemcpyHostToDevice, h->stream);
        if (e != hipSuccess) {
            barq_rocm_cache_destroy(c);
            return fail(BARQ_E_BACKEND, "cache_create: copy of %s: %s", t.name.c_str(), hipGetErrorString(e));
        }
    }
    const hipError_t e = hipStreamSynchronize(h->stream);
    if (e != hipSuccess) {
        barq_rocm_cache_destroy(c);
        return fail(BARQ_E_BACKEND, "cache_create: %s", hipGetErrorString(e));
    }
    *out = c;
    return ok();
}

int barq_rocm_cache_get(const barq_rocm_cache* c, const char* name, int* type, uint64_t* n_rows, uint64_t* k,
                        const void** device_ptr) {
    if (!c || !name) return fail(BARQ_E_INVALID, "cache_get: null argument");
    auto it = c->entries.find(name);
    if (it == c->entries.end()) return fail(BARQ_E_INVALID, "Tensor not found: %s", name);
    if (type) *type = it->second.type;
    if (n_rows) *n_rows = it->second.n_rows;
    if (k) *k = it->second.k;
    if (device_ptr) *device_ptr = static_cast<const uint8_t*>(c->base) + it->second.offset;
    return ok();
}

uint64_t barq_rocm_cache_bytes(const barq_rocm_cache* c) { return c ? c->bytes : 0; }

int barq_rocm_cache_destroy(barq_rocm_cache* c) {
    if (!c) return ok();
    if (c->base) {
        DeviceGuard dg(c->device);
        (void)hipDeviceSynchronize();
        (void)hipFree(c->base);
    }
    delete c;
    return ok();
}

}  // extern "C"
