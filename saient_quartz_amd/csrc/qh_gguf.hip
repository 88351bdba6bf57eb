// qh_gguf.hip -- GGUF container reader / writer and device upload (host code).
//
// Reader: GgufFile::open / parse (src/gguf.rs:61-126): magic 0x46554747,
// versions 1..3 (v1: u32 counts and dims, v2+: u64), typed metadata values
// (scalars, strings, arrays of one element type), tensor infos (name, dims with
// dims[0] fastest-varying, ggml type, offset relative to the data section), data
// section at the next multiple of general.alignment (default 32) after the
// infos.  The file is memory-mapped; tensor data are views into the map.
// Metadata accessors follow GgufValue::as_u32 / as_u64 / as_str
// (src/gguf.rs:18-35): u32 reads Uint32 or Int32, u64 reads Uint64 or Uint32.
// Writer: the layout make_test_model.py produces (version 3, each tensor's data
// padded to the alignment), for any ggml type and metadata value type.
// Upload: GpuWeights::from_weights' per-tensor upload (src/cuda.rs:170-172).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/quartz_hip.h"
#include "qh_internal.h"

namespace {

struct GValue {
    uint32_t type = 0;        // GGUF value type 0..12
    uint32_t elem = 0;        // arrays: element type
    uint64_t u = 0;           // integer / bool / float bits (scalars)
    double f = 0.0;           // float32 / float64 value
    std::string s;            // strings
    std::vector<uint8_t> raw; // arrays of fixed-size elements: little-endian bytes
    std::vector<std::string> strs;  // arrays of strings
    uint64_t count = 0;       // arrays: element count
};

struct GTensor {
    std::string name;
    uint32_t n_dims = 0;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
};

const int kScalarSize[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};

struct Reader {
    const uint8_t* p;
    size_t n, pos = 0;
    std::string err;
    bool need(size_t k, const char* what) {
        if (n - pos < k) {
            if (err.empty()) err = std::string("EOF reading ") + what;
            return false;
        }
        return true;
    }
    bool u8(uint8_t& v) { if (!need(1, "u8")) return false; v = p[pos++]; return true; }
    bool u16(uint16_t& v) { if (!need(2, "u16")) return false; memcpy(&v, p + pos, 2); pos += 2; return true; }
    bool u32(uint32_t& v) { if (!need(4, "u32")) return false; memcpy(&v, p + pos, 4); pos += 4; return true; }
    bool u64(uint64_t& v) { if (!need(8, "u64")) return false; memcpy(&v, p + pos, 8); pos += 8; return true; }
    bool str(std::string& s) {
        uint64_t len;
        if (!u64(len)) return false;
        if (n - pos < len) {
            if (err.empty()) err = "EOF reading string len=" + std::to_string(len);
            return false;
        }
        s.assign(reinterpret_cast<const char*>(p + pos), (size_t)len);
        pos += (size_t)len;
        return true;
    }
    bool scalar(uint32_t t, GValue& v) {
        v.type = t;
        switch (t) {
            case 0: case 1: case 7: { uint8_t x; if (!u8(x)) return false; v.u = t == 1 ? (uint64_t)(int64_t)(int8_t)x : x; return true; }
            case 2: case 3: { uint16_t x; if (!u16(x)) return false; v.u = t == 3 ? (uint64_t)(int64_t)(int16_t)x : x; return true; }
            case 4: case 5: { uint32_t x; if (!u32(x)) return false; v.u = t == 5 ? (uint64_t)(int64_t)(int32_t)x : x; return true; }
            case 6: { uint32_t x; if (!u32(x)) return false; v.u = x; float f; memcpy(&f, &x, 4); v.f = f; return true; }
            case 8: return str(v.s);
            case 10: case 11: { uint64_t x; if (!u64(x)) return false; v.u = x; return true; }
            case 12: { uint64_t x; if (!u64(x)) return false; v.u = x; memcpy(&v.f, &x, 8); return true; }
            default:
                if (err.empty()) err = "Unknown array elem type: " + std::to_string(t);
                return false;
        }
    }
    bool value(uint32_t version, GValue& v) {
        uint32_t t;
        if (!u32(t)) return false;
        if (t != 9) {
            if (t > 12) {
                if (err.empty()) err = "Unknown GGUF value type: " + std::to_string(t);
                return false;
            }
            return scalar(t, v);
        }
        v.type = 9;
        if (!u32(v.elem)) return false;
        if (version == 1) {
            uint32_t c;
            if (!u32(c)) return false;
            v.count = c;
        } else if (!u64(v.count)) {
            return false;
        }
        if (v.elem == 8) {
            for (uint64_t i = 0; i < v.count; i++) {
                std::string s;
                if (!str(s)) return false;
                v.strs.push_back(std::move(s));
            }
            return true;
        }
        if (v.elem > 12 || v.elem == 9) {
            if (err.empty()) err = "Unknown array elem type: " + std::to_string(v.elem);
            return false;
        }
        const uint64_t sz = (uint64_t)kScalarSize[v.elem];
        if (v.count > (n - pos) / sz) return need(n, "array");  // EOF
        v.raw.assign(p + pos, p + pos + v.count * sz);
        pos += (size_t)(v.count * sz);
        return true;
    }
};

}  // namespace

struct qh_gguf {
    uint32_t version = 0;
    std::vector<std::string> keys;  // file order
    std::unordered_map<std::string, GValue> kv;
    std::vector<GTensor> tensors;
    std::unordered_map<std::string, int64_t> by_name;
    uint64_t data_offset = 0, alignment = 32;
    void* map = nullptr;
    size_t size = 0;
    ~qh_gguf() {
        if (map) munmap(map, size);
    }
};

struct qh_gguf_writer {
    std::vector<std::pair<std::string, GValue>> kv;
    struct T { std::string name; std::vector<uint64_t> dims; uint32_t type; const uint8_t* data; size_t bytes; };
    std::vector<T> tensors;
    uint64_t alignment = 32;
};

static int gg_fail(int rc, const std::string& msg) {
    qh_set_error(msg.c_str());
    return rc;
}

static int gg_parse(qh_gguf* g) {
    Reader r{static_cast<const uint8_t*>(g->map), g->size};
    uint32_t magic;
    if (!r.u32(magic)) return gg_fail(QH_ERR_FORMAT, r.err);
    if (magic != 0x46554747u) {
        char b[64];
        snprintf(b, sizeof b, "Not a GGUF file (magic 0x%08X)", magic);
        return gg_fail(QH_ERR_FORMAT, b);
    }
    if (!r.u32(g->version)) return gg_fail(QH_ERR_FORMAT, r.err);
    if (g->version < 1 || g->version > 3)
        return gg_fail(QH_ERR_FORMAT, "Unsupported GGUF version " + std::to_string(g->version));
    uint64_t nt, nkv;
    if (g->version == 1) {
        uint32_t a, b;
        if (!r.u32(a) || !r.u32(b)) return gg_fail(QH_ERR_FORMAT, r.err);
        nt = a;
        nkv = b;
    } else if (!r.u64(nt) || !r.u64(nkv)) {
        return gg_fail(QH_ERR_FORMAT, r.err);
    }
    for (uint64_t i = 0; i < nkv; i++) {
        std::string key;
        GValue v;
        if (!r.str(key) || !r.value(g->version, v)) return gg_fail(QH_ERR_FORMAT, r.err);
        if (!g->kv.count(key)) g->keys.push_back(key);
        g->kv[key] = std::move(v);  // a repeated key keeps the last value (HashMap::insert)
    }
    for (uint64_t i = 0; i < nt; i++) {
        GTensor t;
        if (!r.str(t.name) || !r.u32(t.n_dims)) return gg_fail(QH_ERR_FORMAT, r.err);
        if (t.n_dims > (r.n - r.pos) / 4) return gg_fail(QH_ERR_FORMAT, "EOF reading dims");
        for (uint32_t d = 0; d < t.n_dims; d++) {
            uint64_t v;
            if (g->version == 1) {
                uint32_t v32;
                if (!r.u32(v32)) return gg_fail(QH_ERR_FORMAT, r.err);
                v = v32;
            } else if (!r.u64(v)) {
                return gg_fail(QH_ERR_FORMAT, r.err);
            }
            t.dims.push_back(v);
        }
        if (!r.u32(t.type) || !r.u64(t.offset)) return gg_fail(QH_ERR_FORMAT, r.err);
        g->by_name[t.name] = (int64_t)g->tensors.size();  // a repeated name maps to the last (tensor_map)
        g->tensors.push_back(std::move(t));
    }
    // general.alignment as u32 (Uint32 or Int32), default 32
    auto it = g->kv.find("general.alignment");
    if (it != g->kv.end() && (it->second.type == 4 || it->second.type == 5)) g->alignment = (uint32_t)it->second.u;
    if (g->alignment == 0) return gg_fail(QH_ERR_FORMAT, "general.alignment is 0");
    uint64_t pos = r.pos;
    if (pos % g->alignment) pos += g->alignment - pos % g->alignment;
    g->data_offset = pos;
    return QH_OK;
}

static uint64_t gg_elems(const GTensor& t) {
    uint64_t n = 1;
    for (uint64_t d : t.dims) n *= d;
    return n;
}

extern "C" {

int hip_gguf_open(const char* path, qh_gguf** out) {
    if (!path || !out) return QH_ERR_NULL;
    *out = nullptr;
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return gg_fail(QH_ERR_IO, std::string("Cannot open ") + path);
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return gg_fail(QH_ERR_IO, std::string("Cannot stat ") + path);
    }
    qh_gguf* g = new qh_gguf();
    g->size = (size_t)st.st_size;
    if (g->size) {
        g->map = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (g->map == MAP_FAILED) {
            g->map = nullptr;
            close(fd);
            delete g;
            return gg_fail(QH_ERR_IO, "mmap failed");
        }
    }
    close(fd);
    const int rc = gg_parse(g);
    if (rc) {
        delete g;
        return rc;
    }
    *out = g;
    return QH_OK;
}

void hip_gguf_close(qh_gguf* g) { delete g; }

uint32_t hip_gguf_version(const qh_gguf* g) { return g ? g->version : 0; }
uint64_t hip_gguf_data_offset(const qh_gguf* g) { return g ? g->data_offset : 0; }
uint64_t hip_gguf_alignment(const qh_gguf* g) { return g ? g->alignment : 0; }
int64_t hip_gguf_tensor_count(const qh_gguf* g) { return g ? (int64_t)g->tensors.size() : -1; }
int64_t hip_gguf_kv_count(const qh_gguf* g) { return g ? (int64_t)g->keys.size() : -1; }

const char* hip_gguf_kv_key(const qh_gguf* g, int64_t i) {
    return g && i >= 0 && i < (int64_t)g->keys.size() ? g->keys[(size_t)i].c_str() : nullptr;
}

// Value type of a key (0..12 as in the file), -1 when absent; arrays also give
// their element type and count.
int hip_gguf_kv_type(const qh_gguf* g, const char* key, uint32_t* elem_type, uint64_t* count) {
    if (!g || !key) return -1;
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return -1;
    if (elem_type) *elem_type = it->second.elem;
    if (count) *count = it->second.type == 9 ? it->second.count : 1;
    return (int)it->second.type;
}

int hip_gguf_get_u32(const qh_gguf* g, const char* key, uint32_t* v) {
    if (!g || !key || !v) return QH_ERR_NULL;
    auto it = g->kv.find(key);
    if (it == g->kv.end() || (it->second.type != 4 && it->second.type != 5)) return QH_ERR_RANGE;
    *v = (uint32_t)it->second.u;
    return QH_OK;
}

int hip_gguf_get_u64(const qh_gguf* g, const char* key, uint64_t* v) {
    if (!g || !key || !v) return QH_ERR_NULL;
    auto it = g->kv.find(key);
    if (it == g->kv.end() || (it->second.type != 10 && it->second.type != 4)) return QH_ERR_RANGE;
    *v = it->second.u;
    return QH_OK;
}

// Any integer or bool scalar, sign-extended for the signed types.
int hip_gguf_get_i64(const qh_gguf* g, const char* key, int64_t* v) {
    if (!g || !key || !v) return QH_ERR_NULL;
    auto it = g->kv.find(key);
    const uint32_t t = it == g->kv.end() ? 99u : it->second.type;
    if (t > 11 || t == 6 || t == 8 || t == 9) return QH_ERR_RANGE;
    *v = (int64_t)it->second.u;
    return QH_OK;
}

int hip_gguf_get_f32(const qh_gguf* g, const char* key, float* v) {
    if (!g || !key || !v) return QH_ERR_NULL;
    auto it = g->kv.find(key);
    if (it == g->kv.end() || it->second.type != 6) return QH_ERR_RANGE;
    *v = (float)it->second.f;
    return QH_OK;
}

int hip_gguf_get_f64(const qh_gguf* g, const char* key, double* v) {
    if (!g || !key || !v) return QH_ERR_NULL;
    auto it = g->kv.find(key);
    if (it == g->kv.end() || (it->second.type != 12 && it->second.type != 6)) return QH_ERR_RANGE;
    *v = it->second.f;
    return QH_OK;
}

// String value (not NUL-terminated in the file: *len bytes at the pointer).
const char* hip_gguf_get_str(const qh_gguf* g, const char* key, uint64_t* len) {
    if (!g || !key) return nullptr;
    auto it = g->kv.find(key);
    if (it == g->kv.end() || it->second.type != 8) return nullptr;
    if (len) *len = it->second.s.size();
    return it->second.s.c_str();
}

// Array of fixed-size elements: pointer to count little-endian elements.
const void* hip_gguf_get_array(const qh_gguf* g, const char* key, uint32_t* elem_type, uint64_t* count) {
    if (!g || !key) return nullptr;
    auto it = g->kv.find(key);
    if (it == g->kv.end() || it->second.type != 9 || it->second.elem == 8) return nullptr;
    if (elem_type) *elem_type = it->second.elem;
    if (count) *count = it->second.count;
    return it->second.raw.data();
}

// Element i of an array of strings.
const char* hip_gguf_get_array_str(const qh_gguf* g, const char* key, uint64_t i, uint64_t* len) {
    if (!g || !key) return nullptr;
    auto it = g->kv.find(key);
    if (it == g->kv.end() || it->second.type != 9 || it->second.elem != 8 || i >= it->second.strs.size())
        return nullptr;
    if (len) *len = it->second.strs[(size_t)i].size();
    return it->second.strs[(size_t)i].c_str();
}

int64_t hip_gguf_find_tensor(const qh_gguf* g, const char* name) {
    if (!g || !name) return -1;
    auto it = g->by_name.find(name);
    return it == g->by_name.end() ? -1 : it->second;
}

// TensorInfo i: name, n_dims, up to 8 dims (dims[0] fastest-varying), type, offset.
int hip_gguf_tensor_info(const qh_gguf* g, int64_t i, const char** name, uint32_t* n_dims, uint64_t* dims8,
                         uint32_t* ggml_type, uint64_t* offset) {
    if (!g) return QH_ERR_NULL;
    if (i < 0 || i >= (int64_t)g->tensors.size()) return QH_ERR_RANGE;
    const GTensor& t = g->tensors[(size_t)i];
    if (name) *name = t.name.c_str();
    if (n_dims) *n_dims = t.n_dims;
    if (dims8)
        for (uint32_t d = 0; d < 8; d++) dims8[d] = d < t.n_dims ? t.dims[d] : 1;
    if (ggml_type) *ggml_type = t.type;
    if (offset) *offset = t.offset;
    return QH_OK;
}

// GgufFile::tensor_data (src/gguf.rs:116-121): the tensor's bytes in the map,
// ggml_type_size(type, n_elems) of them.  Errors: unsupported type (the
// reference panics) or a range past the end of the file.
const void* hip_gguf_tensor_data(const qh_gguf* g, int64_t i, size_t* bytes) {
    if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return nullptr;
    const GTensor& t = g->tensors[(size_t)i];
    const uint64_t n = gg_elems(t);
    const size_t b = qh_type_size(t.type, (size_t)n);
    if (b == 0 && n != 0) {
        gg_fail(QH_ERR_TYPE, "unsupported ggml_type: " + std::to_string(t.type));
        return nullptr;
    }
    const uint64_t start = g->data_offset + t.offset;
    if (start > g->size || b > g->size - start) {
        gg_fail(QH_ERR_RANGE, "tensor " + t.name + " runs past the end of the file");
        return nullptr;
    }
    if (bytes) *bytes = b;
    return static_cast<const uint8_t*>(g->map) + start;
}

// Upload tensor i to a new device buffer (hip_alloc; free with hip_drop).
int hip_gguf_upload(const qh_gguf* g, int64_t i, void** d_ptr, size_t* bytes) {
    if (!g || !d_ptr) return QH_ERR_NULL;
    *d_ptr = nullptr;
    size_t b = 0;
    const void* h = hip_gguf_tensor_data(g, i, &b);
    if (!h) return i < 0 || i >= (int64_t)g->tensors.size() ? QH_ERR_RANGE : QH_ERR_FORMAT;
    void* d = nullptr;
    hipError_t e = hipMalloc(&d, b ? b : 1);
    if (e != hipSuccess) return gg_fail(QH_ERR_HIP, std::string("hipMalloc: ") + hipGetErrorString(e));
    e = hipMemcpy(d, h, b, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(d);
        return gg_fail(QH_ERR_HIP, std::string("hipMemcpy: ") + hipGetErrorString(e));
    }
    *d_ptr = d;
    if (bytes) *bytes = b;
    return QH_OK;
}

// ---------------------------------------------------------------- writer

qh_gguf_writer* hip_gguf_writer_new(void) { return new qh_gguf_writer(); }
void hip_gguf_writer_free(qh_gguf_writer* w) { delete w; }

// Scalar value of type 0..7, 10..12 from 8 little-endian bytes (only the low
// bytes of the type's size are used).
int hip_gguf_writer_kv_scalar(qh_gguf_writer* w, const char* key, uint32_t type, const void* le8) {
    if (!w || !key || !le8) return QH_ERR_NULL;
    if (type > 12 || type == 8 || type == 9) return QH_ERR_RANGE;
    GValue v;
    v.type = type;
    memcpy(&v.u, le8, 8);
    if (type == 6) {
        float f;
        memcpy(&f, le8, 4);
        v.f = f;
    }
    if (!strcmp(key, "general.alignment") && (type == 4 || type == 5)) w->alignment = (uint32_t)v.u;
    w->kv.emplace_back(key, std::move(v));
    return QH_OK;
}

int hip_gguf_writer_kv_str(qh_gguf_writer* w, const char* key, const char* s, uint64_t len) {
    if (!w || !key || (!s && len)) return QH_ERR_NULL;
    GValue v;
    v.type = 8;
    v.s.assign(s ? s : "", (size_t)len);
    w->kv.emplace_back(key, std::move(v));
    return QH_OK;
}

// Array of count fixed-size elements (elem_type 0..7, 10..12).
int hip_gguf_writer_kv_array(qh_gguf_writer* w, const char* key, uint32_t elem_type, const void* data,
                             uint64_t count) {
    if (!w || !key || (!data && count)) return QH_ERR_NULL;
    if (elem_type > 12 || elem_type == 8 || elem_type == 9) return QH_ERR_RANGE;
    GValue v;
    v.type = 9;
    v.elem = elem_type;
    v.count = count;
    const uint8_t* p = static_cast<const uint8_t*>(data);
    v.raw.assign(p, p + count * (uint64_t)kScalarSize[elem_type]);
    w->kv.emplace_back(key, std::move(v));
    return QH_OK;
}

// Array of count strings (pointers and byte lengths).
int hip_gguf_writer_kv_array_str(qh_gguf_writer* w, const char* key, const char* const* strs, const uint64_t* lens,
                                 uint64_t count) {
    if (!w || !key || (count && (!strs || !lens))) return QH_ERR_NULL;
    GValue v;
    v.type = 9;
    v.elem = 8;
    v.count = count;
    for (uint64_t i = 0; i < count; i++) v.strs.emplace_back(strs[i] ? strs[i] : "", (size_t)lens[i]);
    w->kv.emplace_back(key, std::move(v));
    return QH_OK;
}

// Tensor with n_dims dims (dims[0] fastest-varying) of a ggml type; the data
// (hip_type_size(type, product of dims) bytes, host memory) must stay valid
// until hip_gguf_writer_write.
int hip_gguf_writer_tensor(qh_gguf_writer* w, const char* name, uint32_t n_dims, const uint64_t* dims,
                           uint32_t ggml_type, const void* data) {
    if (!w || !name || (n_dims && !dims)) return QH_ERR_NULL;
    uint64_t n = 1;
    for (uint32_t d = 0; d < n_dims; d++) n *= dims[d];
    const size_t b = qh_type_size(ggml_type, (size_t)n);
    if (b == 0 && n != 0) return QH_ERR_TYPE;
    if (b && !data) return QH_ERR_NULL;
    w->tensors.push_back({name, std::vector<uint64_t>(dims, dims + n_dims), ggml_type,
                          static_cast<const uint8_t*>(data), b});
    return QH_OK;
}

int hip_gguf_writer_write(const qh_gguf_writer* w, const char* path) {
    if (!w || !path) return QH_ERR_NULL;
    if (w->alignment == 0) return gg_fail(QH_ERR_RANGE, "general.alignment is 0");
    std::vector<uint8_t> h;
    auto put = [&](const void* p, size_t k) { h.insert(h.end(), (const uint8_t*)p, (const uint8_t*)p + k); };
    auto put32 = [&](uint32_t v) { put(&v, 4); };
    auto put64 = [&](uint64_t v) { put(&v, 8); };
    auto putstr = [&](const std::string& s) { put64(s.size()); put(s.data(), s.size()); };
    put32(0x46554747u);
    put32(3);
    put64(w->tensors.size());
    put64(w->kv.size());
    for (const auto& kv : w->kv) {
        putstr(kv.first);
        const GValue& v = kv.second;
        put32(v.type);
        if (v.type == 8) {
            putstr(v.s);
        } else if (v.type == 9) {
            put32(v.elem);
            put64(v.count);
            if (v.elem == 8)
                for (const auto& s : v.strs) putstr(s);
            else
                put(v.raw.data(), v.raw.size());
        } else {
            put(&v.u, (size_t)kScalarSize[v.type]);
        }
    }
    const uint64_t A = w->alignment;
    uint64_t off = 0;
    std::vector<uint64_t> offs;
    for (const auto& t : w->tensors) {
        offs.push_back(off);
        off += (t.bytes + A - 1) / A * A;
    }
    for (size_t i = 0; i < w->tensors.size(); i++) {
        const auto& t = w->tensors[i];
        putstr(t.name);
        put32((uint32_t)t.dims.size());
        for (uint64_t d : t.dims) put64(d);
        put32(t.type);
        put64(offs[i]);
    }
    h.resize((h.size() + A - 1) / A * A, 0);
    FILE* f = fopen(path, "wb");
    if (!f) return gg_fail(QH_ERR_IO, std::string("Cannot create ") + path);
    bool ok = fwrite(h.data(), 1, h.size(), f) == h.size();
    static const uint8_t zeros[4096] = {};
    for (const auto& t : w->tensors) {
        if (!ok) break;
        ok = t.bytes == 0 || fwrite(t.data, 1, t.bytes, f) == t.bytes;
        uint64_t pad = (A - t.bytes % A) % A;
        while (ok && pad) {
            const size_t k = pad < sizeof zeros ? (size_t)pad : sizeof zeros;
            ok = fwrite(zeros, 1, k, f) == k;
            pad -= k;
        }
    }
    if (fclose(f) != 0) ok = false;
    return ok ? QH_OK : gg_fail(QH_ERR_IO, std::string("write failed: ") + path);
}

}  // extern "C"
