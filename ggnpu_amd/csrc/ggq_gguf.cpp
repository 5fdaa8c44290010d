// ggq_gguf.cpp -- GGUF v3 reader over mmap (see include/ggq_gguf.h).
//
// The whole file is mapped read-only and parsed in place through a
// bounds-checked cursor; metadata values and tensor infos are indexed, and
// tensor data is never copied on the host.  Format (the reference reads the
// same layout, src/gguf/gguf.cpp:148-372):
//   u32 magic "GGUF", u32 version, u64 n_tensors, u64 n_kv
//   n_kv x { string key, u32 type, value }    string = u64 len + bytes
//   n_tensors x { string name, u32 n_dims, u64 dims[n_dims], u32 ggml_type, u64 offset }
//   padding to general.alignment (default 32), then the tensor data.
#include "../../include/ggq_gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

// ggml type table: values per block and bytes per block, indexed by type id
// (GGML's numbering; the reference's table is src/gguf/tensor.cpp:18-38).
struct TypeInfo {
    uint32_t blck, bytes;
};
constexpr TypeInfo kTypes[] = {
    {1, 4},     {1, 2},      {32, 18},    {32, 20},   {0, 0},    {0, 0},     // F32 F16 Q4_0 Q4_1 - -
    {32, 22},   {32, 24},    {32, 34},    {32, 36},   {256, 84}, {256, 110}, // Q5_0 Q5_1 Q8_0 Q8_1 Q2_K Q3_K
    {256, 144}, {256, 176},  {256, 210},  {256, 292}, {256, 66}, {256, 74},  // Q4_K Q5_K Q6_K Q8_K IQ2_XXS IQ2_XS
    {256, 98},  {256, 50},   {32, 18},    {256, 110}, {256, 82}, {256, 136}, // IQ3_XXS IQ1_S IQ4_NL IQ3_S IQ2_S IQ4_XS
    {1, 1},     {1, 2},      {1, 4},      {1, 8},     {1, 8},    {256, 56},  // I8 I16 I32 I64 F64 IQ1_M
    {1, 2},     {32, 18},                                                    // BF16 Q4_0_4_4
};
constexpr uint32_t kNumTypes = sizeof(kTypes) / sizeof(kTypes[0]);

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" little-endian
constexpr uint64_t kMaxKey = 1024, kMaxName = 1024, kMaxString = 64ull << 20;

size_t scalar_size(uint32_t t) {
    switch (t) {
    case GGQ_GGUF_UINT8: case GGQ_GGUF_INT8: case GGQ_GGUF_BOOL: return 1;
    case GGQ_GGUF_UINT16: case GGQ_GGUF_INT16: return 2;
    case GGQ_GGUF_UINT32: case GGQ_GGUF_INT32: case GGQ_GGUF_FLOAT32: return 4;
    case GGQ_GGUF_UINT64: case GGQ_GGUF_INT64: case GGQ_GGUF_FLOAT64: return 8;
    default: return 0;
    }
}

thread_local std::string g_open_error;

struct Cursor {
    const uint8_t* base;
    uint64_t size, pos = 0;
    bool ok = true;
    bool need(uint64_t n) {
        if (!ok || n > size - pos) ok = false;
        return ok;
    }
    template <typename T> T get() {
        T v{};
        if (need(sizeof(T))) {
            std::memcpy(&v, base + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    // A GGUF string: returns its position and length, advances past it.
    bool str(uint64_t max, uint64_t* at, uint64_t* len) {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > max || !need(n)) return ok = false;
        *at = pos;
        *len = n;
        pos += n;
        return true;
    }
    bool skip(uint64_t n) {
        if (!need(n)) return false;
        pos += n;
        return true;
    }
};

}  // namespace

struct ggq_gguf {
    struct KV {
        std::string key;
        uint32_t type = 0;
        uint64_t at = 0;  // file offset of the value (after the type field)
        uint64_t len = 0;  // string: bytes
        std::string sval;  // string value (NUL-terminated copy)
        uint32_t elem_type = 0;  // array
        uint64_t count = 0;
        uint64_t elems_at = 0;  // array: offset of the first element
        std::vector<uint64_t> str_at;  // string arrays: offsets of each element's length field
    };
    struct Tensor {
        std::string name;
        uint32_t type = 0;
        int32_t n_dims = 0;
        int64_t dims[4] = {1, 1, 1, 1};
        uint64_t offset = 0, nbytes = 0;
    };
    int fd = -1;
    const uint8_t* map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32, data_offset = 0;
    std::vector<KV> kvs;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int64_t> kv_index, tensor_index;

    ~ggq_gguf() {
        if (map) munmap(const_cast<uint8_t*>(map), size);
        if (fd >= 0) close(fd);
    }
};

namespace {

int fail(ggq_gguf* g, int st, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
int fail(ggq_gguf* g, int st, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_open_error = buf;
    delete g;
    return st;
}

bool parse_value(Cursor& c, ggq_gguf::KV& kv) {
    kv.at = c.pos;
    if (kv.type == GGQ_GGUF_STRING) {
        uint64_t at, len;
        if (!c.str(kMaxString, &at, &len)) return false;
        kv.len = len;
        kv.sval.assign((const char*)c.base + at, len);
        return true;
    }
    if (kv.type == GGQ_GGUF_ARRAY) {
        kv.elem_type = c.get<uint32_t>();
        kv.count = c.get<uint64_t>();
        if (!c.ok) return false;
        kv.elems_at = c.pos;
        if (kv.elem_type == GGQ_GGUF_STRING) {
            if (kv.count > c.size / 8) return false;
            kv.str_at.reserve(kv.count);
            for (uint64_t j = 0; j < kv.count; j++) {
                kv.str_at.push_back(c.pos);
                uint64_t at, len;
                if (!c.str(kMaxString, &at, &len)) return false;
            }
            return true;
        }
        const size_t es = scalar_size(kv.elem_type);
        if (es == 0 || kv.count > (c.size - c.pos) / es) return false;  // nested arrays are not GGUF v3 metadata
        return c.skip(kv.count * es);
    }
    const size_t es = scalar_size(kv.type);
    return es != 0 && c.skip(es);
}

}  // namespace

extern "C" {

const char* ggq_gguf_last_error(void) { return g_open_error.c_str(); }

int ggq_gguf_open(const char* path, ggq_gguf** out) {
    if (!out || !path) return GGQ_INVALID_PARAM;
    *out = nullptr;
    g_open_error.clear();
    ggq_gguf* g = new (std::nothrow) ggq_gguf;
    if (!g) return GGQ_OUT_OF_MEMORY;
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) return fail(g, GGQ_NOT_FOUND, "cannot open %s", path);
    struct stat st;
    if (fstat(g->fd, &st) != 0) return fail(g, GGQ_NOT_FOUND, "cannot stat %s", path);
    g->size = (uint64_t)st.st_size;
    if (g->size < 24) return fail(g, GGQ_INVALID_PARAM, "file too small for a GGUF header");
    void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) return fail(g, GGQ_ERROR, "mmap failed");
    g->map = (const uint8_t*)m;

    Cursor c{g->map, g->size};
    const uint32_t magic = c.get<uint32_t>();
    g->version = c.get<uint32_t>();
    const uint64_t n_tensors = c.get<uint64_t>();
    const uint64_t n_kv = c.get<uint64_t>();
    if (magic != kMagic) return fail(g, GGQ_INVALID_PARAM, "bad magic 0x%08x", magic);
    if (g->version != 3) return fail(g, GGQ_INVALID_PARAM, "GGUF version %u (only 3 is read)", g->version);
    // Every KV and tensor info takes at least 12 bytes.
    if (n_kv > g->size / 12 || n_tensors > g->size / 12) return fail(g, GGQ_INVALID_PARAM, "implausible counts");

    g->kvs.resize(n_kv);
    for (uint64_t i = 0; i < n_kv; i++) {
        ggq_gguf::KV& kv = g->kvs[i];
        uint64_t at, len;
        if (!c.str(kMaxKey, &at, &len)) return fail(g, GGQ_INVALID_PARAM, "bad key %llu", (unsigned long long)i);
        kv.key.assign((const char*)g->map + at, len);
        kv.type = c.get<uint32_t>();
        if (!c.ok || !parse_value(c, kv))
            return fail(g, GGQ_INVALID_PARAM, "bad value of %s (type %u)", kv.key.c_str(), kv.type);
        g->kv_index[kv.key] = (int64_t)i;
    }
    auto al = g->kv_index.find("general.alignment");
    if (al != g->kv_index.end()) {
        const ggq_gguf::KV& kv = g->kvs[al->second];
        int64_t a = 0;
        if (kv.type == GGQ_GGUF_UINT32 || kv.type == GGQ_GGUF_INT32) {
            uint32_t v;
            std::memcpy(&v, g->map + kv.at, 4);
            a = v;
        } else if (kv.type == GGQ_GGUF_UINT64) {
            uint64_t v;
            std::memcpy(&v, g->map + kv.at, 8);
            a = (int64_t)(v > (1u << 30) ? 0 : v);
        }
        if (a <= 0 || (a & (a - 1))) return fail(g, GGQ_INVALID_PARAM, "general.alignment must be a power of two");
        g->alignment = (uint64_t)a;
    }

    g->tensors.resize(n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        ggq_gguf::Tensor& t = g->tensors[i];
        uint64_t at, len;
        if (!c.str(kMaxName, &at, &len)) return fail(g, GGQ_INVALID_PARAM, "bad tensor name %llu", (unsigned long long)i);
        t.name.assign((const char*)g->map + at, len);
        const uint32_t nd = c.get<uint32_t>();
        if (!c.ok || nd < 1 || nd > 4) return fail(g, GGQ_INVALID_PARAM, "tensor %s: %u dims", t.name.c_str(), nd);
        t.n_dims = (int32_t)nd;
        uint64_t elems = 1;
        for (uint32_t d = 0; d < nd; d++) {
            const uint64_t v = c.get<uint64_t>();
            if (!c.ok || v == 0 || v > (1ull << 40) || elems > (1ull << 62) / v)
                return fail(g, GGQ_INVALID_PARAM, "tensor %s: bad dims", t.name.c_str());
            t.dims[d] = (int64_t)v;
            elems *= v;
        }
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        if (!c.ok) return fail(g, GGQ_INVALID_PARAM, "tensor %s: truncated info", t.name.c_str());
        if (t.type < kNumTypes && kTypes[t.type].blck) {
            const TypeInfo ti = kTypes[t.type];
            if ((uint64_t)t.dims[0] % ti.blck)
                return fail(g, GGQ_INVALID_PARAM, "tensor %s: row of %lld not a multiple of the block", t.name.c_str(),
                            (long long)t.dims[0]);
            t.nbytes = elems / ti.blck * ti.bytes;
        }
        if (g->tensor_index.count(t.name)) return fail(g, GGQ_INVALID_PARAM, "duplicate tensor %s", t.name.c_str());
        g->tensor_index[t.name] = (int64_t)i;
    }
    g->data_offset = (c.pos + g->alignment - 1) / g->alignment * g->alignment;
    if (g->data_offset > g->size) return fail(g, GGQ_INVALID_PARAM, "data section past end of file");
    const uint64_t data_size = g->size - g->data_offset;
    for (const ggq_gguf::Tensor& t : g->tensors)
        if (t.offset > data_size || t.nbytes > data_size - t.offset)
            return fail(g, GGQ_INVALID_PARAM, "tensor %s extends past the end of the file", t.name.c_str());
    *out = g;
    return GGQ_OK;
}

void ggq_gguf_close(ggq_gguf* g) { delete g; }

uint32_t ggq_gguf_version(const ggq_gguf* g) { return g ? g->version : 0; }
uint64_t ggq_gguf_alignment(const ggq_gguf* g) { return g ? g->alignment : 0; }
uint64_t ggq_gguf_data_offset(const ggq_gguf* g) { return g ? g->data_offset : 0; }
uint64_t ggq_gguf_file_size(const ggq_gguf* g) { return g ? g->size : 0; }
int64_t ggq_gguf_n_tensors(const ggq_gguf* g) { return g ? (int64_t)g->tensors.size() : 0; }
int64_t ggq_gguf_n_kv(const ggq_gguf* g) { return g ? (int64_t)g->kvs.size() : 0; }

int ggq_gguf_tensor_at(const ggq_gguf* g, int64_t i, ggq_gguf_tensor* out) {
    if (!g || !out || i < 0 || i >= (int64_t)g->tensors.size()) return GGQ_INVALID_PARAM;
    const ggq_gguf::Tensor& t = g->tensors[i];
    out->name = t.name.c_str();
    out->type = t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; d++) out->dims[d] = t.dims[d];
    out->offset = t.offset;
    out->nbytes = t.nbytes;
    out->data = g->map + g->data_offset + t.offset;
    return GGQ_OK;
}

int64_t ggq_gguf_find_tensor(const ggq_gguf* g, const char* name) {
    if (!g || !name) return -1;
    auto it = g->tensor_index.find(name);
    return it == g->tensor_index.end() ? -1 : it->second;
}

const char* ggq_gguf_kv_key(const ggq_gguf* g, int64_t i) {
    if (!g || i < 0 || i >= (int64_t)g->kvs.size()) return nullptr;
    return g->kvs[i].key.c_str();
}

int64_t ggq_gguf_find_kv(const ggq_gguf* g, const char* key) {
    if (!g || !key) return -1;
    auto it = g->kv_index.find(key);
    return it == g->kv_index.end() ? -1 : it->second;
}

uint32_t ggq_gguf_kv_type(const ggq_gguf* g, int64_t i) {
    if (!g || i < 0 || i >= (int64_t)g->kvs.size()) return UINT32_MAX;
    return g->kvs[i].type;
}

int ggq_gguf_kv_int(const ggq_gguf* g, int64_t i, int64_t* out) {
    if (!g || !out || i < 0 || i >= (int64_t)g->kvs.size()) return GGQ_INVALID_PARAM;
    const ggq_gguf::KV& kv = g->kvs[i];
    const uint8_t* p = g->map + kv.at;
    switch (kv.type) {
    case GGQ_GGUF_UINT8: case GGQ_GGUF_BOOL: *out = p[0]; return GGQ_OK;
    case GGQ_GGUF_INT8: *out = (int8_t)p[0]; return GGQ_OK;
    case GGQ_GGUF_UINT16: { uint16_t v; std::memcpy(&v, p, 2); *out = v; return GGQ_OK; }
    case GGQ_GGUF_INT16: { int16_t v; std::memcpy(&v, p, 2); *out = v; return GGQ_OK; }
    case GGQ_GGUF_UINT32: { uint32_t v; std::memcpy(&v, p, 4); *out = v; return GGQ_OK; }
    case GGQ_GGUF_INT32: { int32_t v; std::memcpy(&v, p, 4); *out = v; return GGQ_OK; }
    case GGQ_GGUF_UINT64: case GGQ_GGUF_INT64: { int64_t v; std::memcpy(&v, p, 8); *out = v; return GGQ_OK; }
    default: return GGQ_INVALID_PARAM;
    }
}

int ggq_gguf_kv_uint(const ggq_gguf* g, int64_t i, uint64_t* out) {
    if (!g || !out || i < 0 || i >= (int64_t)g->kvs.size()) return GGQ_INVALID_PARAM;
    if (g->kvs[i].type == GGQ_GGUF_UINT64) {
        std::memcpy(out, g->map + g->kvs[i].at, 8);
        return GGQ_OK;
    }
    int64_t v;
    const int st = ggq_gguf_kv_int(g, i, &v);
    if (st != GGQ_OK || v < 0) return GGQ_INVALID_PARAM;
    *out = (uint64_t)v;
    return GGQ_OK;
}

int ggq_gguf_kv_float(const ggq_gguf* g, int64_t i, double* out) {
    if (!g || !out || i < 0 || i >= (int64_t)g->kvs.size()) return GGQ_INVALID_PARAM;
    const ggq_gguf::KV& kv = g->kvs[i];
    if (kv.type == GGQ_GGUF_FLOAT32) {
        float v;
        std::memcpy(&v, g->map + kv.at, 4);
        *out = v;
        return GGQ_OK;
    }
    if (kv.type == GGQ_GGUF_FLOAT64) {
        std::memcpy(out, g->map + kv.at, 8);
        return GGQ_OK;
    }
    return GGQ_INVALID_PARAM;
}

int ggq_gguf_kv_str(const ggq_gguf* g, int64_t i, const char** s, uint64_t* len) {
    if (!g || !s || i < 0 || i >= (int64_t)g->kvs.size() || g->kvs[i].type != GGQ_GGUF_STRING)
        return GGQ_INVALID_PARAM;
    *s = g->kvs[i].sval.c_str();
    if (len) *len = g->kvs[i].len;
    return GGQ_OK;
}

int ggq_gguf_kv_array(const ggq_gguf* g, int64_t i, uint32_t* elem_type, uint64_t* n, const void** data) {
    if (!g || i < 0 || i >= (int64_t)g->kvs.size() || g->kvs[i].type != GGQ_GGUF_ARRAY) return GGQ_INVALID_PARAM;
    const ggq_gguf::KV& kv = g->kvs[i];
    if (elem_type) *elem_type = kv.elem_type;
    if (n) *n = kv.count;
    if (data) *data = kv.elem_type == GGQ_GGUF_STRING ? nullptr : (const void*)(g->map + kv.elems_at);
    return GGQ_OK;
}

int ggq_gguf_kv_array_str(const ggq_gguf* g, int64_t i, uint64_t j, const char** s, uint64_t* len) {
    if (!g || !s || !len || i < 0 || i >= (int64_t)g->kvs.size()) return GGQ_INVALID_PARAM;
    const ggq_gguf::KV& kv = g->kvs[i];
    if (kv.type != GGQ_GGUF_ARRAY || kv.elem_type != GGQ_GGUF_STRING || j >= kv.count) return GGQ_INVALID_PARAM;
    uint64_t n;
    std::memcpy(&n, g->map + kv.str_at[j], 8);
    *s = (const char*)g->map + kv.str_at[j] + 8;
    *len = n;
    return GGQ_OK;
}

int ggq_gguf_upload(ggq_ctx* ctx, const ggq_gguf* g, const char* name, ggq_weight** out) {
    if (!ctx || !g || !name || !out) return GGQ_INVALID_PARAM;
    *out = nullptr;
    const int64_t i = ggq_gguf_find_tensor(g, name);
    if (i < 0) return GGQ_NOT_FOUND;
    const ggq_gguf::Tensor& t = g->tensors[i];
    int64_t N = 1;
    for (int d = 1; d < t.n_dims; d++) N *= t.dims[d];
    return ggq_weight_upload(ctx, g->map + g->data_offset + t.offset, t.type, N, t.dims[0], out);
}

}  // extern "C"
