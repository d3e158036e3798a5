// GGUF container reader and the Llama loader on top of it (host code).
//
// Replaces GGUFFile (Sources/AlpacaModels/GGUF/GGUFFile.swift:11-217) and
// LlamaLoader (Sources/AlpacaModels/Llama/LlamaLoader.swift:29-126) for a host
// that drives this library through its C ABI: a file is mapped read-only and
// validated without trusting any length field, then its tensors are handed to
// ahip_model_create straight from the mapping (one copy, host mapping -> HBM).
//
// Validation follows the reference rule for rule, in the same order, so every
// file it rejects is rejected here with the same GGUFError case
// (GGUFError.swift:5-19, reported as AHIP_ERR_GGUF plus
// ahip_gguf_last_error_kind()):
//   header: magic "GGUF", version 2 or 3 (a version whose low 16 bits are 0 is
//     a big-endian file), counts bounded by the limits and by the bytes left
//     (a metadata entry needs >= 13 bytes, a tensor record >= 24);
//   metadata: keys <= 4 KiB and unique, value types 0-12, booleans 0/1,
//     strings <= 16 MiB, arrays <= 2^24 elements, nested at most 2 deep, and
//     no longer than the bytes left; general.alignment a power of two <= 1 MiB;
//   tensors: names <= 4 KiB and unique, 1-4 dimensions each in [1, 2^31),
//     element and byte counts without overflow, a known GGML type whose block
//     divides the row, an aligned offset whose range lies inside the file, and
//     no two ranges overlapping.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "../../include/alpaca_hip.h"

// runtime.cpp: the thread-local error message and the config checks of ahip_model_create
int ahip_fail(int code, const std::string& msg);
int ahip_validate_config(const ahip_llama_config* c);

namespace {

thread_local int g_kind = 0;

struct GError {
    int kind;
    std::string msg;
};
[[noreturn]] void gthrow(int kind, std::string msg) { throw GError{kind, std::move(msg)}; }

int report(const GError& e) {
    g_kind = e.kind;
    return ahip_fail(AHIP_ERR_GGUF, e.msg);
}

// GGUFFile.Limits (GGUFFile.swift:13-21).
constexpr uint64_t kMaxMetadata = 1u << 16, kMaxTensors = 1u << 16, kMaxString = 1u << 24, kMaxArray = 1u << 24,
                   kMaxName = 1u << 12;
constexpr int kMaxArrayDepth = 2, kMaxDims = 4;

// GGML storage types: (elements, bytes) per block (GGUFTypes.swift:8-31).
bool block_layout(uint32_t t, int64_t& elems, int64_t& bytes) {
    switch (t) {
    case AHIP_GGML_F32: elems = 1, bytes = 4; return true;
    case AHIP_GGML_F16: case AHIP_GGML_BF16: elems = 1, bytes = 2; return true;
    case AHIP_GGML_Q4_0: elems = 32, bytes = 18; return true;
    case AHIP_GGML_Q4_1: elems = 32, bytes = 20; return true;
    case AHIP_GGML_Q5_0: elems = 32, bytes = 22; return true;
    case AHIP_GGML_Q5_1: elems = 32, bytes = 24; return true;
    case AHIP_GGML_Q8_0: elems = 32, bytes = 34; return true;
    case AHIP_GGML_Q8_1: elems = 32, bytes = 36; return true;
    case AHIP_GGML_Q2_K: elems = 256, bytes = 84; return true;
    case AHIP_GGML_Q3_K: elems = 256, bytes = 110; return true;
    case AHIP_GGML_Q4_K: elems = 256, bytes = 144; return true;
    case AHIP_GGML_Q5_K: elems = 256, bytes = 176; return true;
    case AHIP_GGML_Q6_K: elems = 256, bytes = 210; return true;
    case AHIP_GGML_Q8_K: elems = 256, bytes = 292; return true;
    default: return false;
    }
}

// The library dtype that executes a GGML type directly (GGMLType.nativeDType, GGUFTypes.swift:34-43).
int native_dtype(uint32_t t) {
    switch (t) {
    case AHIP_GGML_F32: return AHIP_F32;
    case AHIP_GGML_F16: return AHIP_F16;
    case AHIP_GGML_Q8_0: return AHIP_Q8_0;
    case AHIP_GGML_Q4_0: return AHIP_Q4_0;
    default: return -1;
    }
}

// Bounds-checked little-endian cursor (ByteReader.swift:5-38).  The host is
// little-endian (x86-64), so fields are copied as they lie.
struct Reader {
    const uint8_t* base;
    size_t count;
    size_t pos = 0;
    size_t remaining() const { return count - pos; }
    template <typename T>
    T read(const std::string& what) {
        if (remaining() < sizeof(T))
            gthrow(AHIP_GGUF_TRUNCATED, "file truncated while reading " + what + " at offset " + std::to_string(pos));
        T v;
        std::memcpy(&v, base + pos, sizeof(T));
        pos += sizeof(T);
        return v;
    }
    std::string read_string(const std::string& what, uint64_t max_len) {
        const uint64_t len = read<uint64_t>(what + " length");
        if (len > max_len)
            gthrow(AHIP_GGUF_LIMIT_EXCEEDED,
                   "GGUF limit exceeded: " + what + " length " + std::to_string(len) + " > " + std::to_string(max_len));
        if (remaining() < len)
            gthrow(AHIP_GGUF_TRUNCATED, "file truncated while reading " + what + " at offset " + std::to_string(pos));
        std::string s(reinterpret_cast<const char*>(base + pos), (size_t)len);
        pos += (size_t)len;
        return s;
    }
};

// GGUFValue (GGUFTypes.swift:46-70): the type id as written, and its payload.
struct Value {
    uint32_t type = 0;
    uint64_t u = 0;  // types 0, 2, 4, 10, and 7 (bool)
    int64_t i = 0;   // types 1, 3, 5, 11
    double f = 0;    // types 6, 12
    std::string s;   // type 8
    uint32_t elem_type = 0;
    std::vector<Value> items;  // type 9
    bool is_uint() const { return type == 0 || type == 2 || type == 4 || type == 10; }
    bool is_int() const { return type == 1 || type == 3 || type == 5 || type == 11; }
    bool is_float() const { return type == 6 || type == 12; }
    // GGUFValue.asInt: integers that fit Int64 exactly
    bool as_int(int64_t& v) const {
        if (is_uint() && u <= (uint64_t)INT64_MAX) return v = (int64_t)u, true;
        if (is_int()) return v = i, true;
        return false;
    }
    // GGUFValue.asDouble: floats and integers
    bool as_double(double& v) const {
        if (is_float()) return v = f, true;
        if (is_uint()) return v = (double)u, true;
        if (is_int()) return v = (double)i, true;
        return false;
    }
};

Value read_value(Reader& r, uint32_t type, const std::string& key, int depth) {
    Value v;
    v.type = type;
    switch (type) {
    case 0: v.u = r.read<uint8_t>(key); break;
    case 1: v.i = r.read<int8_t>(key); break;
    case 2: v.u = r.read<uint16_t>(key); break;
    case 3: v.i = r.read<int16_t>(key); break;
    case 4: v.u = r.read<uint32_t>(key); break;
    case 5: v.i = r.read<int32_t>(key); break;
    case 6: {
        const uint32_t bits = r.read<uint32_t>(key);
        float f;
        std::memcpy(&f, &bits, 4);
        v.f = f;
        break;
    }
    case 7: {
        const uint8_t b = r.read<uint8_t>(key);
        if (b > 1) gthrow(AHIP_GGUF_MALFORMED, "malformed GGUF: bool '" + key + "' has value " + std::to_string(b));
        v.u = b;
        break;
    }
    case 8: v.s = r.read_string(key, kMaxString); break;
    case 9: {
        if (depth >= kMaxArrayDepth) gthrow(AHIP_GGUF_LIMIT_EXCEEDED, "GGUF limit exceeded: array nesting in '" + key + "'");
        v.elem_type = r.read<uint32_t>("array type of " + key);
        const uint64_t n = r.read<uint64_t>("array length of " + key);
        if (n > kMaxArray)
            gthrow(AHIP_GGUF_LIMIT_EXCEEDED, "GGUF limit exceeded: array '" + key + "' length " + std::to_string(n));
        // every element takes at least one byte, so the bytes left bound the real count
        if (n > r.remaining())
            gthrow(AHIP_GGUF_TRUNCATED, "file truncated while reading array '" + key + "' at offset " + std::to_string(r.pos));
        v.items.reserve((size_t)n);
        for (uint64_t k = 0; k < n; k++) v.items.push_back(read_value(r, v.elem_type, key, depth + 1));
        break;
    }
    case 10: v.u = r.read<uint64_t>(key); break;
    case 11: v.i = r.read<int64_t>(key); break;
    case 12: {
        const uint64_t bits = r.read<uint64_t>(key);
        std::memcpy(&v.f, &bits, 8);
        break;
    }
    default:
        gthrow(AHIP_GGUF_MALFORMED, "malformed GGUF: metadata '" + key + "' has unknown value type " + std::to_string(type));
    }
    return v;
}

}  // namespace

struct ahip_gguf {
    // the bytes: a read-only private mapping of the file, or an owned copy
    const uint8_t* base = nullptr;
    size_t size = 0;
    bool mapped = false;
    std::vector<uint8_t> copy;
    uint32_t version = 0;
    int64_t alignment = 32;
    int64_t data_offset = 0;
    std::vector<std::string> keys;  // in file order
    std::map<std::string, Value> meta;
    struct Tensor {
        std::string name;
        std::vector<int64_t> dims;  // GGUF order: dims[0] varies fastest
        uint32_t type;
        int64_t offset, bytes;      // absolute file offset, byte count
    };
    std::vector<Tensor> tensors;    // in directory order
    std::map<std::string, int> index;
    ~ahip_gguf() {
        if (mapped && base) munmap(const_cast<uint8_t*>(base), size);
    }
    const Value* find(const char* key) const {
        auto it = key ? meta.find(key) : meta.end();
        return it == meta.end() ? nullptr : &it->second;
    }
    void parse();
};

// GGUFFile.init(region:limits:), GGUFFile.swift:42-131.
void ahip_gguf::parse() {
    Reader r{base, size};
    if (size < 4 || r.read<uint32_t>("magic") != 0x46554747u) gthrow(AHIP_GGUF_INVALID_MAGIC, "not a GGUF file (bad magic)");
    version = r.read<uint32_t>("version");
    if ((version & 0xFFFFu) == 0 && version != 0)
        gthrow(AHIP_GGUF_BIG_ENDIAN, "big-endian GGUF files are not supported");
    if (version != 2 && version != 3)
        gthrow(AHIP_GGUF_UNSUPPORTED_VERSION, "unsupported GGUF version " + std::to_string(version) + " (supported: 2, 3)");
    const uint64_t n_tensors = r.read<uint64_t>("tensor count");
    const uint64_t n_kv = r.read<uint64_t>("metadata count");
    if (n_kv > kMaxMetadata) gthrow(AHIP_GGUF_LIMIT_EXCEEDED, "GGUF limit exceeded: metadata entries " + std::to_string(n_kv));
    if (n_tensors > kMaxTensors) gthrow(AHIP_GGUF_LIMIT_EXCEEDED, "GGUF limit exceeded: tensor count " + std::to_string(n_tensors));
    if (n_kv > r.remaining() / 13 || n_tensors > r.remaining() / 24)
        gthrow(AHIP_GGUF_TRUNCATED, "file truncated while reading directory at offset " + std::to_string(r.pos));

    for (uint64_t k = 0; k < n_kv; k++) {
        std::string key = r.read_string("metadata key", kMaxName);
        const uint32_t type = r.read<uint32_t>("value type for " + key);
        if (meta.count(key)) gthrow(AHIP_GGUF_MALFORMED, "malformed GGUF: duplicate metadata key '" + key + "'");
        Value v = read_value(r, type, key, 0);
        keys.push_back(key);
        meta.emplace(std::move(key), std::move(v));
    }
    if (const Value* a = find("general.alignment")) {
        int64_t v;
        if (!a->as_int(v) || v <= 0 || (v & (v - 1)) || v > (1 << 20))
            gthrow(AHIP_GGUF_MALFORMED, "malformed GGUF: invalid general.alignment");
        alignment = v;
    }

    struct Raw {
        Tensor t;
        uint64_t rel;
    };
    std::vector<Raw> raws;
    std::set<std::string> seen;
    for (uint64_t k = 0; k < n_tensors; k++) {
        Raw raw;
        Tensor& t = raw.t;
        t.name = r.read_string("tensor name", kMaxName);
        if (!seen.insert(t.name).second) gthrow(AHIP_GGUF_DUPLICATE_TENSOR, "duplicate tensor '" + t.name + "'");
        const uint32_t nd = r.read<uint32_t>("dimension count of " + t.name);
        if (nd < 1 || nd > (uint32_t)kMaxDims)
            gthrow(AHIP_GGUF_MALFORMED, "malformed GGUF: tensor '" + t.name + "' has " + std::to_string(nd) + " dimensions");
        int64_t elements = 1;
        for (uint32_t d = 0; d < nd; d++) {
            const uint64_t x = r.read<uint64_t>("dimension of " + t.name);
            if (x == 0 || x > (uint64_t)INT32_MAX)
                gthrow(AHIP_GGUF_MALFORMED,
                       "malformed GGUF: tensor '" + t.name + "' has invalid dimension " + std::to_string(x));
            if (__builtin_mul_overflow(elements, (int64_t)x, &elements))
                gthrow(AHIP_GGUF_MALFORMED, "malformed GGUF: tensor '" + t.name + "' element count overflows");
            t.dims.push_back((int64_t)x);
        }
        t.type = r.read<uint32_t>("type of " + t.name);
        int64_t be, bb;
        if (!block_layout(t.type, be, bb))
            gthrow(AHIP_GGUF_UNSUPPORTED_TENSOR_TYPE,
                   "tensor '" + t.name + "' uses unsupported GGML type id " + std::to_string(t.type));
        if (t.dims[0] % be)
            gthrow(AHIP_GGUF_MALFORMED, "malformed GGUF: tensor '" + t.name + "': row length " + std::to_string(t.dims[0]) +
                                            " is not a multiple of block size " + std::to_string(be));
        if (__builtin_mul_overflow(elements / be, bb, &t.bytes))
            gthrow(AHIP_GGUF_MALFORMED, "malformed GGUF: tensor '" + t.name + "' byte size overflows");
        raw.rel = r.read<uint64_t>("offset of " + t.name);
        raws.push_back(std::move(raw));
    }

    const uint64_t aligned = ((uint64_t)r.pos + (uint64_t)alignment - 1) / (uint64_t)alignment * (uint64_t)alignment;
    if (aligned > size) gthrow(AHIP_GGUF_TRUNCATED, "file truncated while reading tensor data at offset " + std::to_string(r.pos));
    data_offset = (int64_t)aligned;

    for (Raw& raw : raws) {
        Tensor& t = raw.t;
        if (raw.rel % (uint64_t)alignment)
            gthrow(AHIP_GGUF_MALFORMED, "malformed GGUF: tensor '" + t.name + "' offset " + std::to_string(raw.rel) +
                                            " is not " + std::to_string(alignment) + "-byte aligned");
        if (raw.rel > size - (uint64_t)data_offset)
            gthrow(AHIP_GGUF_TENSOR_OUT_OF_RANGE, "tensor '" + t.name + "' lies outside the file");
        t.offset = data_offset + (int64_t)raw.rel;
        int64_t end;
        if (__builtin_add_overflow(t.offset, t.bytes, &end) || (uint64_t)end > size)
            gthrow(AHIP_GGUF_TENSOR_OUT_OF_RANGE, "tensor '" + t.name + "' lies outside the file");
        tensors.push_back(t);
    }
    std::vector<int> order(tensors.size());
    for (size_t k = 0; k < order.size(); k++) order[k] = (int)k;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return tensors[a].offset < tensors[b].offset; });
    for (size_t k = 1; k < order.size(); k++) {
        const Tensor &a = tensors[order[k - 1]], &b = tensors[order[k]];
        if (a.offset + a.bytes > b.offset)
            gthrow(AHIP_GGUF_TENSORS_OVERLAP, "tensors '" + a.name + "' and '" + b.name + "' overlap");
    }
    for (size_t k = 0; k < tensors.size(); k++) index[tensors[k].name] = (int)k;
}

namespace {

int open_checked(std::unique_ptr<ahip_gguf>& g, ahip_gguf** out) {
    try {
        g->parse();
    } catch (const GError& e) {
        return report(e);
    } catch (const std::bad_alloc&) {
        return ahip_fail(AHIP_ERR_ALLOC, "out of host memory while parsing GGUF");
    }
    *out = g.release();
    g_kind = 0;
    return AHIP_OK;
}

}  // namespace

// ------------------------------------------------------------------ container

extern "C" int ahip_gguf_last_error_kind(void) { return g_kind; }

extern "C" int ahip_gguf_open(const char* path, ahip_gguf** out) {
    if (!path || !out) return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    auto cannot = [&](const std::string& why) { return report(GError{AHIP_GGUF_CANNOT_OPEN, "cannot open " + std::string(path) + ": " + why}); };
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return cannot(std::strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        const int e = errno;
        close(fd);
        return cannot(std::strerror(e));
    }
    if (st.st_size <= 0) {
        close(fd);
        return report(GError{AHIP_GGUF_TRUNCATED, "file truncated while reading header at offset 0"});
    }
    void* p = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    const int e = errno;
    close(fd);
    if (p == MAP_FAILED) return cannot(std::string("mmap failed: ") + std::strerror(e));
    auto g = std::make_unique<ahip_gguf>();
    g->base = static_cast<const uint8_t*>(p);
    g->size = (size_t)st.st_size;
    g->mapped = true;
    return open_checked(g, out);
}

extern "C" int ahip_gguf_open_memory(const void* data, int64_t bytes, ahip_gguf** out) {
    if (!out || bytes < 0 || (bytes && !data)) return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    *out = nullptr;
    auto g = std::make_unique<ahip_gguf>();
    try {
        g->copy.assign(static_cast<const uint8_t*>(data), static_cast<const uint8_t*>(data) + bytes);
    } catch (const std::bad_alloc&) {
        return ahip_fail(AHIP_ERR_ALLOC, "out of host memory copying a GGUF image");
    }
    g->base = g->copy.data();
    g->size = g->copy.size();
    return open_checked(g, out);
}

extern "C" int ahip_gguf_close(ahip_gguf* g) {
    delete g;
    return AHIP_OK;
}

extern "C" int ahip_gguf_header(const ahip_gguf* g, uint32_t* version, int64_t* alignment, int64_t* data_offset,
                                int64_t* file_size) {
    if (!g) return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    if (version) *version = g->version;
    if (alignment) *alignment = g->alignment;
    if (data_offset) *data_offset = g->data_offset;
    if (file_size) *file_size = (int64_t)g->size;
    return AHIP_OK;
}

extern "C" int ahip_gguf_meta_count(const ahip_gguf* g, int* count) {
    if (!g || !count) return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    *count = (int)g->keys.size();
    return AHIP_OK;
}

extern "C" int ahip_gguf_meta_key(const ahip_gguf* g, int i, const char** key, uint32_t* type) {
    if (!g || !key || i < 0 || i >= (int)g->keys.size()) return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "metadata index out of range");
    *key = g->keys[i].c_str();
    if (type) *type = g->meta.at(g->keys[i]).type;
    return AHIP_OK;
}

namespace {

// A metadata value, or one element of an array value (index >= 0).
int meta_value(const ahip_gguf* g, const char* key, int64_t index, const Value** v) {
    if (!g || !key) return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    const Value* m = g->find(key);
    if (!m) return report(GError{AHIP_GGUF_MISSING_METADATA, std::string("required metadata key '") + key + "' is missing or has the wrong type"});
    if (index >= 0) {
        if (m->type != 9 || index >= (int64_t)m->items.size())
            return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, std::string("metadata '") + key + "' has no element " + std::to_string(index));
        m = &m->items[(size_t)index];
    }
    *v = m;
    return AHIP_OK;
}

int wrong_type(const char* key) {
    return report(GError{AHIP_GGUF_MISSING_METADATA, std::string("required metadata key '") + key + "' is missing or has the wrong type"});
}

}  // namespace

extern "C" int ahip_gguf_meta_int(const ahip_gguf* g, const char* key, int64_t index, int64_t* out) {
    const Value* v;
    if (int rc = meta_value(g, key, index, &v)) return rc;
    if (!out || !v->as_int(*out)) return wrong_type(key);
    return AHIP_OK;
}

extern "C" int ahip_gguf_meta_uint(const ahip_gguf* g, const char* key, int64_t index, uint64_t* out) {
    const Value* v;
    if (int rc = meta_value(g, key, index, &v)) return rc;
    if (!out) return wrong_type(key);
    if (v->is_uint()) *out = v->u;
    else if (v->is_int() && v->i >= 0) *out = (uint64_t)v->i;
    else return wrong_type(key);
    return AHIP_OK;
}

extern "C" int ahip_gguf_meta_float(const ahip_gguf* g, const char* key, int64_t index, double* out) {
    const Value* v;
    if (int rc = meta_value(g, key, index, &v)) return rc;
    if (!out || !v->as_double(*out)) return wrong_type(key);
    return AHIP_OK;
}

extern "C" int ahip_gguf_meta_bool(const ahip_gguf* g, const char* key, int64_t index, int* out) {
    const Value* v;
    if (int rc = meta_value(g, key, index, &v)) return rc;
    if (!out || v->type != 7) return wrong_type(key);
    *out = (int)v->u;
    return AHIP_OK;
}

extern "C" int ahip_gguf_meta_string(const ahip_gguf* g, const char* key, int64_t index, const char** data,
                                     int64_t* length) {
    const Value* v;
    if (int rc = meta_value(g, key, index, &v)) return rc;
    if (!data || v->type != 8) return wrong_type(key);
    *data = v->s.data();
    if (length) *length = (int64_t)v->s.size();
    return AHIP_OK;
}

extern "C" int ahip_gguf_meta_array(const ahip_gguf* g, const char* key, uint32_t* elem_type, int64_t* count) {
    const Value* v;
    if (int rc = meta_value(g, key, -1, &v)) return rc;
    if (v->type != 9) return wrong_type(key);
    if (elem_type) *elem_type = v->elem_type;
    if (count) *count = (int64_t)v->items.size();
    return AHIP_OK;
}

extern "C" int ahip_gguf_tensor_count(const ahip_gguf* g, int* count) {
    if (!g || !count) return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    *count = (int)g->tensors.size();
    return AHIP_OK;
}

extern "C" int ahip_gguf_tensor_at(const ahip_gguf* g, int i, ahip_gguf_tensor* out) {
    if (!g || !out || i < 0 || i >= (int)g->tensors.size()) return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "tensor index out of range");
    const ahip_gguf::Tensor& t = g->tensors[i];
    std::memset(out, 0, sizeof(*out));
    out->name = t.name.c_str();
    out->n_dims = (int32_t)t.dims.size();
    for (size_t d = 0; d < t.dims.size(); d++) out->dims[d] = t.dims[d];
    out->type = t.type;
    out->file_offset = t.offset;
    out->byte_count = t.bytes;
    out->data = g->base + t.offset;
    return AHIP_OK;
}

extern "C" int ahip_gguf_find_tensor(const ahip_gguf* g, const char* name, int* index) {
    if (!g || !name || !index) return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    auto it = g->index.find(name);
    if (it == g->index.end()) return report(GError{AHIP_GGUF_MISSING_TENSOR, std::string("required tensor '") + name + "' is missing"});
    *index = it->second;
    return AHIP_OK;
}

// ------------------------------------------------------------------ Llama loader

namespace {

constexpr const char* kLayerTensors[] = {"attn_norm", "attn_q", "attn_k", "attn_v", "attn_output",
                                         "ffn_norm", "ffn_gate", "ffn_up", "ffn_down"};

// LlamaLoader.load, the configuration half (LlamaLoader.swift:36-72).
void llama_config(const ahip_gguf* g, ahip_llama_config& c) {
    const Value* arch = g->find("general.architecture");
    const std::string a = arch && arch->type == 8 ? arch->s : "<missing>";
    if (a != "llama")
        gthrow(AHIP_GGUF_UNSUPPORTED_MODEL, "unsupported model: general.architecture is '" + a + "', only 'llama' is supported");
    auto opt = [&](const char* key, int64_t& v) {
        const Value* m = g->find(key);
        return m && m->as_int(v);
    };
    auto req = [&](const char* key) -> int64_t {
        int64_t v;
        if (!opt(key, v)) gthrow(AHIP_GGUF_MISSING_METADATA, std::string("required metadata key '") + key + "' is missing or has the wrong type");
        return v;
    };
    auto optd = [&](const char* key, double dflt) {
        const Value* m = g->find(key);
        double v;
        return m && m->as_double(v) ? v : dflt;
    };
    const int64_t heads = req("llama.attention.head_count"), hidden = req("llama.embedding_length");
    if (heads <= 0) gthrow(AHIP_GGUF_MALFORMED, "malformed GGUF: llama.attention.head_count is 0");
    int64_t head_dim = hidden / heads, v;
    if (opt("llama.attention.key_length", v)) head_dim = v;
    if (opt("llama.attention.value_length", v) && v != head_dim)
        gthrow(AHIP_GGUF_UNSUPPORTED_MODEL, "unsupported model: attention.value_length " + std::to_string(v) +
                                                " != key_length " + std::to_string(head_dim));
    if (opt("llama.rope.dimension_count", v) && v != head_dim)
        gthrow(AHIP_GGUF_UNSUPPORTED_MODEL, "unsupported model: partial rotary embedding (rope dimension_count " +
                                                std::to_string(v) + " != head dim " + std::to_string(head_dim) +
                                                ") is not supported");
    if (const Value* s = g->find("llama.rope.scaling.type"); s && s->type == 8 && s->s != "none")
        gthrow(AHIP_GGUF_UNSUPPORTED_MODEL, "unsupported model: RoPE scaling '" + s->s + "' is not supported");
    if (g->find("llama.expert_count") && opt("llama.expert_count", v) && v > 0)
        gthrow(AHIP_GGUF_UNSUPPORTED_MODEL, "unsupported model: mixture-of-experts models are not supported");
    auto it = g->index.find("token_embd.weight");
    if (it == g->index.end()) gthrow(AHIP_GGUF_MISSING_TENSOR, "required tensor 'token_embd.weight' is missing");
    const ahip_gguf::Tensor& embd = g->tensors[it->second];
    if (embd.dims.size() != 2) gthrow(AHIP_GGUF_MALFORMED, "malformed GGUF: token_embd.weight must be 2-D");
    const int64_t kv = opt("llama.attention.head_count_kv", v) ? v : heads;
    const int64_t layers = req("llama.block_count"), ffn = req("llama.feed_forward_length"),
                  ctx = req("llama.context_length");
    auto i32 = [](int64_t x, const char* what) {
        if (x < INT32_MIN || x > INT32_MAX) gthrow(AHIP_GGUF_UNSUPPORTED_MODEL, std::string("unsupported model: ") + what + " out of range");
        return (int32_t)x;
    };
    c.vocab_size = i32(embd.dims[1], "vocabulary size");
    c.hidden_size = i32(hidden, "embedding_length");
    c.layer_count = i32(layers, "block_count");
    c.head_count = i32(heads, "head_count");
    c.kv_head_count = i32(kv, "head_count_kv");
    c.head_dim = i32(head_dim, "head dimension");
    c.feed_forward_size = i32(ffn, "feed_forward_length");
    c.context_length = i32(ctx, "context_length");
    c.rms_norm_eps = (float)optd("llama.attention.layer_norm_rms_epsilon", 1e-5);
    c.rope_theta = (float)optd("llama.rope.freq_base", 10000);
    c.rope_interleaved = 1;  // GGUF Llama weights use adjacent RoPE pairs
}

// Q4_1 block: f16 d, f16 m, 16 bytes of nibbles (low = element j, high =
// element j+16); value = d*q + m rounded once to f16 (LlamaLoader.swift:106-125).
uint16_t f32_to_f16_bits_rne(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // rounds past the largest half
    if (ax < 0x38800000u) {                                     // subnormal half (or zero)
        const uint32_t m = (ax & 0x7FFFFFu) | 0x800000u;
        const int shift = 113 - (int)(ax >> 23) + 13;
        if (shift > 24) return (uint16_t)sign;
        const uint32_t q = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        return (uint16_t)(sign | (q + (rem > half || (rem == half && (q & 1)))));
    }
    const uint32_t q = (ax - 0x38000000u) >> 13, rem = ax & 0x1FFFu;
    return (uint16_t)(sign | (q + (rem > 0x1000u || (rem == 0x1000u && (q & 1)))));
}
float f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1F, m = h & 0x3FF;
    uint32_t x;
    if (e == 0) {
        if (m == 0) x = sign;
        else {
            int k = 0;
            uint32_t mm = m;
            while (!(mm & 0x400)) mm <<= 1, k++;
            x = sign | ((uint32_t)(113 - k) << 23) | ((mm & 0x3FF) << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7F800000u | (m << 13);
    } else {
        x = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

void expand_q4_1(const uint8_t* src, int64_t elements, std::vector<uint16_t>& out) {
#pragma clang fp contract(off)
    out.resize((size_t)elements);
    for (int64_t b = 0; b < elements / 32; b++) {
        const uint8_t* p = src + b * 20;
        uint16_t hd, hm;
        std::memcpy(&hd, p, 2);
        std::memcpy(&hm, p + 2, 2);
        const float d = f16_bits_to_f32(hd), m = f16_bits_to_f32(hm);
        for (int j = 0; j < 16; j++) {
            const float lo = d * (float)(p[4 + j] & 0x0F), hi = d * (float)(p[4 + j] >> 4);
            out[(size_t)(b * 32 + j)] = f32_to_f16_bits_rne(lo + m);
            out[(size_t)(b * 32 + j + 16)] = f32_to_f16_bits_rne(hi + m);
        }
    }
}

}  // namespace

extern "C" int ahip_gguf_llama_config(const ahip_gguf* g, ahip_llama_config* out) {
    if (!g || !out) return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    try {
        llama_config(g, *out);
    } catch (const GError& e) {
        return report(e);
    }
    g_kind = 0;
    if (int rc = ahip_validate_config(out)) {
        g_kind = AHIP_GGUF_UNSUPPORTED_MODEL;
        return ahip_fail(AHIP_ERR_GGUF, std::string("unsupported model: ") + ahip_last_error());
    }
    return AHIP_OK;
}

// LlamaLoader.load, the weights half (LlamaLoader.swift:74-104), handed to ahip_model_create.
extern "C" int ahip_model_load_gguf(ahip_context* ctx, const ahip_gguf* g, int prefill_weight_cache, ahip_model** out,
                                    ahip_llama_config* config_out, ahip_load_report* report_out) {
    if (!ctx || !g || !out) return ahip_fail(AHIP_ERR_INVALID_ARGUMENT, "null argument");
    ahip_llama_config cfg;
    if (int rc = ahip_gguf_llama_config(g, &cfg)) return rc;
    ahip_load_report rep;
    std::memset(&rep, 0, sizeof(rep));
    std::string notes;
    std::vector<std::string> names;
    std::vector<ahip_tensor_desc> descs;
    std::vector<std::vector<uint16_t>> converted;  // Q4_1 tensors expanded to f16
    try {
        auto weight = [&](const std::string& gguf_name, bool norm) {
            auto it = g->index.find(gguf_name);
            if (it == g->index.end()) gthrow(AHIP_GGUF_MISSING_TENSOR, "required tensor '" + gguf_name + "' is missing");
            const ahip_gguf::Tensor& t = g->tensors[it->second];
            if (norm && t.type != AHIP_GGML_F32)
                gthrow(AHIP_GGUF_UNSUPPORTED_MODEL, "unsupported model: norm tensor '" + gguf_name + "' is type " +
                                                        std::to_string(t.type) + ", expected F32");
            if (t.dims.size() > 2)
                gthrow(AHIP_GGUF_MALFORMED, "malformed GGUF: tensor '" + gguf_name + "' has more than 2 dimensions");
            ahip_tensor_desc d;
            names.push_back(gguf_name.substr(0, gguf_name.size() - std::strlen(".weight")));
            d.name = nullptr;  // set below, once `names` stops growing
            d.rows = t.dims.size() == 2 ? t.dims[1] : 1;
            d.cols = t.dims[0];
            const int nat = native_dtype(t.type);
            if (nat >= 0) {
                d.dtype = nat;
                d.data = g->base + t.offset;
                d.bytes = t.bytes;
                rep.mapped_weight_bytes += t.bytes;
            } else if (t.type == AHIP_GGML_Q4_1) {
                converted.emplace_back();
                expand_q4_1(g->base + t.offset, d.rows * d.cols, converted.back());
                d.dtype = AHIP_F16;
                d.data = converted.back().data();
                d.bytes = (int64_t)converted.back().size() * 2;
                rep.converted_weight_bytes += d.bytes;
                rep.converted_tensors++;
                notes += gguf_name + ": Q4_1 expanded to F16 at load (" + std::to_string(t.bytes) + " -> " +
                         std::to_string(d.bytes) + " bytes)\n";
            } else {
                gthrow(AHIP_GGUF_UNSUPPORTED_TENSOR_TYPE,
                       "tensor '" + gguf_name + "' uses unsupported GGML type id " + std::to_string(t.type));
            }
            descs.push_back(d);
        };
        converted.reserve(descs.size() + 9 * (size_t)cfg.layer_count + 3);  // pointers into it stay valid
        for (int l = 0; l < cfg.layer_count; l++)
            for (const char* n : kLayerTensors)
                weight("blk." + std::to_string(l) + "." + n + ".weight", std::strcmp(n, "attn_norm") == 0 || std::strcmp(n, "ffn_norm") == 0);
        weight("token_embd.weight", false);
        weight("output_norm.weight", true);
        if (g->index.count("output.weight")) weight("output.weight", false);
    } catch (const GError& e) {
        return report(e);
    } catch (const std::bad_alloc&) {
        return ahip_fail(AHIP_ERR_ALLOC, "out of host memory expanding Q4_1 tensors");
    }
    for (size_t k = 0; k < descs.size(); k++) descs[k].name = names[k].c_str();
    std::strncpy(rep.notes, notes.c_str(), sizeof(rep.notes) - 1);
    if (int rc = ahip_model_create(ctx, &cfg, descs.data(), (int)descs.size(), prefill_weight_cache, out)) return rc;
    if (config_out) *config_out = cfg;
    if (report_out) *report_out = rep;
    return AHIP_OK;
}
