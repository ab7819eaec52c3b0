// GGUF reader and device weight staging behind the C ABI: the format
// boundary before the k-quant path (crates/gguf/src/lib.rs:20-345,1085-1199;
// crates/nvidia/src/cuda.rs:321-387; crates/nvidia/src/staging.rs:230-292).
//
// The parser follows the reference's rules and limits: magic "GGUF",
// version 3, at most 10M tensors and 1M metadata entries / array items,
// strings up to 16 MiB of valid UTF-8, array nesting up to 16, at most 16
// dimensions, a power-of-two general.alignment (default 32), the tensor data
// at the aligned end of the directory, and every tensor offset inside the
// file. Bulk tensor data is not read at open.
//
// Staging reads each tensor's byte range with pread into two pinned host
// buffers in turn and copies them to device memory on the context stream, so
// the next chunk's file read overlaps the previous chunk's copy (the
// reference uploads 1 MiB chunks with a host wait after each). The encoded
// bytes are stored unchanged; k-quant tensors become quantized weights with
// the reference's geometry checks, other types plain device copies.
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <unistd.h>

#include <algorithm>
#include <limits>
#include <map>
#include <new>
#include <string>
#include <vector>

#include "abi_internal.hpp"

namespace {

using namespace ribn_amd_abi;

constexpr uint32_t kMagic = 0x46554747u;
constexpr uint32_t kVersion = 3;
constexpr uint64_t kDefaultAlignment = 32;
constexpr uint64_t kMaxStringBytes = 16ull * 1024 * 1024;
constexpr uint64_t kMaxArrayItems = 1000000;
constexpr uint32_t kMaxDepth = 16;
constexpr uint32_t kMaxDims = 16;
constexpr uint64_t kMaxTensors = 10000000;
constexpr size_t kStageChunk = 8u << 20;  // bytes per pinned staging buffer

struct Value {
    uint32_t type = 0;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0;
    std::string s;
    uint32_t array_type = 0;
    std::vector<Value> items;
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t value_type;
    uint64_t offset;
};

// Block layout of a GGML type id (lib.rs:1050-1083).
bool tensor_layout(uint32_t t, uint64_t& elems, uint64_t& bytes) {
    switch (t) {
    case 0: case 26: elems = 1; bytes = 4; return true;
    case 1: case 25: case 30: elems = 1; bytes = 2; return true;
    case 2: case 20: elems = 32; bytes = 18; return true;
    case 3: elems = 32; bytes = 20; return true;
    case 6: elems = 32; bytes = 22; return true;
    case 7: elems = 32; bytes = 24; return true;
    case 8: elems = 32; bytes = 34; return true;
    case 9: elems = 32; bytes = 36; return true;
    case 10: elems = 256; bytes = 84; return true;
    case 11: case 21: elems = 256; bytes = 110; return true;
    case 12: elems = 256; bytes = 144; return true;
    case 13: elems = 256; bytes = 176; return true;
    case 14: elems = 256; bytes = 210; return true;
    case 15: elems = 256; bytes = 292; return true;
    case 16: case 35: elems = 256; bytes = 66; return true;
    case 17: elems = 256; bytes = 74; return true;
    case 18: elems = 256; bytes = 98; return true;
    case 19: elems = 256; bytes = 50; return true;
    case 22: elems = 256; bytes = 82; return true;
    case 23: elems = 256; bytes = 136; return true;
    case 24: elems = 1; bytes = 1; return true;
    case 27: case 28: elems = 1; bytes = 8; return true;
    case 29: elems = 256; bytes = 56; return true;
    case 34: elems = 256; bytes = 54; return true;
    case 39: elems = 32; bytes = 17; return true;
    case 40: elems = 64; bytes = 36; return true;
    case 41: elems = 128; bytes = 18; return true;
    case 42: elems = 64; bytes = 18; return true;
    default: return false;
    }
}

// TensorInfo::byte_len (lib.rs:128-163).
ribn_amd_status tensor_byte_len(const Tensor& t, uint64_t& out) {
    uint64_t be, bb;
    if (!tensor_layout(t.value_type, be, bb)) {
        return fail(RIBN_AMD_GGUF_UNSUPPORTED_TENSOR_TYPE, 0, t.value_type, "tensor '%s' has unsupported type %u",
                    t.name.c_str(), t.value_type);
    }
    if (t.dims.empty()) return fail(RIBN_AMD_GGUF_INVALID_DIMENSION_COUNT, 0, 0, "tensor '%s' has no dimensions", t.name.c_str());
    if (t.dims[0] % be != 0) {
        return fail(RIBN_AMD_GGUF_QUANTIZATION_MISMATCH, be, t.dims[0],
                    "tensor '%s' first dimension %llu is not a multiple of %llu", t.name.c_str(),
                    (unsigned long long)t.dims[0], (unsigned long long)be);
    }
    uint64_t elems = 1;
    for (uint64_t d : t.dims) {
        if (d != 0 && elems > std::numeric_limits<uint64_t>::max() / d) {
            return fail(RIBN_AMD_GGUF_BYTE_LENGTH_OVERFLOW, 0, 0, "tensor '%s' element count overflows", t.name.c_str());
        }
        elems *= d;
    }
    if (elems % be != 0) {
        return fail(RIBN_AMD_GGUF_QUANTIZATION_MISMATCH, be, elems, "tensor '%s' has %llu elements, not whole blocks",
                    t.name.c_str(), (unsigned long long)elems);
    }
    if (elems / be > std::numeric_limits<uint64_t>::max() / bb) {
        return fail(RIBN_AMD_GGUF_BYTE_LENGTH_OVERFLOW, 0, 0, "tensor '%s' byte length overflows", t.name.c_str());
    }
    out = elems / be * bb;
    return RIBN_AMD_OK;
}

bool valid_utf8(const std::string& s) {
    const unsigned char* p = reinterpret_cast<const unsigned char*>(s.data());
    size_t i = 0, n = s.size();
    while (i < n) {
        const unsigned char c = p[i];
        size_t len;
        uint32_t cp;
        if (c < 0x80) { ++i; continue; }
        if ((c & 0xE0) == 0xC0) { len = 2; cp = c & 0x1F; }
        else if ((c & 0xF0) == 0xE0) { len = 3; cp = c & 0x0F; }
        else if ((c & 0xF8) == 0xF0) { len = 4; cp = c & 0x07; }
        else return false;
        if (i + len > n) return false;
        for (size_t k = 1; k < len; ++k) {
            if ((p[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (p[i + k] & 0x3F);
        }
        // overlong forms, surrogates and values past U+10FFFF are not UTF-8
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000) || cp > 0x10FFFF ||
            (cp >= 0xD800 && cp <= 0xDFFF)) {
            return false;
        }
        i += len;
    }
    return true;
}

// Buffered little-endian reader over a file, tracking its position.
class Reader {
public:
    Reader(FILE* f, const std::string& path) : f_(f), path_(path) {}
    uint64_t pos() const { return pos_; }
    ribn_amd_status bytes(void* dst, size_t n) {
        if (n == 0) return RIBN_AMD_OK;
        if (fread(dst, 1, n, f_) != n) {
            return fail(RIBN_AMD_GGUF_IO, n, 0, "%s: unexpected end of file at byte %llu", path_.c_str(),
                        (unsigned long long)pos_);
        }
        pos_ += n;
        return RIBN_AMD_OK;
    }
    template <typename T>
    ribn_amd_status num(T& v) {
        unsigned char b[sizeof(T)];
        ribn_amd_status st = bytes(b, sizeof(T));
        if (st != RIBN_AMD_OK) return st;
        uint64_t x = 0;
        for (size_t k = 0; k < sizeof(T); ++k) x |= (uint64_t)b[k] << (8 * k);
        memcpy(&v, &x, sizeof(T));  // little-endian host
        return RIBN_AMD_OK;
    }
    ribn_amd_status count(const char* kind, uint64_t max, uint64_t& v) {
        ribn_amd_status st = num(v);
        if (st != RIBN_AMD_OK) return st;
        if (v > max) return fail(RIBN_AMD_GGUF_INVALID_LENGTH, max, v, "invalid %s length %llu", kind, (unsigned long long)v);
        return RIBN_AMD_OK;
    }
    ribn_amd_status string(std::string& s) {
        uint64_t len;
        ribn_amd_status st = num(len);
        if (st != RIBN_AMD_OK) return st;
        if (len > kMaxStringBytes) {
            return fail(RIBN_AMD_GGUF_INVALID_LENGTH, kMaxStringBytes, len, "invalid string length %llu",
                        (unsigned long long)len);
        }
        s.resize(len);
        st = bytes(&s[0], len);
        if (st != RIBN_AMD_OK) return st;
        if (!valid_utf8(s)) return fail(RIBN_AMD_GGUF_INVALID_UTF8, 0, 0, "string is not valid UTF-8");
        return RIBN_AMD_OK;
    }
    // read_value (lib.rs:1085-1127)
    ribn_amd_status value(uint32_t type, uint32_t depth, Value& v) {
        if (depth > kMaxDepth) return fail(RIBN_AMD_GGUF_ARRAY_NESTING_TOO_DEEP, kMaxDepth, depth, "array nesting too deep");
        v.type = type;
        ribn_amd_status st = RIBN_AMD_OK;
        switch (type) {
        case 0: { uint8_t x; st = num(x); v.u = x; break; }
        case 1: { uint8_t x; st = num(x); v.i = (int8_t)x; break; }
        case 2: { uint16_t x; st = num(x); v.u = x; break; }
        case 3: { uint16_t x; st = num(x); v.i = (int16_t)x; break; }
        case 4: { uint32_t x; st = num(x); v.u = x; break; }
        case 5: { uint32_t x; st = num(x); v.i = (int32_t)x; break; }
        case 6: { uint32_t x; st = num(x); float f; memcpy(&f, &x, 4); v.f = f; v.u = x; break; }
        case 7: {
            uint8_t x;
            st = num(x);
            if (st != RIBN_AMD_OK) return st;
            if (x > 1) return fail(RIBN_AMD_GGUF_INVALID_BOOL, 1, x, "invalid bool byte %u", x);
            v.u = x;
            break;
        }
        case 8: st = string(v.s); break;
        case 9: {
            st = num(v.array_type);
            if (st != RIBN_AMD_OK) return st;
            uint64_t n;
            st = count("array", kMaxArrayItems, n);
            if (st != RIBN_AMD_OK) return st;
            v.items.resize(n);
            for (uint64_t k = 0; k < n; ++k) {
                st = value(v.array_type, depth + 1, v.items[k]);
                if (st != RIBN_AMD_OK) return st;
            }
            break;
        }
        case 10: { uint64_t x; st = num(x); v.u = x; break; }
        case 11: { uint64_t x; st = num(x); v.i = (int64_t)x; break; }
        case 12: { uint64_t x; st = num(x); double d; memcpy(&d, &x, 8); v.f = d; v.u = x; break; }
        default: return fail(RIBN_AMD_GGUF_INVALID_VALUE_TYPE, 12, type, "invalid metadata value type %u", type);
        }
        return st;
    }

private:
    FILE* f_;
    std::string path_;
    uint64_t pos_ = 0;
};

// MetadataValue::as_u64 (lib.rs:55-65): unsigned integer types only.
bool as_u64(const Value& v, uint64_t& out) {
    if (v.type == 0 || v.type == 2 || v.type == 4 || v.type == 10) {
        out = v.u;
        return true;
    }
    return false;
}

void fill_value(const Value& v, ribn_amd_gguf_value* out) {
    memset(out, 0, sizeof(*out));
    out->type = v.type;
    out->u = v.u;
    out->i = v.i;
    out->f = v.f;
    if (v.type == 8) {
        out->str = v.s.c_str();
        out->str_len = v.s.size();
    }
    if (v.type == 9) {
        out->array_type = v.array_type;
        out->array_len = v.items.size();
    }
}

}  // namespace

struct ribn_amd_gguf {
    std::string path;
    uint32_t version;
    uint64_t tensor_count;
    std::map<std::string, Value> metadata;  // ordered by key, as the reference's BTreeMap
    std::vector<std::string> keys;
    std::vector<Tensor> tensors;
    uint64_t data_offset;
    uint64_t file_len;
};

namespace {

ribn_amd_status parse(FILE* f, ribn_amd_gguf* g) {
    if (fseeko(f, 0, SEEK_END) != 0) return fail(RIBN_AMD_GGUF_IO, 0, 0, "%s: cannot seek", g->path.c_str());
    g->file_len = (uint64_t)ftello(f);
    if (fseeko(f, 0, SEEK_SET) != 0) return fail(RIBN_AMD_GGUF_IO, 0, 0, "%s: cannot seek", g->path.c_str());
    Reader r(f, g->path);
    uint32_t magic, version;
    ribn_amd_status st = r.num(magic);
    if (st != RIBN_AMD_OK) return st;
    if (magic != kMagic) return fail(RIBN_AMD_GGUF_INVALID_MAGIC, kMagic, magic, "invalid GGUF magic 0x%08x", magic);
    st = r.num(version);
    if (st != RIBN_AMD_OK) return st;
    if (version != kVersion) {
        return fail(RIBN_AMD_GGUF_UNSUPPORTED_VERSION, kVersion, version, "unsupported GGUF version %u", version);
    }
    g->version = version;
    uint64_t metadata_count;
    st = r.count("tensor", kMaxTensors, g->tensor_count);
    if (st != RIBN_AMD_OK) return st;
    st = r.count("metadata", kMaxArrayItems, metadata_count);
    if (st != RIBN_AMD_OK) return st;
    for (uint64_t k = 0; k < metadata_count; ++k) {
        std::string key;
        uint32_t type;
        st = r.string(key);
        if (st != RIBN_AMD_OK) return st;
        st = r.num(type);
        if (st != RIBN_AMD_OK) return st;
        Value v;
        st = r.value(type, 0, v);
        if (st != RIBN_AMD_OK) return st;
        if (!g->metadata.emplace(key, std::move(v)).second) {
            return fail(RIBN_AMD_GGUF_DUPLICATE_METADATA, 0, 0, "duplicate metadata key '%s'", key.c_str());
        }
    }
    g->tensors.reserve(g->tensor_count);
    for (uint64_t k = 0; k < g->tensor_count; ++k) {
        Tensor t;
        st = r.string(t.name);
        if (st != RIBN_AMD_OK) return st;
        uint32_t nd;
        st = r.num(nd);
        if (st != RIBN_AMD_OK) return st;
        if (nd > kMaxDims) return fail(RIBN_AMD_GGUF_INVALID_DIMENSION_COUNT, kMaxDims, nd, "invalid dimension count %u", nd);
        t.dims.resize(nd);
        for (uint32_t d = 0; d < nd; ++d) {
            st = r.num(t.dims[d]);
            if (st != RIBN_AMD_OK) return st;
        }
        st = r.num(t.value_type);
        if (st != RIBN_AMD_OK) return st;
        st = r.num(t.offset);
        if (st != RIBN_AMD_OK) return st;
        g->tensors.push_back(std::move(t));
    }
    uint64_t alignment = kDefaultAlignment;
    auto it = g->metadata.find("general.alignment");
    if (it != g->metadata.end()) {
        uint64_t a;
        if (as_u64(it->second, a)) alignment = a;
    }
    if (alignment == 0 || (alignment & (alignment - 1)) != 0) {
        return fail(RIBN_AMD_GGUF_INVALID_ALIGNMENT, 0, alignment, "invalid alignment %llu", (unsigned long long)alignment);
    }
    const uint64_t end = r.pos();
    const uint64_t rem = end % alignment;
    if (rem != 0 && end > std::numeric_limits<uint64_t>::max() - (alignment - rem)) {
        return fail(RIBN_AMD_GGUF_TRUNCATED, 0, 0, "tensor data offset overflows");
    }
    g->data_offset = rem == 0 ? end : end + (alignment - rem);
    if (g->data_offset > g->file_len) return fail(RIBN_AMD_GGUF_TRUNCATED, g->data_offset, g->file_len, "file truncated");
    for (const Tensor& t : g->tensors) {
        if (t.offset > g->file_len - g->data_offset) {
            return fail(RIBN_AMD_GGUF_TENSOR_OFFSET_OUT_OF_BOUNDS, g->file_len - g->data_offset, t.offset,
                        "tensor '%s' offset %llu is out of bounds", t.name.c_str(), (unsigned long long)t.offset);
        }
    }
    for (const auto& kv : g->metadata) g->keys.push_back(kv.first);
    return RIBN_AMD_OK;
}

const Tensor* find(const ribn_amd_gguf* g, const char* name, uint64_t* index) {
    for (size_t k = 0; k < g->tensors.size(); ++k) {
        if (g->tensors[k].name == name) {
            if (index) *index = k;
            return &g->tensors[k];
        }
    }
    return nullptr;
}

// GgufFile::tensor_data_range (lib.rs:297-327)
ribn_amd_status data_range(const ribn_amd_gguf* g, const char* name, uint64_t& start, uint64_t& end,
                           const Tensor** tensor) {
    const Tensor* t = find(g, name, nullptr);
    if (!t) return fail(RIBN_AMD_MISSING_TENSOR, 0, 0, "missing tensor '%s'", name);
    uint64_t len;
    ribn_amd_status st = tensor_byte_len(*t, len);
    if (st != RIBN_AMD_OK) return st;
    if (t->offset > std::numeric_limits<uint64_t>::max() - g->data_offset) {
        return fail(RIBN_AMD_GGUF_BYTE_LENGTH_OVERFLOW, 0, 0, "tensor '%s' range overflows", name);
    }
    start = g->data_offset + t->offset;
    if (len > std::numeric_limits<uint64_t>::max() - start) {
        return fail(RIBN_AMD_GGUF_BYTE_LENGTH_OVERFLOW, 0, 0, "tensor '%s' range overflows", name);
    }
    end = start + len;
    if (end > g->file_len) {
        return fail(RIBN_AMD_GGUF_TENSOR_OFFSET_OUT_OF_BOUNDS, g->file_len, end, "tensor '%s' ends past the file",
                    name);
    }
    if (tensor) *tensor = t;
    return RIBN_AMD_OK;
}

// Pinned double buffer for staging file bytes to the device.
struct Staging {
    void* host[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool used[2] = {false, false};
    ~Staging() {
        for (int k = 0; k < 2; ++k) {
            if (done[k]) {
                hipEventSynchronize(done[k]);
                hipEventDestroy(done[k]);
            }
            if (host[k]) hipHostFree(host[k]);
        }
    }
};

}  // namespace

extern "C" {

ribn_amd_status ribn_amd_gguf_open(const char* path, ribn_amd_gguf** out) {
    if (!path || !out) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null path or out");
    *out = nullptr;
    FILE* f = fopen(path, "rb");
    if (!f) return fail(RIBN_AMD_GGUF_IO, 0, 0, "%s: %s", path, strerror(errno));
    auto* g = new (std::nothrow) ribn_amd_gguf();
    if (!g) {
        fclose(f);
        return fail(RIBN_AMD_DRIVER, 0, 0, "host allocation failed");
    }
    g->path = path;
    ribn_amd_status st = parse(f, g);
    fclose(f);
    if (st != RIBN_AMD_OK) {
        delete g;
        return st;
    }
    *out = g;
    return ok();
}

void ribn_amd_gguf_close(ribn_amd_gguf* g) { delete g; }

uint32_t ribn_amd_gguf_version(const ribn_amd_gguf* g) { return g ? g->version : 0; }
uint64_t ribn_amd_gguf_tensor_count(const ribn_amd_gguf* g) { return g ? g->tensor_count : 0; }
uint64_t ribn_amd_gguf_tensor_data_offset(const ribn_amd_gguf* g) { return g ? g->data_offset : 0; }
uint64_t ribn_amd_gguf_metadata_count(const ribn_amd_gguf* g) { return g ? g->keys.size() : 0; }

const char* ribn_amd_gguf_metadata_key(const ribn_amd_gguf* g, uint64_t index) {
    if (!g || index >= g->keys.size()) return nullptr;
    return g->keys[index].c_str();
}

ribn_amd_status ribn_amd_gguf_metadata_get(const ribn_amd_gguf* g, const char* key, ribn_amd_gguf_value* out) {
    if (!g || !key || !out) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    auto it = g->metadata.find(key);
    if (it == g->metadata.end()) return fail(RIBN_AMD_GGUF_MISSING_METADATA, 0, 0, "missing metadata '%s'", key);
    fill_value(it->second, out);
    return ok();
}

ribn_amd_status ribn_amd_gguf_metadata_item(const ribn_amd_gguf* g, const char* key, const uint64_t* path,
                                            size_t depth, ribn_amd_gguf_value* out) {
    if (!g || !key || !out || (!path && depth)) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    auto it = g->metadata.find(key);
    if (it == g->metadata.end()) return fail(RIBN_AMD_GGUF_MISSING_METADATA, 0, 0, "missing metadata '%s'", key);
    const Value* v = &it->second;
    for (size_t d = 0; d < depth; ++d) {
        if (v->type != 9) return fail(RIBN_AMD_GGUF_METADATA_TYPE_MISMATCH, 9, v->type, "'%s' is not an array", key);
        if (path[d] >= v->items.size()) {
            return fail(RIBN_AMD_INVALID_ARGUMENT, v->items.size(), path[d], "index past an array of '%s'", key);
        }
        v = &v->items[path[d]];
    }
    fill_value(*v, out);
    return ok();
}

ribn_amd_status ribn_amd_gguf_metadata_array_get(const ribn_amd_gguf* g, const char* key, uint64_t index,
                                                 ribn_amd_gguf_value* out) {
    return ribn_amd_gguf_metadata_item(g, key, &index, 1, out);
}

ribn_amd_status ribn_amd_gguf_tensor_info(const ribn_amd_gguf* g, uint64_t index, ribn_amd_gguf_tensor* out) {
    if (!g || !out) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    if (index >= g->tensors.size()) {
        return fail(RIBN_AMD_INVALID_ARGUMENT, g->tensors.size(), index, "tensor index out of range");
    }
    const Tensor& t = g->tensors[index];
    memset(out, 0, sizeof(*out));
    out->name = t.name.c_str();
    out->n_dims = (uint32_t)t.dims.size();
    for (size_t d = 0; d < t.dims.size(); ++d) out->dims[d] = t.dims[d];
    out->value_type = t.value_type;
    out->offset = t.offset;
    return ok();
}

ribn_amd_status ribn_amd_gguf_find_tensor(const ribn_amd_gguf* g, const char* name, uint64_t* index) {
    if (!g || !name || !index) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    if (!find(g, name, index)) return fail(RIBN_AMD_MISSING_TENSOR, 0, 0, "missing tensor '%s'", name);
    return ok();
}

ribn_amd_status ribn_amd_gguf_tensor_data_range(const ribn_amd_gguf* g, const char* name, uint64_t* start,
                                                uint64_t* end) {
    if (!g || !name || !start || !end) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    ribn_amd_status st = data_range(g, name, *start, *end, nullptr);
    return st == RIBN_AMD_OK ? ok() : st;
}

ribn_amd_status ribn_amd_gguf_stage(ribn_amd_context* ctx, const ribn_amd_gguf* g, const char* const* names,
                                    size_t count, uint64_t budget_bytes, ribn_amd_quantized_weight** out) {
    if (!ctx || !g || (!names && count) || (!out && count)) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null argument");
    for (size_t k = 0; k < count; ++k) out[k] = nullptr;
    // CudaQwen35Weights::stage (staging.rs:238-258): the budget is checked on
    // the encoded sizes before anything is uploaded
    std::vector<uint64_t> starts(count), lens(count);
    std::vector<const Tensor*> ts(count);
    uint64_t required = 0;
    for (size_t k = 0; k < count; ++k) {
        if (!names[k]) return fail(RIBN_AMD_INVALID_ARGUMENT, 0, 0, "null tensor name");
        uint64_t s, e;
        ribn_amd_status st = data_range(g, names[k], s, e, &ts[k]);
        if (st != RIBN_AMD_OK) return st;
        starts[k] = s;
        lens[k] = e - s;
        if (lens[k] == 0) return fail(RIBN_AMD_EMPTY_ENCODING, 0, 0, "tensor '%s' is empty", names[k]);
        if (required > std::numeric_limits<uint64_t>::max() - lens[k]) required = std::numeric_limits<uint64_t>::max();
        else required += lens[k];
    }
    if (required > budget_bytes) {
        return fail(RIBN_AMD_BUDGET_EXCEEDED, budget_bytes, required,
                    "staging needs %llu bytes, over the budget of %llu", (unsigned long long)required,
                    (unsigned long long)budget_bytes);
    }
    const int fd = open(g->path.c_str(), O_RDONLY);
    if (fd < 0) return fail(RIBN_AMD_GGUF_IO, 0, 0, "%s: %s", g->path.c_str(), strerror(errno));
    DeviceGuard guard(ctx->device);
    ribn_amd_status result = RIBN_AMD_OK;
    {
        Staging stg;
        hipError_t e = hipSuccess;
        for (int k = 0; k < 2 && e == hipSuccess; ++k) {
            e = hipHostMalloc(&stg.host[k], kStageChunk, hipHostMallocDefault);
            if (e == hipSuccess) e = hipEventCreateWithFlags(&stg.done[k], hipEventDisableTiming);
        }
        if (e != hipSuccess) result = driver(e, "pinned staging buffers");
        int slot = 0;
        for (size_t k = 0; k < count && result == RIBN_AMD_OK; ++k) {
            const Tensor& t = *ts[k];
            // k-quant tensors keep their [K, N] geometry checks; others (norm
            // vectors, F16 tables) are staged as plain device bytes
            const bool kquant = supported(t.value_type) && t.dims.size() >= 1;
            uint64_t kdim = t.dims.empty() ? 0 : t.dims[0];
            uint64_t ndim = 1;
            for (size_t d = 1; d < t.dims.size(); ++d) ndim *= t.dims[d];
            void* dev = nullptr;
            e = hipMalloc(&dev, lens[k]);
            if (e != hipSuccess) {
                result = driver(e, "hipMalloc staged tensor");
                break;
            }
            auto* w = new (std::nothrow) ribn_amd_quantized_weight{ctx, ctx->device, t.value_type, kdim, ndim, lens[k],
                                                                   static_cast<uint8_t*>(dev), true};
            if (!w) {
                hipFree(dev);
                result = fail(RIBN_AMD_DRIVER, 0, 0, "host allocation failed");
                break;
            }
            context_retain(ctx);  // released by ribn_amd_weight_destroy
            out[k] = w;
            if (kquant) {
                uint64_t vk, vn;
                result = validate_geometry(t.value_type, w, &vk, &vn);
                if (result != RIBN_AMD_OK) break;
            }
            uint64_t done = 0;
            while (done < lens[k] && result == RIBN_AMD_OK) {
                const size_t n = (size_t)std::min<uint64_t>(kStageChunk, lens[k] - done);
                if (stg.used[slot]) {
                    e = hipEventSynchronize(stg.done[slot]);  // the copy that last used this buffer
                    if (e != hipSuccess) {
                        result = driver(e, "staging copy");
                        break;
                    }
                }
                size_t filled = 0;
                while (filled < n) {
                    const ssize_t r = pread(fd, static_cast<char*>(stg.host[slot]) + filled, n - filled,
                                            (off_t)(starts[k] + done + filled));
                    if (r <= 0) {
                        result = fail(RIBN_AMD_SOURCE_INCOMPLETE, lens[k], done + filled,
                                      "tensor '%s': read %llu of %llu bytes", t.name.c_str(),
                                      (unsigned long long)(done + filled), (unsigned long long)lens[k]);
                        break;
                    }
                    filled += (size_t)r;
                }
                if (result != RIBN_AMD_OK) break;
                e = hipMemcpyAsync(static_cast<uint8_t*>(dev) + done, stg.host[slot], n, hipMemcpyHostToDevice,
                                   ctx->stream);
                if (e == hipSuccess) e = hipEventRecord(stg.done[slot], ctx->stream);
                if (e != hipSuccess) {
                    result = driver(e, "staging copy");
                    break;
                }
                stg.used[slot] = true;
                slot ^= 1;
                done += n;
            }
        }
        if (result == RIBN_AMD_OK) {
            e = hipStreamSynchronize(ctx->stream);
            if (e != hipSuccess) result = driver(e, "staging synchronize");
        }
    }
    close(fd);
    if (result != RIBN_AMD_OK) {
        hipStreamSynchronize(ctx->stream);
        for (size_t k = 0; k < count; ++k) {
            if (out[k]) {
                hipFree(out[k]->data);
                delete out[k];
                out[k] = nullptr;
            }
        }
        return result;
    }
    return ok();
}

}  // extern "C"
