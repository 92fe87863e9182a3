// gguf.cpp - GGUF (v2 / v3) reader for the qwen35 engine: header, metadata key/values and tensor table of a
// memory-mapped file.  The reference reads its model through strata::GgufFile (file.get / file.find /
// file.tensor_data at qw:945-957, 1978-2134), a dependency absent from the reference tree; this is a reader of the
// published GGUF layout written for the engine:
//   magic "GGUF", u32 version, u64 tensor count, u64 key/value count;
//   key/values: string key (u64 length + bytes), u32 type, value (types 0-12; 8 string, 9 array of u32 type + u64 n);
//   tensor infos: string name, u32 n_dims, u64 dims[n_dims] (dims[0] innermost), u32 GGML type, u64 offset;
//   data at the first multiple of general.alignment (default 32) after the infos, each tensor at data + offset.
// Every read is bounds-checked against the file size; a malformed file is an error, never a crash.
#include "rmi_common.h"

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

struct rmi_gguf {
    struct Value {
        int type = -1;              // GGUF value type of a scalar, or 9 (array)
        double num = 0.0;           // numeric scalar
        std::string str;            // string scalar
        int elem_type = -1;         // array element type
        uint64_t count = 0;         // array length
        std::vector<std::string> strs;   // string arrays
        std::vector<double> nums;        // numeric arrays
    };
    struct Tensor {
        std::string name;
        int type = 0;
        int n_dims = 0;
        int64_t dims[4] = {1, 1, 1, 1};
        uint64_t offset = 0;
        size_t bytes = 0;
        const uint8_t* data = nullptr;
    };
    int fd = -1;
    const uint8_t* map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint32_t alignment = 32;
    std::unordered_map<std::string, Value> kv;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> by_name;

    ~rmi_gguf() {
        if (map) munmap(const_cast<uint8_t*>(map), size);
        if (fd >= 0) close(fd);
    }
};

namespace rmi {
namespace {

struct Reader {
    const uint8_t* p;
    size_t size, at = 0;
    bool ok = true;
    bool need(size_t n) {
        if (!ok || n > size - at) ok = false;
        return ok;
    }
    template <typename T>
    T get() {
        T v{};
        if (need(sizeof(T))) {
            std::memcpy(&v, p + at, sizeof(T));
            at += sizeof(T);
        }
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!need(n)) return {};
        std::string s(reinterpret_cast<const char*>(p + at), n);
        at += n;
        return s;
    }
};

// size in bytes of a scalar of GGUF value type t (0 if not a fixed-size scalar)
size_t scalar_bytes(uint32_t t) {
    switch (t) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
        default: return 0;
    }
}

double scalar_value(Reader& r, uint32_t t) {
    switch (t) {
        case 0: return r.get<uint8_t>();
        case 1: return r.get<int8_t>();
        case 2: return r.get<uint16_t>();
        case 3: return r.get<int16_t>();
        case 4: return r.get<uint32_t>();
        case 5: return r.get<int32_t>();
        case 6: return r.get<float>();
        case 7: return r.get<uint8_t>() != 0;
        case 10: return static_cast<double>(r.get<uint64_t>());
        case 11: return static_cast<double>(r.get<int64_t>());
        case 12: return r.get<double>();
        default: r.ok = false; return 0.0;
    }
}

// bytes of a GGML tensor of `elems` elements with inner dimension n0, or 0 for a type the engine does not know
size_t tensor_bytes(int type, int64_t n0, int64_t elems) {
    auto blocks = [&](int per, int bytes) -> size_t {
        return n0 % per ? 0 : static_cast<size_t>(elems / per) * bytes;
    };
    switch (type) {
        case 0: return static_cast<size_t>(elems) * 4;      // F32
        case 1: return static_cast<size_t>(elems) * 2;      // F16
        case 30: return static_cast<size_t>(elems) * 2;     // BF16
        case 8: return blocks(32, 34);                      // Q8_0
        case 11: return blocks(256, 110);                   // Q3_K
        case 12: return blocks(256, 144);                   // Q4_K
        case 13: return blocks(256, 176);                   // Q5_K
        case 14: return blocks(256, 210);                   // Q6_K
        case 23: return blocks(256, 136);                   // IQ4_XS
        default: return 0;
    }
}

int parse(rmi_gguf& g) {
    Reader r{g.map, g.size};
    if (!r.need(4) || std::memcmp(g.map, "GGUF", 4) != 0) return fail(RMI_ERR_SHAPE, "gguf: not a GGUF file");
    r.at = 4;
    g.version = r.get<uint32_t>();
    if (g.version != 2 && g.version != 3) return fail(RMI_ERR_UNSUPPORTED, "gguf: unsupported version");
    const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    if (!r.ok || n_tensors > (1u << 24) || n_kv > (1u << 24)) return fail(RMI_ERR_SHAPE, "gguf: bad header");
    for (uint64_t i = 0; i < n_kv && r.ok; ++i) {
        std::string key = r.str();
        rmi_gguf::Value v;
        v.type = static_cast<int>(r.get<uint32_t>());
        if (v.type == 8) {
            v.str = r.str();
        } else if (v.type == 9) {
            v.elem_type = static_cast<int>(r.get<uint32_t>());
            v.count = r.get<uint64_t>();
            if (v.elem_type == 8) {
                for (uint64_t j = 0; j < v.count && r.ok; ++j) v.strs.push_back(r.str());
            } else if (const size_t sb = scalar_bytes(static_cast<uint32_t>(v.elem_type))) {
                if (v.count > (r.size - r.at) / sb) return fail(RMI_ERR_SHAPE, "gguf: truncated array");
                v.nums.reserve(v.count);
                for (uint64_t j = 0; j < v.count; ++j) v.nums.push_back(scalar_value(r, static_cast<uint32_t>(v.elem_type)));
            } else {
                return fail(RMI_ERR_UNSUPPORTED, "gguf: nested or unknown array element type");
            }
        } else if (scalar_bytes(static_cast<uint32_t>(v.type))) {
            v.num = scalar_value(r, static_cast<uint32_t>(v.type));
        } else {
            return fail(RMI_ERR_UNSUPPORTED, "gguf: unknown metadata value type");
        }
        if (key == "general.alignment" && v.type != 9 && v.type != 8) g.alignment = static_cast<uint32_t>(v.num);
        g.kv[key] = std::move(v);
    }
    if (!r.ok) return fail(RMI_ERR_SHAPE, "gguf: truncated metadata");
    if (g.alignment == 0 || (g.alignment & (g.alignment - 1))) return fail(RMI_ERR_SHAPE, "gguf: bad alignment");
    // A tensor record is at least a name length (8), a rank (4), one dimension (8), a type (4) and an offset (8):
    // a count the remaining bytes cannot hold is rejected before anything is sized by it.
    constexpr size_t kMinTensorRecord = 8 + 4 + 8 + 4 + 8;
    if (n_tensors > (r.size - r.at) / kMinTensorRecord) return fail(RMI_ERR_SHAPE, "gguf: truncated tensor table");
    g.tensors.resize(n_tensors);
    for (uint64_t i = 0; i < n_tensors && r.ok; ++i) {
        rmi_gguf::Tensor& t = g.tensors[i];
        t.name = r.str();
        t.n_dims = static_cast<int>(r.get<uint32_t>());
        if (t.n_dims < 1 || t.n_dims > 4) return fail(RMI_ERR_SHAPE, "gguf: bad tensor rank");
        for (int d = 0; d < t.n_dims; ++d) t.dims[d] = static_cast<int64_t>(r.get<uint64_t>());
        t.type = static_cast<int>(r.get<uint32_t>());
        t.offset = r.get<uint64_t>();
    }
    if (!r.ok) return fail(RMI_ERR_SHAPE, "gguf: truncated tensor table");
    const size_t data = (r.at + g.alignment - 1) / g.alignment * g.alignment;
    for (size_t i = 0; i < g.tensors.size(); ++i) {
        rmi_gguf::Tensor& t = g.tensors[i];
        int64_t elems = 1;
        for (int d = 0; d < t.n_dims; ++d) {
            if (t.dims[d] <= 0 || t.dims[d] > (int64_t(1) << 40) / elems) return fail(RMI_ERR_SHAPE, "gguf: bad tensor dims");
            elems *= t.dims[d];
        }
        t.bytes = tensor_bytes(t.type, t.dims[0], elems);
        if (t.bytes == 0) continue;   // a type the engine does not read: listed, no data pointer
        if (data > g.size || t.offset > g.size - data || t.bytes > g.size - data - t.offset)
            return fail(RMI_ERR_SHAPE, "gguf: tensor data outside the file");
        t.data = g.map + data + t.offset;
        g.by_name[t.name] = i;
    }
    for (size_t i = 0; i < g.tensors.size(); ++i)
        if (!g.by_name.count(g.tensors[i].name)) g.by_name[g.tensors[i].name] = i;
    return RMI_OK;
}

}  // namespace
}  // namespace rmi

using namespace rmi;

extern "C" int rmi_gguf_open(const char* path, rmi_gguf** out) {
    if (!path || !out) return fail(RMI_ERR_POINTER, "gguf: null argument");
    *out = nullptr;
    auto* g = new (std::nothrow) rmi_gguf();
    if (!g) return fail(RMI_ERR_STATE, "gguf: out of host memory");
    g->fd = open(path, O_RDONLY);
    struct stat st {};
    if (g->fd < 0 || fstat(g->fd, &st) != 0 || st.st_size < 24) {
        delete g;
        return fail(RMI_ERR_STATE, "gguf: cannot open the file");
    }
    g->size = static_cast<size_t>(st.st_size);
    void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        delete g;
        return fail(RMI_ERR_STATE, "gguf: mmap failed");
    }
    g->map = static_cast<const uint8_t*>(m);
    int rc = RMI_OK;
    try {
        rc = parse(*g);
    } catch (const std::bad_alloc&) {
        rc = fail(RMI_ERR_SHAPE, "gguf: metadata too large for host memory");
    } catch (const std::length_error&) {
        rc = fail(RMI_ERR_SHAPE, "gguf: metadata too large");
    }
    if (rc != RMI_OK) {
        delete g;
        return rc;
    }
    *out = g;
    return RMI_OK;
}

extern "C" void rmi_gguf_close(rmi_gguf* g) { delete g; }

extern "C" int64_t rmi_gguf_tensor_count(const rmi_gguf* g) { return g ? static_cast<int64_t>(g->tensors.size()) : -1; }

extern "C" int64_t rmi_gguf_find(const rmi_gguf* g, const char* name) {
    if (!g || !name) return -1;
    const auto it = g->by_name.find(name);
    return it == g->by_name.end() ? -1 : static_cast<int64_t>(it->second);
}

extern "C" int rmi_gguf_tensor_info(const rmi_gguf* g, int64_t i, const char** name, int* type, int* n_dims,
                                    int64_t* dims, size_t* bytes, const void** data) {
    if (!g || i < 0 || i >= static_cast<int64_t>(g->tensors.size())) return fail(RMI_ERR_SHAPE, "gguf: bad tensor index");
    const rmi_gguf::Tensor& t = g->tensors[static_cast<size_t>(i)];
    if (name) *name = t.name.c_str();
    if (type) *type = t.type;
    if (n_dims) *n_dims = t.n_dims;
    if (dims)
        for (int d = 0; d < 4; ++d) dims[d] = t.dims[d];
    if (bytes) *bytes = t.bytes;
    if (data) *data = t.data;
    return RMI_OK;
}

extern "C" int rmi_gguf_get_num(const rmi_gguf* g, const char* key, double* out) {
    if (!g || !key || !out) return fail(RMI_ERR_POINTER, "gguf: null argument");
    const auto it = g->kv.find(key);
    if (it == g->kv.end() || it->second.type == 8 || it->second.type == 9) return fail(RMI_ERR_STATE, "gguf: no such number");
    *out = it->second.num;
    return RMI_OK;
}

extern "C" int rmi_gguf_get_str(const rmi_gguf* g, const char* key, const char** out) {
    if (!g || !key || !out) return fail(RMI_ERR_POINTER, "gguf: null argument");
    const auto it = g->kv.find(key);
    if (it == g->kv.end() || it->second.type != 8) return fail(RMI_ERR_STATE, "gguf: no such string");
    *out = it->second.str.c_str();
    return RMI_OK;
}

extern "C" int64_t rmi_gguf_array_len(const rmi_gguf* g, const char* key) {
    if (!g || !key) return -1;
    const auto it = g->kv.find(key);
    return it == g->kv.end() || it->second.type != 9 ? -1 : static_cast<int64_t>(it->second.count);
}

extern "C" int rmi_gguf_array_str(const rmi_gguf* g, const char* key, int64_t i, const char** out) {
    if (!g || !key || !out) return fail(RMI_ERR_POINTER, "gguf: null argument");
    const auto it = g->kv.find(key);
    if (it == g->kv.end() || it->second.type != 9 || it->second.elem_type != 8 || i < 0 ||
        i >= static_cast<int64_t>(it->second.strs.size()))
        return fail(RMI_ERR_STATE, "gguf: no such string array element");
    *out = it->second.strs[static_cast<size_t>(i)].c_str();
    return RMI_OK;
}

extern "C" int rmi_gguf_array_num(const rmi_gguf* g, const char* key, int64_t i, double* out) {
    if (!g || !key || !out) return fail(RMI_ERR_POINTER, "gguf: null argument");
    const auto it = g->kv.find(key);
    if (it == g->kv.end() || it->second.type != 9 || i < 0 || i >= static_cast<int64_t>(it->second.nums.size()))
        return fail(RMI_ERR_STATE, "gguf: no such numeric array element");
    *out = it->second.nums[static_cast<size_t>(i)];
    return RMI_OK;
}
