// cbx_gguf.cpp -- the tables of a GGUF model file, for the gather ops.
//
// The reference loads its weights with ggml's gguf reader: metadata first
// (gguf_init_from_file with no_alloc, chatterbox-cpp/src/model.cpp:41-57),
// then each tensor's bytes read from data_offset + tensor offset and
// uploaded to the backend (model.cpp:90-121).  This is the same two-step
// path for libcbxops callers: cbx_gguf_open parses the header, key/values
// and tensor directory (GGUF v2/v3, little endian) and checks every tensor
// lies inside the file; cbx_gguf_upload copies one tensor's bytes into
// device memory the caller owns.  Token tables in F32, F16 or Q8_0 (34-byte
// blocks) can then be described with cbx_gguf_describe and gathered
// directly.  Host code only; nothing here launches a kernel.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "cbx_internal.h"

namespace {

constexpr uint32_t kGgufMagic = 0x46554747u;   // "GGUF" read as a little-endian u32
constexpr uint32_t kDefaultAlignment = 32;
constexpr int kMaxDims = 4;

enum GgufValueType : uint32_t {
    GV_UINT8 = 0, GV_INT8 = 1, GV_UINT16 = 2, GV_INT16 = 3, GV_UINT32 = 4, GV_INT32 = 5, GV_FLOAT32 = 6,
    GV_BOOL = 7, GV_STRING = 8, GV_ARRAY = 9, GV_UINT64 = 10, GV_INT64 = 11, GV_FLOAT64 = 12,
};

// Bytes of one scalar of a GGUF value type (0: not a fixed-size scalar).
size_t scalar_size(uint32_t t) {
    switch (t) {
        case GV_UINT8: case GV_INT8: case GV_BOOL: return 1;
        case GV_UINT16: case GV_INT16: return 2;
        case GV_UINT32: case GV_INT32: case GV_FLOAT32: return 4;
        case GV_UINT64: case GV_INT64: case GV_FLOAT64: return 8;
        default: return 0;
    }
}

// ggml_type -> (elements per block, bytes per block); {0, 0} if unknown.
struct TypeTraits {
    int64_t blck;
    size_t bytes;
};
TypeTraits type_traits(uint32_t t) {
    switch (t) {
        case 0: return {1, 4};      // F32
        case 1: return {1, 2};      // F16
        case 2: return {32, 18};    // Q4_0
        case 3: return {32, 20};    // Q4_1
        case 6: return {32, 22};    // Q5_0
        case 7: return {32, 24};    // Q5_1
        case 8: return {32, 34};    // Q8_0
        case 9: return {32, 36};    // Q8_1
        case 10: return {256, 84};  // Q2_K
        case 11: return {256, 110}; // Q3_K
        case 12: return {256, 144}; // Q4_K
        case 13: return {256, 176}; // Q5_K
        case 14: return {256, 210}; // Q6_K
        case 15: return {256, 292}; // Q8_K
        case 24: return {1, 1};     // I8
        case 25: return {1, 2};     // I16
        case 26: return {1, 4};     // I32
        case 27: return {1, 8};     // I64
        case 28: return {1, 8};     // F64
        case 30: return {1, 2};     // BF16
        default: return {0, 0};
    }
}

struct TensorEntry {
    std::string name;
    uint32_t type = 0;
    int32_t n_dims = 0;
    int64_t ne[kMaxDims] = {1, 1, 1, 1};
    size_t nbytes = 0;
    uint64_t offset = 0;   // from the start of the data section
};

class Reader {
  public:
    explicit Reader(FILE* f, uint64_t size) : f_(f), size_(size) {}
    bool read(void* dst, size_t n) {
        if (n > size_ - pos_ || (n && std::fread(dst, 1, n, f_) != n)) return fail("unexpected end of file");
        pos_ += n;
        return true;
    }
    template <typename T>
    bool get(T* v) { return read(v, sizeof(T)); }
    bool skip(uint64_t n) {
        if (n > size_ - pos_ || std::fseek(f_, static_cast<long>(pos_ + n), SEEK_SET) != 0) {
            return fail("unexpected end of file");
        }
        pos_ += n;
        return true;
    }
    bool str(std::string* s) {
        uint64_t n = 0;
        if (!get(&n)) return false;
        if (n > (uint64_t{1} << 20) || n > size_ - pos_) return fail("string length out of range");
        s->resize(static_cast<size_t>(n));
        return read(&(*s)[0], static_cast<size_t>(n));
    }
    bool fail(const std::string& m) {
        if (err_.empty()) err_ = m;
        return false;
    }
    uint64_t pos() const { return pos_; }
    const std::string& error() const { return err_; }

  private:
    FILE* f_;
    uint64_t size_;
    uint64_t pos_ = 0;
    std::string err_;
};

}  // namespace

struct cbx_gguf {
    std::string path;
    uint32_t version = 0;
    uint32_t alignment = kDefaultAlignment;
    uint64_t data_offset = 0;
    uint64_t file_size = 0;
    std::unordered_map<std::string, std::string> strings;   // string-valued keys
    std::vector<TensorEntry> tensors;
    std::unordered_map<std::string, int64_t> index;
};

using namespace cbx;

namespace {

int gguf_fail(const std::string& path, const std::string& msg) {
    return set_error(CBX_ERR_INVALID_ARG, "cbx_gguf_open: " + path + ": " + msg);
}

// Reads one key's value; keeps strings (and general.alignment) and skips the rest.
bool read_value(Reader& r, cbx_gguf* g, const std::string& key, uint32_t type) {
    if (type == GV_STRING) {
        std::string v;
        if (!r.str(&v)) return false;
        g->strings[key] = v;
        return true;
    }
    if (type == GV_ARRAY) {
        uint32_t et = 0;
        uint64_t n = 0;
        if (!r.get(&et) || !r.get(&n)) return false;
        if (et == GV_STRING) {
            for (uint64_t i = 0; i < n; i++) {
                uint64_t len = 0;
                if (!r.get(&len) || !r.skip(len)) return false;
            }
            return true;
        }
        const size_t es = scalar_size(et);
        if (!es) return r.fail("array of unsupported value type " + std::to_string(et));
        if (n > (UINT64_MAX / es)) return r.fail("array too long");
        return r.skip(n * es);
    }
    const size_t es = scalar_size(type);
    if (!es) return r.fail("unknown value type " + std::to_string(type) + " for key " + key);
    if (key == "general.alignment") {
        if (type != GV_UINT32) return r.fail("general.alignment must be UINT32");
        return r.get(&g->alignment);
    }
    return r.skip(es);
}

}  // namespace

extern "C" {

int cbx_gguf_open(const char* path, cbx_gguf** out) {
    clear_error();
    if (!path || !out) return set_error(CBX_ERR_INVALID_ARG, "cbx_gguf_open: path and out must not be NULL");
    *out = nullptr;
    FILE* f = std::fopen(path, "rb");
    if (!f) return gguf_fail(path, "cannot open");
    std::fseek(f, 0, SEEK_END);
    const long end = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    auto* g = new cbx_gguf();
    g->path = path;
    g->file_size = end > 0 ? static_cast<uint64_t>(end) : 0;
    Reader r(f, g->file_size);
    uint32_t magic = 0;
    uint64_t n_tensors = 0, n_kv = 0;
    bool ok = r.get(&magic) && (magic == kGgufMagic || r.fail("not a GGUF file (bad magic)")) && r.get(&g->version) &&
              ((g->version == 2 || g->version == 3) || r.fail("unsupported GGUF version " + std::to_string(g->version))) &&
              r.get(&n_tensors) && r.get(&n_kv) &&
              (n_tensors < (uint64_t{1} << 24) || r.fail("tensor count out of range")) &&
              (n_kv < (uint64_t{1} << 24) || r.fail("key count out of range"));
    for (uint64_t i = 0; ok && i < n_kv; i++) {
        std::string key;
        uint32_t type = 0;
        ok = r.str(&key) && r.get(&type) && read_value(r, g, key, type);
    }
    if (ok && (g->alignment == 0 || (g->alignment & (g->alignment - 1)))) ok = r.fail("alignment must be a power of two");
    for (uint64_t i = 0; ok && i < n_tensors; i++) {
        TensorEntry t;
        uint32_t nd = 0;
        ok = r.str(&t.name) && r.get(&nd) && (nd >= 1 && nd <= kMaxDims ? true : r.fail("tensor " + t.name + ": n_dims out of range"));
        for (uint32_t d = 0; ok && d < nd; d++) {
            uint64_t v = 0;
            ok = r.get(&v) && (v < (uint64_t{1} << 40) || r.fail("tensor " + t.name + ": dimension out of range"));
            t.ne[d] = static_cast<int64_t>(v);
        }
        ok = ok && r.get(&t.type) && r.get(&t.offset);
        if (!ok) break;
        t.n_dims = static_cast<int32_t>(nd);
        const TypeTraits tt = type_traits(t.type);
        if (!tt.blck) { ok = r.fail("tensor " + t.name + ": unknown ggml type " + std::to_string(t.type)); break; }
        if (t.ne[0] % tt.blck) { ok = r.fail("tensor " + t.name + ": ne[0] not a multiple of the block size"); break; }
        uint64_t nel = 1, nb = 0;
        bool over = false;
        for (int d = 0; d < kMaxDims; d++) over |= __builtin_mul_overflow(nel, static_cast<uint64_t>(t.ne[d]), &nel);
        over |= __builtin_mul_overflow(nel / static_cast<uint64_t>(tt.blck), static_cast<uint64_t>(tt.bytes), &nb);
        if (over) { ok = r.fail("tensor " + t.name + ": size overflows"); break; }
        t.nbytes = static_cast<size_t>(nb);
        if (t.offset % g->alignment) { ok = r.fail("tensor " + t.name + ": offset not aligned"); break; }
        if (g->index.count(t.name)) { ok = r.fail("duplicate tensor name " + t.name); break; }
        g->index[t.name] = static_cast<int64_t>(g->tensors.size());
        g->tensors.push_back(t);
    }
    if (ok) {
        g->data_offset = (r.pos() + g->alignment - 1) / g->alignment * g->alignment;
        for (const TensorEntry& t : g->tensors) {
            if (t.offset > g->file_size || g->data_offset > g->file_size - t.offset ||
                t.nbytes > g->file_size - g->data_offset - t.offset) {
                ok = r.fail("tensor " + t.name + " extends past the end of the file");
                break;
            }
        }
    }
    std::fclose(f);
    if (!ok) {
        const std::string msg = r.error();
        delete g;
        return gguf_fail(path, msg);
    }
    *out = g;
    return CBX_OK;
}

void cbx_gguf_close(cbx_gguf* g) { delete g; }

int64_t cbx_gguf_n_tensors(const cbx_gguf* g) { return g ? static_cast<int64_t>(g->tensors.size()) : -1; }

int64_t cbx_gguf_find_tensor(const cbx_gguf* g, const char* name) {
    if (!g || !name) return -1;
    const auto it = g->index.find(name);
    return it == g->index.end() ? -1 : it->second;
}

const char* cbx_gguf_get_str(const cbx_gguf* g, const char* key) {
    if (!g || !key) return nullptr;
    const auto it = g->strings.find(key);
    return it == g->strings.end() ? nullptr : it->second.c_str();
}

int cbx_gguf_tensor(const cbx_gguf* g, int64_t i, cbx_gguf_tensor_info* out) {
    clear_error();
    if (!g || !out || i < 0 || i >= static_cast<int64_t>(g->tensors.size())) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_gguf_tensor: bad handle, index or output");
    }
    const TensorEntry& t = g->tensors[static_cast<size_t>(i)];
    out->name = t.name.c_str();
    out->type = static_cast<int32_t>(t.type);
    out->n_dims = t.n_dims;
    for (int d = 0; d < kMaxDims; d++) out->ne[d] = t.ne[d];
    out->nbytes = t.nbytes;
    out->file_offset = static_cast<size_t>(g->data_offset + t.offset);
    return CBX_OK;
}

int cbx_gguf_describe(const cbx_gguf* g, int64_t i, void* data, cbx_tensor* out) {
    clear_error();
    if (!g || !out || i < 0 || i >= static_cast<int64_t>(g->tensors.size())) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_gguf_describe: bad handle, index or output");
    }
    const TensorEntry& t = g->tensors[static_cast<size_t>(i)];
    if (t.type != CBX_TYPE_F32 && t.type != CBX_TYPE_F16 && t.type != CBX_TYPE_Q8_0 && t.type != CBX_TYPE_I32) {
        return set_error(CBX_ERR_UNSUPPORTED, "cbx_gguf_describe: tensor " + t.name + " has ggml type " +
                                                  std::to_string(t.type) + " (F32, F16, Q8_0, I32 are supported)");
    }
    const TypeTraits tt = type_traits(t.type);
    std::memset(out, 0, sizeof(*out));
    out->data = data;
    out->type = static_cast<int32_t>(t.type);
    for (int d = 0; d < kMaxDims; d++) out->ne[d] = t.ne[d];
    out->nb[0] = tt.bytes;                                       // ggml: nb[0] = block size
    out->nb[1] = static_cast<size_t>(t.ne[0] / tt.blck) * tt.bytes;
    for (int d = 2; d < kMaxDims; d++) out->nb[d] = out->nb[d - 1] * static_cast<size_t>(t.ne[d - 1]);
    return CBX_OK;
}

int cbx_gguf_upload(const cbx_gguf* g, int64_t i, void* dst, size_t dst_bytes, cbx_stream stream) {
    clear_error();
    if (!g || i < 0 || i >= static_cast<int64_t>(g->tensors.size()) || !dst) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_gguf_upload: bad handle, index or destination");
    }
    const TensorEntry& t = g->tensors[static_cast<size_t>(i)];
    if (dst_bytes < t.nbytes) {
        return set_error(CBX_ERR_INVALID_ARG, "cbx_gguf_upload: destination smaller than tensor " + t.name + " (" +
                                                  std::to_string(t.nbytes) + " bytes)");
    }
    FILE* f = std::fopen(g->path.c_str(), "rb");
    if (!f) return set_error(CBX_ERR_INVALID_ARG, "cbx_gguf_upload: cannot reopen " + g->path);
    // staged through host memory in 64 MiB pieces, each copy finished before the buffer is refilled
    constexpr size_t kPiece = size_t{64} << 20;
    std::vector<char> buf(std::min(kPiece, std::max<size_t>(t.nbytes, 1)));
    int rc = CBX_OK;
    if (std::fseek(f, static_cast<long>(g->data_offset + t.offset), SEEK_SET) != 0) {
        rc = set_error(CBX_ERR_INVALID_ARG, "cbx_gguf_upload: seek failed for " + t.name);
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    for (size_t done = 0; rc == CBX_OK && done < t.nbytes;) {
        const size_t n = std::min(buf.size(), t.nbytes - done);
        if (std::fread(buf.data(), 1, n, f) != n) {
            rc = set_error(CBX_ERR_INVALID_ARG, "cbx_gguf_upload: short read for " + t.name);
            break;
        }
        if (hipMemcpyAsync(static_cast<char*>(dst) + done, buf.data(), n, hipMemcpyHostToDevice, s) != hipSuccess ||
            hipStreamSynchronize(s) != hipSuccess) {
            rc = set_error(CBX_ERR_HIP, "cbx_gguf_upload: copy to the device failed for " + t.name);
            break;
        }
        done += n;
    }
    std::fclose(f);
    return rc;
}

}  // extern "C"
