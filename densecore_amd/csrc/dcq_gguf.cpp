// dcq_gguf.cpp — GGUF weight ingest: parse a GGUF file's header, metadata and tensor table,
// and stream a tensor's bytes into device memory.
//
// Replaces what the reference gets from ggml's gguf_init_from_file (core/src/model_loader.cpp:
// 96-130: the whole file read into host ggml buffers, no_alloc = false), gguf_find_key /
// gguf_get_val_* for metadata, and ggml_get_tensor by name (core/src/model_loader.cpp:294-402).
// Here the weights go to HBM: a tensor is read from the file in chunks into pinned host
// buffers and copied to the device on the caller's stream, two chunks in flight.
//
// Format (GGUF v2/v3, little-endian; restated from the public GGUF specification):
//   u32 magic "GGUF" (0x46554747), u32 version, u64 tensor_count, u64 kv_count
//   kv_count x { string key, u32 value_type, value }      string = u64 length + bytes
//   tensor_count x { string name, u32 n_dims, u64 ne[n_dims], u32 type, u64 offset }
//   padding to `general.alignment` (u32, default 32), then the data section; each tensor's
//   offset is relative to the data section start.
// Every length and count read from the file is bounded by the file size before use.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/dcq.h"

namespace {

enum ValueType : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7, kStr = 8, kArr = 9,
    kU64 = 10, kI64 = 11, kF64 = 12,
};

// (elements per block, bytes per block) of the ggml tensor types a GGUF weight file holds
bool type_geometry(uint32_t t, uint64_t* blck, uint64_t* bytes) {
    switch (t) {
        case 0: *blck = 1; *bytes = 4; return true;      // F32
        case 1: *blck = 1; *bytes = 2; return true;      // F16
        case 2: *blck = 32; *bytes = 18; return true;    // Q4_0
        case 3: *blck = 32; *bytes = 20; return true;    // Q4_1
        case 6: *blck = 32; *bytes = 22; return true;    // Q5_0
        case 7: *blck = 32; *bytes = 24; return true;    // Q5_1
        case 8: *blck = 32; *bytes = 34; return true;    // Q8_0
        case 9: *blck = 32; *bytes = 36; return true;    // Q8_1
        case 10: *blck = 256; *bytes = 84; return true;  // Q2_K
        case 11: *blck = 256; *bytes = 110; return true; // Q3_K
        case 12: *blck = 256; *bytes = 144; return true; // Q4_K
        case 13: *blck = 256; *bytes = 176; return true; // Q5_K
        case 14: *blck = 256; *bytes = 210; return true; // Q6_K
        case 15: *blck = 256; *bytes = 292; return true; // Q8_K
        case 24: *blck = 1; *bytes = 1; return true;     // I8
        case 25: *blck = 1; *bytes = 2; return true;     // I16
        case 26: *blck = 1; *bytes = 4; return true;     // I32
        case 27: *blck = 1; *bytes = 8; return true;     // I64
        case 28: *blck = 1; *bytes = 8; return true;     // F64
        case 30: *blck = 1; *bytes = 2; return true;     // BF16
        default: return false;
    }
}

struct Value {
    uint32_t type = 0;
    uint64_t u = 0;   // integer and bool values (sign-extended for signed types)
    double f = 0;     // float values
    std::string s;    // string values
    uint32_t arr_type = 0;
    uint64_t arr_len = 0;
};

struct Tensor {
    std::string name;
    uint32_t type = 0;
    uint32_t n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0;  // from the data section start
    uint64_t nbytes = 0;
};

// bounded little-endian reader over the mapped file
struct Reader {
    const uint8_t* p;
    uint64_t size, pos = 0;
    bool ok = true;
    bool need(uint64_t n) {
        if (!ok || n > size - pos) ok = false;
        return ok;
    }
    template <class T>
    T get() {
        T v{};
        if (need(sizeof(T))) {
            memcpy(&v, p + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!need(n)) return std::string();
        std::string s(reinterpret_cast<const char*>(p + pos), (size_t)n);
        pos += n;
        return s;
    }
    void skip(uint64_t n) {
        if (need(n)) pos += n;
    }
};

uint64_t scalar_size(uint32_t t) {
    switch (t) {
        case kU8: case kI8: case kBool: return 1;
        case kU16: case kI16: return 2;
        case kU32: case kI32: case kF32: return 4;
        case kU64: case kI64: case kF64: return 8;
        default: return 0;
    }
}

bool read_scalar(Reader& r, uint32_t t, Value& v) {
    switch (t) {
        case kU8: v.u = r.get<uint8_t>(); break;
        case kI8: v.u = (uint64_t)(int64_t)r.get<int8_t>(); break;
        case kU16: v.u = r.get<uint16_t>(); break;
        case kI16: v.u = (uint64_t)(int64_t)r.get<int16_t>(); break;
        case kU32: v.u = r.get<uint32_t>(); break;
        case kI32: v.u = (uint64_t)(int64_t)r.get<int32_t>(); break;
        case kU64: v.u = r.get<uint64_t>(); break;
        case kI64: v.u = (uint64_t)r.get<int64_t>(); break;
        case kBool: v.u = r.get<uint8_t>() != 0; break;
        case kF32: v.f = r.get<float>(); break;
        case kF64: v.f = r.get<double>(); break;
        default: return false;
    }
    return r.ok;
}

}  // namespace

struct dcq_gguf {
    int fd = -1;
    void* map = nullptr;
    uint64_t file_size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32;
    uint64_t data_start = 0;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int64_t> by_name;
    std::unordered_map<std::string, Value> kv;
    // staging for dcq_gguf_load_tensor: two pinned host chunks, allocated by the first load
    // (portable, so any device's stream can copy from them) and freed by dcq_gguf_close
    mutable void* stage[2] = {nullptr, nullptr};
    mutable size_t stage_bytes = 0;
};

namespace {

int parse(dcq_gguf* g) {
    Reader r{static_cast<const uint8_t*>(g->map), g->file_size};
    if (r.get<uint32_t>() != 0x46554747u || !r.ok) return DCQ_ERR_FORMAT;
    g->version = r.get<uint32_t>();
    if (g->version < 2 || g->version > 3) return DCQ_ERR_FORMAT;
    const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    // a kv entry takes at least 13 bytes of the file and a tensor entry at least 32: counts
    // beyond that are malformed (the tables then grow only as entries are actually read)
    if (!r.ok || n_kv > g->file_size / 13 || n_tensors > g->file_size / 32) return DCQ_ERR_FORMAT;
    for (uint64_t i = 0; i < n_kv; ++i) {
        const std::string key = r.str();
        Value v;
        v.type = r.get<uint32_t>();
        if (!r.ok) return DCQ_ERR_FORMAT;
        if (v.type == kStr) {
            v.s = r.str();
        } else if (v.type == kArr) {
            v.arr_type = r.get<uint32_t>();
            v.arr_len = r.get<uint64_t>();
            if (!r.ok) return DCQ_ERR_FORMAT;
            if (v.arr_type == kStr) {
                for (uint64_t j = 0; j < v.arr_len && r.ok; ++j) r.skip(r.get<uint64_t>());
            } else {
                const uint64_t es = scalar_size(v.arr_type);
                if (es == 0 || v.arr_len > (r.size - r.pos) / es) return DCQ_ERR_FORMAT;
                r.skip(es * v.arr_len);
            }
        } else if (!read_scalar(r, v.type, v)) {
            return DCQ_ERR_FORMAT;
        }
        if (!r.ok) return DCQ_ERR_FORMAT;
        // a key may appear once (gguf_init_from_file rejects duplicates as well)
        if (!g->kv.emplace(key, v).second) return DCQ_ERR_FORMAT;
    }
    auto al = g->kv.find("general.alignment");
    if (al != g->kv.end()) {
        if (al->second.type != kU32 || al->second.u == 0 || (al->second.u & (al->second.u - 1))) return DCQ_ERR_FORMAT;
        g->alignment = al->second.u;
    }
    for (uint64_t i = 0; i < n_tensors; ++i) {
        Tensor t;
        t.name = r.str();
        t.n_dims = r.get<uint32_t>();
        if (!r.ok || t.n_dims == 0 || t.n_dims > 4) return DCQ_ERR_FORMAT;
        uint64_t n = 1;
        for (uint32_t d = 0; d < t.n_dims; ++d) {
            const uint64_t e = r.get<uint64_t>();
            if (!r.ok || e == 0 || e > (1ull << 40) || n > (1ull << 50) / e) return DCQ_ERR_FORMAT;
            t.ne[d] = (int64_t)e;
            n *= e;
        }
        t.type = r.get<uint32_t>();
        t.offset = r.get<uint64_t>();
        if (!r.ok) return DCQ_ERR_FORMAT;
        uint64_t blck, bs;
        if (!type_geometry(t.type, &blck, &bs)) return DCQ_ERR_UNSUPPORTED;
        if (t.ne[0] % (int64_t)blck) return DCQ_ERR_FORMAT;
        t.nbytes = n / blck * bs;
        if (t.offset % g->alignment) return DCQ_ERR_FORMAT;
        if (g->by_name.count(t.name)) return DCQ_ERR_FORMAT;
        g->by_name[t.name] = (int64_t)g->tensors.size();
        g->tensors.push_back(t);
    }
    const uint64_t pad = (g->alignment - r.pos % g->alignment) % g->alignment;
    g->data_start = r.pos + pad;
    for (const Tensor& t : g->tensors) {
        if (g->data_start > g->file_size || t.offset > g->file_size - g->data_start ||
            t.nbytes > g->file_size - g->data_start - t.offset)
            return DCQ_ERR_FORMAT;
    }
    return DCQ_OK;
}

}  // namespace

extern "C" {

int dcq_gguf_open(const char* path, dcq_gguf** out) {
    if (!path || !out) return DCQ_ERR_INVALID_ARG;
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return DCQ_ERR_IO;
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return DCQ_ERR_IO;
    }
    if (st.st_size < 24) {
        close(fd);
        return DCQ_ERR_FORMAT;
    }
    void* map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (map == MAP_FAILED) {
        close(fd);
        return DCQ_ERR_IO;
    }
    dcq_gguf* g = new dcq_gguf();
    g->fd = fd;
    g->map = map;
    g->file_size = (uint64_t)st.st_size;
    const int rc = parse(g);
    if (rc != DCQ_OK) {
        dcq_gguf_close(g);
        return rc;
    }
    *out = g;
    return DCQ_OK;
}

void dcq_gguf_close(dcq_gguf* g) {
    if (!g) return;
    for (void* p : g->stage)
        if (p) (void)hipHostFree(p);
    if (g->map) munmap(g->map, (size_t)g->file_size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

int64_t dcq_gguf_tensor_count(const dcq_gguf* g) { return g ? (int64_t)g->tensors.size() : -1; }

int64_t dcq_gguf_find_tensor(const dcq_gguf* g, const char* name) {
    if (!g || !name) return -1;
    auto it = g->by_name.find(name);
    return it == g->by_name.end() ? -1 : it->second;
}

int dcq_gguf_tensor_info(const dcq_gguf* g, int64_t i, const char** name, int* type, int* n_dims, int64_t ne[4],
                         uint64_t* file_offset, uint64_t* nbytes) {
    if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return DCQ_ERR_INVALID_ARG;
    const Tensor& t = g->tensors[(size_t)i];
    if (name) *name = t.name.c_str();
    if (type) *type = (int)t.type;
    if (n_dims) *n_dims = (int)t.n_dims;
    if (ne)
        for (int d = 0; d < 4; ++d) ne[d] = t.ne[d];
    if (file_offset) *file_offset = g->data_start + t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return DCQ_OK;
}

int dcq_gguf_get_int(const dcq_gguf* g, const char* key, int64_t* out) {
    if (!g || !key || !out) return DCQ_ERR_INVALID_ARG;
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return DCQ_ERR_NOT_FOUND;
    const Value& v = it->second;
    if (scalar_size(v.type) == 0 || v.type == kF32 || v.type == kF64) return DCQ_ERR_FORMAT;
    *out = (int64_t)v.u;
    return DCQ_OK;
}

int dcq_gguf_get_str(const dcq_gguf* g, const char* key, const char** out) {
    if (!g || !key || !out) return DCQ_ERR_INVALID_ARG;
    auto it = g->kv.find(key);
    if (it == g->kv.end()) return DCQ_ERR_NOT_FOUND;
    if (it->second.type != kStr) return DCQ_ERR_FORMAT;
    *out = it->second.s.c_str();
    return DCQ_OK;
}

int dcq_gguf_load_tensor(const dcq_gguf* g, int64_t i, void* dst, size_t dst_bytes, void* stream) {
    if (!g || !dst || i < 0 || i >= (int64_t)g->tensors.size()) return DCQ_ERR_INVALID_ARG;
    const Tensor& t = g->tensors[(size_t)i];
    if (dst_bytes < t.nbytes) return DCQ_ERR_INVALID_ARG;
    hipStream_t st = (hipStream_t)stream;
    if (t.nbytes == 0) return DCQ_OK;
    if (!g->stage[0]) {
        // chunk: 32 MB, or the largest tensor when every tensor is smaller
        uint64_t largest = 0;
        for (const Tensor& u : g->tensors) largest = u.nbytes > largest ? u.nbytes : largest;
        const size_t bytes = (size_t)(largest < (32u << 20) ? largest : (32u << 20));
        for (int b = 0; b < 2; ++b) {
            if (hipHostMalloc(&g->stage[b], bytes, hipHostMallocPortable) != hipSuccess) {
                for (void*& p : g->stage) {
                    if (p) (void)hipHostFree(p);
                    p = nullptr;
                }
                return DCQ_ERR_HIP;
            }
        }
        g->stage_bytes = bytes;
    }
    void* const* buf = g->stage;
    const size_t chunk = g->stage_bytes;
    hipEvent_t done[2] = {nullptr, nullptr};
    int rc = DCQ_OK;
    for (int b = 0; b < 2 && rc == DCQ_OK; ++b)
        if (hipEventCreateWithFlags(&done[b], hipEventDisableTiming) != hipSuccess) rc = DCQ_ERR_HIP;
    const uint64_t base = g->data_start + t.offset;
    uint64_t pos = 0;
    for (int k = 0; rc == DCQ_OK && pos < t.nbytes; ++k) {
        const int b = k & 1;
        const size_t n = (size_t)(t.nbytes - pos < chunk ? t.nbytes - pos : chunk);
        // the buffer's previous copy must be done before it is overwritten
        if (k >= 2 && hipEventSynchronize(done[b]) != hipSuccess) { rc = DCQ_ERR_HIP; break; }
        size_t got = 0;
        while (got < n) {
            const ssize_t r = pread(g->fd, static_cast<char*>(buf[b]) + got, n - got, (off_t)(base + pos + got));
            if (r <= 0) { rc = DCQ_ERR_IO; break; }
            got += (size_t)r;
        }
        if (rc != DCQ_OK) break;
        if (hipMemcpyAsync(static_cast<char*>(dst) + pos, buf[b], n, hipMemcpyHostToDevice, st) != hipSuccess ||
            hipEventRecord(done[b], st) != hipSuccess)
            rc = DCQ_ERR_HIP;
        pos += n;
    }
    // the call returns only after its copies have finished: dst is ready, and the staging
    // buffers are free for the next call
    for (int b = 0; b < 2; ++b) {
        if (done[b]) {
            if (hipEventSynchronize(done[b]) != hipSuccess && rc == DCQ_OK) rc = DCQ_ERR_HIP;
            (void)hipEventDestroy(done[b]);
        }
    }
    return rc;
}

}  // extern "C"
