// GGUF v3 reader and device upload of a model file's tensor data (host code).
//
// Follows the container layout the reference reads (src/gguf.cpp:41-71, src/gguf.h): magic
// "GGUF", version 3, tensor and key-value counts, the key-value pairs (typed values, arrays
// of any element type, "general.alignment" overriding the default 32), the tensor infos
// (name, dims, ggml type, offset relative to the data region), then the data region at
// the next multiple of the alignment.  The file is memory-mapped read-only; the data
// region goes to the device in one allocation so that a matrix is a byte offset into it
// (src/engine.cpp:27-37), as kata_dispatch_create expects.  The copy streams through a
// pinned staging buffer (pageable memory cannot be registered for DMA here).
#include "../../include/kata_amd.h"
#include "launch.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

int kata_internal_fail(int code, const char* msg);   // capi.cpp: sets kata_last_error

struct kata_gguf {
    int fd = -1;
    const uint8_t* map = nullptr;
    size_t size = 0;
    uint64_t data_start = 0;
    struct Tensor {
        std::string name;
        uint32_t type = 0, ndims = 0;
        uint64_t dims[4] = {1, 1, 1, 1};
        uint64_t offset = 0, nbytes = 0;
    };
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> by_name;
    std::unordered_map<std::string, uint64_t> ints;        // integer and bool scalars
    std::unordered_map<std::string, std::string> strs;     // string scalars
};

namespace {

// Block geometry of a ggml type: elements and bytes per block; false for a type not known
// here (the reference exits on one, src/gguf.cpp:25-37).
bool type_block(uint32_t type, uint64_t& elems, uint64_t& bytes) {
    switch (type) {
        case 0: elems = 1; bytes = 4; return true;        // F32
        case 1: elems = 1; bytes = 2; return true;        // F16
        case 30: elems = 1; bytes = 2; return true;       // BF16
        case 8: elems = 32; bytes = 34; return true;      // Q8_0
        case 143: elems = 128; bytes = 28; return true;   // PTQ1_0
        case 142: elems = 128; bytes = 34; return true;   // PQ2_0
        case 10: elems = 256; bytes = 84; return true;    // Q2_K
        case 11: elems = 256; bytes = 110; return true;   // Q3_K
        case 12: elems = 256; bytes = 144; return true;   // Q4_K
        case 14: elems = 256; bytes = 210; return true;   // Q6_K
        default: return false;
    }
}

size_t scalar_size(uint32_t t) {
    switch (t) {
        case 0: case 1: case 7: return 1;        // u8 i8 bool
        case 2: case 3: return 2;                // u16 i16
        case 4: case 5: case 6: return 4;        // u32 i32 f32
        case 10: case 11: case 12: return 8;     // u64 i64 f64
        default: return 0;
    }
}

struct Reader {
    const uint8_t* base;
    size_t size, p = 0;
    bool ok = true;
    bool need(size_t n) {
        if (!ok || n > size - p) ok = false;
        return ok;
    }
    template <class T>
    T rd() {
        T v{};
        if (need(sizeof(T))) memcpy(&v, base + p, sizeof(T)), p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = rd<uint64_t>();
        if (!need(n)) return {};
        std::string s((const char*)base + p, n);
        p += n;
        return s;
    }
    void skip(uint64_t n) {
        if (need(n)) p += n;
    }
};

}  // namespace

extern "C" {

kata_gguf* kata_gguf_open(const char* path) {
    if (!path) return kata_internal_fail(KATA_EINVAL, "null path"), nullptr;
    kata_gguf* g = new kata_gguf();
    g->fd = ::open(path, O_RDONLY);
    struct stat st;
    if (g->fd < 0 || fstat(g->fd, &st) != 0 || st.st_size < 24) {
        kata_gguf_close(g);
        return kata_internal_fail(KATA_EINVAL, "cannot open or too short"), nullptr;
    }
    g->size = (size_t)st.st_size;
    void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        kata_gguf_close(g);
        return kata_internal_fail(KATA_EINVAL, "mmap failed"), nullptr;
    }
    g->map = (const uint8_t*)m;
    Reader r{g->map, g->size};
    if (memcmp(g->map, "GGUF", 4) != 0) {
        kata_gguf_close(g);
        return kata_internal_fail(KATA_EINVAL, "not a GGUF file"), nullptr;
    }
    r.p = 4;
    if (r.rd<uint32_t>() != 3) {
        kata_gguf_close(g);
        return kata_internal_fail(KATA_EINVAL, "GGUF version is not 3"), nullptr;
    }
    const uint64_t nt = r.rd<uint64_t>(), nkv = r.rd<uint64_t>();
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < nkv && r.ok; i++) {
        const std::string key = r.str();
        const uint32_t t = r.rd<uint32_t>();
        if (t == 8) {
            g->strs[key] = r.str();
        } else if (t == 9) {                     // array: element type, count, elements
            const uint32_t et = r.rd<uint32_t>();
            const uint64_t n = r.rd<uint64_t>();
            if (et == 8) {
                for (uint64_t k = 0; k < n && r.ok; k++) r.str();
            } else if (scalar_size(et) && n <= (r.size - r.p) / scalar_size(et)) {
                r.skip(n * scalar_size(et));
            } else {
                r.ok = false;
            }
        } else if (scalar_size(t)) {
            uint64_t v = 0;
            switch (t) {
                case 0: case 7: v = r.rd<uint8_t>(); break;
                case 1: v = (uint64_t)(int64_t)r.rd<int8_t>(); break;
                case 2: v = r.rd<uint16_t>(); break;
                case 3: v = (uint64_t)(int64_t)r.rd<int16_t>(); break;
                case 4: v = r.rd<uint32_t>(); break;
                case 5: v = (uint64_t)(int64_t)r.rd<int32_t>(); break;
                case 10: case 11: v = r.rd<uint64_t>(); break;
                default: r.skip(scalar_size(t)); continue;   // floats: not indexed
            }
            g->ints[key] = v;
            if (key == "general.alignment") alignment = v;
        } else {
            r.ok = false;
        }
    }
    const char* why = nullptr;
    for (uint64_t i = 0; i < nt && r.ok && !why; i++) {
        kata_gguf::Tensor t;
        t.name = r.str();
        t.ndims = r.rd<uint32_t>();
        if (t.ndims > 4) r.ok = false;
        uint64_t ne = 1;
        for (uint32_t d = 0; d < t.ndims && r.ok; d++) {
            t.dims[d] = r.rd<uint64_t>();
            if (t.dims[d] != 0 && ne > UINT64_MAX / t.dims[d]) why = "a tensor's element count overflows";
            else ne *= t.dims[d];
        }
        t.type = r.rd<uint32_t>();
        t.offset = r.rd<uint64_t>();
        uint64_t be = 0, bb = 0;
        if (!r.ok || why) break;
        if (!type_block(t.type, be, bb)) why = "a tensor has a ggml type not supported here";
        else if (ne % be != 0) why = "a tensor's element count is not a whole number of blocks";
        else if (ne / be > UINT64_MAX / bb) why = "a tensor's byte size overflows";
        else t.nbytes = ne / be * bb;
        g->by_name[t.name] = g->tensors.size();
        g->tensors.push_back(t);
    }
    if (!why && (!r.ok || alignment == 0 || (alignment & (alignment - 1)) || alignment > ((uint64_t)1 << 30)))
        why = "truncated or malformed GGUF header";
    if (!why) {
        g->data_start = (r.p + alignment - 1) / alignment * alignment;
        if (g->data_start > g->size) why = "the data region starts past the end of the file";
    }
    for (size_t i = 0; i < g->tensors.size() && !why; i++) {
        const auto& t = g->tensors[i];
        const uint64_t room = g->size - g->data_start;   // no wrap-around: each term checked alone
        if (t.offset > room || t.nbytes > room - t.offset) why = "a tensor lies past the end of the file";
    }
    if (why) {
        kata_gguf_close(g);
        return kata_internal_fail(KATA_EINVAL, why), nullptr;
    }
    return g;
}

void kata_gguf_close(kata_gguf* g) {
    if (!g) return;
    if (g->map) munmap((void*)g->map, g->size);
    if (g->fd >= 0) ::close(g->fd);
    delete g;
}

int64_t kata_gguf_tensor_count(const kata_gguf* g) { return g ? (int64_t)g->tensors.size() : KATA_EINVAL; }

uint64_t kata_gguf_data_bytes(const kata_gguf* g) { return g ? g->size - g->data_start : 0; }

int kata_gguf_tensor(const kata_gguf* g, int64_t i, const char** name, uint32_t* type, uint64_t* dims,
                     uint64_t* offset, uint64_t* nbytes) {
    if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return kata_internal_fail(KATA_EINVAL, "no such tensor index");
    const auto& t = g->tensors[(size_t)i];
    if (name) *name = t.name.c_str();
    if (type) *type = t.type;
    if (dims)
        for (int d = 0; d < 4; d++) dims[d] = t.dims[d];
    if (offset) *offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return KATA_OK;
}

int64_t kata_gguf_find(const kata_gguf* g, const char* name) {
    if (!g || !name) return kata_internal_fail(KATA_EINVAL, "null argument");
    auto it = g->by_name.find(name);
    if (it == g->by_name.end()) return kata_internal_fail(KATA_EINVAL, "no such tensor");
    return (int64_t)it->second;
}

int kata_gguf_get_int(const kata_gguf* g, const char* key, uint64_t* value) {
    if (!g || !key || !value) return kata_internal_fail(KATA_EINVAL, "null argument");
    auto it = g->ints.find(key);
    if (it == g->ints.end()) return kata_internal_fail(KATA_EINVAL, "no such integer key");
    *value = it->second;
    return KATA_OK;
}

const char* kata_gguf_get_str(const kata_gguf* g, const char* key) {
    if (!g || !key) return nullptr;
    auto it = g->strs.find(key);
    return it == g->strs.end() ? nullptr : it->second.c_str();
}

int kata_gguf_upload_into(const kata_gguf* g, uint8_t* d, uint64_t capacity) {
    if (!g || !d) return kata_internal_fail(KATA_EINVAL, "null argument");
    const uint64_t n = kata_gguf_data_bytes(g);
    if (capacity < n) return kata_internal_fail(KATA_EINVAL, "device buffer smaller than the data region");
    // double-buffered pinned staging: the host fills one half while the other is copied
    const size_t chunk = 64u << 20;
    uint8_t* stage = nullptr;
    hipStream_t s = nullptr;
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool ok = hipHostMalloc((void**)&stage, 2 * chunk, hipHostMallocDefault) == hipSuccess &&
              hipStreamCreate(&s) == hipSuccess && hipEventCreate(&ev[0]) == hipSuccess &&
              hipEventCreate(&ev[1]) == hipSuccess;
    for (uint64_t o = 0, k = 0; ok && o < n; o += chunk, k ^= 1) {
        const size_t len = (size_t)std::min<uint64_t>(chunk, n - o);
        ok = hipEventSynchronize(ev[k]) == hipSuccess;       // the half's previous copy is done
        if (!ok) break;
        memcpy(stage + k * chunk, g->map + g->data_start + o, len);
        ok = hipMemcpyAsync(d + o, stage + k * chunk, len, hipMemcpyHostToDevice, s) == hipSuccess &&
             hipEventRecord(ev[k], s) == hipSuccess;
    }
    if (s) ok = hipStreamSynchronize(s) == hipSuccess && ok;
    for (auto e : ev)
        if (e) (void)hipEventDestroy(e);
    if (s) (void)hipStreamDestroy(s);
    if (stage) (void)hipHostFree(stage);
    return ok ? KATA_OK : kata_internal_fail(KATA_ELAUNCH, "upload of the data region failed");
}

int kata_gguf_upload(const kata_gguf* g, uint8_t** dev_base) {
    if (!g || !dev_base) return kata_internal_fail(KATA_EINVAL, "null argument");
    const uint64_t n = kata_gguf_data_bytes(g);
    uint8_t* d = nullptr;
    if (hipMalloc((void**)&d, n ? n : 1) != hipSuccess) return kata_internal_fail(KATA_ELAUNCH, "hipMalloc of the data region failed");
    const int rc = kata_gguf_upload_into(g, d, n);
    if (rc != KATA_OK) {
        (void)hipFree(d);
        return rc;
    }
    *dev_base = d;
    return KATA_OK;
}

int kata_gguf_free_device(uint8_t* dev_base) {
    return hipFree(dev_base) == hipSuccess ? KATA_OK : kata_internal_fail(KATA_ELAUNCH, "hipFree failed");
}

}  // extern "C"
