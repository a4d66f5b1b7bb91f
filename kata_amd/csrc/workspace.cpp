// Per-(device, stream) device buffers of the kernels that need scratch memory beyond their
// inputs and outputs: the prefill GEMMs' and the wide GEMV's K-piece partial sums, and the
// argmax's per-workgroup bests.  Each buffer is allocated on the first call on its (device,
// stream, kind) that needs it, so calls on different streams never share scratch memory;
// calls on one stream are ordered by the stream.
//
// A buffer is never freed while the stream may still use it: when a call needs a larger
// buffer than the stream holds, the smaller one is retired, not freed, because a HIP graph
// captured earlier on the stream records its address and may be replayed after the larger
// call.  Retired and current buffers of a stream are freed only by release_stream (the
// caller's promise that the stream's graphs are gone and its work is done).
#include "launch.h"

#include <map>
#include <mutex>
#include <tuple>
#include <vector>

namespace kata {

hipError_t device_cu_count(int* n_cu) {
    static int tab[64] = {};
    static std::mutex mu;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!tab[dev]) {
        int n = 0;
        e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        tab[dev] = n > 0 ? n : 256;
    }
    *n_cu = tab[dev];
    return hipSuccess;
}

namespace {
struct StreamBufs {
    std::map<int, std::pair<void*, size_t>> cur;   // kind -> (buffer, bytes)
    std::vector<void*> retired;                    // outgrown buffers, still referenced by graphs
};
std::map<std::pair<int, hipStream_t>, StreamBufs>& table() {
    static std::map<std::pair<int, hipStream_t>, StreamBufs> tab;
    return tab;
}
std::mutex& table_mutex() {
    static std::mutex mu;
    return mu;
}
}  // namespace

hipError_t stream_buffer(int kind, size_t bytes, hipStream_t s, void** p) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(table_mutex());
    StreamBufs& sb = table()[std::make_pair(dev, s)];
    auto& ent = sb.cur[kind];
    if (ent.second < bytes) {
        // an allocation cannot be recorded into a graph: the first call on a stream that
        // needs this buffer (or a larger one) has to run outside capture.  Checked before
        // anything else touches the stream, so a capture is not invalidated.
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if ((e = hipStreamIsCapturing(s, &cs)) != hipSuccess) return e;
        if (cs != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
        void* q = nullptr;
        if ((e = hipMalloc(&q, bytes)) != hipSuccess) return e;
        if (ent.first) sb.retired.push_back(ent.first);
        ent = {q, bytes};
    }
    *p = ent.first;
    return hipSuccess;
}

hipError_t release_stream(hipStream_t s) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(table_mutex());
    auto it = table().find(std::make_pair(dev, s));
    if (it == table().end()) return hipSuccess;
    if ((e = hipStreamSynchronize(s)) != hipSuccess) return e;
    hipError_t first = hipSuccess;
    for (auto& kv : it->second.cur)
        if (kv.second.first) {
            hipError_t f = hipFree(kv.second.first);
            if (first == hipSuccess) first = f;
        }
    for (void* q : it->second.retired) {
        hipError_t f = hipFree(q);
        if (first == hipSuccess) first = f;
    }
    table().erase(it);
    return first;
}

}  // namespace kata
