// Per-(device, stream) device buffers of the kernels that need scratch memory beyond their
// inputs and outputs: the prefill GEMMs' and the wide GEMV's K-piece partial sums, and the
// argmax's per-workgroup bests.  Each buffer is allocated on the first call on its (device,
// stream, kind) that needs it and kept until the process ends, so calls on different
// streams never share scratch memory; calls on one stream are ordered by the stream.
#include "launch.h"

#include <map>
#include <mutex>
#include <tuple>

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

hipError_t stream_buffer(int kind, size_t bytes, hipStream_t s, void** p) {
    static std::map<std::tuple<int, int, hipStream_t>, std::pair<void*, size_t>> tab;
    static std::mutex mu;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(mu);
    auto& ent = tab[std::make_tuple(dev, kind, s)];
    if (ent.second < bytes) {
        if (ent.first) {
            // a larger buffer: the old one may still be read by work queued on s
            if ((e = hipStreamSynchronize(s)) != hipSuccess) return e;
            if ((e = hipFree(ent.first)) != hipSuccess) return e;
            ent = {nullptr, 0};
        }
        // an allocation cannot be recorded into a graph: the first call on a stream that
        // needs this buffer (or a larger one) has to run outside capture
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if ((e = hipStreamIsCapturing(s, &cs)) != hipSuccess) return e;
        if (cs != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
        void* q = nullptr;
        if ((e = hipMalloc(&q, bytes)) != hipSuccess) return e;
        ent = {q, bytes};
    }
    *p = ent.first;
    return hipSuccess;
}

}  // namespace kata
