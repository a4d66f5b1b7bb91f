// Measurement helpers for the roofline figures (no counterpart in the reference): an empty
// kernel at the decode GEMV's launch geometry (one 1024-thread workgroup per CU) for the
// launch floor, and a plain streaming read of n bytes at the same geometry for the
// achievable HBM read rate at a given size.
//
// The read kernel: each wave streams a contiguous share of the buffer with 16-byte raw
// buffer loads, D in flight per lane, and folds what it read into one word so the loads
// cannot be dropped; bytes past the last whole 1 KB piece of a share are read by the
// share's last wave with the same loads (out-of-range lanes read zero).  Two forms:
//   - the decode GEMV's geometry (1024-thread workgroups, one per CU, ordinary loads);
//   - the read ceiling: the fastest plain read found by a sweep over workgroup size
//     (256/512/1024), workgroups per CU (1/2/4/8), loads in flight (2/4/8/16) and the
//     non-temporal hint (launch_calib_read_cfg, bench.py --calib-sweep), at 19.5 MB, 39 MB
//     and 278 MB: 256-thread workgroups, two per CU, 16-byte non-temporal loads (slc), four
//     in flight.
#include "common.h"
#include "launch.h"

namespace kata {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(1024) void k_calib_empty(uint32_t* out) {
    if (threadIdx.x == 1023 && blockIdx.x == 0x7fffffff) out[0] = 1;
}

template <int BLK, int AUX, int D = 4>
__global__ __launch_bounds__(BLK) void k_calib_read(const uint8_t* __restrict__ p, uint32_t bytes,
                                                    uint32_t* __restrict__ out) {
    constexpr int WPG = BLK / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t nw = gridDim.x * WPG, w = blockIdx.x * WPG + wave;
    const uint32_t pieces = (bytes + 1023) / 1024;            // 1 KB per wave load
    const uint32_t p0 = (uint32_t)(((uint64_t)pieces * w) / nw), p1 = (uint32_t)(((uint64_t)pieces * (w + 1)) / nw);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)p, 0, (int)bytes, 0x00020000);
    auto ld = [&](uint32_t i) -> u32x4 {
        const uint32_t so = i < p1 ? i * 1024u : 0x80000000u;
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, lane * 16, (int)so, AUX));
    };
    u32x4 r[D];
#pragma unroll
    for (int u = 0; u < D; u++) r[u] = ld(p0 + u);
    uint32_t acc = 0;
    for (uint32_t i = p0; i < p1; i += D) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            acc ^= r[u].x + r[u].y + r[u].z + r[u].w;
            r[u] = ld(i + D + u);
        }
    }
    if (acc == 0x9e3779b9u) out[0] = acc;     // practically never: keeps the loads
}

template <int BLK, int AUX, int D>
hipError_t launch_read(const uint8_t* p, uint32_t bytes, uint32_t* out, int wgs, hipStream_t s) {
    hipLaunchKernelGGL((k_calib_read<BLK, AUX, D>), dim3(wgs), dim3(BLK), 0, s, p, bytes, out);
    return hipGetLastError();
}
template <int BLK, int AUX>
hipError_t launch_read_d(const uint8_t* p, uint32_t bytes, uint32_t* out, int wgs, int inflight, hipStream_t s) {
    switch (inflight) {
        case 2: return launch_read<BLK, AUX, 2>(p, bytes, out, wgs, s);
        case 4: return launch_read<BLK, AUX, 4>(p, bytes, out, wgs, s);
        case 8: return launch_read<BLK, AUX, 8>(p, bytes, out, wgs, s);
        default: return launch_read<BLK, AUX, 16>(p, bytes, out, wgs, s);
    }
}
template <int BLK>
hipError_t launch_read_nt(const uint8_t* p, uint32_t bytes, uint32_t* out, int wgs, int inflight, bool nt,
                          hipStream_t s) {
    return nt ? launch_read_d<BLK, 2>(p, bytes, out, wgs, inflight, s) : launch_read_d<BLK, 0>(p, bytes, out, wgs, inflight, s);
}

}  // namespace

hipError_t launch_calib_read_cfg(const uint8_t* p, uint32_t bytes, uint32_t* out, int threads, int wgs, int inflight,
                                 bool nt, hipStream_t s) {
    switch (threads) {
        case 256: return launch_read_nt<256>(p, bytes, out, wgs, inflight, nt, s);
        case 512: return launch_read_nt<512>(p, bytes, out, wgs, inflight, nt, s);
        default: return launch_read_nt<1024>(p, bytes, out, wgs, inflight, nt, s);
    }
}

hipError_t launch_calib_empty(uint32_t* out, int wgs, hipStream_t s) {
    hipLaunchKernelGGL(k_calib_empty, dim3(wgs), dim3(1024), 0, s, out);
    return hipGetLastError();
}

hipError_t launch_calib_read(const uint8_t* p, uint32_t bytes, uint32_t* out, int wgs, hipStream_t s) {
    hipLaunchKernelGGL((k_calib_read<1024, 0>), dim3(wgs), dim3(1024), 0, s, p, bytes, out);
    return hipGetLastError();
}

hipError_t launch_calib_read_peak(const uint8_t* p, uint32_t bytes, uint32_t* out, int cus, hipStream_t s) {
    // aux 2 = slc: the non-temporal hint on the load
    hipLaunchKernelGGL((k_calib_read<256, 2>), dim3(2 * cus), dim3(256), 0, s, p, bytes, out);
    return hipGetLastError();
}

}  // namespace kata
