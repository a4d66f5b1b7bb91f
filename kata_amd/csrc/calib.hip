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
// A third kernel replays the decode GEMV's weight-load stream alone (k_gemv_ptq1, one
// matrix, T = 1): the reads of its loop with the decode, the matrix-core work and the item
// sums left out, which is what that loop could reach if the rest of each item were free.
#include "common.h"
#include "gemv_operand.h"
#include "launch.h"

namespace kata {

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));

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

// The decode GEMV's weight loads for one matrix (gemv_ptq1.hip, k_gemv_ptq1 with T = 1):
// one 1024-thread workgroup per CU owns tpw tiles of 4 rows; its 16 waves walk the items
// (4 consecutive blocks of the tile's 4 rows) in the kernel's run order, or its tile-strided
// order when `strided` (wave w: step pair w % np of tiles h, h + G, ...; h = w / np,
// G = 16 / np); each lane loads the same 12 bytes (row x & 3, block x >> 2 of the step, the
// lane group's window at gemv_dense_byte0) into a ring of 4 items, and item u + 1 is read
// before slot u is reloaded, as in the kernel.
__global__ __launch_bounds__(1024) void k_calib_read_ptq1(const uint8_t* __restrict__ W, int N, int nb, int tpw,
                                                           int strided_ok, uint32_t* __restrict__ out) {
    constexpr int D = 4;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int x_ = lane & 15, g = lane >> 4;
    const int nq = gemv_nq(nb * kGroup), np = nq >> 1, G = 16 / np;
    const int tiles = (N + 3) >> 2, wt0 = (int)blockIdx.x * tpw, Tt = min(tiles, wt0 + tpw) - wt0;
    const uint32_t row_bytes = (uint32_t)nb * kBlockBytes, tstep = 4 * row_bytes, cstep = 4 * kBlockBytes;
    const bool strided = strided_ok && Tt >= 2 * G;
    int n, lt, Tw;
    uint32_t lso, tnext, cwrap;
    if (strided) {
        const int sp = wave % np, sh = wave / np;
        n = wave < G * np && sh < Tt ? 2 * ((Tt - sh + G - 1) / G) : 0;
        lt = sh;
        lso = (uint32_t)(wt0 + sh) * tstep + (uint32_t)(2 * sp) * cstep;
        Tw = 0x7fffffff;
        tnext = (uint32_t)G * tstep - cstep;
        cwrap = 0;
    } else {
        const int S = nq * Tt;
        const int s0 = ((wave * S) / 16) & ~1, s1 = wave == 15 ? S : (((wave + 1) * S) / 16) & ~1;
        n = s1 - s0;
        lt = (s0 % (2 * Tt)) >> 1;
        lso = (uint32_t)(wt0 + lt) * tstep + (uint32_t)(2 * (s0 / (2 * Tt))) * cstep;
        Tw = Tt;
        tnext = tstep - cstep;
        cwrap = cstep - (uint32_t)(Tt - 1) * tstep;
    }
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)W, 0, (int)((uint32_t)N * row_bytes), 0x00020000);
    const uint32_t voff = (uint32_t)(x_ & 3) * row_bytes + (uint32_t)(x_ >> 2) * kBlockBytes + (uint32_t)gemv_dense_byte0(g);
    int lrem = n, par = 0;
    // past the wave's items: an offset beyond the buffer (zeros, no memory access)
    auto ld = [&]() -> u32x4 {
        const uint32_t so = lrem > 0 ? lso : 0x80000000u;
        const u32x3 v = __builtin_bit_cast(u32x3, __builtin_amdgcn_raw_buffer_load_b96(rs, (int)voff, (int)so, 0));
        if (par) {
            const bool wrap = ++lt == Tw;
            lt = wrap ? 0 : lt;
            lso += wrap ? cwrap : tnext;
        } else {
            lso += cstep;
        }
        par ^= 1;
        --lrem;
        return u32x4{v.x, v.y, v.z, 0u};
    };
    u32x4 ring[D];
#pragma unroll
    for (int u = 0; u < D; u++) ring[u] = ld();
    uint32_t acc = ring[0].x + ring[0].y + ring[0].z;
    for (int j = 0; j < n; j += D) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            const int v = (u + 1) % D;
            acc ^= ring[v].x + ring[v].y + ring[v].z;
            ring[u] = ld();
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

// The decode GEMV's split for one matrix at one workgroup per CU, and its rule for the
// tile-strided order at T = 1 (gemv_ptq1.hip, gemv_strided: whole step pairs of 8 blocks,
// 15 or 16 waves busy, >= 64 tiles per workgroup, G <= 12 for the scratch slots).
hipError_t launch_calib_read_ptq1(const uint8_t* W, int K, int N, uint32_t* out, int cus, hipStream_t s) {
    const int nb = K / kGroup, np = gemv_nq(K) / 2, G = np > 0 ? 16 / np : 0;
    const int tiles = (N + 3) / 4, tpw = (tiles + cus - 1) / cus, wgs = (tiles + tpw - 1) / tpw;
    const int strided = nb % 8 == 0 && np > 0 && G >= 2 && G * np >= 15 && tpw >= 64 && G * 64 + 256 <= 1024;
    hipLaunchKernelGGL(k_calib_read_ptq1, dim3(wgs), dim3(1024), 0, s, W, N, nb, tpw, strided, out);
    return hipGetLastError();
}

}  // namespace kata
