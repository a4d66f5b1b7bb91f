// Standalone PTQ1_0 expansions in natural [N][K] order (verification and catch-up uses).
// k_expand_ptq1_v2 / k_expand_i8_v2 semantics (shaders/prefill.metal:457-479):
//   out[n][k] = half(trit * d) exactly;  T8[n][k] = trit;  SW[n][k/128] = d.
// One thread per (row, block, byte pair): the pair's 4-5 digits give adjacent-k weights.
#include "common.h"
#include "launch.h"

namespace kata {

namespace {

template <bool I8>
__global__ __launch_bounds__(256) void k_expand(const uint8_t* __restrict__ W, void* __restrict__ out,
                                                float* __restrict__ SW, int K, int N) {
    const int nb = K / kGroup;
    const size_t id = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t total = (size_t)N * nb * 13;
    if (id >= total) return;
    const int pr = (int)(id % 13);
    const size_t blkid = id / 13;
    const int n = (int)(blkid / nb), b = (int)(blkid % nb);
    const uint8_t* blk = W + blkid * kBlockBytes;
    const int p = 2 * pr;
    const uint32_t b0 = blk[p], b1 = blk[p + 1];
    const float d = half_bits_to_float(*(const uint16_t*)(blk + 26));
    const int nd = p < 24 ? 5 : 4;
    for (int dg = 0; dg < nd; dg++) {
        const int e = ptq1_slot_elem(p, dg);
        const int t0 = (int)ptq1_digit(b0, dg) - 1, t1 = (int)ptq1_digit(b1, dg) - 1;
        const size_t k = (size_t)n * K + (size_t)b * kGroup + e;
        if (I8) {
            ((int8_t*)out)[k] = (int8_t)t0;
            ((int8_t*)out)[k + 1] = (int8_t)t1;
        } else {
            ((_Float16*)out)[k] = (_Float16)((float)t0 * d);
            ((_Float16*)out)[k + 1] = (_Float16)((float)t1 * d);
        }
    }
    if (I8 && pr == 0) SW[(size_t)n * nb + b] = d;
}

}  // namespace

hipError_t launch_expand_f16(const uint8_t* W, uint16_t* out, int K, int N, hipStream_t s) {
    const size_t total = (size_t)N * (K / kGroup) * 13;
    hipLaunchKernelGGL(k_expand<false>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, W, (void*)out,
                       (float*)nullptr, K, N);
    return hipGetLastError();
}

hipError_t launch_expand_i8(const uint8_t* W, int8_t* T8, float* SW, int K, int N, hipStream_t s) {
    const size_t total = (size_t)N * (K / kGroup) * 13;
    hipLaunchKernelGGL(k_expand<true>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, W, (void*)T8, SW,
                       K, N);
    return hipGetLastError();
}

}  // namespace kata
