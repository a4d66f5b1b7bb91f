// Q8_0 GEMV for the MTP head, T = 1 and T = 2 tokens, fp32 accumulation.
//
// Semantics (shaders/mtp.metal:5-20): y[t][n] = sum_b d[n,b] * (sum_i q[n,b,i] * x[t][32b+i]),
// per block the int8 x activation dot in fp32, then acc += d * s.
//
// Design: HBM-bound (1.0625 bytes per weight), so plain VALU fp32 FMAs have ample headroom.
// Each wave owns 4 rows and walks pairs of blocks (68 bytes, dword aligned whenever the row
// holds an even number of blocks, i.e. K % 64 == 0): one lane loads a pair as 17 dwords per
// row and reuses its 64 activations across the 4 rows.  Rows with an odd block count use a
// per-block kernel with 16-bit loads.
#include "common.h"
#include "launch.h"

namespace kata {

namespace {

__device__ inline float byte_s8(uint32_t w, int k) { return (float)(int8_t)(uint8_t)(w >> (8 * k)); }

template <int T, bool XH>
__device__ inline float load_x(const void* x, size_t idx) {
    if (XH) return (float)((const _Float16*)x)[idx];
    return ((const float*)x)[idx];
}

template <int T, bool XH>
__global__ __launch_bounds__(256) void k_gemv_q8_pair(const uint8_t* __restrict__ W, const void* __restrict__ x,
                                                      float* __restrict__ y, int K, int N) {
    constexpr int R = 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row0 = (blockIdx.x * 4 + wave) * R;
    const int nb = K / kQ8Group, np = nb >> 1;
    float acc[T][R];
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[t][r] = 0.0f;

    for (int p = lane; p < np; p += 64) {
        float xv[T][64];
#pragma unroll
        for (int t = 0; t < T; t++) {
            if (XH) {
                const uint4* xp = (const uint4*)((const _Float16*)x + (size_t)t * K + (size_t)p * 64);
#pragma unroll
                for (int c = 0; c < 8; c++) {
                    const uint4 u = xp[c];
                    const uint32_t ws[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                    for (int h = 0; h < 4; h++) {
                        xv[t][c * 8 + 2 * h] = half_bits_to_float(ws[h] & 0xffffu);
                        xv[t][c * 8 + 2 * h + 1] = half_bits_to_float(ws[h] >> 16);
                    }
                }
            } else {
                const float4* xp = (const float4*)((const float*)x + (size_t)t * K + (size_t)p * 64);
#pragma unroll
                for (int c = 0; c < 16; c++) {
                    const float4 u = xp[c];
                    xv[t][4 * c] = u.x; xv[t][4 * c + 1] = u.y; xv[t][4 * c + 2] = u.z; xv[t][4 * c + 3] = u.w;
                }
            }
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = min(row0 + r, N - 1);
            const uint32_t* q = (const uint32_t*)(W + ((size_t)row * nb + 2 * (size_t)p) * kQ8BlockBytes);
            uint32_t wd[17];
#pragma unroll
            for (int i = 0; i < 17; i++) wd[i] = q[i];
            // byte at position pb of the 68-byte pair
#define QB(pb) byte_s8(wd[(pb) >> 2], (pb) & 3)
            const float d0 = half_bits_to_float(wd[0] & 0xffffu);
            const float d1 = half_bits_to_float(wd[8] >> 16);
#pragma unroll
            for (int t = 0; t < T; t++) {
                float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                for (int i = 0; i < 32; i++) s0 += QB(2 + i) * xv[t][i];
#pragma unroll
                for (int i = 0; i < 32; i++) s1 += QB(36 + i) * xv[t][32 + i];
                acc[t][r] += d0 * s0;
                acc[t][r] += d1 * s1;
            }
#undef QB
        }
    }
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int r = 0; r < R; r++) {
            float v = acc[t][r];
            for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
            if (lane == 0 && row0 + r < N) y[(size_t)t * N + row0 + r] = v;
        }
}

// Rows of an odd number of blocks are only 2-byte aligned: one block per lane, 16-bit loads.
template <int T, bool XH>
__global__ __launch_bounds__(256) void k_gemv_q8_block(const uint8_t* __restrict__ W, const void* __restrict__ x,
                                                       float* __restrict__ y, int K, int N) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row = blockIdx.x * 4 + wave;
    if (row >= N) return;
    const int nb = K / kQ8Group;
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] = 0.0f;
    for (int b = lane; b < nb; b += 64) {
        const uint16_t* q = (const uint16_t*)(W + ((size_t)row * nb + b) * kQ8BlockBytes);
        const float d = half_bits_to_float(q[0]);
        float s[T];
#pragma unroll
        for (int t = 0; t < T; t++) s[t] = 0.0f;
        for (int i = 0; i < 16; i++) {
            const uint32_t w = q[1 + i];
#pragma unroll
            for (int t = 0; t < T; t++) {
                s[t] += byte_s8(w, 0) * load_x<T, XH>(x, (size_t)t * K + 32 * (size_t)b + 2 * i);
                s[t] += byte_s8(w, 1) * load_x<T, XH>(x, (size_t)t * K + 32 * (size_t)b + 2 * i + 1);
            }
        }
#pragma unroll
        for (int t = 0; t < T; t++) acc[t] += d * s[t];
    }
#pragma unroll
    for (int t = 0; t < T; t++) {
        float v = acc[t];
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
        if (lane == 0) y[(size_t)t * N + row] = v;
    }
}

template <int T, bool XH>
hipError_t launch_q8_t(const uint8_t* W, const void* x, float* y, int K, int N, hipStream_t s) {
    const int nb = K / kQ8Group;
    if ((nb & 1) == 0 && (((uintptr_t)W) & 3) == 0)
        hipLaunchKernelGGL((k_gemv_q8_pair<T, XH>), dim3((N + 15) / 16), dim3(256), 0, s, W, x, y, K, N);
    else
        hipLaunchKernelGGL((k_gemv_q8_block<T, XH>), dim3((N + 3) / 4), dim3(256), 0, s, W, x, y, K, N);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemv_q8(const uint8_t* W, const void* x, int x_dtype, float* y, int K, int N, int T,
                          hipStream_t s) {
    if (T == 1) return x_dtype == 1 ? launch_q8_t<1, true>(W, x, y, K, N, s) : launch_q8_t<1, false>(W, x, y, K, N, s);
    return x_dtype == 1 ? launch_q8_t<2, true>(W, x, y, K, N, s) : launch_q8_t<2, false>(W, x, y, K, N, s);
}

}  // namespace kata
