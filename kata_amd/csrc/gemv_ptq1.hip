// PTQ1_0 decode GEMV for T = 1 and T = 2 tokens on the gfx950 int8 matrix cores.
//
// Semantics: y[t][n] = sum_b d[n,b] * sum_e trit[n,b,e] * x[t][128b+e]
// (shaders/gemv.metal:5-20; fast forms shaders/gemv_fast.metal:9-50, shaders/mtp.metal:164-205).
//
// Design (MI355X-first, not the reference's simdgroup g/c float decode):
//  * The weight bytes are never expanded in memory.  Each wave owns 16 output rows; per
//    128-weight block every lane loads 8 bytes of one row and turns each byte into its 5
//    base-3 digits {0,1,2} with one LDS lookup (256-entry table, 8 bytes per entry, 32
//    replicas so a wave's lookups spread over all banks).  Digits feed
//    v_mfma_i32_16x16x64_i8 as the B operand (B[k][row]).
//  * The activation enters as the A operand (A[i][k]) in a prepared integer form: per
//    128-block a scale s = amax/32639 and q = rint(x/s) split into two int8 limbs
//    (q = 256*hi + lo); A rows are (token, limb).  The matrix core accumulates exact int32
//    sums of digit*limb; the epilogue forms sum(trit*q) = 256*D_hi + D_lo - sum(q) per
//    block and token, then y += d * s * that (fp32).  The only approximation is the 16-bit
//    block-fixed-point activation (|x - s*q| <= s/2 = amax/65278), far inside the 1e-3
//    relative-L2 contract.
//  * A row tile of 16 rows reuses the prepared activation registers for all its rows; the
//    prepared activation (512*T bytes per block) is shared by every wave through L2.
#include "common.h"
#include "launch.h"

namespace kata {

namespace {

constexpr int kLutReplicas = 32;
constexpr float kQMax = 32639.0f;   // |q| <= 32639 keeps hi = (q+128)>>8 inside int8

// Per (lane group g, MFMA m) the first of the two block bytes a lane feeds to the matrix
// core; -1 = no byte (the activation is zero there).  Lane group 0 holds bytes 20..27 so
// that the row scale (bytes 26..27) sits in the lanes that also hold the result rows.
__host__ __device__ inline int gemv_first_byte(int g, int m) {
    return g == 0 ? 20 + 2 * m : g == 1 ? 2 * m : g == 2 ? 8 + 2 * m : (m < 2 ? 16 + 2 * m : -1);
}

template <int T>
__global__ __launch_bounds__(128) void k_gemv_prep(const void* __restrict__ x, int x_dtype, int x_layout,
                                                   uint8_t* __restrict__ xprep, int K, size_t off_sq,
                                                   size_t off_a) {
    __shared__ int16_t qs[T][128];
    __shared__ float red_f[2][T];
    __shared__ int red_i[2][T];
    const int b = blockIdx.x, e = threadIdx.x, lane = e & 63, wv = e >> 6;
    float v[T];
#pragma unroll
    for (int t = 0; t < T; t++) {
        const size_t idx = x_layout == 1 ? ((size_t)b * 128 + e) * 2 + t : (size_t)t * K + (size_t)b * 128 + e;
        v[t] = x_dtype == 1 ? (float)((const _Float16*)x)[idx] : ((const float*)x)[idx];
        float a = fabsf(v[t]);
        for (int o = 32; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o));
        if (lane == 0) red_f[wv][t] = a;
    }
    __syncthreads();
    int q[T];
#pragma unroll
    for (int t = 0; t < T; t++) {
        const float amax = fmaxf(red_f[0][t], red_f[1][t]);
        const float inv = amax > 0.0f ? kQMax / amax : 0.0f;
        float r = rintf(v[t] * inv);
        r = fminf(fmaxf(r, -kQMax), kQMax);
        q[t] = (int)r;
        qs[t][e] = (int16_t)q[t];
        int s = q[t];
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
        if (lane == 0) red_i[wv][t] = s;
        if (e == 0) ((float*)xprep)[b * T + t] = amax / kQMax;
    }
    __syncthreads();
    if (e < T) ((int*)(xprep + off_sq))[b * T + e] = red_i[0][e] + red_i[1][e];
    // A operand image: [m 4][g 4][i 2T][16 bytes]; i = 2*t + limb; bytes 0..7 = digits 0..7
    // of the lane's first byte, 8..15 of its second (digits 5..7 are padding).
    uint32_t* out = (uint32_t*)(xprep + off_a + (size_t)b * 512 * T);
    for (int w = e; w < 128 * T; w += 128) {
        const int dw = w & 3, i = (w >> 2) % (2 * T), g = (w / (8 * T)) & 3, m = w / (32 * T);
        const int t = i >> 1, limb = i & 1;
        const int p0 = gemv_first_byte(g, m);
        uint32_t word = 0;
        if (p0 >= 0) {
            const int p = p0 + (dw >> 1);
#pragma unroll
            for (int kb = 0; kb < 4; kb++) {
                const int el = ptq1_slot_elem(p, (dw & 1) * 4 + kb);
                if (el >= 0) {
                    const int qq = qs[t][el];
                    const int hi = (qq + 128) >> 8, lo = qq - 256 * hi;
                    word |= (uint32_t)(uint8_t)(int8_t)(limb ? lo : hi) << (8 * kb);
                }
            }
        }
        out[w] = word;
    }
}

template <int T>
__global__ __launch_bounds__(256) void k_gemv_ptq1(const uint8_t* __restrict__ W, const uint8_t* __restrict__ xprep,
                                                   float* __restrict__ y, int K, int N, size_t off_sq,
                                                   size_t off_a) {
    __shared__ uint2 lut[256 * kLutReplicas];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, g = lane >> 4;
    const int nb = K >> 7;
    const int row = (blockIdx.x * 4 + wave) * 16 + j;
    const int rowc = row < N ? row : N - 1;
    const int off_g = g == 0 ? 20 : g == 1 ? 0 : g == 2 ? 8 : 12;
    const uint8_t* wp = W + (size_t)rowc * nb * kBlockBytes + off_g;

    // first block's bytes in flight while the table is built
    uint32_t w0 = ((const uint32_t*)wp)[0], w1 = ((const uint32_t*)wp)[1];

    for (int idx = tid; idx < 256 * kLutReplicas; idx += 256) {
        const uint32_t bv = (uint32_t)idx / kLutReplicas;
        const uint32_t lo = ptq1_digit(bv, 0) | (ptq1_digit(bv, 1) << 8) | (ptq1_digit(bv, 2) << 16) |
                            (ptq1_digit(bv, 3) << 24);
        lut[idx] = make_uint2(lo, ptq1_digit(bv, 4));
    }
    __syncthreads();

    const uint32_t laneoff = (uint32_t)(lane & (kLutReplicas - 1)) * 8u;
    const float* sx = (const float*)xprep;
    const int* sq = (const int*)(xprep + off_sq);
    const bool a_active = j < 2 * T;
    const uint8_t* xa = xprep + off_a + (size_t)g * (2 * T * 16) + (size_t)j * 16;
    const char* lutb = (const char*)lut;

    float acc[T];
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] = 0.0f;

    for (int b = 0; b < nb; ++b) {
        const uint32_t c0 = w0, c1 = w1;
        if (b + 1 < nb) {
            const uint32_t* nq = (const uint32_t*)(wp + (size_t)(b + 1) * kBlockBytes);
            w0 = nq[0];
            w1 = nq[1];
        }
        v4i av[4];
#pragma unroll
        for (int m = 0; m < 4; m++) {
            av[m] = v4i{0, 0, 0, 0};
            if (a_active) av[m] = *(const v4i*)(xa + (size_t)(b * 4 + m) * (4 * 2 * T * 16));
        }
        const uint32_t lo = g == 3 ? c1 : c0, hi = g == 3 ? c0 : c1;
        v4i D = {0, 0, 0, 0};
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const uint32_t w = m < 2 ? lo : hi;
            const int sh = (m & 1) * 16;
            const uint32_t a0 = (((w >> sh) & 0xffu) << 8) | laneoff;
            const uint32_t a1 = (((w >> (sh + 8)) & 0xffu) << 8) | laneoff;
            const uint2 e0 = *(const uint2*)(lutb + a0);
            const uint2 e1 = *(const uint2*)(lutb + a1);
            const v4i bv = {(int)e0.x, (int)e0.y, (int)e1.x, (int)e1.y};
            D = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[m], bv, D, 0, 0, 0);
        }
        const float d = half_bits_to_float(c1 >> 16);
#pragma unroll
        for (int t = 0; t < T; t++) {
            const int v = D[2 * t] * 256 + D[2 * t + 1] - sq[b * T + t];
            acc[t] += (d * sx[b * T + t]) * (float)v;
        }
    }
    if (g == 0 && row < N) {
#pragma unroll
        for (int t = 0; t < T; t++) y[(size_t)t * N + row] = acc[t];
    }
}

}  // namespace

XprepLayout xprep_layout(int K, int T) {
    const size_t nb = (size_t)K / kGroup;
    XprepLayout L;
    L.off_sx = 0;
    L.off_sq = ((nb * T * 4) + 255) & ~(size_t)255;
    L.off_a = (L.off_sq + nb * T * 4 + 255) & ~(size_t)255;
    L.bytes = L.off_a + nb * 512 * (size_t)T;
    return L;
}

hipError_t launch_gemv_prep(const void* x, int x_dtype, int x_layout, uint8_t* xprep, int K, int T,
                            hipStream_t s) {
    const XprepLayout L = xprep_layout(K, T);
    const dim3 grid(K / kGroup), block(128);
    if (T == 1)
        hipLaunchKernelGGL(k_gemv_prep<1>, grid, block, 0, s, x, x_dtype, x_layout, xprep, K, L.off_sq, L.off_a);
    else
        hipLaunchKernelGGL(k_gemv_prep<2>, grid, block, 0, s, x, x_dtype, x_layout, xprep, K, L.off_sq, L.off_a);
    return hipGetLastError();
}

hipError_t launch_gemv_ptq1(const uint8_t* W, const uint8_t* xprep, float* y, int K, int N, int T,
                            hipStream_t s) {
    const XprepLayout L = xprep_layout(K, T);
    const dim3 grid((N + 63) / 64), block(256);
    if (T == 1)
        hipLaunchKernelGGL(k_gemv_ptq1<1>, grid, block, 0, s, W, xprep, y, K, N, L.off_sq, L.off_a);
    else
        hipLaunchKernelGGL(k_gemv_ptq1<2>, grid, block, 0, s, W, xprep, y, K, N, L.off_sq, L.off_a);
    return hipGetLastError();
}

}  // namespace kata
