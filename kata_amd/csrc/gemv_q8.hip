// Q8_0 GEMV for the MTP head, T = 1 and T = 2 tokens, fp32 accumulation.
//
// Semantics (shaders/mtp.metal:5-20): y[t][n] = sum_b d[n,b] * (sum_i q[n,b,i] * x[t][32b+i]),
// per block the int8 x activation dot in fp32, then acc += d * s.
//
// Design: HBM-bound (1.0625 bytes per weight).  One fp16 activation row: each pair of quants
// becomes an exact fp16 pair (a byte permute and a packed add) and v_dot2_f32_f16 multiplies
// it with the activation pair, accumulating in fp32 (27.4 -> 26.4 us at 17408 x 5120; for two
// rows this form was slower, 28.8 -> 35.5 us); otherwise fp32 FMAs per quant.  A lane owns
// whole 34-byte blocks and consecutive lanes own consecutive blocks of a row, so each load
// instruction of a wave covers 2176 contiguous bytes.  A block is read from its
// dword-aligned start as two 16-byte loads, one dword and one 16-bit load (blocks sit at
// 2-byte granularity) and realigned with v_alignbyte.  A wave owns R rows (2 for one
// activation row, 4 for two) and one of KS slices of K, and reuses each block's activations
// (loaded once into registers) for its R rows; the KS waves of a workgroup that share rows
// add their partial sums through LDS in a fixed order (deterministic).
#include "common.h"
#include "launch.h"

#include <algorithm>

namespace kata {

namespace {


__device__ inline float byte_s8(uint32_t w, int k) { return (float)(int8_t)(uint8_t)(w >> (8 * k)); }

// 32 activations x[t][32b .. 32b+31] as floats (fp16 or fp32 rows)
template <int T, bool XH>
__device__ inline void load_x32(const void* x, int K, int b, float (&xv)[T][32]) {
#pragma unroll
    for (int t = 0; t < T; t++) {
        if (XH) {
            const uint4* p = (const uint4*)((const _Float16*)x + (size_t)t * K + (size_t)b * 32);
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint4 u = p[c];
                const uint32_t ws[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int h = 0; h < 4; h++) {
                    const v2h hh = __builtin_bit_cast(v2h, ws[h]);
                    xv[t][c * 8 + 2 * h] = (float)hh[0];
                    xv[t][c * 8 + 2 * h + 1] = (float)hh[1];
                }
            }
        } else {
            const float4* p = (const float4*)((const float*)x + (size_t)t * K + (size_t)b * 32);
#pragma unroll
            for (int c = 0; c < 8; c++) {
                const float4 u = p[c];
                xv[t][4 * c] = u.x;
                xv[t][4 * c + 1] = u.y;
                xv[t][4 * c + 2] = u.z;
                xv[t][4 * c + 3] = u.w;
            }
        }
    }
}

constexpr int kQ8MaxMats = 4;
constexpr int kQ8XlMax = 96 * 1024;   // largest activation copy in LDS (T = 2)
constexpr int kQ8XlRows = 2;          // rows per wave with the LDS copy
constexpr int kQ8XlWaves = 8;         // waves per workgroup with the LDS copy (4 without)

// The 1..4 matrices of one launch (same K, same activation): matrix i is W[i] - w_off[i]
// (its dword-aligned base; w_off[i] = W[i] & 3) with N[i] rows and w_bytes[i] bytes from that
// base, output y[i] [T][N[i]]; workgroups [wg0[i], wg0[i+1]) serve it.
struct Q8Mats {
    const uint8_t* W[kQ8MaxMats];
    float* y[kQ8MaxMats];
    int N[kQ8MaxMats];
    uint32_t w_off[kQ8MaxMats];
    uint32_t w_bytes[kQ8MaxMats];
    int lks[kQ8MaxMats];                         // log2 of the matrix's K slices per row group
    int wg0[kQ8MaxMats + 1];
    int count;
};

// Workgroup = 4 waves = (4 / KS) row groups x KS slices of the row's blocks (KS per matrix,
// the same as a launch of that matrix alone, so a batch equals the single launches bit for bit).
// XL: the activation rows are copied into LDS once per workgroup and every wave reads its
// blocks' activations from there (8 waves: at T = 2 one K slice, 8 row groups; at T = 1 each
// matrix's own K slices; 8 waves copy half as much per row as 4, 24.1 -> 23.5 us at 17408 x
// 5120 T = 2, 16 were slower), instead of each row group reading them from L2.
template <int T, bool XH, int R, bool MULTI, bool XL>
__global__ __launch_bounds__(XL ? kQ8XlWaves * 64 : 256) void k_gemv_q8(Q8Mats P, const void* __restrict__ xg, int K) {
    constexpr int WV = XL ? kQ8XlWaves : 4;
    __shared__ float red[WV][T][R];
    extern __shared__ __align__(16) uint8_t xlds[];
    const void* __restrict__ x = XL ? (const void*)xlds : xg;
    if constexpr (XL) {
        const int n16 = T * K * (XH ? 2 : 4) / 16;
        for (int i = threadIdx.x; i < n16; i += WV * 64) ((uint4*)xlds)[i] = ((const uint4*)xg)[i];
        __syncthreads();
    }
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // this workgroup's matrix: every field is read before one is selected (no branches
    // around dependent argument loads)
    const uint8_t* __restrict__ W = P.W[0];
    float* __restrict__ y = P.y[0];
    int N = P.N[0], wg0 = 0, lks = P.lks[0];
    uint32_t w_off = P.w_off[0], w_bytes = P.w_bytes[0];
    if constexpr (MULTI) {
#pragma unroll
        for (int i = 1; i < kQ8MaxMats; i++) {
            const bool sel = i < P.count && (int)blockIdx.x >= P.wg0[i];
            W = sel ? P.W[i] : W;
            y = sel ? P.y[i] : y;
            N = sel ? P.N[i] : N;
            w_off = sel ? P.w_off[i] : w_off;
            w_bytes = sel ? P.w_bytes[i] : w_bytes;
            lks = sel ? P.lks[i] : lks;
            wg0 = sel ? P.wg0[i] : wg0;
        }
    }
    const int KS = 1 << lks, GROUPS = WV >> lks;
    const int grp = wave >> lks, ks = wave & (KS - 1);
    const int row0 = (((int)blockIdx.x - wg0) * GROUPS + grp) * R;
    const int nb = K / kQ8Group;
    const int b0 = (ks * nb) / KS, b1 = ((ks + 1) * nb) / KS;
    const uint32_t row_bytes = (uint32_t)nb * kQ8BlockBytes;
    // W as a raw buffer from its dword-aligned base (w_off = W & 3); exact bounds
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc((void*)W, 0, (int)w_bytes, 0x00020000);

    float acc[T][R];
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[t][r] = 0.0f;

    // all loads of a block step (4 rows) are issued before its arithmetic
    for (int b = b0 + lane; b < b1; b += 64) {
        uint32_t s[R][9];
        float d[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = min(row0 + r, N - 1);
            const uint32_t base = w_off + (uint32_t)row * row_bytes + (uint32_t)b * kQ8BlockBytes;
            const uint32_t sh = base & 3u, a0 = base - sh;
            typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
            const u32x4 lo = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)a0, 0, 0));
            const u32x4 hi = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, (int)(a0 + 16), 0, 0));
            // block bytes 30..33: the dword at a0 + 32 ends at the block's end when sh = 2
            // (with sh = 0 it would pass it, and past the matrix for the last block: the
            // bounds check returns zeros there, and bytes 32..33 come from a 16-bit load)
            const uint32_t w8 = __builtin_amdgcn_raw_buffer_load_b32(rsrc, (int)(a0 + 32), 0, 0);
            const uint32_t h16 = __builtin_amdgcn_raw_buffer_load_b16(rsrc, (int)(base + 32), 0, 0);
            const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
            // stream s[i] = block bytes 4i .. 4i+3: s[0] = {d, d, q0, q1}, s[i] = q(4i-2) ..,
            // s[8] = {q30, q31}
#pragma unroll
            for (int i = 0; i < 7; i++) s[r][i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
            s[r][7] = __builtin_amdgcn_alignbyte(w8, w[7], sh);
            s[r][8] = h16;
        }
        if constexpr (XH && T == 1) {
            // fp16 activations: pairs of quants as exact fp16 pairs and v_dot2_f32_f16 (the
            // fp16 products are exact in fp32).  Pair m = (q 2m, q 2m+1) sits in bytes 2, 3 of
            // s[0] (m = 0), bytes 0, 1 / 2, 3 of s[i] (m = 2i-1 / 2i) and bytes 0, 1 of s[8]
            // (m = 15).  A byte u = q ^ 0x80 under a 0x64 high byte is the fp16 1152 + q.
            uint32_t xp[T][16];
#pragma unroll
            for (int t = 0; t < T; t++) {
                const uint4* p = (const uint4*)((const _Float16*)x + (size_t)t * K + (size_t)b * 32);
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const uint4 u = p[c];
                    xp[t][4 * c] = u.x;
                    xp[t][4 * c + 1] = u.y;
                    xp[t][4 * c + 2] = u.z;
                    xp[t][4 * c + 3] = u.w;
                }
            }
            const v2h off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
            auto pair = [&](uint32_t w, bool hi) {
                const uint32_t v = __builtin_amdgcn_perm(0x64646464u, w ^ 0x80808080u, hi ? 0x04030402u : 0x04010400u);
                return __builtin_bit_cast(v2h, v) + off;
            };
#pragma unroll
            for (int r = 0; r < R; r++) {
                d[r] = half_bits_to_float(s[r][0] & 0xffffu);
                v2h qp[16];
                qp[0] = pair(s[r][0], true);
#pragma unroll
                for (int i = 1; i < 8; i++) {
                    qp[2 * i - 1] = pair(s[r][i], false);
                    qp[2 * i] = pair(s[r][i], true);
                }
                qp[15] = pair(s[r][8], false);
#pragma unroll
                for (int t = 0; t < T; t++) {
                    float sum = 0.0f;
#pragma unroll
                    for (int m = 0; m < 16; m++) sum = __builtin_amdgcn_fdot2(qp[m], __builtin_bit_cast(v2h, xp[t][m]), sum, false);
                    acc[t][r] += d[r] * sum;
                }
            }
        } else {
            float xv[T][32];
            load_x32<T, XH>(x, K, b, xv);
#pragma unroll
            for (int r = 0; r < R; r++) {
                d[r] = half_bits_to_float(s[r][0] & 0xffffu);
#pragma unroll
                for (int t = 0; t < T; t++) {
                    float sum = 0.0f;
#pragma unroll
                    for (int k = 0; k < 32; k++) sum += byte_s8(s[r][(k + 2) >> 2], (k + 2) & 3) * xv[t][k];
                    acc[t][r] += d[r] * sum;
                }
            }
        }
    }
    // wave sums (fixed butterfly), then the KS slices in slice order
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int r = 0; r < R; r++) {
            float v = acc[t][r];
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
            acc[t][r] = v;
        }
    if (KS == 1) {
        if (lane < T * R) {
            const int t = lane / R, r = lane % R;
            float v = 0.0f;
#pragma unroll
            for (int tt = 0; tt < T; tt++)
#pragma unroll
                for (int rr = 0; rr < R; rr++)
                    if (tt == t && rr == r) v = acc[tt][rr];
            if (row0 + r < N) y[(size_t)t * N + row0 + r] = v;
        }
        return;
    }
    if (lane == 0) {
#pragma unroll
        for (int t = 0; t < T; t++)
#pragma unroll
            for (int r = 0; r < R; r++) red[wave][t][r] = acc[t][r];
    }
    __syncthreads();
    if (ks == 0 && lane < T * R) {
        const int t = lane / R, r = lane % R;
        float v = 0.0f;
#pragma unroll
        for (int k2 = 0; k2 < 4; k2++)
            if (k2 < KS) v += red[wave + k2][t][r];
        if (row0 + r < N) y[(size_t)t * N + row0 + r] = v;
    }
}

template <int T, bool XH, int R>
hipError_t launch_q8_r(Q8Mats& P, const void* x, int K, bool xl, hipStream_t s) {
    const int nb = K / kQ8Group;
    const int xbytes = T * K * (XH ? 2 : 4);
    P.wg0[0] = 0;
    for (int i = 0; i < P.count; i++) {
        const int N = P.N[i];
        P.lks[i] = (xl && T == 2) ? 0 : (T == 1 && nb >= 256) ? 1 : (nb >= 256 || (nb >= 128 && (T == 2 || N < 8192))) ? 2 : 0;
        const int rpw = R * ((xl ? kQ8XlWaves : 4) >> P.lks[i]);     // rows per workgroup
        P.wg0[i + 1] = P.wg0[i] + (N + rpw - 1) / rpw;
    }
    for (int i = P.count; i < kQ8MaxMats; i++) P.wg0[i + 1] = P.wg0[P.count];
    if (xl) {
        // the dynamic-LDS limit of both instantiations, raised once per process
        static const hipError_t attr = [] {
            hipError_t e = hipFuncSetAttribute((const void*)k_gemv_q8<T, XH, R, true, true>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, kQ8XlMax);
            if (e == hipSuccess)
                e = hipFuncSetAttribute((const void*)k_gemv_q8<T, XH, R, false, true>,
                                        hipFuncAttributeMaxDynamicSharedMemorySize, kQ8XlMax);
            return e;
        }();
        if (attr != hipSuccess) return attr;
        if (P.count > 1)
            hipLaunchKernelGGL((k_gemv_q8<T, XH, R, true, true>), dim3(P.wg0[P.count]), dim3(kQ8XlWaves * 64), xbytes, s, P, x, K);
        else
            hipLaunchKernelGGL((k_gemv_q8<T, XH, R, false, true>), dim3(P.wg0[P.count]), dim3(kQ8XlWaves * 64), xbytes, s, P, x, K);
    } else if (P.count > 1) {
        hipLaunchKernelGGL((k_gemv_q8<T, XH, R, true, false>), dim3(P.wg0[P.count]), dim3(256), 0, s, P, x, K);
    } else {
        hipLaunchKernelGGL((k_gemv_q8<T, XH, R, false, false>), dim3(P.wg0[P.count]), dim3(256), 0, s, P, x, K);
    }
    return hipGetLastError();
}

// One fp16 row (v_dot2 form, little VALU per byte): 2 rows per wave, twice the waves of 4
// (17408 x 5120: 26.1 -> 20.9 us); launches of >= 8192 rows with rows of < 256 blocks share
// the activation through LDS too, each matrix keeping its K-slice geometry, so results do not
// change (gate + up batched 41.7 -> 38.4 us; a lone 1024-row matrix was slower that way).  Two rows (fp32 FMAs per quant and token): rows of fewer
// than 256 blocks with the activations shared through LDS (XL) and 2 rows per wave
// (17408 x 5120: 29.8 -> 24.0 us; XL at 4 rows per wave 27.2, at 8 37.9); longer rows read
// them per row group and keep 4 rows per wave to reuse each block's activations (5120 x 17408:
// XL 36.3 us, too few workgroups for one K slice each).  Rows are split over K slices: at
// T = 1 rows of >= 256 blocks over 2 waves (5120 x 17408: 22.1 us with 4 slices, 22.9 with 1,
// 20.9 with 2) and rows of >= 128 blocks over 4 when the one-slice grid would be small
// (5120 x 1024: 6.7 -> 3.7 us); at T = 2 (without XL) rows of >= 128 blocks over 4.
template <int T, bool XH>
hipError_t launch_q8_t(Q8Mats& P, const void* x, int K, hipStream_t s) {
    const int nb = K / kQ8Group;
    int rows = 0;
    for (int i = 0; i < P.count; i++) rows += P.N[i];
    const bool xl = T * K * (XH ? 2 : 4) <= kQ8XlMax && nb < 256 && (T == 2 || rows >= 8192);
    if (xl) return launch_q8_r<T, XH, kQ8XlRows>(P, x, K, true, s);
    return launch_q8_r<T, XH, T == 1 ? 2 : 4>(P, x, K, false, s);
}

}  // namespace

int gemv_q8_max_mats() { return kQ8MaxMats; }

hipError_t launch_gemv_q8_multi(int count, const uint8_t* const* W, float* const* y, const int* N, const void* x,
                                int x_dtype, int K, int T, hipStream_t s) {
    if (count < 1 || count > kQ8MaxMats) return hipErrorInvalidValue;
    const size_t nb = (size_t)(K / kQ8Group);
    Q8Mats P{};
    P.count = count;
    for (int i = 0; i < count; i++) {
        if ((size_t)N[i] * nb * kQ8BlockBytes + 4 > 0x7fffffffu) return hipErrorInvalidValue;
        P.w_off[i] = (uint32_t)((uintptr_t)W[i] & 3);
        P.W[i] = W[i] - P.w_off[i];
        P.y[i] = y[i];
        P.N[i] = N[i];
        P.w_bytes[i] = P.w_off[i] + (uint32_t)((size_t)N[i] * nb * kQ8BlockBytes);
    }
    if (T == 1) return x_dtype == 1 ? launch_q8_t<1, true>(P, x, K, s) : launch_q8_t<1, false>(P, x, K, s);
    return x_dtype == 1 ? launch_q8_t<2, true>(P, x, K, s) : launch_q8_t<2, false>(P, x, K, s);
}

hipError_t launch_gemv_q8(const uint8_t* W, const void* x, int x_dtype, float* y, int K, int N, int T,
                          hipStream_t s) {
    return launch_gemv_q8_multi(1, &W, &y, &N, x, x_dtype, K, T, s);
}

}  // namespace kata
