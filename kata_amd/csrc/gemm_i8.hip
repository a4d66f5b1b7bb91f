// int8 prefill path: activation quantisation and the int8 x trit GEMM with the per-group
// scale epilogue, ternary decode fused into the LDS tile load.
//
// quant_rows (shaders/prefill.metal:369-381): per (token m, group g of 128):
//   scale = amax > 0 ? amax/127 : 1; q = clamp(rint(x * (1/scale)), -127, 127);
//   SX[g*ldS + m] = scale.   IEEE fp32 division and round-half-even, bit-exact.
// gemm (shaders/prefill.metal:382-415): I = sum_{k in g} A8[m][k]*trit[n][k] (exact int32),
//   C[m][n] = sum_g float(I) * (d[n][g] * SX[g][m]) in fp32, groups ascending.
//
// Design: 128x128 C tile per 256-thread workgroup, one K-step per 128-group; A8 tile
// copied to LDS, W tile decoded to int8 trits in LDS (two adjacent-k trits per 16-bit
// store).  Each wave runs 4x4 tiles of v_mfma_i32_16x16x64_i8 (two per group) and folds
// the group's int32 result into fp32 accumulators with the row/column scales.
#include "common.h"
#include "launch.h"
#include "gemm_sched.h"

namespace kata {

namespace {

// max over the 16 lanes of a DPP row
__device__ inline float row16_max(float a) {
    a = fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0xb1, 0xf, 0xf, false)));
    a = fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x4e, 0xf, 0xf, false)));
    a = fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x141, 0xf, 0xf, false)));
    a = fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x140, 0xf, 0xf, false)));
    return a;
}

// One (token, group) per 16 lanes (a DPP row), 8 elements per lane from one 16-byte load;
// groups numbered token-major, 16 per 256-thread workgroup.
__global__ __launch_bounds__(256) void k_quant_rows(const _Float16* __restrict__ X, int8_t* __restrict__ Q,
                                                    float* __restrict__ SX, int M, int K, int ldS) {
    const int G = K / kGroup;
    const int gi = blockIdx.x * 16 + (threadIdx.x >> 4), sub = threadIdx.x & 15;
    if (gi >= M * G) return;                     // whole DPP rows drop out together
    const int m = gi / G, g = gi - m * G;
    const size_t o = (size_t)m * K + (size_t)g * kGroup + 8 * sub;
    const uint4 raw = *(const uint4*)(X + o);
    const uint32_t rw[4] = {raw.x, raw.y, raw.z, raw.w};
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const v2h h = __builtin_bit_cast(v2h, rw[i]);
        v[2 * i] = (float)h[0];
        v[2 * i + 1] = (float)h[1];
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) mx = fmaxf(mx, fabsf(v[i]));
    mx = row16_max(mx);
    const float scale = mx > 0.0f ? mx / 127.0f : 1.0f;
    const float inv = 1.0f / scale;
    uint32_t q[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float qf = fminf(fmaxf(rintf(v[i] * inv), -127.0f), 127.0f);
        q[i >> 2] |= (uint32_t)(uint8_t)(int8_t)qf << (8 * (i & 3));
    }
    *(uint2*)(Q + o) = make_uint2(q[0], q[1]);
    if (sub == 0) SX[(size_t)g * ldS + m] = scale;
}

// digit multipliers 3^n in both 16-bit lanes
__host__ __device__ constexpr uint32_t p3x2(int n) {
    return n == 0 ? 0x00010001u : n == 1 ? 0x00030003u : n == 2 ? 0x00090009u : n == 3 ? 0x001b001bu : 0x00510051u;
}

// int8 trits (digit - 1) of the 4 bytes of w, in byte order: bytes 0, 1 at the digit of
// multiplier p3lo, bytes 2, 3 at p3hi.  The bytes go to 16-bit lanes (v_perm selector 0x0c is
// a zero byte); ((b * 3^n) mod 256) * 3 has the digit in its high byte; a v_perm table maps
// digits 0, 1, 2 to the bytes 0xff, 0x00, 0x01.
__device__ inline uint32_t trits4(uint32_t w, uint32_t p3lo, uint32_t p3hi) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    u16x2 e = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, w, 0x0c010c00u));
    u16x2 o = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, w, 0x0c030c02u));
    e = (e * __builtin_bit_cast(u16x2, p3lo)) & (u16x2){0xff, 0xff};
    o = (o * __builtin_bit_cast(u16x2, p3hi)) & (u16x2){0xff, 0xff};
    e = e * (u16x2){3, 3};
    o = o * (u16x2){3, 3};
    const uint32_t dg = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, o), __builtin_bit_cast(uint32_t, e), 0x07050301u);
    return __builtin_amdgcn_perm(0u, 0x000100ffu, dg);
}

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int LDB_S = BK + 16;   // bytes per LDS row

template <bool C_F16>
__global__ __launch_bounds__(256) void k_gemm_ptq1_i8(const int8_t* __restrict__ A8, const float* __restrict__ SX,
                                                      int ldS, const uint8_t* __restrict__ W, void* __restrict__ C,
                                                      int ldc, float* __restrict__ ws, int M, int K, int N,
                                                      GemmJobs J) {
    __shared__ int8_t As[BM * LDB_S];
    __shared__ int8_t Bs[BN * LDB_S];
    __shared__ float sws[BN];
    __shared__ float sxs[BM];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int nb = K / kGroup;
    int job, tile, kb_lo, kb_n;
    gemm_job(J, nb, job, tile, kb_lo, kb_n);
    const int m0 = (tile / J.G) * BM, n0 = (tile % J.G) * BN;
    const int l16 = lane & 15, lg = lane >> 4;

    v4f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int jx = 0; jx < 4; jx++) acc[i][jx] = v4f{0.f, 0.f, 0.f, 0.f};

    // the operands of the next group are loaded into registers while the matrix cores work
    // on the current one: thread -> 64 bytes of A row tid / 2 and the 7 dwords of W row
    // tid / 2's block (thread tid < BM also the row scale of A row tid)
    const int lr = tid >> 1, lh = tid & 1;
    const bool a_ok = m0 + lr < M, w_ok = n0 + lr < N, s_ok = tid < BM && m0 + tid < M;
    const uint4* asrc = (const uint4*)(A8 + (size_t)min(m0 + lr, M - 1) * K + lh * 64);
    const uint32_t* wsrc = (const uint32_t*)(W + (size_t)min(n0 + lr, N - 1) * nb * kBlockBytes);   // 4-byte aligned
    uint4 pa[4];
    uint32_t pw[7];
    float psx = 0.0f;
    auto fetch = [&](int kb) {
#pragma unroll
        for (int c = 0; c < 4; c++) pa[c] = asrc[kb * (BK / 16) + c];
#pragma unroll
        for (int i = 0; i < 7; i++) pw[i] = wsrc[kb * 7 + i];
        if (tid < BM) psx = SX[(size_t)kb * ldS + min(m0 + tid, M - 1)];
    };
    fetch(kb_lo);
    for (int kb = kb_lo; kb < kb_lo + kb_n; ++kb) {
        __syncthreads();                         // the previous group's LDS tiles are consumed
        {
            uint4* dst = (uint4*)(As + lr * LDB_S + lh * 64);
#pragma unroll
            for (int c = 0; c < 4; c++) dst[c] = a_ok ? pa[c] : make_uint4(0, 0, 0, 0);
            if (tid < BM) sxs[tid] = s_ok ? psx : 0.0f;
        }
        // B tile: thread -> 4 of the 8 16-byte chunks (16 k each) of tile row tid / 2
        {
            uint4* brow = (uint4*)(Bs + lr * LDB_S);
            if (w_ok) {
                const uint32_t w0 = pw[0], w1 = pw[1], w2 = pw[2], w3 = pw[3], w4 = pw[4], w5 = pw[5], w6 = pw[6];
                if (lh == 0) {
                    // chunks 0..3: dwords 0..3 at digit c
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        brow[c] = make_uint4(trits4(w0, p3x2(c), p3x2(c)), trits4(w1, p3x2(c), p3x2(c)),
                                             trits4(w2, p3x2(c), p3x2(c)), trits4(w3, p3x2(c), p3x2(c)));
                    sws[lr] = half_bits_to_float(w6 >> 16);
                } else {
                    brow[4] = make_uint4(trits4(w0, p3x2(4), p3x2(4)), trits4(w1, p3x2(4), p3x2(4)),
                                         trits4(w2, p3x2(4), p3x2(4)), trits4(w3, p3x2(4), p3x2(4)));
                    brow[5] = make_uint4(trits4(w4, p3x2(0), p3x2(0)), trits4(w5, p3x2(0), p3x2(0)),
                                         trits4(w4, p3x2(1), p3x2(1)), trits4(w5, p3x2(1), p3x2(1)));
                    brow[6] = make_uint4(trits4(w4, p3x2(2), p3x2(2)), trits4(w5, p3x2(2), p3x2(2)),
                                         trits4(w4, p3x2(3), p3x2(3)), trits4(w5, p3x2(3), p3x2(3)));
                    const uint32_t qh = __builtin_amdgcn_perm(0u, w6, 0x01000100u);   // (qh0, qh1, qh0, qh1)
                    brow[7] = make_uint4(trits4(w4, p3x2(4), p3x2(4)), trits4(w5, p3x2(4), p3x2(4)),
                                         trits4(qh, p3x2(0), p3x2(1)), trits4(qh, p3x2(2), p3x2(3)));
                }
            } else {
#pragma unroll
                for (int c = 0; c < 4; c++) brow[4 * lh + c] = make_uint4(0, 0, 0, 0);
                if (lh == 0) sws[lr] = 0.0f;
            }
        }
        if (kb + 1 < kb_lo + kb_n) fetch(kb + 1);
        __syncthreads();
        v4i ia[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int jx = 0; jx < 4; jx++) ia[i][jx] = v4i{0, 0, 0, 0};
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
            v4i af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; i++) af[i] = *(const v4i*)(As + (wm * 64 + i * 16 + l16) * LDB_S + kk * 64 + lg * 16);
#pragma unroll
            for (int jx = 0; jx < 4; jx++) bf[jx] = *(const v4i*)(Bs + (wn * 64 + jx * 16 + l16) * LDB_S + kk * 64 + lg * 16);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int jx = 0; jx < 4; jx++)
                    ia[i][jx] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[jx], ia[i][jx], 0, 0, 0);
        }
#pragma unroll
        for (int jx = 0; jx < 4; jx++) {
            const float sw = sws[wn * 64 + jx * 16 + l16];
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    acc[i][jx][r] += (float)ia[i][jx][r] * (sw * sxs[wm * 64 + i * 16 + lg * 4 + r]);
        }
    }
    if (job >= J.n_full) {
        // a piece: the whole fp32 tile, [128][128], into its workspace slot
        float* P = ws + (size_t)(job - J.n_full) * (BM * BN);
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int jx = 0; jx < 4; jx++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float v = acc[i][jx][r];
                    P[(wm * 64 + i * 16 + lg * 4 + r) * BN + wn * 64 + jx * 16 + l16] = v;
                }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int jx = 0; jx < 4; jx++) {
            const int gn = n0 + wn * 64 + jx * 16 + l16;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int gm = m0 + wm * 64 + i * 16 + lg * 4 + r;
                if (gm < M && gn < N) {
                    if (C_F16) ((_Float16*)C)[(size_t)gm * ldc + gn] = (_Float16)acc[i][jx][r];
                    else ((float*)C)[(size_t)gm * ldc + gn] = acc[i][jx][r];
                }
            }
        }
}

}  // namespace

hipError_t launch_quant_rows(const uint16_t* X, int8_t* Q, float* SX, int M, int K, int ldS, hipStream_t s) {
    const long groups = (long)M * (K / kGroup);
    hipLaunchKernelGGL(k_quant_rows, dim3((unsigned)((groups + 15) / 16)), dim3(256), 0, s, (const _Float16*)X, Q, SX,
                       M, K, ldS);
    return hipGetLastError();
}

// Two workgroups are resident per CU (their registers), so the schedule fills 2 n_cu slots.
hipError_t launch_gemm_i8(const int8_t* A8, const float* SX, int ldS, const uint8_t* W, void* C, int c_dtype,
                          int ldc, int M, int K, int N, hipStream_t s) {
    int n_cu = 0;
    float* ws = nullptr;
    hipError_t e = gemm_device(false, s, &n_cu, &ws);
    if (e != hipSuccess) return e;
    const GemmJobs J = plan_gemm_jobs(M, N, K, BM, BN, 2 * n_cu);
    if (J.n_jobs > J.n_full && (e = gemm_device(true, s, &n_cu, &ws)) != hipSuccess) return e;
    if (c_dtype == 1)
        hipLaunchKernelGGL(k_gemm_ptq1_i8<true>, dim3(J.n_jobs), dim3(256), 0, s, A8, SX, ldS, W, C, ldc, ws, M, K, N,
                           J);
    else
        hipLaunchKernelGGL(k_gemm_ptq1_i8<false>, dim3(J.n_jobs), dim3(256), 0, s, A8, SX, ldS, W, C, ldc, ws, M, K,
                           N, J);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_pieces_sum<BM, BN>(ws, C, c_dtype, ldc, M, N, J, s);
}

}  // namespace kata
