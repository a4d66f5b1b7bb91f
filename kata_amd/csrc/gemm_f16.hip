// Exact fp16 prefill GEMM with the PTQ1_0 decode fused into the LDS tile load.
//
// Semantics (shaders/prefill.metal:31-41 after k_expand_ptq1_v2, :472-479):
//   C[m][n] = sum_k A[m][k] * half(trit[n][k] * d[n][k/128]),  fp16 x fp16 -> fp32.
// half(trit*d) is exact, so the product terms equal the reference's; only the fp32
// summation order differs (tolerance-based parity).
//
// Design: no fp16 weight stage ever touches HBM (the reference writes 178 MB per matrix).
// A 256-thread workgroup computes a 128x128 tile of C with K-steps of one PTQ1_0 block
// (128).  Per step it copies the 128x128 fp16 A tile to LDS and decodes the 128-row x
// 28-byte packed W tile straight into an fp16 [n][k] LDS tile: a thread takes two
// neighbouring bytes of a row and emits, for each of their 4-5 base-3 digits, the two
// adjacent-k weights as one 32-bit LDS store (element pairs 16n+m, 80+8n+m, 120+2n+h
// are adjacent for even m, h).  Four waves (2x2) each run 4x4 v_mfma_f32_16x16x32_f16
// tiles over the step.
#include "common.h"
#include "launch.h"

namespace kata {

namespace {

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int LDA_S = BK + 8;   // halves; row stride 272 B

template <bool C_F16>
__global__ __launch_bounds__(256) void k_gemm_ptq1_f16(const _Float16* __restrict__ A, int lda,
                                                       const uint8_t* __restrict__ W, void* __restrict__ C,
                                                       int ldc, int M, int K, int N) {
    __shared__ _Float16 As[BM * LDA_S];
    __shared__ _Float16 Bs[BN * LDA_S];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int nb = K / kGroup;
    const int l16 = lane & 15, lg = lane >> 4;

    v4f acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int jx = 0; jx < 4; jx++) acc[i][jx] = v4f{0.f, 0.f, 0.f, 0.f};

    for (int kb = 0; kb < nb; ++kb) {
        __syncthreads();
        // ---- A tile: 128 rows x 128 halves; thread -> (row tid/2, 64 halves)
        {
            const int r = tid >> 1, h = tid & 1;
            const int gm = m0 + r;
            uint4* dst = (uint4*)(As + r * LDA_S + h * 64);
            if (gm < M) {
                const uint4* src = (const uint4*)(A + (size_t)gm * lda + (size_t)kb * BK + h * 64);
#pragma unroll
                for (int c = 0; c < 8; c++) dst[c] = src[c];
            } else {
#pragma unroll
                for (int c = 0; c < 8; c++) dst[c] = make_uint4(0, 0, 0, 0);
            }
        }
        // ---- W tile: 128 rows x 13 byte pairs -> fp16 [n][k]
        for (int idx = tid; idx < BN * 13; idx += 256) {
            const int r = idx / 13, pr = idx - r * 13;
            const int gn = n0 + r;
            const int p = 2 * pr;
            uint32_t* brow = (uint32_t*)(Bs + r * LDA_S);
            if (gn < N) {
                const uint8_t* blk = W + ((size_t)gn * nb + kb) * kBlockBytes;
                const uint32_t bb = *(const uint16_t*)(blk + p);
                const float d = half_bits_to_float(*(const uint16_t*)(blk + 26));
                const uint32_t b0 = bb & 0xffu, b1 = bb >> 8;
                const int nd = p < 24 ? 5 : 4;
#pragma unroll
                for (int n = 0; n < 5; n++) {
                    if (n < nd) {
                        const float t0 = (float)((int)ptq1_digit(b0, n) - 1) * d;
                        const float t1 = (float)((int)ptq1_digit(b1, n) - 1) * d;
                        const int e = ptq1_slot_elem(p, n);
                        v2h hv = {(_Float16)t0, (_Float16)t1};
                        brow[e >> 1] = *(uint32_t*)&hv;
                    }
                }
            } else {
#pragma unroll
                for (int n = 0; n < 5; n++) {
                    const int e = ptq1_slot_elem(p, n);
                    if (e >= 0) brow[e >> 1] = 0u;
                }
            }
        }
        __syncthreads();
        // ---- 4 k-substeps of 32
#pragma unroll
        for (int kk = 0; kk < BK / 32; kk++) {
            v8h af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                af[i] = *(const v8h*)(As + (wm * 64 + i * 16 + l16) * LDA_S + kk * 32 + lg * 8);
#pragma unroll
            for (int jx = 0; jx < 4; jx++)
                bf[jx] = *(const v8h*)(Bs + (wn * 64 + jx * 16 + l16) * LDA_S + kk * 32 + lg * 8);
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int jx = 0; jx < 4; jx++)
                    acc[i][jx] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[jx], acc[i][jx], 0, 0, 0);
        }
    }
    // ---- store: lane holds D[4*lg + r][l16] of each 16x16 tile
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

hipError_t launch_gemm_f16(const uint16_t* A, int lda, const uint8_t* W, void* C, int c_dtype, int ldc,
                           int M, int K, int N, hipStream_t s) {
    const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM), block(256);
    if (c_dtype == 1)
        hipLaunchKernelGGL(k_gemm_ptq1_f16<true>, grid, block, 0, s, (const _Float16*)A, lda, W, C, ldc, M, K, N);
    else
        hipLaunchKernelGGL(k_gemm_ptq1_f16<false>, grid, block, 0, s, (const _Float16*)A, lda, W, C, ldc, M, K, N);
    return hipGetLastError();
}

}  // namespace kata
