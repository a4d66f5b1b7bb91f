// Tile schedule shared by the prefill GEMMs (gemm_f16.hip, gemm_i8.hip).
//
// C is cut into TBM x TBN tiles, tile t = (row tile t / G, column group t % G).  With
// `slots` workgroups resident at once, the whole rounds of `slots` tiles are taken whole by
// one workgroup each; the r tiles left over are split along K into S = min(slots / r,
// kMaxPieces, K blocks) pieces, one workgroup each, so the last round fills the chip too.
// A piece writes its fp32 partial tile to the per-device workspace and k_gemm_pieces_sum
// adds the pieces of each split tile in piece order (deterministic).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

namespace kata {

constexpr int kMaxPieces = 16;   // K pieces of one split tile

struct GemmJobs {
    int G;        // column groups
    int n_full;   // whole tiles (jobs 0 .. n_full-1)
    int S;        // pieces per split tile
    int n_jobs;   // workgroups: piece slot j = job - n_full is piece j % S of tile n_full + j / S
};

inline GemmJobs plan_gemm_jobs(int M, int N, int K, int TBM, int TBN, int slots) {
    GemmJobs J;
    J.G = (N + TBN - 1) / TBN;
    const long T = (long)((M + TBM - 1) / TBM) * J.G;
    const int nbk = K / 128;
    long rem = T % slots;
    int S = rem ? std::min(std::min(slots / (int)rem, kMaxPieces), nbk) : 1;
    if (S < 2) {
        S = 1;
        rem = 0;
    }
    J.n_full = (int)(T - rem);
    J.S = S;
    J.n_jobs = (int)(J.n_full + rem * S);
    return J;
}

// The job of this workgroup: tile, first K block and K blocks.  Workgroups are dispatched
// round robin over 8 XCDs: within the whole tiles and within the pieces, consecutive jobs
// (tiles sharing A rows) are placed on one XCD, whose L2 then serves them.
__device__ inline void gemm_job(const GemmJobs& J, int nbk, int& job, int& tile, int& kb0, int& nb) {
    job = blockIdx.x;
    const int lo = job < J.n_full ? 0 : J.n_full;
    const int n = job < J.n_full ? J.n_full : J.n_jobs - J.n_full;
    const int i = job - lo;
    if (n % 8 == 0 && lo % 8 == 0) job = lo + (i % 8) * (n / 8) + i / 8;
    if (job < J.n_full) {
        tile = job;
        kb0 = 0;
        nb = nbk;
    } else {
        const int j = job - J.n_full, piece = j % J.S;
        tile = J.n_full + j / J.S;
        kb0 = (int)(((long)piece * nbk) / J.S);
        nb = (int)(((long)(piece + 1) * nbk) / J.S) - kb0;
    }
}

// C[m][n] for the split tiles: the sum of the tile's pieces ([TBM][TBN] fp32 each, slot
// order) in piece order.  One thread per 4 consecutive columns of a tile row; the pieces'
// loads are all in flight before the sum.
template <int TBM, int TBN, bool C_F16>
__global__ __launch_bounds__(256) void k_gemm_pieces_sum(const float* __restrict__ ws, void* __restrict__ C, int ldc,
                                                         int M, int N, GemmJobs J) {
    const int t = J.n_full + blockIdx.y;                    // split tile
    const int e = blockIdx.x * 256 + threadIdx.x;           // quad of the tile
    const int r = e / (TBN / 4), c4 = (e % (TBN / 4)) * 4;
    const int gm = (t / J.G) * TBM + r, gn0 = (t % J.G) * TBN + c4;
    if (gm >= M) return;
    const float* P = ws + (size_t)blockIdx.y * J.S * (TBM * TBN) + r * TBN + c4;
    float4 v[kMaxPieces];
#pragma unroll
    for (int p = 0; p < kMaxPieces; p++)
        if (p < J.S) v[p] = *(const float4*)(P + (size_t)p * (TBM * TBN));
    float4 s = v[0];
#pragma unroll
    for (int p = 1; p < kMaxPieces; p++)
        if (p < J.S) {
            s.x += v[p].x;
            s.y += v[p].y;
            s.z += v[p].z;
            s.w += v[p].w;
        }
    const float o[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (gn0 + i < N) {
            if (C_F16) ((_Float16*)C)[(size_t)gm * ldc + gn0 + i] = (_Float16)o[i];
            else ((float*)C)[(size_t)gm * ldc + gn0 + i] = o[i];
        }
    }
}

template <int TBM, int TBN>
inline hipError_t launch_pieces_sum(const float* ws, void* C, int c_dtype, int ldc, int M, int N, const GemmJobs& J,
                                    hipStream_t s) {
    const int rem = J.n_jobs - J.n_full;
    if (!rem) return hipSuccess;
    const dim3 grid(TBM * TBN / 4 / 256, (unsigned)(rem / J.S));
    if (c_dtype == 1)
        hipLaunchKernelGGL((k_gemm_pieces_sum<TBM, TBN, true>), grid, dim3(256), 0, s, ws, C, ldc, M, N, J);
    else
        hipLaunchKernelGGL((k_gemm_pieces_sum<TBM, TBN, false>), grid, dim3(256), 0, s, ws, C, ldc, M, N, J);
    return hipGetLastError();
}

// The calling thread's device: its CU count and (need_ws) the K-piece workspace of stream s
// (room for one 256 x 128 fp32 tile per CU: 32 MB on MI355X), allocated on the first call on
// that (device, stream) that asks for it and kept; calls on other streams use their own.
hipError_t gemm_device(bool need_ws, hipStream_t s, int* n_cu, float** ws);

}  // namespace kata
