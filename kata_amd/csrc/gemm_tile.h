// Tile machinery shared by the fp16 prefill GEMMs with a fused weight decode
// (gemm_f16.hip: PTQ1_0, gemm_q8.hip: Q8_0).  A workgroup of 8 waves computes a
// 256 x 128 tile of C in stages of 64 k: waves 0..3 (consumers) run v_mfma_f32_32x32x16_f16
// on fp16 A and B tiles in LDS, waves 4..7 (producers) copy A tiles into LDS by DMA two
// stages ahead (three A buffers) and write the decoded fp16 weights of the next stage into
// one of two B buffers.  A stage is released by a workgroup barrier.
//
// LDS: [kABuf][BM rows][ROWB] A tiles, then [2][BN rows][ROWB] B tiles, then whatever the
// producers stage (format specific).  Rows are 64 halves (128 B) of 8 chunks of 16 B; chunk
// c of row r is stored at c ^ ((r >> 1) & 7) (conflict-free fragment reads).
#pragma once
#include "common.h"
#include "gemm_sched.h"

namespace kata {
namespace gemm {

constexpr int BM = 256;          // rows of A / C per workgroup
constexpr int BKS = 64;          // k per stage (halves)
constexpr int ROWB = BKS * 2;    // LDS bytes per tile row
constexpr int NT = 4;            // 32-column MFMA tiles per workgroup
constexpr int BN = 32 * NT;      // columns per tile (128)
constexpr int kABuf = 3;         // A stage buffers (DMA two stages ahead)
constexpr int kTileBytes = kABuf * BM * ROWB + 2 * BN * ROWB;   // LDS before the producers' staging

typedef float v16f __attribute__((ext_vector_type(16)));

__device__ inline uint32_t swz(int row, int chunk) { return (uint32_t)(row * ROWB + ((chunk ^ ((row >> 1) & 7)) << 4)); }
__device__ inline uint8_t* tile_a(uint8_t* smem, int buf) { return smem + buf * (BM * ROWB); }
__device__ inline uint8_t* tile_b(uint8_t* smem, int buf) { return smem + kABuf * BM * ROWB + buf * (BN * ROWB); }

// LDS DMA, 16 bytes per lane to lds + 16*lane (lds wave-uniform); issued through inline
// assembly so that the compiler does not make later LDS accesses wait for every load in
// flight; the kernel waits for these copies explicitly.  M0 is restored.
__device__ inline void dma16(const void* g, uint32_t lds) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(g), "s"(lds)
                 : "memory");
}
__device__ inline uint32_t lds_addr(const void* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(__attribute__((address_space(3))) const void*)p);
}

__device__ inline void barrier_lds() {
    __builtin_amdgcn_s_waitcnt((15 & 15) | ((63 >> 4) << 14) | (7 << 4) | (0 << 8));   // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
}

// Consumer waves (wave < 4) of job `job`: nst stages, then the tile (or, for a piece of a
// split tile, its fp32 partial into the job's workspace slot).  Barriers: two before the
// first stage (the producers' first copies landed, stage 0 produced), one per stage.
template <bool C_F16>
__device__ inline void consume(uint8_t* smem, int wave, int lane, int nst, int job, const GemmJobs& J, float* ws,
                               void* C, int ldc, int M, int m0, int n0, int R) {
    auto As = [&](int buf) { return tile_a(smem, buf); };
    auto Bs = [&](int buf) { return tile_b(smem, buf); };
    auto barrier = [&]() { barrier_lds(); };
    // ================= consumers =================
    const int l32 = lane & 31, lh = lane >> 5;
    v16f acc[2][NT];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int q = 0; q < 16; q++) acc[i][j][q] = 0.0f;
    // lane l reads row / column l % 32 of each 32-row tile at k = 16 kk + 8 (l / 32) .. +7,
    // chunk 2 kk + l / 32; every tile row of this lane has the same swizzle term
    const int xs = (l32 >> 1) & 7;
    const uint32_t a_row = (uint32_t)(wave * 64 + l32) * ROWB, b_row = (uint32_t)l32 * ROWB;
    auto load_frags = [&](int st, int kk, v8h (&af)[2], v8h (&bf)[NT]) {
        const uint32_t c = (uint32_t)(((2 * kk + lh) ^ xs) << 4);
        const uint8_t* at = As(st % kABuf) + a_row + c;
        const uint8_t* bt = Bs(st & 1) + b_row + c;
#pragma unroll
        for (int i = 0; i < 2; i++) af[i] = *(const v8h*)(at + i * 32 * ROWB);
#pragma unroll
        for (int j = 0; j < NT; j++) bf[j] = *(const v8h*)(bt + j * 32 * ROWB);
    };
    auto mfmas = [&](v8h (&af)[2], v8h (&bf)[NT]) {
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int i = 0; i < 2; i++)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    };
    // fragments are loaded one k step ahead of the MFMAs that use them; the last step
    // of a stage is loaded before the barrier that releases the stage's buffers
    v8h a0[2], b0[NT], a1[2], b1[NT];
    barrier();                               // the producers' first copies landed
    barrier();                               // stage 0 produced
    load_frags(0, 0, a0, b0);
    for (int st = 0; st < nst; st++) {
        load_frags(st, 1, a1, b1);
        mfmas(a0, b0);
        load_frags(st, 2, a0, b0);
        mfmas(a1, b1);
        load_frags(st, 3, a1, b1);
        mfmas(a0, b0);
        barrier();                           // stage st + 1 produced; stage st's buffers free
        if (st + 1 < nst) load_frags(st + 1, 0, a0, b0);
        mfmas(a1, b1);
    }
    // store: lane holds D[8(q/4) + 4(l/32) + q%4][l % 32] of each 32x32 tile
    if (job >= J.n_full) {
        // piece: the whole fp32 tile, [256][128], into the job's workspace slot
        float* P = ws + (size_t)(job - J.n_full) * (BM * BN);
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < NT; j++)
#pragma unroll
                for (int q = 0; q < 16; q++)
                    P[(wave * 64 + i * 32 + 8 * (q >> 2) + 4 * lh + (q & 3)) * BN + j * 32 + l32] = acc[i][j][q];
        return;
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int gc = j * 32 + l32;     // tile column
            const int gn = n0 + gc;
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int gm = m0 + wave * 64 + i * 32 + 8 * (q >> 2) + 4 * lh + (q & 3);
                if (gm < M && gc < R) {
                    if (C_F16) ((_Float16*)C)[(size_t)gm * ldc + gn] = (_Float16)acc[i][j][q];
                    else ((float*)C)[(size_t)gm * ldc + gn] = acc[i][j][q];
                }
            }
        }
}

// Producer A copies: DMA instruction i of producer pw copies LDS bytes [1024 (4i + pw), +1024)
// of stage st's A tile: lane l -> tile row r = 8 (4i + pw) + l / 8, LDS slot l % 8, which
// holds global chunk (l % 8) ^ ((r >> 1) & 7) of that row (rows >= M read row M - 1); stages
// past the end copy the last one.  8 vector-memory instructions per call.
__device__ inline void issue_a(uint8_t* smem, int pw, int lane, const _Float16* A, int lda, int M, int m0, int st,
                               int nst) {
    const int ar_lo = 8 * pw + (lane >> 3);      // row for i = 0; + 32 i
    const int aslot = lane & 7;
    const int s2 = min(st, nst - 1);
    const uint32_t base = lds_addr(tile_a(smem, st % kABuf)) + 1024 * pw;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int r = ar_lo + 32 * i;
        const int chunk = aslot ^ ((r >> 1) & 7);
        const _Float16* src = A + (size_t)min(m0 + r, M - 1) * lda + (size_t)s2 * BKS + chunk * 8;
        dma16(src, base + 4096 * i);
    }
}

}  // namespace gemm
}  // namespace kata
