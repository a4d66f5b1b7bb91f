// Exact fp16 prefill GEMM over a Q8_0 matrix with the decode fused into the LDS tile load:
// the MTP head's K/V catch-up (Engine::encMtpKv, src/engine.cpp:392-401: k_expand_q8 then
// dGemm, shaders/mtp.metal:24-33).
//
// Semantics: C[m][n] = sum_k A[m][k] * half(d[n][k/32] * q[n][k]),  fp16 x fp16 -> fp32,
// with half() round-to-nearest-even as the reference's expansion.  Every product term equals
// the reference's; only the fp32 summation order differs (tolerance-based parity).
//
// Design: the tile machinery of gemm_tile.h (256 x 128 tiles, 64-k stages, 4 MFMA consumer
// waves, 4 producer waves, A by DMA two stages ahead); the producers here decode Q8_0:
//  * Staging: a stage covers two 34-byte blocks of each of the tile's 128 weight rows (68
//    bytes, dword-aligned since K is a multiple of 128).  They are copied into LDS by DMA
//    three stages ahead as five 16-byte pieces per row (stage bytes 0, 16, 32, 48 and 52,
//    the last overlapping so that no copy reads past the stage), [row][80 B], three slots.
//    Producer pw copies rows 32 pw .. 32 pw + 31.
//  * Decode: lane `lane` of producer pw takes block q = pw & 1 of tile row 64 (pw >> 1) +
//    lane (q wave-uniform) and writes its 32 fp16 weights as four 16-byte chunks.  The
//    int8 q becomes an exact fp16 through its bits: byte q ^ 0x80 as the low byte under a
//    0x66 high byte is the fp16 1536 + (q + 128), minus 1664 is q; one packed fp16 multiply
//    by d then rounds d * q once, to nearest even, as half(d * float(q)) does (the fp32
//    product of an fp16 and a 7-bit integer is exact).
#include "common.h"
#include "launch.h"

#include "gemm_tile.h"

namespace kata {

namespace {

using namespace gemm;

constexpr int kQ8RowStage = 80;                        // staged bytes per row and stage
constexpr int kQ8Slot = BN * kQ8RowStage;              // one stage of the tile's rows
constexpr int kQ8Slots = 3;                            // copies three stages ahead
constexpr int kQ8LdsBytes = kTileBytes + kQ8Slots * kQ8Slot;
static_assert(kQ8LdsBytes <= 160 * 1024, "LDS");

template <bool C_F16>
__global__ __launch_bounds__(512) void k_gemm_q8_f16(const _Float16* __restrict__ A, int lda,
                                                     const uint8_t* __restrict__ W, void* __restrict__ C, int ldc,
                                                     float* __restrict__ ws, int M, int K, int N, GemmJobs J) {
#pragma clang fp contract(off)
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nbk = K >> 7;
    int job, tile, kb0, nb;
    gemm_job(J, nbk, job, tile, kb0, nb);
    const int m0 = (tile / J.G) * BM;
    const int n0 = (tile % J.G) * BN;
    const int R = min(BN, N - n0);              // columns of this tile
    const int nst = 2 * nb;                      // stages
    A += (size_t)kb0 * 128;

    if (wave < 4) {
        consume<C_F16>(smem, wave, lane, nst, job, J, ws, C, ldc, M, m0, n0, R);
        return;
    }

    // ================= producers =================
    const int pw = wave - 4;
    uint8_t* Ws = smem + kTileBytes;             // [kQ8Slots][BN rows][80 B]
    const size_t row_bytes = (size_t)(K / kQ8Group) * kQ8BlockBytes;
    // copies: lane-load idx = 64 i + lane < 160 of producer pw -> row 32 pw + idx / 5,
    // piece idx % 5, LDS byte 80 row + 16 piece of the slot (DMA lanes are consecutive)
    auto issue_w = [&](int st) {
        const int s2 = min(st, nst - 1);
        const uint32_t base = lds_addr(Ws + (st % kQ8Slots) * kQ8Slot + pw * 32 * kQ8RowStage);
        const size_t stage_off = (size_t)(2 * kb0 + s2) * (2 * kQ8BlockBytes);
#pragma unroll
        for (int i = 0; i < 3; i++) {
            const int idx = 64 * i + lane;
            const int row = 32 * pw + idx / 5, piece = idx % 5;
            const uint8_t* src = W + (size_t)min(n0 + min(row, R - 1), N - 1) * row_bytes + stage_off +
                                 (piece < 4 ? 16 * piece : 52);
            if (i < 2 || lane < 32) dma16(src, base + 1024 * i);
        }
    };
    auto issue_a = [&](int st) { gemm::issue_a(smem, pw, lane, A, lda, M, m0, st, nst); };

    const int wrow = 64 * (pw >> 1) + lane, q = pw & 1;
    const bool wactive = wrow < R;
    auto decode = [&](int st, int buf) {
        if (!wactive) return;
        const uint8_t* sp = Ws + (st % kQ8Slots) * kQ8Slot + wrow * kQ8RowStage;
        // block q of the stage: bytes 34 q .. 34 q + 33, read as 9 dwords from byte 32 q
        // (block 1's last dword, stage bytes 64..67, sits in the overlapping piece at 76)
        const uint4 a0 = *(const uint4*)(sp + 32 * q), a1 = *(const uint4*)(sp + 32 * q + 16);
        const uint32_t a8 = *(const uint32_t*)(sp + (q ? 76 : 32));
        const uint32_t in[9] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w, a8};
        uint32_t qd[8];                          // the block's 32 int8, 4 per dword
        uint32_t dbits;
        if (q) {
            dbits = in[0] >> 16;
#pragma unroll
            for (int i = 0; i < 8; i++) qd[i] = in[i + 1];
        } else {
            dbits = in[0] & 0xffffu;
#pragma unroll
            for (int i = 0; i < 8; i++) qd[i] = __builtin_amdgcn_alignbyte(in[i + 1], in[i], 2);
        }
        const v2h d2 = __builtin_bit_cast(v2h, dbits | (dbits << 16));
        const v2h off2 = {(_Float16)1664.0f, (_Float16)1664.0f};
        uint8_t* bt = tile_b(smem, buf);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            uint32_t o[4];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint32_t w = qd[2 * c + h] ^ 0x80808080u;
                const v2h lo = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x66666666u, w, 0x04010400u)) - off2;
                const v2h hi = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x66666666u, w, 0x04030402u)) - off2;
                o[2 * h] = __builtin_bit_cast(uint32_t, lo * d2);
                o[2 * h + 1] = __builtin_bit_cast(uint32_t, hi * d2);
            }
            *(uint4*)(bt + swz(wrow, 4 * q + c)) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    };
    auto barrier = [&]() { barrier_lds(); };
    // Vector-memory order of a producer (all LDS copies, which the compiler cannot count,
    // so the waits are explicit): prologue w0 w1 w2 a0 a1, then per stage st: a(st+2)
    // w(st+3).  Before the barrier that ends stage st's iteration, a(st+1) (the consumers'
    // next stage) and w(st+2) (the next decode) have landed: 11 copies may still be in
    // flight (a(st+2): 8, w(st+3): 3).
    issue_w(0);
    issue_w(1);
    issue_w(2);
    issue_a(0);
    issue_a(1);
    __builtin_amdgcn_s_waitcnt((22 & 15) | ((22 >> 4) << 14) | (7 << 4) | (15 << 8));   // w0 landed
    barrier();                                   // the producers' first copies landed
    decode(0, 0);
    __builtin_amdgcn_s_waitcnt((8 & 15) | ((8 >> 4) << 14) | (7 << 4) | (15 << 8));    // a0, w1, w2
    barrier();                                   // stage 0 produced
    for (int st = 0; st < nst; st++) {
        issue_a(st + 2);
        issue_w(st + 3);                         // into stage st's slot
        if (st + 1 < nst) decode(st + 1, (st + 1) & 1);
        __builtin_amdgcn_s_waitcnt((11 & 15) | ((11 >> 4) << 14) | (7 << 4) | (15 << 8));   // a(st+1), w(st+2)
        barrier();
    }
}

}  // namespace

hipError_t launch_gemm_q8(const uint16_t* A, int lda, const uint8_t* W, void* C, int c_dtype, int ldc, int M, int K,
                          int N, hipStream_t s) {
    // the dynamic-LDS limit of both instantiations, raised once per process (a function-local
    // static: thread-safe initialisation)
    static const hipError_t attr = [] {
        hipError_t e = hipFuncSetAttribute((const void*)k_gemm_q8_f16<true>, hipFuncAttributeMaxDynamicSharedMemorySize, kQ8LdsBytes);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)k_gemm_q8_f16<false>, hipFuncAttributeMaxDynamicSharedMemorySize, kQ8LdsBytes);
        return e;
    }();
    if (attr != hipSuccess) return attr;
    int n_cu = 0;
    float* ws = nullptr;
    hipError_t e = gemm_device(false, s, &n_cu, &ws);
    if (e != hipSuccess) return e;
    const GemmJobs J = plan_gemm_jobs(M, N, K, BM, BN, n_cu);   // one workgroup per CU
    if (J.n_jobs > J.n_full && (e = gemm_device(true, s, &n_cu, &ws)) != hipSuccess) return e;
    if (c_dtype == 1)
        hipLaunchKernelGGL(k_gemm_q8_f16<true>, dim3(J.n_jobs), dim3(512), kQ8LdsBytes, s, (const _Float16*)A, lda, W,
                           C, ldc, ws, M, K, N, J);
    else
        hipLaunchKernelGGL(k_gemm_q8_f16<false>, dim3(J.n_jobs), dim3(512), kQ8LdsBytes, s, (const _Float16*)A, lda,
                           W, C, ldc, ws, M, K, N, J);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_pieces_sum<BM, BN>(ws, C, c_dtype, ldc, M, N, J, s);
}

}  // namespace kata
