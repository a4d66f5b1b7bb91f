// Exact fp16 prefill GEMM with the PTQ1_0 decode fused into the LDS tile load.
//
// Semantics (shaders/prefill.metal:31-41 after k_expand_ptq1_v2, :472-479):
//   C[m][n] = sum_k A[m][k] * half(trit[n][k] * d[n][k/128]),  fp16 x fp16 -> fp32.
// half(trit*d) is exact, so every product term equals the reference's; only the fp32
// summation order differs (tolerance-based parity).
//
// Design (MI355X-first; the reference expands every matrix to a 178 MB fp16 stage first):
//  * Work is cut into tiles of 256 rows of A / C by 128 columns (8 units of 16).  Tiles are
//    taken whole by one workgroup each for as many full rounds of the CU count as there
//    are; the tiles left over are split along K into pieces, one workgroup each, so the
//    last round fills the chip too.  A piece writes its fp32 partial tile to a workspace
//    and a second kernel adds the pieces of each tile in piece order (deterministic).
//    256-row tiles halve the weight decoding per flop against 128-row ones.  K advances in
//    stages of 64 (half a PTQ1_0 block).
//  * 8 waves, two per SIMD.  Waves 0..3 are consumers: wave w owns rows 64w..64w+63 and all
//    128 columns, 2 x 4 tiles of v_mfma_f32_32x32x16_f16, with the A and B fragments of a
//    16-k step loaded from LDS before the MFMAs of the step before it.  Waves 4..7 are producers:
//    they copy A tiles into LDS by DMA two stages ahead (three A buffers) and decode the
//    next stage's ternary weights from the packed bytes (copied into LDS by DMA two blocks
//    ahead) into fp16 LDS tiles (two B buffers).  No fp16 weight copy ever touches HBM.
//  * Decode: a group is 4 consecutive k of one row from the 4 bytes of one packed dword
//    and one base-3 digit; the bytes go to 16-bit lanes (b0,b1) and (b2,b3), the digit is
//    ((b * 3^n) mod 256) * 3 >> 8 with packed 16-bit multiplies, and v_perm_b32 picks the
//    fp16 value -d, 0 or +d.
//    A producer lane decodes half of one weight row (8 of its 16 groups per stage).
//  * LDS rows are 64 halves (128 B) of 8 chunks of 16 B; chunk c of row r is stored at
//    c ^ ((r >> 1) & 7).
//  * Workgroups are numbered so that the ones on one XCD (dispatched round robin) share
//    row tiles, and with them the A rows in that XCD's L2.
#include "common.h"
#include "launch.h"

#include <mutex>
#include "gemm_tile.h"

#include <algorithm>
#include <type_traits>

namespace kata {

namespace {

using namespace gemm;
constexpr int kWStage = BN * 32;    // staged packed bytes of one block of the tile rows, 32 B per row
constexpr int kLdsBytes = kTileBytes + 2 * kWStage;

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// fp16 of (digit_n(b) - 1) * d for bytes in 16-bit lanes (b_lo, b_hi); lo = (-d, 0),
// hi = (+d, +d) as fp16 bit pairs.  Returns the two halves as one dword.
__device__ inline uint32_t decode_pair(u16x2 b, uint32_t p3n, uint32_t lo, uint32_t hi) {
    u16x2 m = b * __builtin_bit_cast(u16x2, p3n);
    m &= (u16x2){0xff, 0xff};
    const u16x2 dg = (m * (u16x2){3, 3}) >> (u16x2){8, 8};
    const u16x2 sel = dg * (u16x2){0x0202, 0x0202} + (u16x2){0x0100, 0x0100};
    return __builtin_amdgcn_perm(hi, lo, __builtin_bit_cast(uint32_t, sel));
}

// group: bytes (b0, b1, b2, b3) of w -> 4 fp16 in that order as two dwords, digit n of
// b0, b1 by the multipliers p3lo and of b2, b3 by p3hi; the bytes go to 16-bit lanes
// (b0, b1) and (b2, b3) (v_perm selector 0x0c is a zero byte)
__device__ inline uint2 group_vals(uint32_t w, uint32_t p3lo, uint32_t p3hi, uint32_t lo, uint32_t hi) {
    const u16x2 e = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, w, 0x0c010c00u));
    const u16x2 o = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, w, 0x0c030c02u));
    return make_uint2(decode_pair(e, p3lo, lo, hi), decode_pair(o, p3hi, lo, hi));
}
__device__ inline uint2 group_vals(uint32_t w, uint32_t p3n, uint32_t lo, uint32_t hi) {
    return group_vals(w, p3n, p3n, lo, hi);
}

__host__ __device__ constexpr uint32_t p3x2(int n) {
    return n == 0 ? 0x00010001u : n == 1 ? 0x00030003u : n == 2 ? 0x00090009u : n == 3 ? 0x001b001bu : 0x00510051u;
}

// Decode groups of a stage (e = element of the block, dword j = bytes 4j..4j+3, stage
// k = e - 64h; each group covers 4 consecutive k):
//   h=0: dword i, digit n at k = 16n + 4i                        (i, n = 0..3)
//   h=1: dword i digit 4 at k = 4i; dword 4+i digit n at k = 16 + 4i + 8n (n = 0..4);
//        qh bytes (qh0, qh1, qh0, qh1) at digits (a, a, a+1, a+1) at k = 56 (a = 0) and 60 (a = 2)
// Producer half-rows (half q of the row): a 16-byte LDS chunk holds two groups:
//   h=0: chunk 2n + q = dwords 2q, 2q+1 at digit n (n = 0..3)
//   h=1: q=0: chunk 0 = digit 4 of dwords 0,1; chunks 2,3,4 = digits 0,1,2 of dwords 4,5
//        q=1: chunk 1 = digit 4 of dwords 2,3; chunks 5,6 = digits 3,4 of dwords 4,5;
//             chunk 7 = the two qh groups
template <bool C_F16>
__global__ __launch_bounds__(512) void k_gemm_ptq1_f16(const _Float16* __restrict__ A, int lda,
                                                       const uint8_t* __restrict__ W, void* __restrict__ C,
                                                       int ldc, float* __restrict__ ws, int M, int K, int N,
                                                       GemmJobs J) {
    extern __shared__ __align__(16) uint8_t smem[];
    auto Bs = [&](int buf) { return tile_b(smem, buf); };
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nbk = K >> 7;
    int job, tile, kb0, nb;
    gemm_job(J, nbk, job, tile, kb0, nb);
    const int m0 = (tile / J.G) * BM;
    const int n0 = (tile % J.G) * BN;
    const int R = min(BN, N - n0);              // columns of this tile
    const int nst = 2 * nb;                      // stages
    const uint32_t row_bytes = (uint32_t)nbk * kBlockBytes;
    A += (size_t)kb0 * 128;
    auto barrier = [&]() { barrier_lds(); };

    if (wave < 4) {
        consume<C_F16>(smem, wave, lane, nst, job, J, ws, C, ldc, M, m0, n0, R);
        return;
    }

    // ================= producers =================
    const int pw = wave - 4;
    auto issue_a = [&](int st) { gemm::issue_a(smem, pw, lane, A, lda, M, m0, st, nst); };
    // ---- weights: lane `lane` of producer pw decodes half q = pw & 1 of tile row
    // 64 (pw >> 1) + lane (q wave-uniform: no divergence).  The packed bytes of a block of
    // the tile's rows are copied into LDS by DMA (two 16-byte pieces per row, bytes 0..15
    // and 12..27, so no copy reads past the row's block), two blocks ahead; a lane reads
    // its dwords back when it starts the block.  Staging slot layout [piece][BN rows][16 B]:
    // producer pw copies piece pw & 1 of rows 64 (pw >> 1) .. +63.
    const int wrow = 64 * (pw >> 1) + lane, q = pw & 1;
    const bool wactive = wrow < R;
    uint8_t* Ws = smem + kABuf * BM * ROWB + 2 * BN * ROWB;      // [2 slots][2][BN][16 B]
    const uint8_t* wsrc = W + (size_t)min(n0 + min(wrow, R - 1), N - 1) * row_bytes + (size_t)kb0 * kBlockBytes + 12 * q;
    auto issue_w = [&](int blk) {
        dma16(wsrc + (size_t)min(blk, nb - 1) * kBlockBytes,
              lds_addr(Ws + (blk & 1) * kWStage + q * (BN * 16) + (pw >> 1) * 1024));
    };
    uint32_t w_cur[5];
    auto read_w = [&](int blk) {
        const uint8_t* slot = Ws + (blk & 1) * kWStage;
        const uint2 a = *(const uint2*)(slot + wrow * 16 + 8 * q);                  // dwords 2q, 2q+1
        const uint4 c = *(const uint4*)(slot + BN * 16 + wrow * 16);               // bytes 12..27
        w_cur[0] = a.x;
        w_cur[1] = a.y;
        w_cur[2] = c.y;                                                            // dword 4
        w_cur[3] = c.z;                                                            // dword 5
        w_cur[4] = c.w;                                                            // dword 6
    };
    auto decode_w = [&](auto h_c, int buf) {
        constexpr int h = decltype(h_c)::value;
        if (!wactive) return;
        uint8_t* bt = Bs(buf);
        const uint32_t dbits = w_cur[4] >> 16;
        const uint32_t lo = dbits ^ 0x8000u, hi = dbits | (dbits << 16);
        auto put = [&](int chunk, uint2 a, uint2 b) {
            *(uint4*)(bt + swz(wrow, chunk)) = make_uint4(a.x, a.y, b.x, b.y);
        };
        if (h == 0) {
#pragma unroll
            for (int n = 0; n < 4; n++)
                put(2 * n + q, group_vals(w_cur[0], p3x2(n), lo, hi), group_vals(w_cur[1], p3x2(n), lo, hi));
        } else if (q == 0) {
            put(0, group_vals(w_cur[0], p3x2(4), lo, hi), group_vals(w_cur[1], p3x2(4), lo, hi));
#pragma unroll
            for (int n = 0; n < 3; n++)
                put(2 + n, group_vals(w_cur[2], p3x2(n), lo, hi), group_vals(w_cur[3], p3x2(n), lo, hi));
        } else {
            put(1, group_vals(w_cur[0], p3x2(4), lo, hi), group_vals(w_cur[1], p3x2(4), lo, hi));
#pragma unroll
            for (int n = 3; n < 5; n++)
                put(2 + n, group_vals(w_cur[2], p3x2(n), lo, hi), group_vals(w_cur[3], p3x2(n), lo, hi));
            const uint32_t qh = __builtin_amdgcn_perm(0u, w_cur[4], 0x01000100u);
            put(7, group_vals(qh, p3x2(0), p3x2(1), lo, hi), group_vals(qh, p3x2(2), p3x2(3), lo, hi));
        }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // Vector-memory order of a producer (all its loads are LDS copies, which the compiler
    // cannot count, so the waits below do): before the barrier that releases stage s, A
    // batch s (8 copies) must have landed while the copies issued after it may still be in
    // flight; a block's weight copy (1) goes after the A batch of its slot.
    // prologue: weight blocks 0 and 1, A stages 0 and 1
    issue_w(0);
    issue_w(1);
    issue_a(0);
    issue_a(1);
    // blocks 0, 1 and batch 0; a row's two weight pieces come from two waves
    __builtin_amdgcn_s_waitcnt((8 & 15) | ((8 >> 4) << 14) | (7 << 4) | (15 << 8));
    barrier();
    read_w(0);
    decode_w(I0(), 0);
    barrier();
    for (int b = 0; b < nb; b++) {
        // consumers on stage 2b; produce stage 2b+1 (h=1 of block b) into B buffer 1
        issue_a(2 * b + 2);
        decode_w(I1(), 1);
        __builtin_amdgcn_s_waitcnt((8 & 15) | ((8 >> 4) << 14) | (7 << 4) | (15 << 8));    // batch 2b+1, block b+1
        barrier();
        // consumers on stage 2b+1; produce stage 2b+2 (h=0 of block b+1) into B buffer 0
        if (b + 1 < nb) read_w(b + 1);
        issue_a(2 * b + 3);
        issue_w(b + 2);                          // into the staging slot block b freed
        if (b + 1 < nb) decode_w(I0(), 0);
        __builtin_amdgcn_s_waitcnt((9 & 15) | ((9 >> 4) << 14) | (7 << 4) | (15 << 8));    // batch 2b+2
        barrier();
    }
}

}  // namespace

hipError_t gemm_device(bool need_ws, hipStream_t s, int* n_cu, float** ws) {
    hipError_t e = device_cu_count(n_cu);
    if (e != hipSuccess) return e;
    *ws = nullptr;
    if (!need_ws) return hipSuccess;
    void* p = nullptr;
    e = stream_buffer(kBufGemmPieces, (size_t)*n_cu * 256 * 128 * sizeof(float), s, &p);
    *ws = (float*)p;
    return e;
}

hipError_t launch_gemm_f16(const uint16_t* A, int lda, const uint8_t* W, void* C, int c_dtype, int ldc,
                           int M, int K, int N, hipStream_t s) {
    // the dynamic-LDS limit of both instantiations, raised once per process (a function-local
    // static: thread-safe initialisation)
    static const hipError_t attr = [] {
        hipError_t e = hipFuncSetAttribute((const void*)k_gemm_ptq1_f16<true>, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)k_gemm_ptq1_f16<false>, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
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
        hipLaunchKernelGGL(k_gemm_ptq1_f16<true>, dim3(J.n_jobs), dim3(512), kLdsBytes, s, (const _Float16*)A, lda, W,
                           C, ldc, ws, M, K, N, J);
    else
        hipLaunchKernelGGL(k_gemm_ptq1_f16<false>, dim3(J.n_jobs), dim3(512), kLdsBytes, s, (const _Float16*)A, lda,
                           W, C, ldc, ws, M, K, N, J);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_pieces_sum<BM, BN>(ws, C, c_dtype, ldc, M, N, J, s);
}

}  // namespace kata
