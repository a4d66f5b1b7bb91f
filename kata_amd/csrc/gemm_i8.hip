// int8 prefill path: activation quantisation and the int8 x trit GEMM with the per-group
// scale epilogue, ternary decode fused into the LDS tile load.
//
// quant_rows (shaders/prefill.metal:369-381): per (token m, group g of 128):
//   scale = amax > 0 ? amax/127 : 1; q = clamp(rint(x * (1/scale)), -127, 127);
//   SX[g*ldS + m] = scale.   IEEE fp32 division and round-half-even, bit-exact.
// gemm (shaders/prefill.metal:382-415): I = sum_{k in g} A8[m][k]*trit[n][k] (exact int32),
//   C[m][n] = sum_g float(I) * (d[n][g] * SX[g][m]) in fp32, groups ascending.
//
// Design: the tile machinery of the fp16 GEMM (256 x 128 C tiles, 12 waves: 8 consumers
// on v_mfma_i32_32x32x32_i8, two per SIMD, 4 producers copying A by DMA and decoding weights
// into LDS, whole tiles per CU then K pieces summed by a second kernel).  A stage is one 128-group:
// an int8 A row of 128 k is 128 bytes, the byte layout of an fp16 stage row of 64 k, so the
// A copies, swizzle and fragment reads are the fp16 kernel's, with half the stages.  The
// producers also stage the group's row scales (A side) and column scales (decoded weights)
// in LDS; consumers fold each 32 x 32 tile's exact group sum into fp32 right after its
// four MFMAs, groups ascending.
#include "common.h"
#include "launch.h"
#include "gemm_tile.h"
#include <utility>

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
// a zero byte); ((b * 3^n) mod 256) * 3 - 256 has the trit in its high byte (0xff, 0x00, 0x01).
__device__ inline uint32_t trits4(uint32_t w, uint32_t p3lo, uint32_t p3hi) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    u16x2 e = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, w, 0x0c010c00u));
    u16x2 o = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, w, 0x0c030c02u));
    e = (e * __builtin_bit_cast(u16x2, p3lo)) & (u16x2){0xff, 0xff};
    o = (o * __builtin_bit_cast(u16x2, p3hi)) & (u16x2){0xff, 0xff};
    e = e * (u16x2){3, 3} + (u16x2){0xff00, 0xff00};
    o = o * (u16x2){3, 3} + (u16x2){0xff00, 0xff00};
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, o), __builtin_bit_cast(uint32_t, e), 0x07050301u);
}

using namespace gemm;
constexpr int kWStage = BN * 32;                     // staged packed bytes of one block of the tile rows
constexpr int kSxOff = kTileBytes + 2 * kWStage;     // [kABuf][BM] fp32 row scales (with the A buffers)
constexpr int kSwOff = kSxOff + kABuf * BM * 4;      // [2][BN] fp32 column scales (with the B buffers)
constexpr int kLdsBytes = kSwOff + 2 * BN * 4;

typedef int v16i __attribute__((ext_vector_type(16)));
// the value v of lane Q of the caller's 16-lane row (DPP row_newbcast)
template <int Q>
__device__ inline float row_bcast(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x150 + Q, 0xf, 0xf, true));
}
// acc[q] += float(I[q]) * (w * sx[row of output q]), where lane 16 R + Q of the caller's
// 16-lane row R holds the row scale of output q = Q
// (the empty asm gives each call its own copy of sxv, so every broadcast is used once and
// becomes the DPP operand of its multiply instead of a move held across the column tiles)
template <int... Q>
__device__ inline void fold_tile(v16f& acc, const v16i& I, float w, float sxv, std::integer_sequence<int, Q...>) {
    asm volatile("" : "+v"(sxv));
    ((acc[Q] += (float)I[Q] * (w * row_bcast<Q>(sxv))), ...);
}

// LDS DMA of one dword per lane to lds + 4*lane (lds wave-uniform); see dma16
__device__ inline void dma4(const void* g, uint32_t lds) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(g), "s"(lds)
                 : "memory");
}

// Consumer waves (wave < kCW): wave w owns rows 32w..32w+31 and all 128 columns, 4 tiles of
// 32 x 32.  Per stage (one group of 128 k) the A fragments stay in registers; for each column
// tile j the int32 sum is 4 dependent v_mfma_i32_32x32x32_i8, then folded: acc += float(I) *
// (sw[n] * sx[m]), the row scale spread across the lanes by DPP.  The fold of tile j follows
// the MFMAs of tile j + 1.  A wave's VALU does not overlap its own MFMAs; with two consumers
// on each SIMD one's fold can run under the other's MFMAs (2.5 % faster than four consumers
// of 64 rows; 64 x 64 per wave, fewer LDS reads, gains nothing over it).
// Barriers as in the fp16 consumer: two before the first stage, one per stage (after the
// stage's last LDS read).
constexpr int kCW = 8;                   // consumer waves; each owns BM / kCW rows
constexpr int kRH = BM / kCW;             // rows per consumer wave
constexpr int kRT = kRH / 32;             // 32-row MFMA tiles per consumer wave
template <bool C_F16>
__device__ inline void consume_i8(uint8_t* smem, int wave, int lane, int nb, int job, const GemmJobs& J, float* ws,
                                  void* C, int ldc, int M, int m0, int n0, int R) {
    const int l32 = lane & 31, lh = lane >> 5;
    v16f acc[kRT][NT];
#pragma unroll
    for (int i = 0; i < kRT; i++)
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int q = 0; q < 16; q++) acc[i][j][q] = 0.0f;
    const int xs = (l32 >> 1) & 7;
    const uint32_t a_row = (uint32_t)(wave * kRH + l32) * ROWB, b_row = (uint32_t)l32 * ROWB;
    const float* sxs = (const float*)(smem + kSxOff) + wave * kRH + 8 * ((lane & 15) >> 2) + 4 * lh + (lane & 3);
    const float* sws = (const float*)(smem + kSwOff) + l32;
    barrier_lds();                           // the producers' first copies landed
    barrier_lds();                           // stage 0 produced
    for (int st = 0; st < nb; st++) {
        const uint8_t* at = tile_a(smem, st % kABuf) + a_row;
        const uint8_t* bt = tile_b(smem, st & 1) + b_row;
        v4i af[kRT][4];
#pragma unroll
        for (int i = 0; i < kRT; i++)
#pragma unroll
            for (int kk = 0; kk < 4; kk++) af[i][kk] = *(const v4i*)(at + i * 32 * ROWB + (((2 * kk + lh) ^ xs) << 4));
        float sxv[kRT];
#pragma unroll
        for (int i = 0; i < kRT; i++) sxv[i] = sxs[(st % kABuf) * BM + i * 32];
        float sw[NT];
#pragma unroll
        for (int j = 0; j < NT; j++) sw[j] = sws[(st & 1) * BN + j * 32];
        v16i I[2];
        v4i bfA[4], bfB[4];
        auto ldb = [&](int j, v4i (&bf)[4]) {
#pragma unroll
            for (int kk = 0; kk < 4; kk++) bf[kk] = *(const v4i*)(bt + j * 32 * ROWB + (((2 * kk + lh) ^ xs) << 4));
            if (j == NT - 1) barrier_lds();  // stage st + 1 produced; stage st's buffers free
        };
        auto mmi = [&](int i, int slot, v4i (&bf)[4]) {
#pragma unroll
            for (int q = 0; q < 16; q++) I[slot][q] = 0;
#pragma unroll
            for (int kk = 0; kk < 4; kk++)
                I[slot] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i][kk], bf[kk], I[slot], 0, 0, 0);
        };
        auto fold = [&](int i, int j, int slot) {
            fold_tile(acc[i][j], I[slot], sw[j], sxv[i], std::make_integer_sequence<int, 16>());
        };
        // one 32-row tile: the fold of column tile j follows the MFMAs of tile j + 1
        auto step = [&](int j, v4i (&bn)[4]) {
            if (j + 1 < NT) {
                ldb(j + 1, bn);
                mmi(0, (j + 1) & 1, bn);
            }
            fold(0, j, j & 1);
        };
        static_assert(NT == 4, "the steps below cover four column tiles");
        ldb(0, bfA);
        mmi(0, 0, bfA);
        step(0, bfB);
        step(1, bfA);
        step(2, bfB);
        step(3, bfA);
    }
    // store: lane holds D[8(q/4) + 4(l/32) + q%4][l % 32] of each 32x32 tile
    if (job >= J.n_full) {
        float* P = ws + (size_t)(job - J.n_full) * (BM * BN);
#pragma unroll
        for (int i = 0; i < kRT; i++)
#pragma unroll
            for (int j = 0; j < NT; j++)
#pragma unroll
                for (int q = 0; q < 16; q++)
                    P[(wave * kRH + i * 32 + 8 * (q >> 2) + 4 * lh + (q & 3)) * BN + j * 32 + l32] = acc[i][j][q];
        return;
    }
#pragma unroll
    for (int i = 0; i < kRT; i++)
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int gc = j * 32 + l32;
            const int gn = n0 + gc;
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int gm = m0 + wave * kRH + i * 32 + 8 * (q >> 2) + 4 * lh + (q & 3);
                if (gm < M && gc < R) {
                    if (C_F16) ((_Float16*)C)[(size_t)gm * ldc + gn] = (_Float16)acc[i][j][q];
                    else ((float*)C)[(size_t)gm * ldc + gn] = acc[i][j][q];
                }
            }
        }
}

// Stage = one PTQ1_0 block (128 k).  Producer waves kCW..kCW+3: A stage copies (8 DMA per wave)
// plus the stage's row scales (one dword DMA per wave, rows 64 pw .. +63, clamped to M - 1),
// two stages ahead into three buffers; packed weight bytes of a block staged by DMA two
// blocks ahead; decode of the next stage into one of two B buffers.  Producer lane decodes
// half q = pw & 1 of tile row 64 (pw >> 1) + lane: chunks 0..3 (q = 0: dwords 0..3 at digits
// 0..3) or chunks 4..7 (q = 1: digit 4 of dwords 0..3, dwords 4, 5, the qh bytes).
template <bool C_F16>
__global__ __launch_bounds__(64 * (kCW + 4)) void k_gemm_ptq1_i8(const int8_t* __restrict__ A8, const float* __restrict__ SX,
                                                      int ldS, const uint8_t* __restrict__ W, void* __restrict__ C,
                                                      int ldc, float* __restrict__ ws, int M, int K, int N,
                                                      GemmJobs J) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nbk = K >> 7;
    int job, tile, kb0, nb;
    gemm_job(J, nbk, job, tile, kb0, nb);
    const int m0 = (tile / J.G) * BM;
    const int n0 = (tile % J.G) * BN;
    const int R = min(BN, N - n0);
    const uint32_t row_bytes = (uint32_t)nbk * kBlockBytes;

    if (wave < kCW) {
        consume_i8<C_F16>(smem, wave, lane, nb, job, J, ws, C, ldc, M, m0, n0, R);
        return;
    }

    // ================= producers =================
    const int pw = wave - kCW;
    // an int8 row of 128 k has the byte layout of an fp16 stage row of 64 k
    const _Float16* Ah = (const _Float16*)(A8 + (size_t)kb0 * kGroup);
    const float* sxsrc = SX + (size_t)kb0 * ldS + min(m0 + 64 * pw + lane, M - 1);
    const uint32_t sx_lds = lds_addr(smem + kSxOff) + 256 * pw;
    auto issue_a = [&](int st) {
        gemm::issue_a(smem, pw, lane, Ah, K >> 1, M, m0, st, nb);
        dma4(sxsrc + (size_t)min(st, nb - 1) * ldS, sx_lds + (st % kABuf) * (BM * 4));
    };
    const int wrow = 64 * (pw >> 1) + lane, q = pw & 1;
    const bool wactive = wrow < R;
    uint8_t* Ws = smem + kTileBytes;                                  // [2 slots][2][BN][16 B]
    float* sws = (float*)(smem + kSwOff);
    const uint8_t* wsrc = W + (size_t)min(n0 + min(wrow, R - 1), N - 1) * row_bytes + (size_t)kb0 * kBlockBytes + 12 * q;
    auto issue_w = [&](int blk) {
        dma16(wsrc + (size_t)min(blk, nb - 1) * kBlockBytes,
              lds_addr(Ws + (blk & 1) * kWStage + q * (BN * 16) + (pw >> 1) * 1024));
    };
    uint32_t w[7];
    auto read_w = [&](int blk) {
        const uint8_t* slot = Ws + (blk & 1) * kWStage;
        const uint4 a = *(const uint4*)(slot + wrow * 16);           // bytes 0..15
        const uint4 c = *(const uint4*)(slot + BN * 16 + wrow * 16); // bytes 12..27
        w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
        w[4] = c.y; w[5] = c.z; w[6] = c.w;
    };
    auto decode = [&](int buf) {
        uint8_t* bt = tile_b(smem, buf);
        auto put = [&](int chunk, uint32_t x0, uint32_t x1, uint32_t x2, uint32_t x3) {
            *(uint4*)(bt + swz(wrow, chunk)) = make_uint4(x0, x1, x2, x3);
        };
        if (!wactive) {
            if (q == 0) sws[buf * BN + wrow] = 0.0f;
            return;
        }
        if (q == 0) {
#pragma unroll
            for (int c = 0; c < 4; c++)
                put(c, trits4(w[0], p3x2(c), p3x2(c)), trits4(w[1], p3x2(c), p3x2(c)), trits4(w[2], p3x2(c), p3x2(c)),
                    trits4(w[3], p3x2(c), p3x2(c)));
            sws[buf * BN + wrow] = half_bits_to_float(w[6] >> 16);
        } else {
            put(4, trits4(w[0], p3x2(4), p3x2(4)), trits4(w[1], p3x2(4), p3x2(4)), trits4(w[2], p3x2(4), p3x2(4)),
                trits4(w[3], p3x2(4), p3x2(4)));
            put(5, trits4(w[4], p3x2(0), p3x2(0)), trits4(w[5], p3x2(0), p3x2(0)), trits4(w[4], p3x2(1), p3x2(1)),
                trits4(w[5], p3x2(1), p3x2(1)));
            put(6, trits4(w[4], p3x2(2), p3x2(2)), trits4(w[5], p3x2(2), p3x2(2)), trits4(w[4], p3x2(3), p3x2(3)),
                trits4(w[5], p3x2(3), p3x2(3)));
            const uint32_t qh = __builtin_amdgcn_perm(0u, w[6], 0x01000100u);   // (qh0, qh1, qh0, qh1)
            put(7, trits4(w[4], p3x2(4), p3x2(4)), trits4(w[5], p3x2(4), p3x2(4)), trits4(qh, p3x2(0), p3x2(1)),
                trits4(qh, p3x2(2), p3x2(3)));
        }
    };
    // Vector-memory order of a producer (all LDS copies, counted by the waits below):
    // W(b+2) then A(b+2) (9 copies) per iteration; the wait before the barrier that ends
    // iteration b leaves only A(b+2) in flight, so batch b+1 and block b+2 have landed.
    issue_w(0);
    issue_w(1);
    issue_a(0);
    issue_a(1);
    __builtin_amdgcn_s_waitcnt((9 & 15) | ((9 >> 4) << 14) | (7 << 4) | (15 << 8));       // blocks 0, 1, batch 0
    barrier_lds();
    read_w(0);
    decode(0);
    barrier_lds();
    for (int b = 0; b < nb; b++) {
        // consumers on stage b; produce stage b + 1 into B buffer (b + 1) & 1
        if (b + 1 < nb) read_w(b + 1);
        issue_w(b + 2);                          // into the slot read_w(b) freed
        issue_a(b + 2);
        if (b + 1 < nb) decode((b + 1) & 1);
        __builtin_amdgcn_s_waitcnt((9 & 15) | ((9 >> 4) << 14) | (7 << 4) | (15 << 8));   // batch b+1, block b+2
        barrier_lds();
    }
}

}  // namespace

hipError_t launch_quant_rows(const uint16_t* X, int8_t* Q, float* SX, int M, int K, int ldS, hipStream_t s) {
    const long groups = (long)M * (K / kGroup);
    hipLaunchKernelGGL(k_quant_rows, dim3((unsigned)((groups + 15) / 16)), dim3(256), 0, s, (const _Float16*)X, Q, SX,
                       M, K, ldS);
    return hipGetLastError();
}

hipError_t launch_gemm_i8(const int8_t* A8, const float* SX, int ldS, const uint8_t* W, void* C, int c_dtype,
                          int ldc, int M, int K, int N, hipStream_t s) {
    // the dynamic-LDS limit of both instantiations, raised once per process (a function-local
    // static: thread-safe initialisation)
    static const hipError_t attr = [] {
        hipError_t e = hipFuncSetAttribute((const void*)k_gemm_ptq1_i8<true>, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)k_gemm_ptq1_i8<false>, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
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
        hipLaunchKernelGGL(k_gemm_ptq1_i8<true>, dim3(J.n_jobs), dim3(64 * (kCW + 4)), kLdsBytes, s, A8, SX, ldS, W, C, ldc, ws,
                           M, K, N, J);
    else
        hipLaunchKernelGGL(k_gemm_ptq1_i8<false>, dim3(J.n_jobs), dim3(64 * (kCW + 4)), kLdsBytes, s, A8, SX, ldS, W, C, ldc,
                           ws, M, K, N, J);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_pieces_sum<BM, BN>(ws, C, c_dtype, ldc, M, N, J, s);
}

}  // namespace kata
