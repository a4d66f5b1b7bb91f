// Exact fp16 prefill GEMM with the PTQ1_0 decode fused into the LDS tile load.
//
// Semantics (shaders/prefill.metal:31-41 after k_expand_ptq1_v2, :472-479):
//   C[m][n] = sum_k A[m][k] * half(trit[n][k] * d[n][k/128]),  fp16 x fp16 -> fp32.
// half(trit*d) is exact, so every product term equals the reference's; only the fp32
// summation order differs (tolerance-based parity).
//
// Design (MI355X-first; the reference expands every matrix to a 178 MB fp16 stage first):
//  * A workgroup (4 waves) computes a 128 x 16U tile of C, U = 1..18 column units of 16
//    chosen per problem so the grid is close to a multiple of the CU count (pp512 gate/up:
//    128 x 272 -> exactly 256 tiles).  Wave (wm, wn) owns rows 64wm..64wm+63 and about
//    half of the units; each 16x16 output tile is accumulated by v_mfma_f32_16x16x32_f16.
//  * K advances in stages of 64 (half a PTQ1_0 block) through a two-stage LDS pipeline:
//    while the matrix cores consume stage s, the workgroup stores stage s+1's A tile (from
//    registers loaded a stage earlier) and decodes stage s+1's weights straight from the
//    packed bytes into fp16, and the loads for stage s+2 are in flight.  No fp16 weight
//    copy ever touches HBM.
//  * Decode: a group is 4 consecutive k of one row from the 4 bytes of one packed dword
//    and one base-3 digit.  The bytes go to 16-bit lanes (b0,b2) and (b1,b3); the digit is
//    ((b * 3^n) mod 256) * 3 >> 8 with packed 16-bit multiplies, and v_perm_b32 picks the
//    fp16 value -d, 0 or +d for it from one register pair.  Within each group of 4 k the
//    LDS tiles hold the order (k0, k2, k1, k3) - the same permutation for A and for the
//    weights, so the dot products are unchanged - which lets each 16-bit-lane pair be
//    stored as it is.  Wave i of the workgroup decodes the same 4 groups of every row.
//  * LDS rows are 64 halves (128 B) of 8 chunks of 16 B; chunk c of row r is stored at
//    c ^ ((r >> 1) & 7), so the MFMA operand reads and the decode stores spread evenly
//    over the LDS banks.
#include "common.h"
#include "launch.h"

#include <algorithm>
#include <type_traits>

namespace kata {

namespace {

constexpr int BM = 128;          // rows of A / C per workgroup
constexpr int BKS = 64;          // k per stage (halves)
constexpr int kMaxUnits = 18;    // 16-column units per workgroup
constexpr int ROWB = BKS * 2;    // LDS bytes per tile row

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));

// chunk c of row r lives at slot c ^ ((r >> 1) & 7): with the row's parity that gives 16
// distinct 16-byte bank positions over any 16 consecutive rows (MFMA operand reads: 16
// rows x 4 chunks) and over 64 consecutive rows at one chunk (decode stores)
__device__ inline uint32_t swz(int row, int chunk) { return (uint32_t)(row * ROWB + ((chunk ^ ((row >> 1) & 7)) << 4)); }

// (h0..h7) -> (h0,h2,h1,h3, h4,h6,h5,h7): the within-4 k order of the LDS tiles
__device__ inline uint4 permute_k4(uint4 v) {
    uint4 o;
    o.x = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);
    o.y = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);
    o.z = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);
    o.w = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);
    return o;
}

// fp16 of (digit_n(b) - 1) * d for bytes in 16-bit lanes (b_lo, b_hi); lo = (-d, 0),
// hi = (+d, +d) as fp16 bit pairs.  Returns the two halves as one dword.
__device__ inline uint32_t decode_pair(u16x2 b, uint32_t p3n, uint32_t lo, uint32_t hi) {
    u16x2 m = b * __builtin_bit_cast(u16x2, p3n);
    m &= (u16x2){0xff, 0xff};
    const u16x2 dg = (m * (u16x2){3, 3}) >> (u16x2){8, 8};
    const u16x2 sel = dg * (u16x2){0x0202, 0x0202} + (u16x2){0x0100, 0x0100};
    return __builtin_amdgcn_perm(hi, lo, __builtin_bit_cast(uint32_t, sel));
}

// group: bytes of w, digit n -> LDS (b0, b2, b1, b3) at k..k+3 of the row
__device__ inline void decode_group(uint8_t* brow, int row, int k, uint32_t w, uint32_t p3n, uint32_t lo, uint32_t hi) {
    const u16x2 e = __builtin_bit_cast(u16x2, w & 0x00ff00ffu);
    const u16x2 o = __builtin_bit_cast(u16x2, (w >> 8) & 0x00ff00ffu);
    uint2 v;
    v.x = decode_pair(e, p3n, lo, hi);
    v.y = decode_pair(o, p3n, lo, hi);
    *(uint2*)(brow + swz(row, k >> 3) + (k & 7) * 2) = v;
}

__host__ __device__ constexpr uint32_t p3x2(int n) {
    return n == 0 ? 0x00010001u : n == 1 ? 0x00030003u : n == 2 ? 0x00090009u : n == 3 ? 0x001b001bu : 0x00510051u;
}

// Decode groups (e = element of the block, dword j = bytes 4j..4j+3, k = stage-relative
// position = e - 64h).  A row has 16 groups per stage:
//   h=0: dword i, digit n at e = 16n + 4i                         (i, n = 0..3)
//   h=1: dword i digit 4 at e = 64 + 4i; dword 4+i digit n at e = 80 + 4i + 8n (n = 0..4);
//        qh at e = 120..123 and 124..127
// For the extra rows (256..) each wave takes 4 of a row's 16 groups:
//   h=0: dword `wave`, digits 0..3
//   h=1: wave 0: dw0 d4 @64, dw4 d0 @80, dw4 d1 @88, dw4 d2 @96
//        wave 1: dw1 d4 @68, dw4 d3 @104, dw4 d4 @112, dw5 d0 @84
//        wave 2: dw2 d4 @72, dw5 d1 @92, dw5 d2 @100, dw5 d3 @108
//        wave 3: dw3 d4 @76, dw5 d4 @116, qh @120..123, qh @124..127
// weight-tile rows in LDS: 2 waves x 5 tiles of 32 columns (rows past the tile's R are
// read by the MFMAs but never stored)
constexpr int BROWS = 320;
constexpr int kLdsBytes = 2 * BM * ROWB + 2 * BROWS * ROWB;

// Workgroup = 8 waves, two per SIMD: waves 0..3 are consumers (MFMAs over the LDS stage;
// wave (wm, wn) owns rows 64wm.. and about half of the column units), waves 4..7 are
// producers (A tile stores, weight decode and all global loads for the next stages).  The
// SIMD interleaves a consumer's MFMAs with a producer's decode VALU work.  One barrier per
// stage, preceded by an LDS-only wait: the producers' global prefetches stay in flight.
template <bool C_F16, int NWU>
__global__ __launch_bounds__(512) void k_gemm_ptq1_f16(const _Float16* __restrict__ A, int lda,
                                                       const uint8_t* __restrict__ W, void* __restrict__ C,
                                                       int ldc, int M, int K, int N, int G) {
    extern __shared__ __align__(16) uint8_t smem[];
    auto As = [&](int buf) { return smem + buf * (BM * ROWB); };
    auto Bs = [&](int buf) { return smem + 2 * BM * ROWB + buf * (BROWS * ROWB); };
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool consumer = wave < 4;
    const int nb = K >> 7;
    const int m0 = blockIdx.y * BM;
    // column units of this workgroup
    const int U = (N + 15) >> 4;
    const int u0 = (int)(((long)blockIdx.x * U) / G), u1 = (int)(((long)(blockIdx.x + 1) * U) / G);
    const int nu = u1 - u0, n0 = u0 * 16, R = nu * 16;
    auto barrier = [&]() {
        __builtin_amdgcn_s_waitcnt((15 & 15) | ((63 >> 4) << 14) | (7 << 4) | (0 << 8));   // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
    };

    if (consumer) {
        // 32x32x16 MFMAs (the 16x16x32 form issues at half the rate on gfx950): wave (wm, wn)
        // owns rows 64wm..64wm+63 (two 32-row tiles) and 32-column tiles [wt0, wt0 + nwt)
        // of the workgroup's ceil(nu / 2); the last tile may include 16 columns past R,
        // computed from LDS rows that are never stored.
        const int wm = wave >> 1, wn = wave & 1;
        const int l32 = lane & 31, lh = lane >> 5;
        const int T = (nu + 1) >> 1;
        const int wt0 = wn ? (T + 1) >> 1 : 0;
        const int nwt = wn ? T >> 1 : (T + 1) >> 1;
        v16f acc[2][NWU];
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < NWU; j++)
#pragma unroll
                for (int q = 0; q < 16; q++) acc[i][j][q] = 0.0f;
        // all NWU tiles (a wave with fewer computes tiles it never stores; the LDS weight
        // tile has BROWS >= 2 * 32 * NWU rows)
        auto compute = [&](int buf) {
            const uint8_t* at = As(buf);
            const uint8_t* bt = Bs(buf);
#pragma unroll
            for (int kk = 0; kk < BKS / 16; kk++) {
                // lane l: row / column l % 32, k = 16 kk + 8 (l / 32) .. +7 = chunk 2kk + l/32
                v8h af[2], bfs[NWU];
#pragma unroll
                for (int i = 0; i < 2; i++) af[i] = *(const v8h*)(at + swz(wm * 64 + i * 32 + l32, 2 * kk + lh));
#pragma unroll
                for (int j = 0; j < NWU; j++) bfs[j] = *(const v8h*)(bt + swz((wt0 + j) * 32 + l32, 2 * kk + lh));
#pragma unroll
                for (int j = 0; j < NWU; j++)
#pragma unroll
                    for (int i = 0; i < 2; i++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bfs[j], acc[i][j], 0, 0, 0);
            }
        };
        barrier();                                       // stage 0 produced
        for (int b = 0; b < nb; b++) {
            compute(0);
            barrier();
            compute(1);
            barrier();
        }
        // ---- store: lane holds D[8(q/4) + 4(l/32) + q%4][l % 32] of each 32x32 tile
#pragma unroll
        for (int i = 0; i < 2; i++)
#pragma unroll
            for (int j = 0; j < NWU; j++) {
                if (j < nwt) {
                    const int gc = (wt0 + j) * 32 + l32;            // tile column
                    const int gn = n0 + gc;
#pragma unroll
                    for (int q = 0; q < 16; q++) {
                        const int gm = m0 + wm * 64 + i * 32 + 8 * (q >> 2) + 4 * lh + (q & 3);
                        if (gm < M && gc < R && gn < N) {
                            if (C_F16) ((_Float16*)C)[(size_t)gm * ldc + gn] = (_Float16)acc[i][j][q];
                            else ((float*)C)[(size_t)gm * ldc + gn] = acc[i][j][q];
                        }
                    }
                }
            }
        return;
    }

    // ================= producers =================
    const int pw = wave - 4, ptid = tid - 256;
    const uint32_t row_bytes = (uint32_t)nb * kBlockBytes;
    // ---- A: thread -> row ptid/2, chunks 4*(ptid&1) .. +3; stage t's A is loaded into
    // register set t & 1 two stages before it is stored (index clamped to the last stage)
    const int arow = ptid >> 1, achunk = (ptid & 1) * 4;
    const _Float16* a_src = A + (size_t)min(m0 + arow, M - 1) * lda + achunk * 8;
    uint4 areg[2][4];
    const int last_stage = 2 * nb - 1;
    auto load_a = [&](auto set_c, int st) {
        constexpr int set = decltype(set_c)::value;
        const int s2 = min(st, last_stage);
#pragma unroll
        for (int c = 0; c < 4; c++) areg[set][c] = *(const uint4*)(a_src + (size_t)s2 * BKS + c * 8);
    };
    auto store_a = [&](auto set_c, int buf) {
        constexpr int set = decltype(set_c)::value;
#pragma unroll
        for (int c = 0; c < 4; c++) *(uint4*)(As(buf) + swz(arow, achunk + c)) = permute_k4(areg[set][c]);
    };

    // ---- weight bytes: raw buffer loads, 32-bit row offsets, block offset in soffset.
    // Rows 0..255 of the tile: lane `lane` of producer pw owns row 64pw + lane and loads its
    // whole 28-byte block (one x4 and one x3 load, so a load instruction touches one line
    // per row) and decodes all 16 groups of the row per stage.  Rows 256.. (R <= 288): each
    // producer decodes 4 of the 16 groups of row 256 + lane (schedule in the table above).
    const __amdgpu_buffer_rsrc_t wrsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)W, 0, (int)((uint32_t)N * row_bytes), 0x00020000);
    const int rowM = 64 * pw + lane, rowX = 256 + lane;
    const uint32_t offM = (uint32_t)min(n0 + min(rowM, R - 1), N - 1) * row_bytes;
    const uint32_t offX = (uint32_t)min(n0 + min(rowX, R - 1), N - 1) * row_bytes;
    const bool has_x = R > 256;                  // workgroup-uniform
    uint32_t wm_cur[7], wm_nxt[7];               // main row: block being decoded / next
    uint32_t x_cur[4], x_nxt[4];                 // extra row: dword pw, dwb, dword 5, dword 6
    const int dwb = pw < 2 ? 4 : 5;
    auto load_blk = [&](uint32_t* wm7, uint32_t* x4, int blk) {
        const int so = min(blk, nb - 1) * kBlockBytes;
        const uint4 v0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, (int)offM, so, 0));
        typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
        const u32x3 v1 = __builtin_bit_cast(u32x3, __builtin_amdgcn_raw_buffer_load_b96(wrsrc, (int)offM + 16, so, 0));
        wm7[0] = v0.x; wm7[1] = v0.y; wm7[2] = v0.z; wm7[3] = v0.w;
        wm7[4] = v1.x; wm7[5] = v1.y; wm7[6] = v1.z;
        x4[0] = __builtin_amdgcn_raw_buffer_load_b32(wrsrc, (int)(offX + 4 * pw), so, 0);
        x4[1] = __builtin_amdgcn_raw_buffer_load_b32(wrsrc, (int)(offX + 4 * dwb), so, 0);
        x4[2] = __builtin_amdgcn_raw_buffer_load_b32(wrsrc, (int)(offX + 20), so, 0);
        x4[3] = __builtin_amdgcn_raw_buffer_load_b32(wrsrc, (int)(offX + 24), so, 0);
    };
    // Per-producer schedule of the extra row at h=1 as scalars: k (stage-relative) and
    // multiplier pair of groups q = 1..3; group 0 is digit 4 of dword pw at k = 4 * pw.
    // Source: dwb, except producer 1 q3 (dword 5) and producer 3 q2/q3 (the qh bytes as
    // (qh0, qh1, qh0, qh1), digits a, a+1 per lane half).
    const uint32_t k1 = (0x341c2810u >> (8 * pw)) & 0xffu;       // 16, 40, 28, 52
    const uint32_t k2 = (0x38243018u >> (8 * pw)) & 0xffu;       // 24, 48, 36, 56
    const uint32_t k3 = (0x3c2c1420u >> (8 * pw)) & 0xffu;       // 32, 20, 44, 60
    const uint32_t m1 = pw == 0 ? p3x2(0) : pw == 1 ? p3x2(3) : pw == 2 ? p3x2(1) : p3x2(4);
    const uint32_t m2 = pw == 0 ? p3x2(1) : pw == 1 ? p3x2(4) : pw == 2 ? p3x2(2) : 0x00030001u;
    const uint32_t m3 = pw == 0 ? p3x2(2) : pw == 1 ? p3x2(0) : pw == 2 ? p3x2(3) : 0x001b0009u;
    // Main row decode, batched over the 8 independent byte pairs of 4 dwords (the 16-bit
    // lanes (b0,b2), (b1,b3) of each) so the dependent digit chains interleave.  Digits are
    // iterated: t = 3m, digit = t >> 8, next m = t mod 256 (m0 = b); the h=0 stage leaves
    // the pairs' remainders after digit 3 in mrem for digit 4 at h=1.
    u16x2 mrem[8];
    auto emit = [&](uint8_t* bt, int k, u16x2 te, u16x2 to, uint32_t lo, uint32_t hi) {
        const u16x2 se = (te >> (u16x2){8, 8}) * (u16x2){0x0202, 0x0202} + (u16x2){0x0100, 0x0100};
        const u16x2 so = (to >> (u16x2){8, 8}) * (u16x2){0x0202, 0x0202} + (u16x2){0x0100, 0x0100};
        uint2 v;
        v.x = __builtin_amdgcn_perm(hi, lo, __builtin_bit_cast(uint32_t, se));
        v.y = __builtin_amdgcn_perm(hi, lo, __builtin_bit_cast(uint32_t, so));
        *(uint2*)(bt + swz(rowM, k >> 3) + (k & 7) * 2) = v;
    };
    auto split = [&](uint32_t w, u16x2& e, u16x2& o) {
        e = __builtin_bit_cast(u16x2, w & 0x00ff00ffu);
        o = __builtin_bit_cast(u16x2, (w >> 8) & 0x00ff00ffu);
    };
    // stage h of the current block into buffer buf: the main row's 16 groups, then the
    // extra row's 4
    auto decode = [&](auto h_c, int buf) {
        constexpr int h = decltype(h_c)::value;
        uint8_t* bt = Bs(buf);
        {
            const uint32_t dbits = wm_cur[6] >> 16;
            const uint32_t lo = dbits ^ 0x8000u, hi = dbits | (dbits << 16);
            if (h == 0) {
                u16x2 m[8];
#pragma unroll
                for (int i = 0; i < 4; i++) split(wm_cur[i], m[2 * i], m[2 * i + 1]);
#pragma unroll
                for (int n = 0; n < 4; n++) {
                    u16x2 t[8];
#pragma unroll
                    for (int p = 0; p < 8; p++) t[p] = m[p] * (u16x2){3, 3};
#pragma unroll
                    for (int i = 0; i < 4; i++) emit(bt, 16 * n + 4 * i, t[2 * i], t[2 * i + 1], lo, hi);
#pragma unroll
                    for (int p = 0; p < 8; p++) m[p] = t[p] & (u16x2){0xff, 0xff};
                }
#pragma unroll
                for (int p = 0; p < 8; p++) mrem[p] = m[p];
            } else {
                // digit 4 of dwords 0..3 at k = 4i
#pragma unroll
                for (int i = 0; i < 4; i++)
                    emit(bt, 4 * i, mrem[2 * i] * (u16x2){3, 3}, mrem[2 * i + 1] * (u16x2){3, 3}, lo, hi);
                // dwords 4, 5: digits 0..4 at k = 16 + 4i + 8n
                u16x2 m[4];
                split(wm_cur[4], m[0], m[1]);
                split(wm_cur[5], m[2], m[3]);
#pragma unroll
                for (int n = 0; n < 5; n++) {
                    u16x2 t[4];
#pragma unroll
                    for (int p = 0; p < 4; p++) t[p] = m[p] * (u16x2){3, 3};
#pragma unroll
                    for (int i = 0; i < 2; i++) emit(bt, 16 + 4 * i + 8 * n, t[2 * i], t[2 * i + 1], lo, hi);
#pragma unroll
                    for (int p = 0; p < 4; p++) m[p] = t[p] & (u16x2){0xff, 0xff};
                }
                const uint32_t qh = __builtin_amdgcn_perm(0u, wm_cur[6], 0x01000100u);
                decode_group(bt, rowM, 56, qh, 0x00030001u, lo, hi);
                decode_group(bt, rowM, 60, qh, 0x001b0009u, lo, hi);
            }
        }
        if (has_x) {
            const uint32_t dbits = x_cur[3] >> 16;
            const uint32_t lo = dbits ^ 0x8000u, hi = dbits | (dbits << 16);
            if (h == 0) {
#pragma unroll
                for (int q = 0; q < 4; q++) decode_group(bt, rowX, 16 * q + 4 * pw, x_cur[0], p3x2(q), lo, hi);
            } else {
                decode_group(bt, rowX, 4 * pw, x_cur[0], p3x2(4), lo, hi);
                const uint32_t qh = __builtin_amdgcn_perm(0u, x_cur[3], 0x01000100u);
                const uint32_t w23 = pw == 3 ? qh : x_cur[1];
                decode_group(bt, rowX, (int)k1, x_cur[1], m1, lo, hi);
                decode_group(bt, rowX, (int)k2, w23, m2, lo, hi);
                decode_group(bt, rowX, (int)k3, pw == 1 ? x_cur[2] : w23, m3, lo, hi);
            }
        }
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // ---- prologue: stage 0 into buffer 0; stage 1's A, block 1's bytes in flight.  All
    // loads below are unconditional (indices clamped) so the wait counts stay exact.
    load_blk(wm_cur, x_cur, 0);
    load_a(I0(), 0);
    load_a(I1(), 1);
    load_blk(wm_nxt, x_nxt, 1);
    store_a(I0(), 0);
    load_a(I0(), 2);
    decode(I0(), 0);
    barrier();
    for (int b = 0; b < nb; b++) {
        // consumers on stage 2b (buffer 0); produce stage 2b+1 = h1 of block b into buffer 1
        store_a(I1(), 1);
        load_a(I1(), 2 * b + 3);
        decode(I1(), 1);
        barrier();
        // consumers on stage 2b+1 (buffer 1); produce stage 2b+2 = h0 of block b+1
#pragma unroll
        for (int i = 0; i < 7; i++) wm_cur[i] = wm_nxt[i];
#pragma unroll
        for (int i = 0; i < 4; i++) x_cur[i] = x_nxt[i];
        load_blk(wm_nxt, x_nxt, b + 2);
        store_a(I0(), 0);
        load_a(I0(), 2 * b + 4);
        decode(I0(), 0);
        barrier();
    }
}

}  // namespace

// Column groups: about (CUs / row tiles) groups of at most kMaxUnits units; the wave
// unit count selects the kernel instance.
template <int NWU>
static hipError_t launch_nwu(const uint16_t* A, int lda, const uint8_t* W, void* C, int c_dtype, int ldc, int M,
                             int K, int N, int G, dim3 grid, hipStream_t s) {
    static bool attr_done = false;
    if (!attr_done) {
        hipError_t e = hipFuncSetAttribute((const void*)k_gemm_ptq1_f16<true, NWU>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
        if (e == hipSuccess)
            e = hipFuncSetAttribute((const void*)k_gemm_ptq1_f16<false, NWU>,
                                    hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
        if (e != hipSuccess) return e;
        attr_done = true;
    }
    if (c_dtype == 1)
        hipLaunchKernelGGL((k_gemm_ptq1_f16<true, NWU>), grid, dim3(512), kLdsBytes, s, (const _Float16*)A, lda, W, C,
                           ldc, M, K, N, G);
    else
        hipLaunchKernelGGL((k_gemm_ptq1_f16<false, NWU>), grid, dim3(512), kLdsBytes, s, (const _Float16*)A, lda, W,
                           C, ldc, M, K, N, G);
    return hipGetLastError();
}

hipError_t launch_gemm_f16(const uint16_t* A, int lda, const uint8_t* W, void* C, int c_dtype, int ldc,
                           int M, int K, int N, hipStream_t s) {
    static int n_cu = 0;
    if (!n_cu) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 256;
    }
    const int mt = (M + BM - 1) / BM;
    const int U = (N + 15) / 16;
    int G = std::max(1, n_cu / mt);
    G = std::max(G, (U + kMaxUnits - 1) / kMaxUnits);
    G = std::min(G, U);
    const int umax = (U + G - 1) / G;                   // units of the widest workgroup
    const int tmax = ((umax + 1) / 2 + 1) / 2;          // 32-column tiles of its wider wave
    const dim3 grid(G, mt);
    if (tmax <= 1) return launch_nwu<1>(A, lda, W, C, c_dtype, ldc, M, K, N, G, grid, s);
    if (tmax <= 2) return launch_nwu<2>(A, lda, W, C, c_dtype, ldc, M, K, N, G, grid, s);
    if (tmax <= 3) return launch_nwu<3>(A, lda, W, C, c_dtype, ldc, M, K, N, G, grid, s);
    return launch_nwu<5>(A, lda, W, C, c_dtype, ldc, M, K, N, G, grid, s);
}

}  // namespace kata
