// PTQ1_0 decode GEMV for T = 1 and T = 2 tokens on the gfx950 int8 matrix cores.
//
// Semantics: y[t][n] = sum_b d[n,b] * sum_e trit[n,b,e] * x[t][128b+e]
// (shaders/gemv.metal:5-20; fast forms shaders/gemv_fast.metal:9-50, shaders/mtp.metal:164-205).
//
// Design (MI355X-first, not the reference's simdgroup float decode):
//  * The packed weight bytes are never expanded in memory.  Per 128-weight block four lanes
//    each hold 32 of its trits (the dense layout of gemv_operand.h: lane group g = lane/16
//    takes qs bytes 6g..6g+5 and two digits of a qh byte, read as 12 bytes per lane) and
//    turn them into trits {-1,0,1} as int8: the trits of digits 1..4 of a byte come from
//    one 4-byte LDS table entry, the digit-0 trit ((3b) >> 8) - 1 from 16-bit-lane
//    multiply-adds.  The trits are the B operand (B[k][column]) of two
//    v_mfma_i32_16x16x64_i8 per block.
//  * The activation is the A operand (A[i][k]) in an integer form: per 128-block a scale
//    s = amax/32639 and q = rint(x/s) split into two int8 limbs (q = 256*hi + lo), either
//    written once by the activation's producer (the operand form, copied into LDS) or
//    built in LDS by every workgroup from fp16/fp32 rows;
//    A rows are (block, token, limb), so T = 2 costs no extra matrix-core work.  The matrix
//    core sums trit*limb exactly in int32, so sum(trit*q) = 256*D_hi + D_lo per block and
//    token, and y += d * s * that in fp32.  The only approximation is the 16-bit
//    block-fixed-point activation (|x - s*q| <= amax/65278), far inside the 1e-3
//    relative-L2 contract.  A block holding a NaN or an infinity gets s = NaN, so every
//    output row is NaN, as the reference's coefficient-form sum gives (its block `sumy` is
//    then non-finite, shaders/gemv_fast.metal:21-45).
//  * Work item = 4 consecutive blocks of a 4-row tile.  The 16 B columns of the MFMA are
//    (row r, block 4c + kq) and the 16 A rows are (block 4c + kq, token, limb), so one item
//    decodes four 112-byte runs of the matrix and the products of mismatched blocks are
//    never read.  One 1024-thread workgroup per CU; each wave keeps one block step's A
//    operand in registers while it walks the CU's tiles (see the kernel comment); no
//    atomics, deterministic.
#include "common.h"
#include "gemv_operand.h"
#include "launch.h"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace kata {

namespace {

constexpr int kWaves = 16;
constexpr int kChunkMax = 3;   // 8-element activation chunks per thread: K <= 3 * 8 * 1024
constexpr int kMaxMats = 4;    // matrices sharing one activation in one launch
// Where the decode GEMV's activation comes from: raw rows loaded per thread into registers,
// raw rows staged in LDS by wave 0's copies (both quantised by every workgroup), or the
// operand form (gemv_operand.h: quantised once by its producer), copied into LDS.
constexpr int kXmRegs = 0, kXmStage = 1, kXmOperand = 2;
constexpr int kXqChunks = 8;   // 16-byte pieces of the operand form per thread: <= 128 KB

// The matrices of one launch (same K, same activation): matrix i is W[i] (N[i] rows), its
// output rows go to y[i][t * ldy[i] + row], and workgroups [wg0[i], wg0[i+1]) serve it with
// tpw[i] tiles of 4 rows each.
struct GemvMats {
    const uint8_t* W[kMaxMats];
    float* y[kMaxMats];
    int N[kMaxMats];
    int tpw[kMaxMats];
    int ldy[kMaxMats];
    int wg0[kMaxMats + 1];
    int count;
};

typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
// Image offsets of the 8 elements a quantising thread owns: thread index & 63 =
// 16*kq + sub, elements 8*sub .. 8*sub + 7 of a block; [T - 1][idx][e].
struct alignas(16) ImgOffTable {
    uint16_t v[2][64][8];
};
constexpr ImgOffTable make_img_off_table() {
    ImgOffTable t{};
    for (int T = 1; T <= 2; T++)
        for (int idx = 0; idx < 64; idx++)
            for (int e = 0; e < 8; e++) t.v[T - 1][idx][e] = (uint16_t)gemv_dense_img_off(8 * (idx & 15) + e, T);
    return t;
}
__constant__ ImgOffTable kImgOff = make_img_off_table();

// Digit table: 256 entries of 4 bytes (digits 1..4 of the byte value), each replicated
// 2^LR times; lane l reads replica l mod 2^LR so the lanes an LDS cycle serves hit distinct
// banks.  With 64 replicas (LR = 6) an entry row is 256 bytes and one v_perm_b32 forms
// the address [replica*4, byte, 0, 0]; smaller tables (when the activation image needs
// the LDS) use a shift and an or.
template <int LR>
__device__ inline uint32_t lut_addr(uint32_t w, int q, uint32_t laneoff) {
    if (LR == 6) return __builtin_amdgcn_perm(w, laneoff, 0x0c0c0400u | ((uint32_t)(4 + q) << 8));
    return (((w >> (8 * q)) & 0xffu) << (LR + 2)) | laneoff;
}
__host__ __device__ constexpr int lut_bytes(int LR) { return 256 * (4 << LR); }
// The same address for byte q of w where q is a per-lane value: sel = lut_sel<LR>(q)
// (the v_perm selector for LR = 6), computed once per lane.
template <int LR>
__host__ __device__ constexpr uint32_t lut_sel(uint32_t q) { return 0x0c0c0400u | ((4u + q) << 8); }
template <int LR>
__device__ inline uint32_t lut_addr_sel(uint32_t w, uint32_t sel, uint32_t q, uint32_t laneoff) {
    if (LR == 6) return __builtin_amdgcn_perm(w, laneoff, sel);
    return (((w >> (8 * q)) & 0xffu) << (LR + 2)) | laneoff;
}

typedef __attribute__((address_space(3))) const uint8_t lds_u8;
// 32-bit load at byte offset addr of an LDS array; for the digit table, the kernel's first
// static LDS array, the base is address 0 and folds away.
__device__ inline uint32_t lds_u32(lds_u8* base, uint32_t addr) {
    return *(__attribute__((address_space(3))) const uint32_t*)(base + addr);
}

// LDS bytes of the A image (4 quarters, 64 B apart) and of the (scale, 0) pairs
// Pad between the image quarters: with 64 the quarters' A-operand reads are conflict free;
// for T = 2 an 80-byte pad cuts the quantiser's scattered byte stores from ~4.75 LDS passes
// to ~1.25 at the cost of some 2-way read conflicts, measured faster (T = 1: not so).
__host__ __device__ constexpr int gemv_qpad(int T) { return T == 2 ? 80 : 64; }
__host__ __device__ inline int gemv_a_lds_bytes(int qbytes, int T) { return 4 * (qbytes + gemv_qpad(T)); }
__host__ __device__ inline int gemv_s_lds_bytes(int nbv, int T) { return (8 * nbv * T + 15) & ~15; }
// static LDS of the GEMV kernel: the trit table
__host__ __device__ constexpr int gemv_static_lds_bytes(int LR) { return lut_bytes(LR); }

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// LDS DMA of 16 bytes per lane: lane l's 16 bytes at g go to LDS byte address lds + 16*l
// (lds wave-uniform).  Issued through inline assembly so that the compiler does not make
// every later LDS access wait for all vector-memory loads in flight (it cannot tell which
// LDS bytes a DMA writes); the kernel waits for these copies explicitly.  M0 is restored.
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

// 8 consecutive activations x[t][k0..k0+7] as floats.  Layouts: rows x[T][K] (fp16 or
// fp32), or half2-interleaved x[K][2] fp16 (T = 2).
template <int T>
__device__ inline void load_x8(const void* x, int x_dtype, int x_layout, int K, int k0, float (&v)[T][8]) {
    if (x_layout == 1) {
        const uint4* p = (const uint4*)((const _Float16*)x + (size_t)k0 * 2);
        const uint4 a = p[0], b = p[1];
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const v2h h = __builtin_bit_cast(v2h, w[i]);
            v[0][i] = (float)h[0];
            if (T == 2) v[T - 1][i] = (float)h[1];
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < T; t++) {
        if (x_dtype == 1) {
            const uint4 a = *(const uint4*)((const _Float16*)x + (size_t)t * K + k0);
            const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const v2h h = __builtin_bit_cast(v2h, w[i]);
                v[t][2 * i] = (float)h[0];
                v[t][2 * i + 1] = (float)h[1];
            }
        } else {
            const float4* p = (const float4*)((const float*)x + (size_t)t * K + k0);
            const float4 a = p[0], b = p[1];
            v[t][0] = a.x; v[t][1] = a.y; v[t][2] = a.z; v[t][3] = a.w;
            v[t][4] = b.x; v[t][5] = b.y; v[t][6] = b.z; v[t][7] = b.w;
        }
    }
}

// The same from a raw copy of x in LDS (same layouts).
template <int T>
__device__ inline void load_x8_lds(const uint8_t* xs, int x_dtype, int x_layout, int K, int k0, float (&v)[T][8]) {
    if (x_layout == 1) {
        const uint4* p = (const uint4*)(xs + (size_t)k0 * 4);
        const uint4 a = p[0], b = p[1];
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const v2h h = __builtin_bit_cast(v2h, w[i]);
            v[0][i] = (float)h[0];
            if (T == 2) v[T - 1][i] = (float)h[1];
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < T; t++) {
        if (x_dtype == 1) {
            const uint4 a = *(const uint4*)(xs + ((size_t)t * K + k0) * 2);
            const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const v2h h = __builtin_bit_cast(v2h, w[i]);
                v[t][2 * i] = (float)h[0];
                v[t][2 * i + 1] = (float)h[1];
            }
        } else {
            const float4* p = (const float4*)(xs + ((size_t)t * K + k0) * 4);
            const float4 a = p[0], b = p[1];
            v[t][0] = a.x; v[t][1] = a.y; v[t][2] = a.z; v[t][3] = a.w;
            v[t][4] = b.x; v[t][5] = b.y; v[t][6] = b.z; v[t][7] = b.w;
        }
    }
}

// f(integral_constant<int, i>) for i = 0 .. NN-1, unrolled at compile time
template <int I, int NN, typename F>
__device__ inline void static_for_impl(F&& f) {
    if constexpr (I < NN) {
        f(std::integral_constant<int, I>{});
        static_for_impl<I + 1, NN>(f);
    }
}
template <int NN, typename F>
__device__ inline void static_for(F&& f) {
    static_for_impl<0, NN>(f);
}

// Butterfly max / sum over the 16 lanes of a DPP row (xor 1, xor 2, then the half-row
// and row mirrors), every lane ends with the result; fixed order, so deterministic.
__device__ inline float row16_max(float a) {
    a = fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0xb1, 0xf, 0xf, false)));
    a = fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x4e, 0xf, 0xf, false)));
    a = fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x141, 0xf, 0xf, false)));
    a = fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x140, 0xf, 0xf, false)));
    return a;
}
__device__ inline int row16_sum(int a) {
    a += __builtin_amdgcn_mov_dpp(a, 0xb1, 0xf, 0xf, false);
    a += __builtin_amdgcn_mov_dpp(a, 0x4e, 0xf, 0xf, false);
    a += __builtin_amdgcn_mov_dpp(a, 0x141, 0xf, 0xf, false);
    a += __builtin_amdgcn_mov_dpp(a, 0x140, 0xf, 0xf, false);
    return a;
}
__device__ inline float row16_fsum(float a) {
    a += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0xb1, 0xf, 0xf, false));
    a += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x4e, 0xf, 0xf, false));
    a += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x141, 0xf, 0xf, false));
    a += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x140, 0xf, 0xf, false));
    return a;
}

// trit 0 = ((3b) >> 8) - 1 of the four bytes of w as int8, byte k for byte k of w.  Bytes
// (0,2) and (1,3) are spread into 16-bit lanes; 3b - 256 (no carry between the lanes) has
// the trit in its high byte.
__device__ inline uint32_t trit0_word(uint32_t w) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const u16x2 e = __builtin_bit_cast(u16x2, w & 0x00ff00ffu);
    const u16x2 o = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, w, 0x0c030c01u));
    const u16x2 e3 = e * (u16x2){3, 3} + (u16x2){0xff00, 0xff00};
    const u16x2 o3 = o * (u16x2){3, 3} + (u16x2){0xff00, 0xff00};
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, o3), __builtin_bit_cast(uint32_t, e3), 0x07030501u);
}

// Digit-table entry of byte value bv (< 256): the trits of digits 1..4 as int8, byte n - 1
// for digit n.  m_n = (bv * 3^n) mod 256 for two digits at a time in 16-bit lanes (bv * 81
// < 2^16); 3 m_n - 256 holds the trit (digit - 1) in its high byte.
__device__ inline uint32_t trit_entry(uint32_t bv) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const u16x2 b = (u16x2){(unsigned short)bv, (unsigned short)bv};
    const u16x2 m12 = (b * (u16x2){3, 9}) & (u16x2){0xff, 0xff};
    const u16x2 m34 = (b * (u16x2){27, 81}) & (u16x2){0xff, 0xff};
    const u16x2 h12 = m12 * (u16x2){3, 3} + (u16x2){0xff00, 0xff00};
    const u16x2 h34 = m34 * (u16x2){3, 3} + (u16x2){0xff00, 0xff00};
    return __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, h34), __builtin_bit_cast(uint32_t, h12), 0x07050301u);
}

// Dense decode (the layout at gemv_dense_img_off) of one lane's share of a block: w0, w1 the 8
// bytes at gemv_dense_byte0(g), wq the block's bytes 24..27 (qh, scale).  Per-lane constants
// (DenseLane): the byte shift of c0 in the 8 bytes (2 (g & 1)), the perm selectors that take
// c4, c5 and the qh byte, and the multipliers 3^a, 3^(a+1) of the lane's two qh digits
// (a = 2 (g & 1)).  B[0], B[1] are the B operands of the block's two MFMAs.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
struct DenseLane {
    uint32_t csh, sel_c4, sel_c5, sel_z45, sel_q;
    u16x2 qmul;
};
template <int LR>
__device__ inline DenseLane dense_lane(int g) {
    DenseLane L;
    L.csh = 2u * (uint32_t)(g & 1);
    L.sel_c4 = lut_sel<LR>(L.csh);
    L.sel_c5 = lut_sel<LR>(L.csh + 1);
    L.sel_z45 = 0x0c000c00u | ((L.csh + 1) << 16) | L.csh;               // (c4, 0, c5, 0)
    const uint32_t qb = (uint32_t)(g >> 1);
    L.sel_q = 0x0c000c00u | (qb << 16) | qb;                             // (qh, 0, qh, 0)
    L.qmul = (g & 1) ? (u16x2){9, 27} : (u16x2){1, 3};
    return L;
}
template <int LR>
__device__ inline void dense_decode(uint32_t w0, uint32_t w1, uint32_t wq, lds_u8* lb, uint32_t laneoff,
                                    const DenseLane& L, v4i* B) {
    const uint32_t c03 = __builtin_amdgcn_alignbyte(w1, w0, L.csh);       // c0..c3
    B[0] = v4i{(int)lds_u32(lb, lut_addr<LR>(c03, 0, laneoff)), (int)lds_u32(lb, lut_addr<LR>(c03, 1, laneoff)),
               (int)lds_u32(lb, lut_addr<LR>(c03, 2, laneoff)), (int)lds_u32(lb, lut_addr<LR>(c03, 3, laneoff))};
    const u16x2 z45 = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, w1, L.sel_z45)) * (u16x2){3, 3} +
                      (u16x2){0xff00, 0xff00};
    const u16x2 mq = (__builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, wq, L.sel_q)) * L.qmul) & (u16x2){0xff, 0xff};
    const u16x2 hq = mq * (u16x2){3, 3} + (u16x2){0xff00, 0xff00};
    B[1] = v4i{(int)lds_u32(lb, lut_addr_sel<LR>(w1, L.sel_c4, L.csh, laneoff)),
               (int)lds_u32(lb, lut_addr_sel<LR>(w1, L.sel_c5, L.csh + 1, laneoff)), (int)trit0_word(c03),
               (int)__builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, hq), __builtin_bit_cast(uint32_t, z45), 0x07050301u)};
}

// Work split ("activation-stationary").  One 1024-thread workgroup (16 waves) per CU owns
// the contiguous tile range [wt0, wt0 + Tt) (4 rows per tile) of one matrix.  Its work
// items (c, tile) — 4 consecutive blocks 4c..4c+3 of the tile's 4 rows — are numbered by
// pairs of block steps, s = (c / 2) * 2 Tt + 2 tile + c % 2 (nq rounded up to even), and cut
// into 16 contiguous runs of even length, one per wave, so a wave keeps the A operands of
// one pair (c, c + 1) in registers across many tiles and reloads them from LDS only when the
// pair changes.  Consecutive items of a wave read the two halves of 224 contiguous bytes of
// each row, so a 128-byte line shared by block steps c and c + 1 is read twice in a row;
// with the steps a whole pass over the tiles apart, a launch whose weights exceed an XCD's
// L2 fetched such lines twice from memory.  Lane x + 16*g: B column x = (row r = x & 3, block 4c + kq
// with kq = x >> 2), A row x = (block 4c + (x >> 2), token (x >> 1) & 1, limb x & 1);
// result rows 4g..4g+3 belong to block 4c + g, so lane 20*q + r holds row r's sum over
// block 4c + q.  Those 16 lanes store their scaled sums to the item's LDS slot (the other
// lanes store to a scratch slot: no exec-mask changes in the loop; the two items of a step
// pair add in registers first, halving the slots); at the end each output row adds its
// nq * 2 slots in a fixed order (deterministic, no atomics).
//
// Timeline.  (1) Wave 0 (the first wave of the workgroup to launch) copies the scatter
// offsets and (XS) the raw activation into LDS by DMA before any weight load is queued on
// the CU; every wave writes its part of the trit table and clears the A image, then issues
// its first weight items into a register ring of D slots (item j in slot j % D).  (2) After a
// barrier each thread quantises its activation chunks (block amax by DPP) and (3) scatters
// the limbs into the A image.  (4) Every wave decodes item j + 1 while the matrix cores
// run item j and reloads each ring slot after use; the loop body keeps scalar bookkeeping
// to a few instructions per item (the CU issues one scalar instruction per SIMD every
// four cycles, the same rate as the wave64 vector instructions).
// Dynamic LDS: A image (384*T B per virtual block, quarters 64 B apart), (scale, 0)
// pairs [vb][t], the scatter offsets (1 KB), a scratch slot for the off-diagonal lanes
// (512 B), then item sums [S][T][16] floats, which with XS first hold the raw activation.
template <int T, int LR, int D, bool PAD, int XM, bool MULTI, bool STRIDE>
__global__ __launch_bounds__(1024) void k_gemv_ptq1(GemvMats P, const void* __restrict__ x, int x_dtype, int x_layout,
                                                    int K, int nq) {
#pragma clang fp contract(off)
    static_assert(D % 2 == 0 && D >= 4, "operand double buffers alternate by item parity");
    constexpr bool XS = XM == kXmStage, XQ = XM == kXmOperand;
    constexpr int ASTRIDE = 4 * 2 * T * 16;      // A image bytes per (virtual block, MFMA)
    constexpr int BLK = kDenseMfma * ASTRIDE;     // A image bytes per virtual block
    constexpr int REPS = 1 << LR;
    constexpr int QPAD = gemv_qpad(T);
    // trit table first: the kernel's static LDS starts at address 0
    __shared__ uint4 lut[lut_bytes(LR) / 16];
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int x_ = lane & 15, g = lane >> 4;
    const int r = x_ & 3, kq = x_ >> 2;
    const int nb = K >> 7, nbv = 4 * nq;
    // this workgroup's matrix (workgroups [wg0[i], wg0[i+1]) serve matrix i) and tile range
    // One matrix (MULTI false): only entry 0 is read, the kernel arguments span one cache
    // line less.  Several: every field is read before any is selected (the empty asm takes
    // them all as inputs); otherwise the compiler turns the selection into branches around
    // dependent argument loads, a chain of memory latencies at kernel start.
    const uint8_t* __restrict__ W = P.W[0];
    float* __restrict__ y = P.y[0];
    int N = P.N[0], tpw = P.tpw[0], ldy = P.ldy[0], wg0 = 0;
    // the activation pointer and layout are read with the matrix fields, not later inside
    // wave 0's branch (a second argument-load round trip before its first copy)
    asm volatile("" ::"s"(x), "s"(x_dtype), "s"(x_layout), "s"(K), "s"(nq));
    if constexpr (MULTI) {
        const uint8_t* Wv[kMaxMats] = {P.W[0], P.W[1], P.W[2], P.W[3]};
        float* yv[kMaxMats] = {P.y[0], P.y[1], P.y[2], P.y[3]};
        int Nv[kMaxMats] = {P.N[0], P.N[1], P.N[2], P.N[3]};
        int tv[kMaxMats] = {P.tpw[0], P.tpw[1], P.tpw[2], P.tpw[3]};
        int lv[kMaxMats] = {P.ldy[0], P.ldy[1], P.ldy[2], P.ldy[3]};
        int gv[kMaxMats] = {P.wg0[0], P.wg0[1], P.wg0[2], P.wg0[3]};
        const int cnt = P.count;
        asm volatile("" ::"s"(Wv[0]), "s"(Wv[1]), "s"(Wv[2]), "s"(Wv[3]), "s"(yv[0]), "s"(yv[1]), "s"(yv[2]), "s"(yv[3]));
        asm volatile("" ::"s"(Nv[0]), "s"(Nv[1]), "s"(Nv[2]), "s"(Nv[3]), "s"(tv[0]), "s"(tv[1]), "s"(tv[2]), "s"(tv[3]));
        asm volatile("" ::"s"(lv[0]), "s"(lv[1]), "s"(lv[2]), "s"(lv[3]), "s"(gv[1]), "s"(gv[2]), "s"(gv[3]), "s"(cnt));
        int mi = 0;
#pragma unroll
        for (int i = 1; i < kMaxMats; i++) mi = (i < cnt && (int)blockIdx.x >= gv[i]) ? i : mi;
        wg0 = gv[0];
#pragma unroll
        for (int i = 1; i < kMaxMats; i++) {
            W = mi == i ? Wv[i] : W;
            y = mi == i ? yv[i] : y;
            N = mi == i ? Nv[i] : N;
            tpw = mi == i ? tv[i] : tpw;
            ldy = mi == i ? lv[i] : ldy;
            wg0 = mi == i ? gv[i] : wg0;
        }
    }
    const int tiles = (N + 3) >> 2;
    const int wt0 = ((int)blockIdx.x - wg0) * tpw;
    const int Tt = min(tiles, wt0 + tpw) - wt0;
    const int S = nq * Tt;                       // nq is even: whole pairs of block steps
    const int s0 = ((wave * S) / kWaves) & ~1, s1 = wave == kWaves - 1 ? S : (((wave + 1) * S) / kWaves) & ~1;
    // STRIDE (chosen for long tile ranges with few step pairs per row): tile-strided order,
    // wave w takes pair w % np for tiles h, h + G, h + 2G, ... (h = w / np, G = 16 / np
    // phases), so at any time the waves read neighbouring pieces of the same few tiles; the
    // waves past G np stay idle.  Same items and slots as the run order: the same results.
    // Every workgroup of such a launch takes it (a short last range too: the waves whose
    // phase has no tile get no items), so a wave's pair never changes and the loop has no
    // pair-change or tile-wrap test (lm_head 62.1 -> 61.0 us).
    const int np = nq >> 1, G = kWaves / np;
    constexpr bool strided = STRIDE;
    const int sp = strided ? wave % np : 0, sh = strided ? wave / np : 0;
    const int n = !strided ? s1 - s0                     // this wave's run length (even, wave-uniform)
                           : (wave < G * np && sh < Tt ? 2 * ((Tt - sh + G - 1) / G) : 0);
    const int qbytes = nq * BLK;                 // A image bytes per quarter
    uint8_t* As = smem;
    uint8_t* Ss = smem + gemv_a_lds_bytes(qbytes, T);            // (scale, 0) pairs [vb][t]
    uint8_t* Os = Ss + gemv_s_lds_bytes(nbv, T);               // scatter offsets [64][8] u16
    uint8_t* Js = Os + 1024;                                   // scratch slots (1 KB)
    float* part = (float*)(Js + 1024);                         // [S / 2][T][16]
    uint8_t* Xs = (uint8_t*)part;                // XS: raw activation, until the main loop

    // (1a) wave 0: DMA of the scatter offsets and (XS) the raw activation; without XS every
    // thread loads its own chunks.  Chunk j = tid + 1024 i covers k = 8j..8j+7 of every
    // token; the 16 chunks of a block are 16 consecutive lanes (one DPP row), and their
    // quarter (j >> 4) & 3 and sub-block position j & 15 do not depend on i.
    const int nch = K >> 3;
    const int xbytes = T * K * (x_dtype == 1 ? 2 : 4);
    float v[XM != kXmRegs ? 1 : kChunkMax][T][8];
    if (!XQ && wave == 0) {
        dma16((const uint4*)&kImgOff.v[T - 1][0][0] + lane, lds_addr(Os));
        if constexpr (XS) {
            const int xvec = xbytes / 16;
            for (int o = 0; o < xvec; o += 64) dma16((const uint4*)x + min(o + lane, xvec - 1), lds_addr(Xs + o * 16));
        }
    }
    if constexpr (XM == kXmRegs) {
#pragma unroll
        for (int i = 0; i < kChunkMax; i++) {
            const int j = tid + 1024 * i;
            if (j < nch) load_x8<T>(x, x_dtype, x_layout, K, 8 * j, v[i]);
        }
    }
    // XQ: the operand form, 16 bytes per thread and piece, loaded before the weight ring so
    // that it lands first; pieces past its end read zero (whole absent pieces are skipped)
    const int xqb = 4 * qbytes + 8 * nbv * T;     // gemv_xq_bytes(K, T)
    uint4 xr[XQ ? kXqChunks : 1];
    if constexpr (XQ) {
        const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc((void*)x, 0, xqb, 0x00020000);
#pragma unroll
        for (int i = 0; i < kXqChunks; i++)
            if (i * 1024 * 16 < xqb)
                xr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xrs, (tid + 1024 * i) * 16, 0, 0));
    }

    // (1b) trit table.  Consecutive threads store consecutive 16-byte words (no bank
    // conflicts); word o holds 4 replicas of entry o / (REPS / 4): trits of digits 1..4.
    // A batch launch builds it after the first half of its weight ring (below): its longer
    // ring runs gain from the earlier loads (decode sweep step 43.4 -> 42.8 us), one-matrix
    // launches lose 1-5 % that way.
    auto build_table = [&]() {
#pragma unroll
        for (int i = 0; i < lut_bytes(LR) / 16 / 1024; i++) {
            const int o = tid + i * 1024;
            const uint32_t e = trit_entry((uint32_t)o / (REPS / 4));
            lut[o] = make_uint4(e, e, e, e);
        }
    };
    if constexpr (!MULTI) build_table();
    // clear the A image (slots without an element and padding blocks stay zero) and the
    // scales of the padding blocks
    if constexpr (!XQ) {
        for (int o = tid; o < gemv_a_lds_bytes(qbytes, T) / 16; o += 1024) ((uint4*)As)[o] = make_uint4(0, 0, 0, 0);
        for (int o = nb * T + tid; o < nbv * T; o += 1024) ((int2*)Ss)[o] = make_int2(0, 0);
    }

    // (1c) weight ring.  Raw buffer loads: per-lane offset (row r of the tile, block kq of
    // the step, the lane group's 8 bytes, and the block's qh / scale dword) plus a
    // wave-uniform item offset; bytes past the matrix read as 0 (rows >= N; with PAD also the
    // padding blocks of the last row).  Loads past the run's end use an offset beyond the
    // buffer: zeros, no memory access.
    const uint32_t row_bytes = (uint32_t)nb * kBlockBytes;
    const uint32_t tstep = 4 * row_bytes;        // next tile
    const __amdgpu_buffer_rsrc_t wrsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)W, 0, (int)((uint32_t)N * row_bytes), 0x00020000);
    const uint32_t voff = (uint32_t)r * row_bytes + (uint32_t)kq * kBlockBytes + (uint32_t)gemv_dense_byte0(g);
    // item s = (c/2, tile, c%2): pair index s / (2 Tt), tile (s % (2 Tt)) / 2, block step
    // parity s % 2; runs start at even s, so the ring slot's parity is the item's
    int lt = strided ? sh : (s0 % (2 * Tt)) >> 1;   // load cursor: tile, item offset, items left
    uint32_t lso = (uint32_t)(wt0 + lt) * tstep + (uint32_t)(2 * (strided ? sp : s0 / (2 * Tt))) * 4 * kBlockBytes;
    int lrem = n;
    const int Tw = Tt;                           // run order: the pair changes after tile Tw - 1
    const uint32_t cstep = 4 * kBlockBytes;      // even c -> c + 1, same tile
    const uint32_t tnext = (strided ? G : 1) * tstep - cstep;    // odd c -> c - 1, next tile
    const uint32_t cwrap = cstep - (uint32_t)(Tt - 1) * tstep;   // odd c, last tile -> next pair
    // 12 bytes per lane: lane group 3's third dword is the block's bytes 24..27 (qh, scale),
    // which the other lane groups of the column take from it by a cross-lane permute
    uint32_t wl[D], wh[D], wq[D];
    auto load_next = [&](int slot) {
        const uint32_t so = lrem > 0 ? lso : 0x80000000u;
        const u32x3 w = __builtin_bit_cast(u32x3, __builtin_amdgcn_raw_buffer_load_b96(wrsrc, (int)voff, (int)so, 0));
        wq[slot] = w.z;
        wl[slot] = w.x;
        wh[slot] = w.y;
        if (slot & 1) {
            if constexpr (STRIDE) {
                lso += tnext;
            } else {
                const bool wrap = ++lt == Tw;
                lt = wrap ? 0 : lt;
                lso += wrap ? cwrap : tnext;
            }
        } else {
            lso += cstep;
        }
        --lrem;
    };
    // XQ: half the ring now and half once the operand form has landed (below): a smaller first
    // burst of weight loads lets the operand arrive sooner while the stream still starts at
    // once (decode sweep step 45.4 -> 44.9 us; the whole ring after the operand: 3 % slower)
#pragma unroll
    for (int u = 0; u < (XQ ? D / 2 : D); u++) load_next(u);
    if constexpr (MULTI) build_table();

    // XQ: the operand form into the LDS layout (piece at byte o of the form: o plus one pad
    // per quarter before it; the scale pairs follow the fourth quarter's pad)
    if constexpr (XQ) {
#pragma unroll
        for (int i = 0; i < kXqChunks; i++) {
            const int o = (tid + 1024 * i) * 16;
            if (i * 1024 * 16 < xqb && o < xqb) {
                const int q = (o >= qbytes) + (o >= 2 * qbytes) + (o >= 3 * qbytes) + (o >= 4 * qbytes);
                *(uint4*)(As + o + q * QPAD) = xr[i];
            }
        }
    }
    if constexpr (XQ) {
#pragma unroll
        for (int u = D / 2; u < D; u++) load_next(u);
    }
    // the staged offsets and activation (wave 0: everything but the D ring loads has
    // landed), the trit table and the cleared image (XQ: the copied operand) are visible
    // after this barrier
    __builtin_amdgcn_s_waitcnt((D & 15) | ((D >> 4) << 14) | (7 << 4) | (0 << 8));   // vmcnt(D) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();

    // (2) quantise (the quantiser of gemv_operand.h) and (3) scatter the limbs: element
    // 8*(j & 15) + e of block j >> 4 goes to image offset gemv_dense_img_off(8*(j & 15) + e, T)
    // + 16*(2t + limb) of that block.  XQ: done by the operand's producer.
    if constexpr (!XQ) {
        const uint4 offw = *(const uint4*)(Os + (tid & 63) * 16);
        const uint32_t ow[4] = {offw.x, offw.y, offw.z, offw.w};
        int off[8];
#pragma unroll
        for (int e = 0; e < 8; e++) off[e] = (int)((ow[e >> 1] >> (16 * (e & 1))) & 0xffffu);
        auto process = [&](int j, float (&vv)[T][8]) {
            const int b = j >> 4;
            uint8_t* img = As + (b & 3) * (qbytes + QPAD) + (b >> 2) * BLK;
#pragma unroll
            for (int t = 0; t < T; t++) {
                float a = 0.0f;
#pragma unroll
                for (int e = 0; e < 8; e++) a = fmaxf(a, gemv_amax_term(vv[t][e]));
                float inv, sc;
                gemv_block_scale(row16_max(a), inv, sc);
                if ((j & 15) == 0) ((int2*)Ss)[b * T + t] = make_int2(__builtin_bit_cast(int, sc), 0);
#pragma unroll
                for (int e = 0; e < 8; e++) gemv_limbs(vv[t][e], inv, img[off[e] + 32 * t], img[off[e] + 32 * t + 16]);
            }
        };
        if constexpr (XS) {
            for (int j = tid; j < nch; j += 1024) {   // whole 16-lane rows drop out together
                float vv[T][8];
                load_x8_lds<T>(Xs, x_dtype, x_layout, K, 8 * j, vv);
                process(j, vv);
            }
        } else {
#pragma unroll
            for (int i = 0; i < kChunkMax; i++) {
                const int j = tid + 1024 * i;
                if (j < nch) process(j, v[i]);
            }
        }
        // LDS-only barrier: a release fence here would also wait for the weight ring
        __builtin_amdgcn_s_waitcnt((63 & 15) | ((63 >> 4) << 14) | (7 << 4) | (0 << 8));   // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
    }

    // (4) main loop
    const uint32_t laneoff = (uint32_t)(lane & (REPS - 1)) * 4u;
    lds_u8* lb = (lds_u8*)lut;
    // A rows with token >= T only feed result rows that are never stored
    const uint8_t* xa = As + kq * (qbytes + QPAD) + g * (2 * T * 16) + (x_ & (2 * T - 1)) * 16;
    const float* xs = (const float*)Ss + kq * (2 * T);
    // item sums: the two items of a block-step pair (consecutive, same tile) are added in
    // registers; the diagonal lanes 20*q + r store the pair's sum to slot 4q + r of the
    // pair's LDS slot, the others to a scratch word.  Pair u/2 of a ring pass stores at
    // pcur + 64 T (u/2) (an immediate offset); after a pass pcur advances by 64 T D/2 on the
    // diagonal lanes and stays on the others, whose scratch words stay inside the 1 KB area.
    const uint32_t diag = g == kq ? 1u : 0u;
    // (strided: the pair slots of a wave are G tiles apart; the launch takes the strided
    // order only where the other lanes' scratch words still stay inside the 1 KB area)
    const uint32_t pstep = (uint32_t)(strided ? G : 1) * T * 64;
    uint8_t* pcur = diag ? (uint8_t*)part + (g * 4 + r) * 4 + (uint32_t)(strided ? sp * Tt + sh : s0 >> 1) * T * 64
                         : Js + lane * 4;
    const uint32_t pinc = diag * (D / 2) * pstep;
    float vprev[T];
    v4i A[2][kDenseMfma];                        // block steps 2 cp and 2 cp + 1
    float sc[2][T];
    auto load_a = [&](int cp) {
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int c = 2 * cp + h;
#pragma unroll
            for (int m = 0; m < kDenseMfma; m++) A[h][m] = *(const v4i*)(xa + c * BLK + m * ASTRIDE);
#pragma unroll
            for (int t = 0; t < T; t++) sc[h][t] = xs[c * 8 * T + 2 * t];
        }
    };
    const DenseLane dl = dense_lane<LR>(g);
    const int qsrc = (lane | 48) << 2;
    auto decode = [&](uint32_t w0, uint32_t w1, uint32_t& wqv, v4i* B) {
        wqv = (uint32_t)__builtin_amdgcn_ds_bpermute(qsrc, (int)wqv);   // block bytes 24..27, from lane group 3
        dense_decode<LR>(w0, w1, wqv, lb, laneoff, dl, B);
    };
    int ct = strided ? 0 : (s0 % (2 * Tt)) >> 1, cp = strided ? sp : s0 / (2 * Tt);   // compute cursor: tile, pair
    v4i B0[kDenseMfma], B1[kDenseMfma];
    // The pending item: its MFMA results Dp, its scales fp (the activation scale s, and d as
    // the upper half of its qh/scale word dw; with PAD the product d s), its slot dp.  Without
    // PAD the sum is d * (D s): one mixed-precision fma takes d straight from the fp16 bits
    // (decode sweep step -0.7 %).  DEFER (the tile-strided order: long runs): an item is scaled and stored in
    // the next item's body, after that item's MFMAs are issued, so the next decode covers
    // their latency (lm_head 68.3 -> 63.8 us); the first pending item is a dummy (odd, zero)
    // whose store goes to the lane's scratch word, and the run's last item, always odd (runs
    // are whole pairs), is finished after the loop.  Otherwise an item is finished in its own
    // body (short runs: 0.05-0.1 us faster on the sweep's small matrices).
    constexpr bool DEFER = STRIDE;
    v4i Dp = {0, 0, 0, 0};
    float fp[T];
    float* dp = (float*)(Js + lane * 4);
#pragma unroll
    for (int t = 0; t < T; t++) fp[t] = vprev[t] = 0.0f;
    uint32_t dw = 0;
    auto finish = [&](auto oc) {
#pragma unroll
        for (int t = 0; t < T; t++) {
            // explicit fma, contraction off (below): every instantiation (one matrix or a
            // batch) rounds alike, so a batched launch equals the per-matrix launches bit for bit
            const float fi = (float)(Dp[2 * t] * 256 + Dp[2 * t + 1]);
            if constexpr (PAD) {
                if constexpr (decltype(oc)::value)
                    dp[16 * t] = __builtin_fmaf(fi, fp[t], vprev[t]);
                else
                    vprev[t] = fi * fp[t];
            } else {
                const float dd = (float)__builtin_bit_cast(_Float16, (unsigned short)(dw >> 16));
                const float q = fi * fp[t];
                if constexpr (decltype(oc)::value)
                    dp[16 * t] = __builtin_fmaf(dd, q, vprev[t]);
                else
                    vprev[t] = __builtin_fmaf(dd, q, 0.0f);
            }
        }
    };
    // item in ring slot u; `next`: item + 1 is in the run (its operands are read here)
    auto body = [&](auto uc, bool next) {
        constexpr int u = decltype(uc)::value;
        if (next) decode(wl[(u + 1) % D], wh[(u + 1) % D], wq[(u + 1) % D], (u & 1) ? B0 : B1);
        const v4i* B = (u & 1) ? B1 : B0;
        v4i Dm = {0, 0, 0, 0};
#pragma unroll
        for (int m = 0; m < kDenseMfma; m++) Dm = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[u & 1][m], B[m], Dm, 0, 0, 0);
        if constexpr (DEFER) finish(std::integral_constant<bool, (u & 1) == 0>{});   // the previous item
        Dp = Dm;
        dp = (float*)(pcur + (u >> 1) * pstep);
        if constexpr (PAD) {
            float d = half_bits_to_float(wq[u] >> 16);
            if (4 * (2 * cp + (u & 1)) + kq >= nb) d = 0.0f;
#pragma unroll
            for (int t = 0; t < T; t++) fp[t] = d * sc[u & 1][t];
        } else {
            dw = wq[u];
#pragma unroll
            for (int t = 0; t < T; t++) fp[t] = sc[u & 1][t];
        }
        if constexpr (!DEFER) finish(std::integral_constant<bool, (u & 1) == 1>{});
        if constexpr (!STRIDE) {
            if ((u & 1) && ++ct == Tw) {
                ct = 0;
                ++cp;
                if (next) load_a(cp);
            }
        }
    };
    if (n > 0) {
        load_a(cp);
        decode(wl[0], wh[0], wq[0], B0);
    }
    int j = 0;
    for (; j + D < n; j += D) {                  // full passes: every item has a successor
        static_for<D>([&](auto uc) {
            body(uc, true);
            load_next(decltype(uc)::value);
        });
        pcur += pinc;
    }
    static_for<D>([&](auto uc) {                 // the last 1..D items
        constexpr int u = decltype(uc)::value;
        if (j + u < n) body(uc, j + u + 1 < n);
    });
    if constexpr (DEFER) finish(std::true_type{});
    __syncthreads();

    // row sums: output (tile tl, row rr, token t) adds its pair slots over step pairs
    // ascending and quarters ascending, 16 lanes per output (lane sub takes pairs sub,
    // sub + 16, ...), then a fixed-order DPP reduction over the 16 lanes
    for (int o16 = tid; o16 < Tt * 4 * T * 16; o16 += 1024) {
        const int o = o16 >> 4, sub = o16 & 15;
        const int tl = o / (4 * T), rr = (o / T) & 3, t = o % T;
        float sum = 0.0f;
        for (int cp2 = sub; cp2 < nq / 2; cp2 += 16) {
            const float* p = part + ((cp2 * Tt + tl) * T + t) * 16 + rr;
#pragma unroll
            for (int q = 0; q < 4; q++) sum += p[4 * q];
        }
        sum = row16_fsum(sum);
        const int row = (wt0 + tl) * 4 + rr;
        if (sub == 0 && row < N) y[(size_t)t * ldy + row] = sum;
    }
}


// ---------------------------------------------------------------------------------------
// Padded LDS image the wide quantiser scatters into: per lane group 256 B of A rows + 16 B,
// per MFMA 4 groups, per block 2 MFMAs.  The pads spread the quantiser's byte stores over
// the LDS banks (a store instruction of the unpadded layout needs ~15 passes, this one
// ~1.25).  kWideOff[e]: offset of element e's high limb for token 0 in that layout.
constexpr int kWideG = 272, kWideM = 4 * kWideG;
constexpr int kWideBlkBytes = kDenseMfma * kWideM;

struct alignas(16) WideOffTable {
    uint16_t v[128];
};
constexpr WideOffTable make_wide_off_table() {
    WideOffTable t{};
    for (int e = 0; e < 128; e++) {
        const int o = gemv_dense_img_off(e, 8);     // [mfma][g][row 16][16 B], unpadded
        t.v[e] = (uint16_t)((o >> 10) * kWideM + ((o >> 8) & 3) * kWideG + (o & 15));
    }
    return t;
}
__constant__ WideOffTable kWideOff = make_wide_off_table();

// Wide verification GEMV for T = 3..8 token rows: the same integer arithmetic as the decode
// GEMV (16-bit block fixed-point activation in two int8 limbs, exact int32 block sums,
// fp32 scale and accumulate) with the MFMA operands laid out for tokens: B column = one of
// 16 weight rows of a tile (lane group g decodes its dense share of the row's block), A row
// i = (token i >> 1, limb i & 1) of the same block, so all 16 x 16 products are used (2
// v_mfma_i32_16x16x64_i8 per 16 rows x 128 weights).
//
// The A operand image of the T token rows, [block][mfma 2][lane group 4][A row 16][16 B]
// (2048 B per block), and the per (block, token) scales [block][token pair] (float2) are
// the operand form of gemv_operand.h: written once by its producer (an input transform, or
// k_gemv_vw_prep from fp16 / fp32 rows into a stream buffer).  k_gemv_vw: one 512-thread
// workgroup (8 waves) per CU owns a contiguous range of at most kVwTMax tiles of 16 rows
// of the concatenated rows of 1..4 matrices that share the tokens (the batch form) and
// all of K.  Per K chunk of at most kVwCBMax blocks wave w takes blocks [w cb / 8,
// (w+1) cb / 8) of the chunk: it loads their A operands from the image (L2-resident, read by
// every workgroup) into registers, then runs the workgroup's tiles in order, the weight loads
// of tile t + 1 issued before tile t is computed (issuing every tile's loads first left the
// compute waiting for the whole stream: 13.6 against 11.5 us on ffn_gate at T = 8), adding
// into one fp32 accumulator pair per tile, blocks in order (in a whole share of a chunk a
// block's products are added after the next block's MFMAs issue, so that decode covers
// their latency).  At the end the 8 waves' accumulators add in a fixed tree
// order (waves 4..7 into 0..3, 2..3 into 0..1, 1 into 0) through LDS: deterministic, and
// no K split over workgroups (no partial sums, no reduction launch).
constexpr int kVwTMax = 9;                       // tiles per workgroup (the switch in k_gemv_vw)
constexpr int kVwCBMax = 40;                     // blocks per K chunk (the waves' register share)
constexpr int kVwWaves = 8;
constexpr int kVwBB = kVwCBMax / kVwWaves;       // blocks of a wave per chunk
constexpr int kVwLR = 6;                         // 64 trit-table replicas (conflict-free lookups)
constexpr int kVwAhead = 1;                      // tiles whose weight loads run ahead of the compute
constexpr int kVwImgBlk = kWideImgBlk;           // image bytes per block (2048)
constexpr int kVwPrepBlocks = 1;                 // blocks per prep workgroup (one: the shortest chain)
constexpr int kVwPrepThreads = kVwPrepBlocks >= 2 ? 256 : 128;   // 8 tokens x 16 chunks per block
static_assert(8 * kVwPrepBlocks * 16 % kVwPrepThreads == 0, "whole quantisation tasks per prep thread");

struct VwMats {
    const uint8_t* W[kMaxMats];
    float* y[kMaxMats];
    int N[kMaxMats];
    int ldy[kMaxMats];
    int t0[kMaxMats + 1];                        // first tile of matrix i in the concatenation
    int count;
};

// Image of kVwPrepBlocks blocks per workgroup: task j = (token, block, 8-element chunk), 16
// consecutive lanes per (token, block) for the amax; s = amax / 32639, q = rint(x * 32639 /
// amax) (0 for amax = 0; a block holding NaN or an infinity gets s = NaN), limbs hi = (q +
// 128) >> 8 at A row 2t and lo = q - 256 hi at row 2t + 1.  The bytes are scattered into a
// padded LDS copy (strides kWideG: ~1.25 LDS passes per store instruction), then written
// out unpadded with 16-byte stores.  Rows of tokens >= T and slots without an element are
// zero, and so are the scales of tokens >= T.
template <bool XF16>
__global__ __launch_bounds__(kVwPrepThreads) void k_gemv_vw_prep(const void* __restrict__ x, int K, int T,
                                                      uint8_t* __restrict__ img, float2* __restrict__ scl) {
    __shared__ __align__(16) uint8_t im[kVwPrepBlocks * kWideBlkBytes];
    const int tid = threadIdx.x;
    const int nb = K >> 7;
    const int blk0 = blockIdx.x * kVwPrepBlocks, cb = min(kVwPrepBlocks, nb - blk0);
    constexpr int QI = 8 * kVwPrepBlocks * 16 / kVwPrepThreads;
    constexpr int XW = XF16 ? 1 : 2;
    const int ntask = T * cb * 16;
    uint4 xr[QI][XW];
#pragma unroll
    for (int i = 0; i < QI; i++) {
        const int j = tid + kVwPrepThreads * i;
        if (j < ntask) {
            const int ch = j & 15, bt = j >> 4;
            const int t = bt / cb, b = bt - t * cb;
            const size_t k0 = (size_t)t * K + (size_t)(blk0 + b) * 128 + ch * 8;
            if constexpr (XF16) {
                xr[i][0] = *(const uint4*)((const _Float16*)x + k0);
            } else {
                xr[i][0] = *(const uint4*)((const float*)x + k0);
                xr[i][XW - 1] = *(const uint4*)((const float*)x + k0 + 4);
            }
        }
    }
    for (int o = tid; o < kVwPrepBlocks * kWideBlkBytes / 16; o += kVwPrepThreads) ((uint4*)im)[o] = make_uint4(0, 0, 0, 0);
    if (tid < cb * 4) scl[(size_t)(blk0 + tid / 4) * 4 + tid % 4] = make_float2(0.0f, 0.0f);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < QI; i++) {
        const int j = tid + kVwPrepThreads * i;
        if (j >= ntask) continue;                // whole 16-lane rows drop out together
        const int ch = j & 15, bt = j >> 4;
        const int t = bt / cb, b = bt - t * cb;
        float v[8];
        if constexpr (XF16) {
            const uint32_t w4[4] = {xr[i][0].x, xr[i][0].y, xr[i][0].z, xr[i][0].w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const v2h h = __builtin_bit_cast(v2h, w4[q]);
                v[2 * q] = (float)h[0];
                v[2 * q + 1] = (float)h[1];
            }
        } else {
            const uint4 a = xr[i][0], c = xr[i][XW - 1];
            v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y); v[2] = __uint_as_float(a.z);
            v[3] = __uint_as_float(a.w); v[4] = __uint_as_float(c.x); v[5] = __uint_as_float(c.y);
            v[6] = __uint_as_float(c.z); v[7] = __uint_as_float(c.w);
        }
        float a = 0.0f;
        bool bad = false;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const float av = fabsf(v[e]);
            bad |= !(av <= 3.402823466e38f);   // NaN or infinity
            a = fmaxf(a, av);
        }
        a = row16_max(bad ? __builtin_inff() : a);
        const bool blk_bad = !(a <= 3.402823466e38f);
        const float inv = (a > 0.0f && !blk_bad) ? kQMax / a : 0.0f;
        if (ch == 0) {
            float* sp = &scl[(size_t)(blk0 + b) * 4 + (t >> 1)].x;
            sp[t & 1] = blk_bad ? __builtin_nanf("") : a * (1.0f / kQMax);
        }
        const uint4 ow4 = *(const uint4*)&kWideOff.v[8 * ch];
        const uint32_t ow[4] = {ow4.x, ow4.y, ow4.z, ow4.w};
        uint8_t* ib = im + b * kWideBlkBytes + 32 * t;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int off = (int)((ow[e >> 1] >> (16 * (e & 1))) & 0xffffu);
            const int q = (int)rintf(v[e] * inv);
            ib[off] = (uint8_t)((q + 128) >> 8);
            ib[off + 16] = (uint8_t)q;
        }
    }
    __syncthreads();
    // unpadded copy out: 16-byte row r of lane group g of MFMA m of block b
    for (int o = tid; o < cb * kDenseMfma * 4 * 16; o += kVwPrepThreads) {
        const int r = o & 15, g = (o >> 4) & 3, mb = o >> 6, m = mb % kDenseMfma, b = mb / kDenseMfma;
        *(uint4*)(img + (size_t)blk0 * kVwImgBlk + o * 16) =
            *(const uint4*)(im + b * kWideBlkBytes + m * kWideM + g * kWideG + r * 16);
    }
}

__global__ __launch_bounds__(512) void k_gemv_vw(VwMats P, const uint8_t* __restrict__ ximg,
                                                 const float2* __restrict__ xscl, int K, int T, int total_tiles) {
    constexpr int REPS = 1 << kVwLR;
    __shared__ uint4 lut[lut_bytes(kVwLR) / 16];
    __shared__ float2 red[kVwWaves / 2][kVwTMax][64];   // the final tree
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int xn = lane & 15, g = lane >> 4;
    const int nb = K >> 7;
    const size_t row_bytes = (size_t)nb * kBlockBytes;
    // balanced split of the tiles: the first total % grid workgroups take one tile more (32-bit
    // arithmetic; a 64-bit division here was a long software sequence at kernel start)
    const int tq = total_tiles / (int)gridDim.x, tr = total_tiles - tq * (int)gridDim.x;
    const int bx = (int)blockIdx.x;
    const int tw0 = bx * tq + min(bx, tr);
    const int Tt = tq + (bx < tr ? 1 : 0);

    // per tile slot: this lane's row (clamped to the matrix: rows past it read its last row,
    // whose results are not stored) at its segment of block 0
    // (every matrix field is read once, up front, and selected by value: indexing the
    // kernel arguments with a tile's matrix index made a chain of dependent argument loads)
    const uint8_t* Wv[kMaxMats] = {P.W[0], P.W[1], P.W[2], P.W[3]};
    int Nv[kMaxMats] = {P.N[0], P.N[1], P.N[2], P.N[3]};
    int t0v[kMaxMats] = {P.t0[0], P.t0[1], P.t0[2], P.t0[3]};
    const int cnt = P.count;
    asm volatile("" ::"s"(Wv[0]), "s"(Wv[1]), "s"(Wv[2]), "s"(Wv[3]), "s"(Nv[0]), "s"(Nv[1]), "s"(Nv[2]), "s"(Nv[3]));
    asm volatile("" ::"s"(t0v[1]), "s"(t0v[2]), "s"(t0v[3]), "s"(cnt));
    const uint8_t* wp[kVwTMax];
#pragma unroll
    for (int t = 0; t < kVwTMax; t++) {
        const int gt = tw0 + min(t, Tt - 1);
        const uint8_t* Wm = Wv[0];
        int Nm = Nv[0], t0m = t0v[0];
#pragma unroll
        for (int i = 1; i < kMaxMats; i++) {
            const bool sel = i < cnt && gt >= t0v[i];
            Wm = sel ? Wv[i] : Wm;
            Nm = sel ? Nv[i] : Nm;
            t0m = sel ? t0v[i] : t0m;
        }
        const int row = min((gt - t0m) * 16 + xn, Nm - 1);
        wp[t] = Wm + (size_t)row * row_bytes + gemv_dense_byte0(g);
    }

    const uint32_t laneoff = (uint32_t)(lane & (REPS - 1)) * 4u;
    lds_u8* lb = (lds_u8*)lut;
    const DenseLane dl = dense_lane<kVwLR>(g);
    const int qsrc = (lane | 48) << 2;
    const uint8_t* xa = ximg + g * 256 + xn * 16;
    float acc[kVwTMax][2];
#pragma unroll
    for (int t = 0; t < kVwTMax; t++) acc[t][0] = acc[t][1] = 0.0f;

    for (int kb0 = 0; kb0 < nb; kb0 += kVwCBMax) {
        const int cb = min(kVwCBMax, nb - kb0);
        const int bw0 = (wave * cb) / kVwWaves, nbw = ((wave + 1) * cb) / kVwWaves - bw0;
        // (1) the A operands and scales of the wave's blocks, straight from the image (in L2:
        // every workgroup reads it) into registers, issued before the weight loads
        v4i A[kVwBB][kDenseMfma];
        float2 sc[kVwBB];
#pragma unroll
        for (int bb = 0; bb < kVwBB; bb++) {
            const int b = kb0 + min(bw0 + bb, cb - 1);
#pragma unroll
            for (int m = 0; m < kDenseMfma; m++) A[bb][m] = *(const v4i*)(xa + (size_t)b * kVwImgBlk + m * 1024);
            sc[bb] = xscl[(size_t)b * 4 + g];
        }
        // (3) the weight loads of the wave's blocks run kVwAhead tiles ahead of the tile being
        // computed: tiles 0 .. kVwAhead-1 are issued first (and, in the first chunk, the trit
        // table is built while they are in flight), then tile t is computed and tile
        // t + kVwAhead issued, so the weight stream and the decode + MFMA overlap.  The tile
        // loop is instantiated for each tile count (a switch on Tt), so it is straight-line
        // code and each tile waits only for its own loads.  Blocks past the wave's (a ragged
        // chunk) load a valid dummy address.
        auto run = [&](auto ttc) {
            constexpr int TT = decltype(ttc)::value;
            // 12 bytes per lane and block: the lane's 8 and (lane group 3) the qh / scale dword
            uint32_t wl[TT][kVwBB], wh[TT][kVwBB], wq[TT][kVwBB];
            auto issue = [&](int t) {
#pragma unroll
                for (int bb = 0; bb < kVwBB; bb++) {
                    const uint8_t* a = bb < nbw ? wp[t] + (size_t)(kb0 + bw0 + bb) * kBlockBytes : ximg;
                    uint3 w;
                    __builtin_memcpy(&w, a, 12);
                    wl[t][bb] = w.x;
                    wh[t][bb] = w.y;
                    wq[t][bb] = w.z;
                }
            };
#pragma unroll
            for (int t = 0; t < TT && t < kVwAhead; t++) issue(t);
            if (kb0 == 0) {                      // every wave runs the same chunks: uniform
                // the trit table, visible to every wave after this LDS-only barrier
#pragma unroll
                for (int i = 0; i < lut_bytes(kVwLR) / 16 / 512; i++) {
                    const int o = tid + i * 512;
                    const uint32_t e = trit_entry((uint32_t)o / (REPS / 4));
                    lut[o] = make_uint4(e, e, e, e);
                }
                __builtin_amdgcn_s_waitcnt((63 & 15) | ((63 >> 4) << 14) | (7 << 4) | (0 << 8));   // lgkmcnt(0)
                __builtin_amdgcn_s_barrier();
            }
            static_for<TT>([&](auto tc) {
                constexpr int t = decltype(tc)::value;
                if constexpr (t + kVwAhead < TT) issue(t + kVwAhead);
                // block bb's MFMAs and scales (d s of both tokens of the lane's pair)
                auto blk = [&](int bb, v4i& D, float& fx, float& fy) {
                    // the row's qh / scale dword, read by lane group 3
                    const uint32_t wqc = (uint32_t)__builtin_amdgcn_ds_bpermute(qsrc, (int)wq[t][bb]);
                    v4i B[kDenseMfma];
                    dense_decode<kVwLR>(wl[t][bb], wh[t][bb], wqc, lb, laneoff, dl, B);
                    D = v4i{0, 0, 0, 0};
#pragma unroll
                    for (int m = 0; m < kDenseMfma; m++) D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[bb][m], B[m], D, 0, 0, 0);
                    const float d = half_bits_to_float(wqc >> 16);
                    fx = d * sc[bb].x;
                    fy = d * sc[bb].y;
                };
                auto add = [&](const v4i& D, float fx, float fy) {
                    acc[t][0] += (float)(D[0] * 256 + D[1]) * fx;
                    acc[t][1] += (float)(D[2] * 256 + D[3]) * fy;
                };
                if (nbw == kVwBB) {
                    // a whole chunk share (wave-uniform): block bb - 1 is added after block bb's
                    // MFMAs issue, so the next decode covers their latency (same order of adds)
                    v4i Dp;
                    float px, py;
                    blk(0, Dp, px, py);
#pragma unroll
                    for (int bb = 1; bb < kVwBB; bb++) {
                        v4i D;
                        float fx, fy;
                        blk(bb, D, fx, fy);
                        add(Dp, px, py);
                        Dp = D;
                        px = fx;
                        py = fy;
                    }
                    add(Dp, px, py);
                } else {
#pragma unroll
                    for (int bb = 0; bb < kVwBB; bb++) {
                        if (bb < nbw) {
                            v4i D;
                            float fx, fy;
                            blk(bb, D, fx, fy);
                            add(D, fx, fy);
                        }
                    }
                }
            });
        };
        switch (Tt) {
            case 1: run(std::integral_constant<int, 1>{}); break;
            case 2: run(std::integral_constant<int, 2>{}); break;
            case 3: run(std::integral_constant<int, 3>{}); break;
            case 4: run(std::integral_constant<int, 4>{}); break;
            case 5: run(std::integral_constant<int, 5>{}); break;
            case 6: run(std::integral_constant<int, 6>{}); break;
            case 7: run(std::integral_constant<int, 7>{}); break;
            case 8: run(std::integral_constant<int, 8>{}); break;
            default: run(std::integral_constant<int, 9>{}); break;
        }
    }

    // (3) fixed-order tree over the waves through LDS, then wave 0 stores tokens 2g, 2g + 1
    // of row xn of each tile
#pragma unroll
    for (int step = kVwWaves / 2; step >= 1; step /= 2) {
        __syncthreads();
        if (wave >= step && wave < 2 * step) {
#pragma unroll
            for (int t = 0; t < kVwTMax; t++) red[wave - step][t][lane] = make_float2(acc[t][0], acc[t][1]);
        }
        __syncthreads();
        if (wave < step) {
#pragma unroll
            for (int t = 0; t < kVwTMax; t++) {
                const float2 o = red[wave][t][lane];
                acc[t][0] += o.x;
                acc[t][1] += o.y;
            }
        }
    }
    if (wave == 0) {
        float* yv[kMaxMats] = {P.y[0], P.y[1], P.y[2], P.y[3]};
        const int ldv[kMaxMats] = {P.ldy[0], P.ldy[1], P.ldy[2], P.ldy[3]};
#pragma unroll
        for (int t = 0; t < kVwTMax; t++) {
            if (t < Tt) {
                const int gt = tw0 + t;
                float* yy = yv[0];
                int Nm = Nv[0], t0m = t0v[0], ldm = ldv[0];
#pragma unroll
                for (int i = 1; i < kMaxMats; i++) {
                    const bool sel = i < cnt && gt >= t0v[i];
                    yy = sel ? yv[i] : yy;
                    Nm = sel ? Nv[i] : Nm;
                    t0m = sel ? t0v[i] : t0m;
                    ldm = sel ? ldv[i] : ldm;
                }
                const int row = (gt - t0m) * 16 + xn;
                if (row < Nm) {
                    if (2 * g < T) yy[(size_t)(2 * g) * ldm + row] = acc[t][0];
                    if (2 * g + 1 < T) yy[(size_t)(2 * g + 1) * ldm + row] = acc[t][1];
                }
            }
        }
    }
}

}  // namespace


constexpr int kLdsMax = 160 * 1024;

// Weight items in flight per wave.  A deeper ring only stalls the wave at load issue once
// the CU's vector-memory queue is full (16 waves x 4 items x 512 B = 32 KB per CU in
// flight already keep HBM busy), which delays the prologue and the loop.
constexpr int kRing = 4;

// LDS of a GEMV launch: trit table + A image + scales + the larger of the item sums for
// tpw tiles and (xbytes > 0) the staged raw activation, whole 1 KB DMA chunks
static int gemv_lds_bytes(int K, int T, int LR, int tpw, int xbytes) {
    const int nq = gemv_nq(K);
    return gemv_static_lds_bytes(LR) + gemv_a_lds_bytes(nq * kAImageBytes * 2 * T, T) + gemv_s_lds_bytes(4 * nq, T) + 2048 +
           std::max(nq / 2 * tpw * T * 16 * 4, (xbytes + 1023) & ~1023);
}

// the current device's CU count (per device; 256 if it cannot be read)
static int device_cus() {
    int n_cu = 0;
    return device_cu_count(&n_cu) == hipSuccess ? n_cu : 256;
}

template <int T, int LR, bool PAD, int XM, bool MULTI, bool STRIDE = false>
static hipError_t launch_gemv_cfg(const GemvMats& P, const void* x, int x_dtype, int x_layout, int K, int lds,
                                  hipStream_t s) {
    // raised once per process (a function-local static: thread-safe initialisation)
    static const hipError_t attr = hipFuncSetAttribute((const void*)k_gemv_ptq1<T, LR, kRing, PAD, XM, MULTI, STRIDE>,
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       kLdsMax - gemv_static_lds_bytes(LR));
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((k_gemv_ptq1<T, LR, kRing, PAD, XM, MULTI, STRIDE>), dim3(P.wg0[P.count]), dim3(1024),
                       lds - gemv_static_lds_bytes(LR), s, P, x, x_dtype, x_layout, K, gemv_nq(K));
    return hipGetLastError();
}

// The tile-strided order pays off for one matrix with long tile ranges (the 248320-row
// lm_head: 88 -> 78 us) and rows of few step pairs that fill the 16 waves (5 pairs: 15
// waves busy); for the sweep's 6-34 tiles per workgroup it was slower.
// The off-diagonal lanes' scratch stores of a ring pass reach (kRing / 2 - 1) pair slots,
// G T 64 bytes apart, past their word (lane 4 + token 64) in the 1 KB scratch area: the
// strided order is taken only where they stay inside it (G <= 12 for T = 1, <= 5 for T = 2).
static bool gemv_strided(const GemvMats& P, int K, int T) {
    const int np = gemv_nq(K) / 2, G = np > 0 ? 16 / np : 0;
    return P.count == 1 && np > 0 && G >= 2 && G * np >= 15 && P.tpw[0] >= 64 &&
           (kRing / 2 - 1) * G * T * 64 + 64 * (T - 1) + 64 * 4 <= 1024;
}

template <int T, int LR, int XM>
static hipError_t launch_gemv_pad(const GemvMats& P, const void* x, int x_dtype, int x_layout, int K, int lds,
                                  hipStream_t s) {
    if (P.count > 1)
        return (K / kGroup) % 8 ? launch_gemv_cfg<T, LR, true, XM, true>(P, x, x_dtype, x_layout, K, lds, s)
                                : launch_gemv_cfg<T, LR, false, XM, true>(P, x, x_dtype, x_layout, K, lds, s);
    if ((K / kGroup) % 8 == 0 && gemv_strided(P, K, T))
        return launch_gemv_cfg<T, LR, false, XM, false, true>(P, x, x_dtype, x_layout, K, lds, s);
    return (K / kGroup) % 8 ? launch_gemv_cfg<T, LR, true, XM, false>(P, x, x_dtype, x_layout, K, lds, s)
                            : launch_gemv_cfg<T, LR, false, XM, false>(P, x, x_dtype, x_layout, K, lds, s);
}

// Split at most `wgs` workgroups over the matrices in proportion to their tiles (at least
// one each; a launch of more workgroups than CUs would run its last ones as a second
// round), the spare ones to the matrix with the most tiles per workgroup; returns the
// largest tiles-per-workgroup.
static int gemv_split(GemvMats& P, int wgs) {
    int total = 0;
    int w[kMaxMats];
    for (int i = 0; i < P.count; i++) total += (P.N[i] + 3) / 4;
    int used = 0;
    for (int i = 0; i < P.count; i++) {
        w[i] = std::max(1, (int)((long long)((P.N[i] + 3) / 4) * wgs / total));
        used += w[i];
    }
    auto tpw_of = [&](int i) { return ((P.N[i] + 3) / 4 + w[i] - 1) / w[i]; };
    while (used < wgs) {
        int best = 0;
        for (int i = 1; i < P.count; i++)
            if (tpw_of(i) > tpw_of(best)) best = i;
        if (tpw_of(best) == 1) break;
        ++w[best];
        ++used;
    }
    int tmax = 0;
    P.wg0[0] = 0;
    for (int i = 0; i < P.count; i++) {
        const int tiles = (P.N[i] + 3) / 4;
        P.tpw[i] = tpw_of(i);
        P.wg0[i + 1] = P.wg0[i] + (tiles + P.tpw[i] - 1) / P.tpw[i];
        tmax = std::max(tmax, P.tpw[i]);
    }
    for (int i = P.count; i < kMaxMats; i++) P.wg0[i + 1] = P.wg0[P.count];
    return tmax;
}

// Configuration choice, first that fits 160 KB of LDS: about one workgroup per CU, else
// smaller tile ranges (more workgroups); for raw activations the staged copy (kXmStage)
// before per-thread loads, except for K > 8192 (measured: 0.7 us faster at K = 17408,
// slower at 5120); a 64-replica trit table (one v_perm per lookup) before a 16-replica one.
template <int T>
static hipError_t launch_gemv_t(GemvMats& P, const void* x, int x_dtype, int x_layout, int K, hipStream_t s) {
    const int cus = device_cus();
    const int xbytes = T * K * (x_dtype == 1 ? 2 : 4);
    const bool regs_ok = K <= kChunkMax * 8 * 1024;
    for (int wgs = cus;; wgs *= 2) {
        const int tpw = gemv_split(P, wgs);
        int lds;
        if (x_dtype == kXDtypeOperand) {
            if ((lds = gemv_lds_bytes(K, T, 6, tpw, 0)) <= kLdsMax)
                return launch_gemv_pad<T, 6, kXmOperand>(P, x, x_dtype, x_layout, K, lds, s);
            if ((lds = gemv_lds_bytes(K, T, 4, tpw, 0)) <= kLdsMax)
                return launch_gemv_pad<T, 4, kXmOperand>(P, x, x_dtype, x_layout, K, lds, s);
            if (tpw == 1) return hipErrorInvalidValue;
            continue;
        }
        // long activations (K > 8192): per-thread loads start sooner than one wave's copy
        if (K > 8192 && regs_ok && (lds = gemv_lds_bytes(K, T, 6, tpw, 0)) <= kLdsMax)
            return launch_gemv_pad<T, 6, kXmRegs>(P, x, x_dtype, x_layout, K, lds, s);
        if ((lds = gemv_lds_bytes(K, T, 6, tpw, xbytes)) <= kLdsMax)
            return launch_gemv_pad<T, 6, kXmStage>(P, x, x_dtype, x_layout, K, lds, s);
        if ((lds = gemv_lds_bytes(K, T, 4, tpw, xbytes)) <= kLdsMax)
            return launch_gemv_pad<T, 4, kXmStage>(P, x, x_dtype, x_layout, K, lds, s);
        if (regs_ok && (lds = gemv_lds_bytes(K, T, 6, tpw, 0)) <= kLdsMax)
            return launch_gemv_pad<T, 6, kXmRegs>(P, x, x_dtype, x_layout, K, lds, s);
        if (regs_ok && (lds = gemv_lds_bytes(K, T, 4, tpw, 0)) <= kLdsMax)
            return launch_gemv_pad<T, 4, kXmRegs>(P, x, x_dtype, x_layout, K, lds, s);
        if (tpw == 1) return hipErrorInvalidValue;
    }
}

// The operand form (gemv_operand.h) of T raw activation rows: one 256-thread workgroup per 4
// steps (16 blocks, 4 per quarter); thread j quantises elements 8 (j & 15) .. + 7 of block
// 16 w + (j >> 4) (the 16 threads of a block are one DPP row) into an LDS copy of the 16
// block images, which is then written out with 16-byte stores.  Blocks past K are zero.
template <int T>
__global__ __launch_bounds__(256) void k_gemv_prepare(const void* __restrict__ x, int x_dtype, int x_layout, int K,
                                                      uint8_t* __restrict__ xq) {
#pragma clang fp contract(off)
    constexpr int BLK = gemv_xq_blk_bytes(T);
    __shared__ __align__(16) uint8_t stg[16 * BLK];
    const int tid = threadIdx.x, sub = tid & 15, w = blockIdx.x;
    const int nb = K >> 7, nq = gemv_nq(K), qbytes = nq * BLK;
    const int b = 16 * w + (tid >> 4);
    float v[T][8];
    if (b < nb) {
        load_x8<T>(x, x_dtype, x_layout, K, 128 * b + 8 * sub, v);
    } else {
#pragma unroll
        for (int t = 0; t < T; t++)
#pragma unroll
            for (int e = 0; e < 8; e++) v[t][e] = 0.0f;
    }
    uint8_t* img = stg + ((b & 3) * 4 + ((b >> 2) & 3)) * BLK;
#pragma unroll
    for (int t = 0; t < T; t++) {
        float a = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; e++) a = fmaxf(a, gemv_amax_term(v[t][e]));
        float inv, sc;
        gemv_block_scale(row16_max(a), inv, sc);
        if (sub == 0 && b < 4 * nq) ((int2*)(xq + 4 * qbytes))[b * T + t] = make_int2(__builtin_bit_cast(int, sc), 0);
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int off = kImgOff.v[T - 1][sub][e] + 32 * t;
            gemv_limbs(v[t][e], inv, img[off], img[off + 16]);
        }
    }
    __syncthreads();
    // piece p: quarter p / (4 BLK / 16), then 4 consecutive steps of that quarter
    constexpr int PQ = 4 * BLK / 16;
    for (int p = tid; p < 4 * PQ; p += 256) {
        const int q = p / PQ, r = p % PQ, c = 4 * w + (r * 16) / BLK;
        if (c < nq) *(uint4*)(xq + q * qbytes + 4 * w * BLK + r * 16) = *(const uint4*)(stg + p * 16);
    }
}

static hipError_t launch_gemv_vw_prep(const void* x, int x_dtype, int K, int T, uint8_t* ximg, hipStream_t s);

hipError_t launch_gemv_prepare(const void* x, int x_dtype, int x_layout, int K, int T, void* xq, hipStream_t s) {
    if (T > 2) return launch_gemv_vw_prep(x, x_dtype, K, T, (uint8_t*)xq, s);
    const dim3 grid((unsigned)((gemv_nq(K) + 3) / 4));
    if (T == 1)
        hipLaunchKernelGGL(k_gemv_prepare<1>, grid, dim3(256), 0, s, x, x_dtype, x_layout, K, (uint8_t*)xq);
    else
        hipLaunchKernelGGL(k_gemv_prepare<2>, grid, dim3(256), 0, s, x, x_dtype, x_layout, K, (uint8_t*)xq);
    return hipGetLastError();
}

// count matrices of N[i] rows sharing x, one launch.  A matrix whose byte size does not fit
// the 32-bit buffer offsets is split into row chunks (separate entries).
hipError_t launch_gemv_ptq1_multi(int count, const uint8_t* const* W, float* const* y, const int* N, const void* x,
                                  int x_dtype, int x_layout, int K, int T, hipStream_t s) {
    const size_t row_bytes = (size_t)(K / kGroup) * kBlockBytes;
    const int chunk = (int)std::min<size_t>((size_t)1 << 30, ((size_t)1 << 31) / row_bytes / 4 * 4);
    GemvMats P{};
    for (int i = 0; i < count; i++) {
        for (int n0 = 0; n0 < N[i]; n0 += chunk) {
            if (P.count == kMaxMats) return hipErrorInvalidValue;
            P.W[P.count] = W[i] + (size_t)n0 * row_bytes;
            P.y[P.count] = y[i] + n0;
            P.N[P.count] = std::min(chunk, N[i] - n0);
            P.ldy[P.count] = N[i];
            ++P.count;
        }
    }
    return T == 1 ? launch_gemv_t<1>(P, x, x_dtype, x_layout, K, s) : launch_gemv_t<2>(P, x, x_dtype, x_layout, K, s);
}

hipError_t launch_gemv_ptq1(const uint8_t* W, const void* x, int x_dtype, int x_layout, float* y, int K, int N, int T,
                            hipStream_t s) {
    return launch_gemv_ptq1_multi(1, &W, &y, &N, x, x_dtype, x_layout, K, T, s);
}

// ---- wide verification GEMV (T = 3..8): k_gemv_vw_prep writes the token rows' A image
// and scales into `ximg` (nb * kVwImgBytesPerBlock bytes), then one k_gemv_vw launch runs
// the 1..4 matrices sharing them: about one workgroup per CU (more when a CU would get more
// than kVwTMax tiles).
constexpr size_t kVwImgBytesPerBlock = kVwImgBlk + 4 * sizeof(float2);
static_assert(kVwImgBytesPerBlock == kWideImgBlk + kWideSclBlk, "the wide operand form is the prep kernel's image");
size_t gemv_wide_image_bytes(int K) { return (size_t)(K / kGroup) * kVwImgBytesPerBlock; }

// the image and scales of T (1..8) fp16 / fp32 token rows [T][K] into ximg
static hipError_t launch_gemv_vw_prep(const void* x, int x_dtype, int K, int T, uint8_t* ximg, hipStream_t s) {
    const int nb = K / kGroup;
    float2* xscl = (float2*)(ximg + (size_t)nb * kVwImgBlk);
    const dim3 pgrid((nb + kVwPrepBlocks - 1) / kVwPrepBlocks);
    if (x_dtype == 1)
        hipLaunchKernelGGL(k_gemv_vw_prep<true>, pgrid, dim3(kVwPrepThreads), 0, s, x, K, T, ximg, xscl);
    else
        hipLaunchKernelGGL(k_gemv_vw_prep<false>, pgrid, dim3(kVwPrepThreads), 0, s, x, K, T, ximg, xscl);
    return hipGetLastError();
}

static hipError_t launch_gemv_vw(int count, const uint8_t* const* W, float* const* y, const int* N, const void* x,
                                 int x_dtype, int K, int T, uint8_t* ximg, hipStream_t s) {
    if (count < 1 || count > kMaxMats || T < 1 || T > 8) return hipErrorInvalidValue;
    const int nb = K / kGroup;
    const size_t row_bytes = (size_t)nb * kBlockBytes;
    VwMats P{};
    P.count = count;
    long long total = 0;
    for (int i = 0; i < count; i++) {
        P.W[i] = W[i];
        P.y[i] = y[i];
        P.N[i] = N[i];
        P.ldy[i] = N[i];
        P.t0[i] = (int)total;
        total += (N[i] + 15) / 16;
        if ((size_t)N[i] * row_bytes / row_bytes != (size_t)N[i]) return hipErrorInvalidValue;
    }
    for (int i = count; i <= kMaxMats; i++) P.t0[i] = (int)total;
    if (total > 0x3fffffffLL) return hipErrorInvalidValue;
    // the operand form (x_dtype kXDtypeOperand) is the image itself: no prep launch
    if (x_dtype == kXDtypeOperand) ximg = (uint8_t*)x;
    float2* xscl = (float2*)(ximg + (size_t)nb * kVwImgBlk);
    if (x_dtype != kXDtypeOperand) {
        hipError_t e = launch_gemv_vw_prep(x, x_dtype, K, T, ximg, s);
        if (e != hipSuccess) return e;
    }
    const int n_cu = device_cus();
    const long long grid = std::min<long long>(total, std::max<long long>(n_cu, (total + kVwTMax - 1) / kVwTMax));
    hipLaunchKernelGGL(k_gemv_vw, dim3((unsigned)grid), dim3(512), 0, s, P, ximg, xscl, K, T, (int)total);
    return hipGetLastError();
}

// the image in the calling stream's buffer (allocated on the stream's first wide call)
hipError_t launch_gemv_wide_batch(int count, const uint8_t* const* W, float* const* y, const int* N, const void* x,
                                  int x_dtype, int K, int T, hipStream_t s) {
    if (x_dtype == kXDtypeOperand) return launch_gemv_vw(count, W, y, N, x, x_dtype, K, T, nullptr, s);
    void* img = nullptr;
    hipError_t e = stream_buffer(kBufWideImage, gemv_wide_image_bytes(K), s, &img);
    if (e != hipSuccess) return e;
    return launch_gemv_vw(count, W, y, N, x, x_dtype, K, T, (uint8_t*)img, s);
}

hipError_t launch_gemv_wide(const uint8_t* W, const void* x, int x_dtype, float* y, int K, int N, int T,
                            hipStream_t s) {
    return launch_gemv_wide_batch(1, &W, &y, &N, x, x_dtype, K, T, s);
}

// ---- the no-allocation form: the image in a fixed device array.  `scratch` is a host-side
// stand-in for the array, never a device address: the address each device holds its copy at
// comes from hipGetSymbolAddress once per device (with that device current) and only that
// address is handed to kernels.  Calls that overlap on one device share the array and race;
// nothing needs clearing (the prep kernel writes every byte the main kernel reads).
constexpr size_t kNoAllocBytes = (size_t)4 << 20;   // 4 MiB per device
static __device__ __align__(256) uint8_t scratch[kNoAllocBytes];

static hipError_t noalloc_scratch(uint8_t** p) {
    static std::mutex mu;
    static uint8_t* addr[64] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* a = nullptr;
        if ((e = hipGetSymbolAddress(&a, HIP_SYMBOL(scratch))) != hipSuccess) return e;
        addr[dev] = (uint8_t*)a;
    }
    *p = addr[dev];
    return hipSuccess;
}

size_t gemv_wide_noalloc_scratch_bytes() { return kNoAllocBytes; }

bool gemv_wide_noalloc_fits(int K, int T) {
    (void)T;
    return gemv_wide_image_bytes(K) <= kNoAllocBytes;
}

hipError_t launch_gemv_wide_noalloc(const uint8_t* W, const void* x, int x_dtype, float* y, int K, int N, int T,
                                    hipStream_t s) {
    if (x_dtype == kXDtypeOperand) return launch_gemv_vw(1, &W, &y, &N, x, x_dtype, K, T, nullptr, s);
    uint8_t* img = nullptr;
    hipError_t e = noalloc_scratch(&img);
    if (e != hipSuccess) return e;
    return launch_gemv_vw(1, &W, &y, &N, x, x_dtype, K, T, img, s);
}

int gemv_max_mats() { return kMaxMats; }

// Largest K some configuration fits for fp32 activations (fp16 ones never need more LDS).
int gemv_max_k(int T) {
    auto fits = [T](int K) {
        return gemv_lds_bytes(K, T, 4, 1, T * K * 4) <= kLdsMax ||
               (K <= kChunkMax * 8 * 1024 && gemv_lds_bytes(K, T, 4, 1, 0) <= kLdsMax);
    };
    int K = 0;
    while (fits(K + kGroup)) K += kGroup;
    return K;
}

}  // namespace kata
