// The decode GEMV's activation operand (T = 1 or 2 token rows), shared by the GEMV, the
// prepare kernel and the input transform so that every writer quantises alike.
//
// Quantiser: per 128-block and token, amax = max |x| (a block holding a NaN or an infinity
// gets amax = inf), scale s = amax / 32639 (NaN for such a block), q = rint(x * (32639 /
// amax)) (0 when amax = 0), |q| <= 32639, split into int8 limbs hi = (q + 128) >> 8 and
// lo = q - 256 hi (the low byte of q), so q = 256 hi + lo.
//
// A image of a block: [m 2][g 4][row 2T][16 B], row = 2 t + limb, element e of the block
// at byte gemv_dense_img_off(e, T) + 16 row: the A operand (A[row][k]) of the block's two
// v_mfma_i32_16x16x64_i8, matching the dense B layout of the trits (lane group g holds qs
// bytes 6g .. 6g + 5 and two digits of a qh byte).
//
// The operand form in memory (KATA_XQ): K padded to nq steps of 4 blocks (nq even; blocks
// past K are zero), blocks b = 4 c + quarter in quarter-major order,
//   image  [quarter 4][c nq][block image 256 T B]
//   scales [4 nq][T] pairs (s, 0) of fp32 bits (8 B each)
// which is the GEMV's LDS layout less the pads between its quarters, so a workgroup copies
// it with 16-byte loads and stores.
//
// For T = 3..8 rows (the wide verification GEMV) the operand form is that kernel's image:
//   image  [block nb][m 2][g 4][row 16][16 B]   (rows of tokens >= T zero)
//   scales [block nb][token pair 4] (s of token 2p, s of token 2p + 1) fp32
// 2080 bytes per block, read by every workgroup of the wide GEMV from L2.
#pragma once
#include "common.h"

namespace kata {

constexpr int kXDtypeOperand = 2;  // the x_dtype value of the operand form (KATA_XQ)
constexpr int kXqMaxBytes = 8 * 16 * 1024;   // largest operand form the GEMV copies (128 KB)
constexpr float kQMax = 32639.0f;   // |q| <= 32639 keeps hi = (q+128)>>8 inside int8
constexpr int kDenseMfma = 2;      // MFMAs per block: the dense layout, 32 trits per lane group
constexpr int kAImageBytes = kDenseMfma * 4 * 16;   // per block and A row (token, limb)

// The dense operand layout: lane group g of a B column (one row, one block) holds the 32
// trits of qs bytes 6g .. 6g + 5 (all five digits) and two digits of qh byte 24 + (g >> 1)
// (digits 2(g & 1) and 2(g & 1) + 1), so two MFMAs cover the block's 128 trits with no empty
// slot.  With c0..c5 the lane's six qs bytes the B dwords are
//   m=0: L(c0) L(c1) L(c2) L(c3)      m=1: L(c4) L(c5) Z(c0..c3) {Z(c4), Z(c5), Q(a), Q(a+1)}
// (L = digits 1..4, byte n - 1 for digit n; Z = digit 0; Q = the qh digits).  The lane reads
// the 8 bytes at 4-byte aligned gemv_dense_byte0(g) (c0 at byte offset 2 (g & 1)) and the
// dword at block byte 24 (qh and the scale).  Offset of element e in the block's A image
// [m 2][g 4][i 2T][16 B]:
__host__ __device__ constexpr int gemv_dense_byte0(int g) { return g == 0 ? 0 : g == 1 ? 4 : g == 2 ? 12 : 16; }
__host__ __device__ constexpr int gemv_dense_img_off(int e, int T) {
    int p = 0, n = 0;
    ptq1_elem_src(e, p, n);
    int g = 0, m = 1, slot = 0;
    if (p < 24) {
        g = p / 6;
        const int j = p - 6 * g;
        if (n > 0) {
            m = j < 4 ? 0 : 1;
            slot = 4 * (j & 3) + n - 1;
        } else {
            slot = 8 + j;
        }
    } else {
        g = 2 * (p - 24) + (n >> 1);
        slot = 14 + (n & 1);
    }
    return m * (4 * 2 * T * 16) + g * (2 * T * 16) + slot;
}

// steps (of 4 blocks) per row, rounded up to whole pairs; blocks past K are zero padding
__host__ __device__ constexpr int gemv_nq(int K) { return ((K / kGroup + 3) / 4 + 1) & ~1; }
// image bytes of one block and of one quarter
__host__ __device__ constexpr int gemv_xq_blk_bytes(int T) { return kAImageBytes * 2 * T; }
__host__ __device__ constexpr int gemv_xq_qbytes(int K, int T) { return gemv_nq(K) * gemv_xq_blk_bytes(T); }
// the whole operand form: image + scale pairs (T <= 2), the wide image + scales (T = 3..8)
constexpr int kWideImgBlk = kDenseMfma * 4 * 16 * 16;   // wide image bytes per block (2048)
constexpr int kWideSclBlk = 4 * 8;                       // wide scale bytes per block
__host__ __device__ constexpr long long gemv_xq_bytes(int K, int T) {
    return T <= 2 ? 4LL * gemv_xq_qbytes(K, T) + 8LL * 4 * gemv_nq(K) * T
                  : (long long)(K / kGroup) * (kWideImgBlk + kWideSclBlk);
}

// Block scale from the block's amax (inf for a block holding a non-finite value):
// inv = 32639 / amax (0 for amax = 0 or a non-finite block), s = amax / 32639 (NaN for a
// non-finite block: every output row is then NaN, as the reference's coefficient-form sum
// gives -- its block `sumy` is non-finite, shaders/gemv_fast.metal:21-45).
__device__ inline void gemv_block_scale(float amax, float& inv, float& sc) {
    const bool bad = !(amax <= 3.402823466e38f);
    inv = (amax > 0.0f && !bad) ? kQMax / amax : 0.0f;
    sc = bad ? __builtin_nanf("") : amax * (1.0f / kQMax);
}
// max over the 32 lanes of a half wave: the 16 lanes of a DPP row (xor 1, xor 2, the
// half-row and row mirrors), then the other row of the half (a swizzle, xor 16)
__device__ inline float half32_max(float a) {
    a = fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0xb1, 0xf, 0xf, false)));
    a = fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x4e, 0xf, 0xf, false)));
    a = fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x141, 0xf, 0xf, false)));
    a = fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, a), 0x140, 0xf, 0xf, false)));
    // ds_swizzle bit mode: and 0x1f, or 0, xor 0x10
    return fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, a), 0x401f)));
}

// Element e's byte in a block's A image for T = 1, 2 and 8 rows (gemv_dense_img_off), as
// a table for the producers that place elements by a run-time index.
struct alignas(16) DenseImgOff {
    uint16_t v[3][128];
};
constexpr DenseImgOff make_dense_img_off() {
    DenseImgOff t{};
    for (int e = 0; e < 128; e++) {
        t.v[0][e] = (uint16_t)gemv_dense_img_off(e, 1);
        t.v[1][e] = (uint16_t)gemv_dense_img_off(e, 2);
        t.v[2][e] = (uint16_t)gemv_dense_img_off(e, 8);
    }
    return t;
}

// |x| for the amax, infinity for NaN / infinity
__device__ inline float gemv_amax_term(float v) {
    const float a = fabsf(v);
    return a <= 3.402823466e38f ? a : __builtin_inff();
}
// the two int8 limbs of q = rint(v * inv)
__device__ inline void gemv_limbs(float v, float inv, uint8_t& hi, uint8_t& lo) {
    const int q = (int)rintf(v * inv);
    hi = (uint8_t)((q + 128) >> 8);
    lo = (uint8_t)q;
}

}  // namespace kata
