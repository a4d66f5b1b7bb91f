// PTQ1_0 decode GEMV for T = 1 and T = 2 tokens on the gfx950 int8 matrix cores.
//
// Semantics: y[t][n] = sum_b d[n,b] * sum_e trit[n,b,e] * x[t][128b+e]
// (shaders/gemv.metal:5-20; fast forms shaders/gemv_fast.metal:9-50, shaders/mtp.metal:164-205).
//
// Design (MI355X-first, not the reference's simdgroup float decode):
//  * The packed weight bytes are never expanded in memory.  A wave owns a 16-row tile and
//    a slice of its K blocks; per 128-weight block each lane holds 8 bytes of one row
//    (lane group g = lane/16 takes block bytes 20..27, 0..7, 8..15, 16..19) and turns them
//    into base-3 digits {0,1,2}: digits 1..4 of a byte come from one 4-byte LDS table
//    entry, digit 0 = (3b) >> 8 from packed 16-bit multiplies.  The digits are the B
//    operand (B[k][row]) of three v_mfma_i32_16x16x64_i8 per block.
//  * The activation is the A operand (A[i][k]) in a prepared integer form: per 128-block
//    a scale s = amax/32639 and q = rint(x/s) split into two int8 limbs (q = 256*hi + lo);
//    A rows are (token, limb), so T = 2 costs no extra matrix-core work.  The matrix core
//    sums digit*limb exactly in int32; the epilogue forms sum(trit*q) = 256*D_hi + D_lo -
//    sum(q) per block and token and accumulates y += d * s * that in fp32.  The only
//    approximation is the 16-bit block-fixed-point activation (|x - s*q| <= amax/65278),
//    far inside the 1e-3 relative-L2 contract.
//  * Work unit = a 4-row tile.  The 16 B columns of the MFMA are (row r, K-quarter kq) and
//    the 16 A rows are (K-quarter, token, limb), so one wave decodes all four quarters of
//    four rows at once and the off-diagonal quarter products are never read.  Each wave
//    owns whole tiles (wave w takes tiles w, w + waves, ...): no barriers and no partial
//    sums outside the wave; the four quarter sums of a row are added with lane shuffles.
//    The digit table and the prepared activation are put in LDS once per workgroup; each
//    wave loads the next chunk's weight bytes while it decodes the current one.
#include "common.h"
#include "launch.h"

#include <stdlib.h>

namespace kata {

namespace {

constexpr float kQMax = 32639.0f;   // |q| <= 32639 keeps hi = (q+128)>>8 inside int8
constexpr int kMfmaPerBlock = 3;
constexpr int kAImageBytes = kMfmaPerBlock * 4 * 16;   // per block and A row (token, limb)

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// A block is read as four 8-byte segments starting at bytes 20, 0, 8, 16 (segment 3 uses
// only bytes 16..19; bytes 20..23 belong to segment 0).  Segment 0 carries the scale.
// Lane group g working on K-quarter kq reads segment (g - kq) & 3, so the lanes whose
// result rows hold that quarter (g == kq) are the ones holding the scale.
__host__ __device__ inline int gemv_seg_byte0(int seg) { return seg == 0 ? 20 : seg == 1 ? 0 : seg == 2 ? 8 : 16; }

// Byte p and digit n of the A/B operand slot (segment seg, MFMA m, dword dw, byte kb),
// or p = -1 for a slot that multiplies a zero activation.  With w0/w1 the lane's two
// weight dwords (bytes b0..b7) the B dwords are
//   m=0: L(b0) L(b1) L(b2) L(b3)     m=1: E(w0) O(w0) L(b4) L(b5)     m=2: L(b6) L(b7) E(w1) O(w1)
// where L(b) = digits 1..4 of byte b and E/O = digit 0 of bytes (0,2) / (1,3) of the dword
// in the low byte of each 16-bit half.
__host__ __device__ inline void gemv_slot(int seg, int m, int dw, int kb, int& p, int& n) {
    const int base = gemv_seg_byte0(seg);
    const int kind = m * 4 + dw;   // 0..11
    // L slots: byte offset within the lane's 8 bytes; E/O slots: -(1 + word*2 + parity)
    const int desc[12] = {0, 1, 2, 3, -1, -2, 4, 5, 6, 7, -3, -4};
    const int d = desc[kind];
    if (d >= 0) {
        p = base + d;
        n = kb + 1;
    } else {
        const int s = -d - 1, word = s >> 1, par = s & 1;
        if (kb & 1) { p = -1; return; }
        p = base + word * 4 + par + kb;
        n = 0;
    }
    if (seg == 3 && p >= 20) p = -1;   // bytes 20..23 belong to segment 0
}

// One workgroup per virtual block vb (0 <= vb < 4*nq; blocks nb.. are zero padding so the
// four K-quarters have nq blocks each).  Writes scale s and sum(q) per token and the A
// image [m 3][g 4][i 2T][16 B], i = 2*t + limb, laid out for lane group g reading segment
// (g - vb/nq) & 3.
template <int T>
__global__ __launch_bounds__(128) void k_gemv_prep(const void* __restrict__ x, int x_dtype, int x_layout,
                                                   uint8_t* __restrict__ xprep, int K, int nq, size_t off_sq,
                                                   size_t off_a) {
    __shared__ int16_t qs[T][128];
    __shared__ float red_f[2][T];
    __shared__ int red_i[2][T];
    const int b = blockIdx.x, e = threadIdx.x, lane = e & 63, wv = e >> 6;
    const bool real = b < K / kGroup;
    float v[T];
#pragma unroll
    for (int t = 0; t < T; t++) {
        const size_t idx = x_layout == 1 ? ((size_t)b * 128 + e) * 2 + t : (size_t)t * K + (size_t)b * 128 + e;
        v[t] = !real ? 0.0f : x_dtype == 1 ? (float)((const _Float16*)x)[idx] : ((const float*)x)[idx];
        float a = fabsf(v[t]);
        for (int o = 32; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o));
        if (lane == 0) red_f[wv][t] = a;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < T; t++) {
        const float amax = fmaxf(red_f[0][t], red_f[1][t]);
        const float inv = amax > 0.0f ? kQMax / amax : 0.0f;
        const float r = fminf(fmaxf(rintf(v[t] * inv), -kQMax), kQMax);
        const int q = (int)r;
        qs[t][e] = (int16_t)q;
        int s = q;
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
        if (lane == 0) red_i[wv][t] = s;
        if (e == 0) ((float*)xprep)[b * T + t] = amax / kQMax;
    }
    __syncthreads();
    if (e < T) ((int*)(xprep + off_sq))[b * T + e] = red_i[0][e] + red_i[1][e];
    const int kq = b / nq;
    uint32_t* out = (uint32_t*)(xprep + off_a + (size_t)b * kAImageBytes * 2 * T);
    for (int w = e; w < kAImageBytes / 4 * 2 * T; w += 128) {
        const int dw = w & 3, i = (w >> 2) % (2 * T), g = (w / (8 * T)) & 3, m = w / (32 * T);
        const int t = i >> 1, limb = i & 1;
        uint32_t word = 0;
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
            int p, n;
            gemv_slot((g - kq) & 3, m, dw, kb, p, n);
            const int el = p >= 0 ? ptq1_slot_elem(p, n) : -1;
            if (el >= 0) {
                const int qq = qs[t][el];
                const int hi = (qq + 128) >> 8, lo = qq - 256 * hi;
                word |= (uint32_t)(uint8_t)(int8_t)(limb ? lo : hi) << (8 * kb);
            }
        }
        out[w] = word;
    }
}

// Digit table: 256 entries of 4 bytes (digits 1..4 of the byte value), each replicated
// 2^LR times; lane l reads replica l mod 2^LR so the lanes an LDS cycle serves hit distinct
// banks.  With 64 replicas (LR = 6) an entry row is 256 bytes and one v_perm_b32 forms
// the address [replica*4, byte, 0, 0]; smaller tables (when the prepared activation needs
// the LDS) use a shift and an or.
template <int LR>
__device__ inline uint32_t lut_addr(uint32_t w, int q, uint32_t laneoff) {
    if (LR == 6) return __builtin_amdgcn_perm(w, laneoff, 0x0c0c0400u | ((uint32_t)(4 + q) << 8));
    return (((w >> (8 * q)) & 0xffu) << (LR + 2)) | laneoff;
}
__host__ __device__ constexpr int lut_bytes(int LR) { return 256 * (4 << LR); }

// digit 0 of bytes (0,2) (odd = false) or (1,3) (odd = true) of w, in the low byte of each
// 16-bit half; v_perm spreads the two bytes into the halves
__device__ inline uint32_t digit0_pair(uint32_t w, bool odd) {
    const uint32_t spread = __builtin_amdgcn_perm(0u, w, odd ? 0x0c030c01u : 0x0c020c00u);
    u16x2 v = __builtin_bit_cast(u16x2, spread);
    v = (v * (u16x2){3, 3}) >> (u16x2){8, 8};
    return __builtin_bit_cast(uint32_t, v);
}

// 32-bit LDS load at a byte address of this kernel's dynamic LDS, which starts at address 0
// (the kernel declares no static LDS), so table addresses need no base added.
__device__ inline uint32_t lds_u32(uint32_t addr) {
    return *(const __attribute__((address_space(3))) uint32_t*)(size_t)addr;
}

// Work split: one 1024-thread workgroup (16 waves) per CU owns a contiguous range of
// tiles, taken in rounds of up to RMAX tiles.  A round's (tile, block step) pairs are cut
// into 16 equal contiguous runs, one per wave; a wave adds up each tile its run touches and
// writes the partial sum to LDS, and after the round's barrier the partials are summed in
// wave order (deterministic).  Lane x + 16*g: B column x = (row r = x & 3, quarter
// kq = x >> 2), A row x = (quarter x >> 2, token (x >> 1) & 1, limb x & 1); result rows
// 4g..4g+3 belong to quarter g, so lane r + 20*kq holds row r's quarter-kq sum.  Runs are
// walked in chunks of at most CH steps inside one tile, the next chunk's weights in flight,
// each block's operands issued one block ahead of its MFMAs.  Dynamic LDS: digit table,
// A image (384*T B per virtual block, 64 B between quarters), scales and sums, partials.
constexpr int kWaves = 16;
constexpr int kRoundTiles = 32;
template <int T, int LR, int CH>
__global__ __launch_bounds__(1024) void k_gemv_ptq1(const uint8_t* __restrict__ W, const uint8_t* __restrict__ xprep,
                                                    float* __restrict__ y, int K, int N, int nq, int tpw,
                                                    size_t off_sq, size_t off_a) {
    constexpr int ASTRIDE = 4 * 2 * T * 16;      // A image bytes per (virtual block, MFMA)
    constexpr int REPS = 1 << LR;
    constexpr int QPAD = 64;
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int x = lane & 15, g = lane >> 4;
    const int r = x & 3, kq = x >> 2;
    const int nb = K >> 7, nbv = 4 * nq;
    const int tiles = (N + 3) >> 2;
    const int wt0 = blockIdx.x * tpw, wt1 = min(tiles, wt0 + tpw);
    const size_t row_bytes = (size_t)nb * kBlockBytes;
    const int seg_off = gemv_seg_byte0((g - kq) & 3);
    const int qbase = kq * nq;                   // this lane's first (virtual) block

    uint32_t wl[CH], wh[CH];
    auto load_chunk = [&](int tile, int c, int n) {
        const uint8_t* rp = W + (size_t)min(tile * 4 + r, N - 1) * row_bytes + seg_off;
#pragma unroll
        for (int i = 0; i < CH; i++) {
            if (i < n) {
                const int blk = min(qbase + c + i, nb - 1);   // padding blocks read any real block
                const uint32_t* q = (const uint32_t*)(rp + (size_t)blk * kBlockBytes);
                wl[i] = q[0];
                wh[i] = q[1];
            }
        }
    };
    // this wave's run of round rt0..rt1: steps [s0, s1) of (tile - rt0) * nq + c
    auto run_of = [&](int rt0, int rt1, int& s0, int& s1) {
        const int S = (rt1 - rt0) * nq;
        s0 = (wave * S) / kWaves;
        s1 = ((wave + 1) * S) / kWaves;
    };
    auto chunk_len = [&](int s, int s1) { return min(min(CH, nq - s % nq), s1 - s); };
    {
        int s0, s1;
        run_of(wt0, min(wt1, wt0 + kRoundTiles), s0, s1);
        if (s0 < s1) load_chunk(wt0 + s0 / nq, s0 % nq, chunk_len(s0, s1));
    }

    const int qbytes = nq * kAImageBytes * 2 * T;
    uint8_t* As = smem + lut_bytes(LR);
    const int a_bytes = 4 * (qbytes + QPAD);
    float* sxs = (float*)(As + a_bytes);
    int* sqs = (int*)(sxs + nbv * T);
    float* part = (float*)(sqs + nbv * T);       // [kRoundTiles][kWaves][4 rows][T]
    {
        const uint4* src = (const uint4*)(xprep + off_a);
        for (int o = tid; o < 4 * qbytes / 16; o += 1024) {
            const int q = o / (qbytes / 16);
            *(uint4*)(As + o * 16 + q * QPAD) = src[o];
        }
        const float* gsx = (const float*)xprep;
        const int* gsq = (const int*)(xprep + off_sq);
        for (int o = tid; o < nbv * T; o += 1024) { sxs[o] = gsx[o]; sqs[o] = gsq[o]; }
        // table: groups of 4 threads compute one entry each and fill its replicas 4 at a time
        {
            const uint32_t bv = (uint32_t)tid >> 2;
            const uint32_t m1 = (bv * 3u) & 0xffu, m2 = (m1 * 3u) & 0xffu, m3 = (m2 * 3u) & 0xffu,
                           m4 = (m3 * 3u) & 0xffu;
            const uint32_t e = ((m1 * 3u) >> 8) | (((m2 * 3u) >> 8) << 8) | (((m3 * 3u) >> 8) << 16) |
                               (((m4 * 3u) >> 8) << 24);
            uint4* row = (uint4*)smem + bv * (REPS / 4);
            for (int k = tid & 3; k < REPS / 4; k += 4) row[k] = make_uint4(e, e, e, e);
        }
    }

    const uint32_t laneoff = (uint32_t)(lane & (REPS - 1)) * 4u;
    // A rows with token >= T only feed result rows the epilogue never reads: those lanes
    // skip the activation loads and keep whatever their registers hold.
    const bool a_active = ((x >> 1) & 1) < T;
    const uint8_t* xa = As + kq * QPAD + g * (2 * T * 16) + (a_active ? (x & (2 * T - 1)) : 0) * 16;
    v4i A0[kMfmaPerBlock], A1[kMfmaPerBlock];
#pragma unroll
    for (int m = 0; m < kMfmaPerBlock; m++) { A0[m] = v4i{0, 0, 0, 0}; A1[m] = v4i{0, 0, 0, 0}; }

    for (int rt0 = wt0; rt0 < wt1; rt0 += kRoundTiles) {
        const int rt1 = min(wt1, rt0 + kRoundTiles);
        for (int o = tid; o < kRoundTiles * kWaves * 4 * T; o += 1024) part[o] = 0.0f;
        __syncthreads();
        int s, s1;
        run_of(rt0, rt1, s, s1);
        if (rt0 != wt0 && s < s1) load_chunk(rt0 + s / nq, s % nq, chunk_len(s, s1));
        float acc[T];
#pragma unroll
        for (int t = 0; t < T; t++) acc[t] = 0.0f;
        while (s < s1) {
            const int tl = s / nq, c = s - tl * nq;
            const int n = chunk_len(s, s1);
            uint32_t cl[CH], chh[CH];
#pragma unroll
            for (int i = 0; i < CH; i++) { cl[i] = wl[i]; chh[i] = wh[i]; }
            const int sn = s + n;
            if (sn < s1) load_chunk(rt0 + sn / nq, sn % nq, chunk_len(sn, s1));

            auto issue = [&](int i, v4i* A, v4i* B) {
                const int vb = qbase + c + i;
                if (a_active) {
#pragma unroll
                    for (int m = 0; m < kMfmaPerBlock; m++)
                        A[m] = *(const v4i*)(xa + (vb * kMfmaPerBlock + m) * ASTRIDE);
                }
                const uint32_t w0 = cl[i], w1 = chh[i];
                B[0] = v4i{(int)lds_u32(lut_addr<LR>(w0, 0, laneoff)),
                           (int)lds_u32(lut_addr<LR>(w0, 1, laneoff)),
                           (int)lds_u32(lut_addr<LR>(w0, 2, laneoff)),
                           (int)lds_u32(lut_addr<LR>(w0, 3, laneoff))};
                B[1] = v4i{(int)digit0_pair(w0, false), (int)digit0_pair(w0, true),
                           (int)lds_u32(lut_addr<LR>(w1, 0, laneoff)),
                           (int)lds_u32(lut_addr<LR>(w1, 1, laneoff))};
                B[2] = v4i{(int)lds_u32(lut_addr<LR>(w1, 2, laneoff)),
                           (int)lds_u32(lut_addr<LR>(w1, 3, laneoff)),
                           (int)digit0_pair(w1, false), (int)digit0_pair(w1, true)};
            };
            auto finish = [&](int i, const v4i* A, const v4i* B) {
                const int vb = qbase + c + i;
                v4i D = {0, 0, 0, 0};
#pragma unroll
                for (int m = 0; m < kMfmaPerBlock; m++) D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[m], B[m], D, 0, 0, 0);
                const float d = half_bits_to_float(chh[i] >> 16);
#pragma unroll
                for (int t = 0; t < T; t++) {
                    const int v = D[2 * t] * 256 + D[2 * t + 1] - sqs[vb * T + t];
                    acc[t] += (d * sxs[vb * T + t]) * (float)v;
                }
            };
            v4i B0[kMfmaPerBlock], B1[kMfmaPerBlock];
            issue(0, A0, B0);
#pragma unroll
            for (int i = 0; i < CH; i++) {
                if (i < n) {
                    if (i + 1 < n) {
                        if (i & 1) issue(i + 1, A0, B0);
                        else issue(i + 1, A1, B1);
                    }
                    if (i & 1) finish(i, A1, B1);
                    else finish(i, A0, B0);
                }
            }
            s = sn;
            if (c + n == nq || s == s1) {
                // this wave's part of tile tl: add the quarters (lane r + 20*kq) in order
#pragma unroll
                for (int t = 0; t < T; t++) {
                    float sum = 0.0f;
#pragma unroll
                    for (int q = 0; q < 4; q++) sum += __shfl(acc[t], (lane & 3) + 20 * q);
                    if (lane < 4) part[((tl * kWaves + wave) * 4 + lane) * T + t] = sum;
                    acc[t] = 0.0f;
                }
            }
        }
        __syncthreads();
        for (int o = tid; o < (rt1 - rt0) * 4 * T; o += 1024) {
            const int tl = o / (4 * T), rr = (o / T) & 3, t = o % T;
            float sum = 0.0f;
#pragma unroll
            for (int w2 = 0; w2 < kWaves; w2++) sum += part[((tl * kWaves + w2) * 4 + rr) * T + t];
            const int row = (rt0 + tl) * 4 + rr;
            if (row < N) y[(size_t)t * N + row] = sum;
        }
        __syncthreads();
    }
}

}  // namespace

// blocks per K-quarter (the last quarter is zero-padded)
static int gemv_nq(int K) { return (K / kGroup + 3) / 4; }

XprepLayout xprep_layout(int K, int T) {
    const size_t nbv = 4 * (size_t)gemv_nq(K);
    XprepLayout L;
    L.off_sx = 0;
    L.off_sq = ((nbv * T * 4) + 255) & ~(size_t)255;
    L.off_a = (L.off_sq + nbv * T * 4 + 255) & ~(size_t)255;
    L.bytes = L.off_a + nbv * kAImageBytes * 2 * (size_t)T;
    return L;
}

hipError_t launch_gemv_prep(const void* x, int x_dtype, int x_layout, uint8_t* xprep, int K, int T,
                            hipStream_t s) {
    const XprepLayout L = xprep_layout(K, T);
    const int nq = gemv_nq(K);
    const dim3 grid(4 * nq), block(128);
    if (T == 1)
        hipLaunchKernelGGL(k_gemv_prep<1>, grid, block, 0, s, x, x_dtype, x_layout, xprep, K, nq, L.off_sq, L.off_a);
    else
        hipLaunchKernelGGL(k_gemv_prep<2>, grid, block, 0, s, x, x_dtype, x_layout, xprep, K, nq, L.off_sq, L.off_a);
    return hipGetLastError();
}

constexpr int kLdsMax = 160 * 1024;

// dynamic LDS of a GEMV launch: digit table + A image + scales/sums + round partials
static int gemv_lds_bytes(int K, int T, int LR) {
    const int nbv = 4 * gemv_nq(K);
    return lut_bytes(LR) + nbv * kAImageBytes * 2 * T + 4 * 64 + nbv * 8 * T + kRoundTiles * kWaves * 4 * T * 4;
}

static int device_cus() {
    static int n_cu = 0;
    if (!n_cu) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 256;
    }
    return n_cu;
}

template <int T, int LR>
static hipError_t launch_gemv_cfg(const uint8_t* W, const uint8_t* xprep, float* y, int K, int N, hipStream_t s,
                                  const XprepLayout& L) {
    constexpr int CH = 8;
    static bool attr_done = false;
    if (!attr_done) {
        hipError_t e = hipFuncSetAttribute((const void*)k_gemv_ptq1<T, LR, CH>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, kLdsMax);
        if (e != hipSuccess) return e;
        attr_done = true;
    }
    const int tiles = (N + 3) / 4;
    const int tpw = (tiles + device_cus() - 1) / device_cus();   // one workgroup per CU
    const int grid = (tiles + tpw - 1) / tpw;
    hipLaunchKernelGGL((k_gemv_ptq1<T, LR, CH>), dim3(grid), dim3(1024), gemv_lds_bytes(K, T, LR), s, W, xprep, y,
                       K, N, gemv_nq(K), tpw, L.off_sq, L.off_a);
    return hipGetLastError();
}

// Table size: 64 replicas (one v_perm per lookup) when the activation leaves room, else 16.
template <int T>
static hipError_t launch_gemv_t(const uint8_t* W, const uint8_t* xprep, float* y, int K, int N, hipStream_t s,
                                const XprepLayout& L) {
    if (gemv_lds_bytes(K, T, 6) <= kLdsMax) return launch_gemv_cfg<T, 6>(W, xprep, y, K, N, s, L);
    if (gemv_lds_bytes(K, T, 4) <= kLdsMax) return launch_gemv_cfg<T, 4>(W, xprep, y, K, N, s, L);
    return hipErrorInvalidValue;
}

hipError_t launch_gemv_ptq1(const uint8_t* W, const uint8_t* xprep, float* y, int K, int N, int T,
                            hipStream_t s) {
    const XprepLayout L = xprep_layout(K, T);
    return T == 1 ? launch_gemv_t<1>(W, xprep, y, K, N, s, L) : launch_gemv_t<2>(W, xprep, y, K, N, s, L);
}

int gemv_max_k(int T) {
    int K = kGroup;
    while (gemv_lds_bytes(K + kGroup, T, 4) <= kLdsMax) K += kGroup;
    return K;
}


}  // namespace kata
