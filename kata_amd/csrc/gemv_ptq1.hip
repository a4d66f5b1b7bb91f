// PTQ1_0 decode GEMV for T = 1 and T = 2 tokens on the gfx950 int8 matrix cores.
//
// Semantics: y[t][n] = sum_b d[n,b] * sum_e trit[n,b,e] * x[t][128b+e]
// (shaders/gemv.metal:5-20; fast forms shaders/gemv_fast.metal:9-50, shaders/mtp.metal:164-205).
//
// Design (MI355X-first, not the reference's simdgroup float decode):
//  * The packed weight bytes are never expanded in memory.  Per 128-weight block four lanes
//    each hold 8 bytes of it (lane group g = lane/16 takes block bytes 20..27, 0..7, 8..15
//    or 16..19, rotated by the block's position) and turn them into base-3 digits {0,1,2}:
//    digits 1..4 of a byte come from one 4-byte LDS table entry, digit 0 = (3b) >> 8 from
//    16-bit-lane multiplies.  The digits are the B operand (B[k][column]) of three
//    v_mfma_i32_16x16x64_i8 per block.
//  * The activation is the A operand (A[i][k]) in a prepared integer form: per 128-block
//    a scale s = amax/32639 and q = rint(x/s) split into two int8 limbs (q = 256*hi + lo);
//    A rows are (block, token, limb), so T = 2 costs no extra matrix-core work.  The matrix
//    core sums digit*limb exactly in int32; the epilogue forms sum(trit*q) = 256*D_hi +
//    D_lo - sum(q) per block and token and accumulates y += d * s * that in fp32.  The only
//    approximation is the 16-bit block-fixed-point activation (|x - s*q| <= amax/65278),
//    far inside the 1e-3 relative-L2 contract.
//  * Work unit = a 4-row tile.  The 16 B columns of the MFMA are (row r, block 4c + kq)
//    and the 16 A rows are (block 4c + kq, token, limb), so one wave step decodes 4
//    consecutive blocks of 4 rows (four 112-byte runs of the matrix) and the products of
//    mismatched blocks are never read.  One 1024-thread workgroup per CU splits its tile
//    range evenly over its 16 waves (see the kernel comment); no atomics, deterministic.
#include "common.h"
#include "launch.h"

#include <stdlib.h>

namespace kata {

namespace {

constexpr float kQMax = 32639.0f;   // |q| <= 32639 keeps hi = (q+128)>>8 inside int8
constexpr int kMfmaPerBlock = 3;
constexpr int kAImageBytes = kMfmaPerBlock * 4 * 16;   // per block and A row (token, limb)


// A block is read as four 8-byte segments starting at bytes 20, 0, 8, 16 (segment 3 uses
// only bytes 16..19; bytes 20..23 belong to segment 0).  Segment 0 carries the scale.
// Lane group g working on block 4c + kq reads segment (g - kq) & 3, so the lanes whose
// result rows hold that block (g == kq) are the ones holding the scale.
__host__ __device__ inline int gemv_seg_byte0(int seg) { return seg == 0 ? 20 : seg == 1 ? 0 : seg == 2 ? 8 : 16; }

// Byte p and digit n of the A/B operand slot (segment seg, MFMA m, dword dw, byte kb),
// or p = -1 for a slot that multiplies a zero activation.  With w0/w1 the lane's two
// weight dwords (bytes b0..b7) the B dwords are
//   m=0: L(b0) L(b1) L(b2) L(b3)     m=1: Z(w0) L(b4) L(b5) L(b6)     m=2: L(b7) Z(w1) 0 0
// where L(b) = digits 1..4 of byte b and Z(w) = digit 0 of the dword's bytes 0..3.
__host__ __device__ inline void gemv_slot(int seg, int m, int dw, int kb, int& p, int& n) {
    const int base = gemv_seg_byte0(seg);
    const int kind = m * 4 + dw;   // 0..11
    // L slots: byte offset within the lane's 8 bytes; Z slots: -(1 + word); -9: unused
    const int desc[12] = {0, 1, 2, 3, -1, 4, 5, 6, 7, -2, -9, -9};
    const int d = desc[kind];
    if (d == -9) {
        p = -1;
        return;
    }
    if (d >= 0) {
        p = base + d;
        n = kb + 1;
    } else {
        p = base + (-d - 1) * 4 + kb;
        n = 0;
    }
    if (seg == 3 && p >= 20) p = -1;   // bytes 20..23 belong to segment 0
}

// One workgroup per virtual block vb (0 <= vb < 4*nq; blocks nb.. are zero padding so
// every tile has nq steps of 4 blocks).  Writes the pair (scale s as float, sum(q) as int)
// per token at scales[vb][t] and the A image [m 3][g 4][i 2T][16 B], i = 2*t + limb, laid
// out for lane group g reading segment (g - (vb & 3)) & 3.
template <int T>
__global__ __launch_bounds__(128) void k_gemv_prep(const void* __restrict__ x, int x_dtype, int x_layout,
                                                   uint8_t* __restrict__ xprep, int K, int nq, size_t off_a) {
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
        if (e == 0) ((float*)xprep)[(b * T + t) * 2] = amax / kQMax;
    }
    __syncthreads();
    if (e < T) ((int*)xprep)[(b * T + e) * 2 + 1] = red_i[0][e] + red_i[1][e];
    const int kq = b & 3;
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

// digit 0 = (3b) >> 8 of the four bytes of w, byte k of the result for byte k of w.  Bytes
// (0,2) and (1,3) are spread into 16-bit lanes and tripled (3b < 768 cannot carry into the
// next lane); the digit is then byte 1 of its lane.
__device__ inline uint32_t digit0_word(uint32_t w) {
    const uint32_t e = w & 0x00ff00ffu, o = __builtin_amdgcn_perm(0u, w, 0x0c030c01u);
    const uint32_t e3 = e + (e << 1), o3 = o + (o << 1);
    return __builtin_amdgcn_perm(o3, e3, 0x07030501u);
}

typedef __attribute__((address_space(3))) const uint8_t lds_u8;
// 32-bit load at byte offset addr of an LDS array; for the digit table, the kernel's only
// static LDS, the base is address 0 and folds away.
__device__ inline uint32_t lds_u32(lds_u8* base, uint32_t addr) {
    return *(__attribute__((address_space(3))) const uint32_t*)(base + addr);
}

// Work split: one 1024-thread workgroup (16 waves) per CU owns the contiguous tile range
// [wt0, wt0 + tpw).  Its (tile, block step) pairs, numbered s = (tile - wt0) * nq + c, are
// cut into 16 equal contiguous runs, one per wave.  Lane x + 16*g: B column x = (row
// r = x & 3, block 4c + kq with kq = x >> 2), A row x = (block 4c + (x >> 2), token
// (x >> 1) & 1, limb x & 1); result rows 4g..4g+3 belong to block 4c + g, so lane
// 20*q + r holds row r's sum over blocks 4c + q ("quarter" q of the tile's blocks).
//
// Timeline: the digit table is written and the activation staging (global -> LDS DMA) is
// issued by every wave before any wave issues weight loads (vector-memory loads complete
// in order per CU, so staging queued behind the ring would arrive only after it); then
// every wave keeps D weight steps in flight in a register ring (step j in slot j % D) and
// decodes step j as soon as its own load has landed.
// Each step's operands are issued one step ahead of its MFMAs.  When a tile's last step
// of a run is done the 16 diagonal lanes store their sums to the wave's LDS slot for that
// tile; after one barrier the workgroup adds the slots of each tile over waves and quarters
// in fixed order (deterministic).  Dynamic LDS: A image (384*T B per virtual block, 64 B
// between quarters), (scale, sum) pairs, per-wave tile sums [16][slots][T][16].
constexpr int kWaves = 16;
// LDS bytes of the A image (4 quarters, 64 B apart) and of the (scale, sum) pairs, rounded
// up to whole staging chunks
__host__ __device__ inline int gemv_a_lds_bytes(int qbytes) { return (4 * (qbytes + 64) + 1023) & ~1023; }
__host__ __device__ inline int gemv_s_lds_bytes(int nbv, int T) { return (8 * nbv * T + 1023) & ~1023; }
// static LDS of the GEMV kernel: digit table + run_tiles
__host__ __device__ constexpr int gemv_static_lds_bytes(int LR) { return lut_bytes(LR) + kWaves * 8; }

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int T, int LR, int D>
__global__ __launch_bounds__(1024) void k_gemv_ptq1(const uint8_t* __restrict__ W, const uint8_t* __restrict__ xprep,
                                                    float* __restrict__ y, int K, int N, int nq, int tpw, int slots,
                                                    size_t off_a) {
    static_assert(D % 2 == 0 && D >= 4, "operand double buffers alternate by step parity");
    constexpr int ASTRIDE = 4 * 2 * T * 16;      // A image bytes per (virtual block, MFMA)
    constexpr int REPS = 1 << LR;
    constexpr int QPAD = 64;
    // digit table: the kernel's only static LDS besides run_tiles, at LDS address 0
    __shared__ uint4 lut[lut_bytes(LR) / 16];
    __shared__ int2 run_tiles[kWaves];          // first and last tile (local) of each wave's run
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int x = lane & 15, g = lane >> 4;
    const int r = x & 3, kq = x >> 2;
    const int nb = K >> 7, nbv = 4 * nq;
    const int tiles = (N + 3) >> 2;
    const int wt0 = blockIdx.x * tpw, wt1 = min(tiles, wt0 + tpw);
    const int S = (wt1 - wt0) * nq;
    const int s0 = (wave * S) / kWaves, s1 = ((wave + 1) * S) / kWaves;
    const int n = s1 - s0;                       // this wave's run length (wave-uniform)
    const int c0 = s0 % nq;
    if (lane == 0) run_tiles[wave] = n > 0 ? make_int2(s0 / nq, (s1 - 1) / nq) : make_int2(1 << 30, -1);

    // Digit table.  Consecutive threads store consecutive 16-byte words (no bank
    // conflicts); word o holds 4 replicas of entry o / (REPS / 4).
#pragma unroll
    for (int i = 0; i < lut_bytes(LR) / 16 / 1024; i++) {
        const int o = tid + i * 1024;
        const uint32_t bv = (uint32_t)o / (REPS / 4);
        const uint32_t m1 = (bv * 3u) & 0xffu, m2 = (m1 * 3u) & 0xffu, m3 = (m2 * 3u) & 0xffu,
                       m4 = (m3 * 3u) & 0xffu;
        const uint32_t e = ((m1 * 3u) >> 8) | (((m2 * 3u) >> 8) << 8) | (((m3 * 3u) >> 8) << 16) |
                           (((m4 * 3u) >> 8) << 24);
        lut[o] = make_uint4(e, e, e, e);
    }

    // Weight loads: raw buffer loads with 32-bit offsets; bytes past the matrix read as 0
    // (rows >= N).  Padding blocks (past K) reread the row's last block; their activation,
    // scale and sum are zero.  Every ring slot is reloaded once per step, also past the
    // run's end, so all paths issue the same loads and the compiler's wait counts stay
    // exact.
    const uint32_t row_bytes = (uint32_t)nb * kBlockBytes;
    const __amdgpu_buffer_rsrc_t wrsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)W, 0, (int)((uint32_t)N * row_bytes), 0x00020000);
    // loads past the run's end go through an empty descriptor: zeros, no memory access
    const __amdgpu_buffer_rsrc_t wnone = __builtin_amdgcn_make_buffer_rsrc((void*)W, 0, 0, 0x00020000);
    const uint32_t qoff = (uint32_t)kq * kBlockBytes + (uint32_t)gemv_seg_byte0((g - kq) & 3);
    const uint32_t qlim = (uint32_t)(nb - 1) * kBlockBytes + (uint32_t)gemv_seg_byte0((g - kq) & 3);
    uint32_t rowoff = (uint32_t)((wt0 + s0 / nq) * 4 + r) * row_bytes;
    int lc = c0, ld_left = n;                    // load cursor (wave-uniform)
    uint32_t lcb = (uint32_t)c0 * 4 * kBlockBytes;   // lc * 4 blocks
    uint32_t wl[D], wh[D];
    auto load_next = [&](int slot) {
        const uint32_t off = rowoff + min(qoff + lcb, qlim);
        const u32x2 w =
            __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(ld_left > 0 ? wrsrc : wnone, (int)off, 0, 0));
        wl[slot] = w.x;
        wh[slot] = w.y;
        if (ld_left > 1) {
            lcb += 4 * kBlockBytes;
            if (++lc == nq) {
                lc = 0;
                lcb = 0;
                rowoff += 4 * row_bytes;
            }
        }
        --ld_left;
    };
    // Activation staging by DMA; each wave fills whole 1 KB LDS chunks, padding slots load
    // a duplicate in-range element.
    const int qbytes = nq * kAImageBytes * 2 * T;
    const int qvec = qbytes / 16;                // 16-byte vectors per quarter in xprep
    const int a_bytes = gemv_a_lds_bytes(qbytes);
    const int s_bytes = gemv_s_lds_bytes(nbv, T);
    uint8_t* As = smem;
    uint8_t* Ss = smem + a_bytes;                // (scale, sum) pairs [vb][t]
    float* part = (float*)(Ss + s_bytes);        // [kWaves][slots][T][16]
    {
        typedef __attribute__((address_space(3))) void lds_void;
        const uint4* a_src = (const uint4*)(xprep + off_a);
        for (int ch = wave; ch < a_bytes / 1024; ch += kWaves) {
            const int o = ch * 64 + lane;        // LDS vector index
            // LDS quarter q holds blocks 4c + q, c = 0..nq-1, in order
            const int q = o / (qvec + QPAD / 16), w = min(o - q * (qvec + QPAD / 16), qvec - 1);
            const int bv = kAImageBytes * 2 * T / 16;   // vectors per block
            const int src = (4 * (w / bv) + min(q, 3)) * bv + w % bv;
            __builtin_amdgcn_global_load_lds(a_src + src, (lds_void*)(As + ch * 1024), 16, 0, 0);
        }
        const uint4* s_src = (const uint4*)xprep;
        const int svec = nbv * T * 8 / 16;      // (scale, sum) pairs: 16-byte vectors (T=1: 2 blocks)
        for (int ch = wave; ch < s_bytes / 1024; ch += kWaves) {
            const int o = min(ch * 64 + lane, svec - 1);
            __builtin_amdgcn_global_load_lds(s_src + o, (lds_void*)(Ss + ch * 1024), 16, 0, 0);
        }
    }
    // All staging DMA of the workgroup is issued before any wave issues its ring, so the
    // staging is at the head of the CU's in-order vector-memory queue (no wait here).
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int u = 0; u < D; u++) load_next(u);
    // The staging DMA is older than the D ring loads, so "at most D vector-memory loads
    // pending" means it has landed; lgkmcnt(0) covers the table stores.  A bare s_barrier
    // (a release fence would also wait for the ring) then publishes both.
    __builtin_amdgcn_s_waitcnt((D & 15) | ((D >> 4) << 14) | (7 << 4) | (0 << 8));
    __builtin_amdgcn_s_barrier();

    const uint32_t laneoff = (uint32_t)(lane & (REPS - 1)) * 4u;
    lds_u8* lb = (lds_u8*)lut;
    // A rows with token >= T only feed result rows the epilogue never reads: those lanes
    // skip the activation loads and keep whatever their registers hold.
    const bool a_active = ((x >> 1) & 1) < T;
    const uint8_t* xa = As + kq * (qbytes + QPAD) + g * (2 * T * 16) + (a_active ? (x & (2 * T - 1)) : 0) * 16;
    const uint8_t* xs = Ss + kq * (8 * T);
    const bool sum_lane = g == kq;               // lane 20*q + r: the diagonal quarter
    float* my_part = part + (size_t)wave * slots * T * 16 + g * 4 + r;
    v4i A0[kMfmaPerBlock], A1[kMfmaPerBlock], B0[kMfmaPerBlock], B1[kMfmaPerBlock];
    uint4 SQ0, SQ1;
#pragma unroll
    for (int m = 0; m < kMfmaPerBlock; m++) { A0[m] = v4i{0, 0, 0, 0}; A1[m] = v4i{0, 0, 0, 0}; }

    // operands of step c (block qbase + c of this lane's quarter)
    auto issue = [&](int c, uint32_t w0, uint32_t w1, v4i* A, v4i* B, uint4& SQ) {
        const uint8_t* pa = xa + c * (kMfmaPerBlock * ASTRIDE);
        if (a_active) {
#pragma unroll
            for (int m = 0; m < kMfmaPerBlock; m++) A[m] = *(const v4i*)(pa + m * ASTRIDE);
        }
        if (T == 1) {
            const uint2 v = *(const uint2*)(xs + c * 32);
            SQ.x = v.x;
            SQ.y = v.y;
        } else {
            SQ = *(const uint4*)(xs + c * 64);
        }
        B[0] = v4i{(int)lds_u32(lb, lut_addr<LR>(w0, 0, laneoff)), (int)lds_u32(lb, lut_addr<LR>(w0, 1, laneoff)),
                   (int)lds_u32(lb, lut_addr<LR>(w0, 2, laneoff)), (int)lds_u32(lb, lut_addr<LR>(w0, 3, laneoff))};
        B[1] = v4i{(int)digit0_word(w0), (int)lds_u32(lb, lut_addr<LR>(w1, 0, laneoff)),
                   (int)lds_u32(lb, lut_addr<LR>(w1, 1, laneoff)), (int)lds_u32(lb, lut_addr<LR>(w1, 2, laneoff))};
        B[2] = v4i{(int)lds_u32(lb, lut_addr<LR>(w1, 3, laneoff)), (int)digit0_word(w1), 0, 0};
    };
    float acc[T];
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] = 0.0f;
    auto finish = [&](uint32_t dbits, const v4i* A, const v4i* B, const uint4& SQ) {
        v4i Dm = {0, 0, 0, 0};
#pragma unroll
        for (int m = 0; m < kMfmaPerBlock; m++) Dm = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[m], B[m], Dm, 0, 0, 0);
        const float d = half_bits_to_float(dbits >> 16);
        const uint32_t sq[4] = {SQ.x, SQ.y, SQ.z, SQ.w};
#pragma unroll
        for (int t = 0; t < T; t++) {
            const int v = Dm[2 * t] * 256 + Dm[2 * t + 1] - (int)sq[2 * t + 1];
            acc[t] += (d * __builtin_bit_cast(float, sq[2 * t])) * (float)v;
        }
    };

    // compute cursor: step cc of the current tile, `left` steps of it remain in this run's
    // view of the tile, cs = tile slot (0 = the run's first tile)
    int cc = c0, left = nq - c0, cs = 0;
    auto flush_if_done = [&]() {
        if (--left == 0) {
            if (sum_lane) {
#pragma unroll
                for (int t = 0; t < T; t++) my_part[(cs * T + t) * 16] = acc[t];
            }
#pragma unroll
            for (int t = 0; t < T; t++) acc[t] = 0.0f;
            ++cs;
            left = nq;
            cc = 0;
        } else {
            ++cc;
        }
    };
    if (n > 0) issue(cc, wl[0], wh[0], A0, B0, SQ0);
    // One loop over passes of the ring: every slot is reloaded after use (also past the
    // run's end), so the loads do not depend on the branches and their waits stay exact.
    for (int j = 0; j < n; j += D) {
#pragma unroll
        for (int u = 0; u < D; u++) {
            if (j + u < n) {
                const int cn = left == 1 ? 0 : cc + 1;
                if (j + u + 1 < n) {
                    if (u & 1) issue(cn, wl[(u + 1) % D], wh[(u + 1) % D], A0, B0, SQ0);
                    else issue(cn, wl[(u + 1) % D], wh[(u + 1) % D], A1, B1, SQ1);
                }
                if (u & 1) finish(wh[u], A1, B1, SQ1);
                else finish(wh[u], A0, B0, SQ0);
                flush_if_done();
            }
            load_next(u);
        }
    }
    if (left != nq) {                            // the run ended inside a tile: store it
        left = 1;
        flush_if_done();
    }
    __syncthreads();

    // tile sums: every wave whose run touches the tile, in wave order, quarters in order
    for (int o = tid; o < (wt1 - wt0) * 4 * T; o += 1024) {
        const int tl = o / (4 * T), rr = (o / T) & 3, t = o % T;
        float sum = 0.0f;
#pragma unroll
        for (int w2 = 0; w2 < kWaves; w2++) {
            const int f = run_tiles[w2].x, l = run_tiles[w2].y;
            if (tl >= f && tl <= l) {
                const float* p = part + ((size_t)(w2 * slots + tl - f) * T + t) * 16 + rr;
#pragma unroll
                for (int q = 0; q < 4; q++) sum += p[4 * q];
            }
        }
        const int row = (wt0 + tl) * 4 + rr;
        if (row < N) y[(size_t)t * N + row] = sum;
    }
}

}  // namespace

// steps (of 4 blocks) per tile; blocks past K are zero padding
static int gemv_nq(int K) { return (K / kGroup + 3) / 4; }

XprepLayout xprep_layout(int K, int T) {
    const size_t nbv = 4 * (size_t)gemv_nq(K);
    XprepLayout L;
    L.off_s = 0;
    L.off_a = ((nbv * T * 8) + 255) & ~(size_t)255;
    L.bytes = L.off_a + nbv * kAImageBytes * 2 * (size_t)T;
    return L;
}

hipError_t launch_gemv_prep(const void* x, int x_dtype, int x_layout, uint8_t* xprep, int K, int T,
                            hipStream_t s) {
    const XprepLayout L = xprep_layout(K, T);
    const int nq = gemv_nq(K);
    const dim3 grid(4 * nq), block(128);
    if (T == 1)
        hipLaunchKernelGGL(k_gemv_prep<1>, grid, block, 0, s, x, x_dtype, x_layout, xprep, K, nq, L.off_a);
    else
        hipLaunchKernelGGL(k_gemv_prep<2>, grid, block, 0, s, x, x_dtype, x_layout, xprep, K, nq, L.off_a);
    return hipGetLastError();
}

constexpr int kLdsMax = 160 * 1024;

constexpr int kRing = 12;    // weight steps in flight per wave

// tile slots a wave's run can touch when a workgroup owns tpw tiles
static int gemv_slots(int nq, int tpw) {
    const int run = (tpw * nq + kWaves - 1) / kWaves;
    return (run + nq - 1) / nq + 1;
}

// LDS of a GEMV launch (the static digit table, then the dynamic part): digit table + A image + scales/sums + per-wave tile sums
static int gemv_lds_bytes(int K, int T, int LR, int slots) {
    const int nbv = 4 * gemv_nq(K);
    return gemv_static_lds_bytes(LR) + gemv_a_lds_bytes(gemv_nq(K) * kAImageBytes * 2 * T) + gemv_s_lds_bytes(nbv, T) +
           kWaves * slots * T * 16 * 4;
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
static hipError_t launch_gemv_cfg(const uint8_t* W, const uint8_t* xprep, float* y, int K, int N, int tpw,
                                  hipStream_t s, const XprepLayout& L) {
    static bool attr_done = false;
    if (!attr_done) {
        hipError_t e = hipFuncSetAttribute((const void*)k_gemv_ptq1<T, LR, kRing>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           kLdsMax - gemv_static_lds_bytes(LR));
        if (e != hipSuccess) return e;
        attr_done = true;
    }
    const int tiles = (N + 3) / 4, nq = gemv_nq(K);
    const int grid = (tiles + tpw - 1) / tpw;
    const int slots = gemv_slots(nq, tpw);
    hipLaunchKernelGGL((k_gemv_ptq1<T, LR, kRing>), dim3(grid), dim3(1024), gemv_lds_bytes(K, T, LR, slots) - gemv_static_lds_bytes(LR), s, W,
                       xprep, y, K, N, nq, tpw, slots, L.off_a);
    return hipGetLastError();
}

// One workgroup per CU when its tile sums fit in LDS beside the table and activation, else
// smaller tile ranges (more workgroups).  Table: 64 replicas (one v_perm per lookup) when
// there is room, else 16.
template <int T>
static hipError_t launch_gemv_t(const uint8_t* W, const uint8_t* xprep, float* y, int K, int N, hipStream_t s,
                                const XprepLayout& L) {
    const int tiles = (N + 3) / 4, nq = gemv_nq(K), cus = device_cus();
    for (int wgs = cus;; wgs *= 2) {
        const int tpw = (tiles + wgs - 1) / wgs;
        const int slots = gemv_slots(nq, tpw);
        if (gemv_lds_bytes(K, T, 6, slots) <= kLdsMax) return launch_gemv_cfg<T, 6>(W, xprep, y, K, N, tpw, s, L);
        if (gemv_lds_bytes(K, T, 4, slots) <= kLdsMax) return launch_gemv_cfg<T, 4>(W, xprep, y, K, N, tpw, s, L);
        if (tpw == 1) return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_ptq1(const uint8_t* W, const uint8_t* xprep, float* y, int K, int N, int T,
                            hipStream_t s) {
    const XprepLayout L = xprep_layout(K, T);
    return T == 1 ? launch_gemv_t<1>(W, xprep, y, K, N, s, L) : launch_gemv_t<2>(W, xprep, y, K, N, s, L);
}

int gemv_max_k(int T) {
    int K = kGroup;
    while (gemv_lds_bytes(K + kGroup, T, 4, gemv_slots(gemv_nq(K + kGroup), 1)) <= kLdsMax) K += kGroup;
    return K;
}


}  // namespace kata
