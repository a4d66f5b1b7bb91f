// Input transform of every ternary matmul: (residual add +) RMSNorm / SwiGLU / GDN head
// permutation, times the sign vector, then the normalised 1024-point Walsh-Hadamard
// transform of each 1024-block (the model's rotated basis).
//
// Semantics (shaders/common.h:20-42, shaders/ops.metal:30-54,86-106,
// shaders/prefill.metal:59-97,266-285), per token row m and element i < W:
//   mode 0: v = x + y (y optional), xnew = v, inv = 1/sqrt(mean(v^2) + 1e-6),
//           u = v * inv * gs, hout = v * inv * gamma (optional)
//   mode 1: u = silu(src) * src2 * gs          mode 2: u = src[perm(i)] * gs (GDN heads)
//   mode 3: u = src * gs
//   out[block b][j] = (1/32) sum_k (-1)^popcount(j & k) u[1024 b + k]
// fp32 arithmetic; out fp32 or fp16, rows [M][W] or (M = 2) the two tokens interleaved
// per element, [W][2] (the half2 operand of the T = 2 verify GEMV), or (M <= 2) the decode
// GEMV's operand form of the fp32 values (gemv_operand.h), staged per 1024-block in LDS
// and written as whole 16-byte A rows.
//
// Design: a 256-thread workgroup per (1024-block, token) for few rows (more workgroups in
// flight; each reads the row for its sum of squares, L2-resident after the first), per
// token row for many (the row read once, held in registers).  Element k = 4 tid + r of a
// block: bits 0-1 are a thread's registers, bits 2-7 its lane (butterflies by cross-lane
// exchange), bits 8-9 its wave (one LDS transpose).  The sum of squares is reduced in a
// fixed order: a butterfly across the wave's lanes, then the 4 waves through LDS.
#include "common.h"
#include "gemv_operand.h"
#include "launch.h"

namespace kata {

namespace {

constexpr float kRmsEps = 1e-6f;   // config/kata_m6.h:21
__constant__ DenseImgOff kOperandOff = make_dense_img_off();

__device__ inline float wave_sum(float a) {
    // fixed-order butterfly over the 64 lanes
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) a += __shfl_xor(a, o);
    return a;
}

// natural-order butterflies: for bit h the pair (k, k | h) becomes (a + b, a - b)
__device__ inline void fwht1024(float (&v)[4], int tid, float* xs) {
    const int lane = tid & 63;
    float a = v[0] + v[1], b = v[0] - v[1], c = v[2] + v[3], d = v[2] - v[3];
    v[0] = a + c;
    v[1] = b + d;
    v[2] = a - c;
    v[3] = b - d;
    // the partner lane l ^ m: m = 1, 2 by DPP quad permutations, m = 4, 8 by DPP row shifts
    // (the partner is in the lane's row of 16: l + m when bit m is clear, l - m when set;
    // bound_ctrl reads 0 for sources outside the row, so the unselected shift is harmless),
    // m = 16, 32 by a cross-lane permute.  Both shifts are computed in every lane before the
    // select: a conditional expression with the DPP moves as operands evaluates one per lane,
    // which becomes a branch in which the moves read disabled source lanes (zeros).
#pragma unroll
    for (int k = 0; k < 6; k++) {
        const int m = 1 << k;
        const bool hi = lane & m;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int iv = __builtin_bit_cast(int, v[r]);
            int pv;
            if (k == 0) {
                pv = __builtin_amdgcn_mov_dpp(iv, 0xB1, 0xf, 0xf, true);   // quad_perm [1, 0, 3, 2]
            } else if (k == 1) {
                pv = __builtin_amdgcn_mov_dpp(iv, 0x4E, 0xf, 0xf, true);   // quad_perm [2, 3, 0, 1]
            } else if (k == 2) {
                const int up = __builtin_amdgcn_mov_dpp(iv, 0x104, 0xf, 0xf, true);   // row_shl:4
                const int dn = __builtin_amdgcn_mov_dpp(iv, 0x114, 0xf, 0xf, true);   // row_shr:4
                pv = hi ? dn : up;
            } else if (k == 3) {
                const int up = __builtin_amdgcn_mov_dpp(iv, 0x108, 0xf, 0xf, true);   // row_shl:8
                const int dn = __builtin_amdgcn_mov_dpp(iv, 0x118, 0xf, 0xf, true);   // row_shr:8
                pv = hi ? dn : up;
            } else {
                pv = __shfl_xor(iv, m);
            }
            const float p = __builtin_bit_cast(float, pv);
            v[r] = hi ? p - v[r] : v[r] + p;
        }
    }
    // bits 8-9: element k = 4 tid + r; thread t then owns elements t + 256 j (j = 0..3)
#pragma unroll
    for (int r = 0; r < 4; r++) xs[4 * tid + r] = v[r];
    __syncthreads();
    float e[4];
#pragma unroll
    for (int j = 0; j < 4; j++) e[j] = xs[tid + 256 * j];
    const float a2 = e[0] + e[1], b2 = e[0] - e[1], c2 = e[2] + e[3], d2 = e[2] - e[3];
    e[0] = a2 + c2;
    e[1] = b2 + d2;
    e[2] = a2 - c2;
    e[3] = b2 - d2;
#pragma unroll
    for (int j = 0; j < 4; j++) xs[tid + 256 * j] = e[j];
    __syncthreads();
#pragma unroll
    for (int r = 0; r < 4; r++) v[r] = xs[4 * tid + r] * 0.03125f;
}

__device__ inline float silu(float x) { return x / (1.0f + expf(-x)); }

// GDN output order: element i of the grouped head layout reads tiled position
// h + 128 (k + 16 rr) for i = 128 t + h, t = 3 k + rr (shaders/ops.metal:47)
__device__ inline int gdn_perm(int i) {
    const int h = i & 127, t = i >> 7, rr = t % 3, k = t / 3;
    return h + 128 * (k + 16 * rr);
}

// flags: 1 = add y, 2 = write xnew, 4 = write hout, 8 = hout fp16.
// NB blocks per workgroup: NB = 1 -> grid (W/1024, M), every block's workgroup reads the
// row for the sum of squares (few rows: more workgroups in flight); NB = W/1024 -> grid M,
// one workgroup per row, the row read once and held in registers (many rows).
// This workgroup's 8 blocks of token m (elements 4 tid + r of the 1024-block blk) in the
// decode GEMV's operand form: the 32 lanes of a block reduce its amax, the limbs go to an
// LDS copy of the 8 block images, then 128 threads store the token's 16-byte A rows.
__device__ inline void store_operand(const float (&v)[4], uint2 offw, int tid, int blk, int m, int M, int W,
                                     uint8_t* xs, uint8_t* __restrict__ xq) {
#pragma clang fp contract(off)
    const int BLK = gemv_xq_blk_bytes(M), qbytes = gemv_xq_qbytes(W, M);
    float a = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; r++) a = fmaxf(a, gemv_amax_term(v[r]));
    a = half32_max(a);
    float inv, sc;
    gemv_block_scale(a, inv, sc);
    const int bl = tid >> 5, b = 8 * blk + bl;
    __syncthreads();                              // the transform's last reads of xs
    uint8_t* img = xs + bl * BLK + 32 * m;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int off = (int)(((r < 2 ? offw.x : offw.y) >> (16 * (r & 1))) & 0xffffu);
        gemv_limbs(v[r], inv, img[off], img[off + 16]);
    }
    if ((tid & 31) == 0) ((int2*)(xq + 4 * qbytes))[b * M + m] = make_int2(__builtin_bit_cast(int, sc), 0);
    __syncthreads();
    if (tid < 128) {
        // row (mm, g, limb) of block bl: A image bytes mm (8 M 16) + g (2 M 16) + (2 m + limb) 16
        const int pb = tid >> 4, mm = (tid >> 3) & 1, g = (tid >> 1) & 3, limb = tid & 1;
        const int off = mm * (4 * 2 * M * 16) + g * (2 * M * 16) + (2 * m + limb) * 16;
        const int bb = 8 * blk + pb;
        *(uint4*)(xq + (bb & 3) * qbytes + (bb >> 2) * BLK + off) = *(const uint4*)(xs + pb * BLK + off);
    }
}

// The same for M = 3..8 tokens in the wide GEMV's operand form: block b's image at 2048 b,
// A row 2 m + limb of lane group g of MFMA mm at 1024 mm + 256 g + 16 (2 m + limb), the
// scales of token pair p at 2048 nb + 32 b + 8 p.  The workgroups of token 0 also clear
// the rows and scales of tokens M..7 of their blocks.
__device__ inline void store_operand_wide(const float (&v)[4], uint2 offw, int tid, int blk, int m, int M, int W,
                                          uint8_t* xs, uint8_t* __restrict__ xq) {
#pragma clang fp contract(off)
    constexpr int BLK = kWideImgBlk;
    const int nb = W >> 7;
    float a = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; r++) a = fmaxf(a, gemv_amax_term(v[r]));
    a = half32_max(a);
    float inv, sc;
    gemv_block_scale(a, inv, sc);
    const int bl = tid >> 5, b = 8 * blk + bl;
    __syncthreads();                              // the transform's last reads of xs
    // staging: per block the token's 16 A rows [mm 2][g 4][limb 2][16 B] (256 B)
    uint8_t* img = xs + bl * 256;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int o = (int)(((r < 2 ? offw.x : offw.y) >> (16 * (r & 1))) & 0xffffu);   // [mm][g][row 16][16 B]
        const int so = (o >> 10) * 128 + ((o >> 8) & 3) * 32 + (o & 15);
        gemv_limbs(v[r], inv, img[so], img[so + 16]);
    }
    float* scl = (float*)(xq + (size_t)nb * BLK);
    if ((tid & 31) == 0) scl[b * 8 + m] = sc;
    __syncthreads();
    if (tid < 128) {
        const int pb = tid >> 4, mm = (tid >> 3) & 1, g = (tid >> 1) & 3, limb = tid & 1;
        const int bb = 8 * blk + pb;
        *(uint4*)(xq + (size_t)bb * BLK + mm * 1024 + g * 256 + (2 * m + limb) * 16) =
            *(const uint4*)(xs + pb * 256 + mm * 128 + g * 32 + limb * 16);
    }
    if (m == 0) {
        // rows 2 M .. 15 of the 8 blocks' 8 (mm, g) groups, and the scales of tokens M..7
        const int nr = 16 - 2 * M;
        for (int i = tid; i < 8 * 8 * nr; i += 256) {
            const int pb = i / (8 * nr), rem = i % (8 * nr), grp = rem / nr, row = 2 * M + rem % nr;
            *(uint4*)(xq + (size_t)(8 * blk + pb) * BLK + grp * 256 + row * 16) = make_uint4(0, 0, 0, 0);
        }
        if (tid < 8 * (8 - M)) scl[(8 * blk + tid / (8 - M)) * 8 + M + tid % (8 - M)] = 0.0f;
    }
}

template <int NB>
__global__ __launch_bounds__(256) void k_norm_fwht(const float* __restrict__ src, const float* __restrict__ src2,
                                                   const float* __restrict__ gs, void* __restrict__ out, int out_dtype,
                                                   int out_layout, float* __restrict__ xnew,
                                                   const float* __restrict__ gamma, void* __restrict__ hout,
                                                   int flags, int W, int mode) {
    __shared__ float xs[1024];
    __shared__ float part[4];
    const int tid = threadIdx.x;
    const int m = NB == 1 ? blockIdx.y : blockIdx.x, blk0 = NB == 1 ? blockIdx.x : 0;
    const size_t ro = (size_t)m * W;
    // the operand form's image offsets of this thread's 4 elements, loaded first (their
    // latency then overlaps the row loads)
    uint2 offw = make_uint2(0, 0);
    if (out_dtype == 2) {
        const int M = NB == 1 ? gridDim.y : gridDim.x;
        offw = *(const uint2*)&kOperandOff.v[M <= 2 ? M - 1 : 2][(4 * tid) & 127];
    }
    // v = x (+ y) of this thread's elements 1024 (blk0 + b) + 4 tid + r, b < NB
    float s[NB][4];
    if (mode == 0) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int base = (blk0 + b) * 1024 + 4 * tid;
            const float4 a = *(const float4*)(src + ro + base);
            float4 c = make_float4(0.f, 0.f, 0.f, 0.f);
            if (flags & 1) c = *(const float4*)(src2 + ro + base);
            s[b][0] = a.x + c.x;
            s[b][1] = a.y + c.y;
            s[b][2] = a.z + c.z;
            s[b][3] = a.w + c.w;
        }
    }
    float inv = 1.0f;
    if (mode == 0) {
        float ss = 0.0f;
        if (NB == 1) {
            for (int i = 4 * tid; i < W; i += 1024) {
                const float4 a = *(const float4*)(src + ro + i);
                float4 c = make_float4(0.f, 0.f, 0.f, 0.f);
                if (flags & 1) c = *(const float4*)(src2 + ro + i);
                const float v0 = a.x + c.x, v1 = a.y + c.y, v2 = a.z + c.z, v3 = a.w + c.w;
                ss += (v0 * v0 + v1 * v1) + (v2 * v2 + v3 * v3);
            }
        } else {
#pragma unroll
            for (int b = 0; b < NB; b++) ss += (s[b][0] * s[b][0] + s[b][1] * s[b][1]) + (s[b][2] * s[b][2] + s[b][3] * s[b][3]);
        }
        ss = wave_sum(ss);
        if ((tid & 63) == 0) part[tid >> 6] = ss;
        __syncthreads();
        inv = 1.0f / sqrtf((part[0] + part[1] + part[2] + part[3]) / (float)W + kRmsEps);
    }
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int base = (blk0 + b) * 1024 + 4 * tid;
        float v[4];
        const float4 g = *(const float4*)(gs + base);
        const float gv[4] = {g.x, g.y, g.z, g.w};
        if (mode == 0) {
            if (flags & 2) *(float4*)(xnew + ro + base) = make_float4(s[b][0], s[b][1], s[b][2], s[b][3]);
            if (flags & 4) {
                const float4 gm = *(const float4*)(gamma + base);
                const float h[4] = {s[b][0] * inv * gm.x, s[b][1] * inv * gm.y, s[b][2] * inv * gm.z, s[b][3] * inv * gm.w};
                if (flags & 8) {
                    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                    *(h4*)((_Float16*)hout + ro + base) = h4{(_Float16)h[0], (_Float16)h[1], (_Float16)h[2], (_Float16)h[3]};
                } else {
                    *(float4*)((float*)hout + ro + base) = make_float4(h[0], h[1], h[2], h[3]);
                }
            }
#pragma unroll
            for (int r = 0; r < 4; r++) v[r] = s[b][r] * inv * gv[r];
        } else if (mode == 1) {
            const float4 a = *(const float4*)(src + ro + base);
            const float4 c = *(const float4*)(src2 + ro + base);
            const float av[4] = {a.x, a.y, a.z, a.w}, cv[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
            for (int r = 0; r < 4; r++) v[r] = silu(av[r]) * cv[r] * gv[r];
        } else if (mode == 2) {
#pragma unroll
            for (int r = 0; r < 4; r++) v[r] = src[ro + gdn_perm(base + r)] * gv[r];
        } else {
            const float4 a = *(const float4*)(src + ro + base);
            const float av[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int r = 0; r < 4; r++) v[r] = av[r] * gv[r];
        }
        fwht1024(v, tid, xs);
        if (out_dtype == 2) {
            const int M = NB == 1 ? gridDim.y : gridDim.x;
            if (M <= 2)
                store_operand(v, offw, tid, blk0 + b, m, M, W, (uint8_t*)xs, (uint8_t*)out);
            else
                store_operand_wide(v, offw, tid, blk0 + b, m, M, W, (uint8_t*)xs, (uint8_t*)out);
        } else if (out_dtype == 0) {
            *(float4*)((float*)out + ro + base) = make_float4(v[0], v[1], v[2], v[3]);
        } else if (out_layout == 0) {
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            *(h4*)((_Float16*)out + ro + base) = h4{(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
        } else {
            _Float16* o = (_Float16*)out;        // [W][2]: token m at 2 i + m
#pragma unroll
            for (int r = 0; r < 4; r++) o[2 * (base + r) + m] = (_Float16)v[r];
        }
        if (NB > 1) __syncthreads();             // xs is reused by the next block's transform
    }
}

}  // namespace

hipError_t launch_norm_fwht(const float* src, const float* src2, const float* gs, void* out, int out_dtype,
                            int out_layout, float* xnew, const float* gamma, void* hout, int flags, int W, int M,
                            int mode, hipStream_t s) {
    // whole rows per workgroup once there are enough rows to fill the CUs (hidden width 5120);
    // the operand form (out_dtype 2) takes M <= 8
    if (W == 5120 && M >= 64 && out_dtype != 2)
        hipLaunchKernelGGL(k_norm_fwht<5>, dim3(M), dim3(256), 0, s, src, src2, gs, out, out_dtype, out_layout, xnew,
                           gamma, hout, flags, W, mode);
    else
        hipLaunchKernelGGL(k_norm_fwht<1>, dim3(W / 1024, M), dim3(256), 0, s, src, src2, gs, out, out_dtype,
                           out_layout, xnew, gamma, hout, flags, W, mode);
    return hipGetLastError();
}

}  // namespace kata
