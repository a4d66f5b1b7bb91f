/*
 * kata_oracle.c — CPU restatement of the reference's ternary-matmul arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP library in
 * kata_amd/.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only as the checker / the timed CPU baseline — never as the product path.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the reference repository root).  Pinning status of each function
 * (what independent check fixes it) is listed next to it; none is "parity unpinned".
 *
 * Formats:
 *   PTQ1_0 block (28 B): qs[24], qh[2], fp16 d at bytes 26..27
 *       (config/kata_m6.h:44-45, shaders/common.h:18).
 *   Q8_0 block (34 B): fp16 d at bytes 0..1, int8 qs[32] (shaders/mtp.metal:9-16,
 *       src/gguf.cpp:25-38).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_GROUP 128
#define ORC_BLOCK_BYTES 28
#define ORC_Q8_GROUP 32
#define ORC_Q8_BLOCK_BYTES 34

/* ---------------------------------------------------------------- fp16 helpers --------
 * IEEE binary16 <-> binary32.  half->float is exact; float->half rounds to nearest even
 * (the ggml GGML_FP32_TO_FP16 contract used by quantize_row_ptq1_0_ref:17).
 * Pinned by tests against numpy.float16 over every 16-bit pattern and random floats.   */
float orc_half_to_float(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff, u;
    if (e == 0) {
        if (m == 0) { u = s; }
        else {                       /* subnormal: normalise */
            int sh = 0;
            while (!(m & 0x400)) { m <<= 1; sh++; }
            m &= 0x3ff;
            u = s | ((uint32_t)(127 - 15 - sh + 1) << 23) | (m << 13);
        }
    } else if (e == 31) {
        u = s | 0x7f800000u | (m << 13);
    } else {
        u = s | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f; memcpy(&f, &u, 4); return f;
}

uint16_t orc_float_to_half(float f) {
    uint32_t u; memcpy(&u, &f, 4);
    uint32_t s = (u >> 16) & 0x8000u;
    uint32_t a = u & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(s | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0));
    if (a >= 0x477ff000u) return (uint16_t)(s | 0x7c00u);          /* rounds to inf */
    if (a < 0x38800000u) {                                           /* subnormal or zero */
        if (a < 0x33000000u) return (uint16_t)s;                     /* < half of min subnormal */
        uint32_t e = a >> 23, m = (a & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e;                                    /* 14..24 */
        uint32_t q = m >> (shift), rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(s | q);
    }
    uint32_t e = (a >> 23) - 127 + 15, m = a & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13), rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
    return (uint16_t)(s | q);
}

/* ---------------------------------------------------------------- PTQ1_0 decode -------
 * Digit n (0 = most significant) of a packed byte: ((b*3^n mod 256) * 3) >> 8.
 * docs/reference/prism_ptq1_0_quant_dequant.c:60,69-71 ; shaders/common.h:10.
 * Pinned: exhaustive 256x5 table vs floor(b*3^(n+1)/256) mod 3 (tests/golden, closed form). */
static const uint32_t kPow3[6] = {1, 3, 9, 27, 81, 243};

int orc_ptq1_digit(uint32_t b, uint32_t n) {
    uint8_t q = (uint8_t)(b * kPow3[n]);
    return (int)(((uint16_t)q * 3u) >> 8);
}

/* Element e (0..127) of one 28-byte block -> trit in {-1,0,+1}.
 * Order: dequantize_row_ptq1_0 stage loop, prism_ptq1_0_quant_dequant.c:63-80
 * (stage c=16: element n*16+m <- qs[m] digit n; c=8: 80+n*8+m <- qs[16+m]; qh: 120+n*2+h);
 * same map as shaders/common.h:13-17 and docs/MODEL_SPEC.en.md:101-103.
 * Pinned: element-by-element equality with orc_ptq1_dequant_row (the loop form) and with
 * the MODEL_SPEC formula in tests; single-hot pack->decode tests.                         */
int orc_ptq1_elem_trit(const uint8_t* blk, int e) {
    if (e < 80) return orc_ptq1_digit(blk[e & 15], (uint32_t)(e >> 4)) - 1;
    if (e < 120) { int e2 = e - 80; return orc_ptq1_digit(blk[16 + (e2 & 7)], (uint32_t)(e2 >> 3)) - 1; }
    { int e3 = e - 120; return orc_ptq1_digit(blk[24 + (e3 & 1)], (uint32_t)(e3 >> 1)) - 1; }
}

float orc_ptq1_scale(const uint8_t* blk) {
    return orc_half_to_float((uint16_t)(blk[26] | (blk[27] << 8)));
}

/* dequantize_row_ptq1_0: prism_ptq1_0_quant_dequant.c:54-84 (loop form, kept literal in
 * structure: 3 stages {32,16,8} over the 24 qs bytes, then the 2 qh bytes x 4 digits).
 * Pinned: vs per-element form, vs golden fixtures, round trip with the quantiser.       */
static const size_t kStages[3] = {32, 16, 8};

void orc_ptq1_dequant_row(const uint8_t* x, float* y, int64_t k) {
    const int64_t nb = k / ORC_GROUP;
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t* blk = x + i * ORC_BLOCK_BYTES;
        const float d = orc_ptq1_scale(blk);
        size_t j = 0;
        for (size_t s = 0; s < 3; ++s) {
            const size_t c = kStages[s];
            for (; j + c <= 24; j += c)
                for (size_t n = 0; n < 5; ++n)
                    for (size_t m = 0; m < c; ++m) {
                        uint8_t q = (uint8_t)(blk[j + m] * kPow3[n]);
                        int16_t xi = (int16_t)(((uint16_t)q * 3) >> 8);
                        *y++ = (float)(xi - 1) * d;
                    }
        }
        for (size_t n = 0; n < 4; ++n)
            for (size_t h = 0; h < 2; ++h) {
                uint8_t q = (uint8_t)(blk[24 + h] * kPow3[n]);
                int16_t xi = (int16_t)(((uint16_t)q * 3) >> 8);
                *y++ = (float)(xi - 1) * d;
            }
    }
}

/* quantize_row_ptq1_0_ref: prism_ptq1_0_quant_dequant.c:4-52.
 * d = amax (stored fp16); digit = lroundf(x/d)+1; 5 digits per qs byte most significant
 * first, byte = ceil(q*256/243); qh packs 4 digits then x3.
 * Pinned: decode(quant(x)) == sign pattern for ternary inputs, exhaustive over all 3^5 /
 * 3^4 digit tuples (round trip), golden fixtures.                                       */
void orc_ptq1_quant_row(const float* x, uint8_t* y, int64_t k) {
    const int64_t nb = k / ORC_GROUP;
    for (int64_t i = 0; i < nb; i++) {
        uint8_t* blk = y + i * ORC_BLOCK_BYTES;
        float amax = 0.0f;
        for (int j = 0; j < ORC_GROUP; j++) amax = fmaxf(amax, fabsf(x[j]));
        const float d = amax, id = d ? 1.0f / d : 0.0f;
        const uint16_t dh = orc_float_to_half(d);
        blk[26] = (uint8_t)(dh & 0xff); blk[27] = (uint8_t)(dh >> 8);
        size_t j = 0;
        for (size_t s = 0; s < 3; ++s) {
            const size_t c = kStages[s];
            for (; j + c <= 24; j += c) {
                for (size_t m = 0; m < c; ++m) {
                    uint8_t q = 0;
                    for (size_t n = 0; n < 5; ++n) {
                        int xi = (int)lroundf(x[m + n * c] * id) + 1;
                        q = (uint8_t)(q * 3); q = (uint8_t)(q + xi);
                    }
                    q = (uint8_t)(((uint16_t)q * 256 + (243 - 1)) / 243);
                    blk[j + m] = q;
                }
                x += 5 * c;
            }
        }
        for (size_t h = 0; h < 2; ++h) {
            uint8_t q = 0;
            for (size_t m = 0; m < 4; ++m) {
                int xi = (int)lroundf(x[h + m * 2] * id) + 1;
                q = (uint8_t)(q * 3); q = (uint8_t)(q + xi);
            }
            q = (uint8_t)(q * 3);
            q = (uint8_t)(((uint16_t)q * 256 + (243 - 1)) / 243);
            blk[24 + h] = q;
        }
        x += 8;
    }
}

/* Packs given trits (int8 in {-1,0,1}, element order) with a given fp16 scale per block,
 * using the quantiser's byte encoding (prism_ptq1_0_quant_dequant.c:22-31,38-46).  This is
 * quantize_row_ptq1_0_ref with d supplied instead of amax, used to build synthetic
 * weights with |N(0,0.02)| scales.  Pinned by the round trip decode(pack(t)) == t.      */
void orc_ptq1_pack_row(const int8_t* t, const uint16_t* dh, uint8_t* y, int64_t k) {
    const int64_t nb = k / ORC_GROUP;
    for (int64_t i = 0; i < nb; i++) {
        const int8_t* tb = t + i * ORC_GROUP;
        uint8_t* blk = y + i * ORC_BLOCK_BYTES;
        size_t j = 0, base = 0;
        for (size_t s = 0; s < 3; ++s) {
            const size_t c = kStages[s];
            for (; j + c <= 24; j += c) {
                for (size_t m = 0; m < c; ++m) {
                    uint32_t q = 0;
                    for (size_t n = 0; n < 5; ++n) q = q * 3 + (uint32_t)(tb[base + m + n * c] + 1);
                    blk[j + m] = (uint8_t)((q * 256 + 242) / 243);
                }
                base += 5 * c;
            }
        }
        for (size_t h = 0; h < 2; ++h) {
            uint32_t q = 0;
            for (size_t m = 0; m < 4; ++m) q = q * 3 + (uint32_t)(tb[base + h + m * 2] + 1);
            q *= 3;
            blk[24 + h] = (uint8_t)((q * 256 + 242) / 243);
        }
        blk[26] = (uint8_t)(dh[i] & 0xff); blk[27] = (uint8_t)(dh[i] >> 8);
    }
}

/* Float-pipe decode identity: t_n = floor(3^(n+1) u) - 3 floor(3^n u) - 1, u = b/256
 * (docs/reference/prism_metal_dequantize_ptq1_0.h:208-212, shaders/gemv_fast.metal:2-3).
 * Pinned: exhaustive equality with orc_ptq1_digit over all 256x5.                       */
int orc_ptq1_digit_float(uint32_t b, uint32_t n) {
    const float u = (float)b * (1.0f / 256.0f);
    return (int)(floorf((float)kPow3[n + 1] * u) - 3.0f * floorf((float)kPow3[n] * u));
}

/* ---------------------------------------------------------------- GEMV oracles --------
 * y[t][n] = sum_b d[n,b] * sum_e trit[n,b,e] * x[t][128 b + e], accumulated in double.
 * Semantics of k_gemv_ptq1 (shaders/gemv.metal:5-20), k_gemv_v1 (gemv_fast.metal:9-50),
 * k_gemv_v1h (mtp.metal:66-103) and k_gemv_lut2 (mtp.metal:164-205): all compute this sum;
 * they differ only in fp32/fp16 rounding.  x is [T][K] fp32 (fp16 inputs are widened).
 * Pinned: brute force over the dequantised matrix (orc_ptq1_dequant_row + textbook dot),
 * special cases (zero trits, d = 0, single hot element, x = 1 -> d * sum t).            */
void orc_gemv_ptq1(const uint8_t* W, const float* x, double* y, int K, int N, int T) {
    const int nb = K / ORC_GROUP;
    for (int n = 0; n < N; n++) {
        const uint8_t* row = W + (size_t)n * nb * ORC_BLOCK_BYTES;
        for (int t = 0; t < T; t++) {
            double acc = 0.0;
            for (int b = 0; b < nb; b++) {
                const uint8_t* blk = row + (size_t)b * ORC_BLOCK_BYTES;
                double s = 0.0;
                for (int e = 0; e < ORC_GROUP; e++)
                    s += (double)orc_ptq1_elem_trit(blk, e) * (double)x[(size_t)t * K + b * ORC_GROUP + e];
                acc += (double)orc_ptq1_scale(blk) * s;
            }
            y[(size_t)t * N + n] = acc;
        }
    }
}

/* Q8_0 GEMV: y[t][n] = sum_b d[n,b] * sum_i q[n,b,i] * x[t][32 b + i]
 * (shaders/mtp.metal:5-20; block layout mtp.metal:9-11).  Double accumulation.
 * Pinned: brute force against an independently dequantised matrix in tests.            */
void orc_gemv_q8(const uint8_t* W, const float* x, double* y, int K, int N, int T) {
    const int nb = K / ORC_Q8_GROUP;
    for (int n = 0; n < N; n++) {
        const uint8_t* row = W + (size_t)n * nb * ORC_Q8_BLOCK_BYTES;
        for (int t = 0; t < T; t++) {
            double acc = 0.0;
            for (int b = 0; b < nb; b++) {
                const uint8_t* blk = row + (size_t)b * ORC_Q8_BLOCK_BYTES;
                const double d = orc_half_to_float((uint16_t)(blk[0] | (blk[1] << 8)));
                double s = 0.0;
                for (int i = 0; i < ORC_Q8_GROUP; i++)
                    s += (double)(int8_t)blk[2 + i] * (double)x[(size_t)t * K + b * ORC_Q8_GROUP + i];
                acc += d * s;
            }
            y[(size_t)t * N + n] = acc;
        }
    }
}

/* ---------------------------------------------------------------- prefill oracles -----
 * Weight expansion, k_expand_ptq1_v2 (shaders/prefill.metal:472-479, ptq1_slice :445-456):
 * w[n][k] = half(trit * d), exact in fp16.  Written here in natural [N][K] order (the
 * reference writes tile-major [N/64][K][64]; the order is a storage detail).
 * Pinned: bit-exact vs orc_float_to_half(orc_ptq1_dequant_row) and vs fixtures.         */
void orc_expand_ptq1_f16(const uint8_t* W, uint16_t* out, int K, int N) {
    const int nb = K / ORC_GROUP;
    for (int n = 0; n < N; n++)
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = W + ((size_t)n * nb + b) * ORC_BLOCK_BYTES;
            const float d = orc_ptq1_scale(blk);
            for (int e = 0; e < ORC_GROUP; e++)
                out[(size_t)n * K + b * ORC_GROUP + e] = orc_float_to_half((float)orc_ptq1_elem_trit(blk, e) * d);
        }
}

/* Exact fp16 prefill GEMM, k_gemm_f16 (shaders/prefill.metal:31-41):
 * C[m][n] = sum_k A[m][k] * Wexp[n][k], A and Wexp fp16, accumulated in double here
 * (the reference accumulates in fp32; parity is tolerance based).
 * Pinned: textbook GEMM over orc_expand_ptq1_f16 output; tests also compare a numpy
 * matmul of the expanded matrix.                                                          */
void orc_gemm_ptq1_f16(const uint16_t* A, const uint8_t* W, double* C, int M, int K, int N) {
    uint16_t* wexp = (uint16_t*)malloc((size_t)N * K * 2);
    float* af = (float*)malloc((size_t)M * K * 4);
    float* wf = (float*)malloc((size_t)K * 4);
    orc_expand_ptq1_f16(W, wexp, K, N);
    for (size_t i = 0; i < (size_t)M * K; i++) af[i] = orc_half_to_float(A[i]);
    for (int n = 0; n < N; n++) {
        for (int k = 0; k < K; k++) wf[k] = orc_half_to_float(wexp[(size_t)n * K + k]);
        for (int m = 0; m < M; m++) {
            double s = 0.0;
            const float* ar = af + (size_t)m * K;
            for (int k = 0; k < K; k++) s += (double)ar[k] * (double)wf[k];
            C[(size_t)m * N + n] = s;
        }
    }
    free(wexp); free(af); free(wf);
}

/* k_expand_q8 (shaders/mtp.metal:24-33): the fp16 weight of a Q8_0 element is
 * half(d * float(q)), d the block's fp16 scale, rounded to nearest even.
 * Pinned: numpy's float32 -> float16 conversion of d * q in tests.                       */
void orc_expand_q8_f16(const uint8_t* W, uint16_t* out, int K, int N) {
    const int nb = K / ORC_Q8_GROUP;
    for (int n = 0; n < N; n++)
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = W + ((size_t)n * nb + b) * ORC_Q8_BLOCK_BYTES;
            const float d = orc_half_to_float((uint16_t)(blk[0] | (blk[1] << 8)));
            for (int i = 0; i < ORC_Q8_GROUP; i++)
                out[(size_t)n * K + b * ORC_Q8_GROUP + i] = orc_float_to_half(d * (float)(int8_t)blk[2 + i]);
        }
}

/* The MTP K/V catch-up GEMM, k_expand_q8 then dGemm (src/engine.cpp:392-401):
 * C[m][n] = sum_k A[m][k] * Wexp[n][k], A and Wexp fp16, accumulated in double here.
 * Pinned: textbook GEMM over orc_expand_q8_f16; tests compare a numpy matmul too.       */
void orc_gemm_q8_f16(const uint16_t* A, const uint8_t* W, double* C, int M, int K, int N) {
    uint16_t* wexp = (uint16_t*)malloc((size_t)N * K * 2);
    float* af = (float*)malloc((size_t)M * K * 4);
    float* wf = (float*)malloc((size_t)K * 4);
    orc_expand_q8_f16(W, wexp, K, N);
    for (size_t i = 0; i < (size_t)M * K; i++) af[i] = orc_half_to_float(A[i]);
    for (int n = 0; n < N; n++) {
        for (int k = 0; k < K; k++) wf[k] = orc_half_to_float(wexp[(size_t)n * K + k]);
        for (int m = 0; m < M; m++) {
            double s = 0.0;
            const float* ar = af + (size_t)m * K;
            for (int k = 0; k < K; k++) s += (double)ar[k] * (double)wf[k];
            C[(size_t)m * N + n] = s;
        }
    }
    free(wexp); free(af); free(wf);
}

/* Activation quantisation, k_quant_rows (shaders/prefill.metal:369-381):
 * per (token m, 128-group g): amax over the group, scale = amax > 0 ? amax/127 : 1,
 * q = clamp(rint(x * (1/scale)), -127, 127), sx[g*ldS + m] = scale.
 * All arithmetic in fp32 with IEEE division, rint = round half to even.
 * Pinned: closed form in tests (amax = 0 -> scale 1, exact ties, clamp), fixtures.       */
void orc_quant_rows(const uint16_t* X, int8_t* Q, float* SX, int M, int K, int ldS) {
    const int G = K / ORC_GROUP;
    for (int m = 0; m < M; m++)
        for (int g = 0; g < G; g++) {
            const uint16_t* xr = X + (size_t)m * K + g * ORC_GROUP;
            float mx = 0.0f;
            for (int i = 0; i < ORC_GROUP; i++) mx = fmaxf(mx, fabsf(orc_half_to_float(xr[i])));
            const float scale = mx > 0.0f ? mx / 127.0f : 1.0f;
            const float inv = 1.0f / scale;
            for (int i = 0; i < ORC_GROUP; i++) {
                float v = rintf(orc_half_to_float(xr[i]) * inv);
                v = fminf(fmaxf(v, -127.0f), 127.0f);
                Q[(size_t)m * K + g * ORC_GROUP + i] = (int8_t)v;
            }
            SX[(size_t)g * ldS + m] = scale;
        }
}

/* int8 weight expansion, k_expand_i8_v2 (shaders/prefill.metal:457-471): trits as int8
 * and one fp32 scale per (row, group).  Natural [N][K] and [N][K/128] order here.
 * Pinned: trits equal orc_ptq1_elem_trit; scales equal orc_ptq1_scale.                  */
void orc_expand_ptq1_i8(const uint8_t* W, int8_t* T8, float* SW, int K, int N) {
    const int nb = K / ORC_GROUP;
    for (int n = 0; n < N; n++)
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = W + ((size_t)n * nb + b) * ORC_BLOCK_BYTES;
            SW[(size_t)n * nb + b] = orc_ptq1_scale(blk);
            for (int e = 0; e < ORC_GROUP; e++)
                T8[(size_t)n * K + b * ORC_GROUP + e] = (int8_t)orc_ptq1_elem_trit(blk, e);
        }
}

/* int8 GEMM with the per-group scale epilogue, k_gemm_i8 (shaders/prefill.metal:382-415):
 * per group g the int32 sum I = sum_{k in g} A8[m][k]*T8[n][k] (exact), then
 * C += float(I) * (SW[n][g] * SX[g][m]) in fp32, groups in ascending order.
 * GS (optional, may be NULL) receives the exact int32 group sums [M][N][G].
 * Pinned: int32 sums vs brute force (bit-exact), epilogue vs a double re-evaluation.     */
void orc_gemm_i8(const int8_t* A8, const float* SX, int ldS, const uint8_t* W, float* C, int32_t* GS,
                 int M, int K, int N) {
    const int G = K / ORC_GROUP;
    int8_t* t8 = (int8_t*)malloc((size_t)N * K);
    float* sw = (float*)malloc((size_t)N * G * 4);
    orc_expand_ptq1_i8(W, t8, sw, K, N);
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            float acc = 0.0f;
            for (int g = 0; g < G; g++) {
                int32_t s = 0;
                for (int i = 0; i < ORC_GROUP; i++)
                    s += (int32_t)A8[(size_t)m * K + g * ORC_GROUP + i] * (int32_t)t8[(size_t)n * K + g * ORC_GROUP + i];
                if (GS) GS[((size_t)m * N + n) * G + g] = s;
                acc += (float)s * (sw[(size_t)n * G + g] * SX[(size_t)g * ldS + m]);
            }
            C[(size_t)m * N + n] = acc;
        }
    free(t8); free(sw);
}

/* ---------------------------------------------------------------- matmul input --------
 * The input transform of a ternary matmul, in double (shaders/ops.metal:30-54,86-106;
 * shaders/common.h:20-42; shaders/prefill.metal:59-97,266-285).  Per row m:
 *   mode 0: v = src (+ src2 when add), inv = 1/sqrt(mean(v^2) + 1e-6), u = v*inv*gs,
 *           hout = v*inv*gamma (gamma non-NULL)
 *   mode 1: u = silu(src)*src2*gs;  mode 2: u[i] = src[gdn_perm(i)]*gs[i];  mode 3: u = src*gs
 *   out[1024 b + j] = (1/32) sum_k (-1)^popcount(j & k) u[1024 b + k]
 * The transform is the textbook recursive (Sylvester) Walsh-Hadamard butterfly in natural
 * order.  Pinned: against scipy.linalg.hadamard(1024) products, involution (H/32)^2 = I,
 * and closed forms of the norm and SwiGLU on special inputs.                              */
static void orc_fwht_d(double* v, int n) {
    for (int h = 1; h < n; h <<= 1)
        for (int i = 0; i < n; i += 2 * h)
            for (int j = i; j < i + h; j++) {
                const double a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
}

static int orc_gdn_perm(int i) {
    const int h = i & 127, t = i >> 7, rr = t % 3, k = t / 3;
    return h + 128 * (k + 16 * rr);
}

void orc_norm_fwht(const float* src, const float* src2, const float* gs, const float* gamma, double* out,
                   double* hout, int W, int M, int mode, int add) {
    double* u = (double*)malloc((size_t)W * sizeof(double));
    for (int m = 0; m < M; m++) {
        const float* s = src + (size_t)m * W;
        const float* s2 = src2 ? src2 + (size_t)m * W : NULL;
        double inv = 1.0;
        if (mode == 0) {
            double ss = 0.0;
            for (int i = 0; i < W; i++) {
                const double v = (double)s[i] + (add ? (double)s2[i] : 0.0);
                ss += v * v;
            }
            inv = 1.0 / sqrt(ss / W + 1e-6);
        }
        for (int i = 0; i < W; i++) {
            double v;
            if (mode == 0) {
                const double x = (double)s[i] + (add ? (double)s2[i] : 0.0);
                if (gamma) hout[(size_t)m * W + i] = x * inv * gamma[i];
                v = x * inv;
            } else if (mode == 1) {
                const double g = s[i];
                v = g / (1.0 + exp(-g)) * s2[i];
            } else if (mode == 2) {
                v = s[orc_gdn_perm(i)];
            } else {
                v = s[i];
            }
            u[i] = v * gs[i];
        }
        for (int b = 0; b < W; b += 1024) {
            orc_fwht_d(u + b, 1024);
            for (int j = 0; j < 1024; j++) out[(size_t)m * W + b + j] = u[b + j] / 32.0;
        }
    }
    free(u);
}

/* ---------------------------------------------------------------- CPU baseline --------
 * The reference has no CPU matmul; its host-side arithmetic for the path is the PTQ1_0
 * decoder (prism_ptq1_0_quant_dequant.c:54-84).  The baseline timed next to the GPU is
 * that decoder plus an fp32 dot per block with k_gemv_ptq1 semantics
 * (shaders/gemv.metal:12-17): s = sum_e trit*x in fp32, acc += d*s.  OpenMP over rows.
 * Rows [row0, row0+nrows) only, so a bounded sample can be timed.                        */
void orc_cpu_gemv_ptq1_f32(const uint8_t* W, const float* x, float* y, int K, int N, int T,
                           int row0, int nrows, int nthreads) {
    const int nb = K / ORC_GROUP;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel for schedule(static)
#endif
    for (int r = row0; r < row0 + nrows; r++) {
        float tr[ORC_GROUP];
        float acc[4] = {0, 0, 0, 0};
        const uint8_t* row = W + (size_t)r * nb * ORC_BLOCK_BYTES;
        for (int b = 0; b < nb; b++) {
            const uint8_t* blk = row + (size_t)b * ORC_BLOCK_BYTES;
            for (int e = 0; e < ORC_GROUP; e++) tr[e] = (float)orc_ptq1_elem_trit(blk, e);
            const float d = orc_ptq1_scale(blk);
            for (int t = 0; t < T && t < 4; t++) {
                const float* xb = x + (size_t)t * K + b * ORC_GROUP;
                float s = 0.0f;
                for (int e = 0; e < ORC_GROUP; e++) s += tr[e] * xb[e];
                acc[t] += d * s;
            }
        }
        for (int t = 0; t < T && t < 4; t++) y[(size_t)t * N + r] = acc[t];
    }
}

/* CPU baseline in the reference's own host form: each weight row is expanded to fp32 by
 * the stage-loop dequantize_row_ptq1_0 (prism_ptq1_0_quant_dequant.c:54-84, restated in
 * orc_ptq1_dequant_row above; d folded into every weight), then fp32 dots with the T
 * activation rows.  OpenMP over rows, one row buffer per thread.                        */
void orc_cpu_gemv_ptq1_stage(const uint8_t* W, const float* x, float* y, int K, int N, int T, int row0,
                             int nrows, int nthreads) {
    const int nb = K / ORC_GROUP;
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        float* w = (float*)malloc((size_t)K * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int r = row0; r < row0 + nrows; r++) {
            orc_ptq1_dequant_row(W + (size_t)r * nb * ORC_BLOCK_BYTES, w, K);
            for (int t = 0; t < T; t++) {
                const float* xt = x + (size_t)t * K;
                float s = 0.0f;
                for (int k = 0; k < K; k++) s += w[k] * xt[k];
                y[(size_t)t * N + r] = s;
            }
        }
        free(w);
    }
}

/* CPU baseline of the prefill GEMM (k_gemm_f16 semantics after k_expand_ptq1_v2,
 * shaders/prefill.metal:31-41,472-479): each weight row n in [row0, row0+nrows) is decoded
 * once to fp32 (half(t*d) is exact), then C[m][n] = sum_k A[m][k]*w[k] in fp32 for every A
 * row.  OpenMP over weight rows; a bounded sample of columns can be timed.               */
void orc_cpu_gemm_ptq1_f32(const uint16_t* A, const uint8_t* W, float* C, int M, int K, int N, int row0,
                           int nrows, int nthreads) {
    const int nb = K / ORC_GROUP;
    float* af = (float*)malloc((size_t)M * K * 4);
    for (size_t i = 0; i < (size_t)M * K; i++) af[i] = orc_half_to_float(A[i]);
    const int nq = (nrows + 3) / 4;              /* quads of weight rows: each A row is read once per quad */
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
    {
        float* w = (float*)malloc((size_t)4 * K * 4);
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
        for (int q = 0; q < nq; q++) {
            const int n0 = row0 + 4 * q, nr = (4 < row0 + nrows - n0) ? 4 : row0 + nrows - n0;
            for (int r = 0; r < 4; r++) {
                const int n = n0 + (r < nr ? r : 0);
                const uint8_t* row = W + (size_t)n * nb * ORC_BLOCK_BYTES;
                for (int b = 0; b < nb; b++) {
                    const uint8_t* blk = row + (size_t)b * ORC_BLOCK_BYTES;
                    const float d = orc_ptq1_scale(blk);
                    for (int e = 0; e < ORC_GROUP; e++)
                        w[(size_t)r * K + b * ORC_GROUP + e] = (float)orc_ptq1_elem_trit(blk, e) * d;
                }
            }
            for (int m = 0; m < M; m++) {
                const float* ar = af + (size_t)m * K;
                float acc[4][16] = {{0}};        /* 4 rows x 16 lanes: 8 vector accumulators */
                for (int k = 0; k < K; k += 16)
                    for (int r = 0; r < 4; r++)
                        for (int j = 0; j < 16; j++) acc[r][j] += ar[k + j] * w[(size_t)r * K + k + j];
                for (int r = 0; r < nr; r++) {
                    float s = 0.0f;
                    for (int j = 0; j < 16; j++) s += acc[r][j];
                    C[(size_t)m * N + n0 + r] = s;
                }
            }
        }
        free(w);
    }
    free(af);
}

int orc_omp_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
