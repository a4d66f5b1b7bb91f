// Shared definitions of the gfx950 ternary-matmul kernels.
//
// PTQ1_0 block (28 bytes, 128 weights): qs[24] | qh[2] | fp16 d  (config/kata_m6.h:44-45).
// Digit n (0 = most significant) of a packed byte b is ((b*3^n mod 256)*3) >> 8 and the
// weight is (digit-1)*d (docs/reference/prism_ptq1_0_quant_dequant.c:54-84).
// Element map (shaders/common.h:13-17): e<80 -> qs[e&15] digit e>>4; 80<=e<120 ->
// qs[16+(e-80)&7] digit (e-80)>>3; e>=120 -> qh[(e-120)&1] digit (e-120)>>1.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kata {

constexpr int kGroup = 128;
constexpr int kBlockBytes = 28;
constexpr int kQ8Group = 32;
constexpr int kQ8BlockBytes = 34;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

__host__ __device__ inline uint32_t pow3u(uint32_t n) {
    return n == 0 ? 1u : n == 1 ? 3u : n == 2 ? 9u : n == 3 ? 27u : n == 4 ? 81u : 243u;
}

// digit n of byte b, integer form
__host__ __device__ inline uint32_t ptq1_digit(uint32_t b, uint32_t n) {
    return ((((b * pow3u(n)) & 0xffu) * 3u) >> 8);
}

// (byte index, digit) of element e of a block
__host__ __device__ constexpr void ptq1_elem_src(int e, int& p, int& n) {
    if (e < 80) { p = e & 15; n = e >> 4; }
    else if (e < 120) { p = 16 + ((e - 80) & 7); n = (e - 80) >> 3; }
    else { p = 24 + ((e - 120) & 1); n = (e - 120) >> 1; }
}

// element held by (byte p, digit n), or -1 if that slot carries no element
__host__ __device__ inline int ptq1_slot_elem(int p, int n) {
    if (p < 16) return n < 5 ? 16 * n + p : -1;
    if (p < 24) return n < 5 ? 80 + 8 * n + (p - 16) : -1;
    if (p < 26) return n < 4 ? 120 + 2 * n + (p - 24) : -1;
    return -1;
}

__device__ inline float half_bits_to_float(uint32_t h16) {
    union { uint16_t u; _Float16 h; } c;
    c.u = (uint16_t)h16;
    return (float)c.h;
}

}  // namespace kata
