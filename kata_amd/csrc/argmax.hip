// Greedy argmax over n floats for the lm_head logits (shaders/ops.metal:66-78, k_argmax):
// an element is taken only if strictly greater than the best so far (so NaN and -inf never
// are), lowest index on ties; with no such element the result is 0x7fffffff, as there.
//
// Design: a grid of up to 256 workgroups, each reducing a contiguous range (16-byte loads,
// a fixed-order reduction across lanes and waves) to one (value, index) pair in a device
// array of the calling stream, then a one-workgroup launch reduces those pairs in workgroup
// order and writes the index: deterministic, and nothing has to be cleared between calls.
// (A last-arriving-workgroup reduction in one launch needs a device-scope release per
// workgroup, an L2 write-back on this chip, which costs more than the second launch.)
// Each (device, stream) has its own pair array (allocated on its first call): calls on
// different streams do not share it.
#include "launch.h"

#include <math.h>

#include <algorithm>

namespace kata {

namespace {

constexpr int kMaxGroups = 256;
struct Part {
    float v[kMaxGroups];
    int i[kMaxGroups];
};

// element b at index ib after the current best a (indices increasing): strictly greater
__device__ inline void take(float& a, int& ia, float b, int ib) {
    if (b > a) {
        a = b;
        ia = ib;
    }
}
// two partial bests: larger value, then lower index
__device__ inline void better(float& a, int& ia, float b, int ib) {
    if (b > a || (b == a && ib < ia)) {
        a = b;
        ia = ib;
    }
}

__device__ inline void block_best(float& v, int& i, float* sv, int* si) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) better(v, i, __shfl_xor(v, o), __shfl_xor(i, o));
    if ((tid & 63) == 0) {
        sv[tid >> 6] = v;
        si[tid >> 6] = i;
    }
    __syncthreads();
    if (tid == 0)
        for (int w = 1; w < (int)blockDim.x / 64; w++) better(v, i, sv[w], si[w]);
}

__global__ __launch_bounds__(256) void k_argmax(const float* __restrict__ x, int n, Part* __restrict__ part) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int tid = threadIdx.x, G = gridDim.x;
    const int lo = (int)(((long)blockIdx.x * n) / G), hi = (int)(((long)(blockIdx.x + 1) * n) / G);
    float v = -INFINITY;
    int idx = 0x7fffffff;
    // scalar head up to a 4-element boundary, 16-byte loads, scalar tail
    const int a0 = min(hi, (lo + 3) & ~3), a1 = max(a0, hi & ~3);
    for (int k = lo + tid; k < a0; k += 256) take(v, idx, x[k], k);
    for (int k = a0 + 4 * tid; k < a1; k += 1024) {
        const float4 q = *(const float4*)(x + k);
        take(v, idx, q.x, k);
        take(v, idx, q.y, k + 1);
        take(v, idx, q.z, k + 2);
        take(v, idx, q.w, k + 3);
    }
    for (int k = a1 + tid; k < hi; k += 256) take(v, idx, x[k], k);
    block_best(v, idx, sv, si);
    if (tid == 0) {
        part->v[blockIdx.x] = v;
        part->i[blockIdx.x] = idx;
    }
}

__global__ __launch_bounds__(256) void k_argmax_final(int G, const Part* __restrict__ part, int* __restrict__ out) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int tid = threadIdx.x;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int g = tid; g < G; g += 256) better(bv, bi, part->v[g], part->i[g]);
    block_best(bv, bi, sv, si);
    if (tid == 0) *out = bi;
}

}  // namespace

hipError_t launch_argmax(const float* x, int n, int* out, hipStream_t s) {
    const int G = std::max(1, std::min(kMaxGroups, n / 1024));
    void* part = nullptr;
    hipError_t e = stream_buffer(kBufArgmax, sizeof(Part), s, &part);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_argmax, dim3(G), dim3(256), 0, s, x, n, (Part*)part);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s, G, (const Part*)part, out);
    return hipGetLastError();
}

}  // namespace kata
