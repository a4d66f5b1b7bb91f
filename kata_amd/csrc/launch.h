// Internal launch interface between the C ABI (capi.cpp) and the kernel files.
// Arguments are validated by the caller; each function returns the hipError_t of the launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace kata {

// ---- scratch memory (workspace.cpp): the calling thread's device's CU count, and a device
// buffer of at least `bytes` for (device, kind, stream), allocated on first use; a buffer
// outgrown by a larger call is retired, never freed, until release_stream(s)
enum { kBufGemmPieces = 0, kBufArgmax = 1, kBufWideImage = 2 };
hipError_t device_cu_count(int* n_cu);
hipError_t stream_buffer(int kind, size_t bytes, hipStream_t s, void** p);
hipError_t release_stream(hipStream_t s);   // synchronises s, frees every buffer of (device, s)

// ---- PTQ1_0 GEMV (gemv_ptq1.hip); x 16-byte aligned, rows [T][K] or half2 [K][2] (T = 2)
hipError_t launch_gemv_ptq1(const uint8_t* W, const void* x, int x_dtype, int x_layout, float* y, int K, int N, int T,
                            hipStream_t s);
hipError_t launch_gemv_ptq1_multi(int count, const uint8_t* const* W, float* const* y, const int* N, const void* x,
                                  int x_dtype, int x_layout, int K, int T, hipStream_t s);
int gemv_max_k(int T);   // largest K the PTQ1_0 GEMV accepts (its activation image lives in LDS)
int gemv_max_mats();     // most matrices one launch takes
// the operand form of T (1, 2) raw activation rows (x_dtype KATA_XQ of the GEMV)
hipError_t launch_gemv_prepare(const void* x, int x_dtype, int x_layout, int K, int T, void* xq, hipStream_t s);
// wide verification GEMV, T in 1..8 token rows x [T][K] (fp16 or fp32), y [T][N]
hipError_t launch_gemv_wide(const uint8_t* W, const void* x, int x_dtype, float* y, int K, int N, int T,
                            hipStream_t s);
// the same with its activation image in a fixed per-device device array (no allocation)
hipError_t launch_gemv_wide_noalloc(const uint8_t* W, const void* x, int x_dtype, float* y, int K, int N, int T,
                                    hipStream_t s);
bool gemv_wide_noalloc_fits(int K, int T);
// the same for 1..4 matrices sharing the token rows, one launch after the activation prep
hipError_t launch_gemv_wide_batch(int count, const uint8_t* const* W, float* const* y, const int* N, const void* x,
                                  int x_dtype, int K, int T, hipStream_t s);
size_t gemv_wide_noalloc_scratch_bytes();

// ---- Q8_0 GEMV (gemv_q8.hip); the batch form: 1..gemv_q8_max_mats() matrices sharing x
hipError_t launch_gemv_q8(const uint8_t* W, const void* x, int x_dtype, float* y, int K, int N, int T,
                          hipStream_t s);
hipError_t launch_gemv_q8_multi(int count, const uint8_t* const* W, float* const* y, const int* N, const void* x,
                                int x_dtype, int K, int T, hipStream_t s);
int gemv_q8_max_mats();

// ---- prefill (gemm_f16.hip, gemm_i8.hip, expand.hip)
hipError_t launch_gemm_f16(const uint16_t* A, int lda, const uint8_t* W, void* C, int c_dtype, int ldc,
                           int M, int K, int N, hipStream_t s);
hipError_t launch_gemm_q8(const uint16_t* A, int lda, const uint8_t* W, void* C, int c_dtype, int ldc, int M, int K,
                          int N, hipStream_t s);
hipError_t launch_quant_rows(const uint16_t* X, int8_t* Q, float* SX, int M, int K, int ldS,
                             hipStream_t s);
hipError_t launch_gemm_i8(const int8_t* A8, const float* SX, int ldS, const uint8_t* W, void* C,
                          int c_dtype, int ldc, int M, int K, int N, hipStream_t s);
hipError_t launch_expand_f16(const uint8_t* W, uint16_t* out, int K, int N, hipStream_t s);
hipError_t launch_expand_i8(const uint8_t* W, int8_t* T8, float* SW, int K, int N, hipStream_t s);

// ---- matmul input transform (norm_fwht.hip); flags: 1 add src2 (mode 0), 2 write xnew,
// 4 write hout, 8 hout fp16
hipError_t launch_norm_fwht(const float* src, const float* src2, const float* gs, void* out, int out_dtype,
                            int out_layout, float* xnew, const float* gamma, void* hout, int flags, int W, int M,
                            int mode, hipStream_t s);

// ---- measurement helpers (calib.hip): empty kernel and plain streaming read, wgs x 1024
hipError_t launch_calib_empty(uint32_t* out, int wgs, hipStream_t s);
hipError_t launch_calib_read(const uint8_t* p, uint32_t bytes, uint32_t* out, int wgs, hipStream_t s);
// the read ceiling: two 256-thread workgroups per CU, non-temporal 16-byte loads
hipError_t launch_calib_read_peak(const uint8_t* p, uint32_t bytes, uint32_t* out, int cus, hipStream_t s);
// any swept geometry: threads 256/512/1024 per workgroup, wgs workgroups, 2/4/8/16 loads in flight
hipError_t launch_calib_read_cfg(const uint8_t* p, uint32_t bytes, uint32_t* out, int threads, int wgs, int inflight,
                                 bool nt, hipStream_t s);
// the decode GEMV's weight-load stream alone (one matrix, T = 1, one workgroup per CU)
hipError_t launch_calib_read_ptq1(const uint8_t* W, int K, int N, uint32_t* out, int cus, hipStream_t s);

// ---- argmax of the logits (argmax.hip)
hipError_t launch_argmax(const float* x, int n, int* out, hipStream_t s);

}  // namespace kata
