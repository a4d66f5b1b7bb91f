// C ABI of the gfx950 ternary-matmul library: argument validation, error reporting,
// the host packers and the engine-style
// dispatcher.  Declarations and reference citations: include/kata_amd.h.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <string>

#include "../../include/kata_amd.h"
#include "gemv_operand.h"
#include "launch.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

// a byte range [p, p + n); null pointers overlap nothing
struct Span {
    const void* p;
    size_t n;
};
bool overlap(const Span& a, const Span& b) {
    if (!a.p || !b.p || !a.n || !b.n) return false;
    const uintptr_t a0 = (uintptr_t)a.p, b0 = (uintptr_t)b.p;
    return a0 < b0 + b.n && b0 < a0 + a.n;
}

int check_launch(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail(KATA_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
    g_err.clear();
    return KATA_OK;
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p & (a - 1)) == 0; }
size_t align16(size_t n) { return (n + 15) & ~(size_t)15; }

int check_gemv_args(const void* W, const void* x, int x_dtype, int x_layout, const void* y, int K, int N,
                    int T) {
    if (!W || !x || !y) return fail(KATA_EINVAL, "null pointer argument");
    if (K <= 0 || K % 128 != 0) return fail(KATA_EINVAL, "K=%d must be a positive multiple of 128", K);
    if (N <= 0) return fail(KATA_EINVAL, "N=%d must be positive", N);
    if (T != 1 && T != 2) return fail(KATA_EINVAL, "T=%d must be 1 or 2", T);
    if (K > kata::gemv_max_k(T)) return fail(KATA_EINVAL, "K=%d exceeds %d for T=%d", K, kata::gemv_max_k(T), T);
    if (x_dtype != KATA_F32 && x_dtype != KATA_F16 && x_dtype != KATA_XQ) return fail(KATA_EINVAL, "x_dtype=%d", x_dtype);
    if (x_layout != KATA_X_ROWS && x_layout != KATA_X_HALF2) return fail(KATA_EINVAL, "x_layout=%d", x_layout);
    if (x_dtype == KATA_XQ && x_layout != KATA_X_ROWS) return fail(KATA_EINVAL, "the operand form takes KATA_X_ROWS");
    if (x_dtype == KATA_XQ && kata_gemv_xq_bytes(K, T) == 0)
        return fail(KATA_EINVAL, "K=%d: the operand form exceeds %d bytes", K, kata::kXqMaxBytes);
    if (x_layout == KATA_X_HALF2 && (T != 2 || x_dtype != KATA_F16))
        return fail(KATA_EINVAL, "KATA_X_HALF2 needs T=2 and fp16 activations");
    if (!aligned(W, 4)) return fail(KATA_EINVAL, "W must be 4-byte aligned");
    if (!aligned(x, 16)) return fail(KATA_EINVAL, "x must be 16-byte aligned");
    return KATA_OK;
}

}  // namespace

// for the other host sources of the library (gguf.cpp)
int kata_internal_fail(int code, const char* msg) { return fail(code, "%s", msg); }


extern "C" {

const char* kata_last_error(void) { return g_err.c_str(); }
const char* kata_version(void) { return "kata_amd 0.1 (gfx950)"; }

// ------------------------------------------------------------------ PTQ1_0 GEMV
int kata_gemv_ptq1_max_k(int T) { return (T == 1 || T == 2) ? kata::gemv_max_k(T) : 0; }

size_t kata_gemv_xq_bytes(int K, int T) {
    if (T < 1 || T > 8 || K <= 0 || K % 128 != 0) return 0;
    if (T > 2) return (size_t)kata::gemv_xq_bytes(K, T);           // the wide GEMV's image
    if (K > kata::gemv_max_k(T)) return 0;
    const long long b = kata::gemv_xq_bytes(K, T);
    return b <= kata::kXqMaxBytes ? (size_t)b : 0;
}

int kata_gemv_prepare_x(const void* x, int x_dtype, int x_layout, int K, int T, void* xq, void* stream) {
    if (!x || !xq) return fail(KATA_EINVAL, "null pointer argument");
    if (T < 1 || T > 8) return fail(KATA_EINVAL, "T=%d must be 1..8", T);
    if (K <= 0 || K % 128 != 0) return fail(KATA_EINVAL, "K=%d must be a positive multiple of 128", K);
    if (kata_gemv_xq_bytes(K, T) == 0) return fail(KATA_EINVAL, "K=%d unsupported for T=%d", K, T);
    if (x_dtype != KATA_F32 && x_dtype != KATA_F16) return fail(KATA_EINVAL, "x_dtype=%d", x_dtype);
    if (x_layout != KATA_X_ROWS && x_layout != KATA_X_HALF2) return fail(KATA_EINVAL, "x_layout=%d", x_layout);
    if (x_layout == KATA_X_HALF2 && (T != 2 || x_dtype != KATA_F16))
        return fail(KATA_EINVAL, "KATA_X_HALF2 needs T=2 and fp16 activations");
    if (!aligned(x, 16) || !aligned(xq, 16)) return fail(KATA_EINVAL, "x and xq must be 16-byte aligned");
    const size_t xb = (size_t)T * K * (x_dtype == KATA_F16 ? 2 : 4);
    if (overlap({xq, kata_gemv_xq_bytes(K, T)}, {x, xb})) return fail(KATA_EINVAL, "xq overlaps x");
    return check_launch(kata::launch_gemv_prepare(x, x_dtype, x_layout, K, T, xq, (hipStream_t)stream), "gemv prepare x");
}

int kata_gemv_ptq1(const uint8_t* W, const void* x, int x_dtype, int x_layout, float* y, int K, int N, int T,
                   void* stream) {
    int rc = check_gemv_args(W, x, x_dtype, x_layout, y, K, N, T);
    if (rc) return rc;
    return check_launch(kata::launch_gemv_ptq1(W, x, x_dtype, x_layout, y, K, N, T, (hipStream_t)stream),
                        "gemv ptq1");
}

int kata_gemv_ptq1_batch(int count, const uint8_t* const* W, float* const* y, const int* N, const void* x, int x_dtype,
                         int x_layout, int K, int T, void* stream) {
    if (count < 1 || count > kata::gemv_max_mats()) return fail(KATA_EINVAL, "count=%d must be 1..%d", count, kata::gemv_max_mats());
    if (!W || !y || !N) return fail(KATA_EINVAL, "null array argument");
    for (int i = 0; i < count; i++) {
        int rc = check_gemv_args(W[i], x, x_dtype, x_layout, y[i], K, N[i], T);
        if (rc) return rc;
    }
    return check_launch(kata::launch_gemv_ptq1_multi(count, W, y, N, x, x_dtype, x_layout, K, T, (hipStream_t)stream),
                        "gemv ptq1 batch");
}

// activation dtype of the wide entries: fp32 / fp16 rows, or the operand form of T rows
static int check_wide_x(int x_dtype, int K, int T) {
    if (x_dtype != KATA_F32 && x_dtype != KATA_F16 && x_dtype != KATA_XQ) return fail(KATA_EINVAL, "x_dtype=%d", x_dtype);
    if (x_dtype == KATA_XQ && kata_gemv_xq_bytes(K, T) == 0)
        return fail(KATA_EINVAL, "K=%d T=%d has no operand form", K, T);
    return KATA_OK;
}

int kata_gemv_ptq1_wide(const uint8_t* W, const void* x, int x_dtype, float* y, int K, int N, int T, void* stream) {
    if (!W || !x || !y) return fail(KATA_EINVAL, "null pointer argument");
    if (K <= 0 || K % 128 != 0) return fail(KATA_EINVAL, "K=%d must be a positive multiple of 128", K);
    if (N <= 0) return fail(KATA_EINVAL, "N=%d must be positive", N);
    if (T < 1 || T > 8) return fail(KATA_EINVAL, "T=%d must be 1..8", T);
    if (int rc = check_wide_x(x_dtype, K, T)) return rc;
    if (!aligned(W, 4)) return fail(KATA_EINVAL, "W must be 4-byte aligned");
    if (!aligned(x, 16)) return fail(KATA_EINVAL, "x must be 16-byte aligned");
    // one or two tokens: the decode GEMV reads the weights once for both as well, faster
    if (T <= 2 && K <= kata::gemv_max_k(T))
        return check_launch(kata::launch_gemv_ptq1(W, x, x_dtype, KATA_X_ROWS, y, K, N, T, (hipStream_t)stream),
                            "gemv ptq1 wide (T <= 2)");
    return check_launch(kata::launch_gemv_wide(W, x, x_dtype, y, K, N, T, (hipStream_t)stream), "gemv ptq1 wide");
}

int kata_gemv_ptq1_wide_batch(int count, const uint8_t* const* W, float* const* y, const int* N, const void* x,
                              int x_dtype, int K, int T, void* stream) {
    if (count < 1 || count > kata::gemv_max_mats()) return fail(KATA_EINVAL, "count=%d must be 1..%d", count, kata::gemv_max_mats());
    if (!W || !y || !N || !x) return fail(KATA_EINVAL, "null argument");
    if (K <= 0 || K % 128 != 0) return fail(KATA_EINVAL, "K=%d must be a positive multiple of 128", K);
    if (T < 1 || T > 8) return fail(KATA_EINVAL, "T=%d must be 1..8", T);
    if (int rc = check_wide_x(x_dtype, K, T)) return rc;
    if (!aligned(x, 16)) return fail(KATA_EINVAL, "x must be 16-byte aligned");
    for (int i = 0; i < count; i++) {
        if (!W[i] || !y[i]) return fail(KATA_EINVAL, "null pointer in W[] or y[]");
        if (N[i] <= 0) return fail(KATA_EINVAL, "N[%d]=%d must be positive", i, N[i]);
        if (!aligned(W[i], 4)) return fail(KATA_EINVAL, "W[%d] must be 4-byte aligned", i);
    }
    if (T <= 2 && K <= kata::gemv_max_k(T))
        return check_launch(kata::launch_gemv_ptq1_multi(count, W, y, N, x, x_dtype, KATA_X_ROWS, K, T, (hipStream_t)stream),
                            "gemv ptq1 wide batch (T <= 2)");
    return check_launch(kata::launch_gemv_wide_batch(count, W, y, N, x, x_dtype, K, T, (hipStream_t)stream),
                        "gemv ptq1 wide batch");
}

int kata_gemv_ptq1_wide_noalloc(const uint8_t* W, const void* x, int x_dtype, float* y, int K, int N, int T,
                                void* stream) {
    if (!W || !x || !y) return fail(KATA_EINVAL, "null pointer argument");
    if (K <= 0 || K % 128 != 0) return fail(KATA_EINVAL, "K=%d must be a positive multiple of 128", K);
    if (N <= 0) return fail(KATA_EINVAL, "N=%d must be positive", N);
    if (T < 1 || T > 8) return fail(KATA_EINVAL, "T=%d must be 1..8", T);
    if (int rc = check_wide_x(x_dtype, K, T)) return rc;
    if (!aligned(W, 4)) return fail(KATA_EINVAL, "W must be 4-byte aligned");
    if (!aligned(x, 16)) return fail(KATA_EINVAL, "x must be 16-byte aligned");
    // T <= 2: the decode GEMV, which uses no scratch at all
    if (T <= 2 && K <= kata::gemv_max_k(T))
        return check_launch(kata::launch_gemv_ptq1(W, x, x_dtype, KATA_X_ROWS, y, K, N, T, (hipStream_t)stream),
                            "gemv ptq1 wide no-alloc (T <= 2)");
    if (x_dtype != KATA_XQ && !kata::gemv_wide_noalloc_fits(K, T))
        return fail(KATA_EINVAL, "K=%d needs a larger activation image than the %zu-byte no-allocation scratch", K,
                    kata::gemv_wide_noalloc_scratch_bytes());
    return check_launch(kata::launch_gemv_wide_noalloc(W, x, x_dtype, y, K, N, T, (hipStream_t)stream),
                        "gemv ptq1 wide no-alloc");
}

size_t kata_gemv_ptq1_wide_noalloc_scratch_bytes(void) { return kata::gemv_wide_noalloc_scratch_bytes(); }

// ------------------------------------------------------------------ Q8_0 GEMV
int kata_gemv_q8_0(const uint8_t* W, const void* x, int x_dtype, float* y, int K, int N, int T, void* stream) {
    if (!W || !x || !y) return fail(KATA_EINVAL, "null pointer argument");
    if (K <= 0 || K % 32 != 0) return fail(KATA_EINVAL, "K=%d must be a positive multiple of 32", K);
    if (N <= 0) return fail(KATA_EINVAL, "N=%d must be positive", N);
    if (T != 1 && T != 2) return fail(KATA_EINVAL, "T=%d must be 1 or 2", T);
    if (x_dtype != KATA_F32 && x_dtype != KATA_F16) return fail(KATA_EINVAL, "x_dtype=%d", x_dtype);
    if (!aligned(W, 2)) return fail(KATA_EINVAL, "W must be 2-byte aligned");
    if (!aligned(x, 16)) return fail(KATA_EINVAL, "x must be 16-byte aligned");
    return check_launch(kata::launch_gemv_q8(W, x, x_dtype, y, K, N, T, (hipStream_t)stream), "gemv q8_0");
}

int kata_gemv_q8_0_batch(int count, const uint8_t* const* W, float* const* y, const int* N, const void* x, int x_dtype,
                         int K, int T, void* stream) {
    if (count < 1 || count > kata::gemv_q8_max_mats())
        return fail(KATA_EINVAL, "count=%d must be 1..%d", count, kata::gemv_q8_max_mats());
    if (!W || !y || !N || !x) return fail(KATA_EINVAL, "null argument");
    if (K <= 0 || K % 32 != 0) return fail(KATA_EINVAL, "K=%d must be a positive multiple of 32", K);
    if (T != 1 && T != 2) return fail(KATA_EINVAL, "T=%d must be 1 or 2", T);
    if (x_dtype != KATA_F32 && x_dtype != KATA_F16) return fail(KATA_EINVAL, "x_dtype=%d", x_dtype);
    if (!aligned(x, 16)) return fail(KATA_EINVAL, "x must be 16-byte aligned");
    for (int i = 0; i < count; i++) {
        if (!W[i] || !y[i]) return fail(KATA_EINVAL, "null matrix or output %d", i);
        if (N[i] <= 0) return fail(KATA_EINVAL, "N[%d]=%d must be positive", i, N[i]);
        if (!aligned(W[i], 2)) return fail(KATA_EINVAL, "W[%d] must be 2-byte aligned", i);
    }
    return check_launch(kata::launch_gemv_q8_multi(count, W, y, N, x, x_dtype, K, T, (hipStream_t)stream),
                        "gemv q8_0 batch");
}

// ------------------------------------------------------------------ prefill
int kata_gemm_ptq1_f16(const uint16_t* A, int lda, const uint8_t* W, void* C, int c_dtype, int ldc, int M, int K,
                       int N, void* stream) {
    if (!A || !W || !C) return fail(KATA_EINVAL, "null pointer argument");
    if (M <= 0 || N <= 0) return fail(KATA_EINVAL, "M=%d N=%d must be positive", M, N);
    if (K <= 0 || K % 128 != 0) return fail(KATA_EINVAL, "K=%d must be a positive multiple of 128", K);
    if (lda < K || lda % 8 != 0) return fail(KATA_EINVAL, "lda=%d must be >= K and a multiple of 8", lda);
    if (ldc < N) return fail(KATA_EINVAL, "ldc=%d < N=%d", ldc, N);
    if (c_dtype != KATA_F32 && c_dtype != KATA_F16) return fail(KATA_EINVAL, "c_dtype=%d", c_dtype);
    if (!aligned(A, 16)) return fail(KATA_EINVAL, "A must be 16-byte aligned");
    if (!aligned(W, 2)) return fail(KATA_EINVAL, "W must be 2-byte aligned");
    return check_launch(kata::launch_gemm_f16(A, lda, W, C, c_dtype, ldc, M, K, N, (hipStream_t)stream),
                        "gemm ptq1 f16");
}

int kata_gemm_q8_0_f16(const uint16_t* A, int lda, const uint8_t* W, void* C, int c_dtype, int ldc, int M, int K,
                       int N, void* stream) {
    if (!A || !W || !C) return fail(KATA_EINVAL, "null pointer argument");
    if (M <= 0 || N <= 0) return fail(KATA_EINVAL, "M=%d N=%d must be positive", M, N);
    if (K <= 0 || K % 128 != 0) return fail(KATA_EINVAL, "K=%d must be a positive multiple of 128", K);
    if (lda < K || lda % 8 != 0) return fail(KATA_EINVAL, "lda=%d must be >= K and a multiple of 8", lda);
    if (ldc < N) return fail(KATA_EINVAL, "ldc=%d < N=%d", ldc, N);
    if (c_dtype != KATA_F32 && c_dtype != KATA_F16) return fail(KATA_EINVAL, "c_dtype=%d", c_dtype);
    if (!aligned(A, 16)) return fail(KATA_EINVAL, "A must be 16-byte aligned");
    if (!aligned(W, 4)) return fail(KATA_EINVAL, "W must be 4-byte aligned");
    return check_launch(kata::launch_gemm_q8(A, lda, W, C, c_dtype, ldc, M, K, N, (hipStream_t)stream),
                        "gemm q8_0 f16");
}

int kata_quant_rows_i8(const uint16_t* X, int8_t* Q, float* SX, int M, int K, int ldS, void* stream) {
    if (!X || !Q || !SX) return fail(KATA_EINVAL, "null pointer argument");
    if (M <= 0) return fail(KATA_EINVAL, "M=%d must be positive", M);
    if (K <= 0 || K % 128 != 0) return fail(KATA_EINVAL, "K=%d must be a positive multiple of 128", K);
    if (ldS < M) return fail(KATA_EINVAL, "ldS=%d < M=%d", ldS, M);
    if (!aligned(X, 16) || !aligned(Q, 8)) return fail(KATA_EINVAL, "X must be 16-byte and Q 8-byte aligned");
    return check_launch(kata::launch_quant_rows(X, Q, SX, M, K, ldS, (hipStream_t)stream), "quant rows");
}

int kata_gemm_ptq1_i8(const int8_t* A8, const float* SX, int ldS, const uint8_t* W, void* C, int c_dtype, int ldc,
                      int M, int K, int N, void* stream) {
    if (!A8 || !SX || !W || !C) return fail(KATA_EINVAL, "null pointer argument");
    if (M <= 0 || N <= 0) return fail(KATA_EINVAL, "M=%d N=%d must be positive", M, N);
    if (K <= 0 || K % 128 != 0) return fail(KATA_EINVAL, "K=%d must be a positive multiple of 128", K);
    if (ldS < M) return fail(KATA_EINVAL, "ldS=%d < M=%d", ldS, M);
    if (ldc < N) return fail(KATA_EINVAL, "ldc=%d < N=%d", ldc, N);
    if (c_dtype != KATA_F32 && c_dtype != KATA_F16) return fail(KATA_EINVAL, "c_dtype=%d", c_dtype);
    if (!aligned(A8, 16)) return fail(KATA_EINVAL, "A8 must be 16-byte aligned");
    if (!aligned(W, 4)) return fail(KATA_EINVAL, "W must be 4-byte aligned");
    return check_launch(kata::launch_gemm_i8(A8, SX, ldS, W, C, c_dtype, ldc, M, K, N, (hipStream_t)stream),
                        "gemm ptq1 i8");
}

int kata_expand_ptq1_f16(const uint8_t* W, uint16_t* out, int K, int N, void* stream) {
    if (!W || !out) return fail(KATA_EINVAL, "null pointer argument");
    if (N <= 0 || K <= 0 || K % 128 != 0) return fail(KATA_EINVAL, "bad shape K=%d N=%d", K, N);
    if (!aligned(W, 2) || !aligned(out, 2)) return fail(KATA_EINVAL, "misaligned argument");
    return check_launch(kata::launch_expand_f16(W, out, K, N, (hipStream_t)stream), "expand f16");
}

int kata_expand_ptq1_i8(const uint8_t* W, int8_t* T8, float* SW, int K, int N, void* stream) {
    if (!W || !T8 || !SW) return fail(KATA_EINVAL, "null pointer argument");
    if (N <= 0 || K <= 0 || K % 128 != 0) return fail(KATA_EINVAL, "bad shape K=%d N=%d", K, N);
    if (!aligned(W, 2) || !aligned(SW, 4)) return fail(KATA_EINVAL, "misaligned argument");
    return check_launch(kata::launch_expand_i8(W, T8, SW, K, N, (hipStream_t)stream), "expand i8");
}

// ------------------------------------------------------------------ matmul input transform
static size_t fwht_out_bytes(int out_dtype, int W, int M) {
    return out_dtype == KATA_XQ ? kata_gemv_xq_bytes(W, M) : (size_t)W * M * (out_dtype == KATA_F16 ? 2 : 4);
}

static int check_fwht_out(const void* out, int out_dtype, int out_layout, int W, int M) {
    if (out_dtype != KATA_F32 && out_dtype != KATA_F16 && out_dtype != KATA_XQ) return fail(KATA_EINVAL, "out_dtype=%d", out_dtype);
    if (out_dtype == KATA_XQ && (M < 1 || M > 8 || out_layout != KATA_X_ROWS || kata_gemv_xq_bytes(W, M) == 0))
        return fail(KATA_EINVAL, "the operand form takes M <= 8, KATA_X_ROWS and a GEMV-supported W (M=%d W=%d)", M, W);
    if (out_layout != KATA_X_ROWS && out_layout != KATA_X_HALF2) return fail(KATA_EINVAL, "out_layout=%d", out_layout);
    if (out_layout == KATA_X_HALF2 && (out_dtype != KATA_F16 || M != 2))
        return fail(KATA_EINVAL, "the half2 layout is fp16 with M == 2");
    if (W <= 0 || W % 1024 != 0) return fail(KATA_EINVAL, "W=%d must be a positive multiple of 1024", W);
    if (M <= 0 || M > 65535) return fail(KATA_EINVAL, "M=%d out of range", M);
    if (!aligned(out, 16)) return fail(KATA_EINVAL, "out must be 16-byte aligned");
    return KATA_OK;
}

int kata_add_rms_fwht(const float* x, const float* y, const float* gs, void* out, int out_dtype, int out_layout,
                      float* xnew, const float* gamma, void* hout, int hout_dtype, int W, int M, void* stream) {
    if (!x || !gs || !out) return fail(KATA_EINVAL, "null pointer argument");
    if (int rc = check_fwht_out(out, out_dtype, out_layout, W, M)) return rc;
    // no output may overlap an input: a workgroup re-reads its whole row while others write
    // theirs (the reference alternates two residual buffers, src/engine.cpp:136-146)
    {
        const size_t rows = (size_t)W * M * sizeof(float);
        const size_t ob = fwht_out_bytes(out_dtype, W, M);
        const size_t hb = (size_t)W * M * (hout_dtype == KATA_F16 ? 2 : 4);
        const Span ins[] = {{x, rows}, {y, rows}, {gs, (size_t)W * 4}, {gamma, (size_t)W * 4}};
        const Span outs[] = {{out, ob}, {xnew, rows}, {hout, hb}};
        for (const Span& o : outs)
            for (const Span& i : ins)
                if (overlap(o, i)) return fail(KATA_EINVAL, "an output (out, xnew or hout) overlaps an input (x, y, gs or gamma)");
        if (overlap(outs[0], outs[1]) || overlap(outs[0], outs[2]) || overlap(outs[1], outs[2]))
            return fail(KATA_EINVAL, "the outputs out, xnew and hout overlap");
    }
    if ((gamma == nullptr) != (hout == nullptr)) return fail(KATA_EINVAL, "gamma and hout go together");
    if (hout && hout_dtype != KATA_F32 && hout_dtype != KATA_F16) return fail(KATA_EINVAL, "hout_dtype=%d", hout_dtype);
    if (!aligned(x, 16) || (y && !aligned(y, 16)) || !aligned(gs, 16) || (xnew && !aligned(xnew, 16)) ||
        (gamma && !aligned(gamma, 16)) || (hout && !aligned(hout, 16)))
        return fail(KATA_EINVAL, "vectors must be 16-byte aligned");
    const int flags = (y ? 1 : 0) | (xnew ? 2 : 0) | (hout ? 4 : 0) | (hout && hout_dtype == KATA_F16 ? 8 : 0);
    return check_launch(kata::launch_norm_fwht(x, y, gs, out, out_dtype, out_layout, xnew, gamma, hout, flags, W, M, 0,
                                               (hipStream_t)stream),
                        "add_rms_fwht");
}

int kata_rms_fwht(const float* src, const float* src2, const float* gs, void* out, int out_dtype, int out_layout,
                  int W, int M, int mode, void* stream) {
    if (!src || !gs || !out) return fail(KATA_EINVAL, "null pointer argument");
    if (mode < 0 || mode > 3) return fail(KATA_EINVAL, "mode=%d", mode);
    if (mode == 1 && !src2) return fail(KATA_EINVAL, "mode 1 needs src2");
    if (mode == 2 && W != 6144) return fail(KATA_EINVAL, "mode 2 (GDN head order) needs W == 6144");
    if (int rc = check_fwht_out(out, out_dtype, out_layout, W, M)) return rc;
    {
        const size_t rows = (size_t)W * M * sizeof(float);
        const Span o{out, fwht_out_bytes(out_dtype, W, M)};
        if (overlap(o, {src, rows}) || overlap(o, {mode == 1 ? src2 : nullptr, rows}) || overlap(o, {gs, (size_t)W * 4}))
            return fail(KATA_EINVAL, "out overlaps an input (src, src2 or gs)");
    }
    if (!aligned(src, 16) || (src2 && !aligned(src2, 16)) || !aligned(gs, 16))
        return fail(KATA_EINVAL, "vectors must be 16-byte aligned");
    return check_launch(kata::launch_norm_fwht(src, mode == 1 ? src2 : nullptr, gs, out, out_dtype, out_layout, nullptr,
                                               nullptr, nullptr, 0, W, M, mode, (hipStream_t)stream),
                        "rms_fwht");
}

// ------------------------------------------------------------------ argmax
int kata_argmax(const float* x, int n, int* out, void* stream) {
    if (!x || !out) return fail(KATA_EINVAL, "null pointer argument");
    if (n <= 0) return fail(KATA_EINVAL, "n=%d must be positive", n);
    if (!aligned(x, 16) || !aligned(out, 4)) return fail(KATA_EINVAL, "x must be 16-byte aligned");
    return check_launch(kata::launch_argmax(x, n, out, (hipStream_t)stream), "argmax");
}

// ------------------------------------------------------------------ scratch lifetime
int kata_release_stream(void* stream) {
    return check_launch(kata::release_stream((hipStream_t)stream), "release stream");
}

// ------------------------------------------------------------------ measurement helpers
static int calib_wgs(int wgs) {
    if (wgs > 0) return wgs;
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 256;
    return n > 0 ? n : 256;
}

int kata_calib_empty(uint32_t* out, int wgs, void* stream) {
    if (!out) return fail(KATA_EINVAL, "null pointer argument");
    if (wgs > 65536) return fail(KATA_EINVAL, "wgs=%d", wgs);
    return check_launch(kata::launch_calib_empty(out, calib_wgs(wgs), (hipStream_t)stream), "calib_empty");
}

int kata_calib_read(const void* p, size_t bytes, uint32_t* out, int wgs, void* stream) {
    if (!p || !out) return fail(KATA_EINVAL, "null pointer argument");
    if (bytes == 0 || bytes > 0x7fffffffu) return fail(KATA_EINVAL, "bytes=%zu must be in 1..2^31-1", bytes);
    if (!aligned(p, 16)) return fail(KATA_EINVAL, "p must be 16-byte aligned");
    if (wgs > 65536) return fail(KATA_EINVAL, "wgs=%d", wgs);
    return check_launch(kata::launch_calib_read((const uint8_t*)p, (uint32_t)bytes, out, calib_wgs(wgs), (hipStream_t)stream),
                        "calib_read");
}

int kata_calib_read_cfg(const void* p, size_t bytes, uint32_t* out, int threads, int wgs, int inflight, int nt,
                        void* stream) {
    if (!p || !out) return fail(KATA_EINVAL, "null pointer argument");
    if (bytes == 0 || bytes > 0x7fffffffu) return fail(KATA_EINVAL, "bytes=%zu must be in 1..2^31-1", bytes);
    if (!aligned(p, 16)) return fail(KATA_EINVAL, "p must be 16-byte aligned");
    if (threads != 256 && threads != 512 && threads != 1024) return fail(KATA_EINVAL, "threads=%d", threads);
    if (wgs < 1 || wgs > 65536) return fail(KATA_EINVAL, "wgs=%d", wgs);
    if (inflight != 2 && inflight != 4 && inflight != 8 && inflight != 16) return fail(KATA_EINVAL, "inflight=%d", inflight);
    return check_launch(kata::launch_calib_read_cfg((const uint8_t*)p, (uint32_t)bytes, out, threads, wgs, inflight, nt != 0,
                                                    (hipStream_t)stream),
                        "calib_read_cfg");
}

int kata_calib_read_ptq1(const void* W, int K, int N, uint32_t* out, void* stream) {
    if (!W || !out) return fail(KATA_EINVAL, "null pointer argument");
    if (K <= 0 || K % kata::kGroup || N <= 0) return fail(KATA_EINVAL, "K=%d (a positive multiple of 128), N=%d", K, N);
    if ((long long)N * (K / kata::kGroup) * kata::kBlockBytes > 0x7fffffffLL)
        return fail(KATA_EINVAL, "N*K matrix of %lld bytes exceeds 2^31-1", (long long)N * (K / kata::kGroup) * kata::kBlockBytes);
    if (!aligned(W, 16)) return fail(KATA_EINVAL, "W must be 16-byte aligned");
    return check_launch(kata::launch_calib_read_ptq1((const uint8_t*)W, K, N, out, calib_wgs(0), (hipStream_t)stream),
                        "calib_read_ptq1");
}

int kata_calib_read_peak(const void* p, size_t bytes, uint32_t* out, void* stream) {
    if (!p || !out) return fail(KATA_EINVAL, "null pointer argument");
    if (bytes == 0 || bytes > 0x7fffffffu) return fail(KATA_EINVAL, "bytes=%zu must be in 1..2^31-1", bytes);
    if (!aligned(p, 16)) return fail(KATA_EINVAL, "p must be 16-byte aligned");
    return check_launch(kata::launch_calib_read_peak((const uint8_t*)p, (uint32_t)bytes, out, calib_wgs(0), (hipStream_t)stream),
                        "calib_read_peak");
}

// ------------------------------------------------------------------ host packers
// Byte encoding of the quantiser (docs/reference/prism_ptq1_0_quant_dequant.c:20-46):
// stages of 16 and 8 bytes carry 5 digits each (most significant first, element
// m + n*c of the stage), the two qh bytes carry 4 digits then a zero digit; a 5-digit
// base-3 number q is stored as ceil(q*256/243).
}  // extern "C"

namespace {
inline uint8_t enc5(uint32_t q) { return (uint8_t)((q * 256u + 242u) / 243u); }

template <typename DigitOf>
void encode_block(uint8_t* blk, DigitOf digit_of) {
    int base = 0, j = 0;
    for (int c : {16, 8}) {
        for (int m = 0; m < c; m++) {
            uint32_t q = 0;
            for (int n = 0; n < 5; n++) q = q * 3u + digit_of(base + m + n * c);
            blk[j + m] = enc5(q);
        }
        base += 5 * c;
        j += c;
    }
    for (int h = 0; h < 2; h++) {
        uint32_t q = 0;
        for (int n = 0; n < 4; n++) q = q * 3u + digit_of(base + h + n * 2);
        blk[24 + h] = enc5(q * 3u);
    }
}
}  // namespace

extern "C" {

int kata_quantize_ptq1_0(const float* x, uint8_t* out, int64_t nrow, int64_t k) {
    if (!x || !out) return fail(KATA_EINVAL, "null pointer argument");
    if (nrow < 0 || k <= 0 || k % 128 != 0) return fail(KATA_EINVAL, "bad shape");
    const int64_t nb = k / 128;
    for (int64_t i = 0; i < nrow * nb; i++) {
        const float* xb = x + i * 128;
        uint8_t* blk = out + i * 28;
        float amax = 0.0f;
        for (int e = 0; e < 128; e++) amax = std::fmax(amax, std::fabs(xb[e]));
        const float id = amax != 0.0f ? 1.0f / amax : 0.0f;
        encode_block(blk, [&](int e) { return (uint32_t)(std::lround(xb[e] * id) + 1); });
        const _Float16 dh = (_Float16)amax;
        uint16_t bits;
        memcpy(&bits, &dh, 2);
        blk[26] = (uint8_t)(bits & 0xff);
        blk[27] = (uint8_t)(bits >> 8);
    }
    g_err.clear();
    return KATA_OK;
}

int kata_pack_ptq1_0(const int8_t* trits, const uint16_t* scales, uint8_t* out, int64_t nrow, int64_t k) {
    if (!trits || !scales || !out) return fail(KATA_EINVAL, "null pointer argument");
    if (nrow < 0 || k <= 0 || k % 128 != 0) return fail(KATA_EINVAL, "bad shape");
    const int64_t nb = k / 128;
    for (int64_t i = 0; i < nrow * nb; i++) {
        const int8_t* tb = trits + i * 128;
        for (int e = 0; e < 128; e++)
            if (tb[e] < -1 || tb[e] > 1) return fail(KATA_EINVAL, "trit out of range at %lld", (long long)(i * 128 + e));
        uint8_t* blk = out + i * 28;
        encode_block(blk, [&](int e) { return (uint32_t)(tb[e] + 1); });
        blk[26] = (uint8_t)(scales[i] & 0xff);
        blk[27] = (uint8_t)(scales[i] >> 8);
    }
    g_err.clear();
    return KATA_OK;
}

// ------------------------------------------------------------------ dispatcher
static const char* const kI8Names[] = {"qkv", "z", "ssmout", "wq", "wk", "wv", "wo", "gate", "up", "down"};

static uint32_t i8_bit(const char* name, size_t len) {
    for (uint32_t i = 0; i < 10; i++)
        if (strlen(kI8Names[i]) == len && strncmp(kI8Names[i], name, len) == 0) return 1u << i;
    return 0;
}

struct kata_dispatch {
    const uint8_t* wbase;
    uint32_t i8_mask;
};

kata_dispatch* kata_dispatch_create(const uint8_t* wbase) {
    if (!wbase) {
        fail(KATA_EINVAL, "null weight base");
        return nullptr;
    }
    return new kata_dispatch{wbase, 0u};
}

void kata_dispatch_destroy(kata_dispatch* d) { delete d; }

int kata_dispatch_set_i8(kata_dispatch* d, const char* spec) {
    if (!d || !spec) return fail(KATA_EINVAL, "null argument");
    uint32_t m = 0;
    const std::string s(spec);
    if (s == "all") {
        m = (1u << 10) - 1;
    } else if (s == "ffn") {
        m = i8_bit("gate", 4) | i8_bit("up", 2);
    } else if (!s.empty() && s != "none") {
        size_t p = 0;
        while (p <= s.size()) {
            size_t q = s.find(',', p);
            if (q == std::string::npos) q = s.size();
            const uint32_t b = i8_bit(s.c_str() + p, q - p);
            if (!b) return fail(KATA_EINVAL, "unknown matrix name in int8 spec '%s'", spec);
            m |= b;
            p = q + 1;
        }
    }
    d->i8_mask = m;
    g_err.clear();
    return KATA_OK;
}

int kata_dispatch_i8(const kata_dispatch* d, const char* name) {
    if (!d || !name) return 0;
    return (d->i8_mask & i8_bit(name, strlen(name))) != 0;
}

uint32_t kata_dispatch_i8_mask(const kata_dispatch* d) { return d ? d->i8_mask : 0u; }

int kata_dispatch_gemv(kata_dispatch* d, uint64_t wOff, const float* x, float* y, int K, int N, void* stream) {
    if (!d) return fail(KATA_EINVAL, "null dispatcher");
    return kata_gemv_ptq1(d->wbase + wOff, x, KATA_F32, KATA_X_ROWS, y, K, N, 1, stream);
}

int kata_dispatch_gemv_q8(kata_dispatch* d, int count, const uint64_t* offs, const void* x, int x_dtype,
                          float* const* outs, const int* N, int K, int T, void* stream) {
    if (!d || !offs) return fail(KATA_EINVAL, "null argument");
    if (count < 1 || count > kata::gemv_q8_max_mats())
        return fail(KATA_EINVAL, "count=%d must be 1..%d", count, kata::gemv_q8_max_mats());
    const uint8_t* W[4];
    for (int i = 0; i < count; i++) W[i] = d->wbase + offs[i];
    return kata_gemv_q8_0_batch(count, W, outs, N, x, x_dtype, K, T, stream);
}

int kata_dispatch_prefill(kata_dispatch* d, uint64_t wOff, const uint16_t* A, float* C, int M, int K, int N,
                          const char* name, int8_t* A8, float* SX, int ldS, void* stream) {
    if (!d || !name) return fail(KATA_EINVAL, "null argument");
    const uint8_t* W = d->wbase + wOff;
    if (kata_dispatch_i8(d, name)) {
        if (!A8 || !SX) return fail(KATA_EINVAL, "int8 path for '%s' needs A8/SX work buffers", name);
        int rc = kata_quant_rows_i8(A, A8, SX, M, K, ldS, stream);
        if (rc) return rc;
        return kata_gemm_ptq1_i8(A8, SX, ldS, W, C, KATA_F32, N, M, K, N, stream);
    }
    return kata_gemm_ptq1_f16(A, K, W, C, KATA_F32, N, M, K, N, stream);
}


// ------------------------------------------------------------------ layer-level: the FFN sublayer
// Engine::step's FFN (src/engine.cpp:176-182): h = H(rmsnorm(x + y) * gs_in) (the residual
// x + y is kept in xnew), g = W_gate h, u = W_up h (one batched launch), t = H(silu(g) u *
// gs_down), out = W_down t.  work: H + 3F floats; h and t are held in the GEMV's operand form
// (written by the transforms, fewer bytes than the floats).
int kata_dispatch_ffn_decode(kata_dispatch* d, uint64_t offGate, uint64_t offUp, uint64_t offDown, const float* x,
                             const float* y, float* xnew, const float* gs_in, const float* gs_down, float* work,
                             float* out, int H, int F, void* stream) {
    if (!d || !x || !gs_in || !gs_down || !work || !out) return fail(KATA_EINVAL, "null argument");
    if (H % 1024 != 0 || F % 1024 != 0 || H <= 0 || F <= 0) return fail(KATA_EINVAL, "H=%d F=%d must be multiples of 1024", H, F);
    float* h = work;
    float* g = work + H;
    float* u = g + F;
    float* t = u + F;
    int rc = kata_add_rms_fwht(x, y, gs_in, h, KATA_XQ, KATA_X_ROWS, xnew, nullptr, nullptr, 0, H, 1, stream);
    if (rc) return rc;
    const uint8_t* Wg[2] = {d->wbase + offGate, d->wbase + offUp};
    float* Yg[2] = {g, u};
    const int Ng[2] = {F, F};
    if ((rc = kata_gemv_ptq1_batch(2, Wg, Yg, Ng, h, KATA_XQ, KATA_X_ROWS, H, 1, stream))) return rc;
    if ((rc = kata_rms_fwht(g, u, gs_down, t, KATA_XQ, KATA_X_ROWS, F, 1, 1, stream))) return rc;
    return kata_gemv_ptq1(d->wbase + offDown, t, KATA_XQ, KATA_X_ROWS, out, F, H, 1, stream);
}

// The same sublayer for M prefill rows (src/engine.cpp:247-300): the GEMMs take fp16 rows,
// gate / up / down each on the fp16 exact or the int8 path per the dispatcher's selection.
// work: fp32 2 M F (g, u), then fp16 M H (h) and M F (t); with an int8 matrix also int8
// M max(H, F) and fp32 (max(H, F) / 128) M (its quantised rows and scales).  out fp32 [M][H].
int kata_dispatch_ffn_prefill(kata_dispatch* d, uint64_t offGate, uint64_t offUp, uint64_t offDown, const float* x,
                              const float* y, float* xnew, const float* gs_in, const float* gs_down, void* work,
                              float* out, int H, int F, int M, void* stream) {
    if (!d || !x || !gs_in || !gs_down || !work || !out) return fail(KATA_EINVAL, "null argument");
    if (H % 1024 != 0 || F % 1024 != 0 || H <= 0 || F <= 0 || M <= 0)
        return fail(KATA_EINVAL, "H=%d F=%d must be multiples of 1024, M=%d positive", H, F, M);
    float* g = (float*)work;
    float* u = g + (size_t)M * F;
    uint16_t* h = (uint16_t*)(u + (size_t)M * F);
    uint16_t* t = h + (size_t)M * H;
    const size_t kmax = (size_t)std::max(H, F);
    int8_t* A8 = (int8_t*)(t + (size_t)M * F);
    float* SX = (float*)(((uintptr_t)(A8 + (size_t)M * kmax) + 15) & ~(uintptr_t)15);
    int rc = kata_add_rms_fwht(x, y, gs_in, h, KATA_F16, KATA_X_ROWS, xnew, nullptr, nullptr, 0, H, M, stream);
    if (rc) return rc;
    if ((rc = kata_dispatch_prefill(d, offGate, h, g, M, H, F, "gate", A8, SX, M, stream))) return rc;
    if ((rc = kata_dispatch_prefill(d, offUp, h, u, M, H, F, "up", A8, SX, M, stream))) return rc;
    if ((rc = kata_rms_fwht(g, u, gs_down, t, KATA_F16, KATA_X_ROWS, F, M, 1, stream))) return rc;
    return kata_dispatch_prefill(d, offDown, t, out, M, F, H, "down", A8, SX, M, stream);
}

// The sublayer for T <= 8 verification tokens (Engine::verifyWide's FFN, src/engine.cpp:
// 627-629): the transforms write the GEMV operand form of the T token rows (h, t), gate and
// up run as one batched launch.  work: h (kata_gemv_xq_bytes(H, T), 16-byte aligned), fp32
// g, u [T][F], t (kata_gemv_xq_bytes(F, T)).
int kata_dispatch_ffn_verify(kata_dispatch* d, uint64_t offGate, uint64_t offUp, uint64_t offDown, const float* x,
                             const float* y, float* xnew, const float* gs_in, const float* gs_down, void* work,
                             float* out, int H, int F, int T, void* stream) {
    if (!d || !x || !gs_in || !gs_down || !work || !out) return fail(KATA_EINVAL, "null argument");
    if (H % 1024 != 0 || F % 1024 != 0 || H <= 0 || F <= 0 || T < 1 || T > 8)
        return fail(KATA_EINVAL, "H=%d F=%d must be multiples of 1024, T=%d in 1..8", H, F, T);
    const size_t hb = align16(kata_gemv_xq_bytes(H, T));
    if (hb == 0 || kata_gemv_xq_bytes(F, T) == 0) return fail(KATA_EINVAL, "H=%d F=%d T=%d: no operand form", H, F, T);
    uint8_t* h = (uint8_t*)work;
    float* g = (float*)(h + hb);
    float* u = g + (size_t)T * F;
    uint8_t* t = (uint8_t*)(u + (size_t)T * F);
    int rc = kata_add_rms_fwht(x, y, gs_in, h, KATA_XQ, KATA_X_ROWS, xnew, nullptr, nullptr, 0, H, T, stream);
    if (rc) return rc;
    const uint8_t* Wgu[2] = {d->wbase + offGate, d->wbase + offUp};
    float* ygu[2] = {g, u};
    const int Ngu[2] = {F, F};
    if ((rc = kata_gemv_ptq1_wide_batch(2, Wgu, ygu, Ngu, h, KATA_XQ, H, T, stream))) return rc;
    if ((rc = kata_rms_fwht(g, u, gs_down, t, KATA_XQ, KATA_X_ROWS, F, T, 1, stream))) return rc;
    return kata_gemv_ptq1_wide(d->wbase + offDown, t, KATA_XQ, out, F, H, T, stream);
}

// ------------------------------------------------------------------ sublayer halves
// Work layout of kata_dispatch_in / _out for a transform width K and M rows: decode and
// verify the GEMV's operand form of the M rows (kata_gemv_xq_bytes(K, M); decode keeps the
// 4 K bytes of fp32 rows, verify at least 2 M K); prefill fp16 [M][K], then int8 [M][K] and fp32 [K/128][M] for the
// int8 path's quantised rows and scales (16-byte aligned parts).

size_t kata_dispatch_work_bytes(int form, int K, int M) {
    if (K <= 0 || M <= 0) return 0;
    const size_t k = (size_t)K, m = (size_t)M;
    switch (form) {
        case KATA_FORM_DECODE: return align16(4 * k);
        case KATA_FORM_VERIFY: return std::max(align16(2 * m * k), align16(kata_gemv_xq_bytes(K, M)));
        case KATA_FORM_PREFILL: return align16(2 * m * k) + align16(m * k) + align16(4 * (k / 128) * m);
        default: return 0;
    }
}

namespace {
struct HalfWork {
    void* act;      // the transformed activation: the GEMV operand form (decode, verify) or fp16 rows
    int8_t* A8;     // prefill: quantised rows
    float* SX;      // prefill: their group scales [K/128][M]
};
HalfWork half_work(void* work, int K, int M) {
    uint8_t* b = (uint8_t*)work;
    const size_t k = (size_t)K, m = (size_t)M;
    HalfWork w{b, (int8_t*)(b + align16(2 * m * k)), nullptr};
    w.SX = (float*)((uint8_t*)w.A8 + align16(m * k));
    return w;
}
int check_form(int form, int M, int K) {
    if (form != KATA_FORM_DECODE && form != KATA_FORM_PREFILL && form != KATA_FORM_VERIFY)
        return fail(KATA_EINVAL, "form=%d", form);
    if (form == KATA_FORM_DECODE && M != 1) return fail(KATA_EINVAL, "the decode form takes M == 1 (M=%d)", M);
    if (form == KATA_FORM_VERIFY && (M < 1 || M > 8)) return fail(KATA_EINVAL, "the verify form takes 1..8 tokens (M=%d)", M);
    if (M < 1) return fail(KATA_EINVAL, "M=%d must be positive", M);
    if (K <= 0 || K % 1024 != 0) return fail(KATA_EINVAL, "K=%d must be a positive multiple of 1024", K);
    return KATA_OK;
}
// one matmul of the transformed activation (K wide, M rows) with the named matrix
int half_matmul(kata_dispatch* d, int form, uint64_t off, const char* name, const HalfWork& w, float* out, int K,
                int N, int M, bool quantised, hipStream_t st) {
    const uint8_t* Wm = d->wbase + off;
    switch (form) {
        case KATA_FORM_DECODE:
            return kata_gemv_ptq1(Wm, w.act, KATA_XQ, KATA_X_ROWS, out, K, N, 1, st);
        case KATA_FORM_VERIFY:
            return kata_gemv_ptq1_wide(Wm, w.act, KATA_XQ, out, K, N, M, st);
        default:
            if (kata_dispatch_i8(d, name)) {
                int rc = quantised ? KATA_OK : kata_quant_rows_i8((const uint16_t*)w.act, w.A8, w.SX, M, K, M, st);
                return rc ? rc : kata_gemm_ptq1_i8(w.A8, w.SX, M, Wm, out, KATA_F32, N, M, K, N, st);
            }
            return kata_gemm_ptq1_f16((const uint16_t*)w.act, K, Wm, out, KATA_F32, N, M, K, N, st);
    }
}
}  // namespace

int kata_dispatch_in(kata_dispatch* d, int form, int count, const uint64_t* offs, const int* N,
                     const char* const* names, float* const* outs, const float* x, const float* y, float* xnew,
                     const float* gs, const float* gamma, void* hout, int hout_dtype, void* work, int H, int M,
                     void* stream) {
    if (!d || !offs || !N || !names || !outs || !x || !gs || !work) return fail(KATA_EINVAL, "null argument");
    if (count < 1 || count > 4) return fail(KATA_EINVAL, "count=%d must be 1..4", count);
    if (int rc = check_form(form, M, H)) return rc;
    for (int i = 0; i < count; i++) {
        if (!outs[i] || N[i] <= 0) return fail(KATA_EINVAL, "matrix %d: null output or N=%d", i, N[i]);
        if (!names[i] || !i8_bit(names[i], strlen(names[i])))
            return fail(KATA_EINVAL, "matrix %d: unknown name '%s'", i, names[i] ? names[i] : "(null)");
    }
    const hipStream_t st = (hipStream_t)stream;
    const HalfWork w = half_work(work, H, M);
    const int act_dt = form == KATA_FORM_PREFILL ? KATA_F16 : KATA_XQ;
    int rc = kata_add_rms_fwht(x, y, gs, w.act, act_dt, KATA_X_ROWS, xnew, gamma, hout, hout_dtype, H, M, stream);
    if (rc) return rc;
    if (form != KATA_FORM_PREFILL) {                 // one launch for all matrices that read h
        const uint8_t* Wm[4];
        for (int i = 0; i < count; i++) Wm[i] = d->wbase + offs[i];
        if (form == KATA_FORM_DECODE) return kata_gemv_ptq1_batch(count, Wm, outs, N, w.act, KATA_XQ, KATA_X_ROWS, H, 1, stream);
        return kata_gemv_ptq1_wide_batch(count, Wm, outs, N, w.act, KATA_XQ, H, M, stream);
    }
    bool quantised = false;                          // prefill: quantise h once for its int8 matrices
    for (int i = 0; i < count; i++) {
        if ((rc = half_matmul(d, form, offs[i], names[i], w, outs[i], H, N[i], M, quantised, st))) return rc;
        quantised = quantised || (form == KATA_FORM_PREFILL && kata_dispatch_i8(d, names[i]));
    }
    return KATA_OK;
}

int kata_dispatch_out(kata_dispatch* d, int form, uint64_t off, const char* name, const float* src, const float* src2,
                      int mode, const float* gs, void* work, float* out, int W, int H, int M, void* stream) {
    if (!d || !name || !src || !gs || !work || !out) return fail(KATA_EINVAL, "null argument");
    if (!i8_bit(name, strlen(name))) return fail(KATA_EINVAL, "unknown matrix name '%s'", name);
    if (mode < 1 || mode > 3) return fail(KATA_EINVAL, "mode=%d must be 1 (SwiGLU), 2 (GDN order) or 3 (plain)", mode);
    if (int rc = check_form(form, M, W)) return rc;
    if (H <= 0) return fail(KATA_EINVAL, "H=%d must be positive", H);
    const HalfWork w = half_work(work, W, M);
    int rc = kata_rms_fwht(src, src2, gs, w.act, form == KATA_FORM_PREFILL ? KATA_F16 : KATA_XQ, KATA_X_ROWS, W, M, mode,
                           stream);
    if (rc) return rc;
    return half_matmul(d, form, off, name, w, out, W, H, M, false, (hipStream_t)stream);
}

size_t kata_ffn_verify_work_bytes(int H, int F, int T) {
    return align16(kata_gemv_xq_bytes(H, T)) + (size_t)T * F * 8 + kata_gemv_xq_bytes(F, T);
}

size_t kata_ffn_prefill_work_bytes(int H, int F, int M) {
    const size_t kmax = (size_t)std::max(H, F);
    return (size_t)M * F * 8 + (size_t)M * H * 2 + (size_t)M * F * 2 + (size_t)M * kmax + 16 + kmax / 128 * M * 4;
}
}  // extern "C"
