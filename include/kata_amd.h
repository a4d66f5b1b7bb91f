/*
 * kata_amd.h — C ABI of the MI355X (gfx950) ternary-matmul library.
 *
 * Drop-in for the matmul dispatch surface of the reference engine (src/engine.cpp,
 * src/engine.h).  Every entry point:
 *   - is stream ordered on the caller's HIP stream (`stream` is a hipStream_t; NULL means
 *     the default stream) and returns without synchronising;
 *   - takes device pointers only (except the host packers, marked HOST);
 *   - returns 0 on success or a negative KATA_E* code; kata_last_error() then describes
 *     the failure for the calling thread.  No entry point calls exit().
 * Weights are read-only device bytes in the native GGUF block layout (PTQ1_0: 28-byte
 * blocks, Q8_0: 34-byte blocks), row-major [N rows][K/group blocks], at any 4-byte
 * aligned base; no weight copy or dequantised stage is ever made.
 */
#ifndef KATA_AMD_H
#define KATA_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KATA_OK 0
#define KATA_EINVAL (-1)  /* bad shape, alignment, dtype or layout argument */
#define KATA_ELAUNCH (-2) /* a HIP runtime call or kernel launch failed */

/* activation element types */
#define KATA_F32 0
#define KATA_F16 1
/* the decode GEMV's operand form of T (1, 2) activation rows: kata_gemv_xq_bytes(K, T) bytes,
 * written by kata_gemv_prepare_x or by the input transforms (kata_add_rms_fwht,
 * kata_rms_fwht with M == T); an x_dtype of kata_gemv_ptq1 / _batch and an out_dtype of the
 * transforms */
#define KATA_XQ 2
/* activation layouts for the GEMVs */
#define KATA_X_ROWS 0   /* x[T][K], one row per token */
#define KATA_X_HALF2 1  /* x[K][2] fp16, the two tokens interleaved (T == 2 only) */

/* Description of the last failure on the calling thread ("" if none). */
const char* kata_last_error(void);

/* Library version string. */
const char* kata_version(void);

/* ---------------------------------------------------------------- decode GEMVs -------
 * y[t][n] = sum_b d[n,b] * sum_e trit[n,b,e] * x[t][128b+e], fp32 out, t < T, T in {1,2}.
 * K % 128 == 0, K <= kata_gemv_ptq1_max_k(T), N >= 1.  x is 16-byte aligned; y is [T][N]
 * fp32.  One kernel launch, no work buffer: fp16 / fp32 rows are quantised by every
 * workgroup; x_dtype KATA_XQ (x_layout KATA_X_ROWS) takes the operand form of the T rows,
 * quantised once by its producer, with the same y bit for bit.
 * Replaces Engine::dGemvPtq1 (src/engine.cpp:97-101, src/engine.h:155; kernel
 * k_gemv_v1_nr4_sg4, shaders/gemv_fast.metal:9-50) for T = 1, and the `gv` lambda of
 * Engine::verify2 (src/engine.cpp:440-443; k_gemv_lut2_nr4_sg4, shaders/mtp.metal:164-205,
 * or k_gemv_v1h_t2, mtp.metal:66-103) for T = 2.  x_layout KATA_X_HALF2 accepts the
 * interleaved activations k_gemv_lut2 reads (k_ilv2, shaders/mtp.metal:222-224). */
int kata_gemv_ptq1(const uint8_t* W, const void* x, int x_dtype, int x_layout, float* y,
                   int K, int N, int T, void* stream);

/* Largest K the PTQ1_0 GEMV accepts for T tokens (its activation image lives in LDS). */
int kata_gemv_ptq1_max_k(int T);

/* The operand form (KATA_XQ) of T in {1, 2} activation rows for the decode GEMV: each
 * 128-block and token quantised to the 16-bit block fixed point the GEMV computes in (scale
 * amax / 32639, q = rint(x * 32639 / amax) as two int8 limbs), laid out as the GEMV's
 * matrix-core operand.  Writing it once lets every workgroup of a GEMV copy it instead of
 * quantising x itself; kata_gemv_ptq1(W, xq, KATA_XQ, KATA_X_ROWS, ...) gives the same y bit
 * for bit as kata_gemv_ptq1(W, x, x_dtype, x_layout, ...).  x as for kata_gemv_ptq1, K % 128
 * == 0, xq 16-byte aligned, kata_gemv_xq_bytes(K, T) bytes (0 for an unsupported K or T:
 * K beyond kata_gemv_ptq1_max_k(T) or an operand over 128 KB).  No counterpart function in
 * the reference, whose GEMVs read the float activation directly (shaders/gemv_fast.metal:
 * 9-50); it is the producer side of Engine::dGemvPtq1's input (src/engine.cpp:97-101). */
size_t kata_gemv_xq_bytes(int K, int T);
int kata_gemv_prepare_x(const void* x, int x_dtype, int x_layout, int K, int T, void* xq, void* stream);

/* The same GEMV for 1..4 matrices that multiply one activation (same K), in one launch:
 * y[i][t][n] for W[i] with N[i] rows.  W, y and N are HOST arrays of count device
 * pointers / row counts.  The activation is read and quantised once per launch instead
 * of once per matrix.  No counterpart function in the reference, which issues one
 * dGemvPtq1 per matrix; this batches the calls of Engine::step that share an input —
 * qkv + z, q + k + v, gate + up (src/engine.cpp:150-191) — and the matching `gv` calls of
 * verify2 (src/engine.cpp:458-492). */
int kata_gemv_ptq1_batch(int count, const uint8_t* const* W, float* const* y, const int* N,
                         const void* x, int x_dtype, int x_layout, int K, int T, void* stream);

/* Wide verification GEMV: the same y[t][n] for T in 1..8 token rows, x [T][K] fp16 or fp32
 * (16-byte aligned), y [T][N] fp32, any K % 128 == 0, W 4-byte aligned.  T >= 3: a prep
 * launch quantises the token rows once (same 16-bit block fixed point as above) into an
 * activation image held in a buffer of the calling (device, stream), allocated on that
 * stream's first such call (which must not be captured; calls on one stream are ordered,
 * calls on different streams use their own buffers), then one launch reads every weight
 * byte once for all T rows.  T <= 2 runs the decode GEMV above (same result as
 * kata_gemv_ptq1 with these rows, no buffer).  x_dtype KATA_XQ takes the operand form of
 * the T rows (kata_gemv_prepare_x, or an input transform with out_dtype KATA_XQ): no prep
 * launch, no buffer, the same y bit for bit.
 * Replaces Engine::dWide / xWideGemv (src/engine.cpp:542-556, src/engine.h:109,140; kernel
 * k_wide_m16_n16_k128_g4, shaders/wide.metal:41-99, whose x is fp16 rows padded to 16). */
int kata_gemv_ptq1_wide(const uint8_t* W, const void* x, int x_dtype, float* y, int K, int N, int T,
                        void* stream);

/* The wide verification GEMV for 1..4 matrices that multiply the same token rows (same K),
 * in one launch after one quantisation of the rows: y[i][t][n] for W[i] with N[i] rows (W,
 * y and N are HOST arrays of count device pointers / row counts).  Results equal
 * kata_gemv_ptq1_wide's per matrix bit for bit.  No counterpart function in the reference,
 * which issues one dWide per matrix; this batches verifyWide's gate + up
 * (src/engine.cpp:627-629) and the matrices that read one transformed activation in the
 * wide verification of the attention and GDN sublayers. */
int kata_gemv_ptq1_wide_batch(int count, const uint8_t* const* W, float* const* y, const int* N,
                              const void* x, int x_dtype, int K, int T, void* stream);

/* The same wide verification GEMV, allocating nothing: no counterpart in the reference; for
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc).  Same arguments and results as kata_gemv_ptq1_wide (bit
 * for bit); the activation image goes to a fixed per-device array of
 * kata_gemv_ptq1_wide_noalloc_scratch_bytes() bytes (4 MiB) held by each device the library
 * runs on until the process ends, instead of the stream's buffer.  Rejects (KATA_EINVAL) a K
 * whose image would not fit it (K beyond 258 048: 2080 bytes per 128 weights of a row).
 * Calls that overlap in time on one device share the array and race. */
int kata_gemv_ptq1_wide_noalloc(const uint8_t* W, const void* x, int x_dtype, float* y, int K, int N, int T,
                                void* stream);
size_t kata_gemv_ptq1_wide_noalloc_scratch_bytes(void);

/* Q8_0 GEMV for the MTP head: y[t][n] = sum_b d[n,b] * sum_i q[n,b,i] * x[t][32b+i].
 * K % 32 == 0, T in {1,2}, x [T][K] fp32 or fp16 (16-byte aligned), y [T][N] fp32.
 * W is 2-byte aligned (the block layout's granularity).
 * Replaces the `gq` lambda of Engine::mtpRows (src/engine.cpp:351; k_gemv_q8_t1/_t2,
 * shaders/mtp.metal:5-22). */
int kata_gemv_q8_0(const uint8_t* W, const void* x, int x_dtype, float* y, int K, int N, int T,
                   void* stream);

/* The Q8_0 GEMV for 1..4 matrices that multiply one activation (same K), in one launch:
 * y[i] [T][N[i]] for W[i] (W, y and N are HOST arrays of count device pointers / row
 * counts); each matrix's results equal kata_gemv_q8_0's bit for bit.  No counterpart
 * function in the reference, which issues one `gq` per matrix; this batches the calls of
 * Engine::mtpRows that share an input: wq + wk + wv and gate + up (src/engine.cpp:361,369). */
int kata_gemv_q8_0_batch(int count, const uint8_t* const* W, float* const* y, const int* N, const void* x,
                         int x_dtype, int K, int T, void* stream);

/* ---------------------------------------------------------------- prefill ------------
 * Exact fp16 prefill GEMM with the ternary decode fused into the LDS tile load:
 * C[m][n] = sum_k A[m][k] * half(trit[n][k] * d[n][k/128]), fp32 accumulation.
 * A is fp16 [M][lda] (lda >= K), C is [M][ldc] of c_dtype (KATA_F32 or KATA_F16).
 * K % 128 == 0; any M >= 1, N >= 1.
 * The K-pieces of the last round of tiles use a workspace of the calling (device, stream)
 * (at most one fp32 256x128 tile per CU), allocated on the first call on that stream that
 * needs it and kept until kata_release_stream; a call that needs a larger buffer than the
 * stream holds must not be captured, and the outgrown buffer stays allocated (graphs captured
 * earlier may still use it).  Calls on
 * different streams use different workspaces; calls on one stream are ordered by it.  The
 * entry points that use it: kata_gemm_ptq1_f16, kata_gemm_q8_0_f16, kata_gemm_ptq1_i8 and
 * the dispatcher's prefill calls (kata_dispatch_prefill, kata_dispatch_ffn_prefill, the
 * prefill forms of kata_dispatch_in / kata_dispatch_out).
 * Replaces Engine::dExpandGemm's fp16 path (src/engine.cpp:208-219: k_expand_ptq1_v2 into
 * a 178 MB stage, then Engine::dGemm / k_gemm_f16, shaders/prefill.metal:31-41). */
int kata_gemm_ptq1_f16(const uint16_t* A, int lda, const uint8_t* W, void* C, int c_dtype, int ldc,
                       int M, int K, int N, void* stream);

/* The same exact fp16 GEMM over a Q8_0 matrix (34-byte blocks: fp16 d, 32 int8 q), decode
 * fused: C[m][n] = sum_k A[m][k] * half(d[n][k/32] * q[n][k]) (half() rounds to nearest
 * even), fp32 accumulation; K % 128 == 0, W 4-byte aligned, same A / C / workspace rules.
 * Replaces the MTP K/V catch-up's k_expand_q8 + Engine::dGemm (src/engine.cpp:392-401,
 * shaders/mtp.metal:24-33): eh_proj 10240 -> 5120, wk / wv 5120 -> 1024. */
int kata_gemm_q8_0_f16(const uint16_t* A, int lda, const uint8_t* W, void* C, int c_dtype, int ldc,
                       int M, int K, int N, void* stream);

/* Activation quantisation for the int8 prefill path: per (token m, 128-group g)
 * scale = amax > 0 ? amax/127 : 1, Q = clamp(rint(x/scale), +-127), SX[g*ldS + m] = scale.
 * X fp16 [M][K] (16-byte aligned), Q int8 [M][K] (8-byte aligned), SX fp32 [K/128][ldS],
 * ldS >= M.
 * Replaces k_quant_rows (shaders/prefill.metal:369-381; dispatched src/engine.cpp:230). */
int kata_quant_rows_i8(const uint16_t* X, int8_t* Q, float* SX, int M, int K, int ldS, void* stream);

/* int8 prefill GEMM with the ternary decode fused: per 128-group the exact int32 sum
 * I = sum_k A8[m][k] * trit[n][k], then C[m][n] += float(I) * (d[n][g] * SX[g*ldS+m]).
 * C is [M][ldc] of c_dtype.  K % 128 == 0.
 * Replaces Engine::dExpandGemm's int8 path (src/engine.cpp:210-213: k_expand_i8_v2 +
 * k_gemm_i8, shaders/prefill.metal:382-415,457-471). */
int kata_gemm_ptq1_i8(const int8_t* A8, const float* SX, int ldS, const uint8_t* W, void* C,
                      int c_dtype, int ldc, int M, int K, int N, void* stream);

/* Standalone expansions (verification and catch-up uses), natural row-major layout:
 * out[n][k] = half(trit*d) (fp16 bits), T8[n][k] = trit, SW[n][k/128] = d.
 * Replace k_expand_ptq1_v2 / k_expand_i8_v2 (shaders/prefill.metal:457-479); the
 * reference writes tile-major [N/64][K][64], here the order is [N][K]. */
int kata_expand_ptq1_f16(const uint8_t* W, uint16_t* out, int K, int N, void* stream);
int kata_expand_ptq1_i8(const uint8_t* W, int8_t* T8, float* SW, int K, int N, void* stream);

/* ---------------------------------------------------------------- matmul input -------
 * The transform every ternary matmul input goes through (the model's rotated basis), per
 * token row m < M of width W (W % 1024 == 0), fp32 arithmetic:
 *   v = x + y (y may be NULL), xnew = v (may be NULL), inv = 1/sqrt(mean(v^2) + 1e-6),
 *   hout = v * inv * gamma (gamma and hout both NULL or both set; hout_dtype F32 or F16),
 *   out[b][j] = (1/32) sum_k (-1)^popcount(j & k) * (v * inv * gs)[1024 b + k]
 * (gs = the sign vector with the RMSNorm weight folded in).  out is fp32 or fp16 rows
 * [M][W], or for M == 2 fp16 with the two tokens interleaved, [W][2] (KATA_X_HALF2, the
 * half2 operand of the T = 2 GEMV), or for M <= 2 the decode GEMV's operand form
 * (out_dtype KATA_XQ, out_layout KATA_X_ROWS, kata_gemv_xq_bytes(W, M) bytes: the fp32
 * values quantised as kata_gemv_prepare_x does, so the GEMV then gives y bit for bit as
 * from the fp32 rows).  All vectors 16-byte aligned.
 * Replaces k_add_rms_fwht (shaders/ops.metal:86-106), k_add_rms_fwht_b and
 * k_add_rms_fwht_t (shaders/prefill.metal:59-78,266-285). */
int kata_add_rms_fwht(const float* x, const float* y, const float* gs, void* out, int out_dtype, int out_layout,
                      float* xnew, const float* gamma, void* hout, int hout_dtype, int W, int M, void* stream);
/* Outputs (out, xnew, hout) must not overlap each other or any input (x, y, gs, gamma):
 * KATA_EINVAL otherwise; an in-place residual update needs a second buffer, as the
 * reference alternates two (src/engine.cpp:136-146). */

/* The other input transforms, same out formats (out must not overlap src, src2 or gs): mode 0 RMSNorm of src (as above, no
 * residual), 1 SwiGLU v = silu(src) * src2, 2 src in the grouped GDN head order
 * (v[128 t + h] = src[h + 128 (t/3 + 16 (t%3))], W == 6144), 3 v = src; out = H(v * gs).
 * Replaces k_rms_fwht (shaders/ops.metal:30-54) and k_rms_fwht_b (shaders/prefill.metal:81-97). */
int kata_rms_fwht(const float* src, const float* src2, const float* gs, void* out, int out_dtype, int out_layout,
                  int W, int M, int mode, void* stream);

/* Measurement helpers for the roofline figures; no counterpart in the reference (its
 * benchmarks time Metal kernels only).  kata_calib_empty: an empty kernel of wgs
 * 1024-thread workgroups (wgs <= 0: one per CU, the decode GEMV's geometry), the launch
 * floor.  kata_calib_read: a plain streaming read of `bytes` bytes at p (16-byte aligned,
 * < 2^31) at the same geometry, 16-byte loads, the achievable HBM read rate at that size;
 * out (device, one word) is written only in a case that practically never happens.
 * kata_calib_read_peak: the same read at the fastest plain-read geometry a sweep found
 * (two 256-thread workgroups per CU, non-temporal 16-byte loads, four in flight per
 * lane), the read ceiling the decode GEMV is measured against. */
int kata_calib_empty(uint32_t* out, int wgs, void* stream);
int kata_calib_read(const void* p, size_t bytes, uint32_t* out, int wgs, void* stream);
int kata_calib_read_peak(const void* p, size_t bytes, uint32_t* out, void* stream);
/* The same read at any geometry of the sweep that chose the ceiling: threads per workgroup
 * 256, 512 or 1024, wgs workgroups (1..65536), inflight 2, 4, 8 or 16 loads per lane, nt
 * nonzero for the non-temporal hint. */
int kata_calib_read_cfg(const void* p, size_t bytes, uint32_t* out, int threads, int wgs, int inflight, int nt,
                        void* stream);
/* The decode GEMV's weight-load stream alone: the loads kata_gemv_ptq1 issues for one K x N
 * PTQ1_0 matrix at T = 1 (the same workgroups, item order, 12-byte lane windows and ring of
 * four items) with the decode, the matrix-core work and the row sums left out, the rate
 * that loop would reach if the rest of each item were free.  K a multiple of 128, the matrix
 * 16-byte aligned and < 2^31 bytes; out as above. */
int kata_calib_read_ptq1(const void* W, int K, int N, uint32_t* out, void* stream);

/* Greedy argmax of n fp32 logits into *out (device int): an element counts only if strictly
 * greater than the best so far (NaN and -inf never do), lowest index on ties, 0x7fffffff
 * when none does.  x 16-byte aligned.  Deterministic; the per-workgroup partials live in a
 * 2 KB buffer of the calling (device, stream), allocated on its first call (which must not
 * be captured).  Replaces k_argmax (shaders/ops.metal:66-78) after the lm_head
 * GEMV (src/engine.cpp:191-192). */
int kata_argmax(const float* x, int n, int* out, void* stream);

/* Frees the scratch buffers the library holds for the calling device and `stream` (the
 * prefill GEMMs' K pieces, the wide GEMV's activation image, the argmax partials) after
 * synchronising the stream.  Those buffers are kept for the stream's later calls, and a
 * buffer outgrown by a larger call is kept too (not freed), since a HIP graph captured
 * earlier on the stream still holds its address.  Call this before hipStreamDestroy, once
 * no graph that recorded the stream's calls will be replayed again; a new stream that
 * reused a destroyed one's handle would otherwise inherit its buffers.  No counterpart in
 * the reference (its engine allocates every buffer once in load(), src/engine.cpp:48-84). */
int kata_release_stream(void* stream);

/* ---------------------------------------------------------------- HOST packers -------
 * HOST: quantize_row_ptq1_0_ref over nrow rows of k floats (k % 128 == 0)
 * (docs/reference/prism_ptq1_0_quant_dequant.c:4-52, quantize_ptq1_0 :86-96). */
int kata_quantize_ptq1_0(const float* x, uint8_t* out, int64_t nrow, int64_t k);
/* HOST: packs trits (int8 in {-1,0,1}, [nrow][k]) with given fp16 scales ([nrow][k/128],
 * raw bits) using the same byte encoding; used to build synthetic weights. */
int kata_pack_ptq1_0(const int8_t* trits, const uint16_t* scales, uint8_t* out, int64_t nrow, int64_t k);

/* ---------------------------------------------------------------- GGUF model file ----
 * HOST: a GGUF v3 file memory-mapped read-only and indexed (src/gguf.cpp:41-71,
 * src/gguf.h): tensor infos (name, ggml type — 143 PTQ1_0, 8 Q8_0, 0 F32 …, dims with
 * dims[0] the row length, byte offset in the data region, byte size) and integer / string
 * metadata.  A file with a tensor of a ggml type not supported here (the reference exits on
 * one, src/gguf.cpp:25-37), an element count that is not whole blocks or overflows, or any
 * tensor outside the data region is rejected (NULL).  kata_gguf_upload copies the whole data region
 * to one device allocation: a matrix is then dev_base + offset, the weight base that
 * kata_dispatch_create takes and the byte offsets its calls take (src/engine.cpp:27-37).
 * NULL / negative returns set kata_last_error(). */
typedef struct kata_gguf kata_gguf;
kata_gguf* kata_gguf_open(const char* path);
void kata_gguf_close(kata_gguf* g);
int64_t kata_gguf_tensor_count(const kata_gguf* g);
uint64_t kata_gguf_data_bytes(const kata_gguf* g);
/* tensor i: any output pointer may be NULL; dims has room for 4 */
int kata_gguf_tensor(const kata_gguf* g, int64_t i, const char** name, uint32_t* type, uint64_t* dims,
                     uint64_t* offset, uint64_t* nbytes);
int64_t kata_gguf_find(const kata_gguf* g, const char* name);          /* index, or KATA_EINVAL */
int kata_gguf_get_int(const kata_gguf* g, const char* key, uint64_t* value);
const char* kata_gguf_get_str(const kata_gguf* g, const char* key);   /* NULL if absent */
/* synchronous device copy of the data region (a new hipMalloc); free with kata_gguf_free_device */
int kata_gguf_upload(const kata_gguf* g, uint8_t** dev_base);
/* the same copy into caller device memory of at least kata_gguf_data_bytes(g) bytes */
int kata_gguf_upload_into(const kata_gguf* g, uint8_t* dev, uint64_t capacity);
int kata_gguf_free_device(uint8_t* dev_base);

/* ---------------------------------------------------------------- dispatcher ---------
 * An engine-side dispatcher that maps (byte offset into the weight file, K, N, matrix
 * name) to the kernels above, with the reference's per-matrix int8 selection.
 * Mirrors Engine::dGemvPtq1 / dExpandGemm / setI8 / i8 (src/engine.cpp:97-101,208-219,
 * 529-537; src/engine.h:89-95).  Names: qkv z ssmout wq wk wv wo gate up down. */
typedef struct kata_dispatch kata_dispatch;
kata_dispatch* kata_dispatch_create(const uint8_t* wbase);
void kata_dispatch_destroy(kata_dispatch* d);
/* "all", "ffn" (gate+up), "none"/"", or a comma list of names; KATA_EINVAL on unknown. */
int kata_dispatch_set_i8(kata_dispatch* d, const char* spec);
int kata_dispatch_i8(const kata_dispatch* d, const char* name);   /* 1 if int8 path */
uint32_t kata_dispatch_i8_mask(const kata_dispatch* d);
/* T=1 decode GEMV of the matrix at byte offset wOff (x fp32 [K], y fp32 [N]). */
int kata_dispatch_gemv(kata_dispatch* d, uint64_t wOff, const float* x, float* y, int K, int N,
                       void* stream);
/* The `gq` lambda of Engine::mtpRows (src/engine.cpp:351) over the dispatcher's weights, for
 * 1..4 Q8_0 matrices at byte offsets offs[i] (HOST array) that read the same activation x
 * ([T][K] fp32 or fp16, T in {1,2}) into outs[i] ([T][N[i]] fp32, HOST array of device
 * pointers): one kata_gemv_q8_0_batch launch (the MTP block's wq + wk + wv and gate + up,
 * src/engine.cpp:361,369; a single matrix for eh_proj, wo and down). */
int kata_dispatch_gemv_q8(kata_dispatch* d, int count, const uint64_t* offs, const void* x, int x_dtype,
                          float* const* outs, const int* N, int K, int T, void* stream);
/* Prefill matmul of the named matrix: fp16 exact path, or the int8 path when selected
 * (then A is quantised into caller-provided A8 [M][K] / SX [K/128][ldS] work buffers;
 * they may be NULL when the matrix is on the fp16 path).  C fp32 [M][N]. */
int kata_dispatch_prefill(kata_dispatch* d, uint64_t wOff, const uint16_t* A, float* C, int M,
                          int K, int N, const char* name, int8_t* A8, float* SX, int ldS,
                          void* stream);

/* Layer level: the FFN sublayer of Engine::step (src/engine.cpp:176-182) through the
 * dispatcher's weights: h = H(rmsnorm(x + y) * gs_in) (x + y also to xnew when non-NULL; y
 * may be NULL), g = W_gate h and u = W_up h in one launch, t = H(silu(g) * u * gs_down),
 * out = W_down t.  x, y, xnew, out fp32 [H]; work H + 3F floats; H, F multiples of 1024. */
int kata_dispatch_ffn_decode(kata_dispatch* d, uint64_t offGate, uint64_t offUp, uint64_t offDown, const float* x,
                             const float* y, float* xnew, const float* gs_in, const float* gs_down, float* work,
                             float* out, int H, int F, void* stream);
/* The same for M prefill rows (src/engine.cpp:247-300): fp16 rows into the GEMMs, each of
 * gate / up / down on the fp16 exact or int8 path as kata_dispatch_set_i8 selected.  x, y,
 * xnew, out fp32 [M][H]; work of kata_ffn_prefill_work_bytes(H, F, M) bytes, 16-byte aligned. */
int kata_dispatch_ffn_prefill(kata_dispatch* d, uint64_t offGate, uint64_t offUp, uint64_t offDown, const float* x,
                              const float* y, float* xnew, const float* gs_in, const float* gs_down, void* work,
                              float* out, int H, int F, int M, void* stream);
size_t kata_ffn_prefill_work_bytes(int H, int F, int M);
/* The same for T in 1..8 verification tokens (Engine::verifyWide's FFN block,
 * src/engine.cpp:627-629): fp16 token rows through the wide verification GEMV, gate and up
 * as one kata_gemv_ptq1_wide_batch (its buffer rules apply).  x, y, xnew, out fp32 [T][H]; work of kata_ffn_verify_work_bytes(H, F, T)
 * bytes, 16-byte aligned. */
int kata_dispatch_ffn_verify(kata_dispatch* d, uint64_t offGate, uint64_t offUp, uint64_t offDown, const float* x,
                             const float* y, float* xnew, const float* gs_in, const float* gs_down, void* work,
                             float* out, int H, int F, int T, void* stream);
size_t kata_ffn_verify_work_bytes(int H, int F, int T);

/* Any sublayer's matmul halves through the dispatcher's weights, in the three forms of the
 * engine: KATA_FORM_DECODE (M == 1: Engine::step, src/engine.cpp:150-182), KATA_FORM_PREFILL
 * (M rows, GEMMs on the fp16 exact or int8 path as kata_dispatch_set_i8 selected, h quantised
 * once for its int8 matrices: Engine::prefill, src/engine.cpp:247-300) and KATA_FORM_VERIFY
 * (M <= 8 tokens through the wide GEMV: Engine::verify2 / verifyWide, src/engine.cpp:454-491,
 * 627-629).
 * Input half: h = H(rmsnorm(x + y) * gs) (x + y also to xnew; gamma/hout as in
 * kata_add_rms_fwht: the plain normalised rows the GDN alpha/beta projections read), then
 * outs[i] = W_i h (fp32 [M][N[i]]) for the 1..4 matrices that read h, at byte offsets offs[i],
 * named as in kata_dispatch_set_i8 (GDN: "qkv", "z"; GQA: "wq", "wk", "wv"; FFN: "gate",
 * "up").  offs, N, names, outs are HOST arrays; x, y, xnew fp32 [M][H].
 * Output half: t = H(v * gs), v per mode of kata_rms_fwht (1 SwiGLU of src, src2 before
 * "down"; 2 GDN head order of src, W == 6144, before "ssmout"; 3 src before "wo"), then
 * out = W t (fp32 [M][H]).  src, src2 fp32 [M][W].
 * H, W multiples of 1024; work of kata_dispatch_work_bytes(form, H or W, M) bytes, 16-byte
 * aligned; the prefill form uses the workspace of kata_gemm_ptq1_f16, the verify form the
 * buffer of kata_gemv_ptq1_wide (its 1..4 input-half matrices in one batched launch). */
#define KATA_FORM_DECODE 0
#define KATA_FORM_PREFILL 1
#define KATA_FORM_VERIFY 2
int kata_dispatch_in(kata_dispatch* d, int form, int count, const uint64_t* offs, const int* N,
                     const char* const* names, float* const* outs, const float* x, const float* y, float* xnew,
                     const float* gs, const float* gamma, void* hout, int hout_dtype, void* work, int H, int M,
                     void* stream);
int kata_dispatch_out(kata_dispatch* d, int form, uint64_t off, const char* name, const float* src, const float* src2,
                      int mode, const float* gs, void* work, float* out, int W, int H, int M, void* stream);
size_t kata_dispatch_work_bytes(int form, int K, int M);

#ifdef __cplusplus
}
#endif
#endif /* KATA_AMD_H */
