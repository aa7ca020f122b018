/*
 * cmpext3_gemm.h -- C ABI of the MI355X (gfx950) dense matrix-multiply library.
 *
 * Every entry point computes C = A * B (optionally batched, optionally plus a
 * broadcast bias row) with fp32 accumulation and writes C in the input dtype.
 * Matrices are row-major.  All pointers are device pointers owned by the
 * caller; the library never allocates, frees or synchronises.  Work is
 * enqueued on `stream` (a hipStream_t; NULL means the null stream) and the call
 * returns as soon as the kernels are queued.
 *
 * Return value: CMPEXT3_OK (0); a negative CMPEXT3_ERR_* for a rejected
 * argument (nothing was launched); or a positive hipError_t from the launch.
 * cmpext3_status_string() turns any of them into text.
 *
 * The reference library (eastmoe/cmp_ext, `cmpext3`) has no C ABI: its
 * launchers are C++ functions with mangled names declared at
 * src/main.cpp:12-14 and called from src/main.cpp:204-224 and :319-349.  The
 * first three entry points below take their place one for one, with the same
 * argument order and meaning, plus the stream the reference lacks (it always
 * launches on stream 0, fp16_matmul.cu:315).
 */
#ifndef CMPEXT3_GEMM_H
#define CMPEXT3_GEMM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CMPEXT3_OK 0
#define CMPEXT3_ERR_INVALID_ARG (-1)  /* null pointer, negative size, bad stride */
#define CMPEXT3_ERR_UNSUPPORTED (-2)  /* unknown dtype / layout */
#define CMPEXT3_ERR_TOO_LARGE (-3)    /* a size or stride does not fit the kernels' 32-bit offsets */
#define CMPEXT3_ERR_WORKSPACE (-4)    /* a prepared call got less (or less aligned) workspace than it needs */
#define CMPEXT3_ERR_SCRATCH (-5)      /* cmpext3_gemm_ex_noalloc: the call needs more than CMPEXT3_SCRATCH_BYTES */

/* Element types. */
#define CMPEXT3_F16 0
#define CMPEXT3_BF16 1
#define CMPEXT3_F32 2

/* Layout of the B operand. */
#define CMPEXT3_B_KN 0 /* B is [K, N] row-major (matmul / bmm)            */
#define CMPEXT3_B_NK 1 /* B is [N, K] row-major (a Linear weight, W^T is used) */

/*
 * C[M,N] = A[M,K] * B[K,N], fp16 in, fp32 accumulate, fp16 out.
 * Replaces launch_matmul_fp16 (src/cuda/fp16_matmul.cu:301-340), whose strides
 * are lda=K, ldb=N, ldc=N (fp16_matmul.cu:311-313).  Any M, N, K >= 0.
 */
int cmpext3_matmul_fp16(const void* A, const void* B, void* C, int M, int N, int K, void* stream);

/*
 * C[M,N] = A[M,K] * B[K,N], bf16 in, fp32 accumulate, bf16 out.
 * Replaces launch_matmul_bf16 (src/cuda/bf16_matmul.cu:232-254).
 */
int cmpext3_matmul_bf16(const void* A, const void* B, void* C, int M, int N, int K, void* stream);

/*
 * C[M,N] = A[M,K] * B[K,N] in fp32 (fp32 MFMA, fused multiply-add).
 * Replaces launch_matmul_fp32 (src/cuda/fp32_matmul.cu:236-265).
 */
int cmpext3_matmul_fp32(const float* A, const float* B, float* C, int M, int N, int K, void* stream);

/*
 * Strided row-major forms: C[M,N] = A[M,K] * B[K,N] with row pitches lda >= K,
 * ldb >= N, ldc >= N (elements), fp32 accumulation, output in the input dtype
 * (fp32 MFMA for _f32).  The launchers above with explicit pitches, so a caller
 * holding row-pitched views (e.g. a column slice of a larger matrix) needs no
 * copy.  No workspace: M <= 64 products take the unsplit skinny kernel.
 * Replace launch_matmul_fp16/bf16/fp32 (src/cuda/fp16_matmul.cu:301-340,
 * bf16_matmul.cu:232-254, fp32_matmul.cu:236-265), which fix lda=K, ldb=N,
 * ldc=N (fp16_matmul.cu:311-313).
 */
int cmpext3_gemm_f16(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
                     int M, int N, int K, void* stream);
int cmpext3_gemm_bf16(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
                      int M, int N, int K, void* stream);
int cmpext3_gemm_f32(const float* A, int64_t lda, const float* B, int64_t ldb, float* C, int64_t ldc,
                     int M, int N, int K, void* stream);

/*
 * General form used by the Python bindings for matmul, linear and bmm:
 *   for b in [0, batch):  C_b = A_b * op(B_b) (+ bias)
 * with A_b = A + b*stride_a (elements), etc.; op(B) = B for CMPEXT3_B_KN and
 * B^T for CMPEXT3_B_NK.  lda/ldb/ldc are row pitches in elements; bias is
 * NULL or a length-N vector of the same dtype added to every row before the
 * final rounding.  `workspace` (16-byte aligned device memory, or NULL) of
 * `workspace_bytes` bytes lets the skinny-M path split K across workgroups;
 * cmpext3_gemm_workspace_size() says how much it can use.  Its contents need
 * no initialisation and are dead after the call's kernels have run (calls
 * that share a workspace must be ordered on one stream).
 * Replaces the host loop of custom_bmm_forward (src/main.cpp:313-351: one
 * launch per batch entry) with one launch, and the weight.t().contiguous()
 * copy plus separate bias kernel of custom_linear_forward
 * (src/main.cpp:182, :229-246) with the B_NK layout and a fused bias.
 */
int cmpext3_gemm_ex(int dtype, int b_layout,
                    const void* A, int64_t lda, int64_t stride_a,
                    const void* B, int64_t ldb, int64_t stride_b,
                    void* C, int64_t ldc, int64_t stride_c,
                    const void* bias,
                    int M, int N, int K, int batch,
                    void* workspace, int64_t workspace_bytes, void* stream);

/*
 * 1x1 convolution with stride 1, padding 0, dilation 1 and groups 1 on
 * contiguous NCHW tensors:
 *   output[b][o][p] = sum_c weight[o][c] * input[b][c][p] (+ bias[o])
 * with input [batch, c_in, hw], weight [c_out, c_in] (the [c_out, c_in, 1, 1]
 * tensor), bias NULL or [c_out], output [batch, c_out, hw], hw = H * W, all of
 * one dtype.  Each image is one GEMM out_b[c_out, hw] = W * in_b[c_in, hw]
 * (A = the weight, shared; B = the image in the [K, N] layout; the bias added
 * per output row), all images in one launch.  `workspace` is as for
 * cmpext3_gemm_ex; cmpext3_gemm_workspace_size(dtype, CMPEXT3_B_KN, c_out,
 * hw, c_in, batch) says how much helps.
 * Replaces the 1x1 branch of custom_conv2d_forward (src/main.cpp:402-424),
 * which permutes NCHW to NHWC, runs custom_linear_forward on a contiguous
 * copy (with its weight transpose copy and separate bias kernel) and permutes
 * the result back into a second copy; here no copy is made.
 */
int cmpext3_conv2d_1x1(int dtype, const void* input, const void* weight, const void* bias, void* output,
                       int batch, int c_in, int c_out, int hw,
                       void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Prepared calls: cmpext3_gemm_ex in two steps, so that a caller can size the
 * workspace from the very plan that will run (the kernel is chosen once) and
 * can see which kernel that is.
 *
 * cmpext3_gemm_prepare validates the arguments (those of cmpext3_gemm_ex, plus
 * `flags`), picks the kernel and stores the whole call -- pointers, sizes and
 * the plan -- in *call; nothing is launched and no GPU is touched.  A 16-bit
 * product whose last round of output tiles would run mostly empty (M just past
 * what whole rounds of 256-row tiles cover) is planned as two launches over its
 * rows, one for the rows whole rounds cover and one for the rest; they share the
 * workspace, one after the other.
 * `workspace_limit` is the most workspace the caller is willing to provide
 * (0: none; INT64_MAX: whatever helps).  CMPEXT3_BIAS_PER_ROW in `flags` adds
 * the bias per row of C (M elements) instead of per column (N elements).
 * cmpext3_gemm_call_workspace_size says how much workspace the chosen kernels
 * need (<= workspace_limit), cmpext3_gemm_call_describe writes a one-line
 * description of them (up to ~600 characters for two launches) and returns the
 * kernel id (of the first launch), and cmpext3_gemm_run
 * enqueues them on `stream` with a workspace of at least that many bytes
 * (16-byte aligned; NULL when none is needed; CMPEXT3_ERR_WORKSPACE otherwise).
 * A prepared call may be run more than once (e.g. while a graph is captured);
 * the buffers it names must then still be valid.  cmpext3_gemm_ex(...) is
 * cmpext3_gemm_prepare(..., workspace_bytes) followed by cmpext3_gemm_run.
 * No counterpart in the reference, whose launchers take no workspace and
 * choose nothing at run time (src/main.cpp:12-14, fp16_matmul.cu:12-22).
 */
#define CMPEXT3_BIAS_PER_ROW 1
typedef struct cmpext3_gemm_call {
  int64_t opaque[64];
} cmpext3_gemm_call;

int cmpext3_gemm_prepare(cmpext3_gemm_call* call, int dtype, int b_layout,
                         const void* A, int64_t lda, int64_t stride_a,
                         const void* B, int64_t ldb, int64_t stride_b,
                         void* C, int64_t ldc, int64_t stride_c,
                         const void* bias, int flags,
                         int M, int N, int K, int batch, int64_t workspace_limit);
int64_t cmpext3_gemm_call_workspace_size(const cmpext3_gemm_call* call);
int cmpext3_gemm_call_describe(const cmpext3_gemm_call* call, char* buf, int buflen);
int cmpext3_gemm_run(const cmpext3_gemm_call* call, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * cmpext3_gemm_ex without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): the call runs the plan cmpext3_gemm_ex
 * would run with all the workspace it asks for, with the library's own static
 * device scratch buffer of CMPEXT3_SCRATCH_BYTES (64 MiB, held by every GPU the
 * library runs on until the process ends) as that workspace.  When that plan
 * needs more than the scratch holds (zero-padded copies of large unaligned
 * operands, split-K partials of very large products), it runs the plan
 * cmpext3_gemm_ex would run with a workspace of CMPEXT3_SCRATCH_BYTES instead
 * (fewer K splits, or no padded copies); CMPEXT3_ERR_SCRATCH is returned, and
 * nothing launched, only if even that plan does not fit.  It calls no
 * allocating routine.  The scratch contents need no clearing: every byte a call
 * writes is read back by the same call.  All calls on one GPU share its buffer,
 * so calls that may overlap on one GPU (other streams, other threads) race;
 * order them on one stream.  The buffer used is that of the stream's GPU (the
 * current GPU for the null stream); its address is looked up once per GPU.
 * No counterpart in the reference; it is for callers that cannot allocate.
 */
#define CMPEXT3_SCRATCH_BYTES (64ll << 20)
int cmpext3_gemm_ex_noalloc(int dtype, int b_layout,
                            const void* A, int64_t lda, int64_t stride_a,
                            const void* B, int64_t ldb, int64_t stride_b,
                            void* C, int64_t ldc, int64_t stride_c,
                            const void* bias,
                            int M, int N, int K, int batch, void* stream);

/*
 * Bytes of workspace cmpext3_gemm_ex can use for these arguments (zero-padded
 * copies of operands whose rows are not 16-byte aligned, then split-K fp32
 * partial sums; 16-byte aligned); 0 when the chosen kernel needs none, or a
 * negative CMPEXT3_ERR_*.  Host only.  No counterpart in the reference, whose
 * kernels never split K (one launch per product, src/main.cpp:203-227).
 */
int64_t cmpext3_gemm_workspace_size(int dtype, int b_layout, int M, int N, int K, int batch);

/*
 * Kernel selection, host only (no GPU needed): writes a one-line description
 * of the kernel(s) cmpext3_gemm_ex would launch for these arguments into buf and
 * returns the kernel id (of the first launch; >= 0) or a negative CMPEXT3_ERR_*.  `align` is the
 * largest power of two (up to 16) dividing the byte address of every operand;
 * `workspace_bytes` is the workspace the call would provide.
 * No counterpart in the reference, whose tile choice is fixed at compile time
 * (fp16_matmul.cu:12-22, bf16_matmul.cu:11-21, fp32_matmul.cu:10-14).
 */
int cmpext3_gemm_plan(int dtype, int b_layout, int M, int N, int K,
                      int64_t lda, int64_t ldb, int64_t ldc, int align, int has_bias, int batch,
                      int64_t workspace_bytes, char* buf, int buflen);

/* Text for a status code returned by the entry points above. */
const char* cmpext3_status_string(int status);

/* Library version string. */
const char* cmpext3_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CMPEXT3_GEMM_H */
