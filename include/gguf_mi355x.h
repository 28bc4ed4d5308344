/* C ABI of the MI355X (gfx950) GGUF quantized-matmul library, libgguf_mi355x.so.
 *
 * These entry points replace the reference's op boundary, the torch ops of
 * plugin/vllm_gguf_plugin/csrc/lcpp_shim.cu (schemas :973-983, implementations :911-971, guards
 * check_inputs :690-732 and run() :767-791). Plain pointers, sizes and strides only: the host
 * side that owns tensors (vllm_gguf_plugin/_C_gguf.py) passes views, an output buffer, a
 * workspace and the stream; the library allocates nothing.
 *
 * Conventions, as the reference's:
 *  - W: uint8 [>= row, row_bytes] GGUF blocks, unit inner stride, contiguous rows, 16-byte
 *    aligned, K = row_bytes / block_bytes * 256, K % 512 == 0.
 *  - X: fp32 / fp16 / bf16 [n, K], unit inner stride, row stride >= K.
 *  - Y: [n, row] contiguous in X's dtype (the reference's output dtype).
 *  - type: a GGUF type id of the reference's Route L set (lcpp_shim.cu:676-684): Q2_K 10,
 *    Q4_K 12, Q6_K 14, IQ2_XXS 16, IQ2_XS 17, IQ3_XXS 18, IQ3_S 21, IQ2_S 22, IQ4_XS 23,
 *    IQ1_M 29 (no product op for IQ1_M); each op's own type checks are the reference's.
 *  - x_q8 (optional): X already quantised to block_q8_1 by gguf_lcpp_quantize_q8_1(mmq = 0),
 *    contiguous uint8 of >= n*K/32*36 bytes, 16-byte aligned, on X's device.
 *  - Every guard runs before any launch, in the reference's order, with its message; a view
 *    with device < 0 (host memory) passes the shape guards and is then rejected with "must be
 *    CUDA tensors", so the guards are testable without a GPU. Nothing touches the GPU before
 *    the guards pass.
 *  - Launches are stream-ordered on `stream` (a hipStream_t, NULL = the null stream) and never
 *    synchronise the host; results are bit-identical across calls and hipGraph replays.
 *  - Return 0 on success, GGUF_EINVAL when a guard rejects, GGUF_EHIP on a HIP error;
 *    gguf_last_error() gives the message (per thread).
 */
#ifndef GGUF_MI355X_H
#define GGUF_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define GGUF_API __attribute__((visibility("default")))
#else
#define GGUF_API
#endif

#define GGUF_OK 0
#define GGUF_EINVAL 1
#define GGUF_EHIP 2

/* element type codes of a view */
enum { GGUF_DT_F32 = 0, GGUF_DT_F16 = 1, GGUF_DT_BF16 = 2, GGUF_DT_U8 = 3, GGUF_DT_OTHER = 4 };

/* A strided view of a 1-D or 2-D tensor as the guards see it. Sizes and strides in elements;
 * device: GPU index, or -1 for host memory. */
typedef struct gguf_view {
  const void* data;
  int32_t dtype;
  int32_t ndim;
  int64_t size[2];
  int64_t stride[2];
  int32_t device;
} gguf_view;

/* The reference's product ops (lcpp_shim.cu:973-983), by name. */
enum {
  GGUF_OP_MUL_MAT_VEC_Q = 0,           /* lcpp_mul_mat_vec_q (W, X, type, row, x_q8)        */
  GGUF_OP_MUL_MAT_Q = 1,               /* lcpp_mul_mat_q (W, X, type, row)                  */
  GGUF_OP_MUL_MAT_VEC_IQ3 = 2,         /* lcpp_mul_mat_vec_iq3 (W, X, type, row, x_q8)      */
  GGUF_OP_MUL_MAT_VEC_IQ3_MMA = 3,     /* lcpp_mul_mat_vec_iq3_mma (W, X, type, row, x_q8)  */
  GGUF_OP_MUL_MAT_VEC_OWN = 4,         /* lcpp_mul_mat_vec_own (W, X, type, row, x_q8)      */
  GGUF_OP_MUL_MAT_MMA_K = 5,           /* lcpp_mul_mat_mma_k (W, X, type, row)              */
  GGUF_OP_MUL_MAT_VEC_IQ3_MMA_PACKED = 6, /* lcpp_mul_mat_vec_iq3_mma_packed (..., x_q8)    */
  GGUF_OP_MUL_MAT_IQ3_PACKED = 7,      /* lcpp_mul_mat_iq3_packed (W, X, type, row)         */
  GGUF_OP_COUNT = 8
};

/* Last error message of the calling thread ("" if none). */
GGUF_API const char* gguf_last_error(void);

/* Library version string. */
GGUF_API const char* gguf_version(void);

/* The guards of product op `op` (lcpp_shim.cu run() :767-791 then check_inputs :690-732), in
 * the reference's order and wording. x_q8 may be NULL. No GPU access. */
GGUF_API int gguf_check_op(int op, const gguf_view* W, const gguf_view* X, int64_t type, int64_t row,
                  const gguf_view* x_q8);

/* Workspace bytes the op needs for n activation rows of K columns (the q8_1 copy of X unless
 * x_q8 is given). 0 if none. */
GGUF_API size_t gguf_op_workspace_bytes(int op, int64_t type, int64_t row, int64_t k, int64_t n, int has_x_q8);

/* One product: Y[n, row] = X @ W[:row].T, written to y (y_bytes >= n*row*sizeof(X dtype)).
 * The entry points below are this function with `op` fixed. */
GGUF_API int gguf_mul_mat(int op, const gguf_view* W, const gguf_view* X, int64_t type, int64_t row,
                 const gguf_view* x_q8, void* y, size_t y_bytes, void* workspace, size_t workspace_bytes,
                 void* stream);

/* The caller's allocator for gguf_mul_mat_alloc: device memory of `bytes` bytes on X's device,
 * 16-byte aligned, for the output (what = GGUF_ALLOC_OUTPUT; bytes may be 0) or the workspace
 * (GGUF_ALLOC_WORKSPACE), or NULL on failure. It must stay valid until the product's launches have
 * run on `stream`. */
enum { GGUF_ALLOC_OUTPUT = 0, GGUF_ALLOC_WORKSPACE = 1 };
typedef void* (*gguf_alloc_fn)(void* ctx, int what, size_t bytes);

/* gguf_mul_mat that takes its output and workspace from the caller's allocator once the guards
 * have passed: the order of the reference's run() (lcpp_shim.cu:767-805: the guards, then the
 * output from torch's allocator, then the launches), with one guard pass per call. The output is
 * asked for first, also when X has no rows; the workspace only when the plan needs one. */
GGUF_API int gguf_mul_mat_alloc(int op, const gguf_view* W, const gguf_view* X, int64_t type, int64_t row,
                                const gguf_view* x_q8, gguf_alloc_fn alloc, void* alloc_ctx, void* stream);

/* Bytes of the static per-GPU scratch that gguf_mul_mat_noalloc uses as its workspace. */
#define GGUF_SCRATCH_BYTES ((size_t)8 << 20)
GGUF_API size_t gguf_scratch_bytes(void);

/* gguf_mul_mat without a workspace argument and without any allocation: no counterpart in the
 * reference; for callers that cannot allocate (code under stream capture, tight serving loops,
 * harnesses that forbid hipMalloc). The workspace is a statically sized device array of
 * GGUF_SCRATCH_BYTES per GPU, located once per device on the first call there and held until the
 * process ends. A product whose workspace (gguf_op_workspace_bytes) exceeds it is rejected with
 * GGUF_EINVAL; that covers the decode and small-batch products (e.g. 64 activation rows at
 * K = 17408) but not large prefills. Every call on a GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other threads) race, so the caller serialises them; the
 * scratch needs no clearing (every byte a kernel reads is written first by the same call). */
GGUF_API int gguf_mul_mat_noalloc(int op, const gguf_view* W, const gguf_view* X, int64_t type, int64_t row,
                         const gguf_view* x_q8, void* y, size_t y_bytes, void* stream);

/* replaces lcpp_mul_mat_vec_q (lcpp_shim.cu:911-913): 1..8 activation rows */
GGUF_API int gguf_lcpp_mul_mat_vec_q(const gguf_view* W, const gguf_view* X, int64_t type, int64_t row,
                            const gguf_view* x_q8, void* y, size_t y_bytes, void* workspace,
                            size_t workspace_bytes, void* stream);
/* replaces lcpp_mul_mat_q (lcpp_shim.cu:915-917): any number of rows */
GGUF_API int gguf_lcpp_mul_mat_q(const gguf_view* W, const gguf_view* X, int64_t type, int64_t row, void* y,
                        size_t y_bytes, void* workspace, size_t workspace_bytes, void* stream);
/* replaces lcpp_mul_mat_vec_iq3 (lcpp_shim.cu:919-921): IQ3_S, 1..8 rows */
GGUF_API int gguf_lcpp_mul_mat_vec_iq3(const gguf_view* W, const gguf_view* X, int64_t type, int64_t row,
                              const gguf_view* x_q8, void* y, size_t y_bytes, void* workspace,
                              size_t workspace_bytes, void* stream);
/* replaces lcpp_mul_mat_vec_iq3_mma (lcpp_shim.cu:923-925): IQ3_S, 1..8 rows */
GGUF_API int gguf_lcpp_mul_mat_vec_iq3_mma(const gguf_view* W, const gguf_view* X, int64_t type, int64_t row,
                                  const gguf_view* x_q8, void* y, size_t y_bytes, void* workspace,
                                  size_t workspace_bytes, void* stream);
/* replaces lcpp_mul_mat_vec_own (lcpp_shim.cu:927-929): Q4_K, 1..8 rows */
GGUF_API int gguf_lcpp_mul_mat_vec_own(const gguf_view* W, const gguf_view* X, int64_t type, int64_t row,
                              const gguf_view* x_q8, void* y, size_t y_bytes, void* workspace,
                              size_t workspace_bytes, void* stream);
/* replaces lcpp_mul_mat_mma_k (lcpp_shim.cu:931-933): Q4_K / IQ4_XS, 1..64 rows */
GGUF_API int gguf_lcpp_mul_mat_mma_k(const gguf_view* W, const gguf_view* X, int64_t type, int64_t row, void* y,
                            size_t y_bytes, void* workspace, size_t workspace_bytes, void* stream);
/* replaces lcpp_mul_mat_vec_iq3_mma_packed (lcpp_shim.cu:935-938): IQ3_S or IQ3_XXS in the build's
 * unit layout of its type (gguf_iq3_pack), 1..32 rows, row % 16 == 0 */
GGUF_API int gguf_lcpp_mul_mat_vec_iq3_mma_packed(const gguf_view* W, const gguf_view* X, int64_t type, int64_t row,
                                         const gguf_view* x_q8, void* y, size_t y_bytes, void* workspace,
                                         size_t workspace_bytes, void* stream);
/* replaces lcpp_mul_mat_iq3_packed (lcpp_shim.cu:940-942): IQ3_S / IQ3_XXS unit layout, any rows */
GGUF_API int gguf_lcpp_mul_mat_iq3_packed(const gguf_view* W, const gguf_view* X, int64_t type, int64_t row, void* y,
                                 size_t y_bytes, void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of the q8_1 copy of an [n, k] X: block_q8_1 (mmq = 0) or block_q8_1_mmq (mmq = 1). */
GGUF_API size_t gguf_q8_1_bytes(int64_t n, int64_t k, int mmq);

/* replaces lcpp_quantize_q8_1 (lcpp_shim.cu:949-971): X -> q8_1 bytes at out. vendored must be
 * 0 (the reference's vendored fp32 quantizers have no counterpart here). */
GGUF_API int gguf_lcpp_quantize_q8_1(const gguf_view* X, int64_t type, int mmq, int vendored, void* out, size_t out_bytes,
                            void* stream);

/* The build's IQ3_S and IQ3_XXS unit layouts (the reference's load-time repack hook,
 * quantization/iq3_pack.py pack_(w, weight_type) / unpack, replaced by layouts of this build's
 * own). In place on rows % 16 == 0 GGUF rows [rows, row_bytes] of type 21 (IQ3_S) or 18 (IQ3_XXS)
 * (contiguous, 16-byte aligned); scratch: >= gguf_iq3_pack_scratch_bytes. */
GGUF_API size_t gguf_iq3_pack_scratch_bytes(int64_t rows, int64_t row_bytes);
GGUF_API int gguf_iq3_pack(void* w, int64_t type, int64_t rows, int64_t row_bytes, int unpack, void* scratch,
                           size_t scratch_bytes, void* stream);

/* Dense product of a small unquantized weight: Y[n, rows] = X @ W.T in X's dtype, W [rows, K] and
 * X [n, K] of one float dtype (fp32 / fp16 / bf16), 1 <= n <= 8 (n == 0: nothing), K % 32 == 0,
 * unit inner strides, data and row strides 16-byte aligned. Replaces the reference's batched-GEMV
 * route for the GGUF file's F32/F16/BF16 tensors of at most 128 rows at up to 8 activation rows
 * (plugin/vllm_gguf_plugin/quantization/linear.py:281-291); any row count is accepted. */
GGUF_API int gguf_dense_mul_mat(const gguf_view* W, const gguf_view* X, void* y, size_t y_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GGUF_MI355X_H */
