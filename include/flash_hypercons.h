/*
 * flash_hypercons.h -- C ABI of the MI355X (gfx950) batched small-matrix
 * exponential library, libflash_hypercons_hip.so.
 *
 * The library computes, for a batch of [B, n, n] matrices with 2 <= n <= 32
 * stored as float32, float16 or bfloat16:
 *   forward   exp(X)                                   (degree-18 Taylor,
 *             Bader-Blanes-Casas 2019, with scaling and squaring)
 *   Frechet   U block of exp([[X, G], [0, X]])           (the structured
 *             derivative L(X, G); the autograd backward of exp(A) is
 *             L(A^T, grad_output))
 * Arithmetic is FP32 with an FP64 1-norm for the squaring count, as in the
 * reference.  Inputs are read through arbitrary element strides (transposed,
 * expanded stride-0 and lazily negated views need no copy); the output is a
 * contiguous [B, n, n] array in the input dtype.
 *
 * All pointers are device pointers of one HIP device, the current device of
 * the calling thread, and every view (pointer, strides, batch, n) must lie
 * within an allocation on it: the library checks shapes, dtypes and its own
 * addressing limits, not memory bounds.  Launches are asynchronous on `stream`; nothing here
 * synchronises, allocates device memory or keeps state across calls other
 * than the thread-local error message.
 *
 * Return value of every entry point: FH_OK, or an FH_ERR_* code with a
 * message available from fh_last_error() on the same thread.
 */
#ifndef FLASH_HYPERCONS_H
#define FLASH_HYPERCONS_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#if defined(__GNUC__)
#define FH_API __attribute__((visibility("default")))
#else
#define FH_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define FH_OK 0
#define FH_ERR_INVALID_ARGUMENT 1 /* shape, dtype, pointer or stride not accepted */
#define FH_ERR_LAUNCH 2           /* a HIP launch reported an error */

/* Element types; the codes are the reference launcher's
 * (csrc/matrix_exp.cu:17: 0 = float32, 1 = bfloat16, 2 = float16). */
#define FH_DTYPE_F32 0
#define FH_DTYPE_BF16 1
#define FH_DTYPE_F16 2

/* Kernel selection for fh_expm_launch. */
#define FH_VARIANT_AUTO 0    /* the tuned gfx950 kernels (what fh_matrix_exp/fh_frechet run) */
#define FH_VARIANT_GENERIC 1 /* one wavefront per matrix in the reference's exact
                                evaluation order; a checking aid, not a fast path */

/* exp(X) for X = input viewed as [batch, n, n] with element strides
 * strides[0..2] (batch, row, column) and a lazy-negation flag.  Any int64
 * strides are accepted; an operand whose single-matrix footprint exceeds
 * 2 GiB (or has a negative stride) is computed by the 64-bit-indexed
 * one-wavefront-per-matrix kernel when n > 8.
 * Replaces matrix_exp_cuda (csrc/matrix_exp.cu:80-82), the CUDA kernel of the
 * schema flash_hypercons::_matrix_exp(Tensor input) -> Tensor
 * (csrc/register.cpp:11, :16).  Rejects n outside [2, 32] and unknown dtypes
 * with the reference's message (csrc/matrix_exp.cu:52-55).  batch == 0 is a
 * no-op (csrc/matrix_exp.cu:62-64). */
FH_API int fh_matrix_exp(const void* input, const int64_t strides[3], int input_neg, void* out, int dtype,
                  int64_t batch, int n, hipStream_t stream);

/* U block of exp([[X, G], [0, X]]) with X = input and G = direction, both
 * [batch, n, n] of the same dtype, each with its own strides and negation flag.
 * Replaces frechet_cuda (csrc/matrix_exp.cu:84-86), the CUDA kernel of
 * flash_hypercons::_frechet(Tensor input, Tensor direction) -> Tensor
 * (csrc/register.cpp:12, :17). */
FH_API int fh_frechet(const void* input, const int64_t input_strides[3], int input_neg, const void* direction,
               const int64_t direction_strides[3], int direction_neg, void* out, int dtype, int64_t batch,
               int n, hipStream_t stream);

/* The launcher under both entry points: direction == NULL selects exp(X),
 * otherwise the Frechet block.  `variant` picks the kernel family
 * (FH_VARIANT_*).  When s_out is not NULL it also receives the squaring count
 * of every matrix (int32 [batch]; -1 where the non-finite rule fired).
 * Replaces small_matrix_exp_cuda + launch_small_matrix_exp
 * (csrc/matrix_exp.cu:51-78, :13-33). */
FH_API int fh_expm_launch(const void* input, const int64_t input_strides[3], int input_neg, const void* direction,
                   const int64_t direction_strides[3], int direction_neg, void* out, int dtype, int64_t batch,
                   int n, int variant, int32_t* s_out, hipStream_t stream);

/* Selection parameters only: params (int32 [batch, 2]) receives (degree, s)
 * per matrix -- degree 18 and the squaring count, or (-1, -1) for a matrix the
 * non-finite rule sends to NaN -- and norms (double [batch], may be NULL) the
 * FP64 1-norm the count was derived from (NaN for non-finite matrices).
 * direction may be NULL (forward) or the Frechet direction (backward norm of
 * the augmented matrix).  No counterpart in the reference: it exposes the
 * per-matrix choice made inside MatrixExpSmall.cuh:141-154 / :332-361 so that
 * it can be checked bit for bit. */
FH_API int fh_expm_params(const void* input, const int64_t input_strides[3], int input_neg, const void* direction,
                   const int64_t direction_strides[3], int direction_neg, int dtype, int64_t batch, int n,
                   int32_t* params, double* norms, hipStream_t stream);

/* Hyper-connection stream mixing with the exponential fused in:
 * y[b] = exp(h[b]) x[b] for h [batch, n, n] (any strides, lazy negation) and
 * x [batch, n, cols], 2 <= n <= 4 streams; y is a contiguous [batch, n, cols]
 * array of the same dtype.  x's rows must be contiguous and 16-byte aligned,
 * with cols and x's strides multiples of 16 bytes' worth of elements (4 in
 * float32, 8 in float16/bfloat16); each token's rows of x (and of grad) and
 * its n * cols output elements must each span < 2 GiB (FH_ERR_INVALID_ARGUMENT
 * with a span message otherwise).
 * exp(h[b]) is the same as fh_matrix_exp's (bit for bit) and never goes
 * to memory; e_out (float32 [batch, n, n], may be NULL) receives a copy.
 * No counterpart in the reference: its matrix_exp (flash_hypercons/ops/
 * matrix_exp/__init__.py:80-97) returns exp(h) and the caller multiplies; this
 * is the consumer fusion of that product.  Allocates nothing. */
FH_API int fh_hc_mix(const void* h, const int64_t h_strides[3], int h_neg, const void* x, const int64_t x_strides[3],
              void* y, float* e_out, int dtype, int64_t batch, int n, int64_t cols, hipStream_t stream);

/* Gradients of fh_hc_mix for the upstream gradient grad (same layout rules
 * as x): dx = exp(h)^T grad (contiguous [batch, n, cols]) and
 * dh = L(h^T, grad x^T) (contiguous [batch, n, n]), the Frechet derivative
 * computed as fh_frechet does, from the float32 grad x^T reduced in a fixed
 * order (de_out, float32 [batch, n, n], may be NULL, receives it).  One kernel;
 * allocates nothing. */
FH_API int fh_hc_mix_backward(const void* h, const int64_t h_strides[3], int h_neg, const void* x,
                       const int64_t x_strides[3], const void* grad, const int64_t grad_strides[3], void* dh,
                       void* dx, float* de_out, int dtype, int64_t batch, int n, int64_t cols, hipStream_t stream);

/* Stream mixing for 5 <= n <= 8 streams with exp(h) supplied: y[b] = e[b] x[b]
 * for e FP32 [batch, n, n] (contiguous; e.g. fh_matrix_exp of h in float32,
 * which gives the same bits the fused path keeps on chip) and x [batch, n,
 * cols] under fh_hc_mix's row rules; y contiguous [batch, n, cols] in the
 * dtype of x.  No counterpart in the reference (the consumer product of its
 * matrix_exp, ops/matrix_exp/__init__.py:80-97).  Allocates nothing. */
FH_API int fh_hc_apply(const float* e, const void* x, const int64_t x_strides[3], void* y, int dtype, int64_t batch,
                int n, int64_t cols, hipStream_t stream);

/* Gradients through fh_hc_apply for the upstream gradient grad (x's layout
 * rules): dx = e^T grad (contiguous [batch, n, cols]) and de = grad x^T (FP32
 * [batch, n, n], contiguous), reduced in a fixed order; dh then follows as the
 * Frechet derivative L(h^T, de) (fh_frechet in float32).  One kernel;
 * allocates nothing. */
FH_API int fh_hc_apply_backward(const float* e, const void* x, const int64_t x_strides[3], const void* grad,
                         const int64_t grad_strides[3], void* dx, float* de, int dtype, int64_t batch, int n,
                         int64_t cols, hipStream_t stream);

/* Message of the last failing call on this thread ("" if none). */
FH_API const char* fh_last_error(void);

/* Library version string, e.g. "0.1.0". */
FH_API const char* fh_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FLASH_HYPERCONS_H */
