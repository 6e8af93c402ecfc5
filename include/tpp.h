/*
 * tpp.h -- C ABI of libtorchpp_hip.so, the gfx950 (MI355X) kernel set that
 * replaces torchpp's CUDA/CUTLASS native modules.
 *
 * Conventions shared by every entry point
 * ---------------------------------------
 *  - All tensor arguments are caller-owned DEVICE pointers. No entry point
 *    allocates device memory; ops that need scratch take a `workspace`
 *    pointer whose size is returned by the matching *_workspace_size call.
 *  - `stream` is a hipStream_t passed as void* (NULL = the legacy default
 *    stream). Every launch is asynchronous on that stream.
 *  - Element types are `tpp_dtype` codes. Accumulation is always fp32.
 *  - Sizes and strides are int64_t and counted in ELEMENTS, not bytes.
 *  - Return value: TPP_OK (0) or a negative TPP_E_* code. The message for the
 *    last failure on the calling thread is returned by tpp_last_error_string().
 *  - The reference checked arguments with TORCH_CHECK and returned a new
 *    tensor (e.g. csrc/dlops/rmsnorm/rmsnorm_binding.cu:22-46,51); here the
 *    same checks run in C and the caller supplies the output buffer.
 */
#ifndef TPP_H_
#define TPP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  TPP_F16 = 0,  /* IEEE binary16 (the reference's only type, c10::Half)   */
  TPP_BF16 = 1, /* bfloat16                                               */
  TPP_F32 = 2   /* float32 (accepted for RoPE cos/sin tables only)        */
} tpp_dtype;

typedef enum {
  TPP_ACT_NONE = 0,
  TPP_ACT_GELU_TANH = 1, /* csrc/activation/activation.cuh:26-43 (GeluHalf)  */
  TPP_ACT_SILU = 2,      /* csrc/activation/activation.cuh:45-56 (SiluHalf)  */
  TPP_ACT_RELU = 3       /* csrc/activation/activation.cuh:59-67 (ReluHalf)  */
} tpp_act;

#define TPP_OK 0
#define TPP_E_INVALID (-1)     /* bad pointer / shape / stride argument     */
#define TPP_E_UNSUPPORTED (-2) /* dtype or shape the kernels do not handle  */
#define TPP_E_LAUNCH (-3)      /* hipLaunchKernel / hipGetLastError failure  */
#define TPP_E_WORKSPACE (-4)   /* workspace missing or too small            */

/* ---- library ------------------------------------------------------------ */

/* Message of the last failing call on this thread ("" if none). */
const char *tpp_last_error_string(void);
/* ABI version, (major << 16) | minor. */
int tpp_version(void);

/* ---- normalisation ------------------------------------------------------- */

/* y[m,:] = x[m,:] * rsqrt(mean(x[m,:]^2) + eps) * w, fp32 math, one rounding.
 * x: [M, ldx] rows of N valid elements, y: [M, ldy], w: [N].
 * Replaces launch_rmsnorm_fp16 (csrc/dlops/rmsnorm/rmsnorm_binding.cu:11-16)
 * and the kernel it launches (rmsnorm_fp16.cuh:43-137); adds bf16 and row
 * strides. */
int tpp_rmsnorm(const void *x, const void *w, void *y, int64_t M, int64_t N,
                int64_t ldx, int64_t ldy, float eps, int dtype, void *stream);

/* Test hook: inv_rms[m] = rsqrt(mean(x[m,:]^2) + eps) in fp32, the statistic
 * computed at rmsnorm_fp16.cuh:93-95. */
int tpp_rmsnorm_stats(const void *x, float *inv_rms, int64_t M, int64_t N,
                      int64_t ldx, float eps, int dtype, void *stream);

/* Fused residual add + RMSNorm (decoder block entry,
 * examples/LLM/fastqwen3.py:107-116):
 *   h = round(x + residual); residual <- h; y = rmsnorm(h) * w.
 * x, residual, y: [M, N] contiguous. residual is updated in place. */
int tpp_add_rmsnorm(const void *x, void *residual, const void *w, void *y,
                    int64_t M, int64_t N, float eps, int dtype, void *stream);

/* y = (x - mean) * rsqrt(var + eps) * w (+ b if b != NULL), fp32 stats.
 * Replaces launchLayerNorm (csrc/dlops/layernorm/layernorm_fp16.cuh:147-176,
 * bound at layernorm_binding.cu:7-43), which has no bias. */
int tpp_layernorm(const void *x, const void *w, const void *b, void *y,
                  int64_t M, int64_t N, int64_t ldx, int64_t ldy, float eps,
                  int dtype, void *stream);

/* Test hook: fp32 per-row mean and rstd of the LayerNorm above. */
int tpp_layernorm_stats(const void *x, float *mean, float *rstd, int64_t M,
                        int64_t N, int64_t ldx, float eps, int dtype,
                        void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TPP_H_ */
