/*
 * tpp.h -- C ABI of libtorchpp_hip.so, the gfx950 (MI355X) kernel set that
 * replaces torchpp's CUDA/CUTLASS native modules.
 *
 * Conventions shared by every entry point
 * ---------------------------------------
 *  - All tensor arguments are caller-owned DEVICE pointers. No entry point
 *    allocates device memory; ops that need scratch take a `workspace`
 *    pointer whose size is returned by the matching *_workspace_size call.
 *    (The first large plain GEMM on a device creates a hipBLASLt handle,
 *    which loads that library's kernels; its GEMMs use no workspace.)
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
  TPP_F32 = 2   /* float32 (RoPE cos/sin tables only)                     */
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

/* One-time checks of the current device for the kernels that synchronise
 * workgroups inside one XCD (the decode attention's in-kernel split merge,
 * the one-launch decode FFN): the CU count and a probe launch that records
 * each workgroup's XCD. Runs the probe on `stream` and synchronises it; fails
 * with TPP_E_INVALID while `stream` is being captured. Those kernels run the
 * same checks on their first call; a first call made during a capture cannot
 * probe and takes the unfused path (two launches, correct), so call this
 * before capturing a graph. *xcd_local (optional) = 1 if workgroups with
 * equal blockIdx % 8 share an XCD, *cu_count (optional) = the CU count (the
 * one-launch FFN needs 256). No counterpart in the reference, whose kernels
 * never exchange data inside a launch. */
int tpp_prepare_device(void *stream, int *xcd_local, int *cu_count);

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

/* ---- rotary embedding ---------------------------------------------------- */

/* Rotate-half RoPE on x [B, H, S, D] (contiguous) with tables cos/sin [S, D]
 * (row s for sequence index s). out may equal x (in place). cs_dtype is the
 * tables' type (TPP_F16, TPP_BF16 or TPP_F32, independent of dtype; the
 * reference's compute_rope_params returns fp16). fp32 math, one rounding.
 * Replaces rope_apply_half2 (csrc/dlops/rope/apply_rope.cuh:49-64), bound as
 * ropeApplyFunction.rope_apply_cuda (rope_binding.cu:10-67). */
int tpp_rope(const void *x, void *out, const void *cos, const void *sin,
             int64_t B, int64_t H, int64_t S, int64_t D, int dtype,
             int cs_dtype, void *stream);

/* RoPE on q [B, Hq, S, D] and k [B, Hk, S, D] in one launch; Hk may differ
 * from Hq (GQA). Replaces rope_apply_half2_dual
 * (csrc/dlops/qkrope/qkrope.cuh:69-93, qkrope_binding.cu:14-92), which
 * required Hk == Hq. */
int tpp_rope_qk(const void *q, const void *k, void *q_out, void *k_out,
                const void *cos, const void *sin, int64_t B, int64_t Hq,
                int64_t Hk, int64_t S, int64_t D, int dtype, int cs_dtype,
                void *stream);

/* Fused per-layer attention prologue, replacing the chain at
 * torchpp/attention/gqa.py:86-118 (q_norm/k_norm RMSNorm over head_dim,
 * rope_apply on Q and K, KVCache.update at kvcache.py:50-108):
 *   qkv      [B, S, (Hq + 2*Hkv) * D]  fused projection output
 *   q_out    [B, S, Hq, D]             normed + rotated queries
 *   k_cache, v_cache [B, Hkv, Lmax, D] rows pos[b]+s written (K normed+rotated)
 *   q_norm_w, k_norm_w [D] or NULL (no QK-norm)
 *   cos, sin [ctx, D] tables indexed by absolute position
 *   positions int32 [B] device array: first position of each sequence.
 * D must be 64, 128 or 256. Positions >= Lmax are not written. */
int tpp_qkv_rope_cache(const void *qkv, void *q_out, void *k_cache,
                       void *v_cache, const void *q_norm_w,
                       const void *k_norm_w, const void *cos, const void *sin,
                       int64_t ctx, const int32_t *positions, int64_t B,
                       int64_t S, int64_t Hq, int64_t Hkv, int64_t D,
                       int64_t Lmax, float eps, int dtype, int cs_dtype,
                       void *stream);

/* ---- linear layers ------------------------------------------------------- */

/* y[M, N] = act(T(x[M, K] . w[N, K]^T + bias)) on MFMA; w is the nn.Linear
 * weight layout, bias [N] or NULL, act a tpp_act. With act == TPP_ACT_NONE
 * and bias == NULL this is a plain GEMM. Rounding follows the reference
 * epilogue: pre-activation rounded to T, activation in fp32.
 * Replaces linearActvationFp16.LinearGelu/LinearSilu/LinearRelu
 * (csrc/activation/binding.cu:11-160, CUTLASS GEMM fused_gemm.cuh:143-170). */
int tpp_linear_act(const void *x, const void *w, const void *bias, void *y,
                   int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy,
                   int act, int dtype, void *stream);

/* Plain GEMMs of tpp_linear_act (no bias, no activation) with at least as
 * many 256 x 256 output tiles as the device has CUs run on hipBLASLt (zero
 * workspace, plan cached per shape), as the reference runs its plain projections on
 * nn.Linear (examples/LLM/fastqwen3.py:103-116); every other case, and any
 * shape hipBLASLt cannot plan, runs on the MFMA kernels. enable = 0 keeps
 * every GEMM on the MFMA kernels (also set by TPP_GEMM_VENDOR=0 in the
 * environment), 1 restores the dispatch, a negative value only queries.
 * Returns the previous setting. No counterpart in the reference: for
 * comparing the two backends on one shape. */
int tpp_gemm_vendor(int enable);

/* Number of GEMMs hipBLASLt has run in this process (all devices). No
 * counterpart in the reference: lets a test see which backend ran. */
long long tpp_gemm_vendor_runs(void);

/* Fused gate/up SwiGLU FFN projection, y[M, I] = T(silu(T(g))) * T(u) with
 * g = x . Wg^T, u = x . Wu^T, from one weight w_gu [2I, K] whose rows are
 * interleaved in blocks of 32 (rows 64j..64j+31 = Wg rows 32j.., rows
 * 64j+32..64j+63 = Wu rows 32j..). I % 32 == 0. The eager form is
 * examples/TTS/dia/model.py:114-116 (silu(gate(x)) * up(x)), which the
 * reference's FastQwen3 FFN intends (examples/LLM/fastqwen3.py:66-79). */
int tpp_linear_swiglu(const void *x, const void *w_gu, void *y, int64_t M,
                      int64_t I, int64_t K, int64_t ldx, int64_t ldy,
                      int dtype, void *stream);

/* Decode GEMV, y[B, N] = act(T(x[B, K] . W[N, K]^T + bias)), B <= 16,
 * streaming W once for all B rows (MFMA 16x16x32 tiles of 16 weight rows, K
 * split across the waves of a block). bias may be NULL, act a tpp_act.
 * Replaces hgemvK128F16x4Kernel / launchHgemv
 * (csrc/blas/hgemv/hgemv_kernels.cuh:19-85), which had no binding. */
int tpp_gemv(const void *x, const void *W, const void *bias, void *y,
             int64_t B, int64_t N, int64_t K, int64_t ldx, int64_t ldy,
             int act, int dtype, void *stream);

/* Decode GEMV with the decoder-block fusions (x, y, residual contiguous):
 *   norm_w != NULL : the input is RMSNorm(x) * norm_w with eps (the
 *                    RmsNormFused before each projection, fastqwen3.py:108,114)
 *   residual != NULL: residual[B, N] <- T(residual + T(x W^T)) in place, y
 *                    unused (the residual adds of fastqwen3.py:111,116)
 *   swiglu != 0     : W is the interleaved [gate|up] weight of
 *                    tpp_linear_swiglu (N = 2I rows) and y is [B, I]. */
int tpp_gemv_fused(const void *x, const void *norm_w, float eps, const void *W,
                   void *y, void *residual, int64_t B, int64_t N, int64_t K,
                   int swiglu, int dtype, void *stream);

/* Workspace bytes of tpp_ffn_decode. The workspace must be 256-byte aligned
 * and zero-filled before its first use: its first 8 KiB hold counters that
 * every call leaves at zero again (calls of any shape may share it, nothing
 * else may write those bytes; calls that share it must be ordered). */
size_t tpp_ffn_decode_workspace_size(int64_t B, int64_t E, int64_t I);

/* The decoder block's FFN half for B <= 16 new tokens, in place on the
 * residual stream [B, E] (contiguous):
 *   residual <- T(residual + T(down(T(silu(T(g))) * T(u))))
 *   g, u = RMSNorm(residual) * norm_w . Wg^T, . Wu^T
 * replacing rms_norm2 -> ffn -> `x + x_res` of the reference block
 * (examples/LLM/fastqwen3.py:113-116) with the SwiGLU FFN it intends
 * (fastqwen3.py:66-79; examples/TTS/dia/model.py:114-116). w_gu is the
 * interleaved [2I, E] gate/up weight of tpp_linear_swiglu, w_down the
 * nn.Linear weight [E, I]. For E = 1024, I in {1024, 2048, 3072, 4096} on a
 * 256-CU device the whole block is one launch (the down projection split
 * over the 8 XCDs, partials summed in a fixed order); otherwise, or if the
 * workgroup placement check fails, it is the two GEMV launches
 * (tpp_gemv_fused with swiglu, then with the residual). */
int tpp_ffn_decode(void *residual, const void *norm_w, float eps,
                   const void *w_gu, const void *w_down, int64_t B, int64_t E,
                   int64_t I, int dtype, void *workspace, size_t ws_bytes,
                   void *stream);

/* *out = nonzero if a one-launch tpp_ffn_decode on this workspace gave up
 * waiting for its workgroups since the last call. That launch needs all 256
 * workgroups resident at once; if they are not (other work holding CUs),
 * its bounded wait ends, a flag in the workspace is set, and its output is
 * WRONG. When the flag is set this call also zeroes the workspace's counter
 * region and the flag, so later launches are correct again. Call it where
 * the caller synchronises anyway (after a decode loop) with no tpp_ffn_decode
 * on this workspace in flight; it synchronises `stream` and fails during
 * stream capture. No counterpart in the reference, whose kernels never wait
 * on one another. */
int tpp_ffn_decode_sync_errors(void *workspace, int *out, void *stream);

/* Workspace bytes of tpp_gemv_argmax (no initialisation required). */
size_t tpp_gemv_argmax_workspace_size(int64_t B, int64_t N);

/* lm_head + greedy sampling: logits = RMSNorm(x)*norm_w . W^T (norm_w may be
 * NULL; logits may be NULL), out_idx[b] = argmax_n logits[b, n] (first index
 * of the maximum of the T-rounded logits), replacing out_head + sample_greedy
 * (fastqwen3.py:187-188, torchpp/llmops/llm.py:181-186). */
int tpp_gemv_argmax(const void *x, const void *norm_w, float eps,
                    const void *W, void *logits, int64_t *out_idx, int64_t B,
                    int64_t N, int64_t K, int dtype, void *workspace,
                    size_t ws_bytes, void *stream);

/* One greedy decode step's tail: token[b] = argmax of RMSNorm(x)*norm_w . W^T
 * (as tpp_gemv_argmax, no logits written), ids[b] = token[b], the next step's
 * hidden row resid_next[b, :] = emb[token[b], :] (emb [vocab, K], vocab = N),
 * positions[b] += 1 and seqlens[b] += 1 (either may be NULL). Replaces the
 * sample_greedy -> torch.cat -> tok_emb -> pos += 1 tail of the generation
 * loop (torchpp/llmops/llm.py:181-186, 226-236; fastqwen3.py:165-188).
 * Workspace as tpp_gemv_argmax_workspace_size(B, N). */
int tpp_greedy_step(const void *x, const void *norm_w, float eps,
                    const void *W, const void *emb, int64_t *ids,
                    void *resid_next, int32_t *positions, int32_t *seqlens,
                    int64_t B, int64_t N, int64_t K, int dtype,
                    void *workspace, size_t ws_bytes, void *stream);

/* ---- attention ----------------------------------------------------------- */

/* Flash attention forward, the flash_attn_func contract used by the reference
 * (torchpp/attention/gqa.py:128, swa.py:85-89, mha.py:84, mqa.py:87,
 * ca.py:83; the in-repo csrc/attention/flash_attn.cuh:35-604 is an unbound
 * MHA-only spec):
 *   q, o [B, Sq, Hq, D]; k, v [B, Sk, Hkv, D]; each *_strides is
 *   {batch, seq, head} in elements, last dim contiguous. Hq % Hkv == 0
 *   (GQA/MQA). softmax_scale <= 0 means 1/sqrt(D). causal is aligned
 *   bottom-right; window_left/right < 0 = unbounded (causal forces right = 0).
 *   Rows with no visible key are 0. D <= 256; D in {64, 128} with 16-byte
 *   aligned strides runs the MFMA kernel, other shapes a slow generic one. */
int tpp_attn_prefill(const void *q, const void *k, const void *v, void *o,
                     const int64_t *q_strides, const int64_t *k_strides,
                     const int64_t *v_strides, const int64_t *o_strides,
                     int64_t B, int64_t Sq, int64_t Sk, int64_t Hq,
                     int64_t Hkv, int64_t D, float softmax_scale, int causal,
                     int window_left, int window_right, int dtype,
                     void *stream);

/* Bytes of workspace tpp_attn_decode needs. The workspace must be 128-byte
 * aligned and its first 64 KiB zero-filled before the first use: they hold
 * per-(batch, KV head) arrival counters that every call leaves at zero
 * again (calls of any shape may share the workspace, but nothing else may
 * write those bytes). Calls that share it must be ordered (e.g. one stream). */
size_t tpp_attn_decode_workspace_size(int64_t B, int64_t Hq, int64_t Hkv,
                                      int64_t D, int64_t Lmax);

/* Split-KV decode attention: one query per sequence (q, o [B, 1, Hq, D]
 * through {batch, -, head} strides) against the first seqlens[b] keys of a
 * KV cache addressed by {batch, position, head} strides (the KVCache layout
 * [B, Hkv, Lmax, D] of torchpp/llmops/kvcache.py:39-48, batch-generalised).
 * seqlens: int32 [B] on the device, or NULL for Lmax keys everywhere.
 * window_left >= 0 keeps keys >= L-1-window_left. D in {64, 128},
 * Hq/Hkv <= 8. Replaces flash_attn_func with Sq = 1 over the cache prefix
 * (gqa.py:117-128). */
int tpp_attn_decode(const void *q, const void *k_cache, const void *v_cache,
                    void *o, const int64_t *q_strides, const int64_t *k_strides,
                    const int64_t *v_strides, const int64_t *o_strides,
                    const int32_t *seqlens, int64_t B, int64_t Hq, int64_t Hkv,
                    int64_t D, int64_t Lmax, float softmax_scale,
                    int window_left, int dtype, void *workspace,
                    size_t ws_bytes, void *stream);

/* tpp_attn_decode without a workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. The
 * kernels run on a 4 MiB static device array held by each GPU the library
 * runs on until the process ends; shapes whose split plan needs more than
 * that (tpp_attn_decode_workspace_size > 4 MiB) are rejected with
 * TPP_E_UNSUPPORTED. The first call on a device sets the array up (with that
 * device current) and queues a small fill kernel on `stream`. All calls on
 * one GPU share the array: calls that overlap on one GPU (e.g. on two
 * streams without ordering) race. Never calls hipMalloc/hipFree. Arguments
 * and results as tpp_attn_decode. */
int tpp_attn_decode_noalloc(const void *q, const void *k_cache,
                            const void *v_cache, void *o,
                            const int64_t *q_strides, const int64_t *k_strides,
                            const int64_t *v_strides, const int64_t *o_strides,
                            const int32_t *seqlens, int64_t B, int64_t Hq,
                            int64_t Hkv, int64_t D, int64_t Lmax,
                            float softmax_scale, int window_left, int dtype,
                            void *stream);

/* Decode attention with the per-layer prologue fused in (replaces
 * tpp_qkv_rope_cache + tpp_attn_decode for one new token per sequence): the
 * new token's raw projection qkv [B, (Hq + 2*Hkv) * D] is split into heads,
 * q and k get RMSNorm over D (q_norm_w / k_norm_w, NULL = none) and RoPE at
 * position seqlens[b] - 1 (tables cos/sin [ctx, D] of type cs_dtype), the new
 * k and v are written into the caches at that position, and the query
 * attends to keys [0, seqlens[b]) (the cache prefix plus the new key).
 * Caches/o/workspace as in tpp_attn_decode; seqlens is required. */
int tpp_attn_decode_fused(const void *qkv, const void *q_norm_w,
                          const void *k_norm_w, const void *cos,
                          const void *sin, int64_t ctx, int cs_dtype, float eps,
                          void *k_cache, void *v_cache, void *o,
                          const int64_t *k_strides, const int64_t *v_strides,
                          const int64_t *o_strides, const int32_t *seqlens,
                          int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                          int64_t Lmax, float softmax_scale, int window_left,
                          int dtype, void *workspace, size_t ws_bytes,
                          void *stream);

/* Workspace bytes of tpp_attn_decode_oproj (256-byte aligned, zero-filled
 * before first use; counters in it are left at zero by every call; it may be
 * shared with tpp_attn_decode / tpp_attn_decode_fused calls, in order). */
size_t tpp_attn_decode_oproj_workspace_size(int64_t B, int64_t Hq, int64_t Hkv,
                                            int64_t D, int64_t Lmax, int64_t E);

/* tpp_attn_decode_fused followed by the attention block's output projection
 * and residual add (the `x + x_res` after GroupedQueryAttention,
 * torchpp/attention/gqa.py:128-131 and examples/LLM/fastqwen3.py:107-111):
 *   o = attention output [B, 1, Hq, D] (contiguous, rounded to T)
 *   residual[B, E] <- T(residual + T(o W^T)),  W = w_o [E, Hq * D]
 * For Hkv = 8, D = 128, Hq in {8, 16}, E = 1024, B in {1, 2, 4, 8, 16} on
 * a 256-CU device whose workgroup placement probe holds (see
 * tpp_prepare_device) this is ONE launch: the XCD of KV head x computes the
 * projection over its heads' K slice and the 8 slices are summed in a fixed
 * order; that launch needs all 256 workgroups resident at once and reports a
 * failed wait through tpp_attn_decode_oproj_sync_errors. Otherwise it is
 * tpp_attn_decode_fused + tpp_gemv_fused (two launches). `o` is always
 * written. No counterpart in the reference, which runs the projection as a
 * separate nn.Linear. */
int tpp_attn_decode_oproj(const void *qkv, const void *q_norm_w,
                          const void *k_norm_w, const void *cos,
                          const void *sin, int64_t ctx, int cs_dtype, float eps,
                          void *k_cache, void *v_cache, void *o,
                          const int64_t *k_strides, const int64_t *v_strides,
                          const int32_t *seqlens, const void *w_o,
                          void *residual, int64_t B, int64_t Hq, int64_t Hkv,
                          int64_t D, int64_t Lmax, int64_t E,
                          float softmax_scale, int window_left, int dtype,
                          void *workspace, size_t ws_bytes, void *stream);

/* *out = nonzero if a one-launch tpp_attn_decode_oproj on this workspace
 * gave up waiting for its workgroups since the last call (its residual
 * update is WRONG); the flag and the counters are then zeroed. Same calling
 * rules as tpp_ffn_decode_sync_errors. */
int tpp_attn_decode_oproj_sync_errors(void *workspace, int *out, void *stream);

/* Test hook: marks a workspace as if a one-launch decode kernel had given up
 * waiting (kernel 0: tpp_attn_decode_oproj, 1: tpp_ffn_decode): sets its flag
 * and leaves a stray arrival count, by host copies; synchronises `stream`.
 * For tests of the error path that must not make a kernel wait. No
 * counterpart in the reference. */
int tpp_decode_force_sync_error(void *workspace, int kernel, void *stream);

/* ---- sampling ------------------------------------------------------------ */

/* Greedy sampling: out[b] = argmax_n x[b, n] for x [B, ldx] (first index of
 * the maximum, NaN is the maximum), as torch.argmax in
 * LLMInference.sample_greedy (torchpp/llmops/llm.py:181-186). */
int tpp_argmax_rows(const void *x, int64_t *out, int64_t B, int64_t N,
                    int64_t ldx, int dtype, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* TPP_H_ */
