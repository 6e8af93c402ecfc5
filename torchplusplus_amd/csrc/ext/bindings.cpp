// Torch extension over the C ABI of libtorchpp_hip.so (include/tpp.h).
//
// It keeps the function names, argument order and error behaviour of the
// reference's five pybind11 modules:
//   rmsnormFused.rmsnormFused            csrc/dlops/rmsnorm/rmsnorm_binding.cu:20-73
//   layernormFused.applyLayernorm        csrc/dlops/layernorm/layernorm_binding.cu:7-47
//   ropeApplyFunction.rope_apply_cuda    csrc/dlops/rope/rope_binding.cu:10-72
//   qkropeApplyFunction.qkrope_apply_cuda csrc/dlops/qkrope/qkrope_binding.cu:14-101
//   linearActvationFp16.Linear{Gelu,Silu,Relu} csrc/activation/binding.cu:11-166
// and adds bf16 everywhere, optional bias, N-D inputs and the decode/attention
// entry points. Outputs are allocated with torch's caching allocator; kernels
// run on the current HIP stream of the input's device.
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include <limits>
#include <vector>

#include "include/tpp.h"

namespace {

int dtype_code(const at::Tensor &t) {
  switch (t.scalar_type()) {
  case at::kHalf: return TPP_F16;
  case at::kBFloat16: return TPP_BF16;
  case at::kFloat: return TPP_F32;
  default: return -1;
  }
}

void *cur_stream(const at::Tensor &t) {
  return (void *)c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void check_rc(int rc, const char *what) {
  TORCH_CHECK(rc == TPP_OK, what, " failed: ", tpp_last_error_string());
}

bool is_half_or_bf16(const at::Tensor &t) {
  return t.scalar_type() == at::kHalf || t.scalar_type() == at::kBFloat16;
}

// Flatten [..., N] -> (M, N).
void rows_cols(const at::Tensor &x, int64_t &M, int64_t &N) {
  N = x.size(x.dim() - 1);
  M = 1;
  for (int i = 0; i < x.dim() - 1; ++i) M *= x.size(i);
}

// ---- RMSNorm (rmsnorm_binding.cu:20-68) -----------------------------------
at::Tensor rmsnorm_fused(at::Tensor input, at::Tensor weight, double eps) {
  TORCH_CHECK(input.is_cuda(), "input must be CUDA");
  TORCH_CHECK(weight.is_cuda(), "weight must be CUDA");
  TORCH_CHECK(is_half_or_bf16(input), "input must be half or bfloat16");
  TORCH_CHECK(weight.scalar_type() == input.scalar_type(),
              "weight must have the input's dtype (half or bfloat16)");
  TORCH_CHECK(input.dim() >= 2,
              "expected input to have >= 2 dims (leading dims..., embed_dim)");
  if (!input.is_contiguous()) input = input.contiguous();
  if (!weight.is_contiguous()) weight = weight.contiguous();
  int64_t M, N;
  rows_cols(input, M, N);
  TORCH_CHECK(weight.dim() == 1 && weight.size(0) == N,
              "weight must be 1-D and length == embed_dim");
  TORCH_CHECK(M > 0 && N > 0, "invalid shapes");
  TORCH_CHECK(M <= std::numeric_limits<int>::max() &&
                  N <= std::numeric_limits<int>::max(),
              "M or N too large for kernel (must fit in 32-bit int)");
  c10::DeviceGuard g(input.device());
  auto out = torch::empty_like(input);
  check_rc(tpp_rmsnorm(input.data_ptr(), weight.data_ptr(), out.data_ptr(), M, N, N,
                       N, (float)eps, dtype_code(input), cur_stream(input)),
           "rmsnormFused");
  return out;
}

at::Tensor rmsnorm_stats(at::Tensor input, double eps) {
  TORCH_CHECK(input.is_cuda() && is_half_or_bf16(input),
              "input must be a CUDA half/bfloat16 tensor");
  input = input.contiguous();
  int64_t M, N;
  rows_cols(input, M, N);
  c10::DeviceGuard g(input.device());
  auto out = torch::empty({M}, input.options().dtype(at::kFloat));
  check_rc(tpp_rmsnorm_stats(input.data_ptr(), out.data_ptr<float>(), M, N, N,
                             (float)eps, dtype_code(input), cur_stream(input)),
           "rmsnorm_stats");
  return out;
}

// residual <- x + residual ; returns rmsnorm(residual) * weight
at::Tensor add_rmsnorm(at::Tensor x, at::Tensor residual, at::Tensor weight,
                       double eps) {
  TORCH_CHECK(x.is_cuda() && residual.is_cuda() && weight.is_cuda(),
              "tensors must be CUDA");
  TORCH_CHECK(is_half_or_bf16(x), "input must be half or bfloat16");
  TORCH_CHECK(residual.scalar_type() == x.scalar_type() &&
                  weight.scalar_type() == x.scalar_type(),
              "dtype mismatch");
  TORCH_CHECK(x.is_contiguous() && residual.is_contiguous() && weight.is_contiguous(),
              "tensors must be contiguous");
  TORCH_CHECK(x.sizes() == residual.sizes(), "x and residual shapes differ");
  int64_t M, N;
  rows_cols(x, M, N);
  TORCH_CHECK(weight.dim() == 1 && weight.size(0) == N,
              "weight must be 1-D and length == embed_dim");
  c10::DeviceGuard g(x.device());
  auto out = torch::empty_like(x);
  check_rc(tpp_add_rmsnorm(x.data_ptr(), residual.data_ptr(), weight.data_ptr(),
                           out.data_ptr(), M, N, (float)eps, dtype_code(x),
                           cur_stream(x)),
           "add_rmsnorm");
  return out;
}

// ---- LayerNorm (layernorm_binding.cu:7-43) --------------------------------
at::Tensor layernorm_forward(at::Tensor input, at::Tensor weight, double eps,
                             c10::optional<at::Tensor> bias) {
  TORCH_CHECK(input.is_cuda(), "Input tensor must be on CUDA");
  TORCH_CHECK(weight.is_cuda(), "Weight tensor must be on CUDA");
  TORCH_CHECK(is_half_or_bf16(input), "Input must be float16 or bfloat16");
  TORCH_CHECK(weight.scalar_type() == input.scalar_type(),
              "Weight must have the input's dtype");
  TORCH_CHECK(input.is_contiguous(), "Input must be contiguous");
  TORCH_CHECK(weight.is_contiguous(), "Weight must be contiguous");
  TORCH_CHECK(input.dim() >= 2, "Input must be at least 2D");
  int64_t M, N;
  rows_cols(input, M, N);
  TORCH_CHECK(weight.numel() == N, "Weight size must match last dimension of input");
  const void *bp = nullptr;
  if (bias.has_value() && bias->defined()) {
    TORCH_CHECK(bias->is_cuda() && bias->scalar_type() == input.scalar_type() &&
                    bias->is_contiguous() && bias->numel() == N,
                "bias must be a contiguous CUDA tensor of length N with the input's dtype");
    bp = bias->data_ptr();
  }
  c10::DeviceGuard g(input.device());
  auto out = torch::empty_like(input);
  check_rc(tpp_layernorm(input.data_ptr(), weight.data_ptr(), bp, out.data_ptr(), M, N,
                         N, N, (float)eps, dtype_code(input), cur_stream(input)),
           "applyLayernorm");
  return out;
}

std::vector<at::Tensor> layernorm_stats(at::Tensor input, double eps) {
  TORCH_CHECK(input.is_cuda() && is_half_or_bf16(input),
              "input must be a CUDA half/bfloat16 tensor");
  input = input.contiguous();
  int64_t M, N;
  rows_cols(input, M, N);
  c10::DeviceGuard g(input.device());
  auto mean = torch::empty({M}, input.options().dtype(at::kFloat));
  auto rstd = torch::empty({M}, input.options().dtype(at::kFloat));
  check_rc(tpp_layernorm_stats(input.data_ptr(), mean.data_ptr<float>(),
                               rstd.data_ptr<float>(), M, N, N, (float)eps,
                               dtype_code(input), cur_stream(input)),
           "layernorm_stats");
  return {mean, rstd};
}

// ---- RoPE (rope_binding.cu:10-67, qkrope_binding.cu:14-92) -----------------
void check_rope_tables(const at::Tensor &x, const at::Tensor &cos_cache,
                       const at::Tensor &sin_cache, int64_t N, int64_t D) {
  TORCH_CHECK(cos_cache.device().is_cuda(), "cos_cache tensor must be on CUDA device");
  TORCH_CHECK(sin_cache.device().is_cuda(), "sin_cache tensor must be on CUDA device");
  TORCH_CHECK(dtype_code(cos_cache) >= 0,
              "cos_cache tensor must be float16, bfloat16 or float32");
  TORCH_CHECK(sin_cache.scalar_type() == cos_cache.scalar_type(),
              "sin_cache tensor must have cos_cache's dtype");
  TORCH_CHECK(cos_cache.is_contiguous(), "cos_cache tensor must be contiguous");
  TORCH_CHECK(sin_cache.is_contiguous(), "sin_cache tensor must be contiguous");
  TORCH_CHECK(cos_cache.dim() == 2, "cos_cache must be 2D [seq_len, head_dim]");
  TORCH_CHECK(sin_cache.dim() == 2, "sin_cache must be 2D [seq_len, head_dim]");
  TORCH_CHECK(cos_cache.size(0) == N && cos_cache.size(1) == D, "cos_cache shape mismatch");
  TORCH_CHECK(sin_cache.size(0) == N && sin_cache.size(1) == D, "sin_cache shape mismatch");
}

at::Tensor rope_apply_impl(at::Tensor x, at::Tensor cos_cache, at::Tensor sin_cache,
                           bool inplace) {
  TORCH_CHECK(x.device().is_cuda(), "Input tensor must be on CUDA device");
  TORCH_CHECK(is_half_or_bf16(x), "Input tensor must be float16 or bfloat16");
  TORCH_CHECK(x.is_contiguous(), "Input tensor must be contiguous");
  TORCH_CHECK(x.dim() == 4, "Input tensor must be 4D [batch, heads, seq_len, head_dim]");
  const int64_t B = x.size(0), H = x.size(1), N = x.size(2), D = x.size(3);
  TORCH_CHECK(D % 2 == 0, "head dim must be even");
  check_rope_tables(x, cos_cache, sin_cache, N, D);
  c10::DeviceGuard g(x.device());
  at::Tensor out = inplace ? x : torch::empty_like(x);
  check_rc(tpp_rope(x.data_ptr(), out.data_ptr(), cos_cache.data_ptr(), sin_cache.data_ptr(),
                    B, H, N, D, dtype_code(x), dtype_code(cos_cache), cur_stream(x)),
           "rope_apply_cuda");
  return out;
}

at::Tensor rope_apply_cuda(at::Tensor x, at::Tensor cos_cache, at::Tensor sin_cache) {
  return rope_apply_impl(x, cos_cache, sin_cache, false);
}
at::Tensor rope_apply_inplace(at::Tensor x, at::Tensor cos_cache, at::Tensor sin_cache) {
  return rope_apply_impl(x, cos_cache, sin_cache, true);
}

std::vector<at::Tensor> qkrope_apply_cuda(at::Tensor q, at::Tensor k, at::Tensor cos_cache,
                                          at::Tensor sin_cache) {
  TORCH_CHECK(q.device().is_cuda(), "Query tensor must be on CUDA device");
  TORCH_CHECK(is_half_or_bf16(q), "Query tensor must be float16 or bfloat16");
  TORCH_CHECK(q.is_contiguous(), "Query tensor must be contiguous");
  TORCH_CHECK(k.device().is_cuda(), "Key tensor must be on CUDA device");
  TORCH_CHECK(k.scalar_type() == q.scalar_type(), "Key tensor must have the query dtype");
  TORCH_CHECK(k.is_contiguous(), "Key tensor must be contiguous");
  TORCH_CHECK(q.dim() == 4, "Query tensor must be 4D [batch, heads, seq_len, head_dim]");
  TORCH_CHECK(k.dim() == 4, "Key tensor must be 4D [batch, heads, seq_len, head_dim]");
  const int64_t B = q.size(0), H = q.size(1), N = q.size(2), D = q.size(3);
  TORCH_CHECK(D % 2 == 0, "head_dim must be even");
  TORCH_CHECK(k.size(0) == B, "Key batch size must match query");
  TORCH_CHECK(k.size(1) <= H && H % k.size(1) == 0,
              "Key num_heads must divide query num_heads (GQA)");
  TORCH_CHECK(k.size(2) == N, "Key seq_len must match query");
  TORCH_CHECK(k.size(3) == D, "Key head_dim must match query");
  check_rope_tables(q, cos_cache, sin_cache, N, D);
  c10::DeviceGuard g(q.device());
  auto qo = torch::empty_like(q);
  auto ko = torch::empty_like(k);
  check_rc(tpp_rope_qk(q.data_ptr(), k.data_ptr(), qo.data_ptr(), ko.data_ptr(),
                       cos_cache.data_ptr(), sin_cache.data_ptr(), B, H, k.size(1), N, D,
                       dtype_code(q), dtype_code(cos_cache), cur_stream(q)),
           "qkrope_apply_cuda");
  return {qo, ko};
}

void qkv_rope_cache(at::Tensor qkv, at::Tensor q_out, at::Tensor k_cache, at::Tensor v_cache,
                    c10::optional<at::Tensor> q_norm_w, c10::optional<at::Tensor> k_norm_w,
                    at::Tensor cos, at::Tensor sin, at::Tensor positions, double eps) {
  TORCH_CHECK(qkv.is_cuda() && qkv.is_contiguous() && is_half_or_bf16(qkv),
              "qkv must be a contiguous CUDA half/bfloat16 tensor [B, S, (Hq+2Hkv)*D]");
  TORCH_CHECK(q_out.dim() == 4 && q_out.is_contiguous() &&
                  q_out.scalar_type() == qkv.scalar_type(),
              "q_out must be contiguous [B, S, Hq, D]");
  TORCH_CHECK(k_cache.dim() == 4 && k_cache.is_contiguous() && v_cache.is_contiguous() &&
                  k_cache.sizes() == v_cache.sizes() &&
                  k_cache.scalar_type() == qkv.scalar_type() &&
                  v_cache.scalar_type() == qkv.scalar_type(),
              "caches must be contiguous [B, Hkv, Lmax, D] of the qkv dtype");
  TORCH_CHECK(positions.is_cuda() && positions.scalar_type() == at::kInt &&
                  positions.numel() == q_out.size(0),
              "positions must be a CUDA int32 tensor of length B");
  const int64_t B = q_out.size(0), S = q_out.size(1), Hq = q_out.size(2), D = q_out.size(3);
  const int64_t Hkv = k_cache.size(1), Lmax = k_cache.size(2);
  TORCH_CHECK(k_cache.size(0) == B && k_cache.size(3) == D, "cache shape mismatch");
  TORCH_CHECK(qkv.numel() == B * S * (Hq + 2 * Hkv) * D, "qkv size mismatch");
  TORCH_CHECK(cos.is_contiguous() && sin.is_contiguous() && cos.dim() == 2 &&
                  cos.size(1) == D && sin.sizes() == cos.sizes() &&
                  sin.scalar_type() == cos.scalar_type(),
              "cos/sin must be contiguous [ctx, D] tables");
  TORCH_CHECK(cos.size(0) >= Lmax, "cos/sin hold ", cos.size(0),
              " positions, fewer than the cache length ", Lmax);
  const void *qw = nullptr, *kw = nullptr;
  if (q_norm_w.has_value() && q_norm_w->defined()) {
    TORCH_CHECK(q_norm_w->numel() == D && q_norm_w->scalar_type() == qkv.scalar_type() &&
                    q_norm_w->is_contiguous(),
                "q_norm weight must be [D] of the qkv dtype");
    qw = q_norm_w->data_ptr();
  }
  if (k_norm_w.has_value() && k_norm_w->defined()) {
    TORCH_CHECK(k_norm_w->numel() == D && k_norm_w->scalar_type() == qkv.scalar_type() &&
                    k_norm_w->is_contiguous(),
                "k_norm weight must be [D] of the qkv dtype");
    kw = k_norm_w->data_ptr();
  }
  c10::DeviceGuard g(qkv.device());
  check_rc(tpp_qkv_rope_cache(qkv.data_ptr(), q_out.data_ptr(), k_cache.data_ptr(),
                              v_cache.data_ptr(), qw, kw, cos.data_ptr(), sin.data_ptr(),
                              cos.size(0), positions.data_ptr<int32_t>(), B, S, Hq, Hkv, D,
                              Lmax, (float)eps, dtype_code(qkv), dtype_code(cos),
                              cur_stream(qkv)),
           "qkv_rope_cache");
}

// ---- Linear + activation (binding.cu:11-160) --------------------------------
void check_linear(const at::Tensor &input, const at::Tensor &weight) {
  TORCH_CHECK(input.dim() >= 1, "Input must be at least 1D");
  TORCH_CHECK(weight.dim() == 2, "Weight must be 2D");
  TORCH_CHECK(input.size(input.dim() - 1) == weight.size(1), "Dimension mismatch");
  TORCH_CHECK(is_half_or_bf16(input), "Input must be FP16 or BF16");
  TORCH_CHECK(weight.scalar_type() == input.scalar_type(), "Weight must have the input dtype");
  TORCH_CHECK(input.is_cuda(), "Input must be on CUDA");
  TORCH_CHECK(weight.is_cuda(), "Weight must be on CUDA");
  TORCH_CHECK(input.is_contiguous(), "Input must be contiguous");
  TORCH_CHECK(weight.is_contiguous(), "Weight must be contiguous");
}

const void *bias_ptr(const c10::optional<at::Tensor> &bias, const at::Tensor &input,
                     int64_t N) {
  if (!bias.has_value() || !bias->defined()) return nullptr;
  TORCH_CHECK(bias->is_cuda() && bias->scalar_type() == input.scalar_type() &&
                  bias->is_contiguous() && bias->numel() == N,
              "bias must be a contiguous CUDA tensor [N] of the input dtype");
  return bias->data_ptr();
}

std::vector<int64_t> out_shape(const at::Tensor &input, int64_t N) {
  auto s = input.sizes().vec();
  s.back() = N;
  return s;
}

at::Tensor linear_act(at::Tensor input, at::Tensor weight, c10::optional<at::Tensor> bias,
                      int64_t act) {
  check_linear(input, weight);
  const int64_t K = weight.size(1), N = weight.size(0), M = input.numel() / K;
  const void *bp = bias_ptr(bias, input, N);
  c10::DeviceGuard g(input.device());
  auto out = torch::empty(out_shape(input, N), input.options());
  check_rc(tpp_linear_act(input.data_ptr(), weight.data_ptr(), bp, out.data_ptr(), M, N, K, K,
                          N, (int)act, dtype_code(input), cur_stream(input)),
           "linear_act");
  return out;
}

at::Tensor linear_gelu(at::Tensor i, at::Tensor w, c10::optional<at::Tensor> b) {
  return linear_act(i, w, b, TPP_ACT_GELU_TANH);
}
at::Tensor linear_silu(at::Tensor i, at::Tensor w, c10::optional<at::Tensor> b) {
  return linear_act(i, w, b, TPP_ACT_SILU);
}
at::Tensor linear_relu(at::Tensor i, at::Tensor w, c10::optional<at::Tensor> b) {
  return linear_act(i, w, b, TPP_ACT_RELU);
}

at::Tensor linear_swiglu(at::Tensor input, at::Tensor w_gu) {
  check_linear(input, w_gu);
  const int64_t K = w_gu.size(1), I = w_gu.size(0) / 2, M = input.numel() / K;
  TORCH_CHECK(w_gu.size(0) % 64 == 0, "w_gu rows must be a multiple of 64");
  c10::DeviceGuard g(input.device());
  auto out = torch::empty(out_shape(input, I), input.options());
  check_rc(tpp_linear_swiglu(input.data_ptr(), w_gu.data_ptr(), out.data_ptr(), M, I, K, K, I,
                             dtype_code(input), cur_stream(input)),
           "linear_swiglu");
  return out;
}

void check_rows16(const at::Tensor &input, int64_t K) {
  const int64_t B = input.numel() / K;
  TORCH_CHECK(B >= 1 && B <= 16, "gemv supports 1..16 input rows, got ", B);
}

at::Tensor gemv(at::Tensor input, at::Tensor weight, c10::optional<at::Tensor> bias,
                int64_t act) {
  check_linear(input, weight);
  const int64_t K = weight.size(1), N = weight.size(0), B = input.numel() / K;
  check_rows16(input, K);
  const void *bp = bias_ptr(bias, input, N);
  c10::DeviceGuard g(input.device());
  auto out = torch::empty(out_shape(input, N), input.options());
  check_rc(tpp_gemv(input.data_ptr(), weight.data_ptr(), bp, out.data_ptr(), B, N, K, K, N,
                    (int)act, dtype_code(input), cur_stream(input)),
           "gemv");
  return out;
}

const void *norm_ptr(const c10::optional<at::Tensor> &nw, const at::Tensor &input, int64_t K) {
  if (!nw.has_value() || !nw->defined()) return nullptr;
  TORCH_CHECK(nw->is_cuda() && nw->scalar_type() == input.scalar_type() &&
                  nw->is_contiguous() && nw->numel() == K,
              "norm weight must be a contiguous CUDA tensor [K] of the input dtype");
  return nw->data_ptr();
}

// y = [norm](x) @ W^T, or residual += [norm](x) @ W^T (returns residual)
at::Tensor gemv_fused(at::Tensor input, at::Tensor weight, c10::optional<at::Tensor> norm_w,
                      double eps, c10::optional<at::Tensor> residual) {
  check_linear(input, weight);
  const int64_t K = weight.size(1), N = weight.size(0), B = input.numel() / K;
  check_rows16(input, K);
  const void *nw = norm_ptr(norm_w, input, K);
  c10::DeviceGuard g(input.device());
  if (residual.has_value() && residual->defined()) {
    TORCH_CHECK(residual->is_cuda() && residual->is_contiguous() &&
                    residual->scalar_type() == input.scalar_type() && residual->numel() == B * N,
                "residual must be a contiguous [B, N] tensor of the input dtype");
    check_rc(tpp_gemv_fused(input.data_ptr(), nw, (float)eps, weight.data_ptr(), nullptr,
                            residual->data_ptr(), B, N, K, 0, dtype_code(input),
                            cur_stream(input)),
             "gemv_fused");
    return *residual;
  }
  auto out = torch::empty(out_shape(input, N), input.options());
  check_rc(tpp_gemv_fused(input.data_ptr(), nw, (float)eps, weight.data_ptr(), out.data_ptr(),
                          nullptr, B, N, K, 0, dtype_code(input), cur_stream(input)),
           "gemv_fused");
  return out;
}

at::Tensor gemv_swiglu(at::Tensor input, at::Tensor w_gu, c10::optional<at::Tensor> norm_w,
                       double eps) {
  check_linear(input, w_gu);
  const int64_t K = w_gu.size(1), N = w_gu.size(0), B = input.numel() / K;
  check_rows16(input, K);
  TORCH_CHECK(N % 64 == 0, "w_gu rows must be a multiple of 64");
  const void *nw = norm_ptr(norm_w, input, K);
  c10::DeviceGuard g(input.device());
  auto out = torch::empty(out_shape(input, N / 2), input.options());
  check_rc(tpp_gemv_fused(input.data_ptr(), nw, (float)eps, w_gu.data_ptr(), out.data_ptr(),
                          nullptr, B, N, K, 1, dtype_code(input), cur_stream(input)),
           "gemv_swiglu");
  return out;
}

// greedy lm_head: returns (token ids [B] int64, logits or None)
std::vector<at::Tensor> gemv_argmax(at::Tensor input, at::Tensor weight,
                                    c10::optional<at::Tensor> norm_w, double eps,
                                    bool return_logits) {
  check_linear(input, weight);
  const int64_t K = weight.size(1), N = weight.size(0), B = input.numel() / K;
  check_rows16(input, K);
  const void *nw = norm_ptr(norm_w, input, K);
  c10::DeviceGuard g(input.device());
  auto idx = torch::empty({B}, input.options().dtype(at::kLong));
  at::Tensor logits;
  if (return_logits) logits = torch::empty({B, N}, input.options());
  const size_t wsb = tpp_gemv_argmax_workspace_size(B, N);
  auto ws = torch::empty({(int64_t)((wsb + 3) / 4)}, input.options().dtype(at::kFloat));
  check_rc(tpp_gemv_argmax(input.data_ptr(), nw, (float)eps, weight.data_ptr(),
                           return_logits ? logits.data_ptr() : nullptr, idx.data_ptr<int64_t>(),
                           B, N, K, dtype_code(input), ws.data_ptr(), wsb, cur_stream(input)),
           "gemv_argmax");
  if (return_logits) return {idx, logits};
  return {idx};
}

// ---- attention (flash_attn_func contract) ----------------------------------
// Zero-filled per-device scratch, allocated once and reused, so a captured
// decode graph keeps one stable pointer (intentionally leaked: no tensor
// destructor runs after the caching allocator is torn down at exit). When a
// call needs more than the slot holds, a larger buffer replaces it for later
// calls, and the old one is kept alive (`retired`) until the process ends:
// a graph captured earlier still holds its address in its kernel arguments
// and keeps using it (its counters stay zero, since only that graph's calls
// touch it). Slots 1 (decode attention) and 2 (decode FFN) hold counters
// that must be zero before a call and that every call leaves at zero, which
// the kernels guarantee but another user of the same bytes would not; such a
// slot is therefore created or grown only outside stream capture (a zero
// fill recorded into a graph would leave the buffer unset for eager calls
// until the graph ran): the call is refused with a message instead. Calls
// that share a slot must not overlap, so a call on a stream other than the
// slot's last one first makes its stream wait for that stream (an event);
// while a stream is being captured the capture is ordered after earlier
// work by the caller (torch.cuda.graph synchronizes first).
struct ScratchSlot {
  at::Tensor t;
  std::vector<at::Tensor> retired;
  hipStream_t last = nullptr;
  hipEvent_t ev = nullptr;
};

constexpr int kSlots = 3; // 0: greedy-step argmax partials, 1: decode attention, 2: decode FFN

ScratchSlot &scratch_slot(int dev, int slot) {
  static std::vector<ScratchSlot> *cache = new std::vector<ScratchSlot>(64 * kSlots);
  TORCH_CHECK(dev >= 0 && dev < 64 && slot >= 0 && slot < kSlots, "device index out of range");
  return (*cache)[dev * kSlots + slot];
}

at::Tensor cached_workspace(const at::Tensor &like, size_t bytes, int slot = 0) {
  ScratchSlot &e = scratch_slot(like.device().index(), slot);
  hipStream_t s = (hipStream_t)cur_stream(like);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  TORCH_CHECK(hipStreamIsCapturing(s, &cs) == hipSuccess, "hipStreamIsCapturing failed");
  const bool capturing = cs != hipStreamCaptureStatusNone;
  if (!capturing && e.last && e.last != s) {
    if (!e.ev) TORCH_CHECK(hipEventCreateWithFlags(&e.ev, hipEventDisableTiming) == hipSuccess, "hipEventCreate failed");
    TORCH_CHECK(hipEventRecord(e.ev, e.last) == hipSuccess && hipStreamWaitEvent(s, e.ev, 0) == hipSuccess,
                "ordering the shared workspace between streams failed");
  }
  if (!e.t.defined() || (size_t)e.t.numel() * 4 < bytes) {
    TORCH_CHECK(!capturing || slot == 0,
                slot == 1 ? "attn_decode" : "ffn_decode",
                ": its device workspace is created (or grown) on the first call of a shape, which "
                "cannot be inside stream capture; run the call once before capturing");
    int64_t n = (int64_t)((bytes + 3) / 4);
    n = n < (1 << 20) ? (1 << 20) : n;
    if (e.t.defined()) e.retired.push_back(e.t);
    e.t = torch::zeros({n}, like.options().dtype(at::kFloat));
  }
  e.last = capturing ? nullptr : s;
  return e.t;
}

// decode FFN half of a decoder block, in place on the residual stream
void ffn_decode(at::Tensor residual, at::Tensor norm_w, double eps, at::Tensor w_gu,
                at::Tensor w_down) {
  TORCH_CHECK(residual.is_cuda() && is_half_or_bf16(residual) && residual.is_contiguous(),
              "residual must be a contiguous CUDA half/bfloat16 tensor [..., E]");
  const int64_t E = residual.size(-1), B = residual.numel() / E;
  TORCH_CHECK(B >= 1 && B <= 16, "ffn_decode handles 1 to 16 tokens");
  TORCH_CHECK(w_gu.dim() == 2 && w_gu.size(1) == E && w_gu.size(0) % 64 == 0 &&
                  w_gu.is_contiguous() && w_gu.scalar_type() == residual.scalar_type(),
              "w_gu must be a contiguous [2I, E] interleaved gate/up weight (2I % 64 == 0)");
  const int64_t I = w_gu.size(0) / 2;
  TORCH_CHECK(w_down.dim() == 2 && w_down.size(0) == E && w_down.size(1) == I &&
                  w_down.is_contiguous() && w_down.scalar_type() == residual.scalar_type(),
              "w_down must be a contiguous [E, I] weight");
  TORCH_CHECK(norm_w.numel() == E && norm_w.is_contiguous() &&
                  norm_w.scalar_type() == residual.scalar_type(),
              "norm weight must be [E] of the residual dtype");
  c10::DeviceGuard g(residual.device());
  const size_t wsb = tpp_ffn_decode_workspace_size(B, E, I);
  at::Tensor ws = cached_workspace(residual, wsb, 2);
  check_rc(tpp_ffn_decode(residual.data_ptr(), norm_w.data_ptr(), (float)eps, w_gu.data_ptr(),
                          w_down.data_ptr(), B, E, I, dtype_code(residual), ws.data_ptr(),
                          (size_t)ws.numel() * 4, cur_stream(residual)),
           "ffn_decode");
}

// nonzero if a one-launch decode FFN on this device gave up waiting for its
// workgroups (its output was wrong) since the last check; reads and clears
// the flag of every workspace the device's FFN calls may use (the current
// one and the retired ones that captured graphs still hold). Synchronises
// the current stream after ordering it behind the workspace's last stream.
int64_t ffn_decode_sync_errors(at::Tensor like) {
  TORCH_CHECK(like.is_cuda(), "ffn_decode_sync_errors: expected a CUDA tensor");
  c10::DeviceGuard g(like.device());
  ScratchSlot &e = scratch_slot(like.device().index(), 2);
  if (!e.t.defined()) return 0; // no FFN call on this device yet
  cached_workspace(like, 1, 2); // orders this stream after the slot's last one
  int64_t any = 0;
  auto check = [&](at::Tensor &t) {
    int out = 0;
    check_rc(tpp_ffn_decode_sync_errors(t.data_ptr(), &out, cur_stream(like)),
             "ffn_decode_sync_errors");
    any |= out;
  };
  check(e.t);
  for (auto &t : e.retired) check(t);
  return any;
}

// test hook: mark the device's current decode-attention (kernel 0) or decode
// FFN (kernel 1) workspace as if a one-launch kernel had given up waiting
void force_decode_sync_error(at::Tensor like, int64_t kernel) {
  TORCH_CHECK(like.is_cuda() && (kernel == 0 || kernel == 1), "force_decode_sync_error: bad arguments");
  c10::DeviceGuard g(like.device());
  ScratchSlot &e = scratch_slot(like.device().index(), kernel == 0 ? 1 : 2);
  TORCH_CHECK(e.t.defined(), "force_decode_sync_error: no workspace yet");
  cached_workspace(like, 1, kernel == 0 ? 1 : 2);
  check_rc(tpp_decode_force_sync_error(e.t.data_ptr(), (int)kernel, cur_stream(like)),
           "force_decode_sync_error");
}

// One-time device checks of the XCD-local kernels, outside capture
// (tpp_prepare_device): returns (workgroups with equal id % 8 share an XCD,
// CU count).
std::tuple<bool, int64_t> prepare_device(at::Tensor like) {
  TORCH_CHECK(like.is_cuda(), "prepare_device: expected a CUDA tensor");
  c10::DeviceGuard g(like.device());
  int xcd = 0, cus = 0;
  check_rc(tpp_prepare_device(cur_stream(like), &xcd, &cus), "prepare_device");
  return {xcd != 0, (int64_t)cus};
}

// greedy decode tail: ids <- argmax(lm_head(norm(input))), resid_next <-
// emb[ids], positions/seqlens += 1 (all in place)
void greedy_step(at::Tensor input, at::Tensor weight, c10::optional<at::Tensor> norm_w, double eps,
                 at::Tensor emb, at::Tensor ids, at::Tensor resid_next,
                 c10::optional<at::Tensor> positions, c10::optional<at::Tensor> seqlens) {
  check_linear(input, weight);
  const int64_t K = weight.size(1), N = weight.size(0), B = input.numel() / K;
  check_rows16(input, K);
  const void *nw = norm_ptr(norm_w, input, K);
  TORCH_CHECK(emb.is_cuda() && emb.scalar_type() == input.scalar_type() && emb.dim() == 2 &&
                  emb.size(0) == N && emb.size(1) == K && emb.is_contiguous(),
              "emb must be a contiguous [N, K] tensor of the input dtype");
  TORCH_CHECK(ids.is_cuda() && ids.scalar_type() == at::kLong && ids.numel() == B &&
                  ids.is_contiguous(),
              "ids must be a contiguous int64 tensor of B elements");
  TORCH_CHECK(resid_next.is_cuda() && resid_next.scalar_type() == input.scalar_type() &&
                  resid_next.numel() == B * K && resid_next.is_contiguous(),
              "resid_next must be a contiguous [B, K] tensor of the input dtype");
  auto i32 = [&](const c10::optional<at::Tensor> &t, const char *what) -> int32_t * {
    if (!t.has_value() || !t->defined()) return nullptr;
    TORCH_CHECK(t->is_cuda() && t->scalar_type() == at::kInt && t->numel() == B &&
                    t->is_contiguous(),
                what, " must be a contiguous int32 tensor of B elements");
    return t->data_ptr<int32_t>();
  };
  int32_t *pp = i32(positions, "positions"), *sp = i32(seqlens, "seqlens");
  c10::DeviceGuard g(input.device());
  const size_t wsb = tpp_gemv_argmax_workspace_size(B, N);
  auto ws = cached_workspace(input, wsb);
  check_rc(tpp_greedy_step(input.data_ptr(), nw, (float)eps, weight.data_ptr(), emb.data_ptr(),
                           ids.data_ptr<int64_t>(), resid_next.data_ptr(), pp, sp, B, N, K,
                           dtype_code(input), ws.data_ptr(), wsb, cur_stream(input)),
           "greedy_step");
}

void check_bshd(const at::Tensor &t, const char *what) {
  TORCH_CHECK(t.is_cuda(), what, " must be on CUDA");
  TORCH_CHECK(is_half_or_bf16(t), what, " must be float16 or bfloat16");
  TORCH_CHECK(t.dim() == 4, what, " must be 4D [batch, seqlen, heads, head_dim]");
  TORCH_CHECK(t.stride(3) == 1, what, " must have a contiguous last dimension");
}

at::Tensor attn_fwd(at::Tensor q, at::Tensor k, at::Tensor v, bool causal, int64_t window_left,
                    int64_t window_right, double softmax_scale) {
  check_bshd(q, "q");
  check_bshd(k, "k");
  check_bshd(v, "v");
  TORCH_CHECK(k.scalar_type() == q.scalar_type() && v.scalar_type() == q.scalar_type(),
              "q, k, v must share a dtype");
  const int64_t B = q.size(0), Sq = q.size(1), Hq = q.size(2), D = q.size(3);
  const int64_t Sk = k.size(1), Hkv = k.size(2);
  TORCH_CHECK(k.size(0) == B && v.size(0) == B, "batch size mismatch");
  TORCH_CHECK(k.size(3) == D && v.size(3) == D, "head_dim mismatch");
  TORCH_CHECK(v.size(1) == Sk && v.size(2) == Hkv, "k and v shapes differ");
  TORCH_CHECK(Hq % Hkv == 0, "number of query heads must be divisible by KV heads");
  c10::DeviceGuard g(q.device());
  auto o = torch::empty({B, Sq, Hq, D}, q.options());
  const int64_t qs[3] = {q.stride(0), q.stride(1), q.stride(2)};
  const int64_t ks[3] = {k.stride(0), k.stride(1), k.stride(2)};
  const int64_t vs[3] = {v.stride(0), v.stride(1), v.stride(2)};
  const int64_t os[3] = {o.stride(0), o.stride(1), o.stride(2)};
  check_rc(tpp_attn_prefill(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), qs, ks, vs,
                            os, B, Sq, Sk, Hq, Hkv, D, (float)softmax_scale, causal ? 1 : 0,
                            (int)window_left, (int)window_right, dtype_code(q), cur_stream(q)),
           "flash_attn_func");
  return o;
}

// q [B, 1, Hq, D]; caches [B, Hkv, Lmax, D] (strides honoured); seqlens int32 [B]
at::Tensor attn_decode(at::Tensor q, at::Tensor k_cache, at::Tensor v_cache,
                       c10::optional<at::Tensor> seqlens, double softmax_scale,
                       int64_t window_left, c10::optional<at::Tensor> out) {
  check_bshd(q, "q");
  TORCH_CHECK(q.size(1) == 1, "decode expects one query per sequence");
  TORCH_CHECK(k_cache.is_cuda() && v_cache.is_cuda() && k_cache.dim() == 4 &&
                  k_cache.sizes() == v_cache.sizes() && k_cache.stride(3) == 1 &&
                  v_cache.stride(3) == 1,
              "caches must be CUDA [B, Hkv, Lmax, D] with a contiguous last dim");
  TORCH_CHECK(k_cache.scalar_type() == q.scalar_type() &&
                  v_cache.scalar_type() == q.scalar_type(),
              "cache dtype must match q");
  const int64_t B = q.size(0), Hq = q.size(2), D = q.size(3);
  const int64_t Hkv = k_cache.size(1), Lmax = k_cache.size(2);
  TORCH_CHECK(k_cache.size(0) == B && k_cache.size(3) == D, "cache shape mismatch");
  const int32_t *sl = nullptr;
  if (seqlens.has_value() && seqlens->defined()) {
    TORCH_CHECK(seqlens->is_cuda() && seqlens->scalar_type() == at::kInt &&
                    seqlens->numel() == B && seqlens->is_contiguous(),
                "seqlens must be a contiguous CUDA int32 tensor [B]");
    sl = seqlens->data_ptr<int32_t>();
  }
  c10::DeviceGuard g(q.device());
  at::Tensor o;
  if (out.has_value() && out->defined()) {
    o = *out;
    TORCH_CHECK(o.sizes() == q.sizes() && o.scalar_type() == q.scalar_type() &&
                    o.stride(3) == 1,
                "out must match q");
  } else {
    o = torch::empty_like(q);
  }
  const size_t wsb = tpp_attn_decode_workspace_size(B, Hq, Hkv, D, Lmax);
  at::Tensor ws = cached_workspace(q, wsb, 1);
  const int64_t qs[3] = {q.stride(0), q.stride(1), q.stride(2)};
  const int64_t ks[3] = {k_cache.stride(0), k_cache.stride(2), k_cache.stride(1)};
  const int64_t vs[3] = {v_cache.stride(0), v_cache.stride(2), v_cache.stride(1)};
  const int64_t os[3] = {o.stride(0), o.stride(1), o.stride(2)};
  check_rc(tpp_attn_decode(q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), o.data_ptr(),
                           qs, ks, vs, os, sl, B, Hq, Hkv, D, Lmax, (float)softmax_scale,
                           (int)window_left, dtype_code(q), ws.data_ptr(), wsb, cur_stream(q)),
           "attn_decode");
  return o;
}

at::Tensor argmax_rows(at::Tensor x) {
  TORCH_CHECK(x.is_cuda() && is_half_or_bf16(x), "x must be a CUDA half/bfloat16 tensor");
  TORCH_CHECK(x.stride(-1) == 1, "x must have a contiguous last dim");
  const int64_t N = x.size(-1);
  at::Tensor x2 = x.reshape({-1, N});
  TORCH_CHECK(x2.stride(1) == 1, "x must be viewable as rows");
  c10::DeviceGuard g(x.device());
  auto out = torch::empty({x2.size(0)}, x.options().dtype(at::kLong));
  check_rc(tpp_argmax_rows(x2.data_ptr(), out.data_ptr<int64_t>(), x2.size(0), N, x2.stride(0),
                           dtype_code(x), cur_stream(x)),
           "argmax_rows");
  auto shp = x.sizes().vec();
  shp.pop_back();
  return out.view(shp);
}

// decode attention with the new token's QK-norm + RoPE + cache append fused in
at::Tensor attn_decode_fused(at::Tensor qkv, c10::optional<at::Tensor> q_norm_w,
                             c10::optional<at::Tensor> k_norm_w, at::Tensor cos, at::Tensor sin,
                             double eps, at::Tensor k_cache, at::Tensor v_cache,
                             at::Tensor seqlens, double softmax_scale, int64_t window_left) {
  TORCH_CHECK(qkv.is_cuda() && qkv.is_contiguous() && is_half_or_bf16(qkv),
              "qkv must be a contiguous CUDA half/bfloat16 tensor [B, 1, (Hq+2Hkv)*D]");
  TORCH_CHECK(k_cache.is_cuda() && v_cache.is_cuda() && k_cache.dim() == 4 &&
                  k_cache.sizes() == v_cache.sizes() && k_cache.stride(3) == 1 &&
                  v_cache.stride(3) == 1 && k_cache.scalar_type() == qkv.scalar_type() &&
                  v_cache.scalar_type() == qkv.scalar_type(),
              "caches must be CUDA [B, Hkv, Lmax, D] of the qkv dtype");
  const int64_t B = k_cache.size(0), Hkv = k_cache.size(1), Lmax = k_cache.size(2),
                D = k_cache.size(3);
  TORCH_CHECK(qkv.numel() % (B * D) == 0, "qkv size mismatch");
  const int64_t Hq = qkv.numel() / (B * D) - 2 * Hkv;
  TORCH_CHECK(Hq > 0 && Hq % Hkv == 0, "qkv size does not give a valid head count");
  TORCH_CHECK(seqlens.is_cuda() && seqlens.scalar_type() == at::kInt && seqlens.numel() == B &&
                  seqlens.is_contiguous(),
              "seqlens must be a contiguous CUDA int32 tensor [B]");
  TORCH_CHECK(cos.is_contiguous() && sin.is_contiguous() && cos.dim() == 2 && cos.size(1) == D &&
                  sin.sizes() == cos.sizes() && sin.scalar_type() == cos.scalar_type() &&
                  dtype_code(cos) >= 0,
              "cos/sin must be contiguous [ctx, D] tables");
  TORCH_CHECK(cos.size(0) >= Lmax, "cos/sin hold ", cos.size(0),
              " positions, fewer than the cache length ", Lmax);
  const void *qw = norm_ptr(q_norm_w, qkv, D), *kw = norm_ptr(k_norm_w, qkv, D);
  c10::DeviceGuard g(qkv.device());
  auto o = torch::empty({B, 1, Hq, D}, qkv.options());
  const size_t wsb = tpp_attn_decode_workspace_size(B, Hq, Hkv, D, Lmax);
  at::Tensor ws = cached_workspace(qkv, wsb, 1);
  const int64_t ks[3] = {k_cache.stride(0), k_cache.stride(2), k_cache.stride(1)};
  const int64_t vs[3] = {v_cache.stride(0), v_cache.stride(2), v_cache.stride(1)};
  const int64_t os[3] = {o.stride(0), o.stride(1), o.stride(2)};
  check_rc(tpp_attn_decode_fused(qkv.data_ptr(), qw, kw, cos.data_ptr(), sin.data_ptr(),
                                 cos.size(0), dtype_code(cos), (float)eps, k_cache.data_ptr(),
                                 v_cache.data_ptr(), o.data_ptr(), ks, vs, os,
                                 seqlens.data_ptr<int32_t>(), B, Hq, Hkv, D, Lmax,
                                 (float)softmax_scale, (int)window_left, dtype_code(qkv),
                                 ws.data_ptr(), (size_t)ws.numel() * 4, cur_stream(qkv)),
           "attn_decode_fused");
  return o;
}

// decode attention with the fused prologue, then the output projection and
// residual add (in place on `residual`); returns the attention output
at::Tensor attn_decode_oproj(at::Tensor qkv, c10::optional<at::Tensor> q_norm_w,
                             c10::optional<at::Tensor> k_norm_w, at::Tensor cos, at::Tensor sin,
                             double eps, at::Tensor k_cache, at::Tensor v_cache,
                             at::Tensor seqlens, at::Tensor w_o, at::Tensor residual,
                             double softmax_scale, int64_t window_left) {
  TORCH_CHECK(qkv.is_cuda() && qkv.is_contiguous() && is_half_or_bf16(qkv),
              "qkv must be a contiguous CUDA half/bfloat16 tensor [B, 1, (Hq+2Hkv)*D]");
  TORCH_CHECK(k_cache.is_cuda() && v_cache.is_cuda() && k_cache.dim() == 4 &&
                  k_cache.sizes() == v_cache.sizes() && k_cache.stride(3) == 1 &&
                  v_cache.stride(3) == 1 && k_cache.scalar_type() == qkv.scalar_type() &&
                  v_cache.scalar_type() == qkv.scalar_type(),
              "caches must be CUDA [B, Hkv, Lmax, D] of the qkv dtype");
  const int64_t B = k_cache.size(0), Hkv = k_cache.size(1), Lmax = k_cache.size(2),
                D = k_cache.size(3);
  TORCH_CHECK(qkv.numel() % (B * D) == 0, "qkv size mismatch");
  const int64_t Hq = qkv.numel() / (B * D) - 2 * Hkv;
  TORCH_CHECK(Hq > 0 && Hq % Hkv == 0, "qkv size does not give a valid head count");
  TORCH_CHECK(seqlens.is_cuda() && seqlens.scalar_type() == at::kInt && seqlens.numel() == B &&
                  seqlens.is_contiguous(),
              "seqlens must be a contiguous CUDA int32 tensor [B]");
  TORCH_CHECK(cos.is_contiguous() && sin.is_contiguous() && cos.dim() == 2 && cos.size(1) == D &&
                  sin.sizes() == cos.sizes() && sin.scalar_type() == cos.scalar_type() &&
                  dtype_code(cos) >= 0,
              "cos/sin must be contiguous [ctx, D] tables");
  TORCH_CHECK(cos.size(0) >= Lmax, "cos/sin hold ", cos.size(0),
              " positions, fewer than the cache length ", Lmax);
  TORCH_CHECK(w_o.is_cuda() && w_o.dim() == 2 && w_o.size(1) == Hq * D && w_o.is_contiguous() &&
                  w_o.scalar_type() == qkv.scalar_type(),
              "w_o must be a contiguous [E, Hq*D] weight of the qkv dtype");
  const int64_t E = w_o.size(0);
  TORCH_CHECK(residual.is_cuda() && residual.is_contiguous() && residual.numel() == B * E &&
                  residual.scalar_type() == qkv.scalar_type(),
              "residual must be a contiguous [B, E] tensor of the qkv dtype");
  const void *qw = norm_ptr(q_norm_w, qkv, D), *kw = norm_ptr(k_norm_w, qkv, D);
  c10::DeviceGuard g(qkv.device());
  auto o = torch::empty({B, 1, Hq, D}, qkv.options());
  const size_t wsb = tpp_attn_decode_oproj_workspace_size(B, Hq, Hkv, D, Lmax, E);
  at::Tensor ws = cached_workspace(qkv, wsb, 1);
  const int64_t ks[3] = {k_cache.stride(0), k_cache.stride(2), k_cache.stride(1)};
  const int64_t vs[3] = {v_cache.stride(0), v_cache.stride(2), v_cache.stride(1)};
  check_rc(tpp_attn_decode_oproj(qkv.data_ptr(), qw, kw, cos.data_ptr(), sin.data_ptr(),
                                 cos.size(0), dtype_code(cos), (float)eps, k_cache.data_ptr(),
                                 v_cache.data_ptr(), o.data_ptr(), ks, vs,
                                 seqlens.data_ptr<int32_t>(), w_o.data_ptr(), residual.data_ptr(),
                                 B, Hq, Hkv, D, Lmax, E, (float)softmax_scale, (int)window_left,
                                 dtype_code(qkv), ws.data_ptr(), (size_t)ws.numel() * 4,
                                 cur_stream(qkv)),
           "attn_decode_oproj");
  return o;
}

// nonzero if a one-launch attn_decode_oproj on this device gave up waiting for
// its workgroups since the last check; reads and clears the flag of every
// decode-attention workspace of the device (as ffn_decode_sync_errors)
int64_t attn_decode_sync_errors(at::Tensor like) {
  TORCH_CHECK(like.is_cuda(), "attn_decode_sync_errors: expected a CUDA tensor");
  c10::DeviceGuard g(like.device());
  ScratchSlot &e = scratch_slot(like.device().index(), 1);
  if (!e.t.defined()) return 0;
  cached_workspace(like, 1, 1);
  int64_t any = 0;
  auto check = [&](at::Tensor &t) {
    int out = 0;
    check_rc(tpp_attn_decode_oproj_sync_errors(t.data_ptr(), &out, cur_stream(like)),
             "attn_decode_sync_errors");
    any |= out;
  };
  check(e.t);
  for (auto &t : e.retired) check(t);
  return any;
}

} // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("attn_decode_oproj", &attn_decode_oproj,
        "decode attention (fused QK-norm + RoPE + KV append) then the output projection and the "
        "residual add, in place on residual; returns the attention output",
        py::arg("qkv"), py::arg("q_norm_w"), py::arg("k_norm_w"), py::arg("cos"), py::arg("sin"),
        py::arg("eps"), py::arg("k_cache"), py::arg("v_cache"), py::arg("seqlens"),
        py::arg("w_o"), py::arg("residual"), py::arg("softmax_scale") = 0.0,
        py::arg("window_left") = -1);
  m.def("attn_decode_sync_errors", &attn_decode_sync_errors,
        "nonzero if a one-launch attn_decode_oproj gave up waiting for its workgroups since the "
        "last check (its residual update was wrong); clears the flag",
        py::arg("like"));
  m.def("attn_decode_fused", &attn_decode_fused,
        "decode attention with QK-norm + RoPE + KV append of the new token fused in",
        py::arg("qkv"), py::arg("q_norm_w"), py::arg("k_norm_w"), py::arg("cos"), py::arg("sin"),
        py::arg("eps"), py::arg("k_cache"), py::arg("v_cache"), py::arg("seqlens"),
        py::arg("softmax_scale") = 0.0, py::arg("window_left") = -1);
  m.def("ffn_decode", &ffn_decode,
        "decode FFN half of a decoder block (RMSNorm + SwiGLU + down + residual), in place",
        py::arg("residual"), py::arg("norm_weight"), py::arg("eps"), py::arg("w_gu"),
        py::arg("w_down"));
  m.def("ffn_decode_sync_errors", &ffn_decode_sync_errors,
        "nonzero if a one-launch decode FFN gave up waiting for its workgroups since the last "
        "check (its output was wrong); clears the flag",
        py::arg("like"));
  m.def("_force_decode_sync_error", &force_decode_sync_error,
        "test hook: flag the device's decode-attention (0) or decode-FFN (1) workspace as if a "
        "one-launch kernel had given up waiting", py::arg("like"), py::arg("kernel"));
  m.def("prepare_device", &prepare_device,
        "one-time XCD placement probe and CU count of the tensor's device (outside capture)",
        py::arg("like"));
  m.def("argmax_rows", &argmax_rows, "argmax over the last dim (greedy sampling)", py::arg("x"));
  m.def("flash_attn_func", &attn_fwd, "flash attention forward (GQA, causal, window)",
        py::arg("q"), py::arg("k"), py::arg("v"), py::arg("causal") = false,
        py::arg("window_left") = -1, py::arg("window_right") = -1,
        py::arg("softmax_scale") = 0.0);
  m.def("attn_decode", &attn_decode, "split-KV decode attention over a KV cache", py::arg("q"),
        py::arg("k_cache"), py::arg("v_cache"), py::arg("seqlens") = py::none(),
        py::arg("softmax_scale") = 0.0, py::arg("window_left") = -1,
        py::arg("out") = py::none());
  m.def("rope_apply_cuda", &rope_apply_cuda, "RoPE (rotate-half), out of place",
        py::arg("x"), py::arg("cos_cache"), py::arg("sin_cache"));
  m.def("rope_apply_", &rope_apply_inplace, "RoPE (rotate-half), in place", py::arg("x"),
        py::arg("cos_cache"), py::arg("sin_cache"));
  m.def("qkrope_apply_cuda", &qkrope_apply_cuda, "RoPE on Q and K in one launch (Hk | Hq)",
        py::arg("q"), py::arg("k"), py::arg("cos_cache"), py::arg("sin_cache"));
  m.def("qkv_rope_cache", &qkv_rope_cache,
        "fused QK-RMSNorm + RoPE + KV-cache append of a fused qkv projection", py::arg("qkv"),
        py::arg("q_out"), py::arg("k_cache"), py::arg("v_cache"), py::arg("q_norm_w"),
        py::arg("k_norm_w"), py::arg("cos"), py::arg("sin"), py::arg("positions"),
        py::arg("eps") = 1e-6);
  m.def("LinearGelu", &linear_gelu, "Linear + GeLU(tanh) (fp16/bf16, MFMA)", py::arg("input"),
        py::arg("weight"), py::arg("bias") = py::none());
  m.def("LinearSilu", &linear_silu, "Linear + SiLU (fp16/bf16, MFMA)", py::arg("input"),
        py::arg("weight"), py::arg("bias") = py::none());
  m.def("LinearRelu", &linear_relu, "Linear + ReLU (fp16/bf16, MFMA)", py::arg("input"),
        py::arg("weight"), py::arg("bias") = py::none());
  m.def("linear", &linear_act, "act(x @ W^T + b), act: 0 none,1 gelu_tanh,2 silu,3 relu",
        py::arg("input"), py::arg("weight"), py::arg("bias") = py::none(), py::arg("act") = 0);
  m.def("linear_swiglu", &linear_swiglu, "silu(x Wg^T) * (x Wu^T) from interleaved w_gu",
        py::arg("input"), py::arg("w_gu"));
  m.def("gemv", &gemv, "decode GEMV for <= 16 rows", py::arg("input"), py::arg("weight"),
        py::arg("bias") = py::none(), py::arg("act") = 0);
  m.def("gemv_swiglu", &gemv_swiglu, "decode SwiGLU GEMV for <= 16 rows", py::arg("input"),
        py::arg("w_gu"), py::arg("norm_weight") = py::none(), py::arg("eps") = 1e-6);
  m.def("gemv_fused", &gemv_fused,
        "decode GEMV with optional input RMSNorm and in-place residual add", py::arg("input"),
        py::arg("weight"), py::arg("norm_weight") = py::none(), py::arg("eps") = 1e-6,
        py::arg("residual") = py::none());
  m.def("gemv_argmax", &gemv_argmax, "lm_head GEMV fused with greedy argmax", py::arg("input"),
        py::arg("weight"), py::arg("norm_weight") = py::none(), py::arg("eps") = 1e-6,
        py::arg("return_logits") = false);
  m.def("greedy_step", &greedy_step,
        "greedy decode tail: argmax(lm_head) -> ids, embedding gather, position advance",
        py::arg("input"), py::arg("weight"), py::arg("norm_weight"), py::arg("eps"),
        py::arg("emb"), py::arg("ids"), py::arg("resid_next"),
        py::arg("positions") = py::none(), py::arg("seqlens") = py::none());
  m.doc() = "torchpp gfx950 kernel set (binding over libtorchpp_hip.so)";
  m.def("rmsnormFused", &rmsnorm_fused, "Fused RMSNorm (fp16/bf16)", py::arg("input"),
        py::arg("weight"), py::arg("eps") = 1e-6);
  m.def("rmsnorm_stats", &rmsnorm_stats, "fp32 inv-rms per row", py::arg("input"),
        py::arg("eps") = 1e-6);
  m.def("add_rmsnorm", &add_rmsnorm, "residual += x; return rmsnorm(residual)*w",
        py::arg("x"), py::arg("residual"), py::arg("weight"), py::arg("eps") = 1e-6);
  m.def("applyLayernorm", &layernorm_forward, "LayerNorm forward (fp16/bf16)",
        py::arg("input"), py::arg("weight"), py::arg("eps") = 1e-6,
        py::arg("bias") = py::none());
  m.def("layernorm_stats", &layernorm_stats, "fp32 mean, rstd per row",
        py::arg("input"), py::arg("eps") = 1e-6);
}
