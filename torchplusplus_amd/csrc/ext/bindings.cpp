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

} // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
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
