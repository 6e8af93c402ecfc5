// Greedy sampling: idx[b] = argmax_n x[b, n] (first index among equal maxima,
// NaN counts as the maximum), the torch.argmax of LLMInference.sample_greedy
// (torchpp/llmops/llm.py:181-186). One 1024-thread block per row, 128-bit
// loads, DPP/shuffle wave reductions. It allocates and clears nothing, so it
// can sit inside a captured decode graph.
#include "tpp_common.hpp"

namespace tpp {

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

template <typename T>
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const T *__restrict__ x, int64_t ldx,
                                                           int N, int64_t *__restrict__ out) {
  __shared__ float sv[16];
  __shared__ int si[16];
  const T *row = x + (int64_t)blockIdx.x * ldx;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  const bool vec = (N % 8 == 0) && (ldx % 8 == 0) && aligned16(x);
  if (vec) {
    for (int c = threadIdx.x; c < N / 8; c += blockDim.x) {
      float v[8];
      load8(row + (int64_t)c * 8, v);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (better(v[j], c * 8 + j, bv, bi)) bv = v[j], bi = c * 8 + j;
    }
  } else {
    for (int i = threadIdx.x; i < N; i += blockDim.x) {
      const float v = to_f32(row[i]);
      if (better(v, i, bv, bi)) bv = v, bi = i;
    }
  }
#pragma unroll
  for (int sh = 1; sh < kWave; sh <<= 1) {
    const float ov = __shfl_xor(bv, sh, kWave);
    const int oi = __shfl_xor(bi, sh, kWave);
    if (better(ov, oi, bv, bi)) bv = ov, bi = oi;
  }
  if (lane_id() == 0) {
    sv[wave_id()] = bv;
    si[wave_id()] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x / kWave); ++w)
      if (better(sv[w], si[w], bv, bi)) bv = sv[w], bi = si[w];
    out[blockIdx.x] = bi;
  }
}

} // namespace tpp

using namespace tpp;

extern "C" int tpp_argmax_rows(const void *x, int64_t *out, int64_t B, int64_t N, int64_t ldx,
                               int dtype, void *stream) {
  const char *name = "tpp_argmax_rows";
  if (!x || !out) return set_error(TPP_E_INVALID, "%s: null pointer", name);
  if (B < 0 || N < 1 || N > 0x7fffffffLL || ldx < N)
    return set_error(TPP_E_INVALID, "%s: invalid shapes", name);
  if (B == 0) return TPP_OK;
  if (B > 0x7fffffffLL) return set_error(TPP_E_UNSUPPORTED, "%s: too many rows", name);
  hipStream_t st = as_stream(stream);
  return TPP_DISPATCH_HALF(dtype, [&] {
    argmax_rows_kernel<T><<<dim3((unsigned)B), dim3(1024), 0, st>>>((const T *)x, ldx, (int)N, out);
    return check_launch(name);
  });
}
