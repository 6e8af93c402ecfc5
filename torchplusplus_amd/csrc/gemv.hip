// Decode GEMV for gfx950: y[b, n] = sum_k x[b, k] * W[n, k], batch B <= 16.
//
// Reference: hgemvK128F16x4Kernel (csrc/blas/hgemv/hgemv_kernels.cuh:19-67),
// one warp per output row with fp16 accumulation; its CPU check is
// hgemvCpu (hgemv_bench.cpp:10-24). In the model these GEMVs are the
// nn.Linear calls of a decode step (B = batch size, one token each).
//
// Design (HBM-bound on W):
//  * A wave owns a tile of 16 weight rows and a K slice. One
//    v_mfma_f32_16x16x32 consumes 16 rows x 32 K of W (the B operand: each
//    lane loads 16 contiguous bytes of one row) and the matching 16 x 32 of x
//    (the A operand, batch rows >= B are zero). So the batch is free: W is
//    streamed once for all B <= 16 rows of x, with 128-bit loads only.
//  * The K range is split over the 4 waves of a block (LDS reduction) and,
//    when there are too few row tiles to fill 256 CUs, over blocks: the
//    partial sums go to an fp32 workspace with global float atomics and the
//    last block of a row tile (device-scope counter) applies the epilogue,
//    then zeroes its workspace slice and counter. The workspace therefore
//    stays zero between calls (it must be zero when first used), which keeps
//    the op free of memsets and safe to capture in a HIP graph. Calls that
//    share one workspace must be ordered (same stream).
//  * Epilogues: plain; bias + activation with the reference's rounding
//    (pre-activation rounded to T, activation in fp32, csrc/activation/
//    fused_gemm.cuh:93-105); SwiGLU over a [gate|up] weight interleaved in
//    blocks of 32 rows (rows 64j..64j+31 = gate rows 32j.., the next 32 = up),
//    rounding like the eager chain silu(gate(x)) * up(x).
#include "tpp_common.hpp"

namespace tpp {

enum GemvEpi { kEpiPlain = 0, kEpiBiasAct = 1, kEpiSwiGLU = 2 };

constexpr int kGemvU = 2;                  // 64-K steps per load batch
constexpr int kGemvKStep = 64 * kGemvU;    // K elements per load batch

template <typename T>
__device__ __forceinline__ typename VecT<T>::v8 ld16(const T *p, bool ok) {
  typedef typename VecT<T>::v8 V;
  if (ok) return *reinterpret_cast<const V *>(p);
  V z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = (T)0.0f;
  return z;
}

template <typename T>
__device__ __forceinline__ f32x4 mfma16(typename VecT<T>::v8 a, typename VecT<T>::v8 b,
                                        f32x4 c) {
  if constexpr (sizeof(T) == 2 && __is_same(T, bf16))
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

template <typename T, int ACT>
__device__ __forceinline__ T epi_bias_act(float acc, const T *bias, int64_t n) {
  float pre = acc;
  if (bias) pre += to_f32(bias[n]);
  pre = to_f32(from_f32<T>(pre));
  return from_f32<T>(apply_act<ACT>(pre));
}

template <typename T>
__device__ __forceinline__ T epi_swiglu(float g, float u) {
  const float gt = to_f32(from_f32<T>(g));
  const float s = to_f32(from_f32<T>(act_silu(gt)));
  const float ut = to_f32(from_f32<T>(u));
  return from_f32<T>(s * ut);
}

// grid.x: row tiles (16 weight rows; SwiGLU: 16 outputs = 16 gate + 16 up rows)
// grid.y: K splits over blocks. block: 256 threads = 4 waves, each a K slice.
template <typename T, int EPI, int ACT>
__global__ __launch_bounds__(256) void gemv16_kernel(
    const T *__restrict__ x, int64_t ldx, int NB, const T *__restrict__ W, int64_t N,
    int64_t K, T *__restrict__ y, int64_t ldy, const T *__restrict__ bias,
    float *__restrict__ ws, unsigned *__restrict__ cnt, int kslice, int nsplit) {
  typedef typename VecT<T>::v8 V8;
  __shared__ f32x4 red[2][4][64];
  const int lane = lane_id(), w = wave_id();
  const int r = lane & 15, g = lane >> 4;
  const int64_t tile = blockIdx.x;
  int64_t row0, row1 = 0;
  if constexpr (EPI == kEpiSwiGLU) {
    row0 = (tile >> 1) * 64 + (tile & 1) * 16;
    row1 = row0 + 32;
  } else {
    row0 = tile * 16;
  }
  const int64_t k_begin = ((int64_t)blockIdx.y * 4 + w) * kslice;
  const int64_t k_end = k_begin + kslice < K ? k_begin + kslice : K;

  const bool xok = r < NB;
  const T *xr = x + (xok ? r : 0) * ldx;
  const bool w0ok = row0 + r < N;
  const T *w0 = W + (w0ok ? row0 + r : 0) * K;
  const bool w1ok = (EPI == kEpiSwiGLU) && (row1 + r < N);
  const T *w1 = W + (w1ok ? row1 + r : 0) * K;

  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  for (int64_t k = k_begin; k < k_end; k += kGemvKStep) {
    V8 a[2 * kGemvU], b0[2 * kGemvU], b1[2 * kGemvU];
#pragma unroll
    for (int u = 0; u < 2 * kGemvU; ++u) {
      const int64_t c = k + u * 32 + g * 8; // K % 8 == 0: a chunk is all in or all out
      const bool in = c < k_end;
      b0[u] = ld16(w0 + c, in && w0ok);
      if constexpr (EPI == kEpiSwiGLU) b1[u] = ld16(w1 + c, in && w1ok);
      a[u] = ld16(xr + c, in && xok);
    }
#pragma unroll
    for (int u = 0; u < 2 * kGemvU; ++u) {
      acc0 = mfma16<T>(a[u], b0[u], acc0);
      if constexpr (EPI == kEpiSwiGLU) acc1 = mfma16<T>(a[u], b1[u], acc1);
    }
  }
  red[0][w][lane] = acc0;
  if constexpr (EPI == kEpiSwiGLU) red[1][w][lane] = acc1;
  __syncthreads();
  if (w != 0) return;
  acc0 = red[0][0][lane] + red[0][1][lane] + red[0][2][lane] + red[0][3][lane];
  if constexpr (EPI == kEpiSwiGLU)
    acc1 = red[1][0][lane] + red[1][1][lane] + red[1][2][lane] + red[1][3][lane];

  // D layout of 16x16x32: lane -> column r (weight row), rows b = 4g + i.
  const int64_t n0 = row0 + r, n1 = row1 + r;
  if (nsplit > 1) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = 4 * g + i;
      if (b < NB) {
        if (n0 < N) unsafeAtomicAdd(ws + (int64_t)b * N + n0, acc0[i]);
        if constexpr (EPI == kEpiSwiGLU)
          if (n1 < N) unsafeAtomicAdd(ws + (int64_t)b * N + n1, acc1[i]);
      }
    }
    __threadfence();
    unsigned prev = 0;
    if (lane == 0) prev = atomicAdd(cnt + tile, 1u);
    prev = __shfl(prev, 0, kWave);
    if (prev != (unsigned)(nsplit - 1)) return;
    __threadfence();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = 4 * g + i;
      if (b < NB) {
        if (n0 < N) {
          float *p = ws + (int64_t)b * N + n0;
          acc0[i] = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(p, 0.f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if constexpr (EPI == kEpiSwiGLU) {
          if (n1 < N) {
            float *p = ws + (int64_t)b * N + n1;
            acc1[i] = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(p, 0.f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
    }
    if (lane == 0) __hip_atomic_store(cnt + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int b = 4 * g + i;
    if (b >= NB) continue;
    if constexpr (EPI == kEpiSwiGLU) {
      if (n0 < N && n1 < N) {
        const int64_t on = (tile >> 1) * 32 + (tile & 1) * 16 + r;
        y[(int64_t)b * ldy + on] = epi_swiglu<T>(acc0[i], acc1[i]);
      }
    } else if (n0 < N) {
      if constexpr (EPI == kEpiBiasAct)
        y[(int64_t)b * ldy + n0] = epi_bias_act<T, ACT>(acc0[i], bias, n0);
      else
        y[(int64_t)b * ldy + n0] = from_f32<T>(acc0[i]);
    }
  }
}

// Generic fallback (any K, alignment, batch): one thread per output.
template <typename T, int EPI, int ACT>
__global__ __launch_bounds__(256) void gemv_scalar_kernel(
    const T *__restrict__ x, int64_t ldx, int NB, const T *__restrict__ W, int64_t N,
    int64_t K, T *__restrict__ y, int64_t ldy, const T *__restrict__ bias, int64_t NO) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= NO * NB) return;
  const int b = (int)(t / NO);
  const int64_t o = t - (int64_t)b * NO;
  const T *xr = x + b * ldx;
  if constexpr (EPI == kEpiSwiGLU) {
    const int64_t n0 = (o / 32) * 64 + (o % 32), n1 = n0 + 32;
    float g = 0.f, u = 0.f;
    for (int64_t k = 0; k < K; ++k) {
      const float xv = to_f32(xr[k]);
      g += xv * to_f32(W[n0 * K + k]);
      u += xv * to_f32(W[n1 * K + k]);
    }
    y[b * ldy + o] = epi_swiglu<T>(g, u);
  } else {
    float acc = 0.f;
    for (int64_t k = 0; k < K; ++k) acc += to_f32(xr[k]) * to_f32(W[o * K + k]);
    if constexpr (EPI == kEpiBiasAct)
      y[b * ldy + o] = epi_bias_act<T, ACT>(acc, bias, o);
    else
      y[b * ldy + o] = from_f32<T>(acc);
  }
}

struct GemvPlan {
  bool vec;
  int64_t tiles;
  int kslice;
  int nsplit;
  size_t ws_bytes;
};

static GemvPlan plan_gemv(int64_t B, int64_t N, int64_t K, int epi, const void *x,
                          const void *W, const void *y, int64_t ldx) {
  GemvPlan p{};
  p.vec = (K % 8 == 0) && (ldx % 8 == 0) && aligned16(x) && aligned16(W) && B <= 16;
  if (!p.vec) return p;
  p.tiles = (epi == kEpiSwiGLU) ? (N / 64) * 2 : (N + 15) / 16;
  const int64_t steps = (K + kGemvKStep - 1) / kGemvKStep;
  // aim for ~2048 waves in flight (8 per CU) without slicing below one step
  int64_t want_waves = 2048 / (p.tiles > 0 ? p.tiles : 1);
  if (want_waves < 4) want_waves = 4;
  int64_t nsplit = (want_waves + 3) / 4;
  if (nsplit > (steps + 3) / 4) nsplit = (steps + 3) / 4;
  if (nsplit < 1) nsplit = 1;
  const int64_t waves = nsplit * 4;
  const int64_t steps_per_wave = (steps + waves - 1) / waves;
  p.kslice = (int)(steps_per_wave * kGemvKStep);
  p.nsplit = (int)((K + 4LL * p.kslice - 1) / (4LL * p.kslice));
  p.ws_bytes = p.nsplit > 1 ? (size_t)(B * N) * 4 + (size_t)p.tiles * 4 : 0;
  return p;
}

template <typename T, int EPI, int ACT>
static int launch_gemv(const void *x, int64_t ldx, int64_t B, const void *W, int64_t N,
                       int64_t K, void *y, int64_t ldy, const void *bias, void *ws,
                       size_t ws_bytes, hipStream_t st, const char *name) {
  const GemvPlan p = plan_gemv(B, N, K, EPI, x, W, y, ldx);
  const int64_t NO = (EPI == kEpiSwiGLU) ? N / 2 : N;
  if (!p.vec) {
    const int64_t blocks = (NO * B + 255) / 256;
    gemv_scalar_kernel<T, EPI, ACT><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
        (const T *)x, ldx, (int)B, (const T *)W, N, K, (T *)y, ldy, (const T *)bias, NO);
    return check_launch(name);
  }
  float *wsf = nullptr;
  unsigned *cnt = nullptr;
  if (p.nsplit > 1) {
    if (!ws || ws_bytes < p.ws_bytes)
      return set_error(TPP_E_WORKSPACE, "%s: workspace of %zu bytes required, got %zu", name,
                       p.ws_bytes, ws ? ws_bytes : (size_t)0);
    if (!aligned16(ws)) return set_error(TPP_E_INVALID, "%s: workspace alignment", name);
    wsf = (float *)ws;
    cnt = (unsigned *)((char *)ws + (size_t)(B * N) * 4);
  }
  if (p.tiles > 0x7fffffffLL) return set_error(TPP_E_UNSUPPORTED, "%s: N too large", name);
  gemv16_kernel<T, EPI, ACT><<<dim3((unsigned)p.tiles, (unsigned)p.nsplit), dim3(256), 0, st>>>(
      (const T *)x, ldx, (int)B, (const T *)W, N, K, (T *)y, ldy, (const T *)bias, wsf, cnt,
      p.kslice, p.nsplit);
  return check_launch(name);
}

static int gemv_args(const char *name, const void *x, const void *W, const void *y, int64_t B,
                     int64_t N, int64_t K, int64_t ldx, int64_t ldy) {
  if (!x || !W || !y) return set_error(TPP_E_INVALID, "%s: null pointer", name);
  if (B < 1 || N < 1 || K < 1)
    return set_error(TPP_E_INVALID, "%s: invalid shapes (B=%lld N=%lld K=%lld)", name,
                     (long long)B, (long long)N, (long long)K);
  if (B > 16) return set_error(TPP_E_UNSUPPORTED, "%s: batch %lld > 16, use tpp_linear", name,
                               (long long)B);
  if (ldx < K) return set_error(TPP_E_INVALID, "%s: ldx < K", name);
  if (ldy < 1) return set_error(TPP_E_INVALID, "%s: ldy", name);
  return TPP_OK;
}

} // namespace tpp

using namespace tpp;

extern "C" size_t tpp_gemv_workspace_size(int64_t B, int64_t N, int64_t K, int swiglu) {
  // Conservative: assume the vector path (the scalar path needs none).
  GemvPlan p = plan_gemv(B, N, K, swiglu ? kEpiSwiGLU : kEpiPlain, (void *)0, (void *)0,
                         (void *)0, K);
  return p.ws_bytes;
}

extern "C" int tpp_gemv(const void *x, const void *W, const void *bias, void *y, int64_t B,
                        int64_t N, int64_t K, int64_t ldx, int64_t ldy, int act, int dtype,
                        void *workspace, size_t ws_bytes, void *stream) {
  const char *name = "tpp_gemv";
  if (int e = gemv_args(name, x, W, y, B, N, K, ldx, ldy)) return e;
  if (ldy < N) return set_error(TPP_E_INVALID, "%s: ldy < N", name);
  if (act < TPP_ACT_NONE || act > TPP_ACT_RELU)
    return set_error(TPP_E_INVALID, "%s: unknown activation %d", name, act);
  hipStream_t st = as_stream(stream);
  return TPP_DISPATCH_HALF(dtype, [&] {
    if (!bias && act == TPP_ACT_NONE)
      return launch_gemv<T, kEpiPlain, TPP_ACT_NONE>(x, ldx, B, W, N, K, y, ldy, nullptr,
                                                     workspace, ws_bytes, st, name);
    switch (act) {
    case TPP_ACT_GELU_TANH:
      return launch_gemv<T, kEpiBiasAct, TPP_ACT_GELU_TANH>(x, ldx, B, W, N, K, y, ldy, bias,
                                                            workspace, ws_bytes, st, name);
    case TPP_ACT_SILU:
      return launch_gemv<T, kEpiBiasAct, TPP_ACT_SILU>(x, ldx, B, W, N, K, y, ldy, bias,
                                                       workspace, ws_bytes, st, name);
    case TPP_ACT_RELU:
      return launch_gemv<T, kEpiBiasAct, TPP_ACT_RELU>(x, ldx, B, W, N, K, y, ldy, bias,
                                                       workspace, ws_bytes, st, name);
    default:
      return launch_gemv<T, kEpiBiasAct, TPP_ACT_NONE>(x, ldx, B, W, N, K, y, ldy, bias,
                                                       workspace, ws_bytes, st, name);
    }
  });
}

extern "C" int tpp_gemv_swiglu(const void *x, const void *W_gu, void *y, int64_t B,
                               int64_t I, int64_t K, int64_t ldx, int64_t ldy, int dtype,
                               void *workspace, size_t ws_bytes, void *stream) {
  const char *name = "tpp_gemv_swiglu";
  if (int e = gemv_args(name, x, W_gu, y, B, 2 * I, K, ldx, ldy)) return e;
  if (I % 32 != 0)
    return set_error(TPP_E_UNSUPPORTED, "%s: intermediate size %lld must be a multiple of 32",
                     name, (long long)I);
  if (ldy < I) return set_error(TPP_E_INVALID, "%s: ldy < I", name);
  hipStream_t st = as_stream(stream);
  return TPP_DISPATCH_HALF(dtype, [&] {
    return launch_gemv<T, kEpiSwiGLU, TPP_ACT_NONE>(x, ldx, B, W_gu, 2 * I, K, y, ldy, nullptr,
                                                    workspace, ws_bytes, st, name);
  });
}
