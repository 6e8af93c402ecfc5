// RMSNorm / LayerNorm / fused residual-add + RMSNorm for gfx950.
//
// Semantics follow the reference kernels:
//   RMSNorm   csrc/dlops/rmsnorm/rmsnorm_fp16.cuh:63-114
//             sum of squares in fp32, inv = rsqrt(sum/N + eps),
//             y = T( (x * inv) * w )  -- fp32 products, one rounding.
//   LayerNorm csrc/dlops/layernorm/layernorm_fp16.cuh:72-143
//             y = T( ((x - mean) * rstd) * w ), no bias in the reference.
//             The variance here is the two-pass sum((x-mean)^2)/N over the
//             register-resident row instead of the reference's one-pass
//             E[x^2]-mean^2 (same value in exact arithmetic, no cancellation).
//
// Layout: x is [M, ldx] with N valid elements per row; y is [M, ldy].
//
// Fast path (N % 8 == 0, 16-byte aligned rows, N <= 8192): a row lives in the
// VGPRs of one wave (N > 256) or one 16-lane DPP row (N <= 256, so a wave
// normalises 4 rows at once, e.g. the head_dim=128 QK-norm). Loads and stores
// are 128-bit, reductions are DPP + v_readlane, there is no LDS and no
// barrier. Generic path (anything else, including odd N as the reference
// allows): one 256-thread block per row with an LDS block reduction.
#include "tpp_common.hpp"

namespace tpp {

// kLayer: LayerNorm with a bias, kLayerNB: without (no bias loads)
enum NormMode { kRms = 0, kLayer = 1, kRmsStats = 2, kLayerStats = 3, kAddRms = 4, kLayerNB = 5 };
constexpr bool layer_mode(int m) { return m == kLayer || m == kLayerNB || m == kLayerStats; }

template <typename T, int LPR, int MAXV, int MODE>
__global__ __launch_bounds__(256) void norm_rows_kernel(
    const T *__restrict__ x, const T *__restrict__ w, const T *__restrict__ b,
    T *__restrict__ y, T *__restrict__ resid, float *__restrict__ s0,
    float *__restrict__ s1, int64_t M, int N, int64_t ldx, int64_t ldy, float eps) {
  constexpr int RPW = kWave / LPR; // rows per wave
  const int lane = lane_id();
  const int sub = lane / LPR;
  const int l = lane % LPR;
  const int64_t row =
      ((int64_t)blockIdx.x * (blockDim.x / kWave) + wave_id()) * RPW + sub;
  const bool valid = row < M;
  const int64_t rowc = valid ? row : M - 1; // launched only for M >= 1
  const int nvec = N >> 3;

  // Every load of the row goes out first and unconditionally: chunks past the
  // row and rows past M read chunk nvec-1 / row M-1 (values discarded), so the
  // compiler's count of loads in flight stays exact and the row costs one
  // memory round trip (a load under a branch makes the next wait drain every
  // load, one round trip per chunk). The weight (and bias) chunks go with x,
  // so the output pass waits on no further memory.
  typedef typename VecT<T>::v8 V8;
  constexpr bool kOut = (MODE == kRms || MODE == kLayer || MODE == kLayerNB || MODE == kAddRms);
  V8 xr[MAXV], rr[MAXV], wr[MAXV], br[MAXV];
#pragma unroll
  for (int j = 0; j < MAXV; ++j) {
    const int c = j * LPR + l;
    const int64_t cc = (int64_t)(c < nvec ? c : nvec - 1) * 8;
    xr[j] = ld_nt(reinterpret_cast<const V8 *>(x + rowc * ldx + cc));
    if constexpr (MODE == kAddRms) rr[j] = ld_nt(reinterpret_cast<const V8 *>(resid + rowc * ldy + cc));
    if constexpr (kOut) wr[j] = *reinterpret_cast<const V8 *>(w + cc);
    if constexpr (MODE == kLayer) br[j] = *reinterpret_cast<const V8 *>(b + cc);
  }
  __builtin_amdgcn_sched_barrier(0);
  float v[MAXV][8];
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < MAXV; ++j) {
    const bool ok = valid && j * LPR + l < nvec;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float xv = to_f32(xr[j][i]);
      if constexpr (MODE == kAddRms) xv = to_f32(from_f32<T>(xv + to_f32(rr[j][i])));
      v[j][i] = ok ? xv : 0.f;
    }
    if constexpr (layer_mode(MODE)) {
#pragma unroll
      for (int i = 0; i < 8; ++i) sum += v[j][i];
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) sum += v[j][i] * v[j][i];
    }
  }
  sum = (LPR == kWave) ? wave_sum(sum) : row16_sum(sum);

  float scale, mean = 0.f;
  if constexpr (layer_mode(MODE)) {
    mean = sum / (float)N;
    float sq = 0.f;
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
      const int c = j * LPR + l;
      if (c < nvec) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float d = v[j][i] - mean;
          sq += d * d;
        }
      }
    }
    sq = (LPR == kWave) ? wave_sum(sq) : row16_sum(sq);
    scale = rsqrtf(sq / (float)N + eps);
  } else {
    scale = rsqrtf(sum / (float)N + eps);
  }
  if constexpr (kOut) {
    // used only inside the per-chunk store branches below: pinned here so
    // the compiler cannot sink their loads into those branches (a second
    // memory round trip after the reduction)
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
      asm volatile("" ::"v"(wr[j]));
      if constexpr (MODE == kLayer) asm volatile("" ::"v"(br[j]));
    }
  }
  if (!valid) return;

  if constexpr (MODE == kRmsStats) {
    if (l == 0) s0[row] = scale;
    return;
  } else if constexpr (MODE == kLayerStats) {
    if (l == 0) {
      s0[row] = mean;
      s1[row] = scale;
    }
    return;
  } else {
#pragma unroll
    for (int j = 0; j < MAXV; ++j) {
      const int c = j * LPR + l;
      if (c < nvec) {
        float o[8];
        if constexpr (MODE == kLayer || MODE == kLayerNB) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            o[i] = ((v[j][i] - mean) * scale) * to_f32(wr[j][i]);
            if constexpr (MODE == kLayer) o[i] += to_f32(br[j][i]);
          }
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = (v[j][i] * scale) * to_f32(wr[j][i]);
        }
        if constexpr (MODE == kAddRms) store8(resid + row * ldy + (int64_t)c * 8, v[j]);
        store8(y + row * ldy + (int64_t)c * 8, o);
      }
    }
  }
}

// Generic path: one 256-thread block per row, scalar strided loops.
__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  __syncthreads(); // red[] may still be read from a previous reduction
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < (int)(blockDim.x / kWave); ++i) t += red[i];
  return t;
}

template <typename T, int MODE>
__global__ __launch_bounds__(256) void norm_generic_kernel(
    const T *__restrict__ x, const T *__restrict__ w, const T *__restrict__ b,
    T *__restrict__ y, T *__restrict__ resid, float *__restrict__ s0,
    float *__restrict__ s1, int64_t M, int N, int64_t ldx, int64_t ldy, float eps) {
  __shared__ float red[8];
  const int64_t row = blockIdx.x;
  const T *xr = x + row * ldx;
  float sum = 0.f;
  for (int i = threadIdx.x; i < N; i += blockDim.x) {
    float v = to_f32(xr[i]);
    if constexpr (MODE == kAddRms) {
      v = to_f32(from_f32<T>(v + to_f32(resid[row * ldy + i])));
      resid[row * ldy + i] = from_f32<T>(v);
    }
    sum += layer_mode(MODE) ? v : v * v;
  }
  sum = block_sum(sum, red);
  float scale, mean = 0.f;
  if constexpr (layer_mode(MODE)) {
    mean = sum / (float)N;
    float sq = 0.f;
    for (int i = threadIdx.x; i < N; i += blockDim.x) {
      float d = to_f32(xr[i]) - mean;
      sq += d * d;
    }
    sq = block_sum(sq, red);
    scale = rsqrtf(sq / (float)N + eps);
  } else {
    scale = rsqrtf(sum / (float)N + eps);
  }
  if constexpr (MODE == kRmsStats) {
    if (threadIdx.x == 0) s0[row] = scale;
  } else if constexpr (MODE == kLayerStats) {
    if (threadIdx.x == 0) {
      s0[row] = mean;
      s1[row] = scale;
    }
  } else {
    const T *src = (MODE == kAddRms) ? resid + row * ldy : xr;
    for (int i = threadIdx.x; i < N; i += blockDim.x) {
      float v = to_f32(src[i]);
      float o;
      if constexpr (MODE == kLayer || MODE == kLayerNB) {
        o = ((v - mean) * scale) * to_f32(w[i]);
        if constexpr (MODE == kLayer) o += to_f32(b[i]);
      } else {
        o = (v * scale) * to_f32(w[i]);
      }
      y[row * ldy + i] = from_f32<T>(o);
    }
  }
}

template <typename T, int MODE>
static int launch_norm(const void *x_, const void *w_, const void *b_, void *y_,
                       void *r_, float *s0, float *s1, int64_t M, int64_t N,
                       int64_t ldx, int64_t ldy, float eps, hipStream_t st,
                       const char *name) {
  const T *x = (const T *)x_;
  const T *w = (const T *)w_;
  const T *b = (const T *)b_;
  T *y = (T *)y_;
  T *r = (T *)r_;
  if (M == 0) return TPP_OK;
  const bool out_rows = !(MODE == kRmsStats || MODE == kLayerStats);
  bool fast = (N % 8 == 0) && (ldx % 8 == 0) && aligned16(x) && N <= 8192 &&
              (!out_rows || ((ldy % 8 == 0) && aligned16(y) && aligned16(w))) &&
              (b == nullptr || aligned16(b)) && (r == nullptr || aligned16(r));
  const dim3 block(256);
  if (fast) {
    if (N <= 256) {
      const int64_t rows_per_block = 4 * 4;
      dim3 grid((unsigned)((M + rows_per_block - 1) / rows_per_block));
      norm_rows_kernel<T, 16, 2, MODE><<<grid, block, 0, st>>>(
          x, w, b, y, r, s0, s1, M, (int)N, ldx, ldy, eps);
    } else {
      const int64_t rows_per_block = 4;
      dim3 grid((unsigned)((M + rows_per_block - 1) / rows_per_block));
      if (N <= 1024)
        norm_rows_kernel<T, 64, 2, MODE><<<grid, block, 0, st>>>(
            x, w, b, y, r, s0, s1, M, (int)N, ldx, ldy, eps);
      else if (N <= 2048)
        norm_rows_kernel<T, 64, 4, MODE><<<grid, block, 0, st>>>(
            x, w, b, y, r, s0, s1, M, (int)N, ldx, ldy, eps);
      else
        norm_rows_kernel<T, 64, 16, MODE><<<grid, block, 0, st>>>(
            x, w, b, y, r, s0, s1, M, (int)N, ldx, ldy, eps);
    }
  } else {
    if (M > 0x7fffffffLL) return set_error(TPP_E_UNSUPPORTED, "%s: M too large", name);
    norm_generic_kernel<T, MODE><<<dim3((unsigned)M), block, 0, st>>>(
        x, w, b, y, r, s0, s1, M, (int)N, ldx, ldy, eps);
  }
  return check_launch(name);
}

static int check_common(const char *name, const void *x, int64_t M, int64_t N,
                        int64_t ldx) {
  if (!x) return set_error(TPP_E_INVALID, "%s: input pointer is null", name);
  if (M < 0 || N <= 0)
    return set_error(TPP_E_INVALID, "%s: invalid shapes (M=%lld, N=%lld)", name,
                     (long long)M, (long long)N);
  if (N > 0x7fffffffLL)
    return set_error(TPP_E_UNSUPPORTED, "%s: N too large for kernel", name);
  if (ldx < N)
    return set_error(TPP_E_INVALID, "%s: row stride %lld < N %lld", name,
                     (long long)ldx, (long long)N);
  return TPP_OK;
}

} // namespace tpp

using namespace tpp;

extern "C" int tpp_rmsnorm(const void *x, const void *w, void *y, int64_t M,
                           int64_t N, int64_t ldx, int64_t ldy, float eps,
                           int dtype, void *stream) {
  const char *name = "tpp_rmsnorm";
  if (int e = check_common(name, x, M, N, ldx)) return e;
  if (!w || !y) return set_error(TPP_E_INVALID, "%s: null weight/output", name);
  if (ldy < N) return set_error(TPP_E_INVALID, "%s: output stride < N", name);
  return TPP_DISPATCH_HALF(dtype, [&] {
    return launch_norm<T, kRms>(x, w, nullptr, y, nullptr, nullptr, nullptr, M, N,
                                ldx, ldy, eps, as_stream(stream), name);
  });
}

extern "C" int tpp_rmsnorm_stats(const void *x, float *inv_rms, int64_t M,
                                 int64_t N, int64_t ldx, float eps, int dtype,
                                 void *stream) {
  const char *name = "tpp_rmsnorm_stats";
  if (int e = check_common(name, x, M, N, ldx)) return e;
  if (!inv_rms) return set_error(TPP_E_INVALID, "%s: null output", name);
  return TPP_DISPATCH_HALF(dtype, [&] {
    return launch_norm<T, kRmsStats>(x, nullptr, nullptr, nullptr, nullptr, inv_rms,
                                     nullptr, M, N, ldx, N, eps, as_stream(stream),
                                     name);
  });
}

extern "C" int tpp_add_rmsnorm(const void *x, void *residual, const void *w,
                               void *y, int64_t M, int64_t N, float eps,
                               int dtype, void *stream) {
  const char *name = "tpp_add_rmsnorm";
  if (int e = check_common(name, x, M, N, N)) return e;
  if (!w || !y || !residual)
    return set_error(TPP_E_INVALID, "%s: null weight/residual/output", name);
  return TPP_DISPATCH_HALF(dtype, [&] {
    return launch_norm<T, kAddRms>(x, w, nullptr, y, residual, nullptr, nullptr, M,
                                   N, N, N, eps, as_stream(stream), name);
  });
}

extern "C" int tpp_layernorm(const void *x, const void *w, const void *b, void *y,
                             int64_t M, int64_t N, int64_t ldx, int64_t ldy,
                             float eps, int dtype, void *stream) {
  const char *name = "tpp_layernorm";
  if (int e = check_common(name, x, M, N, ldx)) return e;
  if (!w || !y) return set_error(TPP_E_INVALID, "%s: null weight/output", name);
  if (ldy < N) return set_error(TPP_E_INVALID, "%s: output stride < N", name);
  return TPP_DISPATCH_HALF(dtype, [&] {
    if (b)
      return launch_norm<T, kLayer>(x, w, b, y, nullptr, nullptr, nullptr, M, N, ldx,
                                    ldy, eps, as_stream(stream), name);
    return launch_norm<T, kLayerNB>(x, w, nullptr, y, nullptr, nullptr, nullptr, M, N, ldx,
                                    ldy, eps, as_stream(stream), name);
  });
}

extern "C" int tpp_layernorm_stats(const void *x, float *mean, float *rstd,
                                   int64_t M, int64_t N, int64_t ldx, float eps,
                                   int dtype, void *stream) {
  const char *name = "tpp_layernorm_stats";
  if (int e = check_common(name, x, M, N, ldx)) return e;
  if (!mean || !rstd) return set_error(TPP_E_INVALID, "%s: null output", name);
  return TPP_DISPATCH_HALF(dtype, [&] {
    return launch_norm<T, kLayerStats>(x, nullptr, nullptr, nullptr, nullptr, mean,
                                       rstd, M, N, ldx, N, eps, as_stream(stream),
                                       name);
  });
}
