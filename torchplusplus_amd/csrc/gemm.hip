// MFMA GEMM with fused epilogue for gfx950:  C[M,N] = epi(A[M,K] . B[N,K]^T)
//
// Replaces the CUTLASS SM80 tensor-op GEMM + LinearActivationFP16 epilogue of
// csrc/activation/fused_gemm.cuh:20-170 (bound at binding.cu:11-160). B is the
// nn.Linear weight [N, K] (ldb = K, "ColumnMajor" B in CUTLASS terms), so
// both operands are K-contiguous and every load is a 128-bit row segment.
//
// Epilogues (fp32 accumulator in, T out):
//   plain      C = T(acc)
//   bias+act   C = T(act(float(T(acc + bias))))  -- the reference rounds the
//              pre-activation to half before GeluHalf/SiluHalf/ReluHalf
//              (fused_gemm.cuh:93-105); its epilogue as committed reads
//              unconverted registers (:79-89), this is the intended formula.
//   SwiGLU     weight rows interleaved in blocks of 32 ([gate 32 | up 32]...):
//              C[:, 32j+c] = T(T(silu(T(g))) * T(u)), the eager FFN chain.
//
// Tiling: 128x128 block tile, BK = 64, 256 threads = 4 waves in a 2x2 grid,
// each wave a 64x64 tile of 2x2 v_mfma_f32_32x32x16 accumulators (64 fp32
// VGPRs). Global -> VGPR -> LDS with 128-bit accesses, LDS rows XOR-swizzled
// in 16-byte chunks (conflict-free ds_read_b128 for the MFMA operand
// pattern), double-buffered with one barrier per K step. Blocks are mapped
// XCD-aware: the hardware deals blocks round-robin to the 8 XCDs, so block
// ids are remapped so that each XCD works on a compact group of tiles that
// share A rows and B columns in its own L2.
#include "tpp_common.hpp"

namespace tpp {

enum GemmEpi { kGPlain = 0, kGBiasAct = 1, kGSwiGLU = 2 };

constexpr int kBM = 128, kBN = 128, kBK = 64;

template <typename T>
__device__ __forceinline__ f32x16 mfma32(typename VecT<T>::v8 a, typename VecT<T>::v8 b,
                                         f32x16 c) {
  if constexpr (__is_same(T, bf16))
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void tile_coords(int pid, int nb, int ntm, int ntn, int &tm,
                                            int &tn) {
  const int q = nb >> 3, rem = nb & 7;
  const int xcd = pid & 7, idx = pid >> 3;
  const int logical =
      (xcd < rem) ? xcd * (q + 1) + idx : rem * (q + 1) + (xcd - rem) * q + idx;
  constexpr int GM = 8;
  const int width = GM * ntn;
  const int group = logical / width;
  const int first_m = group * GM;
  const int gsz = (ntm - first_m) < GM ? (ntm - first_m) : GM;
  const int within = logical - group * width;
  tm = first_m + within % gsz;
  tn = within / gsz;
}

template <typename T, int EPI, int ACT>
__global__ __launch_bounds__(256) void gemm_kernel(
    const T *__restrict__ A, int64_t lda, const T *__restrict__ B, int64_t ldb,
    T *__restrict__ C, int64_t ldc, const T *__restrict__ bias, int M, int N, int K) {
  typedef typename VecT<T>::v8 V8;
  __shared__ V8 sA[2][kBM * kBK / 8];
  __shared__ V8 sB[2][kBN * kBK / 8];

  const int ntm = (M + kBM - 1) / kBM, ntn = (N + kBN - 1) / kBN;
  int tm, tn;
  tile_coords(blockIdx.x, ntm * ntn, ntm, ntn, tm, tn);
  const int m0 = tm * kBM, n0 = tn * kBN;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w >> 1, wn = w & 1;

  V8 ra[4], rb[4];
  V8 zero;
#pragma unroll
  for (int i = 0; i < 8; ++i) zero[i] = (T)0.0f;

  auto gload = [&](int kt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i, row = c >> 3, kc = c & 7;
      const int gk = kt * kBK + kc * 8;
      const int gm = m0 + row, gn = n0 + row;
      ra[i] = (gm < M && gk < K) ? *reinterpret_cast<const V8 *>(A + (int64_t)gm * lda + gk)
                                 : zero;
      rb[i] = (gn < N && gk < K) ? *reinterpret_cast<const V8 *>(B + (int64_t)gn * ldb + gk)
                                 : zero;
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = tid + 256 * i, row = c >> 3, kc = c & 7;
      sA[buf][row * 8 + (kc ^ (row & 7))] = ra[i];
      sB[buf][row * 8 + (kc ^ (row & 7))] = rb[i];
    }
  };

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  const int nk = (K + kBK - 1) / kBK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      V8 af[2], bfr[2];
      const int kc = ks * 2 + (lane >> 5);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int row = wm * 64 + i * 32 + (lane & 31);
        af[i] = sA[buf][row * 8 + (kc ^ (row & 7))];
        const int col = wn * 64 + i * 32 + (lane & 31);
        bfr[i] = sB[buf][col * 8 + (kc ^ (col & 7))];
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma32<T>(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }

  // Epilogue. 32x32 accumulator layout: lane -> column (lane & 31),
  // register r -> row (r/4)*8 + (lane/32)*4 + (r%4).
  const int half = lane >> 5, cl = lane & 31;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + half * 4 + (r & 3);
      if (row >= M) continue;
      if constexpr (EPI == kGSwiGLU) {
        const int gcol = n0 + wn * 64 + cl; // gate row of W (tile j = 0)
        if (gcol + 32 < N) {
          const float gt = to_f32(from_f32<T>(acc[i][0][r]));
          const float s = to_f32(from_f32<T>(act_silu(gt)));
          const float ut = to_f32(from_f32<T>(acc[i][1][r]));
          const int ocol = (n0 + wn * 64) / 2 + cl;
          C[(int64_t)row * ldc + ocol] = from_f32<T>(s * ut);
        }
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int col = n0 + wn * 64 + j * 32 + cl;
          if (col >= N) continue;
          float v = acc[i][j][r];
          if constexpr (EPI == kGBiasAct) {
            if (bias) v += to_f32(bias[col]);
            v = apply_act<ACT>(to_f32(from_f32<T>(v)));
          }
          C[(int64_t)row * ldc + col] = from_f32<T>(v);
        }
      }
    }
  }
}

// Fallback for K % 8 != 0 or unaligned operands: one thread per output.
template <typename T, int EPI, int ACT>
__global__ __launch_bounds__(256) void gemm_scalar_kernel(
    const T *__restrict__ A, int64_t lda, const T *__restrict__ B, int64_t ldb,
    T *__restrict__ C, int64_t ldc, const T *__restrict__ bias, int M, int NO, int K) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)M * NO) return;
  const int m = (int)(t / NO), o = (int)(t % NO);
  const T *a = A + (int64_t)m * lda;
  if constexpr (EPI == kGSwiGLU) {
    const int64_t n0 = (o / 32) * 64 + (o % 32), n1 = n0 + 32;
    float g = 0.f, u = 0.f;
    for (int k = 0; k < K; ++k) {
      g += to_f32(a[k]) * to_f32(B[n0 * ldb + k]);
      u += to_f32(a[k]) * to_f32(B[n1 * ldb + k]);
    }
    const float s = to_f32(from_f32<T>(act_silu(to_f32(from_f32<T>(g)))));
    C[(int64_t)m * ldc + o] = from_f32<T>(s * to_f32(from_f32<T>(u)));
  } else {
    float v = 0.f;
    for (int k = 0; k < K; ++k) v += to_f32(a[k]) * to_f32(B[(int64_t)o * ldb + k]);
    if constexpr (EPI == kGBiasAct) {
      if (bias) v += to_f32(bias[o]);
      v = apply_act<ACT>(to_f32(from_f32<T>(v)));
    }
    C[(int64_t)m * ldc + o] = from_f32<T>(v);
  }
}

template <typename T, int EPI, int ACT>
static int launch_gemm(const void *A, int64_t lda, const void *B, int64_t ldb, void *C,
                       int64_t ldc, const void *bias, int64_t M, int64_t N, int64_t K,
                       hipStream_t st, const char *name) {
  if (M == 0) return TPP_OK;
  const bool vec = (K % 8 == 0) && (lda % 8 == 0) && (ldb % 8 == 0) && aligned16(A) &&
                   aligned16(B);
  if (vec) {
    const int64_t nb = ((M + kBM - 1) / kBM) * ((N + kBN - 1) / kBN);
    if (nb > 0x7fffffffLL) return set_error(TPP_E_UNSUPPORTED, "%s: too many tiles", name);
    gemm_kernel<T, EPI, ACT><<<dim3((unsigned)nb), dim3(256), 0, st>>>(
        (const T *)A, lda, (const T *)B, ldb, (T *)C, ldc, (const T *)bias, (int)M, (int)N,
        (int)K);
  } else {
    const int64_t NO = (EPI == kGSwiGLU) ? N / 2 : N;
    const int64_t blocks = (M * NO + 255) / 256;
    gemm_scalar_kernel<T, EPI, ACT><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
        (const T *)A, lda, (const T *)B, ldb, (T *)C, ldc, (const T *)bias, (int)M, (int)NO,
        (int)K);
  }
  return check_launch(name);
}

static int gemm_args(const char *name, const void *x, const void *w, const void *y, int64_t M,
                     int64_t N, int64_t K, int64_t ldx) {
  if (!x || !w || !y) return set_error(TPP_E_INVALID, "%s: null pointer", name);
  if (M < 0 || N < 1 || K < 1)
    return set_error(TPP_E_INVALID, "%s: invalid shapes (M=%lld N=%lld K=%lld)", name,
                     (long long)M, (long long)N, (long long)K);
  if (M > 0x7fffffffLL || N > 0x7fffffffLL || K > 0x7fffffffLL)
    return set_error(TPP_E_UNSUPPORTED, "%s: dimension exceeds 2^31-1", name);
  if (ldx < K) return set_error(TPP_E_INVALID, "%s: ldx < K", name);
  return TPP_OK;
}

} // namespace tpp

using namespace tpp;

extern "C" int tpp_linear_act(const void *x, const void *w, const void *bias, void *y,
                              int64_t M, int64_t N, int64_t K, int64_t ldx, int64_t ldy,
                              int act, int dtype, void *stream) {
  const char *name = "tpp_linear_act";
  if (int e = gemm_args(name, x, w, y, M, N, K, ldx)) return e;
  if (ldy < N) return set_error(TPP_E_INVALID, "%s: ldy < N", name);
  if (act < TPP_ACT_NONE || act > TPP_ACT_RELU)
    return set_error(TPP_E_INVALID, "%s: unknown activation %d", name, act);
  hipStream_t st = as_stream(stream);
  return TPP_DISPATCH_HALF(dtype, [&] {
    if (!bias && act == TPP_ACT_NONE)
      return launch_gemm<T, kGPlain, TPP_ACT_NONE>(x, ldx, w, K, y, ldy, nullptr, M, N, K, st,
                                                   name);
    switch (act) {
    case TPP_ACT_GELU_TANH:
      return launch_gemm<T, kGBiasAct, TPP_ACT_GELU_TANH>(x, ldx, w, K, y, ldy, bias, M, N, K,
                                                          st, name);
    case TPP_ACT_SILU:
      return launch_gemm<T, kGBiasAct, TPP_ACT_SILU>(x, ldx, w, K, y, ldy, bias, M, N, K, st,
                                                     name);
    case TPP_ACT_RELU:
      return launch_gemm<T, kGBiasAct, TPP_ACT_RELU>(x, ldx, w, K, y, ldy, bias, M, N, K, st,
                                                     name);
    default:
      return launch_gemm<T, kGBiasAct, TPP_ACT_NONE>(x, ldx, w, K, y, ldy, bias, M, N, K, st,
                                                     name);
    }
  });
}

extern "C" int tpp_linear_swiglu(const void *x, const void *w_gu, void *y, int64_t M,
                                 int64_t I, int64_t K, int64_t ldx, int64_t ldy, int dtype,
                                 void *stream) {
  const char *name = "tpp_linear_swiglu";
  if (int e = gemm_args(name, x, w_gu, y, M, 2 * I, K, ldx)) return e;
  if (I % 32 != 0)
    return set_error(TPP_E_UNSUPPORTED, "%s: intermediate size must be a multiple of 32", name);
  if (ldy < I) return set_error(TPP_E_INVALID, "%s: ldy < I", name);
  hipStream_t st = as_stream(stream);
  return TPP_DISPATCH_HALF(dtype, [&] {
    return launch_gemm<T, kGSwiGLU, TPP_ACT_NONE>(x, ldx, w_gu, K, y, ldy, nullptr, M, 2 * I,
                                                  K, st, name);
  });
}
