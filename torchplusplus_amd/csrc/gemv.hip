// Decode GEMV for gfx950: y[b, n] = sum_k x[b, k] * W[n, k], batch B <= 16.
//
// Reference: hgemvK128F16x4Kernel (csrc/blas/hgemv/hgemv_kernels.cuh:19-67),
// one warp per output row with fp16 accumulation; its CPU check is
// hgemvCpu (hgemv_bench.cpp:10-24). In the model these GEMVs are the
// nn.Linear calls of a decode step (B = batch size, one token each).
//
// Design (HBM-bound on W, latency-bound at decode sizes):
//  * A block owns 16 weight rows. One v_mfma_f32_16x16x32 consumes 16 rows x
//    32 K of W (operand B: each lane loads 16 contiguous bytes of one row)
//    and the matching 16 x 32 of x (operand A, batch rows >= B are zero), so
//    W is streamed once for all B <= 16 rows of x, with 128-bit loads only.
//  * K is split over up to 12 waves of the block (256 K per wave, every W
//    load of a wave issued before the first MFMA), reduced through LDS. No
//    cross-block reduction; at most 1024 blocks loop over the row tiles.
//  * Fusions for the decoder step:
//      norm_w != NULL   the input is RMSNorm(x) * norm_w (fastqwen3.py:108,114:
//                       the block recomputes the 16 row statistics itself)
//      residual != NULL residual <- T(residual + T(x W^T)) in place (the
//                       `x = x + x_res` of fastqwen3.py:111,116)
//      SwiGLU           W = [gate|up] interleaved in blocks of 32 rows; output
//                       T(T(silu(T(g))) * T(u)) (eager silu(gate(x)) * up(x))
//      bias + act       pre-activation rounded to T, activation in fp32
//                       (fused_gemm.cuh:93-105)
//      argmax           per-block (max, first index) over the 16 columns for
//                       every batch row; tpp_argmax_partials finishes it.
#include "tpp_common.hpp"

namespace tpp {

enum GemvEpi { kEpiPlain = 0, kEpiBiasAct = 1, kEpiSwiGLU = 2, kEpiResidual = 3 };

constexpr int kGemvWaveK = 256;   // K elements per wave and load batch
constexpr int kGemvMaxWaves = 12; // 768 threads: 170 VGPRs per lane, no spills

// 16 zero bytes in device memory (zero-initialised, never written): what a
// skipped load reads instead. Not const: a pointer into the constant address
// space mixed with global ones would turn every such load into a flat load.
__device__ uint32_t g_gemv_zero16[4];

// 16-byte load of 8 elements, zero unless ok. The load is always issued, from
// the zero bytes when !ok: a load under a branch makes the compiler's later
// waits drain every load in flight (one memory round trip becomes several),
// and selecting the value after the load would wait for it on the spot.
template <typename T>
__device__ __forceinline__ typename VecT<T>::v8 ld16(const T *p, bool ok) {
  typedef typename VecT<T>::v8 V;
  return *reinterpret_cast<const V *>(ok ? p : reinterpret_cast<const T *>(g_gemv_zero16));
}
// 16 bytes the same way as inline asm, invisible to the compiler's wait
// counts: the caller waits with vm_wait_tied
template <typename T>
__device__ __forceinline__ typename VecT<T>::v8 ld16_asm(const T *p, bool ok) {
  typename VecT<T>::v8 r;
  const void *q = ok ? (const void *)p : (const void *)g_gemv_zero16;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(r) : "v"(q));
  return r;
}
// s_waitcnt vmcnt(N) that also redefines the loaded registers (see
// lds_wait_tied): a and b complete once at most N later loads are in flight
template <int N, typename V>
__device__ __forceinline__ void vm_wait_tied(V (&a)[8], V (&b)[8]) {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%16)"
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]),
                 "+v"(a[6]), "+v"(a[7]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]),
                 "+v"(b[4]), "+v"(b[5]), "+v"(b[6]), "+v"(b[7])
               : "n"(N));
}
// one element the same way, returned unconverted: a conversion next to the
// load would make the wave wait for it (and every load before it) there
template <typename T>
__device__ __forceinline__ T ld1(const T *p, bool ok) {
  return *(ok ? p : reinterpret_cast<const T *>(g_gemv_zero16));
}

template <typename T>
__device__ __forceinline__ f32x4 mfma16(typename VecT<T>::v8 a, typename VecT<T>::v8 b,
                                        f32x4 c) {
  if constexpr (__is_same(T, bf16))
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

template <typename T> __device__ __forceinline__ T epi_swiglu(float g, float u) {
  const float gt = to_f32(from_f32<T>(g));
  const float s = to_f32(from_f32<T>(act_silu(gt)));
  const float ut = to_f32(from_f32<T>(u));
  return from_f32<T>(s * ut);
}

// (value, index) "better than" with first-index ties and NaN as the maximum
__device__ __forceinline__ bool am_better(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

struct GemvArgs {
  const void *x;
  int64_t ldx;
  int NB;
  const void *norm_w;
  float eps;
  const void *W;
  int64_t N, K;
  void *y;
  int64_t ldy;
  const void *bias;
  void *residual; // [NB, N] in/out, ld = ldy
  float *am_val;  // [tiles, NB] argmax partials (or null)
  int *am_idx;
  int kslice;
};

// Row tiles: 16 weight rows each (SwiGLU: 16 outputs from 16 gate + 16 up
// rows). grid.x <= kGemvMaxBlocks blocks loop over the tiles, so the fused
// input RMSNorm is computed once per block; block = 64 * nwaves threads,
// wave w covers K slice w of every tile.
constexpr int kGemvMaxBlocks = 1024;

// RT = weight rows per tile: 16, or 8 for launches with few tiles (the
// MFMA's columns 8..15 then repeat rows 0..7 from LDS and are discarded), so
// twice as many CUs each fetch half the bytes.
template <typename T, int EPI, int ACT, bool NORM, int MAXW, int RT = 16>
__global__ __launch_bounds__(64 * MAXW) void gemv16_kernel(GemvArgs a, int64_t tiles) {
  static_assert(RT == 16 || (RT == 8 && EPI != kEpiSwiGLU), "tile rows");
  typedef typename VecT<T>::v8 V8;
  constexpr int NS = kGemvWaveK / 32; // MFMA steps per wave batch
  __shared__ f32x4 red[EPI == kEpiSwiGLU ? 2 : 1][MAXW][64];
  __shared__ float s_inv[16];
  __shared__ float s_part[MAXW][16];
  const int lane = lane_id(), w = wave_id(), nw = blockDim.x / kWave;
  const int r = lane & 15, g = lane >> 4;
  const int rr = r % RT; // this lane's weight row in the tile
  const int64_t N = a.N, K = a.K;
  const T *X = (const T *)a.x;
  const T *W = (const T *)a.W;
  const bool xok = r < a.NB;
  const T *xr = X + (xok ? r : 0) * a.ldx;
  const int64_t k_begin = (int64_t)w * a.kslice;
  const int64_t k_end = k_begin + a.kslice < K ? k_begin + a.kslice : K;

  auto rows_of = [&](int64_t tile, int64_t &row0, int64_t &row1) {
    if constexpr (EPI == kEpiSwiGLU) {
      row0 = (tile >> 1) * 64 + (tile & 1) * 16;
      row1 = row0 + 32;
    } else {
      row0 = tile * RT;
      row1 = 0;
    }
  };
  // W of one tile for this wave's K batch at k, plus the residual values
  // the tile will update
  auto load_w = [&](int64_t tile, int64_t k, V8 (&b0)[NS], V8 (&b1)[NS], T (&res)[4]) {
    int64_t row0, row1;
    rows_of(tile, row0, row1);
    const bool w0ok = row0 + rr < N;
    const T *w0 = W + (w0ok ? row0 + rr : 0) * K;
    const bool w1ok = (EPI == kEpiSwiGLU) && (row1 + r < N);
    const T *w1 = W + (w1ok ? row1 + r : 0) * K;
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int64_t c = k + u * 32 + g * 8;
      const bool in = c < k_end;
      b0[u] = ld16(w0 + c, in && w0ok);
      if constexpr (EPI == kEpiSwiGLU) b1[u] = ld16(w1 + c, in && w1ok);
    }
    if constexpr (EPI == kEpiResidual) {
      // every wave loads (branch-free); wave 0's values are the ones used
      const T *rs = (const T *)a.residual;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int b = 4 * g + i;
        res[i] = ld1(rs + (int64_t)b * a.ldy + row0 + rr, row0 + rr < N && b < a.NB);
      }
    }
  };
  // One K batch per wave (x stays resident): the tile's weights go HBM ->
  // LDS by LDS-DMA into this wave's slot (16 rows x 512 bytes per row set;
  // instruction j covers rows 2j, 2j+1 with whole 128-byte lines, lane i
  // fetching unit (i % 32) ^ row so that the MFMA-layout reads below hit 16
  // distinct bank groups), then are read back as B operands. Loaded straight
  // into the MFMA layout (16 rows x 64 bytes per instruction) the same
  // weights stream at about a quarter of the rate per CU. Rows past N read
  // row N-1 and units past K read the last unit (finite data, multiplied by
  // x = 0 or discarded). The first tile's DMA is issued right after the
  // input loads (every block has a first tile): the two are in flight
  // together, and since loads complete in issue order the input can be used
  // (row statistics, normalisation) while the weights are still on the way.
  constexpr int NSET = EPI == kEpiSwiGLU ? 2 : 1;
  extern __shared__ __attribute__((aligned(16))) char gemv_smem[];
  V8 *wslot = reinterpret_cast<V8 *>(gemv_smem) + (size_t)w * NSET * (RT * 32);
  const int drow = lane >> 5, dpos = lane & 31;
  auto issue_w = [&](int64_t tile, T (&res)[4]) {
    int64_t row0, row1;
    rows_of(tile, row0, row1);
#pragma unroll
    for (int set = 0; set < NSET; ++set) {
      const int64_t rb = set == 0 ? row0 : row1;
#pragma unroll
      for (int j = 0; j < RT / 2; ++j) {
        const int row = 2 * j + drow;
        const int64_t gr = rb + row < N ? rb + row : N - 1;
        int64_t kk = k_begin + (int64_t)((dpos ^ row) * 8);
        kk = kk < K - 8 ? kk : K - 8;
        __builtin_amdgcn_global_load_lds(
            (const void *)(W + gr * K + kk),
            (__attribute__((address_space(3))) void *)(wslot + set * (RT * 32) + j * 64), 16, 0,
            kCpolNT);
      }
    }
    if constexpr (EPI == kEpiResidual) {
      // wave 0's values are the ones used. With the fused RMSNorm every wave
      // loads them (branch-free): the input's counted asm wait counts these
      // loads. Without it only wave 0 does, which measured faster (o_proj
      // at batch 8 4.48 against 4.65 us cold, decode step 1.2% shorter).
      const T *rs = (const T *)a.residual;
      if (NORM || w == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int b = 4 * g + i;
          res[i] = ld1(rs + (int64_t)b * a.ldy + row0 + rr, row0 + rr < N && b < a.NB);
        }
      }
    }
  };
  // the slot's weights as B operands (waits for this wave's DMA; the slot
  // may be refilled once this returns)
  auto fetch_w = [&](V8 (&b0)[NS], V8 (&b1)[NS]) {
    __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8)); // vmcnt(0)
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      b0[u] = wslot[rr * 32 + ((u * 4 + g) ^ rr)];
      if constexpr (EPI == kEpiSwiGLU) b1[u] = wslot[16 * 32 + r * 32 + ((u * 4 + g) ^ r)];
    }
    __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0): reads done
  };
  const bool x_res = k_end - k_begin <= kGemvWaveK;
  V8 pa0[NS], pa1[NS];
  T ra[4] = {};

  // this wave's slice of the (normalised) input, reused by every tile
  // kept resident when the wave's K slice is one load batch (K <= 4096 for
  // plain GEMVs, 2048 for SwiGLU); longer slices reload x per batch
  V8 xa[NS];
  auto load_x = [&](int64_t k, V8 (&dst)[NS]) {
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int64_t c = k + u * 32 + g * 8; // K % 8 == 0: a chunk is all in or all out
      const bool ok = c < k_end && xok;
      dst[u] = ld16(xr + c, ok);
      if constexpr (NORM) {
        // zero where !ok: both factors are zero there
        const V8 nw8 = ld16((const T *)a.norm_w + c, ok);
        const float inv = s_inv[r];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          dst[u][i] = from_f32<T>((to_f32(dst[u][i]) * inv) * to_f32(nw8[i]));
      }
    }
  };
  if constexpr (NORM) {
    if (x_res) {
      // the wave's raw slice doubles as its share of the row statistics:
      // partial sums of squares over the K slices meet in LDS, so the input
      // is read once and there is one barrier before the normalisation
      V8 nwv[NS];
#pragma unroll
      for (int u = 0; u < NS; ++u) {
        const int64_t c = k_begin + u * 32 + g * 8;
        xa[u] = ld16_asm(xr + c, c < k_end && xok);
        nwv[u] = ld16_asm((const T *)a.norm_w + c, c < k_end);
      }
      __builtin_amdgcn_sched_barrier(0);
      issue_w(blockIdx.x, ra);
      // all loads out before the first use (the scheduler would otherwise
      // start the sums on the first row chunk and wait for it mid-issue);
      // the weight DMA (and residual loads) issued after the input stay in
      // flight: the input loads are asm, since after an LDS-DMA the
      // compiler's own wait for a plain load is vmcnt(0)
      __builtin_amdgcn_sched_barrier(0);
      vm_wait_tied<(RT / 2) * NSET + (EPI == kEpiResidual ? 4 : 0)>(xa, nwv);
      float ss = 0.f;
#pragma unroll
      for (int u = 0; u < NS; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float v = to_f32(xa[u][i]);
          ss += v * v;
        }
      ss += __shfl_xor(ss, 16, kWave); // lanes r, r+16, r+32, r+48: row r
      ss += __shfl_xor(ss, 32, kWave);
      if (g == 0) s_part[w][r] = ss;
      lds_barrier(); // (a fenced barrier would also wait for the weight DMA)
      float tot = 0.f;
      for (int i = 0; i < nw; ++i) tot += s_part[i][r];
      const float inv = rsqrtf(tot / (float)K + a.eps);
#pragma unroll
      for (int u = 0; u < NS; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i)
          xa[u][i] = from_f32<T>((to_f32(xa[u][i]) * inv) * to_f32(nwv[u][i]));
    } else {
      // inv_rms of the <= 16 input rows (wave w: rows w, w + nw, ..)
      for (int row = w; row < a.NB; row += nw) {
        const T *xp = X + row * a.ldx;
        float ss = 0.f;
        for (int64_t c = (int64_t)lane * 8; c < K; c += 64 * 8) {
          float v[8];
          load8(xp + c, v);
#pragma unroll
          for (int i = 0; i < 8; ++i) ss += v[i] * v[i];
        }
        ss = wave_sum(ss);
        if (lane == 0) s_inv[row] = rsqrtf(ss / (float)K + a.eps);
      }
      __syncthreads();
    }
  } else if (x_res) {
    // Rows past the batch skip their input loads (a load under a branch, so
    // the compiler waits for the first of them before the weight DMA goes
    // out). Against the branch-free form (every lane loads, rows past the
    // batch from the zero bytes), measured on three boxes: [1x3072] x
    // [1024x3072]^T 4.08-4.13 against 4.35-4.40 us cold, o_proj at batch 8
    // 4.40-4.65 against 4.66-4.72 us, the decode step equal to 1.4% shorter.
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      const int64_t c = k_begin + u * 32 + g * 8;
      if (c < k_end && xok) {
        xa[u] = *reinterpret_cast<const V8 *>(xr + c);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) xa[u][i] = (T)0.0f;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    issue_w(blockIdx.x, ra);
  }

  // per-block running argmax over all tiles (wave 0, lanes r == 0 hold it)
  float am_v[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  int am_i[4] = {0x7fffffff, 0x7fffffff, 0x7fffffff, 0x7fffffff};

  // block-wide K reduction of a tile's accumulators and its epilogue
  auto finish = [&](int64_t tile, f32x4 acc0, f32x4 acc1, const T (&res_in)[4]) {
    int64_t row0, row1;
    rows_of(tile, row0, row1);
    red[0][w][lane] = acc0;
    if constexpr (EPI == kEpiSwiGLU) red[1][w][lane] = acc1;
    lds_barrier(); // the next tile's weight DMA stays in flight
    if (w == 0) {
      acc0 = red[0][0][lane];
      for (int i = 1; i < nw; ++i) acc0 += red[0][i][lane];
      if constexpr (EPI == kEpiSwiGLU) {
        acc1 = red[1][0][lane];
        for (int i = 1; i < nw; ++i) acc1 += red[1][i][lane];
      }
      // D layout of 16x16x32: lane -> column r (weight row), rows b = 4g + i.
      // (RT = 8: columns 8..15 repeat rows 0..7 and are not stored)
      const int64_t n0 = r < RT ? row0 + r : INT64_MAX, n1 = row1 + r;
      T *Y = (T *)a.y;
      if (a.am_val) { // running argmax over this block's columns
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float bv = n0 < N ? to_f32(from_f32<T>(acc0[i])) : -INFINITY;
          int bix = n0 < N ? (int)n0 : 0x7fffffff;
#pragma unroll
          for (int sh = 1; sh < 16; sh <<= 1) {
            const float ov = __shfl_xor(bv, sh, kWave);
            const int oi = __shfl_xor(bix, sh, kWave);
            if (am_better(ov, oi, bv, bix)) bv = ov, bix = oi;
          }
          if (am_better(bv, bix, am_v[i], am_i[i])) am_v[i] = bv, am_i[i] = bix;
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int b = 4 * g + i;
        if (b >= a.NB) continue;
        if constexpr (EPI == kEpiSwiGLU) {
          if (n0 < N && n1 < N) {
            const int64_t on = (tile >> 1) * 32 + (tile & 1) * 16 + r;
            Y[(int64_t)b * a.ldy + on] = epi_swiglu<T>(acc0[i], acc1[i]);
          }
        } else if (n0 < N) {
          if constexpr (EPI == kEpiResidual) {
            const float v = to_f32(from_f32<T>(acc0[i]));
            ((T *)a.residual)[(int64_t)b * a.ldy + n0] = from_f32<T>(to_f32(res_in[i]) + v);
          } else if constexpr (EPI == kEpiBiasAct) {
            Y[(int64_t)b * a.ldy + n0] = epi_bias_act<T, ACT>(acc0[i], (const T *)a.bias, n0);
          } else if (Y) {
            Y[(int64_t)b * a.ldy + n0] = from_f32<T>(acc0[i]);
          }
        }
      }
    }
    lds_barrier(); // red[] is reused by the next tile
  };
  auto mfma_batch = [&](const V8 (&xv)[NS], const V8 (&b0)[NS], const V8 (&b1)[NS], f32x4 &acc0,
                        f32x4 &acc1) {
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      acc0 = mfma16<T>(xv[u], b0[u], acc0);
      if constexpr (EPI == kEpiSwiGLU) acc1 = mfma16<T>(xv[u], b1[u], acc1);
    }
  };

  const int64_t stride = gridDim.x;
  if (x_res) {
    // two tiles in flight: tile t in registers while the DMA of tile
    // t + stride fills the slot
    for (int64_t t = blockIdx.x; t < tiles; t += stride) {
      fetch_w(pa0, pa1);
      T rc[4] = {ra[0], ra[1], ra[2], ra[3]};
      if (t + stride < tiles) issue_w(t + stride, ra);
      f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
      mfma_batch(xa, pa0, pa1, c0, c1);
      finish(t, c0, c1, rc);
    }
  } else {
    for (int64_t tile = blockIdx.x; tile < tiles; tile += stride) {
      f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
      T res[4] = {};
      for (int64_t k = k_begin; k < k_end; k += kGemvWaveK) {
        V8 b0[NS], b1[NS], xl[NS];
        load_w(tile, k, b0, b1, res);
        load_x(k, xl);
        mfma_batch(xl, b0, b1, c0, c1);
      }
      finish(tile, c0, c1, res);
    }
  }
  if (a.am_val && w == 0 && r == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = 4 * g + i;
      if (b < a.NB) {
        a.am_val[(int64_t)blockIdx.x * a.NB + b] = am_v[i];
        a.am_idx[(int64_t)blockIdx.x * a.NB + b] = am_i[i];
      }
    }
  }
}

// Generic fallback (any K, alignment, batch): one thread per output.
template <typename T, int EPI, int ACT, bool NORM>
__global__ __launch_bounds__(256) void gemv_scalar_kernel(GemvArgs a, int64_t NO) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= NO * a.NB) return;
  const int b = (int)(t / NO);
  const int64_t o = t - (int64_t)b * NO;
  const T *xr = (const T *)a.x + b * a.ldx;
  const T *W = (const T *)a.W;
  const int64_t K = a.K;
  float inv = 1.f;
  if constexpr (NORM) {
    float ss = 0.f;
    for (int64_t k = 0; k < K; ++k) ss += to_f32(xr[k]) * to_f32(xr[k]);
    inv = rsqrtf(ss / (float)K + a.eps);
  }
  auto xin = [&](int64_t k) {
    if constexpr (NORM) return to_f32(from_f32<T>((to_f32(xr[k]) * inv) * to_f32(((const T *)a.norm_w)[k])));
    else return to_f32(xr[k]);
  };
  T *Y = (T *)a.y;
  if constexpr (EPI == kEpiSwiGLU) {
    const int64_t n0 = (o / 32) * 64 + (o % 32), n1 = n0 + 32;
    float gs = 0.f, us = 0.f;
    for (int64_t k = 0; k < K; ++k) {
      const float xv = xin(k);
      gs += xv * to_f32(W[n0 * K + k]);
      us += xv * to_f32(W[n1 * K + k]);
    }
    Y[b * a.ldy + o] = epi_swiglu<T>(gs, us);
  } else {
    float acc = 0.f;
    for (int64_t k = 0; k < K; ++k) acc += xin(k) * to_f32(W[o * K + k]);
    if constexpr (EPI == kEpiResidual) {
      T *res = (T *)a.residual + b * a.ldy + o;
      *res = from_f32<T>(to_f32(*res) + to_f32(from_f32<T>(acc)));
    } else if constexpr (EPI == kEpiBiasAct) {
      Y[b * a.ldy + o] = epi_bias_act<T, ACT>(acc, (const T *)a.bias, o);
    } else {
      Y[b * a.ldy + o] = from_f32<T>(acc);
    }
  }
}

// Final reduction of the per-block argmax partials of row b; block = 1024.
__device__ __forceinline__ int argmax_finish(const float *__restrict__ val,
                                             const int *__restrict__ idx, int nparts, int NB,
                                             int b) {
  __shared__ float sv[16];
  __shared__ int si[16];
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int t = threadIdx.x; t < nparts; t += blockDim.x) {
    const float v = val[(int64_t)t * NB + b];
    const int i = idx[(int64_t)t * NB + b];
    if (am_better(v, i, bv, bi)) bv = v, bi = i;
  }
#pragma unroll
  for (int sh = 1; sh < kWave; sh <<= 1) {
    const float ov = __shfl_xor(bv, sh, kWave);
    const int oi = __shfl_xor(bi, sh, kWave);
    if (am_better(ov, oi, bv, bi)) bv = ov, bi = oi;
  }
  if (lane_id() == 0) {
    sv[wave_id()] = bv;
    si[wave_id()] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x / kWave); ++w)
      if (am_better(sv[w], si[w], bv, bi)) bv = sv[w], bi = si[w];
    si[0] = bi;
  }
  __syncthreads();
  return si[0];
}

__global__ __launch_bounds__(1024) void argmax_partials_kernel(const float *__restrict__ val,
                                                               const int *__restrict__ idx,
                                                               int nparts, int NB,
                                                               int64_t *__restrict__ out) {
  const int tok = argmax_finish(val, idx, nparts, NB, blockIdx.x);
  if (threadIdx.x == 0) out[blockIdx.x] = tok;
}

// Greedy decode step epilogue: token = argmax; ids[b] = token; the next
// step's residual row <- embedding[token]; positions[b]++, seqlens[b]++.
template <typename T>
__global__ __launch_bounds__(1024) void greedy_advance_kernel(
    const float *__restrict__ val, const int *__restrict__ idx, int nparts, int NB,
    const T *__restrict__ emb, int64_t E, int64_t *__restrict__ ids, T *__restrict__ resid,
    int *__restrict__ positions, int *__restrict__ seqlens) {
  const int b = blockIdx.x;
  const int tok = argmax_finish(val, idx, nparts, NB, b);
  if (threadIdx.x == 0) {
    ids[b] = tok;
    if (positions) positions[b] += 1;
    if (seqlens) seqlens[b] += 1;
  }
  const T *src = emb + (int64_t)tok * E;
  T *dst = resid + (int64_t)b * E;
  for (int64_t e = threadIdx.x; e < E; e += blockDim.x) dst[e] = src[e];
}

static bool gemv_vec_ok(const GemvArgs &a) {
  return (a.K % 8 == 0) && (a.ldx % 8 == 0) && aligned16(a.x) && aligned16(a.W) &&
         (a.norm_w == nullptr || aligned16(a.norm_w)) && a.NB <= 16;
}

// ---------------------------------------------------------------------------
// Wide GEMV (many row tiles, K in {256, 512, 768, 1024}, plain epilogue: the
// lm_head). Every
// wave owns whole 16-row tiles, so the stream has no cross-wave reduction and
// no barrier. Weights go HBM -> LDS by LDS-DMA in 16-row x 256-k chunks
// (each row's 512 bytes read by 32 consecutive lanes: whole 128-byte lines)
// through a per-wave ring of kWideRing chunks; MFMA operands are read back
// with ds_read_b128 (16-byte unit u of row r stored at u ^ r: the 16 rows a
// read serves per cycle then sit in 16 distinct 16-byte bank groups);
// the (normalised) input stays in VGPRs as the A operand for the whole K.
constexpr int kWideRing = 4;          // chunks per wave ring (3 in flight)
constexpr int kWideBlocks = 256;      // one 4-wave block per CU
constexpr int64_t kWideMinTiles = 2048;

template <int N> __device__ __forceinline__ void gemv_wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// s_waitcnt vmcnt(N) tied to every register of a (M a multiple of 8): the
// wait redefines the first eight, empty statements after it (kept in order:
// all are volatile) the rest, so no use of any of them moves above the wait
template <int N, typename V, int M>
__device__ __forceinline__ void vm_wait_tied_all(V (&a)[M]) {
  static_assert(N >= 0 && N < 64 && M % 8 == 0, "vmcnt is 6 bits; whole groups of 8");
  asm volatile("s_waitcnt vmcnt(%8)"
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]),
                 "+v"(a[6]), "+v"(a[7])
               : "n"(N));
#pragma unroll
  for (int i = 8; i < M; i += 8)
    asm volatile(""
                 : "+v"(a[i]), "+v"(a[i + 1]), "+v"(a[i + 2]), "+v"(a[i + 3]), "+v"(a[i + 4]),
                   "+v"(a[i + 5]), "+v"(a[i + 6]), "+v"(a[i + 7]));
}

template <typename T, bool NORM, int KC>
__global__ __launch_bounds__(256) void gemv_wide_kernel(GemvArgs a, int64_t tiles) {
  typedef typename VecT<T>::v8 V8;
  constexpr int NWD = (KC * 32 + 63) / 64; // norm weight DMA instructions (64 units each)
  __shared__ V8 ring[4][kWideRing][16 * 32]; // [wave][slot][row * 32 + (unit ^ row)]
  __shared__ V8 s_nw[4][NWD * 64];           // [wave][16-byte unit of the norm weight]
  __shared__ float s_bv[4][16];
  __shared__ int s_bi[4][16];
  const int lane = lane_id(), w = __builtin_amdgcn_readfirstlane(wave_id());
  const int r = lane & 15, g = lane >> 4;
  const int64_t K = a.K, N = a.N;
  const T *X = (const T *)a.x;
  const T *W = (const T *)a.W;
  const int64_t wg = (int64_t)blockIdx.x * 4 + w, nwg = (int64_t)gridDim.x * 4;
  // this wave's tiles: wg, wg + nwg, ...; its chunk stream n = tile_i * KC + c
  const int64_t my_tiles = wg < tiles ? (tiles - 1 - wg) / nwg + 1 : 0;
  const int64_t nchunks = my_tiles * KC;

  // Input rows (<= 16) as A fragments for all K (K = 256 KC): step u covers
  // k = 32u + 8g, so lanes r, r+16, r+32, r+48 hold all of row r and the row
  // statistics need no loads of their own. These loads go out first, as
  // inline asm, then the norm weight and the first weight chunks by LDS-DMA:
  // loads complete in issue order, so counted waits take the input, then the
  // norm weight, while the weights stream in behind them (after an LDS-DMA
  // the compiler's own wait for a plain load would be vmcnt(0)).
  const bool xok = r < a.NB;
  const T *xr = X + (xok ? r : 0) * a.ldx;
  V8 xa[KC * 8];
#pragma unroll
  for (int u = 0; u < KC * 8; ++u) xa[u] = ld16_asm(xr + (int64_t)u * 32 + g * 8, xok);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (NORM) {
    // K / 8 units of 16 bytes into this wave's LDS (lanes past them fetch the
    // last unit again into the array's padding)
#pragma unroll
    for (int i = 0; i < NWD; ++i) {
      const int unit = i * 64 + lane < KC * 32 ? i * 64 + lane : KC * 32 - 1;
      __builtin_amdgcn_global_load_lds((const void *)((const T *)a.norm_w + unit * 8),
                                       (__attribute__((address_space(3))) void *)&s_nw[w][i * 64],
                                       16, 0, 0);
    }
  }

  // DMA of chunk n (16 rows x 256 k of tile wg + (n / KC) nwg) into ring slot
  // n % kWideRing. Instruction j covers rows 2j, 2j+1; lane i lands at slot
  // offset i and so fetches unit (i % 32) ^ row of row 2j + i / 32. Source:
  // the tile's first row (wave-uniform) plus a per-lane 32-bit byte offset;
  // rows past N read row N-1 (finite data, never stored). Past the end of the
  // stream the last chunk is fetched again, so every wave keeps the same
  // issue pattern.
  const int drow = lane >> 5, dpos = lane & 31;
  unsigned xo[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) xo[j] = (unsigned)((dpos ^ (2 * j + drow)) * 8 * (int)sizeof(T));
  const unsigned rowb = (unsigned)(K * (int64_t)sizeof(T)); // bytes per weight row
  auto issue = [&](int64_t n) {
    const int64_t nn = n < nchunks ? n : nchunks - 1;
    const int64_t tile = nn >= 0 ? wg + (nn / KC) * nwg : 0;
    const int c = nn >= 0 ? (int)(nn % KC) : 0;
    const char *tb = reinterpret_cast<const char *>(W + tile * 16 * K) + c * 256 * (int)sizeof(T);
    const int lim = (int)(N - 1 - tile * 16); // last row of the matrix, relative to the tile
    V8 *dst = ring[w][(int)(n % kWideRing)];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int row = 2 * j + drow;
      const unsigned off = (unsigned)(row < lim ? row : lim) * rowb + xo[j];
      __builtin_amdgcn_global_load_lds((const void *)(tb + off),
                                       (__attribute__((address_space(3))) void *)(dst + j * 64),
                                       16, 0, kCpolNT);
    }
  };
#pragma unroll
  for (int p = 0; p < kWideRing - 1; ++p) issue(p);

  // the input landed (norm weight and weight chunks may be in flight)
  constexpr int NDMA0 = (NORM ? NWD : 0) + (kWideRing - 1) * 8;
  vm_wait_tied_all<NDMA0>(xa);
  if constexpr (NORM) {
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < KC * 8; ++u)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = to_f32(xa[u][i]);
        ss += v * v;
      }
    ss += __shfl_xor(ss, 16, kWave);
    ss += __shfl_xor(ss, 32, kWave);
    const float inv = rsqrtf(ss / (float)K + a.eps);
    // the norm weight landed in LDS; read back as asm (the compiler would
    // wait for every LDS-DMA in flight before a plain LDS read)
    gemv_wait_vmcnt<(kWideRing - 1) * 8>();
    const unsigned nwb = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) char *)&s_nw[w][0];
#pragma unroll
    for (int u0 = 0; u0 < KC * 8; u0 += 8) {
      V8 nw8[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) nw8[u] = lds_read_b128<0, V8>(nwb + (unsigned)(((u0 + u) * 4 + g) * 16));
      lds_wait_tied<0>(nw8);
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int i = 0; i < 8; ++i)
          xa[u0 + u][i] = from_f32<T>((to_f32(xa[u0 + u][i]) * inv) * to_f32(nw8[u][i]));
    }
  }

  float bv[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  int bi[4] = {0x7fffffff, 0x7fffffff, 0x7fffffff, 0x7fffffff};
  T *Y = (T *)a.y;
  // MFMA operands from the ring by inline-asm LDS reads with explicit waits:
  // the compiler's wait-count pass cannot tell which slot an LDS-DMA writes
  // and, for plain reads, waited for all of them (vmcnt(0)) once per tile,
  // draining the ring
  const unsigned rbase = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) char *)&ring[w][0][0];
  unsigned roff[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) roff[u] = (unsigned)((r * 32 + ((u * 4 + g) ^ r)) * 16);
  for (int64_t ti = 0; ti < my_tiles; ++ti) {
    const int64_t tile = wg + ti * nwg;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      const int64_t n = ti * KC + c;
      gemv_wait_vmcnt<(kWideRing - 2) * 8>(); // chunk n landed (own DMA)
      // refill the slot read at step n - 1 first (its reads completed: the
      // MFMAs of that step consumed them)
      issue(n + kWideRing - 1);
      const unsigned sb = rbase + (unsigned)(n % kWideRing) * (16 * 32 * 16);
      V8 b[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) b[u] = lds_read_b128<0, V8>(sb + roff[u]);
      lds_wait_tied<0>(b);
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = mfma16<T>(xa[c * 8 + u], b[u], acc);
    }
    // D layout of 16x16x32: lane -> weight row tile*16 + r, rows b = 4g + i
    const int64_t col = tile * 16 + r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = 4 * g + i;
      const T yv = from_f32<T>(acc[i]);
      if (col < N && b < a.NB) {
        if (Y) Y[(int64_t)b * a.ldy + col] = yv;
        const float v = to_f32(yv);
        if (am_better(v, (int)col, bv[i], bi[i])) bv[i] = v, bi[i] = (int)col;
      }
    }
  }
  gemv_wait_vmcnt<0>(); // drain the refetches before the wave exits
  if (!a.am_val) return;
  // argmax over the 16 columns of each lane group, then over the 4 waves
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int sh = 1; sh < 16; sh <<= 1) {
      const float ov = __shfl_xor(bv[i], sh, kWave);
      const int oi = __shfl_xor(bi[i], sh, kWave);
      if (am_better(ov, oi, bv[i], bi[i])) bv[i] = ov, bi[i] = oi;
    }
    if (r == 0) {
      s_bv[w][4 * g + i] = bv[i];
      s_bi[w][4 * g + i] = bi[i];
    }
  }
  __syncthreads();
  if (threadIdx.x < (unsigned)a.NB) {
    const int b = threadIdx.x;
    float v = s_bv[0][b];
    int ix = s_bi[0][b];
    for (int ww = 1; ww < 4; ++ww)
      if (am_better(s_bv[ww][b], s_bi[ww][b], v, ix)) v = s_bv[ww][b], ix = s_bi[ww][b];
    a.am_val[(int64_t)blockIdx.x * a.NB + b] = v;
    a.am_idx[(int64_t)blockIdx.x * a.NB + b] = ix;
  }
}

template <typename T, bool NORM>
static bool launch_wide(const GemvArgs &a, hipStream_t st) {
  const int64_t tiles = (a.N + 15) / 16;
  if (tiles < kWideMinTiles || a.K > 1024 || a.K % 256 != 0) return false;
  const int kc = (int)((a.K + 255) / 256);
  const dim3 grid(kWideBlocks), block(256);
  switch (kc) {
  case 1: gemv_wide_kernel<T, NORM, 1><<<grid, block, 0, st>>>(a, tiles); break;
  case 2: gemv_wide_kernel<T, NORM, 2><<<grid, block, 0, st>>>(a, tiles); break;
  case 3: gemv_wide_kernel<T, NORM, 3><<<grid, block, 0, st>>>(a, tiles); break;
  default: gemv_wide_kernel<T, NORM, 4><<<grid, block, 0, st>>>(a, tiles); break;
  }
  return true;
}

// ---------------------------------------------------------------------------
// One input row (the reference's hgemv, y = A x, hgemv_kernels.cuh:19-85):
// a wave owns one weight row and reads it whole, lane l taking the 16-byte
// chunks l, l + 64, ... (CPL per lane), so each instruction reads a
// contiguous 1 KB of the row. The input row goes to LDS once per workgroup
// by LDS-DMA (its CPL instructions dealt to the waves), ahead of every
// weight load; chunks past the row end read chunk 0 and are multiplied by
// 0. Then fp32 products, a DPP wave reduction and the epilogue in one lane:
// no MFMA padding, one block per CU. (Measured on [1x3072]x[1024x3072]^T: a
// row per wave 3.06 us, two or four rows per wave 3.7 / 4.5 us, a row split
// over two waves with an LDS sum 3.14 us; the input through LDS instead of
// read by every wave (6 MB of L2 reads per launch for 6 MB of weights),
// 3.13-3.17 against 3.20-3.21 us in paired runs, the [1x1024] shape equal;
// the products by v_dot2 instead of conversions and FMAs: 3.28 -> 3.19 us
// and 2.97 -> 2.87 us cold.)
constexpr int kB1MaxLoads = 8; // 16-byte weight loads per lane


template <typename T, int EPI, int ACT, int CPL>
__global__ __launch_bounds__(1024) void gemv_b1_kernel(GemvArgs a) {
  typedef typename VecT<T>::v8 V8;
  __shared__ __attribute__((aligned(16))) V8 s_x[CPL * 64];
  const int lane = lane_id();
  const int w = __builtin_amdgcn_readfirstlane(wave_id()), nwv = blockDim.x / kWave;
  const int64_t n = (int64_t)blockIdx.x * nwv + w;
  const bool live = n < a.N; // waves past N still take part in the barrier
  const int nch = (int)(a.K / 8);
  const T *x = (const T *)a.x;
  const T *W = (const T *)a.W + (live ? n : 0) * a.K;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    if (i % nwv != w) continue; // wave-uniform
    const int c = lane + 64 * i;
    __builtin_amdgcn_global_load_lds((const void *)(x + (int64_t)(c < nch ? c : 0) * 8),
                                     (__attribute__((address_space(3))) void *)(s_x + i * 64),
                                     16, 0, 0);
  }
  __builtin_amdgcn_sched_barrier(0);
  V8 wr[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + 64 * i;
    wr[i] = ld_nt(reinterpret_cast<const V8 *>(W + (int64_t)(c < nch ? c : 0) * 8));
  }
  __builtin_amdgcn_sched_barrier(0);
  vm_wait<CPL>(); // this wave's input DMA (issued before its CPL weight loads)
  lds_barrier();  // every wave's
  if (!live) return;
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    V8 xv = s_x[i * 64 + lane];
    if (lane + 64 * i >= nch) { // a chunk past the row: x read as zeros
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[e] = (T)0.0f;
    }
    acc = dot8<T>(xv, wr[i], acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) {
    if constexpr (EPI == kEpiResidual) {
      T *res = (T *)a.residual + n;
      *res = from_f32<T>(to_f32(*res) + to_f32(from_f32<T>(acc)));
    } else if constexpr (EPI == kEpiBiasAct) {
      ((T *)a.y)[n] = epi_bias_act<T, ACT>(acc, (const T *)a.bias, n);
    } else {
      ((T *)a.y)[n] = from_f32<T>(acc);
    }
  }
}

// B = 1 without fused norm, SwiGLU or argmax, K % 8 == 0 and K <= 4096
template <typename T, int EPI, int ACT>
static bool launch_b1(const GemvArgs &a, hipStream_t st) {
  const int64_t cpl = (a.K / 8 + 63) / 64; // 16-byte chunks per lane
  if (a.NB != 1 || a.am_val || cpl > kB1MaxLoads || cpl < 1 || a.N > (int64_t)1 << 26) return false;
  int64_t wpb = (a.N + 255) / 256; // waves per block: one block per CU
  if (wpb > 16) wpb = 16;
  const dim3 grid((unsigned)((a.N + wpb - 1) / wpb)), block((unsigned)(64 * wpb));
  switch (cpl) {
  case 1: gemv_b1_kernel<T, EPI, ACT, 1><<<grid, block, 0, st>>>(a); break;
  case 2: gemv_b1_kernel<T, EPI, ACT, 2><<<grid, block, 0, st>>>(a); break;
  case 3: gemv_b1_kernel<T, EPI, ACT, 3><<<grid, block, 0, st>>>(a); break;
  case 4: gemv_b1_kernel<T, EPI, ACT, 4><<<grid, block, 0, st>>>(a); break;
  case 5: gemv_b1_kernel<T, EPI, ACT, 5><<<grid, block, 0, st>>>(a); break;
  case 6: gemv_b1_kernel<T, EPI, ACT, 6><<<grid, block, 0, st>>>(a); break;
  case 7: gemv_b1_kernel<T, EPI, ACT, 7><<<grid, block, 0, st>>>(a); break;
  default: gemv_b1_kernel<T, EPI, ACT, 8><<<grid, block, 0, st>>>(a); break;
  }
  return true;
}

template <typename T, int EPI, int ACT, bool NORM>
static int launch_gemv(GemvArgs a, hipStream_t st, const char *name) {
  const int64_t NO = (EPI == kEpiSwiGLU) ? a.N / 2 : a.N;
  if (!gemv_vec_ok(a)) {
    if (a.am_val) return set_error(TPP_E_UNSUPPORTED, "%s: argmax needs the vector path", name);
    const int64_t blocks = (NO * a.NB + 255) / 256;
    gemv_scalar_kernel<T, EPI, ACT, NORM><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(a, NO);
    return check_launch(name);
  }
  // 8-row tiles when 16-row ones would leave most CUs idle (not for SwiGLU,
  // whose tiles pair gate and up rows, nor with argmax partials, whose
  // workspace is sized for 16-row tiles)
  const bool rt8 = EPI != kEpiSwiGLU && !a.am_val && (a.N + 15) / 16 < 128;
  const int64_t tiles = (EPI == kEpiSwiGLU) ? (a.N / 64) * 2 : rt8 ? (a.N + 7) / 8 : (a.N + 15) / 16;
  if (tiles > 0x7fffffffLL) return set_error(TPP_E_UNSUPPORTED, "%s: N too large", name);
  if constexpr (EPI == kEpiPlain) {
    if (launch_wide<T, NORM>(a, st)) return check_launch(name);
  }
  if constexpr (EPI != kEpiSwiGLU && !NORM) {
    if (launch_b1<T, EPI, ACT>(a, st)) return check_launch(name);
  }
  // SwiGLU holds two W tiles per lane: cap its block at 8 waves (256 VGPRs)
  constexpr int MAXW = EPI == kEpiSwiGLU ? 8 : kGemvMaxWaves;
  int64_t nw = (a.K + kGemvWaveK - 1) / kGemvWaveK;
  if (nw > MAXW) nw = MAXW;
  if (nw < 1) nw = 1;
  const int64_t per = (a.K + nw - 1) / nw;
  a.kslice = (int)(((per + 31) / 32) * 32);
  const int64_t blocks = tiles < kGemvMaxBlocks ? tiles : kGemvMaxBlocks;
  // LDS weight slots of the one-batch-per-wave path (16 rows x 512 bytes per
  // row set and wave)
  const size_t lds = (size_t)nw * (EPI == kEpiSwiGLU ? 2 : 1) * (rt8 ? 8 : 16) * 512;
  if constexpr (EPI != kEpiSwiGLU) {
    if (rt8) {
      gemv16_kernel<T, EPI, ACT, NORM, MAXW, 8>
          <<<dim3((unsigned)blocks), dim3((unsigned)(nw * 64)), lds, st>>>(a, tiles);
      return check_launch(name);
    }
  }
  gemv16_kernel<T, EPI, ACT, NORM, MAXW>
      <<<dim3((unsigned)blocks), dim3((unsigned)(nw * 64)), lds, st>>>(a, tiles);
  return check_launch(name);
}

template <typename T, int EPI, int ACT>
static int launch_gemv_n(const GemvArgs &a, hipStream_t st, const char *name) {
  if (a.norm_w) return launch_gemv<T, EPI, ACT, true>(a, st, name);
  return launch_gemv<T, EPI, ACT, false>(a, st, name);
}

static int gemv_args(const char *name, const void *x, const void *W, int64_t B, int64_t N,
                     int64_t K, int64_t ldx) {
  if (!x || !W) return set_error(TPP_E_INVALID, "%s: null pointer", name);
  if (B < 1 || N < 1 || K < 1)
    return set_error(TPP_E_INVALID, "%s: invalid shapes (B=%lld N=%lld K=%lld)", name,
                     (long long)B, (long long)N, (long long)K);
  if (B > 16) return set_error(TPP_E_UNSUPPORTED, "%s: batch %lld > 16, use tpp_linear_act",
                               name, (long long)B);
  if (ldx < K) return set_error(TPP_E_INVALID, "%s: ldx < K", name);
  return TPP_OK;
}

static GemvArgs make_gemv(const void *x, int64_t ldx, int64_t B, const void *norm_w, float eps,
                          const void *W, int64_t N, int64_t K, void *y, int64_t ldy) {
  GemvArgs a{};
  a.x = x;
  a.ldx = ldx;
  a.NB = (int)B;
  a.norm_w = norm_w;
  a.eps = eps;
  a.W = W;
  a.N = N;
  a.K = K;
  a.y = y;
  a.ldy = ldy;
  return a;
}

} // namespace tpp

using namespace tpp;

extern "C" int tpp_gemv(const void *x, const void *W, const void *bias, void *y, int64_t B,
                        int64_t N, int64_t K, int64_t ldx, int64_t ldy, int act, int dtype,
                        void *stream) {
  const char *name = "tpp_gemv";
  if (int e = gemv_args(name, x, W, B, N, K, ldx)) return e;
  if (!y) return set_error(TPP_E_INVALID, "%s: null output", name);
  if (ldy < N) return set_error(TPP_E_INVALID, "%s: ldy < N", name);
  if (act < TPP_ACT_NONE || act > TPP_ACT_RELU)
    return set_error(TPP_E_INVALID, "%s: unknown activation %d", name, act);
  GemvArgs a = make_gemv(x, ldx, B, nullptr, 0.f, W, N, K, y, ldy);
  a.bias = bias;
  hipStream_t st = as_stream(stream);
  return TPP_DISPATCH_HALF(dtype, [&] {
    if (!bias && act == TPP_ACT_NONE) return launch_gemv_n<T, kEpiPlain, TPP_ACT_NONE>(a, st, name);
    switch (act) {
    case TPP_ACT_GELU_TANH: return launch_gemv_n<T, kEpiBiasAct, TPP_ACT_GELU_TANH>(a, st, name);
    case TPP_ACT_SILU: return launch_gemv_n<T, kEpiBiasAct, TPP_ACT_SILU>(a, st, name);
    case TPP_ACT_RELU: return launch_gemv_n<T, kEpiBiasAct, TPP_ACT_RELU>(a, st, name);
    default: return launch_gemv_n<T, kEpiBiasAct, TPP_ACT_NONE>(a, st, name);
    }
  });
}

extern "C" int tpp_gemv_fused(const void *x, const void *norm_w, float eps, const void *W,
                              void *y, void *residual, int64_t B, int64_t N, int64_t K,
                              int swiglu, int dtype, void *stream) {
  const char *name = "tpp_gemv_fused";
  if (int e = gemv_args(name, x, W, B, N, K, K)) return e;
  if (swiglu && (N % 64 != 0))
    return set_error(TPP_E_UNSUPPORTED, "%s: SwiGLU weight rows must be a multiple of 64", name);
  if (swiglu && residual)
    return set_error(TPP_E_INVALID, "%s: SwiGLU output cannot be added to a residual", name);
  if (!residual && !y) return set_error(TPP_E_INVALID, "%s: no output", name);
  const int64_t ldy = swiglu ? N / 2 : N;
  GemvArgs a = make_gemv(x, K, B, norm_w, eps, W, N, K, y, ldy);
  a.residual = residual;
  hipStream_t st = as_stream(stream);
  return TPP_DISPATCH_HALF(dtype, [&] {
    if (swiglu) return launch_gemv_n<T, kEpiSwiGLU, TPP_ACT_NONE>(a, st, name);
    if (residual) return launch_gemv_n<T, kEpiResidual, TPP_ACT_NONE>(a, st, name);
    return launch_gemv_n<T, kEpiPlain, TPP_ACT_NONE>(a, st, name);
  });
}

extern "C" size_t tpp_gemv_argmax_workspace_size(int64_t B, int64_t N) {
  const int64_t tiles = (N + 15) / 16;
  return (size_t)(tiles < kGemvMaxBlocks ? tiles : kGemvMaxBlocks) * (size_t)B * 8;
}

static int gemv_argmax_launch(const char *name, const void *x, const void *norm_w, float eps,
                              const void *W, void *logits, int64_t B, int64_t N, int64_t K,
                              int dtype, void *workspace, size_t ws_bytes, hipStream_t st,
                              GemvArgs &a, int &nparts) {
  if (int e = gemv_args(name, x, W, B, N, K, K)) return e;
  if (N > 0x7fffffffLL) return set_error(TPP_E_UNSUPPORTED, "%s: N too large", name);
  const int64_t tiles = (N + 15) / 16;
  nparts = (int)(tiles < kGemvMaxBlocks ? tiles : kGemvMaxBlocks);
  if (tiles >= kWideMinTiles && K <= 1024 && K % 256 == 0) nparts = kWideBlocks;
  const size_t need = tpp_gemv_argmax_workspace_size(B, N);
  if (!workspace || ws_bytes < need || !aligned16(workspace))
    return set_error(TPP_E_WORKSPACE, "%s: workspace of %zu bytes required", name, need);
  a = make_gemv(x, K, B, norm_w, eps, W, N, K, logits, N);
  a.am_val = (float *)workspace;
  a.am_idx = (int *)((char *)workspace + (size_t)nparts * B * 4);
  if (!gemv_vec_ok(a)) return set_error(TPP_E_UNSUPPORTED, "%s: needs K %% 8 == 0 and 16-byte alignment", name);
  return TPP_DISPATCH_HALF(dtype, [&] {
    return launch_gemv_n<T, kEpiPlain, TPP_ACT_NONE>(a, st, name);
  });
}

extern "C" int tpp_gemv_argmax(const void *x, const void *norm_w, float eps, const void *W,
                               void *logits, int64_t *out_idx, int64_t B, int64_t N, int64_t K,
                               int dtype, void *workspace, size_t ws_bytes, void *stream) {
  const char *name = "tpp_gemv_argmax";
  if (!out_idx) return set_error(TPP_E_INVALID, "%s: null index output", name);
  hipStream_t st = as_stream(stream);
  GemvArgs a;
  int nparts = 0;
  if (int e = gemv_argmax_launch(name, x, norm_w, eps, W, logits, B, N, K, dtype, workspace,
                                 ws_bytes, st, a, nparts))
    return e;
  argmax_partials_kernel<<<dim3((unsigned)B), dim3(1024), 0, st>>>(a.am_val, a.am_idx, nparts,
                                                                   (int)B, out_idx);
  return check_launch(name);
}

extern "C" int tpp_greedy_step(const void *x, const void *norm_w, float eps, const void *W,
                               const void *emb, int64_t *ids, void *resid_next,
                               int32_t *positions, int32_t *seqlens, int64_t B, int64_t N,
                               int64_t K, int dtype, void *workspace, size_t ws_bytes,
                               void *stream) {
  const char *name = "tpp_greedy_step";
  if (!emb || !ids || !resid_next) return set_error(TPP_E_INVALID, "%s: null pointer", name);
  hipStream_t st = as_stream(stream);
  GemvArgs a;
  int nparts = 0;
  if (int e = gemv_argmax_launch(name, x, norm_w, eps, W, nullptr, B, N, K, dtype, workspace,
                                 ws_bytes, st, a, nparts))
    return e;
  return TPP_DISPATCH_HALF(dtype, [&] {
    greedy_advance_kernel<T><<<dim3((unsigned)B), dim3(1024), 0, st>>>(
        a.am_val, a.am_idx, nparts, (int)B, (const T *)emb, K, ids, (T *)resid_next, positions,
        seqlens);
    return check_launch(name);
  });
}
