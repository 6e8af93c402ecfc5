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

// LDS tiles hold 128-byte rows of eight 16-byte chunks; chunk c of row r is
// stored at position c ^ swz(r). A ds_read_b128 serves 16 lanes (16 rows of
// one fragment) per cycle from 16 distinct 16-byte bank groups only if those
// rows land in different groups: rows r and r+1 already differ in the row's
// half of the 256-byte bank space, so the XOR uses row bits 1..3 (bits 0..2
// would put rows r and r+8 on the same banks: a 2-way conflict on every read).
__device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }

// K-tile depth and ring stages of the 256x256 tile (64 KB per stage at BK 64;
// 4- and 5-stage rings of BK 32 tiles measured slower)
#ifndef TPP_BIG_BK
#define TPP_BIG_BK 64
#define TPP_BIG_NST 2
#endif
constexpr int kBigBK = TPP_BIG_BK, kBigNST = TPP_BIG_NST;
// the same for the 128-row tiles: BK 64, as many stages as fit 160 KB of LDS
// (one block per CU): 5 for 128x128, 4 for 128x192, 3 for 128x256 (at the
// Linear+act shape 3 stages were 6% faster than 2, and 4 another 3%)
constexpr int kSmallBK = 64;
// below this many outputs the register-staged kernel's smaller LDS footprint
// (several blocks per CU) wins over the deeper DMA ring
constexpr int64_t kDmaMinMN = 256 * 128 * 128;
// the DMA kernel addresses a tile's rows by 32-bit byte offsets from its
// first row: 256 rows * ld * 2 bytes stays below 2^32 up to this pitch
constexpr int64_t kDmaMaxLd = 1 << 22;

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
      sA[buf][row * 8 + (kc ^ swz(row))] = ra[i];
      sB[buf][row * 8 + (kc ^ swz(row))] = rb[i];
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
        af[i] = sA[buf][row * 8 + (kc ^ swz(row))];
        const int col = wn * 64 + i * 32 + (lane & 31);
        bfr[i] = sB[buf][col * 8 + (kc ^ swz(col))];
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

// ---------------------------------------------------------------------------
// Pipelined variant for K % 64 == 0: operands go HBM/L2 -> LDS directly with
// global_load_lds_dwordx4 (no VGPR staging, no ds_write), through an
// NST-stage ring (NST-1 K tiles in flight while one is multiplied). Block
// tile (32*WM*FM) x (32*WN*FN), WM x WN waves, wave tile (32*FM) x (32*FN).
// Why big tiles: the CU's L1 delivers ~64 B/clk while its four matrix cores
// consume 4096 bf16 flop/clk, so a BM x BN tile needs (BM+BN)/(BM*BN) <=
// 1/64 byte per flop; 128x128 sits exactly at that limit, 256x256 at half.
// Measured on MI355X: 256x256 with 8 waves (4x2 of 64x128, two per SIMD)
// runs ~37-43% of MFMA peak on the prefill shapes vs ~31% for 128x128; with
// fewer tiles than CUs the 128-row tiles (two blocks per CU with a 2-stage
// ring) win.
// An LDS-DMA instruction writes lane i's 16 bytes at base + 16*i; lane i of
// a row group therefore fetches the 16-byte chunk kc = (i%8) ^ swz(row), which
// lands the tile in the same XOR-swizzled layout the fragment reads expect.
// Waits are explicit (s_waitcnt vmcnt / lgkmcnt + s_barrier): a fenced
// __syncthreads() would drain every DMA in flight at each K step.
template <int N> __device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt(0xC07F); }
// Wait until at most min(later, R) K tiles' DMA (NQ instructions each, this
// wave's share) are outstanding: the ring's DMA completes in issue order, so
// every older tile has landed.
template <int NQ, int R> __device__ __forceinline__ void wait_tiles(int later) {
  if constexpr (R <= 0) {
    wait_vmcnt<0>();
  } else {
    if (later >= R) wait_vmcnt<R * NQ>();
    else wait_tiles<NQ, R - 1>(later);
  }
}

template <int BK> __device__ __forceinline__ int swzk(int row) {
  // BK = 64: 128-byte rows, two per 256-byte bank space; BK = 32: 64-byte rows,
  // four per bank space. The XOR uses the row bits above those, so the 16
  // rows one ds_read_b128 cycle serves hit 16 distinct 16-byte bank groups.
  if constexpr (BK == 64) return (row >> 1) & 7;
  else return (row >> 2) & 3;
}

// x[e] <- float(T(x[e])) for four values, converted two at a time (one
// packed conversion per pair instead of one per value)
template <typename T> __device__ __forceinline__ void round_pairs(float (&x)[4]) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef typename VecT<T>::v2 T2;
#pragma unroll
  for (int p = 0; p < 4; p += 2) {
    const f2 in = {x[p], x[p + 1]};
    const f2 out = __builtin_convertvector(__builtin_convertvector(in, T2), f2);
    x[p] = out[0];
    x[p + 1] = out[1];
  }
}

template <typename T, int EPI, int ACT, int FM, int FN, int NST, int WM, int WN, int BK>
__global__ __launch_bounds__(64 * WM * WN) void gemm_dma_kernel(
    const T *__restrict__ A, int64_t lda, const T *__restrict__ B, int64_t ldb,
    T *__restrict__ C, int64_t ldc, const T *__restrict__ bias, int M, int N, int K) {
  typedef typename VecT<T>::v8 V8;
  constexpr int BM = 32 * WM * FM, BN = 32 * WN * FN, NWV = WM * WN;
  constexpr int CPR = BK / 8;                // 16-byte chunks per tile row
  constexpr int RPI = 64 / CPR;              // tile rows per DMA instruction
  constexpr int STG = (BM + BN) * CPR;       // 16-byte slots per stage
  constexpr int NA = BM / RPI / NWV, NB = BN / RPI / NWV; // DMA instructions per wave per stage
  static_assert(NA * RPI * NWV == BM && NB * RPI * NWV == BN, "tile rows per wave");
  // the epilogue's staging tile reuses the ring
  constexpr int OWS = (EPI == kGSwiGLU) ? FN * 16 : FN * 32;
  constexpr int RING = NST * STG, OUTS = NWV * FM * 32 * (OWS + 8) * (int)sizeof(T) / 16;
  __shared__ V8 smem[RING > OUTS ? RING : OUTS];

  const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN;
  int tm, tn;
  tile_coords(blockIdx.x, ntm * ntn, ntm, ntn, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wm = w / WN, wn = w % WN;

  // DMA instruction j of wave w covers tile rows (NWV*j + w)*RPI .. +RPI-1;
  // lane i fetches row +i/CPR, chunk (i%CPR)^swzk(row). swzk(row) depends on
  // w and i only (NWV is even). Source rows are clamped to the matrix: rows
  // past M / N only feed outputs that are never stored.
  const int lrow = lane / CPR, lkc = (lane % CPR) ^ swzk<BK>(RPI * w + lrow);
  // DMA sources: a uniform tile base (row m0 of A, row n0 of B, in scalar
  // registers) plus per-lane 32-bit byte offsets of the lane's clamped rows
  // relative to it, fixed for the whole K loop (the host keeps
  // BM * ld * sizeof(T) below 2^32)
  constexpr int NQ = NA + NB;
  const char *ta = reinterpret_cast<const char *>(A) + (int64_t)m0 * lda * (int64_t)sizeof(T);
  const char *tb = reinterpret_cast<const char *>(B) + (int64_t)n0 * ldb * (int64_t)sizeof(T);
  uint32_t off[NQ];
#pragma unroll
  for (int q = 0; q < NA; ++q)
    off[q] = (uint32_t)((int64_t)(min(m0 + w * RPI + lrow + RPI * NWV * q, M - 1) - m0) * lda + lkc * 8) *
             (uint32_t)sizeof(T);
#pragma unroll
  for (int q = 0; q < NB; ++q)
    off[NA + q] = (uint32_t)((int64_t)(min(n0 + w * RPI + lrow + RPI * NWV * q, N - 1) - n0) * ldb + lkc * 8) *
                  (uint32_t)sizeof(T);
  // DMA instruction q (0 .. NQ - 1) of K tile kt into a stage
  auto issue_one = [&](int stage, int kt, int q) {
    V8 *sa = smem + stage * STG, *sb = sa + BM * CPR;
    const int64_t kb = (int64_t)kt * BK * sizeof(T);
    if (q < NA)
      __builtin_amdgcn_global_load_lds((const void *)(ta + kb + off[q]),
                                       (__attribute__((address_space(3))) void *)(sa + (q * NWV + w) * 64),
                                       16, 0, 0);
    else
      __builtin_amdgcn_global_load_lds((const void *)(tb + kb + off[q]),
                                       (__attribute__((address_space(3))) void *)(sb + ((q - NA) * NWV + w) * 64),
                                       16, 0, 0);
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

  // The bias is added by one more MFMA per accumulator block after the K
  // loop: A' = the bias of the block's 32 W rows in K column 0, B' = ones in
  // K row 0, so acc += bias[n] . 1 with one fp32 rounding, the add of the
  // epilogue formula, with no VALU work per output. Lane l < 32 holds
  // bias[nw0 + 32 j + l] in element 0 of fragment j (requested now, so its
  // latency hides under the main loop); every other element is zero.
  const int nw0 = n0 + wn * FN * 32; // first W row (output column before SwiGLU) of the wave
  V8 bfrag[EPI == kGBiasAct ? FN : 1];
  if constexpr (EPI == kGBiasAct) {
    if (bias) { // uniform
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int c = nw0 + j * 32 + (lane & 31);
        const T bv = bias[c < N ? c : N - 1];
#pragma unroll
        for (int e = 0; e < 8; ++e) bfrag[j][e] = (T)0.0f;
        bfrag[j][0] = (lane < 32 && c < N) ? bv : (T)0.0f;
      }
    }
  }

  // Main loop. Each K tile is KS = BK/16 sub-steps of FM x FN MFMAs, with
  // the operand fragments of sub-step ks + 1 read (into the other register
  // set) while the MFMAs of ks run. The DMA of K tile kt + NST - 1 goes into
  // the slot every wave finished reading before the last barrier and is
  // spread between the MFMAs of the first half of the tile, so no wave
  // stalls on a burst of DMA issue. The wait for K tile kt + 1's DMA and the
  // barrier that publishes it sit in the middle of the last sub-step, right
  // before the next tile's first fragment reads: the second half of the
  // sub-step's MFMAs is still to issue while the barrier resolves and those
  // reads return (measured 3-4% faster on the prefill shapes than a barrier
  // at the top of each K tile).
  constexpr int KS = BK / 16;
  static_assert(KS % 2 == 0, "register sets alternate across the K-tile boundary");
  constexpr int NMF = KS * FM * FN;
  constexpr int MID = NMF - (FM * FN) / 2; // MFMAs of a K tile issued before its barrier
  constexpr int SP = (NMF / 2) / NQ > 0 ? (NMF / 2) / NQ : 1; // MFMAs per DMA instruction
  static_assert(NQ * SP <= MID, "all DMA of a K tile issued before its barrier");
  const int nk = K / BK;
#pragma unroll
  for (int p = 0; p < NST - 1; ++p)
    if (p < nk)
#pragma unroll
      for (int q = 0; q < NQ; ++q) issue_one(p, p, q);
  // K tile 0 landed (tiles 1 .. NST-2 may be in flight)
  wait_tiles<NQ, NST - 2>(nk - 1);
  __builtin_amdgcn_s_barrier();
  V8 af[2][FM], bfr[2][FN];
  auto frag = [&](const V8 *sa, int ks) {
    const V8 *sb = sa + BM * CPR;
    const int kc = ks * 2 + (lane >> 5);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int row = wm * FM * 32 + i * 32 + (lane & 31);
      af[ks & 1][i] = sa[row * CPR + (kc ^ swzk<BK>(row))];
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = wn * FN * 32 + j * 32 + (lane & 31);
      bfr[ks & 1][j] = sb[col * CPR + (kc ^ swzk<BK>(col))];
    }
  };
  frag(smem, 0);
  for (int kt = 0; kt < nk; ++kt) {
    const V8 *sa = smem + (kt % NST) * STG;
    const int kn = kt + NST - 1;
    const bool more = kn < nk, next = kt + 1 < nk;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if (ks + 1 < KS) frag(sa, ks + 1);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          acc[i][j] = mfma32<T>(bfr[ks & 1][j], af[ks & 1][i], acc[i][j]);
          const int m = (ks * FM + i) * FN + j + 1;
          if (m % SP == 0 && m / SP <= NQ && more) issue_one(kn % NST, kn, m / SP - 1);
          if (m == MID && next) {
            // own DMA of K tile kt + 1 landed (tiles kt + 2 .. kt + NST - 1
            // may still be in flight). The fragment reads of tile kt must
            // all have returned before the barrier, since after it any wave
            // may refill that slot: with one row block per wave (FM = 1) the
            // fragments of the second half of this sub-step are not consumed
            // yet, so wait for every LDS read (lgkmcnt(0); the barrier does
            // not wait for them)
            wait_tiles<NQ, NST - 2>(nk - kt - 2);
            wait_lgkmcnt0();
            __builtin_amdgcn_s_barrier();
            frag(smem + ((kt + 1) % NST) * STG, 0);
          }
        }
    }
  }

  if constexpr (EPI == kGBiasAct) {
    if (bias) {
      V8 ones;
#pragma unroll
      for (int e = 0; e < 8; ++e) ones[e] = (T)0.0f;
      ones[0] = lane < 32 ? (T)1.0f : (T)0.0f;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma32<T>(bfrag[j], ones, acc[i][j]);
    }
  }

  // Epilogue. The operands are swapped in the MFMA (W rows first), so the
  // 32x32 accumulator holds lane -> output row m = i*32 + (lane & 31) and
  // registers 4q..4q+3 -> four consecutive output columns
  // n = j*32 + q*8 + (lane/32)*4 + {0..3}. Each wave converts its 32FM x 32FN
  // tile, packs 4 columns per 8-byte LDS write into a padded row-major
  // staging tile (the ring is free by now), then stores whole rows with
  // 16-byte global writes.
  constexpr int OW = (EPI == kGSwiGLU) ? FN * 16 : FN * 32; // output cols per wave
  constexpr int LDR = OW + 8; // staging row pitch in elements (16-byte aligned rows)
  wait_lgkmcnt0();
  __builtin_amdgcn_s_barrier(); // every wave is done reading the ring
  T *stage = reinterpret_cast<T *>(smem) + w * (FM * 32 * LDR);
  const int half = lane >> 5, ml = lane & 31;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    if constexpr (EPI == kGSwiGLU) {
      if (j & 1) continue;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int nl = j * 32 + q * 8 + half * 4; // wave-local W column of register 4q
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        typename VecT<T>::v4 pk;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * q + e];
        if constexpr (EPI == kGSwiGLU) {
          float u[4], sl[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) u[e] = acc[i][j + 1][4 * q + e];
          round_pairs<T>(v);
          round_pairs<T>(u);
#pragma unroll
          for (int e = 0; e < 4; ++e) sl[e] = act_silu(v[e]);
          round_pairs<T>(sl);
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = sl[e] * u[e];
        } else if constexpr (EPI == kGBiasAct) {
          round_pairs<T>(v); // the pre-activation rounded to T (bias already in acc)
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = apply_act<ACT>(v[e]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) pk[e] = from_f32<T>(v[e]);
        const int col = (EPI == kGSwiGLU) ? (j / 2) * 32 + q * 8 + half * 4 : nl;
        *reinterpret_cast<typename VecT<T>::v4 *>(stage + (i * 32 + ml) * LDR + col) = pk;
      }
    }
  }
  wait_lgkmcnt0();
  // rows of the wave tile: OW/8 lanes per row, 16 bytes each; RPI rows per
  // pass (with OW = 96, lanes 60..63 idle)
  constexpr int LPR = OW / 8, OPR = 64 / LPR; // output rows per pass
  const int oc0 = (EPI == kGSwiGLU) ? nw0 / 2 : nw0;
  const int NO = (EPI == kGSwiGLU) ? N / 2 : N;
  const int rr = lane / LPR, cc = (lane % LPR) * 8;
  const bool vec_ok = (ldc % 8 == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
#pragma unroll
  for (int r0 = 0; r0 < FM * 32; r0 += OPR) {
    const int rl = r0 + rr;
    if (rr >= OPR || rl >= FM * 32) continue;
    const int row = m0 + wm * FM * 32 + rl;
    const typename VecT<T>::v8 v =
        *reinterpret_cast<const typename VecT<T>::v8 *>(stage + rl * LDR + cc);
    if (row >= M) continue;
    const int col = oc0 + cc;
    T *dst = C + (int64_t)row * ldc + col;
    if (vec_ok && col + 8 <= NO) {
      *reinterpret_cast<typename VecT<T>::v8 *>(dst) = v;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (col + e < NO) dst[e] = v[e];
    }
  }
}

// ---------------------------------------------------------------------------
// Persistent 256x256 variant for launches with more tiles than CUs (the
// prefill projections: 4-6 tiles per CU). One workgroup per CU loops over the
// tiles b, b + gridDim, ... (all on the workgroup's XCD: gridDim is a
// multiple of 8, and tile_coords keeps an XCD's tiles a compact group). The
// K steps of consecutive tiles form one stream through the 2-stage ring: the
// last K step of a tile issues the DMA of the next tile's first K step, and
// the epilogue, staged through the slot that K step has just finished
// reading (64 KB: 8 KB per wave, two passes), issues the next tile's second
// K step before its global stores, so neither the first DMA of a tile nor the
// store drain sits on the critical path. Measured on the prefill shapes:
// 3-7% faster than one workgroup per tile. Plain and SwiGLU epilogues only
// (a bias prefetch for the next tile does not fit the registers).
template <typename T, int EPI, int ACT>
__global__ __launch_bounds__(512) void gemm_persist_kernel(
    const T *__restrict__ A, int64_t lda, const T *__restrict__ B, int64_t ldb,
    T *__restrict__ C, int64_t ldc, const T *__restrict__ bias, int M, int N, int K) {
  typedef typename VecT<T>::v8 V8;
  typedef typename VecT<T>::v4 V4;
  static_assert(EPI == kGPlain || EPI == kGSwiGLU, "plain or SwiGLU epilogue");
  constexpr int FM = 2, FN = 4, WM = 4, WN = 2, BK = 64, NST = 2;
  constexpr int BM = 32 * WM * FM, BN = 32 * WN * FN, NWV = WM * WN;
  constexpr int CPR = BK / 8, RPI = 64 / CPR;
  constexpr int STG = (BM + BN) * CPR;
  constexpr int NA = BM / RPI / NWV, NB = BN / RPI / NWV, NQ = NA + NB;
  constexpr int KS = BK / 16, NMF = KS * FM * FN, MID = NMF - (FM * FN) / 2;
  constexpr int SP = (NMF / 2) / NQ > 0 ? (NMF / 2) / NQ : 1;
  static_assert(NQ * SP <= MID, "all DMA of a K step issued before its barrier");
  // epilogue staging per wave and pass: 64 rows x OWP output columns, read
  // back in NR rounds of 16 bytes per lane (NSTO global stores per wave)
  constexpr int OWP = (EPI == kGSwiGLU) ? 32 : 64;
  constexpr int RB = OWP * (int)sizeof(T), LPR = RB / 16, OPR = 64 / LPR;
  constexpr int NR = FM * 32 / OPR, NSTO = 2 * NR;
  static_assert(NWV * FM * 32 * RB <= STG * 16, "staging fits one ring slot");
  __shared__ V8 smem[NST * STG];

  const int ntm = (M + BM - 1) / BM, ntn = (N + BN - 1) / BN, ntiles = ntm * ntn;
  // wave index in a scalar register: every per-wave decision (DMA rows,
  // store path, wait counts) is then provably uniform
  const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = w / WN, wn = w % WN;
  const int half = lane >> 5, ml = lane & 31;
  const int lrow = lane / CPR, lkc = (lane % CPR) ^ swzk<BK>(RPI * w + lrow);
  const int nk = K / BK;
  int tile = blockIdx.x;
  if (tile >= ntiles) return;

  // DMA sources of a tile: uniform tile bases plus per-lane 32-bit offsets of
  // the lane's clamped rows (the host keeps BM * ld * sizeof(T) below 2^32)
  struct Src {
    const char *ta, *tb;
    uint32_t off[NQ];
    int m0, n0;
  };
  auto src_of = [&](int t, Src &s) {
    int tm, tn;
    tile_coords(t, ntiles, ntm, ntn, tm, tn);
    s.m0 = tm * BM;
    s.n0 = tn * BN;
    s.ta = reinterpret_cast<const char *>(A) + (int64_t)s.m0 * lda * (int64_t)sizeof(T);
    s.tb = reinterpret_cast<const char *>(B) + (int64_t)s.n0 * ldb * (int64_t)sizeof(T);
#pragma unroll
    for (int q = 0; q < NA; ++q)
      s.off[q] = (uint32_t)((int64_t)(min(s.m0 + w * RPI + lrow + RPI * NWV * q, M - 1) - s.m0) * lda +
                            lkc * 8) * (uint32_t)sizeof(T);
#pragma unroll
    for (int q = 0; q < NB; ++q)
      s.off[NA + q] = (uint32_t)((int64_t)(min(s.n0 + w * RPI + lrow + RPI * NWV * q, N - 1) - s.n0) * ldb +
                                 lkc * 8) * (uint32_t)sizeof(T);
  };
  auto issue = [&](const Src &s, int stage, int kt, int q) {
    V8 *sa = smem + stage * STG, *sb = sa + BM * CPR;
    const int64_t kb = (int64_t)kt * BK * sizeof(T);
    if (q < NA)
      __builtin_amdgcn_global_load_lds((const void *)(s.ta + kb + s.off[q]),
                                       (__attribute__((address_space(3))) void *)(sa + (q * NWV + w) * 64),
                                       16, 0, 0);
    else
      __builtin_amdgcn_global_load_lds((const void *)(s.tb + kb + s.off[q]),
                                       (__attribute__((address_space(3))) void *)(sb + ((q - NA) * NWV + w) * 64),
                                       16, 0, 0);
  };
  V8 af[2][FM], bfr[2][FN];
  auto frag = [&](const V8 *sa, int ks) {
    const V8 *sb = sa + BM * CPR;
    const int kc = ks * 2 + (lane >> 5);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int row = wm * FM * 32 + i * 32 + (lane & 31);
      af[ks & 1][i] = sa[row * CPR + (kc ^ swzk<BK>(row))];
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = wn * FN * 32 + j * 32 + (lane & 31);
      bfr[ks & 1][j] = sb[col * CPR + (kc ^ swzk<BK>(col))];
    }
  };

  Src cur, nxt;
  src_of(tile, cur);
#pragma unroll
  for (int q = 0; q < NQ; ++q) issue(cur, 0, 0, q);
  wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();
  frag(smem, 0);
  int slot = 0;
  // K step 1 of the current tile already in flight (issued in the previous
  // tile's epilogue), with `sto` store instructions of that epilogue issued
  // after it (-1: an unknown number)
  bool pre = false;
  int sto = -1;
  for (;;) {
    const int tnext = tile + (int)gridDim.x;
    const bool has_next = tnext < ntiles;
    if (has_next) src_of(tnext, nxt);
    const int nw0 = cur.n0 + wn * FN * 32; // first W row (output column before SwiGLU) of the wave
    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // K loop: step kt reads slot `slot`; its DMA fills the other slot with
    // K step kt + 1, or with the next tile's first K step after the last
    for (int kt = 0; kt < nk; ++kt) {
      const V8 *sa = smem + slot * STG;
      const bool last = kt + 1 == nk;
      const bool more = !last || has_next;
      const bool early = kt == 0 && pre; // this step's DMA was issued early
      const bool dma = more && !early;
      const Src &ds = last ? nxt : cur;
      const int kd = last ? 0 : kt + 1;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks + 1 < KS) frag(sa, ks + 1);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) {
            acc[i][j] = mfma32<T>(bfr[ks & 1][j], af[ks & 1][i], acc[i][j]);
            const int m = (ks * FM + i) * FN + j + 1;
            if (m % SP == 0 && m / SP <= NQ && dma) issue(ds, slot ^ 1, kd, m / SP - 1);
            if (m == MID && more) {
              // the other slot's DMA landed; this slot's fragment reads all
              // returned (lgkmcnt(0): the slot is refilled after the
              // barrier). Vector memory operations complete in issue order,
              // so behind an early DMA only the epilogue stores issued after
              // it may stay in flight.
              if (early && sto == NSTO) wait_vmcnt<NSTO>();
              else wait_vmcnt<0>();
              wait_lgkmcnt0();
              __builtin_amdgcn_s_barrier();
              frag(smem + (slot ^ 1) * STG, 0);
            }
          }
      }
      slot ^= 1;
    }

    // Epilogue through the slot the last K step read (slot ^ 1 now), which
    // every wave has finished with after this barrier; the next tile's first
    // K step is in the other slot (its first fragments already requested).
    // The output is converted, staged (per wave, two passes of OWP columns)
    // and read back into registers; then the next tile's second K step is
    // issued into the staging slot ahead of the global stores, so the stores
    // drain under the next tile's first K step.
    wait_lgkmcnt0();
    __builtin_amdgcn_s_barrier();
    T *stage = reinterpret_cast<T *>(smem + (slot ^ 1) * STG) + w * (FM * 32 * OWP);
    auto sw = [](int row) { return (RB == 128) ? (row >> 1) & 7 : (row >> 2) & 3; };
    const int NO = (EPI == kGSwiGLU) ? N / 2 : N;
    const int oc0 = (EPI == kGSwiGLU) ? nw0 / 2 : nw0;
    V8 ov[2][NR];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const int j = 2 * p + jj;
        if constexpr (EPI == kGSwiGLU) {
          if (jj == 1) continue;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
#pragma unroll
          for (int i = 0; i < FM; ++i) {
            V4 pk;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * q + e];
            if constexpr (EPI == kGSwiGLU) {
              float u[4], sl[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) u[e] = acc[i][j + 1][4 * q + e];
              round_pairs<T>(v);
              round_pairs<T>(u);
#pragma unroll
              for (int e = 0; e < 4; ++e) sl[e] = act_silu(v[e]);
              round_pairs<T>(sl);
#pragma unroll
              for (int e = 0; e < 4; ++e) v[e] = sl[e] * u[e];
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) pk[e] = from_f32<T>(v[e]);
            const int row = i * 32 + ml;
            const int col = ((EPI == kGSwiGLU) ? 0 : jj * 32) + q * 8 + half * 4; // column in the pass
            const int byte = row * RB + (((col * (int)sizeof(T)) / 16) ^ sw(row)) * 16 +
                             (col * (int)sizeof(T)) % 16;
            *reinterpret_cast<V4 *>(reinterpret_cast<char *>(stage) + byte) = pk;
          }
        }
      }
      wait_lgkmcnt0(); // this wave's staging rows written (the staging is per wave)
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int rl = r * OPR + lane / LPR, ch = lane % LPR;
        ov[p][r] = *reinterpret_cast<const V8 *>(reinterpret_cast<const char *>(stage) + rl * RB +
                                                 (ch ^ sw(rl)) * 16);
      }
      wait_lgkmcnt0(); // the staging reads returned before the next pass overwrites it
    }
    // every wave is done with the staging slot: the next tile's second K step
    // may refill it
    __builtin_amdgcn_s_barrier();
    pre = has_next && nk > 1;
    if (pre) {
#pragma unroll
      for (int q = 0; q < NQ; ++q) issue(nxt, slot ^ 1, 1, q);
    }
    __builtin_amdgcn_sched_barrier(0); // the stores stay behind the DMA
    const int orow0 = cur.m0 + wm * FM * 32;
    const bool vec_ok = (ldc % 8 == 0) && ((reinterpret_cast<uintptr_t>(C) & 15) == 0);
    // whole wave tile inside the output: one 16-byte store per readback round
    const bool full = vec_ok && orow0 + FM * 32 <= M && oc0 + 2 * OWP <= NO;
    if (full) {
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const int rl = r * OPR + lane / LPR, ch = lane % LPR;
          *reinterpret_cast<V8 *>(C + (int64_t)(orow0 + rl) * ldc + oc0 + p * OWP + ch * 8) = ov[p][r];
        }
    } else {
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const int rl = r * OPR + lane / LPR, ch = lane % LPR;
          const int row = orow0 + rl;
          const int col = oc0 + p * OWP + ch * 8;
          if (row >= M) continue;
          T *dst = C + (int64_t)row * ldc + col;
          if (vec_ok && col + 8 <= NO) {
            *reinterpret_cast<V8 *>(dst) = ov[p][r];
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (col + e < NO) dst[e] = ov[p][r][e];
          }
        }
    }
    sto = full ? NSTO : -1;
    if (!has_next) break;
    tile = tnext;
    cur = nxt;
  }
}

// Tile shape for the DMA kernel: minimise (tiles per CU, rounded up) x tile
// area / relative efficiency (one block per CU for every candidate). SwiGLU
// needs whole [gate|up] 64-column pairs per wave (FN even).
static int pick_dma_tile(int64_t M, int64_t N, bool swiglu, int cus) {
  struct Cand { int bm, bn, fn_wave; double eff; };
  // 128x128 / 128x192 / 128x256: 8 waves (4x2) of 32x64 / 32x96 / 32x128, so
  // two waves share each SIMD even at one block per CU (measured 7% faster
  // than 4 waves of 64-row strips at the BASELINE Linear+act shape);
  // 256x256: 8 waves (4x2) of 64x128
  const Cand cands[] = {{128, 128, 2, 0.95}, {128, 192, 3, 1.0}, {128, 256, 4, 1.0},
                        {256, 256, 4, 1.25}};
  int best = -1;
  double best_t = 0.0;
  for (int c = 0; c < 4; ++c) {
    if (swiglu && (cands[c].fn_wave & 1)) continue;
    const int64_t bm = cands[c].bm, bn = cands[c].bn;
    const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    const int64_t per_cu = (tiles + cus - 1) / cus;
    const double t = (double)per_cu * (double)(bm * bn) / cands[c].eff;
    if (best < 0 || t < best_t) best = c, best_t = t;
  }
  return best;
}

static int device_cus() {
  const int n = device_cu_count();
  return n > 0 ? n : 256;
}

template <typename T, int EPI, int ACT, int FM, int FN, int WM, int WN, int BK, int NST>
static void launch_dma(const void *A, int64_t lda, const void *B, int64_t ldb, void *C,
                       int64_t ldc, const void *bias, int64_t M, int64_t N, int64_t K,
                       hipStream_t st) {
  constexpr int BM = 32 * WM * FM, BN = 32 * WN * FN;
  const int64_t nb = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  gemm_dma_kernel<T, EPI, ACT, FM, FN, NST, WM, WN, BK><<<dim3((unsigned)nb), dim3(64 * WM * WN), 0, st>>>(
      (const T *)A, lda, (const T *)B, ldb, (T *)C, ldc, (const T *)bias, (int)M, (int)N, (int)K);
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

// hipBLASLt for plain GEMMs with at least one 256x256 tile per CU (gemm_lt.hip)
bool lt_gemm_wanted(int64_t M, int64_t N, int cus);
bool lt_gemm(const void *X, int64_t ldx, const void *W, int64_t ldw, void *Y, int64_t ldy,
             int64_t M, int64_t N, int64_t K, bool bf16, hipStream_t st);

template <typename T, int EPI, int ACT>
static int launch_gemm(const void *A, int64_t lda, const void *B, int64_t ldb, void *C,
                       int64_t ldc, const void *bias, int64_t M, int64_t N, int64_t K,
                       hipStream_t st, const char *name) {
  if (M == 0) return TPP_OK;
  const bool vec = (K % 8 == 0) && (lda % 8 == 0) && (ldb % 8 == 0) && aligned16(A) &&
                   aligned16(B);
  if constexpr (EPI == kGPlain) {
    if (vec && lt_gemm_wanted(M, N, device_cus()) &&
        lt_gemm(A, lda, B, ldb, C, ldc, M, N, K, __is_same(T, bf16), st))
      return check_launch(name);
  }
  if (vec && K % 64 == 0 && M * N >= (int64_t)kDmaMinMN && lda <= kDmaMaxLd && ldb <= kDmaMaxLd) {
    if ((M + 127) / 128 * ((N + 127) / 128) > 0x7fffffffLL)
      return set_error(TPP_E_UNSUPPORTED, "%s: too many tiles", name);
    switch (pick_dma_tile(M, N, EPI == kGSwiGLU, device_cus())) {
    case 0: launch_dma<T, EPI, ACT, 1, 2, 4, 2, kSmallBK, 5>(A, lda, B, ldb, C, ldc, bias, M, N, K, st); break;
    case 1: launch_dma<T, EPI, ACT, 1, 3, 4, 2, kSmallBK, 4>(A, lda, B, ldb, C, ldc, bias, M, N, K, st); break;
    case 2: launch_dma<T, EPI, ACT, 1, 4, 4, 2, kSmallBK, 3>(A, lda, B, ldb, C, ldc, bias, M, N, K, st); break;
    default: {
      // more tiles than CUs: the persistent kernel (plain / SwiGLU epilogue)
      bool done = false;
      if constexpr (EPI != kGBiasAct && kBigBK == 64 && kBigNST == 2) {
        const int cus = device_cus();
        const int64_t nb = ((M + 255) / 256) * ((N + 255) / 256);
        if (cus % 8 == 0 && nb > cus) {
          gemm_persist_kernel<T, EPI, ACT><<<dim3((unsigned)cus), dim3(512), 0, st>>>(
              (const T *)A, lda, (const T *)B, ldb, (T *)C, ldc, (const T *)bias, (int)M, (int)N, (int)K);
          done = true;
        }
      }
      if (!done) launch_dma<T, EPI, ACT, 2, 4, 4, 2, kBigBK, kBigNST>(A, lda, B, ldb, C, ldc, bias, M, N, K, st);
      break;
    }
    }
  } else if (vec) {
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
