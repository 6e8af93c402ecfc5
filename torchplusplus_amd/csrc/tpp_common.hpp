// Shared device/host helpers for the gfx950 kernel set.
//
// Everything here is written for CDNA4 wave64: reductions use DPP row
// operations inside a 16-lane row plus v_readlane across rows, so no LDS
// round-trip is needed for a row that fits in one wave.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <type_traits>
#include <utility>

#include "../../include/tpp.h"

namespace tpp {

typedef _Float16 f16;
typedef __bf16 bf16;

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// ---- element traits --------------------------------------------------------

template <typename T> struct VecT;
template <> struct VecT<f16> {
  typedef f16x8 v8;
  typedef f16x4 v4;
  typedef f16x2 v2;
};
template <> struct VecT<bf16> {
  typedef bf16x8 v8;
  typedef bf16x4 v4;
  typedef bf16x2 v2;
};

// acc + sum_e x[e] w[e] over 8 elements: four v_dot2 instructions (two
// products each, accumulated in fp32) instead of 16 conversions and 8 FMAs
template <typename T>
__device__ __forceinline__ float dot8(const typename VecT<T>::v8 &x, const typename VecT<T>::v8 &w,
                                      float acc) {
  typedef typename VecT<T>::v2 T2;
#pragma unroll
  for (int p = 0; p < 8; p += 2) {
    const T2 a = {x[p], x[p + 1]}, b = {w[p], w[p + 1]};
    if constexpr (__is_same(T, bf16)) acc = __builtin_amdgcn_fdot2_f32_bf16(a, b, acc, false);
    else acc = __builtin_amdgcn_fdot2(a, b, acc, false);
  }
  return acc;
}

__device__ __forceinline__ float to_f32(f16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(float x) { return x; }

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ f16 from_f32<f16>(float x) { return (f16)x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }

// 16-byte vector load/store of 8 elements, converted to/from fp32.
template <typename T>
__device__ __forceinline__ void load8(const T *p, float (&v)[8]) {
  typedef typename VecT<T>::v8 V;
  V t = *reinterpret_cast<const V *>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = to_f32(t[i]);
}
template <typename T>
__device__ __forceinline__ void store8(T *p, const float (&v)[8]) {
  typedef typename VecT<T>::v8 V;
  V t;
#pragma unroll
  for (int i = 0; i < 8; ++i) t[i] = from_f32<T>(v[i]);
  *reinterpret_cast<V *>(p) = t;
}

// ---- streaming loads ---------------------------------------------------------
// Data a launch reads exactly once (decode weights, the KV cache in decode,
// norm and RoPE input rows) is loaded non-temporal (the NT bit of the cache
// policy). Measured on MI355X: 16-byte streaming reads of 64 MiB - 1 GiB run
// at 5.97-7.0 TB/s with it against 5.4-6.2 TB/s without, and LDS-DMA at 6.5
// against 6.0 TB/s. Data that several workgroups re-read (GEMM operands,
// prefill K/V tiles, GEMV input rows, norm weights, RoPE tables) keeps the
// default policy.
constexpr int kCpolNT = 2; // cache-policy operand of global_load_lds: NT
template <typename V> __device__ __forceinline__ V ld_nt(const V *p) {
  return __builtin_nontemporal_load(p);
}
template <typename T>
__device__ __forceinline__ void load8_nt(const T *p, float (&v)[8]) {
  typedef typename VecT<T>::v8 V;
  const V t = ld_nt(reinterpret_cast<const V *>(p));
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = to_f32(t[i]);
}

// ---- wave64 reductions -----------------------------------------------------
// DPP controls (GFX9 encoding): quad_perm, row_half_mirror, row_mirror.
constexpr int kDppQuadXor1 = 0xB1; // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E; // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowRor8 = 0x128; // row_ror:8, lane i of a 16-lane row reads lane i ^ 8

template <int CTRL> __device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                         0xf, 0xf, false));
}

__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over each 16-lane DPP row; every lane of the row receives the row sum.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f32<kDppQuadXor1>(v);
  v += dpp_f32<kDppQuadXor2>(v);
  v += dpp_f32<kDppRowHalfMirror>(v);
  v += dpp_f32<kDppRowMirror>(v);
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f32<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f32<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f32<kDppRowHalfMirror>(v));
  v = fmaxf(v, dpp_f32<kDppRowMirror>(v));
  return v;
}

// Sum over the whole wave; the result is wave-uniform. Requires all 64
// lanes active (callers keep inactive lanes at 0).
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (readlane_f32(v, 0) + readlane_f32(v, 16)) +
         (readlane_f32(v, 32) + readlane_f32(v, 48));
}

// Sum over lanes {l, l^16, l^32, l^48} after a row16 reduction: gives each
// lane the full-wave value without readlane (used where lane groups differ).
__device__ __forceinline__ float xor_sum(float v, int mask) {
  return v + __shfl_xor(v, mask, kWave);
}

// Sum over aligned groups of LPR lanes (LPR in {2, 4, 8, 16}) with DPP.
template <int LPR> __device__ __forceinline__ float group_sum(float v) {
  v += dpp_f32<kDppQuadXor1>(v);
  if constexpr (LPR >= 4) v += dpp_f32<kDppQuadXor2>(v);
  if constexpr (LPR >= 8) v += dpp_f32<kDppRowHalfMirror>(v);
  if constexpr (LPR >= 16) v += dpp_f32<kDppRowMirror>(v);
  return v;
}

// 8 consecutive RoPE table entries of type CS (fp16, bf16 or fp32) as fp32.
template <typename CS>
__device__ __forceinline__ void load_cs8(const CS *p, float (&v)[8]) {
  if constexpr (sizeof(CS) == 4) {
    f32x4 a = *reinterpret_cast<const f32x4 *>(p);
    f32x4 b = *reinterpret_cast<const f32x4 *>(p + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = a[i];
      v[i + 4] = b[i];
    }
  } else {
    load8(p, v);
  }
}

// Same with the table type chosen at run time (a tpp_dtype code).
__device__ __forceinline__ void load_cs8_rt(const void *p, int64_t idx, int cs_dtype,
                                            float (&v)[8]) {
  if (cs_dtype == TPP_F32) load_cs8((const float *)p + idx, v);
  else if (cs_dtype == TPP_F16) load_cs8((const f16 *)p + idx, v);
  else load_cs8((const bf16 *)p + idx, v);
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }
__device__ __forceinline__ int wave_id() { return threadIdx.x / kWave; }

// ---- activations (fp32), csrc/activation/activation.cuh:26-67 -------------
// Both use the hardware exp2-based __expf and the v_rcp_f32 reciprocal
// (~1 ulp) instead of IEEE division / libm tanhf: the epilogue of a GEMM tile
// evaluates ~100 of these per lane with nothing to overlap them.
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
// 0.5 x (1 + tanh(u)) == x * sigmoid(2u), u = sqrt(2/pi) (x + 0.044715 x^3)
__device__ __forceinline__ float act_gelu_tanh(float x) {
  const float kAlpha = 0.7978845608028654f; // sqrt(2/pi)
  const float kBeta = 0.044715f;
  const float u = kAlpha * (x + kBeta * x * x * x);
  return x * fast_rcp(1.0f + __expf(-2.0f * u));
}
__device__ __forceinline__ float act_silu(float x) { return x * fast_rcp(1.0f + __expf(-x)); }
__device__ __forceinline__ float act_relu(float x) { return fmaxf(0.0f, x); }

template <int ACT> __device__ __forceinline__ float apply_act(float x) {
  if constexpr (ACT == TPP_ACT_GELU_TANH) return act_gelu_tanh(x);
  else if constexpr (ACT == TPP_ACT_SILU) return act_silu(x);
  else if constexpr (ACT == TPP_ACT_RELU) return act_relu(x);
  else return x;
}

// ---- host-side error state -------------------------------------------------
int set_error(int code, const char *fmt, ...);
int check_launch(const char *what);
// Workgroups with equal blockIdx % 8 share an XCD (and its L2) on the current
// device: measured once per device by a probe launch (tpp_capi.hip); false
// while unknown when the probe cannot run (stream capture, !may_probe).
bool xcd_grouping_holds(hipStream_t st, bool may_probe);
// Compute units of the current device (0 if unknown).
int device_cu_count();
__host__ __device__ inline bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }
inline int elem_size(int dtype) { return dtype == TPP_F32 ? 4 : 2; }
inline bool half_type(int dtype) { return dtype == TPP_F16 || dtype == TPP_BF16; }

// s_waitcnt vmcnt(N) alone (N < 64; the count is split over two fields of
// the instruction's immediate, bits 3:0 and 15:14)
template <int N> __device__ __forceinline__ void vm_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Workgroup barrier for data exchanged through LDS by ds_write/ds_read: waits
// for this wave's LDS accesses (lgkmcnt(0)) but, unlike the fenced
// __syncthreads(), not for LDS-DMA (global_load_lds) still in flight.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// LDS reads as inline asm, at byte address addr + OFF. The compiler's
// wait-count pass does not see them, so the caller waits for the results
// with lds_wait_tied. Where the pass does see them it over-waits: the
// transposing read's builtin carries no alias information, so it waits for
// every LDS-DMA in flight (vmcnt(0)), including DMA into other slots; and
// fragment reads a few steps ahead of their MFMAs get lgkmcnt(0) waits that
// also cover the reads still meant to be in flight.
typedef short s16x4 __attribute__((ext_vector_type(4)));
template <int OFF> __device__ __forceinline__ s16x4 lds_read_tr16(unsigned addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  s16x4 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
template <int OFF> __device__ __forceinline__ float lds_read_b32(unsigned addr) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset is 16 bits");
  float r;
  asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
template <int OFF, typename V> __device__ __forceinline__ V lds_read_b128(unsigned addr) {
  static_assert(OFF >= 0 && OFF < 65536 && sizeof(V) == 16, "ds offset is 16 bits");
  V r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}
// s_waitcnt lgkmcnt(N) that also redefines the results in v, which are
// complete once at most N LDS reads are outstanding: uses of v after it see
// the loaded data (the tie keeps the compiler from copying a register the
// load has not yet written before the wait). LDS reads complete in order.
template <int N, typename V, int M> __device__ __forceinline__ void lds_wait_tied(V (&v)[M]) {
  static_assert(N >= 0, "lgkmcnt");
  constexpr int n = N < 15 ? N : 15; // 4-bit field: a smaller count only waits longer
  if constexpr (M == 2)
    asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(v[0]), "+v"(v[1]) : "n"(n));
  else if constexpr (M == 3)
    asm volatile("s_waitcnt lgkmcnt(%3)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]) : "n"(n));
  else if constexpr (M == 4)
    asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]) : "n"(n));
  else if constexpr (M == 5)
    asm volatile("s_waitcnt lgkmcnt(%5)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4])
                 : "n"(n));
  else if constexpr (M == 6)
    asm volatile("s_waitcnt lgkmcnt(%6)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5])
                 : "n"(n));
  else if constexpr (M == 8)
    asm volatile("s_waitcnt lgkmcnt(%8)"
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),
                   "+v"(v[6]), "+v"(v[7])
                 : "n"(n));
  else
    static_assert(M >= 2 && M <= 8 && M != 7, "2 to 6 or 8 registers");
}
// f(std::integral_constant<int, i>) for i = 0 .. N-1, in order
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F> __device__ __forceinline__ void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

} // namespace tpp

// Dispatch a body over fp16/bf16. `T` names the element type inside.
// byte offsets in a tpp_attn_decode_oproj workspace: the folded projection's
// counter region and its give-up flag (attention.hip lays them out)
constexpr size_t kAttnOprojCtrOffset = 32768;
constexpr size_t kAttnOprojErrOffset = kAttnOprojCtrOffset + 48 * 32 * sizeof(int);

#define TPP_DISPATCH_HALF(dtype, ...)                                        \
  [&]() -> int {                                                             \
    if ((dtype) == TPP_F16) {                                                \
      typedef ::tpp::f16 T;                                                  \
      return __VA_ARGS__();                                                  \
    } else if ((dtype) == TPP_BF16) {                                        \
      typedef ::tpp::bf16 T;                                                 \
      return __VA_ARGS__();                                                  \
    }                                                                        \
    return ::tpp::set_error(TPP_E_UNSUPPORTED, "unsupported dtype %d",       \
                            (int)(dtype));                                   \
  }()
