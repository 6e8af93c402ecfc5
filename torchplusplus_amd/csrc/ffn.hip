// Decode FFN block in one launch for gfx950 (MI355X):
//   residual <- T(residual + T(down(T(silu(T(x Wg^T))) * T(x Wu^T))))
//   with x = RMSNorm(residual) * norm_w
// i.e. rms_norm2 -> ffn -> `x + x_res` of the decoder block
// (examples/LLM/fastqwen3.py:113-116), with the SwiGLU FFN the reference
// intends (down(silu(gate(x)) * up(x)), examples/TTS/dia/model.py:114-116).
// The same work as the two decode GEMV launches gemv_swiglu + down GEMV
// with the residual add, without the kernel boundary between them.
//
// Work split (hidden E = 1024, intermediate I = 1024..4096, batch B <= 16;
// 256 workgroups of 4 waves, 8 XCDs x 32, workgroup b on XCD b % 8):
//  * Phase 1: XCD x owns the intermediate columns [x I/8, (x+1) I/8). Its
//    workgroup j computes 16 of them (16 gate + 16 up weight rows, K = E
//    split over the 4 waves, MFMA 16x16x32) from the normalised input, and
//    writes h = T(silu(T(g))) * T(u) into a scratch buffer that only XCD x
//    touches (its lines stay in XCD x's L2).
//  * XCD-local sync: every workgroup of the XCD counts itself in; after all
//    32 have arrived the phase-1 outputs of the XCD are complete in its L2.
//  * Phase 2: workgroup j of XCD x computes the partial down projection of
//    output rows [32 j, 32 j + 32) over the XCD's K slice (h columns
//    [x I/8, (x+1) I/8)) and writes the fp32 partial through to memory
//    (agent-scope stores). An agent-scope counter per 32-row chunk finds the
//    last of the 8 XCDs to finish the chunk; that workgroup sums the 8
//    partials in XCD order (a fixed order: bit-reproducible) and updates the
//    residual rows in place.
// Every weight byte is read once (phase-1 and phase-2 weights go HBM -> LDS
// by LDS-DMA at the start). The sync spins are bounded: if workgroups were
// ever not co-resident, a spin gives up after ~10^6 polls, sets an error
// flag in the workspace and the launch still ends (wrong output, flagged).
// The fused path runs only where the 256 workgroups fit one per CU (256 CUs)
// and the XCD placement probe holds; elsewhere tpp_ffn_decode launches the
// two GEMVs instead.
#include "tpp_common.hpp"

namespace tpp {

constexpr int kFfnXcds = 8;
constexpr int kFfnPerXcd = 32;
constexpr int kFfnBlocks = kFfnXcds * kFfnPerXcd;
constexpr int kFfnWaves = 4;
constexpr int kFfnE = 1024;                 // hidden size of the fused path
constexpr int kFfnKW1 = kFfnE / kFfnWaves;  // phase-1 K per wave
constexpr int kFfnNS1 = kFfnKW1 / 32;       // phase-1 MFMA steps per wave
constexpr int kFfnRows2 = kFfnE / kFfnPerXcd; // phase-2 output rows per workgroup (32)
constexpr unsigned kFfnSpinLimit = 1u << 20;
// workspace: counters (each on its own 128-byte line), then h, then partials
constexpr size_t kFfnOffArrive = 0;                         // [8] x 128 B
constexpr size_t kFfnOffDepart = 1024;                      // [8] x 128 B
constexpr size_t kFfnOffChunk = 2048;                       // [32] x 128 B
constexpr size_t kFfnOffErr = kFfnOffChunk + kFfnPerXcd * 128;
constexpr size_t kFfnCtrBytes = 8192;

__device__ uint32_t g_ffn_zero16[4];

template <typename T>
__device__ __forceinline__ typename VecT<T>::v8 ffn_ld16(const T *p, bool ok) {
  typedef typename VecT<T>::v8 V;
  return *reinterpret_cast<const V *>(ok ? p : reinterpret_cast<const T *>(g_ffn_zero16));
}

// the same 16 bytes as inline asm, invisible to the compiler's wait counts:
// the caller waits with ffn_vm_wait_tied
template <typename T>
__device__ __forceinline__ typename VecT<T>::v8 ffn_ld16_asm(const T *p, bool ok) {
  typename VecT<T>::v8 v;
  const void *q = ok ? (const void *)p : (const void *)g_ffn_zero16;
  asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(q));
  return v;
}
// s_waitcnt vmcnt(N) that also redefines a and b: they are complete once at
// most N later loads are in flight (loads complete in issue order), and no
// copy of them can be made before the wait
template <int N, typename V>
__device__ __forceinline__ void ffn_vm_wait_tied(V (&a)[8], V (&b)[8]) {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%16)"
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]),
                 "+v"(a[6]), "+v"(a[7]), "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]),
                 "+v"(b[4]), "+v"(b[5]), "+v"(b[6]), "+v"(b[7])
               : "n"(N));
}

template <typename T>
__device__ __forceinline__ f32x4 ffn_mfma(typename VecT<T>::v8 a, typename VecT<T>::v8 b, f32x4 c) {
  if constexpr (__is_same(T, bf16))
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

struct FfnArgs {
  void *resid;        // [NB, E] in/out
  const void *norm_w; // [E]
  float eps;
  const void *w_gu;   // [2I, E], gate/up interleaved in blocks of 32 rows
  const void *w_down; // [E, I]
  int NB, I;
  char *ws;
};

__host__ __device__ inline size_t ffn_h_bytes(int64_t B, int64_t I) { return ((size_t)(B * I * 2) + 255) & ~(size_t)255; }

// Phase-2 K units (16 bytes) per weight row and wave: I / 8 / 4 / 8.
template <typename T, int U2>
__global__ __launch_bounds__(256) void ffn_decode_kernel(FfnArgs a) {
  typedef typename VecT<T>::v8 V8;
  constexpr int KW2 = U2 * 8;  // phase-2 K per wave
  constexpr int NS2 = KW2 / 32;
  const int lane = lane_id(), w = wave_id();
  const int r = lane & 15, g = lane >> 4;
  const int x = blockIdx.x % kFfnXcds, j = blockIdx.x / kFfnXcds;
  const int NB = a.NB, I = a.I;
  const int IX = I / kFfnXcds;     // intermediate slice of this XCD
  const bool active1 = j < IX / 16; // this workgroup has a phase-1 tile
  T *resid = (T *)a.resid;
  const T *Wgu = (const T *)a.w_gu;
  const T *Wd = (const T *)a.w_down;
  int *arrive = (int *)(a.ws + kFfnOffArrive + x * 128);
  int *depart = (int *)(a.ws + kFfnOffDepart + x * 128);
  int *chunk = (int *)(a.ws + kFfnOffChunk + j * 128);
  int *err = (int *)(a.ws + kFfnOffErr);
  T *H = (T *)(a.ws + kFfnCtrBytes);
  float *P = (float *)(a.ws + kFfnCtrBytes + ffn_h_bytes(NB, I));

  extern __shared__ __attribute__((aligned(16))) char ffn_smem[];
  V8 *s_gu = reinterpret_cast<V8 *>(ffn_smem);      // [4 waves][2 sets][16 rows][32 units]
  V8 *s_dn = s_gu + kFfnWaves * 2 * 16 * 32;         // [4 waves][32 rows][U2 units]
  f32x4 *s_red = reinterpret_cast<f32x4 *>(s_dn + kFfnWaves * 32 * U2); // [2][4][64]
  float *s_ss = reinterpret_cast<float *>(s_red + 2 * kFfnWaves * 64);  // [4][16]
  __shared__ int s_last;

  // ---- loads: input, then phase-1 and phase-2 weights (HBM -> LDS) -------
  // The input row slice and norm weights go first, as inline asm (after an
  // LDS-DMA the compiler's own wait for a plain load is vmcnt(0), which would
  // also wait for the weights), then the gate/up tile by LDS-DMA, then the
  // down slice. Loads complete in issue order, so counted waits take the
  // input while the weights are on the way, then the gate/up weights while
  // the down weights are.
  const int c0 = x * IX + 16 * j; // phase-1 tile: intermediate columns c0 .. c0 + 15
  const int64_t grow = (int64_t)(c0 / 32) * 64 + (c0 % 32); // first gate row; up rows +32
  V8 *gslot = s_gu + w * (2 * 16 * 32);
  V8 *dslot = s_dn + w * (32 * U2);
  // the down-projection slice by LDS-DMA (every workgroup has one); issued
  // after the phase-1 loads so that counted waits can take those first
  auto issue_down = [&]() {
#pragma unroll
    for (int jj = 0; jj < U2 / 2; ++jj) {
      const int q = jj * 64 + lane; // LDS unit: row q / U2, K unit q % U2
      const int row = q / U2, unit = q % U2;
      const T *src = Wd + (int64_t)(kFfnRows2 * j + row) * I + x * IX + w * KW2 + unit * 8;
      __builtin_amdgcn_global_load_lds(
          (const void *)src, (__attribute__((address_space(3))) void *)(dslot + jj * 64), 16, 0,
          kCpolNT);
    }
  };
  // The workgroups with a phase-1 tile run their loads, DMA, waits and phase 1
  // in one branch (the others only issue the down slice), so no branch on
  // `active1` separates the inline-asm loads from their wait.
  if (active1) {
    V8 xa[kFfnNS1], nwv[kFfnNS1];
    const bool xok = r < NB;
    const T *xr = resid + (xok ? r : 0) * kFfnE;
#pragma unroll
    for (int u = 0; u < kFfnNS1; ++u) {
      const int c = w * kFfnKW1 + u * 32 + g * 8;
      xa[u] = ffn_ld16_asm(xr + c, xok);
      nwv[u] = ffn_ld16_asm((const T *)a.norm_w + c, true);
    }
    __builtin_amdgcn_sched_barrier(0);
    const int drow = lane >> 5, dpos = lane & 31;
#pragma unroll
    for (int set = 0; set < 2; ++set)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        // rows 2jj, 2jj+1 of the set; LDS unit dpos of a row holds K unit
        // dpos ^ row (the MFMA reads below then hit distinct bank groups)
        const int row = 2 * jj + drow;
        const T *src = Wgu + (grow + set * 32 + row) * kFfnE + w * kFfnKW1 + (dpos ^ row) * 8;
        __builtin_amdgcn_global_load_lds(
            (const void *)src,
            (__attribute__((address_space(3))) void *)(gslot + set * 512 + jj * 64), 16, 0,
            kCpolNT);
      }
    issue_down();
    __builtin_amdgcn_sched_barrier(0);

    // ---- phase 1: RMSNorm + gate/up + SwiGLU of this tile -----------------
    ffn_vm_wait_tied<16 + U2 / 2>(xa, nwv); // input in; both weight DMAs in flight
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < kFfnNS1; ++u)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = to_f32(xa[u][i]);
        ss += v * v;
      }
    ss += __shfl_xor(ss, 16, kWave); // lanes r, r+16, r+32, r+48 hold row r
    ss += __shfl_xor(ss, 32, kWave);
    if (g == 0) s_ss[w * 16 + r] = ss;
    lds_barrier(); // (a fenced barrier would also wait for the weight DMA)
    const float tot = s_ss[r] + s_ss[16 + r] + s_ss[32 + r] + s_ss[48 + r];
    const float inv = rsqrtf(tot / (float)kFfnE + a.eps);
#pragma unroll
    for (int u = 0; u < kFfnNS1; ++u)
#pragma unroll
      for (int i = 0; i < 8; ++i)
        xa[u][i] = from_f32<T>((to_f32(xa[u][i]) * inv) * to_f32(nwv[u][i]));
    // gate/up weights landed (the down DMA may still be in flight); the
    // operand reads are inline asm so no compiler wait covers that DMA
    vm_wait<U2 / 2>();
    const unsigned gbase = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) char *)gslot;
    V8 wg[kFfnNS1], wu[kFfnNS1];
#pragma unroll
    for (int u = 0; u < kFfnNS1; ++u)
      wg[u] = lds_read_b128<0, V8>(gbase + (unsigned)((r * 32 + ((u * 4 + g) ^ r)) * 16));
    lds_wait_tied<0>(wg);
#pragma unroll
    for (int u = 0; u < kFfnNS1; ++u)
      wu[u] = lds_read_b128<512 * 16, V8>(gbase + (unsigned)((r * 32 + ((u * 4 + g) ^ r)) * 16));
    f32x4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kFfnNS1; ++u) ag = ffn_mfma<T>(xa[u], wg[u], ag);
    lds_wait_tied<0>(wu);
#pragma unroll
    for (int u = 0; u < kFfnNS1; ++u) au = ffn_mfma<T>(xa[u], wu[u], au);
    s_red[w * 64 + lane] = ag;
    s_red[(kFfnWaves + w) * 64 + lane] = au;
    lds_barrier();
    if (w == 0) {
      f32x4 sg = s_red[lane], su = s_red[kFfnWaves * 64 + lane];
#pragma unroll
      for (int i = 1; i < kFfnWaves; ++i) {
        sg += s_red[i * 64 + lane];
        su += s_red[(kFfnWaves + i) * 64 + lane];
      }
      // D layout: lane -> column r (intermediate c0 + r), batch rows 4g + i
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int b = 4 * g + i;
        const float gt = to_f32(from_f32<T>(sg[i]));
        const float s = to_f32(from_f32<T>(act_silu(gt)));
        const float ut = to_f32(from_f32<T>(su[i]));
        if (b < NB) H[(int64_t)b * I + c0 + r] = from_f32<T>(s * ut);
      }
    }
  } else {
    issue_down();
  }

  // ---- XCD-local sync -------------------------------------------------------
  // h stores reached this XCD's L2 (vmcnt(0), which also covers the down
  // DMA); one thread counts the workgroup in and waits for the XCD's other
  // 31. The counter is reset after phase 2 by the XCD's last workgroup to
  // leave (depart below), off this critical path. The poll is an atomic add
  // of 0, performed in the XCD's L2 where the arrivals are counted; an
  // agent-scope load goes past the L2 on every poll (measured: decode step
  // 1.115 -> 1.082 ms with the atomic). The 0 comes from an asm move: the
  // compiler turns an atomic add of a known 0 back into that load.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned n = 0;
    int zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    while (__hip_atomic_fetch_add(arrive, zero, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < kFfnPerXcd) {
      if (++n > kFfnSpinLimit) {
        __hip_atomic_fetch_or(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
  // leaving: the XCD's last workgroup to leave resets both counters for the
  // next launch (every workgroup of the XCD is past the wait above by then)
  auto depart_xcd = [&]() {
    if (threadIdx.x == 0 &&
        __hip_atomic_fetch_add(depart, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
            kFfnPerXcd - 1) {
      __hip_atomic_store(arrive, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(depart, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  };

  // ---- phase 2: partial down projection over this XCD's K slice -----------
  // The residual rows of this workgroup's output chunk are loaded now: if it
  // turns out to be the chunk's last XCD it adds the summed partials to them
  // without another memory round trip (nobody writes them before that).
  T rres[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int e = threadIdx.x + k * 256;
    const int b = e / kFfnRows2 < NB ? e / kFfnRows2 : 0;
    rres[k] = resid[(int64_t)b * kFfnE + kFfnRows2 * j + e % kFfnRows2];
  }
  {
    const bool hok = r < NB;
    const T *hr = H + (int64_t)(hok ? r : 0) * I + x * IX + w * KW2;
    V8 hv[NS2];
#pragma unroll
    for (int u = 0; u < NS2; ++u) hv[u] = ffn_ld16(hr + u * 32 + g * 8, hok);
    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int u = 0; u < NS2; ++u)
#pragma unroll
      for (int t = 0; t < 2; ++t)
        acc[t] = ffn_mfma<T>(hv[u], dslot[(t * 16 + r) * U2 + u * 4 + g], acc[t]);
    s_red[w * 64 + lane] = acc[0];
    s_red[(kFfnWaves + w) * 64 + lane] = acc[1];
    lds_barrier();
    if (w == 0) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        f32x4 s = s_red[t * kFfnWaves * 64 + lane];
#pragma unroll
        for (int i = 1; i < kFfnWaves; ++i) s += s_red[(t * kFfnWaves + i) * 64 + lane];
        const int n = kFfnRows2 * j + t * 16 + r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int b = 4 * g + i;
          if (b < NB)
            __hip_atomic_store(P + ((int64_t)x * NB + b) * kFfnE + n, s[i], __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
      }
    }
  }
  // partial written through (vmcnt(0)); count this XCD in for the chunk
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(chunk, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = old == kFfnXcds - 1;
    if (old == kFfnXcds - 1) __hip_atomic_store(chunk, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) {
    depart_xcd();
    return;
  }
  // last of the 8 XCDs for this chunk: sum the partials in XCD order, round
  // like the unfused path (T(x W^T), then T(residual + that)), store
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int e = threadIdx.x + k * 256; // blockDim.x == 256, NB * 32 <= 512
    if (e >= NB * kFfnRows2) break;
    const int b = e / kFfnRows2, n = kFfnRows2 * j + e % kFfnRows2;
    float v[kFfnXcds];
#pragma unroll
    for (int xx = 0; xx < kFfnXcds; ++xx)
      v[xx] = __hip_atomic_load(P + ((int64_t)xx * NB + b) * kFfnE + n, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
    float s = 0.f;
#pragma unroll
    for (int xx = 0; xx < kFfnXcds; ++xx) s += v[xx];
    resid[(int64_t)b * kFfnE + n] = from_f32<T>(to_f32(rres[k]) + to_f32(from_f32<T>(s)));
  }
  depart_xcd();
}

template <typename T, int U2>
static int launch_ffn(const FfnArgs &fa, hipStream_t st, const char *name) {
  const size_t lds = (size_t)kFfnWaves * 2 * 16 * 32 * 16 + (size_t)kFfnWaves * 32 * U2 * 16 +
                     2 * kFfnWaves * 64 * 16 + kFfnWaves * 16 * 4;
  static bool attr_set = false; // per instantiation; the attribute is per function
  if (!attr_set) {
    if (hipFuncSetAttribute((const void *)ffn_decode_kernel<T, U2>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return set_error(TPP_E_LAUNCH, "%s: hipFuncSetAttribute failed", name);
    attr_set = true;
  }
  ffn_decode_kernel<T, U2><<<dim3(kFfnBlocks), dim3(64 * kFfnWaves), lds, st>>>(fa);
  return check_launch(name);
}

} // namespace tpp

using namespace tpp;

extern "C" size_t tpp_ffn_decode_workspace_size(int64_t B, int64_t E, int64_t I) {
  if (B <= 0 || E <= 0 || I <= 0) return 0;
  // counters + h [B, I] + 8 fp32 partials [8, B, E] (the unfused path uses
  // the h region only)
  return kFfnCtrBytes + ffn_h_bytes(B, I) + (size_t)kFfnXcds * B * E * sizeof(float);
}

extern "C" int tpp_ffn_decode(void *residual, const void *norm_w, float eps, const void *w_gu,
                              const void *w_down, int64_t B, int64_t E, int64_t I, int dtype,
                              void *workspace, size_t ws_bytes, void *stream) {
  const char *name = "tpp_ffn_decode";
  if (!residual || !norm_w || !w_gu || !w_down)
    return set_error(TPP_E_INVALID, "%s: null pointer argument", name);
  if (B <= 0 || B > 16 || E <= 0 || I <= 0 || I % 32 != 0)
    return set_error(TPP_E_INVALID, "%s: need 1 <= B <= 16 and I a multiple of 32", name);
  if (!half_type(dtype)) return set_error(TPP_E_UNSUPPORTED, "%s: dtype must be f16 or bf16", name);
  const size_t need = tpp_ffn_decode_workspace_size(B, E, I);
  if (!workspace || ws_bytes < need || (uintptr_t)workspace % 256 != 0)
    return set_error(TPP_E_WORKSPACE, "%s: 256-byte aligned workspace of %zu bytes required", name,
                     need);
  hipStream_t st = as_stream(stream);
  char *ws = (char *)workspace;
  const bool fused = E == kFfnE && I % 1024 == 0 && I <= 4096 && aligned16(residual) &&
                     aligned16(norm_w) && aligned16(w_gu) && aligned16(w_down) &&
                     device_cu_count() == kFfnBlocks && xcd_grouping_holds(st, true);
  if (!fused) {
    // two launches: SwiGLU GEMV into h, down GEMV with the residual add
    void *h = ws + kFfnCtrBytes;
    if (int e = tpp_gemv_fused(residual, norm_w, eps, w_gu, h, nullptr, B, 2 * I, E, 1, dtype,
                               stream))
      return e;
    return tpp_gemv_fused(h, nullptr, 0.f, w_down, nullptr, residual, B, E, I, 0, dtype, stream);
  }
  FfnArgs fa{residual, norm_w, eps, w_gu, w_down, (int)B, (int)I, ws};
  return TPP_DISPATCH_HALF(dtype, [&] {
    switch (I / 256) { // K units per phase-2 weight row and wave
    case 4: return launch_ffn<T, 4>(fa, st, name);
    case 8: return launch_ffn<T, 8>(fa, st, name);
    case 12: return launch_ffn<T, 12>(fa, st, name);
    default: return launch_ffn<T, 16>(fa, st, name);
    }
  });
}

extern "C" int tpp_ffn_decode_sync_errors(void *workspace, int *out, void *stream) {
  const char *name = "tpp_ffn_decode_sync_errors";
  if (!workspace || !out) return set_error(TPP_E_INVALID, "%s: null pointer", name);
  hipStream_t st = as_stream(stream);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return set_error(TPP_E_INVALID, "%s: not callable while the stream is being captured", name);
  }
  int flag = 0;
  if (hipMemcpyAsync(&flag, (const char *)workspace + kFfnOffErr, sizeof(int),
                     hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(TPP_E_LAUNCH, "%s: copy failed", name);
  }
  // a launch that gave up leaves its counters in an unknown state (late
  // workgroups count in after the reset): zero them and the flag, so the
  // workspace is usable again
  if (flag && (hipMemsetAsync(workspace, 0, kFfnCtrBytes, st) != hipSuccess ||
               hipStreamSynchronize(st) != hipSuccess)) {
    (void)hipGetLastError();
    return set_error(TPP_E_LAUNCH, "%s: clearing the counters failed", name);
  }
  *out = flag;
  return TPP_OK;
}

extern "C" int tpp_decode_force_sync_error(void *workspace, int kernel, void *stream) {
  const char *name = "tpp_decode_force_sync_error";
  if (!workspace || (kernel != 0 && kernel != 1))
    return set_error(TPP_E_INVALID, "%s: null workspace or unknown kernel %d", name, kernel);
  // kernel 0: tpp_attn_decode_oproj's flag, 1: tpp_ffn_decode's; a stray
  // arrival count is left as well, as a launch that gave up would
  static const int kOne[2] = {1, 5};
  const size_t err_off = kernel == 0 ? kAttnOprojErrOffset : kFfnOffErr;
  const size_t ctr_off = kernel == 0 ? kAttnOprojCtrOffset : kFfnOffArrive;
  hipStream_t st = as_stream(stream);
  if (hipMemcpyAsync((char *)workspace + err_off, &kOne[0], sizeof(int), hipMemcpyHostToDevice, st) !=
          hipSuccess ||
      hipMemcpyAsync((char *)workspace + ctr_off, &kOne[1], sizeof(int), hipMemcpyHostToDevice, st) !=
          hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(TPP_E_LAUNCH, "%s: copy failed", name);
  }
  return TPP_OK;
}
