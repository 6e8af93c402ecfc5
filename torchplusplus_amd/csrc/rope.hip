// Rotary position embedding (rotate-half form) for gfx950.
//
// Semantics: csrc/dlops/rope/apply_rope.cuh:15-46 (one tensor) and
// csrc/dlops/qkrope/qkrope.cuh:20-67 (Q and K in one launch):
//   i <  D/2: out_i = x_i * cos[s,i] - x_{i+D/2} * sin[s,i]
//   i >= D/2: out_i = x_i * cos[s,i] + x_{i-D/2} * sin[s,i]
// where s is the sequence index of the row. The reference does this in fp16
// arithmetic (every __hmul/__hadd rounds); here it is fp32 with one rounding.
//
// Mapping: one thread owns the pair block (i .. i+7, i+D/2 .. i+D/2+7), so it
// reads each input element exactly once (the reference reads every element
// twice: own + partner) with 128-bit loads, and the op is safe in place.
// Q and K rows are one flat grid, so Hk may differ from Hq (GQA), which the
// reference's qkrope rejected (qkrope_binding.cu:52-55).
#include "tpp_common.hpp"

namespace tpp {

__device__ __forceinline__ void rotate8(float (&x1)[8], float (&x2)[8], const float (&c1)[8],
                                        const float (&c2)[8], const float (&s1)[8],
                                        const float (&s2)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    float a = x1[j], b = x2[j];
    x1[j] = a * c1[j] - b * s1[j];
    x2[j] = b * c2[j] + a * s2[j];
  }
}

// x rows are [rows, D] contiguous; row r has sequence index r % S.
template <typename T, typename CS>
__global__ __launch_bounds__(256) void rope_vec_kernel(
    const T *__restrict__ q, T *qo, int64_t rows_q, const T *__restrict__ k, T *ko,
    int64_t rows_k, const CS *__restrict__ cos, const CS *__restrict__ sin, int S,
    int D) {
  const int tpr = D >> 4; // threads per row
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t row = t / tpr;
  const int i0 = (int)(t - row * tpr) * 8;
  const T *src;
  T *dst;
  if (row < rows_q) {
    src = q;
    dst = qo;
  } else {
    row -= rows_q;
    if (row >= rows_k) return;
    src = k;
    dst = ko;
  }
  const int h = D >> 1;
  const int s = (int)(row % S);
  const int64_t base = row * D;
  float x1[8], x2[8], c1[8], c2[8], s1[8], s2[8];
  load8_nt(src + base + i0, x1);
  load8_nt(src + base + h + i0, x2);
  load_cs8(cos + (int64_t)s * D + i0, c1);
  load_cs8(cos + (int64_t)s * D + h + i0, c2);
  load_cs8(sin + (int64_t)s * D + i0, s1);
  load_cs8(sin + (int64_t)s * D + h + i0, s2);
  rotate8(x1, x2, c1, c2, s1, s2);
  store8(dst + base + i0, x1);
  store8(dst + base + h + i0, x2);
}

// Generic: one thread per (i, i + D/2) pair, any even D, any alignment.
template <typename T, typename CS>
__global__ __launch_bounds__(256) void rope_scalar_kernel(
    const T *__restrict__ q, T *qo, int64_t rows_q, const T *__restrict__ k, T *ko,
    int64_t rows_k, const CS *__restrict__ cos, const CS *__restrict__ sin, int S,
    int D) {
  const int h = D >> 1;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t row = t / h;
  const int i = (int)(t - row * h);
  const T *src;
  T *dst;
  if (row < rows_q) {
    src = q;
    dst = qo;
  } else {
    row -= rows_q;
    if (row >= rows_k) return;
    src = k;
    dst = ko;
  }
  const int s = (int)(row % S);
  const int64_t base = row * D;
  const float a = to_f32(src[base + i]), b = to_f32(src[base + i + h]);
  const int64_t cb = (int64_t)s * D;
  const float c1 = to_f32(cos[cb + i]), c2 = to_f32(cos[cb + i + h]);
  const float s1 = to_f32(sin[cb + i]), s2 = to_f32(sin[cb + i + h]);
  dst[base + i] = from_f32<T>(a * c1 - b * s1);
  dst[base + i + h] = from_f32<T>(b * c2 + a * s2);
}

template <typename T, typename CS>
static int launch_rope(const void *q, void *qo, int64_t rows_q, const void *k, void *ko,
                       int64_t rows_k, const void *cos, const void *sin, int64_t S,
                       int64_t D, hipStream_t st, const char *name) {
  const int64_t rows = rows_q + rows_k;
  if (rows == 0) return TPP_OK;
  const bool vec = (D % 16 == 0) && aligned16(q) && aligned16(qo) && aligned16(cos) &&
                   aligned16(sin) && (rows_k == 0 || (aligned16(k) && aligned16(ko)));
  const int64_t per_row = vec ? D / 16 : D / 2;
  const int64_t threads = rows * per_row;
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > 0x7fffffffLL) return set_error(TPP_E_UNSUPPORTED, "%s: too large", name);
  if (vec)
    rope_vec_kernel<T, CS><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
        (const T *)q, (T *)qo, rows_q, (const T *)k, (T *)ko, rows_k, (const CS *)cos,
        (const CS *)sin, (int)S, (int)D);
  else
    rope_scalar_kernel<T, CS><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
        (const T *)q, (T *)qo, rows_q, (const T *)k, (T *)ko, rows_k, (const CS *)cos,
        (const CS *)sin, (int)S, (int)D);
  return check_launch(name);
}

static int rope_dispatch(const void *q, void *qo, int64_t rows_q, const void *k, void *ko,
                         int64_t rows_k, const void *cos, const void *sin, int64_t S,
                         int64_t D, int dtype, int cs_dtype, void *stream,
                         const char *name) {
  if (S <= 0 || D <= 0 || (D & 1))
    return set_error(TPP_E_INVALID, "%s: head dim must be even (S=%lld, D=%lld)", name,
                     (long long)S, (long long)D);
  if (!cos || !sin) return set_error(TPP_E_INVALID, "%s: null cos/sin", name);
  if (cs_dtype != TPP_F16 && cs_dtype != TPP_BF16 && cs_dtype != TPP_F32)
    return set_error(TPP_E_UNSUPPORTED, "%s: cos/sin dtype must be f16, bf16 or f32", name);
  hipStream_t st = as_stream(stream);
  return TPP_DISPATCH_HALF(dtype, [&] {
    if (cs_dtype == TPP_F32)
      return launch_rope<T, float>(q, qo, rows_q, k, ko, rows_k, cos, sin, S, D, st, name);
    if (cs_dtype == TPP_F16)
      return launch_rope<T, f16>(q, qo, rows_q, k, ko, rows_k, cos, sin, S, D, st, name);
    return launch_rope<T, bf16>(q, qo, rows_q, k, ko, rows_k, cos, sin, S, D, st, name);
  });
}

// ---------------------------------------------------------------------------
// Fused QK-RMSNorm + RoPE + KV-cache append for the decoder block.
// Replaces, per layer, the chain at torchpp/attention/gqa.py:86-118:
//   view/transpose -> q_norm/k_norm (nn.RMSNorm(head_dim)) -> .contiguous()
//   -> rope_apply(Q), rope_apply(K) -> kv_cache.update(K, V)
// Input qkv: [B, S, (Hq + 2*Hkv) * D], the fused projection output.
// Outputs: q_out [B, S, Hq, D]; k_cache/v_cache [B, Hkv, Lmax, D] written at
// positions pos[b] + s. cos/sin: [ctx, D] tables indexed by absolute position.
// One 16-byte chunk of each half-row per lane, D/16 lanes per row, the row
// RMS reduced with DPP inside those lanes.
// ---------------------------------------------------------------------------
template <typename T, typename CS, int LPR>
__global__ __launch_bounds__(256) void qkv_rope_cache_kernel(
    const T *__restrict__ qkv, T *__restrict__ q_out, T *__restrict__ k_cache,
    T *__restrict__ v_cache, const T *__restrict__ qw, const T *__restrict__ kw,
    const CS *__restrict__ cos, const CS *__restrict__ sin,
    const int *__restrict__ pos, int B, int S, int Hq, int Hkv, int Lmax, float eps,
    int ctx) {
  constexpr int D = LPR * 16;
  const int H = Hq + 2 * Hkv;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = t / LPR; // (b, s, head)
  const int c = (int)(t % LPR);
  const int64_t nrows = (int64_t)B * S * H;
  const bool valid = row < nrows;
  const int head = valid ? (int)(row % H) : 0;
  const int64_t bs = valid ? row / H : 0;
  const int s = (int)(bs % S);
  const int b = (int)(bs / S);
  const int i0 = c * 8;
  float x1[8] = {0}, x2[8] = {0};
  if (valid) {
    const T *src = qkv + row * D;
    load8(src + i0, x1);
    load8(src + D / 2 + i0, x2);
  }
  const bool is_q = head < Hq, is_k = !is_q && head < Hq + Hkv;
  // RMS over the D elements of this row (all lanes of the group take part).
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) ss += x1[j] * x1[j] + x2[j] * x2[j];
  ss = group_sum<LPR>(ss);
  if (!valid) return;
  const int p = pos[b] + s;
  if (is_q || is_k) {
    const T *nw = is_q ? qw : kw;
    if (nw) {
      const float inv = rsqrtf(ss / (float)D + eps);
      float w1[8], w2[8];
      load8(nw + i0, w1);
      load8(nw + D / 2 + i0, w2);
      // nn.RMSNorm on a half tensor returns that dtype: round before RoPE.
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        x1[j] = to_f32(from_f32<T>((x1[j] * inv) * w1[j]));
        x2[j] = to_f32(from_f32<T>((x2[j] * inv) * w2[j]));
      }
    }
    const int pr = p < 0 ? 0 : (p < ctx ? p : ctx - 1);
    float c1[8], c2[8], s1[8], s2[8];
    load_cs8(cos + (int64_t)pr * D + i0, c1);
    load_cs8(cos + (int64_t)pr * D + D / 2 + i0, c2);
    load_cs8(sin + (int64_t)pr * D + i0, s1);
    load_cs8(sin + (int64_t)pr * D + D / 2 + i0, s2);
    rotate8(x1, x2, c1, c2, s1, s2);
  }
  T *dst;
  if (is_q) {
    dst = q_out + (((int64_t)b * S + s) * Hq + head) * D;
  } else {
    const int hk = is_k ? head - Hq : head - Hq - Hkv;
    T *cache = is_k ? k_cache : v_cache;
    if (p < 0 || p >= Lmax) return; // host checks bounds; never write outside the cache
    dst = cache + (((int64_t)b * Hkv + hk) * Lmax + p) * D;
  }
  store8(dst + i0, x1);
  store8(dst + D / 2 + i0, x2);
}

struct QkvArgs {
  const void *qkv;
  void *q_out, *k_cache, *v_cache;
  const void *qw, *kw, *cos, *sin;
  const int32_t *pos;
  int B, S, Hq, Hkv, Lmax;
  float eps;
  int ctx, lpr;
  unsigned blocks;
  hipStream_t st;
};

template <typename T, typename CS, int LPR>
static void launch_qkv_lpr(const QkvArgs &a) {
  qkv_rope_cache_kernel<T, CS, LPR><<<dim3(a.blocks), dim3(256), 0, a.st>>>(
      (const T *)a.qkv, (T *)a.q_out, (T *)a.k_cache, (T *)a.v_cache, (const T *)a.qw,
      (const T *)a.kw, (const CS *)a.cos, (const CS *)a.sin, a.pos, a.B, a.S, a.Hq, a.Hkv,
      a.Lmax, a.eps, a.ctx);
}

template <typename T, typename CS>
static int launch_qkv(const QkvArgs &a, const char *name) {
  if (a.lpr == 4) launch_qkv_lpr<T, CS, 4>(a);
  else if (a.lpr == 8) launch_qkv_lpr<T, CS, 8>(a);
  else launch_qkv_lpr<T, CS, 16>(a);
  return check_launch(name);
}

} // namespace tpp

using namespace tpp;

extern "C" int tpp_rope(const void *x, void *out, const void *cos, const void *sin,
                        int64_t B, int64_t H, int64_t S, int64_t D, int dtype,
                        int cs_dtype, void *stream) {
  const char *name = "tpp_rope";
  if (!x || !out) return set_error(TPP_E_INVALID, "%s: null input/output", name);
  if (B < 0 || H < 0) return set_error(TPP_E_INVALID, "%s: negative shape", name);
  return rope_dispatch(x, out, B * H * S, nullptr, nullptr, 0, cos, sin, S, D, dtype,
                       cs_dtype, stream, name);
}

extern "C" int tpp_rope_qk(const void *q, const void *k, void *q_out, void *k_out,
                           const void *cos, const void *sin, int64_t B, int64_t Hq,
                           int64_t Hk, int64_t S, int64_t D, int dtype, int cs_dtype,
                           void *stream) {
  const char *name = "tpp_rope_qk";
  if (!q || !k || !q_out || !k_out)
    return set_error(TPP_E_INVALID, "%s: null input/output", name);
  if (B < 0 || Hq < 0 || Hk < 0) return set_error(TPP_E_INVALID, "%s: negative shape", name);
  return rope_dispatch(q, q_out, B * Hq * S, k, k_out, B * Hk * S, cos, sin, S, D, dtype,
                       cs_dtype, stream, name);
}

extern "C" int tpp_qkv_rope_cache(const void *qkv, void *q_out, void *k_cache,
                                  void *v_cache, const void *q_norm_w,
                                  const void *k_norm_w, const void *cos, const void *sin,
                                  int64_t ctx, const int32_t *positions, int64_t B,
                                  int64_t S, int64_t Hq, int64_t Hkv, int64_t D,
                                  int64_t Lmax, float eps, int dtype, int cs_dtype,
                                  void *stream) {
  const char *name = "tpp_qkv_rope_cache";
  if (!qkv || !q_out || !k_cache || !v_cache || !cos || !sin || !positions)
    return set_error(TPP_E_INVALID, "%s: null pointer argument", name);
  if (B <= 0 || S <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0 || Lmax <= 0 || ctx <= 0)
    return set_error(TPP_E_INVALID, "%s: invalid shapes", name);
  if (ctx < Lmax) // every cache position must have a table row (no clamping)
    return set_error(TPP_E_INVALID, "%s: cos/sin hold %lld positions, fewer than the cache length %lld",
                     name, (long long)ctx, (long long)Lmax);
  if (D != 64 && D != 128 && D != 256)
    return set_error(TPP_E_UNSUPPORTED, "%s: head_dim %lld not in {64,128,256}", name,
                     (long long)D);
  if (!aligned16(qkv) || !aligned16(q_out) || !aligned16(k_cache) || !aligned16(v_cache) ||
      !aligned16(cos) || !aligned16(sin) || (q_norm_w && !aligned16(q_norm_w)) ||
      (k_norm_w && !aligned16(k_norm_w)))
    return set_error(TPP_E_INVALID, "%s: pointers must be 16-byte aligned", name);
  if (cs_dtype != TPP_F16 && cs_dtype != TPP_BF16 && cs_dtype != TPP_F32)
    return set_error(TPP_E_UNSUPPORTED, "%s: cos/sin dtype must be f16, bf16 or f32", name);
  const int64_t rows = B * S * (Hq + 2 * Hkv);
  const int lpr = (int)(D / 16);
  const int64_t blocks = (rows * lpr + 255) / 256;
  if (blocks > 0x7fffffffLL) return set_error(TPP_E_UNSUPPORTED, "%s: too large", name);
  QkvArgs a{qkv, q_out, k_cache, v_cache, q_norm_w, k_norm_w, cos, sin, positions,
            (int)B, (int)S, (int)Hq, (int)Hkv, (int)Lmax, eps, (int)ctx, lpr,
            (unsigned)blocks, as_stream(stream)};
  return TPP_DISPATCH_HALF(dtype, [&] {
    if (cs_dtype == TPP_F32) return launch_qkv<T, float>(a, name);
    if (cs_dtype == TPP_F16) return launch_qkv<T, f16>(a, name);
    return launch_qkv<T, bf16>(a, name);
  });
}
