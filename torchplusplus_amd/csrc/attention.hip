// Flash attention for gfx950: GQA/MQA/MHA, causal and sliding-window prefill,
// and split-KV decode against a KV cache.
//
// Contract: the flash_attn_func calls of the reference
// (torchpp/attention/gqa.py:128, swa.py:85-89, mha.py:84, mqa.py:87, ca.py:83):
//   O = softmax(Q K^T * scale + mask) V, fp32 softmax and accumulation,
//   scale = 1/sqrt(D) by default, query head h reads KV head h / (Hq/Hkv),
//   causal aligned bottom-right (key j visible to query i iff
//   j <= i + Sk - Sq), window (left, right) keeps
//   i + Sk - Sq - left <= j <= i + Sk - Sq + right (negative = unbounded),
//   a query with no visible key yields O = 0.
// Layout: q/o [B, S, H, D] and k/v [B, S, Hkv, D] with arbitrary batch/seq/
// head strides and a contiguous last dim (flash-attn's layout); the KV cache
// of the decode path is [B, Hkv, Lmax, D] through the same strides.
//
// Prefill kernel (D = 64 or 128): one wave = 32 queries of one head.
//  * S^T = K . Q^T with v_mfma_f32_32x32x16 (K tile from LDS as operand A,
//    the wave's Q kept in VGPRs as operand B), so every lane owns ONE query
//    and 32 of the 64 scores of a KV tile: the softmax max/sum is an in-lane
//    loop plus a single exchange with lane ^ 32.
//  * O^T += V^T . P^T: P never leaves registers. MFMA operands pair lane half
//    h and element j with a K index; choosing key(c, h, j) =
//    16c + 8(j/4) + 4h + j%4 for the c-th 16-key step makes the score
//    registers of S^T exactly the B operand, and the A operand two 8-byte LDS
//    reads of a transposed V tile.
//  * K and V^T tiles are staged through XOR-swizzled LDS (16-byte chunks for
//    K, 8-byte 4-key slots for V^T), double-buffered, one barrier per tile.
//  * A block is 4 waves over the query heads that share one KV head (GQA),
//    so a K/V tile in LDS serves up to 4 heads; causal/window tiles outside
//    the block's band are skipped, masks are evaluated only on band edges,
//    and the heaviest (latest) query tiles are dispatched first.
// Decode kernel: a block = (batch, KV head, key chunk); each 16-lane DPP row
// (D/8 lanes) handles one key, all query heads of the group are scored
// against it, online softmax per lane, then log-sum-exp merges across rows,
// waves (LDS) and chunks (a small merge kernel per (batch, KV head)).
#include "tpp_common.hpp"

#include <atomic>
#include <mutex>

namespace tpp {

struct AttnArgs {
  const void *q, *k, *v;
  void *o;
  int64_t q_sb, q_ss, q_sh;
  int64_t k_sb, k_ss, k_sh;
  int64_t v_sb, v_ss, v_sh;
  int64_t o_sb, o_ss, o_sh;
  int B, Sq, Sk, Hq, Hkv;
  float scale_log2; // softmax scale * log2(e)
  int left, right;  // window, -1 = unbounded; causal => right = 0
};

// Optional fused decode prologue: the new token's raw QKV projection, QK
// RMSNorm weights and RoPE tables. When set, the decode kernel normalises and
// rotates q itself and appends the new key/value to the cache.
struct DecodeFuse {
  const void *qkv; // [B, (Hq + 2 Hkv) * D]
  const void *qw, *kw;
  const void *cos, *sin;
  int cs_dtype, ctx;
  float eps;
};

// Output projection + residual add folded into the decode attention (the
// OP instantiation): residual[B, E] <- T(residual + T(T(o) W^T)).
struct DecodeOproj {
  const void *w; // [E, Hq * D] (nn.Linear layout)
  void *resid;   // [B, E]
  int *ctr;      // counter region (XCD arrival / departure, chunk counters, error flag)
  float *part;   // [8][B][E] fp32 per-XCD partial projections
  int E;
};

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kKvTile = 64;
// 32-query groups per prefill wave (each K / V^T fragment read from LDS feeds
// every group's products). Two groups need more than the 512 VGPRs of a wave
// at D = 128 and spill, so one group is used.
constexpr int kPrefillQG = 1;
// waves per prefill block: 8 = two per SIMD, so one wave's softmax (VALU)
// overlaps the other's MFMAs
constexpr int kPrefillWaves = 8;

template <typename T>
__device__ __forceinline__ f32x16 mfma32x32(typename VecT<T>::v8 a, typename VecT<T>::v8 b,
                                            f32x16 c) {
  if constexpr (__is_same(T, bf16))
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// V tiles are stored row-major like K ([key][16-byte unit]) and read as
// MFMA operands with ds_read_b64_tr_b16, whose 16-lane groups return lane
// 4a+b the b-th 16-bit element of the words lanes a, a+4, a+8, a+12 point at:
// pointing lane a'+4c' at V[k0 + c'][d0 + 4a'] gives lane l of the group
// V[k0 + 0..3][d0 + l]. Unit u of key row r is stored at u ^ vswz(r): the
// 32 lanes one read cycle serves (4 keys x 32 columns) then hit distinct
// banks (D = 128: 256-byte rows, XOR 4*(r%4); D = 64: 128-byte rows, two
// per bank row, XOR 4*((r/2)%2)).
template <int D> __device__ __forceinline__ int vswz(int r) {
  if constexpr (D == 128) return 4 * (r & 3);
  else return 4 * ((r >> 1) & 1);
}

// K / V ring slots of the prefill kernel: tile t in slot (t - t_begin) % 3
constexpr int kPrefillSlots = 3;
template <typename T, int D> struct PrefillSmem {
  typedef typename VecT<T>::v8 V8;
  V8 k[kPrefillSlots][kKvTile * D / 8];  // [key][chunk ^ (key % (D/8))]
  V8 v[kPrefillSlots][kKvTile * D / 8];  // [key][chunk ^ vswz(key)]
};

template <typename T, int D, int QG, int NW>
__global__ __launch_bounds__(64 * NW) void attn_prefill_kernel(AttnArgs p, int hpb) {
  typedef typename VecT<T>::v8 V8;
  constexpr int CPR = D / 8; // 16-byte chunks per row
  constexpr int NT = D / 32; // 32-row MFMA tiles along D
  __shared__ PrefillSmem<T, D> sm;

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int h = lane >> 5, ql = lane & 31;
  const int G = p.Hq / p.Hkv;
  const int wph = NW / hpb;  // waves per head
  const int qt_len = wph * 32 * QG;
  const int nqt = (p.Sq + qt_len - 1) / qt_len;
  const int nhg = p.Hq / hpb;
  const int npair = p.B * nhg;
  const int nitems = npair * nqt;
  const int off = p.Sk - p.Sq;

  // Work items (query tile qt, batch x head-group pair) in a fixed order,
  // heavy (late) query tiles first; the block loops over its share of them.
  // When the pairs split evenly over the 8 XCDs (workgroups are dealt to
  // them round-robin, XCD = blockIdx % 8), an XCD runs only its own pairs,
  // so the K / V tiles its blocks share stay in its L2, and each of its S
  // blocks takes the XCD's items in boustrophedon order (rounds alternate
  // direction), which evens out the heavy and light tiles per block.
  const bool xcd_split = npair % 8 == 0 && gridDim.x % 8 == 0;
  auto next_item = [&](int &k, int &qt, int &rest) -> bool {
    if (xcd_split) {
      const int S = gridDim.x / 8, slot = blockIdx.x / 8, per = npair / 8, ni = nitems / 8;
      for (;; ++k) {
        if (k * S >= ni) return false;
        const int j = (k & 1) ? (k + 1) * S - 1 - slot : k * S + slot;
        if (j >= ni) continue;
        rest = (blockIdx.x % 8) * per + j % per;
        qt = nqt - 1 - j / per;
        return true;
      }
    }
    const int it = blockIdx.x + k * gridDim.x;
    if (it >= nitems) return false;
    qt = nqt - 1 - it / npair;
    rest = it % npair;
    return true;
  };
  // the item's state (set by setup)
  int b, hq, hk, q0, q_last, qw, t_begin, t_end;
  const T *qp, *kp, *vp;
  auto setup = [&](int qt, int rest) {
    b = rest / nhg;
    const int hg = rest % nhg;
    hq = hg * hpb + w / wph;
    hk = (hg * hpb) / G;
    q0 = qt * qt_len;
    q_last = (q0 + qt_len < p.Sq ? q0 + qt_len : p.Sq) - 1;
    qw = q0 + (w % wph) * 32 * QG; // first query of this wave
    // key band of the whole item
    int hi = p.Sk, lo = 0;
    if (p.right >= 0) {
      const int lim = q_last + off + p.right + 1;
      hi = lim < hi ? lim : hi;
    }
    if (p.left >= 0) {
      const int lim = q0 + off - p.left;
      lo = lim > 0 ? lim : 0;
    }
    t_begin = lo / kKvTile;
    t_end = hi > lo ? (hi + kKvTile - 1) / kKvTile : t_begin;
    qp = (const T *)p.q + (int64_t)b * p.q_sb + (int64_t)hq * p.q_sh;
    kp = (const T *)p.k + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh;
    vp = (const T *)p.v + (int64_t)b * p.v_sb + (int64_t)hk * p.v_sh;
  };

  V8 zero;
#pragma unroll
  for (int i = 0; i < 8; ++i) zero[i] = (T)0.0f;

  // QG groups of 32 queries per wave share every K / V fragment read from LDS
  V8 qf[QG][D / 16];
  auto load_q = [&] {
#pragma unroll
    for (int g = 0; g < QG; ++g) {
      const int qi = qw + g * 32 + ql;
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks)
        qf[g][ks] = qi < p.Sq
                        ? *reinterpret_cast<const V8 *>(qp + (int64_t)qi * p.q_ss + ks * 16 + h * 8)
                        : zero;
    }
  };
  int kitem = 0, qt0, rest0;
  if (!next_item(kitem, qt0, rest0)) return;
  setup(qt0, rest0);
  load_q();

  // The block's waves form two groups of NW/2 (waves w and w + NW/2 share a
  // SIMD). The leading group runs half an iteration ahead of the trailing
  // one, so on every SIMD one wave's MFMA phase (PV of tile t-1, then QK^T of
  // tile t) overlaps the other wave's softmax phase (VALU). Each iteration
  // has two workgroup barriers, one per phase change; the trailing group
  // passes one barrier before its first iteration, the leading group one
  // after its last.
  const bool lead = __builtin_amdgcn_readfirstlane(w) < NW / 2; // wave-uniform
  constexpr int NWL = NW / 2;

  // K and V tiles go HBM/L2 -> LDS by LDS-DMA (no staging registers): the
  // leading group fetches the K tiles, the trailing group the V tiles.
  // Instruction i of a group's wave wu fills 64 slots = 64/CPR keys; lane l
  // fetches the chunk that lands in its slot. The address is a wave-uniform
  // tile base plus a per-lane 32-bit byte offset fixed for the whole kernel
  // (the launch checks 64 rows fit in 2^31 bytes). Keys past Sk are clamped
  // to Sk-1 on the last tile (finite data; those scores are masked, so their
  // P is 0).
  constexpr int KPI = 64 / CPR;                 // keys per DMA instruction
  constexpr int KDMA = kKvTile / KPI / NWL;     // DMA instructions per wave per tile
  constexpr int NDMA = KDMA;                    // ... per wave per iteration
  const int wu = __builtin_amdgcn_readfirstlane(w) % NWL; // wave index within its group
  const int dkey = lane / CPR, dslot = lane % CPR;
  const int64_t dss = lead ? p.k_ss : p.v_ss; // row stride of this wave's tiles
  // Offsets of full tiles, and of the last tile when Sk is not a multiple of
  // the tile: its keys past Sk read key Sk-1 (the clamp computed here once,
  // not per tile)
  const int kb_last = ((p.Sk - 1) / kKvTile) * kKvTile;
  unsigned doff[KDMA], doffl[KDMA];
#pragma unroll
  for (int i = 0; i < KDMA; ++i) {
    const int key = (i * NWL + wu) * KPI + dkey;
    const int kk = min(key, p.Sk - 1 - kb_last);
    const int ch = lead ? dslot ^ (key & (CPR - 1)) : dslot ^ vswz<D>(key); // K / V swizzle
    doff[i] = (unsigned)((key * dss + ch * 8) * (int64_t)sizeof(T));
    doffl[i] = (unsigned)((kk * dss + ch * 8) * (int64_t)sizeof(T));
  }
  // DMA instruction i (< KDMA) of this wave's share of tile t (K tile for the
  // leading group, V tile for the trailing group) into ring slot `slot`
  auto dma = [&](int i, int t, int slot) {
    const int kb = t * kKvTile;
    const char *tb = (const char *)((lead ? kp : vp) + (int64_t)kb * dss);
    V8 *dst = lead ? sm.k[slot] : sm.v[slot];
    const int key0 = (i * NWL + wu) * KPI;
    const unsigned o = kb + kKvTile > p.Sk ? doffl[i] : doff[i];
    __builtin_amdgcn_global_load_lds((const void *)(tb + o),
                                     (__attribute__((address_space(3))) void *)&dst[key0 * CPR],
                                     16, 0, 0);
  };

  f32x16 o[QG][NT];                // reset at the start of every item
  float m_run[QG], l_run[QG];

  f32x16 s[QG][2];
  V8 pb[QG][4];

  // S^T = K Q^T for the K tile in slot buf. The K fragments of step ks + 2
  // are requested before the MFMAs of step ks (scheduling barriers keep the
  // compiler from pulling the reads back next to their use), so LDS latency
  // hides behind the matrix work. The reads are inline asm with explicit
  // waits, like the V reads (from plain LDS loads the compiler waited for
  // all outstanding reads every third step).
  auto qk = [&](int buf) {
    const unsigned kbase = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) char *)&sm.k[buf][0];
    // step ks, key row st * 32 + ql: the st = 1 row is 32 rows (32 * D * 2
    // bytes) after the st = 0 row, with the same swizzle
    auto kfrag = [&](int ks, V8 (&dst)[2]) {
      const unsigned a = kbase + (unsigned)((ql * CPR + ((ks * 2 + h) ^ (ql & (CPR - 1)))) * 16);
      dst[0] = lds_read_b128<0, V8>(a);
      dst[1] = lds_read_b128<32 * D * 2, V8>(a);
    };
    constexpr int KS = D / 16;
    V8 kr[3][2];
#pragma unroll
    for (int g = 0; g < QG; ++g)
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[g][st][r] = 0.f;
    kfrag(0, kr[0]);
    kfrag(1, kr[1]);
    static_for<KS>([&](auto kk) {
      constexpr int ks = decltype(kk)::value;
      if constexpr (ks + 2 < KS) kfrag(ks + 2, kr[(ks + 2) % 3]);
      // the reads of steps ks + 1, ks + 2 stay in flight
      lds_wait_tied<(ks + 2 < KS ? 2 : KS - 1 - ks) * 2>(kr[ks % 3]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int g = 0; g < QG; ++g) s[g][st] = mfma32x32<T>(kr[ks % 3][st], qf[g][ks], s[g][st]);
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // Online softmax on raw scores of tile t: the running max m is kept
  // unscaled and exp2(scale*log2e*(s - m)) is one FMA + v_exp_f32 per score
  // (scale > 0 preserves the max). Masking only on band edges.
  // issue(j) is called at evenly spaced points of the exponentials with
  // j = 0 .. NDMA-1 (the waves put their DMA instructions there: a burst of
  // them would stall issue on the vector-memory queue)
  auto softmax = [&](int t, auto &&issue) {
    const int kb = t * kKvTile;
    const bool edge = (p.right >= 0 && kb + kKvTile - 1 > q0 + off + p.right) ||
                      (p.left >= 0 && kb < q_last + off - p.left) || (kb + kKvTile > p.Sk);
    const float c2 = p.scale_log2;
#pragma unroll
    for (int g = 0; g < QG; ++g) {
      const int qi = qw + g * 32 + ql;
      float mt = -INFINITY;
      if (edge) {
        // score register (st, r) holds key kb + 4h + c, c = 32st + 8(r/4) + r%4;
        // it is kept iff lo <= key <= hi, i.e. c in [lo - jb, hi - jb] with
        // jb = kb + 4h. Per lane one 32-bit mask per st holds the kept c's;
        // each score then costs a bit extract (0 or -1) and a bit select,
        // with no VCC round trip
        const int qpos = qi + off;
        int hi = p.Sk - 1;
        if (p.right >= 0) hi = min(hi, qpos + p.right);
        const int lo = p.left >= 0 ? max(qpos - p.left, 0) : 0;
        const int jb = kb + h * 4;
        const int ca = max(lo - jb, 0), cb = min(hi - jb, 63); // kept c: [ca, cb] (empty if ca > cb)
        const unsigned ninf = __float_as_uint(-INFINITY);
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          const int l0 = max(ca - 32 * st, 0), h0 = min(cb - 32 * st, 31);
          const unsigned keep = l0 <= h0 ? ((2u << h0) - 1u) & ~((1u << l0) - 1u) : 0u;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const unsigned bm = (unsigned)__builtin_amdgcn_sbfe((int)keep, (r >> 2) * 8 + (r & 3), 1);
            s[g][st][r] = __uint_as_float((__float_as_uint(s[g][st][r]) & bm) | (ninf & ~bm));
          }
        }
      }
      // max and sum as trees (a 32-long dependent chain of VALU ops costs
      // its full latency per step); the max as chains of three for v_max3
      auto max3 = [](float a, float b, float c) { return fmaxf(fmaxf(a, b), c); };
      float m1[11];
#pragma unroll
      for (int i = 0; i < 10; ++i) {
        const int a = 3 * i, b = 3 * i + 1, c = 3 * i + 2;
        m1[i] = max3(s[g][a >> 4][a & 15], s[g][b >> 4][b & 15], s[g][c >> 4][c & 15]);
      }
      m1[10] = fmaxf(s[g][1][14], s[g][1][15]);
      const float m2a = max3(m1[0], m1[1], m1[2]), m2b = max3(m1[3], m1[4], m1[5]);
      const float m2c = max3(m1[6], m1[7], m1[8]), m2d = fmaxf(m1[9], m1[10]);
      mt = fmaxf(max3(m2a, m2b, m2c), m2d);
      {
        // the other half of the wave holds the other 4-key groups
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt),
                                                         false, false);
        mt = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      }
      // lazy rescale: the reference max m_run only moves when the tile max
      // exceeds it by more than 8 in the exp2 domain (or on the first finite
      // tile), so P <= 2^8 and O, l keep fp32 headroom; O / l is unchanged by
      // the choice of m_run, and the O rescale then runs on few tiles
      const bool move = (mt - m_run[g]) * c2 > 8.f; // false for NaN (both -inf)
      const float m_new = move ? mt : m_run[g];
      const float mc = m_new == -INFINITY ? 0.f : m_new * c2;
      const float alpha = move ? __builtin_amdgcn_exp2f(m_run[g] * c2 - mc) : 1.f;
      float ps[8];
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          constexpr int kStride = 32 / NDMA;
          if (g == 0 && (st * 16 + r) % kStride == 0) issue((st * 16 + r) / kStride);
          const float e = __builtin_amdgcn_exp2f(fmaf(s[g][st][r], c2, -mc));
          s[g][st][r] = e;
          // the first term of each partial sum starts it (0 + e == e)
          ps[r & 7] = (st == 0 && r < 8) ? e : ps[r & 7] + e;
        }
#pragma unroll
      for (int n = 4; n >= 1; n >>= 1)
#pragma unroll
        for (int i = 0; i < n; ++i) ps[i] += ps[i + n];
      l_run[g] = l_run[g] * alpha + ps[0];
      m_run[g] = m_new;
      if (__any(move)) {
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[g][tt][r] *= alpha;
      }
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) pb[g][c][j] = from_f32<T>(s[g][c >> 1][(c & 1) * 8 + j]);
    }
  };

  // O^T += V^T P^T for the V tile in slot buf: the A operand of 16-key step c
  // for lane half h holds keys 16c + 4h + 0..3 (first read) and
  // 16c + 8 + 4h + 0..3 (second), the key order of the score registers (P
  // stays the B operand unchanged). The V fragments of step c + 2 are
  // requested before the MFMAs of step c.
  //
  // Key rows 16c + kl and 16c + kl + 8 (kl = 4(grp/2) + c4 < 16) have the
  // swizzle of kl, so a lane's address for step c is its step-0 address plus
  // the constant 32cD bytes (+16D for the second read): one base register per
  // 32-column slab, the step in the instruction's offset.
  auto pv = [&](int buf) {
    typedef short s16x8 __attribute__((ext_vector_type(8)));
    constexpr int R = 2 * NT; // LDS reads per 16-key step
    const int grp = lane >> 4, a4 = lane & 3, c4 = (lane >> 2) & 3;
    const int kl = 4 * (grp >> 1) + c4;
    const unsigned vbase = (unsigned)(uintptr_t)(const __attribute__((address_space(3))) char *)&sm.v[buf][0];
    unsigned vb[NT];
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      const int d0 = tt * 32 + 16 * (grp & 1) + 4 * a4; // this lane's 4 columns
      vb[tt] = vbase + kl * D * 2 + (((d0 >> 3) ^ vswz<D>(kl)) << 4) + ((d0 & 7) << 1);
    }
    s16x4 vr[3][R];
    auto vfrag = [&](auto cc) {
      constexpr int c = decltype(cc)::value;
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) {
        vr[c % 3][2 * tt] = lds_read_tr16<c * 32 * D>(vb[tt]);
        vr[c % 3][2 * tt + 1] = lds_read_tr16<c * 32 * D + 16 * D>(vb[tt]);
      }
    };
    auto step = [&](auto cc) {
      constexpr int c = decltype(cc)::value;
      if constexpr (c + 2 < 4) vfrag(std::integral_constant<int, c + 2>{});
      // reads of the later steps already issued stay in flight (LDS reads
      // complete in order)
      constexpr int later = (c + 2 < 4 ? 2 : 3 - c) * R;
      lds_wait_tied<later>(vr[c % 3]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int tt = 0; tt < NT; ++tt) {
        const s16x8 r12 = __builtin_shufflevector(vr[c % 3][2 * tt], vr[c % 3][2 * tt + 1], 0, 1,
                                                  2, 3, 4, 5, 6, 7);
        const V8 a = __builtin_bit_cast(V8, r12);
#pragma unroll
        for (int g = 0; g < QG; ++g) o[g][tt] = mfma32x32<T>(a, pb[g][c], o[g][tt]);
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    vfrag(std::integral_constant<int, 0>{});
    vfrag(std::integral_constant<int, 1>{});
    static_for<4>(step);
  };

  // Slots: K tile t and V tile t live in slot (t - t_begin) % 3. Iteration t
  // is two intervals: (A) the leading group's MFMA phase (PV of V(t-1),
  // QK^T of K(t)) beside the trailing group's softmax of tile t-1, then (B)
  // the leading group's softmax of tile t beside the trailing group's MFMA
  // phase. Each group requests tiles during its softmax: the leading waves
  // K(t+2) in (B), into the slot of K(t-1), last read in iteration t-1, and
  // wait for K(t+1) at the end of it; the trailing waves V(t+1) in (A) of
  // iteration t+1, into the slot of V(t-2), and wait for it at the end of
  // their next MFMA phase. Every wait is before the barrier after which the
  // other group reads the tile. K(t_begin), K(t_begin+1) and V(t_begin) are
  // loaded up front.
  // barrier without the fence of __syncthreads (which would drain the DMA);
  // the empty asm keeps the compiler from moving LDS accesses across it
  auto bar = [] {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  // K(t_begin), K(t_begin + 1) (leading waves), V(t_begin) (trailing waves)
  // of the item, into slot 0, 1 and 0
  auto first_dma = [&] {
    if (t_begin < t_end) {
#pragma unroll
      for (int j = 0; j < NDMA; ++j) dma(j, t_begin, 0);
      if (lead && t_begin + 1 < t_end) {
#pragma unroll
        for (int j = 0; j < NDMA; ++j) dma(j, t_begin + 1, 1);
      }
    }
  };
  // Output staging, 32 rows x D per wave, apart from the K / V slots so the
  // next item's first tiles can land while this item's rows are written out
  typedef typename VecT<T>::v4 V4;
  constexpr int RBY = D * (int)sizeof(T), OCH = RBY / 16, ORPI = 64 / OCH; // row bytes, chunks, rows per pass
  __shared__ V8 stage_all[NW * 32 * OCH];
  char *const stg = reinterpret_cast<char *>(stage_all) + w * (32 * RBY);

  first_dma();
  for (;;) {
    __syncthreads(); // (its fence also drains the DMA and the q loads)
#pragma unroll
    for (int g = 0; g < QG; ++g) {
      m_run[g] = -INFINITY, l_run[g] = 0.f;
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[g][tt][r] = 0.f;
    }
    if (!lead) bar();
    int sc = 0; // slot of tile t
    for (int t = t_begin; t < t_end; ++t) {
      const int sp = sc == 0 ? kPrefillSlots - 1 : sc - 1; // slot of t-1 (and of t+2)
      const int sn = sc == kPrefillSlots - 1 ? 0 : sc + 1; // slot of t+1
      if (t > t_begin) pv(sp);
      qk(sc);
      if (!lead) __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0): V(t) landed
      bar();
      const bool k2 = t + 2 < t_end;
      // K(t+2) into the slot of t-1 (leading waves), V(t+1) into the slot of
      // t+1 (trailing waves)
      const int dt = lead ? (k2 ? t + 2 : -1) : (t + 1 < t_end ? t + 1 : -1);
      const int ds = lead ? sp : sn;
      softmax(t, [&](int j) {
        if (dt >= 0) dma(j, dt, ds);
      });
      if (lead) {
        // K(t+1) landed; K(t+2), issued just now, may stay in flight
        if (k2) __builtin_amdgcn_s_waitcnt((NDMA & 0xF) | ((NDMA >> 4) << 14) | (0x7 << 4) | (0xF << 8));
        else __builtin_amdgcn_s_waitcnt(0x0F70);
      }
      bar();
      sc = sn;
    }
    if (t_begin < t_end) pv(sc == 0 ? kPrefillSlots - 1 : sc - 1);
    if (lead) bar();

    // The item's output rows, then the next item: its q rows are requested
    // now (q is dead after the last QK^T), its first K / V tiles once every
    // wave is past its last PV (the barrier below), after the staging reads.
    const int oqw = qw;
    T *const orow = (T *)p.o + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh;
    int qt1 = 0, rest1 = 0;
    ++kitem;
    const bool more = next_item(kitem, qt1, rest1);
    if (more) {
      setup(qt1, rest1);
      load_q();
    }
    bar(); // every wave is done with the K / V slots

    // Epilogue: each wave stages its 32 x D output rows in LDS and reads
    // them back as whole 16-byte chunks, D / 8 lanes per output row (straight
    // from the accumulators each store would write 8 bytes into each of 32
    // rows: 4x the write requests).
#pragma unroll
    for (int g = 0; g < QG; ++g) {
      const float l = l_run[g] + __shfl_xor(l_run[g], 32, kWave);
      const float inv = l > 0.f ? 1.f / l : 0.f;
      // register 4rg..4rg+3 of tile tt: dims tt*32 + rg*8 + h*4 + 0..3 of query ql,
      // i.e. half h of 16-byte chunk tt*4 + rg of row ql (chunks XOR-swizzled by row)
#pragma unroll
      for (int tt = 0; tt < NT; ++tt)
#pragma unroll
        for (int rg = 0; rg < 4; ++rg) {
          V4 pk;
#pragma unroll
          for (int i = 0; i < 4; ++i) pk[i] = from_f32<T>(o[g][tt][rg * 4 + i] * inv);
          const int ch = (tt * 4 + rg) ^ (ql % OCH);
          *reinterpret_cast<V4 *>(stg + ql * RBY + ch * 16 + h * 8) = pk;
        }
      V8 ov[32 / ORPI];
#pragma unroll
      for (int r = 0; r < 32 / ORPI; ++r) {
        const int row = r * ORPI + lane / OCH, c = lane % OCH;
        ov[r] = *reinterpret_cast<const V8 *>(stg + row * RBY + ((c ^ (row % OCH)) * 16));
      }
      // the DMA goes out after the staging reads: an LDS read issued behind
      // an LDS-DMA waits for it
      if (g == QG - 1 && more) first_dma();
#pragma unroll
      for (int r = 0; r < 32 / ORPI; ++r) {
        const int row = r * ORPI + lane / OCH, c = lane % OCH;
        const int qi = oqw + g * 32 + row;
        if (qi < p.Sq) *reinterpret_cast<V8 *>(orow + (int64_t)qi * p.o_ss + c * 8) = ov[r];
      }
    }
    if (!more) break;
  }
}

// Generic prefill (any D <= 256, any alignment): one wave per (b, query,
// head), keys streamed one at a time with a wave reduction. Slow; exists so
// that every head size flash-attn accepts still runs on the GPU.
template <typename T>
__global__ __launch_bounds__(64) void attn_generic_kernel(AttnArgs p, int D) {
  const int lane = threadIdx.x;
  const int64_t id = blockIdx.x; // (b, qi, hq)
  const int hq = (int)(id % p.Hq);
  const int qi = (int)((id / p.Hq) % p.Sq);
  const int b = (int)(id / ((int64_t)p.Hq * p.Sq));
  const int hk = hq / (p.Hq / p.Hkv);
  const int off = p.Sk - p.Sq;
  const T *qp = (const T *)p.q + b * p.q_sb + (int64_t)qi * p.q_ss + hq * p.q_sh;
  const T *kp = (const T *)p.k + b * p.k_sb + hk * p.k_sh;
  const T *vp = (const T *)p.v + b * p.v_sb + hk * p.v_sh;
  float qv[4], acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    qv[i] = d < D ? to_f32(qp[d]) * p.scale_log2 : 0.f;
  }
  float m = -INFINITY, l = 0.f;
  for (int j = 0; j < p.Sk; ++j) {
    const int rel = j - (qi + off);
    if (p.right >= 0 && rel > p.right) break;
    if (p.left >= 0 && rel < -p.left) continue;
    float sdot = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = lane + 64 * i;
      if (d < D) sdot += qv[i] * to_f32(kp[(int64_t)j * p.k_ss + d]);
    }
    sdot = wave_sum(sdot);
    const float mn = fmaxf(m, sdot);
    const float a = exp2f(m - mn), e = exp2f(sdot - mn);
    l = l * a + e;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d = lane + 64 * i;
      acc[i] = acc[i] * a + (d < D ? e * to_f32(vp[(int64_t)j * p.v_ss + d]) : 0.f);
    }
    m = mn;
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
  T *op = (T *)p.o + b * p.o_sb + (int64_t)qi * p.o_ss + hq * p.o_sh;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int d = lane + 64 * i;
    if (d < D) op[d] = from_f32<T>(acc[i] * inv);
  }
}

// ---------------------------------------------------------------------------
// Decode: one query per sequence against keys [lo_b, L_b) of the cache.
// grid = (nsplit, Hkv, B), block = 256 (4 waves); G = Hq / Hkv <= 8.
// A wave takes KPW keys per pass (one per D/8-lane DPP row) and issues the
// K and V loads of kDecU passes before using any of them; the online
// softmax is updated once per batch of passes.
// ---------------------------------------------------------------------------
constexpr int kDecMaxG = 8;
constexpr int kDecU = 4; // key passes per load batch (two batches in flight)

constexpr int kDecMaxSplit = 256;
#ifndef TPP_DEC_INLINE_MERGE
#define TPP_DEC_INLINE_MERGE 1
#endif
constexpr bool kDecInlineMerge = TPP_DEC_INLINE_MERGE;
constexpr int64_t kDecCounterBytes = 65536; // counters region at the start of the workspace:
constexpr int64_t kDecOpCtrOffset = 32768;  // per-pair arrival counters below, the folded
                                            // projection's counters from here
#ifndef TPP_DEC_WAVES
#define TPP_DEC_WAVES 2048
#endif
constexpr int kDecWaves = TPP_DEC_WAVES; // split-KV target: waves per decode launch
#ifndef TPP_DEC_BIG_NW
#define TPP_DEC_BIG_NW 8
#endif
constexpr int kDecBigNW = TPP_DEC_BIG_NW; // waves per block when G <= 2

// RMSNorm (optional) + rotate-half RoPE of one head row held as 8 values per
// lane by LPK lanes (lane dp owns d = 8 dp .. 8 dp + 7), rounded to T at the
// same points as the unfused path (norm output, rotated output). The norm
// weights w and the table rows c, sn are passed in already loaded.
template <typename T, int LPK>
__device__ __forceinline__ void norm_rope_vals(float (&x)[8], bool norm, const float (&w)[8],
                                               float eps, const float (&c)[8],
                                               const float (&sn)[8], int dp) {
  constexpr int D = LPK * 8;
  if (norm) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
    ss = group_sum<LPK>(ss);
    const float inv = rsqrtf(ss / (float)D + eps);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = to_f32(from_f32<T>((x[j] * inv) * w[j]));
  }
  float pt[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) pt[j] = __shfl_xor(x[j], LPK / 2, kWave); // d +- D/2
  const float sgn = dp < LPK / 2 ? -1.f : 1.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) x[j] = to_f32(from_f32<T>(x[j] * c[j] + sgn * pt[j] * sn[j]));
}

// 8 RoPE table entries from 32 loaded bytes (fp32: lo then hi 16 bytes;
// fp16 / bf16: the low 16 bytes), the table type a tpp_dtype code. All three
// readings are formed and one selected, with no branch: a branch would let the
// compiler sink the load of `hi` into it, and a load under a branch makes
// every later wait a wait for all loads in flight.
__device__ __forceinline__ void cs_vals(u32x4 lo, u32x4 hi, int cs_dtype, float (&v)[8]) {
  const f16x8 h = __builtin_bit_cast(f16x8, lo);
  const bf16x8 bh = __builtin_bit_cast(bf16x8, lo);
  const bool f32 = cs_dtype == TPP_F32, f16t = cs_dtype == TPP_F16;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float a = __uint_as_float(i < 4 ? lo[i & 3] : hi[i & 3]);
    const float b16 = f16t ? (float)h[i] : (float)bh[i];
    v[i] = f32 ? a : b16;
  }
}

// Folded output projection (OP): one workgroup per CU, 8 XCDs x 32, the XCD
// of a workgroup = its KV head (Hkv = 8), so XCD x holds every split of every
// sequence for query heads x G .. x G + G - 1, i.e. the K slice
// [x G D, (x + 1) G D) of the projection. Its workgroup j owns output
// columns [32 j, 32 j + 32). Constants of that layout:
constexpr int kOpXcds = 8, kOpPerXcd = 32, kOpCols = 32;
constexpr unsigned kOpSpinLimit = 1u << 20;
// counter region (ints, each counter on its own 128-byte line) at
// kDecOpCtrOffset of the workspace: arrive[8], depart[8], chunk[32], err
constexpr int kOpArrive = 0, kOpDepart = 8 * 32, kOpChunk = 16 * 32, kOpErr = 48 * 32;
static_assert(kAttnOprojCtrOffset == (size_t)kDecOpCtrOffset &&
                  kAttnOprojErrOffset == (size_t)kDecOpCtrOffset + kOpErr * sizeof(int),
              "counter and flag offsets shared with ffn.hip");

template <typename T>
__device__ __forceinline__ f32x4 mfma16x32(typename VecT<T>::v8 a, typename VecT<T>::v8 b, f32x4 c) {
  if constexpr (__is_same(T, bf16))
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// End of the OP kernel, after this workgroup published its split partial:
//  1. XCD-local sync: the workgroup counts itself in and waits until all 32
//     workgroups of its XCD (every split of every sequence for the XCD's KV
//     head) have published; the partials then sit in this XCD's L2. The wait
//     is bounded: if the workgroups were not all resident it gives up, sets
//     the error flag and the output is wrong (flagged).
//  2. Every workgroup merges the splits of all B sequences for the XCD's G
//     heads into LDS (the attention output, rounded to T like the unfused
//     path's output tensor), and workgroup j < B also stores sequence j's
//     rows to the output tensor.
//  3. Partial projection of output columns [32 j, 32 j + 32) over the XCD's
//     K slice with v_mfma_f32_16x16x32 (batch rows padded to 16), written
//     through to memory as fp32.
//  4. An agent-scope counter per column chunk finds the chunk's last XCD,
//     which sums the 8 partials in XCD order (fixed: bit-reproducible) and
//     updates the residual: T(residual + T(sum)).
template <typename T, int D, int G, int NW, int MG>
__device__ __forceinline__ void attn_decode_oproj_tail(const AttnArgs &p, const float *__restrict__ ws_o,
                                                       int nsplit, const DecodeOproj &op,
                                                       const T *s_w, T *s_o, f32x4 (*s_red)[64]) {
  typedef typename VecT<T>::v8 V8;
  constexpr int KO = G * D, UPR = KO / 8;
  const int lane = lane_id(), w = __builtin_amdgcn_readfirstlane(wave_id());
  const int x = blockIdx.x % kOpXcds, jb = blockIdx.x / kOpXcds;
  const int B = p.B, E = op.E;
  int *arrive = op.ctr + kOpArrive + x * 32;
  int *depart = op.ctr + kOpDepart + x * 32;
  int *chunkc = op.ctr + kOpChunk + jb * 32;
  int *err = op.ctr + kOpErr;
  T *resid = (T *)op.resid;
  __shared__ int s_last;
  // residual values of this workgroup's column chunk (used if it is the
  // chunk's last XCD), requested before the waits below
  const int e = threadIdx.x; // blockDim.x == 512 >= 16 * 32
  const int rb = e / kOpCols < B ? e / kOpCols : 0;
  const T rres = resid[(int64_t)rb * E + kOpCols * jb + e % kOpCols];

  // ---- 1. XCD-local sync (the partial stores and the weight DMA are done:
  // vmcnt(0); the counter lives in this XCD's L2, polled with an atomic add
  // of 0 from an asm move so the compiler keeps it an atomic)
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    unsigned n = 0;
    int zero;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zero));
    while (__hip_atomic_fetch_add(arrive, zero, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < kOpPerXcd) {
      if (++n > kOpSpinLimit) {
        __hip_atomic_fetch_or(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    // the XCD's last workgroup past the wait resets both counters
    if (__hip_atomic_fetch_add(depart, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
        kOpPerXcd - 1) {
      __hip_atomic_store(arrive, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(depart, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();

  // ---- 2. merge the splits: item = (batch row, head, 4 columns); rows past
  // B are zero (MFMA padding). Each split slot is D outputs, m, l, padding;
  // the splits are read in groups of MG (nsplit = 32 / B is a multiple), all
  // loads of a group before any use: one L2 round trip per group.
  for (int it = threadIdx.x; it < 16 * G * (D / 4); it += 64 * NW) {
    const int d4 = it % (D / 4), gi = (it / (D / 4)) % G, bb = it / (D / 4 * G);
    float r[4] = {0.f, 0.f, 0.f, 0.f};
    if (bb < B) {
      const float *sl = ws_o + ((int64_t)bb * p.Hq + x * G + gi) * nsplit * (D + 32);
      float mu = -INFINITY, ls = 0.f, os[4] = {0.f, 0.f, 0.f, 0.f};
      for (int s0 = 0; s0 < nsplit; s0 += MG) {
        float mv[MG], lv[MG];
        f32x4 ov[MG];
#pragma unroll
        for (int jj = 0; jj < MG; ++jj) {
          const float *q = sl + (int64_t)(s0 + jj) * (D + 32);
          const float2 ml = *reinterpret_cast<const float2 *>(q + D);
          mv[jj] = ml.x;
          lv[jj] = ml.y;
          ov[jj] = *reinterpret_cast<const f32x4 *>(q + 4 * d4);
        }
        float mx = mu;
#pragma unroll
        for (int jj = 0; jj < MG; ++jj) mx = fmaxf(mx, mv[jj]);
        const float mn = mx == -INFINITY ? 0.f : mx;
        const float a = mu == -INFINITY ? 0.f : exp2f(mu - mn);
        ls *= a;
#pragma unroll
        for (int c = 0; c < 4; ++c) os[c] *= a;
#pragma unroll
        for (int jj = 0; jj < MG; ++jj) {
          const float wgt = exp2f(mv[jj] - mn);
          ls += wgt * lv[jj];
#pragma unroll
          for (int c = 0; c < 4; ++c) os[c] += wgt * ov[jj][c];
        }
        mu = mx;
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) r[c] = ls > 0.f ? os[c] / ls : 0.f;
    }
    T tv[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) tv[c] = from_f32<T>(r[c]);
    T *so = s_o + bb * (KO + 8) + gi * D + 4 * d4;
#pragma unroll
    for (int c = 0; c < 4; ++c) so[c] = tv[c];
    if (bb < B && bb == jb) {
      T *o = (T *)p.o + (int64_t)bb * p.o_sb + (int64_t)(x * G + gi) * p.o_sh + 4 * d4;
#pragma unroll
      for (int c = 0; c < 4; ++c) o[c] = tv[c];
    }
  }
  __syncthreads();

  // ---- 3. partial projection: waves 0-3 output columns 32 j .. + 15,
  // waves 4-7 the next 16; wave w & 3 takes K steps (w & 3) G .. + G - 1 of 32
  const int t = w >> 2;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int ks = (w & 3) * G + i;
    const int gu = ks * 4 + (lane >> 4);          // 16-byte unit of K
    const int wr = 16 * t + (lane & 15);          // weight row of the tile
    const V8 a = *reinterpret_cast<const V8 *>(s_o + (lane & 15) * (KO + 8) + gu * 8);
    const V8 bw = *reinterpret_cast<const V8 *>(s_w + wr * KO + (gu ^ (wr & (UPR - 1))) * 8);
    acc = mfma16x32<T>(a, bw, acc);
  }
  s_red[w][lane] = acc;
  __syncthreads();
  if ((w & 3) == 0) {
    f32x4 sum = s_red[w][lane];
#pragma unroll
    for (int i = 1; i < 4; ++i) sum += s_red[w + i][lane];
    // D layout: lane -> column lane & 15, batch rows 4 (lane >> 4) + i
    const int n = kOpCols * jb + 16 * t + (lane & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = 4 * (lane >> 4) + i;
      if (b < B)
        __hip_atomic_store(op.part + ((int64_t)x * B + b) * E + n, sum[i], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // ---- 4. partial written through (vmcnt(0)); count this XCD in for the chunk
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(chunkc, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = old == kOpXcds - 1;
    if (old == kOpXcds - 1) __hip_atomic_store(chunkc, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last || e >= B * kOpCols) return;
  const int b = e / kOpCols, n = kOpCols * jb + e % kOpCols;
  float v[kOpXcds];
#pragma unroll
  for (int xx = 0; xx < kOpXcds; ++xx)
    v[xx] = __hip_atomic_load(op.part + ((int64_t)xx * B + b) * E + n, __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
  float sum = 0.f;
#pragma unroll
  for (int xx = 0; xx < kOpXcds; ++xx) sum += v[xx];
  resid[(int64_t)b * E + n] = from_f32<T>(to_f32(rres) + to_f32(from_f32<T>(sum)));
}

template <typename T, int D, int G, int NW, bool OP = false>
__global__ __launch_bounds__(64 * NW) void attn_decode_kernel(AttnArgs p, const int *__restrict__ seqlens,
                                                              int fixed_len, float *__restrict__ ws_o,
                                                              float *__restrict__ ws_ml, int chunk,
                                                              int nsplit, DecodeFuse fz,
                                                              int *__restrict__ counters,
                                                              DecodeOproj op) {
  typedef typename VecT<T>::v8 V8;
  constexpr int LPK = D / 8;        // lanes per key
  constexpr int KPW = kWave / LPK;  // keys per wave pass
  constexpr int U = kDecU;
  __shared__ float red_m[NW][G], red_l[NW][G];
  __shared__ float red_o[NW][G][D];
  // OP: the workgroup's [32 x G D] projection weight tile (LDS-DMA at kernel
  // start, 16-byte units of a row XOR-swizzled by the row), the merged
  // attention output of the XCD's heads for 16 (padded) batch rows, and the
  // cross-wave reduction of the projection
  constexpr int KO = G * D;        // projection K slice of an XCD
  constexpr int UPR = KO / 8;      // 16-byte units per weight row
  __shared__ __attribute__((aligned(16))) T s_w[OP ? kOpCols * KO : 8];
  __shared__ __attribute__((aligned(16))) T s_o[OP ? 16 * (KO + 8) : 8];
  __shared__ f32x4 s_red[OP ? NW : 1][64];
  static_assert(!OP || (D == 128 && NW == 8 && G <= 2), "folded projection: D 128, 8 waves, G <= 2");

  // w through readfirstlane: the compiler then knows it (and every key index
  // derived from it) is wave-uniform, so the key loop's exits are scalar
  // branches rather than exec-mask updates with per-lane live-out copies
  const int lane = lane_id(), w = __builtin_amdgcn_readfirstlane(wave_id());
  const int row = lane / LPK, dp = lane % LPK;
  int split = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  if (counters) {
    // one-dimensional grid; workgroups are dealt to the 8 XCDs round-robin
    // (XCD = blockIdx % 8): all splits of a (batch, KV head) pair share an
    // XCD, so their partials meet in that XCD's L2
    const int xcd = blockIdx.x % 8, slot = blockIdx.x / 8;
    const int pair = (slot / nsplit) * 8 + xcd;
    split = slot % nsplit;
    hk = pair % p.Hkv;
    b = pair / p.Hkv;
  }
  const T *kp = (const T *)p.k + (int64_t)b * p.k_sb + (int64_t)hk * p.k_sh + dp * 8;
  const T *vp = (const T *)p.v + (int64_t)b * p.v_sb + (int64_t)hk * p.v_sh + dp * 8;
  // K/V rows of one batch of keys base + u*NW*KPW + row (u < U), each key
  // clamped to `last`: past the keys a block scores they read a finite cache
  // row whose scores compute_batch masks. Every batch is issued
  // unconditionally: with no load under a branch the compiler's count of
  // loads in flight stays exact, so scoring batch i waits for batch i only (a
  // conditional load makes it wait for everything in flight).
  constexpr int STRIDE = NW * KPW * U; // keys per block-wide batch
  auto load_batch = [&](int base, int last, V8 (&kr)[U], V8 (&vr)[U]) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int key0 = base + u * NW * KPW + row;
      const int key = key0 < last ? key0 : last;
      kr[u] = ld_nt(reinterpret_cast<const V8 *>(kp + (int64_t)key * p.k_ss));
      vr[u] = ld_nt(reinterpret_cast<const V8 *>(vp + (int64_t)key * p.v_ss));
    }
  };
  // The first two batches of the chunk go out before the sequence length is
  // known (their keys depend on the block alone; clamped to the cache), so
  // that round trip overlaps the first K/V loads. Three register sets: while
  // one batch is scored the next two are in flight.
  const int first = split * chunk + w * KPW;
  V8 k0[U], v0[U], k1[U], v1[U], k2[U], v2[U];
  load_batch(first, p.Sk - 1, k0, v0);
  load_batch(first + STRIDE, p.Sk - 1, k1, v1);
  if constexpr (OP) {
    // the projection weight tile W[32 j .. 32 j + 31][x G D .. + G D) by
    // LDS-DMA (1 KB per wave instruction). Issued before the prologue loads,
    // whose first use waits for every load in flight anyway, so the compiler's
    // counted waits of the key loop are not disturbed by it.
    const int jb = blockIdx.x / kOpXcds;
    const T *wsrc = (const T *)op.w + (int64_t)(kOpCols * jb) * (p.Hq * D) + (int64_t)hk * KO;
    constexpr int NQ = kOpCols * KO * (int)sizeof(T) / (NW * 1024); // instructions per wave
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int unit = (w * NQ + q) * 64 + lane; // LDS 16-byte unit
      const int r = unit / UPR, lu = unit % UPR;
      const int gu = lu ^ (r & (UPR - 1));       // global unit stored at LDS unit lu
      __builtin_amdgcn_global_load_lds(
          (const void *)(wsrc + (int64_t)r * (p.Hq * D) + gu * 8),
          (__attribute__((address_space(3))) void *)(s_w + (w * NQ + q) * 64 * 8), 16, 0, 0);
    }
  }

  const int Lraw = seqlens ? seqlens[b] : fixed_len;
  const int L = Lraw < p.Sk ? (Lraw > 0 ? Lraw : 0) : p.Sk; // never read past the cache
  int lo = 0;
  if (p.left >= 0) lo = L - 1 - p.left > 0 ? L - 1 - p.left : 0;
  int k_begin = split * chunk, k_end = k_begin + chunk;
  k_begin = k_begin > lo ? k_begin : lo;
  k_end = k_end < L ? k_end : L;
  // fused prologue: position L-1 is the new token; this block attends to it
  // from registers (if it falls in its chunk) and the cache loop stops before it
  const bool fused = fz.qkv != nullptr;
  const int pnew = L - 1;
  const bool own_new = fused && Lraw <= p.Sk && pnew >= k_begin && pnew < k_end;
  if (fused && k_end > pnew) k_end = pnew;
  const T *qkv_row = fused ? (const T *)fz.qkv + (int64_t)b * (p.Hq + 2 * p.Hkv) * D : nullptr;

  // Every load the prologue needs goes out next, unconditionally (an absent
  // operand reads a valid row instead, never used): the q rows of the group,
  // and when fused the norm weights, the RoPE rows at the new position and
  // the new token's K/V row. One memory round trip then covers all of them
  // and the first K/V batches, where a load under a branch, or a load whose
  // address depends on an earlier one, costs a round trip each.
  const T *qbase = fused ? qkv_row + (int64_t)hk * G * D
                         : (const T *)p.q + (int64_t)b * p.q_sb + (int64_t)(hk * G) * p.q_sh;
  const int64_t qstep = fused ? (int64_t)D : p.q_sh;
  V8 q_raw[G];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) q_raw[gi] = *reinterpret_cast<const V8 *>(qbase + gi * qstep + dp * 8);
  const T *anyrow = qbase + dp * 8;
  const T *qw_src = fz.qw ? (const T *)fz.qw + dp * 8 : anyrow;
  const T *kw_src = fz.kw ? (const T *)fz.kw + dp * 8 : anyrow;
  const V8 qw_raw = *reinterpret_cast<const V8 *>(qw_src);
  const V8 kw_raw = *reinterpret_cast<const V8 *>(kw_src);
  const int pr = fused ? (pnew < 0 ? 0 : (pnew < fz.ctx ? pnew : fz.ctx - 1)) : 0;
  const int64_t cs_es = fz.cs_dtype == TPP_F32 ? 4 : 2;
  const char *c_src = fused ? (const char *)fz.cos + ((int64_t)pr * D + dp * 8) * cs_es
                            : (const char *)anyrow;
  const char *s_src = fused ? (const char *)fz.sin + ((int64_t)pr * D + dp * 8) * cs_es
                            : (const char *)anyrow;
  const int64_t cs_hi = fused && cs_es == 4 ? 16 : 0;
  const u32x4 c_lo = *reinterpret_cast<const u32x4 *>(c_src);
  const u32x4 c_hi = *reinterpret_cast<const u32x4 *>(c_src + cs_hi);
  const u32x4 s_lo = *reinterpret_cast<const u32x4 *>(s_src);
  const u32x4 s_hi = *reinterpret_cast<const u32x4 *>(s_src + cs_hi);
  const V8 knew_raw =
      *reinterpret_cast<const V8 *>(fused ? qkv_row + (int64_t)(p.Hq + hk) * D + dp * 8 : anyrow);
  const V8 vnew_raw = *reinterpret_cast<const V8 *>(
      fused ? qkv_row + (int64_t)(p.Hq + p.Hkv + hk) * D + dp * 8 : anyrow);

  float c[8], sn[8];
  cs_vals(c_lo, c_hi, fz.cs_dtype, c);
  cs_vals(s_lo, s_hi, fz.cs_dtype, sn);
  // q rounded to T after the fused QK-norm and RoPE, as the unfused path
  // stores it in its q tensor; scores by v_dot2 on T pairs accumulated in
  // fp32, scaled after the row reduction
  V8 qh[G];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    float qv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) qv[j] = to_f32(q_raw[gi][j]);
    if (fused) {
      float wq[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) wq[j] = to_f32(qw_raw[j]);
      norm_rope_vals<T, LPK>(qv, fz.qw != nullptr, wq, fz.eps, c, sn, dp);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) qh[gi][j] = from_f32<T>(qv[j]);
  }
  const float qscale = p.scale_log2;
  // the new token's K (normalised, rotated) and V, computed here by every
  // wave and pinned (empty asm uses): left to the block that appends them
  // they would keep their loads in flight across the whole key loop, and the
  // registers the loop reuses would make every iteration wait for all loads
  float kf[8], vf[8];
  {
    float wk[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      kf[j] = to_f32(knew_raw[j]);
      vf[j] = to_f32(vnew_raw[j]);
      wk[j] = to_f32(kw_raw[j]);
    }
    norm_rope_vals<T, LPK>(kf, fz.kw != nullptr, wk, fz.eps, c, sn, dp);
#pragma unroll
    for (int j = 0; j < 8; ++j) asm volatile("" ::"v"(kf[j]), "v"(vf[j]));
  }
  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    m[gi] = -INFINITY;
    l[gi] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[gi][j] = 0.f;
  }
  auto compute_batch = [&](int base, const V8 (&kr)[U], const V8 (&vr)[U]) {
    float sc[U][G];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool ok = (unsigned)(base + u * NW * KPW + row - k_begin) < (unsigned)(k_end - k_begin);
#pragma unroll
      for (int gi = 0; gi < G; ++gi) {
        float sdot = dot8<T>(qh[gi], kr[u], 0.f);
        sdot += dpp_f32<kDppQuadXor1>(sdot);
        sdot += dpp_f32<kDppQuadXor2>(sdot);
        if constexpr (LPK >= 8) sdot += dpp_f32<kDppRowHalfMirror>(sdot);
        if constexpr (LPK >= 16) sdot += dpp_f32<kDppRowMirror>(sdot);
        sc[u][gi] = ok ? sdot * qscale : -INFINITY;
      }
    }
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      float mb = m[gi];
#pragma unroll
      for (int u = 0; u < U; ++u) mb = fmaxf(mb, sc[u][gi]);
      const float mu = mb == -INFINITY ? 0.f : mb;
      const float alpha = exp2f(m[gi] - mu);
      l[gi] *= alpha;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[gi][j] *= alpha;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float e = exp2f(sc[u][gi] - mu);
        l[gi] += e;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[gi][j] += e * to_f32(vr[u][j]);
      }
      m[gi] = mb;
    }
  };
  // Whole triples of batches in the loop (a single exit: with a break after
  // every batch the compiler merges the exits into one latch, whose state
  // then has a batch in flight, and waits for everything at the loop head),
  // the last one or two batches after it. Batches past the chunk that a
  // triple loads are clamped rows and never scored.
  // this wave's keys: first + i*STRIDE + u*NW*KPW + row, scored iff in
  // [k_begin, k_end) (a window can start inside the chunk)
  const int k_last = k_end > 0 ? k_end - 1 : 0;
  int nbat = k_begin < k_end && first < k_end ? (k_end - first + STRIDE - 1) / STRIDE : 0;
  int base = first;
  for (; nbat >= 3; nbat -= 3, base += 3 * STRIDE) {
    asm volatile("" ::: "memory");
    load_batch(base + 2 * STRIDE, k_last, k2, v2);
    asm volatile("" ::: "memory");
    compute_batch(base, k0, v0);
    asm volatile("" ::: "memory");
    load_batch(base + 3 * STRIDE, k_last, k0, v0);
    asm volatile("" ::: "memory");
    compute_batch(base + STRIDE, k1, v1);
    asm volatile("" ::: "memory");
    load_batch(base + 4 * STRIDE, k_last, k1, v1);
    asm volatile("" ::: "memory");
    compute_batch(base + 2 * STRIDE, k2, v2);
  }
  if (nbat >= 1) compute_batch(base, k0, v0);
  if (nbat >= 2) compute_batch(base + STRIDE, k1, v1);
  if (own_new && w == 0) {
    // the new key/value (normalised and rotated in the prologue): append both
    // to the cache (row 0 lanes) and fold the key into row 0's online softmax
    if (row == 0) {
      store8((T *)kp + (int64_t)pnew * p.k_ss, kf);
      store8((T *)vp + (int64_t)pnew * p.v_ss, vf);
    }
    V8 kh; // the key as the cache holds it
#pragma unroll
    for (int j = 0; j < 8; ++j) kh[j] = from_f32<T>(kf[j]);
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      const float sdot = group_sum<LPK>(dot8<T>(qh[gi], kh, 0.f)) * qscale;
      if (row == 0) {
        const float mn = fmaxf(m[gi], sdot);
        const float a = exp2f(m[gi] - mn), e = exp2f(sdot - mn);
        l[gi] = l[gi] * a + e;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[gi][j] = acc[gi][j] * a + e * to_f32(from_f32<T>(vf[j]));
        m[gi] = mn;
      }
    }
  }
  // merge the KPW key rows of the wave (lanes with equal dp): at distance
  // SH = LPK .. 32 every lane gets its own and its partner's (m, l, acc) as an
  // unordered pair (v_permlane16/32_swap, or a row rotation by 8), and
  // combines them symmetrically, so both lanes of a pair get the same value
#pragma unroll
  for (int gi = 0; gi < G; ++gi) {
    auto merge_at = [&](auto pair_of) {
      float ma, mb, la, lb;
      pair_of(m[gi], ma, mb);
      pair_of(l[gi], la, lb);
      const float mn = fmaxf(ma, mb);
      const float mu = mn == -INFINITY ? 0.f : mn;
      const float a = exp2f(ma - mu), c = exp2f(mb - mu);
      l[gi] = la * a + lb * c;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        float xa, xb;
        pair_of(acc[gi][j], xa, xb);
        acc[gi][j] = xa * a + xb * c;
      }
      m[gi] = mn;
    };
    if constexpr (LPK <= 8)
      merge_at([](float x, float &a, float &b) { a = x, b = dpp_f32<kDppRowRor8>(x); });
    if constexpr (LPK <= 16)
      merge_at([](float x, float &a, float &b) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
        a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
      });
    merge_at([](float x, float &a, float &b) {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
      a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
    });
    if (row == 0) {
#pragma unroll
      for (int j = 0; j < 8; ++j) red_o[w][gi][dp * 8 + j] = acc[gi][j];
      if (dp == 0) {
        red_m[w][gi] = m[gi];
        red_l[w][gi] = l[gi];
      }
    }
  }
  __syncthreads();
  // merge the NW waves: thread -> (gi, d); write this chunk's partial, or the
  // final output when the whole key range is one chunk
  for (int idx = threadIdx.x; idx < G * D; idx += blockDim.x) {
    const int gi = idx / D, d = idx % D;
    float mx = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) mx = fmaxf(mx, red_m[ww][gi]);
    const float mu = mx == -INFINITY ? 0.f : mx;
    float ls = 0.f, os = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) {
      const float c = exp2f(red_m[ww][gi] - mu);
      ls += red_l[ww][gi] * c;
      os += red_o[ww][gi][d] * c;
    }
    const int hq = hk * G + gi;
    if (nsplit == 1) {
      T *op = (T *)p.o + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh;
      op[d] = from_f32<T>(ls > 0.f ? os / ls : 0.f);
      continue;
    }
    const int64_t slot = ((int64_t)b * p.Hq + hq) * nsplit + split;
    if (counters) {
      // slot = D partial outputs, m, l, padding: whole 128-byte lines
      float *sl = ws_o + slot * (D + 32);
      sl[d] = os;
      if (d == 0) sl[D] = mx, sl[D + 1] = ls;
    } else {
      ws_o[slot * D + d] = os;
      if (d == 0) ws_ml[slot * 2] = mx, ws_ml[slot * 2 + 1] = ls;
    }
  }
  if constexpr (OP) {
    // nsplit = 32 / B: 2, 4 or a multiple of 8
    if (nsplit == 2) attn_decode_oproj_tail<T, D, G, NW, 2>(p, ws_o, nsplit, op, s_w, s_o, s_red);
    else if (nsplit == 4) attn_decode_oproj_tail<T, D, G, NW, 4>(p, ws_o, nsplit, op, s_w, s_o, s_red);
    else attn_decode_oproj_tail<T, D, G, NW, 8>(p, ws_o, nsplit, op, s_w, s_o, s_red);
    return;
  }
  if (!counters || nsplit == 1) return;
  // The last block of the pair to finish merges the splits. Every thread
  // waits for its partial stores to reach L2 (an explicit vmcnt(0): the
  // workgroup-scope fence of __syncthreads does not wait for global stores),
  // then one thread counts the block in with an atomic in L2; the block that
  // takes the count to nsplit reads the other partials from the same L2.
  // Each partial slot is whole 128-byte lines written by one block only, and
  // a block reads other blocks' slots only here, so this CU's L1 (clean at
  // kernel start) holds no stale copy of them.
  __shared__ int s_last;
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70); // vmcnt(0)
  __syncthreads();
  const int pair = b * p.Hkv + hk;
  if (threadIdx.x == 0) {
    // agent scope: the counter is shared by workgroups (of one XCD); the
    // atomic is performed in that XCD's L2 either way
    const int old = __hip_atomic_fetch_add(&counters[pair], 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    s_last = old == nsplit - 1;
    if (old == nsplit - 1) // leave the counter at 0 for the next launch
      __hip_atomic_store(&counters[pair], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  for (int idx = threadIdx.x; idx < G * D; idx += blockDim.x) {
    const int gi = idx / D, d = idx % D;
    const float *sl = ws_o + (((int64_t)b * p.Hq + hk * G + gi) * nsplit) * (D + 32);
    // the partials in groups of MG splits: a group's loads all go out before
    // any is used (indices past nsplit read the last split and weigh 0), one
    // L2 round trip per group instead of two per split; groups after the
    // first rescale the running sums (online softmax)
    constexpr int MG = 8;
    float mu = -INFINITY, ls = 0.f, os = 0.f;
    for (int s0 = 0; s0 < nsplit; s0 += MG) {
      float mv[MG], lv[MG], ov[MG];
#pragma unroll
      for (int j = 0; j < MG; ++j) {
        const int sp = s0 + j < nsplit ? s0 + j : nsplit - 1;
        const float *q = sl + (int64_t)sp * (D + 32);
        mv[j] = q[D];
        lv[j] = q[D + 1];
        ov[j] = q[d];
      }
      float mx = mu;
#pragma unroll
      for (int j = 0; j < MG; ++j)
        if (s0 + j < nsplit) mx = fmaxf(mx, mv[j]);
      const float mn = mx == -INFINITY ? 0.f : mx;
      const float a = mu == -INFINITY ? 0.f : exp2f(mu - mn);
      ls *= a;
      os *= a;
#pragma unroll
      for (int j = 0; j < MG; ++j) {
        const float wgt = s0 + j < nsplit ? exp2f(mv[j] - mn) : 0.f;
        ls += wgt * lv[j];
        os += wgt * ov[j];
      }
      mu = mx;
    }
    T *op = (T *)p.o + (int64_t)b * p.o_sb + (int64_t)(hk * G + gi) * p.o_sh;
    op[d] = from_f32<T>(ls > 0.f ? os / ls : 0.f);
  }
}

// Merge the chunk partials of one (batch, KV head): grid (Hkv, B), 256
// threads, G query heads. A separate launch on purpose: publishing partials
// across blocks inside one kernel needs device-scope release/acquire fences,
// which on MI355X write back / invalidate the XCD's L2 (the 8 XCD L2s are not
// coherent) and cost far more than a kernel boundary.
template <typename T, int D, int G>
__global__ __launch_bounds__(G * D) void attn_decode_merge_kernel(AttnArgs p,
                                                                  const float *__restrict__ ws_o,
                                                                  const float *__restrict__ ws_ml,
                                                                  int nsplit) {
  constexpr int PRE = 16; // partial outputs prefetched per thread
  __shared__ float s_w[G][kDecMaxSplit], s_l[G][kDecMaxSplit], s_inv[G];
  const int hk = blockIdx.x, b = blockIdx.y, lane = lane_id(), w = wave_id();
  const int gi = threadIdx.x / D, d = threadIdx.x % D;
  const int64_t s0 = ((int64_t)b * p.Hq + hk * G) * nsplit; // slot of (gi = 0, split 0)
  // this thread's partial outputs do not depend on the weights: load first
  const float *po = ws_o + (s0 + (int64_t)gi * nsplit) * D + d;
  float pre[PRE];
#pragma unroll
  for (int j = 0; j < PRE; ++j) pre[j] = j < nsplit ? po[(int64_t)j * D] : 0.f;
  for (int idx = threadIdx.x; idx < G * nsplit; idx += blockDim.x) {
    const int g2 = idx / nsplit, sp = idx % nsplit;
    const float *ml = ws_ml + (s0 + (int64_t)g2 * nsplit + sp) * 2;
    s_w[g2][sp] = ml[0];
    s_l[g2][sp] = ml[1];
  }
  __syncthreads();
  const int nwave = blockDim.x / kWave;
  for (int g2 = w; g2 < G; g2 += nwave) { // one wave per query head
    float mx = -INFINITY;
    for (int sp = lane; sp < nsplit; sp += kWave) mx = fmaxf(mx, s_w[g2][sp]);
#pragma unroll
    for (int sh = 1; sh < kWave; sh <<= 1) mx = fmaxf(mx, __shfl_xor(mx, sh, kWave));
    const float mu = mx == -INFINITY ? 0.f : mx;
    float ls = 0.f;
    for (int sp = lane; sp < nsplit; sp += kWave) {
      const float wgt = exp2f(s_w[g2][sp] - mu);
      s_w[g2][sp] = wgt;
      ls += wgt * s_l[g2][sp];
    }
    ls = wave_sum(ls);
    if (lane == 0) s_inv[g2] = ls > 0.f ? 1.f / ls : 0.f;
  }
  __syncthreads();
  float os = 0.f;
#pragma unroll
  for (int j = 0; j < PRE; ++j) os += j < nsplit ? s_w[gi][j] * pre[j] : 0.f;
  for (int sp = PRE; sp < nsplit; ++sp) os += s_w[gi][sp] * po[(int64_t)sp * D];
  T *op = (T *)p.o + (int64_t)b * p.o_sb + (int64_t)(hk * G + gi) * p.o_sh;
  op[d] = from_f32<T>(os * s_inv[gi]);
}

static int check_attn(const char *name, const AttnArgs &a, int64_t D) {
  if (!a.q || !a.k || !a.v || !a.o) return set_error(TPP_E_INVALID, "%s: null pointer", name);
  if (a.B < 0 || a.Sq < 0 || a.Sk < 0 || a.Hq <= 0 || a.Hkv <= 0 || D <= 0)
    return set_error(TPP_E_INVALID, "%s: invalid shapes", name);
  if (a.Hq % a.Hkv != 0)
    return set_error(TPP_E_INVALID, "%s: Hq (%d) must be a multiple of Hkv (%d)", name, a.Hq,
                     a.Hkv);
  if (D > 256) return set_error(TPP_E_UNSUPPORTED, "%s: head_dim %lld > 256", name, (long long)D);
  return TPP_OK;
}

static bool strides16(const AttnArgs &a) {
  auto al = [](int64_t s) { return s % 8 == 0; };
  return aligned16(a.q) && aligned16(a.k) && aligned16(a.v) && aligned16(a.o) && al(a.q_sb) &&
         al(a.q_ss) && al(a.q_sh) && al(a.k_sb) && al(a.k_ss) && al(a.k_sh) && al(a.v_sb) &&
         al(a.v_ss) && al(a.v_sh) && al(a.o_sb) && al(a.o_ss) && al(a.o_sh);
}

template <typename T>
static int launch_prefill(const AttnArgs &a, int64_t D, hipStream_t st, const char *name) {
  if (a.B == 0 || a.Sq == 0) return TPP_OK;
  const int G = a.Hq / a.Hkv;
  // the tiled kernel addresses a 64-row K / V tile with 32-bit byte offsets
  const bool rows_fit = a.k_ss >= 0 && a.v_ss >= 0 && (int64_t)kKvTile * a.k_ss * 2 < (1LL << 31) &&
                        (int64_t)kKvTile * a.v_ss * 2 < (1LL << 31);
  if ((D == 64 || D == 128) && strides16(a) && rows_fit) {
    const int hpb = (G % 4 == 0) ? 4 : (G % 2 == 0) ? 2 : 1;
    constexpr int QG = kPrefillQG;
    constexpr int NW = kPrefillWaves;
    const int qt_len = (NW / hpb) * 32 * QG;
    const int64_t items =
        (int64_t)a.B * (a.Hq / hpb) * ((a.Sq + qt_len - 1) / qt_len);
    if (items > 0x7fffffffLL) return set_error(TPP_E_UNSUPPORTED, "%s: too large", name);
    // one workgroup per CU loops over the work items (more items than CUs)
    const int cus = device_cu_count();
    const int64_t blocks = (cus > 0 && items > cus) ? cus : items;
    if (D == 128)
      attn_prefill_kernel<T, 128, QG, NW><<<dim3((unsigned)blocks), dim3(64 * NW), 0, st>>>(a, hpb);
    else
      attn_prefill_kernel<T, 64, QG, NW><<<dim3((unsigned)blocks), dim3(64 * NW), 0, st>>>(a, hpb);
  } else {
    const int64_t blocks = (int64_t)a.B * a.Sq * a.Hq;
    if (blocks > 0x7fffffffLL) return set_error(TPP_E_UNSUPPORTED, "%s: too large", name);
    attn_generic_kernel<T><<<dim3((unsigned)blocks), dim3(64), 0, st>>>(a, (int)D);
  }
  return check_launch(name);
}

struct DecodePlan {
  int chunk, nsplit, nw;
  bool inline_merge; // the last split block merges (no merge kernel)
  size_t o_bytes, ml_bytes, ws_bytes;
};

// Partial-slot layout of a split plan: in-kernel merge (one padded slot per
// split) or merge kernel (D outputs, then m/l pairs; the counter region stays
// reserved and untouched, so a workspace shared with in-kernel-merge calls
// keeps its counters at zero).
static void use_merge_layout(DecodePlan &pl, size_t slots, int64_t D, bool inline_merge) {
  pl.inline_merge = inline_merge;
  if (inline_merge) {
    pl.o_bytes = slots * (size_t)(D + 32) * sizeof(float);
    pl.ml_bytes = 0;
  } else {
    pl.o_bytes = slots * (size_t)D * sizeof(float);
    pl.ml_bytes = slots * 2 * sizeof(float);
  }
}

// Split-KV plan: about one 8-wave block per CU, each (batch, KV head) pair's
// keys split into whole load batches; one split needs no merge kernel.
static DecodePlan plan_decode(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t Lmax) {
  DecodePlan pl{};
  const int64_t kpw = kWave / (D / 8);
  const int64_t pairs = B * Hkv > 0 ? B * Hkv : 1;
  pl.nw = (Hkv > 0 && Hq / Hkv <= 2) ? kDecBigNW : 4; // more query heads per KV head: more VGPRs
  const int64_t batch = pl.nw * kpw * kDecU; // keys per block-wide load batch
  // about kDecWaves waves, in whole load batches (a block's loop runs whole
  // batches: a chunk of part batches costs the same time with keys masked,
  // measured 18.3 -> 20.0 us at the model shape with 32-key granularity)
  int64_t want = (kDecWaves / pl.nw + pairs - 1) / pairs;
  int64_t chunk = (Lmax + want - 1) / want;
  chunk = ((chunk + batch - 1) / batch) * batch;
  if (chunk < batch) chunk = batch;
  while ((Lmax + chunk - 1) / chunk > kDecMaxSplit) chunk += batch;
  pl.chunk = (int)chunk;
  pl.nsplit = (int)((Lmax + chunk - 1) / chunk);
  if (pl.nsplit < 1) pl.nsplit = 1;
  pl.inline_merge = pl.nsplit > 1 && pairs % 8 == 0 && pairs * (int64_t)sizeof(int) <= kDecOpCtrOffset &&
                    kDecInlineMerge;
  const size_t slots = (size_t)(B * Hq * pl.nsplit);
  if (pl.nsplit == 1) {
    pl.o_bytes = pl.ml_bytes = 0;
    pl.ws_bytes = 16;
  } else {
    // The size is the in-kernel merge layout's whatever the mode, so a call
    // that falls back to the merge kernel (placement check below) fits too.
    // One arrival counter per (batch, KV head) pair in a fixed region at the
    // start (calls of every shape and mode keep partials out of it), then
    // slots of D partial outputs + m + l padded to whole 128-byte lines.
    pl.ws_bytes = kDecCounterBytes + slots * (size_t)(D + 32) * sizeof(float);
    use_merge_layout(pl, slots, D, pl.inline_merge);
  }
  return pl;
}

template <typename T, int D, int G>
static void launch_decode_g(const AttnArgs &a, dim3 grid, const int *seqlens, int L, float *ws_o,
                            float *ws_ml, int *counters, const DecodePlan &pl, const DecodeFuse &fz,
                            hipStream_t st) {
  const DecodeOproj none{};
  if constexpr (G <= 2) {
    if (pl.nw == kDecBigNW) {
      attn_decode_kernel<T, D, G, kDecBigNW><<<grid, dim3(64 * kDecBigNW), 0, st>>>(
          a, seqlens, L, ws_o, ws_ml, pl.chunk, pl.nsplit, fz, counters, none);
    } else {
      attn_decode_kernel<T, D, G, 4><<<grid, dim3(256), 0, st>>>(a, seqlens, L, ws_o, ws_ml,
                                                                 pl.chunk, pl.nsplit, fz, counters,
                                                                 none);
    }
  } else
    attn_decode_kernel<T, D, G, 4><<<grid, dim3(256), 0, st>>>(a, seqlens, L, ws_o, ws_ml,
                                                               pl.chunk, pl.nsplit, fz, counters,
                                                               none);
  if (pl.nsplit > 1 && !counters)
    attn_decode_merge_kernel<T, D, G><<<dim3(a.Hkv, a.B), dim3(G * D), 0, st>>>(
        a, ws_o, ws_ml, pl.nsplit);
}

template <typename T, int D>
static void launch_decode_d(const AttnArgs &a, int G, dim3 grid, const int *seqlens, int L,
                            float *ws_o, float *ws_ml, int *counters, const DecodePlan &pl,
                            const DecodeFuse &fz, hipStream_t st) {
  switch (G) {
  case 1: launch_decode_g<T, D, 1>(a, grid, seqlens, L, ws_o, ws_ml, counters, pl, fz, st); break;
  case 2: launch_decode_g<T, D, 2>(a, grid, seqlens, L, ws_o, ws_ml, counters, pl, fz, st); break;
  case 3: launch_decode_g<T, D, 3>(a, grid, seqlens, L, ws_o, ws_ml, counters, pl, fz, st); break;
  case 4: launch_decode_g<T, D, 4>(a, grid, seqlens, L, ws_o, ws_ml, counters, pl, fz, st); break;
  case 5: launch_decode_g<T, D, 5>(a, grid, seqlens, L, ws_o, ws_ml, counters, pl, fz, st); break;
  case 6: launch_decode_g<T, D, 6>(a, grid, seqlens, L, ws_o, ws_ml, counters, pl, fz, st); break;
  case 7: launch_decode_g<T, D, 7>(a, grid, seqlens, L, ws_o, ws_ml, counters, pl, fz, st); break;
  default: launch_decode_g<T, D, 8>(a, grid, seqlens, L, ws_o, ws_ml, counters, pl, fz, st); break;
  }
}

template <typename T>
static void launch_decode(const AttnArgs &a, int64_t D, int G, dim3 grid, const int *seqlens,
                          int L, float *ws_o, float *ws_ml, int *counters, const DecodePlan &pl,
                          const DecodeFuse &fz, hipStream_t st) {
  if (D == 128) launch_decode_d<T, 128>(a, G, grid, seqlens, L, ws_o, ws_ml, counters, pl, fz, st);
  else launch_decode_d<T, 64>(a, G, grid, seqlens, L, ws_o, ws_ml, counters, pl, fz, st);
}

} // namespace tpp

using namespace tpp;

static AttnArgs make_args(const void *q, const void *k, const void *v, void *o,
                          const int64_t *qs, const int64_t *ks, const int64_t *vs,
                          const int64_t *os, int64_t B, int64_t Sq, int64_t Sk, int64_t Hq,
                          int64_t Hkv, int64_t D, float scale, int left, int right) {
  AttnArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.q_sb = qs[0], a.q_ss = qs[1], a.q_sh = qs[2];
  a.k_sb = ks[0], a.k_ss = ks[1], a.k_sh = ks[2];
  a.v_sb = vs[0], a.v_ss = vs[1], a.v_sh = vs[2];
  a.o_sb = os[0], a.o_ss = os[1], a.o_sh = os[2];
  a.B = (int)B, a.Sq = (int)Sq, a.Sk = (int)Sk, a.Hq = (int)Hq, a.Hkv = (int)Hkv;
  const float sc = scale > 0.f ? scale : 1.0f / sqrtf((float)D);
  a.scale_log2 = sc * kLog2e;
  a.left = left;
  a.right = right;
  return a;
}

extern "C" int tpp_attn_prefill(const void *q, const void *k, const void *v, void *o,
                                const int64_t *q_strides, const int64_t *k_strides,
                                const int64_t *v_strides, const int64_t *o_strides, int64_t B,
                                int64_t Sq, int64_t Sk, int64_t Hq, int64_t Hkv, int64_t D,
                                float softmax_scale, int causal, int window_left,
                                int window_right, int dtype, void *stream) {
  const char *name = "tpp_attn_prefill";
  if (!q_strides || !k_strides || !v_strides || !o_strides)
    return set_error(TPP_E_INVALID, "%s: null stride array", name);
  if (B > 0x7fffffff || Sq > 0x7fffffff || Sk > 0x7fffffff)
    return set_error(TPP_E_UNSUPPORTED, "%s: dimension too large", name);
  const int right = causal ? 0 : (window_right < 0 ? -1 : window_right);
  const int left = window_left < 0 ? -1 : window_left;
  AttnArgs a = make_args(q, k, v, o, q_strides, k_strides, v_strides, o_strides, B, Sq, Sk, Hq,
                         Hkv, D, softmax_scale, left, right);
  if (int e = check_attn(name, a, D)) return e;
  hipStream_t st = as_stream(stream);
  return TPP_DISPATCH_HALF(dtype, [&] { return launch_prefill<T>(a, D, st, name); });
}

extern "C" size_t tpp_attn_decode_workspace_size(int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                                 int64_t Lmax) {
  return plan_decode(B, Hq, Hkv, D, Lmax).ws_bytes;
}

static int decode_impl(const char *name, AttnArgs &a, int64_t D, int64_t Lmax,
                       const int32_t *seqlens, const DecodeFuse &fz, int dtype, void *workspace,
                       size_t ws_bytes, void *stream, bool may_probe = true) {
  if (int e = check_attn(name, a, D)) return e;
  if (a.B == 0) return TPP_OK;
  // the kernel reads cache row 0 even for empty sequences (clamped loads)
  if (Lmax < 1) return set_error(TPP_E_INVALID, "%s: the cache must hold at least one row", name);
  if (D != 64 && D != 128)
    return set_error(TPP_E_UNSUPPORTED, "%s: head_dim %lld not in {64, 128}", name, (long long)D);
  if (a.Hq / a.Hkv > kDecMaxG)
    return set_error(TPP_E_UNSUPPORTED, "%s: more than %d query heads per KV head", name,
                     kDecMaxG);
  if (!strides16(a)) return set_error(TPP_E_INVALID, "%s: 16-byte alignment required", name);
  DecodePlan pl = plan_decode(a.B, a.Hq, a.Hkv, D, Lmax);
  if (!workspace || ws_bytes < pl.ws_bytes || (uintptr_t)workspace % 128 != 0)
    return set_error(TPP_E_WORKSPACE, "%s: 128-byte aligned workspace of %zu bytes required",
                     name, pl.ws_bytes);
  hipStream_t st = as_stream(stream);
  if (pl.inline_merge && !xcd_grouping_holds(st, may_probe))
    use_merge_layout(pl, (size_t)a.B * a.Hq * pl.nsplit, D, false);
  int *counters = pl.inline_merge ? (int *)workspace : nullptr;
  float *ws_o = (float *)((char *)workspace + kDecCounterBytes);
  float *ws_ml = (float *)((char *)ws_o + pl.o_bytes);
  const dim3 grid = pl.inline_merge
                        ? dim3((unsigned)(pl.nsplit * a.Hkv * a.B))
                        : dim3((unsigned)pl.nsplit, (unsigned)a.Hkv, (unsigned)a.B);
  return TPP_DISPATCH_HALF(dtype, [&] {
    launch_decode<T>(a, D, a.Hq / a.Hkv, grid, seqlens, (int)Lmax, ws_o, ws_ml, counters, pl, fz,
                     st);
    return check_launch(name);
  });
}

extern "C" int tpp_attn_decode(const void *q, const void *k_cache, const void *v_cache, void *o,
                               const int64_t *q_strides, const int64_t *k_strides,
                               const int64_t *v_strides, const int64_t *o_strides,
                               const int32_t *seqlens, int64_t B, int64_t Hq, int64_t Hkv,
                               int64_t D, int64_t Lmax, float softmax_scale, int window_left,
                               int dtype, void *workspace, size_t ws_bytes, void *stream) {
  const char *name = "tpp_attn_decode";
  if (!q_strides || !k_strides || !v_strides || !o_strides)
    return set_error(TPP_E_INVALID, "%s: null stride array", name);
  if (B > 0xffff || Hkv > 0xffff || Lmax > 0x7fffffff)
    return set_error(TPP_E_UNSUPPORTED, "%s: dimension too large", name);
  AttnArgs a = make_args(q, k_cache, v_cache, o, q_strides, k_strides, v_strides, o_strides, B,
                         1, Lmax, Hq, Hkv, D, softmax_scale, window_left < 0 ? -1 : window_left,
                         0);
  DecodeFuse fz{};
  return decode_impl(name, a, D, Lmax, seqlens, fz, dtype, workspace, ws_bytes, stream);
}

// ---- allocation-free decode ------------------------------------------------
// tpp_attn_decode_noalloc runs the decode kernels on a file-scope device
// array instead of a caller workspace, for callers that cannot allocate. Each
// device holds its own copy of `scratch`; its address on a device comes from
// hipGetSymbolAddress at the first call with that device current (the host
// symbol itself is not a device address) and is kept per device. The first
// call also zeroes the arrival-counter region with a fill kernel on the
// caller's stream (every call leaves it at zero again). Calls on one device
// share the array: calls that overlap on one GPU race.
constexpr size_t kNoAllocScratchBytes = (size_t)4 << 20; // plans up to this many bytes
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
static void *g_scratch_ptr[64];
static std::mutex g_scratch_mu;

__global__ __launch_bounds__(256) void zero_words_kernel(int *__restrict__ p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0;
}

static int noalloc_scratch(const char *name, hipStream_t st, void **out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return set_error(TPP_E_LAUNCH, "%s: no current device", name);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      (void)hipGetLastError();
      return set_error(TPP_E_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed: %s", name,
                       hipGetErrorString(e));
    }
    constexpr int words = (int)(kDecCounterBytes / 4);
    zero_words_kernel<<<dim3((words + 255) / 256), dim3(256), 0, st>>>((int *)ptr, words);
    if (int rc = check_launch(name)) return rc;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return TPP_OK;
}

extern "C" int tpp_attn_decode_noalloc(const void *q, const void *k_cache, const void *v_cache,
                                       void *o, const int64_t *q_strides,
                                       const int64_t *k_strides, const int64_t *v_strides,
                                       const int64_t *o_strides, const int32_t *seqlens,
                                       int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                       int64_t Lmax, float softmax_scale, int window_left,
                                       int dtype, void *stream) {
  const char *name = "tpp_attn_decode_noalloc";
  if (!q_strides || !k_strides || !v_strides || !o_strides)
    return set_error(TPP_E_INVALID, "%s: null stride array", name);
  if (B > 0xffff || Hkv > 0xffff || Lmax > 0x7fffffff)
    return set_error(TPP_E_UNSUPPORTED, "%s: dimension too large", name);
  AttnArgs a = make_args(q, k_cache, v_cache, o, q_strides, k_strides, v_strides, o_strides, B,
                         1, Lmax, Hq, Hkv, D, softmax_scale, window_left < 0 ? -1 : window_left,
                         0);
  if (int e = check_attn(name, a, D)) return e;
  if (a.B == 0) return TPP_OK;
  const size_t need = plan_decode(B, Hq, Hkv, D, Lmax).ws_bytes;
  if (need > kNoAllocScratchBytes)
    return set_error(TPP_E_UNSUPPORTED,
                     "%s: this shape needs %zu bytes of scratch, more than the %zu-byte static "
                     "array (use tpp_attn_decode with a workspace)",
                     name, need, kNoAllocScratchBytes);
  void *ws = nullptr;
  if (int e = noalloc_scratch(name, as_stream(stream), &ws)) return e;
  DecodeFuse fz{};
  // no placement probe here (it reads back to the host): the in-kernel merge
  // is used once another decode call has verified the placement on this
  // device, the merge kernel until then
  return decode_impl(name, a, D, Lmax, seqlens, fz, dtype, ws, kNoAllocScratchBytes, stream,
                     false);
}

extern "C" int tpp_attn_decode_fused(const void *qkv, const void *q_norm_w, const void *k_norm_w,
                                     const void *cos, const void *sin, int64_t ctx, int cs_dtype,
                                     float eps, void *k_cache, void *v_cache, void *o,
                                     const int64_t *k_strides, const int64_t *v_strides,
                                     const int64_t *o_strides, const int32_t *seqlens, int64_t B,
                                     int64_t Hq, int64_t Hkv, int64_t D, int64_t Lmax,
                                     float softmax_scale, int window_left, int dtype,
                                     void *workspace, size_t ws_bytes, void *stream) {
  const char *name = "tpp_attn_decode_fused";
  if (!k_strides || !v_strides || !o_strides)
    return set_error(TPP_E_INVALID, "%s: null stride array", name);
  if (!qkv || !cos || !sin || !seqlens)
    return set_error(TPP_E_INVALID, "%s: qkv, cos, sin and seqlens are required", name);
  if (!aligned16(qkv) || !aligned16(cos) || !aligned16(sin) ||
      (q_norm_w && !aligned16(q_norm_w)) || (k_norm_w && !aligned16(k_norm_w)))
    return set_error(TPP_E_INVALID, "%s: 16-byte alignment required", name);
  if (cs_dtype != TPP_F16 && cs_dtype != TPP_BF16 && cs_dtype != TPP_F32)
    return set_error(TPP_E_UNSUPPORTED, "%s: cos/sin dtype", name);
  if (ctx <= 0 || ctx > 0x7fffffff) return set_error(TPP_E_INVALID, "%s: ctx", name);
  if (ctx < Lmax) // every cache position must have a table row (no clamping)
    return set_error(TPP_E_INVALID, "%s: cos/sin hold %lld positions, fewer than the cache length %lld",
                     name, (long long)ctx, (long long)Lmax);
  if (B > 0xffff || Hkv > 0xffff || Lmax > 0x7fffffff)
    return set_error(TPP_E_UNSUPPORTED, "%s: dimension too large", name);
  const int64_t qs[3] = {0, 0, 0};
  AttnArgs a = make_args(qkv, k_cache, v_cache, o, qs, k_strides, v_strides, o_strides, B, 1,
                         Lmax, Hq, Hkv, D, softmax_scale, window_left < 0 ? -1 : window_left, 0);
  DecodeFuse fz{qkv, q_norm_w, k_norm_w, cos, sin, cs_dtype, (int)ctx, eps};
  return decode_impl(name, a, D, Lmax, seqlens, fz, dtype, workspace, ws_bytes, stream);
}

// ---- decode attention + output projection + residual add -------------------
// The OP kernel's plan: one workgroup per CU (Hkv = 8 KV heads x B sequences
// x 32 / B splits = 256), splits in whole 128-key load batches (trailing
// splits may hold no key). Workspace: the counters region (the projection's
// counters at kDecOpCtrOffset), the split partial slots, then the fp32
// per-XCD partial projections [8][B][E].
static bool oproj_shape(int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t E) {
  return Hkv == kOpXcds && D == 128 && (Hq == 8 || Hq == 16) && E == kOpPerXcd * kOpCols &&
         (B == 1 || B == 2 || B == 4 || B == 8 || B == 16);
}

struct OprojPlan {
  int nsplit, chunk;
  size_t part_off, ws_bytes;
};

static OprojPlan plan_oproj(int64_t B, int64_t Hq, int64_t D, int64_t Lmax, int64_t E) {
  OprojPlan pl{};
  constexpr int64_t stride = kDecBigNW * (kWave / 16) * kDecU; // keys per block-wide batch (D 128)
  pl.nsplit = (int)(kOpPerXcd / B);
  int64_t chunk = (Lmax + pl.nsplit - 1) / pl.nsplit;
  chunk = (chunk + stride - 1) / stride * stride;
  pl.chunk = (int)chunk;
  pl.part_off = (size_t)kDecCounterBytes + (size_t)(B * Hq * pl.nsplit) * (size_t)(D + 32) * sizeof(float);
  pl.ws_bytes = pl.part_off + (size_t)kOpXcds * B * E * sizeof(float);
  return pl;
}

extern "C" size_t tpp_attn_decode_oproj_workspace_size(int64_t B, int64_t Hq, int64_t Hkv,
                                                       int64_t D, int64_t Lmax, int64_t E) {
  const size_t plain = plan_decode(B, Hq, Hkv, D, Lmax).ws_bytes;
  if (!oproj_shape(B, Hq, Hkv, D, E) || Lmax < 1) return plain;
  const size_t op = plan_oproj(B, Hq, D, Lmax, E).ws_bytes;
  return op > plain ? op : plain;
}

extern "C" int tpp_attn_decode_oproj(const void *qkv, const void *q_norm_w, const void *k_norm_w,
                                     const void *cos, const void *sin, int64_t ctx, int cs_dtype,
                                     float eps, void *k_cache, void *v_cache, void *o,
                                     const int64_t *k_strides, const int64_t *v_strides,
                                     const int32_t *seqlens, const void *w_o, void *residual,
                                     int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t Lmax,
                                     int64_t E, float softmax_scale, int window_left, int dtype,
                                     void *workspace, size_t ws_bytes, void *stream) {
  const char *name = "tpp_attn_decode_oproj";
  if (!w_o || !residual || !o) return set_error(TPP_E_INVALID, "%s: null pointer argument", name);
  if (!aligned16(w_o) || !aligned16(residual) || !aligned16(o))
    return set_error(TPP_E_INVALID, "%s: 16-byte alignment required", name);
  if (E <= 0 || B <= 0 || B > 16)
    return set_error(TPP_E_INVALID, "%s: need 1 <= B <= 16 and E > 0", name);
  const int64_t os[3] = {Hq * D, Hq * D, D}; // o: contiguous [B, 1, Hq, D]
  hipStream_t st = as_stream(stream);
  const size_t need = tpp_attn_decode_oproj_workspace_size(B, Hq, Hkv, D, Lmax, E);
  if (!workspace || ws_bytes < need || (uintptr_t)workspace % 128 != 0)
    return set_error(TPP_E_WORKSPACE, "%s: 128-byte aligned workspace of %zu bytes required", name,
                     need);
  const bool fold = oproj_shape(B, Hq, Hkv, D, E) && half_type(dtype) &&
                    device_cu_count() == kOpXcds * kOpPerXcd && xcd_grouping_holds(st, true);
  if (!fold) {
    // two launches: fused decode attention into o, then the projection GEMV
    // with the residual add
    if (int rc = tpp_attn_decode_fused(qkv, q_norm_w, k_norm_w, cos, sin, ctx, cs_dtype, eps,
                                       k_cache, v_cache, o, k_strides, v_strides, os, seqlens, B,
                                       Hq, Hkv, D, Lmax, softmax_scale, window_left, dtype,
                                       workspace, ws_bytes, stream))
      return rc;
    return tpp_gemv_fused(o, nullptr, 0.f, w_o, nullptr, residual, B, E, Hq * D, 0, dtype, stream);
  }
  if (!k_strides || !v_strides) return set_error(TPP_E_INVALID, "%s: null stride array", name);
  if (!qkv || !cos || !sin || !seqlens)
    return set_error(TPP_E_INVALID, "%s: qkv, cos, sin and seqlens are required", name);
  if (!aligned16(qkv) || !aligned16(cos) || !aligned16(sin) ||
      (q_norm_w && !aligned16(q_norm_w)) || (k_norm_w && !aligned16(k_norm_w)))
    return set_error(TPP_E_INVALID, "%s: 16-byte alignment required", name);
  if (cs_dtype != TPP_F16 && cs_dtype != TPP_BF16 && cs_dtype != TPP_F32)
    return set_error(TPP_E_UNSUPPORTED, "%s: cos/sin dtype", name);
  if (ctx < Lmax || ctx > 0x7fffffff)
    return set_error(TPP_E_INVALID, "%s: cos/sin hold %lld positions, fewer than the cache length %lld",
                     name, (long long)ctx, (long long)Lmax);
  if (Lmax < 1 || Lmax > 0x7fffffff) return set_error(TPP_E_INVALID, "%s: cache length", name);
  const int64_t qs[3] = {0, 0, 0};
  AttnArgs a = make_args(qkv, k_cache, v_cache, o, qs, k_strides, v_strides, os, B, 1, Lmax, Hq,
                         Hkv, D, softmax_scale, window_left < 0 ? -1 : window_left, 0);
  if (int rc = check_attn(name, a, D)) return rc;
  if (!strides16(a)) return set_error(TPP_E_INVALID, "%s: 16-byte alignment required", name);
  const OprojPlan pl = plan_oproj(B, Hq, D, Lmax, E);
  DecodeFuse fz{qkv, q_norm_w, k_norm_w, cos, sin, cs_dtype, (int)ctx, eps};
  char *ws = (char *)workspace;
  DecodeOproj op{w_o, residual, (int *)(ws + kDecOpCtrOffset), (float *)(ws + pl.part_off), (int)E};
  float *ws_o = (float *)(ws + kDecCounterBytes);
  const dim3 grid(kOpXcds * kOpPerXcd), block(64 * kDecBigNW);
  return TPP_DISPATCH_HALF(dtype, [&] {
    if (Hq == 16)
      attn_decode_kernel<T, 128, 2, kDecBigNW, true><<<grid, block, 0, st>>>(
          a, seqlens, (int)Lmax, ws_o, nullptr, pl.chunk, pl.nsplit, fz, (int *)ws, op);
    else
      attn_decode_kernel<T, 128, 1, kDecBigNW, true><<<grid, block, 0, st>>>(
          a, seqlens, (int)Lmax, ws_o, nullptr, pl.chunk, pl.nsplit, fz, (int *)ws, op);
    return check_launch(name);
  });
}

extern "C" int tpp_attn_decode_oproj_sync_errors(void *workspace, int *out, void *stream) {
  const char *name = "tpp_attn_decode_oproj_sync_errors";
  if (!workspace || !out) return set_error(TPP_E_INVALID, "%s: null pointer", name);
  hipStream_t st = as_stream(stream);
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return set_error(TPP_E_INVALID, "%s: not callable while the stream is being captured", name);
  }
  char *ctr = (char *)workspace + kDecOpCtrOffset;
  int flag = 0;
  if (hipMemcpyAsync(&flag, ctr + kOpErr * sizeof(int), sizeof(int), hipMemcpyDeviceToHost, st) !=
          hipSuccess ||
      hipStreamSynchronize(st) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(TPP_E_LAUNCH, "%s: copy failed", name);
  }
  // a launch that gave up leaves the counters in an unknown state: zero them
  if (flag && (hipMemsetAsync(ctr, 0, (kOpErr + 32) * sizeof(int), st) != hipSuccess ||
               hipStreamSynchronize(st) != hipSuccess)) {
    (void)hipGetLastError();
    return set_error(TPP_E_LAUNCH, "%s: clearing the counters failed", name);
  }
  *out = flag;
  return TPP_OK;
}
