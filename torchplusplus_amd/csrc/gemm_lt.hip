// Plain GEMMs with at least one 256x256 output tile per CU through hipBLASLt.
//
// The reference leaves its plain projections (the prefill q/k/v, output and
// down projections of FastQwen3, examples/LLM/fastqwen3.py:103-116) to
// nn.Linear, i.e. the vendor BLAS; only the GEMMs with a fused epilogue are
// its own kernels (csrc/activation/fused_gemm.cuh:143-170). This build does
// the same split where it measures faster: on MI355X hipBLASLt's persistent
// stream-K kernel (256x256 tiles, 4 waves, no workspace) runs the
// [16384 x 1024..3072] prefill projections 9-20% faster than the
// hand-written persistent MFMA kernel of gemm.hip (identical outputs on those
// shapes), while below one tile per CU (e.g. [2048 x 1024] . [3072 x
// 1024]^T, 96 tiles) the two are equal and the hand-written kernel is kept. Every fused
// epilogue (bias + activation, SwiGLU) stays on the hand-written kernels.
//
// Per device: one hipBLASLt handle and, per (dtype, M, N, K, lda, ldb, ldc),
// the matmul descriptor, the three layouts and the heuristic's first
// algorithm with a zero workspace limit (so no memory is allocated), built
// on first use. A shape whose heuristic returns nothing, or whose matmul
// call fails, is remembered and runs on the hand-written kernel. Nothing is
// created while the stream is being captured into a graph: an uncached shape
// met under capture runs on the hand-written kernel. At most kLtMaxPlans
// shapes are kept per device (M changes with every prompt length in
// serving); shapes past that run on the hand-written kernel, with no
// heuristic query on the host.
#include "tpp_common.hpp"

#include <hipblaslt/hipblaslt.h>

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>

namespace tpp {

namespace {

struct LtPlan {
  bool ok = false;
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

typedef std::tuple<int, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t> LtKey;

struct LtDevice {
  bool tried = false;
  hipblasLtHandle_t handle = nullptr;
  std::map<LtKey, LtPlan> plans;
};

constexpr int kLtMaxDevices = 64;
constexpr size_t kLtMaxPlans = 512;
std::mutex g_lt_mu;
LtDevice g_lt[kLtMaxDevices];

int lt_initial_enable() {
  const char *e = std::getenv("TPP_GEMM_VENDOR");
  return (e && e[0] == '0' && e[1] == '\0') ? 0 : 1;
}
std::atomic<int> g_lt_enable{lt_initial_enable()};
std::atomic<long long> g_lt_runs{0};

// Build the plan of one shape: W [N, K] row-major is hipBLASLt's A (a
// column-major K x N matrix, transposed), X [M, K] its B (column-major K x M),
// Y [M, N] row-major its D (column-major N x M): D = A^T . B.
LtPlan make_plan(hipblasLtHandle_t h, hipDataType dt, int64_t M, int64_t N, int64_t K,
                 int64_t ldx, int64_t ldw, int64_t ldy) {
  LtPlan p;
  if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) {
    p.desc = nullptr;
    return p;
  }
  const int32_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  bool good =
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) ==
          HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) ==
          HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatrixLayoutCreate(&p.la, dt, (uint64_t)K, (uint64_t)N, ldw) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatrixLayoutCreate(&p.lb, dt, (uint64_t)K, (uint64_t)M, ldx) == HIPBLAS_STATUS_SUCCESS &&
      hipblasLtMatrixLayoutCreate(&p.lc, dt, (uint64_t)N, (uint64_t)M, ldy) == HIPBLAS_STATUS_SUCCESS;
  if (good) {
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS) {
      const uint64_t ws = 0;
      hipblasLtMatmulHeuristicResult_t res[4];
      int nret = 0;
      if (hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                                sizeof(ws)) == HIPBLAS_STATUS_SUCCESS &&
          hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.la, p.lb, p.lc, p.lc, pref, 4, res, &nret) ==
              HIPBLAS_STATUS_SUCCESS) {
        for (int i = 0; i < nret; ++i) {
          if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize == 0) {
            p.algo = res[i].algo;
            p.ok = true;
            break;
          }
        }
      }
      hipblasLtMatmulPreferenceDestroy(pref);
    }
  }
  return p;
}

} // namespace

bool lt_gemm_wanted(int64_t M, int64_t N, int cus) {
  if (!g_lt_enable.load(std::memory_order_relaxed)) return false;
  const int64_t tiles = ((M + 255) / 256) * ((N + 255) / 256);
  return tiles >= (int64_t)cus;
}

// Y[M, N] = X[M, K] . W[N, K]^T in fp32 accumulation, T output. Returns true
// when hipBLASLt ran it; false leaves the GEMM to the caller.
bool lt_gemm(const void *X, int64_t ldx, const void *W, int64_t ldw, void *Y, int64_t ldy,
             int64_t M, int64_t N, int64_t K, bool bf16, hipStream_t st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kLtMaxDevices) return false;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cap) != hipSuccess) return false;
  const bool capturing = cap != hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> lock(g_lt_mu);
  LtDevice &d = g_lt[dev];
  if (!d.handle) {
    if (d.tried || capturing) return false;
    d.tried = true;
    if (hipblasLtCreate(&d.handle) != HIPBLAS_STATUS_SUCCESS) {
      d.handle = nullptr;
      return false;
    }
  }
  const LtKey key(bf16 ? 1 : 0, M, N, K, ldx, ldw, ldy);
  auto it = d.plans.find(key);
  if (it == d.plans.end()) {
    if (capturing || d.plans.size() >= kLtMaxPlans) return false;
    it = d.plans.emplace(key, make_plan(d.handle, bf16 ? HIP_R_16BF : HIP_R_16F, M, N, K, ldx, ldw, ldy))
             .first;
  }
  LtPlan &p = it->second;
  if (!p.ok) return false;
  const float alpha = 1.f, beta = 0.f;
  if (hipblasLtMatmul(d.handle, p.desc, &alpha, W, p.la, X, p.lb, &beta, Y, p.lc, Y, p.lc, &p.algo,
                      nullptr, 0, st) != HIPBLAS_STATUS_SUCCESS) {
    p.ok = false; // this shape runs on the hand-written kernel from now on
    return false;
  }
  g_lt_runs.fetch_add(1, std::memory_order_relaxed);
  return true;
}

} // namespace tpp

extern "C" int tpp_gemm_vendor(int enable) {
  if (enable < 0) return tpp::g_lt_enable.load();
  return tpp::g_lt_enable.exchange(enable ? 1 : 0);
}

extern "C" long long tpp_gemm_vendor_runs(void) { return tpp::g_lt_runs.load(); }
