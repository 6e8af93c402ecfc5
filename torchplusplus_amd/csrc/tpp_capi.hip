// Library-level C ABI: per-thread error message and version; per-device
// placement facts shared by the kernels that synchronise inside one XCD.
#include "tpp_common.hpp"

#include <atomic>
#include <mutex>

namespace tpp {

static thread_local char g_err[512] = {0};

int set_error(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(TPP_E_LAUNCH, "%s: kernel launch failed: %s", what,
                     hipGetErrorString(e));
  g_err[0] = 0;
  return TPP_OK;
}

// ---- workgroup placement ----------------------------------------------------
// Kernels that exchange data through one XCD's L2 (the decode attention's
// in-kernel split merge, the fused decode FFN) rely on workgroups with equal
// blockIdx % 8 running on one XCD. Once per device a probe launch records
// HW_REG_XCC_ID for 512 workgroups; if any workgroup's XCD differs from that
// of workgroup (id % 8), those kernels take their unfused paths on that
// device. The probe needs a synchronous read back, so it is skipped (answer
// "no", nothing cached) while the caller's stream is being captured, or when
// the caller may not synchronise (may_probe false).
constexpr int kXcdProbeBlocks = 512;
static __device__ int g_xcd_probe[kXcdProbeBlocks];
static std::atomic<int> g_xcd_state[64]; // 0 unknown, 1 holds, 2 does not hold
static std::atomic<int> g_cu_count[64];  // 0 unknown
static std::mutex g_xcd_mu;

__global__ __launch_bounds__(64) void xcd_probe_kernel(int *__restrict__ out) {
  unsigned v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  if (threadIdx.x == 0) out[blockIdx.x] = (int)(v & 0xfu);
}

bool xcd_grouping_holds(hipStream_t st, bool may_probe) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return false;
  }
  int s = g_xcd_state[dev].load(std::memory_order_acquire);
  if (s || !may_probe) return s == 1;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return false;
  }
  std::lock_guard<std::mutex> lock(g_xcd_mu);
  s = g_xcd_state[dev].load(std::memory_order_acquire);
  if (s) return s == 1;
  int *d = nullptr;
  int h[kXcdProbeBlocks];
  hipError_t e = hipGetSymbolAddress((void **)&d, HIP_SYMBOL(g_xcd_probe));
  if (e == hipSuccess) {
    xcd_probe_kernel<<<dim3(kXcdProbeBlocks), dim3(64), 0, st>>>(d);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpyAsync(h, d, sizeof(h), hipMemcpyDeviceToHost, st);
  if (e == hipSuccess) e = hipStreamSynchronize(st);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  bool ok = true;
  for (int i = 0; i < kXcdProbeBlocks; ++i) ok = ok && h[i] == h[i % 8];
  g_xcd_state[dev].store(ok ? 1 : 2, std::memory_order_release);
  return ok;
}

int device_cu_count() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return 0;
  }
  int n = g_cu_count[dev].load(std::memory_order_acquire);
  if (n) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  g_cu_count[dev].store(n, std::memory_order_release);
  return n;
}

} // namespace tpp

extern "C" int tpp_prepare_device(void *stream, int *xcd_local, int *cu_count) {
  using namespace tpp;
  const char *name = "tpp_prepare_device";
  hipStream_t st = (hipStream_t)stream;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return set_error(TPP_E_INVALID, "%s: hipStreamIsCapturing failed", name);
  }
  if (cs != hipStreamCaptureStatusNone)
    return set_error(TPP_E_INVALID, "%s: the stream is being captured; call it before the capture",
                     name);
  const int cus = device_cu_count();
  if (cus <= 0) return set_error(TPP_E_LAUNCH, "%s: no current HIP device", name);
  const bool ok = xcd_grouping_holds(st, true);
  if (xcd_local) *xcd_local = ok ? 1 : 0;
  if (cu_count) *cu_count = cus;
  g_err[0] = 0;
  return TPP_OK;
}

extern "C" const char *tpp_last_error_string(void) { return tpp::g_err; }
extern "C" int tpp_version(void) { return (1 << 16) | 0; }
