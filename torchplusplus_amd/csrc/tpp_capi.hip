// Library-level C ABI: per-thread error message and version.
#include "tpp_common.hpp"

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

} // namespace tpp

extern "C" const char *tpp_last_error_string(void) { return tpp::g_err; }
extern "C" int tpp_version(void) { return (1 << 16) | 0; }
