// Status strings, version and the per-thread error message of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "common.h"

static thread_local char g_last_error[512] = "";

namespace qo {
std::atomic<unsigned> g_route_mask{0u};
thread_local hipError_t g_launch_error = hipSuccess;
}  // namespace qo

void qo_set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

extern "C" const char* qo_last_error(void) { return g_last_error; }

extern "C" const char* qo_version(void) { return "0.1.0"; }

extern "C" unsigned qo_set_kernel_routing(unsigned mask) {
  return qo::g_route_mask.exchange(mask & QO_ROUTE_ALL, std::memory_order_relaxed);
}

extern "C" const char* qo_status_string(int status) {
  switch (status) {
    case QO_OK: return "ok";
    case QO_ERR_NULL_POINTER: return "null pointer";
    case QO_ERR_SHAPE: return "invalid shape";
    case QO_ERR_DTYPE: return "unsupported dtype";
    case QO_ERR_ALIGNMENT: return "misaligned pointer or stride";
    case QO_ERR_UNSUPPORTED: return "unsupported configuration";
    case QO_ERR_LAUNCH: return "kernel launch failed";
    default: return "unknown status";
  }
}
