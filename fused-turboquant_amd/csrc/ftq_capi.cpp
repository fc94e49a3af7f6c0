// Error reporting and version query for the fused-turboquant C ABI.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>

#include "ftq_internal.h"

namespace {
thread_local char g_err[512] = "";
}

namespace ftq {
void set_error(const char* msg) {
  std::strncpy(g_err, msg, sizeof(g_err) - 1);
  g_err[sizeof(g_err) - 1] = 0;
}
int hip_status(hipError_t e) {
  if (e == hipSuccess) return FTQ_OK;
  std::snprintf(g_err, sizeof(g_err), "HIP error %d: %s", (int)e, hipGetErrorString(e));
  return (int)e;
}
}  // namespace ftq

extern "C" const char* ftq_last_error(void) { return g_err; }
extern "C" int ftq_version(void) { return FTQ_ABI_VERSION; }
