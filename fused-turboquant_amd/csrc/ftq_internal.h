// Host-side helpers shared by the C entry points: argument checks that set a
// thread-local error message and return FTQ_ERR_ARG, and HIP status mapping.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fused_tq.h"  // from include/ (on the -I path)

namespace ftq {
void set_error(const char* msg);
int hip_status(hipError_t e);
inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
inline bool aligned4(const void* p) { return ((uintptr_t)p & 3u) == 0; }

// Workgroups of 256 threads of kernel k that fit on the current device at
// once (512 if the runtime cannot tell): the grid of a kernel whose waves loop
// over the work.
template <typename K>
inline int resident_workgroups(K k) {
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, 256, 0) != hipSuccess || cus <= 0 ||
      per_cu <= 0)
    return 512;
  return cus * per_cu;
}
}  // namespace ftq

#define FTQ_REQUIRE(cond, msg)      \
  do {                              \
    if (!(cond)) {                  \
      ::ftq::set_error(msg);        \
      return FTQ_ERR_ARG;           \
    }                               \
  } while (0)
