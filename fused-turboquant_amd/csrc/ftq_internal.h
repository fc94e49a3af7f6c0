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
}  // namespace ftq

#define FTQ_REQUIRE(cond, msg)      \
  do {                              \
    if (!(cond)) {                  \
      ::ftq::set_error(msg);        \
      return FTQ_ERR_ARG;           \
    }                               \
  } while (0)
