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

// Bytes of a split-K workspace: the partial outputs [batch][heads][splits][d]
// plus the log-sum-exps [batch][heads][splits], float32; -1 for a negative
// count, a non-positive head_dim or split count, or a size past int64.
inline int64_t split_workspace_bytes(int batch, int heads, int d, int splits) {
  if (batch < 0 || heads < 0 || d <= 0 || splits <= 0) return -1;
  int64_t r = 0;
  if (__builtin_mul_overflow((int64_t)batch * heads, (int64_t)splits, &r) ||
      __builtin_mul_overflow(r, (int64_t)d + 1, &r) || __builtin_mul_overflow(r, (int64_t)4, &r))
    return -1;
  return r;
}

// Strides (bytes) of a [num_blocks][block_size][num_kv_heads][slot] cache:
// positive, each at least the span of the dimension inside it, and the whole
// cache's byte span within int64 (checked by division, so huge strides cannot
// overflow the products here or the kernels' offsets).
inline bool cache_strides_ok(int64_t num_blocks, int64_t s_blk, int64_t s_pos, int64_t s_head, int num_kv_heads,
                             int block_size) {
  return s_head > 0 && num_kv_heads > 0 && block_size > 0 && s_pos / num_kv_heads >= s_head &&
         s_blk / block_size >= s_pos && num_blocks >= 0 && num_blocks <= INT64_MAX / s_blk;
}

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
