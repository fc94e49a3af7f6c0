// Slot geometry and value-dtype rounding shared by the vLLM v1 slot-format
// kernels (store and decode).
#pragma once

#include "ftq_device.h"

namespace ftq {

// Byte offsets of one (token, kv head) slot: [K codes mse][K norm f16]
// [V codes vdb][V scale f16][V min f16]; raw = the bytes that hold data
// (reference boundary_tq_config.py:66-81).
struct V1Geom {
  int mse, kps, vdb, raw;
};
__host__ __device__ constexpr V1Geom v1_geom(int d, int kb, int vb) {
  return V1Geom{d * kb / 8, d * kb / 8 + 2, d * vb / 8, d * kb / 8 + 2 + d * vb / 8 + 4};
}

// x rounded to the value dtype and back (the reference rounds the pre-rotated
// V to the value tensor's dtype, v1_backend.py:736-740)
template <int DT>
__device__ __forceinline__ float round_to_dtype(float x) {
  if constexpr (DT == BF16) return bf16_bits_to_f32(f32_to_bf16_bits(x));
  else if constexpr (DT == F16) return f16_bits_to_f32(f32_to_f16_bits(x));
  else return x;
}

}  // namespace ftq
