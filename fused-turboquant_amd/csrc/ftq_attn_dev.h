// Device helpers shared by the decode-attention kernels (gfx950 MFMA operand
// types, packed-code field extraction, cross-lane reductions).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ftq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

union Op8 {
  uint32_t u[4];
  half8 h;
};

template <int NDW>
__device__ __forceinline__ void load_dwords(const uint8_t* p, uint32_t (&w)[NDW]) {
  const uint32_t* q = reinterpret_cast<const uint32_t*>(p);
#pragma unroll
  for (int i = 0; i < NDW; ++i) w[i] = q[i];
}

// entry_bytes * bits [P, P+W) of a little-endian multi-dword value: the byte
// offset of a table entry (P, W compile-time after unrolling)
template <int SH, int N>
__device__ __forceinline__ uint32_t field_off(const uint32_t (&w)[N], int P, int W) {
  const uint32_t m = ((1u << W) - 1u) << SH;
  if (P >= SH) {
    const int Q = P - SH, i = Q >> 5, o = Q & 31;
    uint32_t v = w[i] >> o;
    if (o + W + SH > 32 && i + 1 < N) v |= w[i + 1] << (32 - o);
    return v & m;
  }
  return (w[0] << (SH - P)) & m;
}

// Reductions over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the 16-lane rows):
// v_permlane16_swap (x, x) leaves rows (0, 0, 2, 2) in one result and
// (1, 1, 3, 3) in the other, v_permlane32_swap pairs row r with row r ^ 2.
// Each stage combines the same two values in every lane of a pair, so all
// four lanes end with the same bits.
__device__ __forceinline__ float warp_max_q(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float warp_sum_q(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace ftq
