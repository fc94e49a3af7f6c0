// Device-side pieces of the library-format codec shared by the flat codec
// kernels (ftq_codec.hip) and the paged store (ftq_paged.hip): the lane
// layout, the fused RHT + norm + Lloyd-Max quantiser, and the code packers.
#pragma once

#include "ftq_device.h"

namespace ftq {

template <int D> struct CodecShape {
  static constexpr int E = (D == 256) ? 16 : 8;
  static constexpr int LPV = D / E;
  static constexpr int GPB = 256 / LPV;
};

// Pack the E codes of this lane (BITS each) into the vector's packed row.
template <int E, int BITS>
__device__ __forceinline__ void pack_store(const uint32_t (&c)[E], uint8_t* row, int lane) {
  if constexpr (E == 8 && BITS == 4) {
    uint32_t w = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) w |= c[k] << (4 * k);
    reinterpret_cast<uint32_t*>(row)[lane] = w;
  } else if constexpr (E == 8 && BITS == 2) {
    uint32_t w = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) w |= c[k] << (2 * k);
    uint32_t wn = dpp_xor1_u(w);
    if ((lane & 1) == 0) reinterpret_cast<uint32_t*>(row)[lane >> 1] = w | (wn << 16);
  } else if constexpr (E == 8 && BITS == 3) {
    uint32_t w = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) w |= c[k] << (3 * k);
    uint32_t wn = dpp_quad_next(w);
    const int q = lane & 3;
    if (q < 3)
      reinterpret_cast<uint32_t*>(row)[3 * (lane >> 2) + q] = (w >> (8 * q)) | (wn << (24 - 8 * q));
  } else if constexpr (E == 16 && BITS == 4) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) { lo |= c[k] << (4 * k); hi |= c[k + 8] << (4 * k); }
    reinterpret_cast<uint2*>(row)[lane] = make_uint2(lo, hi);
  } else if constexpr (E == 16 && BITS == 2) {
    uint32_t w = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) w |= c[k] << (2 * k);
    reinterpret_cast<uint32_t*>(row)[lane] = w;
  } else if constexpr (E == 16 && BITS == 3) {
    uint64_t w = 0;
#pragma unroll
    for (int k = 0; k < 16; ++k) w |= (uint64_t)c[k] << (3 * k);
    uint32_t lo = (uint32_t)w, hi = (uint32_t)(w >> 32);
    uint32_t plo = dpp_xor1_u(lo), phi = dpp_xor1_u(hi);
    if ((lane & 1) == 0) {
      uint32_t* dst = reinterpret_cast<uint32_t*>(row) + 3 * (lane >> 1);
      dst[0] = lo;
      dst[1] = (hi & 0xffffu) | (plo << 16);
      dst[2] = (plo >> 16) | (phi << 16);
    }
  } else {
    static_assert(BITS == 2 || BITS == 3 || BITS == 4, "unsupported bit width");
  }
}

// Read the E codes of this lane from the vector's packed row.
template <int E, int BITS>
__device__ __forceinline__ void unpack_load(const uint8_t* row, int lane, uint32_t (&c)[E]) {
  constexpr int B = E * BITS / 8;  // packed bytes per lane
  const int o = lane * B;
  const uint32_t* dw = reinterpret_cast<const uint32_t*>(row);
  uint64_t win;
  if constexpr (B == 8) {
    uint2 v = reinterpret_cast<const uint2*>(row)[lane];
    win = ((uint64_t)v.y << 32) | v.x;
  } else if constexpr (B == 4) {
    win = dw[lane];
  } else if constexpr (B == 2) {
    win = reinterpret_cast<const uint16_t*>(row)[lane];
  } else {
    uint32_t d0 = dw[o >> 2];
    uint32_t d1 = dw[(o + B - 1) >> 2];
    win = ((((uint64_t)d1) << 32) | d0) >> (8 * (o & 3));
  }
  constexpr uint32_t mask = (1u << BITS) - 1u;
#pragma unroll
  for (int k = 0; k < E; ++k) c[k] = (uint32_t)(win >> (BITS * k)) & mask;
}

// RHT + per-vector norm + Lloyd-Max bucketize of one vector held as E
// elements per lane in LPV lanes (x is overwritten with the rotated vector).
// Matches TurboQuantMSE._encode_unfused (reference core/quantizer.py:137-160):
// y = fwht(x * s) * d^-1/2, n = ||y||, u = y / (n + 1e-8),
// code = #{interior boundaries b : b < u}  (== clamp(bucketize(u) - 1)).
template <int E, int LPV, int BITS>
__device__ __forceinline__ float encode_core(float (&y)[E], const float (&sg)[E],
                                             const float (&bnd)[(1 << BITS) - 1], float scale,
                                             int lane, uint32_t (&c)[E]) {
  constexpr int L = 1 << BITS;
#pragma unroll
  for (int i = 0; i < E; ++i) y[i] *= sg[i];
  fwht_lanes<E, LPV>(y, lane);
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    y[i] *= scale;
    ss = __builtin_fmaf(y[i], y[i], ss);
  }
  ss = group_sum<LPV>(ss);
  const float nrm = __builtin_sqrtf(ss);
  const float den = nrm + 1e-8f;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const float u = y[i] / den;
    uint32_t q = 0;
#pragma unroll
    for (int j = 0; j < L - 1; ++j) q += (bnd[j] < u) ? 1u : 0u;
    c[i] = q;
  }
  return nrm;
}

}  // namespace ftq
