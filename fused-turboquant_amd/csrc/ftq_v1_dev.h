// Slot geometry and value-dtype rounding shared by the vLLM v1 slot-format
// kernels (store and decode).
#pragma once

#include "ftq_device.h"

namespace ftq {

// Byte offsets of one (token, kv head) slot: [K codes mse][K norm f16]
// [V codes vdb][V scale f16][V min f16]; raw = the bytes that hold data
// (reference boundary_tq_config.py:66-81).  FP8 keys (kf8, 8 bits) take d
// bytes and have no norm: kps = mse = d.
struct V1Geom {
  int mse, kps, vdb, raw;
};
__host__ __device__ constexpr V1Geom v1_geom(int d, int kb, int vb, bool kf8 = false) {
  return V1Geom{d * kb / 8, d * kb / 8 + (kf8 ? 0 : 2), d * vb / 8, d * kb / 8 + (kf8 ? 0 : 2) + d * vb / 8 + 4};
}

// v_flags bits of the slot store and decode entry points
constexpr int V1F_VROT = 1;   // V rotated before its quantisation (un-rotated after the decode)
constexpr int V1F_VLM = 2;    // Lloyd-Max V codes (4-bit V)
constexpr int V1F_KFP8 = 4;   // fp8 e4m3fn keys (key_bits 8)
constexpr int V1F_FP32 = 8;   // decode: fp32 products on the VALU instead of f16 matrix-core operands

// x rounded to the value dtype and back (the reference rounds the pre-rotated
// V to the value tensor's dtype, v1_backend.py:736-740)
template <int DT>
__device__ __forceinline__ float round_to_dtype(float x) {
  if constexpr (DT == BF16) return bf16_bits_to_f32(f32_to_bf16_bits(x));
  else if constexpr (DT == F16) return f16_bits_to_f32(f32_to_f16_bits(x));
  else return x;
}

// x <- x M for a vector spread over 16 lanes, E contiguous elements per lane
// (M row-major D x D fp32, the rotation of a matrix strategy: planar, rotor,
// iso or a caller's own).  The vector goes through `row` (D floats of LDS
// private to this 16-lane group, which lies inside one wave), and each lane
// forms its E columns.
template <int D, int E>
__device__ __forceinline__ void rot_matrix_lanes(float (&x)[E], const float* __restrict__ M, float* row, int lane) {
#pragma unroll
  for (int i = 0; i < E; ++i) row[lane * E + i] = x[i];
  __asm__ volatile("" ::: "memory");  // a wave's LDS accesses run in order
  float y[E];
#pragma unroll
  for (int i = 0; i < E; ++i) y[i] = 0.f;
  for (int k = 0; k < D; ++k) {
    const float xk = row[k];
#pragma unroll
    for (int i = 0; i < E; ++i) y[i] = __builtin_fmaf(xk, M[(int64_t)k * D + lane * E + i], y[i]);
  }
  __asm__ volatile("" ::: "memory");
#pragma unroll
  for (int i = 0; i < E; ++i) x[i] = y[i];
}

// Arguments of one decode-attention call (stage 1 + merge), shared by the
// launchers of the matrix-core and the fp32 VALU kernels.
struct V1Args {
  const void* q;
  int qt;
  const uint8_t* cache;
  const int32_t *bt, *sl, *ks;
  int B, hq, hkv, lbs, max_blocks;
  int64_t nb, sblk, spos, shead;
  const float* cent;
  float qscale;
  int splits, vrot;
  float *wo, *wl;
  void* out;
  int ot;
  float* lse;  // optional per-row natural-log LSE (B*Hq floats)
  const float* rot;  // rotation matrix (D x D fp32, x M), or null for H/sqrt(D)
};

// Code widths with a store and a decode (defined with the store).
bool v1_widths_ok(int kb, int vb, int flags);

// The fp32 VALU decode (any head_dim of 64, 128, 256; every code width);
// defined in ftq_v1_valu.hip.
hipError_t v1_valu_launch(const V1Args& a, int d, int kb, int vb, int flags, hipStream_t st);
// The same kernel over raw fp16 [K | V] slots (boundary layers; a.vrot = 0,
// a.rot = null, a.qscale = scale * log2 e).
hipError_t raw_valu_launch(const V1Args& a, int d, hipStream_t st);

}  // namespace ftq
