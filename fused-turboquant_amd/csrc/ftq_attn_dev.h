// Device helpers shared by the decode-attention kernels (gfx950 MFMA operand
// types, packed-code field extraction, cross-lane reductions).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ftq_device.h"

namespace ftq {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// LDS address of a __shared__ object
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p;
}

union Op8 {
  uint32_t u[4];
  half8 h;
};

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

// Byte offset, inside a code table, of the entry whose index is bits
// [P, P + W) of the code words, ORed with the lane's copy offset (< 2^SH):
// one funnel shift that puts the field at bit SH and one v_and_or_b32, as
// plain arithmetic the compiler schedules itself.  With the table in static
// LDS its address folds into the DS instruction's offset field.
template <int SH, int W, int N>
__device__ __forceinline__ uint32_t lut_field(const uint32_t (&w)[N], int P, uint32_t laneoff) {
  constexpr uint32_t M = ((1u << W) - 1u) << SH;
  uint32_t v;
  if (P >= SH) {
    const int Q = P - SH, i = Q >> 5, o = Q & 31;  // compile-time after unrolling
    v = (o + W + SH > 32 && i + 1 < N) ? __builtin_amdgcn_alignbit(w[i + 1], w[i], o) : (w[i] >> o);
  } else {
    v = w[0] << (SH - P);
  }
  return (v & M) | laneoff;
}

// dword at byte offset off of a table in static LDS
__device__ __forceinline__ uint32_t lds_dword_at(const uint32_t* table, uint32_t off) {
  typedef __attribute__((address_space(3))) const uint8_t lds_u8;
  lds_u8* t = (lds_u8*)(__attribute__((address_space(3))) const void*)table;
  return *(__attribute__((address_space(3))) const uint32_t*)(t + off);
}

// A pair table built by one wave: entry e = h[e & (2^B - 1)] | h[e >> B] << 16,
// where lane i < 2^B holds the f16 bits h[i] (the other lanes' values are not
// read), stored in 2^LOGC consecutive copies (lane l of a reader takes copy
// l % 2^LOGC).  Each lane assembles its entries with two lane reads (every
// lane takes part) and writes their copies, 4 per ds_write_b128.
template <int B, int LOGC>
__device__ __forceinline__ void build_pair_table_wave(uint32_t* lut, uint32_t hbits, int lane) {
  constexpr int NL = 1 << B, ENTRIES = 1 << (2 * B), COPIES = 1 << LOGC;
  constexpr int PER = (ENTRIES + 63) / 64;  // entries per lane
  uint32_t v[PER];
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int e = lane + 64 * k;
    const uint32_t lo = (uint32_t)__shfl((int)hbits, e & (NL - 1));
    const uint32_t hi = (uint32_t)__shfl((int)hbits, (e >> B) & (NL - 1));
    v[k] = (lo & 0xffffu) | (hi << 16);
  }
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int e = lane + 64 * k;
    if (e < ENTRIES) {
      if constexpr (COPIES >= 4) {
        uint4* dst = reinterpret_cast<uint4*>(lut + e * COPIES);
#pragma unroll
        for (int c = 0; c < COPIES / 4; ++c) dst[c] = make_uint4(v[k], v[k], v[k], v[k]);
      } else {
#pragma unroll
        for (int c = 0; c < COPIES; ++c) lut[e * COPIES + c] = v[k];
      }
    }
  }
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

// min over the 64 lanes of a wave; every lane ends with the result
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
  x = min(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0xB1, 0xF, 0xF, true));   // lane ^ 1
  x = min(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x4E, 0xF, 0xF, true));   // lane ^ 2
  x = min(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x141, 0xF, 0xF, true));  // 7 - lane in 8
  x = min(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x128, 0xF, 0xF, true));  // lane + 8 in 16
  auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  x = min((uint32_t)r[0], (uint32_t)r[1]);
  r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return min((uint32_t)r[0], (uint32_t)r[1]);
}

// Scale of a code table (centroids / levels) that enters f16 MFMA operands
// as f16(sigma c).  f16 rounding errs by a relative r(x) = (f16(x) - x) / x of
// up to 2^-11 that differs per table value; with keys 8x the typical norm
// that moves softmax weights by about 0.5%.  A common factor (1 + r) is
// harmless where the kernel divides by the norm of the same f16 values, and
// is divided out elsewhere (rmid), so what matters is the spread of r across
// the table.  sigma = base (1 + j/128), j = 0..127 (two per lane), keeping
// the j with the smallest spread (lowest j on ties: every wave and every
// workgroup picks the same).  For the Lloyd-Max tables of 2-, 3- and 4-bit
// codes at d = 128 the spread drops from up to 8e-4 to 2e-6, 3e-5 and 2e-4.
// base = 1, or (pow2) the power of two that puts the largest |c| in
// [512, 1024).  Wave-local: no LDS, no barrier; c[0, N) read with uniform
// addresses.
struct TableScale {
  float sigma;  // the scale
  float rmid;   // (max r + min r) / 2 of f16(sigma c) over the table
};
template <int N>
__device__ __forceinline__ TableScale table_scale(const float* __restrict__ c, bool pow2) {
  float cv[N], rc[N];
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    cv[i] = c[i];
    mx = fmaxf(mx, fabsf(cv[i]));
  }
  if (!(mx > 0.f) || !(mx < INFINITY)) return TableScale{1.f, 0.f};
  float base = 1.f;
  if (pow2) {
    const int e = (int)((__float_as_uint(mx) >> 23) & 255u);  // mx in [2^(e-127), 2^(e-126))
    base = __uint_as_float((uint32_t)min(max(263 - e, 1), 254) << 23);  // 2^(136 - e)
  }
#pragma unroll
  for (int i = 0; i < N; ++i) rc[i] = cv[i] != 0.f ? __builtin_amdgcn_rcpf(cv[i]) : 0.f;
  const int lane = (int)(threadIdx.x & 63u);
  uint32_t best = ~0u;
  float best_mid = 0.f;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int j = lane + 64 * k;
    const float sg = base * (1.f + (float)j * (1.f / 128.f));
    float tlo = INFINITY, thi = -INFINITY;  // t = f16(sigma c) / c = sigma (1 + r)
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (cv[i] == 0.f) continue;
      const float t = f16_bits_to_f32(f32_to_f16_bits(sg * cv[i])) * rc[i];
      tlo = fminf(tlo, t);
      thi = fmaxf(thi, t);
    }
    const float rs = __builtin_amdgcn_rcpf(sg);
    const uint32_t key = (__float_as_uint((thi - tlo) * rs) & ~127u) | (uint32_t)j;  // spread >= 0: bits order
    if (key < best) {
      best = key;
      best_mid = 0.5f * (thi + tlo) * rs - 1.f;
    }
  }
  const int j = (int)(__builtin_amdgcn_readfirstlane(wave_min_u32(best)) & 127);
  const float mid = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(best_mid), j & 63));
  return TableScale{base * (1.f + (float)j * (1.f / 128.f)), mid};
}

}  // namespace ftq
