// Fast exact library-format encoder for gfx950 (used by the flat encode
// kernel).  Produces the same codes as TurboQuantMSE._encode_unfused
// (reference core/quantizer.py:137-160) for the same rotated vector and norm:
//
//   t    = unscaled FWHT of (x * signs)       stages h = 1, 2, 4, ..., d/2
//   y    = RN(t * c), c = f32(d^-1/2)
//   norm = ||y||,  den = RN(norm + 1e-8)
//   u    = RN(y / den)
//   code = #{interior boundaries B_j : B_j < u}
//
// Work per element is cut in three ways:
//  * one vector per 4 lanes (or 8 for d = 256): all butterfly stages with
//    stride < d/4 run in registers; each cross-lane stage is one v_fmac with a
//    DPP operand.  Lanes keep a statically known sign flip sigma instead of
//    selecting between a+b and b-a: lane value = sigma * true value, and
//    a + (+-1)*b is rounded exactly like the reference's a+b / a-b because
//    round-to-nearest-even commutes with negation.
//  * no per-element multiply by c and no division: per vector, the exact fp32
//    threshold T_j = min{t : B_j < RN(RN(t*c)/den)} is computed once (in fp64,
//    where the products involved are exact), so code = #{j : t >= T_j}.
//  * the count is a binary search over the thresholds (3 compares for 3 bits).
#pragma once

#include "ftq_device.h"

namespace ftq {

__device__ __forceinline__ float f32_next_up(float x) {
  int i = __float_as_int(x);
  if ((i & 0x7fffffff) == 0) return __int_as_float(1);  // +-0 -> smallest positive subnormal
  i += (i >= 0) ? 1 : -1;
  return __int_as_float(i);
}
__device__ __forceinline__ float f32_next_down(float x) { return -f32_next_up(-x); }
__device__ __forceinline__ bool f32_even(float x) { return (__float_as_uint(x) & 1u) == 0u; }

// smallest float >= p (p finite)
__device__ __forceinline__ float f32_round_up(double p) {
  float f = (float)p;
  if ((double)f < p) f = f32_next_up(f);
  return f;
}

// Smallest fp32 t with  B < RN32( RN32(t*c) / den ),  c > 0, den > 0.
//   B < RN(q)  <=>  RN(q) >= B+  <=>  q > M1, or q == M1 and B+ is even
//   (M1 = midpoint of B and B+; ties round to even).  With q = y/den and
//   P = M1*den (exact in fp64), the smallest such y is Y = RU(P), bumped once
//   if Y == P and B+ is odd.  Likewise RN(t*c) >= Y  <=>  t*c > M2, or
//   t*c == M2 and Y is even (M2 = midpoint of Y- and Y).  t0 = RN(M2 / c)
//   is within half an ulp of the real root, so the answer is t0 or its
//   successor; t*c is exact in fp64, which decides between them.
__device__ __forceinline__ float exact_threshold(float B, float den, float c, double rc) {
  const float Bp = f32_next_up(B);
  const double M1 = ((double)B + (double)Bp) * 0.5;
  const double P = M1 * (double)den;
  float Y = f32_round_up(P);
  if ((double)Y == P && !f32_even(Bp)) Y = f32_next_up(Y);
  const double M2 = ((double)f32_next_down(Y) + (double)Y) * 0.5;
  const float t0 = (float)(M2 * rc);
  const double tc = (double)t0 * (double)c;
  const bool ok = (tc > M2) || (tc == M2 && f32_even(Y));
  return ok ? t0 : f32_next_up(t0);
}

// DPP helpers (quad_perm within 4-lane groups; see ftq_device.h for encodings)
__device__ __forceinline__ float dpp_bcast_quad(float v, int k) {
  // every lane of a quad reads lane k of the quad (k compile-time)
  switch (k) {
    case 0: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x00, 0xF, 0xF, false));
    case 1: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x55, 0xF, 0xF, false));
    case 2: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xAA, 0xF, 0xF, false));
    default: return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xFF, 0xF, 0xF, false));
  }
}

template <int D> struct FastShape {
  static constexpr int LPV = (D == 256) ? 8 : 4;  // lanes per vector
  static constexpr int E = D / LPV;               // elements per lane
  static constexpr int VPW = 64 / LPV;            // vectors per wave
};

// Exact RHT-domain quantisation of one vector held as E elements per lane in
// LPV lanes.  On entry x holds the input; on exit codes[] holds the codes of
// this lane's elements (in element order) -- complemented (c ^ (2^BITS - 1))
// when flip is set -- and the return value is the fp32 norm of the rotated
// vector.
template <int D, int BITS>
__device__ __forceinline__ float encode_fast(float (&x)[FastShape<D>::E], const float* __restrict__ bnd_sh,
                                             float c, double rc, int lane, uint32_t (&codes)[FastShape<D>::E],
                                             bool& flip) {
  constexpr int LPV = FastShape<D>::LPV, E = FastShape<D>::E;
  constexpr int L = 1 << BITS;
  // ---- FWHT, in-register stages ----
#pragma unroll
  for (int h = 1; h < E; h <<= 1) {
#pragma unroll
    for (int i = 0; i < E; ++i) {
      if ((i & h) == 0) {
        const float a = x[i], b = x[i + h];
        x[i] = a + b;
        x[i + h] = a - b;
      }
    }
  }
  // ---- cross-lane stages with lazily tracked sign ----
  // stage m: lower lane needs v_l + v_m, upper lane v_m - v_l.  With a = sigma*v,
  // lower computes a_l + (s_l s_m) a_m (new sigma = s_l), upper computes
  // a_l - (s_l s_m) a_m (new sigma = -s_l).  Partners always share the sigma
  // accumulated from lower-order bits, so s_l s_m = 1 within a stage.
  bool neg = false;  // final sigma == -1
  {
    const float k1 = (lane & 1) ? -1.f : 1.f;
#pragma unroll
    for (int i = 0; i < E; ++i) x[i] = __builtin_fmaf(dpp_xor1(x[i]), k1, x[i]);
    neg ^= (lane & 1) != 0;
  }
  if constexpr (LPV >= 4) {
    const float k2 = (lane & 2) ? -1.f : 1.f;
#pragma unroll
    for (int i = 0; i < E; ++i) x[i] = __builtin_fmaf(dpp_xor2(x[i]), k2, x[i]);
    neg ^= (lane & 2) != 0;
  }
  if constexpr (LPV >= 8) {
    const float k4 = (lane & 4) ? -1.f : 1.f;
#pragma unroll
    for (int i = 0; i < E; ++i) x[i] = __builtin_fmaf(dpp_xor4(x[i]), k4, x[i]);
    neg ^= (lane & 4) != 0;
  }
  // ---- norm ----
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < E; ++i) ss = __builtin_fmaf(x[i], x[i], ss);
  ss += dpp_xor1(ss);
  if constexpr (LPV >= 4) ss += dpp_xor2(ss);
  if constexpr (LPV >= 8) ss += dpp_xor4(ss);
  const float nrm = __builtin_sqrtf(ss) * c;
  const float den = nrm + 1e-8f;
  // ---- thresholds: lane k of the group computes T_j for j-1 == k (mod LPV) ----
  constexpr int NT = L - 1;
  constexpr int PER = (NT + LPV - 1) / LPV;
  float mine[PER];
#pragma unroll
  for (int r = 0; r < PER; ++r) {
    const int j = r * LPV + (lane & (LPV - 1));  // 0-based threshold index
    mine[r] = (j < NT) ? exact_threshold(bnd_sh[j], den, c, rc) : 0.f;
  }
  float T[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int src = j % LPV, r = j / LPV;
    if constexpr (LPV == 4) {
      T[j] = dpp_bcast_quad(mine[r], src);
    } else {
      T[j] = __shfl(mine[r], (lane & ~(LPV - 1)) + src);
    }
  }
  // lanes holding negated values a = -t count #{k : a >= V_k} with
  // V_k = next_up(-T_{NT-1-k}); their codes are then (L-1) - count.
  float V[NT];
#pragma unroll
  for (int k = 0; k < NT; ++k) V[k] = neg ? f32_next_up(-T[NT - 1 - k]) : T[k];
  // ---- per-element binary search: code = #{k : a >= V_k}, four elements per
  // step so each compare has independent work before its result is used ----
#pragma unroll
  for (int i0 = 0; i0 < E; i0 += 4) {
    uint32_t cd[4];
    if constexpr (BITS == 2) {
      bool s1[4], s0[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) s1[u] = x[i0 + u] >= V[1];
#pragma unroll
      for (int u = 0; u < 4; ++u) s0[u] = x[i0 + u] >= (s1[u] ? V[2] : V[0]);
#pragma unroll
      for (int u = 0; u < 4; ++u) cd[u] = (s1[u] ? 2u : 0u) | (s0[u] ? 1u : 0u);
    } else if constexpr (BITS == 3) {
      bool s2[4], s1[4], s0[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) s2[u] = x[i0 + u] >= V[3];
#pragma unroll
      for (int u = 0; u < 4; ++u) s1[u] = x[i0 + u] >= (s2[u] ? V[5] : V[1]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float lo = s1[u] ? V[2] : V[0];
        const float hi = s1[u] ? V[6] : V[4];
        s0[u] = x[i0 + u] >= (s2[u] ? hi : lo);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) cd[u] = (s2[u] ? 4u : 0u) | (s1[u] ? 2u : 0u) | (s0[u] ? 1u : 0u);
    } else {
      bool s3[4], s2[4], s1[4], s0[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) s3[u] = x[i0 + u] >= V[7];
#pragma unroll
      for (int u = 0; u < 4; ++u) s2[u] = x[i0 + u] >= (s3[u] ? V[11] : V[3]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float a = s3[u] ? V[13] : V[5], bq = s3[u] ? V[9] : V[1];
        s1[u] = x[i0 + u] >= (s2[u] ? a : bq);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        // last threshold: V[8*s3 + 4*s2 + 2*s1]
        const float t00 = s3[u] ? V[8] : V[0], t01 = s3[u] ? V[10] : V[2];
        const float t10 = s3[u] ? V[12] : V[4], t11 = s3[u] ? V[14] : V[6];
        const float lo = s1[u] ? t01 : t00, hi = s1[u] ? t11 : t10;
        s0[u] = x[i0 + u] >= (s2[u] ? hi : lo);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
        cd[u] = (s3[u] ? 8u : 0u) | (s2[u] ? 4u : 0u) | (s1[u] ? 2u : 0u) | (s0[u] ? 1u : 0u);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) codes[i0 + u] = cd[u];
  }
  flip = neg;
  return nrm;
}

// Store this lane's E codes (element order) at byte offset lane*E*BITS/8 of row.
// (codes complemented when flip is set: undone here on the packed words)
template <int E, int BITS>
__device__ __forceinline__ void store_lane_codes(const uint32_t (&codes)[E], bool flip, uint8_t* row,
                                                 int lane_in_vec) {
  constexpr int NB = E * BITS;          // bits per lane
  constexpr int NDW = (NB + 31) / 32;
  uint32_t w[NDW];
#pragma unroll
  for (int k = 0; k < NDW; ++k) w[k] = 0;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int P = i * BITS, k = P >> 5, o = P & 31;
    w[k] |= codes[i] << o;
    if (o + BITS > 32) w[k + 1] |= codes[i] >> (32 - o);
  }
  const uint32_t fm = flip ? 0xffffffffu : 0u;
#pragma unroll
  for (int k = 0; k < NDW; ++k) {
    const int bits_here = (NB - 32 * k) >= 32 ? 32 : (NB - 32 * k);
    w[k] ^= fm & (bits_here == 32 ? 0xffffffffu : ((1u << bits_here) - 1u));
  }
  uint8_t* dst = row + lane_in_vec * (NB / 8);
  if constexpr (NB % 32 == 0) {
    if constexpr (NDW == 4) {
      *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
    } else if constexpr (NDW == 2) {
      *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
    } else {
#pragma unroll
      for (int k = 0; k < NDW; ++k) reinterpret_cast<uint32_t*>(dst)[k] = w[k];
    }
  } else {
    // NB % 16 == 0 (e.g. 48 bits): 16-bit stores
#pragma unroll
    for (int k = 0; k < NB / 16; ++k)
      reinterpret_cast<uint16_t*>(dst)[k] = (uint16_t)(w[k >> 1] >> (16 * (k & 1)));
  }
}

}  // namespace ftq
