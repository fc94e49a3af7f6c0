// Library-format encoder for 16-bit inputs (bf16 / f16) whose Hadamard
// transform runs on the matrix cores.  Same outputs as
// TurboQuantMSE._encode_unfused (reference core/quantizer.py:137-160):
//
//   t    = H (x * signs)        unnormalised Sylvester transform, fp32
//   norm = sqrt(d sum x^2) * c  c = f32(d^-1/2); = ||t|| c by Parseval, the
//                               sum taken from the diagonal of X X^T on the
//                               matrix cores
//   code = #{interior boundaries B_j : B_j < RN(RN(t*c) / (norm + 1e-8))}
//
// The quantiser is the exact per-vector threshold search of ftq_encode_fast.h
// (T_j in the t domain, binary search, no per-element division).
//
// Transform.  A wave encodes 16 vectors at a time.  The input, sign-flipped,
// is the B operand of v_mfma_f32_16x16x32_{bf16,f16} (K = input element,
// N = vector) and the Hadamard matrix is the A operand (M = output element),
// with its rows and columns permuted so that every lane needs only four
// operand registers and ends up holding contiguous outputs:
//   lane l = 16 q + j  (q = l / 16, j = l % 16 = vector of the group)
//   B operand, K step s: input elements e = EL q + 8 s + t, t = 0..7
//   A operand, M block mb: row i = 4 q' + r holds output o = EL q' + 4 mb + r
//   H[o][e] = (-1)^popc(o & e) = (-1)^(popc(r & t) + mb0 t2 + popc((mb >> 1) & s) + popc(q' & q))
// (EL = d/4; o and e split into bit fields r|mb|q' and t|s|q that line up).
// So A(mb, s) = (-1)^popc((mb >> 1) & s) * P_{mb & 1}, a compile-time sign
// times one of two per-lane patterns, and the accumulator of M block mb in
// lane (q, j) holds outputs EL q + 4 mb + 0..3 of vector j: lane q owns the
// contiguous elements [EL q, EL q + EL) and stores their codes with one
// EL*bits/8-byte write.
//
// Products with +-1 are exact; the fp32 sums follow the matrix core's
// accumulation order instead of the reference's butterfly order, so t can
// differ from the reference's rotated value in its last bits.  A code can
// then differ only where u lies within that distance of a boundary; the
// tests count such ties.
#pragma once

#include "ftq_encode_fast.h"

namespace ftq {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

union Op16x8 {
  uint32_t u[4];
  uint4 v;
  bf16x8_t b;
  f16x8_t h;
};

template <int DT>
__device__ __forceinline__ f32x4_t mfma_16x16x32(const Op16x8& a, const Op16x8& b, f32x4_t c) {
  if constexpr (DT == BF16) return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.b, b.b, c, 0, 0, 0);
  else return __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, b.h, c, 0, 0, 0);
}

// next representable float above / below a nonzero finite x (integer step
// on the bit pattern: +1 away from zero for positives, toward zero for negatives)
__device__ __forceinline__ float nz_next_up(float x) {
  const int i = __float_as_int(x);
  return __int_as_float(i + ((i >> 31) | 1));
}
__device__ __forceinline__ float nz_next_down(float x) {
  const int i = __float_as_int(x);
  return __int_as_float(i - ((i >> 31) | 1));
}

// Per-boundary constants of the exact threshold: m1 = (B + B+) / 2 (exact in
// fp64, B+ the float after B) and whether B+ has an odd significand.
struct BoundaryK {
  double m1;
  bool odd;
};
__device__ __forceinline__ BoundaryK boundary_k(float B) {
  const float Bp = nz_next_up(B == 0.f ? 0.f : B);  // +-0 -> smallest subnormal
  return BoundaryK{((double)B + (double)Bp) * 0.5, (__float_as_uint(Bp) & 1u) != 0u};
}

// Smallest fp32 t with  B < RN(RN(t c) / den)  (same value as exact_threshold
// in ftq_encode_fast.h, without branches):
//   Y = smallest float with RN(Y / den) > B: Y > P = m1 den (exact in fp64),
//       or Y == P when B+ is even (the tie then rounds up to B+);
//   T = smallest float with RN(T c) >= Y: T c > M2 = (Y- + Y) / 2, or
//       T c == M2 when Y is even.  t0 = RN(M2 / c) is T or the float below it;
//       t0 c (exact in fp64) decides.  S = Y- + Y and t0 (2c) are exact.
// The integer steps never meet +0 (Y = +0 would need P > 0 rounding to +0
// without a bump) and are exact for every other finite value.
__device__ __forceinline__ float exact_threshold_k(const BoundaryK& k, double den, double c2,
                                                   double rc_half) {
  const double P = k.m1 * den;
  const float Yr = (float)P;
  const double Yd = (double)Yr;
  const bool bump = (Yd < P) || (Yd == P && k.odd);
  const float Y = bump ? nz_next_up(Yr) : Yr;
  const double S = (double)nz_next_down(Y) + (double)Y;
  const float t0 = (float)(S * rc_half);
  const double tc2 = (double)t0 * c2;
  const bool ok = (tc2 > S) || (tc2 == S && (__float_as_uint(Y) & 1u) == 0u);
  return ok ? t0 : nz_next_up(t0);
}

// w = 2 w + (lane's bit of mask m): one v_addc per code bit.  m is the
// wave's compare mask (EXEC must be full where this is used).
__device__ __forceinline__ uint32_t shift_in(uint32_t w, bool bit) {
  const uint64_t m = __builtin_amdgcn_ballot_w64(bit);
  uint32_t r;
  uint64_t co;
  asm("v_addc_co_u32_e64 %0, %1, %2, %2, %3" : "=v"(r), "=s"(co) : "v"(w), "s"(m));
  return r;
}

// Codes of E elements, code = #{k : a >= V_k} over NT = 2^BITS - 1 sorted
// thresholds by binary search, packed little-endian (element e at bits
// [BITS e, BITS e + BITS)) into E*BITS/32 words.  Bits are shifted in from
// the highest position down; four elements per step keep independent
// compares queued behind each select.
template <int BITS, int E>
__device__ __forceinline__ void quantize_pack(const float (&x)[E], const float (&V)[(1 << BITS) - 1],
                                              uint32_t (&w)[E * BITS / 32]) {
  static_assert((E * BITS) % 32 == 0, "whole words per lane");
#pragma unroll
  for (int k = 0; k < E * BITS / 32; ++k) w[k] = 0;
#pragma unroll
  for (int i0 = E - 4; i0 >= 0; i0 -= 4) {
    bool s[4][BITS];
    if constexpr (BITS == 2) {
#pragma unroll
      for (int u = 0; u < 4; ++u) s[u][1] = x[i0 + u] >= V[1];
#pragma unroll
      for (int u = 0; u < 4; ++u) s[u][0] = x[i0 + u] >= (s[u][1] ? V[2] : V[0]);
    } else if constexpr (BITS == 3) {
#pragma unroll
      for (int u = 0; u < 4; ++u) s[u][2] = x[i0 + u] >= V[3];
#pragma unroll
      for (int u = 0; u < 4; ++u) s[u][1] = x[i0 + u] >= (s[u][2] ? V[5] : V[1]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float lo = s[u][2] ? V[4] : V[0];
        const float hi = s[u][2] ? V[6] : V[2];
        s[u][0] = x[i0 + u] >= (s[u][1] ? hi : lo);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) s[u][3] = x[i0 + u] >= V[7];
#pragma unroll
      for (int u = 0; u < 4; ++u) s[u][2] = x[i0 + u] >= (s[u][3] ? V[11] : V[3]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float a = s[u][3] ? V[13] : V[5], bq = s[u][3] ? V[9] : V[1];
        s[u][1] = x[i0 + u] >= (s[u][2] ? a : bq);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float t00 = s[u][3] ? V[8] : V[0], t01 = s[u][3] ? V[10] : V[2];
        const float t10 = s[u][3] ? V[12] : V[4], t11 = s[u][3] ? V[14] : V[6];
        const float lo = s[u][1] ? t01 : t00, hi = s[u][1] ? t11 : t10;
        s[u][0] = x[i0 + u] >= (s[u][2] ? hi : lo);
      }
    }
#pragma unroll
    for (int u = 3; u >= 0; --u) {
#pragma unroll
      for (int b = BITS - 1; b >= 0; --b) {
        const int k = (BITS * (i0 + u) + b) >> 5;
        w[k] = shift_in(w[k], s[u][b]);
      }
    }
  }
}

template <int D, int BITS, int DT>
__global__ __launch_bounds__(256) void encode_mfma_kernel(const void* __restrict__ x, int64_t n,
                                                          const float* __restrict__ signs,
                                                          const float* __restrict__ boundaries,
                                                          float c, double rc,
                                                          uint8_t* __restrict__ packed,
                                                          uint16_t* __restrict__ norms) {
  static_assert(D == 128 || D == 256, "MFMA encoder covers d = 128 and 256");
  static_assert(DT == BF16 || DT == F16, "MFMA encoder takes 16-bit inputs");
  constexpr int EL = D / 4;   // outputs (and inputs) per lane
  constexpr int KS = D / 32;  // K steps
  constexpr int MB = D / 16;  // M blocks
  constexpr int NT = (1 << BITS) - 1;
  constexpr int PERQ = (NT + 3) / 4;  // thresholds computed per lane
  constexpr int PD = D * BITS / 8;

  const int lane = threadIdx.x & 63;
  const int q = lane >> 4, j = lane & 15;
  const int qp = (lane >> 2) & 3, r = lane & 3;
  // boundary constants of the thresholds this lane computes (j = PERQ q + k)
  BoundaryK bk[PERQ];
#pragma unroll
  for (int k = 0; k < PERQ; ++k) {
    const int jj = PERQ * q + k;
    bk[k] = boundary_k(boundaries[1 + (jj < NT ? jj : 0)]);
  }
  const double c2 = 2.0 * (double)c, rc_half = 0.5 * rc;
  // A patterns: P0[t] = (-1)^(popc(r & t) + popc(q' & q)), P1[t] = P0[t] (-1)^(t >> 2)
  const uint32_t one = (DT == BF16) ? 0x3F80u : 0x3C00u;
  Op16x8 P0, P1, N0, N1;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t p0 = 0, p1 = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int t = 2 * w + h;
      const uint32_t s0 = (uint32_t)(__popc(r & t) + __popc(qp & q)) & 1u;
      const uint32_t s1 = s0 ^ (uint32_t)(t >> 2);
      p0 |= (one | (s0 << 15)) << (16 * h);
      p1 |= (one | (s1 << 15)) << (16 * h);
    }
    P0.u[w] = p0;
    P1.u[w] = p1;
    N0.u[w] = p0 ^ 0x80008000u;
    N1.u[w] = p1 ^ 0x80008000u;
  }
  // RHT sign flips of this lane's input elements EL q + 8 s + t, as xor masks
  uint32_t sm[KS][4];
#pragma unroll
  for (int s = 0; s < KS; ++s) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int e = EL * q + 8 * s + 2 * w;
      sm[s][w] = (signs[e] < 0.f ? 0x8000u : 0u) | (signs[e + 1] < 0.f ? 0x80000000u : 0u);
    }
  }
  // G[j][j] of the Gram MFMA sits in lane (j / 4, j), accumulator j % 4:
  // every lane picks accumulator j % 4 and reads lane (j / 4, j)'s pick
  const bool jr_hi = (j & 2) != 0, jr_lo = (j & 1) != 0;
  const int diag_src = (((j >> 2) << 4) | j) << 2;  // ds_bpermute byte address

  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t wstride = (int64_t)gridDim.x * 4 * 16;
  const uint16_t* xb = static_cast<const uint16_t*>(x);

  // groups of 16 vectors; the next group's input is loaded while the
  // current one is encoded
  auto load_group = [&](int64_t g0, Op16x8 (&dst)[KS]) {
    const int64_t vv = g0 + j < n ? g0 + j : g0;
    const uint4* src = reinterpret_cast<const uint4*>(xb + vv * D + EL * q);
#pragma unroll
    for (int s = 0; s < KS; ++s) dst[s].v = src[s];
  };
  auto flip_signs = [&](Op16x8 (&v)[KS]) {
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int w = 0; w < 4; ++w) v[s].u[w] ^= sm[s][w];
  };
  // norm and the NT thresholds of the group held (sign-flipped) in v
  auto norm_thresholds = [&](const Op16x8 (&v)[KS], float& nrm, float (&T)[NT]) {
    f32x4_t gram = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) gram = mfma_16x16x32<DT>(v[s], v[s], gram);
    const float pick = jr_hi ? (jr_lo ? gram[3] : gram[2]) : (jr_lo ? gram[1] : gram[0]);
    const float xx = __int_as_float(__builtin_amdgcn_ds_bpermute(diag_src, __float_as_int(pick)));
    // ||t||^2 = D ||x||^2 (Parseval for the unnormalised transform)
    nrm = __builtin_sqrtf(xx * (float)D) * c;
    const double den = (double)(nrm + 1e-8f);
    float mine[PERQ];
#pragma unroll
    for (int k = 0; k < PERQ; ++k) mine[k] = exact_threshold_k(bk[k], den, c2, rc_half);
#pragma unroll
    for (int jj = 0; jj < NT; ++jj) T[jj] = __shfl(mine[jj % PERQ], ((jj / PERQ) << 4) | j);
  };

  int64_t v0 = wave * 16;
  if (v0 >= n) return;
  Op16x8 nxt[KS];
  load_group(v0, nxt);
  for (; v0 < n; v0 += wstride) {
    Op16x8 cur[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) cur[s] = nxt[s];
    if (v0 + wstride < n) load_group(v0 + wstride, nxt);
    flip_signs(cur);
    f32x4_t acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const bool neg = (__builtin_popcount((mb >> 1) & s) & 1) != 0;
        const Op16x8& a = (mb & 1) ? (neg ? N1 : P1) : (neg ? N0 : P0);
        acc[mb] = mfma_16x16x32<DT>(a, cur[s], acc[mb]);
      }
    }
    float T[NT], nrm;
    norm_thresholds(cur, nrm, T);
    float t[EL];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) t[4 * mb + i] = acc[mb][i];
    constexpr int NW = EL * BITS / 32;
    uint32_t w[NW];
    quantize_pack<BITS, EL>(t, T, w);
    const int64_t v = v0 + j;
    if (v < n) {
      uint32_t* dst = reinterpret_cast<uint32_t*>(packed + v * PD) + NW * q;
      if constexpr (NW == 2) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(w[0], w[1]);
      } else if constexpr (NW % 4 == 0) {
#pragma unroll
        for (int k = 0; k < NW; k += 4) *reinterpret_cast<uint4*>(dst + k) = make_uint4(w[k], w[k + 1], w[k + 2], w[k + 3]);
      } else {
#pragma unroll
        for (int k = 0; k < NW; ++k) dst[k] = w[k];
      }
      if (q == 0) norms[v] = (uint16_t)f32_to_f16_bits(nrm);
    }
  }
}

}  // namespace ftq
