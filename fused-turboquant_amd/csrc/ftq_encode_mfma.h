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
// Quantiser.  code = #{j : t > T_j} with per-vector thresholds in the t
// domain, T_j = RN(B_j * RN((norm + 1e-8) / c)) in fp32: no per-element
// division.  T_j sits within a few ulp of the exact preimage of B_j under
// t -> RN(RN(t c) / den), so a code can differ from the reference's only where
// u lies within that distance of B_j (a boundary tie, like those of the
// accumulation order below).  When the codebook is symmetric in fp32
// (B[2^b - j] == -B[j] for every j but the middle one, as the Lloyd-Max
// codebooks of d = 64 and 128 are) the search runs on |t| over the positive
// thresholds, the sign test against the middle threshold picking the half:
// 3 compares, 1 select and 3 carry-adds per 3-bit element instead of 3, 4, 3.
// The symmetric form is a separate instantiation (SYM), chosen by the host
// from its copy of the codebook: one loop per kernel keeps the register count
// at 100 (4 waves per SIMD) at d = 128 and 149 (3 waves) at d = 256.
//
// Transform.  A wave encodes 16 vectors (a group) at a time.  A launch may
// cover two tensors of the same shape (K and V of one store): the groups of
// the second follow those of the first in one numbering, so the waves stream
// both without a second launch.  The transform runs in 128-element blocks:
// H_256 = [[H_128, H_128], [H_128, -H_128]] (the top index bit of the
// Sylvester matrix contributes (-1)^(o7 e7)), so at d = 256 each half of the
// input goes through the 128-point transform on the matrix cores and one fp32
// add and subtract per output pair finish it: half the matrix-core work of the
// dense 256 x 256 product, for one VALU operation per element.
//
// The 128-point transform: the input block, sign-flipped, is the B operand of
// v_mfma_f32_16x16x32_{bf16,f16} (K = input element, N = vector) and the
// Hadamard matrix is the A operand (M = output element), with its rows and
// columns permuted so that every lane needs only four operand registers and
// ends up holding contiguous outputs:
//   lane l = 16 q + j  (q = l / 16, j = l % 16 = vector of the group)
//   B operand, K step s: block elements e = 32 q + 8 s + t, t = 0..7
//   A operand, M block mb: row i = 4 q' + r holds output o = 32 q' + 4 mb + r
//   H[o][e] = (-1)^popc(o & e) = (-1)^(popc(r & t) + mb0 t2 + popc((mb >> 1) & s) + popc(q' & q))
// (o and e split into bit fields r|mb|q' and t|s|q that line up).
// So A(mb, s) = (-1)^popc((mb >> 1) & s) * P_{mb & 1}, a compile-time sign
// times one of two per-lane patterns, and the accumulator of M block mb in
// lane (q, j) holds outputs 32 q + 4 mb + 0..3 of vector j: lane q owns the
// contiguous outputs [32 q, 32 q + 32) of every 128-element block and stores
// their codes with one 4*bits-byte write per block.
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

// The tensors one launch encodes: nseg (1 or 2) segments of n vectors each,
// segment 1 being the V of a fused K + V store.  Unused pointers may be null.
struct EncodeSegs {
  const void* x0;
  const void* x1;
  uint8_t* packed0;
  uint8_t* packed1;
  uint16_t* norms0;
  uint16_t* norms1;
  int nseg;
};

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

// w = 2 w + (lane's bit of mask m): one v_addc per code bit.  m is the
// wave's compare mask (EXEC must be full where this is used).
__device__ __forceinline__ uint32_t shift_in(uint32_t w, bool bit) {
  const uint64_t m = __builtin_amdgcn_ballot_w64(bit);
  uint32_t r;
  uint64_t co;
  asm("v_addc_co_u32_e64 %0, %1, %2, %2, %3" : "=v"(r), "=s"(co) : "v"(w), "s"(m));
  return r;
}

// Codes of E elements, code = #{k : a > V_k} over NT = 2^BITS - 1 sorted
// thresholds by binary search, packed little-endian (element e at bits
// [BITS e, BITS e + BITS)) into E*BITS/32 words.  Element e is compared with
// threshold set e % NS (NS = 4: four vectors interleaved element by element).
// Bits are shifted in from the highest position down; four elements per step
// keep independent compares queued behind each select.  Strict, like the
// reference's bucketize(right=False): a value on a threshold takes the lower
// code.
template <int BITS, int E, int NS = 1>
__device__ __forceinline__ void quantize_pack(const float (&x)[E], const float (&VS)[NS][(1 << BITS) - 1],
                                              uint32_t (&w)[E * BITS / 32]) {
  static_assert((E * BITS) % 32 == 0, "whole words per lane");
  static_assert(NS == 1 || NS == 2 || NS == 4, "threshold sets repeat every 4 elements");
  auto V = [&](int u, int k) { return VS[u % NS][k]; };
#pragma unroll
  for (int k = 0; k < E * BITS / 32; ++k) w[k] = 0;
#pragma unroll
  for (int i0 = E - 4; i0 >= 0; i0 -= 4) {
    bool s[4][BITS];
    // element i0 + u takes threshold set u % NS (i0 is a multiple of 4): V(u, k)
    if constexpr (BITS == 2) {
#pragma unroll
      for (int u = 0; u < 4; ++u) s[u][1] = x[i0 + u] > V(u, 1);
#pragma unroll
      for (int u = 0; u < 4; ++u) s[u][0] = x[i0 + u] > (s[u][1] ? V(u, 2) : V(u, 0));
    } else if constexpr (BITS == 3) {
#pragma unroll
      for (int u = 0; u < 4; ++u) s[u][2] = x[i0 + u] > V(u, 3);
#pragma unroll
      for (int u = 0; u < 4; ++u) s[u][1] = x[i0 + u] > (s[u][2] ? V(u, 5) : V(u, 1));
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float lo = s[u][2] ? V(u, 4) : V(u, 0);
        const float hi = s[u][2] ? V(u, 6) : V(u, 2);
        s[u][0] = x[i0 + u] > (s[u][1] ? hi : lo);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) s[u][3] = x[i0 + u] > V(u, 7);
#pragma unroll
      for (int u = 0; u < 4; ++u) s[u][2] = x[i0 + u] > (s[u][3] ? V(u, 11) : V(u, 3));
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float a = s[u][3] ? V(u, 13) : V(u, 5), bq = s[u][3] ? V(u, 9) : V(u, 1);
        s[u][1] = x[i0 + u] > (s[u][2] ? a : bq);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float t00 = s[u][3] ? V(u, 8) : V(u, 0), t01 = s[u][3] ? V(u, 10) : V(u, 2);
        const float t10 = s[u][3] ? V(u, 12) : V(u, 4), t11 = s[u][3] ? V(u, 14) : V(u, 6);
        const float lo = s[u][1] ? t01 : t00, hi = s[u][1] ? t11 : t10;
        s[u][0] = x[i0 + u] > (s[u][2] ? hi : lo);
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

// sqrt rounded to nearest: the hardware estimate r, then r - ulp or r + ulp
// when the residual a - r' r (one fma, sign exact) shows the true root lies
// nearer to it.  No rescaling for inputs below 2^-96 (norms that small store
// as fp16 zero either way); fewer registers than the library sqrt.
__device__ __forceinline__ float sqrt_rn(float a) {
  float r = __builtin_amdgcn_sqrtf(a);
  const float rd = __int_as_float(__float_as_int(r) - 1);
  const float ru = __int_as_float(__float_as_int(r) + 1);
  if (__builtin_fmaf(-rd, r, a) <= 0.f) r = rd;
  if (__builtin_fmaf(-ru, r, a) > 0.f) r = ru;
  return r;
}

// shift_in with the lane mask given directly
__device__ __forceinline__ uint32_t shift_in_mask(uint32_t w, uint64_t m) {
  uint32_t r;
  uint64_t co;
  asm("v_addc_co_u32_e64 %0, %1, %2, %2, %3" : "=v"(r), "=s"(co) : "v"(w), "s"(m));
  return r;
}

// Symmetric codebook: sg = (a > Tm) against the middle threshold, then a
// binary search of |a| over the H = 2^(BITS-1) - 1 positive thresholds P,
// m = #{k : |a| > P_k}.  code = 2^(BITS-1) + m when sg, else
// 2^(BITS-1) - 1 - m (the negative thresholds are -P_k), so the top bit is sg
// and the low bits are m XNOR sg, combined on the compare masks.  (a == -P_k
// exactly gives the code one below #{j : a > T_j}: a boundary tie.)  Bits go
// in from the highest element down, as in quantize_pack.
template <int BITS, int E>
__device__ __forceinline__ void quantize_pack_sym(const float (&x)[E], float Tm,
                                                  const float (&P)[(1 << (BITS - 1)) - 1],
                                                  uint32_t (&w)[E * BITS / 32]) {
  static_assert((E * BITS) % 32 == 0, "whole words per lane");
#pragma unroll
  for (int k = 0; k < E * BITS / 32; ++k) w[k] = 0;
#pragma unroll
  for (int i = E - 1; i >= 0; --i) {
    const float xv = x[i];
    const float a = __builtin_fabsf(xv);
    const uint64_t sg = __builtin_amdgcn_ballot_w64(xv > Tm);
    uint64_t mb[BITS - 1];
    if constexpr (BITS == 2) {
      mb[0] = __builtin_amdgcn_ballot_w64(a > P[0]);
    } else if constexpr (BITS == 3) {
      const bool m1 = a > P[1];
      mb[1] = __builtin_amdgcn_ballot_w64(m1);
      mb[0] = __builtin_amdgcn_ballot_w64(a > (m1 ? P[2] : P[0]));
    } else {
      const bool m2 = a > P[3];
      const bool m1 = a > (m2 ? P[5] : P[1]);
      const float lo = m2 ? P[4] : P[0], hi = m2 ? P[6] : P[2];
      mb[2] = __builtin_amdgcn_ballot_w64(m2);
      mb[1] = __builtin_amdgcn_ballot_w64(m1);
      mb[0] = __builtin_amdgcn_ballot_w64(a > (m1 ? hi : lo));
    }
    {
      const int k = (BITS * i + BITS - 1) >> 5;
      w[k] = shift_in_mask(w[k], sg);
    }
#pragma unroll
    for (int b = BITS - 2; b >= 0; --b) {
      const int k = (BITS * i + b) >> 5;
      w[k] = shift_in_mask(w[k], ~(mb[b] ^ sg));
    }
  }
}

// Per-lane constants of the 128-point Hadamard transform on the matrix cores
// (layout above) and of the Gram-diagonal norm.
template <int DT>
struct Rht128 {
  Op16x8 P0, P1, N0, N1;  // A operand patterns, +-
  uint32_t jr_hi, jr_lo;  // bits 1 and 0 of j as all-ones / all-zero masks
  int diag_src;           // ds_bpermute byte address of lane (j / 4, j)

  __device__ __forceinline__ void init(int lane) {
    const int q = lane >> 4, j = lane & 15;
    const int qp = (lane >> 2) & 3, r = lane & 3;
    // A patterns: P0[t] = (-1)^(popc(r & t) + popc(q' & q)), P1[t] = P0[t] (-1)^(t >> 2)
    const uint32_t one = (DT == BF16) ? 0x3F80u : 0x3C00u;
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
    // G[j][j] of the Gram MFMA sits in lane (j / 4, j), accumulator j % 4:
    // every lane picks accumulator j % 4 and reads lane (j / 4, j)'s pick.
    // The empty asm keeps the compiler from turning the masks back into
    // compares inside the caller's loop.
    jr_hi = (j & 2) ? ~0u : 0u;
    jr_lo = (j & 1) ? ~0u : 0u;
    asm volatile("" : "+v"(jr_hi), "+v"(jr_lo));
    diag_src = (((j >> 2) << 4) | j) << 2;
  }

  // acc[8 b + mb] = H_128 x (block b of the group in cur, K steps 4 b .. 4 b + 3)
  template <int NB>
  __device__ __forceinline__ void transform(const Op16x8 (&cur)[4 * NB], f32x4_t (&acc)[8 * NB]) const {
#pragma unroll
    for (int mb = 0; mb < 8 * NB; ++mb) acc[mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int b = 0; b < NB; ++b) {
#pragma unroll
        for (int mb = 0; mb < 8; ++mb) {
          const bool neg = (__builtin_popcount((mb >> 1) & s) & 1) != 0;
          const Op16x8& a = (mb & 1) ? (neg ? N1 : P1) : (neg ? N0 : P0);
          acc[8 * b + mb] = mfma_16x16x32<DT>(a, cur[4 * b + s], acc[8 * b + mb]);
        }
      }
    }
  }

  // sum of squares of vector j (the Gram diagonal), in every lane of vector j
  template <int KS>
  __device__ __forceinline__ float sumsq(const Op16x8 (&cur)[KS]) const {
    f32x4_t gram = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) gram = mfma_16x16x32<DT>(cur[s], cur[s], gram);
    auto bsel = [](uint32_t m, float a, float b) {
      return __uint_as_float((__float_as_uint(a) & m) | (__float_as_uint(b) & ~m));
    };
    const float pick = bsel(jr_hi, bsel(jr_lo, gram[3], gram[2]), bsel(jr_lo, gram[1], gram[0]));
    return __int_as_float(__builtin_amdgcn_ds_bpermute(diag_src, __float_as_int(pick)));
  }
};

// RHT sign flips of input elements 128 b + 32 q + 8 s + t (K step 4 b + s) as
// xor masks, table[q KS + 4 b + s] for the lanes of quarter q.  The table sits
// in LDS and is read once per group (16 lanes share each entry): held in
// registers it would take KS * 4 VGPRs for the kernel's lifetime, which at
// d = 256 is the difference between 2 and 3 waves per SIMD.  Filled by the
// threads with tid in [0, 4 KS); the caller synchronises.
template <int KS>
__device__ __forceinline__ void fill_sign_table(uint4* table, const float* __restrict__ signs, int tid) {
  if (tid >= 0 && tid < 4 * KS) {
    const int qq = tid / KS, s = tid % KS;
    uint32_t m[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const int e = 128 * (s >> 2) + 32 * qq + 8 * (s & 3) + 2 * w;
      m[w] = (signs[e] < 0.f ? 0x8000u : 0u) | (signs[e + 1] < 0.f ? 0x80000000u : 0u);
    }
    table[tid] = make_uint4(m[0], m[1], m[2], m[3]);
  }
}

// z is an opaque zero (an empty asm result inside the caller's loop): the
// table reads stay inside the loop instead of being hoisted out of it into
// registers
template <int KS>
__device__ __forceinline__ void flip_signs(Op16x8 (&v)[KS], const uint4* table, int q, int z) {
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const uint4 m = table[q * KS + s + z];
    v[s].u[0] ^= m.x;
    v[s].u[1] ^= m.y;
    v[s].u[2] ^= m.z;
    v[s].u[3] ^= m.w;
  }
}

template <int D, int BITS, int DT, bool SYM>
__global__ __launch_bounds__(256) void encode_mfma_kernel(EncodeSegs io, int64_t n,
                                                          const float* __restrict__ signs,
                                                          const float* __restrict__ boundaries,
                                                          float c, double rc) {
  static_assert(D == 128 || D == 256, "MFMA encoder covers d = 128 and 256");
  static_assert(DT == BF16 || DT == F16, "MFMA encoder takes 16-bit inputs");
  constexpr int NB = D / 128;  // 128-element transform blocks
  constexpr int EL = D / 4;    // outputs (and inputs) per lane, 32 per block
  constexpr int KS = D / 32;   // K steps, 4 per block
  constexpr int MB = D / 16;   // M blocks, 8 per block
  constexpr int NT = (1 << BITS) - 1;
  constexpr int MID = 1 << (BITS - 1);  // boundaries[MID] is the middle one
  constexpr int NH = MID - 1;
  constexpr int PD = D * BITS / 8;

  const int lane = threadIdx.x & 63;
  const int q = lane >> 4, j = lane & 15;
  Rht128<DT> H;
  H.init(lane);
  __shared__ uint4 smt[4 * KS];
  fill_sign_table<KS>(smt, signs, (int)threadIdx.x);
  __syncthreads();

  // wave-uniform, so the group bookkeeping below stays on the scalar unit
  const int wave = (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gstride = (int)gridDim.x * 4;
  // groups of 16 vectors, numbered over the segments one after the other (the
  // host keeps their count below 2^31 - 2^20, so g + gstride cannot overflow)
  const int gps = (int)((n + 15) >> 4);
  const int ngroups = gps * io.nseg;

  // interior boundaries (wave-uniform)
  float Bv[NT];
#pragma unroll
  for (int k = 0; k < NT; ++k) Bv[k] = boundaries[1 + k];
  const float rcf = (float)rc;

  // groups of 16 vectors; the next group's input is loaded while the current
  // one is encoded.  Past the end the load repeats the last vector, so every
  // iteration issues the same loads and the wait counts stay static.
  // group g (clamped to the last one, so a prefetch past the end stays in
  // bounds): its segment and the index of its first vector there
  auto locate = [&](int g, int& seg, int64_t& g0) {
    g = g < ngroups ? g : ngroups - 1;
    seg = g >= gps ? 1 : 0;
    g0 = (int64_t)(g - (seg ? gps : 0)) << 4;
  };
  auto load_group = [&](int g, Op16x8 (&dst)[KS]) {
    int seg;
    int64_t g0;
    locate(g, seg, g0);
    // wave-uniform group base plus a 32-bit lane offset; rows past the end
    // read the last row (the lane's row within the group, clamped)
    const uint16_t* xb = static_cast<const uint16_t*>(seg ? io.x1 : io.x0) + g0 * D;
    const int last = (int)(n - 1 - g0 < 15 ? n - 1 - g0 : 15);
    const int jj = j < last ? j : last;
    const uint4* src = reinterpret_cast<const uint4*>(xb + (jj * D + 32 * q));
#pragma unroll
    for (int s = 0; s < KS; ++s) dst[s].v = src[16 * (s >> 2) + (s & 3)];
  };
  // t domain scale of the thresholds, RN((norm + 1e-8) / c), of the group held
  // (sign-flipped) in v; the norm itself goes to nrm
  auto norm_scale = [&](const Op16x8 (&v)[KS], float& nrm) {
    const float xx = H.sumsq(v);
    // ||t||^2 = D ||x||^2 (Parseval for the unnormalised transform)
    nrm = sqrt_rn(xx * (float)D) * c;
    return (nrm + 1e-8f) * rcf;
  };
  // encodes group g held in cur, and reloads cur with group gnext once the
  // transform and the norm no longer need it
  auto encode_group = [&](Op16x8 (&cur)[KS], int g, int gnext) {
    int z = 0;
    asm volatile("" : "+s"(z));
    flip_signs<KS>(cur, smt, q, z);
    f32x4_t acc[MB];
    H.template transform<NB>(cur, acc);
    // t[32 b + 4 mb + i] = output 128 b + 32 q + 4 mb + i
    float t[EL];
#pragma unroll
    for (int mb = 0; mb < 8; ++mb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if constexpr (NB == 1) {
          t[4 * mb + i] = acc[mb][i];
        } else {
          const float z0 = acc[mb][i], z1 = acc[8 + mb][i];
          t[4 * mb + i] = z0 + z1;
          t[32 + 4 * mb + i] = z0 - z1;
        }
      }
    constexpr int NW = EL * BITS / 32;
    uint32_t w[NW];
    float nrm;
    const float sv = norm_scale(cur, nrm);
    // the next group's loads go out here, ahead of the quantiser (whose VALU
    // work covers their latency), and no earlier: before this point the
    // registers hold the current group
    __builtin_amdgcn_sched_barrier(0);
    load_group(gnext, cur);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (SYM) {
      float P[NH];
#pragma unroll
      for (int k = 0; k < NH; ++k) P[k] = Bv[MID + k] * sv;
      quantize_pack_sym<BITS, EL>(t, Bv[MID - 1] * sv, P, w);
    } else {
      float T[1][NT];
#pragma unroll
      for (int k = 0; k < NT; ++k) T[0][k] = Bv[k] * sv;
      quantize_pack<BITS, EL>(t, T, w);
    }
    int seg;
    int64_t g0;
    locate(g, seg, g0);
    uint8_t* packed = (seg ? io.packed1 : io.packed0) + g0 * PD;
    uint16_t* norms = (seg ? io.norms1 : io.norms0) + g0;
    const int rows = (int)(n - g0 < 16 ? n - g0 : 16);
    if (j < rows) {
      // block b's codes: BITS words at word BITS (4 b + q) of the row.
      // Non-temporal stores: the codes are not read back by this launch, and
      // streaming them past the caches keeps those for the input reads (4-5%
      // faster at d = 128, K + V, and 3% at d = 256, inputs not cache
      // resident).  (Non-temporal input loads measured slower.)
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        uint32_t* dst = reinterpret_cast<uint32_t*>(packed + j * PD) + BITS * (4 * b + q);
        const uint32_t* wb = w + BITS * b;
#pragma unroll
        for (int k = 0; k < BITS; ++k) __builtin_nontemporal_store(wb[k], dst + k);
      }
      if (q == 0) __builtin_nontemporal_store((uint16_t)f32_to_f16_bits(nrm), norms + j);
    }
  };
  if (wave >= ngroups) return;
  // one register set: group g + gstride is loaded into it while group g is
  // quantised.  (Two alternating sets, loaded a whole group ahead, cost KS * 4
  // more VGPRs: 3 waves per SIMD instead of 2 at d = 256, and no faster at
  // d = 128.)
  int g = wave;
  Op16x8 cur[KS];
  load_group(g, cur);
  for (;;) {
    encode_group(cur, g, g + gstride);
    g += gstride;
    if (g >= ngroups) break;
  }
}

}  // namespace ftq
