// vLLM v1 TURBOQUANT slot store, Hadamard rotation (kind = rht) at d = 128
// with 16-bit inputs: K's rotation and V's pre-rotation on the matrix cores.
//
// Same slot bytes as v1_store_fast_kernel (reference
// vllm_plugin/triton_inkernel_store.py:38-440, 554-616; V pre-rotation
// v1_backend.py:736-740), computed in another order:
//
//   K: t = H k (unnormalised Sylvester product of the 16-bit input, fp32
//      accumulation), norm = sqrt(sum k^2 + 1e-16) from the Gram diagonal,
//      and the codes compare t with per-vector thresholds in the t domain,
//      T_j = RN(m_j * RN((norm + 1e-8) / c)), c = f32(d^-1/2): the number of
//      midpoints m_j <= y for y = (k / (norm + 1e-8)) H c.  t and T_j differ
//      from the reference's butterflies of the divided k by a few fp32 ulps,
//      so a code can differ only for y within that distance of a midpoint (a
//      tie; the tests bound and count them).  With a symmetric midpoint set
//      (m_j == -m_{2^KB-2-j}, so the middle one is 0, as the Lloyd-Max sets
//      of d = 64 and 128 are) the search runs on |t| over the positive
//      thresholds with the sign test picking the half; otherwise over all.
//   V: rotated (V1F_VROT) as bf16/f16(f32(H v) * c), the dense product of the
//      reference's fp32 matrix H c up to its summation order (ties counted by
//      the tests); then the min/max uniform codes of v1_store_fast_kernel.
//
// Layout of the work (as the library-format encoder, ftq_encode_mfma.h): a
// wave takes 16 consecutive (token, head) vectors at a time; lane
// (q, j) = (lane / 16, lane % 16) holds elements [32 q, 32 q + 32) of vector
// j before and after the transform, so its codes are 4 KB / 4 VB contiguous
// bytes of the slot.  The next group's K is loaded once K's transform and
// norm are done, its V once V's are, so the loads overlap the quantisers.
#pragma once

#include "ftq_encode_mfma.h"
#include "ftq_v1_dev.h"

namespace ftq {

// n / d for 0 <= n < 2^31 and 1 <= d < 2^31 with a wave-uniform multiplier
// (kernel arguments, so no reciprocal in a vector register): with
// s = max(1, ceil(log2 d)) and m = floor(2^(31+s) / d) + 1 < 2^32,
// floor(n m / 2^(31+s)) = floor(n / d), since m d - 2^(31+s) lies in (0, d]
// and n (m d - 2^(31+s)) < 2^(31+s).  d = 1 (whose m would need 33 bits) is
// its own case.
struct FastDiv {
  uint32_t m;
  int sh;  // s - 1
  int d;
  static FastDiv make(int d) {
    FastDiv f{0u, 0, d};
    if (d > 1) {
      int s = 1;
      while ((1ll << s) < d) ++s;
      f.m = (uint32_t)(((uint64_t)1 << (31 + s)) / (uint64_t)d + 1u);
      f.sh = s - 1;
    }
    return f;
  }
  __device__ __forceinline__ int div(int n) const {
    return d == 1 ? n : (int)(__umulhi((uint32_t)n, m) >> sh);
  }
};

// Codes of E elements = number of the 2^KB - 1 sorted thresholds T_j <= x
// (binary search, y >= m going up as the reference's store), packed
// little-endian into E * KB / 32 words from the highest element down.
template <int KB, int E>
__device__ __forceinline__ void v1_kcodes_search(const float (&x)[E], const float (&T)[(1 << KB) - 1],
                                                 uint32_t (&w)[E * KB / 32]) {
  static_assert((E * KB) % 32 == 0, "whole words per lane");
#pragma unroll
  for (int k = 0; k < E * KB / 32; ++k) w[k] = 0;
#pragma unroll
  for (int i = E - 1; i >= 0; --i) {
    const float xv = x[i];
    bool b[KB];
    if constexpr (KB == 2) {
      b[1] = xv >= T[1];
      b[0] = xv >= (b[1] ? T[2] : T[0]);
    } else if constexpr (KB == 3) {
      b[2] = xv >= T[3];
      b[1] = xv >= (b[2] ? T[5] : T[1]);
      const float lo = b[2] ? T[4] : T[0], hi = b[2] ? T[6] : T[2];
      b[0] = xv >= (b[1] ? hi : lo);
    } else {
      static_assert(KB == 4, "2, 3 or 4-bit keys");
      b[3] = xv >= T[7];
      b[2] = xv >= (b[3] ? T[11] : T[3]);
      const float a = b[3] ? T[13] : T[5], bq = b[3] ? T[9] : T[1];
      b[1] = xv >= (b[2] ? a : bq);
      const float t00 = b[3] ? T[8] : T[0], t01 = b[3] ? T[10] : T[2];
      const float t10 = b[3] ? T[12] : T[4], t11 = b[3] ? T[14] : T[6];
      const float lo = b[1] ? t01 : t00, hi = b[1] ? t11 : t10;
      b[0] = xv >= (b[2] ? hi : lo);
    }
#pragma unroll
    for (int bit = KB - 1; bit >= 0; --bit) {
      const int k = (KB * i + bit) >> 5;
      w[k] = shift_in_mask(w[k], __builtin_amdgcn_ballot_w64(b[bit]));
    }
  }
}

// The same codes for a symmetric threshold set (middle threshold 0, the
// positive ones P[0 .. 2^(KB-1) - 2]): sg = x >= 0 gives the top bit and
// m = #{k : P_k <= |x|} the low bits, m itself when sg, its complement
// (2^(KB-1) - 1 - m) otherwise.  Exact but at x == -P_k, where the reference
// counts P_k and this form does not (a tie).
template <int KB, int E>
__device__ __forceinline__ void v1_kcodes_sym(const float (&x)[E], const float (&P)[(1 << (KB - 1)) - 1],
                                              uint32_t (&w)[E * KB / 32]) {
  static_assert((E * KB) % 32 == 0 && E % 4 == 0, "whole words per lane, 4 elements a step");
#pragma unroll
  for (int k = 0; k < E * KB / 32; ++k) w[k] = 0;
  // four elements a step: their compares are independent, so each select
  // and each carry-add finds its mask written a few instructions earlier
#pragma unroll
  for (int i0 = E - 4; i0 >= 0; i0 -= 4) {
    uint64_t sg[4], mb[4][KB - 1];
    float a[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      a[u] = __builtin_fabsf(x[i0 + u]);
      sg[u] = __builtin_amdgcn_ballot_w64(x[i0 + u] >= 0.f);
    }
    if constexpr (KB == 2) {
#pragma unroll
      for (int u = 0; u < 4; ++u) mb[u][0] = __builtin_amdgcn_ballot_w64(a[u] >= P[0]);
    } else if constexpr (KB == 3) {
      bool m1[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        m1[u] = a[u] >= P[1];
        mb[u][1] = __builtin_amdgcn_ballot_w64(m1[u]);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) mb[u][0] = __builtin_amdgcn_ballot_w64(a[u] >= (m1[u] ? P[2] : P[0]));
    } else {
      bool m2[4], m1[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        m2[u] = a[u] >= P[3];
        mb[u][2] = __builtin_amdgcn_ballot_w64(m2[u]);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        m1[u] = a[u] >= (m2[u] ? P[5] : P[1]);
        mb[u][1] = __builtin_amdgcn_ballot_w64(m1[u]);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float lo = m2[u] ? P[4] : P[0], hi = m2[u] ? P[6] : P[2];
        mb[u][0] = __builtin_amdgcn_ballot_w64(a[u] >= (m1[u] ? hi : lo));
      }
    }
#pragma unroll
    for (int u = 3; u >= 0; --u) {
      const int i = i0 + u;
      {
        const int k = (KB * i + KB - 1) >> 5;
        w[k] = shift_in_mask(w[k], sg[u]);
      }
#pragma unroll
      for (int bit = KB - 2; bit >= 0; --bit) {
        const int k = (KB * i + bit) >> 5;
        w[k] = shift_in_mask(w[k], ~(mb[u][bit] ^ sg[u]));
      }
    }
  }
}

// Min / max uniform codes of the lane's E elements, code = trunc((v - mn) /
// sc + 0.5) clamped to [0, 2^VB - 1] (reference
// triton_inkernel_store.py:202-330), with the division correctly rounded by
// one fused correction of the reciprocal's quotient: rs = RN(1 / sc) (an IEEE
// division, once per vector), q0 = RN(d rs), r = d - q0 sc (exact, one fma),
// q = RN(q0 + r rs) = RN(d / sc) (Markstein's theorem: rs within half an ulp
// of 1 / sc and q0 within an ulp of d / sc make the corrected quotient the
// rounded one).  Codes are packed at bit VB e of E * VB / 32 words.
template <int VB, int E>
__device__ __forceinline__ void v1_vcodes_uniform(const float (&v)[E], float mn, float sc,
                                                  uint32_t (&w)[E * VB / 32]) {
  constexpr int VTOP = (1 << VB) - 1;
  const float rs = 1.f / sc;
#pragma unroll
  for (int k = 0; k < E * VB / 32; ++k) w[k] = 0;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const float d = v[i] - mn;
    const float q0 = d * rs;
    const float q = __builtin_fmaf(__builtin_fmaf(-q0, sc, d), rs, q0);
    // trunc(q + 0.5) clamped to [0, VTOP]; NaN -> 0 (fmaxf takes the number)
    const uint32_t c = (uint32_t)fminf(fmaxf(q + 0.5f, 0.f), (float)VTOP);
    const int p = VB * i, k = p >> 5, o = p & 31;
    w[k] |= c << o;
    if (o + VB > 32) w[k + 1] |= c >> (32 - o);
  }
}

template <int DT, int KB, int VB>
__global__ __launch_bounds__(256, 4) void v1_store_mfma_kernel(
    const void* __restrict__ key, const void* __restrict__ value, int nvec, int hkv, FastDiv hdiv,
    const float* __restrict__ mid_g, int vflags, const int64_t* __restrict__ slot_mapping,
    uint8_t* __restrict__ cache, int slots_total, int block_size, FastDiv bdiv, int64_t s_blk, int64_t s_pos,
    int64_t s_head, float c) {
  constexpr int D = 128, KS = 4, EL = 32;
  constexpr int NMK = (1 << KB) - 1, MID = 1 << (KB - 1), NH = MID - 1;
  constexpr V1Geom G = v1_geom(D, KB, VB, false);
  constexpr int VTOP = (1 << VB) - 1;
  static_assert(DT == BF16 || DT == F16, "16-bit inputs");

  const int lane = threadIdx.x & 63;
  const int q = lane >> 4, j = lane & 15;
  Rht128<DT> H;
  H.init(lane);
  const int wave = (int)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gstride = (int)gridDim.x * 4;
  const int ngroups = (nvec + 15) >> 4;
  if (wave >= ngroups) return;

  // midpoints (wave-uniform) and whether they are symmetric about 0
  float M[NMK];
#pragma unroll
  for (int k = 0; k < NMK; ++k) M[k] = mid_g[k];
  bool sym = true;
#pragma unroll
  for (int k = 0; k < NMK; ++k) sym = sym && (M[k] == -M[NMK - 1 - k]);
  const bool vrot = (vflags & 1) != 0;

  // rows past the end read the last row (every iteration issues the same
  // loads); the lane's row of group g is 16 g + j.  A wave-uniform group base
  // plus a 32-bit lane offset, the same for K and V.
  auto load_group = [&](const void* src, int g, Op16x8 (&dst)[KS]) __attribute__((always_inline)) {
    g = g < ngroups ? g : ngroups - 1;
    const uint8_t* gb = static_cast<const uint8_t*>(src) + (int64_t)g * (16 * D * 2);
    const int last = nvec - 1 - 16 * g;
    const uint32_t off = (uint32_t)((j < last ? j : last) * (D * 2) + 64 * q);
#pragma unroll
    for (int s = 0; s < KS; ++s) dst[s].v = *reinterpret_cast<const uint4*>(gb + off + 16 * s);
  };

  Op16x8 ck[KS], cv[KS];
  int g = wave;
  load_group(key, g, ck);
  for (;;) {
    const int gn = g + gstride;
    // the lane's vector: its slot (-1: no store)
    const int vi = 16 * g + j;
    int live_slot = -1;
    int tok = 0, head = 0;
    if (vi < nvec) {
      tok = hdiv.div(vi);
      head = vi - tok * hkv;
      const int64_t s = slot_mapping[tok];
      if (s >= 0 && s < (int64_t)slots_total) live_slot = (int)s;
    }
    const bool live = live_slot >= 0;
    uint8_t* sp = cache;
    if (live) {
      const int blk = bdiv.div(live_slot);
      sp = cache + (int64_t)blk * s_blk + (int64_t)(live_slot - blk * block_size) * s_pos + (int64_t)head * s_head;
    }

    // ---- K: t = H k on the matrix cores; the norm by Parseval, ||k||^2 =
    // ||t||^2 / d, summed over the lane's 32 outputs and the vector's 4 lanes
    f32x4_t acc[8];
    float nrm;
    H.template transform<1>(ck, acc);
    __builtin_amdgcn_sched_barrier(0);
    load_group(value, g, cv);
    load_group(key, gn, ck);
    __builtin_amdgcn_sched_barrier(0);
    {
      float t[EL];
#pragma unroll
      for (int mb = 0; mb < 8; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) t[4 * mb + i] = acc[mb][i];
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < EL; ++i) ss = __builtin_fmaf(t[i], t[i], ss);
      ss += __shfl_xor(ss, 16);
      ss += __shfl_xor(ss, 32);
      nrm = sqrt_rn(ss * (1.f / D) + 1e-16f);
      const float S = (nrm + 1e-8f) / c;  // y >= m  <=>  t >= m S
      uint32_t w[KB];
      if (sym) {
        float P[NH];
#pragma unroll
        for (int k = 0; k < NH; ++k) P[k] = M[MID + k] * S;
        v1_kcodes_sym<KB, EL>(t, P, w);
      } else {
        float T[NMK];
#pragma unroll
        for (int k = 0; k < NMK; ++k) T[k] = M[k] * S;
        v1_kcodes_search<KB, EL>(t, T, w);
      }
      if (live) {
        uint32_t* dst = reinterpret_cast<uint32_t*>(sp) + KB * q;
#pragma unroll
        for (int k = 0; k < KB; ++k) dst[k] = w[k];
        if (q == 0) *reinterpret_cast<uint16_t*>(sp + G.mse) = (uint16_t)f32_to_f16_bits(nrm);
      }
    }

    // ---- V: rotated on the matrix cores and rounded to the input dtype, or as loaded
    float v[EL];
    if (vrot) {
      H.template transform<1>(cv, acc);
#pragma unroll
      for (int mb = 0; mb < 8; ++mb)
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
          const float a0 = acc[mb][i] * c, a1 = acc[mb][i + 1] * c;
          if constexpr (DT == BF16) {
            // v_cvt_pk_bf16_f32: two roundings to nearest even in one instruction
            typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
            typedef float f32x2_t __attribute__((ext_vector_type(2)));
            const bf16x2_t r = __builtin_convertvector((f32x2_t{a0, a1}), bf16x2_t);
            v[4 * mb + i] = (float)r.x;
            v[4 * mb + i + 1] = (float)r.y;
          } else {
            v[4 * mb + i] = round_to_dtype<DT>(a0);
            v[4 * mb + i + 1] = round_to_dtype<DT>(a1);
          }
        }
    } else {
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          v[8 * s + 2 * h] = half_bits_to_f32(DT, cv[s].u[h] & 0xffffu);
          v[8 * s + 2 * h + 1] = half_bits_to_f32(DT, cv[s].u[h] >> 16);
        }
    }
    float mn = v[0], mx = v[0];
#pragma unroll
    for (int i = 1; i < EL; ++i) {
      mn = fminf(mn, v[i]);
      mx = fmaxf(mx, v[i]);
    }
    // lanes j, j + 16, j + 32, j + 48 hold the vector's four quarters
    mn = fminf(mn, __shfl_xor(mn, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mn = fminf(mn, __shfl_xor(mn, 32));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // a rotated zero minimum is stored as +0 (the dense product's zeros are
    // +0); an input's own -0.0 minimum is kept
    if (vrot) mn = mn + 0.f;
    float sc = (mx - mn) / (float)VTOP;
    sc = sc > 1e-8f ? sc : 1e-8f;
    uint32_t w[VB];
    v1_vcodes_uniform<VB, EL>(v, mn, sc, w);
    if (live) {
      // V codes start 2 bytes past a 4-byte boundary: 16-bit stores
      uint16_t* dst = reinterpret_cast<uint16_t*>(sp + G.kps + 4 * VB * q);
#pragma unroll
      for (int k = 0; k < 2 * VB; ++k) dst[k] = (uint16_t)(w[k >> 1] >> (16 * (k & 1)));
      if (q == 0) {
        *reinterpret_cast<uint16_t*>(sp + G.kps + G.vdb) = (uint16_t)f32_to_f16_bits(sc);
        *reinterpret_cast<uint16_t*>(sp + G.kps + G.vdb + 2) = (uint16_t)f32_to_f16_bits(mn);
      }
    }
    g = gn;
    if (g >= ngroups) break;
  }
}

}  // namespace ftq
