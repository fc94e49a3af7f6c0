// vLLM v1 TURBOQUANT slot store kernel on gfx950 (shared by the translation
// units that instantiate it): quantise K and V of n tokens x Hkv heads and
// write them into their slots, for the unsigned Hadamard rotation (kind = rht)
// and for the block-diagonal rotations (planar 2x2, rotor 3x3, iso 4x4), in
// one launch.
//
// Per (token, kv head) (reference vllm_plugin/triton_inkernel_store.py:38-440,
// 554-616 for rht, 649-860 for the block-diagonal kinds):
//   K: norm = sqrt(sum k^2 + 1e-16); rht: x = k / (norm + 1e-8) through the
//      butterflies, y = x * d^-1/2; block-diagonal: x = k * (1 / (norm + 1e-8)),
//      y[e] = sum_j x[(e / B) B + j] c[j][e] in fp32 fused multiply-adds;
//      code = number of midpoints <= y (1, 2, 3, 4 or 8 bits); fp16 norm after
//      the codes.  FP8 keys (KF8, :59-83): y * norm rounded to fp8 e4m3fn
//      (nearest-even, saturating at +-448), one byte per dim, no norm.
//   V (optionally rotated first -- the same rotation, without the
//      normalisation -- and rounded back to the input dtype, v1_backend.py:
//      736-740): min / max uniform codes trunc((v - min) / scale + 0.5),
//      scale = (max - min) / (2^vb - 1) (>= 1e-8), vb = 1, 2, 3, 4 or 8
//      (:202-330), or with the Lloyd-Max flag (4-bit V) the K midpoint search
//      on v / (|v| + 1e-8), its fp16 norm in the scale field and 0 in the min
//      field (:159-200).
//
// Layout of the work: one vector per LPV = min(16, D / 8) lanes, E = D / LPV
// contiguous elements per lane (E = 8 at d = 64 and 128, 16 at d = 256), so
// a lane's codes form E * bits (8 ... 128) whole bits; they are packed in
// registers and written straight to the slot with 1-, 2- and 4-byte stores
// (no staging).  The midpoint search is a branch-free binary search on
// midpoints held in registers (bits compares and 2^bits - 1 - bits selects
// per element instead of 2^bits - 1 compares and adds); the 255 midpoints of
// 8-bit codes live in LDS and are searched by binary lifting.
// K is divided by its norm through the reciprocal and one fma correction.
// The uniform V codes divide by the scale through its correctly rounded
// reciprocal and one fused correction of the quotient, which gives the
// correctly rounded division (Markstein's theorem).
#pragma once

#include "ftq_internal.h"
#include "ftq_v1_dev.h"

namespace ftq {

float fwht_scale(int d);

// lane l reads lane l - 1 / l + 1 of its 16-lane row (0 past the row's edge)
__device__ __forceinline__ float dpp_prev(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x111, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_next(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x101, 0xF, 0xF, true));
}

// number of the NM = 2^NB - 1 sorted midpoints m[] that are <= y, as a
// binary search: each level compares against the middle of the remaining
// candidates and keeps the upper or lower half by selects.  The empty asm
// makes the two operands of each select opaque values: left alone, LLVM
// turns a select of two array elements into one element at a run-time
// index, which it then expands into an NM-way compare-and-select.
template <int NB>
__device__ __forceinline__ uint32_t mid_search(float y, const float (&m)[(1 << NB) - 1]) {
  constexpr int NM = (1 << NB) - 1;
  float cand[NM];
#pragma unroll
  for (int i = 0; i < NM; ++i) cand[i] = m[i];
  uint32_t code = 0;
#pragma unroll
  for (int lvl = 0; lvl < NB; ++lvl) {
    const int half = (1 << (NB - 1 - lvl)) - 1;  // candidates left on each side of the middle
    const bool up = y >= cand[half];
    code = (code << 1) | (up ? 1u : 0u);
#pragma unroll
    for (int i = 0; i < half; ++i) {
      float hi = cand[half + 1 + i], lo = cand[i];
      asm("" : "+v"(hi), "+v"(lo));
      cand[i] = up ? hi : lo;
    }
  }
  return code;
}

// the same count over 255 sorted midpoints in LDS, by binary lifting: the
// count is built from its high bit down, taking 2^s more whenever y >= the
// midpoint just below that step
__device__ __forceinline__ uint32_t mid_search_lds8(float y, const float* m) {
  uint32_t pos = 0;
#pragma unroll
  for (int s = 7; s >= 0; --s) {
    const uint32_t step = 1u << s;
    pos += (y >= m[pos + step - 1]) ? step : 0u;
  }
  return pos;
}

// fp32 -> fp8 e4m3fn byte: round to nearest even, saturating at +-448
// (infinities included), NaN -> 0x7f with the sign kept.  Normal results
// round the fp32 bits at mantissa bit 20 and rebias the exponent (127 -> 7);
// values below 2^-6 are multiples of 2^-9 (subnormals, and 2^-6 itself when
// they round up, whose encoding 0x08 is the same integer).
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  const uint32_t u = __float_as_uint(x);
  const uint32_t s = (u >> 24) & 0x80u;
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return s | 0x7fu;
  if (a >= 0x43e00000u) return s | 0x7eu;  // |x| >= 448
  if (a < 0x3c800000u)                     // |x| < 2^-6
    return s | (uint32_t)__builtin_rintf(__uint_as_float(a) * 512.f);
  const uint32_t r = (a + 0x7ffffu + ((a >> 20) & 1u)) >> 20;
  return s | (r - 960u);
}

// E codes of NB bits (code i at bit i * NB) into w[0 .. NW)
template <int E, int NB, int NW>
__device__ __forceinline__ void pack_codes(const uint32_t (&c)[E], uint32_t (&w)[NW]) {
  static_assert(NW * 32 >= E * NB, "room for the codes");
#pragma unroll
  for (int k = 0; k < NW; ++k) w[k] = 0;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int p = i * NB;  // compile-time after unrolling
    const int k = p >> 5, o = p & 31;
    w[k] |= c[i] << o;
    if (o + NB > 32) w[k + 1] |= c[i] >> (32 - o);  // NB = 3 across a word boundary
  }
}

// Write W = E * NB bits of lane `li` at byte base + li * W / 8.  base is
// 2-byte aligned (4-byte aligned when ALIGN4).
template <int W, bool ALIGN4, int NW>
__device__ __forceinline__ void store_bits(uint8_t* base, int li, const uint32_t (&w)[NW]) {
  static_assert(W % 8 == 0, "whole bytes per lane");
  uint8_t* p = base + li * (W / 8);
  if constexpr (W == 8) {
    p[0] = (uint8_t)w[0];
  } else if constexpr (W == 16) {
    *reinterpret_cast<uint16_t*>(p) = (uint16_t)w[0];
  } else if constexpr (W == 24) {  // 3 bytes at an odd or even offset
    if ((li & 1) == 0) {
      *reinterpret_cast<uint16_t*>(p) = (uint16_t)w[0];
      p[2] = (uint8_t)(w[0] >> 16);
    } else {
      p[0] = (uint8_t)w[0];
      *reinterpret_cast<uint16_t*>(p + 1) = (uint16_t)(w[0] >> 8);
    }
  } else if constexpr (W == 48) {
    *reinterpret_cast<uint16_t*>(p) = (uint16_t)w[0];
    *reinterpret_cast<uint16_t*>(p + 2) = (uint16_t)(w[0] >> 16);
    *reinterpret_cast<uint16_t*>(p + 4) = (uint16_t)w[1];
  } else {
    static_assert(W == 32 || W == 64 || W == 128, "8 ... 128 bits per lane");
    constexpr int ND = W / 32;
    if constexpr (ALIGN4) {
#pragma unroll
      for (int h = 0; h < ND; ++h) *reinterpret_cast<uint32_t*>(p + 4 * h) = w[h];
    } else {
#pragma unroll
      for (int h = 0; h < 2 * ND; ++h)
        *reinterpret_cast<uint16_t*>(p + 2 * h) = (uint16_t)(w[h >> 1] >> (16 * (h & 1)));
    }
  }
}

// x <- x M for a block-diagonal M with RB x RB blocks, from its coefficients
// cf[j][i] = M[(e / RB) RB + j][e] of the lane's elements e = li * E + i:
// y[e] = fma(x_{RB-1}, c_{RB-1}, ... fma(x_1, c_1, x_0 c_0)) with the partners
// x_j = x[(e / RB) RB + j].  For RB = 2 and 4 they are in the lane; for
// RB = 3 a group can start up to 2 elements before the lane's first element
// or end up to 2 after its last, so the lane also takes the last two
// elements of the previous lane and the first two of the next (DPP row
// moves) and picks each partner from that window by the element's position
// in its group, p = (li * E + i) mod 3.
template <int D, int E, int LPV, int RB>
__device__ __forceinline__ void rot_blockdiag(float (&x)[E], const float (&cf)[RB][E], int li) {
  float y[E];
  if constexpr (RB == 3) {
    float win[E + 4];  // x[-2 .. E + 1] relative to the lane's first element
    // The row moves run with every lane of the row enabled: a DPP read from a
    // lane that is switched off returns 0, so they must not be sunk into the
    // select below (the empty asm pins them before it).
    float p0v = dpp_prev(x[E - 2]), p1v = dpp_prev(x[E - 1]);
    float n0v = dpp_next(x[0]), n1v = dpp_next(x[1]);
    asm volatile("" : "+v"(p0v), "+v"(p1v), "+v"(n0v), "+v"(n1v));
    win[0] = p0v;
    win[1] = p1v;
#pragma unroll
    for (int i = 0; i < E; ++i) win[i + 2] = x[i];
    const bool last = li == LPV - 1;  // partners past D: zero coefficients, and no neighbour to read
    win[E + 2] = last ? 0.f : n0v;
    win[E + 3] = last ? 0.f : n1v;
    const int r = (li * E) % 3;  // position of element 0 in its group
#pragma unroll
    for (int i = 0; i < E; ++i) {
      // p = (r + i) mod 3 is 0 / 1 / 2 when r is (3 - i % 3) % 3, (4 - i % 3) % 3, (5 - i % 3) % 3
      const bool p0 = r == (3 - i % 3) % 3;
      const bool p1 = r == (4 - i % 3) % 3;
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        // partner index e - p + j, as a window slot: i + 2 - p + j
        const float xp = p0 ? win[i + 2 + j] : (p1 ? win[i + 1 + j] : win[i + j]);
        y[i] = j == 0 ? xp * cf[j][i] : __builtin_fmaf(xp, cf[j][i], y[i]);
      }
    }
  } else {
    static_assert(E % RB == 0, "2x2 and 4x4 blocks lie inside a lane");
#pragma unroll
    for (int i = 0; i < E; ++i)
#pragma unroll
      for (int j = 0; j < RB; ++j) {
        const float xp = x[(i / RB) * RB + j];
        y[i] = j == 0 ? xp * cf[j][i] : __builtin_fmaf(xp, cf[j][i], y[i]);
      }
  }
#pragma unroll
  for (int i = 0; i < E; ++i) x[i] = y[i];
}

// KB: key code bits (1, 2, 3, 4 or 8; 8 with KF8 = fp8 keys); VB: value bits
// (1, 2, 3, 4 or 8).
template <int D, int DT, int KB, int VB, int RB, bool KF8 = false>
__global__ __launch_bounds__(256) void v1_store_fast_kernel(
    const void* __restrict__ key, const void* __restrict__ value, int64_t n_tokens, int hkv,
    const float* __restrict__ mid_g, int vflags, const int64_t* __restrict__ slot_mapping,
    uint8_t* __restrict__ cache, int64_t num_blocks, int block_size, int64_t s_blk, int64_t s_pos,
    int64_t s_head, float rscale, const float* __restrict__ coeffs) {
  constexpr int LPV = D >= 128 ? 16 : D / 8;
  constexpr int E = D / LPV;
  constexpr int VPB = 256 / LPV;  // vectors per workgroup pass
  constexpr bool MIDS_LDS = KB == 8 && !KF8;
  constexpr int NMK = (KB <= 4) ? (1 << KB) - 1 : 1;  // midpoints held in registers
  constexpr V1Geom G = v1_geom(D, KB, VB, KF8);
  constexpr int VTOP = (1 << VB) - 1;
  constexpr int NWK = (E * KB + 31) / 32, NWV = (E * VB + 31) / 32;
  constexpr int NW = NWK > NWV ? NWK : NWV;
  static_assert(RB == 0 || RB == 2 || RB == 3 || RB == 4, "rotation: Hadamard or 2/3/4 blocks");
  static_assert(!KF8 || KB == 8, "fp8 keys take one byte per dim");
  // li: the vector chunk the lane holds (the Hadamard rotation uses the
  // permuted lane layout of fwht_lanes_perm; rsg is its sign times the scale)
  const int li = RB == 0 ? fwht_perm_lane<LPV>((int)threadIdx.x % LPV) : (int)threadIdx.x % LPV;
  const int grp = threadIdx.x / LPV;
  const float rsg = rscale * fwht_perm_sign<LPV>(li);

  float mids[NMK];
  __shared__ float mid_l[MIDS_LDS ? 256 : 1];
  if constexpr (MIDS_LDS) {
    if (threadIdx.x < 255) mid_l[threadIdx.x] = mid_g[threadIdx.x];
    __syncthreads();
  } else if constexpr (!KF8) {
#pragma unroll
    for (int j = 0; j < NMK; ++j) mids[j] = mid_g[j];
  }
  float cf[RB == 0 ? 1 : RB][E];
  if constexpr (RB != 0) {
#pragma unroll
    for (int j = 0; j < RB; ++j)
#pragma unroll
      for (int i = 0; i < E; ++i) cf[j][i] = coeffs[j * D + li * E + i];
  }
  const bool vrot = (vflags & 1) != 0;
  const bool vlm = (vflags & 2) != 0 && VB == 4 && KB <= 4 && !KF8;
  const int64_t nvec = n_tokens * hkv;

  for (int64_t base = (int64_t)blockIdx.x * VPB; base < nvec; base += (int64_t)gridDim.x * VPB) {
    const int64_t vi = base + grp;
    if (vi >= nvec) continue;  // uniform over the vector's lanes
    const int64_t tok = vi / hkv;
    const int head = (int)(vi - tok * hkv);
    const int64_t slot = slot_mapping[tok];
    if (slot < 0) continue;  // skipped token
    const int64_t blk = slot / block_size;
    if (blk >= num_blocks) continue;
    uint8_t* sp = cache + blk * s_blk + (slot - blk * block_size) * s_pos + (int64_t)head * s_head;

    // ---- K
    float x[E];
    load_elems<DT, E>(key, vi * D + li * E, x);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < E; ++i) ss = __builtin_fmaf(x[i], x[i], ss);
    ss = RB == 0 ? group_sum_perm<LPV>(ss) : group_sum<LPV>(ss);
    const float nrm = __builtin_sqrtf(ss + 1e-16f);
    const float den = nrm + 1e-8f;
    if constexpr (RB == 0) {
      // x / den through the reciprocal and one fma correction of the
      // quotient (Markstein): the correctly rounded quotient in all but rare
      // cases, and within an ulp there, where only a code within a few ulps
      // of a midpoint can change
      const float rd = 1.f / den;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const float q0 = x[i] * rd;
        x[i] = __builtin_fmaf(__builtin_fmaf(-q0, den, x[i]), rd, q0);
      }
      fwht_lanes_perm<E, LPV>(x, li);
#pragma unroll
      for (int i = 0; i < E; ++i) x[i] *= rsg;
    } else {
      const float inv = 1.f / den;
#pragma unroll
      for (int i = 0; i < E; ++i) x[i] *= inv;
      rot_blockdiag<D, E, LPV, RB>(x, cf, li);
    }
    uint32_t c[E], w[NW];
#pragma unroll
    for (int i = 0; i < E; ++i) {
      if constexpr (KF8) c[i] = f32_to_e4m3(x[i] * nrm);
      else if constexpr (MIDS_LDS) c[i] = mid_search_lds8(x[i], mid_l);
      else c[i] = mid_search<KB>(x[i], mids);
    }
    pack_codes<E, KB, NW>(c, w);
    store_bits<E * KB, true, NW>(sp, li, w);

    // ---- V
    float v[E];
    load_elems<DT, E>(value, vi * D + li * E, v);
    if (vrot) {
      if constexpr (RB == 0) {
        fwht_lanes_perm<E, LPV>(v, li);
#pragma unroll
        for (int i = 0; i < E; ++i) v[i] = round_to_dtype<DT>(v[i] * rsg);
      } else {
        rot_blockdiag<D, E, LPV, RB>(v, cf, li);
#pragma unroll
        for (int i = 0; i < E; ++i) v[i] = round_to_dtype<DT>(v[i]);
      }
    }
    float sc = 0.f, mn = 0.f;
    bool coded = false;
    if constexpr (VB == 4 && KB <= 4 && !KF8) {
      if (vlm) {
        float vs = 0.f;
#pragma unroll
        for (int i = 0; i < E; ++i) vs = __builtin_fmaf(v[i], v[i], vs);
        vs = RB == 0 ? group_sum_perm<LPV>(vs) : group_sum<LPV>(vs);
        sc = __builtin_sqrtf(vs + 1e-16f);
        const float vden = sc + 1e-8f;
#pragma unroll
        for (int i = 0; i < E; ++i) c[i] = mid_search<KB>(v[i] / vden, mids);
        pack_codes<E, 4, NW>(c, w);
        coded = true;
      }
    }
    if (!coded) {
      mn = v[0];
      float mx = v[0];
#pragma unroll
      for (int i = 1; i < E; ++i) {
        mn = fminf(mn, v[i]);
        mx = fmaxf(mx, v[i]);
      }
#pragma unroll
      for (int m = 1; m < LPV; m <<= 1) {
        if (m == 1) { mn = fminf(mn, lane_xor<1>(mn)); mx = fmaxf(mx, lane_xor<1>(mx)); }
        else if (m == 2) { mn = fminf(mn, lane_xor<2>(mn)); mx = fmaxf(mx, lane_xor<2>(mx)); }
        else if (m == 4) {
          mn = fminf(mn, RB == 0 ? lane_pair<4>(mn) : lane_xor<4>(mn));
          mx = fmaxf(mx, RB == 0 ? lane_pair<4>(mx) : lane_xor<4>(mx));
        } else { mn = fminf(mn, lane_xor<8>(mn)); mx = fmaxf(mx, lane_xor<8>(mx)); }
      }
      // a rotated zero minimum is stored as +0 (the butterflies' zeros can
      // carry either sign, the dense product's are +0; no code or scale
      // depends on which); an input's own -0.0 minimum is kept
      if (vrot) mn = mn + 0.f;
      sc = (VB == 1) ? (mx - mn) : (mx - mn) / (float)VTOP;
      sc = sc > 1e-8f ? sc : 1e-8f;
      // (v - mn) / sc correctly rounded: the reciprocal's quotient and one
      // fused correction (Markstein: rs = RN(1 / sc), q0 within an ulp)
      const float rs = 1.f / sc;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const float dv = v[i] - mn;
        const float q0 = dv * rs;
        const float q = __builtin_fmaf(__builtin_fmaf(-q0, sc, dv), rs, q0);
        // trunc(q + 0.5) clamped to [0, VTOP]; NaN -> 0 (fmaxf takes the number)
        c[i] = (uint32_t)fminf(fmaxf(q + 0.5f, 0.f), (float)VTOP);
      }
      pack_codes<E, VB, NW>(c, w);
    }
    store_bits<E * VB, false, NW>(sp + G.kps, li, w);
    if (li == 0) {
      if constexpr (!KF8) *reinterpret_cast<uint16_t*>(sp + G.mse) = (uint16_t)f32_to_f16_bits(nrm);
      *reinterpret_cast<uint16_t*>(sp + G.kps + G.vdb) = (uint16_t)f32_to_f16_bits(sc);
      *reinterpret_cast<uint16_t*>(sp + G.kps + G.vdb + 2) = (uint16_t)f32_to_f16_bits(mn);
    }
  }
}

template <int D, int KB, int VB, int RB, bool KF8 = false>
static hipError_t launch_fast_store4(const void* k, const void* v, int dt, int64_t n, int hkv, const float* mids,
                                     int vflags, const int64_t* slots, uint8_t* cache, int64_t nb, int bs,
                                     int64_t sb, int64_t sp, int64_t sh, const float* coeffs, hipStream_t st) {
  constexpr int LPV = D >= 128 ? 16 : D / 8;
  constexpr int VPB = 256 / LPV;
  const int64_t nvec = n * hkv;
  int64_t g = (nvec + VPB - 1) / VPB;
  if (g > 256 * 16) g = 256 * 16;
  const float rs = fwht_scale(D);
  dim3 grid((unsigned)g), block(256);
  if (dt == F32)
    v1_store_fast_kernel<D, F32, KB, VB, RB, KF8><<<grid, block, 0, st>>>(k, v, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, rs, coeffs);
  else if (dt == F16)
    v1_store_fast_kernel<D, F16, KB, VB, RB, KF8><<<grid, block, 0, st>>>(k, v, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, rs, coeffs);
  else
    v1_store_fast_kernel<D, BF16, KB, VB, RB, KF8><<<grid, block, 0, st>>>(k, v, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, rs, coeffs);
  return hipGetLastError();
}

template <int D, int KB, int VB, bool KF8 = false>
static hipError_t launch_fast_store3(int rb, const void* k, const void* v, int dt, int64_t n, int hkv,
                                     const float* mids, int vflags, const int64_t* slots, uint8_t* cache,
                                     int64_t nb, int bs, int64_t sb, int64_t sp, int64_t sh, const float* coeffs,
                                     hipStream_t st) {
  switch (rb) {
    case 2: return launch_fast_store4<D, KB, VB, 2, KF8>(k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
    case 3: return launch_fast_store4<D, KB, VB, 3, KF8>(k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
    case 4: return launch_fast_store4<D, KB, VB, 4, KF8>(k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
    default: return launch_fast_store4<D, KB, VB, 0, KF8>(k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
  }
}

// The launch of the combinations outside K, V in {2, 3, 4} (1-bit codes,
// 8-bit K and V, fp8 keys); defined in ftq_v1_store_ext.hip.
hipError_t v1_store_ext_launch(int d, int kb, int vb, bool kf8, int rb, const void* k, const void* v, int dt,
                               int64_t n, int hkv, const float* mids, int vflags, const int64_t* slots,
                               uint8_t* cache, int64_t nb, int bs, int64_t sb, int64_t sp, int64_t sh,
                               const float* coeffs, hipStream_t st);

}  // namespace ftq
