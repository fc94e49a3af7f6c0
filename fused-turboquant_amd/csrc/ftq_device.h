// Device helpers shared by the fused-turboquant HIP kernels (gfx950 / CDNA4).
//
// Lane layout used by the codec kernels: one vector of D elements is held by
// a group of LPV = D / E lanes, lane j holding the E contiguous elements
// [j*E, (j+1)*E).  The Walsh-Hadamard butterflies with stride h < E run inside
// the lane's registers; strides h >= E pair lane j with lane j ^ (h / E) and
// use DPP row permutes (no LDS traffic).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

namespace ftq {

// ---- DPP cross-lane moves inside a 16-lane row ----------------------------
// dpp_ctrl encodings (GFX9 DPP): quad_perm = p0 | p1<<2 | p2<<4 | p3<<6,
// row_shl:n = 0x100+n (lane l reads l+n), row_shr:n = 0x110+n (lane l reads
// l-n), row_ror:n = 0x120+n.
// (mov_dpp with bound_ctrl set: every lane's source is inside its row, so no
// "old" value is needed and LLVM can fold the permute into the consuming VALU op)
__device__ __forceinline__ float dpp_xor1(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_xor2(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_xor4(float v) {
  int x = __float_as_int(v);
  // banks 0 and 2 (lanes 0-3, 8-11 of each row) read lane+4, banks 1 and 3 read lane-4
  int t = __builtin_amdgcn_update_dpp(x, x, 0x104, 0xF, 0x5, false);
  t = __builtin_amdgcn_update_dpp(t, x, 0x114, 0xF, 0xA, false);
  return __int_as_float(t);
}
__device__ __forceinline__ float dpp_xor8(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, true));
}
__device__ __forceinline__ uint32_t dpp_xor1_u(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
}
// lane q of each quad reads lane min(q+1, 3) of the same quad
__device__ __forceinline__ uint32_t dpp_quad_next(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xF9, 0xF, 0xF, false);
}

template <int M>
__device__ __forceinline__ float lane_xor(float v) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8, "lane xor within a 16-lane row");
  if constexpr (M == 1) return dpp_xor1(v);
  else if constexpr (M == 2) return dpp_xor2(v);
  else if constexpr (M == 4) return dpp_xor4(v);
  else return dpp_xor8(v);
}

// Sum over the LPV lanes of a vector group.  Every lane ends with the same
// bits: each xor stage adds the same two operands in either order.
template <int LPV>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (LPV >= 2) v += lane_xor<1>(v);
  if constexpr (LPV >= 4) v += lane_xor<2>(v);
  if constexpr (LPV >= 8) v += lane_xor<4>(v);
  if constexpr (LPV >= 16) v += lane_xor<8>(v);
  return v;
}

// ---- Walsh-Hadamard butterflies ------------------------------------------
// Unnormalised FWHT of a D-vector held as E elements per lane in LPV lanes,
// stages in the order h = 1, 2, 4, ..., D/2.  Each stage maps the pair
// (x[i], x[i+h]) to (x[i] + x[i+h], x[i] - x[i+h]), so the result is
// bit-identical to any implementation that uses the same stage order.
template <int E, int LPV>
__device__ __forceinline__ void fwht_lanes(float (&x)[E], int lane_in_group) {
#pragma unroll
  for (int h = 1; h < E; h <<= 1) {
#pragma unroll
    for (int i = 0; i < E; ++i) {
      if ((i & h) == 0) {
        float a = x[i], b = x[i + h];
        x[i] = a + b;
        x[i + h] = a - b;
      }
    }
  }
#pragma unroll
  for (int m = 1; m < LPV; m <<= 1) {
    const bool upper = (lane_in_group & m) != 0;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      float p;
      if (m == 1) p = lane_xor<1>(x[i]);
      else if (m == 2) p = lane_xor<2>(x[i]);
      else if (m == 4) p = lane_xor<4>(x[i]);
      else p = lane_xor<8>(x[i]);
      x[i] = upper ? (p - x[i]) : (x[i] + p);
    }
  }
}

// ---- the same butterflies, one VALU op per element per cross-lane stage ----
// Two changes to the lane layout and the arithmetic; neither changes which
// values are added in which order, so the magnitudes are fwht_lanes' bits:
//  - Chunk j of the vector (elements [jE, (j+1)E)) sits in lane
//    fwht_perm_lane(j) of its group: chunks with bit 2 set swap their low two
//    lane bits. The stride-4 partner j ^ 4 is then the row_half_mirror
//    partner (lane l <-> 7 - l of each 8), one DPP move; strides 1, 2 and 8
//    stay quad_perm / row_ror:8 moves. (The map is its own inverse.)
//  - The upper lane of a pair takes x - p, the negated p - x, so every lane
//    does x + c p with c = +1 or -1: one v_fmac with the partner as a DPP
//    operand (the product by +-1 is exact, so the fma rounds the sum or
//    difference once, as the add does). The negations accumulate: the value
//    held is (-1)^popc(j) times the transform's; fwht_perm_sign gives that
//    factor, which the caller folds into its scale. A result that is an exact
//    zero may carry the other sign than fwht_lanes' zero.
template <int LPV>
__device__ __forceinline__ int fwht_perm_lane(int j) {
  return LPV >= 8 ? (j ^ ((j & 4) ? 3 : 0)) : j;
}
template <int M>
__device__ __forceinline__ float lane_pair(float v) {
  static_assert(M == 1 || M == 2 || M == 4 || M == 8, "pair within a 16-lane row");
  constexpr int ctrl = M == 1 ? 0xB1 : M == 2 ? 0x4E : M == 4 ? 0x141 : 0x128;
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, true));
}
// x[o .. o+7] += c * (the same element of the pair partner): one
// v_fmac_f32_dpp each. Inline asm, since LLVM does not fold a DPP move into
// v_fmac. A DPP read needs 2 wait states after a VALU write of its register
// and 5 after a VALU write of EXEC; the block starts with NOP wait states
// (s_nop n gives n + 1), and no element is written in between.
#define FTQ_FMAC_DPP8(NOP, DPP)                                                   \
  asm(NOP "\n"                                                                    \
      "v_fmac_f32_dpp %0, %0, %8 " DPP " row_mask:0xf bank_mask:0xf bound_ctrl:1\n" \
      "v_fmac_f32_dpp %1, %1, %8 " DPP " row_mask:0xf bank_mask:0xf bound_ctrl:1\n" \
      "v_fmac_f32_dpp %2, %2, %8 " DPP " row_mask:0xf bank_mask:0xf bound_ctrl:1\n" \
      "v_fmac_f32_dpp %3, %3, %8 " DPP " row_mask:0xf bank_mask:0xf bound_ctrl:1\n" \
      "v_fmac_f32_dpp %4, %4, %8 " DPP " row_mask:0xf bank_mask:0xf bound_ctrl:1\n" \
      "v_fmac_f32_dpp %5, %5, %8 " DPP " row_mask:0xf bank_mask:0xf bound_ctrl:1\n" \
      "v_fmac_f32_dpp %6, %6, %8 " DPP " row_mask:0xf bank_mask:0xf bound_ctrl:1\n" \
      "v_fmac_f32_dpp %7, %7, %8 " DPP " row_mask:0xf bank_mask:0xf bound_ctrl:1"   \
      : "+v"(x[o]), "+v"(x[o + 1]), "+v"(x[o + 2]), "+v"(x[o + 3]), "+v"(x[o + 4]),   \
        "+v"(x[o + 5]), "+v"(x[o + 6]), "+v"(x[o + 7])                                \
      : "v"(c))

template <int M, bool FIRST, int E>
__device__ __forceinline__ void fmac_pair8(float (&x)[E], int o, float c) {
  if constexpr (FIRST) {
    if constexpr (M == 1) FTQ_FMAC_DPP8("s_nop 4", "quad_perm:[1,0,3,2]");
    else if constexpr (M == 2) FTQ_FMAC_DPP8("s_nop 4", "quad_perm:[2,3,0,1]");
    else if constexpr (M == 4) FTQ_FMAC_DPP8("s_nop 4", "row_half_mirror");
    else FTQ_FMAC_DPP8("s_nop 4", "row_ror:8");
  } else {
    if constexpr (M == 1) FTQ_FMAC_DPP8("s_nop 1", "quad_perm:[1,0,3,2]");
    else if constexpr (M == 2) FTQ_FMAC_DPP8("s_nop 1", "quad_perm:[2,3,0,1]");
    else if constexpr (M == 4) FTQ_FMAC_DPP8("s_nop 1", "row_half_mirror");
    else FTQ_FMAC_DPP8("s_nop 1", "row_ror:8");
  }
}
#undef FTQ_FMAC_DPP8

template <int LPV>
__device__ __forceinline__ float fwht_perm_sign(int j) {
  return (__builtin_popcount((unsigned)j & (LPV - 1)) & 1) ? -1.f : 1.f;
}
// j: the chunk index (fwht_perm_lane of the lane in the group)
template <int E, int LPV>
__device__ __forceinline__ void fwht_lanes_perm(float (&x)[E], int j) {
#pragma unroll
  for (int h = 1; h < E; h <<= 1) {
#pragma unroll
    for (int i = 0; i < E; ++i) {
      if ((i & h) == 0) {
        float a = x[i], b = x[i + h];
        x[i] = a + b;
        x[i + h] = a - b;
      }
    }
  }
  static_assert(E % 8 == 0, "blocks of 8 elements");
  // The first block waits 5 states (an EXEC write may precede the transform);
  // every later one 2, whatever the compiler schedules between the blocks.
#pragma unroll
  for (int o = 0; o < E; o += 8) {
    if (o == 0) fmac_pair8<1, true>(x, o, (j & 1) ? -1.f : 1.f);
    else fmac_pair8<1, false>(x, o, (j & 1) ? -1.f : 1.f);
  }
  if constexpr (LPV >= 4) {
#pragma unroll
    for (int o = 0; o < E; o += 8) fmac_pair8<2, false>(x, o, (j & 2) ? -1.f : 1.f);
  }
  if constexpr (LPV >= 8) {
#pragma unroll
    for (int o = 0; o < E; o += 8) fmac_pair8<4, false>(x, o, (j & 4) ? -1.f : 1.f);
  }
  if constexpr (LPV >= 16) {
#pragma unroll
    for (int o = 0; o < E; o += 8) fmac_pair8<8, false>(x, o, (j & 8) ? -1.f : 1.f);
  }
}
// group_sum over the permuted layout: the same pairs of chunks as group_sum
// over the plain one, so the same bits
template <int LPV>
__device__ __forceinline__ float group_sum_perm(float v) {
  if constexpr (LPV >= 2) v += lane_pair<1>(v);
  if constexpr (LPV >= 4) v += lane_pair<2>(v);
  if constexpr (LPV >= 8) v += lane_pair<4>(v);
  if constexpr (LPV >= 16) v += lane_pair<8>(v);
  return v;
}

// ---- element loads / stores ----------------------------------------------
enum DType : int { F32 = 0, F16 = 1, BF16 = 2 };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// float -> bf16 bits, round to nearest even (NaN kept quiet)
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
// fp32 -> fp16 bits, round to nearest even, as an instruction of its own: left
// to the compiler, a conversion of a product becomes one v_fma_mix* (a single
// rounding of the exact product to fp16), where the reference rounds the
// product to fp32 first and then to fp16 (.half() of a float32 tensor)
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  uint32_t r;
  asm("v_cvt_f16_f32 %0, %1" : "=v"(r) : "v"(f));
  return r & 0xffffu;
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  return __half2float(__ushort_as_half((unsigned short)b));
}

__device__ __forceinline__ float half_bits_to_f32(int DT, uint32_t h) {
  return DT == BF16 ? bf16_bits_to_f32(h) : f16_bits_to_f32(h);
}

// Load E contiguous elements (E a multiple of 4; 16-byte chunks, then one
// 8-byte chunk when E % 8 == 4 for 16-bit types).
template <int DT, int E>
__device__ __forceinline__ void load_elems(const void* base, int64_t elem_off, float (&x)[E]) {
  static_assert(E % 4 == 0, "E must be a multiple of 4");
  if constexpr (DT == F32) {
    const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(base) + elem_off);
#pragma unroll
    for (int k = 0; k < E / 4; ++k) {
      float4 v = p[k];
      x[4 * k + 0] = v.x; x[4 * k + 1] = v.y; x[4 * k + 2] = v.z; x[4 * k + 3] = v.w;
    }
  } else {
    const uint16_t* b16 = static_cast<const uint16_t*>(base) + elem_off;
    const uint4* p = reinterpret_cast<const uint4*>(b16);
#pragma unroll
    for (int k = 0; k < E / 8; ++k) {
      uint4 v = p[k];
      uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[8 * k + 2 * j] = half_bits_to_f32(DT, w[j] & 0xffffu);
        x[8 * k + 2 * j + 1] = half_bits_to_f32(DT, w[j] >> 16);
      }
    }
    if constexpr (E % 8 == 4) {
      const uint2 v = *reinterpret_cast<const uint2*>(b16 + (E / 8) * 8);
      x[E - 4] = half_bits_to_f32(DT, v.x & 0xffffu);
      x[E - 3] = half_bits_to_f32(DT, v.x >> 16);
      x[E - 2] = half_bits_to_f32(DT, v.y & 0xffffu);
      x[E - 1] = half_bits_to_f32(DT, v.y >> 16);
    }
  }
}

__device__ __forceinline__ uint32_t f32_to_half_bits(int DT, float f) {
  return DT == BF16 ? f32_to_bf16_bits(f) : f32_to_f16_bits(f);
}

// Store E contiguous elements (same chunking as load_elems).
template <int DT, int E>
__device__ __forceinline__ void store_elems(void* base, int64_t elem_off, const float (&x)[E]) {
  static_assert(E % 4 == 0, "E must be a multiple of 4");
  if constexpr (DT == F32) {
    float4* p = reinterpret_cast<float4*>(static_cast<float*>(base) + elem_off);
#pragma unroll
    for (int k = 0; k < E / 4; ++k) p[k] = make_float4(x[4 * k], x[4 * k + 1], x[4 * k + 2], x[4 * k + 3]);
  } else {
    uint16_t* b16 = static_cast<uint16_t*>(base) + elem_off;
    uint4* p = reinterpret_cast<uint4*>(b16);
#pragma unroll
    for (int k = 0; k < E / 8; ++k) {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        w[j] = f32_to_half_bits(DT, x[8 * k + 2 * j]) | (f32_to_half_bits(DT, x[8 * k + 2 * j + 1]) << 16);
      p[k] = make_uint4(w[0], w[1], w[2], w[3]);
    }
    if constexpr (E % 8 == 4) {
      const uint32_t lo = f32_to_half_bits(DT, x[E - 4]) | (f32_to_half_bits(DT, x[E - 3]) << 16);
      const uint32_t hi = f32_to_half_bits(DT, x[E - 2]) | (f32_to_half_bits(DT, x[E - 1]) << 16);
      *reinterpret_cast<uint2*>(b16 + (E / 8) * 8) = make_uint2(lo, hi);
    }
  }
}

}  // namespace ftq
