// vLLM v1 TURBOQUANT slot store on gfx950: quantise K and V of n tokens x
// Hkv heads and write them into their slots, for the unsigned Hadamard
// rotation (kind = rht) and for the block-diagonal rotations (planar 2x2,
// rotor 3x3, iso 4x4), in one launch.
//
// Per (token, kv head) (reference vllm_plugin/triton_inkernel_store.py:38-440,
// 554-616 for rht, 649-860 for the block-diagonal kinds):
//   K: norm = sqrt(sum k^2 + 1e-16); rht: x = k / (norm + 1e-8) through the
//      butterflies, y = x * d^-1/2; block-diagonal: x = k * (1 / (norm + 1e-8)),
//      y[e] = sum_j x[(e / B) B + j] c[j][e] in fp32 fused multiply-adds;
//      code = number of midpoints <= y; fp16 norm after the codes.
//   V (optionally rotated first -- the same rotation, without the
//      normalisation -- and rounded back to the input dtype, v1_backend.py:
//      736-740): min / max uniform codes trunc((v - min) / scale + 0.5),
//      scale = (max - min) / (2^vb - 1) (>= 1e-8), or with the Lloyd-Max flag
//      (4-bit V) the K midpoint search on v / (|v| + 1e-8), its fp16 norm in
//      the scale field and 0 in the min field.
//
// Layout of the work: one vector per LPV = min(16, D / 8) lanes, E = D / LPV
// contiguous elements per lane (E = 8 at d = 64 and 128, 16 at d = 256), so
// a lane's codes form E * bits (16 ... 64) whole bits; they are packed in
// registers and written straight to the slot with 1-, 2- and 4-byte stores
// (no LDS).  The midpoint search is a branch-free binary search on
// midpoints held in registers: bits compares and 2^bits - 1 - bits selects
// per element instead of 2^bits - 1 compares and adds.
// K is divided by its norm through the reciprocal and one fma correction.
// The uniform V codes divide by the scale through its reciprocal; where that
// quotient lies within 1e-5 of a half-integer (the only place trunc(q + 0.5)
// can differ from the correctly rounded division), the wave recomputes the
// lane's elements with the IEEE division.
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

// E codes of NB bits (code i at bit i * NB) into w[0..1]
template <int E, int NB>
__device__ __forceinline__ void pack_codes(const uint32_t (&c)[E], uint32_t (&w)[2]) {
  w[0] = 0;
  w[1] = 0;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int p = i * NB;  // compile-time after unrolling; fields do not straddle for NB = 2, 4
    if (p + NB <= 32) {
      w[0] |= c[i] << p;
    } else if (p >= 32) {
      w[1] |= c[i] << (p - 32);
    } else {  // NB = 3 across the word boundary
      w[0] |= c[i] << p;
      w[1] |= c[i] >> (32 - p);
    }
  }
}

// Write W = E * NB bits of lane `li` at byte base + li * W / 8.  base is
// 2-byte aligned (4-byte aligned when ALIGN4).
template <int W, bool ALIGN4>
__device__ __forceinline__ void store_bits(uint8_t* base, int li, const uint32_t (&w)[2]) {
  static_assert(W % 8 == 0, "whole bytes per lane");
  uint8_t* p = base + li * (W / 8);
  if constexpr (W == 16) {
    *reinterpret_cast<uint16_t*>(p) = (uint16_t)w[0];
  } else if constexpr (W == 24) {  // 3 bytes at an odd or even offset
    if ((li & 1) == 0) {
      *reinterpret_cast<uint16_t*>(p) = (uint16_t)w[0];
      p[2] = (uint8_t)(w[0] >> 16);
    } else {
      p[0] = (uint8_t)w[0];
      *reinterpret_cast<uint16_t*>(p + 1) = (uint16_t)(w[0] >> 8);
    }
  } else if constexpr (W == 32) {
    if constexpr (ALIGN4) {
      *reinterpret_cast<uint32_t*>(p) = w[0];
    } else {
      *reinterpret_cast<uint16_t*>(p) = (uint16_t)w[0];
      *reinterpret_cast<uint16_t*>(p + 2) = (uint16_t)(w[0] >> 16);
    }
  } else if constexpr (W == 48) {
    *reinterpret_cast<uint16_t*>(p) = (uint16_t)w[0];
    *reinterpret_cast<uint16_t*>(p + 2) = (uint16_t)(w[0] >> 16);
    *reinterpret_cast<uint16_t*>(p + 4) = (uint16_t)w[1];
  } else {
    static_assert(W == 64, "16 ... 64 bits per lane");
    if constexpr (ALIGN4) {
      *reinterpret_cast<uint32_t*>(p) = w[0];
      *reinterpret_cast<uint32_t*>(p + 4) = w[1];
    } else {
#pragma unroll
      for (int h = 0; h < 4; ++h)
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

template <int D, int DT, int KB, int VB, int RB>
__global__ __launch_bounds__(256) void v1_store_fast_kernel(
    const void* __restrict__ key, const void* __restrict__ value, int64_t n_tokens, int hkv,
    const float* __restrict__ mid_g, int vflags, const int64_t* __restrict__ slot_mapping,
    uint8_t* __restrict__ cache, int64_t num_blocks, int block_size, int64_t s_blk, int64_t s_pos,
    int64_t s_head, float rscale, const float* __restrict__ coeffs) {
  constexpr int LPV = D >= 128 ? 16 : D / 8;
  constexpr int E = D / LPV;
  constexpr int VPB = 256 / LPV;  // vectors per workgroup pass
  constexpr int NMK = (1 << KB) - 1;
  constexpr V1Geom G = v1_geom(D, KB, VB);
  constexpr int VTOP = (1 << VB) - 1;
  static_assert(RB == 0 || RB == 2 || RB == 3 || RB == 4, "rotation: Hadamard or 2/3/4 blocks");
  const int li = threadIdx.x % LPV;
  const int grp = threadIdx.x / LPV;

  float mids[NMK];
#pragma unroll
  for (int j = 0; j < NMK; ++j) mids[j] = mid_g[j];
  float cf[RB == 0 ? 1 : RB][E];
  if constexpr (RB != 0) {
#pragma unroll
    for (int j = 0; j < RB; ++j)
#pragma unroll
      for (int i = 0; i < E; ++i) cf[j][i] = coeffs[j * D + li * E + i];
  }
  const bool vrot = (vflags & 1) != 0;
  const bool vlm = (vflags & 2) != 0 && VB == 4;
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
    ss = group_sum<LPV>(ss);
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
      fwht_lanes<E, LPV>(x, li);
#pragma unroll
      for (int i = 0; i < E; ++i) x[i] *= rscale;
    } else {
      const float inv = 1.f / den;
#pragma unroll
      for (int i = 0; i < E; ++i) x[i] *= inv;
      rot_blockdiag<D, E, LPV, RB>(x, cf, li);
    }
    uint32_t c[E], w[2];
#pragma unroll
    for (int i = 0; i < E; ++i) c[i] = mid_search<KB>(x[i], mids);
    pack_codes<E, KB>(c, w);
    store_bits<E * KB, true>(sp, li, w);

    // ---- V
    float v[E];
    load_elems<DT, E>(value, vi * D + li * E, v);
    if (vrot) {
      if constexpr (RB == 0) {
        fwht_lanes<E, LPV>(v, li);
#pragma unroll
        for (int i = 0; i < E; ++i) v[i] = round_to_dtype<DT>(v[i] * rscale);
      } else {
        rot_blockdiag<D, E, LPV, RB>(v, cf, li);
#pragma unroll
        for (int i = 0; i < E; ++i) v[i] = round_to_dtype<DT>(v[i]);
      }
    }
    float sc, mn;
    if (vlm) {
      float vs = 0.f;
#pragma unroll
      for (int i = 0; i < E; ++i) vs = __builtin_fmaf(v[i], v[i], vs);
      vs = group_sum<LPV>(vs);
      sc = __builtin_sqrtf(vs + 1e-16f);
      mn = 0.f;
      const float vden = sc + 1e-8f;
#pragma unroll
      for (int i = 0; i < E; ++i) c[i] = mid_search<KB>(v[i] / vden, mids);
      pack_codes<E, 4>(c, w);
    } else {
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
        else if (m == 4) { mn = fminf(mn, lane_xor<4>(mn)); mx = fmaxf(mx, lane_xor<4>(mx)); }
        else { mn = fminf(mn, lane_xor<8>(mn)); mx = fmaxf(mx, lane_xor<8>(mx)); }
      }
      sc = (VB == 1) ? (mx - mn) : (mx - mn) / (float)VTOP;
      sc = sc > 1e-8f ? sc : 1e-8f;
      const float rs = 1.f / sc;
      float q[E];
      bool near = false;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        q[i] = (v[i] - mn) * rs;
        const float f = q[i] - __builtin_floorf(q[i]);
        near = near || (__builtin_fabsf(f - 0.5f) < 1e-5f * fmaxf(q[i], 1.f));
      }
      if (__builtin_amdgcn_ballot_w64(near) != 0) {  // rare: the correctly rounded quotient
#pragma unroll
        for (int i = 0; i < E; ++i) q[i] = (v[i] - mn) / sc;
      }
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const float t = q[i] + 0.5f;
        // trunc toward zero, clamped to [0, VTOP]; NaN -> 0
        c[i] = t >= 1.f ? (uint32_t)fminf(t, (float)VTOP) : 0u;
      }
      pack_codes<E, VB>(c, w);
    }
    store_bits<E * VB, false>(sp + G.kps, li, w);
    if (li == 0) {
      *reinterpret_cast<uint16_t*>(sp + G.mse) = (uint16_t)f32_to_f16_bits(nrm);
      *reinterpret_cast<uint16_t*>(sp + G.kps + G.vdb) = (uint16_t)f32_to_f16_bits(sc);
      *reinterpret_cast<uint16_t*>(sp + G.kps + G.vdb + 2) = (uint16_t)f32_to_f16_bits(mn);
    }
  }
}

template <int D, int KB, int VB, int RB>
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
    v1_store_fast_kernel<D, F32, KB, VB, RB><<<grid, block, 0, st>>>(k, v, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, rs, coeffs);
  else if (dt == F16)
    v1_store_fast_kernel<D, F16, KB, VB, RB><<<grid, block, 0, st>>>(k, v, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, rs, coeffs);
  else
    v1_store_fast_kernel<D, BF16, KB, VB, RB><<<grid, block, 0, st>>>(k, v, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, rs, coeffs);
  return hipGetLastError();
}

template <int D, int KB, int VB>
static hipError_t launch_fast_store3(int rb, const void* k, const void* v, int dt, int64_t n, int hkv,
                                     const float* mids, int vflags, const int64_t* slots, uint8_t* cache,
                                     int64_t nb, int bs, int64_t sb, int64_t sp, int64_t sh, const float* coeffs,
                                     hipStream_t st) {
  switch (rb) {
    case 2: return launch_fast_store4<D, KB, VB, 2>(k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
    case 3: return launch_fast_store4<D, KB, VB, 3>(k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
    case 4: return launch_fast_store4<D, KB, VB, 4>(k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
    default: return launch_fast_store4<D, KB, VB, 0>(k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
  }
}

template <int D, int KB>
static hipError_t launch_fast_store2(int vb, int rb, const void* k, const void* v, int dt, int64_t n, int hkv,
                                     const float* mids, int vflags, const int64_t* slots, uint8_t* cache,
                                     int64_t nb, int bs, int64_t sb, int64_t sp, int64_t sh, const float* coeffs,
                                     hipStream_t st) {
  if (vb == 2) return launch_fast_store3<D, KB, 2>(rb, k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
  if (vb == 3) return launch_fast_store3<D, KB, 3>(rb, k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
  return launch_fast_store3<D, KB, 4>(rb, k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
}

template <int D>
static hipError_t launch_fast_store1(int kb, int vb, int rb, const void* k, const void* v, int dt, int64_t n,
                                     int hkv, const float* mids, int vflags, const int64_t* slots, uint8_t* cache,
                                     int64_t nb, int bs, int64_t sb, int64_t sp, int64_t sh, const float* coeffs,
                                     hipStream_t st) {
  if (kb == 2) return launch_fast_store2<D, 2>(vb, rb, k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
  if (kb == 3) return launch_fast_store2<D, 3>(vb, rb, k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
  return launch_fast_store2<D, 4>(vb, rb, k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
}

// Shared argument checks of the slot stores; 0 = fine.
int v1_store_checks(int d, int key_bits, int value_bits, int64_t n_tokens, int num_kv_heads, int64_t num_blocks,
                    int block_size, int dtype, int v_rotate, int64_t stride_block, int64_t stride_pos,
                    int64_t stride_head) {
  FTQ_REQUIRE(d == 64 || d == 128 || d == 256, "v1 store: head_dim must be 64, 128 or 256");
  FTQ_REQUIRE(key_bits >= 2 && key_bits <= 4 && value_bits >= 2 && value_bits <= 4,
              "v1 store: key_bits and value_bits must be 2, 3 or 4");
  FTQ_REQUIRE(n_tokens >= 0 && num_kv_heads > 0 && num_blocks >= 0 && block_size > 0,
              "bad token / head / block counts");
  FTQ_REQUIRE(dtype >= F32 && dtype <= BF16, "dtype must be FTQ_F32, FTQ_F16 or FTQ_BF16");
  FTQ_REQUIRE(v_rotate >= 0 && v_rotate <= 3, "v_rotate: bit 0 = rotate V, bit 1 = Lloyd-Max V codes");
  const V1Geom g = v1_geom(d, key_bits, value_bits);
  FTQ_REQUIRE(stride_head >= g.raw, "stride_head is smaller than the slot bytes (see ftq_v1_slot_bytes)");
  FTQ_REQUIRE(stride_pos >= stride_head * num_kv_heads && stride_block >= stride_pos * block_size,
              "kv_cache strides must describe [num_blocks][block_size][num_kv_heads][slot]");
  FTQ_REQUIRE(stride_head % 4 == 0 && stride_pos % 4 == 0 && stride_block % 4 == 0,
              "kv_cache strides must be multiples of 4 bytes");
  return FTQ_OK;
}

static int v1_store_fast(const void* key, const void* value, int dtype, int64_t n_tokens, int num_kv_heads, int d,
                         const float* midpoints, int key_bits, int value_bits, int v_rotate,
                         const int64_t* slot_mapping, uint8_t* kv_cache, int64_t num_blocks, int block_size,
                         int64_t stride_block, int64_t stride_pos, int64_t stride_head, const float* coeffs,
                         int rb, void* stream) {
  const int rc = v1_store_checks(d, key_bits, value_bits, n_tokens, num_kv_heads, num_blocks, block_size, dtype,
                                 v_rotate, stride_block, stride_pos, stride_head);
  if (rc != FTQ_OK) return rc;
  if (n_tokens == 0) return FTQ_OK;
  FTQ_REQUIRE(key && value && midpoints && slot_mapping && kv_cache, "null pointer argument");
  FTQ_REQUIRE(rb == 0 || coeffs != nullptr, "null coefficient pointer");
  FTQ_REQUIRE(aligned16(key) && aligned16(value), "key/value must be 16-byte aligned");
  FTQ_REQUIRE(aligned4(kv_cache), "kv_cache must be 4-byte aligned");
  FTQ_REQUIRE(coeffs == nullptr || aligned4(coeffs), "coefficients must be 4-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (d == 64)
    e = launch_fast_store1<64>(key_bits, value_bits, rb, key, value, dtype, n_tokens, num_kv_heads, midpoints, v_rotate, slot_mapping, kv_cache, num_blocks, block_size, stride_block, stride_pos, stride_head, coeffs, st);
  else if (d == 128)
    e = launch_fast_store1<128>(key_bits, value_bits, rb, key, value, dtype, n_tokens, num_kv_heads, midpoints, v_rotate, slot_mapping, kv_cache, num_blocks, block_size, stride_block, stride_pos, stride_head, coeffs, st);
  else
    e = launch_fast_store1<256>(key_bits, value_bits, rb, key, value, dtype, n_tokens, num_kv_heads, midpoints, v_rotate, slot_mapping, kv_cache, num_blocks, block_size, stride_block, stride_pos, stride_head, coeffs, st);
  return hip_status(e);
}

}  // namespace ftq

using namespace ftq;

extern "C" int ftq_v1_store(const void* key, const void* value, int dtype, int64_t n_tokens, int num_kv_heads,
                            int d, const float* midpoints, int key_bits, int value_bits, int v_rotate,
                            const int64_t* slot_mapping, uint8_t* kv_cache, int64_t num_blocks, int block_size,
                            int64_t stride_block, int64_t stride_pos, int64_t stride_head, void* stream) {
  return v1_store_fast(key, value, dtype, n_tokens, num_kv_heads, d, midpoints, key_bits, value_bits, v_rotate,
                       slot_mapping, kv_cache, num_blocks, block_size, stride_block, stride_pos, stride_head,
                       nullptr, 0, stream);
}

extern "C" int ftq_v1_store_blockdiag(const void* key, const void* value, int dtype, int64_t n_tokens,
                                      int num_kv_heads, int d, const float* midpoints, int key_bits,
                                      int value_bits, int v_rotate, const int64_t* slot_mapping,
                                      uint8_t* kv_cache, int64_t num_blocks, int block_size, int64_t stride_block,
                                      int64_t stride_pos, int64_t stride_head, const float* coeffs, int block,
                                      void* stream) {
  FTQ_REQUIRE(block == 2 || block == 3 || block == 4, "block-diagonal rotation: block must be 2, 3 or 4");
  return v1_store_fast(key, value, dtype, n_tokens, num_kv_heads, d, midpoints, key_bits, value_bits, v_rotate,
                       slot_mapping, kv_cache, num_blocks, block_size, stride_block, stride_pos, stride_head,
                       coeffs, block, stream);
}
