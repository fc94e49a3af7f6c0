// vLLM v1 TURBOQUANT slot-format KV cache on gfx950: fused store and split-K
// decode attention over the packed slots.
//
// Slot format (reference vllm_plugin/triton_inkernel_store.py:38-440,
// boundary_tq_config.py:66-81, v1_backend.py:171-220), per (token, kv head),
// byte-addressed inside kv_cache[num_blocks][block_size][Hkv][slot]:
//   [K codes: MSE = D*KB/8][K norm f16][V codes: VDB = D*VB/8][V scale f16][V min f16][pad]
// K codes use the library bit layout (4-bit: low nibble = even dim; 3-bit: 8
// codes in 24 bits; 2-bit: LSB first).
//
// Store semantics (reference triton_inkernel_store.py:394-440, :91-100, :202-330):
//   K: n = sqrt(sum k^2 + 1e-16); y = H (k / (n + 1e-8)) / sqrt(D) with the
//      unsigned Sylvester butterflies; code = #{midpoints m : y >= m}; n -> f16.
//   V (optionally rotated first, v' = dtype(v H / sqrt(D)), v1_backend.py:736-740):
//      sc = max((max - min) / (2^VB - 1), 1e-8); q = clamp(trunc((v - min)/sc + 0.5));
//      sc, min -> f16.
// Decode semantics (reference triton_decode_offset.py:42-442, v1_backend.py:975-1093):
//   q_rot = q H / sqrt(D); c^ = C[idx] / sqrt(sum C[idx]^2 + 1e-16);
//   s_t = ||k_t||_16 <q_rot, c^_t> scale; o = softmax(s) . (q_v sc_16 + min_16);
//   o <- o H / sqrt(D) when V was rotated; out = dtype(o).
//
// Decode kernel: one workgroup (4 waves) per (batch, kv head, split); a wave
// walks 32-token tiles (two 16-token S-tiles), reading each slot's K codes,
// K norm, V codes and V scale/min once for the whole GQA group.
//   S^T[t][h] = K[t][:] . Q^T[:][h]   v_mfma_f32_16x16x32_f16; A = K codes as f16
//                pairs from an LDS pair table, B = rotated query (scale*log2 e folded)
//   Gram[t][t'] = K[t][:] . K[t'][:]   same MFMA with A = B = the K operand; its
//                diagonal is sum C[idx]^2 for the norm correction
//   O^T[d][h] += V^T[d][t] . P'^T[t][h]  A = V codes as f16 2^e_t (1 + q / 2^VB),
//                taken straight from the packed bits with one shift and one
//                and-or, e_t the exponent of the token's fp16 V scale sc_t;
//                B = p_t * sc_t / 2^e_t (in [p, 2p)), so
//                o = 2^VB (acc - sum p sc) + sum p * min.
// Precision: P' and the rotated query enter the MFMAs as f16 hi + lo pairs (two
// MFMAs each), ~22 bits: with uniform V, sc * q cancels against min, and one
// f16 rounding of P' would show in the output.  Keeping sc's exponent in the A
// operand keeps P' in [p, 2p) <= 2^(TAU+1): never subnormal for the tokens that
// matter, never above the f16 range for any fp16 scale.
// Online softmax in the log2 domain with lazy rescaling (the reference max is
// only raised when a tile exceeds it by 2^8).  Waves merge through LDS; splits
// merge in a second kernel that also un-rotates V and writes the output dtype.
#include "ftq_attn_dev.h"
#include "ftq_merge.h"
#include "ftq_codec_dev.h"
#include "ftq_internal.h"
#include "ftq_v1_dev.h"

#include <cmath>
#include <type_traits>
#include <mutex>

namespace ftq {

float fwht_scale(int d);

typedef unsigned short us2 __attribute__((ext_vector_type(2)));


// ---------------------------------------------------------------------------
// store
// ---------------------------------------------------------------------------

// bits [pos, pos + n) (n <= 32) of the little-endian stream of B-bit codes c[0..D)
template <int D>
__device__ __forceinline__ uint32_t packed_bits(const uint8_t* c, int B, int pos, int n) {
  uint32_t r = 0;
  const int d0 = pos / B;
  int d1 = (pos + n - 1) / B;
  if (d1 > D - 1) d1 = D - 1;
  for (int d = d0; d <= d1; ++d) {
    const int sh = d * B - pos;
    const uint32_t v = c[d];
    r |= sh >= 0 ? (v << sh) : (v >> -sh);
  }
  return n == 32 ? r : (r & ((1u << n) - 1u));
}


// One (token, kv head) per 16 lanes, D/16 contiguous elements per lane.
// ROTM: K (and V when rotated) rotated by the matrix rot instead of H/sqrt(D).
template <int D, int DT, bool ROTM = false>
__global__ __launch_bounds__(256) void v1_store_kernel(
    const void* __restrict__ key, const void* __restrict__ value, int64_t n_tokens, int hkv,
    const float* __restrict__ mid_g, int kb, int vb, int v_rotate,
    const int64_t* __restrict__ slot_mapping, uint8_t* __restrict__ cache, int64_t num_blocks,
    int block_size, int64_t s_blk, int64_t s_pos, int64_t s_head, float rscale,
    const float* __restrict__ rot) {
  constexpr int E = D / 16;
  __shared__ uint8_t kc[16][D];
  __shared__ uint8_t vc[16][D];
  __shared__ float xs[ROTM ? 16 : 1][ROTM ? D : 1];  // ROTM: the group's vector for the matrix product
  __shared__ float mids[16];
  const int lane = threadIdx.x & 15, grp = threadIdx.x >> 4;
  const int nmid = (1 << kb) - 1;
  if ((int)threadIdx.x < nmid) mids[threadIdx.x] = mid_g[threadIdx.x];
  __syncthreads();
  const V1Geom g = v1_geom(D, kb, vb);
  const int vtop = (1 << vb) - 1;
  const int64_t nvec = n_tokens * hkv;

  for (int64_t base = (int64_t)blockIdx.x * 16; base < nvec; base += (int64_t)gridDim.x * 16) {
    const int64_t vi = base + grp;
    bool active = vi < nvec;
    const int64_t tok = active ? vi / hkv : 0;
    const int head = active ? (int)(vi % hkv) : 0;
    const int64_t slot = active ? slot_mapping[tok] : -1;
    const int64_t blk = slot >= 0 ? slot / block_size : -1;
    active = active && slot >= 0 && blk < num_blocks;  // negative slots are skipped
    float nrm = 0.f, sc = 0.f, mn = 0.f;
    if (active) {  // uniform over the 16 lanes of the vector
      // ---- K: norm, normalise, unsigned Hadamard, midpoint search
      float x[E];
      load_elems<DT, E>(key, vi * D + lane * E, x);
      float ss = 0.f;
#pragma unroll
      for (int i = 0; i < E; ++i) ss += x[i] * x[i];
      ss = group_sum<16>(ss);
      nrm = sqrtf(ss + 1e-16f);
      const float den = nrm + 1e-8f;
#pragma unroll
      for (int i = 0; i < E; ++i) x[i] = x[i] / den;
      if constexpr (ROTM) rot_matrix_lanes<D, E>(x, rot, &xs[grp][0], lane);
      else fwht_lanes<E, 16>(x, lane);
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const float y = x[i] * rscale;
        int c = 0;
        for (int j = 0; j < nmid; ++j) c += (y >= mids[j]) ? 1 : 0;
        kc[grp][lane * E + i] = (uint8_t)c;
      }
      // ---- V: optional rotation (rounded back to the value dtype), then
      // Lloyd-Max codes (flag 2, 4-bit V) or the min/max quantiser
      float v[E];
      load_elems<DT, E>(value, vi * D + lane * E, v);
      if (v_rotate & 1) {
        if constexpr (ROTM) rot_matrix_lanes<D, E>(v, rot, &xs[grp][0], lane);
        else fwht_lanes<E, 16>(v, lane);
#pragma unroll
        for (int i = 0; i < E; ++i) v[i] = round_to_dtype<DT>(v[i] * rscale);
      }
      if ((v_rotate & 2) && vb == 4) {
        // norm into the scale field, codes of v / (norm + 1e-8) by the K
        // midpoint search, 0 in the min field
        float vs = 0.f;
#pragma unroll
        for (int i = 0; i < E; ++i) vs += v[i] * v[i];
        vs = group_sum<16>(vs);
        sc = sqrtf(vs + 1e-16f);
        mn = 0.f;
        const float vden = sc + 1e-8f;
#pragma unroll
        for (int i = 0; i < E; ++i) {
          const float u = v[i] / vden;
          int c = 0;
          for (int j = 0; j < nmid; ++j) c += (u >= mids[j]) ? 1 : 0;
          vc[grp][lane * E + i] = (uint8_t)c;
        }
      } else {
      mn = v[0];
      float mx = v[0];
#pragma unroll
      for (int i = 1; i < E; ++i) {
        mn = fminf(mn, v[i]);
        mx = fmaxf(mx, v[i]);
      }
      mn = fminf(mn, lane_xor<1>(mn)); mx = fmaxf(mx, lane_xor<1>(mx));
      mn = fminf(mn, lane_xor<2>(mn)); mx = fmaxf(mx, lane_xor<2>(mx));
      mn = fminf(mn, lane_xor<4>(mn)); mx = fmaxf(mx, lane_xor<4>(mx));
      mn = fminf(mn, lane_xor<8>(mn)); mx = fmaxf(mx, lane_xor<8>(mx));
      sc = (vb == 1) ? (mx - mn) : (mx - mn) / (float)vtop;
      sc = sc > 1e-8f ? sc : 1e-8f;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const float t = (v[i] - mn) / sc + 0.5f;
        // trunc toward zero, clamped; NaN -> 0
        const int q = t >= 1.f ? (int)fminf(t, (float)vtop) : 0;
        vc[grp][lane * E + i] = (uint8_t)q;
      }
      }
    }
    __syncthreads();
    if (active) {
      const int off = (int)(slot - blk * block_size);
      uint8_t* sp = cache + blk * s_blk + off * s_pos + head * s_head;
      for (int w = lane; w < g.mse / 4; w += 16)
        *reinterpret_cast<uint32_t*>(sp + 4 * w) = packed_bits<D>(kc[grp], kb, 32 * w, 32);
      for (int w = lane; w < g.vdb / 2; w += 16)
        *reinterpret_cast<uint16_t*>(sp + g.kps + 2 * w) = (uint16_t)packed_bits<D>(vc[grp], vb, 16 * w, 16);
      if (lane == 0) {
        *reinterpret_cast<uint16_t*>(sp + g.mse) = (uint16_t)f32_to_f16_bits(nrm);
        *reinterpret_cast<uint16_t*>(sp + g.kps + g.vdb) = (uint16_t)f32_to_f16_bits(sc);
        *reinterpret_cast<uint16_t*>(sp + g.kps + g.vdb + 2) = (uint16_t)f32_to_f16_bits(mn);
      }
    }
    __syncthreads();
  }
}

// One split (num_splits == 1) and no caller matrix: the workgroup writes the
// output itself (the merge's arithmetic for a single partial: o / L, then the
// un-rotation and the dtype) and no merge launch follows.  mode -1: partials
// to the workspace as usual; 0: output, V not rotated; 1: output, V rotated
// (o <- (H o) d^-1/2).
struct V1Direct {
  void* out;
  float* lse;  // optional natural-log LSE per row
  float scale;  // d^-1/2 (the merge's factor)
  int ot, mode;
};

// Rows of one (batch, kv head) written straight to the output: wave w takes
// heads w, w + 4, ...; lane l elements [2 l, 2 l + 2).  Bit for bit what the
// merge writes for one split: y = o / L (its workspace value, times the merge's
// weight 1 and 1 / W = 1), then the inverse transform and the dtype.
template <int D, int RW, int RS>
__device__ __forceinline__ void v1_direct_rows(const float (&red_m)[4][RW], const float (&red_l)[4][RW],
                                               const float (*red_o)[RW][RS], int G, int wave, int lane,
                                               int64_t row0, const V1Direct& dout) {
  constexpr int E2 = D / 64;
  for (int gg = wave; gg < G; gg += 4) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, red_m[w][gg]);
    float L = 0.f, o[E2];
#pragma unroll
    for (int i = 0; i < E2; ++i) o[i] = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float f = __builtin_amdgcn_exp2f(red_m[w][gg] - M);
        L += f * red_l[w][gg];
#pragma unroll
        for (int i = 0; i < E2; ++i) o[i] += f * red_o[w][gg][E2 * lane + i];
      }
    }
    float y[E2];
#pragma unroll
    for (int i = 0; i < E2; ++i) y[i] = (L > 0.f) ? o[i] / L : 0.f;
    if (dout.mode == 1) {
      fwht_wave64<E2>(y, lane);
#pragma unroll
      for (int i = 0; i < E2; ++i) y[i] *= dout.scale;
    }
    const int64_t row = row0 + gg;
    if (dout.lse != nullptr && lane == 0)
      dout.lse[row] = (L > 0.f) ? (M + __builtin_log2f(L)) * 0.69314718055994531f : -INFINITY;
    if (dout.ot == F32) store_small<F32, E2>(dout.out, row * D + lane * E2, y);
    else if (dout.ot == F16) store_small<F16, E2>(dout.out, row * D + lane * E2, y);
    else store_small<BF16, E2>(dout.out, row * D + lane * E2, y);
  }
}

// ---------------------------------------------------------------------------
// decode attention, stage 1 (per split)
// ---------------------------------------------------------------------------

template <int D, int KB, int VB>
struct V1A {
  static constexpr V1Geom G = v1_geom(D, KB, VB);
  static constexpr int MSE = G.mse, KPS = G.kps, VDB = G.vdb;
  static constexpr int KQ = MSE / 4;      // K bytes one lane reads per token
  static constexpr int KQW = KQ / 4;      // ... in dwords
  static constexpr int NS = D / 32;       // Q.K MFMAs per S-tile
  static constexpr int NB = D / 16;       // P.V MFMAs per tile
  static constexpr int NV = VB == 2 ? 4 : 8;  // V operand registers per tile
  static_assert(D == 128, "the v1 decode kernel is laid out for head_dim 128");
  static_assert(KQ % 4 == 0, "K lane chunk must be whole dwords");
};

template <int D, int KB, int VB, bool DEFER>
struct V1Tile {
  using A = V1A<D, KB, VB>;
  uint32_t k[2][A::KQW];  // per S-tile: K code dwords of token (lane & 15), bytes (lane >> 4) * KQ
  // V codes of the lane's 8 tokens (see v1_load).  DEFER: as loaded, 16 bits
  // each; operand word j is va[j] | vb[j] << 16, formed where it is used, in
  // the next tile's step -- formed at the load, the OR waits in the loading
  // step for loads it has just issued, a full memory round trip per step.
  // Without DEFER (where the registers are not there) va holds the words.
  // The halves stay 16-bit values until then, so that no zero-extension
  // either is computed in the loading step.
  using VH = typename std::conditional<DEFER, uint16_t, uint32_t>::type;
  VH va[A::NV];
  uint16_t vb[DEFER ? A::NV : 1];
  uint16_t tail[2];       // per S-tile: K norm / V scale / V min (by lane >> 4), f16 bits
  uint32_t vt[2][4];      // Lloyd-Max V only: token (lane & 15)'s V codes, bytes (lane >> 4) * 16 ..
  bool ok[2];             // wave-uniform: S-tile has a real page
  __device__ __forceinline__ uint32_t vword(int j) const {
    if constexpr (DEFER) return (uint32_t)va[j] | ((uint32_t)vb[j] << 16);
    else return va[j];
  }
};

// Loads of one 32-token tile, as raw buffer loads: one wave-uniform buffer
// descriptor per S-tile (its page base; the byte range ends after its 16 token
// rows, so no lane can read past them) plus a lane offset fixed for the
// kernel.  An S-tile past the sequence (or on a bad block id) reads block 0
// instead -- the loads always issue, so the wait counts stay static -- and the
// consumer masks it.
//   K:    lane (m, g) = token m, K bytes [g*KQ, (g+1)*KQ)
//   tail: lane (m, g) = token m, field g (0 K norm, 1 V scale, 2 V min, 3 unused)
//   V:    lane (m, g) = tokens 4g+i (i < 4) of each S-tile, the codes of dims
//         8m .. 8m+7.  P.V operand pair j holds tokens (4g + 2(j&1), +1) of S-tile j/2:
//         VB 2: v[j] = the two 16-bit chunks;  VB 4: v[j] / v[4+j] = low / high
//         16 bits of the two 32-bit chunks;  VB 3: v[2j], v[2j+1] = 32 bits around
//         each 24-bit chunk (starting at an even byte).
struct V1Addr {
  const uint8_t* cache;
  __amdgpu_buffer_rsrc_t bt_rs;  // the sequence's block-table row as a buffer
  int64_t s_blk, kvh_off;
  uint32_t s_pos;
  int lbs, max_blocks, seq_len, nb32;  // nb32 = min(num_blocks, 2^31 - 1)
  uint32_t koff, toff, voff;  // lane offsets; token 4g+i of a V load adds i * s_pos (scalar)
  uint32_t vtoff;              // Lloyd-Max V: token-major V codes of the lane
};

__device__ __forceinline__ void v1_addr_rows(V1Addr& ad, const int32_t* bt_row, int64_t num_blocks) {
  ad.bt_rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<int32_t*>(bt_row), (short)0,
                                               (int)min((int64_t)ad.max_blocks * 4, (int64_t)0x7ffffffc),
                                               0x00020000);
  ad.nb32 = (int)min(num_blocks, (int64_t)0x7fffffff);
}

// Is S-tile st of `tile` a real position range with a block-table entry?
__device__ __forceinline__ bool v1_stile_ok(const V1Addr& ad, int tile, int st, bool active) {
  const int pos0 = tile * 32 + st * 16;
  return active && pos0 < ad.seq_len && (pos0 >> ad.lbs) < ad.max_blocks;
}

// Block-table entries of a tile's two S-tiles, as a vector load issued one tile
// ahead of the loads that need them (lane l holds S-tile l & 1; entry 0 is
// read where the S-tile is inactive, past seq_len or past the row).  LATE:
// the entry is returned as loaded and v1_load makes the inactive ones -1,
// so nothing in the fetching step waits for this load; otherwise -1 here.
// A vector load retires in order, so the wait before v1_load's readlane
// covers only this load.
template <bool LATE>
__device__ __forceinline__ int v1_fetch_bt(const V1Addr& ad, int tile, bool active, int lane) {
  const bool ok = v1_stile_ok(ad, tile, lane & 1, active);
  const int page = (tile * 32 + (lane & 1) * 16) >> ad.lbs;
  const int v = (int)__builtin_amdgcn_raw_buffer_load_b32(ad.bt_rs, (uint32_t)(ok ? page : 0) * 4u, 0, 0);
  if constexpr (LATE) return v;
  else return ok ? v : -1;
}

__device__ __forceinline__ uint32_t buf_u16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0);
}

// DEFER tiles take their block-table entries from v1_fetch_bt<true> (the
// inactive test here); the others from v1_fetch_bt<false>.
template <int D, int KB, int VB, bool VLM = false, bool DEFER>
__device__ __forceinline__ void v1_load(V1Tile<D, KB, VB, DEFER>& r, const V1Addr& ad, int tile, bool active,
                                        int btv) {
  using A = V1A<D, KB, VB>;
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const int pos0 = tile * 32 + st * 16;
    int phys;
    if constexpr (DEFER) phys = v1_stile_ok(ad, tile, st, active) ? __builtin_amdgcn_readlane(btv, st) : -1;
    else phys = __builtin_amdgcn_readlane(btv, st);
    const bool valid = (uint32_t)phys < (uint32_t)ad.nb32;  // -1 (no entry) and ids >= num_blocks fail
    if (!valid) phys = 0;
    const uint32_t within = valid ? (uint32_t)(pos0 & ((1 << ad.lbs) - 1)) : 0u;
    const uint8_t* bst = ad.cache + ((int64_t)phys * ad.s_blk + (int64_t)(within * ad.s_pos) + ad.kvh_off);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(bst), (short)0, (int)(16u * ad.s_pos), 0x00020000);
    if constexpr (A::KQW == 4) {
      const uint4 k = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, ad.koff, 0, 0));
      r.k[st][0] = k.x; r.k[st][1] = k.y; r.k[st][2] = k.z; r.k[st][3] = k.w;
    } else if constexpr (A::KQW == 3) {
      typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
      const u32x3 k = __builtin_bit_cast(u32x3, __builtin_amdgcn_raw_buffer_load_b96(rs, ad.koff, 0, 0));
      r.k[st][0] = k.x; r.k[st][1] = k.y; r.k[st][2] = k.z;
    } else {
      const uint2 k = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, ad.koff, 0, 0));
      r.k[st][0] = k.x; r.k[st][1] = k.y;
    }
    r.tail[st] = (uint16_t)buf_u16(rs, ad.toff, 0);
    if constexpr (VLM) {
      const uint4 x = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, ad.vtoff, 0, 0));
      r.vt[st][0] = x.x; r.vt[st][1] = x.y; r.vt[st][2] = x.z; r.vt[st][3] = x.w;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // scalar offset of token 4g+i; uniform, but LLVM otherwise keeps the
      // i >= 2 products in VGPRs and wraps each load in a waterfall loop
      const uint32_t so = __builtin_amdgcn_readfirstlane((uint32_t)i * ad.s_pos);
      // half (i & 1) of word w: into vb[w] (DEFER) or the high half of va[w]
      auto put = [&](int w, int half, uint32_t x) __attribute__((always_inline)) {
        if constexpr (DEFER) {
          if (half) r.vb[w] = (uint16_t)x;
          else r.va[w] = (uint16_t)x;
        } else {
          if (half) r.va[w] |= x << 16;
          else r.va[w] = x;
        }
      };
      if constexpr (VB == 2) {
        put(2 * st + (i >> 1), i & 1, buf_u16(rs, ad.voff, so));
      } else if constexpr (VB == 4) {
        const uint32_t lo = buf_u16(rs, ad.voff, so);
        const uint32_t hi = buf_u16(rs, ad.voff + 2u, so);
        put(2 * st + (i >> 1), i & 1, lo);
        put(4 + 2 * st + (i >> 1), i & 1, hi);
      } else {
        put(4 * st + i, 0, buf_u16(rs, ad.voff, so));
        put(4 * st + i, 1, buf_u16(rs, ad.voff + 2u, so));
      }
    }
    r.ok[st] = valid;
  }
}

// f16 pair (1 + q_a / 2^VB, 1 + q_b / 2^VB) for dim 8m + bb of the two tokens of pair j
// ex = the two tokens' f16 exponent fields (2^e_t (1 + q / 2^VB) once the code
// bits fill the top of the mantissa)
template <int VB, int NV>
__device__ __forceinline__ uint32_t v1_vpair(const uint32_t (&v)[NV], const uint32_t (&w)[8], int j, int bb,
                                             uint32_t ex) {
  const uint32_t ONE2 = ex;
  if constexpr (VB == 2) {
    const int sh = 8 - 2 * bb;
    const uint32_t x = sh >= 0 ? (v[j] << sh) : (v[j] >> -sh);
    return (x & 0x03000300u) | ONE2;
  } else if constexpr (VB == 4) {
    const uint32_t X = bb < 4 ? v[j] : v[4 + j];
    const int sh = 6 - 4 * (bb & 3);
    const uint32_t x = sh >= 0 ? (X << sh) : (X >> -sh);
    return (x & 0x03C003C0u) | ONE2;
  } else {
    // w[2j] = bytes 0-1 of each chunk (dims 0..4 + 1 bit), w[2j+1] = bytes 1-2 (dims 3..7)
    const uint32_t X = bb <= 2 ? w[2 * j] : w[2 * j + 1];
    const int sh = bb <= 2 ? 7 - 3 * bb : 15 - 3 * bb;
    const uint32_t x = sh >= 0 ? (X << sh) : (X >> -sh);
    return (x & 0x03800380u) | ONE2;
  }
}

__device__ __forceinline__ void wave_lds_fence() {
  // LDS accesses of one wave execute in order, so a write by one lane is seen
  // by a later read of another lane of the same wave; only the compiler must
  // not reorder them (a hardware fence here would also wait for the prefetch
  // loads in flight)
  __asm__ volatile("" ::: "memory");
}

// f16 pairs (a, b): hi | hi << 16 and lo | lo << 16, lo = f16(x - f16(x))
__device__ __forceinline__ uint2 cent_hilo_pair(float a, float b) {
  const uint32_t ha = f32_to_f16_bits(a), hb = f32_to_f16_bits(b);
  const uint32_t la = f32_to_f16_bits(a - f16_bits_to_f32(ha));
  const uint32_t lb = f32_to_f16_bits(b - f16_bits_to_f32(hb));
  return make_uint2(ha | (hb << 16), la | (lb << 16));
}

// VLM: Lloyd-Max V (TURBOQUANT_V_LLOYD_MAX, 4-bit V; reference
// triton_decode_offset.py:399-419): V = c[code] * ||v||_16 / ||c[codes]||,
// the K centroids shared.  The V codes become f16 centroid pairs (hi + lo)
// through a 4-bit pair table, ||c[codes]|| comes from the Gram diagonal of a
// token-major copy of the codes (as the K norm correction does), and
// P' = p ||v|| / ||c|| 2^-8 (hi + lo) feeds the P.V MFMA; accumulators are
// scaled back by 2^8.  With p <= 2^8 and ||c[codes]|| near 1 (unit-norm
// rotated vectors), P' stays below the f16 maximum for every f16 ||v||.
template <int D, int KB, int VB, int QT, bool VLM = false>
__global__ __launch_bounds__(256, 2) void v1_attn_kernel(
    const void* __restrict__ query, const uint8_t* __restrict__ cache,
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ seq_lens,
    const int32_t* __restrict__ kv_start, int hq, int hkv, int lbs, int max_blocks,
    int64_t num_blocks, int64_t s_blk, int64_t s_pos, int64_t s_head,
    const float* __restrict__ cent, float qscale, int num_splits, float* __restrict__ ws_o,
    float* __restrict__ ws_lse, const float* __restrict__ rot, V1Direct dout) {
  using A = V1A<D, KB, VB>;
  constexpr int NS = A::NS, NB = A::NB, E = D / 16;
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int G = hq / hkv;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m = lane & 15, g = lane >> 4;

  // K pair table: entry e = f16(sigma c[e & mask]) | f16(sigma c[e >> KB]) << 16, in LUT_C
  // interleaved copies (lane l reads copy l % LUT_C), so the random lookups of
  // a 32-lane LDS phase spread over the banks.  Static, so its address folds
  // into the lookups' DS offsets; a separate pool holds the rotated queries
  // (prologue) and the wave-merge buffer (epilogue).
  constexpr int LUT_LOGC = 5;
  constexpr int LUT_BYTES = (4 << (2 * KB)) << LUT_LOGC;
  constexpr int RED_BYTES = 4 * 16 * (D + 1) * 4;
  constexpr int QS_BYTES = 16 * (D + 4) * 4;
  constexpr int POOL = RED_BYTES > QS_BYTES ? RED_BYTES : QS_BYTES;
  __shared__ __attribute__((aligned(16))) uint32_t lut[LUT_BYTES / 4];
  __shared__ __attribute__((aligned(16))) uint8_t pool[POOL];
  __shared__ float red_m[4][16], red_l[4][16];
  __shared__ __attribute__((aligned(16))) uint16_t tail_l[4][2][4][16];
  __shared__ __attribute__((aligned(16))) float diag_l[4][2][16];
  __shared__ float tab_sc;   // sigma of the pair tables
  static_assert(!VLM || VB == 4, "Lloyd-Max V needs the 4-bit V layout");
  __shared__ uint2 lutv[VLM ? 256 : 1];  // Lloyd-Max V: centroid pairs (c[e & 15], c[e >> 4]), hi and lo
  __shared__ float diagv_l[VLM ? 4 : 1][2][16];   // Lloyd-Max V: sum c^2 per token
  float (*qs)[D + 4] = reinterpret_cast<float (*)[D + 4]>(pool);
  float (*red_o)[16][D + 1] = reinterpret_cast<float (*)[16][D + 1]>(pool);
  const uint32_t laneoff = 4u * (uint32_t)(lane & ((1 << LUT_LOGC) - 1));  // this lane's copy of the table
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);

  // Prologue, one barrier.  The last wave sizes and builds the pair tables;
  // the query heads' loads go out ahead of the dependent block-table loads,
  // and the first waves rotate them (one head per 16 lanes) once the first
  // tile's loads are out: q_rot = q H / sqrt(D), scale * log2(e) folded in.
  if (wave_u == 3) {
    const float csc = table_scale<1 << KB>(cent, true).sigma;
    build_pair_table_wave<KB, LUT_LOGC>(lut, f32_to_f16_bits(csc * cent[lane & ((1 << KB) - 1)]), lane);
    if constexpr (VLM) {
      constexpr int NC = 1 << KB;  // codes >= NC do not occur; they read the top centroid
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int e = lane + 64 * k, c0 = e & 15, c1 = e >> 4;
        lutv[e] = cent_hilo_pair(csc * cent[c0 < NC ? c0 : NC - 1], csc * cent[c1 < NC ? c1 : NC - 1]);
      }
    }
    if (lane == 0) tab_sc = csc;
  }
  const int qg = tid >> 4, ql16 = tid & 15;
  float y[E];
  if (qg < G) load_elems<QT, E>(query, ((int64_t)b * hq + kvh * G + qg) * D + ql16 * E, y);

  const int seq_len = seq_lens[b];
  int k0 = kv_start ? kv_start[b] : 0;
  if (k0 < 0) k0 = 0;
  const int t_first = k0 >> 5;
  const int t_last = (seq_len + 31) >> 5;
  const int n_tiles = t_last > t_first ? t_last - t_first : 0;
  const int tps = (n_tiles + num_splits - 1) / num_splits;
  const int t_begin = t_first + split * tps;
  const int t_end = min(t_begin + tps, t_last);
  const int32_t* bt_row = block_table + (int64_t)b * max_blocks;
  const int64_t kvh_off = (int64_t)kvh * s_head;

  // lane offsets (fixed for the kernel)
  V1Addr ad;
  ad.cache = cache;
  ad.s_blk = s_blk;
  ad.kvh_off = kvh_off;
  ad.s_pos = (uint32_t)s_pos;
  ad.lbs = lbs;
  ad.max_blocks = max_blocks;
  ad.seq_len = seq_len;
  v1_addr_rows(ad, bt_row, num_blocks);
  ad.koff = (uint32_t)m * ad.s_pos + (uint32_t)(g * A::KQ);
  ad.toff = (uint32_t)m * ad.s_pos +
            (uint32_t)(g == 1 ? A::KPS + A::VDB : (g == 2 ? A::KPS + A::VDB + 2 : A::MSE));
  ad.voff = (uint32_t)(4 * g) * ad.s_pos +
            (VB == 3 ? (uint32_t)((A::KPS + 3 * m) & ~1) : (uint32_t)(A::KPS + VB * m));
  ad.vtoff = (uint32_t)m * ad.s_pos + (uint32_t)A::KPS + 16u * (uint32_t)g;
  // VB 3: byte selectors that re-align each chunk to its first code bit
  const uint32_t o3 = (uint32_t)((A::KPS + 3 * m) & 1);
  const uint32_t sel0 = o3 | ((o3 + 1) << 8) | ((o3 + 4) << 16) | ((o3 + 5) << 24);
  const uint32_t sel1 = (o3 + 1) | ((o3 + 2) << 8) | ((o3 + 5) << 16) | ((o3 + 6) << 24);

  // the first tile's loads (two register sets: the next tile's loads overlap
  // this tile's math, and the block-table entries come one tile further ahead).
  // V words formed at the load: deferred, the raw halves would cost this
  // kernel a wave per SIMD at several widths (e.g. K2 V3 165 -> 187 VGPRs).
  V1Tile<D, KB, VB, false> ra, rb;
  int tile = t_begin + wave_u;
  int btv = 0;
  if (tile < t_end) {
    v1_load<D, KB, VB, VLM>(ra, ad, tile, true, v1_fetch_bt<false>(ad, tile, true, lane));
    btv = v1_fetch_bt<false>(ad, tile + 4, tile + 4 < t_end, lane);
  }

  if (qg < G) {
    if (rot != nullptr) rot_matrix_lanes<D, E>(y, rot, &qs[qg][0], ql16);  // q M (matrix strategies)
    else fwht_lanes<E, 16>(y, ql16);
#pragma unroll
    for (int i = 0; i < E; ++i) qs[qg][ql16 * E + i] = y[i] * qscale;
  }
  __syncthreads();
  const float csc = tab_sc;
  const float vk = csc * (1.f / 256.f), vinv = 256.f / csc;  // Lloyd-Max V: P' scale and its inverse
  // B operand of the Q.K MFMAs (f16 hi + lo): lane (n, g), MFMA s -> Q[n][g*D/4 + 8s + j]
  Op8 qb[NS], ql[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    float x[8];
    if (m < G) {
      const float4 a4 = *reinterpret_cast<const float4*>(&qs[m][g * (D / 4) + 8 * s]);
      const float4 c4 = *reinterpret_cast<const float4*>(&qs[m][g * (D / 4) + 8 * s + 4]);
      x[0] = a4.x; x[1] = a4.y; x[2] = a4.z; x[3] = a4.w; x[4] = c4.x; x[5] = c4.y; x[6] = c4.z; x[7] = c4.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t wh = 0, wl = 0;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float xv = x[2 * j + e];
        const _Float16 hi = (_Float16)xv;
        const _Float16 lo = (_Float16)(xv - (float)hi);
        wh |= (uint32_t)__builtin_bit_cast(uint16_t, hi) << (16 * e);
        wl |= (uint32_t)__builtin_bit_cast(uint16_t, lo) << (16 * e);
      }
      qb[s].u[j] = wh;
      ql[s].u[j] = wl;
    }
  }

  float m_run = -INFINITY, l_run = 0.f, z_run = 0.f, u_run = 0.f;
  floatx4 acc[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};

  constexpr float TAU = 8.f;  // p <= 2^TAU
  auto process = [&](const V1Tile<D, KB, VB, false>& cur, int tile) __attribute__((always_inline)) {
    // scores and Gram diagonal per S-tile; the per-token fields (K norm, V
    // scale, V min, sum C^2) go to the score layout (lane (n, g) holds tokens
    // 4g+i) through LDS
    floatx4 sacc[2];
    wave_lds_fence();
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      sacc[st] = floatx4{0.f, 0.f, 0.f, 0.f};
      floatx4 gacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        Op8 a;
#pragma unroll
        for (int p = 0; p < 4; ++p)
          a.u[p] = lds_dword_at(lut, lut_field<2 + LUT_LOGC, 2 * KB>(cur.k[st], (8 * s + 2 * p) * KB, laneoff));
        sacc[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, qb[s].h, sacc[st], 0, 0, 0);
        sacc[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, ql[s].h, sacc[st], 0, 0, 0);
        gacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, a.h, gacc, 0, 0, 0);
      }
      tail_l[wave][st][g][m] = (uint16_t)cur.tail[st];
      if ((m >> 2) == g) {
        const int i = m & 3;
        diag_l[wave][st][m] = i == 0 ? gacc[0] : i == 1 ? gacc[1] : i == 2 ? gacc[2] : gacc[3];
      }
      if constexpr (VLM) {
        // sum over the 128 dims of c[code]^2 per token: Gram diagonal of the
        // token-major V codes through the pair table (MFMA s takes codes 8s..8s+7)
        floatx4 gv = {0.f, 0.f, 0.f, 0.f}, gv2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          Op8 a, alo;
#pragma unroll
          for (int p = 0; p < 4; ++p) {
            const uint2 e = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(lutv) +
                                                            field_off<3>(cur.vt[st], (8 * s4 + 2 * p) * 4, 8));
            a.u[p] = e.x;
            alo.u[p] = e.y;
          }
          gv = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, a.h, gv, 0, 0, 0);
          gv2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo.h, a.h, gv2, 0, 0, 0);
        }
        if ((m >> 2) == g) {
          const int i = m & 3;
          const floatx4 gd = gv + 2.f * gv2;
          diagv_l[wave][st][m] = i == 0 ? gd[0] : i == 1 ? gd[1] : i == 2 ? gd[2] : gd[3];
        }
      }
    }
    wave_lds_fence();
    float s[2][4];
    float dvv[2][4];      // Lloyd-Max V: sum c^2 of token 4g+i
    uint2 scw[2], zw[2];  // f16 pairs: tokens (4g, 4g+1), (4g+2, 4g+3)
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const uint2 kn = *reinterpret_cast<const uint2*>(&tail_l[wave][st][0][4 * g]);
      scw[st] = *reinterpret_cast<const uint2*>(&tail_l[wave][st][1][4 * g]);
      zw[st] = *reinterpret_cast<const uint2*>(&tail_l[wave][st][2][4 * g]);
      const float4 dg = *reinterpret_cast<const float4*>(&diag_l[wave][st][4 * g]);
      const float dga[4] = {dg.x, dg.y, dg.z, dg.w};
      if constexpr (VLM) {
        const float4 dv = *reinterpret_cast<const float4*>(&diagv_l[wave][st][4 * g]);
        dvv[st][0] = dv.x; dvv[st][1] = dv.y; dvv[st][2] = dv.z; dvv[st][3] = dv.w;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t kw = (i < 2 ? kn.x : kn.y) >> (16 * (i & 1));
        const float knf = (float)__builtin_bit_cast(_Float16, (uint16_t)kw);
        s[st][i] = sacc[st][i] * knf * __builtin_amdgcn_rsqf(dga[i] + 1e-16f);
      }
    }
    // edge tiles: positions outside [k0, seq_len) and S-tiles without a page
    if (tile * 32 < k0 || tile * 32 + 32 > seq_len || !cur.ok[0] || !cur.ok[1]) {
#pragma unroll
      for (int st = 0; st < 2; ++st)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int pos = tile * 32 + st * 16 + 4 * g + i;
          if (pos >= seq_len || pos < k0 || !cur.ok[st]) {
            s[st][i] = -INFINITY;
            const uint32_t keep = (i & 1) ? 0x0000FFFFu : 0xFFFF0000u;
            if (i < 2) { scw[st].x &= keep; zw[st].x &= keep; }
            else { scw[st].y &= keep; zw[st].y &= keep; }
          }
        }
    }
    float tmax = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                       fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
    tmax = warp_max_q(tmax);
    if (__builtin_amdgcn_ballot_w64(tmax > m_run + TAU) != 0) {  // wave-uniform, rare
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
      z_run *= alpha;
      u_run *= alpha;
#pragma unroll
      for (int bb = 0; bb < NB; ++bb) acc[bb] *= alpha;
    }
    float psum = 0.f;
    Op8 pb, pl;
    uint32_t ex[4];  // per P.V operand pair: the two tokens' V-scale exponent fields
    if constexpr (VLM) {
      // P' = p ||v||_16 / sqrt(sum x^2 + 1e-16) 2^(k-8) for the scaled centroids x = c 2^k, hi + lo
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        uint32_t h16[4], l16[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = __builtin_amdgcn_exp2f(s[st][i] - m_run);
          psum += p;
          const uint32_t vw = (i < 2 ? scw[st].x : scw[st].y) >> (16 * (i & 1));
          const float vn = (float)__builtin_bit_cast(_Float16, (uint16_t)vw);
          const float u = p * vn * __builtin_amdgcn_rsqf(dvv[st][i] + 1e-16f) * vk;
          const _Float16 uh = (_Float16)u;
          h16[i] = __builtin_bit_cast(uint16_t, uh);
          l16[i] = __builtin_bit_cast(uint16_t, (_Float16)(u - (float)uh));
        }
        pb.u[2 * st] = h16[0] | (h16[1] << 16);
        pb.u[2 * st + 1] = h16[2] | (h16[3] << 16);
        pl.u[2 * st] = l16[0] | (l16[1] << 16);
        pl.u[2 * st + 1] = l16[2] | (l16[3] << 16);
      }
    } else {
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      uint32_t h16[4], l16[4];
#pragma unroll
      for (int hp = 0; hp < 2; ++hp) {
        const uint32_t scp = hp ? scw[st].y : scw[st].x;
        // exponent field clamped to [1, 29]: a zero / subnormal scale uses 2^-14
        // and carries its value in P'; a scale >= 2^15 uses 2^14 and P' < 2^(TAU+2)
        us2 e2 = __builtin_bit_cast(us2, scp & 0x7C007C00u);
        e2 = __builtin_elementwise_max(e2, us2{0x0400, 0x0400});
        e2 = __builtin_elementwise_min(e2, us2{0x7400, 0x7400});
        const uint32_t e = __builtin_bit_cast(uint32_t, e2);
        ex[2 * st + hp] = e;
        const uint32_t r = 0x78007800u - e;  // f16 2^(15 - exponent field) per token
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int i = 2 * hp + t;
          const float p = __builtin_amdgcn_exp2f(s[st][i] - m_run);
          psum += p;
          const uint32_t zq = (hp ? zw[st].y : zw[st].x) >> (16 * t);
          const float scf = (float)__builtin_bit_cast(_Float16, (uint16_t)(scp >> (16 * t)));
          z_run = __builtin_fmaf(p, (float)__builtin_bit_cast(_Float16, (uint16_t)zq), z_run);
          const float ps = p * scf;
          u_run += ps;
          const float u = ps * (float)__builtin_bit_cast(_Float16, (uint16_t)(r >> (16 * t)));
          const _Float16 uh = (_Float16)u;
          h16[i] = __builtin_bit_cast(uint16_t, uh);
          l16[i] = __builtin_bit_cast(uint16_t, (_Float16)(u - (float)uh));
        }
      }
      pb.u[2 * st] = h16[0] | (h16[1] << 16);
      pb.u[2 * st + 1] = h16[2] | (h16[3] << 16);
      pl.u[2 * st] = l16[0] | (l16[1] << 16);
      pl.u[2 * st + 1] = l16[2] | (l16[3] << 16);
    }
    }
    l_run += psum;
    uint32_t cv[A::NV];  // the V operand words
#pragma unroll
    for (int k = 0; k < A::NV; ++k) cv[k] = cur.vword(k);
    uint32_t w3[8];
    if constexpr (VB == 3) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        w3[2 * j] = __builtin_amdgcn_perm(cv[2 * j + 1], cv[2 * j], sel0);
        w3[2 * j + 1] = __builtin_amdgcn_perm(cv[2 * j + 1], cv[2 * j], sel1);
      }
    }
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) {
      Op8 a;
      if constexpr (VLM) {
        // pair j: the 4-bit codes of dim 8m + bb of its two tokens -> f16 centroid
        // pair (hi), plus its remainder (lo) against P'_hi
        Op8 alo;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t X = bb < 4 ? cv[j] : cv[4 + j];
          const uint32_t idx = __builtin_amdgcn_ubfe(X, 4 * (bb & 3), 4) |
                               (__builtin_amdgcn_ubfe(X, 16 + 4 * (bb & 3), 4) << 4);
          const uint2 e = lutv[idx];
          a.u[j] = e.x;
          alo.u[j] = e.y;
        }
        acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo.h, pb.h, acc[bb], 0, 0, 0);
      } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) a.u[j] = v1_vpair<VB>(cv, w3, j, bb, ex[j]);
      }
      acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, pb.h, acc[bb], 0, 0, 0);
      acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, pl.h, acc[bb], 0, 0, 0);
    }
  };

  // The uniform V codes enter the P.V MFMAs as 2^e (1 + q 2^-k): the sums
  // carry an offset, sum p sc (u_run), that the epilogue subtracts.  Its fp32
  // rounding grows with the tiles summed (a wave of ~950 tiles erred by 8e-2
  // on fp32 outputs of a 122K-position sequence, K4 V2), so every 16 tiles
  // the offset so far leaves both sums.
  int since = 0;
  auto rebase = [&]() __attribute__((always_inline)) {
    if constexpr (!VLM) {
      if (++since == 16) {
        since = 0;
        const float u = warp_sum_q(u_run);
#pragma unroll
        for (int bb = 0; bb < NB; ++bb) acc[bb] -= u;
        u_run = 0.f;
      }
    }
  };
  // each wave takes every 4th tile (a fixed assignment, so the sums and the
  // output bits do not depend on how fast the waves progress)
  while (tile < t_end) {
    int btn = v1_fetch_bt<false>(ad, tile + 8, tile + 8 < t_end, lane);
    v1_load<D, KB, VB, VLM>(rb, ad, tile + 4, true, btv);
    btv = btn;
    process(ra, tile);
    rebase();
    tile += 4;
    if (tile >= t_end) break;
    btn = v1_fetch_bt<false>(ad, tile + 8, tile + 8 < t_end, lane);
    v1_load<D, KB, VB, VLM>(ra, ad, tile + 4, true, btv);
    btv = btn;
    process(rb, tile);
    rebase();
    tile += 4;
  }

  // ---- merge the 4 waves through LDS (the pool of the rotated queries) ----
  __syncthreads();
  const float l_tot = warp_sum_q(l_run);
  const float z_tot = warp_sum_q(z_run);
  const float u_tot = warp_sum_q(u_run);
  if (g == 0) {
    red_m[wave][m] = m_run;
    red_l[wave][m] = l_tot;
  }
  constexpr float VSC = (float)(1 << VB);
#pragma unroll
  for (int bb = 0; bb < NB; ++bb)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      red_o[wave][m][8 * (4 * g + i) + bb] = VLM ? acc[bb][i] * vinv : __builtin_fmaf(acc[bb][i] - u_tot, VSC, z_tot);
  __syncthreads();

  if (dout.mode >= 0) {  // one split: the output itself
    v1_direct_rows<D, 16, D + 1>(red_m, red_l, red_o, G, wave, lane, (int64_t)b * hq + kvh * G, dout);
    return;
  }
  const int64_t row0 = ((int64_t)b * hq + kvh * G) * num_splits + split;  // (b, head 0 of the group, split)
  for (int idx = tid; idx < G * D; idx += 256) {
    const int gg = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, red_m[w][gg]);
    float L = 0.f, o = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float f = __builtin_amdgcn_exp2f(red_m[w][gg] - M);
        L += f * red_l[w][gg];
        o += f * red_o[w][gg][d];
      }
    }
    const int64_t row = row0 + (int64_t)gg * num_splits;
    ws_o[row * D + d] = (L > 0.f) ? o / L : 0.f;
    if (d == 0) ws_lse[row] = (L > 0.f) ? M + __builtin_log2f(L) : -INFINITY;
  }
}

// ---------------------------------------------------------------------------
// decode attention, stage 1, GQA group of 4 (e.g. 32 query / 8 kv heads)
// ---------------------------------------------------------------------------
// Same tiles, loads and MFMAs as v1_attn_kernel, but the per-(token, head)
// work runs in a compact layout: after the score MFMA only 4 of its 16
// columns are real heads, so the scores of an S-tile (16 tokens x 4 heads) are
// moved with three DPP row shifts to one value per lane,
//   compact lane 16g + 4i + n  <->  token 4g + i of the S-tile, head n,
// the softmax, P' and its hi/lo split run once per value, and three DPP row
// shifts plus byte permutes build the P.V operand back.
// The V operand needs no shift: dim 8m + bb's code stays at its bit position
// inside the 16-bit chunk (for the first 8 bits; the rest from the chunk
// shifted by 8), which is mantissa bit pos_bb of the f16 2^e (1 + q 2^(pos_bb-10));
// accumulator bb is scaled by 2^(10 - pos_bb) at the end.

// mantissa position of the code of dim 8m + bb in the V operand, and the
// source word: 0 = the chunk pair, 1 = it shifted right by 8, 2 = by 16 (VB 3)
template <int VB> __host__ __device__ constexpr int v1_vpos(int bb) {
  return VB == 2 ? (bb <= 4 ? 2 * bb : 2 * bb - 8)
       : VB == 4 ? (4 * (bb & 1))
       : (bb <= 2 ? 3 * bb : bb <= 5 ? 3 * bb - 8 : 3 * bb - 16);
}

// 2-bit V: 4 workgroups per CU (<= 128 VGPRs, no spills; B = 4, 32 / 8 heads,
// 64K-128K positions, K4 V2 ran 83 us
// against 90 us at 3 per CU); 3- and 4-bit V need more registers
template <int D, int KB, int VB, int QT>
__global__ __launch_bounds__(256, VB == 2 ? 4 : 2) void v1_attn_g4_kernel(
    const void* __restrict__ query, const uint8_t* __restrict__ cache,
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ seq_lens,
    const int32_t* __restrict__ kv_start, int hq, int hkv, int lbs, int max_blocks,
    int64_t num_blocks, int64_t s_blk, int64_t s_pos, int64_t s_head,
    const float* __restrict__ cent, float qscale, int num_splits, float* __restrict__ ws_o,
    float* __restrict__ ws_lse, const float* __restrict__ rot, V1Direct dout) {
  using A = V1A<D, KB, VB>;
  constexpr int NS = A::NS, NB = A::NB, E = D / 16;
  constexpr int G = 4;
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m = lane & 15, g = lane >> 4;      // MFMA layout: row / column m, k-group g
  const int ci = (lane >> 2) & 3;  // compact layout: head lane & 3, token 4g + ci

  // K pair table in LUT_C interleaved copies (lane l reads copy l % LUT_C):
  // 32 for 2- and 3-bit keys; 16 for 4-bit (16 KB, so that 4 workgroups still
  // fit a CU's LDS).  Static, so its address folds into the lookups' DS
  // offsets; a separate pool holds the rotated queries (prologue) and the
  // wave-merge buffer (epilogue).
  constexpr int LUT_LOGC = KB == 4 ? 4 : 5;
  constexpr int LUT_BYTES = (4 << (2 * KB)) << LUT_LOGC;
  constexpr int RED_BYTES = 4 * G * (D + 1) * 4;
  constexpr int QS_BYTES = G * (D + 4) * 4;
  constexpr int POOL = RED_BYTES > QS_BYTES ? RED_BYTES : QS_BYTES;
  __shared__ __attribute__((aligned(16))) uint32_t lut[LUT_BYTES / 4];
  __shared__ __attribute__((aligned(16))) uint8_t pool[POOL];
  __shared__ float red_m[4][G], red_l[4][G];
  __shared__ __attribute__((aligned(16))) uint16_t tail_l[4][2][4][16];  // [wave][S-tile][field][token]
  __shared__ __attribute__((aligned(16))) float diag_l[4][2][64][4];  // [wave][S-tile][lane][register]
  float (*qs)[D + 4] = reinterpret_cast<float (*)[D + 4]>(pool);
  float (*red_o)[G][D + 1] = reinterpret_cast<float (*)[G][D + 1]>(pool);
  const uint32_t laneoff = 4u * (uint32_t)(lane & ((1 << LUT_LOGC) - 1));  // this lane's copy of the table
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);

  // Prologue, one barrier.  The last wave sizes and builds the K pair table
  // (f16(sigma c), sigma from table_scale; the norm correction divides by the
  // norm of the same f16 values, so sigma cancels); the query heads' loads go
  // out ahead of the dependent block-table loads, and wave 0 rotates them
  // (one head per 16 lanes) once the first tile's loads are out.
  if (wave_u == 3) {
    const float csc = table_scale<1 << KB>(cent, true).sigma;
    build_pair_table_wave<KB, LUT_LOGC>(lut, f32_to_f16_bits(csc * cent[lane & ((1 << KB) - 1)]), lane);
  }
  const int qg = tid >> 4, ql16 = tid & 15;
  float y[E];
  if (qg < G) load_elems<QT, E>(query, ((int64_t)b * hq + kvh * G + qg) * D + ql16 * E, y);

  const int seq_len = seq_lens[b];
  int k0 = kv_start ? kv_start[b] : 0;
  if (k0 < 0) k0 = 0;
  const int t_first = k0 >> 5;
  const int t_last = (seq_len + 31) >> 5;
  const int n_tiles = t_last > t_first ? t_last - t_first : 0;
  const int tps = (n_tiles + num_splits - 1) / num_splits;
  const int t_begin = t_first + split * tps;
  const int t_end = min(t_begin + tps, t_last);
  const int32_t* bt_row = block_table + (int64_t)b * max_blocks;
  const int64_t kvh_off = (int64_t)kvh * s_head;

  V1Addr ad;
  ad.cache = cache;
  ad.s_blk = s_blk;
  ad.kvh_off = kvh_off;
  ad.s_pos = (uint32_t)s_pos;
  ad.lbs = lbs;
  ad.max_blocks = max_blocks;
  ad.seq_len = seq_len;
  v1_addr_rows(ad, bt_row, num_blocks);
  ad.koff = (uint32_t)m * ad.s_pos + (uint32_t)(g * A::KQ);
  ad.toff = (uint32_t)m * ad.s_pos +
            (uint32_t)(g == 1 ? A::KPS + A::VDB : (g == 2 ? A::KPS + A::VDB + 2 : A::MSE));
  ad.voff = (uint32_t)(4 * g) * ad.s_pos +
            (VB == 3 ? (uint32_t)((A::KPS + 3 * m) & ~1) : (uint32_t)(A::KPS + VB * m));
  // VB 3: byte selectors giving chunk bits [0,16), [8,24), [16,24) of both tokens of a pair
  const uint32_t o3 = (uint32_t)((A::KPS + 3 * m) & 1);
  const uint32_t sel0 = o3 | ((o3 + 1) << 8) | ((o3 + 4) << 16) | ((o3 + 5) << 24);
  const uint32_t sel1 = (o3 + 1) | ((o3 + 2) << 8) | ((o3 + 5) << 16) | ((o3 + 6) << 24);
  const uint32_t sel2 = (o3 + 2) | (0x0Cu << 8) | ((o3 + 6) << 16) | (0x0Cu << 24);

  // the first tile's loads (two register sets: the next tile's loads overlap
  // this tile's math, and the block-table entries come one tile further ahead)
  // DEFER (3- and 4-bit V): the V words and the block-table test are formed
  // in the step that uses them, so no wait in a loading step covers the
  // loads it has just issued (two splits over 64 x 8 (batch, kv head) units,
  // K3 V3: 49.6 -> 44.2 us).  2-bit V forms them at the load: deferred, its
  // registers would pass the 128 of 4 workgroups per CU.
  constexpr bool DEFER = VB != 2;
  V1Tile<D, KB, VB, DEFER> ra, rb;
  int tile = t_begin + wave_u;
  int btv = 0;
  if (tile < t_end) {
    v1_load(ra, ad, tile, true, v1_fetch_bt<DEFER>(ad, tile, true, lane));
    btv = v1_fetch_bt<DEFER>(ad, tile + 4, tile + 4 < t_end, lane);
  }

  if (qg < G) {
    if (rot != nullptr) rot_matrix_lanes<D, E>(y, rot, &qs[qg][0], ql16);  // q M (matrix strategies)
    else fwht_lanes<E, 16>(y, ql16);
#pragma unroll
    for (int i = 0; i < E; ++i) qs[qg][ql16 * E + i] = y[i] * qscale;
  }
  __syncthreads();
  // B operand of the Q.K MFMAs: column n < G holds f16(q) of head n, column
  // G + n its remainder q - f16(q); the two score columns are summed after the
  // K loop, so q enters in about fp32 precision at no extra MFMA
  Op8 qb[NS];
  {
    const int hq_ = m < G ? m : m - G;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      float x[8];
      if (m < 2 * G) {
        const float4 a4 = *reinterpret_cast<const float4*>(&qs[hq_][g * (D / 4) + 8 * s]);
        const float4 c4 = *reinterpret_cast<const float4*>(&qs[hq_][g * (D / 4) + 8 * s + 4]);
        x[0] = a4.x; x[1] = a4.y; x[2] = a4.z; x[3] = a4.w; x[4] = c4.x; x[5] = c4.y; x[6] = c4.z; x[7] = c4.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = 0.f;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float xv = x[2 * j + e];
          const _Float16 hi = (_Float16)xv;
          const _Float16 v = m < G ? hi : (_Float16)(xv - (float)hi);
          w |= (uint32_t)__builtin_bit_cast(uint16_t, v) << (16 * e);
        }
        qb[s].u[j] = w;
      }
    }
  }

  float m_run = -INFINITY, l_run = 0.f, z_run = 0.f, u_run = 0.f;  // per compact lane, head cn
  floatx4 acc[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};

  constexpr float TAU = 8.f;  // p <= 2^TAU
  auto process = [&](const V1Tile<D, KB, VB, DEFER>& cur, int tile) __attribute__((always_inline)) {
    floatx4 sacc[2];
    wave_lds_fence();
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      sacc[st] = floatx4{0.f, 0.f, 0.f, 0.f};
      floatx4 gacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        Op8 a;
#pragma unroll
        for (int p = 0; p < 4; ++p)
          a.u[p] = lds_dword_at(lut, lut_field<2 + LUT_LOGC, 2 * KB>(cur.k[st], (8 * s + 2 * p) * KB, laneoff));
        sacc[st] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, qb[s].h, sacc[st], 0, 0, 0);
        gacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, a.h, gacc, 0, 0, 0);
      }
      tail_l[wave][st][g][m] = (uint16_t)cur.tail[st];
      // Gram[t][t] of token t sits in lane 16(t/4) + t, register t % 4: every
      // lane stores its 4 registers and the readers pick the diagonal
      *reinterpret_cast<floatx4*>(&diag_l[wave][st][lane][0]) = gacc;
    }
    wave_lds_fence();
    // score column n += column n + G (the q remainder), then to the compact
    // layout: lane 16g + 4i + n <- lane 16g + n, register i
    float sc_[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        sacc[st][i] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sacc[st][i]), 0x100 + G, 0xF, 0xF, true));
      int x = __float_as_int(sacc[st][0]);
      x = __builtin_amdgcn_update_dpp(x, __float_as_int(sacc[st][1]), 0x114, 0xF, 0x2, false);
      x = __builtin_amdgcn_update_dpp(x, __float_as_int(sacc[st][2]), 0x118, 0xF, 0x4, false);
      x = __builtin_amdgcn_update_dpp(x, __float_as_int(sacc[st][3]), 0x11C, 0xF, 0x8, false);
      sc_[st] = __int_as_float(x);
    }
    // per-token fields of token 4g + ci (compact) and the V scale pairs (MFMA layout)
    float s[2], scf[2], zf[2];
    uint2 scw[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const int tok = 4 * g + ci;
      const float knf = (float)__builtin_bit_cast(_Float16, tail_l[wave][st][0][tok]);
      scf[st] = (float)__builtin_bit_cast(_Float16, tail_l[wave][st][1][tok]);
      zf[st] = (float)__builtin_bit_cast(_Float16, tail_l[wave][st][2][tok]);
      const float dg = diag_l[wave][st][16 * g + tok][ci];
      s[st] = sc_[st] * knf * __builtin_amdgcn_rsqf(dg + 1e-16f);
      scw[st] = *reinterpret_cast<const uint2*>(&tail_l[wave][st][1][4 * g]);
    }
    if (tile * 32 < k0 || tile * 32 + 32 > seq_len || !cur.ok[0] || !cur.ok[1]) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        // the MFMA-layout scale pairs of masked tokens only feed exponents (P' is 0 there)
        const int pos = tile * 32 + st * 16 + 4 * g + ci;
        const bool bad = pos >= seq_len || pos < k0 || !cur.ok[st];
        s[st] = bad ? -INFINITY : s[st];
        scf[st] = bad ? 0.f : scf[st];
        zf[st] = bad ? 0.f : zf[st];
      }
    }
    if (__builtin_amdgcn_ballot_w64(fmaxf(s[0], s[1]) > m_run + TAU) != 0) {  // wave-uniform, rare
      float t = fmaxf(s[0], s[1]);
      t = fmaxf(t, dpp_xor4(t));
      t = fmaxf(t, dpp_xor8(t));
      t = fmaxf(t, __shfl_xor(t, 16));
      t = fmaxf(t, __shfl_xor(t, 32));
      const float m_new = fmaxf(m_run, t);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
      z_run *= alpha;
      u_run *= alpha;
      // acc column (lane & 15) < 4 is head lane & 3: the same lane's alpha
#pragma unroll
      for (int bb = 0; bb < NB; ++bb) acc[bb] *= alpha;
    }
    // P' = p sc / 2^e (f16 hi + lo), packed hi | lo << 16 per compact lane
    uint32_t w[2];
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const float p = __builtin_amdgcn_exp2f(s[st] - m_run);
      l_run += p;
      z_run = __builtin_fmaf(p, zf[st], z_run);
      const float ps = p * scf[st];
      u_run += ps;
      uint32_t eb = __builtin_bit_cast(uint16_t, (_Float16)scf[st]) & 0x7C00u;
      eb = eb < 0x0400u ? 0x0400u : (eb > 0x7400u ? 0x7400u : eb);
      const float r = (float)__builtin_bit_cast(_Float16, (uint16_t)(0x7800u - eb));
      const float u = ps * r;
      const _Float16 uh = (_Float16)u;
      const _Float16 ul = (_Float16)(u - (float)uh);
      w[st] = (uint32_t)__builtin_bit_cast(uint16_t, uh) | ((uint32_t)__builtin_bit_cast(uint16_t, ul) << 16);
    }
    // back to the P.V operand: lane (n, g) takes tokens 4g..4g+3 of head n from
    // compact lanes n, n+4, n+8, n+12 of its row
    Op8 pb, pl;
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const uint32_t w0 = w[st];
      const uint32_t w1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)w0, 0x104, 0xF, 0xF, true);
      const uint32_t w2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)w0, 0x108, 0xF, 0xF, true);
      const uint32_t w3 = (uint32_t)__builtin_amdgcn_mov_dpp((int)w0, 0x10C, 0xF, 0xF, true);
      pb.u[2 * st] = __builtin_amdgcn_perm(w1, w0, 0x05040100u);
      pb.u[2 * st + 1] = __builtin_amdgcn_perm(w3, w2, 0x05040100u);
      pl.u[2 * st] = __builtin_amdgcn_perm(w1, w0, 0x07060302u);
      pl.u[2 * st + 1] = __builtin_amdgcn_perm(w3, w2, 0x07060302u);
    }
    // V operand exponent words (pair j: tokens 4g + 2(j&1), +1 of S-tile j/2)
    uint32_t ex[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t scp = (j & 1) ? scw[j >> 1].y : scw[j >> 1].x;
      us2 e2 = __builtin_bit_cast(us2, scp & 0x7C007C00u);
      e2 = __builtin_elementwise_max(e2, us2{0x0400, 0x0400});
      e2 = __builtin_elementwise_min(e2, us2{0x7400, 0x7400});
      ex[j] = __builtin_bit_cast(uint32_t, e2);
    }
    // V code words: [0] the chunk pairs, [1] shifted by 8, [2] by 16 (VB 3 only)
    uint32_t vw[3][A::NV];
#pragma unroll
    for (int j = 0; j < A::NV; ++j) {
      if constexpr (VB == 3) {
        if (j < 4) {
          const uint32_t v0 = cur.vword(2 * j), v1 = cur.vword(2 * j + 1);
          vw[0][j] = __builtin_amdgcn_perm(v1, v0, sel0);
          vw[1][j] = __builtin_amdgcn_perm(v1, v0, sel1);
          vw[2][j] = __builtin_amdgcn_perm(v1, v0, sel2);
        }
      } else {
        vw[0][j] = cur.vword(j);
        vw[1][j] = vw[0][j] >> 8;
      }
    }
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) {
      const int pos = v1_vpos<VB>(bb);
      const uint32_t msk = ((uint32_t)((1 << VB) - 1) << pos) * 0x00010001u;
      Op8 a;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t x;
        if constexpr (VB == 2) x = bb <= 4 ? vw[0][j] : vw[1][j];
        else if constexpr (VB == 4) x = vw[(bb >> 1) & 1][(bb < 4 ? 0 : 4) + j];
        else x = vw[bb <= 2 ? 0 : (bb <= 5 ? 1 : 2)][j];
        a.u[j] = (x & msk) | ex[j];
      }
      acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, pb.h, acc[bb], 0, 0, 0);
      acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, pl.h, acc[bb], 0, 0, 0);
    }
  };

  auto head_sum = [](float x) __attribute__((always_inline)) {
    x += dpp_xor4(x);
    x += dpp_xor8(x);
    x += __shfl_xor(x, 16);
    x += __shfl_xor(x, 32);
    return x;
  };
  // The V codes enter the P.V MFMAs as 2^e (1 + q 2^-k): the sums carry an
  // offset, sum p sc (u_run), that the epilogue subtracts.  Its fp32 rounding
  // grows with the tiles summed (a wave of ~950 tiles erred by 8e-2 on fp32
  // outputs of a 122K-position sequence, K4 V2), so every 16 tiles the offset
  // so far leaves both sums (acc column m < 4 is head lane & 3, whose compact
  // lanes head_sum adds).
  int since = 0;
  auto rebase = [&]() __attribute__((always_inline)) {
    if (++since == 16) {
      since = 0;
      const float u = head_sum(u_run);
#pragma unroll
      for (int bb = 0; bb < NB; ++bb) acc[bb] -= u;
      u_run = 0.f;
    }
  };
  // each wave takes every 4th tile (a fixed assignment, so the sums and the
  // output bits do not depend on how fast the waves progress)
  while (tile < t_end) {
    int btn = v1_fetch_bt<DEFER>(ad, tile + 8, tile + 8 < t_end, lane);
    v1_load(rb, ad, tile + 4, tile + 4 < t_end, btv);
    btv = btn;
    process(ra, tile);
    rebase();
    tile += 4;
    if (tile >= t_end) break;
    btn = v1_fetch_bt<DEFER>(ad, tile + 8, tile + 8 < t_end, lane);
    v1_load(ra, ad, tile + 4, tile + 4 < t_end, btv);
    btv = btn;
    process(rb, tile);
    rebase();
    tile += 4;
  }

  // ---- per-head totals over the 16 compact lanes of each head, wave merge ----
  __syncthreads();
  const float l_tot = head_sum(l_run);
  const float z_tot = head_sum(z_run);
  const float u_tot = head_sum(u_run);
  if (lane < G) {
    red_m[wave][lane] = m_run;
    red_l[wave][lane] = l_tot;
  }
  if (m < G) {  // MFMA column m is head m; this lane's compact head (lane & 3) is m too
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) {
      const float vsc = (float)(1 << (10 - v1_vpos<VB>(bb)));
#pragma unroll
      for (int i = 0; i < 4; ++i)
        red_o[wave][m][8 * (4 * g + i) + bb] = __builtin_fmaf(acc[bb][i] - u_tot, vsc, z_tot);
    }
  }
  __syncthreads();

  if (dout.mode >= 0) {  // one split: the output itself
    v1_direct_rows<D, G, D + 1>(red_m, red_l, red_o, G, wave, lane, (int64_t)b * hq + kvh * G, dout);
    return;
  }
  const int64_t row0 = ((int64_t)b * hq + kvh * G) * num_splits + split;
  for (int idx = tid; idx < G * D; idx += 256) {
    const int gg = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, red_m[w][gg]);
    float L = 0.f, o = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const float f = __builtin_amdgcn_exp2f(red_m[w][gg] - M);
        L += f * red_l[w][gg];
        o += f * red_o[w][gg][d];
      }
    }
    const int64_t row = row0 + (int64_t)gg * num_splits;
    ws_o[row * D + d] = (L > 0.f) ? o / L : 0.f;
    if (d == 0) ws_lse[row] = (L > 0.f) ? M + __builtin_log2f(L) : -INFINITY;
  }
}

// ---------------------------------------------------------------------------
// host launchers (stage 2 -- LSE merge of the splits, V un-rotation, output
// cast, the merge of vLLM's stage-2 kernel, v1_backend.py:1070-1093 -- is
// merge_splits_kernel in ftq_merge.h)
// ---------------------------------------------------------------------------

// dense matrix rotation (a caller's own M): x M through a per-group LDS row
template <int D>
static hipError_t v1_launch_store_dense(const void* k, const void* v, int dt, int64_t n, int hkv,
                                        const float* mids, int kb, int vb, int vrot, const int64_t* slots,
                                        uint8_t* cache, int64_t nb, int bs, int64_t sb, int64_t sp,
                                        int64_t sh, const float* rot, hipStream_t st) {
  const int64_t nvec = n * hkv;
  int64_t gsz = (nvec + 15) / 16;
  if (gsz > 256 * 16) gsz = 256 * 16;
  dim3 grid((unsigned)gsz), block(256);
  if (dt == F32)
    v1_store_kernel<D, F32, true><<<grid, block, 0, st>>>(k, v, n, hkv, mids, kb, vb, vrot, slots, cache, nb, bs, sb, sp, sh, 1.f, rot);
  else if (dt == F16)
    v1_store_kernel<D, F16, true><<<grid, block, 0, st>>>(k, v, n, hkv, mids, kb, vb, vrot, slots, cache, nb, bs, sb, sp, sh, 1.f, rot);
  else
    v1_store_kernel<D, BF16, true><<<grid, block, 0, st>>>(k, v, n, hkv, mids, kb, vb, vrot, slots, cache, nb, bs, sb, sp, sh, 1.f, rot);
  return hipGetLastError();
}



template <int D, int KB, int VB>
static hipError_t v1_launch_attn3(const V1Args& a, hipStream_t st) {
  dim3 grid(a.splits, a.hkv, a.B), block(256);
  // one split and no caller matrix: the kernel writes the output, no merge
  const bool direct = a.splits == 1 && !((a.vrot & 1) && a.rot != nullptr);
  const V1Direct dout{a.out, a.lse, fwht_scale(D), a.ot, direct ? (a.vrot & 1) : -1};
  if constexpr (VB == 4) {
    if (a.vrot & 2) {  // Lloyd-Max V codes
      if (a.qt == F32)
        v1_attn_kernel<D, KB, VB, F32, true><<<grid, block, 0, st>>>(a.q, a.cache, a.bt, a.sl, a.ks, a.hq, a.hkv, a.lbs, a.max_blocks, a.nb, a.sblk, a.spos, a.shead, a.cent, a.qscale, a.splits, a.wo, a.wl, a.rot, dout);
      else if (a.qt == F16)
        v1_attn_kernel<D, KB, VB, F16, true><<<grid, block, 0, st>>>(a.q, a.cache, a.bt, a.sl, a.ks, a.hq, a.hkv, a.lbs, a.max_blocks, a.nb, a.sblk, a.spos, a.shead, a.cent, a.qscale, a.splits, a.wo, a.wl, a.rot, dout);
      else
        v1_attn_kernel<D, KB, VB, BF16, true><<<grid, block, 0, st>>>(a.q, a.cache, a.bt, a.sl, a.ks, a.hq, a.hkv, a.lbs, a.max_blocks, a.nb, a.sblk, a.spos, a.shead, a.cent, a.qscale, a.splits, a.wo, a.wl, a.rot, dout);
      goto merge;
    }
  }
  if (a.hq == 4 * a.hkv) {
    if (a.qt == F32)
      v1_attn_g4_kernel<D, KB, VB, F32><<<grid, block, 0, st>>>(a.q, a.cache, a.bt, a.sl, a.ks, a.hq, a.hkv, a.lbs, a.max_blocks, a.nb, a.sblk, a.spos, a.shead, a.cent, a.qscale, a.splits, a.wo, a.wl, a.rot, dout);
    else if (a.qt == F16)
      v1_attn_g4_kernel<D, KB, VB, F16><<<grid, block, 0, st>>>(a.q, a.cache, a.bt, a.sl, a.ks, a.hq, a.hkv, a.lbs, a.max_blocks, a.nb, a.sblk, a.spos, a.shead, a.cent, a.qscale, a.splits, a.wo, a.wl, a.rot, dout);
    else
      v1_attn_g4_kernel<D, KB, VB, BF16><<<grid, block, 0, st>>>(a.q, a.cache, a.bt, a.sl, a.ks, a.hq, a.hkv, a.lbs, a.max_blocks, a.nb, a.sblk, a.spos, a.shead, a.cent, a.qscale, a.splits, a.wo, a.wl, a.rot, dout);
  } else if (a.qt == F32)
    v1_attn_kernel<D, KB, VB, F32><<<grid, block, 0, st>>>(a.q, a.cache, a.bt, a.sl, a.ks, a.hq, a.hkv, a.lbs, a.max_blocks, a.nb, a.sblk, a.spos, a.shead, a.cent, a.qscale, a.splits, a.wo, a.wl, a.rot, dout);
  else if (a.qt == F16)
    v1_attn_kernel<D, KB, VB, F16><<<grid, block, 0, st>>>(a.q, a.cache, a.bt, a.sl, a.ks, a.hq, a.hkv, a.lbs, a.max_blocks, a.nb, a.sblk, a.spos, a.shead, a.cent, a.qscale, a.splits, a.wo, a.wl, a.rot, dout);
  else
    v1_attn_kernel<D, KB, VB, BF16><<<grid, block, 0, st>>>(a.q, a.cache, a.bt, a.sl, a.ks, a.hq, a.hkv, a.lbs, a.max_blocks, a.nb, a.sblk, a.spos, a.shead, a.cent, a.qscale, a.splits, a.wo, a.wl, a.rot, dout);
merge:
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || direct) return e;
  const int64_t rows = (int64_t)a.B * a.hq;
  const float rs = fwht_scale(D);
  if ((a.vrot & 1) && a.rot != nullptr) {  // o M^T
    if (a.ot == F32) return launch_merge_splits<D, F32, ROT_MATRIX>(a.wo, a.wl, rows, a.splits, a.rot, 1.f, a.out, st, a.lse);
    if (a.ot == F16) return launch_merge_splits<D, F16, ROT_MATRIX>(a.wo, a.wl, rows, a.splits, a.rot, 1.f, a.out, st, a.lse);
    return launch_merge_splits<D, BF16, ROT_MATRIX>(a.wo, a.wl, rows, a.splits, a.rot, 1.f, a.out, st, a.lse);
  }
  if (a.vrot & 1) {
    if (a.ot == F32) return launch_merge_splits<D, F32, ROT_PLAIN>(a.wo, a.wl, rows, a.splits, nullptr, rs, a.out, st, a.lse);
    if (a.ot == F16) return launch_merge_splits<D, F16, ROT_PLAIN>(a.wo, a.wl, rows, a.splits, nullptr, rs, a.out, st, a.lse);
    return launch_merge_splits<D, BF16, ROT_PLAIN>(a.wo, a.wl, rows, a.splits, nullptr, rs, a.out, st, a.lse);
  }
  if (a.ot == F32) return launch_merge_splits<D, F32, ROT_NONE>(a.wo, a.wl, rows, a.splits, nullptr, rs, a.out, st, a.lse);
  if (a.ot == F16) return launch_merge_splits<D, F16, ROT_NONE>(a.wo, a.wl, rows, a.splits, nullptr, rs, a.out, st, a.lse);
  return launch_merge_splits<D, BF16, ROT_NONE>(a.wo, a.wl, rows, a.splits, nullptr, rs, a.out, st, a.lse);
}

template <int D, int KB>
static hipError_t v1_launch_attn2(int vb, const V1Args& a, hipStream_t st) {
  if (vb == 2) return v1_launch_attn3<D, KB, 2>(a, st);
  if (vb == 3) return v1_launch_attn3<D, KB, 3>(a, st);
  return v1_launch_attn3<D, KB, 4>(a, st);
}

int auto_splits(int batch, int hkv, int seq_hint, int target_wgs);

}  // namespace ftq

using namespace ftq;

extern "C" int64_t ftq_v1_slot_bytes_flags(int d, int key_bits, int value_bits, int v_flags) {
  if (!(d == 64 || d == 128 || d == 256) || !v1_widths_ok(key_bits, value_bits, v_flags)) return -1;
  return v1_geom(d, key_bits, value_bits, (v_flags & V1F_KFP8) != 0).raw;
}

extern "C" int64_t ftq_v1_slot_bytes(int d, int key_bits, int value_bits) {
  return ftq_v1_slot_bytes_flags(d, key_bits, value_bits, 0);
}

namespace ftq {
int v1_store_checks(int d, int key_bits, int value_bits, int64_t n_tokens, int num_kv_heads, int64_t num_blocks,
                    int block_size, int dtype, int v_rotate, int64_t stride_block, int64_t stride_pos,
                    int64_t stride_head);
}

extern "C" int ftq_v1_store_rot(const void* key, const void* value, int dtype, int64_t n_tokens,
                            int num_kv_heads, int d, const float* midpoints, int key_bits,
                            int value_bits, int v_rotate, const int64_t* slot_mapping,
                            uint8_t* kv_cache, int64_t num_blocks, int block_size,
                            int64_t stride_block, int64_t stride_pos, int64_t stride_head,
                            const float* rotation, void* stream) {
  if (rotation == nullptr)
    return ftq_v1_store(key, value, dtype, n_tokens, num_kv_heads, d, midpoints, key_bits, value_bits, v_rotate,
                        slot_mapping, kv_cache, num_blocks, block_size, stride_block, stride_pos, stride_head, stream);
  const int rc = v1_store_checks(d, key_bits, value_bits, n_tokens, num_kv_heads, num_blocks, block_size, dtype,
                                 v_rotate, stride_block, stride_pos, stride_head);
  if (rc != FTQ_OK) return rc;
  FTQ_REQUIRE(key_bits <= 4 && value_bits <= 4 && (v_rotate & V1F_KFP8) == 0,
              "dense-matrix store: key_bits and value_bits in 1..4, no fp8 keys");
  FTQ_REQUIRE(aligned4(rotation), "rotation must be 4-byte aligned");
  if (n_tokens == 0) return FTQ_OK;
  FTQ_REQUIRE(key && value && midpoints && slot_mapping && kv_cache, "null pointer argument");
  FTQ_REQUIRE(aligned16(key) && aligned16(value), "key/value must be 16-byte aligned");
  FTQ_REQUIRE(aligned4(kv_cache), "kv_cache must be 4-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (d == 64)
    e = v1_launch_store_dense<64>(key, value, dtype, n_tokens, num_kv_heads, midpoints, key_bits, value_bits, v_rotate, slot_mapping, kv_cache, num_blocks, block_size, stride_block, stride_pos, stride_head, rotation, st);
  else if (d == 128)
    e = v1_launch_store_dense<128>(key, value, dtype, n_tokens, num_kv_heads, midpoints, key_bits, value_bits, v_rotate, slot_mapping, kv_cache, num_blocks, block_size, stride_block, stride_pos, stride_head, rotation, st);
  else
    e = v1_launch_store_dense<256>(key, value, dtype, n_tokens, num_kv_heads, midpoints, key_bits, value_bits, v_rotate, slot_mapping, kv_cache, num_blocks, block_size, stride_block, stride_pos, stride_head, rotation, st);
  return hip_status(e);
}

extern "C" int64_t ftq_v1_workspace_bytes(int batch, int num_q_heads, int d, int num_splits) {
  return split_workspace_bytes(batch, num_q_heads, d, num_splits);
}

extern "C" int ftq_v1_default_splits(int batch, int num_kv_heads, int max_seq_len) {
  // 384 or more (batch, kv head) workgroups already give each CU 1.5 of them:
  // one split writes the output directly and saves the merge launch (64
  // sequences x 8 kv heads over ~2200 positions, K3 V3: 39.8 us at one split
  // against 49.5 us at two)
  if ((int64_t)batch * num_kv_heads >= 384) return 1;
  return auto_splits(batch, num_kv_heads, max_seq_len, 1024);
}

namespace {
// Workgroups of the matrix-core decode kernel that runs this shape that the
// GPU holds at once (the occupancy of the bf16-query instantiation; the query
// type does not change the register count).
template <int KB, int VB>
int v1_attn_resident(int group, bool lloyd) {
  if constexpr (VB == 4) {
    if (lloyd) {
      static const int c = resident_workgroups(v1_attn_kernel<128, KB, VB, BF16, true>);
      return c;
    }
  }
  if (group == 4) {
    static const int c = resident_workgroups(v1_attn_g4_kernel<128, KB, VB, BF16>);
    return c;
  }
  static const int c = resident_workgroups(v1_attn_kernel<128, KB, VB, BF16>);
  return c;
}
template <int KB>
int v1_attn_resident_k(int value_bits, int group, bool lloyd) {
  if (value_bits == 2) return v1_attn_resident<KB, 2>(group, lloyd);
  if (value_bits == 3) return v1_attn_resident<KB, 3>(group, lloyd);
  return v1_attn_resident<KB, 4>(group, lloyd);
}
}  // namespace

extern "C" int ftq_v1_choose_splits(int batch, int num_q_heads, int num_kv_heads, int d, int key_bits,
                                    int value_bits, int v_flags, int max_seq_len) {
  if (batch <= 0 || num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0) return 1;
  const bool mfma = d == 128 && (v_flags & (V1F_KFP8 | V1F_FP32)) == 0 && key_bits >= 2 && key_bits <= 4 &&
                    value_bits >= 2 && value_bits <= 4;
  if (!mfma) return ftq_v1_default_splits(batch, num_kv_heads, max_seq_len);
  // The most splits whose grid the GPU holds in one round: past that a second
  // round of workgroups (or an uneven first one) costs more than the longer
  // tiles per wave.  Measured on 32 query / 8 kv heads, K3 V3 (3 workgroups
  // per CU) and K4 V2 (4): 384 units, 2K-32K positions, 2 splits 11-22%
  // faster than 1; 448 and 512 units at K3 V3, 1 split best (two splits
  // would need a second round); K4 V2 at 448 and 512, 2 splits 1-11%
  // faster; 4 x 8 units at 64K-128K, K4 V2, 32 splits.  No more splits than
  // leave 8 tiles per wave, and at most 64.
  const int group = num_q_heads / num_kv_heads;
  const bool lloyd = value_bits == 4 && (v_flags & V1F_VLM) != 0;
  int cap;
  if (key_bits == 2) cap = v1_attn_resident_k<2>(value_bits, group, lloyd);
  else if (key_bits == 3) cap = v1_attn_resident_k<3>(value_bits, group, lloyd);
  else cap = v1_attn_resident_k<4>(value_bits, group, lloyd);
  const int64_t units = std::min<int64_t>((int64_t)batch * num_kv_heads, 1 << 20);
  int64_t s = cap / units;
  const int64_t by_len = max_seq_len / (32 * 4 * 8);
  if (s > by_len) s = by_len;
  if (s > 64) s = 64;
  return s < 1 ? 1 : (int)s;
}

namespace {
// Argument checks of the v1 decode attention entry points and the launch
// arguments they imply.  check_ws: the caller's workspace (the no-alloc form
// brings its own afterwards).  FTQ_OK with a.B == 0: nothing to launch.
int v1_attn_prepare(V1Args& a, const void* query, int q_dtype, const uint8_t* kv_cache, int64_t num_blocks,
                    int block_size, int64_t stride_block, int64_t stride_pos, int64_t stride_head,
                    const int32_t* block_table, int max_blocks_per_seq, const int32_t* seq_lens,
                    const int32_t* kv_start, int batch, int num_q_heads, int num_kv_heads, int d,
                    const float* centroids, int key_bits, int value_bits, float scale, int v_rotate,
                    int num_splits, void* workspace, int64_t workspace_bytes, bool check_ws, void* out,
                    int out_dtype, float* lse_out, const float* rotation) {
  FTQ_REQUIRE(d == 64 || d == 128 || d == 256, "v1 decode attention: head_dim must be 64, 128 or 256");
  FTQ_REQUIRE(v_rotate >= 0 && v_rotate <= 15,
              "v_flags: bit 0 = un-rotate V, bit 1 = Lloyd-Max V codes, bit 2 = fp8 keys, bit 3 = fp32 products");
  FTQ_REQUIRE(rotation == nullptr || aligned4(rotation), "rotation must be 4-byte aligned");
  FTQ_REQUIRE(v1_widths_ok(key_bits, value_bits, v_rotate),
              "v1 decode attention: key_bits and value_bits must both be in 1..4, or both 8 (fp8 keys: both 8)");
  FTQ_REQUIRE(block_size >= 16 && block_size <= 4096 && (block_size & (block_size - 1)) == 0,
              "block_size must be a power of two in [16, 4096]");
  FTQ_REQUIRE(batch >= 0 && num_kv_heads > 0 && num_q_heads > 0 && num_blocks >= 0,
              "bad batch / head / block counts");
  FTQ_REQUIRE(num_q_heads % num_kv_heads == 0, "num_q_heads must be a multiple of num_kv_heads");
  FTQ_REQUIRE(num_q_heads / num_kv_heads <= 16, "GQA group (num_q_heads / num_kv_heads) must be <= 16");
  FTQ_REQUIRE(num_splits >= 1 && num_splits <= 1024, "num_splits must be in [1, 1024]");
  FTQ_REQUIRE(max_blocks_per_seq >= 0, "max_blocks_per_seq must be >= 0");
  FTQ_REQUIRE(q_dtype >= F32 && q_dtype <= BF16 && out_dtype >= F32 && out_dtype <= BF16,
              "dtype must be FTQ_F32, FTQ_F16 or FTQ_BF16");
  const bool kf8 = (v_rotate & V1F_KFP8) != 0;
  const V1Geom g = v1_geom(d, key_bits, value_bits, kf8);
  FTQ_REQUIRE(stride_head >= g.raw, "stride_head is smaller than the slot bytes (see ftq_v1_slot_bytes)");
  FTQ_REQUIRE(cache_strides_ok(num_blocks, stride_block, stride_pos, stride_head, num_kv_heads, block_size),
              "kv_cache strides must describe [num_blocks][block_size][num_kv_heads][slot]");
  FTQ_REQUIRE(stride_head % 4 == 0 && stride_pos % 4 == 0 && stride_block % 4 == 0,
              "kv_cache strides must be multiples of 4 bytes");
  FTQ_REQUIRE(stride_pos * 16 < ((int64_t)1 << 31), "stride_pos too large");
  a.B = batch;
  if (batch == 0) return FTQ_OK;
  FTQ_REQUIRE(num_blocks >= 1, "kv_cache must hold at least one block");
  FTQ_REQUIRE(query && kv_cache && block_table && seq_lens && out, "null pointer argument");
  FTQ_REQUIRE(centroids != nullptr || kf8, "null centroids");
  if (check_ws) {
    FTQ_REQUIRE(workspace != nullptr, "null pointer argument");
    FTQ_REQUIRE(workspace_bytes >= ftq_v1_workspace_bytes(batch, num_q_heads, d, num_splits),
                "workspace too small (see ftq_v1_workspace_bytes)");
    FTQ_REQUIRE(aligned16(workspace), "workspace must be 16-byte aligned");
  }
  FTQ_REQUIRE(aligned16(query) && aligned16(out) && aligned4(kv_cache),
              "query and out must be 16-byte aligned, kv_cache 4-byte aligned");
  a.q = query; a.qt = q_dtype; a.cache = kv_cache; a.bt = block_table; a.sl = seq_lens; a.ks = kv_start;
  a.B = batch; a.hq = num_q_heads; a.hkv = num_kv_heads; a.max_blocks = max_blocks_per_seq;
  a.lbs = 0;
  while ((1 << a.lbs) < block_size) ++a.lbs;
  a.nb = num_blocks; a.sblk = stride_block; a.spos = stride_pos; a.shead = stride_head;
  a.cent = centroids;
  a.qscale = (rotation != nullptr ? 1.f : fwht_scale(d)) * scale * 1.4426950408889634f;
  a.rot = rotation;
  a.splits = num_splits; a.vrot = v_rotate;
  a.out = out; a.ot = out_dtype; a.lse = lse_out;
  return FTQ_OK;
}

// The launches for prepared arguments (a.wo / a.wl set).
int v1_attn_launch(const V1Args& a, int d, int key_bits, int value_bits, int v_rotate, void* stream) {
  hipStream_t st = (hipStream_t)stream;
  const bool kf8 = (v_rotate & V1F_KFP8) != 0;
  hipError_t e;
  // the matrix-core kernels: head_dim 128, 2-4 bit codes, f16 operands; every
  // other format, and fp32 products on request, on the VALU kernel
  const bool mfma = d == 128 && !kf8 && (v_rotate & V1F_FP32) == 0 && key_bits >= 2 && key_bits <= 4 &&
                    value_bits >= 2 && value_bits <= 4;
  if (!mfma) e = v1_valu_launch(a, d, key_bits, value_bits, v_rotate, st);
  else if (key_bits == 2) e = v1_launch_attn2<128, 2>(value_bits, a, st);
  else if (key_bits == 3) e = v1_launch_attn2<128, 3>(value_bits, a, st);
  else e = v1_launch_attn2<128, 4>(value_bits, a, st);
  return hip_status(e);
}
}  // namespace

extern "C" int ftq_v1_decode_attention_rot(
    const void* query, int q_dtype, const uint8_t* kv_cache, int64_t num_blocks, int block_size,
    int64_t stride_block, int64_t stride_pos, int64_t stride_head, const int32_t* block_table,
    int max_blocks_per_seq, const int32_t* seq_lens, const int32_t* kv_start, int batch,
    int num_q_heads, int num_kv_heads, int d, const float* centroids, int key_bits,
    int value_bits, float scale, int v_rotate, int num_splits, void* workspace,
    int64_t workspace_bytes, void* out, int out_dtype, float* lse_out, const float* rotation,
    void* stream) {
  V1Args a;
  const int rc = v1_attn_prepare(a, query, q_dtype, kv_cache, num_blocks, block_size, stride_block, stride_pos,
                                 stride_head, block_table, max_blocks_per_seq, seq_lens, kv_start, batch,
                                 num_q_heads, num_kv_heads, d, centroids, key_bits, value_bits, scale, v_rotate,
                                 num_splits, workspace, workspace_bytes, true, out, out_dtype, lse_out, rotation);
  if (rc != FTQ_OK || batch == 0) return rc;
  a.wo = static_cast<float*>(workspace);
  a.wl = a.wo + (int64_t)batch * num_q_heads * num_splits * d;
  return v1_attn_launch(a, d, key_bits, value_bits, v_rotate, stream);
}

extern "C" int ftq_v1_decode_attention_lse(
    const void* query, int q_dtype, const uint8_t* kv_cache, int64_t num_blocks, int block_size,
    int64_t stride_block, int64_t stride_pos, int64_t stride_head, const int32_t* block_table,
    int max_blocks_per_seq, const int32_t* seq_lens, const int32_t* kv_start, int batch,
    int num_q_heads, int num_kv_heads, int d, const float* centroids, int key_bits,
    int value_bits, float scale, int v_rotate, int num_splits, void* workspace,
    int64_t workspace_bytes, void* out, int out_dtype, float* lse_out, void* stream) {
  return ftq_v1_decode_attention_rot(query, q_dtype, kv_cache, num_blocks, block_size, stride_block, stride_pos, stride_head, block_table, max_blocks_per_seq, seq_lens, kv_start, batch, num_q_heads, num_kv_heads, d, centroids, key_bits, value_bits, scale, v_rotate, num_splits, workspace, workspace_bytes, out, out_dtype, lse_out, nullptr, stream);
}

extern "C" int ftq_v1_decode_attention(
    const void* query, int q_dtype, const uint8_t* kv_cache, int64_t num_blocks, int block_size,
    int64_t stride_block, int64_t stride_pos, int64_t stride_head, const int32_t* block_table,
    int max_blocks_per_seq, const int32_t* seq_lens, const int32_t* kv_start, int batch,
    int num_q_heads, int num_kv_heads, int d, const float* centroids, int key_bits,
    int value_bits, float scale, int v_rotate, int num_splits, void* workspace,
    int64_t workspace_bytes, void* out, int out_dtype, void* stream) {
  return ftq_v1_decode_attention_lse(query, q_dtype, kv_cache, num_blocks, block_size, stride_block, stride_pos,
                                     stride_head, block_table, max_blocks_per_seq, seq_lens, kv_start, batch,
                                     num_q_heads, num_kv_heads, d, centroids, key_bits, value_bits, scale,
                                     v_rotate, num_splits, workspace, workspace_bytes, out, out_dtype, nullptr,
                                     stream);
}

// ---------------------------------------------------------------------------
// Allocation-free decode attention.  The split-K partials (per (row, split):
// D floats of output and one log2-sum-exp) go to `scratch`, a file-scope
// device array, instead of a caller's workspace.  Every stage-1 workgroup
// writes all of its partials (zeros and -inf for an empty split) before the
// merge reads them, so nothing in the array has to start at zero and the
// contents a previous call left behind are never read.
// All calls on one GPU share that GPU's copy of the array: calls that overlap
// on one GPU (two host threads, or two streams without an ordering between
// them) race on it.
// ---------------------------------------------------------------------------
namespace {
constexpr int64_t kV1ScratchBytes = (int64_t)16 << 20;  // 16 MiB per device
constexpr int kMaxDevices = 64;
static __device__ __align__(256) float scratch[kV1ScratchBytes / 4];

std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};  // device address of `scratch`, per device

// Device address of this device's `scratch`, looked up once per device (the
// array's host-side name is not a device address).
int current_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return ftq::hip_status(e);
  FTQ_REQUIRE(dev >= 0 && dev < kMaxDevices, "device ordinal beyond the scratch table (64 devices)");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return ftq::hip_status(e);
    FTQ_REQUIRE(p != nullptr, "hipGetSymbolAddress returned no address for the scratch array");
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return FTQ_OK;
}
}  // namespace

extern "C" int64_t ftq_v1_scratch_bytes(void) { return kV1ScratchBytes; }

extern "C" int ftq_v1_decode_attention_noalloc(
    const void* query, int q_dtype, const uint8_t* kv_cache, int64_t num_blocks, int block_size,
    int64_t stride_block, int64_t stride_pos, int64_t stride_head, const int32_t* block_table,
    int max_blocks_per_seq, const int32_t* seq_lens, const int32_t* kv_start, int batch,
    int num_q_heads, int num_kv_heads, int d, const float* centroids, int key_bits,
    int value_bits, float scale, int v_rotate, int num_splits, void* out, int out_dtype,
    void* stream) {
  V1Args a;
  int rc = v1_attn_prepare(a, query, q_dtype, kv_cache, num_blocks, block_size, stride_block, stride_pos,
                           stride_head, block_table, max_blocks_per_seq, seq_lens, kv_start, batch, num_q_heads,
                           num_kv_heads, d, centroids, key_bits, value_bits, scale, v_rotate, num_splits, nullptr,
                           0, false, out, out_dtype, nullptr, nullptr);
  if (rc != FTQ_OK) return rc;
  const int64_t need = ftq_v1_workspace_bytes(batch, num_q_heads, d, num_splits);
  FTQ_REQUIRE(need >= 0, "bad batch / head / split counts");
  FTQ_REQUIRE(need <= kV1ScratchBytes,
              "batch * num_q_heads * num_splits * (head_dim + 1) * 4 exceeds the 16 MiB scratch of "
              "ftq_v1_decode_attention_noalloc: lower num_splits or the batch");
  if (batch == 0) return FTQ_OK;
  if (stream != nullptr) {  // the scratch address is per device: the stream must be the current device's
    int cur = -1, sdev = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess) e = hipStreamGetDevice((hipStream_t)stream, &sdev);
    if (e != hipSuccess) return hip_status(e);
    FTQ_REQUIRE(cur == sdev, "stream belongs to another device than the current one");
  }
  void* ws = nullptr;
  rc = current_scratch(&ws);
  if (rc != FTQ_OK) return rc;
  a.wo = static_cast<float*>(ws);
  a.wl = a.wo + (int64_t)batch * num_q_heads * num_splits * d;
  return v1_attn_launch(a, d, key_bits, value_bits, v_rotate, stream);
}
