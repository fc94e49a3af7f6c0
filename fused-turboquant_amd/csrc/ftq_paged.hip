// Paged library-format KV cache on gfx950: fused store (encode + scatter) and
// split-K decode attention computed directly over the packed codes.
//
// Semantics: decode attention of the library format, i.e.
//   q_rot = RHT_K(q);  s_t = ||k_t||_16 * <q_rot, C_K[idx_t]> * scale
//   o = RHT_V^-1( sum_t softmax(s)_t * ||v_t||_16 * C_V[vidx_t] )
// == softmax(q . K^T * scale) . V with K, V the decoded cache
// (reference vllm_plugin/attention_impl.py:431-521 for the paged semantics,
// kernels/triton_flash_decode.py:66-221 for the fused rotated-domain form).
//
// HBM layout (this library's page format; the reference's paged format for
// this codec is the Python v0 slot [2, nb, bs, Hkv, packed + fp32 norm],
// vllm_plugin/cache_ops.py:64-108):
//   kv_cache[num_blocks][Hkv][page_size/16][SUB] bytes, where one 16-token
//   sub-block of one kv head holds
//     K codes  [16 tokens][D*BK/8]   per-token packed, reference bit layout
//     V codes  [64 lanes][D*BV/32]   "lane-major": chunk (q, r) holds, for each
//              d-block b = 0..D/16-1, the codes of tokens 4q..4q+3 at
//              d = 16b + r, token i at bit (4b + i) * BV
//     K norms  [16] fp16, V norms [16] fp16
//   The V order is the operand order of the P.V MFMA below, so a lane's V
//   operand for a whole sub-block is one contiguous D*BV/32-byte load.
//
// Decode attention kernel: one workgroup (4 waves) per (batch, kv head,
// split); each wave walks 32-token tiles (two sub-blocks) of its split.
//   S^T[t][h] = K[t][:] . Q^T[:][h]  : v_mfma_f32_16x16x32_f16, A = K codes
//               turned into f16 pairs by a pair lookup table, B = rotated
//               query of the GQA group (columns h >= G are zero)
//   O^T[d][h] += V^T[d][t] . P'^T[t][h] : same MFMA, A = V codes (lane-major
//               layout), B = softmax weights * ||v_t|| kept in registers from
//               the S^T output (no shuffle: the k-slot order of the P.V MFMA
//               is chosen to be the row order of the S^T output).
// Online softmax in the log2 domain (scale * log2 e folded into q).  Waves
// merge through LDS; splits merge in a second kernel that also applies the
// inverse RHT of V and writes the output dtype.
#include "ftq_attn_dev.h"
#include "ftq_merge.h"
#include "ftq_codec_dev.h"
#include "ftq_encode_mfma.h"
#include "ftq_internal.h"

#include <algorithm>
#include <cmath>

namespace ftq {

template <int D, int BK, int BV> struct PagedGeom {
  static constexpr int KTOK = D * BK / 8;   // K code bytes per token
  static constexpr int KSEC = 16 * KTOK;    // K codes of one sub-block
  static constexpr int KLANE = KTOK / 4;    // K bytes one lane reads per sub-block
  static constexpr int VLANE = D * BV / 32; // V bytes of one lane chunk
  static constexpr int VSEC = 64 * VLANE;
  static constexpr int KNORM = KSEC + VSEC;
  static constexpr int VNORM = KNORM + 32;
  static constexpr int SUB = VNORM + 32;    // bytes per (sub-block, kv head)
  static constexpr int NS = D / 32;         // Q.K MFMAs per sub-block
  static constexpr int NB = D / 16;         // P.V MFMAs per tile (d-blocks)
  static_assert(KLANE % 4 == 0 && VLANE % 4 == 0, "lane chunks must be dword multiples");
};

int64_t paged_sub_bytes(int d, int bk, int bv) {
  return (int64_t)2 * d * (bk + bv) + 64;
}

// ---------------------------------------------------------------------------
// store: encode K and V of n tokens x Hkv heads and scatter into the pages.
// One wave per (group of 16 consecutive input tokens, kv head).  K codes, K
// and V norms are per token and written directly.  V codes go to the
// lane-major chunks, where 4 tokens share each chunk's words:
//   * a group whose 16 tokens fill one whole 16-token sub-block in order (a
//     prefill: slot_mapping[16 g + j] = S + j, S a multiple of 16) writes
//     every chunk whole, with plain stores;
//   * any other group (decode steps, ragged tails, scattered slots) merges
//     each token's bits into the chunk words with atomic and / or, which is
//     correct for any slot mapping.
// paged_store_mfma_kernel (16-bit input) encodes whole groups on the matrix
// cores and the others token by token (paged_store_tokens); paged_store_kernel
// (fp32 input) does every group token by token.
// ---------------------------------------------------------------------------

// The tokens of group t0 .. t0 + 15 (one kv head), 4 at a time, 16 lanes each
// (row `sub` of the wave takes token t0 + 4 p + sub): K codes, both norms and,
// for a group that is not a whole sub-block, V's bits merged into the shared
// chunk words with atomic and / or.  Each token's V codes are also staged in
// vcode[token][d] (this wave's LDS), from which a whole group's chunks are
// written by the caller.
template <int D, int BK, int BV, int DT>
__device__ __forceinline__ void paged_store_tokens(
    const void* __restrict__ key, const void* __restrict__ value, int64_t n_tokens, int hkv,
    const float* __restrict__ ksigns, const float* __restrict__ vsigns, const float* __restrict__ kbnd_g,
    const float* __restrict__ vbnd_g, const int64_t* __restrict__ slot_mapping, uint8_t* __restrict__ cache,
    int page_size, int64_t num_blocks, float scale, int64_t t0, int head, bool whole, uint8_t (*vcode)[D]) {
  using Gm = PagedGeom<D, BK, BV>;
  constexpr int E = D / 16, LPV = 16;
  constexpr int NDW = Gm::VLANE / 4;  // dwords of one lane chunk
  const int lane = threadIdx.x & 63;
  const int l16 = lane & 15, sub = lane >> 4;
  const int nsub = page_size / 16;
  float kb[(1 << BK) - 1], vb[(1 << BV) - 1];
#pragma unroll
  for (int j = 0; j < (1 << BK) - 1; ++j) kb[j] = kbnd_g[j + 1];
#pragma unroll
  for (int j = 0; j < (1 << BV) - 1; ++j) vb[j] = vbnd_g[j + 1];
  float ks[E], vs[E];
#pragma unroll
  for (int i = 0; i < E; ++i) {
    ks[i] = ksigns[l16 * E + i];
    vs[i] = vsigns[l16 * E + i];
  }
#pragma unroll 1
  for (int p = 0; p < 4; ++p) {
    const int tt = 4 * p + sub;  // token of the group this 16-lane vector encodes
    const int64_t tok = t0 + tt;
    const int64_t slot = tok < n_tokens ? slot_mapping[tok] : -1;
    const bool active = slot >= 0 && slot / page_size < num_blocks;
    if (active) {  // uniform over the vector's 16 lanes
      const int64_t blk = slot / page_size;
      const int off = (int)(slot - blk * page_size);
      const int ts = off & 15;
      uint8_t* sbp = cache + (((blk * hkv + head) * nsub) + (off >> 4)) * (int64_t)Gm::SUB;
      const int64_t eoff = (tok * hkv + head) * D + l16 * E;
      float y[E];
      uint32_t c[E];
      load_elems<DT, E>(key, eoff, y);
      const float kn = encode_core<E, LPV, BK>(y, ks, kb, scale, l16, c);
      pack_store<E, BK>(c, sbp + ts * Gm::KTOK, l16);
      load_elems<DT, E>(value, eoff, y);
      const float vn = encode_core<E, LPV, BV>(y, vs, vb, scale, l16, c);
      if (l16 == 0) {
        reinterpret_cast<uint16_t*>(sbp + Gm::KNORM)[ts] = (uint16_t)f32_to_f16_bits(kn);
        reinterpret_cast<uint16_t*>(sbp + Gm::VNORM)[ts] = (uint16_t)f32_to_f16_bits(vn);
      }
#pragma unroll
      for (int i = 0; i < E; ++i) vcode[tt][l16 * E + i] = (uint8_t)c[i];
      __asm__ volatile("" ::: "memory");  // a wave's LDS accesses run in order
      if (!whole) {
        // lane r owns chunk (ts / 4, r): this token's code for d = 16 b + r sits
        // at bit (4 b + ts % 4) BV; other tokens share the chunk's words, so
        // clear and set only this token's bits
        uint32_t v0[NDW], m0[NDW];  // this token's bits as if it were token 0 of its quad
#pragma unroll
        for (int w = 0; w < NDW; ++w) { v0[w] = 0; m0[w] = 0; }
#pragma unroll
        for (int b = 0; b < D / 16; ++b) {
          const uint32_t code = vcode[tt][16 * b + l16];
          const int P = 4 * b * BV;  // compile-time after unrolling; fields never straddle here
          v0[P >> 5] |= code << (P & 31);
          m0[P >> 5] |= ((1u << BV) - 1u) << (P & 31);
        }
        const int sh = (ts & 3) * BV;
        uint32_t* chunk = reinterpret_cast<uint32_t*>(sbp + Gm::KSEC + ((ts >> 2) * 16 + l16) * Gm::VLANE);
#pragma unroll
        for (int w = 0; w < NDW; ++w) {
          const uint64_t vv = ((uint64_t)v0[w] << 32) | (w ? v0[w - 1] : 0u);
          const uint64_t mm = ((uint64_t)m0[w] << 32) | (w ? m0[w - 1] : 0u);
          const uint32_t val = (uint32_t)((vv << sh) >> 32), msk = (uint32_t)((mm << sh) >> 32);
          if (msk) {
            atomicAnd(chunk + w, ~msk);
            atomicOr(chunk + w, val);
          }
        }
      }
    }
  }
}

// The VALU store: every group, for the input the matrix-core kernel below
// does not take (fp32).
template <int D, int BK, int BV, int DT>
__global__ __launch_bounds__(256) void paged_store_kernel(
    const void* __restrict__ key, const void* __restrict__ value, int64_t n_tokens, int hkv,
    const float* __restrict__ ksigns, const float* __restrict__ vsigns,
    const float* __restrict__ kbnd_g, const float* __restrict__ vbnd_g,
    const int64_t* __restrict__ slot_mapping, uint8_t* __restrict__ cache, int page_size,
    int64_t num_blocks, float scale) {
  using Gm = PagedGeom<D, BK, BV>;
  constexpr int NDW = Gm::VLANE / 4;  // dwords of one lane chunk
  __shared__ uint8_t vcode[4][16][D];  // per wave: the V codes of its group's 16 tokens
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int l16 = lane & 15, sub = lane >> 4;
  const int nsub = page_size / 16;
  const int64_t n_groups = (n_tokens + 15) / 16;
  const int64_t items = n_groups * hkv;

  for (int64_t item = (int64_t)blockIdx.x * 4 + wave; item < items; item += (int64_t)gridDim.x * 4) {
    const int64_t grp = item / hkv;
    const int head = (int)(item - grp * hkv);
    const int64_t t0 = grp * 16;
    // whole-sub-block group?  (lanes l, l + 16, l + 32, l + 48 check token t0 + l)
    const int64_t sl = (t0 + l16 < n_tokens) ? slot_mapping[t0 + l16] : -1;
    const int64_t s0 = ((int64_t)__builtin_amdgcn_readfirstlane((int)(sl >> 32)) << 32) |
                       (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)sl);
    const bool lane_ok = s0 >= 0 && (s0 & 15) == 0 && sl == s0 + l16 && s0 / page_size < num_blocks;
    const bool whole = __builtin_amdgcn_ballot_w64(lane_ok) == ~0ull;
    paged_store_tokens<D, BK, BV, DT>(key, value, n_tokens, hkv, ksigns, vsigns, kbnd_g, vbnd_g, slot_mapping,
                                      cache, page_size, num_blocks, scale, t0, head, whole, vcode[wave]);
    if (whole) {  // wave-uniform: every chunk of the sub-block, written whole
      __asm__ volatile("" ::: "memory");
      const int64_t blk = s0 / page_size;
      const int off = (int)(s0 - blk * page_size);
      uint8_t* sbp = cache + (((blk * hkv + head) * nsub) + (off >> 4)) * (int64_t)Gm::SUB;
      // lane (q, r) = (lane >> 4, lane & 15): tokens 4q..4q+3 at d = 16 b + r
      uint32_t w[NDW];
#pragma unroll
      for (int k = 0; k < NDW; ++k) w[k] = 0;
#pragma unroll
      for (int b = 0; b < D / 16; ++b)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int P = (4 * b + i) * BV;  // compile-time; a field never straddles a word (BV | 32 or 3 * 4 fits)
          const uint32_t code = vcode[wave][4 * sub + i][16 * b + l16];
          if ((P & 31) + BV <= 32) {
            w[P >> 5] |= code << (P & 31);
          } else {
            w[P >> 5] |= code << (P & 31);
            w[(P >> 5) + 1] |= code >> (32 - (P & 31));
          }
        }
      uint32_t* chunk = reinterpret_cast<uint32_t*>(sbp + Gm::KSEC + lane * Gm::VLANE);
#pragma unroll
      for (int k = 0; k < NDW; ++k) chunk[k] = w[k];
    }
    __asm__ volatile("" ::: "memory");
  }
}

// ---------------------------------------------------------------------------
// store on the matrix cores (d = 128 and 256, 16-bit input).  A group whose slots are
// one whole 16-token sub-block in order (a prefill chunk) is encoded here;
// every other group goes token by token through paged_store_tokens, with this
// wave's LDS tile as its staging area.  The 16 vectors of K (then V) go through the encoder's
// 128-point Hadamard transform and norm on the matrix cores (Rht128,
// ftq_encode_mfma.h), lane (q, j) ending up with outputs 32 q .. 32 q + 31 of
// token j, so K's codes (per token, reference bit layout) and both norms are
// written straight from there.  V's codes go to the lane-major chunks: chunk
// (q', r) holds tokens 4 q' .. 4 q' + 3 at d = 16 b + r, which sit in 16
// different lanes.  The rotated V values therefore go through LDS (fp32, one
// 8 KB [dim][token] tile per wave) and each lane quantises its own chunk's 32
// values, element 4 b + i against token 4 q' + i's thresholds, and writes the
// chunk whole.  The quantiser is the general one (any codebook), as the
// encoder's general instantiation.
// LDS tile, dword address of (dim, token): row dim ^ (dim >> 5 & 1) (the two
// 32-dim quarters of one write phase land in opposite bank halves), token
// xor 4 ((row >> 1) & 3) (the 8 rows of one 128-byte read phase land in
// distinct 4-bank groups): conflict-free for both the per-token writes and
// the 4-token reads.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int pstore_row(int dim) { return dim ^ ((dim >> 5) & 1); }
__device__ __forceinline__ int pstore_addr(int dim, int token) {
  const int row = pstore_row(dim);
  return row * 16 + (token ^ (((row >> 1) & 3) << 2));
}

template <int D, int BK, int BV, int DT>
__global__ __launch_bounds__(256) void paged_store_mfma_kernel(
    const void* __restrict__ key, const void* __restrict__ value, int64_t n_tokens, int hkv,
    const float* __restrict__ ksigns, const float* __restrict__ vsigns,
    const float* __restrict__ kbnd_g, const float* __restrict__ vbnd_g,
    const int64_t* __restrict__ slot_mapping, uint8_t* __restrict__ cache, int page_size,
    int64_t num_blocks, float c, double rc) {
  static_assert(D == 128 || D == 256, "the matrix-core store covers d = 128 and 256");
  constexpr int KS = D / 32;   // K steps of the transform, 4 per 128-element block
  constexpr int NB = D / 128;  // 128-element blocks (the encoder's factored d = 256)
  using Gm = PagedGeom<D, BK, BV>;
  constexpr int NTK = (1 << BK) - 1, NTV = (1 << BV) - 1;
  const int lane = threadIdx.x & 63, q = lane >> 4, j = lane & 15;
  const int wv = threadIdx.x >> 6;
  Rht128<DT> H;
  H.init(lane);
  __shared__ uint4 ksm[4 * KS], vsm[4 * KS];
  __shared__ __align__(16) float tile[4][128 * 16];  // per wave: 128 of V's rotated dims
  __shared__ __align__(16) float vsc[4][16];       // per wave: V's threshold scale per token
  fill_sign_table<KS>(ksm, ksigns, (int)threadIdx.x);
  fill_sign_table<KS>(vsm, vsigns, (int)threadIdx.x - 64);  // threads 64 .. 64 + 4 KS - 1
  __syncthreads();
  float kb[NTK], vb[NTV];  // interior boundaries (wave-uniform)
#pragma unroll
  for (int k = 0; k < NTK; ++k) kb[k] = kbnd_g[1 + k];
#pragma unroll
  for (int k = 0; k < NTV; ++k) vb[k] = vbnd_g[1 + k];
  const float rcf = (float)rc;
  const int nsub = page_size / 16;
  const int64_t items = (n_tokens + 15) / 16 * hkv;
  float* tw = tile[wv];

  // 16 vectors of one tensor: lane (q, j) gets outputs 128 b + 32 q .. 128 b +
  // 32 q + 31 of token t0 + j in t[32 b ..] (at d = 256 the two 128-point
  // transforms and their butterfly, as the encoder) and the norm in nrm;
  // returns the threshold scale
  auto rotate = [&](const void* x, int64_t t0, int head, const uint4* signs, float (&t)[32 * NB],
                    float& nrm) {
    const uint16_t* src = static_cast<const uint16_t*>(x) + ((t0 + j) * hkv + head) * D + 32 * q;
    Op16x8 cur[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) cur[s].v = reinterpret_cast<const uint4*>(src)[16 * (s >> 2) + (s & 3)];
    int z = 0;
    asm volatile("" : "+s"(z));
    flip_signs<KS>(cur, signs, q, z);
    f32x4_t acc[8 * NB];
    H.template transform<NB>(cur, acc);
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
    nrm = sqrt_rn(H.sumsq(cur) * (float)D) * c;
    return (nrm + 1e-8f) * rcf;
  };

  for (int64_t item = (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(wv); item < items;
       item += (int64_t)gridDim.x * 4) {
    const int64_t grp = item / hkv;
    const int head = (int)(item - grp * hkv);
    const int64_t t0 = grp * 16;
    const int64_t sl = t0 + j < n_tokens ? slot_mapping[t0 + j] : -1;
    const int64_t s0 = ((int64_t)__builtin_amdgcn_readfirstlane((int)(sl >> 32)) << 32) |
                       (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)sl);
    const bool lane_ok = s0 >= 0 && (s0 & 15) == 0 && sl == s0 + j && s0 / page_size < num_blocks;
    if (__builtin_amdgcn_ballot_w64(lane_ok) != ~0ull) {  // wave-uniform
      paged_store_tokens<D, BK, BV, DT>(key, value, n_tokens, hkv, ksigns, vsigns, kbnd_g, vbnd_g, slot_mapping,
                                        cache, page_size, num_blocks, c, t0, head, false,
                                        reinterpret_cast<uint8_t(*)[D]>(tw));
      __asm__ volatile("" ::: "memory");  // the tile is rewritten by the next group
      continue;
    }
    const int64_t blk = s0 / page_size;
    const int off = (int)(s0 - blk * page_size);
    uint8_t* sbp = cache + (((blk * hkv + head) * nsub) + (off >> 4)) * (int64_t)Gm::SUB;

    float t[32 * NB];
    float nrm;
    // The cache writes are non-temporal (streamed past the caches, which then
    // hold the K / V reads): 9% faster on 65 536 tokens x 8 heads, K3 V3.  (Full-line fp32
    // output streams, as the decoder's, measured 2x slower that way.)
    {  // K: codes per token, block b's BK words of token j at word BK (4 b + q) of its row
      const float sv = rotate(key, t0, head, ksm, t, nrm);
      float T[1][NTK];
#pragma unroll
      for (int k = 0; k < NTK; ++k) T[0][k] = kb[k] * sv;
      uint32_t w[BK * NB];
      quantize_pack<BK, 32 * NB>(t, T, w);
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        uint32_t* dst = reinterpret_cast<uint32_t*>(sbp + j * Gm::KTOK) + BK * (4 * b + q);
#pragma unroll
        for (int k = 0; k < BK; ++k) __builtin_nontemporal_store(w[BK * b + k], dst + k);
      }
      if (q == 0)
        __builtin_nontemporal_store((uint16_t)f32_to_f16_bits(nrm), reinterpret_cast<uint16_t*>(sbp + Gm::KNORM) + j);
    }
    {  // V: through the LDS tile into lane-major chunks, 128 dims at a time
      const float sv = rotate(value, t0, head, vsm, t, nrm);
      if (q == 0) {
        __builtin_nontemporal_store((uint16_t)f32_to_f16_bits(nrm), reinterpret_cast<uint16_t*>(sbp + Gm::VNORM) + j);
        vsc[wv][j] = sv;
      }
      __asm__ volatile("" ::: "memory");
      // this lane owns chunk (q, j): tokens 4 q + i at d = 16 b + j
      const float4 s4 = *reinterpret_cast<const float4*>(&vsc[wv][4 * q]);
      float T[4][NTV];
#pragma unroll
      for (int k = 0; k < NTV; ++k) {
        T[0][k] = vb[k] * s4.x;
        T[1][k] = vb[k] * s4.y;
        T[2][k] = vb[k] * s4.z;
        T[3][k] = vb[k] * s4.w;
      }
      uint32_t* chunk = reinterpret_cast<uint32_t*>(sbp + Gm::KSEC + lane * Gm::VLANE);
#pragma unroll
      for (int hb = 0; hb < NB; ++hb) {  // dims 128 hb ..: d-blocks 8 hb .. 8 hb + 7, chunk words BV hb ..
#pragma unroll
        for (int e = 0; e < 32; ++e) tw[pstore_addr(32 * q + e, j)] = t[32 * hb + e];
        __asm__ volatile("" ::: "memory");  // a wave's LDS accesses run in order
        float x[32];
#pragma unroll
        for (int b = 0; b < 8; ++b) {
          const float4 x4 = *reinterpret_cast<const float4*>(&tw[pstore_addr(16 * b + j, 4 * q)]);
          x[4 * b] = x4.x;
          x[4 * b + 1] = x4.y;
          x[4 * b + 2] = x4.z;
          x[4 * b + 3] = x4.w;
        }
        uint32_t w[BV];
        quantize_pack<BV, 32, 4>(x, T, w);
#pragma unroll
        for (int k = 0; k < BV; ++k) __builtin_nontemporal_store(w[k], chunk + BV * hb + k);
        __asm__ volatile("" ::: "memory");  // the tile is rewritten next
      }
    }
  }
}

// ---------------------------------------------------------------------------
// decode attention, stage 1 (per split)
// ---------------------------------------------------------------------------

// Code lookup tables in LDS: an entry holds the f16 levels of two codes
// (index = c0 | c1 << B, one ds_read_b32 dequantises two codes).  The LDS
// serves a wave in 32-lane phases over 32 four-byte banks, so a 64-entry
// table (3-bit codes) has two entries per bank and random indices collide.
// For 3 bits the table is therefore stored in 32 copies, one per bank: entry
// e of copy c sits at dword e * 32 + c, and lane l reads copy l % 32, so every
// lane of a phase hits its own bank.  (2-bit tables have 16 entries and are
// conflict-free as they are; 4-bit tables keep one 256-entry copy.)
// Looking codes up through a register table with ds_bpermute_b32 instead
// (one shift per pair, no address add) measured slower on gfx950: the
// permute's throughput is below a conflict-free ds_read_b32's.
template <int B>
struct CodeLut {
  static constexpr int IDX_BITS = 2 * B;
  static constexpr int ENTRIES = 1 << IDX_BITS;
  static constexpr int LOG_COPIES = (B == 3) ? 5 : 0;
  static constexpr int COPIES = 1 << LOG_COPIES;
  static constexpr int BYTES = ENTRIES * 4 * COPIES;
};

// fill a code table from the fp16 level values already staged in LDS:
// entry e -> f16(levels[e & (2^B - 1)]) | f16(levels[e >> B]) << 16, in every copy
template <int B>
__device__ void build_code_lut(uint8_t* lut, const uint16_t* single, int tid, int nthreads) {
  using C = CodeLut<B>;
  for (int k = tid; k < C::ENTRIES * C::COPIES; k += nthreads) {
    const int e = k >> C::LOG_COPIES;
    reinterpret_cast<uint32_t*>(lut)[k] =
        (uint32_t)single[e & ((1 << B) - 1)] | ((uint32_t)single[e >> B] << 16);
  }
}

typedef __attribute__((address_space(3))) const uint32_t lds_u32;

// LDS address of this lane's copy of a code table
template <int B>
__device__ __forceinline__ uint32_t lut_lane_base(int lane, uint32_t table_addr) {
  return table_addr + (((uint32_t)lane & (CodeLut<B>::COPIES - 1u)) << 2);
}

// Byte offset of the table entry whose index is bits [P, P + W) of the code
// words: (field << SH) + base, as v_bfe_u32 + v_lshl_add_u32 (LLVM would
// otherwise split it into shift, and, add).  A field across two words first
// goes through v_alignbit_b32.
template <int SH, int W, int N>
__device__ __forceinline__ uint32_t lut_entry_off(const uint32_t (&w)[N], int P, uint32_t base) {
  const int i = P >> 5, o = P & 31;  // compile-time after unrolling
  uint32_t src = w[i], f, r;
  int off = o;
  if (o + W > 32 && i + 1 < N) {
    src = __builtin_amdgcn_alignbit(w[i + 1], w[i], o);
    off = 0;
  }
  asm("v_bfe_u32 %0, %1, %2, %3" : "=v"(f) : "v"(src), "n"(off), "n"(W));
  asm("v_lshl_add_u32 %0, %1, %2, %3" : "=v"(r) : "v"(f), "n"(SH), "v"(base));
  return r;
}

// dequantise the 4 codes at bits [P, P + 4B) into two f16x2 dwords;
// base = LDS address of this lane's copy of the table
template <int B, int N>
__device__ __forceinline__ uint2 lut_quad(const uint32_t (&w)[N], int P, uint32_t base) {
  using C = CodeLut<B>;
  constexpr int SH = 2 + C::LOG_COPIES;
  const uint32_t lo = *(lds_u32*)(uintptr_t)lut_entry_off<SH, C::IDX_BITS>(w, P, base);
  const uint32_t hi = *(lds_u32*)(uintptr_t)lut_entry_off<SH, C::IDX_BITS>(w, P + 2 * B, base);
  return make_uint2(lo, hi);
}

// lut_quad over a table in static LDS (its address a link-time constant the
// compiler folds into the DS instructions' offset field)
template <int B, int N>
__device__ __forceinline__ uint2 lut_quad_s(const uint32_t (&w)[N], int P, uint32_t laneoff, const uint32_t* table) {
  using C = CodeLut<B>;
  constexpr int SH = 2 + C::LOG_COPIES;
  const uint32_t lo = lds_dword_at(table, lut_field<SH, C::IDX_BITS>(w, P, laneoff));
  const uint32_t hi = lds_dword_at(table, lut_field<SH, C::IDX_BITS>(w, P + 2 * B, laneoff));
  return make_uint2(lo, hi);
}


// Schedule of a run of NM MFMAs whose A operands come from RD table reads
// each: the reads of MFMA i+1 issue before MFMA i waits for its own (a
// two-deep LDS pipeline; left alone, the scheduler waits for every read).
template <int NM, int RD>
__device__ __forceinline__ void sched_lds_mfma() {
  __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);
#pragma unroll
  for (int i = 0; i < NM - 1; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x100, RD, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
}

// max without the NaN canonicalisation fmaxf carries (scores are finite or -inf)
__device__ __forceinline__ float vmax(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float vmax3(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
// max over lanes l, l^16, l^32, l^48
__device__ __forceinline__ float row_max4(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// f16x2 {p0 * vn.lo, p1 * vn.hi}, each product rounded once to f16
__device__ __forceinline__ uint32_t pv_pair(float p0, float p1, uint32_t vn) {
  uint32_t r;
  asm("v_fma_mixlo_f16 %0, %1, %2, 0 op_sel_hi:[0,1,0]\n\t"
      "v_fma_mixhi_f16 %0, %3, %2, 0 op_sel:[0,1,0] op_sel_hi:[0,1,0]"
      : "=&v"(r) : "v"(p0), "v"(vn), "v"(p1));
  return r;
}
template <int D, int BK, int BV>
struct TileRegs {
  using Gm = PagedGeom<D, BK, BV>;
  uint32_t k[2][Gm::KLANE / 4];
  uint32_t v[2][Gm::VLANE / 4];
  uint32_t kn[2][2];  // 4 fp16 K norms per sub-block (tokens 4q..4q+3)
  uint32_t vn[2][2];  // zero for a sub-block without tokens (see load_tile)
};

// Page of sub-block j (16 tokens) of a sequence as a multiply-high:
// (2j * m) >> 32 with m = ceil(2^31 / nsub) equals floor(j / nsub) whenever
// j * nsub < 2^31, and always when nsub is a power of two (m is then exact).
// Only sub-blocks of the block table (j < j_cap = max_blocks * nsub) are
// divided, and the launcher checks j_cap * nsub < 2^31 for other page sizes.
struct SubDiv {
  uint32_t m;
  int nsub, j_cap;
  __device__ __forceinline__ int page(int j) const { return (int)__umulhi((uint32_t)j << 1, m); }
};

// Block-table entries of a tile's two sub-blocks, as a vector load issued one
// tile ahead of the code loads that need them (lane l holds sub-block l & 1;
// -1 past the split, past seq_len or past the row).  A vector load retires in
// order, so the wait before the consumer's readlane covers only this load;
// the table is a buffer (its row), so no lane reads outside it.
__device__ __forceinline__ int fetch_bt(__amdgpu_buffer_rsrc_t bt_rs, int tile, bool active, int seq_subs,
                                        const SubDiv& sd, uint32_t lane) {
  const int j = 2 * tile + (int)(lane & 1u);
  const bool ok = active && j < seq_subs && j < sd.j_cap;
  const int page = sd.page(ok ? j : 0);
  const int v = (int)__builtin_amdgcn_raw_buffer_load_b32(bt_rs, (uint32_t)page * 4u, 0, 0);
  return ok ? v : -1;
}

// The same two entries as wave-uniform scalar loads (no vector registers, no
// lane reads); the branch keeps the loads inside the table row.
struct BtPair {
  int e[2];
};
__device__ __forceinline__ BtPair fetch_bt_s(const int32_t* __restrict__ bt_row, int tile, bool active,
                                             int seq_subs, const SubDiv& sd) {
  BtPair r;
#pragma unroll
  for (int sb = 0; sb < 2; ++sb) {
    const int j = 2 * tile + sb;
    r.e[sb] = (active && j < seq_subs && j < sd.j_cap) ? bt_row[sd.page(j)] : -1;
  }
  return r;
}

// dwords [I, NDW) at lane offset voff of a buffer, as 16/12/8/4-byte loads
template <int I = 0, int NDW>
__device__ __forceinline__ void buf_dwords(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t (&w)[NDW]) {
  typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
  constexpr int R = NDW - I;
  const uint32_t o = voff + 4u * I;
  if constexpr (R >= 4) {
    const uint4 x = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, o, 0, 0));
    w[I] = x.x; w[I + 1] = x.y; w[I + 2] = x.z; w[I + 3] = x.w;
    if constexpr (R > 4) buf_dwords<I + 4>(rs, voff, w);
  } else if constexpr (R == 3) {
    const u32x3 x = __builtin_bit_cast(u32x3, __builtin_amdgcn_raw_buffer_load_b96(rs, o, 0, 0));
    w[I] = x.x; w[I + 1] = x.y; w[I + 2] = x.z;
  } else if constexpr (R == 2) {
    const uint2 x = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, o, 0, 0));
    w[I] = x.x; w[I + 1] = x.y;
  } else if constexpr (R == 1) {
    w[I] = __builtin_amdgcn_raw_buffer_load_b32(rs, o, 0, 0);
  }
}

// Lane offsets of the tile loads inside one sub-block (fixed for the kernel)
struct TileOff {
  uint32_t k, v, n;  // K codes, V codes, K norms (V norms at n + 32)
};

// Loads of one 32-token tile: per sub-block one wave-uniform buffer descriptor
// (its base; the byte range ends with the sub-block, so no lane reads past it)
// plus the lane offsets.
template <int D, int BK, int BV>
__device__ __forceinline__ void load_tile(TileRegs<D, BK, BV>& r, const uint8_t* __restrict__ cache, BtPair bt,
                                          int tile, const SubDiv& sd, int64_t blk_stride, int64_t kvh_off,
                                          int nb32, const TileOff& lo) {
  using Gm = PagedGeom<D, BK, BV>;
#pragma unroll
  for (int sb = 0; sb < 2; ++sb) {
    // block id and base are wave-uniform (scalar).  An inactive or invalid
    // sub-block (past seq_len, or a bad block id) gets a descriptor of range
    // 0 at block 0: the loads still issue (the wait counts stay static) and
    // return zeros, so its V norms are 0 and it adds nothing to P.V; past
    // seq_len its scores are masked to -inf by the consumer.
    int phys = bt.e[sb];
    const bool valid = (uint32_t)phys < (uint32_t)nb32;  // -1 (no entry) and ids >= num_blocks fail
    const int j = 2 * tile + sb;
    const int sub = valid ? j - sd.page(j) * sd.nsub : 0;
    if (!valid) phys = 0;
    const uint8_t* base = cache + ((int64_t)phys * blk_stride + kvh_off + (int64_t)sub * Gm::SUB);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, valid ? Gm::SUB : 0, 0x00020000);
    buf_dwords(rs, lo.k, r.k[sb]);
    buf_dwords(rs, lo.v, r.v[sb]);
    buf_dwords(rs, lo.n, r.kn[sb]);
    buf_dwords(rs, lo.n + 32u, r.vn[sb]);
  }
}

// LDS bytes of one paged_attn_kernel workgroup of NW waves for a GQA group of
// G heads: one pool reused for the rotated queries (prologue), the code tables
// (tile loop) and the wave-merge buffer (epilogue)
template <int D, int BK, int BV, bool SHARE, int NW>
__host__ __device__ constexpr int paged_attn_lds(int G) {
  const int red = NW * G * (D + 1) * 4;
  const int qs = G * (D + 4) * 4;
  return red > qs ? red : qs;
}

// Output of a finished (batch, q head) row: o / L, inverse RHT of V
// (unnormalised FWHT, times the 1/sqrt(d) scale and the signs), the output
// dtype; lane l of the wave holds elements [E l, E l + E).  L == 0 (no token
// attended) writes zeros.
template <int D>
__device__ __forceinline__ void finish_row(float (&y)[D / 64], float L, const float* __restrict__ vsigns,
                                           float scale, int lane, void* __restrict__ out, int ot, int64_t row) {
  constexpr int E = D / 64;
  const float inv = (L > 0.f) ? 1.f / L : 0.f;
#pragma unroll
  for (int i = 0; i < E; ++i) y[i] *= inv;
  fwht_wave64<E>(y, lane);
#pragma unroll
  for (int i = 0; i < E; ++i) y[i] = y[i] * scale * vsigns[lane * E + i];
  if (ot == F32) store_small<F32, E>(out, row * D + lane * E, y);
  else if (ot == F16) store_small<F16, E>(out, row * D + lane * E, y);
  else store_small<BF16, E>(out, row * D + lane * E, y);
}

// One workgroup per (split, kv head, batch) with NW waves.
//   NW = 4: the split form.  Each workgroup writes its split's partial
//     output (divided by its own softmax sum) and log2-sum-exp to the
//     workspace; merge_splits_kernel combines the splits.  d = 128 runs 4
//     workgroups per CU (<= 128 VGPRs); d = 256 holds twice the accumulators
//     and tile registers and runs 2 per CU (<= 256 VGPRs, no spills).
//   NW = 16 (d = 128, G <= 4, one split): the whole sequence in one workgroup
//     of 4 waves per SIMD (<= 128 VGPRs).  The waves merge in LDS and the
//     workgroup writes the output itself (inverse RHT, output dtype): no
//     workspace and no second launch.
//   QL (more than 8 query heads per kv head, no spare MFMA columns): the
//     query's f16 remainder is a second B operand with an MFMA of its own
//     (16 more registers: 3 workgroups per CU at d = 128).
template <int D, int BK, int BV, int QT, bool SHARE, int NW, bool QL = false>
__global__ __launch_bounds__(NW * 64, NW == 16 ? 1 : (D == 128 ? (QL ? 3 : 4) : 2)) void paged_attn_kernel(
    const void* __restrict__ query, const uint8_t* __restrict__ cache,
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ seq_lens, int hq, int hkv,
    int page_size, int max_blocks, int64_t num_blocks, const float* __restrict__ ksigns,
    const float* __restrict__ klev, const float* __restrict__ vlev, float qscale, int num_splits,
    float* __restrict__ ws_o, float* __restrict__ ws_lse, const float* __restrict__ vsigns, float vscale,
    void* __restrict__ out, int ot) {
  static_assert(NW == 4 || (NW == 16 && D == 128), "4 waves, or 16 waves at d = 128");
  static_assert(!QL || NW == 4, "the 16-wave form takes at most 4 query heads per kv head");
  using Gm = PagedGeom<D, BK, BV>;
  constexpr int NS = Gm::NS, NB = Gm::NB;
  constexpr int E = D / 16;
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int G = hq / hkv;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int h = lane & 15, q = lane >> 4;

  // LDS: the code tables in static arrays; a dynamic pool
  // (paged_attn_lds(G) bytes) reused for the rotated queries (prologue) and
  // the wave-merge buffer (epilogue)
  __shared__ __attribute__((aligned(16))) uint32_t lutK[CodeLut<BK>::BYTES / 4];
  __shared__ __attribute__((aligned(16))) uint32_t lutV_own[SHARE ? 1 : CodeLut<BV>::BYTES / 4];
  uint32_t* lutV = SHARE ? lutK : lutV_own;
  extern __shared__ __attribute__((aligned(16))) uint8_t pool[];
  __shared__ float red_m[NW][16], red_l[NW][16];
  __shared__ float tab_inv[2];       // 1 / (sigma (1 + rmid)), K / V
  float (*qs)[D + 4] = reinterpret_cast<float (*)[D + 4]>(pool);
  float* red_o = reinterpret_cast<float*>(pool);  // [NW waves][G heads][D + 1]

  // The code tables first, each sized and built by one wave (its level loads
  // and search overlap the other waves' first loads), and the query heads'
  // loads (one head per 16 lanes), ahead of the dependent block-table loads.
  const int wave_s = __builtin_amdgcn_readfirstlane(wave);
  if (wave_s == NW - 1) {
    const TableScale t = table_scale<1 << BK>(klev, false);
    build_pair_table_wave<BK, CodeLut<BK>::LOG_COPIES>(lutK, f32_to_f16_bits(t.sigma * klev[lane & ((1 << BK) - 1)]), lane);
    if (lane == 0) tab_inv[0] = 1.f / (t.sigma * (1.f + t.rmid));
  }
  if (!SHARE && wave_s == NW - 2) {
    const TableScale t = table_scale<1 << BV>(vlev, false);
    build_pair_table_wave<BV, CodeLut<BV>::LOG_COPIES>(lutV, f32_to_f16_bits(t.sigma * vlev[lane & ((1 << BV) - 1)]), lane);
    if (lane == 0) tab_inv[1] = 1.f / (t.sigma * (1.f + t.rmid));
  }
  const int qg = tid >> 4, ql16 = tid & 15;
  float y[E];
  if (qg < G) load_elems<QT, E>(query, ((int64_t)b * hq + kvh * G + qg) * D + ql16 * E, y);

  // tile range and the first tile's loads, issued before the rest of the
  // prologue so that their latency overlaps it
  const int seq_len = seq_lens[b];
  const int n_tiles = (seq_len + 31) >> 5;
  const int tps = (n_tiles + num_splits - 1) / num_splits;
  const int t_begin = split * tps;
  const int t_end = min(t_begin + tps, n_tiles);
  SubDiv sd;
  sd.nsub = page_size >> 4;
  sd.m = (0x80000000u + (uint32_t)sd.nsub - 1u) / (uint32_t)sd.nsub;
  sd.j_cap = (int)min((int64_t)max_blocks * sd.nsub, (int64_t)0x7fffffff);
  const int seq_subs = (int)(((int64_t)seq_len + 15) >> 4);
  const int nb32 = (int)min(num_blocks, (int64_t)0x7fffffff);
  const int64_t blk_stride = (int64_t)hkv * sd.nsub * Gm::SUB;
  const int64_t kvh_off = (int64_t)kvh * sd.nsub * Gm::SUB;
  const int32_t* bt_row = block_table + (int64_t)b * max_blocks;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);  // wave-uniform -> scalar tile math
  TileRegs<D, BK, BV> ra, rb;
  int tile = t_begin + wave_u;
  auto bt_of = [&](int t) __attribute__((always_inline)) { return fetch_bt_s(bt_row, t, t < t_end, seq_subs, sd); };
  TileOff lo;
  lo.k = (uint32_t)h * Gm::KTOK + (uint32_t)q * Gm::KLANE;
  lo.v = (uint32_t)Gm::KSEC + (uint32_t)lane * Gm::VLANE;
  lo.n = (uint32_t)Gm::KNORM + (uint32_t)q * 8u;
  auto load = [&](TileRegs<D, BK, BV>& r, BtPair bt, int t) __attribute__((always_inline)) {
    load_tile(r, cache, bt, t, sd, blk_stride, kvh_off, nb32, lo);
  };
  BtPair btv{{-1, -1}};
  if (tile < t_end) {
    load(ra, bt_of(tile), tile);
    btv = bt_of(tile + NW);
  }

  // Prologue, one barrier: the query heads are rotated by the first waves
  // (one head per 16 lanes); the last wave has built the K code table and
  // the one before it the V table; every wave then reads its MFMA operands of
  // the query.  Code tables hold f16(sigma level) with sigma chosen to
  // equalise the relative rounding errors; the scores and the output are
  // divided by sigma (1 + rmid), which leaves an error of at most half the
  // spread (one codebook array for K and V: one table, the K scale).
  {
    if (qg < G) {
#pragma unroll
      for (int i = 0; i < E; ++i) y[i] *= ksigns[ql16 * E + i];
      fwht_lanes<E, 16>(y, ql16);
      const float sc = (float)(1.0 / __builtin_sqrt((double)D)) * qscale;
#pragma unroll
      for (int i = 0; i < E; ++i) qs[qg][ql16 * E + i] = y[i] * sc;
    }
  }
  __syncthreads();

  // B operand of the Q.K MFMAs: lane (h, q), MFMA s -> Q[h][q*D/4 + 8s + j] as
  // f16; the remainder q - f16(q) goes to column 8 + h when G <= 8 (summed into
  // column h after the K loop, no extra MFMA), else (QL) to a second operand
  const bool qrem = !QL && G <= 8;
  const float kinv = tab_inv[0];
  Op8 qb[NS], ql[QL ? NS : 1];
  {
    const int hh = (qrem && h >= 8) ? h - 8 : h;
    const bool lo_col = hh != h;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      float x[8];
      if (hh < G) {
        const float4 a = *reinterpret_cast<const float4*>(&qs[hh][q * (D / 4) + 8 * s]);
        const float4 c = *reinterpret_cast<const float4*>(&qs[hh][q * (D / 4) + 8 * s + 4]);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = c.x; x[5] = c.y; x[6] = c.z; x[7] = c.w;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = 0.f;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t w = 0, wl = 0;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const float xv = x[2 * j + e] * kinv;
          const _Float16 hi = (_Float16)xv;
          const _Float16 lo = (_Float16)(xv - (float)hi);
          w |= (uint32_t)__builtin_bit_cast(uint16_t, lo_col ? lo : hi) << (16 * e);
          wl |= (uint32_t)__builtin_bit_cast(uint16_t, lo) << (16 * e);
        }
        qb[s].u[j] = w;
        if constexpr (QL) ql[s].u[j] = wl;
      }
    }
  }
  const uint32_t tabK = lut_lane_base<BK>(lane, 0u);  // the lane's copy offset in the table
  const uint32_t tabV = lut_lane_base<BV>(lane, 0u);


  float m_run = -INFINITY, l_run = 0.f;
  floatx4 acc[NB];
#pragma unroll
  for (int i = 0; i < NB; ++i) acc[i] = floatx4{0.f, 0.f, 0.f, 0.f};

  // One 32-token tile: scores, lazily rescaled online softmax, P.V.
  // Exponentials use the running reference max m_run; it is only raised (and
  // acc / l rescaled) when a tile max exceeds it by more than TAU, so
  // p <= 2^TAU.  P' = p * ||v|| * 2^-(TAU+1) then stays below the f16 maximum
  // for any fp16 norm; the final output is multiplied back by 2^(TAU+1).
  constexpr float TAU = 8.f;  // 2^(TAU+1) == 512
  auto process = [&](const TileRegs<D, BK, BV>& cur, int tile) __attribute__((always_inline)) {
    float s[2][4];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      floatx4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        Op8 a;
        const uint2 c01 = lut_quad_s<BK>(cur.k[sb], (8 * st) * BK, tabK, lutK);
        const uint2 c23 = lut_quad_s<BK>(cur.k[sb], (8 * st + 4) * BK, tabK, lutK);
        a.u[0] = c01.x; a.u[1] = c01.y; a.u[2] = c23.x; a.u[3] = c23.y;
        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, qb[st].h, c, 0, 0, 0);
        if constexpr (QL) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, ql[st].h, c, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const _Float16 kn = __builtin_bit_cast(_Float16, (uint16_t)(cur.kn[sb][i >> 1] >> (16 * (i & 1))));
        s[sb][i] = __builtin_fmaf(c[i], (float)kn, 0.f);
      }
    }
    if constexpr (BK <= 3 && BV <= 3) sched_lds_mfma<2 * NS, 4>();  // (4-bit tables: registers run out)
    // add the q remainder's column h + 8 (the same token, so the same K norm)
    if (qrem)
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int i = 0; i < 4; ++i) s[sb][i] += dpp_xor8(s[sb][i]);
    if (tile * 32 + 32 > seq_len) {  // only the last tile of a sequence is partial
#pragma unroll
      for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (tile * 32 + sb * 16 + 4 * q + i >= seq_len) s[sb][i] = -INFINITY;
    }
    float tmax = vmax3(s[0][0], s[0][1], s[0][2]);
    tmax = vmax3(tmax, s[0][3], s[1][0]);
    tmax = vmax3(tmax, s[1][1], s[1][2]);
    tmax = row_max4(vmax(tmax, s[1][3]));
    if (__builtin_amdgcn_ballot_w64(tmax > m_run + TAU) != 0) {  // wave-uniform, rare
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int bb = 0; bb < NB; ++bb) acc[bb] *= alpha;
    }
    // p is taken pre-scaled by 2^-(TAU+1) (folded into the exponent); l gets it back
    const float m_sc = m_run + (TAU + 1.f);
    float pr[8];
    Op8 pb;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
      for (int i2 = 0; i2 < 2; ++i2) {
        // V norms of two tokens as f16 halves (zero for a sub-block without
        // tokens); the products are rounded straight into the two halves of
        // the operand
        const uint32_t vn = cur.vn[sb][i2];
        const float p0 = __builtin_amdgcn_exp2f(s[sb][2 * i2] - m_sc);
        const float p1 = __builtin_amdgcn_exp2f(s[sb][2 * i2 + 1] - m_sc);
        pr[4 * sb + 2 * i2] = p0;
        pr[4 * sb + 2 * i2 + 1] = p1;
        pb.u[2 * sb + i2] = pv_pair(p0, p1, vn);
      }
    }
    // l_run holds the sum of the pre-scaled p (the 2^(TAU+1) goes back at the end)
    l_run += ((pr[0] + pr[1]) + (pr[2] + pr[3])) + ((pr[4] + pr[5]) + (pr[6] + pr[7]));
#pragma unroll
    for (int bb = 0; bb < NB; ++bb) {
      Op8 a;
#pragma unroll
      for (int sb = 0; sb < 2; ++sb) {
        const uint2 t4 = lut_quad_s<BV>(cur.v[sb], (4 * bb) * BV, tabV, lutV);
        a.u[2 * sb] = t4.x;
        a.u[2 * sb + 1] = t4.y;
      }
      acc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, pb.h, acc[bb], 0, 0, 0);
    }
    if constexpr (BK <= 3 && BV <= 3) sched_lds_mfma<NB, 4>();
  };

  // ping-pong over two register sets so the next tile's loads overlap this
  // tile's math and the block-table entries one tile further ahead.  Each
  // wave takes every NW-th tile: a fixed assignment, so the sums (and the
  // output bits) do not depend on how fast the waves progress.
  int tile1 = tile + NW;  // the tile whose loads go out next
  while (tile < t_end) {
    const int tile2 = tile1 + NW;
    BtPair btn = bt_of(tile2);
    load(rb, btv, tile1);
    btv = btn;
    process(ra, tile);
    tile = tile1;
    tile1 = tile2;
    if (tile >= t_end) break;
    const int tile3 = tile1 + NW;
    btn = bt_of(tile3);
    load(ra, btv, tile1);
    btv = btn;
    process(rb, tile);
    tile = tile1;
    tile1 = tile3;
  }
  // undo the P' pre-scale and the V table scale
  const float osc = 512.f * tab_inv[SHARE ? 0 : 1];
#pragma unroll
  for (int bb = 0; bb < NB; ++bb) acc[bb] *= osc;
  l_run *= 512.f;

  // ---- merge the 4 waves through LDS (the code tables' LDS is reused) ----
  __syncthreads();
  const float l_tot = warp_sum_q(l_run);
  if (q == 0) {
    red_m[wave][h] = m_run;
    red_l[wave][h] = l_tot;
  }
  if (h < G) {
    float* ro = red_o + (wave * G + h) * (D + 1);
#pragma unroll
    for (int bb = 0; bb < NB; ++bb)
#pragma unroll
      for (int i = 0; i < 4; ++i) ro[16 * bb + 4 * q + i] = acc[bb][i];
  }
  __syncthreads();

  if constexpr (NW == 16) {
    // wave g < G finishes q head g: lane l combines elements [E2 l, E2 l + E2)
    if (wave < G) {
      constexpr int E2 = D / 64;
      const int g = wave;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < NW; ++w) M = fmaxf(M, red_m[w][g]);
      float L = 0.f, y[E2];
#pragma unroll
      for (int i = 0; i < E2; ++i) y[i] = 0.f;
      if (M != -INFINITY) {
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const float f = __builtin_amdgcn_exp2f(red_m[w][g] - M);
          L += f * red_l[w][g];
#pragma unroll
          for (int i = 0; i < E2; ++i) y[i] += f * red_o[(w * G + g) * (D + 1) + lane * E2 + i];
        }
      }
      finish_row<D>(y, L, vsigns, vscale, lane, out, ot, (int64_t)b * hq + kvh * G + g);
    }
  } else {
    const int64_t row0 = ((int64_t)b * hq + kvh * G) * num_splits + split;  // (b, head g=0, split)
    for (int idx = tid; idx < G * D; idx += NW * 64) {
      const int g = idx / D, d = idx % D;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < NW; ++w) M = fmaxf(M, red_m[w][g]);
      float L = 0.f, o = 0.f;
      if (M != -INFINITY) {
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const float f = __builtin_amdgcn_exp2f(red_m[w][g] - M);
          L += f * red_l[w][g];
          o += f * red_o[(w * G + g) * (D + 1) + d];
        }
      }
      const int64_t row = row0 + (int64_t)g * num_splits;
      ws_o[row * D + d] = (L > 0.f) ? o / L : 0.f;
      if (d == 0) ws_lse[row] = (L > 0.f) ? M + __builtin_log2f(L) : -INFINITY;
    }
  }
}

// ---------------------------------------------------------------------------
// decode attention with fp32 operands on the VALU (the reference's arithmetic:
// fp32 products of the rotated query with the fp32 K levels, fp32 softmax
// weights times the fp32 V norms and levels), kept beside the MFMA kernel
// above to measure what the f16 matrix-core operands buy.  Split form only
// (4 waves per (split, kv head, batch), partials merged by merge_splits_kernel),
// d = 128, at most 4 query heads per kv head.
//
// Lane (m, g) = (lane & 15, lane >> 4) of a wave, per 16-token sub-block:
//   Q.K: token m, dims [32 g, 32 g + 32): 16 pair lookups of fp32 levels and
//        4 heads x 32 FMAs against the rotated query read from LDS (one
//        16-byte read gives the 4 heads of one dim); the four quarter sums of
//        a token are added over lanes m, m + 16, m + 32, m + 48.
//   P.V: the lane-major V chunk of lane (g, m) -- tokens 4g..4g+3, dims
//        16 b + m, b = 0..7 -- into acc[b][h] (fp32), summed over g after the
//        last tile.  The softmax weights move from the score layout (lane
//        (m, g) holds head g of token m) to the chunk layout through 512
//        bytes of LDS per wave.
// ---------------------------------------------------------------------------
template <int B>
struct CodeLut32 {  // fp32 pair tables: entry = (level[c0], level[c1]), 8 bytes
  static constexpr int ENTRIES = 1 << (2 * B);
  static constexpr int LOG_COPIES = (B <= 3) ? 4 : 0;  // 16 copies: a 16-lane phase of 8-byte reads
  static constexpr int COPIES = 1 << LOG_COPIES;
  static constexpr int BYTES = ENTRIES * 8 * COPIES;
};

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) const f32x2 lds_f2;
typedef __attribute__((address_space(3))) const f32x4 lds_f4;

template <int B>
__device__ void build_code_lut32(uint8_t* lut, const float* __restrict__ lev, int tid, int nthreads) {
  using C = CodeLut32<B>;
  for (int k = tid; k < C::ENTRIES * C::COPIES; k += nthreads) {
    const int e = k >> C::LOG_COPIES;
    reinterpret_cast<f32x2*>(lut)[k] = f32x2{lev[e & ((1 << B) - 1)], lev[e >> B]};
  }
}

// the fp32 levels of the 2 codes at bits [P, P + 2B) of the code words
template <int B, int N>
__device__ __forceinline__ f32x2 lut32_pair(const uint32_t (&w)[N], int P, uint32_t base) {
  using C = CodeLut32<B>;
  return *(lds_f2*)(uintptr_t)lut_entry_off<3 + C::LOG_COPIES, 2 * B>(w, P, base);
}

template <int D, int BK, int BV>
struct ValuTile {
  using Gm = PagedGeom<D, BK, BV>;
  uint32_t k[2][Gm::KLANE / 4];  // token m, K bytes [g KLANE, (g + 1) KLANE)
  uint32_t v[2][Gm::VLANE / 4];  // V chunk of lane (g, m)
  uint32_t kn[2];                // K norm of token m (f16 bits, low half)
  uint32_t vn[2][2];             // V norms of tokens 4g..4g+3
  bool ok[2];
};

template <int D, int BK, int BV>
__device__ __forceinline__ void load_tile_valu(ValuTile<D, BK, BV>& r, const uint8_t* __restrict__ cache, int btv,
                                               int tile, const SubDiv& sd, int64_t blk_stride, int64_t kvh_off,
                                               int nb32, uint32_t ok_off, uint32_t ov_off, uint32_t okn, uint32_t ovn) {
  using Gm = PagedGeom<D, BK, BV>;
#pragma unroll
  for (int sb = 0; sb < 2; ++sb) {
    int phys = __builtin_amdgcn_readlane(btv, sb);
    const bool valid = (uint32_t)phys < (uint32_t)nb32;
    const int j = 2 * tile + sb;
    const int sub = valid ? j - sd.page(j) * sd.nsub : 0;
    if (!valid) phys = 0;
    const uint8_t* base = cache + ((int64_t)phys * blk_stride + kvh_off + (int64_t)sub * Gm::SUB);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, Gm::SUB, 0x00020000);
    buf_dwords(rs, ok_off, r.k[sb]);
    buf_dwords(rs, ov_off, r.v[sb]);
    r.kn[sb] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, okn, 0, 0);
    buf_dwords(rs, ovn, r.vn[sb]);
    r.ok[sb] = valid;
  }
}

template <int D, int BK, int BV, int QT, bool SHARE>
__global__ __launch_bounds__(256, 2) void paged_attn_valu_kernel(
    const void* __restrict__ query, const uint8_t* __restrict__ cache,
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ seq_lens, int hq, int hkv,
    int page_size, int max_blocks, int64_t num_blocks, const float* __restrict__ ksigns,
    const float* __restrict__ klev, const float* __restrict__ vlev, float qscale, int num_splits,
    float* __restrict__ ws_o, float* __restrict__ ws_lse) {
  static_assert(D == 128, "laid out for head_dim 128");
  using Gm = PagedGeom<D, BK, BV>;
  constexpr int NW = 4, GM = 4;  // waves, query heads per kv head (at most)
  constexpr int E = D / 16;
  constexpr int QG = 32 * GM + 4;  // floats per quarter of the query block (padded: conflict-free reads)
  constexpr int LK = CodeLut32<BK>::BYTES, LV = SHARE ? 0 : CodeLut32<BV>::BYTES;
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int G = hq / hkv;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m = lane & 15, g = lane >> 4;

  // LDS: code tables | rotated query [4 quarters][32 dims][4 heads] | per-wave
  // softmax weights [2 sub-blocks][16 tokens][4 heads]; the tables' bytes are
  // reused for the wave merge at the end
  extern __shared__ __attribute__((aligned(16))) uint8_t pool[];
  __shared__ float red_m[NW][GM], red_l[NW][GM];
  uint8_t* lutK = pool;
  uint8_t* lutV = SHARE ? pool : pool + LK;
  float* qv = reinterpret_cast<float*>(pool + LK + LV);
  float* pw = qv + 4 * QG + wave * 128;
  float* red_o = reinterpret_cast<float*>(pool);

  const int seq_len = seq_lens[b];
  const int n_tiles = (seq_len + 31) >> 5;
  const int tps = (n_tiles + num_splits - 1) / num_splits;
  const int t_begin = split * tps;
  const int t_end = min(t_begin + tps, n_tiles);
  SubDiv sd;
  sd.nsub = page_size >> 4;
  sd.m = (0x80000000u + (uint32_t)sd.nsub - 1u) / (uint32_t)sd.nsub;
  sd.j_cap = (int)min((int64_t)max_blocks * sd.nsub, (int64_t)0x7fffffff);
  const int seq_subs = (int)(((int64_t)seq_len + 15) >> 4);
  const int nb32 = (int)min(num_blocks, (int64_t)0x7fffffff);
  const int64_t blk_stride = (int64_t)hkv * sd.nsub * Gm::SUB;
  const int64_t kvh_off = (int64_t)kvh * sd.nsub * Gm::SUB;
  const __amdgpu_buffer_rsrc_t bt_rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int32_t*>(block_table + (int64_t)b * max_blocks), (short)0,
      (int)min((int64_t)max_blocks * 4, (int64_t)0x7ffffffc), 0x00020000);
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const uint32_t ok_off = (uint32_t)m * Gm::KTOK + (uint32_t)g * Gm::KLANE;
  const uint32_t ov_off = (uint32_t)Gm::KSEC + (uint32_t)lane * Gm::VLANE;
  const uint32_t okn = (uint32_t)Gm::KNORM + 2u * (uint32_t)m;
  const uint32_t ovn = (uint32_t)Gm::VNORM + 8u * (uint32_t)g;
  ValuTile<D, BK, BV> ra, rb;
  int tile = t_begin + wave_u;
  auto bt_of = [&](int t) __attribute__((always_inline)) {
    return fetch_bt(bt_rs, t, t < t_end, seq_subs, sd, (uint32_t)lane);
  };
  auto load = [&](ValuTile<D, BK, BV>& r, int btv, int t) __attribute__((always_inline)) {
    load_tile_valu(r, cache, btv, t, sd, blk_stride, kvh_off, nb32, ok_off, ov_off, okn, ovn);
  };
  int btv = 0;
  if (tile < t_end) {
    load(ra, bt_of(tile), tile);
    btv = bt_of(tile + NW);
  }

  // prologue: fp32 pair tables, rotated and scaled query (one head per 16 lanes)
  build_code_lut32<BK>(lutK, klev, tid, NW * 64);
  if (!SHARE) build_code_lut32<BV>(lutV, vlev, tid, NW * 64);
  {
    const int hh = tid >> 4, l16 = tid & 15;
    if (hh < GM) {
      float y[E];
      if (hh < G) {
        load_elems<QT, E>(query, ((int64_t)b * hq + kvh * G + hh) * D + l16 * E, y);
#pragma unroll
        for (int i = 0; i < E; ++i) y[i] *= ksigns[l16 * E + i];
      } else {
#pragma unroll
        for (int i = 0; i < E; ++i) y[i] = 0.f;
      }
      fwht_lanes<E, 16>(y, l16);
      const float sc = (float)(1.0 / __builtin_sqrt((double)D)) * qscale;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const int dd = l16 * E + i;
        qv[(dd >> 5) * QG + (dd & 31) * GM + hh] = y[i] * sc;
      }
    }
  }
  __syncthreads();
  const uint32_t tabK = lds_addr(lutK) + (((uint32_t)lane & (CodeLut32<BK>::COPIES - 1u)) << 3);
  const uint32_t tabV = lds_addr(lutV) + (((uint32_t)lane & (CodeLut32<BV>::COPIES - 1u)) << 3);
  const uint32_t qaddr = lds_addr(qv) + (uint32_t)g * QG * 4u;
  const uint32_t pw_addr = lds_addr(pw);

  float m_run[GM], l_run = 0.f;
  float acc[8][GM];
#pragma unroll
  for (int h = 0; h < GM; ++h) m_run[h] = -INFINITY;
#pragma unroll
  for (int bb = 0; bb < 8; ++bb)
#pragma unroll
    for (int h = 0; h < GM; ++h) acc[bb][h] = 0.f;

  constexpr float TAU = 8.f;
  auto process = [&](const ValuTile<D, BK, BV>& cur, int tile) __attribute__((always_inline)) {
    float s[2][GM];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      float sq[GM];
#pragma unroll
      for (int h = 0; h < GM; ++h) sq[h] = 0.f;
#pragma unroll
      for (int j = 0; j < 32; j += 2) {
        const f32x2 lv = lut32_pair<BK>(cur.k[sb], j * BK, tabK);
        const f32x4 q0 = *(lds_f4*)(uintptr_t)(qaddr + 16u * (uint32_t)j);
        const f32x4 q1 = *(lds_f4*)(uintptr_t)(qaddr + 16u * (uint32_t)(j + 1));
        sq[0] = __builtin_fmaf(q0.x, lv.x, sq[0]);
        sq[1] = __builtin_fmaf(q0.y, lv.x, sq[1]);
        sq[2] = __builtin_fmaf(q0.z, lv.x, sq[2]);
        sq[3] = __builtin_fmaf(q0.w, lv.x, sq[3]);
        sq[0] = __builtin_fmaf(q1.x, lv.y, sq[0]);
        sq[1] = __builtin_fmaf(q1.y, lv.y, sq[1]);
        sq[2] = __builtin_fmaf(q1.z, lv.y, sq[2]);
        sq[3] = __builtin_fmaf(q1.w, lv.y, sq[3]);
      }
      const float kn = (float)__builtin_bit_cast(_Float16, (uint16_t)cur.kn[sb]);
      const bool live = tile * 32 + sb * 16 + m < seq_len;
#pragma unroll
      for (int h = 0; h < GM; ++h) {
        const float t = warp_sum_q(sq[h]) * kn;
        s[sb][h] = live ? t : -INFINITY;
      }
    }
    float tmax[GM];
    bool raise = false;
#pragma unroll
    for (int h = 0; h < GM; ++h) {
      float x = vmax(s[0][h], s[1][h]);
      x = vmax(x, lane_xor<1>(x));
      x = vmax(x, lane_xor<2>(x));
      x = vmax(x, lane_xor<4>(x));
      tmax[h] = vmax(x, lane_xor<8>(x));
      raise = raise || (tmax[h] > m_run[h] + TAU);
    }
    if (__builtin_amdgcn_ballot_w64(raise) != 0) {  // wave-uniform, rare
      float al[GM];
#pragma unroll
      for (int h = 0; h < GM; ++h) {
        const float m_new = fmaxf(m_run[h], tmax[h]);
        al[h] = __builtin_amdgcn_exp2f(m_run[h] - m_new);
        m_run[h] = m_new;
#pragma unroll
        for (int bb = 0; bb < 8; ++bb) acc[bb][h] *= al[h];
      }
      l_run *= g == 0 ? al[0] : g == 1 ? al[1] : g == 2 ? al[2] : al[3];
    }
    // softmax weights of head g for token m of both sub-blocks
    const float mg = g == 0 ? m_run[0] : g == 1 ? m_run[1] : g == 2 ? m_run[2] : m_run[3];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      const float sg = g == 0 ? s[sb][0] : g == 1 ? s[sb][1] : g == 2 ? s[sb][2] : s[sb][3];
      const float p = __builtin_amdgcn_exp2f(sg - mg);
      l_run += p;
      pw[(sb * 16 + m) * GM + g] = p;
    }
    __asm__ volatile("" ::: "memory");  // a wave's LDS accesses run in order
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
      float pv[4][GM];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 pp = *(lds_f4*)(uintptr_t)(pw_addr + 16u * (uint32_t)(sb * 16 + 4 * g + i));
        const uint32_t vw = cur.vn[sb][i >> 1];
        const float vn = cur.ok[sb] ? (float)__builtin_bit_cast(_Float16, (uint16_t)(vw >> (16 * (i & 1)))) : 0.f;
        pv[i][0] = pp.x * vn;
        pv[i][1] = pp.y * vn;
        pv[i][2] = pp.z * vn;
        pv[i][3] = pp.w * vn;
      }
#pragma unroll
      for (int bb = 0; bb < 8; ++bb) {
#pragma unroll
        for (int pr = 0; pr < 2; ++pr) {
          const f32x2 lv = lut32_pair<BV>(cur.v[sb], (4 * bb + 2 * pr) * BV, tabV);
#pragma unroll
          for (int h = 0; h < GM; ++h) {
            acc[bb][h] = __builtin_fmaf(pv[2 * pr][h], lv.x, acc[bb][h]);
            acc[bb][h] = __builtin_fmaf(pv[2 * pr + 1][h], lv.y, acc[bb][h]);
          }
        }
      }
    }
    __asm__ volatile("" ::: "memory");
  };

  int tile1 = tile + NW;  // the tile whose loads go out next
  while (tile < t_end) {
    const int tile2 = tile1 + NW;
    int btn = bt_of(tile2);
    load(rb, btv, tile1);
    btv = btn;
    process(ra, tile);
    tile = tile1;
    tile1 = tile2;
    if (tile >= t_end) break;
    const int tile3 = tile1 + NW;
    btn = bt_of(tile3);
    load(ra, btv, tile1);
    btv = btn;
    process(rb, tile);
    tile = tile1;
    tile1 = tile3;
  }

  // ---- wave totals, then the 4 waves merged through LDS ----
  const float l_tot = group_sum<16>(l_run);  // head g, over the 16 tokens of a row
#pragma unroll
  for (int bb = 0; bb < 8; ++bb)
#pragma unroll
    for (int h = 0; h < GM; ++h) acc[bb][h] = warp_sum_q(acc[bb][h]);
  __syncthreads();  // the code tables are dead: their LDS takes the merge buffer
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < GM; ++h) red_m[wave][h] = m_run[h];
  }
  if (m == 0) red_l[wave][g] = l_tot;
  if (g == 0) {
#pragma unroll
    for (int h = 0; h < GM; ++h)
      if (h < G)
#pragma unroll
        for (int bb = 0; bb < 8; ++bb) red_o[(wave * G + h) * (D + 1) + 16 * bb + m] = acc[bb][h];
  }
  __syncthreads();
  const int64_t row0 = ((int64_t)b * hq + kvh * G) * num_splits + split;
  for (int idx = tid; idx < G * D; idx += NW * 64) {
    const int gg = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, red_m[w][gg]);
    float L = 0.f, o = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float f = __builtin_amdgcn_exp2f(red_m[w][gg] - M);
        L += f * red_l[w][gg];
        o += f * red_o[(w * G + gg) * (D + 1) + d];
      }
    }
    const int64_t row = row0 + (int64_t)gg * num_splits;
    ws_o[row * D + d] = (L > 0.f) ? o / L : 0.f;
    if (d == 0) ws_lse[row] = (L > 0.f) ? M + __builtin_log2f(L) : -INFINITY;
  }
}

template <int D, int BK, int BV, bool SHARE>
__host__ constexpr int paged_attn_valu_lds() {
  const int tabs = CodeLut32<BK>::BYTES + (SHARE ? 0 : CodeLut32<BV>::BYTES);
  const int front = tabs + (4 * (32 * 4 + 4) + 4 * 128) * 4;
  const int red = 4 * 4 * (D + 1) * 4;
  return front > red ? front : red;
}

// ---------------------------------------------------------------------------
// host launchers (stage 2 -- merge of the splits, inverse RHT of V, output
// cast -- is merge_splits_kernel in ftq_merge.h)
// ---------------------------------------------------------------------------
float fwht_scale(int d);

template <int D, int BK, int BV>
static hipError_t launch_store3(const void* k, const void* v, int dt, int64_t n, int hkv,
                                const float* ks, const float* vs, const float* kb, const float* vb,
                                const int64_t* slots, uint8_t* cache, int page_size,
                                int64_t num_blocks, hipStream_t st) {
  const int64_t items = (n + 15) / 16 * hkv;  // (16-token group, kv head), 4 per workgroup
  int64_t g = (items + 3) / 4;
  if (g > 256 * 8) g = 256 * 8;
  const float sc = fwht_scale(D);
  dim3 grid((unsigned)g), block(256);
  if (dt == F32) {
    paged_store_kernel<D, BK, BV, F32><<<grid, block, 0, st>>>(k, v, n, hkv, ks, vs, kb, vb, slots, cache, page_size, num_blocks, sc);
  } else {  // one launch: whole sub-blocks on the matrix cores, the rest per token
    const double rsc = 1.0 / (double)sc;
    if (dt == F16) {
      static const int cap = resident_workgroups(paged_store_mfma_kernel<D, BK, BV, F16>);
      paged_store_mfma_kernel<D, BK, BV, F16><<<dim3((unsigned)(g < cap ? g : cap)), block, 0, st>>>(
          k, v, n, hkv, ks, vs, kb, vb, slots, cache, page_size, num_blocks, sc, rsc);
    } else {
      static const int cap = resident_workgroups(paged_store_mfma_kernel<D, BK, BV, BF16>);
      paged_store_mfma_kernel<D, BK, BV, BF16><<<dim3((unsigned)(g < cap ? g : cap)), block, 0, st>>>(
          k, v, n, hkv, ks, vs, kb, vb, slots, cache, page_size, num_blocks, sc, rsc);
    }
  }
  return hipGetLastError();
}

template <int D, int BK>
static hipError_t launch_store2(int bv, const void* k, const void* v, int dt, int64_t n, int hkv,
                                const float* ks, const float* vs, const float* kb, const float* vb,
                                const int64_t* slots, uint8_t* cache, int page_size,
                                int64_t num_blocks, hipStream_t st) {
  if (bv == 2) return launch_store3<D, BK, 2>(k, v, dt, n, hkv, ks, vs, kb, vb, slots, cache, page_size, num_blocks, st);
  if (bv == 3) return launch_store3<D, BK, 3>(k, v, dt, n, hkv, ks, vs, kb, vb, slots, cache, page_size, num_blocks, st);
  return launch_store3<D, BK, 4>(k, v, dt, n, hkv, ks, vs, kb, vb, slots, cache, page_size, num_blocks, st);
}

template <int D>
static hipError_t launch_store1(int bk, int bv, const void* k, const void* v, int dt, int64_t n,
                                int hkv, const float* ks, const float* vs, const float* kb,
                                const float* vb, const int64_t* slots, uint8_t* cache,
                                int page_size, int64_t num_blocks, hipStream_t st) {
  if (bk == 2) return launch_store2<D, 2>(bv, k, v, dt, n, hkv, ks, vs, kb, vb, slots, cache, page_size, num_blocks, st);
  if (bk == 3) return launch_store2<D, 3>(bv, k, v, dt, n, hkv, ks, vs, kb, vb, slots, cache, page_size, num_blocks, st);
  return launch_store2<D, 4>(bv, k, v, dt, n, hkv, ks, vs, kb, vb, slots, cache, page_size, num_blocks, st);
}

struct AttnArgs {
  const void* q;
  int qt;
  const uint8_t* cache;
  const int32_t* bt;
  const int32_t* sl;
  int B, hq, hkv, page_size, max_blocks;
  int64_t num_blocks;
  const float *ks, *vs, *kl, *vl;
  float qscale;
  int splits;
  float *wo, *wl;
  void* out;
  int ot;
};

// the single-workgroup form applies: d = 128, GQA group <= 4, one split
static bool fused_form(int d, int hq, int hkv, int splits) {
  return d == 128 && hq / hkv <= 4 && splits == 1;
}

template <int D, int BK, int BV, bool SHARE, int NW, bool QL = false>
static void launch_attn_nw(const AttnArgs& a, hipStream_t st) {
  dim3 grid(a.splits, a.hkv, a.B), block(NW * 64);
  const size_t lds = (size_t)paged_attn_lds<D, BK, BV, SHARE, NW>(a.hq / a.hkv);
  const float sc = fwht_scale(D);
  if (a.qt == F32)
    paged_attn_kernel<D, BK, BV, F32, SHARE, NW, QL><<<grid, block, lds, st>>>(a.q, a.cache, a.bt, a.sl, a.hq, a.hkv, a.page_size, a.max_blocks, a.num_blocks, a.ks, a.kl, a.vl, a.qscale, a.splits, a.wo, a.wl, a.vs, sc, a.out, a.ot);
  else if (a.qt == F16)
    paged_attn_kernel<D, BK, BV, F16, SHARE, NW, QL><<<grid, block, lds, st>>>(a.q, a.cache, a.bt, a.sl, a.hq, a.hkv, a.page_size, a.max_blocks, a.num_blocks, a.ks, a.kl, a.vl, a.qscale, a.splits, a.wo, a.wl, a.vs, sc, a.out, a.ot);
  else
    paged_attn_kernel<D, BK, BV, BF16, SHARE, NW, QL><<<grid, block, lds, st>>>(a.q, a.cache, a.bt, a.sl, a.hq, a.hkv, a.page_size, a.max_blocks, a.num_blocks, a.ks, a.kl, a.vl, a.qscale, a.splits, a.wo, a.wl, a.vs, sc, a.out, a.ot);
}

template <int D, int BK, int BV, bool SHARE>
static void launch_attn_kernel(const AttnArgs& a, hipStream_t st) {
  if constexpr (D == 128) {
    if (fused_form(D, a.hq, a.hkv, a.splits)) {
      launch_attn_nw<D, BK, BV, SHARE, 16>(a, st);
      return;
    }
  }
  if (a.hq / a.hkv > 8) launch_attn_nw<D, BK, BV, SHARE, 4, true>(a, st);
  else launch_attn_nw<D, BK, BV, SHARE, 4>(a, st);
}

template <int D, int BK, int BV>
static hipError_t launch_attn3(const AttnArgs& a, hipStream_t st) {
  // K and V share one code table when they use the same codebook array
  if constexpr (BK == BV) {
    if (a.kl == a.vl) launch_attn_kernel<D, BK, BV, true>(a, st);
    else launch_attn_kernel<D, BK, BV, false>(a, st);
  } else {
    launch_attn_kernel<D, BK, BV, false>(a, st);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (fused_form(D, a.hq, a.hkv, a.splits)) return hipSuccess;  // the kernel wrote the output
  const int64_t rows = (int64_t)a.B * a.hq;
  const float sc = fwht_scale(D);
  if (a.ot == F32) return launch_merge_splits<D, F32, ROT_SIGNS>(a.wo, a.wl, rows, a.splits, a.vs, sc, a.out, st);
  if (a.ot == F16) return launch_merge_splits<D, F16, ROT_SIGNS>(a.wo, a.wl, rows, a.splits, a.vs, sc, a.out, st);
  return launch_merge_splits<D, BF16, ROT_SIGNS>(a.wo, a.wl, rows, a.splits, a.vs, sc, a.out, st);
}

template <int D, int BK>
static hipError_t launch_attn2(int bv, const AttnArgs& a, hipStream_t st) {
  if (bv == 2) return launch_attn3<D, BK, 2>(a, st);
  if (bv == 3) return launch_attn3<D, BK, 3>(a, st);
  return launch_attn3<D, BK, 4>(a, st);
}

template <int D>
static hipError_t launch_attn1(int bk, int bv, const AttnArgs& a, hipStream_t st) {
  if (bk == 2) return launch_attn2<D, 2>(bv, a, st);
  if (bk == 3) return launch_attn2<D, 3>(bv, a, st);
  return launch_attn2<D, 4>(bv, a, st);
}

// merge of the split partials: inverse RHT of V, output dtype
static hipError_t launch_attn_merge(const AttnArgs& a, int d, hipStream_t st) {
  const int64_t rows = (int64_t)a.B * a.hq;
  const float sc = fwht_scale(d);
  if (d == 256) {
    if (a.ot == F32) return launch_merge_splits<256, F32, ROT_SIGNS>(a.wo, a.wl, rows, a.splits, a.vs, sc, a.out, st);
    if (a.ot == F16) return launch_merge_splits<256, F16, ROT_SIGNS>(a.wo, a.wl, rows, a.splits, a.vs, sc, a.out, st);
    return launch_merge_splits<256, BF16, ROT_SIGNS>(a.wo, a.wl, rows, a.splits, a.vs, sc, a.out, st);
  }
  if (a.ot == F32) return launch_merge_splits<128, F32, ROT_SIGNS>(a.wo, a.wl, rows, a.splits, a.vs, sc, a.out, st);
  if (a.ot == F16) return launch_merge_splits<128, F16, ROT_SIGNS>(a.wo, a.wl, rows, a.splits, a.vs, sc, a.out, st);
  return launch_merge_splits<128, BF16, ROT_SIGNS>(a.wo, a.wl, rows, a.splits, a.vs, sc, a.out, st);
}

template <int D, int BK, int BV, bool SHARE>
static void launch_attn_valu_kernel(const AttnArgs& a, hipStream_t st) {
  dim3 grid(a.splits, a.hkv, a.B), block(256);
  constexpr size_t lds = (size_t)paged_attn_valu_lds<D, BK, BV, SHARE>();
  if (a.qt == F32)
    paged_attn_valu_kernel<D, BK, BV, F32, SHARE><<<grid, block, lds, st>>>(a.q, a.cache, a.bt, a.sl, a.hq, a.hkv, a.page_size, a.max_blocks, a.num_blocks, a.ks, a.kl, a.vl, a.qscale, a.splits, a.wo, a.wl);
  else if (a.qt == F16)
    paged_attn_valu_kernel<D, BK, BV, F16, SHARE><<<grid, block, lds, st>>>(a.q, a.cache, a.bt, a.sl, a.hq, a.hkv, a.page_size, a.max_blocks, a.num_blocks, a.ks, a.kl, a.vl, a.qscale, a.splits, a.wo, a.wl);
  else
    paged_attn_valu_kernel<D, BK, BV, BF16, SHARE><<<grid, block, lds, st>>>(a.q, a.cache, a.bt, a.sl, a.hq, a.hkv, a.page_size, a.max_blocks, a.num_blocks, a.ks, a.kl, a.vl, a.qscale, a.splits, a.wo, a.wl);
}

template <int BK, int BV>
static hipError_t launch_attn_valu(const AttnArgs& a, hipStream_t st) {
  if constexpr (BK == BV) {
    if (a.kl == a.vl) launch_attn_valu_kernel<128, BK, BV, true>(a, st);
    else launch_attn_valu_kernel<128, BK, BV, false>(a, st);
  } else {
    launch_attn_valu_kernel<128, BK, BV, false>(a, st);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return launch_attn_merge(a, 128, st);
}

template <int BK>
static hipError_t launch_attn_valu2(int bv, const AttnArgs& a, hipStream_t st) {
  if (bv == 2) return launch_attn_valu<BK, 2>(a, st);
  if (bv == 3) return launch_attn_valu<BK, 3>(a, st);
  return launch_attn_valu<BK, 4>(a, st);
}

int auto_splits(int batch, int hkv, int seq_hint, int target_wgs) {
  // aim for target_wgs workgroups with at least 8 tiles per wave (an empty
  // batch or head count counts as one unit)
  const int64_t units = (batch > 0 && hkv > 0) ? (int64_t)batch * hkv : 1;
  int s = (int)std::min<int64_t>((target_wgs + units - 1) / units, 64);
  const int max_by_len = seq_hint / (32 * 4 * 8);
  if (s > max_by_len) s = max_by_len;
  if (s < 1) s = 1;
  if (s > 64) s = 64;
  return s;
}

}  // namespace ftq

using namespace ftq;

extern "C" int64_t ftq_paged_subblock_bytes(int d, int bits_k, int bits_v) {
  if (!(d == 128 || d == 256) || bits_k < 2 || bits_k > 4 || bits_v < 2 || bits_v > 4) return -1;
  return paged_sub_bytes(d, bits_k, bits_v);
}

extern "C" int64_t ftq_paged_workspace_bytes(int batch, int num_q_heads, int d, int num_splits) {
  return split_workspace_bytes(batch, num_q_heads, d, num_splits);
}

extern "C" int ftq_paged_default_splits(int batch, int num_kv_heads, int max_seq_len) {
  return auto_splits(batch, num_kv_heads, max_seq_len, 1024);  // 4 workgroups per CU
}

extern "C" int ftq_paged_choose_splits(int batch, int num_q_heads, int num_kv_heads, int d, int max_seq_len) {
  if (batch <= 0 || num_kv_heads <= 0 || num_q_heads <= 0) return 1;
  // one split when the single-workgroup form applies and its 16-wave
  // workgroups (one per CU at a time) keep the 256 CUs at least 3/4 busy
  // (past 768 units every whole-round count fills 3/4: the cap keeps the
  // products small without changing the answer)
  const int64_t units = std::min<int64_t>((int64_t)batch * num_kv_heads, 1 << 20);
  if (fused_form(d, num_q_heads, num_kv_heads, 1) && units >= 256) {
    const int64_t rounds = (units + 255) / 256;
    if (units * 4 >= rounds * 256 * 3) return 1;
  }
  return ftq_paged_default_splits(batch, num_kv_heads, max_seq_len);
}

extern "C" int ftq_paged_store(const void* key, const void* value, int dtype, int64_t n_tokens,
                               int num_kv_heads, int d, const float* k_signs, const float* v_signs,
                               const float* k_boundaries, const float* v_boundaries, int bits_k,
                               int bits_v, const int64_t* slot_mapping, uint8_t* kv_cache,
                               int page_size, int64_t num_blocks, void* stream) {
  FTQ_REQUIRE(d == 128 || d == 256, "paged cache: head_dim must be 128 or 256");
  FTQ_REQUIRE(num_blocks >= 0, "num_blocks must be >= 0");
  FTQ_REQUIRE(bits_k >= 2 && bits_k <= 4 && bits_v >= 2 && bits_v <= 4, "bits must be 2, 3, or 4");
  FTQ_REQUIRE(page_size >= 16 && page_size % 16 == 0, "page_size must be a multiple of 16");
  FTQ_REQUIRE(n_tokens >= 0 && num_kv_heads > 0, "bad token / head count");
  FTQ_REQUIRE(dtype >= F32 && dtype <= BF16, "dtype must be FTQ_F32, FTQ_F16 or FTQ_BF16");
  if (n_tokens == 0) return FTQ_OK;
  FTQ_REQUIRE(key && value && k_signs && v_signs && k_boundaries && v_boundaries && slot_mapping && kv_cache,
              "null pointer argument");
  FTQ_REQUIRE(aligned16(key) && aligned16(value), "key/value must be 16-byte aligned");
  FTQ_REQUIRE(aligned16(kv_cache), "kv_cache must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (d == 128)
    e = launch_store1<128>(bits_k, bits_v, key, value, dtype, n_tokens, num_kv_heads, k_signs, v_signs,
                           k_boundaries, v_boundaries, slot_mapping, kv_cache, page_size, num_blocks, st);
  else
    e = launch_store1<256>(bits_k, bits_v, key, value, dtype, n_tokens, num_kv_heads, k_signs, v_signs,
                           k_boundaries, v_boundaries, slot_mapping, kv_cache, page_size, num_blocks, st);
  return hip_status(e);
}

// Argument checks and launch arguments shared by the two decode entry points.
static int paged_attn_args(AttnArgs& a, const void* query, int q_dtype, const uint8_t* kv_cache,
                           const int32_t* block_table, const int32_t* seq_lens, int batch, int num_q_heads,
                           int num_kv_heads, int d, int page_size, int max_blocks_per_seq, int64_t num_blocks,
                           const float* k_signs, const float* v_signs, const float* k_levels,
                           const float* v_levels, int bits_k, int bits_v, float scale, int num_splits,
                           void* workspace, int64_t workspace_bytes, void* out, int out_dtype) {
  FTQ_REQUIRE(d == 128 || d == 256, "paged attention: head_dim must be 128 or 256");
  FTQ_REQUIRE(bits_k >= 2 && bits_k <= 4 && bits_v >= 2 && bits_v <= 4, "bits must be 2, 3, or 4");
  FTQ_REQUIRE(page_size >= 16 && page_size % 16 == 0, "page_size must be a multiple of 16");
  FTQ_REQUIRE(batch >= 0 && num_kv_heads > 0 && num_q_heads > 0, "bad batch / head counts");
  FTQ_REQUIRE(num_q_heads % num_kv_heads == 0, "num_q_heads must be a multiple of num_kv_heads");
  FTQ_REQUIRE(num_q_heads / num_kv_heads <= 16, "GQA group (num_q_heads / num_kv_heads) must be <= 16");
  FTQ_REQUIRE(num_splits >= 1 && num_splits <= 1024, "num_splits must be in [1, 1024]");
  FTQ_REQUIRE(max_blocks_per_seq >= 0, "max_blocks_per_seq must be >= 0");
  {
    const int64_t nsub = page_size / 16;
    FTQ_REQUIRE((nsub & (nsub - 1)) == 0 || (int64_t)max_blocks_per_seq * nsub * nsub < ((int64_t)1 << 31),
                "max_blocks_per_seq * (page_size / 16)^2 must be below 2^31 when page_size / 16 is not a power of two");
  }
  FTQ_REQUIRE(q_dtype >= F32 && q_dtype <= BF16 && out_dtype >= F32 && out_dtype <= BF16,
              "dtype must be FTQ_F32, FTQ_F16 or FTQ_BF16");
  if (batch == 0) return FTQ_OK;
  FTQ_REQUIRE(query && kv_cache && block_table && seq_lens && k_signs && v_signs && k_levels &&
                  v_levels && workspace && out,
              "null pointer argument");
  FTQ_REQUIRE(workspace_bytes >= ftq_paged_workspace_bytes(batch, num_q_heads, d, num_splits),
              "workspace too small (see ftq_paged_workspace_bytes)");
  FTQ_REQUIRE(aligned16(query) && aligned16(out) && aligned16(workspace) && aligned16(kv_cache),
              "query, out, workspace and kv_cache must be 16-byte aligned");
  a.q = query; a.qt = q_dtype; a.cache = kv_cache; a.bt = block_table; a.sl = seq_lens;
  a.B = batch; a.hq = num_q_heads; a.hkv = num_kv_heads; a.page_size = page_size;
  a.max_blocks = max_blocks_per_seq; a.num_blocks = num_blocks; a.ks = k_signs; a.vs = v_signs; a.kl = k_levels; a.vl = v_levels;
  a.qscale = scale * 1.4426950408889634f;
  a.splits = num_splits;
  a.wo = static_cast<float*>(workspace);
  a.wl = a.wo + (int64_t)batch * num_q_heads * num_splits * d;
  a.out = out; a.ot = out_dtype;
  return FTQ_OK;
}

extern "C" int ftq_paged_decode_attention(
    const void* query, int q_dtype, const uint8_t* kv_cache, const int32_t* block_table,
    const int32_t* seq_lens, int batch, int num_q_heads, int num_kv_heads, int d, int page_size,
    int max_blocks_per_seq, int64_t num_blocks, const float* k_signs, const float* v_signs, const float* k_levels,
    const float* v_levels, int bits_k, int bits_v, float scale, int num_splits, void* workspace,
    int64_t workspace_bytes, void* out, int out_dtype, void* stream) {
  AttnArgs a;
  const int rc = paged_attn_args(a, query, q_dtype, kv_cache, block_table, seq_lens, batch, num_q_heads,
                                 num_kv_heads, d, page_size, max_blocks_per_seq, num_blocks, k_signs, v_signs,
                                 k_levels, v_levels, bits_k, bits_v, scale, num_splits, workspace,
                                 workspace_bytes, out, out_dtype);
  if (rc != FTQ_OK || batch == 0) return rc;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = (d == 128) ? launch_attn1<128>(bits_k, bits_v, a, st) : launch_attn1<256>(bits_k, bits_v, a, st);
  return hip_status(e);
}

extern "C" int ftq_paged_decode_attention_valu(
    const void* query, int q_dtype, const uint8_t* kv_cache, const int32_t* block_table,
    const int32_t* seq_lens, int batch, int num_q_heads, int num_kv_heads, int d, int page_size,
    int max_blocks_per_seq, int64_t num_blocks, const float* k_signs, const float* v_signs, const float* k_levels,
    const float* v_levels, int bits_k, int bits_v, float scale, int num_splits, void* workspace,
    int64_t workspace_bytes, void* out, int out_dtype, void* stream) {
  FTQ_REQUIRE(d == 128, "fp32 VALU paged attention: head_dim must be 128");
  FTQ_REQUIRE(num_kv_heads > 0 && num_q_heads % num_kv_heads == 0 && num_q_heads / num_kv_heads <= 4,
              "fp32 VALU paged attention: at most 4 query heads per kv head");
  AttnArgs a;
  const int rc = paged_attn_args(a, query, q_dtype, kv_cache, block_table, seq_lens, batch, num_q_heads,
                                 num_kv_heads, d, page_size, max_blocks_per_seq, num_blocks, k_signs, v_signs,
                                 k_levels, v_levels, bits_k, bits_v, scale, num_splits, workspace,
                                 workspace_bytes, out, out_dtype);
  if (rc != FTQ_OK || batch == 0) return rc;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (bits_k == 2) e = launch_attn_valu2<2>(bits_v, a, st);
  else if (bits_k == 3) e = launch_attn_valu2<3>(bits_v, a, st);
  else e = launch_attn_valu2<4>(bits_v, a, st);
  return hip_status(e);
}
