// Raw fp16 KV slots of the vLLM TURBOQUANT backend's boundary layers: store
// and split-K decode attention.
//
// Boundary-protection layers (reference vllm_plugin/v1_backend.py:1446-1545,
// triton_boundary_attn.py:28-219) keep K and V unquantised in the same
// [num_blocks][block_size][Hkv][slot] byte allocation as the TurboQuant layers,
// per (token, kv head):
//   [K fp16 (2 D bytes)][V fp16 (2 D bytes)][pad]
// Store: K and V rounded to fp16 (.to(float16), round to nearest even);
// negative slot entries are skipped.
// Decode: o = softmax(q . K^T * scale) . V over positions [kv_start, seq_len).
//
// Decode kernel: one workgroup (4 waves) per (batch, kv head, split); a wave
// walks 16-token tiles of one page.
//   S^T[t][h] = K[t][:] . Q^T[:][h]   v_mfma_f32_16x16x32_f16, A = the fp16 K
//                rows straight from the cache (lane (m, g): token m, dims
//                32 s + 8 g .. +7), B = the query of the GQA group as f16 hi + lo
//                (scale * log2 e folded), so the product keeps ~22 bits
//   O[h][d]  += p[h][t] V[t][d]       VALU: lane (m, g) owns dims 8 m .. 8 m + 7
//                of the tokens t = 4 k + g of the tile; p goes from the score
//                layout to this one through LDS
// Online softmax in the log2 domain with lazy rescaling (the reference max is
// raised only when a tile exceeds it by 2^8).  The 4 waves merge through LDS;
// the splits merge in merge_splits_kernel (ROT_NONE), which writes the output
// dtype.  HBM-bound: 4 D bytes per (token, kv head).
#include "ftq_attn_dev.h"
#include "ftq_device.h"
#include "ftq_internal.h"
#include "ftq_merge.h"
#include "ftq_v1_dev.h"

namespace ftq {

int auto_splits(int batch, int hkv, int seq_hint, int target_wgs);

// ---------------------------------------------------------------------------
// store
// ---------------------------------------------------------------------------

// One (token, kv head) per 16 lanes, D/16 contiguous elements per lane.
template <int D, int DT>
__global__ __launch_bounds__(256) void raw_store_kernel(const void* __restrict__ key,
                                                        const void* __restrict__ value, int64_t n_rows,
                                                        int hkv, const int64_t* __restrict__ slot_mapping,
                                                        uint8_t* __restrict__ cache, int64_t num_blocks,
                                                        int block_size, int64_t s_blk, int64_t s_pos,
                                                        int64_t s_head) {
  constexpr int E = D / 16;
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int l16 = threadIdx.x & 15;
  if (row >= n_rows) return;
  const int64_t tok = row / hkv;
  const int h = (int)(row - tok * hkv);
  const int64_t slot = slot_mapping[tok];
  if (slot < 0) return;
  const int64_t blk = slot / block_size, pos = slot - blk * block_size;
  if (blk >= num_blocks) return;
  uint8_t* dst = cache + blk * s_blk + pos * s_pos + h * s_head;
#pragma unroll
  for (int kv = 0; kv < 2; ++kv) {
    float x[E];
    load_elems<DT, E>(kv ? value : key, row * D + l16 * E, x);
    uint32_t w[E / 2];
#pragma unroll
    for (int i = 0; i < E / 2; ++i) w[i] = f32_to_f16_bits(x[2 * i]) | (f32_to_f16_bits(x[2 * i + 1]) << 16);
    uint32_t* p = reinterpret_cast<uint32_t*>(dst + kv * 2 * D + l16 * E * 2);
    if constexpr (E == 8) {
      *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
#pragma unroll
      for (int i = 0; i < E / 2; ++i) p[i] = w[i];
    }
  }
}

// ---------------------------------------------------------------------------
// decode attention, stage 1 (per split)
// ---------------------------------------------------------------------------

struct RawTile {
  uint32_t k[4][4];  // K operand per MFMA step s: token m, dims 32 s + 8 g .. +7 (f16)
  uint32_t v[4][4];  // V rows: token 4 k + g, dims 8 m .. 8 m + 7 (f16)
  bool ok;           // the tile's page is in range
};

struct RawAddr {
  const uint8_t* cache;
  __amdgpu_buffer_rsrc_t bt_rs;  // the sequence's block-table row as a buffer
  int64_t s_blk, kvh_off;
  uint32_t s_pos;
  int lbs, max_blocks, seq_len, nb32;  // nb32 = min(num_blocks, 2^31 - 1)
  uint32_t koff, voff;  // lane offsets in the tile's descriptor
};

// Block-table entry of a 16-token tile, as a vector load issued one tile
// ahead of the loads that need it (-1 when inactive, past seq_len or past the
// row).  A vector load retires in order, so the wait before raw_load's
// readfirstlane covers only this load.
__device__ __forceinline__ int raw_fetch_bt(const RawAddr& ad, int tile, bool active) {
  const int pos0 = tile * 16;
  const int page = pos0 >> ad.lbs;
  const bool ok = active && pos0 < ad.seq_len && page < ad.max_blocks;
  const int v = (int)__builtin_amdgcn_raw_buffer_load_b32(ad.bt_rs, (uint32_t)(ok ? page : 0) * 4u, 0, 0);
  return ok ? v : -1;
}

// Loads of one 16-token tile through one wave-uniform buffer descriptor (its
// page base; the byte range ends after its 16 token rows, so no lane reads past
// them).  A tile past the sequence or on a bad block id reads block 0 instead
// -- the loads always issue, so the wait counts stay static -- and the
// consumer masks it.
template <int D>
__device__ __forceinline__ void raw_load(RawTile& r, const RawAddr& ad, int tile, int btv) {
  const int pos0 = tile * 16;
  int phys = __builtin_amdgcn_readfirstlane(btv);
  const bool valid = (uint32_t)phys < (uint32_t)ad.nb32;  // -1 (no entry) and ids >= num_blocks fail
  if (!valid) phys = 0;
  const uint32_t within = valid ? (uint32_t)(pos0 & ((1 << ad.lbs) - 1)) : 0u;
  const uint8_t* base = ad.cache + ((int64_t)phys * ad.s_blk + (int64_t)(within * ad.s_pos) + ad.kvh_off);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, (int)(16u * ad.s_pos), 0x00020000);
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const uint4 x = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, ad.koff + 64u * s, 0, 0));
    r.k[s][0] = x.x; r.k[s][1] = x.y; r.k[s][2] = x.z; r.k[s][3] = x.w;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint4 x = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, ad.voff, 4u * k * ad.s_pos, 0));
    r.v[k][0] = x.x; r.v[k][1] = x.y; r.v[k][2] = x.z; r.v[k][3] = x.w;
  }
  r.ok = valid;
}

__device__ __forceinline__ void raw_lds_fence() {
  // LDS accesses of one wave execute in order; only the compiler must not
  // reorder them across this point
  __asm__ volatile("" ::: "memory");
}

// GP = the GQA group size rounded up to a power of two (<= 8): P.V accumulators
// per lane are GP x 8 floats.
template <int D, int GP, int QT>
__global__ __launch_bounds__(256) void raw_attn_kernel(
    const void* __restrict__ query, const uint8_t* __restrict__ cache,
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ seq_lens,
    const int32_t* __restrict__ kv_start, int hq, int hkv, int lbs, int max_blocks,
    int64_t num_blocks, int64_t s_blk, int64_t s_pos, int64_t s_head, float qscale, int num_splits,
    float* __restrict__ ws_o, float* __restrict__ ws_lse) {
  static_assert(D == 128, "raw decode attention covers head_dim 128");
  static_assert(GP == 1 || GP == 2 || GP == 4 || GP == 8, "GQA group padded to 1, 2, 4 or 8");
  const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z;
  const int G = hq / hkv;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m = lane & 15, g = lane >> 4;

  __shared__ __attribute__((aligned(16))) float p_l[4][16][GP];   // per wave: p[token][head] of a tile
  __shared__ __attribute__((aligned(16))) float alpha_l[4][GP];   // per wave: rescale factors
  __shared__ float red_m[4][GP], red_l[4][GP];
  __shared__ float red_o[4][GP][D + 1];

  // B operand of the score MFMAs (f16 hi + lo): lane (n = m, g), step s ->
  // Q[n][32 s + 8 g .. +7] * qscale; columns n >= G stay zero
  Op8 qb[4], ql[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    float x[8];
    if (m < G) {
      load_elems<QT, 8>(query, ((int64_t)b * hq + kvh * G + m) * D + 32 * s + 8 * g, x);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = 0.f;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t wh = 0, wl = 0;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float y = x[2 * j + e] * qscale;
        const _Float16 hi = (_Float16)y;
        const _Float16 lo = (_Float16)(y - (float)hi);
        wh |= (uint32_t)__builtin_bit_cast(uint16_t, hi) << (16 * e);
        wl |= (uint32_t)__builtin_bit_cast(uint16_t, lo) << (16 * e);
      }
      qb[s].u[j] = wh;
      ql[s].u[j] = wl;
    }
  }

  const int seq_len = seq_lens[b];
  int k0 = kv_start ? kv_start[b] : 0;
  if (k0 < 0) k0 = 0;
  const int t_first = k0 >> 4;
  const int t_last = (seq_len + 15) >> 4;
  const int n_tiles = t_last > t_first ? t_last - t_first : 0;
  const int tps = (n_tiles + num_splits - 1) / num_splits;
  const int t_begin = t_first + split * tps;
  const int t_end = min(t_begin + tps, t_last);
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);

  RawAddr ad;
  ad.cache = cache;
  ad.bt_rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<int32_t*>(block_table + (int64_t)b * max_blocks),
                                               (short)0, (int)min((int64_t)max_blocks * 4, (int64_t)0x7ffffffc),
                                               0x00020000);
  ad.nb32 = (int)min(num_blocks, (int64_t)0x7fffffff);
  ad.s_blk = s_blk;
  ad.kvh_off = (int64_t)kvh * s_head;
  ad.s_pos = (uint32_t)s_pos;
  ad.lbs = lbs;
  ad.max_blocks = max_blocks;
  ad.seq_len = seq_len;
  ad.koff = (uint32_t)m * ad.s_pos + 16u * (uint32_t)g;
  ad.voff = (uint32_t)g * ad.s_pos + 2u * D + 16u * (uint32_t)m;

  // score layout: lane (m, g) holds head m, tokens 4 g + i; its m_run / l_run
  // are head m's (l_run a partial sum over its tokens)
  float m_run = -INFINITY, l_run = 0.f;
  float acc[GP][8];
#pragma unroll
  for (int h = 0; h < GP; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;

  constexpr float TAU = 8.f;  // p <= 2^TAU
  auto process = [&](const RawTile& cur, int tile) __attribute__((always_inline)) {
    floatx4 sacc = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      Op8 a;
      a.u[0] = cur.k[s][0]; a.u[1] = cur.k[s][1]; a.u[2] = cur.k[s][2]; a.u[3] = cur.k[s][3];
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, qb[s].h, sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.h, ql[s].h, sacc, 0, 0, 0);
    }
    float s4[4] = {sacc[0], sacc[1], sacc[2], sacc[3]};
    // positions outside [k0, seq_len) and tiles without a page
    if (tile * 16 < k0 || tile * 16 + 16 > seq_len || !cur.ok) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int pos = tile * 16 + 4 * g + i;
        if (pos >= seq_len || pos < k0 || !cur.ok) s4[i] = -INFINITY;
      }
    }
    const float tmax = warp_max_q(fmaxf(fmaxf(s4[0], s4[1]), fmaxf(s4[2], s4[3])));
    if (__builtin_amdgcn_ballot_w64(tmax > m_run + TAU) != 0) {  // wave-uniform, rare
      const float m_new = fmaxf(m_run, tmax);
      const float alpha = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
      if (g == 0 && m < GP) alpha_l[wave][m] = alpha;
      raw_lds_fence();
#pragma unroll
      for (int h = 0; h < GP; ++h) {
        const float ah = alpha_l[wave][h];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] *= ah;
      }
      raw_lds_fence();
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // a masked score (or a head that has seen no position yet) weighs 0
      p[i] = (s4[i] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(s4[i] - m_run);
      l_run += p[i];
    }
    if (m < GP) {
#pragma unroll
      for (int i = 0; i < 4; ++i) p_l[wave][4 * g + i][m] = p[i];
    }
    raw_lds_fence();
    // P.V: lane (m, g) accumulates tokens 4 k + g, dims 8 m .. 8 m + 7
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float pk[GP];
      if constexpr (GP >= 4) {
#pragma unroll
        for (int h4 = 0; h4 < GP; h4 += 4) {
          const float4 q4 = *reinterpret_cast<const float4*>(&p_l[wave][4 * k + g][h4]);
          pk[h4] = q4.x; pk[h4 + 1] = q4.y; pk[h4 + 2] = q4.z; pk[h4 + 3] = q4.w;
        }
      } else {
#pragma unroll
        for (int h = 0; h < GP; ++h) pk[h] = p_l[wave][4 * k + g][h];
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const half2_t v2 = __builtin_bit_cast(half2_t, cur.v[k][j]);
        const float v0 = (float)v2[0], v1 = (float)v2[1];
#pragma unroll
        for (int h = 0; h < GP; ++h) {
          acc[h][2 * j] = __builtin_fmaf(pk[h], v0, acc[h][2 * j]);
          acc[h][2 * j + 1] = __builtin_fmaf(pk[h], v1, acc[h][2 * j + 1]);
        }
      }
    }
    raw_lds_fence();
  };

  // two register sets: the next tile's loads overlap this tile's math, and
  // the block-table entry comes one tile further ahead
  RawTile ra, rb;
  int tile = t_begin + wave_u;
  int btv = 0;
  if (tile < t_end) {
    raw_load<D>(ra, ad, tile, raw_fetch_bt(ad, tile, true));
    btv = raw_fetch_bt(ad, tile + 4, tile + 4 < t_end);
  }
  while (tile < t_end) {
    int btn = raw_fetch_bt(ad, tile + 8, tile + 8 < t_end);
    raw_load<D>(rb, ad, tile + 4, btv);
    btv = btn;
    process(ra, tile);
    tile += 4;
    if (tile >= t_end) break;
    btn = raw_fetch_bt(ad, tile + 8, tile + 8 < t_end);
    raw_load<D>(ra, ad, tile + 4, btv);
    btv = btn;
    process(rb, tile);
    tile += 4;
  }

  // ---- merge the 4 waves through LDS ----
  const float l_tot = warp_sum_q(l_run);
  if (g == 0 && m < GP) {
    red_m[wave][m] = m_run;
    red_l[wave][m] = l_tot;
  }
  // the 4 lanes of a dim block (g = 0..3) hold disjoint token sets: sum them
#pragma unroll
  for (int h = 0; h < GP; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = warp_sum_q(acc[h][e]);
      if (g == 0) red_o[wave][h][8 * m + e] = x;
    }
  __syncthreads();

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
        const float f = red_m[w][gg] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(red_m[w][gg] - M);
        L += f * red_l[w][gg];
        o += f * red_o[w][gg][d];
      }
    }
    const int64_t row = row0 + (int64_t)gg * num_splits;
    ws_o[row * D + d] = (L > 0.f) ? o / L : 0.f;
    if (d == 0) ws_lse[row] = (L > 0.f) ? M + __builtin_log2f(L) : -INFINITY;
  }
}

struct RawArgs {
  const void* q;
  int qt;
  const uint8_t* cache;
  const int32_t* bt;
  const int32_t* sl;
  const int32_t* ks;
  int B, hq, hkv, lbs, max_blocks;
  int64_t nb, sblk, spos, shead;
  float qscale;
  int splits;
  float *wo, *wl;
  void* out;
  int ot;
  float* lse;  // optional per-row natural-log LSE (B*Hq floats)
};

template <int GP, int QT>
static hipError_t raw_launch_q(const RawArgs& a, hipStream_t st) {
  dim3 grid((unsigned)a.splits, (unsigned)a.hkv, (unsigned)a.B), block(256);
  raw_attn_kernel<128, GP, QT><<<grid, block, 0, st>>>(a.q, a.cache, a.bt, a.sl, a.ks, a.hq, a.hkv, a.lbs,
                                                        a.max_blocks, a.nb, a.sblk, a.spos, a.shead, a.qscale,
                                                        a.splits, a.wo, a.wl);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t rows = (int64_t)a.B * a.hq;
  if (a.ot == F32) return launch_merge_splits<128, F32, ROT_NONE>(a.wo, a.wl, rows, a.splits, nullptr, 1.f, a.out, st, a.lse);
  if (a.ot == F16) return launch_merge_splits<128, F16, ROT_NONE>(a.wo, a.wl, rows, a.splits, nullptr, 1.f, a.out, st, a.lse);
  return launch_merge_splits<128, BF16, ROT_NONE>(a.wo, a.wl, rows, a.splits, nullptr, 1.f, a.out, st, a.lse);
}

template <int GP>
static hipError_t raw_launch_g(const RawArgs& a, hipStream_t st) {
  if (a.qt == F32) return raw_launch_q<GP, F32>(a, st);
  if (a.qt == F16) return raw_launch_q<GP, F16>(a, st);
  return raw_launch_q<GP, BF16>(a, st);
}

}  // namespace ftq

using namespace ftq;

extern "C" int64_t ftq_raw_slot_bytes(int d) {
  if (d != 64 && d != 128 && d != 256) return -1;
  return 4 * (int64_t)d;
}

extern "C" int ftq_raw_store(const void* key, const void* value, int dtype, int64_t n_tokens,
                             int num_kv_heads, int d, const int64_t* slot_mapping, uint8_t* kv_cache,
                             int64_t num_blocks, int block_size, int64_t stride_block,
                             int64_t stride_pos, int64_t stride_head, void* stream) {
  FTQ_REQUIRE(d == 64 || d == 128 || d == 256, "raw store: head_dim must be 64, 128 or 256");
  FTQ_REQUIRE(dtype >= F32 && dtype <= BF16, "dtype must be FTQ_F32, FTQ_F16 or FTQ_BF16");
  FTQ_REQUIRE(n_tokens >= 0 && num_kv_heads > 0 && num_blocks >= 0 && block_size > 0,
              "bad token / head / block counts");
  FTQ_REQUIRE(stride_head >= 4 * (int64_t)d, "stride_head is smaller than the raw slot (4 * head_dim bytes)");
  FTQ_REQUIRE(cache_strides_ok(num_blocks, stride_block, stride_pos, stride_head, num_kv_heads, block_size),
              "kv_cache strides must describe [num_blocks][block_size][num_kv_heads][slot]");
  FTQ_REQUIRE(stride_head % 16 == 0 && stride_pos % 16 == 0 && stride_block % 16 == 0,
              "kv_cache strides must be multiples of 16 bytes");
  if (n_tokens == 0) return FTQ_OK;
  FTQ_REQUIRE(key && value && slot_mapping && kv_cache, "null pointer argument");
  FTQ_REQUIRE(aligned16(key) && aligned16(value) && aligned16(kv_cache),
              "key, value and kv_cache must be 16-byte aligned");
  const int64_t rows = n_tokens * num_kv_heads;
  dim3 grid((unsigned)((rows + 15) / 16)), block(256);
  hipStream_t st = (hipStream_t)stream;
#define FTQ_RAW_STORE(DD, TT)                                                                              \
  raw_store_kernel<DD, TT><<<grid, block, 0, st>>>(key, value, rows, num_kv_heads, slot_mapping, kv_cache, \
                                                   num_blocks, block_size, stride_block, stride_pos, stride_head)
  if (d == 64) {
    if (dtype == F32) FTQ_RAW_STORE(64, F32); else if (dtype == F16) FTQ_RAW_STORE(64, F16); else FTQ_RAW_STORE(64, BF16);
  } else if (d == 128) {
    if (dtype == F32) FTQ_RAW_STORE(128, F32); else if (dtype == F16) FTQ_RAW_STORE(128, F16); else FTQ_RAW_STORE(128, BF16);
  } else {
    if (dtype == F32) FTQ_RAW_STORE(256, F32); else if (dtype == F16) FTQ_RAW_STORE(256, F16); else FTQ_RAW_STORE(256, BF16);
  }
#undef FTQ_RAW_STORE
  return hip_status(hipGetLastError());
}

extern "C" int64_t ftq_raw_workspace_bytes(int batch, int num_q_heads, int d, int num_splits) {
  if (num_q_heads <= 0) return -1;
  return split_workspace_bytes(batch, num_q_heads, d, num_splits);
}

extern "C" int ftq_raw_default_splits(int batch, int num_kv_heads, int max_seq_len) {
  // tiles are 16 tokens here (32 in the packed formats): same fill target
  return auto_splits(batch, num_kv_heads, max_seq_len / 2, 1024);
}

extern "C" int ftq_raw_decode_attention_lse(
    const void* query, int q_dtype, const uint8_t* kv_cache, int64_t num_blocks, int block_size,
    int64_t stride_block, int64_t stride_pos, int64_t stride_head, const int32_t* block_table,
    int max_blocks_per_seq, const int32_t* seq_lens, const int32_t* kv_start, int batch,
    int num_q_heads, int num_kv_heads, int d, float scale, int num_splits, void* workspace,
    int64_t workspace_bytes, void* out, int out_dtype, float* lse_out, void* stream) {
  FTQ_REQUIRE(d == 64 || d == 128 || d == 256, "raw decode attention: head_dim must be 64, 128 or 256");
  FTQ_REQUIRE(block_size >= 16 && block_size <= 4096 && (block_size & (block_size - 1)) == 0,
              "block_size must be a power of two in [16, 4096]");
  FTQ_REQUIRE(batch >= 0 && num_kv_heads > 0 && num_q_heads > 0 && num_blocks >= 0,
              "bad batch / head / block counts");
  FTQ_REQUIRE(num_q_heads % num_kv_heads == 0, "num_q_heads must be a multiple of num_kv_heads");
  FTQ_REQUIRE(num_q_heads / num_kv_heads <= (d == 128 ? 8 : 16),
              "raw decode attention: GQA group must be <= 8 at head_dim 128, <= 16 otherwise");
  FTQ_REQUIRE(num_splits >= 1 && num_splits <= 1024, "num_splits must be in [1, 1024]");
  FTQ_REQUIRE(max_blocks_per_seq >= 0, "max_blocks_per_seq must be >= 0");
  FTQ_REQUIRE(q_dtype >= F32 && q_dtype <= BF16 && out_dtype >= F32 && out_dtype <= BF16,
              "dtype must be FTQ_F32, FTQ_F16 or FTQ_BF16");
  FTQ_REQUIRE(stride_head >= 4 * (int64_t)d, "stride_head is smaller than the raw slot (4 * head_dim bytes)");
  FTQ_REQUIRE(cache_strides_ok(num_blocks, stride_block, stride_pos, stride_head, num_kv_heads, block_size),
              "kv_cache strides must describe [num_blocks][block_size][num_kv_heads][slot]");
  FTQ_REQUIRE(stride_head % 16 == 0 && stride_pos % 16 == 0 && stride_block % 16 == 0,
              "kv_cache strides must be multiples of 16 bytes");
  FTQ_REQUIRE(stride_pos * 16 < ((int64_t)1 << 31), "stride_pos too large");
  if (batch == 0) return FTQ_OK;
  FTQ_REQUIRE(num_blocks >= 1, "kv_cache must hold at least one block");
  FTQ_REQUIRE(query && kv_cache && block_table && seq_lens && workspace && out, "null pointer argument");
  FTQ_REQUIRE(workspace_bytes >= ftq_raw_workspace_bytes(batch, num_q_heads, d, num_splits),
              "workspace too small (see ftq_raw_workspace_bytes)");
  FTQ_REQUIRE(aligned16(query) && aligned16(out) && aligned16(workspace) && aligned16(kv_cache),
              "query, out, workspace and kv_cache must be 16-byte aligned");
  if (d != 128) {  // head_dim 64 / 256: the fp32 VALU kernel over the same slots
    V1Args v;
    v.q = query; v.qt = q_dtype; v.cache = kv_cache; v.bt = block_table; v.sl = seq_lens; v.ks = kv_start;
    v.B = batch; v.hq = num_q_heads; v.hkv = num_kv_heads; v.max_blocks = max_blocks_per_seq;
    v.lbs = 0;
    while ((1 << v.lbs) < block_size) ++v.lbs;
    v.nb = num_blocks; v.sblk = stride_block; v.spos = stride_pos; v.shead = stride_head;
    v.cent = nullptr; v.qscale = scale * 1.4426950408889634f; v.splits = num_splits; v.vrot = 0;
    v.wo = static_cast<float*>(workspace);
    v.wl = v.wo + (int64_t)batch * num_q_heads * num_splits * d;
    v.out = out; v.ot = out_dtype; v.lse = lse_out; v.rot = nullptr;
    return hip_status(raw_valu_launch(v, d, (hipStream_t)stream));
  }
  RawArgs a;
  a.q = query; a.qt = q_dtype; a.cache = kv_cache; a.bt = block_table; a.sl = seq_lens; a.ks = kv_start;
  a.B = batch; a.hq = num_q_heads; a.hkv = num_kv_heads; a.max_blocks = max_blocks_per_seq;
  a.lbs = 0;
  while ((1 << a.lbs) < block_size) ++a.lbs;
  a.nb = num_blocks; a.sblk = stride_block; a.spos = stride_pos; a.shead = stride_head;
  a.qscale = scale * 1.4426950408889634f;
  a.splits = num_splits;
  a.wo = static_cast<float*>(workspace);
  a.wl = a.wo + (int64_t)batch * num_q_heads * num_splits * d;
  a.out = out; a.ot = out_dtype; a.lse = lse_out;
  const int G = num_q_heads / num_kv_heads;
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (G == 1) e = raw_launch_g<1>(a, st);
  else if (G == 2) e = raw_launch_g<2>(a, st);
  else if (G <= 4) e = raw_launch_g<4>(a, st);
  else e = raw_launch_g<8>(a, st);
  return hip_status(e);
}

extern "C" int ftq_raw_decode_attention(
    const void* query, int q_dtype, const uint8_t* kv_cache, int64_t num_blocks, int block_size,
    int64_t stride_block, int64_t stride_pos, int64_t stride_head, const int32_t* block_table,
    int max_blocks_per_seq, const int32_t* seq_lens, const int32_t* kv_start, int batch,
    int num_q_heads, int num_kv_heads, int d, float scale, int num_splits, void* workspace,
    int64_t workspace_bytes, void* out, int out_dtype, void* stream) {
  return ftq_raw_decode_attention_lse(query, q_dtype, kv_cache, num_blocks, block_size, stride_block, stride_pos,
                                      stride_head, block_table, max_blocks_per_seq, seq_lens, kv_start, batch,
                                      num_q_heads, num_kv_heads, d, scale, num_splits, workspace, workspace_bytes,
                                      out, out_dtype, nullptr, stream);
}
