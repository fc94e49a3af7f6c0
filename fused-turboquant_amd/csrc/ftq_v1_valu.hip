// vLLM v1 TURBOQUANT slot decode attention with fp32 products on the VALU:
// the reference's arithmetic (reference vllm_plugin/triton_decode_offset.py:
// 42-442, every product and sum in fp32), for every slot format the store
// writes -- head_dim 64, 128 or 256; K codes of 1, 2, 3, 4 or 8 bits or fp8
// e4m3fn keys; V codes of 1, 2, 3, 4 or 8 bits, uniform or Lloyd-Max (4-bit).
// The matrix-core kernels of ftq_v1.hip cover head_dim 128 with 2-4 bit codes
// at f16 operand precision; this kernel is the path for everything else, and
// for callers that ask for fp32 products.  The same kernel reads the raw fp16
// [K | V] slots of the boundary layers (KB = VB = 16: no codes, no norms, no
// rotation; reference triton_boundary_attn.py:28-219) at head_dim 64 and 256,
// where ftq_raw.hip's matrix-core kernel covers 128.
//
// Per split (one workgroup of 4 waves per (batch, kv head, group of <= 4 query
// heads, split)); a wave takes every 4th 16-token S-tile of the split.
//   scores:  lane (m, g) = token m of the S-tile, dims [g D/4, (g+1) D/4):
//            sum_d q[h][d] c[code_d] (4 heads) and sum_d c[code_d]^2 in fp32
//            FMAs, c from an LDS table (32 copies, lane l reads copy l % 32:
//            one bank per lane); the four quarter sums meet over lanes m,
//            m + 16, m + 32, m + 48.  s = ||k||_16 * dot / sqrt(sum c^2 +
//            1e-16) (norm correction, :210-242), or for fp8 keys the plain
//            dot with the fp8 values (:174-192).  The query is rotated and
//            scaled (scale * log2 e) in the prologue.
//   softmax: log2 domain, per head, lazily rescaled (the running max is only
//            raised when a tile exceeds it by 2^8).  Lane (m, g) forms the
//            weight of head g for token m: w = p * scale (uniform V; sum p *
//            min is kept aside) or p * ||v|| / sqrt(sum c[vcode]^2 + 1e-16)
//            (Lloyd-Max V, :399-419), and passes it through LDS.
//   P.V:     lane (dg, tg): dims [8 dg, 8 dg + 8) of tokens tg * TPL ...,
//            TPL = D / 32 tokens per S-tile; acc[dim][head] += w * code (or
//            w * c[code]); summed over the token groups after the last tile.
// Waves merge through LDS; the split merge, the V un-rotation and the output
// cast are merge_splits_kernel (ftq_merge.h), as for the matrix-core kernels.
#include "ftq_attn_dev.h"
#include "ftq_internal.h"
#include "ftq_merge.h"
#include "ftq_v1_dev.h"

#include <cmath>

namespace ftq {

float fwht_scale(int d);

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int NW = 4;  // waves per workgroup
constexpr int GM = 4;  // query heads per workgroup

// fp8 e4m3fn byte -> fp32: sign, 4-bit exponent (bias 7), 3-bit mantissa;
// exponent 0 holds the subnormals m * 2^-9; 0x7f / 0xff are NaN
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  const uint32_t e = (b >> 3) & 15u, m = b & 7u;
  float v;
  if (e == 0) v = (float)m * (1.f / 512.f);
  else if (e == 15 && m == 7) v = __builtin_nanf("");
  else v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return (b & 0x80u) ? -v : v;
}

// bits [i * B, i * B + B) of a little-endian dword array (i compile-time after unrolling)
template <int B, int N>
__device__ __forceinline__ uint32_t code_at(const uint32_t (&w)[N], int i) {
  const int p = i * B, k = p >> 5, o = p & 31;
  uint32_t x = w[k] >> o;
  if (o + B > 32) x |= w[k + 1] << (32 - o);
  return B == 32 ? x : (x & ((1u << B) - 1u));
}

// NB bytes at byte offset `off` of a buffer: whole dwords when NB % 4 == 0 and
// the offset is a multiple of 4 (A4), else 16-bit loads (NB even, offset
// even), else bytes
template <int NB, bool A4>
__device__ __forceinline__ void load_bytes(__amdgpu_buffer_rsrc_t rs, uint32_t off, uint32_t (&w)[(NB + 3) / 4]) {
  constexpr int N = (NB + 3) / 4;
  if constexpr (A4 && NB % 4 == 0) {
    int k = 0;
#pragma unroll
    for (; k + 4 <= N; k += 4) {
      const uint4 x = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs, off + 4u * k, 0, 0));
      w[k] = x.x; w[k + 1] = x.y; w[k + 2] = x.z; w[k + 3] = x.w;
    }
    if constexpr (N % 4 == 3) {
      typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
      const u32x3 x = __builtin_bit_cast(u32x3, __builtin_amdgcn_raw_buffer_load_b96(rs, off + 4u * k, 0, 0));
      w[k] = x.x; w[k + 1] = x.y; w[k + 2] = x.z;
    } else if constexpr (N % 4 == 2) {
      const uint2 x = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rs, off + 4u * k, 0, 0));
      w[k] = x.x; w[k + 1] = x.y;
    } else if constexpr (N % 4 == 1) {
      w[k] = __builtin_amdgcn_raw_buffer_load_b32(rs, off + 4u * k, 0, 0);
    }
  } else if constexpr (NB % 2 == 0) {
#pragma unroll
    for (int k = 0; k < N; ++k) w[k] = 0;
#pragma unroll
    for (int h = 0; h < NB / 2; ++h)
      w[h >> 1] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, off + 2u * h, 0, 0) << (16 * (h & 1));
  } else {
#pragma unroll
    for (int k = 0; k < N; ++k) w[k] = 0;
#pragma unroll
    for (int h = 0; h < NB; ++h)
      w[h >> 2] |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rs, off + (uint32_t)h, 0, 0) << (8 * (h & 3));
  }
}

template <int D, int KB, int VB, bool KF8, bool VLM>
struct VGeo {
  static constexpr bool RAW = KB == 16;      // raw fp16 K and V: [K 2D bytes][V 2D bytes]
  static constexpr V1Geom G = RAW ? V1Geom{2 * D, 2 * D, 2 * D, 4 * D} : v1_geom(D, KB, VB, KF8);
  static constexpr bool VA4 = RAW;           // V chunks at 4-byte aligned offsets
  static constexpr int KQ = D * KB / 32;     // K bytes of one quarter of a vector
  static constexpr int KQW = (KQ + 3) / 4;
  static constexpr int DG = D / 8;           // P.V dim groups (8 dims each)
  static constexpr int TG = 64 / DG;         // P.V token groups
  static constexpr int TPL = 16 / TG;        // tokens of one S-tile per P.V lane
  static constexpr int VW = (VB * 8 + 31) / 32;  // dwords of one token's 8 V codes
  static constexpr int VTB = D / 8;          // Lloyd-Max V: V code bytes of one quarter (4-bit codes)
  static constexpr int VTW = VLM ? (VTB + 3) / 4 : 1;
  static constexpr int KTB = RAW ? 0 : KF8 ? 8 : KB;  // bits of a K table index (no table for raw K)
  static constexpr int QG = D + 4;           // floats per query quarter (4 heads x D/4 dims, padded)
};

template <int D, int KB, int VB, bool KF8, bool VLM>
struct VTile {
  using Q = VGeo<D, KB, VB, KF8, VLM>;
  uint32_t k[Q::KQW];
  uint32_t v[Q::TPL][Q::VW];
  uint32_t vt[Q::VTW];
  uint32_t kn, vs, vm;  // f16 bits of token m's K norm, V scale (or norm), V min
  bool ok;              // wave-uniform: the S-tile has a real page
};

template <int D, int KB, int VB, bool KF8, bool VLM>
__device__ __forceinline__ void vtile_load(VTile<D, KB, VB, KF8, VLM>& r, const uint8_t* cache, int phys, bool ok,
                                           uint32_t within, int64_t s_blk, uint32_t s_pos, int64_t kvh_off,
                                           int lane) {
  using Q = VGeo<D, KB, VB, KF8, VLM>;
  const int m = lane & 15, g = lane >> 4;
  const int dg = lane % Q::DG, tg = lane / Q::DG;
  if (!ok) { phys = 0; within = 0; }
  const uint8_t* bst = cache + ((int64_t)phys * s_blk + (int64_t)within * s_pos + kvh_off);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(bst), (short)0, (int)(16u * s_pos), 0x00020000);
  const uint32_t row = (uint32_t)m * s_pos;
  load_bytes<Q::KQ, true>(rs, row + (uint32_t)(g * Q::KQ), r.k);
  if constexpr (Q::RAW) {
    r.kn = r.vs = r.vm = 0u;
  } else {
    r.kn = KF8 ? 0u : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, row + Q::G.mse, 0, 0);
    r.vs = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, row + Q::G.kps + Q::G.vdb, 0, 0);
    r.vm = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, row + Q::G.kps + Q::G.vdb + 2, 0, 0);
  }
  if constexpr (VLM) load_bytes<Q::VTB, false>(rs, row + Q::G.kps + (uint32_t)(g * Q::VTB), r.vt);
#pragma unroll
  for (int i = 0; i < Q::TPL; ++i) {
    const uint32_t t = (uint32_t)(tg * Q::TPL + i);
    load_bytes<VB, Q::VA4>(rs, t * s_pos + Q::G.kps + (uint32_t)(dg * VB), r.v[i]);
  }
  r.ok = ok;
}

template <int D, int KB, int VB, bool KF8, bool VLM>
__global__ __launch_bounds__(256, 2) void v1_attn_valu_kernel(
    const void* __restrict__ query, int qt, const uint8_t* __restrict__ cache,
    const int32_t* __restrict__ block_table, const int32_t* __restrict__ seq_lens,
    const int32_t* __restrict__ kv_start, int hq, int hkv, int lbs, int max_blocks, int64_t num_blocks,
    int64_t s_blk, int64_t s_pos, int64_t s_head, const float* __restrict__ cent, float qscale,
    int num_splits, float* __restrict__ ws_o, float* __restrict__ ws_lse, const float* __restrict__ rot) {
  using Q = VGeo<D, KB, VB, KF8, VLM>;
  constexpr int E16 = D / 16;                 // query elements per lane in the prologue
  // K table entries; Lloyd-Max V reads it with 4-bit codes, and codes at or
  // above 2^KB (never stored) read the top centroid
  constexpr int NK = Q::RAW ? 0 : (VLM && Q::KTB < 4) ? 16 : 1 << Q::KTB;
  constexpr int TAB_BYTES = NK * 32 * 4;
  constexpr int RED_BYTES = NW * GM * (D + 1) * 4;
  constexpr int ROT_BYTES = GM * D * 4;
  constexpr int P0 = TAB_BYTES > RED_BYTES ? TAB_BYTES : RED_BYTES;
  constexpr int POOL = P0 > ROT_BYTES ? P0 : ROT_BYTES;
  __shared__ __attribute__((aligned(16))) uint8_t pool[POOL];  // K table | prologue rows | wave merge
  __shared__ __attribute__((aligned(16))) float qv[4 * Q::QG];
  __shared__ __attribute__((aligned(16))) float pw[NW][16][GM];
  __shared__ float red_m[NW][GM], red_l[NW][GM];

  const int split = blockIdx.x, b = blockIdx.z;
  const int G = hq / hkv;
  const int hchunks = (G + GM - 1) / GM;
  const int kvh = blockIdx.y / hchunks, hc = blockIdx.y % hchunks;
  const int h0 = hc * GM;                     // first head of the group handled here
  const int nh = min(GM, G - h0);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int m = lane & 15, g = lane >> 4;
  const int dg = lane % Q::DG, tg = lane / Q::DG;

  // ---- prologue: rotated, scaled query of the <= 4 heads (16 lanes each) ----
  if (tid < 64) {
    const int hh = tid >> 4, l16 = tid & 15;
    float y[E16];
    if (hh < nh) {
      const int64_t off = ((int64_t)b * hq + kvh * G + h0 + hh) * D + l16 * E16;
      if (qt == F32) load_elems<F32, E16>(query, off, y);
      else if (qt == F16) load_elems<F16, E16>(query, off, y);
      else load_elems<BF16, E16>(query, off, y);
    } else {
#pragma unroll
      for (int i = 0; i < E16; ++i) y[i] = 0.f;
    }
    if constexpr (!Q::RAW) {  // raw K is not rotated
      if (rot != nullptr) rot_matrix_lanes<D, E16>(y, rot, reinterpret_cast<float*>(pool) + hh * D, l16);
      else fwht_lanes<E16, 16>(y, l16);
    }
#pragma unroll
    for (int i = 0; i < E16; ++i) {
      const int d = l16 * E16 + i, qq = d / (D / 4), di = d % (D / 4);
      qv[qq * Q::QG + di * GM + hh] = y[i] * qscale;
    }
  }
  __syncthreads();  // the prologue rows are dead: the pool takes the K table
  float* ktab = reinterpret_cast<float*>(pool);
  if constexpr (!Q::RAW) {
    for (int e = tid; e < NK * 32; e += NW * 64) {
      const int c = e >> 5;
      ktab[e] = KF8 ? e4m3_to_f32((uint32_t)c) : cent[c < (1 << KB) ? c : (1 << KB) - 1];
    }
    __syncthreads();
  }
  const uint32_t tab = lds_addr(ktab) + 4u * (uint32_t)(lane & 31);
  auto tabv = [&](uint32_t c) __attribute__((always_inline)) {
    return *(__attribute__((address_space(3))) const float*)(uintptr_t)(tab + (c << 7));
  };
  const uint32_t qaddr = lds_addr(qv) + 4u * (uint32_t)(g * Q::QG);

  // ---- the split's S-tiles ----
  const int seq_len = seq_lens[b];
  int k0 = kv_start ? kv_start[b] : 0;
  if (k0 < 0) k0 = 0;
  const int s_first = k0 >> 4;
  const int s_last = (seq_len + 15) >> 4;
  const int n_st = s_last > s_first ? s_last - s_first : 0;
  const int sps = (n_st + num_splits - 1) / num_splits;
  const int st_begin = s_first + split * sps;
  const int st_end = min(st_begin + sps, s_last);
  const int32_t* bt_row = block_table + (int64_t)b * max_blocks;
  const int64_t kvh_off = (int64_t)kvh * s_head;
  const int nb32 = (int)min(num_blocks, (int64_t)0x7fffffff);
  const uint32_t sp32 = (uint32_t)s_pos;
  auto load = [&](VTile<D, KB, VB, KF8, VLM>& r, int j) __attribute__((always_inline)) {
    const int pos0 = j * 16;
    const int page = pos0 >> lbs;
    int phys = page < max_blocks ? bt_row[page] : -1;
    const bool ok = (uint32_t)phys < (uint32_t)nb32;
    vtile_load(r, cache, phys, ok, (uint32_t)(pos0 & ((1 << lbs) - 1)), s_blk, sp32, kvh_off, lane);
  };

  float m_run[GM], l_run = 0.f, z_run = 0.f;
  float acc[8][GM];
#pragma unroll
  for (int h = 0; h < GM; ++h) m_run[h] = -INFINITY;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int h = 0; h < GM; ++h) acc[j][h] = 0.f;
  float* pwl = &pw[wave][0][0];

  constexpr float TAU = 8.f;
  auto process = [&](const VTile<D, KB, VB, KF8, VLM>& cur, int j) __attribute__((always_inline)) {
    // scores of token m, quarter g
    float dot[GM] = {0.f, 0.f, 0.f, 0.f};
    float csq = 0.f;
#pragma unroll
    for (int i = 0; i < D / 4; ++i) {
      float c;
      if constexpr (Q::RAW) c = (float)__builtin_bit_cast(_Float16, (uint16_t)code_at<16>(cur.k, i));
      else c = tabv(code_at<Q::KTB>(cur.k, i));
      const f32x4 q4 = *(__attribute__((address_space(3))) const f32x4*)(uintptr_t)(qaddr + 16u * (uint32_t)i);
      dot[0] = __builtin_fmaf(q4.x, c, dot[0]);
      dot[1] = __builtin_fmaf(q4.y, c, dot[1]);
      dot[2] = __builtin_fmaf(q4.z, c, dot[2]);
      dot[3] = __builtin_fmaf(q4.w, c, dot[3]);
      if constexpr (!KF8 && !Q::RAW) csq = __builtin_fmaf(c, c, csq);
    }
    const int pos = j * 16 + m;
    const bool live = cur.ok && pos >= k0 && pos < seq_len;
    float kf = 1.f;
    if constexpr (!KF8 && !Q::RAW) {
      const float kn = (float)__builtin_bit_cast(_Float16, (uint16_t)cur.kn);
      kf = kn / __builtin_sqrtf(warp_sum_q(csq) + 1e-16f);
    }
    float s[GM];
#pragma unroll
    for (int h = 0; h < GM; ++h) {
      const float t = warp_sum_q(dot[h]) * kf;
      s[h] = live ? t : -INFINITY;
    }
    // V weight factor of token m (lane (m, g) serves head g); zero for tokens
    // that are not attended, whose fields may hold anything
    float wf, zm = 0.f;
    const float vs = (float)__builtin_bit_cast(_Float16, (uint16_t)cur.vs);
    if constexpr (Q::RAW) {
      wf = 1.f;
    } else if constexpr (VLM) {
      float vsq = 0.f;
#pragma unroll
      for (int i = 0; i < D / 4; ++i) {
        const float c = tabv(code_at<4>(cur.vt, i));
        vsq = __builtin_fmaf(c, c, vsq);
      }
      wf = vs / __builtin_sqrtf(warp_sum_q(vsq) + 1e-16f);
    } else {
      wf = vs;
      zm = (float)__builtin_bit_cast(_Float16, (uint16_t)cur.vm);
    }
    if (!live) {
      wf = 0.f;
      zm = 0.f;
    }
    float tmax[GM];
    bool raise = false;
#pragma unroll
    for (int h = 0; h < GM; ++h) {
      float x = s[h];
      x = fmaxf(x, lane_xor<1>(x));
      x = fmaxf(x, lane_xor<2>(x));
      x = fmaxf(x, lane_xor<4>(x));
      tmax[h] = fmaxf(x, lane_xor<8>(x));
      raise = raise || (tmax[h] > m_run[h] + TAU);
    }
    if (__builtin_amdgcn_ballot_w64(raise) != 0) {  // wave-uniform, rare
#pragma unroll
      for (int h = 0; h < GM; ++h) {
        const float m_new = fmaxf(m_run[h], tmax[h]);
        const float al = m_new == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m_run[h] - m_new);
        m_run[h] = m_new;
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) acc[jj][h] *= al;
        if (g == h) {
          l_run *= al;
          z_run *= al;
        }
      }
    }
    const float mg = g == 0 ? m_run[0] : g == 1 ? m_run[1] : g == 2 ? m_run[2] : m_run[3];
    const float sg = g == 0 ? s[0] : g == 1 ? s[1] : g == 2 ? s[2] : s[3];
    const float p = live ? __builtin_amdgcn_exp2f(sg - mg) : 0.f;
    l_run += p;
    z_run = __builtin_fmaf(p, zm, z_run);
    pwl[m * GM + g] = p * wf;
    __asm__ volatile("" ::: "memory");  // a wave's LDS accesses run in order
    // P.V of the lane's tokens, 8 dims each
#pragma unroll
    for (int i = 0; i < Q::TPL; ++i) {
      const f32x4 w4 = *(__attribute__((address_space(3))) const f32x4*)(uintptr_t)(
          lds_addr(pwl) + 16u * (uint32_t)(tg * Q::TPL + i));
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const uint32_t cd = code_at<VB>(cur.v[i], jj);
        float val;
        if constexpr (Q::RAW) val = (float)__builtin_bit_cast(_Float16, (uint16_t)cd);
        else val = VLM ? tabv(cd) : (float)cd;
        acc[jj][0] = __builtin_fmaf(w4.x, val, acc[jj][0]);
        acc[jj][1] = __builtin_fmaf(w4.y, val, acc[jj][1]);
        acc[jj][2] = __builtin_fmaf(w4.z, val, acc[jj][2]);
        acc[jj][3] = __builtin_fmaf(w4.w, val, acc[jj][3]);
      }
    }
    __asm__ volatile("" ::: "memory");
  };

  VTile<D, KB, VB, KF8, VLM> ra, rb;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  int j = st_begin + wave_u;
  if (j < st_end) load(ra, j);
  while (j < st_end) {
    if (j + NW < st_end) load(rb, j + NW);
    process(ra, j);
    j += NW;
    if (j >= st_end) break;
    if (j + NW < st_end) load(ra, j + NW);
    process(rb, j);
    j += NW;
  }

  // ---- wave totals, then the 4 waves merged through LDS ----
  const float l_tot = group_sum<16>(l_run);  // head g over the 16 token lanes
  const float z_tot = group_sum<16>(z_run);
#pragma unroll
  for (int jj = 0; jj < 8; ++jj)
#pragma unroll
    for (int h = 0; h < GM; ++h) {
      float x = acc[jj][h];
#pragma unroll
      for (int o = Q::DG; o < 64; o <<= 1) x += __shfl_xor(x, o);
      acc[jj][h] = x;
    }
  __syncthreads();  // the K table is dead: the pool takes the merge buffer
  float* red_o = reinterpret_cast<float*>(pool);
  float* red_z = qv;  // the query is dead too
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < GM; ++h) red_m[wave][h] = m_run[h];
  }
  if (m == 0) {
    red_l[wave][g] = l_tot;
    red_z[wave * GM + g] = z_tot;
  }
  if (tg == 0) {
#pragma unroll
    for (int h = 0; h < GM; ++h)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) red_o[(wave * GM + h) * (D + 1) + 8 * dg + jj] = acc[jj][h];
  }
  __syncthreads();
  const int64_t row0 = ((int64_t)b * hq + kvh * G + h0) * num_splits + split;
  for (int idx = tid; idx < nh * D; idx += NW * 64) {
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
        o += f * (red_o[(w * GM + gg) * (D + 1) + d] + red_z[w * GM + gg]);
      }
    }
    const int64_t row = row0 + (int64_t)gg * num_splits;
    ws_o[row * D + d] = (L > 0.f) ? o / L : 0.f;
    if (d == 0) ws_lse[row] = (L > 0.f) ? M + __builtin_log2f(L) : -INFINITY;
  }
}

template <int D, int KB, int VB, bool KF8, bool VLM>
hipError_t launch_valu(const V1Args& a, hipStream_t st) {
  const int G = a.hq / a.hkv;
  dim3 grid(a.splits, a.hkv * ((G + GM - 1) / GM), a.B), block(NW * 64);
  v1_attn_valu_kernel<D, KB, VB, KF8, VLM><<<grid, block, 0, st>>>(
      a.q, a.qt, a.cache, a.bt, a.sl, a.ks, a.hq, a.hkv, a.lbs, a.max_blocks, a.nb, a.sblk, a.spos, a.shead,
      a.cent, a.qscale, a.splits, a.wo, a.wl, a.rot);
  return hipGetLastError();
}

template <int D, int KB, int VB>
hipError_t launch_valu_v(const V1Args& a, bool vlm, hipStream_t st) {
  if constexpr (VB == 4 && KB <= 4) {
    if (vlm) return launch_valu<D, KB, VB, false, true>(a, st);
  }
  return launch_valu<D, KB, VB, false, false>(a, st);
}

template <int D, int KB>
hipError_t launch_valu_k(int vb, const V1Args& a, bool vlm, hipStream_t st) {
  if constexpr (KB == 8) {
    return launch_valu_v<D, 8, 8>(a, vlm, st);
  } else {
    if (vb == 1) return launch_valu_v<D, KB, 1>(a, vlm, st);
    if (vb == 2) return launch_valu_v<D, KB, 2>(a, vlm, st);
    if (vb == 3) return launch_valu_v<D, KB, 3>(a, vlm, st);
    return launch_valu_v<D, KB, 4>(a, vlm, st);
  }
}

template <int D>
hipError_t launch_valu_d(int kb, int vb, bool kf8, bool vlm, const V1Args& a, hipStream_t st) {
  if (kf8) return launch_valu<D, 8, 8, true, false>(a, st);
  if (kb == 1) return launch_valu_k<D, 1>(vb, a, vlm, st);
  if (kb == 2) return launch_valu_k<D, 2>(vb, a, vlm, st);
  if (kb == 3) return launch_valu_k<D, 3>(vb, a, vlm, st);
  if (kb == 4) return launch_valu_k<D, 4>(vb, a, vlm, st);
  return launch_valu_k<D, 8>(vb, a, vlm, st);
}

template <int D>
hipError_t merge_d(const V1Args& a, hipStream_t st) {
  const int64_t rows = (int64_t)a.B * a.hq;
  const float rs = fwht_scale(D);
  if ((a.vrot & V1F_VROT) && a.rot != nullptr) {  // o M^T
    if (a.ot == F32) return launch_merge_splits<D, F32, ROT_MATRIX>(a.wo, a.wl, rows, a.splits, a.rot, 1.f, a.out, st, a.lse);
    if (a.ot == F16) return launch_merge_splits<D, F16, ROT_MATRIX>(a.wo, a.wl, rows, a.splits, a.rot, 1.f, a.out, st, a.lse);
    return launch_merge_splits<D, BF16, ROT_MATRIX>(a.wo, a.wl, rows, a.splits, a.rot, 1.f, a.out, st, a.lse);
  }
  if (a.vrot & V1F_VROT) {
    if (a.ot == F32) return launch_merge_splits<D, F32, ROT_PLAIN>(a.wo, a.wl, rows, a.splits, nullptr, rs, a.out, st, a.lse);
    if (a.ot == F16) return launch_merge_splits<D, F16, ROT_PLAIN>(a.wo, a.wl, rows, a.splits, nullptr, rs, a.out, st, a.lse);
    return launch_merge_splits<D, BF16, ROT_PLAIN>(a.wo, a.wl, rows, a.splits, nullptr, rs, a.out, st, a.lse);
  }
  if (a.ot == F32) return launch_merge_splits<D, F32, ROT_NONE>(a.wo, a.wl, rows, a.splits, nullptr, rs, a.out, st, a.lse);
  if (a.ot == F16) return launch_merge_splits<D, F16, ROT_NONE>(a.wo, a.wl, rows, a.splits, nullptr, rs, a.out, st, a.lse);
  return launch_merge_splits<D, BF16, ROT_NONE>(a.wo, a.wl, rows, a.splits, nullptr, rs, a.out, st, a.lse);
}

}  // namespace

hipError_t raw_valu_launch(const V1Args& a, int d, hipStream_t st) {
  hipError_t e;
  if (d == 64) e = launch_valu<64, 16, 16, false, false>(a, st);
  else if (d == 128) e = launch_valu<128, 16, 16, false, false>(a, st);
  else e = launch_valu<256, 16, 16, false, false>(a, st);
  if (e != hipSuccess) return e;
  if (d == 64) return merge_d<64>(a, st);
  if (d == 128) return merge_d<128>(a, st);
  return merge_d<256>(a, st);
}

hipError_t v1_valu_launch(const V1Args& a, int d, int kb, int vb, int flags, hipStream_t st) {
  const bool kf8 = (flags & V1F_KFP8) != 0, vlm = (flags & V1F_VLM) != 0;
  hipError_t e;
  if (d == 64) e = launch_valu_d<64>(kb, vb, kf8, vlm, a, st);
  else if (d == 128) e = launch_valu_d<128>(kb, vb, kf8, vlm, a, st);
  else e = launch_valu_d<256>(kb, vb, kf8, vlm, a, st);
  if (e != hipSuccess) return e;
  if (d == 64) return merge_d<64>(a, st);
  if (d == 128) return merge_d<128>(a, st);
  return merge_d<256>(a, st);
}

}  // namespace ftq
