// Split-K merge of the decode-attention kernels: for every (batch, q head)
// row, combine the per-split partial outputs o_s (already divided by their
// own softmax sums) and their log2-domain log-sum-exps:
//   M = max_s lse_s,  w_s = 2^(lse_s - M),  o = sum_s w_s o_s / sum_s w_s
// (the stage-2 merge of reference vllm_plugin/v1_backend.py:975-1093 and the
// flash-decode combine of kernels/triton_flash_decode.py:66-221), then the
// output transform of the cache format:
//   ROT_SIGNS  o <- (H o) * scale * signs   inverse RHT of library-format V
//   ROT_PLAIN  o <- (H o) * scale            un-rotation of v1 V (v_rotate)
//   ROT_MATRIX o <- o M^T, M = signs (row-major D x D fp32): un-rotation of v1 V
//              rotated by a matrix strategy (x M)
//   ROT_NONE   o unchanged
// A row with every split empty (lse = -inf) is written as zeros.  With
// lse_out, the row's natural-log log-sum-exp of the scaled scores goes there
// too (-inf for an empty row): ln 2 * (M + log2 sum_s w_s).
//
// Layout: a row is handled by WPR waves (WPR = 1 or 4).  Lane l of a wave owns
// elements [E l, E l + E) of the row (E = D / 64), so each split's partial
// output is one coalesced D*4-byte read per wave.  With WPR = 4 the waves take
// every fourth split and meet in LDS.
#pragma once

#include "ftq_device.h"

namespace ftq {

enum MergeRot : int { ROT_NONE = 0, ROT_PLAIN = 1, ROT_SIGNS = 2, ROT_MATRIX = 3 };

__device__ __forceinline__ float wave_max64(float x) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m));
  return x;
}

// Unnormalised Walsh-Hadamard transform of a D-vector held as E contiguous
// elements per lane over all 64 lanes.
template <int E>
__device__ __forceinline__ void fwht_wave64(float (&y)[E], int lane) {
#pragma unroll
  for (int h = 1; h < E; h <<= 1) {
#pragma unroll
    for (int i = 0; i < E; ++i) {
      if ((i & h) == 0) {
        const float a = y[i], b = y[i + h];
        y[i] = a + b;
        y[i + h] = a - b;
      }
    }
  }
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) {
    const bool upper = (lane & m) != 0;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      float p;
      if (m == 1) p = lane_xor<1>(y[i]);
      else if (m == 2) p = lane_xor<2>(y[i]);
      else if (m == 4) p = lane_xor<4>(y[i]);
      else if (m == 8) p = lane_xor<8>(y[i]);
      else p = __shfl_xor(y[i], m);
      y[i] = upper ? (p - y[i]) : (y[i] + p);
    }
  }
}

// E = 1, 2 or 4 contiguous fp32 loads / dtype stores (4, 8 or 16 bytes per lane)
template <int E>
__device__ __forceinline__ void load_f32_small(const float* p, float (&x)[E]) {
  static_assert(E == 1 || E == 2 || E == 4, "1, 2 or 4 elements");
  if constexpr (E == 1) {
    x[0] = *p;
  } else if constexpr (E == 2) {
    const float2 v = *reinterpret_cast<const float2*>(p);
    x[0] = v.x; x[1] = v.y;
  } else {
    const float4 v = *reinterpret_cast<const float4*>(p);
    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
  }
}
template <int OT, int E>
__device__ __forceinline__ void store_small(void* base, int64_t off, const float (&y)[E]) {
  if constexpr (OT == F32) {
    float* p = static_cast<float*>(base) + off;
    if constexpr (E == 1) *p = y[0];
    else if constexpr (E == 2) *reinterpret_cast<float2*>(p) = make_float2(y[0], y[1]);
    else *reinterpret_cast<float4*>(p) = make_float4(y[0], y[1], y[2], y[3]);
  } else if constexpr (E == 1) {
    *(static_cast<uint16_t*>(base) + off) = (uint16_t)f32_to_half_bits(OT, y[0]);
  } else {
    uint32_t w[E / 2];
#pragma unroll
    for (int k = 0; k < E / 2; ++k) w[k] = f32_to_half_bits(OT, y[2 * k]) | (f32_to_half_bits(OT, y[2 * k + 1]) << 16);
    uint16_t* p = static_cast<uint16_t*>(base) + off;
    if constexpr (E == 2) *reinterpret_cast<uint32_t*>(p) = w[0];
    else *reinterpret_cast<uint2*>(p) = make_uint2(w[0], w[1]);
  }
}

template <int D, int OT, int ROT, int WPR>
__global__ __launch_bounds__(256) void merge_splits_kernel(const float* __restrict__ ws_o,
                                                           const float* __restrict__ ws_lse,
                                                           int64_t rows, int num_splits,
                                                           const float* __restrict__ signs,
                                                           float scale, void* __restrict__ out,
                                                           float* __restrict__ lse_out) {
  static_assert(WPR == 1 || WPR == 4, "one or four waves per row");
  constexpr int E = D / 64;
  constexpr int RPB = 4 / WPR;  // rows per workgroup
  __shared__ float part[WPR == 4 ? 4 : 1][WPR == 4 ? D : 1];
  __shared__ float wpart[4];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int64_t r = (int64_t)blockIdx.x * RPB + (WPR == 4 ? 0 : wv);
  const bool live = r < rows;  // uniform per wave (and per workgroup when WPR == 4)
  const float* lse = ws_lse + (live ? r : 0) * num_splits;

  // The partial outputs do not depend on the max: the first CH of this
  // wave's splits are requested together with the log-sum-exps, so the two
  // reads overlap.
  constexpr int CH = 8;
  const int s0 = (WPR == 4) ? wv : 0;
  const float* po = ws_o + ((live ? r : 0) * num_splits) * D + lane * E;
  float x[CH][E], lw[CH];
#pragma unroll
  for (int k = 0; k < CH; ++k) {
    const int s = s0 + k * WPR;
    if (s < num_splits) {
      load_f32_small<E>(po + (int64_t)s * D, x[k]);
      lw[k] = lse[s];
    }
  }
  float M = -INFINITY;
  for (int s = lane; s < num_splits; s += 64) M = fmaxf(M, lse[s]);
  M = wave_max64(M);
  float y[E];
#pragma unroll
  for (int i = 0; i < E; ++i) y[i] = 0.f;
  float W = 0.f;
  if (live && M != -INFINITY) {
    for (int c0 = s0; c0 < num_splits; c0 += CH * WPR) {
      if (c0 != s0) {  // later chunks (more than CH splits per wave)
#pragma unroll
        for (int k = 0; k < CH; ++k) {
          const int s = c0 + k * WPR;
          if (s < num_splits) {
            load_f32_small<E>(po + (int64_t)s * D, x[k]);
            lw[k] = lse[s];
          }
        }
      }
#pragma unroll
      for (int k = 0; k < CH; ++k) {
        if (c0 + k * WPR < num_splits) {
          const float w = __builtin_amdgcn_exp2f(lw[k] - M);
          W += w;
#pragma unroll
          for (int i = 0; i < E; ++i) y[i] = __builtin_fmaf(w, x[k][i], y[i]);
        }
      }
    }
  }
  if constexpr (WPR == 4) {
#pragma unroll
    for (int i = 0; i < E; ++i) part[wv][lane * E + i] = y[i];
    if (lane == 0) wpart[wv] = W;
    __syncthreads();
    if (wv != 0) return;
    W = (wpart[0] + wpart[1]) + (wpart[2] + wpart[3]);
#pragma unroll
    for (int i = 0; i < E; ++i)
      y[i] = (part[0][lane * E + i] + part[1][lane * E + i]) + (part[2][lane * E + i] + part[3][lane * E + i]);
  }
  if (!live) return;
  if (lse_out != nullptr && lane == 0)
    lse_out[r] = (W > 0.f) ? (M + __builtin_log2f(W)) * 0.69314718055994531f : -INFINITY;
  const float inv = (W > 0.f) ? 1.f / W : 0.f;
#pragma unroll
  for (int i = 0; i < E; ++i) y[i] *= inv;
  if constexpr (ROT == ROT_MATRIX) {
    __shared__ float mrow[4][D];  // this wave's row; a wave's LDS accesses run in order
    const int w = (int)(threadIdx.x >> 6);
#pragma unroll
    for (int i = 0; i < E; ++i) mrow[w][lane * E + i] = y[i];
    __asm__ volatile("" ::: "memory");
    float z[E];
#pragma unroll
    for (int i = 0; i < E; ++i) z[i] = 0.f;
    for (int j = 0; j < D; ++j) {
      const float oj = mrow[w][j];
#pragma unroll
      for (int i = 0; i < E; ++i) z[i] = __builtin_fmaf(oj, signs[(int64_t)(lane * E + i) * D + j], z[i]);
    }
#pragma unroll
    for (int i = 0; i < E; ++i) y[i] = z[i];
  } else if constexpr (ROT != ROT_NONE) {
    fwht_wave64<E>(y, lane);
#pragma unroll
    for (int i = 0; i < E; ++i) {
      y[i] *= scale;
      if constexpr (ROT == ROT_SIGNS) y[i] *= signs[lane * E + i];
    }
  }
  store_small<OT, E>(out, r * D + lane * E, y);
}

// Launch helper: four waves per row when there are enough splits to share.
template <int D, int OT, int ROT>
hipError_t launch_merge_splits(const float* ws_o, const float* ws_lse, int64_t rows, int num_splits,
                               const float* signs, float scale, void* out, hipStream_t st,
                               float* lse_out = nullptr) {
  if (rows <= 0) return hipSuccess;
  if (num_splits >= 8) {
    merge_splits_kernel<D, OT, ROT, 4><<<dim3((unsigned)rows), dim3(256), 0, st>>>(
        ws_o, ws_lse, rows, num_splits, signs, scale, out, lse_out);
  } else {
    merge_splits_kernel<D, OT, ROT, 1><<<dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st>>>(
        ws_o, ws_lse, rows, num_splits, signs, scale, out, lse_out);
  }
  return hipGetLastError();
}

}  // namespace ftq
