// Library-format encode / decode / RHT for the power-of-two head dims without
// a tuned kernel: 8, 16, 32, 512, 1024, 2048 and 4096 (the tuned kernels in
// ftq_codec.hip and ftq_encode_mfma.h cover 64, 128 and 256).  The reference
// accepts any power of two (core/quantizer.py:77-80) and computes, per vector
// (core/quantizer.py:137-160, 191-205; core/hadamard.py:23-100):
//   encode: y = fwht(x * s) * d^-1/2, n = ||y||, u = y / (n + 1e-8),
//           code = #{interior boundaries b : b < u}, n -> fp16
//   decode: x = fwht(level[code] * n16) * d^-1/2 * s
// One vector per LPV = min(64, d / 8) lanes, E = d / LPV contiguous elements
// per lane (8 ... 64): the butterflies run in registers, then across lanes
// (DPP within 16-lane rows, ds_bpermute beyond), in the reference's stage
// order, so decode and RHT are bit-identical to it.  Rows are d * bits / 8
// bytes (3 bytes at d = 8, 3 bits), so codes move with byte loads and stores.
#include "ftq_codec_dev.h"
#include "ftq_device.h"
#include "ftq_internal.h"

namespace ftq {

float fwht_scale(int d);

namespace {

template <int M>
__device__ __forceinline__ float xor_any(float v) {
  if constexpr (M <= 8) return lane_xor<M>(v);
  else return __shfl_xor(v, M);
}

// unnormalised FWHT, stages h = 1, 2, ..., D/2 (E in the lane, then LPV lanes)
template <int E, int LPV>
__device__ __forceinline__ void fwht_any(float (&x)[E], int li) {
#pragma unroll
  for (int h = 1; h < E; h <<= 1) {
#pragma unroll
    for (int i = 0; i < E; ++i) {
      if ((i & h) == 0) {
        const float a = x[i], b = x[i + h];
        x[i] = a + b;
        x[i + h] = a - b;
      }
    }
  }
#pragma unroll
  for (int m = 1; m < LPV; m <<= 1) {
    const bool upper = (li & m) != 0;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      float p;
      if (m == 1) p = xor_any<1>(x[i]);
      else if (m == 2) p = xor_any<2>(x[i]);
      else if (m == 4) p = xor_any<4>(x[i]);
      else if (m == 8) p = xor_any<8>(x[i]);
      else if (m == 16) p = xor_any<16>(x[i]);
      else p = xor_any<32>(x[i]);
      x[i] = upper ? (p - x[i]) : (x[i] + p);
    }
  }
}

template <int LPV>
__device__ __forceinline__ float sum_any(float v) {
  if constexpr (LPV >= 2) v += xor_any<1>(v);
  if constexpr (LPV >= 4) v += xor_any<2>(v);
  if constexpr (LPV >= 8) v += xor_any<4>(v);
  if constexpr (LPV >= 16) v += xor_any<8>(v);
  if constexpr (LPV >= 32) v += xor_any<16>(v);
  if constexpr (LPV >= 64) v += xor_any<32>(v);
  return v;
}

template <int E, int LPV, int DT, int BITS>
__global__ __launch_bounds__(256) void any_encode_kernel(const void* __restrict__ x, int64_t n,
                                                         const float* __restrict__ signs,
                                                         const float* __restrict__ boundaries, float scale,
                                                         uint8_t* __restrict__ packed,
                                                         uint16_t* __restrict__ norms) {
  constexpr int D = E * LPV, L = 1 << BITS, PB = E * BITS / 8, VPB = 256 / LPV;
  const int li = threadIdx.x % LPV, grp = threadIdx.x / LPV;
  float sg[E], bnd[L - 1];
#pragma unroll
  for (int i = 0; i < E; ++i) sg[i] = signs[li * E + i];
#pragma unroll
  for (int j = 0; j < L - 1; ++j) bnd[j] = boundaries[j + 1];
  for (int64_t v = (int64_t)blockIdx.x * VPB + grp; v < n; v += (int64_t)gridDim.x * VPB) {
    float y[E];
    load_elems<DT, E>(x, v * D + li * E, y);
#pragma unroll
    for (int i = 0; i < E; ++i) y[i] *= sg[i];
    fwht_any<E, LPV>(y, li);
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      y[i] *= scale;
      ss = __builtin_fmaf(y[i], y[i], ss);
    }
    const float nrm = __builtin_sqrtf(sum_any<LPV>(ss));
    const float den = nrm + 1e-8f;
    uint8_t* row = packed + v * (D * BITS / 8) + li * PB;
    uint32_t acc = 0;
    int nbits = 0, out = 0;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const float u = y[i] / den;
      uint32_t q = 0;
#pragma unroll
      for (int j = 0; j < L - 1; ++j) q += (bnd[j] < u) ? 1u : 0u;
      acc |= q << nbits;  // codes LSB first, as the reference packs them
      nbits += BITS;
      while (nbits >= 8) {
        row[out++] = (uint8_t)acc;
        acc >>= 8;
        nbits -= 8;
      }
    }
    if (li == 0) norms[v] = (uint16_t)f32_to_f16_bits(nrm);
  }
}

template <int E, int LPV, int BITS, int OT>
__global__ __launch_bounds__(256) void any_decode_kernel(const uint8_t* __restrict__ packed,
                                                         const uint16_t* __restrict__ norms, int64_t n,
                                                         const float* __restrict__ levels,
                                                         const float* __restrict__ signs, float scale,
                                                         void* __restrict__ out) {
  constexpr int D = E * LPV, L = 1 << BITS, PB = E * BITS / 8, VPB = 256 / LPV;
  __shared__ float slev[L];
  if (threadIdx.x < L) slev[threadIdx.x] = levels[threadIdx.x];
  __syncthreads();
  const int li = threadIdx.x % LPV, grp = threadIdx.x / LPV;
  float sg[E];
#pragma unroll
  for (int i = 0; i < E; ++i) sg[i] = signs[li * E + i];
  for (int64_t v = (int64_t)blockIdx.x * VPB + grp; v < n; v += (int64_t)gridDim.x * VPB) {
    const uint8_t* row = packed + v * (D * BITS / 8) + li * PB;
    const float nrm = f16_bits_to_f32(norms[v]);
    float y[E];
    uint32_t acc = 0;
    int nbits = 0, in = 0;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      while (nbits < BITS) {
        acc |= (uint32_t)row[in++] << nbits;
        nbits += 8;
      }
      y[i] = slev[acc & (L - 1)] * nrm;
      acc >>= BITS;
      nbits -= BITS;
    }
    fwht_any<E, LPV>(y, li);
#pragma unroll
    for (int i = 0; i < E; ++i) y[i] = (y[i] * scale) * sg[i];
    store_elems<OT, E>(out, v * D + li * E, y);
  }
}

template <int E, int LPV, int IT, int OT>
__global__ __launch_bounds__(256) void any_rht_kernel(const void* __restrict__ x, int64_t n,
                                                      const float* __restrict__ signs, float scale, int inverse,
                                                      void* __restrict__ out) {
  constexpr int D = E * LPV, VPB = 256 / LPV;
  const int li = threadIdx.x % LPV, grp = threadIdx.x / LPV;
  float sg[E];
#pragma unroll
  for (int i = 0; i < E; ++i) sg[i] = signs[li * E + i];
  for (int64_t v = (int64_t)blockIdx.x * VPB + grp; v < n; v += (int64_t)gridDim.x * VPB) {
    float y[E];
    load_elems<IT, E>(x, v * D + li * E, y);
    if (!inverse) {
#pragma unroll
      for (int i = 0; i < E; ++i) y[i] *= sg[i];
    }
    fwht_any<E, LPV>(y, li);
#pragma unroll
    for (int i = 0; i < E; ++i) {
      y[i] *= scale;
      if (inverse) y[i] *= sg[i];
    }
    store_elems<OT, E>(out, v * D + li * E, y);
  }
}

dim3 grid_for(int64_t n, int lpv) {
  const int64_t vpb = 256 / lpv;
  int64_t g = (n + vpb - 1) / vpb;
  if (g > 256 * 32) g = 256 * 32;
  return dim3((unsigned)(g < 1 ? 1 : g));
}

template <int E, int LPV>
hipError_t enc_e(const void* x, int dt, int64_t n, const float* s, const float* b, int bits, uint8_t* p,
                 uint16_t* nr, hipStream_t st) {
  const float sc = fwht_scale(E * LPV);
  const dim3 g = grid_for(n, LPV), blk(256);
#define FTQ_ENC(DT, B) any_encode_kernel<E, LPV, DT, B><<<g, blk, 0, st>>>(x, n, s, b, sc, p, nr)
  if (bits == 2) { if (dt == F32) FTQ_ENC(F32, 2); else if (dt == F16) FTQ_ENC(F16, 2); else FTQ_ENC(BF16, 2); }
  else if (bits == 3) { if (dt == F32) FTQ_ENC(F32, 3); else if (dt == F16) FTQ_ENC(F16, 3); else FTQ_ENC(BF16, 3); }
  else { if (dt == F32) FTQ_ENC(F32, 4); else if (dt == F16) FTQ_ENC(F16, 4); else FTQ_ENC(BF16, 4); }
#undef FTQ_ENC
  return hipGetLastError();
}

template <int E, int LPV>
hipError_t dec_e(const uint8_t* p, const uint16_t* nr, int64_t n, const float* lev, const float* s, int bits,
                 void* out, int ot, hipStream_t st) {
  const float sc = fwht_scale(E * LPV);
  const dim3 g = grid_for(n, LPV), blk(256);
#define FTQ_DEC(B, OT) any_decode_kernel<E, LPV, B, OT><<<g, blk, 0, st>>>(p, nr, n, lev, s, sc, out)
  if (bits == 2) { if (ot == F32) FTQ_DEC(2, F32); else if (ot == F16) FTQ_DEC(2, F16); else FTQ_DEC(2, BF16); }
  else if (bits == 3) { if (ot == F32) FTQ_DEC(3, F32); else if (ot == F16) FTQ_DEC(3, F16); else FTQ_DEC(3, BF16); }
  else { if (ot == F32) FTQ_DEC(4, F32); else if (ot == F16) FTQ_DEC(4, F16); else FTQ_DEC(4, BF16); }
#undef FTQ_DEC
  return hipGetLastError();
}

template <int E, int LPV>
hipError_t rht_e(const void* x, int it, int64_t n, const float* s, int inverse, void* out, int ot,
                 hipStream_t st) {
  const float sc = fwht_scale(E * LPV);
  const dim3 g = grid_for(n, LPV), blk(256);
#define FTQ_RHT(IT, OT) any_rht_kernel<E, LPV, IT, OT><<<g, blk, 0, st>>>(x, n, s, sc, inverse, out)
#define FTQ_RHT_O(IT) { if (ot == F32) FTQ_RHT(IT, F32); else if (ot == F16) FTQ_RHT(IT, F16); else FTQ_RHT(IT, BF16); }
  if (it == F32) FTQ_RHT_O(F32) else if (it == F16) FTQ_RHT_O(F16) else FTQ_RHT_O(BF16)
#undef FTQ_RHT_O
#undef FTQ_RHT
  return hipGetLastError();
}

}  // namespace

bool codec_any_dim(int d) {
  return d == 8 || d == 16 || d == 32 || d == 512 || d == 1024 || d == 2048 || d == 4096;
}

#define FTQ_ANY_DISPATCH(FN, ...)                                    \
  switch (d) {                                                       \
    case 8: return FN<8, 1>(__VA_ARGS__);                            \
    case 16: return FN<8, 2>(__VA_ARGS__);                           \
    case 32: return FN<8, 4>(__VA_ARGS__);                           \
    case 512: return FN<8, 64>(__VA_ARGS__);                         \
    case 1024: return FN<16, 64>(__VA_ARGS__);                       \
    case 2048: return FN<32, 64>(__VA_ARGS__);                       \
    default: return FN<64, 64>(__VA_ARGS__);                         \
  }

hipError_t codec_any_encode(int d, const void* x, int dt, int64_t n, const float* signs, const float* boundaries,
                            int bits, uint8_t* packed, uint16_t* norms, hipStream_t st) {
  FTQ_ANY_DISPATCH(enc_e, x, dt, n, signs, boundaries, bits, packed, norms, st)
}

hipError_t codec_any_decode(int d, const uint8_t* packed, const uint16_t* norms, int64_t n, const float* levels,
                            const float* signs, int bits, void* out, int ot, hipStream_t st) {
  FTQ_ANY_DISPATCH(dec_e, packed, norms, n, levels, signs, bits, out, ot, st)
}

hipError_t codec_any_rht(int d, const void* x, int it, int64_t n, const float* signs, int inverse, void* out,
                         int ot, hipStream_t st) {
  FTQ_ANY_DISPATCH(rht_e, x, it, n, signs, inverse, out, ot, st)
}

#undef FTQ_ANY_DISPATCH

}  // namespace ftq
