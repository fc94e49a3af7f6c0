// Library-format TurboQuant codec kernels for gfx950:
//   encode  = RHT (sign flip + FWHT) -> per-vector L2 norm -> u = y / (norm + 1e-8)
//             -> Lloyd-Max bucketize -> 2/3/4-bit pack, fp16 norm
//   decode  = unpack -> levels[code] * norm -> FWHT -> sign flip
//   rht     = forward / inverse randomized Hadamard transform
//
// Semantics follow the reference's unfused PyTorch path
// (core/quantizer.py:137-160 encode, :191-205 decode, core/hadamard.py:23-100),
// which the Triton kernels (kernels/triton_encode.py, triton_decode.py,
// triton_rht.py) replace on CUDA.  The C entry points are declared in
// include/fused_tq.h.
//
// Mapping: one vector per LPV lanes (E elements per lane, see ftq_device.h);
// a 256-thread workgroup holds 256/LPV vectors and walks the batch with a
// grid-stride loop.  Codes are packed with DPP neighbour exchanges into
// dword stores; nothing goes through HBM scratch.
#include "ftq_codec_dev.h"
#include "ftq_encode_fast.h"
#include "ftq_encode_mfma.h"
#include "ftq_internal.h"
#include "ftq_merge.h"

#include <cmath>

namespace ftq {

template <int D, int BITS, int DT>
__global__ __launch_bounds__(256) void encode_kernel(const void* __restrict__ x, int64_t n,
                                                     const float* __restrict__ signs,
                                                     const float* __restrict__ boundaries,
                                                     float scale, double rscale,
                                                     uint8_t* __restrict__ packed,
                                                     uint16_t* __restrict__ norms) {
  using S = FastShape<D>;
  constexpr int E = S::E, LPV = S::LPV, VPB = 256 / LPV;
  constexpr int PD = D * BITS / 8;
  constexpr int NT = (1 << BITS) - 1;
  __shared__ float bnd[NT];
  if (threadIdx.x < NT) bnd[threadIdx.x] = boundaries[threadIdx.x + 1];
  const int lane = threadIdx.x & 63;        // lane in the wave
  const int lv = threadIdx.x & (LPV - 1);   // lane in the vector
  const int grp = threadIdx.x / LPV;
  // sign flips of this lane's elements, as xor masks on the input bits
  constexpr int PER_DW = (DT == F32) ? 1 : 2;
  uint32_t smask[E / PER_DW];
#pragma unroll
  for (int k = 0; k < E / PER_DW; ++k) {
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < PER_DW; ++j)
      if (signs[lv * E + k * PER_DW + j] < 0.f) m |= (DT == F32) ? 0x80000000u : (0x8000u << (16 * j));
    smask[k] = m;
  }
  __syncthreads();

  for (int64_t v = (int64_t)blockIdx.x * VPB + grp; v < n; v += (int64_t)gridDim.x * VPB) {
    float y[E];
    if constexpr (DT == F32) {
      const uint4* p = reinterpret_cast<const uint4*>(static_cast<const float*>(x) + v * D + lv * E);
#pragma unroll
      for (int k = 0; k < E / 4; ++k) {
        const uint4 w = p[k];
        y[4 * k + 0] = __uint_as_float(w.x ^ smask[4 * k + 0]);
        y[4 * k + 1] = __uint_as_float(w.y ^ smask[4 * k + 1]);
        y[4 * k + 2] = __uint_as_float(w.z ^ smask[4 * k + 2]);
        y[4 * k + 3] = __uint_as_float(w.w ^ smask[4 * k + 3]);
      }
    } else {
      const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + v * D + lv * E);
#pragma unroll
      for (int k = 0; k < E / 8; ++k) {
        const uint4 w4 = p[k];
        const uint32_t w[4] = {w4.x ^ smask[4 * k], w4.y ^ smask[4 * k + 1], w4.z ^ smask[4 * k + 2],
                               w4.w ^ smask[4 * k + 3]};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (DT == BF16) {
            y[8 * k + 2 * j] = __uint_as_float(w[j] << 16);
            y[8 * k + 2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
          } else {
            y[8 * k + 2 * j] = f16_bits_to_f32(w[j] & 0xffffu);
            y[8 * k + 2 * j + 1] = f16_bits_to_f32(w[j] >> 16);
          }
        }
      }
    }
    uint32_t c[E];
    bool flip;
    const float nrm = encode_fast<D, BITS>(y, bnd, scale, rscale, lane, c, flip);
    store_lane_codes<E, BITS>(c, flip, packed + v * PD, lv);
    if (lv == 0) norms[v] = (uint16_t)f32_to_f16_bits(nrm);
  }
}

// Store a d = 256 row held as 16 contiguous elements per lane over 16 lanes
// (lane l: elements [16 l, 16 l + 16)) through the group's LDS row, so that
// each store instruction writes one contiguous run per vector (lane l:
// elements [64 k + 4 l, 64 k + 4 l + 4)) instead of 16 bytes of every lane's
// 64; the scattered form left the write stream at 3.0 TB/s.  A wave's LDS
// accesses run in order and each 16-lane group reads back only its own row.
template <int OT>
__device__ __forceinline__ void store_row256(float* rb, const float (&y)[16], void* out, int64_t off, int lane) {
#pragma unroll
  for (int k = 0; k < 4; ++k)
    *reinterpret_cast<float4*>(rb + lane * 16 + 4 * k) = make_float4(y[4 * k], y[4 * k + 1], y[4 * k + 2], y[4 * k + 3]);
  __asm__ volatile("" ::: "memory");
  float z[4][4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float4 t = *reinterpret_cast<const float4*>(rb + 64 * k + 4 * lane);
    z[k][0] = t.x;
    z[k][1] = t.y;
    z[k][2] = t.z;
    z[k][3] = t.w;
  }
  __asm__ volatile("" ::: "memory");  // the row is rewritten by the next vector
#pragma unroll
  for (int k = 0; k < 4; ++k) store_small<OT, 4>(out, off + 64 * k + 4 * lane, z[k]);
}

template <int D, int BITS, int OT>
__global__ __launch_bounds__(256) void decode_kernel(const uint8_t* __restrict__ packed,
                                                     const uint16_t* __restrict__ norms, int64_t n,
                                                     const float* __restrict__ levels,
                                                     const float* __restrict__ signs, float scale,
                                                     void* __restrict__ out) {
  using S = CodecShape<D>;
  constexpr int E = S::E, LPV = S::LPV, GPB = S::GPB;
  constexpr int L = 1 << BITS;
  constexpr int PD = D * BITS / 8;
  __shared__ float slev[L];
  if (threadIdx.x < L) slev[threadIdx.x] = levels[threadIdx.x];
  __syncthreads();
  const int lane = threadIdx.x % LPV;
  const int grp = threadIdx.x / LPV;
  float sg[E];
#pragma unroll
  for (int i = 0; i < E; ++i) sg[i] = signs[lane * E + i];

  constexpr bool XPOSE = (D == 256);  // rows through LDS (store_row256)
  __shared__ __attribute__((aligned(16))) float rowbuf[XPOSE ? GPB : 1][XPOSE ? D : 1];

  for (int64_t v = (int64_t)blockIdx.x * GPB + grp; v < n; v += (int64_t)gridDim.x * GPB) {
    uint32_t c[E];
    unpack_load<E, BITS>(packed + v * PD, lane, c);
    const float nrm = f16_bits_to_f32(norms[v]);
    float y[E];
#pragma unroll
    for (int i = 0; i < E; ++i) y[i] = slev[c[i]] * nrm;
    fwht_lanes<E, LPV>(y, lane);
#pragma unroll
    for (int i = 0; i < E; ++i) y[i] = (y[i] * scale) * sg[i];
    if constexpr (XPOSE) {
      store_row256<OT>(rowbuf[grp], y, out, v * D, lane);
    } else {
      store_elems<OT, E>(out, v * D + lane * E, y);
    }
  }
}

template <int D, int IT, int OT>
__global__ __launch_bounds__(256) void rht_kernel(const void* __restrict__ x, int64_t n,
                                                  const float* __restrict__ signs, float scale,
                                                  int inverse, void* __restrict__ out) {
  using S = CodecShape<D>;
  constexpr int E = S::E, LPV = S::LPV, GPB = S::GPB;
  const int lane = threadIdx.x % LPV;
  const int grp = threadIdx.x / LPV;
  float sg[E];
#pragma unroll
  for (int i = 0; i < E; ++i) sg[i] = signs[lane * E + i];
  constexpr bool XPOSE = (D == 256);  // rows through LDS (store_row256)
  __shared__ __attribute__((aligned(16))) float rowbuf[XPOSE ? GPB : 1][XPOSE ? D : 1];
  for (int64_t v = (int64_t)blockIdx.x * GPB + grp; v < n; v += (int64_t)gridDim.x * GPB) {
    float y[E];
    load_elems<IT, E>(x, v * D + lane * E, y);
    if (!inverse) {
#pragma unroll
      for (int i = 0; i < E; ++i) y[i] *= sg[i];
    }
    fwht_lanes<E, LPV>(y, lane);
#pragma unroll
    for (int i = 0; i < E; ++i) {
      y[i] *= scale;
      if (inverse) y[i] *= sg[i];
    }
    if constexpr (XPOSE) store_row256<OT>(rowbuf[grp], y, out, v * D, lane);
    else store_elems<OT, E>(out, v * D + lane * E, y);
  }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

// power-of-two head dims without a tuned kernel (ftq_codec_any.hip)
bool codec_any_dim(int d);
hipError_t codec_any_encode(int d, const void* x, int dt, int64_t n, const float* signs, const float* boundaries,
                            int bits, uint8_t* packed, uint16_t* norms, hipStream_t st);
hipError_t codec_any_decode(int d, const uint8_t* packed, const uint16_t* norms, int64_t n, const float* levels,
                            const float* signs, int bits, void* out, int ot, hipStream_t st);
hipError_t codec_any_rht(int d, const void* x, int it, int64_t n, const float* signs, int inverse, void* out,
                         int ot, hipStream_t st);

float fwht_scale(int d) { return (float)std::pow((double)d, -0.5); }

int codec_grid(int64_t n, int gpb) {
  int64_t want = (n + gpb - 1) / gpb;
  const int64_t cap = 256 * 16;  // 16 workgroups per CU on 256 CUs
  if (want > cap) want = cap;
  if (want < 1) want = 1;
  return (int)want;
}

template <int D, int BITS, int DT, bool SYM>
static void launch_encode_mfma(const EncodeSegs& io, int64_t n, const float* signs, const float* bnd,
                               float sc, double rsc, hipStream_t st) {
  // one pass of resident workgroups, each wave looping over groups of 16 vectors
  static const int cap = resident_workgroups(encode_mfma_kernel<D, BITS, DT, SYM>);
  const int64_t want = ((n + 15) / 16 * io.nseg + 3) / 4;
  encode_mfma_kernel<D, BITS, DT, SYM><<<dim3((unsigned)(want < cap ? want : cap)), dim3(256), 0, st>>>(
      io, n, signs, bnd, sc, rsc);
}

// The matrix-core encoder takes this input: d = 128 / 256, 16-bit elements,
// nseg tensors of n vectors in fewer than 2^31 - 2^20 groups of 16 (its
// 32-bit group numbering; 2^35 vectors, far beyond device memory).
static bool encode_mfma_ok(int d, int dt, int64_t n, int nseg) {
  return (d == 128 || d == 256) && dt != F32 && (n + 15) / 16 * nseg < ((int64_t)1 << 31) - (1 << 20);
}

template <int D, int BITS>
static void launch_encode_mfma_db(const EncodeSegs& io, int dt, int64_t n, const float* signs,
                                  const float* bnd, int cb_class, hipStream_t st) {
  if constexpr (D == 128 || D == 256) {
    const float sc = fwht_scale(D);
    const double rsc = 1.0 / (double)sc;
    const bool sym = cb_class == FTQ_CB_SYMMETRIC;
    if (dt == F16) {
      if (sym) launch_encode_mfma<D, BITS, F16, true>(io, n, signs, bnd, sc, rsc, st);
      else launch_encode_mfma<D, BITS, F16, false>(io, n, signs, bnd, sc, rsc, st);
    } else {
      if (sym) launch_encode_mfma<D, BITS, BF16, true>(io, n, signs, bnd, sc, rsc, st);
      else launch_encode_mfma<D, BITS, BF16, false>(io, n, signs, bnd, sc, rsc, st);
    }
  }
}

template <int D>
static hipError_t launch_encode_mfma_d(const EncodeSegs& io, int dt, int64_t n, const float* signs,
                                       const float* bnd, int bits, int cb_class, hipStream_t st) {
  if (bits == 2) launch_encode_mfma_db<D, 2>(io, dt, n, signs, bnd, cb_class, st);
  else if (bits == 3) launch_encode_mfma_db<D, 3>(io, dt, n, signs, bnd, cb_class, st);
  else launch_encode_mfma_db<D, 4>(io, dt, n, signs, bnd, cb_class, st);
  return hipGetLastError();
}

template <int D, int BITS>
static hipError_t launch_encode_db(const void* x, int dt, int64_t n, const float* signs,
                                   const float* bnd, int cb_class, uint8_t* packed, uint16_t* norms,
                                   hipStream_t st) {
  const float sc = fwht_scale(D);
  const double rsc = 1.0 / (double)sc;
  if (encode_mfma_ok(D, dt, n, 1)) {  // 16-bit inputs: Hadamard transform on the matrix cores
    const EncodeSegs io{x, nullptr, packed, nullptr, norms, nullptr, 1};
    launch_encode_mfma_db<D, BITS>(io, dt, n, signs, bnd, cb_class, st);
    return hipGetLastError();
  }
  constexpr int VPB = 256 / FastShape<D>::LPV;
  dim3 grid(codec_grid(n, VPB)), block(256);
  if (dt == F32) encode_kernel<D, BITS, F32><<<grid, block, 0, st>>>(x, n, signs, bnd, sc, rsc, packed, norms);
  else if (dt == F16) encode_kernel<D, BITS, F16><<<grid, block, 0, st>>>(x, n, signs, bnd, sc, rsc, packed, norms);
  else encode_kernel<D, BITS, BF16><<<grid, block, 0, st>>>(x, n, signs, bnd, sc, rsc, packed, norms);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_encode_d(const void* x, int dt, int64_t n, const float* signs,
                                  const float* bnd, int bits, int cb_class, uint8_t* packed,
                                  uint16_t* norms, hipStream_t st) {
  if (bits == 2) return launch_encode_db<D, 2>(x, dt, n, signs, bnd, cb_class, packed, norms, st);
  if (bits == 3) return launch_encode_db<D, 3>(x, dt, n, signs, bnd, cb_class, packed, norms, st);
  return launch_encode_db<D, 4>(x, dt, n, signs, bnd, cb_class, packed, norms, st);
}

template <int D, int BITS>
static hipError_t launch_decode_db(const uint8_t* packed, const uint16_t* norms, int64_t n,
                                   const float* lev, const float* signs, void* out, int ot,
                                   hipStream_t st) {
  using S = CodecShape<D>;
  dim3 grid(codec_grid(n, S::GPB)), block(256);
  const float sc = fwht_scale(D);
  if (ot == F32) decode_kernel<D, BITS, F32><<<grid, block, 0, st>>>(packed, norms, n, lev, signs, sc, out);
  else if (ot == F16) decode_kernel<D, BITS, F16><<<grid, block, 0, st>>>(packed, norms, n, lev, signs, sc, out);
  else decode_kernel<D, BITS, BF16><<<grid, block, 0, st>>>(packed, norms, n, lev, signs, sc, out);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_decode_d(const uint8_t* packed, const uint16_t* norms, int64_t n,
                                  const float* lev, const float* signs, int bits, void* out, int ot,
                                  hipStream_t st) {
  if (bits == 2) return launch_decode_db<D, 2>(packed, norms, n, lev, signs, out, ot, st);
  if (bits == 3) return launch_decode_db<D, 3>(packed, norms, n, lev, signs, out, ot, st);
  return launch_decode_db<D, 4>(packed, norms, n, lev, signs, out, ot, st);
}

template <int D, int IT>
static hipError_t launch_rht_di(const void* x, int64_t n, const float* signs, int inverse,
                                void* out, int ot, hipStream_t st) {
  using S = CodecShape<D>;
  dim3 grid(codec_grid(n, S::GPB)), block(256);
  const float sc = fwht_scale(D);
  if (ot == F32) rht_kernel<D, IT, F32><<<grid, block, 0, st>>>(x, n, signs, sc, inverse, out);
  else if (ot == F16) rht_kernel<D, IT, F16><<<grid, block, 0, st>>>(x, n, signs, sc, inverse, out);
  else rht_kernel<D, IT, BF16><<<grid, block, 0, st>>>(x, n, signs, sc, inverse, out);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_rht_d(const void* x, int it, int64_t n, const float* signs, int inverse,
                               void* out, int ot, hipStream_t st) {
  if (it == F32) return launch_rht_di<D, F32>(x, n, signs, inverse, out, ot, st);
  if (it == F16) return launch_rht_di<D, F16>(x, n, signs, inverse, out, ot, st);
  return launch_rht_di<D, BF16>(x, n, signs, inverse, out, ot, st);
}

}  // namespace ftq

using namespace ftq;

extern "C" int ftq_codebook_class(const float* boundaries, int bits) {
  FTQ_REQUIRE(bits >= 2 && bits <= 4, "bits must be 2, 3, or 4");
  FTQ_REQUIRE(boundaries, "null pointer argument");
  const int mid = 1 << (bits - 1), nb = (1 << bits) + 1;
  for (int k = 1; k < nb; ++k)
    if (!(boundaries[k - 1] <= boundaries[k])) return FTQ_CB_ANY;  // unsorted or NaN: no claims
  if (!(std::fabs(boundaries[mid]) < boundaries[mid + 1])) return FTQ_CB_ANY;
  for (int k = 1; k < mid; ++k)
    if (!(boundaries[mid + k] == -boundaries[mid - k])) return FTQ_CB_ANY;
  return FTQ_CB_SYMMETRIC;
}

extern "C" int ftq_encode_cb(const void* x, int x_dtype, int64_t n, int d, const float* signs,
                             const float* boundaries, int bits, int codebook_class,
                             uint8_t* packed_out, uint16_t* norms_out, void* stream) {
  FTQ_REQUIRE(n >= 0, "n must be >= 0");
  FTQ_REQUIRE(d == 64 || d == 128 || d == 256 || codec_any_dim(d), "head_dim must be a power of two in [8, 4096]");
  FTQ_REQUIRE(bits >= 2 && bits <= 4, "bits must be 2, 3, or 4");
  FTQ_REQUIRE(x_dtype >= F32 && x_dtype <= BF16, "x_dtype must be FTQ_F32, FTQ_F16 or FTQ_BF16");
  FTQ_REQUIRE(codebook_class == FTQ_CB_ANY || codebook_class == FTQ_CB_SYMMETRIC,
              "codebook_class must be FTQ_CB_ANY or FTQ_CB_SYMMETRIC");
  if (n == 0) return FTQ_OK;
  FTQ_REQUIRE(x && signs && boundaries && packed_out && norms_out, "null pointer argument");
  FTQ_REQUIRE(aligned16(x), "x must be 16-byte aligned");
  FTQ_REQUIRE(codec_any_dim(d) || aligned4(packed_out), "packed_out must be 4-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (codec_any_dim(d)) e = codec_any_encode(d, x, x_dtype, n, signs, boundaries, bits, packed_out, norms_out, st);
  else if (d == 64) e = launch_encode_d<64>(x, x_dtype, n, signs, boundaries, bits, codebook_class, packed_out, norms_out, st);
  else if (d == 128) e = launch_encode_d<128>(x, x_dtype, n, signs, boundaries, bits, codebook_class, packed_out, norms_out, st);
  else e = launch_encode_d<256>(x, x_dtype, n, signs, boundaries, bits, codebook_class, packed_out, norms_out, st);
  return hip_status(e);
}

extern "C" int ftq_encode_kv(const void* k, const void* v, int x_dtype, int64_t n, int d,
                             const float* signs, const float* boundaries, int bits, int codebook_class,
                             uint8_t* k_packed_out, uint16_t* k_norms_out, uint8_t* v_packed_out,
                             uint16_t* v_norms_out, void* stream) {
  FTQ_REQUIRE(n >= 0, "n must be >= 0");
  FTQ_REQUIRE(d == 64 || d == 128 || d == 256 || codec_any_dim(d), "head_dim must be a power of two in [8, 4096]");
  FTQ_REQUIRE(bits >= 2 && bits <= 4, "bits must be 2, 3, or 4");
  FTQ_REQUIRE(x_dtype >= F32 && x_dtype <= BF16, "x_dtype must be FTQ_F32, FTQ_F16 or FTQ_BF16");
  FTQ_REQUIRE(codebook_class == FTQ_CB_ANY || codebook_class == FTQ_CB_SYMMETRIC,
              "codebook_class must be FTQ_CB_ANY or FTQ_CB_SYMMETRIC");
  if (n == 0) return FTQ_OK;
  FTQ_REQUIRE(k && v && signs && boundaries && k_packed_out && k_norms_out && v_packed_out && v_norms_out,
              "null pointer argument");
  if (!encode_mfma_ok(d, x_dtype, n, 2)) {  // no fused kernel for this input: one launch per tensor
    const int e = ftq_encode_cb(k, x_dtype, n, d, signs, boundaries, bits, codebook_class, k_packed_out,
                                k_norms_out, stream);
    if (e != FTQ_OK) return e;
    return ftq_encode_cb(v, x_dtype, n, d, signs, boundaries, bits, codebook_class, v_packed_out,
                         v_norms_out, stream);
  }
  FTQ_REQUIRE(aligned16(k) && aligned16(v), "k and v must be 16-byte aligned");
  FTQ_REQUIRE(aligned4(k_packed_out) && aligned4(v_packed_out), "packed outputs must be 4-byte aligned");
  const EncodeSegs io{k, v, k_packed_out, v_packed_out, k_norms_out, v_norms_out, 2};
  hipStream_t st = (hipStream_t)stream;
  hipError_t e = d == 128 ? launch_encode_mfma_d<128>(io, x_dtype, n, signs, boundaries, bits, codebook_class, st)
                          : launch_encode_mfma_d<256>(io, x_dtype, n, signs, boundaries, bits, codebook_class, st);
  return hip_status(e);
}

extern "C" int ftq_encode(const void* x, int x_dtype, int64_t n, int d, const float* signs,
                          const float* boundaries, int bits, uint8_t* packed_out,
                          uint16_t* norms_out, void* stream) {
  return ftq_encode_cb(x, x_dtype, n, d, signs, boundaries, bits, FTQ_CB_ANY, packed_out, norms_out, stream);
}

extern "C" int ftq_decode(const uint8_t* packed, const uint16_t* norms, int64_t n, int d,
                          const float* levels, const float* signs, int bits, void* out,
                          int out_dtype, void* stream) {
  FTQ_REQUIRE(n >= 0, "n must be >= 0");
  FTQ_REQUIRE(d == 64 || d == 128 || d == 256 || codec_any_dim(d), "head_dim must be a power of two in [8, 4096]");
  FTQ_REQUIRE(bits >= 2 && bits <= 4, "bits must be 2, 3, or 4");
  FTQ_REQUIRE(out_dtype >= F32 && out_dtype <= BF16, "out_dtype must be FTQ_F32, FTQ_F16 or FTQ_BF16");
  if (n == 0) return FTQ_OK;
  FTQ_REQUIRE(packed && norms && levels && signs && out, "null pointer argument");
  FTQ_REQUIRE(aligned16(out), "out must be 16-byte aligned");
  FTQ_REQUIRE(codec_any_dim(d) || aligned4(packed), "packed must be 4-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (codec_any_dim(d)) e = codec_any_decode(d, packed, norms, n, levels, signs, bits, out, out_dtype, st);
  else if (d == 64) e = launch_decode_d<64>(packed, norms, n, levels, signs, bits, out, out_dtype, st);
  else if (d == 128) e = launch_decode_d<128>(packed, norms, n, levels, signs, bits, out, out_dtype, st);
  else e = launch_decode_d<256>(packed, norms, n, levels, signs, bits, out, out_dtype, st);
  return hip_status(e);
}

extern "C" int ftq_rht(const void* x, int x_dtype, int64_t n, int d, const float* signs,
                       int inverse, void* out, int out_dtype, void* stream) {
  FTQ_REQUIRE(n >= 0, "n must be >= 0");
  FTQ_REQUIRE(d == 64 || d == 128 || d == 256 || codec_any_dim(d), "head_dim must be a power of two in [8, 4096]");
  FTQ_REQUIRE(x_dtype >= F32 && x_dtype <= BF16 && out_dtype >= F32 && out_dtype <= BF16,
              "dtype must be FTQ_F32, FTQ_F16 or FTQ_BF16");
  if (n == 0) return FTQ_OK;
  FTQ_REQUIRE(x && signs && out, "null pointer argument");
  FTQ_REQUIRE(aligned16(x) && aligned16(out), "x and out must be 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  if (codec_any_dim(d)) e = codec_any_rht(d, x, x_dtype, n, signs, inverse, out, out_dtype, st);
  else if (d == 64) e = launch_rht_d<64>(x, x_dtype, n, signs, inverse, out, out_dtype, st);
  else if (d == 128) e = launch_rht_d<128>(x, x_dtype, n, signs, inverse, out, out_dtype, st);
  else e = launch_rht_d<256>(x, x_dtype, n, signs, inverse, out, out_dtype, st);
  return hip_status(e);
}
