// vLLM v1 TURBOQUANT slot store on gfx950: the entry points and the
// launches of the K, V in {2, 3, 4} combinations (the kernel itself is in
// ftq_v1_store_kernel.h; 1-bit codes, 8-bit K / V and fp8 keys are launched
// from ftq_v1_store_ext.hip).
#include "ftq_v1_store_kernel.h"
#include "ftq_v1_store_mfma.h"

namespace ftq {

// The matrix-core store (ftq_v1_store_mfma.h) takes: the Hadamard rotation at
// d = 128, 16-bit inputs, K and V in 2..4 bits, no Lloyd-Max V, and 32-bit
// vector and slot numbers; and at least 32768 (token, head) vectors.  Below
// that its one wave per 16 vectors leaves the GPU part idle, and the VALU
// store (16 lanes per vector) is faster: 1024 tokens x 8 heads took 4.1 us
// there against 5.3 us on the matrix cores; 32768 x 8 took 72 us against 41.
static bool v1_store_mfma_ok(int d, int dt, int kb, int vb, int flags, int rb, int64_t nvec, int64_t slots_total) {
  const bool vlm = (flags & V1F_VLM) != 0 && vb == 4;
  return rb == 0 && d == 128 && dt != F32 && kb >= 2 && kb <= 4 && vb >= 2 && vb <= 4 && !vlm &&
         (flags & V1F_KFP8) == 0 && nvec >= 32768 && nvec < ((int64_t)1 << 31) - 64 &&
         slots_total < ((int64_t)1 << 31);
}

template <int DT, int KB, int VB>
static hipError_t launch_store_mfma3(const void* k, const void* v, int64_t nvec, int hkv, const float* mids,
                                     int vflags, const int64_t* slots, uint8_t* cache, int64_t slots_total, int bs,
                                     int64_t sb, int64_t sp, int64_t sh, hipStream_t st) {
  // one pass of resident workgroups, each wave looping over groups of 16 vectors
  static const int cap = resident_workgroups(v1_store_mfma_kernel<DT, KB, VB>);
  const int64_t want = ((nvec + 15) / 16 + 3) / 4;
  v1_store_mfma_kernel<DT, KB, VB><<<dim3((unsigned)(want < cap ? want : cap)), dim3(256), 0, st>>>(
      k, v, (int)nvec, hkv, FastDiv::make(hkv), mids, vflags, slots, cache, (int)slots_total, bs,
      FastDiv::make(bs), sb, sp, sh, fwht_scale(128));
  return hipGetLastError();
}

template <int DT, int KB>
static hipError_t launch_store_mfma2(int vb, const void* k, const void* v, int64_t nvec, int hkv, const float* mids,
                                     int vflags, const int64_t* slots, uint8_t* cache, int64_t slots_total, int bs,
                                     int64_t sb, int64_t sp, int64_t sh, hipStream_t st) {
  if (vb == 2) return launch_store_mfma3<DT, KB, 2>(k, v, nvec, hkv, mids, vflags, slots, cache, slots_total, bs, sb, sp, sh, st);
  if (vb == 3) return launch_store_mfma3<DT, KB, 3>(k, v, nvec, hkv, mids, vflags, slots, cache, slots_total, bs, sb, sp, sh, st);
  return launch_store_mfma3<DT, KB, 4>(k, v, nvec, hkv, mids, vflags, slots, cache, slots_total, bs, sb, sp, sh, st);
}

template <int DT>
static hipError_t launch_store_mfma1(int kb, int vb, const void* k, const void* v, int64_t nvec, int hkv,
                                     const float* mids, int vflags, const int64_t* slots, uint8_t* cache,
                                     int64_t slots_total, int bs, int64_t sb, int64_t sp, int64_t sh, hipStream_t st) {
  if (kb == 2) return launch_store_mfma2<DT, 2>(vb, k, v, nvec, hkv, mids, vflags, slots, cache, slots_total, bs, sb, sp, sh, st);
  if (kb == 3) return launch_store_mfma2<DT, 3>(vb, k, v, nvec, hkv, mids, vflags, slots, cache, slots_total, bs, sb, sp, sh, st);
  return launch_store_mfma2<DT, 4>(vb, k, v, nvec, hkv, mids, vflags, slots, cache, slots_total, bs, sb, sp, sh, st);
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

// Code widths with a store and a decode: K, V in 1..4, or both 8 (8-bit
// Lloyd-Max keys with 8-bit values, or fp8 keys with 8-bit values -- the
// boundary-layer modes of reference vllm_plugin/boundary_tq_config.py).
bool v1_widths_ok(int kb, int vb, int flags) {
  if (flags & V1F_KFP8) return kb == 8 && vb == 8;
  if (kb == 8 || vb == 8) return kb == 8 && vb == 8;
  return kb >= 1 && kb <= 4 && vb >= 1 && vb <= 4;
}

// Shared argument checks of the slot stores; 0 = fine.
int v1_store_checks(int d, int key_bits, int value_bits, int64_t n_tokens, int num_kv_heads, int64_t num_blocks,
                    int block_size, int dtype, int v_rotate, int64_t stride_block, int64_t stride_pos,
                    int64_t stride_head) {
  FTQ_REQUIRE(d == 64 || d == 128 || d == 256, "v1 store: head_dim must be 64, 128 or 256");
  FTQ_REQUIRE(v_rotate >= 0 && v_rotate <= 7,
              "v_flags: bit 0 = rotate V, bit 1 = Lloyd-Max V codes, bit 2 = fp8 keys");
  FTQ_REQUIRE(v1_widths_ok(key_bits, value_bits, v_rotate),
              "v1 store: key_bits and value_bits must both be in 1..4, or both 8 (fp8 keys: both 8)");
  FTQ_REQUIRE(n_tokens >= 0 && num_kv_heads > 0 && num_blocks >= 0 && block_size > 0,
              "bad token / head / block counts");
  FTQ_REQUIRE(dtype >= F32 && dtype <= BF16, "dtype must be FTQ_F32, FTQ_F16 or FTQ_BF16");
  const V1Geom g = v1_geom(d, key_bits, value_bits, (v_rotate & V1F_KFP8) != 0);
  FTQ_REQUIRE(stride_head >= g.raw, "stride_head is smaller than the slot bytes (see ftq_v1_slot_bytes)");
  FTQ_REQUIRE(cache_strides_ok(num_blocks, stride_block, stride_pos, stride_head, num_kv_heads, block_size),
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
  FTQ_REQUIRE(key && value && slot_mapping && kv_cache, "null pointer argument");
  FTQ_REQUIRE(midpoints != nullptr || (v_rotate & V1F_KFP8) != 0, "null midpoints");
  FTQ_REQUIRE(rb == 0 || coeffs != nullptr, "null coefficient pointer");
  FTQ_REQUIRE(aligned16(key) && aligned16(value), "key/value must be 16-byte aligned");
  FTQ_REQUIRE(aligned4(kv_cache), "kv_cache must be 4-byte aligned");
  FTQ_REQUIRE(coeffs == nullptr || aligned4(coeffs), "coefficients must be 4-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  hipError_t e;
  const bool kf8 = (v_rotate & V1F_KFP8) != 0;
  const int64_t nvec = n_tokens * num_kv_heads;
  const int64_t slots_total = num_blocks * (int64_t)block_size;
  if (v1_store_mfma_ok(d, dtype, key_bits, value_bits, v_rotate, rb, nvec, slots_total)) {
    if (dtype == F16)
      e = launch_store_mfma1<F16>(key_bits, value_bits, key, value, nvec, num_kv_heads, midpoints, v_rotate,
                                  slot_mapping, kv_cache, slots_total, block_size, stride_block, stride_pos,
                                  stride_head, st);
    else
      e = launch_store_mfma1<BF16>(key_bits, value_bits, key, value, nvec, num_kv_heads, midpoints, v_rotate,
                                   slot_mapping, kv_cache, slots_total, block_size, stride_block, stride_pos,
                                   stride_head, st);
  } else if (kf8 || key_bits < 2 || key_bits > 4 || value_bits < 2 || value_bits > 4)
    e = v1_store_ext_launch(d, key_bits, value_bits, kf8, rb, key, value, dtype, n_tokens, num_kv_heads, midpoints,
                            v_rotate, slot_mapping, kv_cache, num_blocks, block_size, stride_block, stride_pos,
                            stride_head, coeffs, st);
  else if (d == 64)
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
