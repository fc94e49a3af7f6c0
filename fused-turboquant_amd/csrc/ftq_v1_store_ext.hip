// vLLM v1 TURBOQUANT slot store: launches of the code widths outside
// K, V in {2, 3, 4} -- 1-bit K or V (the turboquant_k{K}v{V}_nc aliases with
// a 1, reference vllm_plugin/plugin.py:322, triton_inkernel_store.py:138-146,
// 205-229), 8-bit Lloyd-Max keys with 8-bit values, and fp8 keys with 8-bit
// values (the boundary-layer modes 8 and fp8, boundary_tq_config.py,
// triton_inkernel_store.py:59-83, 132-137).  A translation unit of its own so
// that the two sets of instantiations compile in parallel.
#include "ftq_v1_store_kernel.h"

namespace ftq {

template <int D>
static hipError_t ext_launch_d(int kb, int vb, bool kf8, int rb, const void* k, const void* v, int dt, int64_t n,
                               int hkv, const float* mids, int vflags, const int64_t* slots, uint8_t* cache,
                               int64_t nb, int bs, int64_t sb, int64_t sp, int64_t sh, const float* coeffs,
                               hipStream_t st) {
#define FTQ_EXT(KB, VB, F8) \
  return launch_fast_store3<D, KB, VB, F8>(rb, k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st)
  if (kf8) FTQ_EXT(8, 8, true);
  if (kb == 8) FTQ_EXT(8, 8, false);
  if (kb == 1) {
    if (vb == 1) FTQ_EXT(1, 1, false);
    if (vb == 2) FTQ_EXT(1, 2, false);
    if (vb == 3) FTQ_EXT(1, 3, false);
    FTQ_EXT(1, 4, false);
  }
  // vb == 1, kb in 2..4
  if (kb == 2) FTQ_EXT(2, 1, false);
  if (kb == 3) FTQ_EXT(3, 1, false);
  FTQ_EXT(4, 1, false);
#undef FTQ_EXT
}

hipError_t v1_store_ext_launch(int d, int kb, int vb, bool kf8, int rb, const void* k, const void* v, int dt,
                               int64_t n, int hkv, const float* mids, int vflags, const int64_t* slots,
                               uint8_t* cache, int64_t nb, int bs, int64_t sb, int64_t sp, int64_t sh,
                               const float* coeffs, hipStream_t st) {
  if (d == 64) return ext_launch_d<64>(kb, vb, kf8, rb, k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
  if (d == 128) return ext_launch_d<128>(kb, vb, kf8, rb, k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
  return ext_launch_d<256>(kb, vb, kf8, rb, k, v, dt, n, hkv, mids, vflags, slots, cache, nb, bs, sb, sp, sh, coeffs, st);
}

}  // namespace ftq
