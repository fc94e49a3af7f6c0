/*
 * fused_tq.h -- C ABI of the MI355X (gfx950) fused-turboquant KV-cache hot path.
 *
 * Every entry point takes plain device pointers, sizes and a hipStream_t
 * (passed as void*), enqueues its kernels on that stream, performs no host
 * synchronisation and allocates nothing unless its comment says otherwise.
 * Return value: FTQ_OK (0) on success, FTQ_ERR_ARG (-1) for a rejected
 * argument (message in ftq_last_error()), or a positive hipError_t from the
 * launch.
 *
 * Pointers to floats (signs, boundaries, levels, centroids, midpoints) are
 * device pointers, float32.  fp16 values (norms, scales) are passed as raw
 * uint16_t bit patterns.  dtype codes: FTQ_F32, FTQ_F16, FTQ_BF16.
 */
#ifndef FUSED_TQ_H
#define FUSED_TQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FTQ_ABI_VERSION 1
#define FTQ_OK 0
#define FTQ_ERR_ARG (-1)

enum { FTQ_F32 = 0, FTQ_F16 = 1, FTQ_BF16 = 2 };

/* Message of the last FTQ_ERR_ARG / HIP error raised on this host thread. */
const char* ftq_last_error(void);
int ftq_version(void);

/*
 * Fused library-format encode: RHT (x * signs, FWHT, * d^-1/2), per-vector
 * L2 norm, u = y / (norm + 1e-8), code = clamp(bucketize(u, boundaries) - 1),
 * 2/3/4-bit pack, norm stored as fp16.
 *   x          [n, d] (x_dtype), 16-byte aligned, rows contiguous
 *   signs      [d] (+-1), boundaries [2^bits + 1] (interior ones are used)
 *   packed_out [n, d*bits/8] uint8, norms_out [n] fp16 bits
 * Replaces triton_fused_encode (reference kernels/triton_encode.py:150-209)
 * as called by TurboQuantMSE._encode_fused (core/quantizer.py:121-135), with
 * the numerics of TurboQuantMSE._encode_unfused (core/quantizer.py:137-160).
 */
int ftq_encode(const void* x, int x_dtype, int64_t n, int d, const float* signs,
               const float* boundaries, int bits, uint8_t* packed_out, uint16_t* norms_out,
               void* stream);

/*
 * Fused library-format decode: unpack, levels[code] * norm, FWHT, * d^-1/2,
 * * signs.  out [n, d] in out_dtype (FTQ_F32 matches the reference).
 * Replaces triton_fused_decode (reference kernels/triton_decode.py:104-155)
 * as called by TurboQuantMSE._decode_fused (core/quantizer.py:175-189), with
 * the numerics of _decode_unfused (core/quantizer.py:191-205).
 */
int ftq_decode(const uint8_t* packed, const uint16_t* norms, int64_t n, int d,
               const float* levels, const float* signs, int bits, void* out, int out_dtype,
               void* stream);

/*
 * Randomized Hadamard transform of n rows of d elements:
 *   forward: fwht(x * signs), inverse: fwht(x) * signs (orthonormal).
 * Replaces triton_rht (reference kernels/triton_rht.py:82-121) as called by
 * RHTRotation.forward / inverse (core/hadamard.py:141-153).
 */
int ftq_rht(const void* x, int x_dtype, int64_t n, int d, const float* signs, int inverse,
            void* out, int out_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FUSED_TQ_H */
