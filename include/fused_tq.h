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

/* Codebook classes for ftq_encode_cb (see ftq_codebook_class). */
enum { FTQ_CB_ANY = 0, FTQ_CB_SYMMETRIC = 1 };

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
 * Class of a codebook, from a HOST copy of boundaries [2^bits + 1]:
 * FTQ_CB_SYMMETRIC when it is sorted, boundaries[2^bits - j] == -boundaries[j]
 * in fp32 for every interior j but the middle one (j = 2^(bits-1)), and
 * |middle| < boundaries[middle + 1] -- the Lloyd-Max codebooks of d = 64 and
 * 128 are; else FTQ_CB_ANY.  Host-only: reads no device memory.
 * No reference counterpart: the reference's encode has a single path
 * (kernels/triton_encode.py:150-209).
 */
int ftq_codebook_class(const float* boundaries_host, int bits);

/*
 * ftq_encode with the codebook's class, as ftq_codebook_class returned it for
 * the values behind `boundaries`.  FTQ_CB_SYMMETRIC selects, for 16-bit x at
 * d = 128 / 256, a kernel whose search runs on |t| over the positive
 * thresholds (fewer instructions per element); given a codebook that is not
 * symmetric it returns codes as if the negative boundaries were the negated
 * positive ones.  FTQ_CB_ANY is correct for every sorted codebook.
 * ftq_encode(...) == ftq_encode_cb(..., FTQ_CB_ANY, ...).
 */
int ftq_encode_cb(const void* x, int x_dtype, int64_t n, int d, const float* signs,
                  const float* boundaries, int bits, int codebook_class, uint8_t* packed_out,
                  uint16_t* norms_out, void* stream);

/*
 * ftq_encode_cb of two tensors of the same shape with one codebook, K and V
 * of one store: k, v [n, d] (x_dtype) to k_packed_out / v_packed_out
 * [n, d*bits/8] and k_norms_out / v_norms_out [n].  For 16-bit input at
 * d = 128 / 256 one kernel launch streams both tensors (2n vectors); other
 * inputs are encoded one tensor after the other on the stream.  Outputs are
 * those of two ftq_encode_cb calls.
 * Replaces the stacked single-launch encode of
 * FusedTurboQuantCache.store_compressed_kv (reference hf/fused_cache.py:274-330),
 * which encodes torch.stack([k, v]) with one TurboQuantMSE.encode.
 */
int ftq_encode_kv(const void* k, const void* v, int x_dtype, int64_t n, int d, const float* signs,
                  const float* boundaries, int bits, int codebook_class, uint8_t* k_packed_out,
                  uint16_t* k_norms_out, uint8_t* v_packed_out, uint16_t* v_norms_out, void* stream);

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

/* ---------------------------------------------------------------------------
 * Paged library-format KV cache (this library's page format).
 *
 * kv_cache: uint8 [num_blocks][num_kv_heads][page_size/16][sub_bytes], one
 * 16-token sub-block of one kv head = K codes [16][d*bits_k/8] (reference bit
 * layout) | V codes in MFMA lane order [64][d*bits_v/32] | K norms fp16[16] |
 * V norms fp16[16].  sub_bytes = 2*d*(bits_k+bits_v) + 64.  d in {128, 256},
 * page_size a multiple of 16.  A token's slot is block*page_size + offset.
 * ------------------------------------------------------------------------- */
int64_t ftq_paged_subblock_bytes(int d, int bits_k, int bits_v);

/*
 * Encode K and V ([n_tokens][num_kv_heads][d], dtype) with the library
 * codec and scatter them to slot_mapping[n_tokens] (int64; slots < 0 or in a
 * block >= num_blocks are skipped).  Replaces the reference's per-token
 * compressed-slot writes (vllm_plugin/attention_impl.py:217-254 with
 * cache_ops.py:85-108 write_compressed_to_slot) and the fused v1 store
 * launch (vllm_plugin/triton_inkernel_store.py:554-616) for this codec.
 */
int ftq_paged_store(const void* key, const void* value, int dtype, int64_t n_tokens,
                    int num_kv_heads, int d, const float* k_signs, const float* v_signs,
                    const float* k_boundaries, const float* v_boundaries, int bits_k, int bits_v,
                    const int64_t* slot_mapping, uint8_t* kv_cache, int page_size,
                    int64_t num_blocks, void* stream);

/* Workspace bytes ftq_paged_decode_attention needs: batch*Hq*splits*(d+1)*4. */
int64_t ftq_paged_workspace_bytes(int batch, int num_q_heads, int d, int num_splits);
/* Split-K factor that fills the GPU for this shape (host-side heuristic). */
int ftq_paged_default_splits(int batch, int num_kv_heads, int max_seq_len);
/* Split factor for ftq_paged_decode_attention with the head geometry known: 1
 * (the single-launch form below) when d = 128, Hq/Hkv <= 4 and batch*Hkv fills
 * the 256 CUs in whole rounds of at least 3/4, else ftq_paged_default_splits.
 * Host-side heuristic; no counterpart in the reference, whose Triton launch
 * picks its grid in kernels/triton_flash_decode.py:224-324. */
int ftq_paged_choose_splits(int batch, int num_q_heads, int num_kv_heads, int d, int max_seq_len);

/*
 * Decode attention (one query token per sequence) over the paged cache:
 * out[b][h] = softmax(q[b][h] . K_b^T * scale) . V_b, K/V the decoded cache,
 * kv head = h / (Hq/Hkv), positions >= seq_lens[b] masked, block_table
 * [batch][max_blocks_per_seq] int32 physical block ids.  q is RHT-rotated
 * in-kernel with k_signs; the output is un-rotated with v_signs.
 * Replaces the library-format decode of the reference
 * (vllm_plugin/attention_impl.py:431-521: _gather_compressed_k +
 * randomized_hadamard + fused_qk_scores_rht + softmax + V decode + matmul) and
 * flash_decode_compressed (kernels/triton_flash_decode.py:224-324).
 * num_splits == 1 with d = 128 and Hq/Hkv <= 4: one launch on `stream`, one
 * 16-wave workgroup per (batch, kv head) that merges its waves and writes the
 * output (inverse RHT, out_dtype); the workspace is not touched.  Otherwise
 * two launches: split-K stage 1 into the workspace, then merge + inverse RHT.
 */
int ftq_paged_decode_attention(const void* query, int q_dtype, const uint8_t* kv_cache,
                               const int32_t* block_table, const int32_t* seq_lens, int batch,
                               int num_q_heads, int num_kv_heads, int d, int page_size,
                               int max_blocks_per_seq, int64_t num_blocks, const float* k_signs,
                               const float* v_signs, const float* k_levels, const float* v_levels,
                               int bits_k, int bits_v, float scale, int num_splits, void* workspace,
                               int64_t workspace_bytes, void* out, int out_dtype, void* stream);

/*
 * ftq_paged_decode_attention with every product in fp32 on the VALU (fp32
 * level tables, fp32 rotated query, fp32 weights times norms), the
 * arithmetic of the reference's flash_decode_compressed
 * (kernels/triton_flash_decode.py:66-221); same arguments and semantics.
 * Always the split form (stage 1 into the workspace, then the merge + inverse
 * RHT launch).  d = 128 and at most 4 query heads per kv head.  About 2.3x the
 * time of the default matrix-core form at B = 32, 32 / 8 heads, 8192
 * positions, 3-bit K and V.
 */
int ftq_paged_decode_attention_valu(const void* query, int q_dtype, const uint8_t* kv_cache,
                                    const int32_t* block_table, const int32_t* seq_lens, int batch,
                                    int num_q_heads, int num_kv_heads, int d, int page_size,
                                    int max_blocks_per_seq, int64_t num_blocks, const float* k_signs,
                                    const float* v_signs, const float* k_levels,
                                    const float* v_levels, int bits_k, int bits_v, float scale,
                                    int num_splits, void* workspace, int64_t workspace_bytes, void* out,
                                    int out_dtype, void* stream);

/* ---- vLLM v1 TURBOQUANT slot format ------------------------------------
 * kv_cache uint8 [num_blocks][block_size][num_kv_heads][slot] (strides in
 * bytes); per (token, kv head) slot:
 *   [K codes d*kb/8][K norm f16][V codes d*vb/8][V scale f16][V min f16][pad]
 * (reference vllm_plugin/triton_inkernel_store.py:38-330,
 * boundary_tq_config.py:66-81, v1_backend.py:171-220).  Code widths: K and V
 * both in 1..4, or both 8 (the 8-bit boundary layers: 256 Lloyd-Max
 * centroids for K, 8-bit uniform V).  FP8 keys (v_flags bit 2, key_bits 8):
 * d bytes of fp8 e4m3fn K, no K norm: [K fp8 d][V codes][V scale][V min].
 * The int v_rotate argument of the store and decode entry points is this
 * bit set (FTQ_V1_*): bit 0 V rotated, bit 1 Lloyd-Max V codes (4-bit V),
 * bit 2 fp8 keys, bit 3 (decode only) fp32 products on the VALU.
 */
#define FTQ_V1_VROT 1
#define FTQ_V1_VLLOYD 2
#define FTQ_V1_KFP8 4
#define FTQ_V1_FP32 8

/* Bytes of a slot that hold data (key_packed_size + value bytes + 4), or -1
 * for an unsupported shape.  Replaces BoundaryTurboQuantConfig.key_packed_size /
 * value_data_bytes (boundary_tq_config.py:66-81); the slot stride itself is the
 * caller's (v1_backend.py:171-209 rounds it up to a power of two). */
int64_t ftq_v1_slot_bytes(int d, int key_bits, int value_bits);
/* ftq_v1_slot_bytes for a v_flags bit set: with FTQ_V1_KFP8 the key part is d
 * bytes of fp8 and no norm (BoundaryTurboQuantConfig.key_packed_size with
 * key_fp8, boundary_tq_config.py:66-73). */
int64_t ftq_v1_slot_bytes_flags(int d, int key_bits, int value_bits, int v_flags);

/*
 * Store n_tokens x num_kv_heads K/V vectors ([n][Hkv][d], dtype) into their
 * slots: K normalised, rotated by the unsigned Hadamard H/sqrt(d), quantised
 * against `midpoints` (2^key_bits - 1 sorted float32; code = number of
 * midpoints <= y), norm stored fp16; V (rotated first and rounded back to
 * dtype when v_rotate) quantised uniformly between its min and max.
 * v_rotate is a bit set: bit 0 rotates V; bit 1 (value_bits 4 only, with
 * bit 0) stores V as Lloyd-Max codes instead (TURBOQUANT_V_LLOYD_MAX): the
 * rotated V is normalised and coded against `midpoints` like K, its fp16 norm
 * goes to the scale field and 0 to the min field (v1_backend.py:736-749,
 * triton_inkernel_store.py:159-200); bit 2 stores K as fp8 e4m3fn
 * (key_bits 8; y * norm rounded to nearest even, saturating at +-448; no
 * norm; `midpoints` unused, triton_inkernel_store.py:59-83).  1-bit codes
 * (:138-146, :205-229) and 8-bit K / V (:132-137, 8-bit V :202-330) as the
 * reference packs them.
 * slot_mapping[i] < 0 skips token i.  Replaces _launch_rht / _fused_store_rht
 * (vllm_plugin/triton_inkernel_store.py:376-440, 554-616) and the V
 * pre-rotation of _launch_store (v1_backend.py:712-749).  One launch.
 */
int ftq_v1_store(const void* key, const void* value, int dtype, int64_t n_tokens,
                 int num_kv_heads, int d, const float* midpoints, int key_bits, int value_bits,
                 int v_rotate, const int64_t* slot_mapping, uint8_t* kv_cache,
                 int64_t num_blocks, int block_size, int64_t stride_block, int64_t stride_pos,
                 int64_t stride_head, void* stream);
/*
 * ftq_v1_store with the rotation of a matrix strategy: K (and V when
 * v_rotate) rotated by x M, `rotation` = M row-major d x d float32 on the
 * device (NULL = the unsigned Hadamard H/sqrt(d)).  Replaces the in-kernel
 * (D, D) and block-diagonal rotations of _fused_store_matrix /
 * _fused_store_block_diag (vllm_plugin/triton_inkernel_store.py:459-541,
 * 649-744) behind MatrixRotationStrategy.launch_store
 * (vllm_plugin/rotation/matrix.py:50-70): planar, rotor, iso.
 */
int ftq_v1_store_rot(const void* key, const void* value, int dtype, int64_t n_tokens,
                     int num_kv_heads, int d, const float* midpoints, int key_bits, int value_bits,
                     int v_rotate, const int64_t* slot_mapping, uint8_t* kv_cache,
                     int64_t num_blocks, int block_size, int64_t stride_block, int64_t stride_pos,
                     int64_t stride_head, const float* rotation, void* stream);

/*
 * ftq_v1_store for the block-diagonal rotation strategies (planar B = 2,
 * rotor B = 3, iso_fast / iso_full B = 4): K (and V when v_rotate) rotated
 * by x M with M given by its coefficients coeffs[B][d] (float32, device),
 * coeffs[j][e] = M[(e / B) B + j][e] (0 where that row is past d); K is
 * normalised by multiplying with 1 / (norm + 1e-8) and y[e] =
 * sum_j x[(e / B) B + j] coeffs[j][e] is formed by fused multiply-adds in
 * j order.  O(B d) work per vector.  Replaces _launch_block_diag /
 * _fused_store_block_diag (vllm_plugin/triton_inkernel_store.py:649-860)
 * behind BlockDiagonalRotationStrategy.launch_store
 * (vllm_plugin/rotation/matrix.py:126-148) and the V pre-rotation of
 * _launch_store (v1_backend.py:736-740).
 */
int ftq_v1_store_blockdiag(const void* key, const void* value, int dtype, int64_t n_tokens,
                           int num_kv_heads, int d, const float* midpoints, int key_bits,
                           int value_bits, int v_rotate, const int64_t* slot_mapping,
                           uint8_t* kv_cache, int64_t num_blocks, int block_size,
                           int64_t stride_block, int64_t stride_pos, int64_t stride_head,
                           const float* coeffs, int block, void* stream);

/* Workspace bytes ftq_v1_decode_attention needs: batch*Hq*splits*(d+1)*4. */
int64_t ftq_v1_workspace_bytes(int batch, int num_q_heads, int d, int num_splits);
/* Split-K factor that fills the GPU for this shape (host-side heuristic): 1
 * once batch*Hkv >= 384.  With one split ftq_v1_decode_attention writes the
 * output from the attention kernel itself (no merge launch; the workspace is
 * still checked but not written) unless a caller rotation matrix is given. */
int ftq_v1_default_splits(int batch, int num_kv_heads, int max_seq_len);
/* Split-K factor with the head geometry and slot format known: for the
 * matrix-core kernels (d = 128, 2-4 bit K and V, no FTQ_V1_KFP8 / FTQ_V1_FP32
 * flag) the most splits whose batch*Hkv*splits workgroups the GPU holds at
 * once (the kernel's occupancy, from the HIP runtime), leaving at least 8
 * tiles of 32 positions per wave, at most 64; other formats take
 * ftq_v1_default_splits.  Host-side heuristic; no counterpart in the
 * reference, whose decode takes vLLM's fixed NUM_KV_SPLITS
 * (vllm_plugin/v1_backend.py:568-573, 895). */
int ftq_v1_choose_splits(int batch, int num_q_heads, int num_kv_heads, int d, int key_bits,
                         int value_bits, int v_flags, int max_seq_len);

/*
 * Decode attention over the slot cache, one query token per sequence:
 * positions [kv_start[b], seq_lens[b]) of block_table row b (kv_start may be
 * NULL = 0), kv head = h / (Hq/Hkv); scores use the rotated query q H/sqrt(d)
 * against the norm-corrected centroids (2^key_bits sorted float32) times the
 * fp16 K norm; V = code * scale + min; with v_rotate the output is multiplied
 * by H/sqrt(d).  v_rotate bit 1 (as in ftq_v1_store) reads Lloyd-Max V
 * codes: V = c[code] * ||v|| / ||c[codes]|| (triton_decode_offset.py:399-419);
 * bit 2 reads fp8 keys (scores q_rot . k_fp8, :174-192; `centroids` unused
 * then).  Rows with no positions give 0.  Replaces the stage-1 kernel
 * _tq_decode_stage1_offset (vllm_plugin/triton_decode_offset.py:42-442), the
 * stage-2 merge, the un-rotation and the output cast of
 * _decode_attention_offset_only (v1_backend.py:975-1093).  Head dim 64, 128
 * or 256.  Two launches on `stream`: split-K stage 1, then merge.  Head dim
 * 128 with 2-4 bit codes runs the matrix-core kernels (f16 operands, fp32
 * accumulation); every other format, or v_rotate bit 3, runs a kernel with
 * every product in fp32 on the VALU (the reference's arithmetic).
 */
int ftq_v1_decode_attention(const void* query, int q_dtype, const uint8_t* kv_cache,
                            int64_t num_blocks, int block_size, int64_t stride_block,
                            int64_t stride_pos, int64_t stride_head, const int32_t* block_table,
                            int max_blocks_per_seq, const int32_t* seq_lens,
                            const int32_t* kv_start, int batch, int num_q_heads, int num_kv_heads,
                            int d, const float* centroids, int key_bits, int value_bits,
                            float scale, int v_rotate, int num_splits, void* workspace,
                            int64_t workspace_bytes, void* out, int out_dtype, void* stream);
/*
 * ftq_v1_decode_attention that also writes each row's natural-log
 * log-sum-exp of the scaled scores to lse_out[batch * Hq] (float32; -inf for a
 * row with no positions; NULL = not written).  Replaces the (output, lse)
 * pair of the quantised phase of _decode_attention_hybrid
 * (vllm_plugin/v1_backend.py:1185-1262), merged there with the fp16 prefix.
 */
int ftq_v1_decode_attention_lse(const void* query, int q_dtype, const uint8_t* kv_cache,
                                int64_t num_blocks, int block_size, int64_t stride_block,
                                int64_t stride_pos, int64_t stride_head, const int32_t* block_table,
                                int max_blocks_per_seq, const int32_t* seq_lens,
                                const int32_t* kv_start, int batch, int num_q_heads, int num_kv_heads,
                                int d, const float* centroids, int key_bits, int value_bits,
                                float scale, int v_rotate, int num_splits, void* workspace,
                                int64_t workspace_bytes, void* out, int out_dtype, float* lse_out,
                                void* stream);
/*
 * ftq_v1_decode_attention_lse for a matrix strategy: the query is rotated
 * by q M and, with v_rotate, the output by o M^T, `rotation` = M row-major
 * d x d float32 on the device (NULL = H/sqrt(d)).  Replaces
 * rotate_for_decode's q @ M (vllm_plugin/rotation/matrix.py:47-48) and the
 * o @ M^T un-rotation (v1_backend.py:1086-1092) around stage 1.
 */
int ftq_v1_decode_attention_rot(const void* query, int q_dtype, const uint8_t* kv_cache,
                                int64_t num_blocks, int block_size, int64_t stride_block,
                                int64_t stride_pos, int64_t stride_head, const int32_t* block_table,
                                int max_blocks_per_seq, const int32_t* seq_lens,
                                const int32_t* kv_start, int batch, int num_q_heads, int num_kv_heads,
                                int d, const float* centroids, int key_bits, int value_bits,
                                float scale, int v_rotate, int num_splits, void* workspace,
                                int64_t workspace_bytes, void* out, int out_dtype, float* lse_out,
                                const float* rotation, void* stream);

/* Bytes of the device scratch array ftq_v1_decode_attention_noalloc uses in
 * place of a workspace (16 MiB per device). */
int64_t ftq_v1_scratch_bytes(void);
/*
 * ftq_v1_decode_attention without the workspace argument: allocates nothing
 * and takes no workspace.  The split-K partials go to a file-scope device
 * array of ftq_v1_scratch_bytes() bytes, which each GPU the library runs on
 * holds until the process ends; its device address is looked up once per
 * device on the first call there.  Rejects (FTQ_ERR_ARG) a shape whose
 * ftq_v1_workspace_bytes exceeds that size, and a stream of another device
 * than the current one.  All calls on one GPU share its array: calls that
 * overlap on one GPU race.  Results equal ftq_v1_decode_attention's.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).
 */
int ftq_v1_decode_attention_noalloc(const void* query, int q_dtype, const uint8_t* kv_cache,
                                    int64_t num_blocks, int block_size, int64_t stride_block,
                                    int64_t stride_pos, int64_t stride_head,
                                    const int32_t* block_table, int max_blocks_per_seq,
                                    const int32_t* seq_lens, const int32_t* kv_start, int batch,
                                    int num_q_heads, int num_kv_heads, int d,
                                    const float* centroids, int key_bits, int value_bits,
                                    float scale, int v_rotate, int num_splits, void* out,
                                    int out_dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Raw fp16 slots of the boundary-protection layers (TURBOQUANT_BOUNDARY_PROTECT
 * = fp16): the same [num_blocks][block_size][Hkv][slot] byte cache, per
 * (token, kv head) [K fp16 (2 d bytes)][V fp16 (2 d bytes)][pad], the layout of
 * the reference's _store_raw_kv (vllm_plugin/v1_backend.py:1449-1505).
 * ------------------------------------------------------------------------- */

/* Bytes of a raw slot that hold data: 4 * d (-1 for an unsupported d). */
int64_t ftq_raw_slot_bytes(int d);

/*
 * Store n_tokens x num_kv_heads K/V vectors ([n][Hkv][d], dtype) as fp16
 * (round to nearest even) into their raw slots; slot_mapping[i] < 0 skips
 * token i (and a slot past the cache is skipped too).  Replaces _store_raw_kv
 * (vllm_plugin/v1_backend.py:1449-1505).  One launch.  Strides in bytes,
 * multiples of 16.
 */
int ftq_raw_store(const void* key, const void* value, int dtype, int64_t n_tokens,
                  int num_kv_heads, int d, const int64_t* slot_mapping, uint8_t* kv_cache,
                  int64_t num_blocks, int block_size, int64_t stride_block, int64_t stride_pos,
                  int64_t stride_head, void* stream);

/* Workspace bytes ftq_raw_decode_attention needs: batch*Hq*splits*(d+1)*4. */
int64_t ftq_raw_workspace_bytes(int batch, int num_q_heads, int d, int num_splits);
/* Split-K factor that fills the GPU for this shape (host-side heuristic). */
int ftq_raw_default_splits(int batch, int num_kv_heads, int max_seq_len);

/*
 * Decode attention over raw fp16 slots, one query token per sequence:
 * softmax(q . K^T * scale) . V over positions [kv_start[b], seq_lens[b]) of
 * block_table row b (kv_start may be NULL = 0), kv head = h / (Hq/Hkv); rows
 * with no positions give 0.  Replaces boundary_fp16_decode_attention
 * (vllm_plugin/triton_boundary_attn.py:28-219) as called by _forward_raw
 * (v1_backend.py:1547-1640).  Head dim 128, GQA group <= 8.  Two launches on
 * `stream`: split-K stage 1, then merge.
 */
int ftq_raw_decode_attention(const void* query, int q_dtype, const uint8_t* kv_cache,
                             int64_t num_blocks, int block_size, int64_t stride_block,
                             int64_t stride_pos, int64_t stride_head, const int32_t* block_table,
                             int max_blocks_per_seq, const int32_t* seq_lens,
                             const int32_t* kv_start, int batch, int num_q_heads,
                             int num_kv_heads, int d, float scale, int num_splits, void* workspace,
                             int64_t workspace_bytes, void* out, int out_dtype, void* stream);
/*
 * ftq_raw_decode_attention that also writes each row's natural-log
 * log-sum-exp of the scaled scores to lse_out[batch * Hq] (float32; -inf for a
 * row with no positions; NULL = not written).  Replaces the flash-attention
 * call over the deferred fp16 prefix (out, softmax lse) of
 * _decode_attention_hybrid (vllm_plugin/v1_backend.py:1131-1172).
 */
int ftq_raw_decode_attention_lse(const void* query, int q_dtype, const uint8_t* kv_cache,
                                 int64_t num_blocks, int block_size, int64_t stride_block,
                                 int64_t stride_pos, int64_t stride_head, const int32_t* block_table,
                                 int max_blocks_per_seq, const int32_t* seq_lens,
                                 const int32_t* kv_start, int batch, int num_q_heads,
                                 int num_kv_heads, int d, float scale, int num_splits, void* workspace,
                                 int64_t workspace_bytes, void* out, int out_dtype, float* lse_out,
                                 void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FUSED_TQ_H */
