/* C ABI of the MI355X compressed-KV attention library (libttkv_hip.so).
 *
 * Drop-in boundary for the hot path of ttkv-vllm's `vllm_ttkv` AttentionImpl. Every entry point
 * takes raw device pointers, sizes and the caller's HIP stream, allocates nothing, never
 * synchronises, and returns 0 on success or a TTKV_E_* code (message via ttkv_last_error(),
 * thread-local). Geometry/shape errors the host can see are refused before any launch; conditions
 * only the device can see (a block id outside the cache, a request without a registered decoder,
 * a padded slot id) set bits in the caller's `error_word` and leave the affected rows NaN-filled
 * or unwritten, never silently plausible.
 *
 * Byte format: the reference's slot layout, bit for bit (vllm_ttkv/layout.py:56-261;
 * codec/ttkv_packed_cache.py:50-271; vllm_ttkv/select_triton.py:24-91).
 */
#ifndef TTKV_HIP_H
#define TTKV_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* ttkv_stream_t; /* == hipStream_t */

enum {
  TTKV_DTYPE_F32 = 0,
  TTKV_DTYPE_F16 = 1,
  TTKV_DTYPE_BF16 = 2,
};

enum {
  TTKV_OK = 0,
  TTKV_E_INVALID = 1,     /* bad geometry / argument, refused before launch */
  TTKV_E_UNSUPPORTED = 2, /* a geometry the compiled kernels do not cover */
  TTKV_E_LAUNCH = 3,      /* hipLaunch / HIP runtime error */
  TTKV_E_WORKSPACE = 4,   /* workspace too small */
};

/* Device-side condition bits written (OR-ed) into `error_word`. */
enum {
  TTKV_ERR_NO_DECODER = 1,   /* block_table[r,0] maps to no decoder slot */
  TTKV_ERR_BAD_BLOCK = 2,    /* a block id outside [0, num_blocks) inside a request's used prefix */
  TTKV_ERR_BAD_SLOT = 4,     /* slot_mapping entry past the cache (PAD entries, < 0, are skipped) */
  TTKV_ERR_SEQ_LEN = 8,      /* seq_lens[r] (or a query count) beyond what the call was sized for (clamped), or a continuation with seq_len < q_len */
};

/* One layer's allocation. Mirrors TTKLayout(H, d, r1, qbits, res_k, res_bits, v_lanes, v_bits)
 * (vllm_ttkv/layout.py:56-74); all byte offsets are derived from these by layout.py:98-157's
 * formulas. The kernels are built for d == 128 and res_bits/v_bits in {3, 4}.
 * qbits selects the coefficient field: 8 is the reference's (r1 int8 values + one fp16 ruler);
 * 16 (r1 fp16 values, no ruler) and 4 (4-bit values in [-7, 7] as 4 * ceil(r1/8) bytes of
 * word-interleaved nibbles, then one fp16 scale per 32 ranks) are this library's own modes, with
 * no counterpart in the reference, built for num_heads / H == 3 and 64 < r1 <= 128 (other
 * shapes: TTKV_E_UNSUPPORTED). The residual rows follow the coefficient field in every mode. */
typedef struct ttkv_layout {
  int32_t H, d, r1, qbits, res_k, res_bits, v_lanes, v_bits;
} ttkv_layout;

/* Bytes of one token's blob (K slot + V slot) for `lay`, or -1 if the geometry is invalid.
 * Replaces TTKLayout.compressed_bytes_per_token (vllm_ttkv/layout.py:152-154). */
int64_t ttkv_blob_bytes(const ttkv_layout* lay);

/* Ranks R each decoder column holds in the decoder pool (dec_q [n_dec_slots, H*d, R]): 64 for
 * r1 <= 64, 128 for r1 <= 128, else r1 rounded up to a multiple of 64; -1 for r1 <= 0. Replaces
 * the reference's [r1, H*d] decoder shape (codec/ttkv_packed_cache.py:284-293), padded so that
 * every kernel reads whole 8-, 16- and 64-byte groups of ranks. */
int32_t ttkv_decoder_ranks(int32_t r1);

/* Workspaces (all four `*_workspace_bytes`): the first 64 KiB of a workspace are arrival
 * counters at a fixed place, followed by per-call partial results. A workspace must be
 * zero-filled before its first use; every call leaves the counters zero again, and no call writes
 * partials into them, so one buffer, once large enough, serves calls of any shape in turn.
 * Calls that share a workspace must not overlap in time (run them on one stream).
 *
 * Workspace bytes `ttkv_decode_paged` needs for this batch shape. */
int64_t ttkv_decode_workspace_bytes(const ttkv_layout* lay, int32_t num_heads,
                                    int32_t num_reqs, int32_t max_seq_len, int32_t block_size);

/* K1 -- fused paged decode read, ONE launch for the whole batch of decode requests.
 *
 * Replaces, per layer and step, the reference's per-request loop (vllm_ttkv/impl.py:452-493)
 * of `_decode_one` (impl.py:511-540): block_slots + gather_slots + split_blob +
 * cos_sin_from_cache (decode.py:54-122, 160-197, 286-339), `krt_from_slots`
 * (krt_triton.py:320-371), softmax(scores * scale) (impl.py:538) and `v_out_from_slots`
 * (v_out_triton.py:121-155). Semantics are vllm_ttkv/reference.py:149-163 per request:
 *   K_pre[t] = (cq[t] * float(cs16[t])) @ decoder_f[:, h*d:(h+1)*d] + residual[h, t]
 *   s[p, t]  = scale * q[p] . RoPE_t(K_pre[t])           (t = 0 .. seq_len-1, absolute position t)
 *   out[p]   = sum_t softmax_t(s[p, :]) * V[h(p), t]      h(p) = p / (num_heads / H)
 *
 * query        [N, num_heads, d] (dtype q_dtype), row of request r at query_start_loc[r].
 * page         per-layer cache viewed as bytes; slot s at page + s*slot_stride (>= blob bytes).
 * block_table  [num_reqs, bt_row_stride] int32; slot of position t = bt[r, t/bs]*bs + t%bs.
 * dec_slot_of_block [num_blocks] int32: the registry rope_store.register_decoder keys by
 *              block_table[r, 0] (rope_store.py:148-237), as a device map; -1 = none.
 * dec_q, dec_scale  the decoder pool: each slot holds one decoder_f (encode.py:178-211) in the
 *              codec's own form (ttkv_packed_cache.py:284-293), decoder_f[a, j] =
 *              float(dec_q[slot, j, a]) * dec_scale[slot, a], laid out column-major:
 *              dec_q [n_dec_slots, H*d, R] int8, dec_scale [n_dec_slots, R] fp32, R =
 *              ttkv_decoder_ranks(r1); ranks a >= r1 hold 0. Both 16-byte aligned.
 * cos_sin_cache [max_position, d] fp32, vLLM layout: cos in columns [0,d/2), sin in [d/2,d)
 *              (decode.py:54-122).
 * out          [N, num_heads, d] (dtype out_dtype); only the decode rows are written.
 * Precision: the reconstruction and the scores are carried at fp32 accuracy (hi + lo fp16 MFMA
 * operands; the query is taken as fp16); the softmax weight times the V row ruler is rounded to
 * fp16 once for the P.V MFMA (the V codes are exact integers), at a power-of-two scale that keeps
 * it below 2^15 whatever the rulers, so no finite V row overflows it. */
int ttkv_decode_paged(const ttkv_layout* lay, int32_t num_heads, float scale,
                      const void* query, int32_t q_dtype, int64_t q_row_stride,
                      const uint8_t* page, int64_t n_slots, int64_t slot_stride,
                      int32_t block_size, const int32_t* block_table, int64_t bt_row_stride,
                      int32_t max_blocks, const int32_t* seq_lens,
                      const int32_t* query_start_loc, int32_t num_reqs, int32_t max_seq_len,
                      const int32_t* dec_slot_of_block, int64_t num_blocks,
                      const int8_t* dec_q, const float* dec_scale, int64_t n_dec_slots,
                      const float* cos_sin_cache, int64_t max_position,
                      void* out, int32_t out_dtype, int64_t out_row_stride,
                      void* workspace, int64_t workspace_bytes, int32_t* error_word,
                      ttkv_stream_t stream);

/* K1 without a workspace -- NO COUNTERPART IN THE REFERENCE. For callers that cannot allocate
 * (code under HIP graph capture, serving loops or harnesses that forbid hipMalloc): the same
 * read as ttkv_decode_paged, same arguments minus `workspace`/`workspace_bytes`, same kernels and
 * results, with the split-K counters and partials in a file-scope device array of 8 MiB that
 * each device holds until the process ends. Allocates nothing (no hipMalloc / hipFree / torch).
 * A batch whose split-K state exceeds 8 MiB (ttkv_decode_workspace_bytes) is refused with
 * TTKV_E_WORKSPACE. Calls on one device share the array: calls that overlap in time on one
 * device race (issue them on one stream). Every call leaves the array's counters zero. */
int ttkv_decode_paged_noalloc(const ttkv_layout* lay, int32_t num_heads, float scale,
                              const void* query, int32_t q_dtype, int64_t q_row_stride,
                              const uint8_t* page, int64_t n_slots, int64_t slot_stride,
                              int32_t block_size, const int32_t* block_table,
                              int64_t bt_row_stride, int32_t max_blocks, const int32_t* seq_lens,
                              const int32_t* query_start_loc, int32_t num_reqs,
                              int32_t max_seq_len, const int32_t* dec_slot_of_block,
                              int64_t num_blocks, const int8_t* dec_q, const float* dec_scale, int64_t n_dec_slots,
                              const float* cos_sin_cache, int64_t max_position, void* out,
                              int32_t out_dtype, int64_t out_row_stride, int32_t* error_word,
                              ttkv_stream_t stream);

/* K3 -- write/encode of `num_tokens` new tokens into their slots, one launch per layer.
 *
 * Replaces the reference's per-request write (vllm_ttkv/impl.py:543-653): `encode_frozen(_batch)`
 * (encode.py:301-428) + `pack_and_write` / `_fused_write` (encode.py:511-603) with the coefficient
 * index_put (encode.py:570-573) and `select_triton.write_k_residual` / `write_v_rows`
 * (select_triton.py:235-303). Per token i of request r (query_start_loc[r] <= i < [r+1]):
 *   c   = M_i @ pinv                      (M_i = key[i] flattened h*d + j; pinv [H*d, r1])
 *   cs  = max|c| * fp32(1/127), 1 if 0;   cq = clamp(rint(c / cs), -128, 127)
 *   R   = key[i] - (cq * cs) @ decoder_f   -> K residual rows; value[i] -> V rows
 * written at slot_mapping[i] as the reference slot bytes (layout.py:161-239), padding zeroed.
 * When coeff_q_in/coeff_scale_in ([N, r1] int8, [N] fp32) are given, they replace the projection
 * (a first chunk written with its fit's own coefficients, encode.py:257-298).
 * In the qbits 16 / 4 modes (see ttkv_layout) c is stored as fp16(c) (round to nearest even), or
 * as q * scale per group of 32 ranks (scale = max|c| / 7 rounded up to 8 significant bits, within
 * [2^-14, 9344]; q = clamp(rint(c / scale), -7, 7)), and R = key[i] - value(c) @ decoder_f;
 * coeff_q_in must then be null (TTKV_E_INVALID).
 * Bytes are bit-exact functions of R and value (select_triton.py:24-91): exact top-k by magnitude
 * (ties -> lowest lane), ruler = rowmax * fp32(1/(2^(b-1)-1)), q = rint(x / ruler) (IEEE div).
 * coeff_out [N, r1] and resid_out [N, H*d] (optional, fp32) receive c and R.
 * dec_slot_used (optional, [n_dec_slots] int32): set to 1 for the decoder slot of every token
 *   written, so the host registry can evict decoders by last use (the caller clears it).
 * slot_mapping entries < 0 are vLLM's PAD_SLOT_ID (padded tokens of a replayed graph): skipped
 *   silently, as vLLM's cache writers do; entries past the cache set TTKV_ERR_BAD_SLOT.
 * key/value: [N, H, d] rows with the given element stride between tokens. The decoder pool
 *   (dec_q, dec_scale) is laid out as for ttkv_decode_paged; pinv_pool [n_dec_slots, r1, H*d]
 *   fp32 holds each decoder's pseudo-inverse (encode.py:193-206) transposed: row a is rank a's
 *   projection vector (the reference's pinv is [H*d, r1]; rank-major rows let the projection read
 *   whole rows).
 * Work is spread over two launches: the projection, one workgroup per (token, 4 ranks), each
 * rank's sum complete in its workgroup; then, per (token, KV head), the quantisation (every head
 * alike), the residual and the K and V rows. The projection and each token's decoder slot live in
 * `workspace` (ttkv_write_workspace_bytes). */
int ttkv_write_paged(const ttkv_layout* lay, const void* key, int32_t k_dtype, int64_t k_row_stride,
                     const void* value, int32_t v_dtype, int64_t v_row_stride,
                     const int64_t* slot_mapping, int32_t num_tokens,
                     const int32_t* query_start_loc, int32_t num_reqs, const int32_t* block_table,
                     int64_t bt_row_stride, const int32_t* dec_slot_of_block, int64_t num_blocks,
                     const int8_t* dec_q, const float* dec_scale, const float* pinv_pool,
                     int64_t n_dec_slots,
                     int32_t* dec_slot_used, const int8_t* coeff_q_in,
                     const float* coeff_scale_in, uint8_t* page, int64_t n_slots,
                     int64_t slot_stride, float* coeff_out, float* resid_out, void* workspace,
                     int64_t workspace_bytes, int32_t* error_word, ttkv_stream_t stream);

/* Workspace bytes `ttkv_write_paged` needs for `num_tokens` projected tokens (none when the
 * coefficients come from coeff_q_in); see the workspace note above ttkv_decode_workspace_bytes. */
int64_t ttkv_write_workspace_bytes(const ttkv_layout* lay, int32_t num_tokens);

/* Workspace bytes `ttkv_prefill_paged` needs for this batch shape: the split-K counters and
 * partials, and for chunks of two or more queries the expanded key tiles (49,408 B per request,
 * KV head and 64 keys, at most 1 GiB per request slice); 0 when one key split covers every query
 * block of a fused launch. See the workspace note above ttkv_decode_workspace_bytes. */
int64_t ttkv_prefill_workspace_bytes(const ttkv_layout* lay, int32_t num_heads, int32_t num_reqs,
                                     int32_t max_q_len, int32_t max_seq_len, int32_t block_size);

/* K2 -- multi-query read for chunked-prefill continuations, ONE launch over the batch.
 *
 * Replaces the reference's per-request `_prefill_continuation` (vllm_ttkv/impl.py:725-778):
 * `krt_multi_from_slots` (krt_triton.py:268-317) with p0 = seq_len - q_len, the softmax over the
 * materialised [num_heads, Q, n] scores (impl.py:771) and `v_out_multi_from_slots`
 * (v_out_triton.py:249-293). Per request r with Q = qsl[r+1]-qsl[r] queries and n = seq_lens[r]
 * stored keys (the chunk's own keys included, written before the read), p0 = n - Q:
 *   s[p, j, t] = scale * q[qsl[r]+j, p] . RoPE_t(K_pre[t]),   -inf where t > p0 + j
 *   out[qsl[r]+j, p] = sum_t softmax_t(s[p, j, :]) * V[h(p), t]
 * Chunks of two or more queries (G <= 3, r1 <= 128) run as two launches: every stored key is
 * decoded and reconstructed once into the workspace (rotated key hi + lo fp16, exact V codes, V
 * rulers), then flash attention on MFMA reads it for every 128-query block. Single queries (and
 * G = 4, 8 or r1 > 128) run one fused launch that reconstructs each key tile once per 64-query
 * block. Scores never leave the chip. Precision as for ttkv_decode_paged (the softmax weight times
 * the V ruler rounded to fp16 once, at a power-of-two scale that keeps it below 2^15).
 * req_index    optional [num_reqs] int32: batch rows to process (block_table / seq_lens /
 *              query_start_loc are indexed by it); NULL = rows 0..num_reqs-1.
 * max_q_len / max_seq_len bound Q and n over the processed rows (they size the grid).
 * Other arguments as for ttkv_decode_paged. Refused device-side: a request whose n < Q (bit
 * TTKV_ERR_SEQ_LEN), one without a decoder (TTKV_ERR_NO_DECODER, its rows are NaN). */
int ttkv_prefill_paged(const ttkv_layout* lay, int32_t num_heads, float scale,
                       const void* query, int32_t q_dtype, int64_t q_row_stride,
                       const uint8_t* page, int64_t n_slots, int64_t slot_stride,
                       int32_t block_size, const int32_t* block_table, int64_t bt_row_stride,
                       int32_t max_blocks, const int32_t* seq_lens,
                       const int32_t* query_start_loc, const int32_t* req_index,
                       int32_t num_reqs, int32_t max_q_len, int32_t max_seq_len,
                       const int32_t* dec_slot_of_block, int64_t num_blocks,
                       const int8_t* dec_q, const float* dec_scale, int64_t n_dec_slots,
                       const float* cos_sin_cache, int64_t max_position,
                       void* out, int32_t out_dtype, int64_t out_row_stride,
                       void* workspace, int64_t workspace_bytes, int32_t* error_word,
                       ttkv_stream_t stream);

/* K2, scores mode -- the continuation score tensor of ONE request (num_reqs == 1), as
 * `krt_multi_from_slots` returns it (krt_triton.py:268-317; reference.py:112-146):
 *   scores[p * s_head_stride + j * s_q_stride + t] = s[p, j, t]   fp32, -inf where t > p0 + j
 * for p < num_heads, j < Q, t < n. Reconstruction and rotated keys are carried at fp32 accuracy
 * (hi + lo fp16 MFMA operands); the query is taken as fp16. With a workspace of
 * ttkv_multi_scores_workspace_bytes (256-byte aligned; NULL / 0 allowed), a chunk of two or more
 * queries is computed from every stored key expanded once; otherwise by the fused kernel. */
int ttkv_multi_scores_paged(const ttkv_layout* lay, int32_t num_heads, float scale,
                            const void* query, int32_t q_dtype, int64_t q_row_stride,
                            const uint8_t* page, int64_t n_slots, int64_t slot_stride,
                            int32_t block_size, const int32_t* block_table,
                            int64_t bt_row_stride, int32_t max_blocks, const int32_t* seq_lens,
                            const int32_t* query_start_loc, int32_t max_q_len,
                            int32_t max_seq_len, const int32_t* dec_slot_of_block,
                            int64_t num_blocks, const int8_t* dec_q, const float* dec_scale, int64_t n_dec_slots,
                            const float* cos_sin_cache, int64_t max_position, float* scores,
                            int64_t s_head_stride, int64_t s_q_stride, void* workspace,
                            int64_t workspace_bytes, int32_t* error_word, ttkv_stream_t stream);

/* Workspace bytes with which `ttkv_multi_scores_paged` computes a chunk of two or more queries
 * (G <= 3, r1 <= 128) from every stored key expanded once (49,408 B per KV head and 64 keys);
 * 0 when the chunk takes the fused kernel. With a NULL or smaller workspace the call runs the
 * fused kernel, with the same results. -1 for an invalid layout / head count. */
int64_t ttkv_multi_scores_workspace_bytes(const ttkv_layout* lay, int32_t num_heads,
                                          int32_t max_q_len, int32_t max_seq_len);

/* Benchmark comparator (no counterpart in the compressed path): dense paged decode attention over
 * an uncompressed fp16/bf16 KV cache of the same shapes as ttkv_decode_paged's workload, for the
 * "per-cached-token cost vs dense" comparison the reference's bench makes
 * (bench_decode_read.py:132-151). Two launches: split-K over (request, token chunk) items that
 * read whole slot rows (all H heads), with a work plan computed on the device from the batch's
 * lengths, then a reduction of the chunks' partials.
 * k_cache / v_cache [n_slots, H, d] (dtype = TTKV_DTYPE_F16 or _BF16 for q, caches and out);
 * built for H = 8, G = num_heads / H in 1..4, d = 128 and a power-of-two block size. */
int64_t ttkv_dense_workspace_bytes(int32_t H, int32_t num_heads, int32_t num_reqs,
                                   int32_t max_seq_len, int32_t block_size);
int ttkv_dense_decode_paged(int32_t H, int32_t num_heads, int32_t d, float scale,
                            const void* query, int64_t q_row_stride, const void* k_cache,
                            const void* v_cache, int32_t dtype, int64_t n_slots,
                            int32_t block_size, const int32_t* block_table,
                            int64_t bt_row_stride, int32_t max_blocks, const int32_t* seq_lens,
                            const int32_t* query_start_loc, int32_t num_reqs,
                            int32_t max_seq_len, void* out, int64_t out_row_stride,
                            void* workspace, int64_t workspace_bytes, ttkv_stream_t stream);

/* Container-layout reads (the codec's pooled container, not slots): drop-ins for the codec's
 * fused container kernels `ttkv_krt` and `ttkv_v_out` (codec/ttkv_kernels.cu:208-277, 338-513),
 * as launched by codec/ttkv_cuda.py:169-257 (`krt`) and :144-166 (`v_out`).
 *
 * Container of B equal-length sequences of n tokens (codec/ttkv_packed_cache.py:337-385):
 *   coeff_q [B*n, r1] int8 and coeff_scale [B*n] fp32 (row b*n + i);
 *   decoder_f fp32 = dec_q * dec_scale, [r1, H*d] shared by the batch (decoder_per_seq = 0) or
 *     [B, r1, H*d] (decoder_per_seq = 1);
 *   rows (K residual or V): bitmap [B*H*n, d/8] u8 (16-byte aligned), packed [B*H*n, PB] u8
 *     (MSB-first codes of the set lanes in lane order), scale [B*H*n] fp32, row b*H*n + h*n + i.
 *
 * ttkv_container_krt: scores [B, num_heads, n] fp32, UNSCALED,
 *   s[b, p, i] = q[b, p] . RoPE_i((cq[i] * cs[i]) @ decoder_f[:, h*d:(h+1)*d] + resid[h, i]),
 *   h = p / (num_heads / H); cos / sin [n, d] fp32 in rope_apply's frame (absolute position i)
 *   with duplicated halves (column j == column j + d/2, as rotate-half tables are built): only
 *   columns [0, d/2) are read, as the codec kernel does (codec/ttkv_kernels.cu:472-491);
 *   query [B, num_heads, d] fp32 post-RoPE. cos, sin, query and the bitmaps are 16-byte aligned. res_bitmap = NULL: no residual (mode without rows).
 *   Carried at fp32 accuracy (hi + lo fp16 MFMA operands).
 * ttkv_container_v_out: out [B, num_heads, d] fp32 += sum_i p[b, p, i] * V[b, h, i, :];
 *   p[b, p, i] at p + b*p_batch_stride + p*p_head_stride + i. `out` must be zero-filled: the
 *   launch accumulates tile partials with atomic adds (the codec kernel's contract). Carried at
 *   fp32 accuracy (MFMA on exact integer codes against p * row scale split hi + lo in fp16 after
 *   an exact power-of-two scaling: 2^8 while every |p * scale| is below 128, and lowered by the
 *   workgroup, with its partial sums rescaled exactly, when a larger product arrives, so no
 *   finite product overflows the fp16 operand).
 * Built for d = 128, r1 <= 160, 3- or 4-bit rows of <= 48 packed bytes, num_heads / H in
 * {1, 2, 3, 4, 8}. */
int ttkv_container_krt(int32_t H, int32_t num_heads, int32_t d, int32_t B, int32_t n, int32_t r1,
                       const int8_t* coeff_q, const float* coeff_scale, const float* decoder_f,
                       int32_t decoder_per_seq, const uint8_t* res_bitmap,
                       const uint8_t* res_packed, const float* res_scale, int32_t res_pb,
                       int32_t res_bits, const float* cos, const float* sin, const float* query,
                       float* scores, ttkv_stream_t stream);
int ttkv_container_v_out(int32_t H, int32_t num_heads, int32_t d, int32_t B, int32_t n,
                         const float* p, int64_t p_head_stride, int64_t p_batch_stride,
                         const uint8_t* v_bitmap, const uint8_t* v_packed, const float* v_scale,
                         int32_t v_pb, int32_t v_bits, float* out, ttkv_stream_t stream);

/* Message for the last nonzero return on this thread. */
const char* ttkv_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* TTKV_HIP_H */
