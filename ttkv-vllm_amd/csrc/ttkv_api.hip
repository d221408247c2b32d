// extern "C" entry points of libttkv_hip (declared in include/ttkv_hip.h).
#include <mutex>
#include <unordered_map>
#include <vector>

#include "ttkv_host.h"

namespace ttkv {

static thread_local std::string t_err;

int host_fail(int code, const std::string& msg) {
  t_err = msg;
  return code;
}

int device_cu_count() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lk(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
  if (!cache[dev]) {
    int cu = 0;
    if (hipDeviceGetAttribute(&cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cu <= 0)
      cu = 256;
    cache[dev] = cu;
  }
  return cache[dev];
}

int raise_smem_limit(const void* kfn, size_t smem) {
  static std::mutex mu;
  static std::unordered_map<const void*, uint64_t> raised;  // kernel -> bit per device ordinal
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return host_fail(TTKV_E_LAUNCH, "hipGetDevice failed");
  const uint64_t bit = 1ull << (dev & 63);
  std::lock_guard<std::mutex> lk(mu);
  uint64_t& mask = raised[kfn];
  if (mask & bit) return TTKV_OK;
  if (hipFuncSetAttribute(kfn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem) !=
      hipSuccess)
    return host_fail(TTKV_E_LAUNCH, "hipFuncSetAttribute(MaxDynamicSharedMemorySize) failed");
  mask |= bit;
  return TTKV_OK;
}

}  // namespace ttkv

using namespace ttkv;

extern "C" {

const char* ttkv_last_error(void) { return t_err.c_str(); }

int32_t ttkv_decoder_ranks(int32_t r1) { return r1 > 0 ? dec_ranks(r1) : -1; }

int64_t ttkv_blob_bytes(const ttkv_layout* lay) {
  Geom g;
  return make_geom(lay, &g) ? g.blob : -1;
}

int64_t ttkv_decode_workspace_bytes(const ttkv_layout* lay, int32_t num_heads, int32_t num_reqs,
                                    int32_t max_seq_len, int32_t block_size) {
  Geom g;
  if (!make_geom(lay, &g) || num_heads <= 0 || num_heads % g.H || num_reqs < 0) return -1;
  if (block_size <= 0) return -1;
  return decode_workspace_bytes(g, num_heads / g.H, num_reqs, max_seq_len, block_size);
}

int ttkv_decode_paged(const ttkv_layout* lay, int32_t num_heads, float scale, const void* query,
                      int32_t q_dtype, int64_t q_row_stride, const uint8_t* page, int64_t n_slots,
                      int64_t slot_stride, int32_t block_size, const int32_t* block_table,
                      int64_t bt_row_stride, int32_t max_blocks, const int32_t* seq_lens,
                      const int32_t* query_start_loc, int32_t num_reqs, int32_t max_seq_len,
                      const int32_t* dec_slot_of_block, int64_t num_blocks, const int8_t* dec_q,
                      const float* dec_scale, int64_t n_dec_slots, const float* cos_sin_cache,
                      int64_t max_position, void* out, int32_t out_dtype, int64_t out_row_stride,
                      void* workspace, int64_t workspace_bytes, int32_t* error_word,
                      ttkv_stream_t stream) {
  Geom g;
  if (!make_geom(lay, &g)) return host_fail(TTKV_E_INVALID, "invalid layout");
  return decode_paged(g, num_heads, scale, query, q_dtype, q_row_stride, page, n_slots,
                      slot_stride, block_size, block_table, bt_row_stride, max_blocks, seq_lens,
                      query_start_loc, num_reqs, max_seq_len, dec_slot_of_block, num_blocks,
                      dec_q, dec_scale, n_dec_slots, cos_sin_cache, max_position, out, out_dtype,
                      out_row_stride, workspace, workspace_bytes, error_word,
                      (hipStream_t)stream);
}

int ttkv_decode_paged_noalloc(const ttkv_layout* lay, int32_t num_heads, float scale,
                              const void* query, int32_t q_dtype, int64_t q_row_stride,
                              const uint8_t* page, int64_t n_slots, int64_t slot_stride,
                              int32_t block_size, const int32_t* block_table, int64_t bt_row_stride,
                              int32_t max_blocks, const int32_t* seq_lens,
                              const int32_t* query_start_loc, int32_t num_reqs, int32_t max_seq_len,
                              const int32_t* dec_slot_of_block, int64_t num_blocks,
                              const int8_t* dec_q, const float* dec_scale, int64_t n_dec_slots,
                              const float* cos_sin_cache, int64_t max_position, void* out,
                              int32_t out_dtype, int64_t out_row_stride, int32_t* error_word,
                              ttkv_stream_t stream) {
  Geom g;
  if (!make_geom(lay, &g)) return host_fail(TTKV_E_INVALID, "invalid layout");
  return decode_paged_noalloc(g, num_heads, scale, query, q_dtype, q_row_stride, page, n_slots,
                              slot_stride, block_size, block_table, bt_row_stride, max_blocks,
                              seq_lens, query_start_loc, num_reqs, max_seq_len, dec_slot_of_block,
                              num_blocks, dec_q, dec_scale, n_dec_slots, cos_sin_cache,
                              max_position, out, out_dtype, out_row_stride, error_word,
                              (hipStream_t)stream);
}

int ttkv_write_paged(const ttkv_layout* lay, const void* key, int32_t k_dtype, int64_t k_row_stride,
                     const void* value, int32_t v_dtype, int64_t v_row_stride,
                     const int64_t* slot_mapping, int32_t num_tokens,
                     const int32_t* query_start_loc, int32_t num_reqs, const int32_t* block_table,
                     int64_t bt_row_stride, const int32_t* dec_slot_of_block, int64_t num_blocks,
                     const int8_t* dec_q, const float* dec_scale, const float* pinv_pool,
                     int64_t n_dec_slots, int32_t* dec_slot_used, const int8_t* coeff_q_in,
                     const float* coeff_scale_in, uint8_t* page, int64_t n_slots,
                     int64_t slot_stride, float* coeff_out, float* resid_out, void* workspace,
                     int64_t workspace_bytes, int32_t* error_word, ttkv_stream_t stream) {
  Geom g;
  if (!make_geom(lay, &g)) return host_fail(TTKV_E_INVALID, "invalid layout");
  return write_paged(g, key, k_dtype, k_row_stride, value, v_dtype, v_row_stride, slot_mapping,
                     num_tokens, query_start_loc, num_reqs, block_table, bt_row_stride,
                     dec_slot_of_block, num_blocks, dec_q, dec_scale, pinv_pool, n_dec_slots,
                     dec_slot_used, coeff_q_in,
                     coeff_scale_in, page, n_slots, slot_stride, coeff_out, resid_out, workspace,
                     workspace_bytes, error_word, (hipStream_t)stream);
}

int64_t ttkv_write_workspace_bytes(const ttkv_layout* lay, int32_t num_tokens) {
  Geom g;
  if (!make_geom(lay, &g) || num_tokens < 0) return -1;
  return write_workspace_bytes(g, num_tokens);
}

int64_t ttkv_prefill_workspace_bytes(const ttkv_layout* lay, int32_t num_heads, int32_t num_reqs,
                                     int32_t max_q_len, int32_t max_seq_len, int32_t block_size) {
  Geom g;
  if (!make_geom(lay, &g) || num_heads <= 0 || num_heads % g.H || num_reqs < 0 || block_size <= 0)
    return -1;
  return prefill_workspace_bytes(g, num_heads / g.H, num_reqs, max_q_len, max_seq_len, block_size);
}

int ttkv_prefill_paged(const ttkv_layout* lay, int32_t num_heads, float scale, const void* query,
                       int32_t q_dtype, int64_t q_row_stride, const uint8_t* page, int64_t n_slots,
                       int64_t slot_stride, int32_t block_size, const int32_t* block_table,
                       int64_t bt_row_stride, int32_t max_blocks, const int32_t* seq_lens,
                       const int32_t* query_start_loc, const int32_t* req_index, int32_t num_reqs,
                       int32_t max_q_len, int32_t max_seq_len, const int32_t* dec_slot_of_block,
                       int64_t num_blocks, const int8_t* dec_q, const float* dec_scale,
                       int64_t n_dec_slots, const float* cos_sin_cache, int64_t max_position,
                       void* out, int32_t out_dtype, int64_t out_row_stride, void* workspace,
                       int64_t workspace_bytes, int32_t* error_word, ttkv_stream_t stream) {
  Geom g;
  if (!make_geom(lay, &g)) return host_fail(TTKV_E_INVALID, "invalid layout");
  return prefill_paged(g, num_heads, scale, query, q_dtype, q_row_stride, page, n_slots,
                       slot_stride, block_size, block_table, bt_row_stride, max_blocks, seq_lens,
                       query_start_loc, req_index, num_reqs, max_q_len, max_seq_len,
                       dec_slot_of_block, num_blocks, dec_q, dec_scale, n_dec_slots, cos_sin_cache,
                       max_position, out, out_dtype, out_row_stride, nullptr, 0, 0, workspace,
                       workspace_bytes, error_word, (hipStream_t)stream);
}

int ttkv_multi_scores_paged(const ttkv_layout* lay, int32_t num_heads, float scale,
                            const void* query, int32_t q_dtype, int64_t q_row_stride,
                            const uint8_t* page, int64_t n_slots, int64_t slot_stride,
                            int32_t block_size, const int32_t* block_table, int64_t bt_row_stride,
                            int32_t max_blocks, const int32_t* seq_lens,
                            const int32_t* query_start_loc, int32_t max_q_len, int32_t max_seq_len,
                            const int32_t* dec_slot_of_block, int64_t num_blocks,
                            const int8_t* dec_q, const float* dec_scale, int64_t n_dec_slots,
                            const float* cos_sin_cache, int64_t max_position, float* scores,
                            int64_t s_head_stride, int64_t s_q_stride, void* workspace,
                            int64_t workspace_bytes, int32_t* error_word, ttkv_stream_t stream) {
  Geom g;
  if (!make_geom(lay, &g)) return host_fail(TTKV_E_INVALID, "invalid layout");
  if (!scores) return host_fail(TTKV_E_INVALID, "scores is null");
  if (workspace_bytes < 0) return host_fail(TTKV_E_INVALID, "negative workspace_bytes");
  return prefill_paged(g, num_heads, scale, query, q_dtype, q_row_stride, page, n_slots,
                       slot_stride, block_size, block_table, bt_row_stride, max_blocks, seq_lens,
                       query_start_loc, nullptr, 1, max_q_len, max_seq_len, dec_slot_of_block,
                       num_blocks, dec_q, dec_scale, n_dec_slots, cos_sin_cache, max_position,
                       nullptr, 0, 0, scores, s_head_stride, s_q_stride, workspace, workspace_bytes,
                       error_word, (hipStream_t)stream);
}

int64_t ttkv_multi_scores_workspace_bytes(const ttkv_layout* lay, int32_t num_heads,
                                          int32_t max_q_len, int32_t max_seq_len) {
  Geom g;
  if (!make_geom(lay, &g) || num_heads <= 0 || num_heads % g.H || max_q_len < 0 ||
      max_seq_len < 0)
    return -1;
  return continuation_scores_workspace_bytes(g, num_heads / g.H, max_q_len, max_seq_len);
}

int64_t ttkv_dense_workspace_bytes(int32_t H, int32_t num_heads, int32_t num_reqs,
                                   int32_t max_seq_len, int32_t block_size) {
  if (H <= 0 || num_heads <= 0 || num_heads % H || num_reqs < 0 || block_size <= 0) return -1;
  return dense_workspace_bytes(H, num_heads / H, num_reqs, max_seq_len, block_size);
}

int ttkv_dense_decode_paged(int32_t H, int32_t num_heads, int32_t d, float scale,
                            const void* query, int64_t q_row_stride, const void* k_cache,
                            const void* v_cache, int32_t dtype, int64_t n_slots,
                            int32_t block_size, const int32_t* block_table,
                            int64_t bt_row_stride, int32_t max_blocks, const int32_t* seq_lens,
                            const int32_t* query_start_loc, int32_t num_reqs,
                            int32_t max_seq_len, void* out, int64_t out_row_stride,
                            void* workspace, int64_t workspace_bytes, ttkv_stream_t stream) {
  return dense_decode_paged(H, num_heads, d, scale, query, q_row_stride, k_cache, v_cache, dtype,
                            n_slots, block_size, block_table, bt_row_stride, max_blocks, seq_lens,
                            query_start_loc, num_reqs, max_seq_len, out, out_row_stride,
                            workspace, workspace_bytes, (hipStream_t)stream);
}

int ttkv_container_krt(int32_t H, int32_t num_heads, int32_t d, int32_t B, int32_t n, int32_t r1,
                       const int8_t* coeff_q, const float* coeff_scale, const float* decoder_f,
                       int32_t decoder_per_seq, const uint8_t* res_bitmap,
                       const uint8_t* res_packed, const float* res_scale, int32_t res_pb,
                       int32_t res_bits, const float* cos, const float* sin, const float* query,
                       float* scores, ttkv_stream_t stream) {
  return container_krt(H, num_heads, d, B, n, r1, coeff_q, coeff_scale, decoder_f,
                       decoder_per_seq, res_bitmap, res_packed, res_scale, res_pb, res_bits, cos,
                       sin, query, scores, (hipStream_t)stream);
}

int ttkv_container_v_out(int32_t H, int32_t num_heads, int32_t d, int32_t B, int32_t n,
                         const float* p, int64_t p_head_stride, int64_t p_batch_stride,
                         const uint8_t* v_bitmap, const uint8_t* v_packed, const float* v_scale,
                         int32_t v_pb, int32_t v_bits, float* out, ttkv_stream_t stream) {
  return container_v_out(H, num_heads, d, B, n, p, p_head_stride, p_batch_stride, v_bitmap,
                         v_packed, v_scale, v_pb, v_bits, out, (hipStream_t)stream);
}

}  // extern "C"
