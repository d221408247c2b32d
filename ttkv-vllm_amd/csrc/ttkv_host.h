// Host-side shared state of libttkv_hip: thread-local error text and device properties.
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <string>

#include "ttkv_common.h"

namespace ttkv {

int host_fail(int code, const std::string& msg);
int device_cu_count();

// Raise a kernel's dynamic LDS limit to `smem` bytes on the current device, once per (kernel,
// device): the attribute is per device.
int raise_smem_limit(const void* kfn, size_t smem);

// The decoder pool (dec_q / dec_scale, laid out as dec_ranks describes): the kernels read 8 and
// 16 ranks of a column, and 4 rulers, per load, so both arrays start 16-byte aligned.
inline int check_dec_pool(const int8_t* dec_q, const float* dec_scale) {
  if (!dec_q || !dec_scale) return host_fail(TTKV_E_INVALID, "null decoder pool");
  if ((uintptr_t)dec_q % 16 || (uintptr_t)dec_scale % 16)
    return host_fail(TTKV_E_INVALID, "dec_q and dec_scale must be 16-byte aligned");
  return TTKV_OK;
}

// Every workspace starts with a fixed region of arrival counters: zero before first use (a fresh
// zero-filled buffer), left zero by every call. It sits at the same offset with the same size
// whatever the call's shape, so one buffer can serve calls of any shape in turn: a call's data
// never lands where a later call expects zeroed counters. A launch uses at most kMaxCounters of
// them; larger batches run as several launches.
constexpr int64_t kCounterBytes = 65536;
constexpr int kMaxCounters = (int)(kCounterBytes / 4);

int64_t decode_workspace_bytes(const Geom& g, int G, int num_reqs, int max_seq_len,
                               int block_size);
int decode_paged(const Geom& g, int HQ, float scale, const void* q, int q_dtype,
                 int64_t q_row_stride, const uint8_t* page, int64_t n_slots, int64_t slot_stride,
                 int block_size, const int32_t* bt, int64_t bt_row_stride, int max_blocks,
                 const int32_t* seq_lens, const int32_t* qsl, int num_reqs, int max_seq_len,
                 const int32_t* dec_map, int64_t num_blocks, const int8_t* dec_q,
                 const float* dec_scale, int64_t n_dec_slots, const float* cs_cache,
                 int64_t max_pos, void* out, int out_dtype, int64_t out_row_stride, void* ws,
                 int64_t ws_bytes, int32_t* err, hipStream_t st);
// decode_paged with its split-K scratch in a file-scope device array (no workspace argument)
int decode_paged_noalloc(const Geom& g, int HQ, float scale, const void* q, int q_dtype,
                         int64_t q_row_stride, const uint8_t* page, int64_t n_slots,
                         int64_t slot_stride, int block_size, const int32_t* bt,
                         int64_t bt_row_stride, int max_blocks, const int32_t* seq_lens,
                         const int32_t* qsl, int num_reqs, int max_seq_len, const int32_t* dec_map,
                         int64_t num_blocks, const int8_t* dec_q, const float* dec_scale,
                         int64_t n_dec_slots, const float* cs_cache, int64_t max_pos, void* out,
                         int out_dtype, int64_t out_row_stride, int32_t* err, hipStream_t st);

}  // namespace ttkv

namespace ttkv {
int write_paged(const Geom& g, const void* key, int k_dtype, int64_t k_row_stride, const void* val,
                int v_dtype, int64_t v_row_stride, const int64_t* slot_mapping, int num_tokens,
                const int32_t* qsl, int num_reqs, const int32_t* bt, int64_t bt_row_stride,
                const int32_t* dec_map, int64_t num_blocks, const int8_t* dec_q,
                const float* dec_scale, const float* pinv_pool, int64_t n_dec_slots,
                int32_t* dec_used, const int8_t* cq_in, const float* cs_in, uint8_t* page,
                int64_t n_slots, int64_t slot_stride, float* c_out, float* r_out, void* ws,
                int64_t ws_bytes, int32_t* err, hipStream_t st);
int64_t write_workspace_bytes(const Geom& g, int num_tokens);
}  // namespace ttkv

namespace ttkv {
int64_t prefill_workspace_bytes(const Geom& g, int G, int num_reqs, int max_q_len,
                                int max_seq_len, int block_size);
// The two-launch continuation read (expand + attend) for chunks of two or more queries.
bool continuation_applies(const Geom& g, int G, int max_q_len);
int64_t continuation_workspace_bytes(const Geom& g, int G, int num_reqs, int max_q_len,
                                     int max_seq_len);
int64_t continuation_scores_workspace_bytes(const Geom& g, int G, int max_q_len,
                                            int max_seq_len);
int continuation_scores(const Geom& g, int HQ, float scale, const void* q, int q_dtype,
                        int64_t q_row_stride, const uint8_t* page, int64_t n_slots,
                        int64_t slot_stride, int block_size, const int32_t* bt,
                        int64_t bt_row_stride, const int32_t* seq_lens, const int32_t* qsl,
                        int max_q_len, int max_seq_len, const int32_t* dec_map, int64_t num_blocks,
                        const int8_t* dec_q, const float* dec_scale, int64_t n_dec_slots,
                        const float* cs_cache, float* s_out, int64_t s_head_stride,
                        int64_t s_q_stride, void* ws, int32_t* err, hipStream_t st);
int continuation_paged(const Geom& g, int HQ, float scale, const void* q, int q_dtype,
                       int64_t q_row_stride, const uint8_t* page, int64_t n_slots,
                       int64_t slot_stride, int block_size, const int32_t* bt,
                       int64_t bt_row_stride, const int32_t* seq_lens, const int32_t* qsl,
                       const int32_t* req_index, int num_reqs, int max_q_len, int max_seq_len,
                       const int32_t* dec_map, int64_t num_blocks, const int8_t* dec_q,
                       const float* dec_scale, int64_t n_dec_slots, const float* cs_cache,
                       void* out, int out_dtype, int64_t out_row_stride, void* ws, int32_t* err,
                       hipStream_t st);
int prefill_paged(const Geom& g, int HQ, float scale, const void* q, int q_dtype,
                  int64_t q_row_stride, const uint8_t* page, int64_t n_slots, int64_t slot_stride,
                  int block_size, const int32_t* bt, int64_t bt_row_stride, int max_blocks,
                  const int32_t* seq_lens, const int32_t* qsl, const int32_t* req_index,
                  int num_reqs, int max_q_len, int max_seq_len, const int32_t* dec_map,
                  int64_t num_blocks, const int8_t* dec_q, const float* dec_scale,
                  int64_t n_dec_slots, const float* cs_cache, int64_t max_pos, void* out,
                  int out_dtype, int64_t out_row_stride, float* s_out, int64_t s_head_stride,
                  int64_t s_q_stride, void* ws, int64_t ws_bytes, int32_t* err, hipStream_t st);
}  // namespace ttkv

namespace ttkv {
int64_t dense_workspace_bytes(int H, int G, int num_reqs, int max_seq_len, int block_size);
int dense_decode_paged(int H, int HQ, int d, float scale, const void* q, int64_t q_row_stride,
                       const void* k_cache, const void* v_cache, int dtype, int64_t n_slots,
                       int block_size, const int32_t* bt, int64_t bt_row_stride, int max_blocks,
                       const int32_t* seq_lens, const int32_t* qsl, int num_reqs, int max_seq_len,
                       void* out, int64_t out_row_stride, void* ws, int64_t ws_bytes,
                       hipStream_t st);
}  // namespace ttkv

namespace ttkv {
int container_krt(int H, int HQ, int d, int B, int n, int r1, const int8_t* cq, const float* cs,
                  const float* dec, int dec_per_seq, const uint8_t* bm, const uint8_t* pk,
                  const float* rs, int pb, int bits, const float* cosv, const float* sinv,
                  const float* q, float* s, hipStream_t st);
int container_v_out(int H, int HQ, int d, int B, int n, const float* p, int64_t p_head_stride,
                    int64_t p_batch_stride, const uint8_t* bm, const uint8_t* pk, const float* rs,
                    int pb, int bits, float* o, hipStream_t st);
}  // namespace ttkv
