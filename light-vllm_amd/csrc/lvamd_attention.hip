// One layer's attention step through one C entry point: the decode launch and
// its merge, then the prefill launch and its merge, from the launch facts the
// host bound once per step and layer shape (lvamd_attention_plan).

#include "lvamd_common.h"

extern "C" int lvamd_paged_attention(const lvamd_attention_plan* plan,
                                     const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                     const void* new_key, int64_t new_key_token_stride,
                                     int64_t new_key_head_stride, const void* new_value,
                                     int64_t new_value_token_stride, int64_t new_value_head_stride,
                                     void* key_pool, void* value_pool,
                                     void* out, int64_t out_token_stride, int64_t out_head_stride,
                                     float scale, lvamd_stream_t stream) {
  if (!plan) return LVAMD_ERR_INVALID_ARGUMENT;
  const lvamd_attention_plan& p = *plan;
  int status = LVAMD_OK;
  if (p.waves_per_head > 0) {
    status = lvamd_paged_decode(q, q_token_stride, q_head_stride, new_key, new_key_token_stride,
                                new_key_head_stride, new_value, new_value_token_stride, new_value_head_stride,
                                key_pool, value_pool, out, out_token_stride, out_head_stride, p.pieces,
                                p.wave_first, p.waves_per_head, p.tables, p.vis, p.part_acc, p.part_ml,
                                p.num_partial_slots, p.num_kv_heads, p.group, p.head_size,
                                p.col_tiles, p.group_waves, p.block_size, scale, p.dtype, stream);
    if (status != LVAMD_OK) return status;
    if (p.num_jobs > 0) {
      status = lvamd_paged_attention_merge(p.part_acc, p.part_ml, out, out_token_stride, out_head_stride, p.jobs,
                                           p.num_jobs, p.num_kv_heads, p.group, p.head_size, p.col_tiles,
                                           p.merge_columns, p.dtype, stream);
      if (status != LVAMD_OK) return status;
    }
  }
  if (p.num_units > 0) {
    status = lvamd_paged_prefill(q, q_token_stride, q_head_stride, new_key, new_key_token_stride,
                                 new_key_head_stride, new_value, new_value_token_stride, new_value_head_stride,
                                 key_pool, value_pool, out, out_token_stride, out_head_stride, p.tables, p.vis,
                                 p.units, p.num_units, p.prefill_part_acc, p.prefill_part_ml,
                                 p.num_prefill_partial_slots, p.num_kv_heads, p.group, p.head_size, p.prefill_waves,
                                 p.block_size, scale, p.dtype, stream);
    if (status != LVAMD_OK) return status;
    if (p.num_prefill_jobs > 0) {
      status = lvamd_paged_attention_merge(p.prefill_part_acc, p.prefill_part_ml, out, out_token_stride,
                                           out_head_stride, p.prefill_jobs, p.num_prefill_jobs, p.num_kv_heads,
                                           p.group, p.head_size, p.prefill_col_tiles, p.prefill_merge_columns,
                                           p.dtype, stream);
    }
  }
  return status;
}

static_assert(sizeof(lvamd_attention_plan) == 168, "the Python binding (native.AttentionPlan) assumes this layout");
