// Chunked-prefill paged attention (MFMA) — entry point.
#include "lvamd_common.h"

extern "C" int lvamd_paged_prefill(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                   const void* key_pool, const void* value_pool,
                                   void* out, int64_t out_token_stride, int64_t out_head_stride,
                                   const int32_t* req_meta, const int32_t* tables, const uint32_t* vis,
                                   const int32_t* units, int32_t num_units,
                                   int32_t num_kv_heads, int32_t group, int32_t head_size,
                                   int32_t block_size, float scale, int32_t dtype, lvamd_stream_t stream) {
  (void)q; (void)q_token_stride; (void)q_head_stride; (void)key_pool; (void)value_pool; (void)out;
  (void)out_token_stride; (void)out_head_stride; (void)req_meta; (void)tables; (void)vis; (void)units;
  (void)num_kv_heads; (void)group; (void)head_size; (void)block_size; (void)scale; (void)dtype; (void)stream;
  return num_units == 0 ? LVAMD_OK : LVAMD_ERR_UNSUPPORTED;
}
