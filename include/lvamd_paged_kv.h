/*
 * lvamd_paged_kv.h — C ABI of the MI355X (gfx950) paged-KV attention backend.
 *
 * Every entry point takes raw device pointers, element strides and sizes,
 * enqueues its kernels on the given HIP stream, performs no host
 * synchronisation and no device allocation, and returns an lvamd_status
 * (0 = success, negative = error; lvamd_status_string names it).
 *
 * Physical KV layout (unchanged from light-vllm): per layer two tensors,
 * keys and values, each [num_blocks, block_size, num_kv_heads, head_size],
 * contiguous, of the cache dtype.  A physical "slot" is
 * block_id * block_size + offset, so slot s addresses the row
 * pool + s * num_kv_heads * head_size.
 *
 * Reference interfaces each entry point replaces are cited per function
 * (paths relative to the light-vllm source tree).
 */
#ifndef LVAMD_PAGED_KV_H
#define LVAMD_PAGED_KV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* lvamd_stream_t; /* a hipStream_t; NULL = the legacy default stream */

enum lvamd_status {
  LVAMD_OK = 0,
  LVAMD_ERR_INVALID_ARGUMENT = -1,  /* null pointer, negative size, misaligned row  */
  LVAMD_ERR_UNSUPPORTED = -2,       /* dtype / head_size / group size not built     */
  LVAMD_ERR_WORKSPACE = -3,         /* missing or undersized workspace              */
  LVAMD_ERR_LAUNCH = -4,            /* hipLaunchKernel / hipGetLastError failed     */
  LVAMD_ERR_SCRATCH_LIMIT = -5,     /* input needs more than the static scratch     */
  LVAMD_ERR_RUNTIME = -6            /* a HIP runtime call (copy, event) failed      */
};

enum lvamd_dtype { LVAMD_F32 = 0, LVAMD_F16 = 1, LVAMD_BF16 = 2 };

/* Number of int32 fields per request in the attention metadata
 * (table_off, num_table_blocks, computed, q_len, q_start, vis_off, vis_words, 0). */
#define LVAMD_REQ_FIELDS 8
/* Number of int32 fields per decode piece: (req, column_group, token_begin, token_end,
 * partial_slot, table_off, computed, q_len, q_start, vis_off, vis_words, b0, b1, b2, b3, b4).
 * column_group g covers column tiles [g * col_tiles, (g + 1) * col_tiles) of
 * the request.  A piece with partial_slot -1 covers its whole segment.
 * b0..b4 are the physical ids of the piece's first five logical blocks
 * (token_begin / block_size onwards; 0 past the request's table): the kernel
 * issues the piece's first tile from them when that tile spans at most five
 * blocks, without waiting for the block table. */
#define LVAMD_PIECE_FIELDS 16
/* Number of int32 fields per merge job:
 * (req, column_group, first_partial_slot, num_partials, q_start, q_len,
 *  span_slot, span_columns).
 * span_slot 0: no span.  Otherwise (prefill jobs of a request whose shared
 * prefix was attended by span units, below) span_slot - 1 is the span's first
 * partial slot and span_columns = the request's first column within the span
 * | pieces per span unit << 24: the job also combines, for its column c
 * (v = that offset + c), the partials of span unit v / unit columns at
 * column v % unit columns, slots span_slot - 1 + (v / unit columns) * pieces
 * + [0, pieces). */
#define LVAMD_MERGE_FIELDS 8
/* Number of int32 fields per prefill work unit:
 * (req, first column, columns, key_begin, key_end, partial_slot,
 *  table_off, q_start, computed, q_len, vis_off, vis_words, b0, b1, b2, b3).
 * key_begin and key_end are multiples of lvamd_paged_prefill_key_tokens();
 * key_end 0 means up to the unit's last visible key.  A unit with
 * partial_slot -1 covers all its keys and writes out; the others write
 * partials.  Fields 6-11 are the request's (as in its row of the
 * attention metadata), so the kernel reads nothing else per unit; b0..b3 are the physical ids of the logical
 * blocks key_begin / block_size onwards when the unit's first key tile spans
 * at most four blocks (0 past the table), else b0 = -1 (read from tables).
 * A span unit (req < 0): columns of the packed queries from token q_start on
 * (column c = token q_start + c / group, head c % group) of requests whose
 * tables all list the blocks at table_off over keys [0, key_end), each of
 * those keys below every such query's computed count; its fields read as a
 * linear request with computed = key_end and q_len 0, and it always writes
 * partials (key_end > 0). */
#define LVAMD_PREFILL_FIELDS 16

const char* lvamd_status_string(int status);

/* Library version, for the Python loader's compatibility check. */
int lvamd_abi_version(void);

/* XCDs (accelerator complex dies, each with its own L2) of the current
 * device, or LVAMD_ERR_RUNTIME.  The planner orders the prefill grid per XCD
 * (workgroup b runs on XCD b % count).  A device query with no counterpart in
 * the reference. */
int lvamd_xcd_count(void);

/*
 * Slot-mapped KV append:  key_pool[slots[t]] = key[t], value_pool[slots[t]] = value[t]
 * for every token t with slots[t] >= 0 (a negative slot marks an inactive token
 * and is skipped, as in the validated write path).  Slots must be unique and
 * < num_blocks * block_size (the caller proves this on the host, as
 * PagedAttentionMetadata.validate_block_tables does).  Bit-exact row copy.
 *
 * key/value: [num_tokens, num_kv_heads, head_size] with the given token and
 * head strides (elements); the head_size dimension must be contiguous.
 *
 * Replaces: PagedKVCache.write_prepared / write
 *   (src/light_vllm/runtime/execution/paged_cache.py:209-254) and the Triton
 *   _write_paged_kv_kernel (src/light_vllm/runtime/execution/triton_paged_attention.py:31-104).
 */
int lvamd_kv_append(const void* key, int64_t key_token_stride, int64_t key_head_stride,
                    const void* value, int64_t value_token_stride, int64_t value_head_stride,
                    void* key_pool, void* value_pool, const int64_t* slots, int64_t num_tokens,
                    int32_t num_kv_heads, int32_t head_size, int32_t dtype,
                    lvamd_stream_t stream);

/*
 * Rotary append: the RoPE half rotation fused with the KV append.  For every
 * packed token t (cosines / sines rows t, head_size wide, in the cache dtype):
 *   query_out[t, h] = rotate(query[t, h])         for h < num_query_heads
 *   key_pool[slots[t], h] = rotate(key[t, h])     for h < num_kv_heads
 *   value_pool[slots[t], h] = value[t, h]         (bit-exact copy)
 * with rotate(x)[d] = x[d]*cos[d] + r[d]*sin[d], r = (-x[D/2:], x[:D/2]),
 * rounded as the PyTorch path rounds it: each product to the dtype, then the
 * sum (fp32 add) to the dtype.  Negative slots skip the pool writes.
 * query_out may alias query (each thread reads a chunk pair before writing
 * it).  One launch replaces the model's rotary kernel and the append.
 *
 * Replaces: apply_rotary (src/light_vllm/modeling/models/_qwen2_kernels.py:205-245,
 *   called at src/light_vllm/modeling/models/qwen2.py:411) followed by
 *   PagedKVCache.write_prepared (src/light_vllm/runtime/execution/paged_cache.py:209-248).
 */
int lvamd_kv_append_rotary(const void* query, int64_t query_token_stride, int64_t query_head_stride,
                           void* query_out, int64_t query_out_token_stride, int64_t query_out_head_stride,
                           const void* key, int64_t key_token_stride, int64_t key_head_stride,
                           const void* value, int64_t value_token_stride, int64_t value_head_stride,
                           const void* cosines, int64_t cosines_token_stride,
                           const void* sines, int64_t sines_token_stride,
                           void* key_pool, void* value_pool, const int64_t* slots, int64_t num_tokens,
                           int32_t num_query_heads, int32_t num_kv_heads, int32_t head_size, int32_t dtype,
                           lvamd_stream_t stream);

/*
 * Split-K paged attention for short query runs (decode, speculative tree
 * verification), stream-K scheduled, with this step's KV append fused in.
 *
 * Work: one wave computes col_tiles (1 or 4) column tiles of 16 MFMA columns
 * each.  The decode rows' (request, column group) segments are laid end to
 * end in tile-sized units (lvamd_paged_decode_tile_tokens) and cut into
 * waves_per_head contiguous shares; wave w of kv head h (workgroup
 * h * waves_per_head + w, one wave64 each) processes pieces
 * [wave_first[w], wave_first[w + 1]) (LVAMD_PIECE_FIELDS int32 each).  A
 * piece with partial_slot -1 covers its whole segment and writes out; the
 * others write partials for lvamd_paged_attention_merge: each column's
 * output row normalised by its own softmax sum, in the pool's element type,
 * to part_acc [slots][num_kv_heads][16 * col_tiles][head_size], and its fp32
 * (max, sum) to part_ml [slots][num_kv_heads][16 * col_tiles][2].
 *
 * Workgroup split: with group_waves W = lvamd_paged_decode_split_waves(...)
 * (col_tiles 1) the waves run in workgroups of W, waves W*b .. W*b + W - 1 of
 * a kv head in workgroup b, each workgroup holds one segment, and pieces
 * holds exactly one record per wave (wave w's at index w; wave_first is not
 * read): a piece of the segment, or an idle record with req -1 (idle waves
 * follow the active ones).  A segment left whole in its workgroup's first
 * wave (partial_slot -1) is written by that wave; the pieces of a split one
 * (partial_slot >= 0) are combined in the workgroup's LDS and written by the
 * workgroup: no partials, no merge launch.  waves_per_head must then be a
 * multiple of W.  group_waves 1 is the stream-K layout above.
 *
 * Append: when new_key / new_value are given ([tokens][num_kv_heads][D] with
 * the given strides), keys and values at positions >= computed are read from
 * them, and each such token's row is written to its pool slot (bit-exact copy;
 * the slot comes from the block table, exactly PagedAttentionMetadata.slot_mapping).
 * When they are NULL the pool must already hold this step's K/V.
 *
 * MFMA columns are (query, head-in-group) pairs of one kv head, 16 per column
 * tile.  bf16/fp16 QK^T and PV on MFMA (fp32 on 16x16x4), fp32 online softmax;
 * K/V gathered through the block table (tables: flat int32 block ids); vis
 * holds uint32 ancestor bit rows for requests with vis_off >= 0.  scale is the
 * caller's softmax scale.  head_size: a multiple of 16 from 32 to 256 (the
 * merge and prefill entry points take the same set); any other returns
 * LVAMD_ERR_UNSUPPORTED.
 *
 * Together with lvamd_paged_attention_merge and lvamd_paged_prefill this
 * replaces TorchPagedAttention.forward / _attend_query_token
 * (src/light_vllm/runtime/execution/paged_attention.py:268-380), the
 * write-before-attend of PagedKVCache.write_prepared (paged_cache.py:209-254,
 * called at paged_attention.py:294-301) and the Triton _write_paged_kv_kernel /
 * _grouped_paged_attention_kernel / _paged_attention_kernel
 *   (src/light_vllm/runtime/execution/triton_paged_attention.py:31-104, 107-391,
 *   launch :498-559).
 */
int lvamd_paged_decode(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                       const void* new_key, int64_t new_key_token_stride, int64_t new_key_head_stride,
                       const void* new_value, int64_t new_value_token_stride, int64_t new_value_head_stride,
                       void* key_pool, void* value_pool,
                       void* out, int64_t out_token_stride, int64_t out_head_stride,
                       const int32_t* pieces, const int32_t* wave_first, int32_t waves_per_head,
                       const int32_t* tables, const uint32_t* vis,
                       void* part_acc, float* part_ml, int64_t num_partial_slots,
                       int32_t num_kv_heads, int32_t group, int32_t head_size, int32_t col_tiles,
                       int32_t group_waves, int32_t block_size, float scale, int32_t dtype, lvamd_stream_t stream);

/* Workgroups of the workgroup-split decode kernel (one column tile) the
 * current device holds at once for this dtype and head size: the planner uses
 * the split only when a step's segments fit them.  Needs a GPU. */
int lvamd_paged_decode_split_groups(int32_t dtype, int32_t head_size);

/* Waves per workgroup of the workgroup-split decode kernel for this dtype and
 * head size (the group_waves it takes): 8, or 4 where eight would spill or
 * exceed the LDS. */
int lvamd_paged_decode_split_waves(int32_t dtype, int32_t head_size);

/* How many decode waves (workgroups) the current device holds at once for this
 * dtype, head size and col_tiles: the planner's stream-K width.  Needs a GPU. */
int lvamd_paged_decode_resident_waves(int32_t dtype, int32_t head_size, int32_t col_tiles);

/* Tokens per decode-kernel tile for this dtype, head size and col_tiles (32
 * for one column tile, 16 for four; 16 for rows above 256 bytes): the planner
 * cuts pieces on multiples of it.  A piece may start anywhere; tile-aligned
 * pieces avoid partial tiles. */
int lvamd_paged_decode_tile_tokens(int32_t dtype, int32_t head_size, int32_t col_tiles);

/*
 * Log-sum-exp merge of split-K partials into out, one wave per (job, kv head,
 * column), four columns per workgroup, over the first max_columns (1 to
 * 16 * col_tiles) columns of each job (the most any job has; the host knows
 * it); jobs [num_jobs][LVAMD_MERGE_FIELDS]; col_tiles (1 to 16) is
 * the number of 16-column tiles per partial slot the partials were written
 * with (the decode kernel's col_tiles, or prefill unit columns / 16).
 * Partial i of a column weighs sum_i * 2^(max_i - max) (max, sum in the
 * log2 domain); part_acc holds rows of dtype.  Same reference functions as lvamd_paged_decode:
 * the reference has no split-K, and this is the cross-partition half of that
 * computation.
 */
int lvamd_paged_attention_merge(const void* part_acc, const float* part_ml,
                                void* out, int64_t out_token_stride, int64_t out_head_stride,
                                const int32_t* jobs, int32_t num_jobs,
                                int32_t num_kv_heads, int32_t group, int32_t head_size, int32_t col_tiles,
                                int32_t max_columns, int32_t dtype, lvamd_stream_t stream);

/*
 * Chunked-prefill paged attention for query runs of more than one column
 * tile (prompt chunks, tree verification; bf16 / fp16, head sizes that are
 * multiples of 16 from 32 to 256): one workgroup per (unit, kv head); a unit
 * (units [num_units][LVAMD_PREFILL_FIELDS]) is a run of MFMA columns of one
 * request over a key range, a column being a (query, head-in-group) pair,
 * column c = query (c / group), head (c % group).  K/V tiles (64 tokens up to
 * head size 128, else 32) are copied through the block table straight into
 * LDS (direct loads, double-buffered) and shared by the workgroup's waves; QK^T and PV on MFMA 16x16x32, fp32 online
 * softmax.  waves (4 or 8) picks the workgroup shape for the same unit: four
 * waves of two 16-column tiles or eight waves of one (8 only where
 * lvamd_paged_prefill_waves_built says so).  Units with a partial slot write partials in the
 * decode kernel's format (normalised rows of the pool's type to part_acc
 * [slots][num_kv_heads][unit columns][head_size], fp32 (max, sum) to part_ml
 * [slots][num_kv_heads][unit columns][2]); lvamd_paged_attention_merge with
 * col_tiles = unit columns / 16 combines them.
 * A record with zero columns (field 2) is padding and does nothing (the
 * planner orders units per XCD).
 * Append: when new_key / new_value are given
 * ([tokens][num_kv_heads][D] with the given strides), keys at positions >=
 * computed are read from them, and each such token's row is written to its
 * pool slot by the unit that holds the token's own query (bit-exact copy).
 * When they are NULL the pool must already hold this step's K/V
 * (lvamd_kv_append).  Each unit record carries its request's fields
 * (LVAMD_PREFILL_FIELDS), so no per-request table is passed.  Replaces the
 * prefill half of the same reference functions as lvamd_paged_decode.
 */
int lvamd_paged_prefill(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                        const void* new_key, int64_t new_key_token_stride, int64_t new_key_head_stride,
                        const void* new_value, int64_t new_value_token_stride, int64_t new_value_head_stride,
                        void* key_pool, void* value_pool,
                        void* out, int64_t out_token_stride, int64_t out_head_stride,
                        const int32_t* tables, const uint32_t* vis,
                        const int32_t* units, int32_t num_units,
                        void* part_acc, float* part_ml, int64_t num_partial_slots,
                        int32_t num_kv_heads, int32_t group, int32_t head_size, int32_t waves,
                        int32_t block_size, float scale, int32_t dtype, lvamd_stream_t stream);

/*
 * One layer's attention in one call: the launch facts of a layer shape in one
 * step plan, bound once per step (every layer of that shape shares them), so
 * that a layer only adds its tensors.  Fields mirror the arguments of
 * lvamd_paged_decode, lvamd_paged_attention_merge and lvamd_paged_prefill.
 */
typedef struct lvamd_attention_plan {
  /* Decode rows (waves_per_head 0: none). */
  const int32_t* pieces;
  const int32_t* wave_first;
  int32_t waves_per_head;
  int32_t col_tiles;
  void* part_acc;
  float* part_ml;
  int64_t num_partial_slots;
  const int32_t* jobs;
  int32_t num_jobs;
  int32_t merge_columns;
  int32_t group_waves; /* 1: stream-K; lvamd_paged_decode_split_waves: workgroup split */
  /* Prefill rows (num_units 0: none). */
  const int32_t* units;
  int32_t num_units;
  int32_t prefill_waves;
  void* prefill_part_acc;
  float* prefill_part_ml;
  int64_t num_prefill_partial_slots;
  const int32_t* prefill_jobs;
  int32_t num_prefill_jobs;
  int32_t prefill_merge_columns;
  int32_t prefill_col_tiles; /* prefill unit columns / 16 */
  /* Step facts and layer shape. */
  int32_t num_kv_heads;
  const int32_t* tables;
  const uint32_t* vis;
  int32_t group;
  int32_t head_size;
  int32_t block_size;
  int32_t dtype;
} lvamd_attention_plan;

/*
 * A layer's whole attention step: the decode launch and its merge launch,
 * then the prefill launch and its merge launch, on one stream, with this
 * step's K/V appended by the kernels (or new_key / new_value NULL when the
 * pool already holds them).  Returns the first failing launch's status.
 *
 * Replaces: TorchPagedAttention.forward's write-then-attend for one layer
 *   (src/light_vllm/runtime/execution/paged_attention.py:268-380) and the
 *   Triton backend's per-layer launches (triton_paged_attention.py:454-560),
 *   called from Qwen2Attention.forward (src/light_vllm/modeling/models/qwen2.py:417-423).
 */
int lvamd_paged_attention(const lvamd_attention_plan* plan,
                          const void* q, int64_t q_token_stride, int64_t q_head_stride,
                          const void* new_key, int64_t new_key_token_stride, int64_t new_key_head_stride,
                          const void* new_value, int64_t new_value_token_stride, int64_t new_value_head_stride,
                          void* key_pool, void* value_pool,
                          void* out, int64_t out_token_stride, int64_t out_head_stride,
                          float scale, lvamd_stream_t stream);

/* Columns per prefill unit for this dtype and head size (the planner's unit
 * width), or 0 when the prefill kernel does not support them. */
int lvamd_paged_prefill_unit_columns(int32_t dtype, int32_t head_size);

/* Keys per prefill tile (unit key ranges start on multiples of it). */
int lvamd_paged_prefill_key_tokens(int32_t dtype, int32_t head_size);

/* Prefill workgroups of the given shape (waves 4 or 8) the current device
 * holds at once for this dtype and head size: the planner splits units' key
 * ranges to fill them.  Needs a GPU. */
int lvamd_paged_prefill_resident_units(int32_t dtype, int32_t head_size, int32_t waves);

/* 1 when the prefill kernel is built with that many waves per workgroup for
 * this dtype and head size (4 always; 8 up to head size 128), else 0. */
int lvamd_paged_prefill_waves_built(int32_t dtype, int32_t head_size, int32_t waves);

/*
 * Tree-KV compact across all layers: for every layer l and pair i,
 * row dst_slots[i] of keys[l] and values[l] receives the bytes row
 * src_slots[i] held before the call (every source is read before any
 * destination is written, so overlapping paths are safe).  Pairs with
 * src == dst may be passed or omitted.  Destinations must be unique.
 * layer_key_ptrs / layer_value_ptrs: device arrays of num_layers pool base
 * addresses (uint64).  row_bytes = num_kv_heads * head_size * element size,
 * equal for all layers of one call.  When num_pairs exceeds
 * lvamd_kv_compact_inline_pairs(), workspace must hold
 * lvamd_kv_compact_workspace_size(...) bytes; otherwise it may be NULL.
 *
 * Replaces: PagedKVCache.compact's gather / clone / scatter loop
 *   (src/light_vllm/runtime/execution/paged_cache.py:315-326); host-side
 *   validation and the moved-token count stay in Python (:269-314, :326).
 */
int lvamd_kv_compact(const uint64_t* layer_key_ptrs, const uint64_t* layer_value_ptrs,
                     int32_t num_layers, int64_t row_bytes,
                     const int64_t* src_slots, const int64_t* dst_slots, int64_t num_pairs,
                     void* workspace, int64_t workspace_bytes, lvamd_stream_t stream);
int64_t lvamd_kv_compact_inline_pairs(void);

/*
 * lvamd_kv_compact in one HBM pass, in place, for pair lists whose order makes
 * that safe (no workspace): the pairs come in num_groups groups, group g being
 * pairs [group_starts[g], group_starts[g + 1]) (device int64 array).  The
 * caller guarantees that (1) no pair's destination is the source of a later
 * pair of its group, and (2) no destination of one group is a source or
 * destination of another; destinations are unique.  Rows are then moved in
 * order, so row dst_slots[i] receives what row src_slots[i] held before the
 * call, as with lvamd_kv_compact.  A step's compacts qualify with one group
 * per request whenever each request's retained indices are strictly
 * increasing (speculative decoding's accepted root-to-leaf paths).
 *
 * Replaces: the gather / clone / scatter of PagedKVCache.compact
 *   (src/light_vllm/runtime/execution/paged_cache.py:315-326), which moves
 *   each row once per layer, for calls above lvamd_kv_compact_inline_pairs().
 */
int lvamd_kv_compact_ordered(const uint64_t* layer_key_ptrs, const uint64_t* layer_value_ptrs,
                             int32_t num_layers, int64_t row_bytes,
                             const int64_t* src_slots, const int64_t* dst_slots, const int64_t* group_starts,
                             int64_t num_groups, lvamd_stream_t stream);

/*
 * lvamd_kv_compact for at most lvamd_kv_compact_inline_pairs() pairs given
 * in HOST memory: the pairs travel in the kernel's arguments (one launch, no
 * device index buffer, no upload).  Same rules and result as
 * lvamd_kv_compact; more pairs return LVAMD_ERR_INVALID_ARGUMENT.
 *
 * Replaces: the same reference loop as lvamd_kv_compact
 *   (src/light_vllm/runtime/execution/paged_cache.py:315-326), for the
 *   per-step compacts of speculative decoding (a few accepted tokens).
 */
int lvamd_kv_compact_small(const uint64_t* layer_key_ptrs, const uint64_t* layer_value_ptrs,
                           int32_t num_layers, int64_t row_bytes,
                           const int64_t* src_slots, const int64_t* dst_slots, int64_t num_pairs,
                           lvamd_stream_t stream);

/*
 * Allocation-free variant of lvamd_kv_compact: the same kernels and result,
 * but calls with more than lvamd_kv_compact_inline_pairs() pairs stage their
 * rows in a device array the library holds (LVAMD_COMPACT_STATIC_SCRATCH_BYTES
 * per GPU, for the life of the process) instead of a caller workspace, so the
 * call itself allocates nothing (no hipMalloc, no library allocation).
 * Returns LVAMD_ERR_SCRATCH_LIMIT, without launching, when
 * num_pairs * num_layers * 2 * row_bytes exceeds that size.  Every call on
 * one GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams, other threads) race and must be serialised by the caller.
 *
 * No counterpart in the reference.  It is for callers that cannot allocate:
 * code under HIP graph capture, tight serving loops, and harnesses that
 * forbid hipMalloc.
 */
#define LVAMD_COMPACT_STATIC_SCRATCH_BYTES (16LL << 20)
int lvamd_kv_compact_static(const uint64_t* layer_key_ptrs, const uint64_t* layer_value_ptrs,
                            int32_t num_layers, int64_t row_bytes,
                            const int64_t* src_slots, const int64_t* dst_slots, int64_t num_pairs,
                            lvamd_stream_t stream);
int64_t lvamd_kv_compact_workspace_size(int64_t num_pairs, int32_t num_layers, int64_t row_bytes);

/*
 * Copy-on-write block copy across all layers: block dst_blocks[i] of keys[l]
 * and values[l] becomes a byte copy of block src_blocks[i].  Sources and
 * destinations must be disjoint sets and destinations unique (checked by the
 * Python caller).  block_bytes = block_size * row_bytes.
 *
 * No reference counterpart: light-vllm's prefix cache shares only complete
 * read-only pages (src/light_vllm/runtime/kv_cache.py:661-723).  This is the
 * primitive a partial-page prefix share needs.
 */
int lvamd_kv_block_copy(const uint64_t* layer_key_ptrs, const uint64_t* layer_value_ptrs,
                        int32_t num_layers, int64_t block_bytes,
                        const int64_t* src_blocks, const int64_t* dst_blocks, int64_t num_pairs,
                        lvamd_stream_t stream);

/*
 * lvamd_kv_block_copy for at most lvamd_kv_block_copy_small_pairs() pairs
 * given in HOST memory: the pairs travel in the kernel's arguments (no device
 * index buffer, no upload).  Same rules and result as lvamd_kv_block_copy;
 * more pairs return LVAMD_ERR_INVALID_ARGUMENT.  No reference counterpart
 * (as lvamd_kv_block_copy): a step's copy-on-write of a few partial pages.
 */
int lvamd_kv_block_copy_small(const uint64_t* layer_key_ptrs, const uint64_t* layer_value_ptrs,
                              int32_t num_layers, int64_t block_bytes,
                              const int64_t* src_blocks, const int64_t* dst_blocks, int64_t num_pairs,
                              lvamd_stream_t stream);
int64_t lvamd_kv_block_copy_small_pairs(void);

/*
 * The per-step upload of a staged plan: copies bytes from pinned host memory
 * to device memory on stream (asynchronous), then records event (a
 * hipEvent_t; NULL for none) on stream, so the caller can tell when the
 * pinned buffer may be refilled.  Replaces the pinned-buffer copy of
 * light-vllm's CudaStaging (src/light_vllm/runtime/execution/cuda_staging.py:27-49)
 * plus its event, in one call.  LVAMD_ERR_RUNTIME if either HIP call fails.
 */
int lvamd_stage_upload(void* device_dst, const void* pinned_src, int64_t bytes, void* event,
                       lvamd_stream_t stream);

/*
 * Measurement only: streams bytes (a multiple of 16) of buf from HBM with
 * workgroups x 64 lanes, 16-byte loads, and writes the XOR of every lane's
 * words to sink[workgroups * 64] (so the XOR of sink equals the XOR of buf).
 * bench.py times it to report the practical HBM read ceiling beside the
 * decode kernel's bandwidth.  No counterpart in the reference.
 */
int lvamd_hbm_read_probe(const void* buf, int64_t bytes, uint32_t* sink, int32_t workgroups,
                         lvamd_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* LVAMD_PAGED_KV_H */
