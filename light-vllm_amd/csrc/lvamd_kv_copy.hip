// KV movement kernels for gfx950: slot-mapped append, tree-path compact and
// copy-on-write block copy.  All three are bit-exact byte copies, HBM-bound,
// and use the widest vector access the row alignment allows (16 B when the
// head row, strides and base addresses are 16-byte aligned).
//
// Behaviour follows light-vllm's PyTorch correctness path:
//   append  - PagedKVCache.write_prepared (src/light_vllm/runtime/execution/paged_cache.py:209-248)
//   compact - PagedKVCache.compact        (src/light_vllm/runtime/execution/paged_cache.py:257-326)
//   block copy has no reference counterpart (copy-on-write of a whole block).

#include <initializer_list>

#include "lvamd_common.h"

namespace lvamd {

// ---------------------------------------------------------------------------
// Append: one workgroup per packed token; its threads stride over
// (K|V, kv head, chunk).  A negative slot marks an inactive token.
// ---------------------------------------------------------------------------
struct AppendArgs {
  const char* key;
  const char* value;
  int64_t key_tok_bytes, key_head_bytes;
  int64_t value_tok_bytes, value_head_bytes;
  char* key_pool;
  char* value_pool;
  const int64_t* slots;
  int32_t num_kv_heads;
  int32_t head_bytes;  // head_size * element size
};

template <typename V>
__global__ __launch_bounds__(256) void kv_append_kernel(const AppendArgs a) {
  const int64_t t = blockIdx.x;
  const int64_t slot = a.slots[t];
  if (slot < 0) return;
  const int cpr = a.head_bytes / (int)sizeof(V);  // chunks per head row
  const int per_tensor = a.num_kv_heads * cpr;
  const int64_t row_bytes = (int64_t)a.num_kv_heads * a.head_bytes;
  for (int i = threadIdx.x; i < 2 * per_tensor; i += blockDim.x) {
    const bool is_v = i >= per_tensor;
    const int j = is_v ? i - per_tensor : i;
    const int h = j / cpr;
    const int c = j - h * cpr;
    const char* src = is_v ? a.value + t * a.value_tok_bytes + h * a.value_head_bytes
                           : a.key + t * a.key_tok_bytes + h * a.key_head_bytes;
    char* dst = (is_v ? a.value_pool : a.key_pool) + slot * row_bytes + (int64_t)h * a.head_bytes;
    reinterpret_cast<V*>(dst)[c] = reinterpret_cast<const V*>(src)[c];
  }
}

// Largest access width (16/8/4/2 bytes) dividing every address and stride.
static int common_vector_bytes(std::initializer_list<uint64_t> values) {
  uint64_t acc = 0;
  for (uint64_t v : values) acc |= v;
  if ((acc & 15u) == 0) return 16;
  if ((acc & 7u) == 0) return 8;
  if ((acc & 3u) == 0) return 4;
  if ((acc & 1u) == 0) return 2;
  return 1;
}

// ---------------------------------------------------------------------------
// Compact.  Inline path (num_pairs <= kCompactInline): one thread per
// (layer, K|V, 16-byte column chunk) holds the chunk of every source row in
// registers before it writes any destination, so every source is read before
// it can be overwritten.  Larger calls gather into a workspace first and
// scatter in a second, stream-ordered kernel.
// ---------------------------------------------------------------------------
constexpr int kCompactInline = 16;

struct CompactArgs {
  const uint64_t* kptrs;
  const uint64_t* vptrs;
  int32_t num_layers;
  int64_t row_bytes;
  const int64_t* src;
  const int64_t* dst;
  int64_t num_pairs;
  char* ws;
};

template <typename V>
__global__ __launch_bounds__(256) void kv_compact_inline_kernel(const CompactArgs a) {
  const int64_t cpr = a.row_bytes / (int64_t)sizeof(V);
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= (int64_t)a.num_layers * 2 * cpr) return;
  const int64_t c = item % cpr;
  const int64_t rest = item / cpr;
  const int is_v = (int)(rest & 1);
  const int layer = (int)(rest >> 1);
  char* base = reinterpret_cast<char*>(is_v ? a.vptrs[layer] : a.kptrs[layer]);
  const int n = (int)a.num_pairs;
  V tmp[kCompactInline];
#pragma unroll
  for (int i = 0; i < kCompactInline; ++i) {
    if (i < n) tmp[i] = reinterpret_cast<const V*>(base + a.src[i] * a.row_bytes)[c];
  }
  // Every gather has landed before the first scatter is issued.
  __threadfence_block();
#pragma unroll
  for (int i = 0; i < kCompactInline; ++i) {
    if (i < n) reinterpret_cast<V*>(base + a.dst[i] * a.row_bytes)[c] = tmp[i];
  }
}

// Workspace layout: [pair][layer][K|V][row_bytes].
template <typename V, bool kGather>
__global__ __launch_bounds__(256) void kv_compact_phase_kernel(const CompactArgs a) {
  const int64_t cpr = a.row_bytes / (int64_t)sizeof(V);
  const int64_t per_pair = (int64_t)a.num_layers * 2 * cpr;
  const int64_t total = a.num_pairs * per_pair;
  for (int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; item < total;
       item += (int64_t)gridDim.x * blockDim.x) {
    const int64_t pair = item / per_pair;
    const int64_t r = item - pair * per_pair;
    const int64_t c = r % cpr;
    const int64_t lk = r / cpr;  // layer * 2 + is_v
    const int is_v = (int)(lk & 1);
    const int layer = (int)(lk >> 1);
    char* base = reinterpret_cast<char*>(is_v ? a.vptrs[layer] : a.kptrs[layer]);
    V* wsrow = reinterpret_cast<V*>(a.ws + (pair * a.num_layers * 2 + lk) * a.row_bytes);
    if (kGather) {
      wsrow[c] = reinterpret_cast<const V*>(base + a.src[pair] * a.row_bytes)[c];
    } else {
      reinterpret_cast<V*>(base + a.dst[pair] * a.row_bytes)[c] = wsrow[c];
    }
  }
}

// ---------------------------------------------------------------------------
// Block copy: grid over (pair, layer, K|V); threads stride over the block.
// ---------------------------------------------------------------------------
struct BlockCopyArgs {
  const uint64_t* kptrs;
  const uint64_t* vptrs;
  int32_t num_layers;
  int64_t block_bytes;
  const int64_t* src;
  const int64_t* dst;
};

template <typename V>
__global__ __launch_bounds__(256) void kv_block_copy_kernel(const BlockCopyArgs a) {
  const int64_t idx = blockIdx.x;
  const int64_t pair = idx / (2 * a.num_layers);
  const int64_t lk = idx - pair * 2 * a.num_layers;
  const int is_v = (int)(lk & 1);
  const int layer = (int)(lk >> 1);
  char* base = reinterpret_cast<char*>(is_v ? a.vptrs[layer] : a.kptrs[layer]);
  const V* s = reinterpret_cast<const V*>(base + a.src[pair] * a.block_bytes);
  V* d = reinterpret_cast<V*>(base + a.dst[pair] * a.block_bytes);
  const int64_t n = a.block_bytes / (int64_t)sizeof(V);
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) d[i] = s[i];
}

// Launch KERNEL<V> with V the unsigned type of WIDTH bytes.
#define LVAMD_LAUNCH_BY_WIDTH(KERNEL, WIDTH, GRID, BLOCK, STREAM, ARGS)                  \
  do {                                                                                  \
    switch (WIDTH) {                                                                    \
      case 16: hipLaunchKernelGGL(KERNEL<uint4>, GRID, BLOCK, 0, STREAM, ARGS); break;    \
      case 8: hipLaunchKernelGGL(KERNEL<uint2>, GRID, BLOCK, 0, STREAM, ARGS); break;     \
      case 4: hipLaunchKernelGGL(KERNEL<uint32_t>, GRID, BLOCK, 0, STREAM, ARGS); break;  \
      case 2: hipLaunchKernelGGL(KERNEL<uint16_t>, GRID, BLOCK, 0, STREAM, ARGS); break;  \
      default: hipLaunchKernelGGL(KERNEL<uint8_t>, GRID, BLOCK, 0, STREAM, ARGS); break;  \
    }                                                                                   \
  } while (0)

}  // namespace lvamd

using namespace lvamd;

extern "C" {

const char* lvamd_status_string(int status) {
  switch (status) {
    case LVAMD_OK: return "ok";
    case LVAMD_ERR_INVALID_ARGUMENT: return "invalid argument";
    case LVAMD_ERR_UNSUPPORTED: return "unsupported dtype, head size or group size";
    case LVAMD_ERR_WORKSPACE: return "workspace missing or too small";
    case LVAMD_ERR_LAUNCH: return "kernel launch failed";
    default: return "unknown status";
  }
}

int lvamd_abi_version(void) { return 8; }

int lvamd_kv_append(const void* key, int64_t key_token_stride, int64_t key_head_stride,
                    const void* value, int64_t value_token_stride, int64_t value_head_stride,
                    void* key_pool, void* value_pool, const int64_t* slots, int64_t num_tokens,
                    int32_t num_kv_heads, int32_t head_size, int32_t dtype,
                    lvamd_stream_t stream) {
  const int es = dtype_size(dtype);
  if (es == 0) return LVAMD_ERR_UNSUPPORTED;
  if (num_tokens < 0 || num_kv_heads <= 0 || head_size <= 0) return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_tokens == 0) return LVAMD_OK;
  if (!key || !value || !key_pool || !value_pool || !slots) return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_tokens > 0x7fffffffLL) return LVAMD_ERR_INVALID_ARGUMENT;
  AppendArgs a;
  a.key = static_cast<const char*>(key);
  a.value = static_cast<const char*>(value);
  a.key_tok_bytes = key_token_stride * es;
  a.key_head_bytes = key_head_stride * es;
  a.value_tok_bytes = value_token_stride * es;
  a.value_head_bytes = value_head_stride * es;
  a.key_pool = static_cast<char*>(key_pool);
  a.value_pool = static_cast<char*>(value_pool);
  a.slots = slots;
  a.num_kv_heads = num_kv_heads;
  a.head_bytes = head_size * es;
  const int width = common_vector_bytes(
      {(uint64_t)(uintptr_t)key, (uint64_t)(uintptr_t)value, (uint64_t)(uintptr_t)key_pool,
       (uint64_t)(uintptr_t)value_pool, (uint64_t)a.key_tok_bytes, (uint64_t)a.key_head_bytes,
       (uint64_t)a.value_tok_bytes, (uint64_t)a.value_head_bytes, (uint64_t)a.head_bytes});
  const int chunks = 2 * num_kv_heads * (a.head_bytes / width);
  const int threads = chunks >= 256 ? 256 : ((chunks + 63) / 64) * 64;
  LVAMD_LAUNCH_BY_WIDTH(kv_append_kernel, width, dim3((unsigned)num_tokens), dim3(threads),
                        static_cast<hipStream_t>(stream), a);
  return launch_status();
}

int64_t lvamd_kv_compact_inline_pairs(void) { return kCompactInline; }

int64_t lvamd_kv_compact_workspace_size(int64_t num_pairs, int32_t num_layers, int64_t row_bytes) {
  if (num_pairs <= kCompactInline) return 0;
  return num_pairs * (int64_t)num_layers * 2 * row_bytes;
}

int lvamd_kv_compact(const uint64_t* layer_key_ptrs, const uint64_t* layer_value_ptrs,
                     int32_t num_layers, int64_t row_bytes,
                     const int64_t* src_slots, const int64_t* dst_slots, int64_t num_pairs,
                     void* workspace, int64_t workspace_bytes, lvamd_stream_t stream) {
  if (num_pairs < 0 || num_layers <= 0 || row_bytes <= 0) return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_pairs == 0) return LVAMD_OK;
  if (!layer_key_ptrs || !layer_value_ptrs || !src_slots || !dst_slots)
    return LVAMD_ERR_INVALID_ARGUMENT;
  CompactArgs a;
  a.kptrs = layer_key_ptrs;
  a.vptrs = layer_value_ptrs;
  a.num_layers = num_layers;
  a.row_bytes = row_bytes;
  a.src = src_slots;
  a.dst = dst_slots;
  a.num_pairs = num_pairs;
  a.ws = static_cast<char*>(workspace);
  // Pool bases come from torch allocations (>= 256-byte aligned); the row
  // size alone decides the access width.
  const int width = common_vector_bytes({(uint64_t)row_bytes});
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (num_pairs <= kCompactInline) {
    const int64_t items = (int64_t)num_layers * 2 * (row_bytes / width);
    const unsigned blocks = (unsigned)((items + 255) / 256);
    LVAMD_LAUNCH_BY_WIDTH(kv_compact_inline_kernel, width, dim3(blocks), dim3(256), s, a);
    return launch_status();
  }
  const int64_t need = lvamd_kv_compact_workspace_size(num_pairs, num_layers, row_bytes);
  if (!workspace || workspace_bytes < need) return LVAMD_ERR_WORKSPACE;
  const int64_t items = num_pairs * num_layers * 2 * (row_bytes / width);
  int64_t blocks = (items + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  switch (width) {
    case 16:
      hipLaunchKernelGGL((kv_compact_phase_kernel<uint4, true>), dim3((unsigned)blocks), dim3(256), 0, s, a);
      hipLaunchKernelGGL((kv_compact_phase_kernel<uint4, false>), dim3((unsigned)blocks), dim3(256), 0, s, a);
      break;
    case 8:
      hipLaunchKernelGGL((kv_compact_phase_kernel<uint2, true>), dim3((unsigned)blocks), dim3(256), 0, s, a);
      hipLaunchKernelGGL((kv_compact_phase_kernel<uint2, false>), dim3((unsigned)blocks), dim3(256), 0, s, a);
      break;
    case 4:
      hipLaunchKernelGGL((kv_compact_phase_kernel<uint32_t, true>), dim3((unsigned)blocks), dim3(256), 0, s, a);
      hipLaunchKernelGGL((kv_compact_phase_kernel<uint32_t, false>), dim3((unsigned)blocks), dim3(256), 0, s, a);
      break;
    case 2:
      hipLaunchKernelGGL((kv_compact_phase_kernel<uint16_t, true>), dim3((unsigned)blocks), dim3(256), 0, s, a);
      hipLaunchKernelGGL((kv_compact_phase_kernel<uint16_t, false>), dim3((unsigned)blocks), dim3(256), 0, s, a);
      break;
    default:
      hipLaunchKernelGGL((kv_compact_phase_kernel<uint8_t, true>), dim3((unsigned)blocks), dim3(256), 0, s, a);
      hipLaunchKernelGGL((kv_compact_phase_kernel<uint8_t, false>), dim3((unsigned)blocks), dim3(256), 0, s, a);
      break;
  }
  return launch_status();
}

int lvamd_kv_block_copy(const uint64_t* layer_key_ptrs, const uint64_t* layer_value_ptrs,
                        int32_t num_layers, int64_t block_bytes,
                        const int64_t* src_blocks, const int64_t* dst_blocks, int64_t num_pairs,
                        lvamd_stream_t stream) {
  if (num_pairs < 0 || num_layers <= 0 || block_bytes <= 0) return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_pairs == 0) return LVAMD_OK;
  if (!layer_key_ptrs || !layer_value_ptrs || !src_blocks || !dst_blocks)
    return LVAMD_ERR_INVALID_ARGUMENT;
  const int64_t grid = num_pairs * 2 * num_layers;
  if (grid > 0x7fffffffLL) return LVAMD_ERR_INVALID_ARGUMENT;
  BlockCopyArgs a;
  a.kptrs = layer_key_ptrs;
  a.vptrs = layer_value_ptrs;
  a.num_layers = num_layers;
  a.block_bytes = block_bytes;
  a.src = src_blocks;
  a.dst = dst_blocks;
  const int width = common_vector_bytes({(uint64_t)block_bytes});
  LVAMD_LAUNCH_BY_WIDTH(kv_block_copy_kernel, width, dim3((unsigned)grid), dim3(256),
                        static_cast<hipStream_t>(stream), a);
  return launch_status();
}

}  // extern "C"
