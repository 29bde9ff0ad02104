// KV movement kernels for gfx950: slot-mapped append, tree-path compact and
// copy-on-write block copy.  All three are bit-exact byte copies, HBM-bound,
// and use the widest vector access the row alignment allows (16 B when the
// head row, strides and base addresses are 16-byte aligned).
//
// Behaviour follows light-vllm's PyTorch correctness path:
//   append  - PagedKVCache.write_prepared (src/light_vllm/runtime/execution/paged_cache.py:209-248)
//   compact - PagedKVCache.compact        (src/light_vllm/runtime/execution/paged_cache.py:257-326)
//   block copy has no reference counterpart (copy-on-write of a whole block).

#include <atomic>
#include <initializer_list>
#include <mutex>
#include <type_traits>

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

// ---------------------------------------------------------------------------
// Rotary append: one workgroup per packed token.  The token's query heads and
// key heads get the half rotation of light-vllm's apply_rotary
//   out[d]     = x[d] * cos[d]     + (-x[d + D/2]) * sin[d]       (d < D/2)
//   out[d+D/2] = x[d+D/2] * cos[d+D/2] + x[d] * sin[d+D/2]
// with the rounding of its PyTorch path (_qwen2_kernels.py:214-224): each
// product is rounded to the tensor dtype, then their sum is (an fp32 add,
// rounded to the dtype).  Rotated queries go to query_out; rotated keys and
// the values are written to their pool slots (negative slot: no pool write).
// A thread takes one chunk pair (d, d + D/2) of one head, or one value chunk.
// ---------------------------------------------------------------------------
struct RotaryArgs {
  const char* q;
  char* q_out;
  const char* key;
  const char* value;
  const char* cosines;
  const char* sines;
  int64_t q_tok_bytes, q_head_bytes, qo_tok_bytes, qo_head_bytes;
  int64_t key_tok_bytes, key_head_bytes, value_tok_bytes, value_head_bytes;
  int64_t cos_tok_bytes, sin_tok_bytes;
  char* key_pool;
  char* value_pool;
  const int64_t* slots;
  int32_t num_q_heads, num_kv_heads;
  int32_t head_bytes;
};

template <int VB> struct RawChunk;
template <> struct RawChunk<16> { using type = uint4; };
template <> struct RawChunk<8> { using type = uint2; };
template <> struct RawChunk<4> { using type = uint32_t; };
template <> struct RawChunk<2> { using type = uint16_t; };

// One product of the rotation, rounded as the PyTorch expression rounds it.
// The rounded product passes through an empty asm statement: the device
// code generator fuses a multiply feeding an add into an FMA whatever the
// contraction flags say (also the mixed-precision fma_mix / packed forms it
// builds from a 16-bit product extended into an fp32 add), which would skip
// the product's rounding.  The asm makes the product an opaque register.
template <typename T>
__device__ __forceinline__ float rope_product(float x, float y) {
  float p;
  if constexpr (std::is_same_v<T, float>) {
    p = x * y;
  } else {
    p = to_f32(from_f32<T>(x * y));  // exact in fp32, then rounded to T
  }
  __asm__("" : "+v"(p));
  return p;
}

template <typename T, int VB>
__device__ __forceinline__ void rotate_pair(const char* src, char* dst_lo, char* dst_hi, int64_t half_bytes,
                                            const char* cs, const char* sn) {
  using R = typename RawChunk<VB>::type;
  constexpr int W = VB / (int)sizeof(T);
  const R xl = *reinterpret_cast<const R*>(src);
  const R xh = *reinterpret_cast<const R*>(src + half_bytes);
  const R cl = *reinterpret_cast<const R*>(cs);
  const R ch = *reinterpret_cast<const R*>(cs + half_bytes);
  const R sl = *reinterpret_cast<const R*>(sn);
  const R sh = *reinterpret_cast<const R*>(sn + half_bytes);
  T x0[W], x1[W], c0[W], c1[W], s0[W], s1[W], o0[W], o1[W];
  __builtin_memcpy(x0, &xl, VB);
  __builtin_memcpy(x1, &xh, VB);
  __builtin_memcpy(c0, &cl, VB);
  __builtin_memcpy(c1, &ch, VB);
  __builtin_memcpy(s0, &sl, VB);
  __builtin_memcpy(s1, &sh, VB);
#pragma unroll
  for (int e = 0; e < W; ++e) {
    const float lo = to_f32(x0[e]), hi = to_f32(x1[e]);
    // x + round(-h*s) is x - round(h*s) exactly (rounding is sign-symmetric).
    o0[e] = from_f32<T>(rope_product<T>(lo, to_f32(c0[e])) - rope_product<T>(hi, to_f32(s0[e])));
    o1[e] = from_f32<T>(rope_product<T>(hi, to_f32(c1[e])) + rope_product<T>(lo, to_f32(s1[e])));
  }
  R rl, rh;
  __builtin_memcpy(&rl, o0, VB);
  __builtin_memcpy(&rh, o1, VB);
  *reinterpret_cast<R*>(dst_lo) = rl;
  *reinterpret_cast<R*>(dst_hi) = rh;
}

template <typename T, int VB>
__global__ __launch_bounds__(256) void kv_append_rotary_kernel(const RotaryArgs a) {
  const int64_t t = blockIdx.x;
  const int64_t slot = a.slots[t];
  const int half_bytes = a.head_bytes / 2;
  const int pairs = half_bytes / VB;  // chunk pairs per head row
  const int vchunks = a.head_bytes / VB;
  const int q_items = a.num_q_heads * pairs;
  const int k_items = a.num_kv_heads * pairs;
  const int items = q_items + (slot >= 0 ? k_items + a.num_kv_heads * vchunks : 0);
  const int64_t row_bytes = (int64_t)a.num_kv_heads * a.head_bytes;
  const char* cs = a.cosines + t * a.cos_tok_bytes;
  const char* sn = a.sines + t * a.sin_tok_bytes;
  for (int i = threadIdx.x; i < items; i += blockDim.x) {
    if (i < q_items) {
      const int h = i / pairs;
      const int off = (i - h * pairs) * VB;
      const char* src = a.q + t * a.q_tok_bytes + h * a.q_head_bytes + off;
      char* dst = a.q_out + t * a.qo_tok_bytes + h * a.qo_head_bytes + off;
      rotate_pair<T, VB>(src, dst, dst + half_bytes, half_bytes, cs + off, sn + off);
    } else if (i < q_items + k_items) {
      const int j = i - q_items;
      const int h = j / pairs;
      const int off = (j - h * pairs) * VB;
      const char* src = a.key + t * a.key_tok_bytes + h * a.key_head_bytes + off;
      char* dst = a.key_pool + slot * row_bytes + (int64_t)h * a.head_bytes + off;
      rotate_pair<T, VB>(src, dst, dst + half_bytes, half_bytes, cs + off, sn + off);
    } else {
      const int j = i - q_items - k_items;
      const int h = j / vchunks;
      const int off = (j - h * vchunks) * VB;
      using R = typename RawChunk<VB>::type;
      *reinterpret_cast<R*>(a.value_pool + slot * row_bytes + (int64_t)h * a.head_bytes + off) =
          *reinterpret_cast<const R*>(a.value + t * a.value_tok_bytes + h * a.value_head_bytes + off);
    }
  }
}

template <typename T>
static int launch_rotary(int width, dim3 grid, dim3 block, hipStream_t s, const RotaryArgs& a) {
  switch (width) {
    case 16: hipLaunchKernelGGL((kv_append_rotary_kernel<T, 16>), grid, block, 0, s, a); break;
    case 8: hipLaunchKernelGGL((kv_append_rotary_kernel<T, 8>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((kv_append_rotary_kernel<T, 4>), grid, block, 0, s, a); break;
    default:
      if constexpr (sizeof(T) == 2) {
        hipLaunchKernelGGL((kv_append_rotary_kernel<T, 2>), grid, block, 0, s, a);
        break;
      }
      return LVAMD_ERR_INVALID_ARGUMENT;
  }
  return launch_status();
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
// scatter in a second, stream-ordered kernel.  lvamd_kv_compact_small runs
// the inline kernel with the pairs in its kernel arguments (the launch
// carries them: no index buffer, no upload).
// ---------------------------------------------------------------------------
constexpr int kCompactInline = 32;

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

// The pairs of lvamd_kv_compact_small, in the kernel arguments.
struct CompactSmallArgs {
  const uint64_t* kptrs;
  const uint64_t* vptrs;
  int32_t num_layers;
  int64_t row_bytes;
  int64_t num_pairs;
  int64_t src[kCompactInline];
  int64_t dst[kCompactInline];
};

// N (8, 16 or 32) is the smallest bucket holding the call's pairs.  Every
// one of the N gathers is issued (entries past the pairs re-read pair 0),
// so the row chunks stay in registers: conditional gathers into the array
// made the compiler keep it in scratch memory (512 bytes per lane).
template <typename V, typename Args, int N>
__global__ __launch_bounds__(256) void kv_compact_inline_kernel(const Args a) {
  const int64_t cpr = a.row_bytes / (int64_t)sizeof(V);
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= (int64_t)a.num_layers * 2 * cpr) return;
  const int64_t c = item % cpr;
  const int64_t rest = item / cpr;
  const int is_v = (int)(rest & 1);
  const int layer = (int)(rest >> 1);
  char* base = reinterpret_cast<char*>(is_v ? a.vptrs[layer] : a.kptrs[layer]);
  const int n = (int)a.num_pairs;
  V tmp[N];
#pragma unroll
  for (int i = 0; i < N; ++i) tmp[i] = reinterpret_cast<const V*>(base + a.src[i < n ? i : 0] * a.row_bytes)[c];
  // Every gather has landed before the first scatter is issued.
  __threadfence_block();
#pragma unroll
  for (int i = 0; i < N; ++i) {
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
// Ordered compact (lvamd_kv_compact_ordered): one HBM pass for pair lists
// whose order makes moving in place safe.  The pairs come in groups (one per
// request) that touch disjoint rows; inside a group no pair's destination is
// the source of a later pair (the host proves both; a step's accepted tree
// paths, retained indices strictly increasing, always qualify).  One thread
// per (group, layer, K|V, column chunk) moves its group's rows in order,
// kOrderedBatch pairs at a time: every source of a batch is read before its
// destinations are written, and a later batch reads no row an earlier one
// wrote.  Unlike the two-phase path, no row crosses HBM twice and no
// workspace is needed.
// ---------------------------------------------------------------------------
constexpr int kOrderedBatch = 16;

struct OrderedCompactArgs {
  const uint64_t* kptrs;
  const uint64_t* vptrs;
  int32_t num_layers;
  int64_t row_bytes;
  const int64_t* src;
  const int64_t* dst;
  const int64_t* group_starts;  // [num_groups + 1]
  int64_t num_groups;
};

// V is the chunk type: the native 4 x u32 vector for 16-byte chunks (an
// array of HIP's uint4 struct stayed in scratch memory, 272 bytes per lane,
// and the scratch traffic made this one-pass kernel slower than the
// two-phase one).  Eight 16-byte chunks per batch (sixteen narrower ones)
// keep the batch in registers.  Every gather of a batch is issued (entries
// past the group re-read its last source): conditional gathers into the
// array also leave it in scratch.
template <typename V>
__global__ __launch_bounds__(256) void kv_compact_ordered_kernel(const OrderedCompactArgs a) {
  constexpr int kBatch = sizeof(V) >= 16 ? kOrderedBatch / 2 : kOrderedBatch;
  const int64_t cpr = a.row_bytes / (int64_t)sizeof(V);
  const int64_t per_group = (int64_t)a.num_layers * 2 * cpr;
  const int64_t item = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= a.num_groups * per_group) return;
  const int64_t group = item / per_group;
  const int64_t r = item - group * per_group;
  const int64_t c = r % cpr;
  const int64_t lk = r / cpr;  // layer * 2 + is_v
  char* base = reinterpret_cast<char*>((lk & 1) ? a.vptrs[lk >> 1] : a.kptrs[lk >> 1]);
  const int64_t p0 = a.group_starts[group], p1 = a.group_starts[group + 1];
  for (int64_t b = p0; b < p1; b += kBatch) {
    V tmp[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int64_t p = b + i < p1 ? b + i : p1 - 1;
      tmp[i] = reinterpret_cast<const V*>(base + a.src[p] * a.row_bytes)[c];
    }
    // Every gather of the batch has landed before its first scatter.
    __threadfence_block();
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      if (b + i < p1) reinterpret_cast<V*>(base + a.dst[b + i] * a.row_bytes)[c] = tmp[i];
    }
    __threadfence_block();
  }
}

// ---------------------------------------------------------------------------
// Allocation-free compact (lvamd_kv_compact_static): the two-phase kernels
// stage their rows in this file-scope array instead of a caller workspace.
// Each GPU holds its own copy for the life of the process; its device
// address is looked up once per device (hipGetSymbolAddress, with that device
// current) and kept, and only that address is handed to kernels.  Every call
// on a GPU shares the array: calls that overlap on one GPU race.  Nothing in
// it needs clearing (the gather phase writes every staged byte before the
// scatter phase reads it).
// ---------------------------------------------------------------------------
constexpr int64_t kStaticScratchBytes = LVAMD_COMPACT_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
static std::atomic<char*> g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mutex;

// The current device's address of ``scratch``.
static int static_scratch(char** out) {
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return LVAMD_ERR_LAUNCH;
  if (device < 0 || device >= kMaxDevices) return LVAMD_ERR_UNSUPPORTED;
  char* ptr = g_scratch_ptr[device].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ptr = g_scratch_ptr[device].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      void* addr = nullptr;
      if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || addr == nullptr) return LVAMD_ERR_LAUNCH;
      ptr = static_cast<char*>(addr);
      g_scratch_ptr[device].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return LVAMD_OK;
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

// The pairs of lvamd_kv_block_copy_small, in the kernel arguments.
constexpr int kBlockCopySmall = 32;
struct BlockCopySmallArgs {
  const uint64_t* kptrs;
  const uint64_t* vptrs;
  int32_t num_layers;
  int64_t block_bytes;
  int64_t src[kBlockCopySmall];
  int64_t dst[kBlockCopySmall];
};

template <typename V, typename Args = BlockCopyArgs>
__global__ __launch_bounds__(256) void kv_block_copy_kernel(const Args a) {
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

template <typename Args, int N>
static int launch_compact_inline_n(int width, const dim3 grid, hipStream_t s, const Args& a) {
  switch (width) {
    case 16: hipLaunchKernelGGL((kv_compact_inline_kernel<u32x4, Args, N>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((kv_compact_inline_kernel<uint2, Args, N>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((kv_compact_inline_kernel<uint32_t, Args, N>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((kv_compact_inline_kernel<uint16_t, Args, N>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((kv_compact_inline_kernel<uint8_t, Args, N>), grid, dim3(256), 0, s, a); break;
  }
  return launch_status();
}

// One thread per row chunk of every (layer, K|V): a step's few pairs over 28
// layers of 512-byte rows make only seven workgroups at 16-byte chunks, so
// the chunk narrows (to 4 bytes at least) until about 32 workgroups share the
// latency-bound gather and scatter.
template <typename Args>
static int launch_compact_inline(int width, int32_t num_layers, int64_t row_bytes, hipStream_t s, const Args& a) {
  static_assert(kCompactInline == 32, "buckets of 8, 16 and 32 pairs");
  while (width > 4 && (int64_t)num_layers * 2 * (row_bytes / width) < 32 * 256) width /= 2;
  const int64_t items = (int64_t)num_layers * 2 * (row_bytes / width);
  const dim3 grid((unsigned)((items + 255) / 256));
  if (a.num_pairs <= 8) return launch_compact_inline_n<Args, 8>(width, grid, s, a);
  if (a.num_pairs <= 16) return launch_compact_inline_n<Args, 16>(width, grid, s, a);
  return launch_compact_inline_n<Args, 32>(width, grid, s, a);
}

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
    case LVAMD_ERR_SCRATCH_LIMIT: return "call needs more than the library's static scratch holds";
    case LVAMD_ERR_RUNTIME: return "HIP runtime call failed";
    default: return "unknown status";
  }
}

int lvamd_abi_version(void) { return 20; }

int lvamd_xcd_count(void) {
  int device = 0, xcds = 0;
  if (hipGetDevice(&device) != hipSuccess) return LVAMD_ERR_RUNTIME;
  if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, device) != hipSuccess) return LVAMD_ERR_RUNTIME;
  return xcds;
}

int lvamd_stage_upload(void* device_dst, const void* pinned_src, int64_t bytes, void* event, lvamd_stream_t stream) {
  if (bytes < 0 || (bytes > 0 && (!device_dst || !pinned_src))) return LVAMD_ERR_INVALID_ARGUMENT;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (bytes > 0 && hipMemcpyAsync(device_dst, pinned_src, (size_t)bytes, hipMemcpyHostToDevice, s) != hipSuccess)
    return LVAMD_ERR_RUNTIME;
  if (event != nullptr && hipEventRecord(static_cast<hipEvent_t>(event), s) != hipSuccess) return LVAMD_ERR_RUNTIME;
  return LVAMD_OK;
}

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

int lvamd_kv_append_rotary(const void* query, int64_t query_token_stride, int64_t query_head_stride,
                           void* query_out, int64_t query_out_token_stride, int64_t query_out_head_stride,
                           const void* key, int64_t key_token_stride, int64_t key_head_stride,
                           const void* value, int64_t value_token_stride, int64_t value_head_stride,
                           const void* cosines, int64_t cosines_token_stride,
                           const void* sines, int64_t sines_token_stride,
                           void* key_pool, void* value_pool, const int64_t* slots, int64_t num_tokens,
                           int32_t num_query_heads, int32_t num_kv_heads, int32_t head_size, int32_t dtype,
                           lvamd_stream_t stream) {
  const int es = dtype_size(dtype);
  if (es == 0) return LVAMD_ERR_UNSUPPORTED;
  if (num_tokens < 0 || num_query_heads <= 0 || num_kv_heads <= 0 || head_size <= 0 || head_size % 2 != 0)
    return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_tokens == 0) return LVAMD_OK;
  if (!query || !query_out || !key || !value || !cosines || !sines || !key_pool || !value_pool || !slots)
    return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_tokens > 0x7fffffffLL) return LVAMD_ERR_INVALID_ARGUMENT;
  RotaryArgs a;
  a.q = static_cast<const char*>(query);
  a.q_out = static_cast<char*>(query_out);
  a.key = static_cast<const char*>(key);
  a.value = static_cast<const char*>(value);
  a.cosines = static_cast<const char*>(cosines);
  a.sines = static_cast<const char*>(sines);
  a.q_tok_bytes = query_token_stride * es;
  a.q_head_bytes = query_head_stride * es;
  a.qo_tok_bytes = query_out_token_stride * es;
  a.qo_head_bytes = query_out_head_stride * es;
  a.key_tok_bytes = key_token_stride * es;
  a.key_head_bytes = key_head_stride * es;
  a.value_tok_bytes = value_token_stride * es;
  a.value_head_bytes = value_head_stride * es;
  a.cos_tok_bytes = cosines_token_stride * es;
  a.sin_tok_bytes = sines_token_stride * es;
  a.key_pool = static_cast<char*>(key_pool);
  a.value_pool = static_cast<char*>(value_pool);
  a.slots = slots;
  a.num_q_heads = num_query_heads;
  a.num_kv_heads = num_kv_heads;
  a.head_bytes = head_size * es;
  const int width = common_vector_bytes(
      {(uint64_t)(uintptr_t)query, (uint64_t)(uintptr_t)query_out, (uint64_t)(uintptr_t)key,
       (uint64_t)(uintptr_t)value, (uint64_t)(uintptr_t)cosines, (uint64_t)(uintptr_t)sines,
       (uint64_t)(uintptr_t)key_pool, (uint64_t)(uintptr_t)value_pool, (uint64_t)a.q_tok_bytes,
       (uint64_t)a.q_head_bytes, (uint64_t)a.qo_tok_bytes, (uint64_t)a.qo_head_bytes, (uint64_t)a.key_tok_bytes,
       (uint64_t)a.key_head_bytes, (uint64_t)a.value_tok_bytes, (uint64_t)a.value_head_bytes,
       (uint64_t)a.cos_tok_bytes, (uint64_t)a.sin_tok_bytes, (uint64_t)(a.head_bytes / 2)});
  if (width < es) return LVAMD_ERR_INVALID_ARGUMENT;  // misaligned element rows
  const int items = (num_query_heads + num_kv_heads) * (a.head_bytes / 2 / width) + num_kv_heads * (a.head_bytes / width);
  const int threads = items >= 256 ? 256 : ((items + 63) / 64) * 64;
  const dim3 grid((unsigned)num_tokens);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case LVAMD_BF16: return launch_rotary<__bf16>(width, grid, dim3(threads), s, a);
    case LVAMD_F16: return launch_rotary<_Float16>(width, grid, dim3(threads), s, a);
    default: return launch_rotary<float>(width, grid, dim3(threads), s, a);
  }
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
  if (num_pairs <= kCompactInline) return launch_compact_inline(width, num_layers, row_bytes, s, a);
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

int lvamd_kv_compact_ordered(const uint64_t* layer_key_ptrs, const uint64_t* layer_value_ptrs,
                             int32_t num_layers, int64_t row_bytes,
                             const int64_t* src_slots, const int64_t* dst_slots, const int64_t* group_starts,
                             int64_t num_groups, lvamd_stream_t stream) {
  if (num_groups < 0 || num_layers <= 0 || row_bytes <= 0) return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_groups == 0) return LVAMD_OK;
  if (!layer_key_ptrs || !layer_value_ptrs || !src_slots || !dst_slots || !group_starts)
    return LVAMD_ERR_INVALID_ARGUMENT;
  OrderedCompactArgs a;
  a.kptrs = layer_key_ptrs;
  a.vptrs = layer_value_ptrs;
  a.num_layers = num_layers;
  a.row_bytes = row_bytes;
  a.src = src_slots;
  a.dst = dst_slots;
  a.group_starts = group_starts;
  a.num_groups = num_groups;
  int width = common_vector_bytes({(uint64_t)row_bytes});
  // Narrow the chunks (to 4 bytes at least) until about 64 workgroups share
  // a latency-bound call.
  while (width > 4 && num_groups * num_layers * 2 * (row_bytes / width) < 64 * 256) width /= 2;
  const int64_t items = num_groups * num_layers * 2 * (row_bytes / width);
  if ((items + 255) / 256 > 0x7fffffffLL) return LVAMD_ERR_INVALID_ARGUMENT;
  const dim3 grid((unsigned)((items + 255) / 256));
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (width) {
    case 16: hipLaunchKernelGGL(kv_compact_ordered_kernel<u32x4>, grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL(kv_compact_ordered_kernel<uint2>, grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL(kv_compact_ordered_kernel<uint32_t>, grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL(kv_compact_ordered_kernel<uint16_t>, grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(kv_compact_ordered_kernel<uint8_t>, grid, dim3(256), 0, s, a); break;
  }
  return launch_status();
}

int lvamd_kv_compact_small(const uint64_t* layer_key_ptrs, const uint64_t* layer_value_ptrs,
                           int32_t num_layers, int64_t row_bytes,
                           const int64_t* src_slots, const int64_t* dst_slots, int64_t num_pairs,
                           lvamd_stream_t stream) {
  if (num_pairs < 0 || num_pairs > kCompactInline || num_layers <= 0 || row_bytes <= 0)
    return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_pairs == 0) return LVAMD_OK;
  if (!layer_key_ptrs || !layer_value_ptrs || !src_slots || !dst_slots) return LVAMD_ERR_INVALID_ARGUMENT;
  CompactSmallArgs a;
  a.kptrs = layer_key_ptrs;
  a.vptrs = layer_value_ptrs;
  a.num_layers = num_layers;
  a.row_bytes = row_bytes;
  a.num_pairs = num_pairs;
  for (int64_t i = 0; i < kCompactInline; ++i) {
    a.src[i] = i < num_pairs ? src_slots[i] : 0;
    a.dst[i] = i < num_pairs ? dst_slots[i] : 0;
  }
  const int width = common_vector_bytes({(uint64_t)row_bytes});
  return launch_compact_inline(width, num_layers, row_bytes, static_cast<hipStream_t>(stream), a);
}

int lvamd_kv_compact_static(const uint64_t* layer_key_ptrs, const uint64_t* layer_value_ptrs,
                            int32_t num_layers, int64_t row_bytes,
                            const int64_t* src_slots, const int64_t* dst_slots, int64_t num_pairs,
                            lvamd_stream_t stream) {
  if (num_pairs < 0 || num_layers <= 0 || row_bytes <= 0) return LVAMD_ERR_INVALID_ARGUMENT;
  char* ws = nullptr;
  if (num_pairs > kCompactInline) {
    // Staged rows: num_pairs * num_layers * 2 * row_bytes, without overflow.
    const int64_t per_pair = (int64_t)num_layers * 2 * row_bytes;
    if (per_pair > kStaticScratchBytes || num_pairs > kStaticScratchBytes / per_pair) return LVAMD_ERR_SCRATCH_LIMIT;
    const int status = static_scratch(&ws);
    if (status != LVAMD_OK) return status;
  }
  return lvamd_kv_compact(layer_key_ptrs, layer_value_ptrs, num_layers, row_bytes, src_slots, dst_slots, num_pairs,
                          ws, ws ? kStaticScratchBytes : 0, stream);
}

int64_t lvamd_kv_block_copy_small_pairs(void) { return kBlockCopySmall; }

int lvamd_kv_block_copy_small(const uint64_t* layer_key_ptrs, const uint64_t* layer_value_ptrs,
                              int32_t num_layers, int64_t block_bytes,
                              const int64_t* src_blocks, const int64_t* dst_blocks, int64_t num_pairs,
                              lvamd_stream_t stream) {
  if (num_pairs < 0 || num_pairs > kBlockCopySmall || num_layers <= 0 || block_bytes <= 0)
    return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_pairs == 0) return LVAMD_OK;
  if (!layer_key_ptrs || !layer_value_ptrs || !src_blocks || !dst_blocks) return LVAMD_ERR_INVALID_ARGUMENT;
  BlockCopySmallArgs a;
  a.kptrs = layer_key_ptrs;
  a.vptrs = layer_value_ptrs;
  a.num_layers = num_layers;
  a.block_bytes = block_bytes;
  for (int64_t i = 0; i < kBlockCopySmall; ++i) {
    a.src[i] = i < num_pairs ? src_blocks[i] : 0;
    a.dst[i] = i < num_pairs ? dst_blocks[i] : 0;
  }
  const dim3 grid((unsigned)(num_pairs * 2 * num_layers));
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (common_vector_bytes({(uint64_t)block_bytes})) {
    case 16: hipLaunchKernelGGL((kv_block_copy_kernel<uint4, BlockCopySmallArgs>), grid, dim3(256), 0, s, a); break;
    case 8: hipLaunchKernelGGL((kv_block_copy_kernel<uint2, BlockCopySmallArgs>), grid, dim3(256), 0, s, a); break;
    case 4: hipLaunchKernelGGL((kv_block_copy_kernel<uint32_t, BlockCopySmallArgs>), grid, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL((kv_block_copy_kernel<uint16_t, BlockCopySmallArgs>), grid, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL((kv_block_copy_kernel<uint8_t, BlockCopySmallArgs>), grid, dim3(256), 0, s, a); break;
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
