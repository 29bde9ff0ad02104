// Split-K paged attention for short query runs on gfx950 (decode and
// speculative tree verification), plus the cross-partition merge.
//
// Semantics (light-vllm TorchPagedAttention, src/light_vllm/runtime/execution/
// paged_attention.py:323-380): query token j of request r with c = computed
// tokens sees logical positions [0, c) plus {c + i : i in ancestors(j) + {j}}
// (linear layouts: i <= j); q head h reads kv head h / group; scores are
// q.k * scale in fp32; softmax in fp32; output = (sum p v) / (sum p) in the
// query dtype.  There is no split-K in the reference; this kernel splits each
// sequence into partitions and merges their (max, sum, acc) partials.
//
// Mapping onto CDNA4 (one wave64 per workgroup):
//   * A work unit is (request, partition, column tile); the grid is
//     units x num_kv_heads, consecutive workgroups are the kv heads of the same
//     unit so a physical block's rows are streamed together.
//   * MFMA columns are (query, head-in-group) pairs of one kv head: 16 per
//     column tile, so a GQA group of 7 heads shares every K/V byte.
//   * S^T = K Q^T on MFMA 16x16x32 (bf16/fp16) or 16x16x4 (fp32): the A operand
//     is read straight from HBM in its MFMA layout (lane l holds 16 bytes of
//     token l%16), the B operand is Q held in registers for the whole unit.
//   * The S^T accumulator layout (lane l: column l%16, tokens 4*(l/16)+r) is
//     exactly the B-operand layout of O^T = V^T P^T, so P never leaves its lane.
//     V^T is staged through LDS (16 KB-padded rows, per-wave tile of 32 tokens).
//   * The online softmax state (max, sum) of column l%16 lives in lanes
//     l%16 + 16k; the max is reduced with two cross-row shuffles per tile, the
//     sum only once at the end.  exp2 with scale*log2(e) folded in.

#include <cmath>
#include <type_traits>

#include "lvamd_common.h"

namespace lvamd {

struct DecodeArgs {
  const void* q;
  int64_t q_tok_stride, q_head_stride;
  const void* k_pool;
  const void* v_pool;
  void* out;
  int64_t out_tok_stride, out_head_stride;
  const int32_t* __restrict__ req_meta;
  const int32_t* __restrict__ tables;
  const uint32_t* __restrict__ vis;
  const int32_t* __restrict__ units;
  float* part_acc;
  float* part_ml;
  int32_t num_kv_heads;
  int32_t group;
  int32_t block_size;
  int32_t bs_shift;  // log2(block_size) when a power of two, else -1
  int32_t partition_tokens;
  float scale_log2;
};

// MFMA building blocks per storage type.
template <typename T> struct Mma;

template <> struct Mma<__bf16> {
  // One 16-byte chunk = 8 elements = one 16x16x32 MFMA k-step.
  __device__ static __forceinline__ f32x4 qk(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(bitcast<bf16x8>(a), bitcast<bf16x8>(b), c, 0, 0, 0);
  }
};
template <> struct Mma<_Float16> {
  __device__ static __forceinline__ f32x4 qk(uint4 a, uint4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(bitcast<f16x8>(a), bitcast<f16x8>(b), c, 0, 0, 0);
  }
};
template <> struct Mma<float> {
  // One 16-byte chunk = 4 elements = four 16x16x4 MFMA k-steps.
  __device__ static __forceinline__ f32x4 qk(uint4 a, uint4 b, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.x), __uint_as_float(b.x), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.y), __uint_as_float(b.y), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.z), __uint_as_float(b.z), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a.w), __uint_as_float(b.w), c, 0, 0, 0);
    return c;
  }
};

template <typename T, int D>
struct DecodeShape {
  static constexpr int E16 = 16 / (int)sizeof(T);             // elements per 16-byte chunk
  static constexpr int NCH = (D + 4 * E16 - 1) / (4 * E16);    // chunk steps per lane per row
  static constexpr int NT = D / 16;                            // 16-row tiles of O^T
  static constexpr int RSE = D + E16;                          // LDS row stride, +16 bytes
  static_assert(D % 16 == 0 && D <= 256, "head size must be a multiple of 16, at most 256");
};

template <typename T, int D>
__global__ __launch_bounds__(64) void paged_decode_kernel(const DecodeArgs a) {
  using S = DecodeShape<T, D>;
  constexpr int E16 = S::E16, NCH = S::NCH, NT = S::NT, RSE = S::RSE;
  __shared__ __attribute__((aligned(16))) T vtile[32 * RSE];

  const int lane = threadIdx.x;
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int Hkv = a.num_kv_heads;
  const int unit = blockIdx.x / Hkv;
  const int kvh = blockIdx.x - unit * Hkv;

  const int32_t* u = a.units + unit * LVAMD_UNIT_FIELDS;
  const int req = u[0], part = u[1], ctile = u[2], pslot = u[3];
  const int32_t* rm = a.req_meta + req * LVAMD_REQ_FIELDS;
  const int table_off = rm[0], computed = rm[2], q_len = rm[3], q_start = rm[4];
  const int vis_off = rm[5], vis_words = rm[6];
  const int G = a.group;
  const int seq_len = computed + q_len;
  const int t_begin = part * a.partition_tokens;
  const int t_end = min(seq_len, t_begin + a.partition_tokens);

  // This lane's MFMA column: (query qi, head h of the group).
  const int ncols = q_len * G;
  const int col = ctile * 16 + l16;
  const bool col_ok = col < ncols;
  const int colc = col_ok ? col : ncols - 1;
  const int qi = colc / G;
  const int h = colc - qi * G;
  const int qhead = kvh * G + h;

  // B operand: Q^T chunks, kept in registers for the whole unit.
  const T* qrow = static_cast<const T*>(a.q) + (int64_t)(q_start + qi) * a.q_tok_stride +
                  (int64_t)qhead * a.q_head_stride;
  uint4 qf[NCH];
#pragma unroll
  for (int kk = 0; kk < NCH; ++kk) {
    const int d0 = (kk * 4 + g) * E16;
    qf[kk] = (col_ok && d0 < D) ? load16(qrow + d0) : zero_u4();
  }

  const uint32_t* vrow = (vis_off >= 0) ? a.vis + vis_off + (int64_t)qi * vis_words : nullptr;
  const int lin_last = computed + qi;  // linear layouts: last visible position

  const int64_t row_elems = (int64_t)Hkv * D;
  const T* kbase = static_cast<const T*>(a.k_pool) + (int64_t)kvh * D;
  const T* vbase = static_cast<const T*>(a.v_pool) + (int64_t)kvh * D;

  auto row_of = [&](int pos) -> int64_t {
    const int pc = pos < seq_len ? pos : seq_len - 1;
    int lb, off;
    if (a.bs_shift >= 0) {
      lb = pc >> a.bs_shift;
      off = pc & (a.block_size - 1);
    } else {
      lb = pc / a.block_size;
      off = pc - lb * a.block_size;
    }
    return (int64_t)a.tables[table_off + lb] * a.block_size + off;
  };

  uint4 kf[2][NCH], vf[2][NCH];
  auto load_tile = [&](int t0) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int64_t row = row_of(t0 + 16 * s + l16);
      const T* kp = kbase + row * row_elems;
      const T* vp = vbase + row * row_elems;
#pragma unroll
      for (int kk = 0; kk < NCH; ++kk) {
        const int d0 = (kk * 4 + g) * E16;
        if (d0 < D) {
          kf[s][kk] = load16(kp + d0);
          vf[s][kk] = load16(vp + d0);
        } else {
          kf[s][kk] = zero_u4();
          vf[s][kk] = zero_u4();
        }
      }
    }
  };

  float m_run = -INFINITY;
  float l_run = 0.f;
  f32x4 acc[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};

  load_tile(t_begin);
  for (int t0 = t_begin; t0 < t_end; t0 += 32) {
    // S^T tile: rows = 32 tokens (two 16-row halves), columns = this lane's col.
    f32x4 st[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      st[s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < NCH; ++kk) st[s] = Mma<T>::qk(kf[s][kk], qf[kk], st[s]);
    }

    // Stage this tile's V rows (natural [token][dim] order) in LDS; rows past
    // the sequence end are zero so 0-weight * value stays exactly 0.
    __syncthreads();
    const bool tail = t0 + 32 > seq_len;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const bool row_ok = !tail || (t0 + 16 * s + l16 < seq_len);
#pragma unroll
      for (int kk = 0; kk < NCH; ++kk) {
        const int d0 = (kk * 4 + g) * E16;
        if (d0 < D) {
          *reinterpret_cast<uint4*>(&vtile[(16 * s + l16) * RSE + d0]) = row_ok ? vf[s][kk] : zero_u4();
        }
      }
    }

    if (t0 + 32 < t_end) load_tile(t0 + 32);

    // Scale, mask, online softmax (log2 domain).
    const bool need_mask = t0 + 32 > computed;
    float sv[2][4];
    float mt = -INFINITY;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int pos = t0 + 16 * s + 4 * g + r;
        bool vis = true;
        if (need_mask) {
          if (pos >= seq_len) {
            vis = false;
          } else if (pos >= computed) {
            if (vrow == nullptr) {
              vis = pos <= lin_last;
            } else {
              const int j = pos - computed;
              vis = (vrow[j >> 5] >> (j & 31)) & 1u;
            }
          }
        }
        const float x = vis ? st[s][r] * a.scale_log2 : -INFINITY;
        sv[s][r] = x;
        mt = fmaxf(mt, x);
      }
    mt = wave_max_across_rows(mt);
    const float m_new = fmaxf(m_run, mt);
    const float base = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - base);
    float p[2][4];
    float psum = 0.f;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[s][r] = fast_exp2(sv[s][r] - base);
        psum += p[s][r];
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[n] *= alpha;

    __syncthreads();

    // O^T += V^T P^T.
    if constexpr (sizeof(T) == 2) {
      using V8 = typename std::conditional<std::is_same<T, __bf16>::value, bf16x8, f16x8>::type;
      V8 b;
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int r = 0; r < 4; ++r) b[s * 4 + r] = from_f32<T>(p[s][r]);
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        V8 av;
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) av[s * 4 + r] = vtile[(16 * s + 4 * g + r) * RSE + 16 * n + l16];
        if constexpr (std::is_same<T, __bf16>::value) {
          acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b, acc[n], 0, 0, 0);
        } else {
          acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b, acc[n], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int n = 0; n < NT; ++n) {
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float av = vtile[(16 * s + 4 * g + r) * RSE + 16 * n + l16];
            acc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, p[s][r], acc[n], 0, 0, 0);
          }
      }
    }
  }

  l_run = wave_sum_across_rows(l_run);

  if (pslot < 0) {
    if (!col_ok) return;
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
    T* orow = static_cast<T*>(a.out) + (int64_t)(q_start + qi) * a.out_tok_stride +
              (int64_t)qhead * a.out_head_stride;
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) orow[16 * n + 4 * g + r] = from_f32<T>(acc[n][r] * inv);
  } else {
    const int64_t cslot = ((int64_t)pslot * Hkv + kvh) * 16 + l16;
    float* pacc = a.part_acc + cslot * D;
#pragma unroll
    for (int n = 0; n < NT; ++n) *reinterpret_cast<f32x4*>(pacc + 16 * n + 4 * g) = acc[n];
    if (g == 0) {
      a.part_ml[cslot * 2 + 0] = m_run;
      a.part_ml[cslot * 2 + 1] = l_run;
    }
  }
}

// ---------------------------------------------------------------------------
// Merge: one 256-thread workgroup per (job, kv head); thread (col, d-lane).
// ---------------------------------------------------------------------------
struct MergeArgs {
  const float* part_acc;
  const float* part_ml;
  void* out;
  int64_t out_tok_stride, out_head_stride;
  const int32_t* __restrict__ req_meta;
  const int32_t* __restrict__ jobs;
  int32_t num_kv_heads;
  int32_t group;
};

template <typename T, int D>
__global__ __launch_bounds__(256) void paged_merge_kernel(const MergeArgs a) {
  const int Hkv = a.num_kv_heads;
  const int job = blockIdx.x / Hkv;
  const int kvh = blockIdx.x - job * Hkv;
  const int32_t* jb = a.jobs + job * LVAMD_MERGE_FIELDS;
  const int req = jb[0], ctile = jb[1], ps0 = jb[2], np = jb[3];
  const int32_t* rm = a.req_meta + req * LVAMD_REQ_FIELDS;
  const int q_len = rm[3], q_start = rm[4];
  const int G = a.group;
  const int cl = threadIdx.x >> 4;
  const int dl = threadIdx.x & 15;
  const int col = ctile * 16 + cl;
  if (col >= q_len * G) return;
  const int qi = col / G;
  const int h = col - qi * G;

  const int64_t pstride = (int64_t)Hkv * 16;  // column slots per partial
  const int64_t c0 = ((int64_t)ps0 * Hkv + kvh) * 16 + cl;
  float mmax = -INFINITY;
  for (int p = 0; p < np; ++p) mmax = fmaxf(mmax, a.part_ml[(c0 + p * pstride) * 2]);
  const float base = (mmax == -INFINITY) ? 0.f : mmax;
  float lsum = 0.f;
  constexpr int PER = D / 16;
  float o[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) o[i] = 0.f;
  for (int p = 0; p < np; ++p) {
    const int64_t cs = c0 + p * pstride;
    const float w = fast_exp2(a.part_ml[cs * 2] - base);
    lsum += w * a.part_ml[cs * 2 + 1];
    const float* pacc = a.part_acc + cs * D;
#pragma unroll
    for (int i = 0; i < PER; ++i) o[i] += w * pacc[16 * i + dl];
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  T* orow = static_cast<T*>(a.out) + (int64_t)(q_start + qi) * a.out_tok_stride +
            (int64_t)(kvh * G + h) * a.out_head_stride;
#pragma unroll
  for (int i = 0; i < PER; ++i) orow[16 * i + dl] = from_f32<T>(o[i] * inv);
}

template <typename T>
static int launch_decode_t(int head_size, dim3 grid, hipStream_t s, const DecodeArgs& a) {
  switch (head_size) {
    case 32: hipLaunchKernelGGL((paged_decode_kernel<T, 32>), grid, dim3(64), 0, s, a); break;
    case 64: hipLaunchKernelGGL((paged_decode_kernel<T, 64>), grid, dim3(64), 0, s, a); break;
    case 80: hipLaunchKernelGGL((paged_decode_kernel<T, 80>), grid, dim3(64), 0, s, a); break;
    case 96: hipLaunchKernelGGL((paged_decode_kernel<T, 96>), grid, dim3(64), 0, s, a); break;
    case 128: hipLaunchKernelGGL((paged_decode_kernel<T, 128>), grid, dim3(64), 0, s, a); break;
    case 256: hipLaunchKernelGGL((paged_decode_kernel<T, 256>), grid, dim3(64), 0, s, a); break;
    default: return LVAMD_ERR_UNSUPPORTED;
  }
  return launch_status();
}

template <typename T>
static int launch_merge_t(int head_size, dim3 grid, hipStream_t s, const MergeArgs& a) {
  switch (head_size) {
    case 32: hipLaunchKernelGGL((paged_merge_kernel<T, 32>), grid, dim3(256), 0, s, a); break;
    case 64: hipLaunchKernelGGL((paged_merge_kernel<T, 64>), grid, dim3(256), 0, s, a); break;
    case 80: hipLaunchKernelGGL((paged_merge_kernel<T, 80>), grid, dim3(256), 0, s, a); break;
    case 96: hipLaunchKernelGGL((paged_merge_kernel<T, 96>), grid, dim3(256), 0, s, a); break;
    case 128: hipLaunchKernelGGL((paged_merge_kernel<T, 128>), grid, dim3(256), 0, s, a); break;
    case 256: hipLaunchKernelGGL((paged_merge_kernel<T, 256>), grid, dim3(256), 0, s, a); break;
    default: return LVAMD_ERR_UNSUPPORTED;
  }
  return launch_status();
}

static bool head_size_supported(int d) {
  return d == 32 || d == 64 || d == 80 || d == 96 || d == 128 || d == 256;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace lvamd

using namespace lvamd;

extern "C" int lvamd_paged_decode(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                  const void* key_pool, const void* value_pool,
                                  void* out, int64_t out_token_stride, int64_t out_head_stride,
                                  const int32_t* req_meta, const int32_t* tables, const uint32_t* vis,
                                  const int32_t* units, int32_t num_units,
                                  float* part_acc, float* part_ml, int64_t num_partial_slots,
                                  int32_t num_kv_heads, int32_t group, int32_t head_size,
                                  int32_t block_size, int32_t partition_tokens, float scale,
                                  int32_t dtype, lvamd_stream_t stream) {
  const int es = dtype_size(dtype);
  if (es == 0 || !head_size_supported(head_size)) return LVAMD_ERR_UNSUPPORTED;
  if (num_units < 0 || num_kv_heads <= 0 || group <= 0 || block_size <= 0) return LVAMD_ERR_INVALID_ARGUMENT;
  if (partition_tokens <= 0 || partition_tokens % 32 != 0) return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_units == 0) return LVAMD_OK;
  if (!q || !key_pool || !value_pool || !out || !req_meta || !tables || !units)
    return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_partial_slots > 0 && (!part_acc || !part_ml)) return LVAMD_ERR_WORKSPACE;
  // 16-byte row chunks: base pointers and token/head strides must keep rows aligned.
  if (!aligned16(q) || !aligned16(key_pool) || !aligned16(value_pool) ||
      (q_token_stride * es) % 16 != 0 || (q_head_stride * es) % 16 != 0)
    return LVAMD_ERR_INVALID_ARGUMENT;
  if ((int64_t)num_units * num_kv_heads > 0x7fffffffLL) return LVAMD_ERR_INVALID_ARGUMENT;
  DecodeArgs a;
  a.q = q;
  a.q_tok_stride = q_token_stride;
  a.q_head_stride = q_head_stride;
  a.k_pool = key_pool;
  a.v_pool = value_pool;
  a.out = out;
  a.out_tok_stride = out_token_stride;
  a.out_head_stride = out_head_stride;
  a.req_meta = req_meta;
  a.tables = tables;
  a.vis = vis;
  a.units = units;
  a.part_acc = part_acc;
  a.part_ml = part_ml;
  a.num_kv_heads = num_kv_heads;
  a.group = group;
  a.block_size = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.partition_tokens = partition_tokens;
  a.scale_log2 = scale * 1.4426950408889634f;
  const dim3 grid((unsigned)(num_units * num_kv_heads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case LVAMD_BF16: return launch_decode_t<__bf16>(head_size, grid, s, a);
    case LVAMD_F16: return launch_decode_t<_Float16>(head_size, grid, s, a);
    default: return launch_decode_t<float>(head_size, grid, s, a);
  }
}

extern "C" int lvamd_paged_attention_merge(const float* part_acc, const float* part_ml,
                                           void* out, int64_t out_token_stride, int64_t out_head_stride,
                                           const int32_t* req_meta, const int32_t* jobs, int32_t num_jobs,
                                           int32_t num_kv_heads, int32_t group, int32_t head_size,
                                           int32_t dtype, lvamd_stream_t stream) {
  const int es = dtype_size(dtype);
  if (es == 0 || !head_size_supported(head_size)) return LVAMD_ERR_UNSUPPORTED;
  if (num_jobs < 0 || num_kv_heads <= 0 || group <= 0) return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_jobs == 0) return LVAMD_OK;
  if (!part_acc || !part_ml || !out || !req_meta || !jobs) return LVAMD_ERR_INVALID_ARGUMENT;
  if ((int64_t)num_jobs * num_kv_heads > 0x7fffffffLL) return LVAMD_ERR_INVALID_ARGUMENT;
  MergeArgs a;
  a.part_acc = part_acc;
  a.part_ml = part_ml;
  a.out = out;
  a.out_tok_stride = out_token_stride;
  a.out_head_stride = out_head_stride;
  a.req_meta = req_meta;
  a.jobs = jobs;
  a.num_kv_heads = num_kv_heads;
  a.group = group;
  const dim3 grid((unsigned)(num_jobs * num_kv_heads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case LVAMD_BF16: return launch_merge_t<__bf16>(head_size, grid, s, a);
    case LVAMD_F16: return launch_merge_t<_Float16>(head_size, grid, s, a);
    default: return launch_merge_t<float>(head_size, grid, s, a);
  }
}
