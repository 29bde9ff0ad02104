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
//   * Per 32-token tile, lane (g = l/16, l%16) reads 16-byte chunks 4kk+g of
//     token rows l%16 and 16+l%16: the K chunks land in VGPRs already in the
//     A-operand layout of S^T = K Q^T (MFMA 16x16x32 bf16/fp16, 16x16x4 fp32);
//     the V chunks of the same addresses go HBM -> LDS by 16-byte LDS DMA
//     (global_load_lds), never through VGPRs.
//   * The S^T accumulator layout (lane l: column l%16, tokens 4*(l/16)+r) is
//     the B-operand layout of O^T = V^T P^T, so P never leaves its lane; the
//     V^T A operand comes out of LDS with ds_read_b64_tr_b16 transpose reads
//     (two per 16-row output tile).
//   * The block-table slice of a partition sits in LDS, so tile addresses
//     never wait on a table load; V is double-buffered in LDS and the next
//     tile's K/V are in flight while the current tile computes.
//   * Online softmax in the log2 domain (scale*log2(e) folded in) with lazy
//     rescaling: the running base only moves when a tile's max exceeds it by
//     more than 2^8, decided by a wave vote, so most tiles skip the O^T rescale.
//     The max is reduced across the four 16-lane rows with permlane swaps.

#include <cmath>
#include <type_traits>

#include "lvamd_common.h"

namespace lvamd {

// Block-table entries of one partition staged in LDS (the host keeps
// partition_tokens / block_size + 2 within this bound).
constexpr int kTableSlice = 256;
// Lazy-rescale threshold in log2 units: probabilities stay below 2^8.
constexpr float kRescaleSlack = 8.0f;

struct DecodeArgs {
  const void* q;
  int64_t q_tok_stride, q_head_stride;
  const void* k_pool;
  const void* v_pool;
  void* out;
  int64_t out_tok_stride, out_head_stride;
  const int32_t* __restrict__ pieces;      // [n_pieces][LVAMD_PIECE_FIELDS]
  const int32_t* __restrict__ wave_first;  // [waves_per_head + 1]
  const int32_t* __restrict__ tables;
  const uint32_t* __restrict__ vis;
  float* part_acc;
  float* part_ml;
  int32_t waves_per_head;
  int32_t num_kv_heads;
  int32_t group;
  int32_t block_size;
  int32_t bs_shift;  // log2(block_size) when a power of two, else -1
  float scale_log2;
};

// s_waitcnt vmcnt(0) in the gfx9 encoding (expcnt and lgkmcnt left at their
// maxima), through the builtin so LLVM's wait-insertion pass sees the wait.
constexpr int kWaitVmcnt0 = 0x0F70;

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4_t;
typedef __attribute__((address_space(3))) void lds_void_t;

// Max across the four 16-lane rows of a wave64 (xor 16 then xor 32) in VALU.
__device__ __forceinline__ float row_max4(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float row_sum4(float v) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// LDS slot (16-byte units) of V row r (0..31) chunk c of a 32-token tile:
// the DMA of instruction (s = r/16, kk = c/4) writes 64 consecutive slots,
// lane 16*(c%4) + r%16 at slot 16*(c%4) + r%16.
template <int NCH>
__device__ __forceinline__ int vslot(int r, int c) {
  return ((r >> 4) * NCH + (c >> 2)) * 64 + (c & 3) * 16 + (r & 15);
}

// One piece of a wave's share: a contiguous token range of one
// (request, column tile), with the request fields the kernel needs.
struct Piece {
  int req, ctile, tok_begin, tok_end, slot;
  int table_off, computed, q_len, q_start, vis_off, vis_words;
};

__device__ __forceinline__ Piece read_piece(const int32_t* __restrict__ pieces, int p) {
  const int32_t* r = pieces + (int64_t)p * LVAMD_PIECE_FIELDS;
  Piece x;
  x.req = r[0];
  x.ctile = r[1];
  x.tok_begin = r[2];
  x.tok_end = r[3];
  x.slot = r[4];
  x.table_off = r[5];
  x.computed = r[6];
  x.q_len = r[7];
  x.q_start = r[8];
  x.vis_off = r[9];
  x.vis_words = r[10];
  return x;
}

// This lane's MFMA column of a piece: (query qi, head h of the group).
struct LaneCol {
  int qi, qhead, lin_last;
  bool ok;
  const uint32_t* vrow;
};

template <typename T, int D>
__global__ __launch_bounds__(64) void paged_decode_kernel(const DecodeArgs a) {
  using S = TileShape<T, D>;
  constexpr int E16 = S::E16, NCH = S::NCH, NT = S::NT, CPR = S::CPR;
  constexpr int VSLOTS = 2 * NCH * 64;  // 16-byte LDS slots per V tile
  __shared__ __attribute__((aligned(16))) uint4 vlds[2][VSLOTS];
  __shared__ int32_t tab[2][kTableSlice];

  const int lane = threadIdx.x;
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int Hkv = a.num_kv_heads;
  const int G = a.group;
  // Head-major grid: the waves of one kv head are consecutive workgroups, so
  // the heads' slices of a row are not all requested at the same moment.
  const int kvh = blockIdx.x / a.waves_per_head;
  const int w = blockIdx.x - kvh * a.waves_per_head;
  int p = a.wave_first[w];
  const int p_end = a.wave_first[w + 1];
  if (p >= p_end) return;

  const int64_t row_elems = (int64_t)Hkv * D;
  const T* kbase = static_cast<const T*>(a.k_pool) + (int64_t)kvh * D;
  const T* vbase = static_cast<const T*>(a.v_pool) + (int64_t)kvh * D;

  auto logical_block = [&](int pos) -> int {
    return a.bs_shift >= 0 ? (pos >> a.bs_shift) : (pos / a.block_size);
  };

  // Block-table slice of a piece into tab[b] by 4-byte LDS DMA (the host keeps
  // a piece within kTableSlice - 2 blocks).
  auto issue_table = [&](const Piece& x, int b) {
    const int lb0 = logical_block(x.tok_begin);
    const int n = logical_block(x.tok_end - 1) - lb0 + 1;
    for (int i = 0; i < n; i += 64) {
      if (i + lane < n) {
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(a.tables + x.table_off + lb0 + i + lane),
                                         (lds_void_t*)(&tab[b][i]), 4, 0, 0);
      }
    }
  };

  auto lane_col = [&](const Piece& x) -> LaneCol {
    LaneCol c;
    const int ncols = x.q_len * G;
    const int col = x.ctile * 16 + l16;
    c.ok = col < ncols;
    const int colc = c.ok ? col : ncols - 1;
    c.qi = colc / G;
    c.qhead = kvh * G + (colc - c.qi * G);
    c.lin_last = x.computed + c.qi;
    c.vrow = (x.vis_off >= 0) ? a.vis + x.vis_off + (int64_t)c.qi * x.vis_words : nullptr;
    return c;
  };

  // B operand: Q^T chunks of this lane's column.
  auto issue_q = [&](const Piece& x, uint4 (&qdst)[NCH]) {
    const LaneCol c = lane_col(x);
    const T* qrow = static_cast<const T*>(a.q) + (int64_t)(x.q_start + c.qi) * a.q_tok_stride +
                    (int64_t)c.qhead * a.q_head_stride;
#pragma unroll
    for (int kk = 0; kk < NCH; ++kk) {
      const int ch = kk * 4 + g;
      qdst[kk] = (c.ok && ch < CPR) ? load16(qrow + ch * E16) : zero_u4();
    }
  };

  auto row_of = [&](const Piece& x, int b, int pos) -> int64_t {
    const int seq_len = x.computed + x.q_len;
    const int pc = pos < seq_len ? pos : seq_len - 1;
    const int lb = logical_block(pc);
    return (int64_t)tab[b][lb - logical_block(x.tok_begin)] * a.block_size + (pc - lb * a.block_size);
  };

  // Issue one 32-token tile of piece x: K chunks into registers, V chunks by
  // 16-byte LDS DMA into V buffer vb.  Rows past the sequence end read the
  // last real row (finite data whose probability is exactly 0).
  auto issue_tile = [&](const Piece& x, int tb, int t0, int vb, uint4 (&kdst)[2][NCH]) {
    const int64_t row0 = row_of(x, tb, t0 + l16);
    const int64_t row1 = row_of(x, tb, t0 + 16 + l16);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int64_t off = (s == 0 ? row0 : row1) * row_elems;
#pragma unroll
      for (int kk = 0; kk < NCH; ++kk) {
        const int c = kk * 4 + g;
        if (c < CPR) {
          kdst[s][kk] = load16(kbase + off + c * E16);
          __builtin_amdgcn_global_load_lds(static_cast<const void*>(vbase + off + c * E16),
                                           (lds_void_t*)(&vlds[vb][(s * NCH + kk) * 64]), 16, 0, 0);
        } else {
          kdst[s][kk] = zero_u4();
        }
      }
    }
  };

  // Prologue: this piece's table and Q, the next piece's table and Q, then
  // the first tile.
  Piece cur = read_piece(a.pieces, p);
  int tb = 0;
  uint4 qf[NCH], qn[NCH];
  issue_table(cur, tb);
  issue_q(cur, qf);
  bool have_nxt = p + 1 < p_end;
  Piece nxt = cur;
  if (have_nxt) {
    nxt = read_piece(a.pieces, p + 1);
    issue_table(nxt, tb ^ 1);
    issue_q(nxt, qn);
  }
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  uint4 kf[2][NCH];
  int vb = 0;
  issue_tile(cur, tb, cur.tok_begin, vb, kf);
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  bool nxt_pending = false;  // the next piece's table DMA is not known to have landed

  LaneCol lc = lane_col(cur);
  float m_run = -INFINITY;  // per-column base (log2 domain), uniform across the column's lanes
  float l_run = 0.f;        // this lane's share of the column's probability sum
  f32x4 acc[NT];
#pragma unroll
  for (int n = 0; n < NT; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  int t0 = cur.tok_begin;

  while (true) {
    // Keep the next tile in flight: the rest of this piece, else the first
    // tile of the next piece.
    const int nt0 = t0 + 32;
    const bool next_in_cur = nt0 < cur.tok_end;
    uint4 kn[2][NCH];
    if (next_in_cur) {
      issue_tile(cur, tb, nt0, vb ^ 1, kn);
    } else if (have_nxt) {
      if (nxt_pending) __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      issue_tile(nxt, tb ^ 1, nxt.tok_begin, vb ^ 1, kn);
    }

    // S^T tile: rows = 32 tokens (two 16-row halves), columns = this lane's col.
    f32x4 st[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      st[s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < NCH; ++kk) st[s] = Mma<T>::qk(kf[s][kk], qf[kk], st[s]);
    }

    // Scale and mask (only the tiles that reach the query region need masks).
    const int computed = cur.computed;
    const int seq_len = computed + cur.q_len;
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
            if (lc.vrow == nullptr) {
              vis = pos <= lc.lin_last;
            } else {
              const int j = pos - computed;
              vis = (lc.vrow[j >> 5] >> (j & 31)) & 1u;
            }
          }
        }
        const float x = vis ? st[s][r] * a.scale_log2 : -INFINITY;
        sv[s][r] = x;
        mt = fmaxf(mt, x);
      }
    mt = row_max4(mt);
    // Lazy rescale: move the base only when some column's max outgrows it.
    if (__any(mt > m_run + kRescaleSlack)) {
      const float m_new = fmaxf(m_run, mt);
      const float alpha = (m_new == -INFINITY) ? 1.f : fast_exp2(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int n = 0; n < NT; ++n) acc[n] *= alpha;
      m_run = m_new;
    }
    const float base = (m_run == -INFINITY) ? 0.f : m_run;
    float p4[2][4];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p4[s][r] = fast_exp2(sv[s][r] - base);
        l_run += p4[s][r];
      }

    // O^T += V^T P^T with V^T from the LDS tile.
    char* vbytes = reinterpret_cast<char*>(&vlds[vb][0]);
    if constexpr (sizeof(T) == 2) {
      using V8 = typename std::conditional<std::is_same<T, __bf16>::value, bf16x8, f16x8>::type;
      V8 pb;
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int r = 0; r < 4; ++r) pb[s * 4 + r] = from_f32<T>(p4[s][r]);
      const int q4 = l16 & 3;
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        // Lane (g, l16) addresses row 16j + 4g + l16/4, dims 16n + 4*(l16%4)..+3;
        // the transpose hands it dims 16n + l16 of rows 16j + 4g + 0..3.
        const int c = 2 * n + (q4 >> 1);
        const int lo = vslot<NCH>(4 * g + (l16 >> 2), c) * 16 + (q4 & 1) * 8;
        const int hi = vslot<NCH>(16 + 4 * g + (l16 >> 2), c) * 16 + (q4 & 1) * 8;
        const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vbytes + lo));
        const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vbytes + hi));
        const s16x4 both[2] = {v0, v1};
        const V8 av = bitcast<V8>(both);
        if constexpr (std::is_same<T, __bf16>::value) {
          acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pb, acc[n], 0, 0, 0);
        } else {
          acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, pb, acc[n], 0, 0, 0);
        }
      }
    } else {
      const float* vfl = reinterpret_cast<const float*>(vbytes);
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        const int d = 16 * n + l16;
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float av = vfl[vslot<NCH>(16 * s + 4 * g + r, d >> 2) * 4 + (d & 3)];
            acc[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, p4[s][r], acc[n], 0, 0, 0);
          }
      }
    }

    // The next tile (K registers and V DMA) and any table/Q prefetch have
    // landed once this wait returns.
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    nxt_pending = false;

    if (!next_in_cur) {
      // Piece finished: write the output (whole segment) or its partial.
      const float l_tot = row_sum4(l_run);
      if (cur.slot < 0) {
        if (lc.ok) {
          const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
          T* orow = static_cast<T*>(a.out) + (int64_t)(cur.q_start + lc.qi) * a.out_tok_stride +
                    (int64_t)lc.qhead * a.out_head_stride;
#pragma unroll
          for (int n = 0; n < NT; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) orow[16 * n + 4 * g + r] = from_f32<T>(acc[n][r] * inv);
        }
      } else if (lc.ok) {
        const int64_t cslot = ((int64_t)cur.slot * Hkv + kvh) * 16 + l16;
        float* pacc = a.part_acc + cslot * D;
#pragma unroll
        for (int n = 0; n < NT; ++n) *reinterpret_cast<f32x4*>(pacc + 16 * n + 4 * g) = acc[n];
        if (g == 0) {
          a.part_ml[cslot * 2 + 0] = m_run;
          a.part_ml[cslot * 2 + 1] = l_tot;
        }
      }
      if (!have_nxt) break;
      // Switch to the next piece (its first tile is already in flight) and
      // start fetching the one after.
      cur = nxt;
      tb ^= 1;
#pragma unroll
      for (int kk = 0; kk < NCH; ++kk) qf[kk] = qn[kk];
      lc = lane_col(cur);
      m_run = -INFINITY;
      l_run = 0.f;
#pragma unroll
      for (int n = 0; n < NT; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
      t0 = cur.tok_begin;
      ++p;
      have_nxt = p + 1 < p_end;
      if (have_nxt) {
        nxt = read_piece(a.pieces, p + 1);
        issue_table(nxt, tb ^ 1);
        issue_q(nxt, qn);
        nxt_pending = true;
      }
    } else {
      t0 = nt0;
    }
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int kk = 0; kk < NCH; ++kk) kf[s][kk] = kn[s][kk];
    vb ^= 1;
  }
}

// ---------------------------------------------------------------------------
// Merge: one thread per (job, kv head, column, 4-float chunk of the row);
// partials are combined in one pass with a running log-sum-exp base.
// ---------------------------------------------------------------------------
struct MergeArgs {
  const float* part_acc;
  const float* part_ml;
  void* out;
  int64_t out_tok_stride, out_head_stride;
  const int32_t* __restrict__ req_meta;
  const int32_t* __restrict__ jobs;
  int32_t num_jobs;
  int32_t num_kv_heads;
  int32_t group;
};

template <typename T, int D>
__global__ __launch_bounds__(256) void paged_merge_kernel(const MergeArgs a) {
  constexpr int DC = D / 4;  // 16-byte chunks of one partial row
  const int Hkv = a.num_kv_heads;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int dc = (int)(gid % DC);
  int64_t r = gid / DC;
  const int cl = (int)(r % 16);
  r /= 16;
  const int kvh = (int)(r % Hkv);
  const int64_t job = r / Hkv;
  if (job >= a.num_jobs) return;
  const int32_t* jb = a.jobs + job * LVAMD_MERGE_FIELDS;
  const int req = jb[0], ctile = jb[1], ps0 = jb[2], np = jb[3];
  const int32_t* rm = a.req_meta + req * LVAMD_REQ_FIELDS;
  const int q_len = rm[3], q_start = rm[4];
  const int G = a.group;
  const int col = ctile * 16 + cl;
  if (col >= q_len * G) return;
  const int qi = col / G;
  const int h = col - qi * G;

  const int64_t pstride = (int64_t)Hkv * 16;  // column slots per partial slot
  const int64_t c0 = ((int64_t)ps0 * Hkv + kvh) * 16 + cl;
  float mrun = -INFINITY;
  float lsum = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int p = 0; p < np; ++p) {
    const int64_t cs = c0 + p * pstride;
    const float2 ml = *reinterpret_cast<const float2*>(a.part_ml + cs * 2);
    const f32x4 pa = *reinterpret_cast<const f32x4*>(a.part_acc + cs * D + 4 * dc);
    const float mnew = fmaxf(mrun, ml.x);
    if (mnew == -INFINITY) continue;  // nothing visible so far
    const float sc = fast_exp2(mrun - mnew);  // 0 while mrun is -inf
    const float w = fast_exp2(ml.x - mnew);   // 0 for an empty partial
    lsum = lsum * sc + w * ml.y;
    o = o * sc + w * pa;
    mrun = mnew;
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  T* orow = static_cast<T*>(a.out) + (int64_t)(q_start + qi) * a.out_tok_stride +
            (int64_t)(kvh * G + h) * a.out_head_stride + 4 * dc;
#pragma unroll
  for (int i = 0; i < 4; ++i) orow[i] = from_f32<T>(o[i] * inv);
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
                                  const int32_t* pieces, const int32_t* wave_first, int32_t waves_per_head,
                                  const int32_t* tables, const uint32_t* vis,
                                  float* part_acc, float* part_ml, int64_t num_partial_slots,
                                  int32_t num_kv_heads, int32_t group, int32_t head_size,
                                  int32_t block_size, float scale, int32_t dtype, lvamd_stream_t stream) {
  const int es = dtype_size(dtype);
  if (es == 0 || !head_size_supported(head_size)) return LVAMD_ERR_UNSUPPORTED;
  if (waves_per_head < 0 || num_kv_heads <= 0 || group <= 0 || block_size <= 0) return LVAMD_ERR_INVALID_ARGUMENT;
  if (waves_per_head == 0) return LVAMD_OK;
  if (!q || !key_pool || !value_pool || !out || !pieces || !wave_first || !tables)
    return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_partial_slots > 0 && (!part_acc || !part_ml)) return LVAMD_ERR_WORKSPACE;
  // 16-byte row chunks: base pointers and token/head strides must keep rows aligned.
  if (!aligned16(q) || !aligned16(key_pool) || !aligned16(value_pool) ||
      (q_token_stride * es) % 16 != 0 || (q_head_stride * es) % 16 != 0)
    return LVAMD_ERR_INVALID_ARGUMENT;
  if ((int64_t)waves_per_head * num_kv_heads > 0x7fffffffLL) return LVAMD_ERR_INVALID_ARGUMENT;
  DecodeArgs a;
  a.q = q;
  a.q_tok_stride = q_token_stride;
  a.q_head_stride = q_head_stride;
  a.k_pool = key_pool;
  a.v_pool = value_pool;
  a.out = out;
  a.out_tok_stride = out_token_stride;
  a.out_head_stride = out_head_stride;
  a.pieces = pieces;
  a.wave_first = wave_first;
  a.tables = tables;
  a.vis = vis;
  a.part_acc = part_acc;
  a.part_ml = part_ml;
  a.waves_per_head = waves_per_head;
  a.num_kv_heads = num_kv_heads;
  a.group = group;
  a.block_size = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.scale_log2 = scale * 1.4426950408889634f;
  const dim3 grid((unsigned)(waves_per_head * num_kv_heads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case LVAMD_BF16: return launch_decode_t<__bf16>(head_size, grid, s, a);
    case LVAMD_F16: return launch_decode_t<_Float16>(head_size, grid, s, a);
    default: return launch_decode_t<float>(head_size, grid, s, a);
  }
}

template <typename T>
static const void* decode_kernel_ptr(int head_size) {
  switch (head_size) {
    case 32: return reinterpret_cast<const void*>(&paged_decode_kernel<T, 32>);
    case 64: return reinterpret_cast<const void*>(&paged_decode_kernel<T, 64>);
    case 80: return reinterpret_cast<const void*>(&paged_decode_kernel<T, 80>);
    case 96: return reinterpret_cast<const void*>(&paged_decode_kernel<T, 96>);
    case 128: return reinterpret_cast<const void*>(&paged_decode_kernel<T, 128>);
    case 256: return reinterpret_cast<const void*>(&paged_decode_kernel<T, 256>);
    default: return nullptr;
  }
}

extern "C" int lvamd_paged_decode_resident_waves(int32_t dtype, int32_t head_size) {
  if (dtype_size(dtype) == 0 || !head_size_supported(head_size)) return LVAMD_ERR_UNSUPPORTED;
  const void* fn = dtype == LVAMD_BF16 ? decode_kernel_ptr<__bf16>(head_size)
                   : dtype == LVAMD_F16 ? decode_kernel_ptr<_Float16>(head_size)
                                        : decode_kernel_ptr<float>(head_size);
  int device = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&device) != hipSuccess) return LVAMD_ERR_LAUNCH;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return LVAMD_ERR_LAUNCH;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 64, 0) != hipSuccess) return LVAMD_ERR_LAUNCH;
  return per_cu * cus;
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
  if ((int64_t)num_jobs * num_kv_heads * 16 * (head_size / 4) / 256 > 0x7fffffffLL) return LVAMD_ERR_INVALID_ARGUMENT;
  MergeArgs a;
  a.part_acc = part_acc;
  a.part_ml = part_ml;
  a.out = out;
  a.out_tok_stride = out_token_stride;
  a.out_head_stride = out_head_stride;
  a.req_meta = req_meta;
  a.jobs = jobs;
  a.num_jobs = num_jobs;
  a.num_kv_heads = num_kv_heads;
  a.group = group;
  const int64_t threads = (int64_t)num_jobs * num_kv_heads * 16 * (head_size / 4);
  const dim3 grid((unsigned)((threads + 255) / 256));
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case LVAMD_BF16: return launch_merge_t<__bf16>(head_size, grid, s, a);
    case LVAMD_F16: return launch_merge_t<_Float16>(head_size, grid, s, a);
    default: return launch_merge_t<float>(head_size, grid, s, a);
  }
}
