// Split-K paged attention for short query runs on gfx950 (decode and
// speculative tree verification) with the step's KV append fused in, plus the
// cross-partition merge.
//
// Semantics (light-vllm TorchPagedAttention, src/light_vllm/runtime/execution/
// paged_attention.py:323-380): query token j of request r with c = computed
// tokens sees logical positions [0, c) plus {c + i : i in ancestors(j) + {j}}
// (linear layouts: i <= j); q head h reads kv head h / group; scores are
// q.k * scale in fp32; softmax in fp32; output = (sum p v) / (sum p) in the
// query dtype.  There is no split-K in the reference; this kernel splits each
// sequence into partitions and merges their partials: each column's output
// row normalised by its own sum (in the pool's type) and its fp32 (max, sum).
//
// Mapping onto CDNA4 (one wave64 per workgroup, one workgroup per SIMD):
//   * MFMA columns are (query, head-in-group) pairs of one kv head, 16 per
//     column tile, so a GQA group shares every K/V byte.  A wave owns CTW
//     column tiles of one request (CTW = 1 for decode; 4 when a request's
//     queries x group need more than 16 columns, as in tree verification),
//     so every K/V byte it loads serves all of them.
//   * Stream-K: the (request, column-tile group) segments of all decode rows
//     are laid end to end in tile-sized units and cut into balanced
//     contiguous shares (the fewest shares that give the largest share the
//     resident waves would get), one per wave; wave w of kv head h is workgroup
//     h * waves_per_head + w and walks its pieces (the parts of segments
//     inside its share).  A piece covering a whole segment writes the output;
//     the others write partials that the merge kernel combines by
//     log-sum-exp, one wave per (segment, kv head, output column).  (Merging in
//     the decode kernel, by the wave that completes a segment, put ~1000
//     instructions of cold code in the kernel's tail: the instruction-cache
//     misses cost more than a separate launch.)
//   * Fused append: this step's tokens are read from the input K/V and
//     written to their pool slots by the piece that covers them.
//   * Per tile (32 tokens for one column tile, 16 for four or for wide
//     rows), lane (g = l/16, l%16) loads 16-byte chunks 4kk+g of token rows
//     16s + l%16 of K and V: the K chunks land in VGPRs already in the
//     A-operand layout of S^T = K Q^T (MFMA 16x16x32 bf16/fp16, 16x16x4
//     fp32); the V chunks are written to LDS after the current tile's PV.
//     (No LDS DMA: LLVM cannot tell an in-flight DMA into one buffer from
//     reads of the other and would make every LDS read wait for the next
//     tile's loads.)
//   * The S^T accumulator layout (lane l: column l%16, tokens 4*(l/16)+r) is
//     the B-operand layout of O^T = V^T P^T, so P never leaves its lane; the
//     V^T A operand comes out of LDS with ds_read_b64_tr_b16 transpose reads
//     (two per 16-row output tile, shared by the wave's column tiles).
//   * The block-table slice of a piece sits in LDS, so tile addresses
//     never wait on a table load; K is double-buffered in VGPRs and V in
//     LDS, and the next tile's K/V are in flight while the current tile
//     computes.
//   * Online softmax in the log2 domain (scale*log2(e) folded in) with lazy
//     rescaling: the running base only moves when a tile's max exceeds it by
//     more than 2^8, decided by a wave vote, so most tiles skip the O^T rescale.
//     The max is reduced across the four 16-lane rows with permlane swaps.

#include <cmath>
#include <type_traits>

#include "lvamd_common.h"

namespace lvamd {

// Block-table entries of one piece staged in LDS (the host keeps a piece
// within kTableSlice - 2 blocks).
constexpr int kTableSlice = 256;
// Lazy-rescale threshold in log2 units: probabilities stay below 2^8.
constexpr float kRescaleSlack = 8.0f;
// Piece fields 11..15: physical ids of the piece's first logical blocks.
constexpr int kPieceBlockField = 11;
constexpr int kPieceBlocks = 5;

struct DecodeArgs {
  const void* q;
  int64_t q_tok_stride, q_head_stride;
  const void* k_new;  // this step's K/V [tokens][kv heads][D], or null
  const void* v_new;
  int64_t kn_tok_stride, kn_head_stride, vn_tok_stride, vn_head_stride;
  void* k_pool;
  void* v_pool;
  void* out;
  int64_t out_tok_stride, out_head_stride;
  const int32_t* __restrict__ tables;
  const uint32_t* __restrict__ vis;
  void* part_acc;   // [slots][Hkv][CTW * 16][D] of T, each row normalised by its sum
  float* part_ml;   // [slots][Hkv][CTW * 16][2]: (max, sum)
  int32_t num_kv_heads;
  int32_t group;
  int32_t block_size;
  int32_t bs_shift;  // log2(block_size) when a power of two, else -1
  float scale_log2;
};

// LDS slot (16-byte units) of V row r chunk c of a tile: the (s = r/16,
// kk = c/4) chunk group is 64 consecutive slots, lane 16*(c%4) + r%16 at slot
// 16*(c%4) + r%16 (the order in which the lanes load it).
template <int NCH>
__device__ __forceinline__ int vslot(int r, int c) {
  return ((r >> 4) * NCH + (c >> 2)) * 64 + (c & 3) * 16 + (r & 15);
}

// Decode tile shape: a tile is TT tokens of one kv head.  With one column
// tile per wave, TT = 32 when a head's row slice is at most 256 bytes
// (bf16/fp16 up to D = 128, fp32 up to D = 64), else 16; with four column
// tiles TT = 16, which leaves registers for their Q operands and accumulators
// (at TT = 32 the bf16 D = 128 kernel spills).  32-token tiles beat 64 on the
// Qwen2.5-7B decode (62.8 against 65.3 us in one process): the stream-K
// shares, cut on whole tiles, then differ by a half tile instead of a whole
// one, and the memory system stays saturated with 16 KiB per wave in flight.
template <typename T, int D, int CTW>
struct DecodeTile {
  static constexpr int ROW = (int)sizeof(T) * D;
  static constexpr int TT1 = ROW <= 256 ? 32 : 16;
  static constexpr int TT = CTW == 1 ? TT1 : 16;
  static constexpr int SUB = TT / 16;                                // 16-row groups per tile
  static constexpr int VSLOTS = SUB * TileShape<T, D>::NCH * 64;     // 16-byte LDS slots per V tile
  // Each workgroup reserves more than 32 KiB of LDS (two V buffers of at
  // least 1024 slots plus the table slice), so a CU holds at most four decode
  // waves: one per SIMD.  Two waves sharing a SIMD stream at unequal rates
  // (the older one wins arbitration), which left the younger waves of a
  // static split finishing last.
  static constexpr int VALLOC = VSLOTS < 1024 ? 1024 : VSLOTS;
  // Line-order loads (one column tile, 16-bit pools with 16 chunks per head
  // row, i.e. bf16/fp16 at D = 128): each load instruction covers four whole
  // 256-byte row slices, i.e. whole 128-byte lines, instead of a 64-byte
  // piece of sixteen rows, and the loads are non-temporal.  K then goes
  // through LDS (into the MFMA operand layout) like V.  Gathering C2's blocks
  // this way takes 48.7 us against 53.9 for the operand-order pattern, whose
  // half-line accesses with non-temporal loads take 56.5 (probe kernels,
  // one process).  The K tile sits in the V buffer's padding.
  static constexpr int CPR = TileShape<T, D>::CPR;
  // (fp32 at D = 64 has 16 chunks per row too, but its latency-bound C1
  // step ran 15.7 -> 19.9 us with them: the K round trip through LDS.)
  static constexpr bool LINES_OK = sizeof(T) == 2 && CTW == 1 && CPR == 16 && TT == 32;
  static constexpr int RPI = 64 / CPR;     // token rows per line-order load
  static constexpr int LROWS = TT / RPI;   // line-order loads per lane per tensor
  static constexpr int KSLOTS = TT * CPR;  // 16-byte LDS slots of a K tile
  static_assert(!LINES_OK || (LROWS == SUB * TileShape<T, D>::NCH && VSLOTS + KSLOTS <= VALLOC),
                "line-order tiles reuse the operand-order register arrays and the V padding");
};

// Line-order LDS slots of a tile (row r, 16-byte chunk c of its head slice,
// CPR chunks per row): V rows XOR chunk bits 1-3 with row bits 0-2, so the
// transpose reads of four rows x two chunk pairs hit distinct banks; K rows
// XOR the chunk with row bits 0-3, so the 16 rows of an operand read hit
// distinct banks.  The line-order writes (one row per 16 lanes) are a
// permutation of one row's chunks either way.
template <int CPR>
__device__ __forceinline__ int vslot_lines(int r, int c) {
  return r * CPR + (c ^ ((2 * r) & (CPR - 2)));
}
template <int CPR>
__device__ __forceinline__ int kslot_lines(int r, int c) {
  return r * CPR + (c ^ (r & (CPR - 1)));
}

// One piece of a wave's share: a contiguous token range of one
// (request, column-tile group), with the request fields the kernel needs.
struct Piece {
  int req, cgroup, tok_begin, tok_end, slot;
  int table_off, computed, q_len, q_start, vis_off, vis_words;
};

__device__ __forceinline__ Piece read_piece(const int32_t* __restrict__ pieces, int p) {
  const int32_t* r = pieces + (int64_t)p * LVAMD_PIECE_FIELDS;
  Piece x;
  x.req = r[0];
  x.cgroup = r[1];
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

// This lane's MFMA column of one column tile: (query qi, head h of the group).
struct LaneCol {
  int qi, qhead, lin_last;
  bool ok;
  const uint32_t* vrow;
};

// Workgroup split (WG > 1): a latency-bound step (few short segments) is
// spread over workgroups of WG waves, one segment each: each wave runs one
// piece of its segment, the waves combine their results in LDS, and the
// segment's output is written by the workgroup, with no partials in memory
// and no merge launch.  WG = 1 is the stream-K kernel (one wave per
// workgroup, split segments merged by lvamd_paged_attention_merge).
//
// WG is eight where eight waves fit a CU without spilling (two waves per
// SIMD: at most 256 registers each) and their V buffers fit its LDS:
// bf16/fp16 up to D = 128 and fp32 up to D = 96; four otherwise.  With one
// piece per wave the kernel needs no next-piece prefetch registers.
template <typename T, int D>
constexpr int split_waves() {
  return (sizeof(T) == 2 && D <= 128) || (sizeof(T) == 4 && D <= 96) ? 8 : 4;
}
// Wave i's result lives in its own LDS: (max, sum) of column c at ml + i *
// ml_stride + 2c, the fp32 row at acc + i * acc_stride + c * D.
template <typename T, int D, int CTW, int WG>
__device__ __forceinline__ void merge_workgroup(const DecodeArgs& a, const float* ml, int ml_stride,
                                                const float* acc, int acc_stride, int kvh, int cgroup, int q_start,
                                                int q_len) {
  // Thread t < 256: column t % 16 of the segment's column tile (column
  // group cgroup), dims [(t / 16) * D / 16, + D / 16); the waves' rows weigh
  // sum_i * 2^(max_i - max) (each row normalised by its own sum).
  constexpr int DPT = D / 16;
  const int t = threadIdx.x;
  if (t >= 256) return;
  const int c = t & 15;
  const int d0 = (t >> 4) * DPT;
  const int col = cgroup * 16 + c;
  if (col >= q_len * a.group) return;
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < WG; ++i) m = fmaxf(m, ml[i * ml_stride + 2 * c]);
  float o[DPT];
#pragma unroll
  for (int e = 0; e < DPT; ++e) o[e] = 0.f;
  float lsum = 0.f;
#pragma unroll
  for (int i = 0; i < WG; ++i) {
    const float mi = ml[i * ml_stride + 2 * c];
    if (mi == -INFINITY) continue;  // an idle wave (its row holds nothing)
    const float wt = fast_exp2(mi - m) * ml[i * ml_stride + 2 * c + 1];
    lsum += wt;
    const float* row = acc + i * acc_stride + c * D + d0;
#pragma unroll
    for (int e = 0; e < DPT; ++e) o[e] += wt * row[e];
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  const int qi = col / a.group;
  const int qhead = kvh * a.group + (col - qi * a.group);
  T* orow = static_cast<T*>(a.out) + (int64_t)(q_start + qi) * a.out_tok_stride + (int64_t)qhead * a.out_head_stride;
#pragma unroll
  for (int e = 0; e < DPT; ++e) orow[d0 + e] = from_f32<T>(o[e] * inv);
}

template <typename T, int D, int CTW, int WG>
// The fields a wave needs first (its share's bounds, then its first piece)
// are scalar kernel arguments ahead of the struct: the build preloads leading
// scalar arguments into SGPRs, so those loads wait for no argument load.
__global__ __launch_bounds__(64 * WG) void paged_decode_kernel(
    const int32_t* __restrict__ wave_first,  // [waves_per_head + 1]
    const int32_t* __restrict__ pieces,      // [n_pieces][LVAMD_PIECE_FIELDS]
    const int32_t waves_per_head, const DecodeArgs a) {
  using S = TileShape<T, D>;
  using DT = DecodeTile<T, D, CTW>;
  constexpr int E16 = S::E16, NCH = S::NCH, NT = S::NT, CPR = S::CPR;
  constexpr int TT = DT::TT, SUB = DT::SUB;
  constexpr int TAB_PER_LANE = kTableSlice / 64;
  static_assert(WG == 1 || CTW == 1, "the workgroup split runs one column tile per wave");
  // One column tile prefetches the next piece's Q; four load theirs at the
  // piece switch (their registers hold the extra accumulators instead).
  // (In the workgroup split a wave has one piece: nothing to prefetch.)
  constexpr bool kPrefetchQ = CTW == 1 && WG == 1;
  // Line-order loads in the stream-K kernel (the workgroup split's LDS has no
  // room for K tiles): register array entry i = s * NCH + kk holds chunk
  // lane % CPR of tile row RPI * i + lane / CPR.
  constexpr bool LINES = DT::LINES_OK && WG == 1;
  constexpr int FR = LINES ? DT::LROWS : SUB;  // rows per lane a tile may append
  auto vs = [](int r, int c) -> int {
    if constexpr (LINES) {
      return vslot_lines<CPR>(r, c);
    } else {
      return vslot<NCH>(r, c);
    }
  };
  // Per wave: two V buffers (contiguous) and a table slice pair; in the
  // workgroup split the V buffers also take the wave's results at the end
  // (fp32 rows), and they are not padded (the stream-K kernel's padding
  // keeps it at one wave per SIMD).
  constexpr int VAL = WG == 1 ? DT::VALLOC : DT::VSLOTS;
  __shared__ __attribute__((aligned(16))) uint4 vlds_all[WG][2][VAL];
  __shared__ int32_t tab_all[WG][2][kTableSlice];
  static_assert(WG == 1 || 16 * D * 4 <= 2 * VAL * 16, "a wave's result rows must fit its V buffers");

  const int lane = threadIdx.x & 63;  // (the mask tells LLVM lane < 64)
  const int wid = WG == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  uint4* const vlds_a = &vlds_all[wid][0][0];
  uint4* const vlds_b = &vlds_all[wid][1][0];
  int32_t(*const tab)[kTableSlice] = tab_all[wid];
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int Hkv = a.num_kv_heads;
  const int G = a.group;
  // Head-major grid: the waves of one kv head are consecutive (in workgroups
  // of WG waves).
  constexpr int kWG = WG;
  const int wg_per_head = waves_per_head / kWG;
  const int kvh = blockIdx.x / wg_per_head;
  const int w = (blockIdx.x - kvh * wg_per_head) * kWG + wid;
  // The workgroup split holds one record per wave (wave w's at index w; an
  // idle wave's has request -1), so no wave_first lookup delays it.
  int p = WG == 1 ? wave_first[w] : w;
  const int p_end = WG == 1 ? wave_first[w + 1] : (pieces[(int64_t)w * LVAMD_PIECE_FIELDS] >= 0 ? w + 1 : w);
  // Workgroup split: each wave's result rows (fp32, normalised) in its own
  // V buffers and its (max, sum) pairs in its own table slices, then the
  // segment's merge once every wave has written.
  constexpr int kAccStride = 2 * VAL * 4;     // floats per wave's V buffers
  constexpr int kMlStride = 2 * kTableSlice;  // floats per wave's table slices
  float* const wg_acc = reinterpret_cast<float*>(vlds_a);
  float* const wg_ml = reinterpret_cast<float*>(&tab[0][0]);
  auto finish_workgroup = [&]() {
    if constexpr (WG > 1) {
      __syncthreads();
      const int32_t* lead = pieces + (int64_t)(w - wid) * LVAMD_PIECE_FIELDS;
      // A segment left whole in its first wave was written by that wave.
      if (lead[4] >= 0)
        merge_workgroup<T, D, CTW, WG>(a, reinterpret_cast<const float*>(&tab_all[0][0][0]), kMlStride,
                                       reinterpret_cast<const float*>(&vlds_all[0][0][0]), kAccStride, kvh,
                                       lead[1], lead[8], lead[7]);
    }
  };
  if (p >= p_end) {
    if constexpr (WG > 1) {
      // An idle wave of a split workgroup: no result (max -inf).
      if (lane < 16) {
        wg_ml[2 * lane] = -INFINITY;
        wg_ml[2 * lane + 1] = 0.f;
      }
      finish_workgroup();
    }
    return;
  }

  const int64_t row_elems = (int64_t)Hkv * D;
  // Global-address-space pointers: the tile loads select between the pool
  // and the input K/V per lane, and generic pointers would become flat loads.
  gptr<T> const kbase = (gptr<T>)(a.k_pool) + (int64_t)kvh * D;
  gptr<T> const vbase = (gptr<T>)(a.v_pool) + (int64_t)kvh * D;
  // Fused append: this step's tokens are read from the input K/V (so no
  // wave waits for another's pool write) and written to their pool slots by
  // the column-group-0 piece that covers them.
  gptr<const T> const knew =
      a.k_new ? (gptr<const T>)(a.k_new) + (int64_t)kvh * a.kn_head_stride : nullptr;
  gptr<const T> const vnew =
      a.v_new ? (gptr<const T>)(a.v_new) + (int64_t)kvh * a.vn_head_stride : nullptr;

  auto logical_block = [&](int pos) -> int {
    return a.bs_shift >= 0 ? (pos >> a.bs_shift) : (pos / a.block_size);
  };

  // Block-table slice of a piece: loaded into registers (lane i holds entries
  // i + 64j), stored to LDS when the piece's first tile is issued.
  auto load_table = [&](const Piece& x, int (&t)[TAB_PER_LANE]) {
    const int lb0 = logical_block(x.tok_begin);
    const int n = logical_block(x.tok_end - 1) - lb0 + 1;
#pragma unroll
    for (int j = 0; j < TAB_PER_LANE; ++j) {
      const int i = j * 64 + lane;
      t[j] = i < n ? a.tables[x.table_off + lb0 + i] : 0;
    }
  };
  auto store_table = [&](int b, const int (&t)[TAB_PER_LANE]) {
#pragma unroll
    for (int j = 0; j < TAB_PER_LANE; ++j) tab[b][j * 64 + lane] = t[j];
  };

  auto lane_col = [&](const Piece& x, int ct) -> LaneCol {
    LaneCol c;
    const int ncols = x.q_len * G;
    const int col = (x.cgroup * CTW + ct) * 16 + l16;
    c.ok = col < ncols;
    const int colc = c.ok ? col : ncols - 1;
    c.qi = colc / G;
    c.qhead = kvh * G + (colc - c.qi * G);
    c.lin_last = x.computed + c.qi;
    c.vrow = (x.vis_off >= 0) ? a.vis + x.vis_off + (int64_t)c.qi * x.vis_words : nullptr;
    return c;
  };

  // B operands: Q^T chunks of this lane's columns.
  auto load_q = [&](const Piece& x, uint4 (&qdst)[CTW][NCH]) {
#pragma unroll
    for (int ct = 0; ct < CTW; ++ct) {
      const LaneCol c = lane_col(x, ct);
      const T* qrow = static_cast<const T*>(a.q) + (int64_t)(x.q_start + c.qi) * a.q_tok_stride +
                      (int64_t)c.qhead * a.q_head_stride;
#pragma unroll
      for (int kk = 0; kk < NCH; ++kk) {
        const int ch = kk * 4 + g;
        qdst[ct][kk] = (c.ok && ch < CPR) ? load16(qrow + ch * E16) : zero_u4();
      }
    }
  };

  // Issue one TT-token tile of piece x (table slice in tab[tb]): K chunks and
  // V chunks into registers.  Positions past the piece read its last row
  // (finite data, masked to probability 0, already in cache).  All row
  // offsets are read from LDS before any load is issued.  fresh[s] is the
  // pool offset of row group s's row when this tile must append it, else -1.
  auto issue_tile_ids = [&](const Piece& x, int t0, auto block_id, uint4 (&kdst)[SUB][NCH],
                            uint4 (&vdst)[SUB][NCH], int64_t (&fresh)[FR]) {
    const int lb0 = logical_block(x.tok_begin);
    if constexpr (LINES) {
      // Line order: entry i is chunk lane % CPR of row RPI * i + lane / CPR.
      constexpr int RPI = DT::RPI;
      const int c = lane % CPR;
      gptr<const T> kp[FR];
      gptr<const T> vp[FR];
#pragma unroll
      for (int i = 0; i < FR; ++i) {
        const int pos = t0 + RPI * i + lane / CPR;
        const int pc = pos < x.tok_end ? pos : x.tok_end - 1;
        const int lb = logical_block(pc);
        const int64_t off = ((int64_t)block_id(lb - lb0) * a.block_size + (pc - lb * a.block_size)) * row_elems;
        kp[i] = kbase + off;
        vp[i] = vbase + off;
        fresh[i] = -1;
        if (knew != nullptr && pc >= x.computed) {
          const int64_t t = x.q_start + (pc - x.computed);
          kp[i] = knew + t * a.kn_tok_stride;
          vp[i] = vnew + t * a.vn_tok_stride;
          if (x.cgroup == 0 && pc == pos) fresh[i] = off;
        }
      }
#pragma unroll
      for (int i = 0; i < FR; ++i) {
        kdst[i / NCH][i % NCH] = load16_stream(kp[i] + c * E16);
        vdst[i / NCH][i % NCH] = load16_stream(vp[i] + c * E16);
      }
      return;
    }
    gptr<const T> kp[SUB];
    gptr<const T> vp[SUB];
#pragma unroll
    for (int s = 0; s < SUB; ++s) {
      const int pos = t0 + 16 * s + l16;
      const int pc = pos < x.tok_end ? pos : x.tok_end - 1;
      const int lb = logical_block(pc);
      const int64_t off = ((int64_t)block_id(lb - lb0) * a.block_size + (pc - lb * a.block_size)) * row_elems;
      kp[s] = kbase + off;
      vp[s] = vbase + off;
      fresh[s] = -1;
      if (knew != nullptr && pc >= x.computed) {
        const int64_t t = x.q_start + (pc - x.computed);
        kp[s] = knew + t * a.kn_tok_stride;
        vp[s] = vnew + t * a.vn_tok_stride;
        if (x.cgroup == 0 && pc == pos) fresh[s] = off;
      }
    }
#pragma unroll
    for (int s = 0; s < SUB; ++s)
#pragma unroll
      for (int kk = 0; kk < NCH; ++kk) {
        const int c = kk * 4 + g;
        if (c < CPR) {
          kdst[s][kk] = load16(kp[s] + c * E16);
          vdst[s][kk] = load16(vp[s] + c * E16);
        } else {
          kdst[s][kk] = zero_u4();
          vdst[s][kk] = zero_u4();
        }
      }
  };
  auto issue_tile = [&](const Piece& x, int tb, int t0, uint4 (&kdst)[SUB][NCH], uint4 (&vdst)[SUB][NCH],
                        int64_t (&fresh)[FR]) {
    issue_tile_ids(x, t0, [&](int rel) { return tab[tb][rel]; }, kdst, vdst, fresh);
  };
  // Append the tile's fresh rows to the pool (bit-exact row copies).
  auto store_fresh = [&](const uint4 (&kr)[SUB][NCH], const uint4 (&vr)[SUB][NCH], const int64_t (&fresh)[FR]) {
    if constexpr (LINES) {
      const int c = lane % CPR;
#pragma unroll
      for (int i = 0; i < FR; ++i) {
        if (fresh[i] >= 0) {
          store16(kbase + fresh[i] + c * E16, kr[i / NCH][i % NCH]);
          store16(vbase + fresh[i] + c * E16, vr[i / NCH][i % NCH]);
        }
      }
      return;
    }
#pragma unroll
    for (int s = 0; s < SUB; ++s) {
      if (fresh[s] >= 0) {
#pragma unroll
        for (int kk = 0; kk < NCH; ++kk) {
          const int c = kk * 4 + g;
          if (c < CPR) {
            store16(kbase + fresh[s] + c * E16, kr[s][kk]);
            store16(vbase + fresh[s] + c * E16, vr[s][kk]);
          }
        }
      }
    }
  };
  // Tile into LDS.  Operand order: V chunk (s, kk) of lane l at slot
  // (s * NCH + kk) * 64 + l (K stays in registers).  Line order: V and K rows
  // at their swizzled slots, K after the V tile.
  auto stage_v = [&](uint4* vdst, const uint4 (&vr)[SUB][NCH], const uint4 (&kr)[SUB][NCH]) {
    if constexpr (LINES) {
      const int c = lane % CPR;
#pragma unroll
      for (int i = 0; i < FR; ++i) {
        const int r = DT::RPI * i + lane / CPR;
        vdst[vslot_lines<CPR>(r, c)] = vr[i / NCH][i % NCH];
        vdst[DT::VSLOTS + kslot_lines<CPR>(r, c)] = kr[i / NCH][i % NCH];
      }
      return;
    }
#pragma unroll
    for (int s = 0; s < SUB; ++s)
#pragma unroll
      for (int kk = 0; kk < NCH; ++kk) vdst[(s * NCH + kk) * 64 + lane] = vr[s][kk];
  };
  // Line order: this tile's K operands (A layout of S^T = K Q^T: lane
  // (g, l16) holds chunk 4kk + g of row 16s + l16) from the LDS tile.
  auto read_k = [&](const uint4* vsrc, uint4 (&kdst)[SUB][NCH]) {
#pragma unroll
    for (int s = 0; s < SUB; ++s)
#pragma unroll
      for (int kk = 0; kk < NCH; ++kk)
        kdst[s][kk] = vsrc[DT::VSLOTS + kslot_lines<CPR>(16 * s + l16, kk * 4 + g)];
  };

  // Prologue.  The first tile is issued straight from the block ids the
  // piece record carries (when the tile spans at most kPieceBlocks blocks),
  // so it does not wait for the table slice; then this piece's table and Q,
  // the next piece's table (and Q).
  Piece cur = read_piece(pieces, p);
  int tb = 0;
  uint4 qf[CTW][NCH];
  uint4 qn[kPrefetchQ ? CTW : 1][NCH];
  int tn[TAB_PER_LANE];
  uint4 ka[SUB][NCH], kb[SUB][NCH];
  uint4 vr0[SUB][NCH];
  int64_t fresh0[FR];
  int tc[TAB_PER_LANE];
  const int first_span = logical_block(min(cur.tok_begin + TT, cur.tok_end) - 1) - logical_block(cur.tok_begin);
  const bool direct = first_span < kPieceBlocks;
  if (direct) {
    const int32_t* ids = pieces + (int64_t)p * LVAMD_PIECE_FIELDS + kPieceBlockField;
    const int b0 = ids[0], b1 = ids[1], b2 = ids[2], b3 = ids[3], b4 = ids[4];
    issue_tile_ids(
        cur, cur.tok_begin,
        [&](int rel) { return rel == 0 ? b0 : rel == 1 ? b1 : rel == 2 ? b2 : rel == 3 ? b3 : b4; }, ka, vr0,
        fresh0);
    load_table(cur, tc);
  } else {
    load_table(cur, tc);
    store_table(tb, tc);
    issue_tile(cur, tb, cur.tok_begin, ka, vr0, fresh0);
  }
  load_q(cur, qf);
  bool have_nxt = WG == 1 && p + 1 < p_end;
  bool nxt_stored = false;  // the next piece's table slice is in tab[tb ^ 1]
  Piece nxt = cur;
  if (have_nxt) {
    nxt = read_piece(pieces, p + 1);
    load_table(nxt, tn);
    if constexpr (kPrefetchQ) load_q(nxt, qn);
  }
  if (direct) store_table(tb, tc);
  stage_v(vlds_a, vr0, ka);
  store_fresh(ka, vr0, fresh0);

  LaneCol lc[CTW];
  float m_run[CTW];  // per-column base (log2 domain), uniform across the column's lanes
  float l_run[CTW];  // this lane's share of the column's probability sum
  f32x4 acc[CTW][NT];
#pragma unroll
  for (int ct = 0; ct < CTW; ++ct) {
    lc[ct] = lane_col(cur, ct);
    m_run[ct] = -INFINITY;
    l_run[ct] = 0.f;
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[ct][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  int t0 = cur.tok_begin;

  // One tile: start loading the next tile into (kx, registers for vx), then
  // compute the current one from (kc, vc), then stage the next V into vx.
  // Returns true when the current piece has ended.
  auto step = [&](uint4 (&kc)[SUB][NCH], uint4 (&kx)[SUB][NCH], uint4* vc, uint4* vx) -> bool {
    // Masks: only tiles that reach the piece end or the query region need
    // them.  A tree request's visibility words for this tile's query
    // positions (j = pos - computed spans at most three words) are loaded
    // before the next tile is issued.
    const int computed = cur.computed;
    const int tok_end = cur.tok_end;
    const bool need_mask = t0 + TT > (computed < tok_end ? computed : tok_end);
    // (One-dimensional word arrays: LLVM turns a two-dimensional one into
    // an LDS allocation.)
    uint32_t vw0[CTW], vw1[CTW], vw2[CTW];
    const int jw0 = (t0 > computed ? t0 - computed : 0) >> 5;
#pragma unroll
    for (int ct = 0; ct < CTW; ++ct) vw0[ct] = vw1[ct] = vw2[ct] = 0u;
    if (need_mask && lc[0].vrow != nullptr) {
      const int last_word = (cur.q_len - 1) >> 5;
      const int w0 = jw0 <= last_word ? jw0 : last_word;
      const int w1 = jw0 + 1 <= last_word ? jw0 + 1 : last_word;
      const int w2 = jw0 + 2 <= last_word ? jw0 + 2 : last_word;
#pragma unroll
      for (int ct = 0; ct < CTW; ++ct) {
        vw0[ct] = lc[ct].vrow[w0];
        vw1[ct] = lc[ct].vrow[w1];
        vw2[ct] = lc[ct].vrow[w2];
      }
    }

    // Line order: this tile's K operands come out of LDS (their reads
    // overlap the next tile's address arithmetic).
    uint4 kl[LINES ? SUB : 1][NCH];
    if constexpr (LINES) read_k(vc, kl);

    const int nt0 = t0 + TT;
    const bool next_in_cur = nt0 < cur.tok_end;
    uint4 vr[SUB][NCH];
    int64_t fresh[FR];
    const bool issued = next_in_cur || have_nxt;
    if (next_in_cur) {
      issue_tile(cur, tb, nt0, kx, vr, fresh);
    } else if (have_nxt) {
      if (!nxt_stored) {
        store_table(tb ^ 1, tn);
        nxt_stored = true;
      }
      issue_tile(nxt, tb ^ 1, nxt.tok_begin, kx, vr, fresh);
    }

    // S^T tiles: rows = TT tokens (16-row groups), columns = this lane's
    // column of each column tile; the K operands serve every column tile.
    f32x4 st[CTW][SUB];
#pragma unroll
    for (int s = 0; s < SUB; ++s)
#pragma unroll
      for (int ct = 0; ct < CTW; ++ct) {
        st[ct][s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < NCH; ++kk)
          st[ct][s] = Mma<T>::qk(LINES ? kl[s][kk] : kc[s][kk], qf[ct][kk], st[ct][s]);
      }

    // Scale, mask and the online softmax of each column tile.
    float p4[CTW][SUB][4];
#pragma unroll
    for (int ct = 0; ct < CTW; ++ct) {
      float sv[SUB][4];
      float mt = -INFINITY;
#pragma unroll
      for (int s = 0; s < SUB; ++s)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int pos = t0 + 16 * s + 4 * g + r;
          bool vis = true;
          if (need_mask) {
            if (pos >= tok_end) {
              vis = false;
            } else if (pos >= computed) {
              const int j = pos - computed;
              if (lc[ct].vrow == nullptr) {
                vis = pos <= lc[ct].lin_last;
              } else {
                const int wi = (j >> 5) - jw0;
                const uint32_t word = wi == 0 ? vw0[ct] : (wi == 1 ? vw1[ct] : vw2[ct]);
                vis = (word >> (j & 31)) & 1u;
              }
            }
          }
          const float x = vis ? st[ct][s][r] * a.scale_log2 : -INFINITY;
          sv[s][r] = x;
          mt = fmaxf(mt, x);
        }
      mt = row_max4(mt);
      // Lazy rescale: move the base only when some column's max outgrows it.
      if (__any(mt > m_run[ct] + kRescaleSlack)) {
        const float m_new = fmaxf(m_run[ct], mt);
        const float alpha = (m_new == -INFINITY) ? 1.f : fast_exp2(m_run[ct] - m_new);
        l_run[ct] *= alpha;
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[ct][n] *= alpha;
        m_run[ct] = m_new;
      }
      const float nbase = (m_run[ct] == -INFINITY) ? 0.f : -m_run[ct];
#pragma unroll
      for (int s = 0; s < SUB; ++s)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          p4[ct][s][r] = fast_exp2(sv[s][r] + nbase);  // sv is already scaled
          l_run[ct] += p4[ct][s][r];
        }
    }

    // O^T += V^T P^T with V^T from the LDS tile (each transpose read serves
    // every column tile): 32 tokens per MFMA k-step (16x16x32), or 16
    // (16x16x16) for a single 16-row group.
    char* vbytes = reinterpret_cast<char*>(vc);
    if constexpr (sizeof(T) == 2 && SUB == 1) {
      using V4 = typename std::conditional<std::is_same<T, __bf16>::value, s16x4, f16x4>::type;
      const int q4 = l16 & 3;
      V4 pb[CTW];
#pragma unroll
      for (int ct = 0; ct < CTW; ++ct) {
        T pt[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) pt[r] = from_f32<T>(p4[ct][0][r]);
        pb[ct] = bitcast<V4>(pt);
      }
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        // The transpose hands lane (g, l16) dims 16n + l16 of rows 4g + 0..3:
        // the A operand of a 16x16x16 step whose k index is 4g + e.
        const int c = 2 * n + (q4 >> 1);
        const int lo = vs(4 * g + (l16 >> 2), c) * 16 + (q4 & 1) * 8;
        const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vbytes + lo));
#pragma unroll
        for (int ct = 0; ct < CTW; ++ct) {
          if constexpr (std::is_same<T, __bf16>::value) {
            acc[ct][n] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v0, pb[ct], acc[ct][n], 0, 0, 0);
          } else {
            acc[ct][n] = __builtin_amdgcn_mfma_f32_16x16x16f16(bitcast<f16x4>(v0), pb[ct], acc[ct][n], 0, 0, 0);
          }
        }
      }
    } else if constexpr (sizeof(T) == 2) {
      using V8 = typename std::conditional<std::is_same<T, __bf16>::value, bf16x8, f16x8>::type;
      const int q4 = l16 & 3;
#pragma unroll
      for (int h = 0; h < SUB / 2; ++h) {
        V8 pb[CTW];
#pragma unroll
        for (int ct = 0; ct < CTW; ++ct)
#pragma unroll
          for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int r = 0; r < 4; ++r) pb[ct][s * 4 + r] = from_f32<T>(p4[ct][2 * h + s][r]);
#pragma unroll
        for (int n = 0; n < NT; ++n) {
          // Lane (g, l16) addresses row 32h + 16j + 4g + l16/4, dims
          // 16n + 4*(l16%4)..+3; the transpose hands it dims 16n + l16 of rows
          // 32h + 16j + 4g + 0..3.
          const int c = 2 * n + (q4 >> 1);
          const int lo = vs(32 * h + 4 * g + (l16 >> 2), c) * 16 + (q4 & 1) * 8;
          const int hi = vs(32 * h + 16 + 4 * g + (l16 >> 2), c) * 16 + (q4 & 1) * 8;
          const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vbytes + lo));
          const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vbytes + hi));
          const s16x4 both[2] = {v0, v1};
          const V8 av = bitcast<V8>(both);
#pragma unroll
          for (int ct = 0; ct < CTW; ++ct) {
            if constexpr (std::is_same<T, __bf16>::value) {
              acc[ct][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pb[ct], acc[ct][n], 0, 0, 0);
            } else {
              acc[ct][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, pb[ct], acc[ct][n], 0, 0, 0);
            }
          }
        }
      }
    } else {
      const float* vfl = reinterpret_cast<const float*>(vbytes);
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        const int d = 16 * n + l16;
#pragma unroll
        for (int s = 0; s < SUB; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float av = vfl[vs(16 * s + 4 * g + r, d >> 2) * 4 + (d & 3)];
#pragma unroll
            for (int ct = 0; ct < CTW; ++ct)
              acc[ct][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, p4[ct][s][r], acc[ct][n], 0, 0, 0);
          }
      }
    }

    // Next tile's V into the other LDS buffer (this waits for its loads),
    // and its fresh rows into the pool.
    if (issued) {
      stage_v(vx, vr, kx);
      store_fresh(kx, vr, fresh);
    }
    if (next_in_cur) t0 = nt0;
    return !next_in_cur;
  };

  // Results of a finished piece: the normalised output rows (a whole
  // segment) or its partials (normalised rows, max and sum).
  auto write_piece = [&](const Piece& x, const LaneCol (&lx)[CTW], const f32x4 (&ax)[CTW][NT],
                         const float (&mx)[CTW], const float (&sx)[CTW]) {
#pragma unroll
    for (int ct = 0; ct < CTW; ++ct) {
      if (!lx[ct].ok) continue;
      if (x.slot < 0) {
        const float inv = sx[ct] > 0.f ? 1.f / sx[ct] : 0.f;
        T* orow = static_cast<T*>(a.out) + (int64_t)(x.q_start + lx[ct].qi) * a.out_tok_stride +
                  (int64_t)lx[ct].qhead * a.out_head_stride;
#pragma unroll
        for (int n = 0; n < NT; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r) orow[16 * n + 4 * g + r] = from_f32<T>(ax[ct][n][r] * inv);
      } else if constexpr (WG > 1) {
        // Workgroup split: this wave's fp32 rows and (max, sum) into LDS
        // (the wave's own V buffers, free once its last tile is done).
        const float inv = sx[ct] > 0.f ? 1.f / sx[ct] : 0.f;
        float* racc = wg_acc + l16 * D;
#pragma unroll
        for (int n = 0; n < NT; ++n)
          *reinterpret_cast<f32x4*>(racc + 16 * n + 4 * g) =
              f32x4{ax[ct][n][0] * inv, ax[ct][n][1] * inv, ax[ct][n][2] * inv, ax[ct][n][3] * inv};
        if (g == 0) {
          wg_ml[2 * l16] = mx[ct];
          wg_ml[2 * l16 + 1] = sx[ct];
        }
      } else {
        const int64_t cs = ((int64_t)x.slot * Hkv + kvh) * (16 * CTW) + ct * 16 + l16;
        T* pacc = static_cast<T*>(a.part_acc) + cs * D;
        const float inv = sx[ct] > 0.f ? 1.f / sx[ct] : 0.f;
#pragma unroll
        for (int n = 0; n < NT; ++n) store_partial4<false, T>(pacc + 16 * n + 4 * g, ax[ct][n], inv);
        if (g == 0) *reinterpret_cast<float2*>(a.part_ml + cs * 2) = make_float2(mx[ct], sx[ct]);
      }
    }
  };

  // With one column tile a piece that is not the wave's last keeps its
  // results in registers and writes them after the wave's last piece: its
  // stores would otherwise enter the memory queues behind every wave's
  // in-flight tile loads, and reusing the accumulators would wait for them
  // (about 2 us per switch, measured).  Four column tiles and rows above 256
  // bytes have no registers to spare and write at once.
  constexpr bool kDeferWrite = CTW == 1 && WG == 1 && (int)sizeof(T) * D <= 256;
  bool pend = false;
  Piece pend_piece = cur;
  LaneCol pend_lc[CTW];
  f32x4 pend_acc[CTW][kDeferWrite ? NT : 1];
  float pend_m[CTW], pend_s[CTW];

  // Piece finished: write (or keep) its results, then switch to the next
  // piece (its first tile is already staged) and start fetching the one
  // after.  Returns false after the wave's last piece.
  auto end_piece = [&]() -> bool {
    if (!have_nxt) return false;
    float l_tot[CTW];
#pragma unroll
    for (int ct = 0; ct < CTW; ++ct) l_tot[ct] = row_sum4(l_run[ct]);
    if constexpr (kDeferWrite) {
      if (pend) write_piece(pend_piece, pend_lc, pend_acc, pend_m, pend_s);
      pend = true;
      pend_piece = cur;
#pragma unroll
      for (int ct = 0; ct < CTW; ++ct) {
        pend_lc[ct] = lc[ct];
        pend_m[ct] = m_run[ct];
        pend_s[ct] = l_tot[ct];
#pragma unroll
        for (int n = 0; n < NT; ++n) pend_acc[ct][n] = acc[ct][n];
      }
    } else {
      write_piece(cur, lc, acc, m_run, l_tot);
    }
    cur = nxt;
    tb ^= 1;
    if constexpr (kPrefetchQ) {
#pragma unroll
      for (int ct = 0; ct < CTW; ++ct)
#pragma unroll
        for (int kk = 0; kk < NCH; ++kk) qf[ct][kk] = qn[ct][kk];
    } else {
      load_q(cur, qf);
    }
#pragma unroll
    for (int ct = 0; ct < CTW; ++ct) {
      lc[ct] = lane_col(cur, ct);
      m_run[ct] = -INFINITY;
      l_run[ct] = 0.f;
#pragma unroll
      for (int n = 0; n < NT; ++n) acc[ct][n] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    t0 = cur.tok_begin;
    ++p;
    have_nxt = WG == 1 && p + 1 < p_end;
    nxt_stored = false;
    if (have_nxt) {
      nxt = read_piece(pieces, p + 1);
      load_table(nxt, tn);
      if constexpr (kPrefetchQ) load_q(nxt, qn);
    }
    return true;
  };

  // The K registers and V buffers swap roles every tile; two step copies keep
  // those roles static (a run-time choice would keep both K sets live).
  while (true) {
    if (step(ka, kb, vlds_a, vlds_b) && !end_piece()) break;
    if (step(kb, ka, vlds_b, vlds_a) && !end_piece()) break;
  }
  // The wave's last piece, written once after the loop (its code is not
  // duplicated into the two step copies).
  {
    float l_tot[CTW];
#pragma unroll
    for (int ct = 0; ct < CTW; ++ct) l_tot[ct] = row_sum4(l_run[ct]);
    write_piece(cur, lc, acc, m_run, l_tot);
    if constexpr (kDeferWrite) {
      if (pend) write_piece(pend_piece, pend_lc, pend_acc, pend_m, pend_s);
    }
  }
  finish_workgroup();
}

// ---------------------------------------------------------------------------
// Merge: one wave per (job, kv head, column); a workgroup holds the four
// waves of four consecutive columns.  Lane l combines dims EPL*l..+EPL-1 of
// its column over the job's partials, MCP partials per round trip (their
// (max, sum) pairs and normalised rows are all requested before any is
// used), by log-sum-exp in the log2 domain: partial i weighs
// sum_i * 2^(max_i - max).  Every lane computes the chunk's weights itself
// from the same (max, sum) values, so no cross-lane step is needed.
// ---------------------------------------------------------------------------
// The fields a wave needs first (its job record's address) are scalar kernel
// arguments ahead of the rest: the build preloads leading scalar arguments
// into SGPRs, so the job record's load does not wait for a kernel-argument
// load; the struct's fields are loaded meanwhile.
struct MergeArgs {
  const void* part_acc;  // rows of T, normalised
  const float* part_ml;
  void* out;
  int64_t out_tok_stride, out_head_stride;
};

constexpr int kMergeWaves = 4;  // columns (waves) per merge workgroup

template <typename T, int D>
__global__ __launch_bounds__(64 * kMergeWaves) void paged_merge_kernel(
    const int32_t* __restrict__ jobs,  // [num_jobs][LVAMD_MERGE_FIELDS]
    const int32_t quads,               // workgroups (of kMergeWaves columns) per (job, kv head)
    const int32_t num_kv_heads, const int32_t group,
    const int32_t col_tiles,           // column tiles per partial slot (the decode launch's)
    const MergeArgs a) {
  constexpr int EPL = D <= 64 ? 1 : (D <= 128 ? 2 : 4);  // dims per lane
  constexpr int MCP = 16;
  const int Hkv = num_kv_heads;
  const int G = group;
  const int cols = 16 * col_tiles;  // columns per partial slot
  const int jh = (int)blockIdx.x / quads;
  const int c = ((int)blockIdx.x - jh * quads) * kMergeWaves +
                __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int job = jh / Hkv;
  const int kvh = jh - job * Hkv;
  const int lane = threadIdx.x & 63;
  const int32_t* jb = jobs + (int64_t)job * LVAMD_MERGE_FIELDS;
  const int cgroup = jb[1], slot0 = jb[2], np = jb[3], q_start = jb[4], q_len = jb[5];
  const int col = cgroup * cols + c;
  if (col >= q_len * G) return;
  const int qi = col / G;
  const int qhead = kvh * G + (col - qi * G);
  const int e0 = lane * EPL;
  const bool act = e0 < D;
  // A request whose shared prefix was attended by span units (prefill jobs
  // only): fields 6 = first span partial slot + 1, 7 = the request's first
  // column within the span | pieces per span unit << 24.  Column v of the
  // span lies in span unit v / cols at column v % cols, and that unit's
  // pieces are consecutive slots.
  const int span_slot = jb[6] - 1;
  const int span_pieces = span_slot >= 0 ? (int)((uint32_t)jb[7] >> 24) : 0;
  const int sv = (jb[7] & 0xffffff) + col;
  const int sunit = sv / cols;
  const int scol = sv - sunit * cols;
  const int ntot = np + span_pieces;

  float mrun = -INFINITY;
  float lsum = 0.f;
  float o[EPL];
#pragma unroll
  for (int k = 0; k < EPL; ++k) o[k] = 0.f;
  for (int p0 = 0; p0 < ntot; p0 += MCP) {
    const int n = ntot - p0 < MCP ? ntot - p0 : MCP;
    typedef typename PartialVec<T, EPL>::type Raw;
    float2 ml[MCP];
    Raw raw[MCP];
    // Entries past the job load nothing and carry max -inf (weight 0).  No
    // loaded value is used before the barrier, so the round trip's loads all
    // issue before the first wait: the (max, sum) pairs are scalar loads,
    // and a use scheduled between them (a 16-bit row's conversion) waits for
    // every one issued so far.
#pragma unroll
    for (int i = 0; i < MCP; ++i) {
      ml[i] = make_float2(-INFINITY, 0.f);
      raw[i] = Raw{};
      if (i < n) {
        const int p = p0 + i;
        const int64_t r = p < np ? ((int64_t)(slot0 + p) * Hkv + kvh) * cols + c
                                 : ((int64_t)(span_slot + sunit * span_pieces + (p - np)) * Hkv + kvh) * cols + scol;
        ml[i] = *reinterpret_cast<const float2*>(a.part_ml + r * 2);
        if (act) raw[i] = *reinterpret_cast<const Raw*>(static_cast<const T*>(a.part_acc) + r * D + e0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    float pa[MCP][EPL];
#pragma unroll
    for (int i = 0; i < MCP; ++i)
#pragma unroll
      for (int k = 0; k < EPL; ++k) pa[i][k] = partial_f32<T, EPL>(raw[i], k);
    float mc = -INFINITY;
#pragma unroll
    for (int i = 0; i < MCP; ++i) mc = fmaxf(mc, ml[i].x);
    const float mnew = fmaxf(mrun, mc);
    const bool any = mnew != -INFINITY;
    const float sc = (any && mrun != -INFINITY) ? fast_exp2(mrun - mnew) : (any ? 0.f : 1.f);
    lsum *= sc;
#pragma unroll
    for (int k = 0; k < EPL; ++k) o[k] *= sc;
#pragma unroll
    for (int i = 0; i < MCP; ++i) {
      // Entries past the job and empty partials carry max -inf: weight 0.
      const float wt = ml[i].x != -INFINITY ? fast_exp2(ml[i].x - mnew) * ml[i].y : 0.f;
      lsum += wt;
#pragma unroll
      for (int k = 0; k < EPL; ++k) o[k] += wt * pa[i][k];
    }
    mrun = mnew;
  }
  if (!act) return;
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  T* orow = static_cast<T*>(a.out) + (int64_t)(q_start + qi) * a.out_tok_stride + (int64_t)qhead * a.out_head_stride;
#pragma unroll
  for (int k = 0; k < EPL; ++k) orow[e0 + k] = from_f32<T>(o[k] * inv);
}

// ---------------------------------------------------------------------------
// Launch tables: (dtype, head size, column tiles per wave) -> kernel.
// ---------------------------------------------------------------------------
// Head sizes: multiples of 16 from 32 to 256.
static bool head_size_supported(int d) { return d >= 32 && d <= 256 && d % 16 == 0; }
static bool col_tiles_supported(int ctw) { return ctw == 1 || ctw == 4; }

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Four column tiles per wave are built for rows of at most 256 bytes: wider
// rows leave no registers for four accumulator sets.
template <typename T, int D, int CTW>
constexpr bool decode_built = CTW == 1 || (int)sizeof(T) * D <= 256;

template <typename T, int D, int CTW, typename F>
static int with_kernel(F& f) {
  if constexpr (decode_built<T, D, CTW>) {
    return f.template operator()<T, D, CTW>();
  } else {
    return LVAMD_ERR_UNSUPPORTED;
  }
}

// Calls F.template operator()<T, D, CTW>() for the run-time triple; returns
// LVAMD_ERR_UNSUPPORTED for a combination without a kernel.
template <typename T, int CTW, typename F>
static int with_head_size(int head_size, F& f) {
  switch (head_size) {
    case 32: return with_kernel<T, 32, CTW>(f);
    case 48: return with_kernel<T, 48, CTW>(f);
    case 64: return with_kernel<T, 64, CTW>(f);
    case 80: return with_kernel<T, 80, CTW>(f);
    case 96: return with_kernel<T, 96, CTW>(f);
    case 112: return with_kernel<T, 112, CTW>(f);
    case 128: return with_kernel<T, 128, CTW>(f);
    case 144: return with_kernel<T, 144, CTW>(f);
    case 160: return with_kernel<T, 160, CTW>(f);
    case 176: return with_kernel<T, 176, CTW>(f);
    case 192: return with_kernel<T, 192, CTW>(f);
    case 208: return with_kernel<T, 208, CTW>(f);
    case 224: return with_kernel<T, 224, CTW>(f);
    case 240: return with_kernel<T, 240, CTW>(f);
    case 256: return with_kernel<T, 256, CTW>(f);
    default: return LVAMD_ERR_UNSUPPORTED;
  }
}
template <typename F>
static int dispatch_decode(int dtype, int head_size, int col_tiles, F f) {
  if (dtype_size(dtype) == 0 || !head_size_supported(head_size) || !col_tiles_supported(col_tiles))
    return LVAMD_ERR_UNSUPPORTED;
  if (col_tiles == 4) {
    switch (dtype) {
      case LVAMD_BF16: return with_head_size<__bf16, 4>(head_size, f);
      case LVAMD_F16: return with_head_size<_Float16, 4>(head_size, f);
      default: return with_head_size<float, 4>(head_size, f);
    }
  }
  switch (dtype) {
    case LVAMD_BF16: return with_head_size<__bf16, 1>(head_size, f);
    case LVAMD_F16: return with_head_size<_Float16, 1>(head_size, f);
    default: return with_head_size<float, 1>(head_size, f);
  }
}

template <typename T>
static int launch_merge_t(int head_size, dim3 grid, hipStream_t s, const int32_t* jobs, int32_t quads,
                          int32_t num_kv_heads, int32_t group, int32_t col_tiles, const MergeArgs& a) {
  const dim3 block(64 * kMergeWaves);
  switch (head_size) {
    case 32: hipLaunchKernelGGL((paged_merge_kernel<T, 32>), grid, block, 0, s, jobs, quads, num_kv_heads, group, col_tiles, a); break;
    case 48: hipLaunchKernelGGL((paged_merge_kernel<T, 48>), grid, block, 0, s, jobs, quads, num_kv_heads, group, col_tiles, a); break;
    case 64: hipLaunchKernelGGL((paged_merge_kernel<T, 64>), grid, block, 0, s, jobs, quads, num_kv_heads, group, col_tiles, a); break;
    case 80: hipLaunchKernelGGL((paged_merge_kernel<T, 80>), grid, block, 0, s, jobs, quads, num_kv_heads, group, col_tiles, a); break;
    case 96: hipLaunchKernelGGL((paged_merge_kernel<T, 96>), grid, block, 0, s, jobs, quads, num_kv_heads, group, col_tiles, a); break;
    case 112: hipLaunchKernelGGL((paged_merge_kernel<T, 112>), grid, block, 0, s, jobs, quads, num_kv_heads, group, col_tiles, a); break;
    case 128: hipLaunchKernelGGL((paged_merge_kernel<T, 128>), grid, block, 0, s, jobs, quads, num_kv_heads, group, col_tiles, a); break;
    case 144: hipLaunchKernelGGL((paged_merge_kernel<T, 144>), grid, block, 0, s, jobs, quads, num_kv_heads, group, col_tiles, a); break;
    case 160: hipLaunchKernelGGL((paged_merge_kernel<T, 160>), grid, block, 0, s, jobs, quads, num_kv_heads, group, col_tiles, a); break;
    case 176: hipLaunchKernelGGL((paged_merge_kernel<T, 176>), grid, block, 0, s, jobs, quads, num_kv_heads, group, col_tiles, a); break;
    case 192: hipLaunchKernelGGL((paged_merge_kernel<T, 192>), grid, block, 0, s, jobs, quads, num_kv_heads, group, col_tiles, a); break;
    case 208: hipLaunchKernelGGL((paged_merge_kernel<T, 208>), grid, block, 0, s, jobs, quads, num_kv_heads, group, col_tiles, a); break;
    case 224: hipLaunchKernelGGL((paged_merge_kernel<T, 224>), grid, block, 0, s, jobs, quads, num_kv_heads, group, col_tiles, a); break;
    case 240: hipLaunchKernelGGL((paged_merge_kernel<T, 240>), grid, block, 0, s, jobs, quads, num_kv_heads, group, col_tiles, a); break;
    case 256: hipLaunchKernelGGL((paged_merge_kernel<T, 256>), grid, block, 0, s, jobs, quads, num_kv_heads, group, col_tiles, a); break;
    default: return LVAMD_ERR_UNSUPPORTED;
  }
  return launch_status();
}

}  // namespace lvamd

using namespace lvamd;

extern "C" int lvamd_paged_decode(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                  const void* new_key, int64_t new_key_token_stride, int64_t new_key_head_stride,
                                  const void* new_value, int64_t new_value_token_stride,
                                  int64_t new_value_head_stride,
                                  void* key_pool, void* value_pool,
                                  void* out, int64_t out_token_stride, int64_t out_head_stride,
                                  const int32_t* pieces, const int32_t* wave_first, int32_t waves_per_head,
                                  const int32_t* tables, const uint32_t* vis,
                                  void* part_acc, float* part_ml, int64_t num_partial_slots,
                                  int32_t num_kv_heads, int32_t group, int32_t head_size, int32_t col_tiles,
                                  int32_t group_waves, int32_t block_size, float scale, int32_t dtype,
                                  lvamd_stream_t stream) {
  const int es = dtype_size(dtype);
  if (es == 0 || !head_size_supported(head_size) || !col_tiles_supported(col_tiles)) return LVAMD_ERR_UNSUPPORTED;
  if (group_waves != 1 && (col_tiles != 1 || group_waves != lvamd_paged_decode_split_waves(dtype, head_size)))
    return LVAMD_ERR_UNSUPPORTED;
  if (waves_per_head < 0 || num_kv_heads <= 0 || group <= 0 || block_size <= 0 || num_partial_slots < 0 ||
      waves_per_head % group_waves != 0)
    return LVAMD_ERR_INVALID_ARGUMENT;
  if (waves_per_head == 0) return LVAMD_OK;
  if (!q || !key_pool || !value_pool || !out || !pieces || !wave_first || !tables)
    return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_partial_slots > 0 && (!part_acc || !part_ml)) return LVAMD_ERR_WORKSPACE;
  if ((new_key == nullptr) != (new_value == nullptr)) return LVAMD_ERR_INVALID_ARGUMENT;
  // 16-byte row chunks: base pointers and token/head strides must keep rows aligned.
  if (!aligned16(q) || !aligned16(key_pool) || !aligned16(value_pool) ||
      (q_token_stride * es) % 16 != 0 || (q_head_stride * es) % 16 != 0)
    return LVAMD_ERR_INVALID_ARGUMENT;
  if (new_key && (!aligned16(new_key) || !aligned16(new_value) || (new_key_token_stride * es) % 16 != 0 ||
                  (new_key_head_stride * es) % 16 != 0 || (new_value_token_stride * es) % 16 != 0 ||
                  (new_value_head_stride * es) % 16 != 0))
    return LVAMD_ERR_INVALID_ARGUMENT;
  if ((int64_t)waves_per_head * num_kv_heads > 0x7fffffffLL) return LVAMD_ERR_INVALID_ARGUMENT;
  DecodeArgs a;
  a.q = q;
  a.q_tok_stride = q_token_stride;
  a.q_head_stride = q_head_stride;
  a.k_new = new_key;
  a.v_new = new_value;
  a.kn_tok_stride = new_key_token_stride;
  a.kn_head_stride = new_key_head_stride;
  a.vn_tok_stride = new_value_token_stride;
  a.vn_head_stride = new_value_head_stride;
  a.k_pool = key_pool;
  a.v_pool = value_pool;
  a.out = out;
  a.out_tok_stride = out_token_stride;
  a.out_head_stride = out_head_stride;
  a.tables = tables;
  a.vis = vis;
  a.part_acc = part_acc;
  a.part_ml = part_ml;
  a.num_kv_heads = num_kv_heads;
  a.group = group;
  a.block_size = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.scale_log2 = scale * 1.4426950408889634f;
  const dim3 grid((unsigned)(waves_per_head / group_waves * num_kv_heads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dispatch_decode(dtype, head_size, col_tiles, [&]<typename T, int D, int CTW>() -> int {
    if constexpr (CTW == 1) {
      constexpr int WG = split_waves<T, D>();
      if (group_waves == WG) {
        hipLaunchKernelGGL((paged_decode_kernel<T, D, CTW, WG>), grid, dim3(64 * WG), 0, s, wave_first, pieces,
                           waves_per_head, a);
        return launch_status();
      }
    }
    if (group_waves != 1) return LVAMD_ERR_UNSUPPORTED;
    hipLaunchKernelGGL((paged_decode_kernel<T, D, CTW, 1>), grid, dim3(64), 0, s, wave_first, pieces,
                       waves_per_head, a);
    return launch_status();
  });
}

extern "C" int lvamd_paged_decode_split_groups(int32_t dtype, int32_t head_size) {
  return dispatch_decode(dtype, head_size, 1, []<typename T, int D, int CTW>() -> int {
    if constexpr (CTW != 1) {
      return 0;  // (not reached: one column tile asked for)
    } else {
      int device = 0, cus = 0, per_cu = 0;
      if (hipGetDevice(&device) != hipSuccess) return LVAMD_ERR_LAUNCH;
      if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
        return LVAMD_ERR_LAUNCH;
      constexpr int WG = split_waves<T, D>();
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
              &per_cu, reinterpret_cast<const void*>(&paged_decode_kernel<T, D, CTW, WG>), 64 * WG, 0) !=
          hipSuccess)
        return LVAMD_ERR_LAUNCH;
      return per_cu * cus;
    }
  });
}

extern "C" int lvamd_paged_decode_split_waves(int32_t dtype, int32_t head_size) {
  return dispatch_decode(dtype, head_size, 1, []<typename T, int D, int CTW>() -> int {
    return split_waves<T, D>();
  });
}

extern "C" int lvamd_paged_decode_tile_tokens(int32_t dtype, int32_t head_size, int32_t col_tiles) {
  return dispatch_decode(dtype, head_size, col_tiles,
                         []<typename T, int D, int CTW>() -> int { return DecodeTile<T, D, CTW>::TT; });
}

extern "C" int lvamd_paged_decode_resident_waves(int32_t dtype, int32_t head_size, int32_t col_tiles) {
  return dispatch_decode(dtype, head_size, col_tiles, []<typename T, int D, int CTW>() -> int {
    int device = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&device) != hipSuccess) return LVAMD_ERR_LAUNCH;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
      return LVAMD_ERR_LAUNCH;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(&paged_decode_kernel<T, D, CTW, 1>), 64, 0) != hipSuccess)
      return LVAMD_ERR_LAUNCH;
    return per_cu * cus;
  });
}

extern "C" int lvamd_paged_attention_merge(const void* part_acc, const float* part_ml,
                                           void* out, int64_t out_token_stride, int64_t out_head_stride,
                                           const int32_t* jobs, int32_t num_jobs,
                                           int32_t num_kv_heads, int32_t group, int32_t head_size, int32_t col_tiles,
                                           int32_t max_columns, int32_t dtype, lvamd_stream_t stream) {
  if (dtype_size(dtype) == 0 || !head_size_supported(head_size) || col_tiles < 1 || col_tiles > 16)
    return LVAMD_ERR_UNSUPPORTED;
  if (max_columns < 1 || max_columns > 16 * col_tiles) return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_jobs < 0 || num_kv_heads <= 0 || group <= 0) return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_jobs == 0) return LVAMD_OK;
  if (!part_acc || !part_ml || !out || !jobs) return LVAMD_ERR_INVALID_ARGUMENT;
  const int64_t quads = (max_columns + kMergeWaves - 1) / kMergeWaves;
  if ((int64_t)num_jobs * num_kv_heads * quads > 0x7fffffffLL) return LVAMD_ERR_INVALID_ARGUMENT;
  MergeArgs a;
  a.part_acc = part_acc;
  a.part_ml = part_ml;
  a.out = out;
  a.out_tok_stride = out_token_stride;
  a.out_head_stride = out_head_stride;
  // One workgroup per (job, kv head, kMergeWaves columns), over the columns
  // the jobs use; columns past a job's own count exit at once.
  const dim3 grid((unsigned)(num_jobs * num_kv_heads * quads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int32_t q = (int32_t)quads;
  switch (dtype) {
    case LVAMD_BF16: return launch_merge_t<__bf16>(head_size, grid, s, jobs, q, num_kv_heads, group, col_tiles, a);
    case LVAMD_F16: return launch_merge_t<_Float16>(head_size, grid, s, jobs, q, num_kv_heads, group, col_tiles, a);
    default: return launch_merge_t<float>(head_size, grid, s, jobs, q, num_kv_heads, group, col_tiles, a);
  }
}
