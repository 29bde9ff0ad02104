// Chunked-prefill paged attention on gfx950: long query runs (prompt chunks,
// long tree verifications) of bf16/fp16 requests.
//
// Semantics are those of the decode kernel (light-vllm TorchPagedAttention,
// src/light_vllm/runtime/execution/paged_attention.py:323-380): query j of a
// request with c computed tokens sees logical positions [0, c) and
// {c + i : i <= j} (linear) or {c + i : i an ancestor of j, or j} (tree);
// q head h reads kv head h / group; fp32 scores and softmax.
//
// Mapping onto CDNA4:
//   * A work unit is up to 128 MFMA columns of one request, a column being a
//     (query, head-in-group) pair of one kv head, so the GQA group shares
//     every K/V byte.  One workgroup per (unit, kv head): four waves of two
//     16-column tiles, or eight waves of one (the host picks per step).
//   * Keys go in 64-token tiles (32 for D = 256).  Each lane copies one
//     16-byte chunk of one row per load straight from the pool (or this
//     step's K/V) into LDS (global_load_lds_dwordx4: no registers, no LDS
//     store instructions), double-buffered, one barrier per tile: tile t+1
//     lands while tile t computes, tile t+2's table entries are in flight.
//     The LDS layout is unpadded and XOR-swizzled (below) so that the
//     loads, the K reads and the V transpose reads are all free of bank
//     conflicts.
//   * S^T = K Q^T on MFMA 16x16x32: the K A operand is read from LDS once per
//     wave and used for all its column tiles; the accumulator layout (lane l:
//     column l%16, keys 4*(l/16)+r) is the B operand of O^T = V^T P^T, whose
//     V^T A operand comes from LDS by ds_read_b64_tr_b16 transpose reads, also
//     shared by the column tiles.
//   * Online softmax in the log2 domain with lazy rescaling (wave vote), the
//     max across the four 16-lane rows with permlane swaps; the sums come
//     from the matrix cores (a ones row times P^T).
//   * The append is fused: keys of this step's tokens are read from the
//     step's K/V, and the unit that holds a token's own query writes its row
//     to the pool.
//   * A record with zero columns is padding of the planner's per-XCD order.
//   * Split-K: a unit may cover a key range of its request (a piece); a piece
//     that is not the whole range writes partials (its normalised output
//     rows in T, fp32 max and sum) that lvamd_paged_attention_merge combines.  The host splits units when there
//     are fewer units than resident workgroups (tree verification, short
//     chunks), so each workgroup's waves share fewer, wider K/V tiles.

#include <cmath>
#include <type_traits>

#include "lvamd_common.h"

namespace lvamd {

namespace {

constexpr float kRescaleSlack = 8.0f;  // log2 units: probabilities stay below 2^8

}  // namespace

// Keys per LDS tile up to head size 128 (32 above).
constexpr int kPrefillKeyTile = 64;
// Two shapes of the same 128-column unit, chosen per step by the planner:
// * W = 4 waves of two 16-column tiles: each K/V LDS read feeds two MFMAs;
//   up to 256 registers per wave, two waves per SIMD (two workgroups per CU).
// * W = 8 waves of one column tile: half the registers (128), four waves per
//   SIMD to hide the softmax's dependency chain, twice the LDS reads per MFMA.
// W = 8 is faster on split-K and short units (tree verification, chunks
// without history), W = 4 on long unsplit units.  Keys per LDS tile: 64 (32
// for D = 256, which is built for W = 4 only).
constexpr int prefill_col_tiles_per_wave(int d, int w) { return w == 8 ? 1 : 2; }
constexpr bool prefill_built(int d, int w) { return w == 4 || (w == 8 && d <= 128); }
constexpr int prefill_key_tile(int d) { return d <= 128 ? kPrefillKeyTile : 32; }
constexpr int prefill_unit_columns(int d) { return 16 * prefill_col_tiles_per_wave(d, 4) * 4; }
static_assert(16 * 1 * 8 == 16 * 2 * 4, "both shapes cover the same unit columns");

// LDS tile layout.  A K (or V) tile of KT rows is stored as CG column groups
// (64 bytes = four 16-byte chunks of every row), group-major: byte
//   cg * KT * 64 + row * 64 + 16 * (c ^ swz(row))
// holds chunk 4 cg + c of the row.  One direct load of a wave fills 1 KB =
// 16 rows of one group.  swz permutes the four chunk slots of a row by row
// bits, which makes
//   * the K reads (lanes 0-31 read rows 0-15 at two chunks) and
//   * the V transpose reads (lanes 0-31 read 8 rows x 32 bytes)
// cover every bank once, and the loads write contiguous bytes.  Measured on
// MI355X with the LDS bank-conflict counter over lane patterns of known
// conflict degree: ds_read_b128 serves half a wave from a 512-byte bank
// window, so rows r and r + 8 must differ in slot bit 1, and the transpose
// reads need rows r and r + 4 to differ in slot bit 1; slot bit 1 = b2 ^ b3
// gives both.  Slot bit 0 is free for these reads and is chosen per shape by
// wall time (conflict-free choices differ by up to 4% for reasons the
// counters do not show): b2 for four waves, b0 for eight.  The first layout
// (slot = b2 b3 as bits 1, 0) left every K read 2-way conflicted.
// Source and LDS pointers of global_load_lds.
typedef const __attribute__((address_space(1))) void* lds_gptr;
typedef __attribute__((address_space(3))) void* lds_lptr;

template <int W>
__device__ __forceinline__ constexpr int prefill_swz(int row) {
  return ((row >> (W == 4 ? 2 : 0)) & 1) | ((((row >> 2) ^ (row >> 3)) & 1) << 1);
}

template <typename T, int D, int W>
struct PrefillShape {
  static constexpr int KT = prefill_key_tile(D);               // keys per tile
  static constexpr int KS = KT / 16;                           // 16-key groups per tile
  static constexpr int CPR = D * (int)sizeof(T) / 16;          // 16-byte chunks per row
  static constexpr int CG = (CPR + 3) / 4;                     // 64-byte column groups (D = 80: the last half used)
  static constexpr int RB = KT / 16;                           // 16-row blocks per tile
  static constexpr int GROUP_BYTES = KT * 64;                  // one column group of a tile
  static constexpr int TILE_BYTES = CG * GROUP_BYTES;          // a K or V tile
  static constexpr int THREADS = 64 * W;
  static_assert(W % RB == 0, "every wave loads one row block");
  static constexpr int CT = prefill_col_tiles_per_wave(D, W);
  static constexpr int NCH = (D + 31) / 32;                    // 16x16x32 k-steps of QK^T
  static constexpr int NT = D / 16;                            // 16-row tiles of O^T
  static_assert(KT % 32 == 0, "PV steps take 32 keys");
  static_assert(sizeof(T) == 2, "the prefill kernel is built for 16-bit types");
};

struct PrefillArgs {
  const void* q;
  int64_t q_tok_stride, q_head_stride;
  const void* k_new;  // this step's K/V, or null when the pool already holds them
  const void* v_new;
  int64_t kn_tok_stride, kn_head_stride, vn_tok_stride, vn_head_stride;
  void* k_pool;
  void* v_pool;
  void* out;
  int64_t out_tok_stride, out_head_stride;
  const int32_t* __restrict__ tables;
  const uint32_t* __restrict__ vis;
  void* part_acc;                        // [slots][Hkv][unit columns][D] of T, rows normalised
  float* part_ml;                        // [slots][Hkv][unit columns][2]: (max, sum)
  int32_t group;
  int32_t block_size;
  int32_t bs_shift;
  float scale_log2;
};

template <typename T, int D, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(W == 8 ? 4 : (D <= 128 ? 2 : 1)))) void paged_prefill_kernel(
    const int32_t* __restrict__ units,  // [n][LVAMD_PREFILL_FIELDS]
    const int32_t num_kv_heads, const PrefillArgs a) {
  using P = PrefillShape<T, D, W>;
  constexpr int CPR = P::CPR, CG = P::CG, RB = P::RB, CT = P::CT, NCH = P::NCH, NT = P::NT;
  constexpr int KT = P::KT, KS = P::KS, GB = P::GROUP_BYTES;
  using V8 = typename std::conditional<std::is_same<T, __bf16>::value, bf16x8, f16x8>::type;
  // Two K and two V buffers as four objects: the compiler then sees that a
  // load into one buffer does not alias reads of the other.
  __shared__ __attribute__((aligned(1024))) char klds0[P::TILE_BYTES];
  __shared__ __attribute__((aligned(1024))) char klds1[P::TILE_BYTES];
  __shared__ __attribute__((aligned(1024))) char vlds0[P::TILE_BYTES];
  __shared__ __attribute__((aligned(1024))) char vlds1[P::TILE_BYTES];

  constexpr int kThreads = P::THREADS;
  const int tid = threadIdx.x & (kThreads - 1);  // (the mask tells LLVM the thread range)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar registers
  const int lane = tid & 63;
  const int l16 = lane & 15;
  const int g = lane >> 4;
  const int Hkv = num_kv_heads;
  const int G = a.group;
  const int unit = blockIdx.x / Hkv;
  const int kvh = blockIdx.x - unit * Hkv;
  // The unit record carries everything the unit needs, so the first tile's
  // loads depend on one load (the record) only: its request's fields (a span
  // unit, over keys every query of the span sees, reads as a linear request
  // whose computed count is its key_end: no tile masked, nothing appended)
  // and, when the piece's first tile spans at most four blocks, their ids.
  const int32_t* u = units + (int64_t)unit * LVAMD_PREFILL_FIELDS;
  const int col0 = u[1], ncols = u[2], key_begin = u[3], key_end = u[4], slot = u[5];
  const int table_off = u[6], q_start = u[7], computed = u[8], q_len = u[9], vis_off = u[10], vis_words = u[11];
  const int first_blocks[4] = {u[12], u[13], u[14], u[15]};  // -1: take them from the table
  if (ncols <= 0) return;  // a padding record (the host's per-XCD unit order)
  const int col_end = col0 + ncols;  // exclusive: <= q_len * G (a span unit: its packed columns)
  // Keys the unit needs: up to its last query's position, within the piece's
  // key range [key_begin, key_end) (key_begin a multiple of KT; key_end 0 =
  // no bound).  Tiles are numbered from position 0.
  const int kneed = computed + (col_end - 1) / G + 1;
  const int kmax = key_end > 0 && key_end < kneed ? key_end : kneed;
  const int tile0 = key_begin / KT;
  const int ntiles = (kmax + KT - 1) / KT - tile0;  // tiles of this piece
  const int bs = a.block_size;

  const int64_t row_elems = (int64_t)Hkv * D;
  // Global-address-space pointers: the gather picks the pool or the step's
  // input per row, and generic pointers would become flat loads.
  gptr<T> const kbase = (gptr<T>)(a.k_pool);
  gptr<T> const vbase = (gptr<T>)(a.v_pool);
  const int32_t* table = a.tables + table_off;

  // ---- tile loads.  Wave w loads row block w % RB of every tile, column
  // groups w / RB, w / RB + W / RB, ...; lane l the row 16 (w % RB) + l / 4
  // into chunk slot l % 4 of each group (chunk 4 cg + ((l % 4) ^ swz(row))):
  // one table entry and one row address per tile.
  const int lrow = 16 * (wave % RB) + (lane >> 2);
  const int lchunk = (lane & 3) ^ prefill_swz<W>(lrow);
  // Fused append: keys at positions >= computed are this step's tokens, read
  // from the input K/V; the unit that holds a token's own query (its first
  // column) also writes the row to its pool slot, so no other launch appends.
  gptr<const T> const knew = a.k_new ? (gptr<const T>)(a.k_new) + (int64_t)kvh * a.kn_head_stride : nullptr;
  gptr<const T> const vnew = a.v_new ? (gptr<const T>)(a.v_new) + (int64_t)kvh * a.vn_head_stride : nullptr;
  auto key_pos = [&](int t) -> int {
    const int pos = (tile0 + t) * KT + lrow;
    return pos < kmax ? pos : kmax - 1;  // rows past the piece read its last key (masked)
  };
  auto logical_block = [&](int pos) -> int { return a.bs_shift >= 0 ? (pos >> a.bs_shift) : (pos / bs); };
  auto load_entry = [&](int t) -> int { return table[logical_block(key_pos(t))]; };
  // Tile 0's entry from the record (its rows lie in the tile's blocks, the
  // first of which is logical block key_begin / block_size).
  auto first_entry = [&]() -> int {
    if (first_blocks[0] < 0) return load_entry(0);
    const int k = logical_block(key_pos(0)) - logical_block(key_begin);
    return k == 0 ? first_blocks[0] : k == 1 ? first_blocks[1] : k == 2 ? first_blocks[2] : first_blocks[3];
  };
  // Chunk of column group cg this lane copies (D = 80: the half-used last
  // group's spare slots copy the row's last chunk again; nothing reads them).
  auto chunk_of = [&](int cg) -> int {
    const int ch = 4 * cg + lchunk;
    if constexpr (4 * CG > CPR) return ch < CPR ? ch : CPR - 1;
    return ch;
  };
  // Issues tile t's loads into (kdst, vdst); te is the row's table entry.
  auto issue_tile = [&](int t, int te, char* kdst, char* vdst) {
    const int pos = key_pos(t);
    const uint32_t slot = (uint32_t)te * (uint32_t)bs + (uint32_t)(pos - logical_block(pos) * bs);
    const int64_t off = (int64_t)slot * row_elems + kvh * D;
    gptr<const T> kp = kbase + off;
    gptr<const T> vp = vbase + off;
    bool append = false;
    if (knew != nullptr && pos >= computed) {
      const int j = pos - computed;  // query index of the row's token
      kp = knew + (int64_t)(q_start + j) * a.kn_tok_stride;
      vp = vnew + (int64_t)(q_start + j) * a.vn_tok_stride;
      const int raw = (tile0 + t) * KT + lrow;
      append = raw == pos && j * G >= col0;  // (j * G < col_end: pos < kmax <= kneed)
    }
    const int lds_row = (wave % RB) * 1024;
    for (int cg = wave / RB; cg < CG; cg += W / RB) {
      const int ch = chunk_of(cg);
      __builtin_amdgcn_global_load_lds((lds_gptr)(kp + ch * 8), (lds_lptr)(kdst + cg * GB + lds_row), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((lds_gptr)(vp + ch * 8), (lds_lptr)(vdst + cg * GB + lds_row), 16, 0, 0);
      if (append) {
        store16((gptr<T>)(kbase + off + ch * 8), load16(kp + ch * 8));
        store16((gptr<T>)(vbase + off + ch * 8), load16(vp + ch * 8));
      }
    }
  };

  // ---- this wave's columns: (query qi, head) per column tile, and Q^T chunks
  int qi[CT];
  bool colok[CT];
  uint4 qf[CT][NCH];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int col = col0 + 16 * (CT * wave + ct) + l16;
    colok[ct] = col < col_end;
    const int colc = colok[ct] ? col : col_end - 1;
    qi[ct] = colc / G;
    const int qhead = kvh * G + (colc - qi[ct] * G);
    const T* qrow = static_cast<const T*>(a.q) + (int64_t)(q_start + qi[ct]) * a.q_tok_stride +
                    (int64_t)qhead * a.q_head_stride;
#pragma unroll
    for (int kk = 0; kk < NCH; ++kk) {
      const int ch = kk * 4 + g;
      qf[ct][kk] = (colok[ct] && ch < CPR) ? load16(qrow + ch * 8) : zero_u4();
    }
  }
  // Keys this wave's columns can see at most (its last valid query).
  const int wave_col_last = col0 + 16 * CT * (wave + 1) - 1;
  const int wave_kmax = computed + ((wave_col_last < col_end ? wave_col_last : col_end - 1) / G) + 1;
  const bool wave_active = col0 + 16 * CT * wave < col_end;
  // Tiles below this bound are visible to every column of the unit (for a
  // tree request only the computed prefix is).
  const int full_tiles = (vis_off >= 0 ? computed : computed + col0 / G + 1) / KT;
  const bool tree = vis_off >= 0;
  const float c_log2 = a.scale_log2;
  // A tree of at most 32 queries has one ancestor word per query: each
  // column's word is loaded once here instead of per score in the masks.
  const bool tree_word = tree && vis_words == 1;
  uint32_t vrow[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) vrow[ct] = tree_word ? a.vis[vis_off + qi[ct]] : 0u;

  // m_run in the scaled log2 domain.  The softmax denominators come from the
  // matrix cores: l_run += ones(16 x 32) P^T puts each column's sum of its
  // (rounded) probabilities in every row of its accumulator, so the VALU
  // adds no probabilities and the epilogue needs no cross-lane sum.
  float m_run[CT];
  f32x4 l_run[CT];
  f32x4 acc[CT][NT];
  V8 ones;
#pragma unroll
  for (int i = 0; i < 8; ++i) ones[i] = from_f32<T>(1.f);
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    m_run[ct] = -INFINITY;
    l_run[ct] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[ct][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // LDS read offsets of this lane: K row l16 (+16 s), chunk 4 kk + g; V^T
  // transpose reads of row 4 g + l16 / 4 (+32 h, +16), bytes 32 n + 8 q4 of
  // the row (chunk 2 n + q4 / 2: group n / 2, slot 2 (n % 2) + q4 / 2).
  const int q4 = l16 & 3;
  const int k_off = l16 * 64 + 16 * (g ^ prefill_swz<W>(l16));
  const int v_row = 4 * g + (l16 >> 2);
  const int v_off0 = v_row * 64 + 16 * ((q4 >> 1) ^ prefill_swz<W>(v_row)) + 8 * (q4 & 1);
  const int v_off1 = v_row * 64 + 16 * ((2 + (q4 >> 1)) ^ prefill_swz<W>(v_row)) + 8 * (q4 & 1);

  // ---- one tile of attention from LDS (t: tile of the piece)
  auto compute_tile = [&](int tr, const char* kt, const char* vt) {
    const int t = tile0 + tr;
    if (!wave_active || t * KT >= wave_kmax) return;
    // S^T for each column tile, K chunks shared.  Each MFMA block runs at
    // raised wave priority: the SIMD's other wave then does its softmax
    // VALU work while this one feeds the matrix core, and the two phases
    // overlap (measured 7% on a chunked-prefill step in both shapes).
    // iglp_opt(0) asks the scheduler to interleave the block's LDS reads with
    // its MFMAs (a further 4% in the 4-wave shape).
    __builtin_amdgcn_s_setprio(1);
    __builtin_amdgcn_iglp_opt(0);
    f32x4 st[CT][KS];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int s = 0; s < KS; ++s) st[ct][s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s)
#pragma unroll
      for (int kk = 0; kk < NCH; ++kk) {
        const int ch = kk * 4 + g;
        const uint4 kc = ch < CPR ? *reinterpret_cast<const uint4*>(kt + kk * GB + s * 1024 + k_off) : zero_u4();
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) st[ct][s] = Mma<T>::qk(kc, qf[ct][kk], st[ct][s]);
      }
    __builtin_amdgcn_s_setprio(0);
    const bool masked = t >= full_tiles;
    // Masks only past the fully visible prefix: one compare per score for a
    // linear request, the ancestor bits for a tree.  (A piece ends on a tile
    // boundary or at the unit's last key, so no unmasked tile reaches past
    // it; rows past kmax in a masked tile fail the visibility test.)
    if (masked && !tree) {
      // Linear: key pos is visible to query qi iff pos <= computed + qi.
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        const int last = computed + qi[ct] - t * KT - 4 * g;  // last visible pos, tile- and lane-relative
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (16 * s + r > last) st[ct][s][r] = -INFINITY;
      }
    } else if (masked) {
      // Tree: keys before computed are visible, key j = pos - computed < q_len
      // iff bit j of the query's ancestor row.  The tile's keys span at most
      // NW words of the row; each column loads them once per tile, always in
      // bounds (clamped), so the loads carry no condition.
      constexpr int NW = KT / 32 + 1;
      const int j0 = t * KT - computed;  // j of the tile's first key
      const int w0 = j0 >> 5;            // (arithmetic: j0 may be negative)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        uint32_t words[NW];
#pragma unroll
        for (int i = 0; i < NW; ++i) {
          const int w = min(max(w0 + i, 0), vis_words - 1);
          words[i] = tree_word ? vrow[ct] : a.vis[vis_off + qi[ct] * vis_words + w];
        }
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = j0 + 16 * s + 4 * g + r;
            const int wi = (j >> 5) - w0;  // 0 .. NW - 1
            const uint32_t word = wi == 0 ? words[0] : wi == 1 ? words[1] : words[NW - 1];
            const bool vis = j < 0 || (j < q_len && ((word >> (j & 31)) & 1u));
            if (!vis) st[ct][s][r] = -INFINITY;
          }
      }
    }
    // Online softmax on raw scores: max first, scale folded into the exp.
    V8 pb[CT][KS / 2];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      float mt = -INFINITY;
#pragma unroll
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int r = 0; r < 4; ++r) mt = fmaxf(mt, st[ct][s][r]);
      mt = row_max4(mt) * c_log2;
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
      for (int s = 0; s < KS; ++s)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = fast_exp2(__builtin_fmaf(st[ct][s][r], c_log2, nbase));
          pb[ct][s >> 1][(s & 1) * 4 + r] = from_f32<T>(p);
        }
    }
    // O^T += V^T P^T: transpose reads shared by the column tiles.
    __builtin_amdgcn_s_setprio(1);
    __builtin_amdgcn_iglp_opt(0);
#pragma unroll
    for (int h = 0; h < KS / 2; ++h)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        if constexpr (std::is_same<T, __bf16>::value) {
          l_run[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[ct][h], l_run[ct], 0, 0, 0);
        } else {
          l_run[ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pb[ct][h], l_run[ct], 0, 0, 0);
        }
      }
#pragma unroll
    for (int h = 0; h < KS / 2; ++h)
#pragma unroll
      for (int n = 0; n < NT; ++n) {
        const int lo = (n & 1 ? v_off1 : v_off0) + (n >> 1) * GB + h * 32 * 64;
        const int hi = lo + 16 * 64;
        const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vt + lo));
        const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)(vt + hi));
        const s16x4 both[2] = {v0, v1};
        const V8 av = bitcast<V8>(both);
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
          if constexpr (std::is_same<T, __bf16>::value) {
            acc[ct][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, pb[ct][h], acc[ct][n], 0, 0, 0);
          } else {
            acc[ct][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, pb[ct][h], acc[ct][n], 0, 0, 0);
          }
        }
      }
    __builtin_amdgcn_s_setprio(0);
  };

  // ---- pipeline: tile t computes from one buffer pair while tile t+1's
  // loads land in the other and tile t+2's table entries are fetched; then
  // every wave waits for its own loads and the barrier publishes the tile
  // (and frees the buffers just read).  The barrier carries no fence: the
  // vmcnt wait is what orders the direct loads before it.
  auto tile_done = [&]() {
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __builtin_amdgcn_s_barrier();
  };
  int ea = first_entry(), eb = 0;
  issue_tile(0, ea, klds0, vlds0);
  if (ntiles > 1) ea = load_entry(1);
  tile_done();
  // en: tile t+1's entry (in), ef: receives tile t+2's.
  auto step = [&](int t, const char* kc, const char* vc, char* kn, char* vn, const int en, int& ef) {
    // The entry load goes first: a wait for it then never waits for the
    // tile's loads (the vector memory counter retires in issue order).
    if (t + 2 < ntiles) ef = load_entry(t + 2);
    if (t + 1 < ntiles) issue_tile(t + 1, en, kn, vn);
    compute_tile(t, kc, vc);
    tile_done();
  };
  for (int t = 0; t < ntiles; t += 2) {
    step(t, klds0, vlds0, klds1, vlds1, ea, eb);
    if (t + 1 < ntiles) step(t + 1, klds1, vlds1, klds0, vlds0, eb, ea);
  }

  // ---- normalised output rows, or this piece's partials
  if (!wave_active) return;
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const float l_tot = l_run[ct][0];
    if (!colok[ct]) continue;
    if (slot >= 0) {
      constexpr int UC = prefill_unit_columns(D);
      const int64_t cs = ((int64_t)slot * Hkv + kvh) * UC + 16 * (CT * wave + ct) + l16;
      T* pacc = static_cast<T*>(a.part_acc) + cs * D;
      const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
#pragma unroll
      for (int n = 0; n < NT; ++n) store_partial4<true, T>(pacc + 16 * n + 4 * g, acc[ct][n], inv);
      if (g == 0) __builtin_nontemporal_store(f32x2{m_run[ct], l_tot}, reinterpret_cast<f32x2*>(a.part_ml + cs * 2));
      continue;
    }
    const int col = col0 + 16 * (CT * wave + ct) + l16;
    const int qhead = kvh * G + (col - qi[ct] * G);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    T* orow = static_cast<T*>(a.out) + (int64_t)(q_start + qi[ct]) * a.out_tok_stride +
              (int64_t)qhead * a.out_head_stride;
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
      for (int r = 0; r < 4; ++r) orow[16 * n + 4 * g + r] = from_f32<T>(acc[ct][n][r] * inv);
  }
}

template <typename T, int D>
static int launch_prefill_d(int waves, dim3 grid, hipStream_t s, const int32_t* units, int32_t num_kv_heads,
                            const PrefillArgs& a) {
  if (waves == 8) {
    if constexpr (prefill_built(D, 8)) {
      hipLaunchKernelGGL((paged_prefill_kernel<T, D, 8>), grid, dim3(512), 0, s, units, num_kv_heads, a);
      return launch_status();
    }
    return LVAMD_ERR_UNSUPPORTED;
  }
  hipLaunchKernelGGL((paged_prefill_kernel<T, D, 4>), grid, dim3(256), 0, s, units, num_kv_heads, a);
  return launch_status();
}

template <typename T>
static int launch_prefill_t(int head_size, int waves, dim3 grid, hipStream_t s, const int32_t* units,
                            int32_t num_kv_heads, const PrefillArgs& a) {
  switch (head_size) {
    case 32: return launch_prefill_d<T, 32>(waves, grid, s, units, num_kv_heads, a);
    case 48: return launch_prefill_d<T, 48>(waves, grid, s, units, num_kv_heads, a);
    case 64: return launch_prefill_d<T, 64>(waves, grid, s, units, num_kv_heads, a);
    case 80: return launch_prefill_d<T, 80>(waves, grid, s, units, num_kv_heads, a);
    case 96: return launch_prefill_d<T, 96>(waves, grid, s, units, num_kv_heads, a);
    case 112: return launch_prefill_d<T, 112>(waves, grid, s, units, num_kv_heads, a);
    case 128: return launch_prefill_d<T, 128>(waves, grid, s, units, num_kv_heads, a);
    case 144: return launch_prefill_d<T, 144>(waves, grid, s, units, num_kv_heads, a);
    case 160: return launch_prefill_d<T, 160>(waves, grid, s, units, num_kv_heads, a);
    case 176: return launch_prefill_d<T, 176>(waves, grid, s, units, num_kv_heads, a);
    case 192: return launch_prefill_d<T, 192>(waves, grid, s, units, num_kv_heads, a);
    case 208: return launch_prefill_d<T, 208>(waves, grid, s, units, num_kv_heads, a);
    case 224: return launch_prefill_d<T, 224>(waves, grid, s, units, num_kv_heads, a);
    case 240: return launch_prefill_d<T, 240>(waves, grid, s, units, num_kv_heads, a);
    case 256: return launch_prefill_d<T, 256>(waves, grid, s, units, num_kv_heads, a);
    default: return LVAMD_ERR_UNSUPPORTED;
  }
}

template <typename T, int D>
static const void* prefill_fn(int waves) {
  if (waves == 8) {
    if constexpr (prefill_built(D, 8)) return (const void*)&paged_prefill_kernel<T, D, 8>;
    return nullptr;
  }
  return (const void*)&paged_prefill_kernel<T, D, 4>;
}

template <typename T>
static const void* prefill_fn_t(int head_size, int waves) {
  switch (head_size) {
    case 32: return prefill_fn<T, 32>(waves);
    case 48: return prefill_fn<T, 48>(waves);
    case 64: return prefill_fn<T, 64>(waves);
    case 80: return prefill_fn<T, 80>(waves);
    case 96: return prefill_fn<T, 96>(waves);
    case 112: return prefill_fn<T, 112>(waves);
    case 128: return prefill_fn<T, 128>(waves);
    case 144: return prefill_fn<T, 144>(waves);
    case 160: return prefill_fn<T, 160>(waves);
    case 176: return prefill_fn<T, 176>(waves);
    case 192: return prefill_fn<T, 192>(waves);
    case 208: return prefill_fn<T, 208>(waves);
    case 224: return prefill_fn<T, 224>(waves);
    case 240: return prefill_fn<T, 240>(waves);
    case 256: return prefill_fn<T, 256>(waves);
    default: return nullptr;
  }
}

// 16-bit pools, head sizes that are multiples of 16 from 32 to 256.
static bool prefill_supported(int dtype, int head_size) {
  return (dtype == LVAMD_BF16 || dtype == LVAMD_F16) && head_size >= 32 && head_size <= 256 && head_size % 16 == 0;
}

}  // namespace lvamd

using namespace lvamd;

extern "C" int lvamd_paged_prefill_unit_columns(int32_t dtype, int32_t head_size) {
  if (!prefill_supported(dtype, head_size)) return 0;
  return prefill_unit_columns(head_size);
}

extern "C" int lvamd_paged_prefill_key_tokens(int32_t dtype, int32_t head_size) {
  if (!prefill_supported(dtype, head_size)) return LVAMD_ERR_UNSUPPORTED;
  return prefill_key_tile(head_size);
}

extern "C" int lvamd_paged_prefill_resident_units(int32_t dtype, int32_t head_size, int32_t waves) {
  if (!prefill_supported(dtype, head_size)) return LVAMD_ERR_UNSUPPORTED;
  if (waves != 4 && waves != 8) return LVAMD_ERR_INVALID_ARGUMENT;
  const void* fn = dtype == LVAMD_BF16 ? prefill_fn_t<__bf16>(head_size, waves) : prefill_fn_t<_Float16>(head_size, waves);
  if (fn == nullptr) return LVAMD_ERR_UNSUPPORTED;
  int device = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&device) != hipSuccess) return LVAMD_ERR_LAUNCH;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return LVAMD_ERR_LAUNCH;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 64 * waves, 0) != hipSuccess) return LVAMD_ERR_LAUNCH;
  return per_cu * cus;
}

extern "C" int lvamd_paged_prefill_waves_built(int32_t dtype, int32_t head_size, int32_t waves) {
  if (!prefill_supported(dtype, head_size)) return 0;
  return (waves == 4 || (waves == 8 && head_size <= 128)) ? 1 : 0;
}

extern "C" int lvamd_paged_prefill(const void* q, int64_t q_token_stride, int64_t q_head_stride,
                                   const void* new_key, int64_t new_key_token_stride, int64_t new_key_head_stride,
                                   const void* new_value, int64_t new_value_token_stride,
                                   int64_t new_value_head_stride, void* key_pool, void* value_pool,
                                   void* out, int64_t out_token_stride, int64_t out_head_stride,
                                   const int32_t* tables, const uint32_t* vis,
                                   const int32_t* units, int32_t num_units,
                                   void* part_acc, float* part_ml, int64_t num_partial_slots,
                                   int32_t num_kv_heads, int32_t group, int32_t head_size, int32_t waves,
                                   int32_t block_size, float scale, int32_t dtype, lvamd_stream_t stream) {
  if (num_units < 0 || num_kv_heads <= 0 || group <= 0 || block_size <= 0 || num_partial_slots < 0)
    return LVAMD_ERR_INVALID_ARGUMENT;
  if (waves != 4 && waves != 8) return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_units == 0) return LVAMD_OK;
  if (!prefill_supported(dtype, head_size)) return LVAMD_ERR_UNSUPPORTED;
  if (!q || !key_pool || !value_pool || !out || !tables || !vis || !units)
    return LVAMD_ERR_INVALID_ARGUMENT;
  if (num_partial_slots > 0 && (!part_acc || !part_ml)) return LVAMD_ERR_WORKSPACE;
  const int es = dtype_size(dtype);
  if (((uintptr_t)q & 15u) || ((uintptr_t)key_pool & 15u) || ((uintptr_t)value_pool & 15u) ||
      (q_token_stride * es) % 16 != 0 || (q_head_stride * es) % 16 != 0)
    return LVAMD_ERR_INVALID_ARGUMENT;
  if ((int64_t)num_units * num_kv_heads > 0x7fffffffLL) return LVAMD_ERR_INVALID_ARGUMENT;
  if ((new_key == nullptr) != (new_value == nullptr)) return LVAMD_ERR_INVALID_ARGUMENT;
  if (new_key && (((uintptr_t)new_key & 15u) || ((uintptr_t)new_value & 15u) ||
                  (new_key_token_stride * es) % 16 != 0 || (new_key_head_stride * es) % 16 != 0 ||
                  (new_value_token_stride * es) % 16 != 0 || (new_value_head_stride * es) % 16 != 0))
    return LVAMD_ERR_INVALID_ARGUMENT;
  PrefillArgs a;
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
  a.group = group;
  a.block_size = block_size;
  a.bs_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  a.scale_log2 = scale * 1.4426950408889634f;
  const dim3 grid((unsigned)(num_units * num_kv_heads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  return dtype == LVAMD_BF16 ? launch_prefill_t<__bf16>(head_size, waves, grid, s, units, num_kv_heads, a)
                             : launch_prefill_t<_Float16>(head_size, waves, grid, s, units, num_kv_heads, a);
}
