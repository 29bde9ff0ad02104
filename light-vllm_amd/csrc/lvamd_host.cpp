// lvamd_host.cpp — native host side of the paged-KV backend (CPython
// extension module _lvamd_host, built with g++ against the interpreter's
// headers; no numpy or torch headers).
//
// One model step of light-vllm hands the backend Python tuples: a block
// table per request, computed-token counts, query layouts.  Everything the
// gfx950 kernels need is derived from them here, in single passes over the
// Python objects, into flat int32/int64 arrays the caller stages to the GPU:
//
//   flatten     block tables -> flat int32 ids + per-request counts (or any
//               int sequences -> int64), with the metadata constructor's
//               "non-negative int" rule
//               (src/light_vllm/runtime/execution/paged_attention.py:51-62);
//   validate    the block-table rules of validate_block_tables
//               (paged_attention.py:138-172), reporting the rule that fires
//               first in the reference's order, and the request;
//   layouts     query lengths and uint32 ancestor bit rows of tree layouts
//               (query_visibility, src/light_vllm/runtime/execution/layout.py:44-55);
//   metadata    the metadata constructor's field rules and defaults
//               (paged_attention.py:29-62) plus flatten and layouts, in one call;
//   stage       slots (slot_mapping, paged_attention.py:110-136) and the
//               per-request records, written straight into a staging buffer;
//   decode_work / prefill_work / layer_work
//               the stream-K split of decode rows and the prefill units, and
//               (layer_work) the per-step kernel choices of a layer shape;
//   plan_step   validate + stage + layer_work for every layer shape, written
//               into one pinned staging buffer (the backend's per-step call);
//   compact_pairs
//               the rules and slots of PagedKVCache.compact
//               (src/light_vllm/runtime/execution/paged_cache.py:257-314) for
//               many requests in one call.
//
// Every function returns status codes; the Python layer turns them into the
// host's exception classes and messages.  Functions run with the GIL held
// and keep per-process scratch (epoch-stamped owner arrays) between calls.

#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <algorithm>
#include <climits>
#include <cstdint>
#include <cstring>
#include <functional>
#include <limits>
#include <numeric>
#include <unordered_map>
#include <vector>

namespace {

// Fields per record, equal to the LVAMD_* constants of include/lvamd_paged_kv.h.
constexpr int kReqFields = 8;
constexpr int kPieceFields = 16;
constexpr int kMergeFields = 8;
constexpr int kPrefillFields = 16;
// Field 0 of a padding record of the prefill grid (its column count, field
// 2, is zero: the kernel does nothing for it).
constexpr int32_t kPadRecord = INT32_MAX;
constexpr int kPieceBlocks = 5;  // first-tile block ids in piece fields 11..15
constexpr int kTableSlice = 256;  // decode kernel's LDS copy of a piece's table slice

// A contiguous buffer argument (numpy array, bytearray, memoryview).
class Buf {
 public:
  Buf(PyObject* obj, bool writable, Py_ssize_t itemsize, const char* what) {
    const int flags = PyBUF_C_CONTIGUOUS | (writable ? PyBUF_WRITABLE : 0);
    if (PyObject_GetBuffer(obj, &view_, flags) != 0) return;
    held_ = true;
    if (view_.itemsize != itemsize && !(view_.itemsize == 1 && view_.len % itemsize == 0)) {
      PyErr_Format(PyExc_TypeError, "%s: expected %zd-byte items", what, itemsize);
      return;
    }
    ok_ = true;
    count_ = view_.len / itemsize;
  }
  ~Buf() {
    if (held_) PyBuffer_Release(&view_);
  }
  Buf(const Buf&) = delete;
  Buf& operator=(const Buf&) = delete;
  bool ok() const { return ok_; }
  Py_ssize_t count() const { return count_; }
  template <typename T>
  T* data() const {
    return static_cast<T*>(view_.buf);
  }

 private:
  Py_buffer view_{};
  bool held_ = false;
  bool ok_ = false;
  Py_ssize_t count_ = 0;
};

// A bytearray of n items of T, zero-filled when asked.
template <typename T>
PyObject* new_array(Py_ssize_t n, T** out, bool zero = false) {
  PyObject* arr = PyByteArray_FromStringAndSize(nullptr, n * (Py_ssize_t)sizeof(T));
  if (arr == nullptr) return nullptr;
  *out = reinterpret_cast<T*>(PyByteArray_AS_STRING(arr));
  if (zero && n) std::memset(*out, 0, (size_t)n * sizeof(T));
  return arr;
}

bool want_args(Py_ssize_t got, Py_ssize_t want, const char* name) {
  if (got == want) return true;
  PyErr_Format(PyExc_TypeError, "%s takes %zd arguments (%zd given)", name, want, got);
  return false;
}

bool as_i64(PyObject* o, int64_t* v) {
  *v = PyLong_AsLongLong(o);
  return !(*v == -1 && PyErr_Occurred());
}

// Counts of how calls were served: incremental table proofs, full table
// checks, and block ids taken from the previous flatten without reading
// their int objects (against ids read).
struct PlannerCounts {
  long long incremental_proofs = 0, full_checks = 0, reused_ids = 0, read_ids = 0;
};
PlannerCounts g_counts;

// ---------------------------------------------------------------------------
// flatten(sequences, wide) -> (flat bytearray, counts int64 bytearray, status)
// The concatenation of a sequence of int sequences (block tables, or one
// sequence of per-request counts), as int32 (wide 0) or int64 (wide 1).
// status 0: ok; 1: an item is not an exact int (bool and numpy integers are
// not) or is negative.  Values past the item type are clamped to its
// maximum (the range rules then reject them).
// ---------------------------------------------------------------------------
template <typename T>
int flatten_into(const std::vector<PyObject*>& rows, T* flat, int64_t* counts) {
  int status = 0;
  const long long vmax = std::numeric_limits<T>::max();
  Py_ssize_t k = 0;
  for (size_t r = 0; r < rows.size(); ++r) {
    const Py_ssize_t n = PySequence_Fast_GET_SIZE(rows[r]);
    PyObject** items = PySequence_Fast_ITEMS(rows[r]);
    counts[r] = n;
    for (Py_ssize_t i = 0; i < n; ++i, ++k) {
      PyObject* o = items[i];
      T v = 0;
      if (!PyLong_CheckExact(o)) {
        status = 1;
      } else {
        int overflow = 0;
        const long long x = PyLong_AsLongLongAndOverflow(o, &overflow);
        if (overflow < 0 || (overflow == 0 && x < 0)) {
          status = 1;
        } else {
          v = (overflow > 0 || x > vmax) ? (T)vmax : (T)x;
        }
      }
      flat[k] = v;
    }
  }
  return status;
}

// The block tables of the previous int32 flatten.  Only tuple rows are kept,
// with a reference each: a tuple cannot change and keeps its items alive, so
// an item pointer equal to the previous row's is the same int object, of
// the same value.  light-vllm builds every step's tables as
// ``tuple(allocation.block_ids)`` over the same int objects, so a decode
// step's rows repeat the previous step's items and add at most a block.
struct PrevFlatten {
  std::vector<PyObject*> rows;  // owned references (tuples), or nullptr
  std::vector<int64_t> offsets;
  std::vector<int32_t> values;
  // Set when the table check passed on exactly these tables (for a pool of
  // proven_blocks blocks): every id of every row is then in range and
  // appears once in its row, which compact_pairs relies on for a row it
  // receives as the same tuple object.
  int64_t proven_blocks = -1;

  void reset() {
    for (PyObject* row : rows) Py_XDECREF(row);
    rows.clear();
    offsets.clear();
    values.clear();
    proven_blocks = -1;
  }

  // Marks the rows proven when the checked tables (ids, cnt) are these.
  void note_proven(const int32_t* ids, const int64_t* cnt, int64_t batch, int64_t num_blocks) {
    proven_blocks = -1;
    if ((int64_t)rows.size() != batch) return;
    int64_t total = 0;
    for (int64_t r = 0; r < batch; ++r) {
      if (offsets[(size_t)r] != total) return;
      total += cnt[r];
    }
    if (total != (int64_t)values.size() || std::memcmp(ids, values.data(), (size_t)total * sizeof(int32_t)) != 0)
      return;
    proven_blocks = num_blocks;
  }
};
PrevFlatten g_prev_flatten;

// flatten_into for block tables, reusing the values of the leading items a
// row shares (by identity) with the same row of the previous call.
int flatten_tables_into(const std::vector<PyObject*>& rows, int32_t* flat, int64_t* counts) {
  PrevFlatten& prev = g_prev_flatten;
  int status = 0;
  Py_ssize_t k = 0;
  for (size_t r = 0; r < rows.size(); ++r) {
    PyObject* row = rows[r];
    const Py_ssize_t n = PySequence_Fast_GET_SIZE(row);
    PyObject** items = PySequence_Fast_ITEMS(row);
    counts[r] = n;
    Py_ssize_t same = 0;
    if (r < prev.rows.size() && prev.rows[r] != nullptr && PyTuple_CheckExact(row)) {
      PyObject** old = PySequence_Fast_ITEMS(prev.rows[r]);
      const Py_ssize_t limit = std::min(n, PyTuple_GET_SIZE(prev.rows[r]));
      if (std::memcmp(items, old, (size_t)limit * sizeof(PyObject*)) == 0) {
        same = limit;  // the usual decode step: the whole old row, maybe a block more
      } else {
        while (same < limit && items[same] == old[same]) ++same;
      }
      if (same) std::memcpy(flat + k, prev.values.data() + prev.offsets[r], (size_t)same * sizeof(int32_t));
    }
    g_counts.reused_ids += same;
    g_counts.read_ids += n - same;
    for (Py_ssize_t i = same; i < n; ++i) {
      PyObject* o = items[i];
      int32_t v = 0;
      if (!PyLong_CheckExact(o)) {
        status = 1;
      } else {
        int overflow = 0;
        const long long x = PyLong_AsLongLongAndOverflow(o, &overflow);
        if (overflow < 0 || (overflow == 0 && x < 0)) {
          status = 1;
        } else {
          v = (overflow > 0 || x > INT32_MAX) ? INT32_MAX : (int32_t)x;
        }
      }
      flat[k + i] = v;
    }
    k += n;
  }
  // Keep this call's tuple rows for the next one (only a fully valid call).
  prev.reset();
  if (status == 0) {
    prev.rows.resize(rows.size(), nullptr);
    prev.offsets.resize(rows.size(), 0);
    prev.values.assign(flat, flat + k);
    for (size_t r = 0, off = 0; r < rows.size(); ++r) {
      prev.offsets[r] = (int64_t)off;
      off += (size_t)PySequence_Fast_GET_SIZE(rows[r]);
      if (PyTuple_CheckExact(rows[r])) {
        Py_INCREF(rows[r]);
        prev.rows[r] = rows[r];
      }
    }
  }
  return status;
}

PyObject* flatten(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!want_args(nargs, 2, "flatten")) return nullptr;
  const int wide = PyObject_IsTrue(args[1]);
  if (wide < 0) return nullptr;
  PyObject* outer = PySequence_Fast(args[0], "block tables must be a sequence");
  if (outer == nullptr) return nullptr;
  const Py_ssize_t batch = PySequence_Fast_GET_SIZE(outer);
  std::vector<PyObject*> rows((size_t)batch, nullptr);
  Py_ssize_t total = 0;
  PyObject* result = nullptr;
  PyObject* flat_obj = nullptr;
  PyObject* counts_obj = nullptr;
  int64_t* counts = nullptr;
  int status = 0;
  for (Py_ssize_t r = 0; r < batch; ++r) {
    rows[r] = PySequence_Fast(PySequence_Fast_GET_ITEM(outer, r), "a block table must be a sequence");
    if (rows[r] == nullptr) goto done;
    total += PySequence_Fast_GET_SIZE(rows[r]);
  }
  counts_obj = new_array<int64_t>(batch, &counts);
  if (counts_obj == nullptr) goto done;
  if (wide) {
    int64_t* flat = nullptr;
    flat_obj = new_array<int64_t>(total, &flat);
    if (flat_obj == nullptr) goto done;
    status = flatten_into<int64_t>(rows, flat, counts);
  } else {
    int32_t* flat = nullptr;
    flat_obj = new_array<int32_t>(total, &flat);
    if (flat_obj == nullptr) goto done;
    status = flatten_tables_into(rows, flat, counts);
  }
  result = Py_BuildValue("(OOi)", flat_obj, counts_obj, status);
done:
  Py_XDECREF(flat_obj);
  Py_XDECREF(counts_obj);
  for (PyObject* row : rows) Py_XDECREF(row);
  Py_DECREF(outer);
  return result;
}

// ---------------------------------------------------------------------------
// Per-block scratch, one 16-byte record per physical block, valid when its
// epoch equals the current call's: the request that last listed the block,
// and that request's logical index of it with its readonly bit.  Epochs
// avoid clearing the array per call; a wrap clears it once.
// ---------------------------------------------------------------------------
struct BlockRecord {
  uint32_t epoch;
  int32_t request;
  uint32_t owner;  // logical index << 1 | readonly
  uint32_t pad;
};

struct BlockScratch {
  std::vector<BlockRecord> rec;
  uint32_t epoch = 0;

  void reserve(int64_t num_blocks) {
    if ((int64_t)rec.size() < num_blocks) {
      rec.assign((size_t)num_blocks, BlockRecord{0u, -1, 0u, 0u});
      epoch = 0;
    }
  }
  uint32_t next_epoch() {
    if (++epoch == 0) {
      std::fill(rec.begin(), rec.end(), BlockRecord{0u, -1, 0u, 0u});
      epoch = 1;
    }
    return epoch;
  }
};
BlockScratch g_scratch;          // validate's block owners
BlockScratch g_compact_scratch;  // compact_pairs' per-table repeat check

// Rule codes of validate, in the order the reference checks them per request.
enum TableRule {
  kTablesOk = 0,
  kTableShort = 1,      // "block table does not cover all scheduled tokens"
  kTableLong = 2,       // "block table contains unused physical blocks"
  kTableRange = 3,      // "block table contains an out-of-range physical block"
  kTableReadonly = 4,   // "readonly prefix blocks exceed the computed prefix"
  kTableAliasOne = 5,   // "block table aliases a physical block within one request"
  kTableAliasMany = 6,  // "block tables alias a physical block across requests"
};

// The tables of the last call of validate that passed, with the epoch whose
// block records they own.
struct PrevTables {
  std::vector<int32_t> flat;
  std::vector<int64_t> counts, readonly;
  int64_t num_blocks = -1, block_size = -1;
  uint32_t epoch = 0;
  bool valid = false;

  void save(const int32_t* ids, const int64_t* cnt, const int64_t* ro, int64_t batch, int64_t nb, int64_t bs,
            uint32_t ep) {
    int64_t total = 0;
    for (int64_t r = 0; r < batch; ++r) total += cnt[r];
    flat.assign(ids, ids + total);
    counts.assign(cnt, cnt + batch);
    readonly.assign(ro, ro + batch);
    num_blocks = nb;
    block_size = bs;
    epoch = ep;
    valid = true;
  }
};
PrevTables g_prev_tables;

// The incremental proof of a decode step: every table of the last passing
// call is a prefix of the same request's table now (same batch, same
// readonly counts), and the block records of that call are still current.
// Then the old blocks keep their proof; coverage and the readonly bound are
// re-checked per request, and each appended block is checked for range and
// for being listed nowhere else (an appended block lies past the readonly
// prefix, so any other listing breaks a rule).  Returns true when the step
// is proven; false sends it to the full check, which also names the first
// broken rule.
bool validate_appended(const int32_t* ids, const int64_t* cnt, const int64_t* comp, const int64_t* res,
                       const int64_t* ro, int64_t batch, int64_t num_blocks, int64_t bs) {
  PrevTables& prev = g_prev_tables;
  BlockScratch& s = g_scratch;
  if (!prev.valid || prev.num_blocks != num_blocks || prev.block_size != bs || prev.epoch != s.epoch ||
      (int64_t)prev.counts.size() != batch)
    return false;
  for (int64_t r = 0, off = 0, old_off = 0; r < batch; off += cnt[r], old_off += prev.counts[r], ++r) {
    const int64_t n = cnt[r], old_n = prev.counts[r];
    if (n < old_n || ro[r] != prev.readonly[r]) return false;
    if (n != (comp[r] + res[r] + bs - 1) / bs || ro[r] > n || ro[r] * bs > comp[r]) return false;
    if (std::memcmp(ids + off, prev.flat.data() + old_off, (size_t)old_n * sizeof(int32_t)) != 0) return false;
  }
  // Appended blocks: stamped into the current epoch's records as they pass,
  // so one appended twice is caught too.  A failure leaves stamps behind; the
  // full check starts a new epoch, which voids them.
  BlockRecord* rec = s.rec.data();
  for (int64_t r = 0, off = 0; r < batch; off += cnt[r], ++r) {
    for (int64_t i = prev.counts[r]; i < cnt[r]; ++i) {
      const int32_t b = ids[off + i];
      if ((uint32_t)b >= (uint32_t)num_blocks || rec[b].epoch == s.epoch) return false;
      rec[b].epoch = s.epoch;
      rec[b].request = (int32_t)r;
      rec[b].owner = ((uint32_t)i << 1) | (uint32_t)(i < ro[r]);
    }
  }
  prev.save(ids, cnt, ro, batch, num_blocks, bs, s.epoch);
  g_prev_flatten.note_proven(ids, cnt, batch, num_blocks);
  ++g_counts.incremental_proofs;
  return true;
}

// counts() -> (incremental table proofs, full table checks, reused ids, read ids)
PyObject* counts(PyObject*, PyObject* const*, Py_ssize_t nargs) {
  if (!want_args(nargs, 0, "counts")) return nullptr;
  const PlannerCounts& c = g_counts;
  return Py_BuildValue("(LLLL)", c.incremental_proofs, c.full_checks, c.reused_ids, c.read_ids);
}

int check_tables(const int32_t* ids, const int64_t* cnt, const int64_t* comp, const int64_t* res, const int64_t* ro,
                 int64_t batch, int64_t num_blocks, int64_t bs, int64_t* bad);

// validate(flat i32, counts i64, computed i64, reserved i64, readonly i64,
//          num_blocks, block_size) -> (rule, request)
//
// A decode step that only appends blocks to the last proven tables takes the
// incremental proof (validate_appended); any other step, and any step it
// cannot prove, takes the full check below.
//
// Per request, in order: coverage, range and readonly are checked first
// (cheap, sequential); then one pass over the table visits each block's
// record once, noting a repeat inside the table (this request already
// listed the block) and a bad share (another request listed it at another
// logical index, or one side is not readonly).  A repeat is reported before
// a bad share of the same request, as the reference checks the whole table
// for repeats before it looks at sharing.
PyObject* validate(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!want_args(nargs, 7, "validate")) return nullptr;
  Buf flat(args[0], false, 4, "flat"), counts(args[1], false, 8, "counts"), computed(args[2], false, 8, "computed"),
      reserved(args[3], false, 8, "reserved"), readonly(args[4], false, 8, "readonly");
  if (!flat.ok() || !counts.ok() || !computed.ok() || !reserved.ok() || !readonly.ok()) return nullptr;
  int64_t num_blocks = 0, bs = 0;
  if (!as_i64(args[5], &num_blocks) || !as_i64(args[6], &bs)) return nullptr;
  const Py_ssize_t batch = counts.count();
  if (computed.count() != batch || reserved.count() != batch || readonly.count() != batch || bs <= 0 ||
      num_blocks <= 0 || num_blocks > INT32_MAX) {
    PyErr_SetString(PyExc_ValueError, "validate: inconsistent arguments");
    return nullptr;
  }
  const int32_t* ids = flat.data<int32_t>();
  const int64_t* cnt = counts.data<int64_t>();
  const int64_t* comp = computed.data<int64_t>();
  const int64_t* res = reserved.data<int64_t>();
  const int64_t* ro = readonly.data<int64_t>();
  int64_t total = 0;
  for (Py_ssize_t r = 0; r < batch; ++r) total += cnt[r];
  if (total != flat.count()) {
    PyErr_SetString(PyExc_ValueError, "validate: counts do not match the flat table");
    return nullptr;
  }
  int64_t bad = -1;
  const int rule = check_tables(ids, cnt, comp, res, ro, batch, num_blocks, bs, &bad);
  return Py_BuildValue("(in)", rule, (Py_ssize_t)bad);
}

// The rule check behind validate (arguments already consistent): the
// incremental proof when it applies, else the full check.  Returns the
// first broken rule (kTablesOk if none) and sets *bad to its request.
int check_tables(const int32_t* ids, const int64_t* cnt, const int64_t* comp, const int64_t* res, const int64_t* ro,
                 int64_t batch, int64_t num_blocks, int64_t bs, int64_t* bad) {
  BlockScratch& s = g_scratch;
  s.reserve(num_blocks);
  *bad = -1;
  if (validate_appended(ids, cnt, comp, res, ro, batch, num_blocks, bs)) return kTablesOk;
  ++g_counts.full_checks;
  const uint32_t epoch = s.next_epoch();
  BlockRecord* rec = s.rec.data();
  int rule = kTablesOk;
  int64_t r = 0;
  for (int64_t off = 0; r < batch; off += cnt[r], ++r) {
    const int64_t n = cnt[r];
    const int64_t required = (comp[r] + res[r] + bs - 1) / bs;
    if (n < required) { rule = kTableShort; break; }
    if (n > required) { rule = kTableLong; break; }
    const int32_t* t = ids + off;
    bool in_range = true;
    for (int64_t i = 0; i < n; ++i) in_range &= (uint32_t)t[i] < (uint32_t)num_blocks;
    if (!in_range) { rule = kTableRange; break; }
    if (ro[r] > n || ro[r] * bs > comp[r]) { rule = kTableReadonly; break; }
    bool repeat = false, bad_share = false;
    for (int64_t i = 0; i < n; ++i) {
      BlockRecord& b = rec[t[i]];
      const uint32_t mine = ((uint32_t)i << 1) | (uint32_t)(i < ro[r]);
      if (b.epoch == epoch) {
        if (b.request == (int32_t)r) {
          repeat = true;
        } else {
          bad_share |= !((b.owner >> 1) == (uint32_t)i && (b.owner & 1u) && (mine & 1u));
        }
      }
      b.epoch = epoch;
      b.request = (int32_t)r;
      b.owner = mine;
    }
    if (repeat) { rule = kTableAliasOne; break; }
    if (bad_share) { rule = kTableAliasMany; break; }
  }
  if (rule == kTablesOk) {
    g_prev_tables.save(ids, cnt, ro, batch, num_blocks, bs, epoch);
    g_prev_flatten.note_proven(ids, cnt, batch, num_blocks);
  } else {
    g_prev_tables.valid = false;
    g_prev_flatten.proven_blocks = -1;
    *bad = r;
  }
  return rule;
}

// ---------------------------------------------------------------------------
// layouts(query_layouts) -> (q_lens i64, vis_off i64, vis_words i64, vis u32, status)
// A layout is anything with a ``parent_indices`` sequence of exact ints.
// Linear layouts (parent i - 1 for every i) get vis_off -1; the others one
// uint32 row per query: bit j of word w of row q set iff query 32w + j is q
// or an ancestor of q.  status 1: a parent is not an int in [-1, index).
// ---------------------------------------------------------------------------
PyObject* g_parent_indices = nullptr;  // interned "parent_indices"
// Interned keys of a compact request: block_ids, num_computed_tokens,
// num_query_tokens, num_reserved_query_tokens, num_readonly_prefix_blocks,
// retained_query_indices.
PyObject* g_compact_keys[6] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};

// layouts' body over ``batch`` layout objects: fills the per-request arrays
// and appends the ancestor rows to ``vis``.  Returns the status, or -1 with
// a Python error set (no parent_indices, not a sequence).
int parse_layouts(PyObject* const* layouts, Py_ssize_t batch, int64_t* qlen, int64_t* voff, int64_t* vwords,
                  std::vector<uint32_t>& vis) {
  static std::vector<int32_t> parents;
  int status = 0;
  for (Py_ssize_t r = 0; r < batch; ++r) {
    PyObject* attr = PyObject_GetAttr(layouts[r], g_parent_indices);
    if (attr == nullptr) return -1;
    PyObject* seq = PySequence_Fast(attr, "parent_indices must be a sequence");
    Py_DECREF(attr);
    if (seq == nullptr) return -1;
    const Py_ssize_t q = PySequence_Fast_GET_SIZE(seq);
    PyObject** items = PySequence_Fast_ITEMS(seq);
    parents.resize((size_t)q);
    bool linear = true;
    for (Py_ssize_t i = 0; i < q; ++i) {
      long v = PyLong_CheckExact(items[i]) ? PyLong_AsLong(items[i]) : LONG_MIN;
      if (v == -1 && PyErr_Occurred()) {
        PyErr_Clear();
        v = LONG_MIN;
      }
      if (v < -1 || v >= i) status = 1;
      parents[(size_t)i] = (int32_t)std::max<long>(-1, std::min<long>(v, i - 1));
      linear &= parents[(size_t)i] == i - 1;
    }
    Py_DECREF(seq);
    qlen[r] = q;
    if (linear) {
      voff[r] = -1;
      vwords[r] = 0;
      continue;
    }
    const int64_t words = (q + 31) / 32;
    voff[r] = (int64_t)vis.size();
    vwords[r] = words;
    vis.resize(vis.size() + (size_t)(q * words), 0u);
    uint32_t* rows = vis.data() + voff[r];
    for (Py_ssize_t i = 0; i < q; ++i) {
      uint32_t* row = rows + i * words;
      // Ancestors precede their children: row i = row of its parent + bit i.
      const int32_t p = parents[(size_t)i];
      if (p >= 0) std::memcpy(row, rows + p * words, (size_t)words * 4);
      row[i >> 5] |= 1u << (i & 31);
    }
  }
  return status;
}

PyObject* layouts(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!want_args(nargs, 1, "layouts")) return nullptr;
  PyObject* outer = PySequence_Fast(args[0], "query layouts must be a sequence");
  if (outer == nullptr) return nullptr;
  const Py_ssize_t batch = PySequence_Fast_GET_SIZE(outer);
  int64_t *qlen = nullptr, *voff = nullptr, *vwords = nullptr;
  PyObject* qlen_obj = new_array<int64_t>(batch, &qlen);
  PyObject* voff_obj = new_array<int64_t>(batch, &voff);
  PyObject* vwords_obj = new_array<int64_t>(batch, &vwords);
  std::vector<uint32_t> vis;
  PyObject* result = nullptr;
  int status = 0;
  if (qlen_obj == nullptr || voff_obj == nullptr || vwords_obj == nullptr) goto done;
  status = parse_layouts(PySequence_Fast_ITEMS(outer), batch, qlen, voff, vwords, vis);
  if (status < 0) goto done;
  {
    uint32_t* out = nullptr;
    PyObject* vis_obj = new_array<uint32_t>((Py_ssize_t)vis.size(), &out);
    if (vis_obj == nullptr) goto done;
    if (!vis.empty()) std::memcpy(out, vis.data(), vis.size() * 4);
    result = Py_BuildValue("(OOOOi)", qlen_obj, voff_obj, vwords_obj, vis_obj, status);
    Py_DECREF(vis_obj);
  }
done:
  Py_XDECREF(qlen_obj);
  Py_XDECREF(voff_obj);
  Py_XDECREF(vwords_obj);
  Py_DECREF(outer);
  return result;
}

// ---------------------------------------------------------------------------
// metadata(block_tables, num_computed_tokens, query_layouts,
//          num_reserved_query_tokens, num_readonly_prefix_blocks)
//   -> rule (int 1..9) when a field rule fails, or
//      ((tables, computed, layouts, reserved, readonly),
//       (flat i32, counts i64, computed i64, reserved i64, readonly i64,
//        q_lens i64, vis_off i64, vis_words i64, vis u32), tokens, linear)
//
// The construction of PagedAttentionMetadata in one pass
// (src/light_vllm/runtime/execution/paged_attention.py:29-62): the fields
// as tuples (every block table a tuple), the empty reserved field defaulting
// to each layout's query count and the empty readonly field to zeros, and
// the field rules in the reference's order:
//   1 no request; 2 computed or layouts batch differs from the tables';
//   3 reserved batch; 4 readonly batch; 5 a computed count not a
//   non-negative exact int; 6 a reserved count not an exact int covering its
//   layout's queries; 7 a readonly count not a non-negative exact int;
//   8 a block id not a non-negative exact int; 9 a parent not -1 or an
//   earlier query (checked by QueryLayout itself in the reference).
// Then the step facts: flatten, the int fields as int64, layouts' rows.
// A layout's query count is the length of its parent_indices.
// ---------------------------------------------------------------------------
enum MetadataRule {
  kMdEmpty = 1,
  kMdBatch = 2,
  kMdReservedBatch = 3,
  kMdReadonlyBatch = 4,
  kMdComputed = 5,
  kMdReserved = 6,
  kMdReadonly = 7,
  kMdBlockIds = 8,
  kMdParents = 9,
};

// Exact non-negative ints of a tuple into int64 (clamped at INT64_MAX);
// false when an item is not one.
bool counts_of(PyObject* tuple, int64_t* out) {
  const Py_ssize_t n = PyTuple_GET_SIZE(tuple);
  bool ok = true;
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* o = PyTuple_GET_ITEM(tuple, i);
    int64_t v = -1;
    if (PyLong_CheckExact(o)) {
      int overflow = 0;
      const long long x = PyLong_AsLongLongAndOverflow(o, &overflow);
      v = overflow > 0 ? INT64_MAX : (overflow < 0 ? -1 : x);
    }
    ok &= v >= 0;
    out[i] = v;
  }
  return ok;
}

PyObject* metadata(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!want_args(nargs, 5, "metadata")) return nullptr;
  PyObject* fields[5] = {nullptr, nullptr, nullptr, nullptr, nullptr};  // the five fields as tuples
  PyObject* arrays[9] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  PyObject* result = nullptr;
  int rule = 0;
  Py_ssize_t batch = 0, total = 0;
  int64_t *counts = nullptr, *computed = nullptr, *reserved = nullptr, *readonly = nullptr, *qlen = nullptr,
          *voff = nullptr, *vwords = nullptr;
  int32_t* flat = nullptr;
  static std::vector<uint32_t> vis;
  static std::vector<PyObject*> rows;
  vis.clear();
  int64_t tokens = 0;
  bool linear = true;
  for (int i = 0; i < 5; ++i) {
    fields[i] = PySequence_Tuple(args[i]);
    if (fields[i] == nullptr) goto done;
  }
  {
    // Every block table as a tuple (a new outer tuple only if a row changes).
    PyObject* tables = fields[0];
    batch = PyTuple_GET_SIZE(tables);
    PyObject* rebuilt = nullptr;
    for (Py_ssize_t r = 0; r < batch; ++r) {
      PyObject* row = PyTuple_GET_ITEM(tables, r);
      if (PyTuple_CheckExact(row) && rebuilt == nullptr) continue;
      if (rebuilt == nullptr) {
        rebuilt = PyTuple_New(batch);
        if (rebuilt == nullptr) goto done;
        for (Py_ssize_t k = 0; k < r; ++k) PyTuple_SET_ITEM(rebuilt, k, Py_NewRef(PyTuple_GET_ITEM(tables, k)));
      }
      PyObject* as_tuple = PySequence_Tuple(row);
      if (as_tuple == nullptr) {
        Py_DECREF(rebuilt);
        goto done;
      }
      PyTuple_SET_ITEM(rebuilt, r, as_tuple);
    }
    if (rebuilt != nullptr) {
      Py_DECREF(fields[0]);
      fields[0] = rebuilt;
    }
  }
  if (batch == 0) {
    rule = kMdEmpty;
    goto done;
  }
  if (PyTuple_GET_SIZE(fields[1]) != batch || PyTuple_GET_SIZE(fields[2]) != batch) {
    rule = kMdBatch;
    goto done;
  }
  arrays[5] = new_array<int64_t>(batch, &qlen);
  arrays[6] = new_array<int64_t>(batch, &voff);
  arrays[7] = new_array<int64_t>(batch, &vwords);
  if (arrays[5] == nullptr || arrays[6] == nullptr || arrays[7] == nullptr) goto done;
  {
    // Query counts (len of parent_indices; len(layout) where there is none).
    PyObject** layouts = &PyTuple_GET_ITEM(fields[2], 0);
    for (Py_ssize_t r = 0; r < batch; ++r) {
      PyObject* attr = PyObject_GetAttr(layouts[r], g_parent_indices);
      Py_ssize_t q;
      if (attr != nullptr) {
        q = PyObject_Size(attr);
        Py_DECREF(attr);
      } else {
        PyErr_Clear();
        q = PyObject_Size(layouts[r]);
      }
      if (q < 0) goto done;
      qlen[r] = q;
      tokens += q;
    }
  }
  if (PyTuple_GET_SIZE(fields[3]) == 0) {
    PyObject* filled = PyTuple_New(batch);
    if (filled == nullptr) goto done;
    for (Py_ssize_t r = 0; r < batch; ++r) {
      PyObject* n = PyLong_FromLongLong(qlen[r]);
      if (n == nullptr) {
        Py_DECREF(filled);
        goto done;
      }
      PyTuple_SET_ITEM(filled, r, n);
    }
    Py_SETREF(fields[3], filled);
  }
  if (PyTuple_GET_SIZE(fields[3]) != batch) {
    rule = kMdReservedBatch;
    goto done;
  }
  if (PyTuple_GET_SIZE(fields[4]) == 0) {
    PyObject* zeros = PyTuple_New(batch);
    if (zeros == nullptr) goto done;
    for (Py_ssize_t r = 0; r < batch; ++r) PyTuple_SET_ITEM(zeros, r, PyLong_FromLong(0));
    Py_SETREF(fields[4], zeros);
  }
  if (PyTuple_GET_SIZE(fields[4]) != batch) {
    rule = kMdReadonlyBatch;
    goto done;
  }
  arrays[2] = new_array<int64_t>(batch, &computed);
  arrays[3] = new_array<int64_t>(batch, &reserved);
  arrays[4] = new_array<int64_t>(batch, &readonly);
  if (arrays[2] == nullptr || arrays[3] == nullptr || arrays[4] == nullptr) goto done;
  if (!counts_of(fields[1], computed)) {
    rule = kMdComputed;
    goto done;
  }
  {
    bool ok = counts_of(fields[3], reserved);
    for (Py_ssize_t r = 0; r < batch; ++r) ok &= reserved[r] >= qlen[r];
    if (!ok) {
      rule = kMdReserved;
      goto done;
    }
  }
  if (!counts_of(fields[4], readonly)) {
    rule = kMdReadonly;
    goto done;
  }
  rows.assign(&PyTuple_GET_ITEM(fields[0], 0), &PyTuple_GET_ITEM(fields[0], 0) + batch);
  for (PyObject* row : rows) total += PyTuple_GET_SIZE(row);
  arrays[0] = new_array<int32_t>(total, &flat);
  arrays[1] = new_array<int64_t>(batch, &counts);
  if (arrays[0] == nullptr || arrays[1] == nullptr) goto done;
  if (flatten_tables_into(rows, flat, counts) != 0) {
    rule = kMdBlockIds;
    goto done;
  }
  {
    const int status = parse_layouts(&PyTuple_GET_ITEM(fields[2], 0), batch, qlen, voff, vwords, vis);
    if (status < 0) goto done;
    if (status > 0) {
      rule = kMdParents;
      goto done;
    }
    for (Py_ssize_t r = 0; r < batch; ++r) linear &= voff[r] < 0;
  }
  {
    uint32_t* out = nullptr;
    arrays[8] = new_array<uint32_t>((Py_ssize_t)vis.size(), &out);
    if (arrays[8] == nullptr) goto done;
    if (!vis.empty()) std::memcpy(out, vis.data(), vis.size() * 4);
    PyObject* norm = PyTuple_New(5);
    PyObject* facts = PyTuple_New(9);
    if (norm == nullptr || facts == nullptr) {
      Py_XDECREF(norm);
      Py_XDECREF(facts);
      goto done;
    }
    for (int i = 0; i < 5; ++i) {
      PyTuple_SET_ITEM(norm, i, fields[i]);
      fields[i] = nullptr;
    }
    for (int i = 0; i < 9; ++i) {
      PyTuple_SET_ITEM(facts, i, arrays[i]);
      arrays[i] = nullptr;
    }
    result = Py_BuildValue("(NNLO)", norm, facts, (long long)tokens, linear ? Py_True : Py_False);
  }
done:
  for (PyObject* f : fields) Py_XDECREF(f);
  for (PyObject* a : arrays) Py_XDECREF(a);
  if (result == nullptr && rule != 0 && !PyErr_Occurred()) return PyLong_FromLong(rule);
  return result;
}

// ---------------------------------------------------------------------------
// stage(flat i32, counts i64, computed i64, q_lens i64, vis_off i64,
//       vis_words i64, block_size, slots_out i64[T], req_meta_out i32[B*8]) -> status
// slots_out[t] = table[pos // bs] * bs + pos % bs for pos = computed + offset;
// req_meta rows (table_off, blocks, computed, q_len, q_start, vis_off,
// vis_words, 0).  status 1: a query position past its table (only possible
// when the tables were not validated).
// ---------------------------------------------------------------------------
int stage_rows(const int32_t* ids, const int64_t* cnt, const int64_t* comp, const int64_t* ql, const int64_t* voff,
               const int64_t* vwords, int64_t batch, int64_t bs, int64_t* out, int32_t* rm);

PyObject* stage(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!want_args(nargs, 9, "stage")) return nullptr;
  Buf flat(args[0], false, 4, "flat"), counts(args[1], false, 8, "counts"), computed(args[2], false, 8, "computed"),
      q_lens(args[3], false, 8, "q_lens"), vis_off(args[4], false, 8, "vis_off"),
      vis_words(args[5], false, 8, "vis_words");
  int64_t bs = 0;
  if (!flat.ok() || !counts.ok() || !computed.ok() || !q_lens.ok() || !vis_off.ok() || !vis_words.ok() ||
      !as_i64(args[6], &bs))
    return nullptr;
  Buf slots(args[7], true, 8, "slots_out"), meta(args[8], true, 4, "req_meta_out");
  if (!slots.ok() || !meta.ok()) return nullptr;
  const Py_ssize_t batch = counts.count();
  const int64_t* cnt = counts.data<int64_t>();
  const int64_t* comp = computed.data<int64_t>();
  const int64_t* ql = q_lens.data<int64_t>();
  int64_t tokens = 0;
  for (Py_ssize_t r = 0; r < batch; ++r) tokens += ql[r];
  if (bs <= 0 || computed.count() != batch || q_lens.count() != batch || vis_off.count() != batch ||
      vis_words.count() != batch || slots.count() != tokens || meta.count() != batch * kReqFields) {
    PyErr_SetString(PyExc_ValueError, "stage: inconsistent arguments");
    return nullptr;
  }
  const int status = stage_rows(flat.data<int32_t>(), cnt, comp, ql, vis_off.data<int64_t>(),
                                vis_words.data<int64_t>(), batch, bs, slots.data<int64_t>(), meta.data<int32_t>());
  return PyLong_FromLong(status);
}

// stage's body: slots and req_meta rows; returns 1 when a query position
// lies past its table (its slot is -1), else 0.
int stage_rows(const int32_t* ids, const int64_t* cnt, const int64_t* comp, const int64_t* ql, const int64_t* voff,
               const int64_t* vwords, int64_t batch, int64_t bs, int64_t* out, int32_t* rm) {
  int status = 0;
  int64_t off = 0, t = 0;
  for (int64_t r = 0; r < batch; ++r) {
    int32_t* m = rm + r * kReqFields;
    m[0] = (int32_t)off;
    m[1] = (int32_t)cnt[r];
    m[2] = (int32_t)comp[r];
    m[3] = (int32_t)ql[r];
    m[4] = (int32_t)t;
    m[5] = (int32_t)voff[r];
    m[6] = (int32_t)vwords[r];
    m[7] = 0;
    for (int64_t i = 0; i < ql[r]; ++i, ++t) {
      const int64_t pos = comp[r] + i;
      const int64_t lb = pos / bs;
      if (lb >= cnt[r]) {
        status = 1;
        out[t] = -1;
        continue;
      }
      out[t] = (int64_t)ids[off + lb] * bs + (pos - lb * bs);
    }
    off += cnt[r];
  }
  return status;
}

// ---------------------------------------------------------------------------
// Work lists of one layer shape.
//
// Decode rows are the requests whose q_len * group columns fit
// decode_max_columns (every request when it is 0); a request has
// ceil(ceil(q_len * group / 16) / col_tiles) column groups, each a segment
// of computed + q_len tokens.  Stream-K: the segments are laid end to end in
// unit_tokens units, and the unit range is cut into W balanced contiguous
// shares (wave w: units [w*total/W, (w+1)*total/W)), W the fewest shares
// that give the largest share the resident waves would get, and no share
// above what the kernel's LDS table slice covers.  A wave's share is a list
// of pieces (the part of each segment inside it); a segment cut into several
// pieces gets consecutive partial slots and one merge job.
//
// Prefill rows are the others.  A unit is up to ``columns`` MFMA columns
// (query, head-in-group pairs) of one request; it needs the keys up to its
// last query.  With fewer units than slots_per_head, every unit's tile range
// is cut into near-equal pieces of at least min_tiles tiles; the pieces of a
// split unit write consecutive partial slots and one merge job combines
// them.  Units come heaviest first (key tiles x columns, stable).
// ---------------------------------------------------------------------------
struct Requests {
  const int32_t* meta;  // [batch][kReqFields]
  int64_t batch;
  int64_t q_len(int64_t r) const { return meta[r * kReqFields + 3]; }
  int64_t computed(int64_t r) const { return meta[r * kReqFields + 2]; }
  const int32_t* row(int64_t r) const { return meta + r * kReqFields; }
};

struct DecodeLists {
  std::vector<int32_t> pieces, first, jobs;
  int64_t waves = 0, per_wave = 0, merge_cols = 1;
  int64_t group_waves = 1;  // 1: stream-K; kSplitWaves: workgroup split
  int32_t slots = 0;
  void reset() {
    pieces.clear();
    first.clear();
    jobs.clear();
    waves = per_wave = 0;
    merge_cols = 1;
    group_waves = 1;
    slots = 0;
  }
};

struct DecodeParams {
  int64_t group, col_tiles, max_cols, hkv, resident, bs, min_units, max_units, unit;
  int64_t split_groups = 0;  // resident workgroups of the workgroup-split kernel (0: not built)
  int64_t split_waves = 0;   // its waves per workgroup
};

// Workgroup split of the decode kernel: workgroups of split_waves waves, one
// segment each, its pieces combined in LDS.  The planner takes it for
// latency-bound steps: the step's segments fit the resident workgroups and
// the longest piece is no longer than stream-K's largest share plus what the
// merge launch it saves costs (kSplitMergeTiles tiles).  A workgroup's time
// grows by about one tile's load latency per tile of its longest wave, so
// the split is taken at one tile per wave, and at two only where stream-K is
// slower too: when the pieces average at most 1.5 tiles, or the step has
// kSplitBusyGroups segments or more.  (Measured on 28 bf16 layers of 28 / 4
// heads, D 128, per layer: one tile 4.3-12.6 us against stream-K's 4.9-18.3;
// two tiles 13.4 vs 12.7 at 1 x 512 tokens, 15.6 vs 15.1 at 16 x 512, 13.6
// vs 14.7 at 16 x 384, 16.6 vs 18.0 at 32 x 512, 19.8 vs 22.6 at 64 x 512;
// three and four tiles lose, 19.3 vs 16.9 and 20.7 vs 13.7.  Without a cap
// C2's 64 contexts of 512-4096 tokens took one CU per segment: 84 us against
// 59 us on stream-K shares.  Against stream-K at one tile per share, in a HIP
// graph of 8 layers: one tile 6.5-9.1 us against 9.5-15.0; two tiles at 256
// tokens 10.8 vs 9.9 (1 sequence), 10.9 vs 10.0 (4), 11.3 vs 11.4 (16),
// 11.5 vs 14.5 (32), 13.4 vs 18.0 (64).  The two-tile split is kept where
// stream-K's GPU time is lower by up to a tenth: it is one launch per layer
// where stream-K makes two, and the host submits about 4 us more per layer
// for the second (the 28-layer small config: 325 us of GPU time and 5.3 us of
// host time per layer on the split, 313 us and 9.3 us on stream-K).)
constexpr int64_t kSplitMergeTiles = 3;
constexpr int64_t kMergePiecesMax = 48;
constexpr int64_t kSplitMaxTiles = 2;
constexpr int64_t kSplitBusyGroups = 128;

void build_decode(const Requests& q, const int32_t* ids, int64_t nflat, const DecodeParams& d, DecodeLists& out) {
  struct Seg {
    int32_t req, group;
    int64_t start, tiles;
  };
  std::vector<Seg> segs;
  int64_t total = 0;
  for (int64_t r = 0; r < q.batch; ++r) {
    const int64_t columns = q.q_len(r) * d.group;
    if (d.max_cols > 0 && columns > d.max_cols) continue;
    const int64_t tiles = (q.computed(r) + q.q_len(r) + d.unit - 1) / d.unit;
    const int64_t ngroups = ((columns + 15) / 16 + d.col_tiles - 1) / d.col_tiles;
    for (int64_t g = 0; g < ngroups; ++g) {
      segs.push_back({(int32_t)r, (int32_t)g, total, tiles});
      total += tiles;
    }
  }
  if (total == 0) return;
  int64_t cap = std::max<int64_t>(1, ((kTableSlice - 2) * d.bs) / d.unit);
  if (d.max_units > 0) cap = std::max<int64_t>(1, std::min(cap, d.max_units));
  // Shares of at least min_units tiles, and long enough that no segment is
  // cut into more than kMergePiecesMax pieces (a segment of T tiles over
  // shares of P takes at most ceil(T / P) + 1; the merge reads 16 partials
  // per round trip: one sequence of 2048 tokens in 65 one-tile pieces took
  // 15.7 us per layer against 14.9 in 33).
  int64_t longest_seg = 0;
  for (const Seg& sg : segs) longest_seg = std::max(longest_seg, sg.tiles);
  const int64_t min_units =
      std::max<int64_t>(d.min_units, (longest_seg + kMergePiecesMax - 2) / (kMergePiecesMax - 1));
  int64_t waves = std::max<int64_t>(
      1, std::min(std::max<int64_t>(1, d.resident / d.hkv), (total + min_units - 1) / min_units));
  waves = std::max(waves, (total + cap - 1) / cap);
  const int64_t per_wave = (total + waves - 1) / waves;
  waves = (total + per_wave - 1) / per_wave;
  // Walk segment ends and share bounds together: one piece per step.  The
  // bound of share w, floor((w + 1) * total / waves), is stepped with a
  // running remainder (no division per piece).
  struct PieceRec {
    int32_t seg, wave;
    int64_t lo, hi;
  };
  std::vector<PieceRec> recs;
  recs.reserve(segs.size() + (size_t)waves);
  std::vector<int32_t> seg_pieces(segs.size(), 0);
  const int64_t share_q = total / waves, share_r = total % waves;
  int64_t bound = share_q, rem = share_r;
  if (rem >= waves) {
    rem -= waves;
    ++bound;
  }
  for (size_t s = 0, pos = 0, w = 0; (int64_t)pos < total;) {
    const int64_t seg_end = segs[s].start + segs[s].tiles;
    const int64_t end = std::min(seg_end, bound);
    recs.push_back({(int32_t)s, (int32_t)w, (int64_t)pos, end});
    ++seg_pieces[s];
    pos = (size_t)end;
    if (end == seg_end) ++s;
    if (end == bound) {
      ++w;
      bound += share_q;
      rem += share_r;
      if (rem >= waves) {
        rem -= waves;
        ++bound;
      }
    }
  }
  const int64_t per_slot = 16 * d.col_tiles;  // columns of one partial slot
  // Whole blocks per unit when units are whole blocks (the usual case), so
  // a piece's first logical block needs no division.
  const int64_t blocks_per_unit = d.unit % d.bs == 0 ? d.unit / d.bs : 0;
  out.pieces.assign(recs.size() * kPieceFields, 0);
  out.first.assign((size_t)waves + 1, 0);
  out.waves = waves;
  out.per_wave = per_wave;
  int64_t w = 0;
  for (size_t p = 0; p < recs.size(); ++p) {
    const PieceRec& x = recs[p];
    const Seg& sg = segs[(size_t)x.seg];
    const int32_t* m = q.row(sg.req);
    int32_t* o = out.pieces.data() + p * kPieceFields;
    while (w <= x.wave) out.first[(size_t)w++] = (int32_t)p;
    const bool multi = seg_pieces[(size_t)x.seg] > 1;
    const int64_t tok_begin = (x.lo - sg.start) * d.unit;
    o[0] = sg.req;
    o[1] = sg.group;
    o[2] = (int32_t)tok_begin;
    o[3] = (int32_t)std::min((x.hi - sg.start) * d.unit, q.computed(sg.req) + q.q_len(sg.req));
    o[4] = multi ? out.slots : -1;
    o[5] = m[0];   // table_off
    o[6] = m[2];   // computed
    o[7] = m[3];   // q_len
    o[8] = m[4];   // q_start
    o[9] = m[5];   // vis_off
    o[10] = m[6];  // vis_words
    const int64_t lb0 = blocks_per_unit ? (x.lo - sg.start) * blocks_per_unit : tok_begin / d.bs;
    for (int k = 0; k < kPieceBlocks; ++k) {
      const int64_t lb = lb0 + k, idx = m[0] + lb;
      o[11 + k] = (lb < m[1] && idx < nflat) ? ids[idx] : 0;
    }
    if (multi && x.lo == sg.start) {
      const int32_t job[kMergeFields] = {sg.req, sg.group, out.slots, seg_pieces[(size_t)x.seg], m[4], m[3], 0, 0};
      out.jobs.insert(out.jobs.end(), job, job + kMergeFields);
      // The merge grid covers the most columns any job has.
      out.merge_cols = std::max(out.merge_cols, std::min(per_slot, (int64_t)m[3] * d.group - sg.group * per_slot));
    }
    if (multi) ++out.slots;
  }
  while (w <= waves) out.first[(size_t)w++] = (int32_t)recs.size();

  // The workgroup split instead, when it is no slower (see kSplitMergeTiles):
  // one record per wave, an idle wave's with request -1.
  const int64_t gw = d.split_waves;
  if (d.split_groups <= 0 || gw <= 1 || d.col_tiles != 1) return;
  int64_t longest = 0;
  for (const Seg& sg : segs) longest = std::max(longest, sg.tiles);
  const int64_t split_share = (longest + gw - 1) / gw;
  const int64_t nseg = (int64_t)segs.size();
  if (nseg * d.hkv > d.split_groups || split_share > cap || split_share > kSplitMaxTiles) return;
  if (split_share == kSplitMaxTiles && 2 * longest > 3 * gw && nseg * d.hkv < kSplitBusyGroups) return;
  if (split_share > per_wave + (out.jobs.empty() ? 0 : kSplitMergeTiles)) return;
  out.reset();
  out.group_waves = gw;
  out.waves = gw * nseg;
  out.per_wave = split_share;
  out.first.resize((size_t)out.waves + 1);
  std::iota(out.first.begin(), out.first.end(), 0);
  out.pieces.assign((size_t)(out.waves * kPieceFields), 0);
  for (int64_t s = 0; s < nseg; ++s) {
    const Seg& sg = segs[(size_t)s];
    const int32_t* m = q.row(sg.req);
    const int64_t n = std::min(gw, sg.tiles);
    const int64_t seq_end = q.computed(sg.req) + q.q_len(sg.req);
    for (int64_t i = 0; i < gw; ++i) {
      int32_t* o = out.pieces.data() + (s * gw + i) * kPieceFields;
      if (i >= n) {
        o[0] = -1;  // an idle wave
        o[4] = -1;
        continue;
      }
      const int64_t lo = i * sg.tiles / n, hi = (i + 1) * sg.tiles / n;
      o[0] = sg.req;
      o[1] = sg.group;
      o[2] = (int32_t)(lo * d.unit);
      o[3] = (int32_t)std::min(hi * d.unit, seq_end);
      o[4] = n > 1 ? (int32_t)i : -1;
      o[5] = m[0];
      o[6] = m[2];
      o[7] = m[3];
      o[8] = m[4];
      o[9] = m[5];
      o[10] = m[6];
      const int64_t lb0 = blocks_per_unit ? lo * blocks_per_unit : (lo * d.unit) / d.bs;
      for (int k = 0; k < kPieceBlocks; ++k) {
        const int64_t lb = lb0 + k, idx = m[0] + lb;
        o[11 + k] = (lb < m[1] && idx < nflat) ? ids[idx] : 0;
      }
    }
  }
}

struct PrefillLists {
  std::vector<int32_t> units, jobs;
  int32_t slots = 0;
  int64_t merge_cols = 1;
  double mean_tiles = 0.0;
  void reset() {
    units.clear();
    jobs.clear();
    slots = 0;
    merge_cols = 1;
    mean_tiles = 0.0;
  }
};

struct PrefillParams {
  int64_t group, columns, key_tokens, slots_per_head, min_tiles, max_cols;
  const int32_t* ids = nullptr;  // flat block tables, for shared-prefix spans (null: no spans)
  int64_t block_size = 0;
  bool spans = false;
  int64_t kv_heads = 1, xcds = 0;  // the device's XCDs (0 or 1: no per-XCD order)
  int64_t resident_per_head = 0;   // resident workgroups / kv heads (0: unknown)
  int64_t order = 0;               // per-XCD order: 0 the faster (simulated), 1 grouped, 2 plain
};

// A prefill unit: columns [col0, col0 + cols) of request req over key tiles
// [first, first + tiles).  A span unit covers columns of a span (below): its
// columns are the (token, head) pairs of the span's packed queries.
struct Unit {
  int32_t req;
  int64_t col0, cols, tiles, first;
  int32_t span;    // the span of a span unit or of a member's unit, else -1
  bool span_unit;
};

// Shared-prefix decomposition.  A span is a run of consecutive prefill rows
// [r0, r1) whose block tables list the same block ids over the key tokens
// [0, prefix), with prefix a whole number of key tiles and at most every
// member's computed count: those keys are the same K/V rows for every
// member, visible to every query, and not written this step.  They are
// attended once per 128 columns of the span's packed queries (span units),
// and each member's own units cover only keys [prefix, end); every member
// unit writes partials, and its merge job adds the span units' partials of
// its columns (merge fields 6 and 7).  light-vllm's prefix cache produces
// such runs: sequences sharing a prompt prefix hold the same readonly blocks
// at the same logical indices (paged_attention.py:138-172 allows sharing
// only there).
struct Span {
  int64_t r0, r1, prefix, t0, ntok, table_off;
  int64_t pieces = 1;  // pieces per span unit
  int32_t base = -1;   // partial slot of the first span unit's first piece
};

constexpr int64_t kSpanMaxPieces = 127;         // merge field 7 holds pieces << 24
constexpr int64_t kSpanMaxColumns = 1 << 24;    // ... and the column offset below it

std::vector<Span> find_spans(const Requests& q, const PrefillParams& p) {
  std::vector<Span> spans;
  if (!p.spans || p.ids == nullptr || p.block_size <= 0) return spans;
  const int64_t KT = p.key_tokens, G = p.group, bs = p.block_size;
  auto wide = [&](int64_t r) { return q.q_len(r) * G > p.max_cols; };
  auto units_of = [&](int64_t cols) { return (cols + p.columns - 1) / p.columns; };
  for (int64_t r = 0; r < q.batch;) {
    if (!wide(r) || q.row(r)[1] == 0) {
      ++r;
      continue;
    }
    const int32_t* first = p.ids + q.row(r)[0];
    int64_t lcp = q.row(r)[1], min_comp = q.computed(r);
    int64_t prefix = std::min(lcp * bs, min_comp) / KT * KT;
    int64_t end = r + 1, cols = q.q_len(r) * G, member_units = units_of(q.q_len(r) * G);
    while (end < q.batch && wide(end)) {
      const int32_t* t = p.ids + q.row(end)[0];
      const int64_t n = std::min<int64_t>(lcp, q.row(end)[1]);
      int64_t l = 0;
      while (l < n && t[l] == first[l]) ++l;
      const int64_t mc = std::min(min_comp, q.computed(end));
      const int64_t pre = std::min(l * bs, mc) / KT * KT;
      // A member that would halve the prefix the run already shares ends it.
      if (pre < 2 * KT || (end - r >= 2 && 2 * pre < prefix)) break;
      lcp = l;
      min_comp = mc;
      prefix = pre;
      cols += q.q_len(end) * G;
      member_units += units_of(q.q_len(end) * G);
      ++end;
    }
    // Worth it when the span's columns pack into fewer units than the
    // members' own (each unit streams the prefix once).
    if (end - r >= 2 && prefix >= 2 * KT && units_of(cols) < member_units && cols < kSpanMaxColumns) {
      Span s;
      s.r0 = r;
      s.r1 = end;
      s.prefix = prefix;
      s.t0 = q.row(r)[4];
      s.ntok = cols / G;
      s.table_off = q.row(r)[0];
      spans.push_back(s);
    }
    r = end;
  }
  return spans;
}

std::vector<Unit> prefill_units_of(const Requests& q, const PrefillParams& p, const std::vector<Span>& spans) {
  std::vector<Unit> units;
  const int64_t KT = p.key_tokens;
  size_t s = 0;
  for (int64_t r = 0; r < q.batch; ++r) {
    const int64_t ncols = q.q_len(r) * p.group;
    if (ncols <= p.max_cols) continue;
    const Span* sp = (s < spans.size() && spans[s].r0 <= r && r < spans[s].r1) ? &spans[s] : nullptr;
    const int64_t first = sp ? sp->prefix / KT : 0;
    if (sp && r == sp->r0) {
      const int64_t scols = sp->ntok * p.group;
      for (int64_t c0 = 0; c0 < scols; c0 += p.columns)
        units.push_back({-1 - (int32_t)s, c0, std::min(p.columns, scols - c0), first, 0, (int32_t)s, true});
    }
    for (int64_t c0 = 0; c0 < ncols; c0 += p.columns) {
      const int64_t cols = std::min(p.columns, ncols - c0);
      const int64_t kneed = q.computed(r) + (c0 + cols - 1) / p.group + 1;
      units.push_back({(int32_t)r, c0, cols, (kneed + KT - 1) / KT - first, first, sp ? (int32_t)s : -1, false});
    }
    if (sp && r + 1 == sp->r1) ++s;
  }
  return units;
}

// Per-XCD order of the prefill grid.  The hardware hands workgroup b to XCD
// b % X (X XCDs, each with its own L2), and workgroup b is (unit position
// u = b / H, kv head b % H) for H kv heads, so position u runs kv head h on
// XCD (u H + h) % X.  That XCD depends on h and on u modulo
// P = X / gcd(H, X) only: positions congruent modulo P form a bin whose
// units, per kv head, all run on one XCD and share its L2.  A request's
// units read the same keys, so the planner keeps each request (a span
// unit's group: its span) in as few bins as the dispatch order allows.
int64_t xcd_bins(const PrefillParams& p) {
  if (p.xcds <= 1 || p.kv_heads <= 0) return 1;
  return p.xcds / std::gcd(p.kv_heads, p.xcds);
}

// Bins of near-equal work: whole groups, heaviest first, each to the
// lightest bin; then single records move from the heaviest bin to the
// lightest while that lowers the heaviest by more than 1/32 of a bin.
void assign_bins(const std::vector<int64_t>& group_of, const std::vector<int64_t>& work, int64_t nbins,
                 std::vector<int64_t>& bin_of) {
  std::unordered_map<int64_t, int64_t> gwork;
  for (size_t k = 0; k < work.size(); ++k) gwork[group_of[k]] += work[k];
  std::vector<std::pair<int64_t, int64_t>> groups(gwork.begin(), gwork.end());  // (group, work)
  std::sort(groups.begin(), groups.end(), [](const auto& a, const auto& b) {
    return a.second != b.second ? a.second > b.second : a.first < b.first;
  });
  std::vector<int64_t> load((size_t)nbins, 0);
  std::unordered_map<int64_t, int64_t> gbin;
  for (const auto& [g, w] : groups) {
    const size_t b = (size_t)(std::min_element(load.begin(), load.end()) - load.begin());
    gbin[g] = (int64_t)b;
    load[b] += w;
  }
  for (size_t k = 0; k < work.size(); ++k) bin_of[k] = gbin[group_of[k]];
  const int64_t total = std::accumulate(load.begin(), load.end(), (int64_t)0);
  for (size_t iter = 0; iter < work.size(); ++iter) {
    const size_t hi = (size_t)(std::max_element(load.begin(), load.end()) - load.begin());
    const size_t lo = (size_t)(std::min_element(load.begin(), load.end()) - load.begin());
    const int64_t gap = load[hi] - load[lo];
    if (gap * 32 * nbins <= total) break;
    int64_t best = -1;
    for (size_t k = 0; k < work.size(); ++k)
      if (bin_of[k] == (int64_t)hi && work[k] < gap && (best < 0 || work[k] > work[(size_t)best])) best = (int64_t)k;
    if (best < 0) break;
    bin_of[(size_t)best] = (int64_t)lo;
    load[hi] -= work[(size_t)best];
    load[lo] += work[(size_t)best];
  }
}

// The latest finish over the bins when each bin's records (position k of
// ``order`` in bin k % nbins; -1: padding) start in order on ``slots``
// workgroup slots, each on the first slot to free (the dispatcher's rule).
int64_t packed_makespan(const std::vector<int64_t>& order, const std::vector<int64_t>& work, int64_t nbins,
                        int64_t slots) {
  int64_t worst = 0;
  std::vector<int64_t> heap;
  for (int64_t b = 0; b < nbins; ++b) {
    heap.assign((size_t)slots, 0);
    for (size_t k = (size_t)b; k < order.size(); k += (size_t)nbins) {
      if (order[k] < 0) continue;
      std::pop_heap(heap.begin(), heap.end(), std::greater<int64_t>());
      heap.back() += work[(size_t)order[k]];
      std::push_heap(heap.begin(), heap.end(), std::greater<int64_t>());
    }
    worst = std::max(worst, *std::max_element(heap.begin(), heap.end()));
  }
  return worst;
}

void build_prefill(const Requests& q, const PrefillParams& p, PrefillLists& out) {
  std::vector<Span> spans = find_spans(q, p);
  const std::vector<Unit> units = prefill_units_of(q, p, spans);
  const int64_t n = (int64_t)units.size();
  int64_t tile_sum = 0;
  for (const Unit& u : units) tile_sum += u.tiles;
  out.mean_tiles = n ? (double)tile_sum / (double)n : 0.0;
  std::vector<int64_t> npieces((size_t)n, 1);
  if (p.slots_per_head > 0 && n < p.slots_per_head) {
    const int64_t target = std::max(p.min_tiles, (tile_sum + p.slots_per_head - 1) / p.slots_per_head);
    for (int64_t u = 0; u < n; ++u) {
      const Unit& un = units[(size_t)u];
      const int64_t k = std::max<int64_t>(1, (un.tiles + target - 1) / target);
      npieces[(size_t)u] = un.span_unit ? std::min(k, kSpanMaxPieces) : k;
    }
  }
  struct PRec {
    int64_t unit, t0, t1, i, work;
    int32_t slot;
  };
  std::vector<PRec> recs;
  for (int64_t u = 0; u < n; ++u) {
    const Unit& un = units[(size_t)u];
    const int64_t k = npieces[(size_t)u], tiles = un.tiles;
    // Partial slots in (unit, piece) order, before the heaviest-first sort:
    // a span's units are consecutive, so piece i of its span unit j is slot
    // base + j * pieces + i.  Span units and members' units always write
    // partials (their merge job combines both parts).
    if (un.span_unit && spans[(size_t)un.span].base < 0) {
      spans[(size_t)un.span].base = out.slots;
      spans[(size_t)un.span].pieces = k;
    }
    for (int64_t i = 0; i < k; ++i) {
      const int64_t t0 = (i * tiles) / k, t1 = ((i + 1) * tiles) / k;
      const bool partial = k > 1 || un.span >= 0;
      recs.push_back({u, t0, t1, i, (t1 - t0) * un.cols, partial ? out.slots++ : -1});
    }
  }
  for (const PRec& x : recs) {
    const Unit& un = units[(size_t)x.unit];
    if (x.slot < 0 || x.i != 0 || un.span_unit) continue;
    const int32_t* m = q.row(un.req);
    int32_t span_slot = 0, span_cols = 0;
    if (un.span >= 0) {
      const Span& sp = spans[(size_t)un.span];
      span_slot = sp.base + 1;
      span_cols = (int32_t)(((int64_t)m[4] - sp.t0) * p.group | (sp.pieces << 24));
    }
    const int32_t job[kMergeFields] = {un.req, (int32_t)(un.col0 / p.columns), x.slot,
                                       (int32_t)npieces[(size_t)x.unit], m[4], m[3], span_slot, span_cols};
    out.jobs.insert(out.jobs.end(), job, job + kMergeFields);
    out.merge_cols = std::max(out.merge_cols, un.cols);
  }
  // Heaviest first: the dispatch order that packs the resident workgroups
  // best.  With several per-XCD bins the planner also builds the grouped
  // order (each request, or span, in one bin; bins interleaved, padding in
  // the shorter ones) and keeps it when the bins' simulated packing is no
  // slower (within 1/64): the plain order's bins (position parity) mix
  // every request's units, so each XCD's L2 holds all of their keys.
  std::vector<int64_t> order(recs.size());
  std::iota(order.begin(), order.end(), (int64_t)0);
  std::stable_sort(order.begin(), order.end(),
                   [&](int64_t x, int64_t y) { return recs[(size_t)x].work > recs[(size_t)y].work; });
  const int64_t nbins = xcd_bins(p);
  if (nbins > 1) {
    std::vector<int64_t> group_of(recs.size()), work(recs.size()), bin_of(recs.size());
    for (size_t k = 0; k < recs.size(); ++k) {
      const Unit& un = units[(size_t)recs[k].unit];
      group_of[k] = un.span_unit ? q.batch + un.span : un.req;
      work[k] = recs[k].work;
    }
    assign_bins(group_of, work, nbins, bin_of);
    std::vector<std::vector<int64_t>> bins((size_t)nbins);
    for (int64_t k : order) bins[(size_t)bin_of[(size_t)k]].push_back(k);  // heaviest first within a bin
    size_t longest = 0;
    for (const auto& b : bins) longest = std::max(longest, b.size());
    std::vector<int64_t> grouped;
    grouped.reserve(longest * (size_t)nbins);
    for (size_t i = 0; i < longest; ++i)
      for (const auto& b : bins) grouped.push_back(i < b.size() ? b[i] : -1);
    bool keep = p.order != 2;
    if (p.order == 0 && p.resident_per_head > 0) {
      const int64_t slots = std::max<int64_t>(1, p.resident_per_head / nbins);
      const int64_t mg = packed_makespan(grouped, work, nbins, slots);
      const int64_t mp = packed_makespan(order, work, nbins, slots);
      keep = mg * 64 <= mp * 65;
    }
    if (keep) order.swap(grouped);
  }
  out.units.assign(order.size() * kPrefillFields, 0);
  for (size_t k = 0; k < order.size(); ++k) {
    if (order[k] < 0) {  // padding: zero columns, nothing to do
      int32_t* o = out.units.data() + k * kPrefillFields;
      o[0] = kPadRecord;
      o[5] = -1;
      o[10] = -1;
      o[12] = -1;
      continue;
    }
    const PRec& x = recs[(size_t)order[k]];
    const Unit& un = units[(size_t)x.unit];
    int32_t* o = out.units.data() + k * kPrefillFields;
    const bool last = x.i + 1 == npieces[(size_t)x.unit];
    o[0] = un.req;
    o[1] = (int32_t)un.col0;
    o[2] = (int32_t)un.cols;
    o[3] = (int32_t)((un.first + x.t0) * p.key_tokens);
    // A request's last piece runs to its queries' keys (0: no bound); a
    // span unit's pieces always end at a tile boundary within the prefix.
    o[4] = (last && !un.span_unit) ? 0 : (int32_t)((un.first + x.t1) * p.key_tokens);
    o[5] = x.slot;
    // The request's fields (a span unit reads as a linear request whose
    // computed count is its key_end), then the first tile's block ids.
    int64_t table_off, table_len;
    if (un.span_unit) {
      const Span& sp = spans[(size_t)un.span];
      table_off = sp.table_off;
      table_len = (sp.prefix + p.block_size - 1) / std::max<int64_t>(1, p.block_size);
      o[6] = (int32_t)sp.table_off;
      o[7] = (int32_t)sp.t0;
      o[8] = o[4];
      o[9] = 0;
      o[10] = -1;
      o[11] = 0;
    } else {
      const int32_t* m = q.row(un.req);
      table_off = m[0];
      table_len = m[1];
      o[6] = m[0];
      o[7] = m[4];
      o[8] = m[2];
      o[9] = m[3];
      o[10] = m[5];
      o[11] = m[6];
    }
    o[12] = -1;
    if (p.ids != nullptr && p.block_size > 0) {
      const int64_t k0 = o[3], lb0 = k0 / p.block_size, lb1 = (k0 + p.key_tokens - 1) / p.block_size;
      if (lb1 - lb0 < 4) {
        for (int b = 0; b < 4; ++b) o[12 + b] = lb0 + b < table_len ? p.ids[table_off + lb0 + b] : 0;
      }
    }
  }
}

// Column tiles per decode wave: 4 when the decode rows' K/V re-reads at one
// tile per wave cost more than the four-tile kernel's slower tiles
//   sum(seq * ceil(tiles / 4)) * cost4 < sum(seq * tiles),
// else 1 (always 1 when the four-tile kernel is not built, max_ctw < 4).
int64_t choose_col_tiles(const Requests& q, int64_t group, int64_t max_cols, int64_t max_ctw, double cost4) {
  if (max_ctw < 4) return 1;
  double one = 0.0, four = 0.0;
  for (int64_t r = 0; r < q.batch; ++r) {
    const int64_t columns = q.q_len(r) * group;
    if (max_cols > 0 && columns > max_cols) continue;
    const double seq = (double)(q.computed(r) + q.q_len(r));
    const int64_t nct = (columns + 15) / 16;
    one += seq * (double)nct;
    four += seq * (double)((nct + 3) / 4);
  }
  return four * cost4 < one ? 4 : 1;
}

// Prefill workgroup shape: 8 waves of one column tile when the units will
// be split over the resident workgroups or are short (mean key tiles per
// unit at most wide_max_tiles), else 4 waves of two column tiles.
int64_t choose_prefill_waves(const Requests& q, const PrefillParams& p, int64_t slots_per_head8, bool wide_built,
                             double wide_max_tiles) {
  if (!wide_built) return 4;
  const std::vector<Unit> units = prefill_units_of(q, p, find_spans(q, p));
  if (units.empty()) return 4;
  int64_t tile_sum = 0;
  for (const Unit& u : units) tile_sum += u.tiles;
  const bool split = slots_per_head8 > 0 && (int64_t)units.size() < slots_per_head8;
  return split || (double)tile_sum / (double)units.size() <= wide_max_tiles ? 8 : 4;
}

template <typename T>
PyObject* to_bytearray(const std::vector<T>& v) {
  T* out = nullptr;
  PyObject* arr = new_array<T>((Py_ssize_t)v.size(), &out);
  if (arr != nullptr && !v.empty()) std::memcpy(out, v.data(), v.size() * sizeof(T));
  return arr;
}

PyObject* decode_result(const DecodeLists& d) {
  PyObject* a = to_bytearray(d.pieces);
  PyObject* b = to_bytearray(d.first);
  PyObject* c = to_bytearray(d.jobs);
  PyObject* result = (a && b && c) ? Py_BuildValue("(OOOLLiLL)", a, b, c, (long long)d.waves, (long long)d.per_wave,
                                                   d.slots, (long long)d.merge_cols, (long long)d.group_waves)
                                   : nullptr;
  Py_XDECREF(a);
  Py_XDECREF(b);
  Py_XDECREF(c);
  return result;
}

PyObject* prefill_result(const PrefillLists& p) {
  PyObject* a = to_bytearray(p.units);
  PyObject* b = to_bytearray(p.jobs);
  PyObject* result =
      (a && b) ? Py_BuildValue("(OOidL)", a, b, p.slots, p.mean_tiles, (long long)p.merge_cols) : nullptr;
  Py_XDECREF(a);
  Py_XDECREF(b);
  return result;
}

// Whether every request's table (table_off, blocks) lies inside the flat
// array of nflat ids (req_meta handed in from Python is not trusted).
bool tables_fit(const Requests& q, int64_t nflat) {
  for (int64_t r = 0; r < q.batch; ++r) {
    const int64_t off = q.row(r)[0], n = q.row(r)[1];
    if (off < 0 || n < 0 || off + n > nflat) return false;
  }
  return true;
}

bool requests_of(const Buf& meta, Requests* q, const char* name) {
  q->meta = meta.data<int32_t>();
  q->batch = meta.count() / kReqFields;
  if (meta.count() != q->batch * kReqFields) {
    PyErr_Format(PyExc_ValueError, "%s: req_meta is not [batch][%d]", name, kReqFields);
    return false;
  }
  return true;
}

// decode_work(req_meta i32[B*8], flat i32, group, col_tiles, decode_max_columns,
//             num_kv_heads, resident_waves, block_size, min_units_per_wave,
//             max_units_per_wave (0 = none), unit_tokens, split_groups, split_waves)
//   -> (pieces i32 [n, 16], wave_first i32 [W + 1], jobs i32 [m, 8],
//       W, largest share, partial slots, most columns of a merge job,
//       waves per workgroup)
// split_groups: resident workgroups of the workgroup-split kernel (0: never
// split in workgroups) and split_waves its waves per workgroup.
PyObject* decode_work(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!want_args(nargs, 13, "decode_work")) return nullptr;
  Buf meta(args[0], false, 4, "req_meta"), flat(args[1], false, 4, "flat");
  if (!meta.ok() || !flat.ok()) return nullptr;
  Requests q;
  if (!requests_of(meta, &q, "decode_work")) return nullptr;
  DecodeParams d;
  int64_t* fields[] = {&d.group,     &d.col_tiles, &d.max_cols, &d.hkv,          &d.resident,   &d.bs,
                       &d.min_units, &d.max_units, &d.unit,     &d.split_groups, &d.split_waves};
  for (int i = 0; i < 11; ++i)
    if (!as_i64(args[2 + i], fields[i])) return nullptr;
  if (d.group <= 0 || d.col_tiles <= 0 || d.hkv <= 0 || d.bs <= 0 || d.unit <= 0 || d.min_units <= 0) {
    PyErr_SetString(PyExc_ValueError, "decode_work: inconsistent arguments");
    return nullptr;
  }
  DecodeLists out;
  build_decode(q, flat.data<int32_t>(), flat.count(), d, out);
  return decode_result(out);
}

// prefill_work(req_meta i32[B*8], flat i32, group, columns, key_tokens,
//              slots_per_head, min_tiles, decode_max_columns, block_size,
//              shared_prefix, num_kv_heads, xcds, order)
//   -> (units i32 [n, 8], jobs i32 [m, 8], partial slots, mean key tiles per
//       unit, most columns of a merge job)
// shared_prefix (0/1) enables the shared-prefix spans; xcds > 1 orders the
// units per XCD for num_kv_heads kv heads (padding records included) by the
// order policy (kernel fact 22's values).
PyObject* prefill_work(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!want_args(nargs, 13, "prefill_work")) return nullptr;
  Buf meta(args[0], false, 4, "req_meta"), flat(args[1], false, 4, "flat");
  if (!meta.ok() || !flat.ok()) return nullptr;
  Requests q;
  if (!requests_of(meta, &q, "prefill_work")) return nullptr;
  PrefillParams p;
  int64_t spans = 0;
  int64_t* fields[] = {&p.group, &p.columns, &p.key_tokens, &p.slots_per_head, &p.min_tiles, &p.max_cols,
                       &p.block_size, &spans, &p.kv_heads, &p.xcds, &p.order};
  for (int i = 0; i < 11; ++i)
    if (!as_i64(args[2 + i], fields[i])) return nullptr;
  if (p.group <= 0 || p.columns <= 0 || p.key_tokens <= 0 || p.min_tiles <= 0 || p.block_size <= 0 ||
      p.kv_heads <= 0 || p.xcds < 0 || p.order < 0 || p.order > 2) {
    PyErr_SetString(PyExc_ValueError, "prefill_work: inconsistent arguments");
    return nullptr;
  }
  if (!tables_fit(q, flat.count())) {
    PyErr_SetString(PyExc_ValueError, "prefill_work: req_meta names tables past the flat array");
    return nullptr;
  }
  p.ids = flat.data<int32_t>();
  p.spans = spans != 0;
  p.resident_per_head = p.slots_per_head;
  PrefillLists out;
  build_prefill(q, p, out);
  return prefill_result(out);
}

// layer_work(req_meta i32[B*8], flat i32, kernel facts (int64 array, 23
//            entries, below), cost4, wide_max_tiles)
//   -> (col_tiles, prefill_waves, decode result or None, prefill result or None)
//
// Everything one layer shape needs in one call: the decode kernel's column
// tiles per wave and the prefill workgroup shape are chosen for this step
// (unless forced), then both work lists are built.  Kernel facts:
//   0 group, 1 num_kv_heads, 2 block_size, 3 prefill columns (0: no prefill
//   kernel), 4 prefill key tokens, 5 split prefill (0/1), 6 forced col tiles
//   (0: choose), 7 forced prefill waves (0: choose), 8 widest col tiles built,
//   9 8-wave prefill built (0/1), 10 resident decode waves at 1 col tile,
//   11 tile tokens at 1, 12 resident at 4, 13 tile tokens at 4, 14 resident
//   4-wave prefill workgroups, 15 resident 8-wave ones, 16 max tokens per
//   decode wave (0: no cap), 17 decode max columns, 18 min units per wave,
//   19 prefill min tiles, 20 shared-prefix spans (0/1), 21 the device's XCDs
//   (0: no per-XCD order of the prefill grid), 22 per-XCD order (0: grouped
//   when its simulated packing is no slower, 1: grouped, 2: plain), 23
//   resident workgroups of the workgroup-split decode kernel (0: never), 24
//   its waves per workgroup.
constexpr int kKernelFacts = 25;

// One layer shape's plan: the choices and the lists of both kernels.
struct LayerPlan {
  int64_t ctw = 1, waves = 4;
  bool has_dec = false, has_pre = false;
  DecodeLists dec;
  PrefillLists pre;
  void reset() {
    ctw = 1;
    waves = 4;
    has_dec = has_pre = false;
    dec.reset();
    pre.reset();
  }
};

const char* plan_layer(const Requests& q, const int32_t* ids, int64_t nflat, const int64_t* k, double cost4,
                       double wide_max, LayerPlan& out);

PyObject* layer_work(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!want_args(nargs, 5, "layer_work")) return nullptr;
  Buf meta(args[0], false, 4, "req_meta"), flat(args[1], false, 4, "flat"), kf(args[2], false, 8, "facts");
  if (!meta.ok() || !flat.ok() || !kf.ok()) return nullptr;
  const double cost4 = PyFloat_AsDouble(args[3]), wide_max = PyFloat_AsDouble(args[4]);
  if (PyErr_Occurred()) return nullptr;
  Requests q;
  if (!requests_of(meta, &q, "layer_work")) return nullptr;
  if (kf.count() != kKernelFacts) {
    PyErr_Format(PyExc_ValueError, "layer_work: expected %d kernel facts", kKernelFacts);
    return nullptr;
  }
  if (!tables_fit(q, flat.count())) {
    PyErr_SetString(PyExc_ValueError, "layer_work: req_meta names tables past the flat array");
    return nullptr;
  }
  LayerPlan plan;
  if (const char* err = plan_layer(q, flat.data<int32_t>(), flat.count(), kf.data<int64_t>(), cost4, wide_max, plan)) {
    PyErr_Format(PyExc_ValueError, "layer_work: %s", err);
    return nullptr;
  }
  PyObject* dec = plan.has_dec ? decode_result(plan.dec) : Py_NewRef(Py_None);
  PyObject* pre = plan.has_pre ? prefill_result(plan.pre) : Py_NewRef(Py_None);
  PyObject* result =
      (dec && pre) ? Py_BuildValue("(LLOO)", (long long)plan.ctw, (long long)plan.waves, dec, pre) : nullptr;
  Py_XDECREF(dec);
  Py_XDECREF(pre);
  return result;
}

// layer_work's body: the choices for this step, then both work lists.
// Returns an error message, or nullptr when ``out`` holds the plan.
const char* plan_layer(const Requests& q, const int32_t* ids, int64_t nflat, const int64_t* k, double cost4,
                       double wide_max, LayerPlan& out) {
  const int64_t group = k[0], hkv = k[1], bs = k[2], columns = k[3];
  const int64_t max_cols = columns > 0 ? k[17] : 0;
  if (group <= 0 || hkv <= 0 || bs <= 0) return "inconsistent arguments";
  out.reset();
  int64_t ctw = k[6] > 0 ? std::min(k[6], k[8]) : choose_col_tiles(q, group, max_cols, k[8], cost4);
  if (ctw != 4) ctw = 1;
  PrefillParams p{group, columns > 0 ? columns : 1, k[4] > 0 ? k[4] : 1, 0, k[19] > 0 ? k[19] : 1, max_cols};
  p.ids = ids;
  p.block_size = bs;
  p.spans = k[20] != 0;
  p.kv_heads = hkv;
  p.xcds = k[21];
  p.order = k[22];
  int64_t waves = 4;
  bool any_decode = false, any_prefill = false;
  for (int64_t r = 0; r < q.batch; ++r) {
    const bool wide = max_cols > 0 && q.q_len(r) * group > max_cols;
    any_decode |= !wide;
    any_prefill |= wide;
  }
  if (any_prefill) {
    if (k[7] > 0) {
      waves = (k[7] == 8 && k[9]) ? 8 : 4;
    } else {
      waves = choose_prefill_waves(q, p, k[5] ? k[14] / hkv : 0, k[9] != 0, wide_max);
    }
    p.resident_per_head = (waves == 8 ? k[15] : k[14]) / hkv;
    p.slots_per_head = k[5] ? p.resident_per_head : 0;
  }
  out.ctw = ctw;
  out.waves = waves;
  if (any_decode) {
    const int64_t unit = ctw == 4 ? k[13] : k[11];
    const int64_t max_units = (k[16] > 0 && unit > 0) ? std::max<int64_t>(1, k[16] / unit) : 0;
    DecodeParams d{group, ctw, max_cols, hkv, ctw == 4 ? k[12] : k[10], bs, k[18] > 0 ? k[18] : 4, max_units, unit,
                   k[23], k[24]};
    if (d.unit <= 0 || d.resident <= 0) return "missing decode kernel facts";
    build_decode(q, ids, nflat, d, out.dec);
    out.has_dec = true;
  }
  if (any_prefill) {
    build_prefill(q, p, out.pre);
    out.has_pre = true;
  }
  return nullptr;
}

// ---------------------------------------------------------------------------
// plan_step(flat i32, counts i64, computed i64, reserved i64, readonly i64,
//           q_lens i64, vis_off i64, vis_words i64, vis u32, num_blocks,
//           block_size, kernel facts i64 [n][25], cost4, wide_max_tiles,
//           out i32 (writable))
//   -> rule (int 1..6): a block-table rule fails (validate's codes);
//      (needed, None, None): ``out`` holds fewer than ``needed`` entries;
//      (used, (slots, req_meta, tables, vis offsets), shapes) otherwise.
//
// A whole step in one call: validate's rules, then stage's slots and
// records, the flat tables and ancestor rows, and layer_work for each of the
// n kernel-fact rows, all written into ``out`` (a pinned staging buffer),
// each part starting on a 16-entry (64-byte) boundary.  Offsets are in
// int32 entries; slots take two entries per token.  Per shape:
//   (col_tiles, prefill_waves, decode waves per head, largest share,
//    decode partial slots, decode merge jobs, decode merge columns,
//    prefill units, prefill merge jobs, prefill partial slots,
//    prefill merge columns, pieces, wave_first, jobs, units, prefill jobs,
//    decode pieces, decode waves per workgroup)
// with the five offsets -1 for an absent list.
// ---------------------------------------------------------------------------
std::vector<LayerPlan> g_layer_plans;

int64_t align16(int64_t n) { return (n + 15) & ~int64_t(15); }

PyObject* plan_step(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!want_args(nargs, 15, "plan_step")) return nullptr;
  Buf flat(args[0], false, 4, "flat"), counts(args[1], false, 8, "counts"), computed(args[2], false, 8, "computed"),
      reserved(args[3], false, 8, "reserved"), readonly(args[4], false, 8, "readonly"),
      q_lens(args[5], false, 8, "q_lens"), vis_off(args[6], false, 8, "vis_off"),
      vis_words(args[7], false, 8, "vis_words"), vis(args[8], false, 4, "vis");
  if (!flat.ok() || !counts.ok() || !computed.ok() || !reserved.ok() || !readonly.ok() || !q_lens.ok() ||
      !vis_off.ok() || !vis_words.ok() || !vis.ok())
    return nullptr;
  int64_t num_blocks = 0, bs = 0;
  if (!as_i64(args[9], &num_blocks) || !as_i64(args[10], &bs)) return nullptr;
  Buf kf(args[11], false, 8, "kernel facts");
  if (!kf.ok()) return nullptr;
  const double cost4 = PyFloat_AsDouble(args[12]), wide_max = PyFloat_AsDouble(args[13]);
  if (PyErr_Occurred()) return nullptr;
  Buf out(args[14], true, 4, "out");
  if (!out.ok()) return nullptr;
  const int64_t batch = counts.count();
  const int64_t* cnt = counts.data<int64_t>();
  const int64_t* ql = q_lens.data<int64_t>();
  int64_t total_blocks = 0, tokens = 0;
  for (int64_t r = 0; r < batch; ++r) {
    total_blocks += cnt[r];
    tokens += ql[r];
  }
  if (batch <= 0 || computed.count() != batch || reserved.count() != batch || readonly.count() != batch ||
      q_lens.count() != batch || vis_off.count() != batch || vis_words.count() != batch ||
      total_blocks != flat.count() || bs <= 0 || num_blocks <= 0 || num_blocks > INT32_MAX ||
      kf.count() % kKernelFacts != 0 || batch > INT32_MAX / kReqFields) {
    PyErr_SetString(PyExc_ValueError, "plan_step: inconsistent arguments");
    return nullptr;
  }
  const int32_t* ids = flat.data<int32_t>();
  int64_t bad = -1;
  const int rule = check_tables(ids, cnt, computed.data<int64_t>(), reserved.data<int64_t>(),
                                readonly.data<int64_t>(), batch, num_blocks, bs, &bad);
  if (rule != kTablesOk) return PyLong_FromLong(rule);
  // Offsets of the step's facts; the requests' records are staged first
  // into scratch (the planner reads them), then copied.
  const int64_t o_slots = 0, o_meta = align16(2 * tokens), o_tables = o_meta + align16(batch * kReqFields),
                o_vis = o_tables + align16(std::max<int64_t>(1, total_blocks));
  int64_t used = o_vis + align16(std::max<Py_ssize_t>(1, vis.count()));
  static std::vector<int32_t> meta;
  static std::vector<int64_t> slots;
  meta.resize((size_t)(batch * kReqFields));
  slots.resize((size_t)tokens);
  if (stage_rows(ids, cnt, computed.data<int64_t>(), ql, vis_off.data<int64_t>(), vis_words.data<int64_t>(), batch,
                 bs, slots.data(), meta.data()) != 0) {
    PyErr_SetString(PyExc_ValueError, "plan_step: a query position lies past its block table");
    return nullptr;
  }
  const int64_t nshapes = kf.count() / kKernelFacts;
  if ((int64_t)g_layer_plans.size() < nshapes) g_layer_plans.resize((size_t)nshapes);
  Requests q{meta.data(), batch};
  struct Offsets {
    int64_t pieces, first, jobs, units, pjobs;
  };
  std::vector<Offsets> offs((size_t)nshapes);
  for (int64_t s = 0; s < nshapes; ++s) {
    LayerPlan& plan = g_layer_plans[(size_t)s];
    if (const char* err = plan_layer(q, ids, total_blocks, kf.data<int64_t>() + s * kKernelFacts, cost4, wide_max,
                                     plan)) {
      PyErr_Format(PyExc_ValueError, "plan_step: %s", err);
      return nullptr;
    }
    Offsets& o = offs[(size_t)s];
    auto place = [&used](const std::vector<int32_t>& v, bool present) -> int64_t {
      if (!present || v.empty()) return -1;
      const int64_t at = used;
      used += align16((int64_t)v.size());
      return at;
    };
    o.pieces = place(plan.dec.pieces, plan.has_dec);
    o.first = place(plan.dec.first, plan.has_dec);
    o.jobs = place(plan.dec.jobs, plan.has_dec);
    o.units = place(plan.pre.units, plan.has_pre);
    o.pjobs = place(plan.pre.jobs, plan.has_pre);
  }
  if (used > out.count()) return Py_BuildValue("(LOO)", (long long)used, Py_None, Py_None);
  int32_t* dst = out.data<int32_t>();
  std::memcpy(dst + o_slots, slots.data(), (size_t)tokens * 8);
  std::memcpy(dst + o_meta, meta.data(), meta.size() * 4);
  std::memcpy(dst + o_tables, ids, (size_t)total_blocks * 4);
  std::memcpy(dst + o_vis, vis.data<int32_t>(), (size_t)vis.count() * 4);
  PyObject* shapes = PyTuple_New((Py_ssize_t)nshapes);
  if (shapes == nullptr) return nullptr;
  for (int64_t s = 0; s < nshapes; ++s) {
    const LayerPlan& plan = g_layer_plans[(size_t)s];
    const Offsets& o = offs[(size_t)s];
    auto put = [dst](const std::vector<int32_t>& v, int64_t at) {
      if (at >= 0) std::memcpy(dst + at, v.data(), v.size() * 4);
    };
    put(plan.dec.pieces, o.pieces);
    put(plan.dec.first, o.first);
    put(plan.dec.jobs, o.jobs);
    put(plan.pre.units, o.units);
    put(plan.pre.jobs, o.pjobs);
    const DecodeLists& d = plan.dec;
    const PrefillLists& p = plan.pre;
    PyObject* one = Py_BuildValue(
        "(LLLLLLLLLLLLLLLLLL)", (long long)plan.ctw, (long long)plan.waves, (long long)(plan.has_dec ? d.waves : 0),
        (long long)(plan.has_dec ? d.per_wave : 0), (long long)(plan.has_dec ? d.slots : 0),
        (long long)(plan.has_dec ? (int64_t)d.jobs.size() / kMergeFields : 0),
        (long long)(plan.has_dec ? d.merge_cols : 1),
        (long long)(plan.has_pre ? (int64_t)p.units.size() / kPrefillFields : 0),
        (long long)(plan.has_pre ? (int64_t)p.jobs.size() / kMergeFields : 0), (long long)(plan.has_pre ? p.slots : 0),
        (long long)(plan.has_pre ? p.merge_cols : 1), (long long)o.pieces, (long long)o.first, (long long)o.jobs,
        (long long)o.units, (long long)o.pjobs,
        (long long)(plan.has_dec ? (int64_t)d.pieces.size() / kPieceFields : 0),
        (long long)(plan.has_dec ? d.group_waves : 1));
    if (one == nullptr) {
      Py_DECREF(shapes);
      return nullptr;
    }
    PyTuple_SET_ITEM(shapes, (Py_ssize_t)s, one);
  }
  PyObject* result = Py_BuildValue("(L(LLLL)N)", (long long)used, (long long)o_slots, (long long)o_meta,
                                   (long long)o_tables, (long long)o_vis, shapes);
  return result;
}

// ---------------------------------------------------------------------------
// compact_pairs(requests, num_blocks, block_size, keep_equal) ->
//   (rule, request index, moved counts i64[R], src i64[n], dst i64[n])
//
// Each request is a mapping with PagedKVCache.compact's arguments
// (block_ids, num_computed_tokens, num_query_tokens,
// num_reserved_query_tokens, retained_query_indices and optionally
// num_readonly_prefix_blocks).  Rules in the reference's order
// (paged_cache.py:276-302); the first failing one is reported:
//   1 counts not non-negative ints          (ValueError)
//   2 reserved < queries                     (ValueError)
//   3 retained index not a non-negative int  (ValueError)
//   4 retained indices not unique            (ValueError)
//   5 retained index >= queries              (KVCacheError)
//   6 table size != blocks the reserve needs (KVCacheError)
//   7 an id not an int in [0, num_blocks)    (KVCacheError)
//   8 an id repeated in the table            (KVCacheError)
//   9 readonly blocks past the computed prefix (KVCacheError)
//  10 two requests write the same slot       (KVCacheError)
//  11 a request is missing an argument       (TypeError)
// moved[r] counts the pairs with src != dst; those with src == dst are
// dropped from src/dst unless keep_equal is true.
// ---------------------------------------------------------------------------
PyObject* compact_pairs(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!want_args(nargs, 4, "compact_pairs")) return nullptr;
  int64_t num_blocks = 0, bs = 0;
  if (!as_i64(args[1], &num_blocks) || !as_i64(args[2], &bs)) return nullptr;
  const int keep_equal = PyObject_IsTrue(args[3]);
  if (keep_equal < 0) return nullptr;
  if (bs <= 0 || num_blocks <= 0 || num_blocks > INT32_MAX) {
    PyErr_SetString(PyExc_ValueError, "compact_pairs: inconsistent arguments");
    return nullptr;
  }
  PyObject* reqs = PySequence_Fast(args[0], "compact requests must be a sequence");
  if (reqs == nullptr) return nullptr;
  const Py_ssize_t nreq = PySequence_Fast_GET_SIZE(reqs);
  BlockScratch& s = g_compact_scratch;
  s.reserve(num_blocks);
  std::vector<int64_t> src, dst, moved((size_t)nreq, 0);
  std::vector<int64_t> ret;
  static std::vector<int32_t> vals;  // one request's block ids
  const PrevFlatten& proven = g_prev_flatten;
  int rule = 0;
  Py_ssize_t r = 0;
  for (; r < nreq && rule == 0; ++r) {
    PyObject* req = PySequence_Fast_GET_ITEM(reqs, r);
    if (!PyDict_Check(req)) {
      rule = 11;
      break;
    }
    int64_t cnt[4] = {0, 0, 0, 0};
    for (int k = 0; k < 4 && rule == 0; ++k) {
      PyObject* v = PyDict_GetItem(req, g_compact_keys[1 + k]);
      if (v == nullptr) {
        if (k == 3) continue;  // num_readonly_prefix_blocks defaults to 0
        rule = 11;
        break;
      }
      int overflow = 0;
      cnt[k] = PyLong_CheckExact(v) ? PyLong_AsLongLongAndOverflow(v, &overflow) : -1;
      if (cnt[k] < 0 || overflow) rule = 1;
    }
    if (rule) break;
    const int64_t computed = cnt[0], queries = cnt[1], reserved = cnt[2], readonly = cnt[3];
    if (reserved < queries) { rule = 2; break; }
    PyObject* ids_obj = PyDict_GetItem(req, g_compact_keys[0]);
    PyObject* ret_obj = PyDict_GetItem(req, g_compact_keys[5]);
    if (ids_obj == nullptr || ret_obj == nullptr) { rule = 11; break; }
    PyObject* rseq = PySequence_Fast(ret_obj, "retained query indices must be a sequence");
    if (rseq == nullptr) { Py_DECREF(reqs); return nullptr; }
    const Py_ssize_t nret = PySequence_Fast_GET_SIZE(rseq);
    ret.assign((size_t)nret, 0);
    for (Py_ssize_t i = 0; i < nret && rule == 0; ++i) {
      PyObject* v = PySequence_Fast_ITEMS(rseq)[i];
      int overflow = 0;
      ret[(size_t)i] = PyLong_CheckExact(v) ? PyLong_AsLongLongAndOverflow(v, &overflow) : -1;
      if (ret[(size_t)i] < 0 || overflow) rule = 3;
    }
    Py_DECREF(rseq);
    if (rule) break;
    {
      std::vector<int64_t> sorted(ret);
      std::sort(sorted.begin(), sorted.end());
      if (std::adjacent_find(sorted.begin(), sorted.end()) != sorted.end()) { rule = 4; break; }
    }
    bool tail_ok = true;
    for (int64_t x : ret) tail_ok &= x < queries;
    if (!tail_ok) { rule = 5; break; }
    const int64_t required = (computed + reserved + bs - 1) / bs;
    const int32_t* ids = nullptr;
    Py_ssize_t n = 0;
    // The very tuple this step's metadata listed for some request (looked
    // for from this request's index on: a step's compacts usually come in
    // table order), whose ids the step's table check proved in range and
    // unique in the row.
    int64_t row = -1;
    if (proven.proven_blocks == num_blocks && PyTuple_CheckExact(ids_obj)) {
      const size_t nrows = proven.rows.size();
      for (size_t k = 0; k < nrows && row < 0; ++k) {
        const size_t i = ((size_t)r + k) % nrows;
        if (proven.rows[i] == ids_obj) row = (int64_t)i;
      }
    }
    if (row >= 0) {
      n = PyTuple_GET_SIZE(ids_obj);
      ids = proven.values.data() + proven.offsets[(size_t)row];
      if (n != required) { rule = 6; break; }
    } else {
      PyObject* tseq = PySequence_Fast(ids_obj, "block_ids must be a sequence");
      if (tseq == nullptr) { Py_DECREF(reqs); return nullptr; }
      n = PySequence_Fast_GET_SIZE(tseq);
      PyObject** items = PySequence_Fast_ITEMS(tseq);
      if (n != required) {
        Py_DECREF(tseq);
        rule = 6;
        break;
      }
      vals.resize((size_t)n);
      bool ids_ok = true;
      for (Py_ssize_t i = 0; i < n && ids_ok; ++i) {
        int overflow = 0;
        const long long v = PyLong_CheckExact(items[i]) ? PyLong_AsLongLongAndOverflow(items[i], &overflow) : -1;
        ids_ok = overflow == 0 && v >= 0 && v < num_blocks;
        vals[(size_t)i] = (int32_t)v;
      }
      Py_DECREF(tseq);
      if (!ids_ok) { rule = 7; break; }
      const uint32_t seen = s.next_epoch();
      bool unique = true;
      for (Py_ssize_t i = 0; i < n && unique; ++i) {
        BlockRecord& b = s.rec[(size_t)vals[(size_t)i]];
        unique = b.epoch != seen;
        b.epoch = seen;
      }
      if (!unique) { rule = 8; break; }
      ids = vals.data();
    }
    if (readonly * bs > computed) { rule = 9; break; }
    auto slot_of = [&](int64_t pos) -> int64_t {
      const int64_t lb = pos / bs;
      return (int64_t)ids[lb] * bs + (pos - lb * bs);
    };
    for (Py_ssize_t i = 0; i < nret; ++i) {
      const int64_t from = slot_of(computed + ret[(size_t)i]);
      const int64_t to = slot_of(computed + i);
      if (from != to || keep_equal) {
        src.push_back(from);
        dst.push_back(to);
      }
      moved[(size_t)r] += from != to;
    }
  }
  Py_DECREF(reqs);
  if (rule == 0 && dst.size() > 1) {
    std::vector<int64_t> sorted(dst);
    std::sort(sorted.begin(), sorted.end());
    if (std::adjacent_find(sorted.begin(), sorted.end()) != sorted.end()) {
      rule = 10;
      r = nreq;
    }
  }
  if (rule) return Py_BuildValue("(inOOO)", rule, r, Py_None, Py_None, Py_None);
  int64_t *m = nullptr, *so = nullptr, *d = nullptr;
  PyObject* m_obj = new_array<int64_t>(nreq, &m);
  PyObject* s_obj = new_array<int64_t>((Py_ssize_t)src.size(), &so);
  PyObject* d_obj = new_array<int64_t>((Py_ssize_t)dst.size(), &d);
  PyObject* result = nullptr;
  if (m_obj && s_obj && d_obj) {
    std::copy(moved.begin(), moved.end(), m);
    std::copy(src.begin(), src.end(), so);
    std::copy(dst.begin(), dst.end(), d);
    result = Py_BuildValue("(inOOO)", 0, (Py_ssize_t)-1, m_obj, s_obj, d_obj);
  }
  Py_XDECREF(m_obj);
  Py_XDECREF(s_obj);
  Py_XDECREF(d_obj);
  return result;
}

// ---------------------------------------------------------------------------
// attend(fn, plan, q, qs0, qs1, k, ks0, ks1, v, vs0, vs1, key_pool, value_pool,
//        out, os0, os1, scale, stream) -> status
//
// Calls the HIP library's lvamd_paged_attention (fn: its address, handed over
// once by the Python loader) with plain integers: the per-layer call of the
// backend's forward, without ctypes' per-argument conversion.  Pointers are
// ints (0 for NULL); the status is the library's.
// ---------------------------------------------------------------------------
typedef int (*AttendFn)(const void*, const void*, int64_t, int64_t, const void*, int64_t, int64_t, const void*,
                        int64_t, int64_t, void*, void*, void*, int64_t, int64_t, float, void*);

PyObject* attend(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!want_args(nargs, 18, "attend")) return nullptr;
  int64_t v[18];
  for (int i = 0; i < 18; ++i) {
    if (i == 16) continue;
    v[i] = (int64_t)PyLong_AsLongLong(args[i]);
  }
  const double scale = PyFloat_AsDouble(args[16]);
  if (PyErr_Occurred()) return nullptr;
  if (v[0] == 0 || v[1] == 0) {
    PyErr_SetString(PyExc_ValueError, "attend: null function or plan");
    return nullptr;
  }
  auto ptr = [&](int i) { return reinterpret_cast<void*>((intptr_t)v[i]); };
  const AttendFn fn = reinterpret_cast<AttendFn>((intptr_t)v[0]);
  const int status = fn(ptr(1), ptr(2), v[3], v[4], ptr(5), v[6], v[7], ptr(8), v[9], v[10], ptr(11), ptr(12), ptr(13),
                        v[14], v[15], (float)scale, ptr(17));
  return PyLong_FromLong(status);
}

// ---------------------------------------------------------------------------
// attend_tensors(shape, key_pool, value_pool, out, q, k, v, scale) -> status,
// or kNotFast
//
// forward's common case in one call: reads each tensor's dtype, device,
// shape, strides and data pointer itself and, when every rule of the fast
// path holds (the layer's shapes, its dtype and device, contiguous 16-byte
// rows), calls lvamd_paged_attention.  Any other tensor returns kNotFast and
// the caller takes its general path, which raises the reference's message
// for the first broken rule.  shape = (fn, plan, out_s0, out_s1, dtype
// object, device index, element size, tokens, query heads, kv heads, head
// size, raw-stream getter), made once per layer shape and step; the pools
// are the layer's (fixed for a cache) and out its output rows.
// ---------------------------------------------------------------------------
constexpr long kNotFast = 1 << 30;
PyObject* g_str_dtype = nullptr;
PyObject* g_str_get_device = nullptr;
PyObject* g_str_shape = nullptr;
PyObject* g_str_stride = nullptr;
PyObject* g_str_data_ptr = nullptr;

// 1: the tensor fits (facts filled), 0: it does not, -1: a Python error.
int tensor_facts(PyObject* t, PyObject* dtype, long device, int64_t n0, int64_t n1, int64_t n2, int64_t es,
                 int64_t* ptr, int64_t* s0, int64_t* s1) {
  PyObject* dt = PyObject_GetAttr(t, g_str_dtype);
  if (dt == nullptr) return -1;
  const bool same_dtype = dt == dtype;
  Py_DECREF(dt);
  if (!same_dtype) return 0;
  PyObject* dev = PyObject_CallMethodNoArgs(t, g_str_get_device);
  if (dev == nullptr) return -1;
  const long d = PyLong_AsLong(dev);
  Py_DECREF(dev);
  if (d == -1 && PyErr_Occurred()) return -1;
  if (d != device) return 0;
  PyObject* shape = PyObject_GetAttr(t, g_str_shape);
  if (shape == nullptr) return -1;
  bool fits = PyTuple_Check(shape) && PyTuple_GET_SIZE(shape) == 3;
  if (fits) {
    const int64_t want[3] = {n0, n1, n2};
    for (int i = 0; i < 3 && fits; ++i) fits = PyLong_AsLongLong(PyTuple_GET_ITEM(shape, i)) == want[i];
  }
  Py_DECREF(shape);
  if (PyErr_Occurred()) return -1;
  if (!fits) return 0;
  PyObject* stride = PyObject_CallMethodNoArgs(t, g_str_stride);
  if (stride == nullptr) return -1;
  int64_t st[3] = {0, 0, 0};
  fits = PyTuple_Check(stride) && PyTuple_GET_SIZE(stride) == 3;
  for (int i = 0; i < 3 && fits; ++i) st[i] = PyLong_AsLongLong(PyTuple_GET_ITEM(stride, i));
  Py_DECREF(stride);
  if (PyErr_Occurred()) return -1;
  if (!fits || st[2] != 1 || ((st[0] * es) & 15) || ((st[1] * es) & 15)) return 0;
  PyObject* dp = PyObject_CallMethodNoArgs(t, g_str_data_ptr);
  if (dp == nullptr) return -1;
  const int64_t p = PyLong_AsLongLong(dp);
  Py_DECREF(dp);
  if (PyErr_Occurred()) return -1;
  if (p & 15) return 0;
  *ptr = p;
  *s0 = st[0];
  *s1 = st[1];
  return 1;
}

PyObject* attend_tensors(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (!want_args(nargs, 8, "attend_tensors")) return nullptr;
  PyObject* b = args[0];
  if (!PyTuple_Check(b) || PyTuple_GET_SIZE(b) != 12) {
    PyErr_SetString(PyExc_ValueError, "attend_tensors: shape facts must be a 12-tuple");
    return nullptr;
  }
  int64_t f[12];
  for (int i = 0; i < 12; ++i) {
    if (i == 4 || i == 11) continue;
    f[i] = (int64_t)PyLong_AsLongLong(PyTuple_GET_ITEM(b, i));
  }
  const int64_t k_pool = (int64_t)PyLong_AsLongLong(args[1]);
  const int64_t v_pool = (int64_t)PyLong_AsLongLong(args[2]);
  const int64_t out = (int64_t)PyLong_AsLongLong(args[3]);
  if (PyErr_Occurred()) return nullptr;
  PyObject* dtype = PyTuple_GET_ITEM(b, 4);
  const long device = (long)f[5];
  const int64_t es = f[6], tokens = f[7], hq = f[8], hkv = f[9], d = f[10];
  int64_t qp, qs0, qs1, kp, ks0, ks1, vp, vs0, vs1;
  int r = tensor_facts(args[4], dtype, device, tokens, hq, d, es, &qp, &qs0, &qs1);
  if (r == 1) r = tensor_facts(args[5], dtype, device, tokens, hkv, d, es, &kp, &ks0, &ks1);
  if (r == 1) r = tensor_facts(args[6], dtype, device, tokens, hkv, d, es, &vp, &vs0, &vs1);
  if (r < 0) return nullptr;
  if (r == 0) return PyLong_FromLong(kNotFast);
  const double scale = PyFloat_AsDouble(args[7]);
  if (PyErr_Occurred()) return nullptr;
  PyObject* dev = PyLong_FromLong(device);
  if (dev == nullptr) return nullptr;
  PyObject* stream = PyObject_CallOneArg(PyTuple_GET_ITEM(b, 11), dev);
  Py_DECREF(dev);
  if (stream == nullptr) return nullptr;
  const int64_t sp = PyLong_AsLongLong(stream);
  Py_DECREF(stream);
  if (PyErr_Occurred()) return nullptr;
  if (f[0] == 0 || f[1] == 0) {
    PyErr_SetString(PyExc_ValueError, "attend_tensors: null function or plan");
    return nullptr;
  }
  auto ptr = [](int64_t v) { return reinterpret_cast<void*>((intptr_t)v); };
  const AttendFn fn = reinterpret_cast<AttendFn>((intptr_t)f[0]);
  const int status = fn(ptr(f[1]), ptr(qp), qs0, qs1, ptr(kp), ks0, ks1, ptr(vp), vs0, vs1, ptr(k_pool), ptr(v_pool),
                        ptr(out), f[2], f[3], (float)scale, ptr(sp));
  return PyLong_FromLong(status);
}

PyMethodDef kMethods[] = {
    {"flatten", (PyCFunction)(void (*)(void))flatten, METH_FASTCALL, "int sequences -> (flat, counts int64, status)"},
    {"validate", (PyCFunction)(void (*)(void))validate, METH_FASTCALL, "block-table rules -> (rule, request)"},
    {"layouts", (PyCFunction)(void (*)(void))layouts, METH_FASTCALL, "query layouts -> lengths and ancestor bit rows"},
    {"metadata", (PyCFunction)(void (*)(void))metadata, METH_FASTCALL, "metadata fields -> rule or (fields, facts)"},
    {"stage", (PyCFunction)(void (*)(void))stage, METH_FASTCALL, "slots and per-request records into buffers"},
    {"decode_work", (PyCFunction)(void (*)(void))decode_work, METH_FASTCALL, "stream-K decode pieces"},
    {"prefill_work", (PyCFunction)(void (*)(void))prefill_work, METH_FASTCALL, "prefill units and merge jobs"},
    {"layer_work", (PyCFunction)(void (*)(void))layer_work, METH_FASTCALL, "one layer shape's choices and lists"},
    {"plan_step", (PyCFunction)(void (*)(void))plan_step, METH_FASTCALL, "a whole step, staged into one buffer"},
    {"counts", (PyCFunction)(void (*)(void))counts, METH_FASTCALL, "how the planner's calls were served"},
    {"compact_pairs", (PyCFunction)(void (*)(void))compact_pairs, METH_FASTCALL, "compact rules and moved slot pairs"},
    {"attend", (PyCFunction)(void (*)(void))attend, METH_FASTCALL, "one layer's lvamd_paged_attention call"},
    {"attend_tensors", (PyCFunction)(void (*)(void))attend_tensors, METH_FASTCALL,
     "forward's fast path: tensor rules and the lvamd_paged_attention call"},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_lvamd_host", "Native host-side step planner of the paged-KV backend.",
                       -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__lvamd_host(void) {
  g_parent_indices = PyUnicode_InternFromString("parent_indices");
  if (g_parent_indices == nullptr) return nullptr;
  g_str_dtype = PyUnicode_InternFromString("dtype");
  g_str_get_device = PyUnicode_InternFromString("get_device");
  g_str_shape = PyUnicode_InternFromString("shape");
  g_str_stride = PyUnicode_InternFromString("stride");
  g_str_data_ptr = PyUnicode_InternFromString("data_ptr");
  if (!g_str_dtype || !g_str_get_device || !g_str_shape || !g_str_stride || !g_str_data_ptr) return nullptr;
  static const char* kCompactKeys[6] = {"block_ids", "num_computed_tokens", "num_query_tokens",
                                        "num_reserved_query_tokens", "num_readonly_prefix_blocks",
                                        "retained_query_indices"};
  for (int i = 0; i < 6; ++i) {
    g_compact_keys[i] = PyUnicode_InternFromString(kCompactKeys[i]);
    if (g_compact_keys[i] == nullptr) return nullptr;
  }
  return PyModule_Create(&kModule);
}
