// _pkvhost: the per-entry host work of one ModelRunner iteration, in C++ (a CPython extension).
//
// A batch is a tuple of BatchEntry objects (the reference's or this package's: anything with
// seq_id, token_ids, positions, block_table and logits_index). Walking them in Python costs about
// a microsecond per entry and attribute; here one pass reads each entry once. Functions:
//
//   gather(entries, block_size, tokens, positions, slots, lengths, contexts, logits[, stats])
//       -> (total, problem, entry, position)
//       Flattens token ids and positions, computes every slot with the reference's rule
//       (runner.py:149-159: block_table[p // B] * B + p % B with Python's floor division and a
//       negative index counting from the table's end), and per entry its token count, context
//       length (positions[-1] + 1) and the flat row of its logits (-1 when it asks for none).
//       The first slot that cannot be formed is reported, not raised, so the caller can check
//       token ids and positions first, in the reference's order: problem 1 = a position past
//       the table (the reference's ValueError), 2 = a negative index before its start
//       (IndexError). Returns total = -(tokens needed), writing nothing, when the token buffers
//       are too small. The optional int64 `stats` buffer (>= 9 entries) receives what the
//       caller validates and sizes, so it needs no pass of its own: [min token, max token, min
//       position, max position, min slot, max slot, min context, 1 if two single-token entries'
//       tables start with the same block id else 0, max context] (slots of unformed positions
//       count as -1).
//   prefix_order_rows(rows, lengths, host, held_len, lead, min_rows, out) -> bool
//       The row order that puts decode entries sharing their first `lead` blocks next to each
//       other (runner.shared_prefix_order), written to the int64 buffer `out` (>= one entry per
//       row); False (out untouched) when no such run would change. Read from
//       the block-table arena after its update: entry e has lengths[e] tokens and its table in
//       arena row rows[e] (held_len[rows[e]] entries of host[rows[e]]), so no block id is
//       converted from a Python object.
//   arena_update(entries, row_of, key_of, held_len, held_obj, last_use, host, step, rows, index,
//                values) -> (changed entries, changed rows) | (-1, longest) | (-2, needed)
//       The block-table arena's step (tables.BlockTableArena.update): a row per entry (claiming the
//       least recently used row for a new sequence), and the flat indices and values of the
//       table entries that differ from what each row holds. Asks for a larger arena, before
//       changing anything, when the batch needs more rows or a wider table than it has.
//       held_obj keeps, per row, the tuple it was last filled from: a scheduler rebuilds each
//       table tuple from the same int objects every step, so an unchanged table compares equal
//       by identity (its pointer array against the held one's, 16 at a time) without converting
//       a single id; ids that are other objects are converted and compared with the mirror.
//   CopyQueue(num_blocks)
//       A runner's queued copy-on-write copies. push(src, dst) checks and queues one copy (the
//       runner's copy_block); groups() gives the sizes of the consecutive groups that may each
//       run as one concurrent pkv_copy_blocks launch (ops.independent_groups: a copy starts a
//       new group when it reads a block an earlier copy of the group writes, or writes a block
//       an earlier copy of the group reads or writes); flush(...) sends the pairs to the device
//       and launches one pkv_copy_blocks per group; clear() and items() drop and list them.
//   exclusive_writes(rows, contexts, host, block_size, marks[, tiles, partition]) -> bool
//       Whether a batch of single-token entries at their last positions (entry e: arena row
//       rows[e], context contexts[e], so it writes position contexts[e] - 1) may append inside
//       the attention call: False when a tile of the plan (int32 [n, 4] records over planner
//       rows, the entries' order here; `partition` keys per partition) covers an entry's own
//       position, since only the row pass appends; else True when each written block occurs
//       exactly once among the blocks
//       every entry reads (host[rows[e]][0 .. ceil(contexts[e] / B))), which is its own writer's
//       entry for that position. Otherwise some row reads a slot another row (or its own row,
//       through a repeated table entry) writes in the same step, and only an append that
//       completes before attention reads it as the reference does (runner.py:195-212). `marks`
//       is a uint8 buffer with one zero per pool block (small enough to stay in the L1 cache for
//       tens of thousands of blocks); it is left all zero.
//   bind(plan_batch, paged_attention, paged_attention_append, copy_blocks, rms_norm, silu_mul,
//        rope_append, memcpy_async[, gather_rows, greedy_tokens, get_device, set_device,
//        event_create, event_record, event_synchronize, event_destroy, append])
//       Takes the addresses of those libpkv.so entry points (include/pkv.h), so the calls below
//       reach the library without ctypes' per-argument conversions, and of hipMemcpyAsync,
//       hipGetDevice, hipSetDevice and hipEventCreateWithFlags / Record / Synchronize / Destroy
//       as the HIP runtime that libpkv.so is linked against exports them.
//   event_create(device) -> int, event_destroy(event)
//       A timing-free HIP event on `device` as an integer handle (for stage), and its release.
//   forward(fields, layers, eps, scale) -> None
//       One ModelRunner iteration's forward pass (the reference's runner.py:189-227 with
//       model.py:243-264), every launch enqueued from here on `stream` with the device made
//       current for the call: the embedding rows (pkv_gather_rows), per layer RMSNorm, the QKV
//       product, RoPE + append, paged attention, the output product with its residual add fused
//       into the next norm, the [gate | up] product, the SwiGLU gate and the down product; then
//       the logits rows, their product with the tied embedding, and greedy sampling when an
//       output address is given. The products are rocBLAS sgemm calls (the rocBLAS the process
//       has loaded, one handle per device, used by one forward pass at a time). `fields` holds
//       the integers of the Field enum below (addresses, sizes, the attention plan); `layers`
//       one tuple of six weight addresses per layer (attn_norm, qkv, out_proj, ffn_norm,
//       [gate | up], down). Raises RuntimeError naming the first step that failed.
//   stage(parts64, parts32, host, device_address, stream[, event]) -> list of byte offsets | None
//       A runner call's metadata transfer: the int64 arrays of the list parts64, then the int32
//       arrays of parts32, packed back to back into the pinned uint8 buffer `host` and copied to
//       device_address with one hipMemcpyAsync on `stream`. With an event (event_create), it
//       first waits for the event (the previous copy out of `host` has finished) and records it
//       after the copy. Returns each part's byte offset, or None (nothing written) when `host` is
//       too small; the caller keeps the device buffer at least as large as `host`.
//   plan(query_seq, query_positions | None, tables, contexts, block_size, num_heads, head_dim,
//        kv_dtype, partition_size, min_tile_rows, rows, tiles, merge, counts, launch) -> int
//       pkv_plan_batch on NumPy buffers; returns its PKV_* code.
//   paged_attention(...), paged_attention_append(...), copy_blocks(...), rms_norm(...),
//   silu_mul(...), rope_append(...), append(...) -> int
//       The entry points of the same names, with every pointer, stream and handle passed as a
//       Python int (0 for NULL) in the order of their C declarations; returns the PKV_* code.
//
// Buffers are NumPy arrays passed through the buffer protocol (C-contiguous, of the stated
// element type; writable where written); nothing here allocates Python-visible memory besides
// the returned lists.
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <structmember.h>
#if PY_VERSION_HEX < 0x030C0000
#include <longintrepr.h>
#endif

#include <dlfcn.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_set>
#include <vector>

#include "pkv.h"

namespace {

// A writable C-contiguous buffer of T, released on scope exit.
template <typename T>
class Buf {
 public:
  Buf() { view_.obj = nullptr; }
  ~Buf() {
    if (view_.obj != nullptr) PyBuffer_Release(&view_);
  }
  bool get(PyObject* obj, const char* what, bool writable = true) {
    const int flags = (writable ? PyBUF_WRITABLE : 0) | PyBUF_C_CONTIGUOUS | PyBUF_FORMAT;
    if (PyObject_GetBuffer(obj, &view_, flags) != 0) return false;
    if (view_.itemsize != static_cast<Py_ssize_t>(sizeof(T))) {
      PyErr_Format(PyExc_TypeError, "%s must hold %d-byte integers", what, static_cast<int>(sizeof(T)));
      return false;
    }
    return true;
  }
  T* data() const { return static_cast<T*>(view_.buf); }
  Py_ssize_t size() const { return view_.len / view_.itemsize; }
  Py_ssize_t dim(int i) const { return view_.ndim > i ? view_.shape[i] : 1; }
  int ndim() const { return view_.ndim; }

 private:
  Py_buffer view_;
};

// Interned attribute names.
PyObject* s_seq_id;
PyObject* s_token_ids;
PyObject* s_positions;
PyObject* s_block_table;
PyObject* s_logits_index;

// One attribute of the batch entries, read for a whole walk over them. For a class that keeps
// the attribute in a __slots__ slot (BatchEntry is a slotted frozen dataclass) and uses the
// generic attribute lookup, the slot's member descriptor gives its offset in the object, and the
// value is read there: what getattr returns for that class, without the descriptor call (about
// a fifth of the time per read). Objects of any other class go through PyObject_GetAttr.
class EntryField {
 public:
  explicit EntryField(PyObject* name) : name_(name) {}
  // A new reference, or null with an exception set.
  PyObject* get(PyObject* obj) {
    PyTypeObject* type = Py_TYPE(obj);
    if (type != type_) resolve(type);
    if (offset_ >= 0) {
      PyObject* value = *reinterpret_cast<PyObject**>(reinterpret_cast<char*>(obj) + offset_);
      if (value != nullptr) {
        Py_INCREF(value);
        return value;
      }
    }
    return PyObject_GetAttr(obj, name_);  // an unset slot raises AttributeError here
  }

 private:
  void resolve(PyTypeObject* type) {
    type_ = type;
    offset_ = -1;
    if (type->tp_getattro != PyObject_GenericGetAttr) return;
    PyObject* descr = _PyType_Lookup(type, name_);  // borrowed
    if (descr == nullptr || Py_TYPE(descr) != &PyMemberDescr_Type) return;
    const PyMemberDef* member = reinterpret_cast<PyMemberDescrObject*>(descr)->d_member;
    if (member->type == T_OBJECT_EX && (member->flags & READ_RESTRICTED) == 0) offset_ = member->offset;
  }

  PyObject* name_;
  PyTypeObject* type_ = nullptr;
  Py_ssize_t offset_ = -1;
};

// A sequence attribute as a fast sequence (a new reference), or null with an exception set.
PyObject* fast_attr(PyObject* obj, EntryField& field) {
  PyObject* value = field.get(obj);
  if (value == nullptr) return nullptr;
  PyObject* fast = PySequence_Fast(value, "a batch entry field must be a sequence");
  Py_DECREF(value);
  return fast;
}

// An int's value. Exact ints of at most one digit (|v| < 2**30: every block id, slot and
// position of a pool) are read from the object, in the layout of CPython before 3.12
// (longintrepr.h); anything else goes through PyLong_AsLongLong, which raises for non-ints.
inline bool as_i64(PyObject* v, int64_t* out) {
#if PY_VERSION_HEX < 0x030C0000
  if (PyLong_CheckExact(v)) {
    const Py_ssize_t size = Py_SIZE(v);
    if (size == 0) {
      *out = 0;
      return true;
    }
    if (size == 1 || size == -1) {
      const int64_t digit = reinterpret_cast<PyLongObject*>(v)->ob_digit[0];
      *out = size < 0 ? -digit : digit;
      return true;
    }
  }
#endif
  const long long x = PyLong_AsLongLong(v);
  if (x == -1 && PyErr_Occurred()) return false;
  *out = x;
  return true;
}

int64_t floor_div(int64_t a, int64_t b) {  // Python's a // b for b > 0
  int64_t q = a / b;
  if ((a % b != 0) && (a < 0)) --q;
  return q;
}

PyObject* gather(PyObject*, PyObject* args) {
  PyObject *entries_obj, *tokens_o, *positions_o, *slots_o, *lengths_o, *contexts_o, *logits_o;
  PyObject* stats_o = Py_None;
  long long block_size;
  if (!PyArg_ParseTuple(args, "OLOOOOOO|O", &entries_obj, &block_size, &tokens_o, &positions_o, &slots_o,
                        &lengths_o, &contexts_o, &logits_o, &stats_o)) {
    return nullptr;
  }
  if (block_size < 1) {
    PyErr_SetString(PyExc_ValueError, "block_size must be >= 1");
    return nullptr;
  }
  PyObject* entries = PySequence_Fast(entries_obj, "entries must be a sequence");
  if (entries == nullptr) return nullptr;
  const Py_ssize_t count = PySequence_Fast_GET_SIZE(entries);
  PyObject** items = PySequence_Fast_ITEMS(entries);
  Buf<int64_t> tokens, positions, slots, lengths, logits, stats;
  Buf<int32_t> contexts;
  PyObject* result = nullptr;
  std::vector<PyObject*> toks(count, nullptr), poss(count, nullptr);
  std::vector<int64_t> firsts;  // first block ids of single-token entries
  EntryField token_ids(s_token_ids), positions_f(s_positions), block_table(s_block_table),
      logits_index(s_logits_index);
  int64_t total = 0;
  if (!tokens.get(tokens_o, "tokens") || !positions.get(positions_o, "positions") ||
      !slots.get(slots_o, "slots") || !lengths.get(lengths_o, "lengths") ||
      !contexts.get(contexts_o, "contexts") || !logits.get(logits_o, "logits")) {
    goto done;
  }
  if (stats_o != Py_None && (!stats.get(stats_o, "stats") || stats.size() < 9)) {
    if (!PyErr_Occurred()) PyErr_SetString(PyExc_ValueError, "stats must hold 9 entries");
    goto done;
  }
  if (lengths.size() < count || contexts.size() < count || logits.size() < count) {
    PyErr_SetString(PyExc_ValueError, "per-entry buffers are shorter than the batch");
    goto done;
  }
  for (Py_ssize_t e = 0; e < count; ++e) {
    toks[e] = fast_attr(items[e], token_ids);
    if (toks[e] == nullptr) goto done;
    poss[e] = fast_attr(items[e], positions_f);
    if (poss[e] == nullptr) goto done;
    total += PySequence_Fast_GET_SIZE(toks[e]);
  }
  if (total > tokens.size() || total > positions.size() || total > slots.size()) {
    result = Py_BuildValue("(LiLL)", static_cast<long long>(-total), 0, 0LL, 0LL);
    goto done;
  }
  {
    int64_t at = 0;
    int problem = 0;
    long long bad_entry = 0, bad_position = 0;
    int64_t lo_tok = INT64_MAX, hi_tok = INT64_MIN, lo_pos = INT64_MAX, hi_pos = INT64_MIN;
    int64_t lo_slot = INT64_MAX, hi_slot = INT64_MIN, lo_ctx = INT64_MAX, hi_ctx = INT64_MIN;
    for (Py_ssize_t e = 0; e < count; ++e) {
      PyObject* entry = items[e];
      const Py_ssize_t n = PySequence_Fast_GET_SIZE(toks[e]);
      if (PySequence_Fast_GET_SIZE(poss[e]) != n) {
        PyErr_SetString(PyExc_ValueError, "token_ids and positions must have the same length");
        goto done;
      }
      PyObject** tok = PySequence_Fast_ITEMS(toks[e]);
      PyObject** pos = PySequence_Fast_ITEMS(poss[e]);
      PyObject* table = fast_attr(entry, block_table);
      if (table == nullptr) goto done;
      const Py_ssize_t width = PySequence_Fast_GET_SIZE(table);
      PyObject** blocks = PySequence_Fast_ITEMS(table);
      bool ok = true;
      for (Py_ssize_t i = 0; i < n && ok; ++i) {
        int64_t t, p;
        if (!as_i64(tok[i], &t) || !as_i64(pos[i], &p)) {
          ok = false;
          break;
        }
        tokens.data()[at + i] = t;
        positions.data()[at + i] = p;
        lo_tok = std::min(lo_tok, t);
        hi_tok = std::max(hi_tok, t);
        lo_pos = std::min(lo_pos, p);
        hi_pos = std::max(hi_pos, p);
        int64_t index = floor_div(p, block_size);
        if (index < 0) index += width;
        if (index >= width || index < 0) {
          if (problem == 0) {
            problem = floor_div(p, block_size) >= width ? 1 : 2;
            bad_entry = e;
            bad_position = p;
          }
          slots.data()[at + i] = -1;
          lo_slot = std::min<int64_t>(lo_slot, -1);
          hi_slot = std::max<int64_t>(hi_slot, -1);
          continue;
        }
        int64_t block;
        if (!as_i64(blocks[index], &block)) {
          ok = false;
          break;
        }
        const int64_t slot = block * block_size + (p - floor_div(p, block_size) * block_size);
        slots.data()[at + i] = slot;
        lo_slot = std::min(lo_slot, slot);
        hi_slot = std::max(hi_slot, slot);
      }
      if (ok && n == 1 && width > 0) {
        int64_t first;
        if (!as_i64(blocks[0], &first)) ok = false;
        else firsts.push_back(first);
      }
      Py_DECREF(table);
      if (!ok) goto done;
      lengths.data()[e] = n;
      int64_t last = 0;
      if (n > 0) last = positions.data()[at + n - 1];
      contexts.data()[e] = static_cast<int32_t>(last + 1);
      lo_ctx = std::min<int64_t>(lo_ctx, static_cast<int32_t>(last + 1));
      hi_ctx = std::max<int64_t>(hi_ctx, static_cast<int32_t>(last + 1));
      PyObject* index = logits_index.get(entry);
      if (index == nullptr) goto done;
      int64_t li = -1;
      if (index != Py_None && !as_i64(index, &li)) {
        Py_DECREF(index);
        goto done;
      }
      Py_DECREF(index);
      logits.data()[e] = li < 0 ? -1 : at + li;
      at += n;
    }
    if (stats_o != Py_None) {
      std::sort(firsts.begin(), firsts.end());
      const bool repeat = std::adjacent_find(firsts.begin(), firsts.end()) != firsts.end();
      const int64_t values[9] = {lo_tok, hi_tok, lo_pos, hi_pos, lo_slot, hi_slot, lo_ctx, repeat ? 1 : 0, hi_ctx};
      std::memcpy(stats.data(), values, sizeof(values));
    }
    result = Py_BuildValue("(LiLL)", static_cast<long long>(total), problem, bad_entry, bad_position);
  }
done:
  for (PyObject* o : toks) Py_XDECREF(o);
  for (PyObject* o : poss) Py_XDECREF(o);
  Py_DECREF(entries);
  return result;
}

// A hash of `n` block ids: four interleaved FNV-1a lanes (independent multiply chains), folded.
uint64_t hash_ids(const int32_t* ids, long long n) {
  constexpr uint64_t kPrime = 1099511628211ull;
  uint64_t h[4] = {1469598103934665603ull, 0x9e3779b97f4a7c15ull, 0xc2b2ae3d27d4eb4full, 0x165667b19e3779f9ull};
  long long c = 0;
  for (; c + 4 <= n; c += 4) {
    for (int j = 0; j < 4; ++j) h[j] = (h[j] ^ static_cast<uint32_t>(ids[c + j])) * kPrime;
  }
  for (; c < n; ++c) h[0] = (h[0] ^ static_cast<uint32_t>(ids[c])) * kPrime;
  uint64_t x = h[0] ^ (h[1] << 16 | h[1] >> 48) ^ (h[2] << 32 | h[2] >> 32) ^ (h[3] << 48 | h[3] >> 16);
  x ^= x >> 33;
  x *= 0xff51afd7ed558ccdull;
  return x ^ (x >> 33);
}

// The row order of prefix_order from the decode entries' positions in the batch (decode, in
// batch order) and their `lead` leading block ids (keys[k] points at entry k's), written to
// out[count]; false when nothing would move. An entry whose key equals the previous entry's
// (sharers are usually adjacent) takes its id from one comparison; other keys are found through
// a hash of the key confirmed by comparing the ids, so each entry's key is read about twice
// whatever the number of sharers; only the distinct keys are sorted.
bool order_decode_entries(const std::vector<Py_ssize_t>& decode, const std::vector<const int32_t*>& keys,
                          long long lead, long long min_rows, Py_ssize_t count, int64_t* out) {
  const Py_ssize_t nd = static_cast<Py_ssize_t>(decode.size());
  if (nd < min_rows || lead < 1 || nd < 2) return false;
  const size_t key_bytes = static_cast<size_t>(lead) * sizeof(int32_t);
  auto key = [&](Py_ssize_t k) { return keys[k]; };
  // 1. A key id per entry (ids numbered in order of first appearance).
  size_t slots = 4;
  while (slots < 2 * static_cast<size_t>(nd)) slots *= 2;
  std::vector<int32_t> table(slots, -1);  // open addressing: the first entry holding each key
  std::vector<int32_t> id(nd), first_of;  // entry -> key id; key id -> its first entry
  for (Py_ssize_t k = 0; k < nd; ++k) {
    const int32_t* kk = key(k);
    if (k > 0 && std::memcmp(kk, key(k - 1), key_bytes) == 0) {  // the previous entry's key
      id[k] = id[k - 1];
      continue;
    }
    size_t at = static_cast<size_t>(hash_ids(kk, lead)) & (slots - 1);
    while (true) {
      const int32_t e = table[at];
      if (e < 0) {
        table[at] = static_cast<int32_t>(k);
        id[k] = static_cast<int32_t>(first_of.size());
        first_of.push_back(static_cast<int32_t>(k));
        break;
      }
      if (std::memcmp(key(e), kk, key_bytes) == 0) {
        id[k] = id[e];
        break;
      }
      at = (at + 1) & (slots - 1);
    }
  }
  const Py_ssize_t distinct = static_cast<Py_ssize_t>(first_of.size());
  if (distinct == nd) return false;  // no two entries share their leading blocks
  // 2. Already grouped: every key's entries form one run of consecutive batch entries.
  {
    std::vector<char> ended(distinct, 0);
    bool grouped = true;
    for (Py_ssize_t k = 1; k < nd && grouped; ++k) {
      if (decode[k] == decode[k - 1] + 1 && id[k] == id[k - 1]) continue;
      ended[id[k - 1]] = 1;
      grouped = ended[id[k]] == 0;
    }
    if (grouped) return false;
  }
  // 3. The entries stably sorted by key: the distinct keys in lexicographic order of their ids,
  // then a counting sort of the entries by their key's rank.
  std::vector<int32_t> by_key(distinct);
  for (Py_ssize_t d = 0; d < distinct; ++d) by_key[d] = static_cast<int32_t>(d);
  std::sort(by_key.begin(), by_key.end(), [&](int32_t a, int32_t b) {
    const int32_t* ka = key(first_of[a]);
    const int32_t* kb = key(first_of[b]);
    return std::lexicographical_compare(ka, ka + lead, kb, kb + lead);
  });
  std::vector<int32_t> start(distinct + 1, 0);  // by rank
  std::vector<int32_t> rank(distinct);
  for (Py_ssize_t r = 0; r < distinct; ++r) rank[by_key[r]] = static_cast<int32_t>(r);
  for (Py_ssize_t k = 0; k < nd; ++k) ++start[rank[id[k]] + 1];
  for (Py_ssize_t r = 0; r < distinct; ++r) start[r + 1] += start[r];
  // 4. Nothing to gain when the entries that share are already adjacent in the batch: the sorted
  // order has nd - distinct equal neighbours; count those the batch order already has.
  Py_ssize_t adjacent = 0;
  for (Py_ssize_t k = 0; k + 1 < nd; ++k) adjacent += decode[k + 1] == decode[k] + 1 && id[k] == id[k + 1];
  if (adjacent == nd - distinct) return false;
  for (Py_ssize_t k = 0; k < nd; ++k) out[start[rank[id[k]]]++] = decode[k];
  std::vector<char> is_decode(count, 0);
  for (Py_ssize_t k = 0; k < nd; ++k) is_decode[decode[k]] = 1;
  Py_ssize_t at = nd;
  for (Py_ssize_t e = 0; e < count; ++e) {
    if (!is_decode[e]) out[at++] = e;
  }
  return true;
}

PyObject* prefix_order_rows(PyObject*, PyObject* args) {
  PyObject *rows_o, *lengths_o, *host_o, *held_o, *out_o;
  long long lead, min_rows;
  if (!PyArg_ParseTuple(args, "OOOOLLO", &rows_o, &lengths_o, &host_o, &held_o, &lead, &min_rows, &out_o)) {
    return nullptr;
  }
  Buf<int32_t> rows, host, held;
  Buf<int64_t> lengths, out;
  if (!rows.get(rows_o, "rows", false) || !lengths.get(lengths_o, "lengths", false) ||
      !host.get(host_o, "host", false) || !held.get(held_o, "held_len", false) || !out.get(out_o, "out")) {
    return nullptr;
  }
  const Py_ssize_t count = rows.size();
  const Py_ssize_t num_rows = host.dim(0), width = host.dim(1);
  if (host.ndim() != 2 || lengths.size() < count || held.size() != num_rows || out.size() < count) {
    PyErr_SetString(PyExc_ValueError, "prefix_order_rows buffers disagree");
    return nullptr;
  }
  std::vector<Py_ssize_t> decode;
  std::vector<const int32_t*> keys;
  if (lead >= 1) {
    for (Py_ssize_t e = 0; e < count; ++e) {
      const int32_t row = rows.data()[e];
      if (row < 0 || row >= num_rows) {
        PyErr_SetString(PyExc_ValueError, "an arena row is out of range");
        return nullptr;
      }
      if (lengths.data()[e] != 1 || held.data()[row] < lead || lead > width) continue;
      const int32_t* table = host.data() + static_cast<int64_t>(row) * width;
      decode.push_back(e);
      keys.push_back(table);
    }
  }
  return PyBool_FromLong(order_decode_entries(decode, keys, lead, min_rows, count, out.data()));
}

PyObject* arena_update(PyObject*, PyObject* args) {
  PyObject *entries_obj, *row_of, *key_of, *held_o, *held_obj, *last_o, *host_o, *rows_o, *index_o, *values_o;
  long long step;
  if (!PyArg_ParseTuple(args, "OO!O!OO!OOLOOO", &entries_obj, &PyDict_Type, &row_of, &PyList_Type, &key_of,
                        &held_o, &PyList_Type, &held_obj, &last_o, &host_o, &step, &rows_o, &index_o,
                        &values_o)) {
    return nullptr;
  }
  PyObject* entries = PySequence_Fast(entries_obj, "entries must be a sequence");
  if (entries == nullptr) return nullptr;
  const Py_ssize_t count = PySequence_Fast_GET_SIZE(entries);
  PyObject** items = PySequence_Fast_ITEMS(entries);
  Buf<int32_t> held, host, rows, values;
  Buf<int64_t> last, index;
  PyObject* result = nullptr;
  std::vector<PyObject*> tables(count, nullptr);
  EntryField block_table(s_block_table), seq_ids(s_seq_id);
  Py_ssize_t num_rows = 0, width = 0, longest = 0;
  if (!held.get(held_o, "held_len") || !last.get(last_o, "last_use") || !host.get(host_o, "host") ||
      !rows.get(rows_o, "rows") || !index.get(index_o, "index") || !values.get(values_o, "values")) {
    goto done;
  }
  num_rows = host.dim(0);
  width = host.dim(1);
  if (host.ndim() != 2 || held.size() != num_rows || last.size() != num_rows ||
      PyList_GET_SIZE(key_of) != num_rows || PyList_GET_SIZE(held_obj) != num_rows || rows.size() < count) {
    PyErr_SetString(PyExc_ValueError, "arena buffers disagree on their row count");
    goto done;
  }
  for (Py_ssize_t e = 0; e < count; ++e) {
    tables[e] = fast_attr(items[e], block_table);
    if (tables[e] == nullptr) goto done;
    longest = std::max(longest, PySequence_Fast_GET_SIZE(tables[e]));
  }
  if (count > num_rows || longest > width) {  // the caller grows the arena and calls again
    result = Py_BuildValue("(nn)", static_cast<Py_ssize_t>(-1), longest);
    goto done;
  }
  {
    // Every value that could change must fit the index/values buffers: at most the sum of the
    // table lengths.
    Py_ssize_t worst = 0;
    for (PyObject* t : tables) worst += PySequence_Fast_GET_SIZE(t);
    if (index.size() < worst || values.size() < worst) {
      result = Py_BuildValue("(nn)", static_cast<Py_ssize_t>(-2), worst);
      goto done;
    }
    int32_t* hostp = host.data();
    int32_t* heldp = held.data();
    int64_t* lastp = last.data();
    Py_ssize_t changed = 0, nchanged_rows = 0, reached = 0;
    PyObject* seen = nullptr;  // seq id -> occurrences so far, built once a sequence repeats
    bool ok = true;
    for (Py_ssize_t e = 0; e < count && ok; ++e) {
      PyObject* seq_id = seq_ids.get(items[e]);
      if (seq_id == nullptr) {
        ok = false;
        break;
      }
      // The same sequence twice in one batch gets a row per occurrence, keyed (seq_id, k) for
      // its k-th repeat. A repeat shows as a row this iteration has used already; only then are
      // the batch's occurrences counted.
      PyObject* key = seq_id;
      Py_INCREF(key);
      PyObject* found = PyDict_GetItemWithError(row_of, key);
      if (found == nullptr && PyErr_Occurred()) ok = false;
      const Py_ssize_t held_row = found == nullptr ? -1 : PyLong_AsSsize_t(found);
      const bool used = held_row >= 0 && held_row < num_rows && lastp[held_row] == step;
      if (ok && (used || seen != nullptr)) {
        if (seen == nullptr) {  // count the occurrences of every sequence before this entry
          seen = PyDict_New();
          for (Py_ssize_t f = 0; f < e && seen != nullptr; ++f) {
            PyObject* id = seq_ids.get(items[f]);
            PyObject* prior = id == nullptr ? nullptr : PyDict_GetItemWithError(seen, id);
            PyObject* next = id == nullptr || (prior == nullptr && PyErr_Occurred())
                                 ? nullptr
                                 : PyLong_FromLongLong(prior == nullptr ? 1 : PyLong_AsLongLong(prior) + 1);
            if (next == nullptr || PyDict_SetItem(seen, id, next) != 0) Py_CLEAR(seen);
            Py_XDECREF(next);
            Py_XDECREF(id);
          }
          if (seen == nullptr) ok = false;
        }
        long long repeat = 0;
        if (ok) {
          PyObject* prior = PyDict_GetItemWithError(seen, seq_id);
          if (prior != nullptr) repeat = PyLong_AsLongLong(prior);
          else if (PyErr_Occurred()) ok = false;
          PyObject* next = ok ? PyLong_FromLongLong(repeat + 1) : nullptr;
          if (next == nullptr || PyDict_SetItem(seen, seq_id, next) != 0) ok = false;
          Py_XDECREF(next);
        }
        if (ok && repeat > 0) {
          Py_DECREF(key);
          key = Py_BuildValue("(OL)", seq_id, repeat);
          if (key == nullptr) ok = false;
          found = key == nullptr ? nullptr : PyDict_GetItemWithError(row_of, key);
          if (found == nullptr && PyErr_Occurred()) ok = false;
        }
      }
      Py_DECREF(seq_id);
      if (!ok) {
        Py_XDECREF(key);
        break;
      }
      Py_ssize_t row = -1;
      if (found != nullptr) {
        row = PyLong_AsSsize_t(found);
      } else if (PyErr_Occurred()) {
        ok = false;
      } else {
        // claim the least recently used row not used in this iteration
        int64_t best = step;
        for (Py_ssize_t r = 0; r < num_rows; ++r) {
          if (lastp[r] < best) {
            best = lastp[r];
            row = r;
          }
        }
        if (row < 0) {  // cannot happen: count <= num_rows
          PyErr_SetString(PyExc_RuntimeError, "block-table arena has no free row");
          ok = false;
        } else {
          PyObject* previous = PyList_GET_ITEM(key_of, row);
          if (previous != Py_None && PyDict_DelItem(row_of, previous) != 0) ok = false;
          PyObject* r_obj = PyLong_FromSsize_t(row);
          if (ok && (r_obj == nullptr || PyDict_SetItem(row_of, key, r_obj) != 0)) ok = false;
          Py_XDECREF(r_obj);
          if (ok) {
            Py_INCREF(key);
            PyList_SetItem(key_of, row, key);  // steals the new reference, drops the old key
            heldp[row] = 0;  // nothing the row holds may be trusted for the new key
            Py_INCREF(Py_None);
            PyList_SetItem(held_obj, row, Py_None);
          }
        }
      }
      Py_DECREF(key);
      if (!ok) break;
      lastp[row] = step;
      rows.data()[e] = static_cast<int32_t>(row);
      reached = e + 1;
      const Py_ssize_t n = PySequence_Fast_GET_SIZE(tables[e]);
      PyObject** blocks = PySequence_Fast_ITEMS(tables[e]);
      const bool is_tuple = PyTuple_CheckExact(tables[e]);
      PyObject* before = PyList_GET_ITEM(held_obj, row);  // None or the tuple the mirror holds
      if (before == tables[e] && heldp[row] == n) continue;  // the row already holds this tuple
      int32_t* mirror = hostp + row * width;
      const Py_ssize_t old = heldp[row];
      // The ids against the row's mirror. An id that is the very object the held tuple has at
      // that index needs no conversion: the mirror holds that object's value (the reference's
      // scheduler builds each step's tuples from its sequences' lists of ids, so the objects
      // repeat; a comparison of the two tuples would convert every id that is not, both sides).
      // Runs of identical objects are found by comparing the pointer arrays 16 at a time.
      PyObject** held_ids = before != Py_None ? PySequence_Fast_ITEMS(before) : nullptr;
      const Py_ssize_t held_n = held_ids != nullptr ? std::min(old, PyTuple_GET_SIZE(before)) : 0;
      Py_ssize_t start = 0;
      const Py_ssize_t common = std::min(old, n);
      constexpr Py_ssize_t kRun = 16;
      const Py_ssize_t same_limit = std::min(held_n, common);
      while (start + kRun <= same_limit &&
             std::memcmp(held_ids + start, blocks + start, kRun * sizeof(PyObject*)) == 0) {
        start += kRun;
      }
      for (; start < common; ++start) {
        if (start < held_n && held_ids[start] == blocks[start]) continue;
        int64_t b;
        if (!as_i64(blocks[start], &b)) {
          ok = false;
          break;
        }
        if (mirror[start] != b) break;
      }
      if (!ok) break;
      if (!(start == n && old == n)) {
        for (Py_ssize_t c = start; c < n; ++c) {
          int64_t b;
          if (!as_i64(blocks[c], &b)) {
            ok = false;
            break;
          }
          mirror[c] = static_cast<int32_t>(b);
          index.data()[changed] = static_cast<int64_t>(row) * width + c;
          values.data()[changed] = static_cast<int32_t>(b);
          ++changed;
        }
        if (!ok) break;
        heldp[row] = static_cast<int32_t>(n);
        ++nchanged_rows;
      }
      // Keep the tuple (immutable) to compare the next step's table with; a list may change
      // under us, so it is converted and compared every time.
      PyObject* keep = is_tuple ? tables[e] : Py_None;
      Py_INCREF(keep);
      PyList_SetItem(held_obj, row, keep);
    }
    Py_XDECREF(seen);
    if (ok) {
      result = Py_BuildValue("(nn)", changed, nchanged_rows);
    } else {
      // The caller raises and applies nothing: no row this walk reached may be trusted.
      for (Py_ssize_t r = 0; r < reached; ++r) {
        const int32_t row = rows.data()[r];
        heldp[row] = 0;
        Py_INCREF(Py_None);
        PyList_SetItem(held_obj, row, Py_None);
      }
    }
  }
done:
  for (PyObject* t : tables) Py_XDECREF(t);
  Py_DECREF(entries);
  return result;
}

PyObject* exclusive_writes(PyObject*, PyObject* args) {
  PyObject *rows_o, *contexts_o, *host_o, *marks_o, *tiles_o = Py_None;
  long long block_size, partition = 0;
  if (!PyArg_ParseTuple(args, "OOOLO|OL", &rows_o, &contexts_o, &host_o, &block_size, &marks_o, &tiles_o, &partition)) {
    return nullptr;
  }
  Buf<int32_t> rows, contexts, host, tiles;
  Buf<uint8_t> marks;
  if (!rows.get(rows_o, "rows", false) || !contexts.get(contexts_o, "contexts", false) ||
      !host.get(host_o, "host", false) || !marks.get(marks_o, "marks") ||
      (tiles_o != Py_None && !tiles.get(tiles_o, "tiles", false))) {
    return nullptr;
  }
  const Py_ssize_t count = rows.size();
  const Py_ssize_t num_rows = host.dim(0), width = host.dim(1);
  const Py_ssize_t tile_ints = tiles_o == Py_None ? 0 : tiles.size();
  if (host.ndim() != 2 || contexts.size() < count || block_size < 1 || tile_ints % 4 != 0 ||
      (tile_ints > 0 && partition < 1)) {
    PyErr_SetString(PyExc_ValueError, "exclusive_writes buffers disagree");
    return nullptr;
  }
  // 0. A tile must cover no row's own position (context - 1): only the row pass appends.
  for (Py_ssize_t i = 0; i + 3 < tile_ints; i += 4) {
    const int32_t* t = tiles.data() + i;
    const bool whole = t[3] == PKV_TILE_WHOLE;
    const int64_t lo = whole ? 0 : static_cast<int64_t>(t[2]) * partition;
    const int64_t hi = whole || t[3] <= t[2] ? INT64_MAX : static_cast<int64_t>(t[3]) * partition;
    for (int64_t r = t[0]; r < static_cast<int64_t>(t[0]) + t[1]; ++r) {
      if (r < 0 || r >= count) Py_RETURN_FALSE;
      const int64_t own = static_cast<int64_t>(contexts.data()[r]) - 1;
      if (own >= lo && own < hi) Py_RETURN_FALSE;
    }
  }
  const int64_t num_blocks = marks.size();
  uint8_t* mark = marks.data();
  // The visible blocks of entry e, [0, ceil(context / B)), clamped to the row; -1 on a bad row.
  auto visible = [&](Py_ssize_t e, const int32_t** table) -> int64_t {
    const int32_t row = rows.data()[e];
    const int64_t ctx = contexts.data()[e];
    if (row < 0 || row >= num_rows || ctx < 1) return -1;
    *table = host.data() + static_cast<int64_t>(row) * width;
    return std::min<int64_t>((ctx + block_size - 1) / block_size, width);
  };
  // 1. Flag every written block (the block of position context - 1).
  bool ok = true;
  std::vector<int32_t> written;
  written.reserve(count);
  for (Py_ssize_t e = 0; e < count; ++e) {
    const int32_t* table = nullptr;
    const int64_t nb = visible(e, &table);
    const int64_t index = nb < 0 ? -1 : (contexts.data()[e] - 1) / block_size;
    if (index < 0 || index >= nb) {
      ok = false;  // a row the kernels cannot place: take the general path, which reports it
      break;
    }
    const int32_t w = table[index];
    if (w < 0 || w >= num_blocks) continue;  // outside the pool: no row reads or writes it
    if (mark[w] != 0) {
      ok = false;  // two rows write one block
      break;
    }
    mark[w] = 1;
    written.push_back(w);
  }
  // 2. Count the occurrences of flagged blocks among every entry's visible blocks: each written
  // block must occur once, in its writer's own table. Entries that share a prefix (the common
  // case the check serves: sequences forked from one parent) repeat the previous entry's leading
  // blocks; those need no second look when none of them is flagged (a flagged one among them
  // occurs in both tables, which already fails), so only the rest of each table is scanned.
  const int32_t* prev_table = nullptr;
  int64_t prev_nb = 0, prev_flagged = 0;  // the previous entry's first flagged index (nb: none)
  for (Py_ssize_t e = 0; e < count && ok; ++e) {
    const int32_t* table = nullptr;
    const int64_t nb = visible(e, &table);
    int64_t start = 0;
    if (prev_table != nullptr) {
      const int64_t limit = std::min(nb, prev_nb);
      // The common prefix, 16 ids at a time (a vectorised compare), then id by id.
      constexpr int64_t kChunk = 16;
      while (start + kChunk <= limit &&
             std::memcmp(table + start, prev_table + start, kChunk * sizeof(int32_t)) == 0) {
        start += kChunk;
      }
      while (start < limit && table[start] == prev_table[start]) ++start;
      if (prev_flagged < start) {
        ok = false;  // a written block in both tables
        break;
      }
    }
    int64_t flagged = nb;
    for (int64_t i = start; i < nb; ++i) {
      const int32_t b = table[i];
      if (b >= 0 && b < num_blocks && mark[b] != 0) {
        if (flagged == nb) flagged = i;
        if (++mark[b] > 2) {
          ok = false;
          break;
        }
      }
    }
    prev_table = table;
    prev_nb = nb;
    prev_flagged = flagged;
  }
  for (int32_t w : written) mark[w] = 0;
  return PyBool_FromLong(ok);
}

// Entry points of libpkv.so, bound once by bind().
decltype(&pkv_plan_batch) g_plan_batch = nullptr;
decltype(&pkv_paged_attention) g_paged_attention = nullptr;
decltype(&pkv_paged_attention_append) g_paged_attention_append = nullptr;
decltype(&pkv_copy_blocks) g_copy_blocks = nullptr;
decltype(&pkv_rms_norm) g_rms_norm = nullptr;
decltype(&pkv_silu_mul) g_silu_mul = nullptr;
decltype(&pkv_rope_append) g_rope_append = nullptr;
decltype(&pkv_append) g_append = nullptr;
decltype(&pkv_gather_rows) g_gather_rows = nullptr;
decltype(&pkv_greedy_tokens) g_greedy_tokens = nullptr;
// hipGetDevice / hipSetDevice of the same runtime, by their C signatures.
using GetDeviceFn = int (*)(int* device);
using SetDeviceFn = int (*)(int device);
GetDeviceFn g_get_device = nullptr;
SetDeviceFn g_set_device = nullptr;
// hipMemcpyAsync by its C signature (hipError_t and hipMemcpyKind are int-sized enums, hipStream_t
// a pointer), so this host-only extension needs no HIP headers.
using MemcpyAsyncFn = int (*)(void* dst, const void* src, size_t bytes, int kind, void* stream);
MemcpyAsyncFn g_memcpy_async = nullptr;
constexpr int kHostToDevice = 1;  // hipMemcpyHostToDevice
// hipEventCreateWithFlags / hipEventRecord / hipEventSynchronize / hipEventDestroy, likewise
// (hipEvent_t is a pointer).
using EventCreateFn = int (*)(void** event, unsigned flags);
using EventRecordFn = int (*)(void* event, void* stream);
using EventFn = int (*)(void* event);
EventCreateFn g_event_create = nullptr;
EventRecordFn g_event_record = nullptr;
EventFn g_event_synchronize = nullptr;
EventFn g_event_destroy = nullptr;
constexpr unsigned kEventDisableTiming = 2;  // hipEventDisableTiming

// A timing-free event created on `device` (made current for the call, then restored); null with
// a RuntimeError set on failure.
void* make_event(int device) {
  if (g_event_create == nullptr || g_get_device == nullptr || g_set_device == nullptr) {
    PyErr_SetString(PyExc_RuntimeError, "_pkvhost.bind() has not been given the HIP event entry points");
    return nullptr;
  }
  int previous = 0;
  void* event = nullptr;
  int rc = g_get_device(&previous);
  if (rc == 0 && previous != device) rc = g_set_device(device);
  if (rc == 0) rc = g_event_create(&event, kEventDisableTiming);
  if (previous != device) g_set_device(previous);
  if (rc != 0 || event == nullptr) {
    PyErr_Format(PyExc_RuntimeError, "hipEventCreateWithFlags failed (hipError_t %d)", rc);
    return nullptr;
  }
  return event;
}

bool bound(const void* fn) {
  if (fn != nullptr) return true;
  PyErr_SetString(PyExc_RuntimeError, "_pkvhost.bind() has not been given the library's entry points");
  return false;
}

template <typename T>
T* ptr(unsigned long long address) {
  return reinterpret_cast<T*>(static_cast<uintptr_t>(address));
}

PyObject* bind(PyObject*, PyObject* args) {
  unsigned long long plan, attention, attention_append, copy, norm, gate, rope, memcpy_async;
  unsigned long long gather_rows = 0, greedy = 0, get_device = 0, set_device = 0;
  unsigned long long event_create = 0, event_record = 0, event_synchronize = 0, event_destroy = 0, append = 0;
  if (!PyArg_ParseTuple(args, "KKKKKKKK|KKKKKKKKK", &plan, &attention, &attention_append, &copy, &norm, &gate, &rope,
                        &memcpy_async, &gather_rows, &greedy, &get_device, &set_device, &event_create,
                        &event_record, &event_synchronize, &event_destroy, &append)) {
    return nullptr;
  }
  if (plan == 0 || attention == 0 || attention_append == 0 || copy == 0 || norm == 0 || gate == 0 || rope == 0 ||
      memcpy_async == 0) {
    PyErr_SetString(PyExc_ValueError, "bind() needs eight non-null entry points");
    return nullptr;
  }
  g_gather_rows = reinterpret_cast<decltype(g_gather_rows)>(static_cast<uintptr_t>(gather_rows));
  g_greedy_tokens = reinterpret_cast<decltype(g_greedy_tokens)>(static_cast<uintptr_t>(greedy));
  g_get_device = reinterpret_cast<GetDeviceFn>(static_cast<uintptr_t>(get_device));
  g_set_device = reinterpret_cast<SetDeviceFn>(static_cast<uintptr_t>(set_device));
  g_plan_batch = reinterpret_cast<decltype(g_plan_batch)>(static_cast<uintptr_t>(plan));
  g_paged_attention = reinterpret_cast<decltype(g_paged_attention)>(static_cast<uintptr_t>(attention));
  g_paged_attention_append =
      reinterpret_cast<decltype(g_paged_attention_append)>(static_cast<uintptr_t>(attention_append));
  g_copy_blocks = reinterpret_cast<decltype(g_copy_blocks)>(static_cast<uintptr_t>(copy));
  g_rms_norm = reinterpret_cast<decltype(g_rms_norm)>(static_cast<uintptr_t>(norm));
  g_silu_mul = reinterpret_cast<decltype(g_silu_mul)>(static_cast<uintptr_t>(gate));
  g_rope_append = reinterpret_cast<decltype(g_rope_append)>(static_cast<uintptr_t>(rope));
  g_memcpy_async = reinterpret_cast<MemcpyAsyncFn>(static_cast<uintptr_t>(memcpy_async));
  g_event_create = reinterpret_cast<EventCreateFn>(static_cast<uintptr_t>(event_create));
  g_event_record = reinterpret_cast<EventRecordFn>(static_cast<uintptr_t>(event_record));
  g_event_synchronize = reinterpret_cast<EventFn>(static_cast<uintptr_t>(event_synchronize));
  g_event_destroy = reinterpret_cast<EventFn>(static_cast<uintptr_t>(event_destroy));
  g_append = reinterpret_cast<decltype(g_append)>(static_cast<uintptr_t>(append));
  Py_RETURN_NONE;
}

PyObject* event_create(PyObject*, PyObject* args) {
  int device;
  if (!PyArg_ParseTuple(args, "i", &device)) return nullptr;
  void* event = make_event(device);
  if (event == nullptr) return nullptr;
  return PyLong_FromVoidPtr(event);
}

PyObject* event_destroy(PyObject*, PyObject* args) {
  unsigned long long event;
  if (!PyArg_ParseTuple(args, "K", &event)) return nullptr;
  if (event != 0 && g_event_destroy != nullptr) g_event_destroy(reinterpret_cast<void*>(static_cast<uintptr_t>(event)));
  Py_RETURN_NONE;
}

PyObject* stage(PyObject*, PyObject* args) {
  PyObject *p64_o, *p32_o, *host_o;
  unsigned long long device_address, stream, event = 0;
  if (!PyArg_ParseTuple(args, "O!O!OKK|K", &PyList_Type, &p64_o, &PyList_Type, &p32_o, &host_o, &device_address,
                        &stream, &event)) {
    return nullptr;
  }
  if (!bound(reinterpret_cast<const void*>(g_memcpy_async))) return nullptr;
  if (event != 0 && (g_event_record == nullptr || g_event_synchronize == nullptr)) {
    PyErr_SetString(PyExc_RuntimeError, "_pkvhost.bind() has not been given the HIP event entry points");
    return nullptr;
  }
  const Py_ssize_t n64 = PyList_GET_SIZE(p64_o), n32 = PyList_GET_SIZE(p32_o);
  Buf<uint8_t> host;
  std::unique_ptr<Buf<int64_t>[]> b64(new Buf<int64_t>[n64]);
  std::unique_ptr<Buf<int32_t>[]> b32(new Buf<int32_t>[n32]);
  if (!host.get(host_o, "host")) return nullptr;
  Py_ssize_t bytes = 0;
  for (Py_ssize_t i = 0; i < n64; ++i) {
    if (!b64[i].get(PyList_GET_ITEM(p64_o, i), "an int64 part", false)) return nullptr;
    bytes += 8 * b64[i].size();
  }
  for (Py_ssize_t i = 0; i < n32; ++i) {
    if (!b32[i].get(PyList_GET_ITEM(p32_o, i), "an int32 part", false)) return nullptr;
    bytes += 4 * b32[i].size();
  }
  if (bytes > host.size()) Py_RETURN_NONE;
  if (bytes > 0 && device_address == 0) {
    PyErr_SetString(PyExc_ValueError, "stage() needs a device buffer");
    return nullptr;
  }
  // The copy the previous call queued from this buffer must have read it before it is rewritten.
  if (event != 0) {
    const int rc = g_event_synchronize(reinterpret_cast<void*>(static_cast<uintptr_t>(event)));
    if (rc != 0) {
      PyErr_Format(PyExc_RuntimeError, "hipEventSynchronize failed (hipError_t %d)", rc);
      return nullptr;
    }
  }
  PyObject* offsets = PyList_New(n64 + n32);
  if (offsets == nullptr) return nullptr;
  uint8_t* base = host.data();
  Py_ssize_t at = 0;
  for (Py_ssize_t i = 0; i < n64 + n32; ++i) {
    const bool wide = i < n64;
    const void* src = wide ? static_cast<const void*>(b64[i].data()) : static_cast<const void*>(b32[i - n64].data());
    const Py_ssize_t len = wide ? 8 * b64[i].size() : 4 * b32[i - n64].size();
    PyObject* offset = PyLong_FromSsize_t(at);
    if (offset == nullptr) {
      Py_DECREF(offsets);
      return nullptr;
    }
    PyList_SET_ITEM(offsets, i, offset);
    if (len > 0) std::memcpy(base + at, src, static_cast<size_t>(len));
    at += len;
  }
  if (bytes > 0) {
    const int rc = g_memcpy_async(reinterpret_cast<void*>(static_cast<uintptr_t>(device_address)), base,
                                  static_cast<size_t>(bytes), kHostToDevice,
                                  reinterpret_cast<void*>(static_cast<uintptr_t>(stream)));
    if (rc != 0) {
      Py_DECREF(offsets);
      PyErr_Format(PyExc_RuntimeError, "hipMemcpyAsync of the call's metadata failed (hipError_t %d)", rc);
      return nullptr;
    }
    if (event != 0) {
      const int rec = g_event_record(reinterpret_cast<void*>(static_cast<uintptr_t>(event)),
                                     reinterpret_cast<void*>(static_cast<uintptr_t>(stream)));
      if (rec != 0) {
        Py_DECREF(offsets);
        PyErr_Format(PyExc_RuntimeError, "hipEventRecord failed (hipError_t %d)", rec);
        return nullptr;
      }
    }
  }
  return offsets;
}

PyObject* plan(PyObject*, PyObject* args) {
  PyObject *seq_o, *pos_o, *tables_o, *ctx_o, *rows_o, *tiles_o, *merge_o, *counts_o, *launch_o;
  int block_size, num_heads, head_dim, kv_dtype, partition_size, min_tile_rows;
  if (!PyArg_ParseTuple(args, "OOOOiiiiiiOOOOO", &seq_o, &pos_o, &tables_o, &ctx_o, &block_size, &num_heads,
                        &head_dim, &kv_dtype, &partition_size, &min_tile_rows, &rows_o, &tiles_o, &merge_o,
                        &counts_o, &launch_o)) {
    return nullptr;
  }
  if (!bound(reinterpret_cast<const void*>(g_plan_batch))) return nullptr;
  Buf<int32_t> seq, pos, tables, ctx, rows, tiles, merge, launch;
  Buf<int64_t> counts;
  if (!seq.get(seq_o, "query_seq", false) || (pos_o != Py_None && !pos.get(pos_o, "query_positions", false)) ||
      !tables.get(tables_o, "tables", false) || !ctx.get(ctx_o, "contexts", false) || !rows.get(rows_o, "rows") ||
      !tiles.get(tiles_o, "tiles") || !merge.get(merge_o, "merge") || !counts.get(counts_o, "counts") ||
      !launch.get(launch_o, "launch")) {
    return nullptr;
  }
  if (tables.ndim() != 2 || (pos_o != Py_None && pos.size() != seq.size()) || counts.size() < 3 ||
      launch.size() < 2 || rows.size() % 2 != 0 || tiles.size() % 4 != 0) {
    PyErr_SetString(PyExc_ValueError, "plan buffers have inconsistent shapes");
    return nullptr;
  }
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = g_plan_batch(seq.data(), pos_o == Py_None ? nullptr : pos.data(), seq.size(), tables.data(),
                    static_cast<int32_t>(tables.dim(1)), ctx.data(), static_cast<int32_t>(ctx.size()), block_size,
                    num_heads, head_dim, static_cast<pkv_dtype>(kv_dtype), partition_size, min_tile_rows,
                    rows.data(), rows.size() / 2, tiles.data(),
                    tiles.size() / 4, merge.data(), merge.size(), counts.data(), launch.data());
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(rc);
}

PyObject* paged_attention(PyObject*, PyObject* args) {
  unsigned long long out, queries, qpos, qseq, caller_rows, rows, tiles, merge, kc, vc, tables, ctx, ws, stream;
  long long q_stride, nq, nrows, ntiles, nmerge, nblocks, ws_bytes;
  int dtype, block_size, table_stride, nseqs, heads, head_dim, max_ctx, partition, flags, device;
  float scale;
  if (!PyArg_ParseTuple(args, "KKLKKLKKLKLKLKKiLiKiKiiifiiiKLiK", &out, &queries, &q_stride, &qpos, &qseq, &nq,
                        &caller_rows, &rows, &nrows, &tiles, &ntiles, &merge, &nmerge, &kc, &vc, &dtype, &nblocks,
                        &block_size,
                        &tables, &table_stride, &ctx, &nseqs, &heads, &head_dim, &scale, &max_ctx, &partition,
                        &flags, &ws, &ws_bytes, &device, &stream)) {
    return nullptr;
  }
  if (!bound(reinterpret_cast<const void*>(g_paged_attention))) return nullptr;
  const int rc = g_paged_attention(
      ptr<float>(out), ptr<const float>(queries), q_stride, ptr<const int32_t>(qpos), ptr<const int32_t>(qseq), nq,
      ptr<const int32_t>(caller_rows), ptr<const int32_t>(rows), nrows, ptr<const int32_t>(tiles), ntiles,
      ptr<const int32_t>(merge), nmerge,
      ptr<const void>(kc), ptr<const void>(vc), static_cast<pkv_dtype>(dtype), nblocks, block_size,
      ptr<const int32_t>(tables), table_stride, ptr<const int32_t>(ctx), nseqs, heads, head_dim, scale, max_ctx,
      partition, flags, ptr<float>(ws), ws_bytes, device, ptr<void>(stream));
  return PyLong_FromLong(rc);
}

PyObject* paged_attention_append(PyObject*, PyObject* args) {
  unsigned long long out, queries, qpos, qseq, caller_rows, rows, tiles, merge, kc, vc, tables, ctx, ws, new_k, new_v,
      slots, stream;
  long long q_stride, nq, nrows, ntiles, nmerge, nblocks, ws_bytes, k_stride, v_stride;
  int dtype, block_size, table_stride, nseqs, heads, head_dim, max_ctx, partition, flags, new_dtype, device;
  float scale;
  if (!PyArg_ParseTuple(args, "KKLKKLKKLKLKLKKiLiKiKiiifiiiKLKKiLLKiK", &out, &queries, &q_stride, &qpos, &qseq, &nq,
                        &caller_rows, &rows, &nrows, &tiles, &ntiles, &merge, &nmerge, &kc, &vc, &dtype, &nblocks,
                        &block_size, &tables,
                        &table_stride, &ctx, &nseqs, &heads, &head_dim, &scale, &max_ctx, &partition, &flags, &ws,
                        &ws_bytes, &new_k, &new_v, &new_dtype, &k_stride, &v_stride, &slots, &device, &stream)) {
    return nullptr;
  }
  if (!bound(reinterpret_cast<const void*>(g_paged_attention_append))) return nullptr;
  const int rc = g_paged_attention_append(
      ptr<float>(out), ptr<const float>(queries), q_stride, ptr<const int32_t>(qpos), ptr<const int32_t>(qseq), nq,
      ptr<const int32_t>(caller_rows), ptr<const int32_t>(rows), nrows, ptr<const int32_t>(tiles), ntiles,
      ptr<const int32_t>(merge), nmerge, ptr<void>(kc), ptr<void>(vc),
      static_cast<pkv_dtype>(dtype), nblocks, block_size, ptr<const int32_t>(tables), table_stride,
      ptr<const int32_t>(ctx), nseqs, heads, head_dim, scale, max_ctx, partition, flags, ptr<float>(ws), ws_bytes,
      ptr<const void>(new_k), ptr<const void>(new_v), static_cast<pkv_dtype>(new_dtype), k_stride, v_stride,
      ptr<const int64_t>(slots), device, ptr<void>(stream));
  return PyLong_FromLong(rc);
}

PyObject* copy_blocks(PyObject*, PyObject* args) {
  unsigned long long kp, vp, pairs, stream;
  long long npairs, nblocks, block_elems;
  int dtype, layers, device;
  if (!PyArg_ParseTuple(args, "KKiKLiLLiK", &kp, &vp, &dtype, &pairs, &npairs, &layers, &nblocks, &block_elems,
                        &device, &stream)) {
    return nullptr;
  }
  if (!bound(reinterpret_cast<const void*>(g_copy_blocks))) return nullptr;
  const int rc = g_copy_blocks(ptr<void>(kp), ptr<void>(vp), static_cast<pkv_dtype>(dtype), ptr<const int64_t>(pairs),
                               npairs, layers, nblocks, block_elems, device, ptr<void>(stream));
  return PyLong_FromLong(rc);
}

// ---- CopyQueue: the runner's queued copy-on-write copies ----------------------------------------

struct CopyQueue {
  PyObject_HEAD
  std::vector<int64_t>* pairs;  // flat (src, dst), in queue order
  std::vector<uint8_t>* marks;  // one per pool block, all zero between flushes
  int64_t num_blocks;
  void* event;  // recorded after the pairs' copy to the device; created at the first flush
};

PyObject* copy_queue_new(PyTypeObject* type, PyObject* args, PyObject* kwds) {
  static const char* kwlist[] = {"num_blocks", nullptr};
  long long num_blocks;
  if (!PyArg_ParseTupleAndKeywords(args, kwds, "L", const_cast<char**>(kwlist), &num_blocks)) return nullptr;
  if (num_blocks < 1) {
    PyErr_SetString(PyExc_ValueError, "num_blocks must be >= 1");
    return nullptr;
  }
  CopyQueue* self = reinterpret_cast<CopyQueue*>(type->tp_alloc(type, 0));
  if (self == nullptr) return nullptr;
  self->num_blocks = num_blocks;
  self->event = nullptr;
  try {
    self->pairs = new std::vector<int64_t>();
    self->marks = new std::vector<uint8_t>(static_cast<size_t>(num_blocks), 0);
  } catch (const std::bad_alloc&) {
    Py_DECREF(self);
    return PyErr_NoMemory();
  }
  return reinterpret_cast<PyObject*>(self);
}

void copy_queue_dealloc(CopyQueue* self) {
  delete self->pairs;
  delete self->marks;
  if (self->event != nullptr && g_event_destroy != nullptr) g_event_destroy(self->event);
  Py_TYPE(self)->tp_free(reinterpret_cast<PyObject*>(self));
}

// push(source, destination): the reference's copy_block checks (runner.py:128-133 and this
// package's ModelRunner.copy_block), then the pair joins the queue.
PyObject* copy_queue_push(CopyQueue* self, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != 2) {
    PyErr_SetString(PyExc_TypeError, "copy_block() takes a source and a destination block id");
    return nullptr;
  }
  const int same = PyObject_RichCompareBool(args[0], args[1], Py_EQ);
  if (same < 0) return nullptr;
  if (same) {
    PyErr_SetString(PyExc_ValueError, "copy-on-write must not copy a block onto itself");
    return nullptr;
  }
  int64_t ids[2];
  for (int i = 0; i < 2; ++i) {
    const long long v = PyLong_AsLongLong(args[i]);
    if (v == -1 && PyErr_Occurred()) {
      if (!PyErr_ExceptionMatches(PyExc_OverflowError)) return nullptr;
      PyErr_Clear();
      ids[i] = -1;  // beyond int64: outside the pool
    } else {
      ids[i] = v;
    }
  }
  for (int i = 0; i < 2; ++i) {
    if (ids[i] < 0 || ids[i] >= self->num_blocks) {
      PyErr_Format(PyExc_IndexError, "block id %S is outside the pool", args[i]);
      return nullptr;
    }
  }
  try {
    self->pairs->push_back(ids[0]);
    self->pairs->push_back(ids[1]);
  } catch (const std::bad_alloc&) {
    return PyErr_NoMemory();
  }
  Py_RETURN_NONE;
}

// Sizes of the consecutive groups of independent queued copies, tracked with one mark byte per
// block (bit 0 read, bit 1 written by the current group; left all zero). Every id was checked
// against the pool at push.
std::vector<size_t> copy_groups(CopyQueue* self) {
  const std::vector<int64_t>& p = *self->pairs;
  const size_t n = p.size() / 2;
  std::vector<size_t> sizes;
  uint8_t* mark = self->marks->data();
  std::vector<int64_t> touched;
  touched.reserve(2 * n);
  size_t current = 0;
  for (size_t i = 0; i < n; ++i) {
    const int64_t src = p[2 * i], dst = p[2 * i + 1];
    if (current > 0 && ((mark[src] & 2) != 0 || mark[dst] != 0)) {
      sizes.push_back(current);
      current = 0;
      for (int64_t b : touched) mark[b] = 0;
      touched.clear();
    }
    mark[src] |= 1;
    mark[dst] |= 2;
    touched.push_back(src);
    touched.push_back(dst);
    ++current;
  }
  if (current > 0) sizes.push_back(current);
  for (int64_t b : touched) mark[b] = 0;
  return sizes;
}

PyObject* copy_queue_groups(CopyQueue* self, PyObject*) {
  const std::vector<size_t> sizes = copy_groups(self);
  PyObject* out = PyList_New(static_cast<Py_ssize_t>(sizes.size()));
  if (out == nullptr) return nullptr;
  for (size_t g = 0; g < sizes.size(); ++g) {
    PyObject* size = PyLong_FromSize_t(sizes[g]);
    if (size == nullptr) {
      Py_DECREF(out);
      return nullptr;
    }
    PyList_SET_ITEM(out, static_cast<Py_ssize_t>(g), size);
  }
  return out;
}

Py_ssize_t copy_queue_len(CopyQueue* self) { return static_cast<Py_ssize_t>(self->pairs->size() / 2); }

PyObject* copy_queue_clear(CopyQueue* self, PyObject*) {
  self->pairs->clear();
  Py_RETURN_NONE;
}

PyObject* copy_queue_items(CopyQueue* self, PyObject*) {
  const std::vector<int64_t>& p = *self->pairs;
  PyObject* out = PyList_New(static_cast<Py_ssize_t>(p.size() / 2));
  if (out == nullptr) return nullptr;
  for (size_t i = 0; i < p.size() / 2; ++i) {
    PyObject* pair = Py_BuildValue("(LL)", static_cast<long long>(p[2 * i]), static_cast<long long>(p[2 * i + 1]));
    if (pair == nullptr) {
      Py_DECREF(out);
      return nullptr;
    }
    PyList_SET_ITEM(out, static_cast<Py_ssize_t>(i), pair);
  }
  return out;
}

// flush(key_pool, value_pool, kv_dtype, layers, block_elems, host, device_address, device, stream)
//   -> (rc, n)
// Launches the queued copies in order, as pkv_copy_blocks launches of consecutive groups of
// independent copies (a copy starts a new group when it reads a block an earlier copy of the
// group writes, or writes a block an earlier copy of the group reads or writes), their pairs
// sent in one hipMemcpyAsync from the pinned uint8 buffer `host` to device_address. Before it
// rewrites `host` it waits for the event recorded after the previous flush's copy. (0, n): n
// copies launched and dequeued. (0, -bytes): `host` is smaller than the `bytes` the pairs need;
// nothing was done. (rc, 0): a launch failed with PKV code rc; every copy stays queued (a group
// reads no block it writes, so a group that ran already leaves the same bytes when it runs again).
PyObject* copy_queue_flush(CopyQueue* self, PyObject* args) {
  unsigned long long kp, vp, device_address, stream;
  int dtype, layers, device;
  long long block_elems;
  PyObject* host_o;
  if (!PyArg_ParseTuple(args, "KKiiLOKiK", &kp, &vp, &dtype, &layers, &block_elems, &host_o, &device_address, &device,
                        &stream)) {
    return nullptr;
  }
  const std::vector<int64_t>& p = *self->pairs;
  const size_t n = p.size() / 2;
  if (n == 0) return Py_BuildValue("(ii)", 0, 0);
  if (!bound(reinterpret_cast<const void*>(g_copy_blocks)) || !bound(reinterpret_cast<const void*>(g_memcpy_async))) {
    return nullptr;
  }
  if (g_event_record == nullptr || g_event_synchronize == nullptr) {
    PyErr_SetString(PyExc_RuntimeError, "_pkvhost.bind() has not been given the HIP event entry points");
    return nullptr;
  }
  Buf<uint8_t> host;
  if (!host.get(host_o, "host")) return nullptr;
  const Py_ssize_t bytes = static_cast<Py_ssize_t>(16 * n);
  if (host.size() < bytes) return Py_BuildValue("(in)", 0, -bytes);
  if (device_address == 0) {
    PyErr_SetString(PyExc_ValueError, "flush() needs a device buffer");
    return nullptr;
  }
  const std::vector<size_t> sizes = copy_groups(self);
  if (self->event == nullptr) {
    self->event = make_event(device);
    if (self->event == nullptr) return nullptr;
  } else {
    const int rc = g_event_synchronize(self->event);
    if (rc != 0) {
      PyErr_Format(PyExc_RuntimeError, "hipEventSynchronize failed (hipError_t %d)", rc);
      return nullptr;
    }
  }
  std::memcpy(host.data(), p.data(), static_cast<size_t>(bytes));
  void* dev = reinterpret_cast<void*>(static_cast<uintptr_t>(device_address));
  void* strm = reinterpret_cast<void*>(static_cast<uintptr_t>(stream));
  int rc = g_memcpy_async(dev, host.data(), static_cast<size_t>(bytes), kHostToDevice, strm);
  if (rc != 0) {
    PyErr_Format(PyExc_RuntimeError, "hipMemcpyAsync of the copy pairs failed (hipError_t %d)", rc);
    return nullptr;
  }
  rc = g_event_record(self->event, strm);
  if (rc != 0) {
    PyErr_Format(PyExc_RuntimeError, "hipEventRecord failed (hipError_t %d)", rc);
    return nullptr;
  }
  size_t start = 0;
  for (size_t size : sizes) {
    rc = g_copy_blocks(ptr<void>(kp), ptr<void>(vp), static_cast<pkv_dtype>(dtype),
                       reinterpret_cast<const int64_t*>(static_cast<uint8_t*>(dev) + 16 * start),
                       static_cast<int64_t>(size), layers, self->num_blocks, block_elems, device, strm);
    if (rc != 0) return Py_BuildValue("(ii)", rc, 0);
    start += size;
  }
  self->pairs->clear();
  return Py_BuildValue("(in)", 0, static_cast<Py_ssize_t>(n));
}

PyMethodDef kCopyQueueMethods[] = {
    {"push", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)(void)>(copy_queue_push)), METH_FASTCALL,
     "Queue one block copy (source, destination), checked against the pool."},
    {"flush", reinterpret_cast<PyCFunction>(copy_queue_flush), METH_VARARGS,
     "Launch the queued copies as batched pkv_copy_blocks launches: (rc, copies) or (0, -bytes needed)."},
    {"groups", reinterpret_cast<PyCFunction>(copy_queue_groups), METH_NOARGS,
     "Sizes of the consecutive groups of independent queued copies (one launch each)."},
    {"clear", reinterpret_cast<PyCFunction>(copy_queue_clear), METH_NOARGS, "Drop every queued copy."},
    {"items", reinterpret_cast<PyCFunction>(copy_queue_items), METH_NOARGS, "The queued (source, destination) pairs."},
    {nullptr, nullptr, 0, nullptr},
};

PySequenceMethods kCopyQueueSequence = {
    reinterpret_cast<lenfunc>(copy_queue_len),  // sq_length
};

PyTypeObject kCopyQueueType = {PyVarObject_HEAD_INIT(nullptr, 0) "_pkvhost.CopyQueue"};

PyObject* rms_norm(PyObject*, PyObject* args) {
  unsigned long long out, hidden, delta, weight, stream;
  long long out_stride, hidden_stride, delta_stride, rows;
  int dim, device;
  float eps;
  if (!PyArg_ParseTuple(args, "KLKLKLKLifiK", &out, &out_stride, &hidden, &hidden_stride, &delta, &delta_stride,
                        &weight, &rows, &dim, &eps, &device, &stream)) {
    return nullptr;
  }
  if (!bound(reinterpret_cast<const void*>(g_rms_norm))) return nullptr;
  const int rc = g_rms_norm(ptr<float>(out), out_stride, ptr<float>(hidden), hidden_stride, ptr<const float>(delta),
                            delta_stride, ptr<const float>(weight), rows, dim, eps, device, ptr<void>(stream));
  return PyLong_FromLong(rc);
}

PyObject* silu_mul(PyObject*, PyObject* args) {
  unsigned long long out, gate, up, stream;
  long long out_stride, in_stride, rows;
  int width, device;
  if (!PyArg_ParseTuple(args, "KLKKLLiiK", &out, &out_stride, &gate, &up, &in_stride, &rows, &width, &device,
                        &stream)) {
    return nullptr;
  }
  if (!bound(reinterpret_cast<const void*>(g_silu_mul))) return nullptr;
  const int rc = g_silu_mul(ptr<float>(out), out_stride, ptr<const float>(gate), ptr<const float>(up), in_stride,
                            rows, width, device, ptr<void>(stream));
  return PyLong_FromLong(rc);
}

PyObject* append(PyObject*, PyObject* args) {
  unsigned long long kp, vp, k, v, slots, stream;
  long long nslots, k_stride, v_stride, tokens;
  int pool_dtype, src_dtype, heads, dim, device;
  if (!PyArg_ParseTuple(args, "KKiLKKiLLKLiiiK", &kp, &vp, &pool_dtype, &nslots, &k, &v, &src_dtype, &k_stride,
                        &v_stride, &slots, &tokens, &heads, &dim, &device, &stream)) {
    return nullptr;
  }
  if (!bound(reinterpret_cast<const void*>(g_append))) return nullptr;
  const int rc = g_append(ptr<void>(kp), ptr<void>(vp), static_cast<pkv_dtype>(pool_dtype), nslots, ptr<const void>(k),
                          ptr<const void>(v), static_cast<pkv_dtype>(src_dtype), k_stride, v_stride,
                          ptr<const int64_t>(slots), tokens, heads, dim, device, ptr<void>(stream));
  return PyLong_FromLong(rc);
}

PyObject* rope_append(PyObject*, PyObject* args) {
  unsigned long long rot, q, k, v, pos, cos_t, sin_t, kp, vp, slots, stream;
  long long rot_stride, q_stride, k_stride, v_stride, table_rows, nslots, tokens;
  int dtype, heads, dim, device;
  if (!PyArg_ParseTuple(args, "KLKKKLLLKKKLKKiLKLiiiK", &rot, &rot_stride, &q, &k, &v, &q_stride, &k_stride,
                        &v_stride, &pos, &cos_t, &sin_t, &table_rows, &kp, &vp, &dtype, &nslots, &slots, &tokens,
                        &heads, &dim, &device, &stream)) {
    return nullptr;
  }
  if (!bound(reinterpret_cast<const void*>(g_rope_append))) return nullptr;
  const int rc = g_rope_append(ptr<float>(rot), rot_stride, ptr<const float>(q), ptr<const float>(k),
                               ptr<const float>(v), q_stride, k_stride, v_stride, ptr<const int64_t>(pos),
                               ptr<const float>(cos_t), ptr<const float>(sin_t), table_rows, ptr<void>(kp),
                               ptr<void>(vp), static_cast<pkv_dtype>(dtype), nslots, ptr<const int64_t>(slots),
                               tokens, heads, dim, device, ptr<void>(stream));
  return PyLong_FromLong(rc);
}

// --- the forward pass of one iteration ---------------------------------------------------------

// rocBLAS by its C signatures (rocblas_handle is a pointer, rocblas_status and rocblas_operation
// are int-sized enums, rocblas_int is int32), so this extension needs no ROCm headers. The library
// is the one already loaded in the process (torch's), found by its soname, else loaded.
using BlasCreateFn = int (*)(void** handle);
using BlasSetStreamFn = int (*)(void* handle, void* stream);
using BlasSgemmFn = int (*)(void* handle, int trans_a, int trans_b, int32_t m, int32_t n, int32_t k,
                            const float* alpha, const float* a, int32_t lda, const float* b, int32_t ldb,
                            const float* beta, float* c, int32_t ldc);
constexpr int kBlasNone = 111;       // rocblas_operation_none
constexpr int kBlasTranspose = 112;  // rocblas_operation_transpose
constexpr int kMaxDevices = 64;

struct Blas {
  BlasCreateFn create = nullptr;
  BlasSetStreamFn set_stream = nullptr;
  BlasSgemmFn sgemm = nullptr;
  void* handles[kMaxDevices] = {};
  // A device's handle is bound to one stream at a time: its forward passes run one after another.
  std::mutex device_mu[kMaxDevices];
};
Blas g_blas;

bool load_blas() {
  if (g_blas.sgemm != nullptr) return true;
  void* lib = dlopen("librocblas.so.5", RTLD_NOW | RTLD_NOLOAD);
  if (lib == nullptr) lib = dlopen("librocblas.so.5", RTLD_NOW | RTLD_LOCAL);
  if (lib == nullptr) lib = dlopen("/opt/rocm/lib/librocblas.so.5", RTLD_NOW | RTLD_LOCAL);
  if (lib == nullptr) {
    PyErr_Format(PyExc_RuntimeError, "rocBLAS is not available: %s", dlerror());
    return false;
  }
  g_blas.create = reinterpret_cast<BlasCreateFn>(dlsym(lib, "rocblas_create_handle"));
  g_blas.set_stream = reinterpret_cast<BlasSetStreamFn>(dlsym(lib, "rocblas_set_stream"));
  g_blas.sgemm = reinterpret_cast<BlasSgemmFn>(dlsym(lib, "rocblas_sgemm"));
  if (g_blas.create == nullptr || g_blas.set_stream == nullptr || g_blas.sgemm == nullptr) {
    g_blas.sgemm = nullptr;
    PyErr_SetString(PyExc_RuntimeError, "rocBLAS lacks rocblas_create_handle / rocblas_set_stream / rocblas_sgemm");
    return false;
  }
  return true;
}

// Row-major C[m, n] = A[m, k] B[k, n] (B given transposed, as [n, k], when b_transposed), leading
// dimensions in elements. In rocBLAS's column-major terms: C^T = B^T A^T.
int gemm(void* handle, int64_t m, int64_t n, int64_t k, const float* a, int64_t lda, const float* b, int64_t ldb,
         bool b_transposed, float* c, int64_t ldc) {
  static const float one = 1.f, zero = 0.f;
  return g_blas.sgemm(handle, b_transposed ? kBlasTranspose : kBlasNone, kBlasNone, static_cast<int32_t>(n),
                      static_cast<int32_t>(m), static_cast<int32_t>(k), &one, b, static_cast<int32_t>(ldb), a,
                      static_cast<int32_t>(lda), &zero, c, static_cast<int32_t>(ldc));
}

// Integer fields of forward()'s first argument, in order.
enum Field {
  kDevice, kStream, kTokens, kWanted, kModel, kHeads, kHeadDim, kFf, kVocab,
  kTokenIds, kRopePositions, kSlots, kLogitsRows,
  kEmbedding, kFinalNorm, kCos, kSin, kTableRows,
  kKeyPool, kValuePool, kLayerBytes, kKvDtype, kNumSlots,
  kHidden, kNormed, kFused, kAttended, kTmp, kGate, kGated, kPicked, kLogits,
  kQueryPositions, kQuerySeq, kPlanRows, kNumPlanRows, kPlanTiles, kNumTiles, kMerge, kNumMerge,
  kNumBlocks, kBlockSize, kTables, kTableStride, kContexts, kNumSeqs,
  kMaxContext, kPartition, kFlags, kWorkspace, kWorkspaceBytes, kGreedyOut,
  kNumFields
};

PyObject* forward(PyObject*, PyObject* args) {
  PyObject *ints_o, *layers_o;
  float eps, scale;
  if (!PyArg_ParseTuple(args, "OO!ff", &ints_o, &PyList_Type, &layers_o, &eps, &scale)) return nullptr;
  for (const void* fn : {reinterpret_cast<const void*>(g_rms_norm), reinterpret_cast<const void*>(g_rope_append),
                         reinterpret_cast<const void*>(g_paged_attention), reinterpret_cast<const void*>(g_silu_mul),
                         reinterpret_cast<const void*>(g_gather_rows), reinterpret_cast<const void*>(g_greedy_tokens),
                         reinterpret_cast<const void*>(g_get_device), reinterpret_cast<const void*>(g_set_device)}) {
    if (!bound(fn)) return nullptr;
  }
  if (!load_blas()) return nullptr;
  PyObject* ints = PySequence_Fast(ints_o, "forward() takes a sequence of integers");
  if (ints == nullptr) return nullptr;
  if (PySequence_Fast_GET_SIZE(ints) != kNumFields) {
    Py_DECREF(ints);
    PyErr_Format(PyExc_ValueError, "forward() takes %d integers", static_cast<int>(kNumFields));
    return nullptr;
  }
  int64_t v[kNumFields];
  for (int i = 0; i < kNumFields; ++i) {
    PyObject* item = PySequence_Fast_GET_ITEM(ints, i);
    v[i] = PyLong_AsLongLong(item);
    if (PyErr_Occurred()) {
      Py_DECREF(ints);
      return nullptr;
    }
  }
  Py_DECREF(ints);
  const Py_ssize_t num_layers = PyList_GET_SIZE(layers_o);
  std::vector<int64_t> layer(6 * num_layers);
  for (Py_ssize_t l = 0; l < num_layers; ++l) {
    PyObject* t = PyList_GET_ITEM(layers_o, l);
    if (!PyTuple_Check(t) || PyTuple_GET_SIZE(t) != 6) {
      PyErr_SetString(PyExc_ValueError, "a layer is a tuple of six weight addresses");
      return nullptr;
    }
    for (int j = 0; j < 6; ++j) {
      layer[6 * l + j] = PyLong_AsLongLong(PyTuple_GET_ITEM(t, j));
      if (PyErr_Occurred()) return nullptr;
    }
  }
  const int device = static_cast<int>(v[kDevice]);
  void* stream = ptr<void>(v[kStream]);
  const int64_t T = v[kTokens], W = v[kWanted], d = v[kModel], ff = v[kFf], vocab = v[kVocab];
  const int heads = static_cast<int>(v[kHeads]), dim = static_cast<int>(v[kHeadDim]);
  if (device < 0 || device >= kMaxDevices || T < 1 || W < 0 || d != static_cast<int64_t>(heads) * dim || ff < 1 ||
      vocab < 1 || 3 * d > INT32_MAX || 2 * ff > INT32_MAX || T > INT32_MAX) {
    PyErr_SetString(PyExc_ValueError, "forward() sizes are out of range");
    return nullptr;
  }
  auto f = [&](Field i) { return ptr<float>(v[i]); };
  const char* failed = nullptr;
  int rc = 0;
  int previous = -1;
  if (g_get_device(&previous) != 0 || (previous != device && g_set_device(device) != 0)) {
    PyErr_Format(PyExc_RuntimeError, "cannot make device %d current", device);
    return nullptr;
  }
  Py_BEGIN_ALLOW_THREADS
  std::lock_guard<std::mutex> device_lock(g_blas.device_mu[device]);
  void*& handle = g_blas.handles[device];
  if (handle == nullptr && g_blas.create(&handle) != 0) {
    handle = nullptr;
    failed = "rocblas_create_handle";
  }
  if (failed == nullptr && g_blas.set_stream(handle, stream) != 0) failed = "rocblas_set_stream";
  auto check = [&](int code, const char* what) {
    if (failed == nullptr && code != 0) {
      rc = code;
      failed = what;
    }
    return failed == nullptr;
  };
  // hidden = embedding[tokens]; normed = rms_norm(hidden) with the first norm's weights
  float* hidden = f(kHidden);
  float* normed = f(kNormed);
  float* fused = f(kFused);
  float* attended = f(kAttended);
  float* tmp = f(kTmp);
  float* gate = f(kGate);
  float* gated = f(kGated);
  auto norm = [&](int64_t weight, const float* delta) {
    return check(g_rms_norm(normed, d, hidden, d, delta, d, ptr<const float>(weight), T, static_cast<int32_t>(d), eps,
                            device, stream),
                 "pkv_rms_norm");
  };
  if (failed == nullptr) {
    check(g_gather_rows(hidden, d, ptr<const float>(v[kEmbedding]), d, vocab, ptr<const int64_t>(v[kTokenIds]), T,
                        static_cast<int32_t>(d), device, stream),
          "pkv_gather_rows (embedding)");
  }
  if (failed == nullptr) norm(num_layers > 0 ? layer[0] : v[kFinalNorm], nullptr);
  const int64_t row = d;  // heads * head_dim
  for (Py_ssize_t l = 0; l < num_layers && failed == nullptr; ++l) {
    const int64_t* w = &layer[6 * l];  // attn_norm, qkv, out_proj, ffn_norm, gate_up, down
    char* kp = ptr<char>(v[kKeyPool]) + l * v[kLayerBytes];
    char* vp = ptr<char>(v[kValuePool]) + l * v[kLayerBytes];
    // fused = normed @ qkv: [T, 3d], q | k | v per token (model.py:248-249)
    if (!check(gemm(handle, T, 3 * d, d, normed, d, ptr<const float>(w[1]), 3 * d, false, fused, 3 * d), "rocblas_sgemm (qkv)")) break;
    // RoPE on q (in place) and k, and the append of k and v (model.py:251-252, runner.py:195-196)
    if (!check(g_rope_append(fused, 3 * row, fused, fused + row, fused + 2 * row, 3 * row, 3 * row, 3 * row,
                             ptr<const int64_t>(v[kRopePositions]), ptr<const float>(v[kCos]), ptr<const float>(v[kSin]),
                             v[kTableRows], kp, vp, static_cast<pkv_dtype>(v[kKvDtype]), v[kNumSlots],
                             ptr<const int64_t>(v[kSlots]), T, heads, dim, device, stream),
               "pkv_rope_append")) {
      break;
    }
    // attention over the pools (runner.py:198-212)
    if (v[kNumPlanRows] > 0 || v[kNumTiles] > 0) {
      if (!check(g_paged_attention(attended, fused, 3 * row, ptr<const int32_t>(v[kQueryPositions]),
                                   ptr<const int32_t>(v[kQuerySeq]), T, nullptr, ptr<const int32_t>(v[kPlanRows]),
                                   v[kNumPlanRows],
                                   ptr<const int32_t>(v[kPlanTiles]), v[kNumTiles], ptr<const int32_t>(v[kMerge]),
                                   v[kNumMerge], kp, vp, static_cast<pkv_dtype>(v[kKvDtype]), v[kNumBlocks],
                                   static_cast<int32_t>(v[kBlockSize]), ptr<const int32_t>(v[kTables]),
                                   static_cast<int32_t>(v[kTableStride]), ptr<const int32_t>(v[kContexts]),
                                   static_cast<int32_t>(v[kNumSeqs]), heads, dim, scale,
                                   static_cast<int32_t>(v[kMaxContext]), static_cast<int32_t>(v[kPartition]),
                                   static_cast<int32_t>(v[kFlags]), f(kWorkspace), v[kWorkspaceBytes], device, stream),
                 "pkv_paged_attention")) {
        break;
      }
    }
    // hidden += attended @ out_proj, then the feed-forward norm (model.py:283, 256)
    if (!check(gemm(handle, T, d, d, attended, d, ptr<const float>(w[2]), d, false, tmp, d), "rocblas_sgemm (out_proj)")) break;
    if (!norm(w[3], tmp)) break;
    // gated = silu(normed @ gate) * (normed @ up), one product of [gate | up] (model.py:257-258)
    if (!check(gemm(handle, T, 2 * ff, d, normed, d, ptr<const float>(w[4]), 2 * ff, false, gate, 2 * ff), "rocblas_sgemm (gate_up)")) break;
    if (!check(g_silu_mul(gated, ff, gate, gate + ff, 2 * ff, T, static_cast<int32_t>(ff), device, stream), "pkv_silu_mul")) break;
    // hidden += gated @ down, then the next norm (the next layer's attention norm, or the final one)
    if (!check(gemm(handle, T, d, ff, gated, ff, ptr<const float>(w[5]), d, false, tmp, d), "rocblas_sgemm (down)")) break;
    norm(l + 1 < num_layers ? layer[6 * (l + 1)] : v[kFinalNorm], tmp);
  }
  // logits of the rows that ask for them: normed[rows] @ embedding^T (runner.py:215-227,
  // model.py:259-261), then greedy sampling when asked
  if (failed == nullptr && W > 0) {
    float* picked = f(kPicked);
    float* logits = f(kLogits);
    if (check(g_gather_rows(picked, d, normed, d, T, ptr<const int64_t>(v[kLogitsRows]), W, static_cast<int32_t>(d),
                            device, stream),
              "pkv_gather_rows (logits rows)") &&
        check(gemm(handle, W, vocab, d, picked, d, ptr<const float>(v[kEmbedding]), d, true, logits, vocab),
              "rocblas_sgemm (logits)") &&
        v[kGreedyOut] != 0) {
      check(g_greedy_tokens(ptr<int32_t>(v[kGreedyOut]), logits, vocab, W, vocab, device, stream), "pkv_greedy_tokens");
    }
  }
  if (previous != device) g_set_device(previous);
  Py_END_ALLOW_THREADS
  if (failed != nullptr) {
    PyErr_Format(PyExc_RuntimeError, "%s failed (code %d)", failed, rc);
    return nullptr;
  }
  Py_RETURN_NONE;
}

PyMethodDef kMethods[] = {
    {"gather", gather, METH_VARARGS, "Flatten a batch: tokens, positions, slots, lengths, contexts, logits rows."},
    {"prefix_order_rows", prefix_order_rows, METH_VARARGS, "prefix_order from the block-table arena's rows."},
    {"arena_update", arena_update, METH_VARARGS, "One step of the block-table arena."},
    {"exclusive_writes", exclusive_writes, METH_VARARGS,
     "True when no decode row reads a block another row (or its own, elsewhere) writes."},
    {"bind", bind, METH_VARARGS, "Bind the libpkv.so entry points the calls below use."},
    {"plan", plan, METH_VARARGS, "pkv_plan_batch on NumPy buffers."},
    {"paged_attention", paged_attention, METH_VARARGS, "pkv_paged_attention with integer pointers."},
    {"paged_attention_append", paged_attention_append, METH_VARARGS,
     "pkv_paged_attention_append with integer pointers."},
    {"copy_blocks", copy_blocks, METH_VARARGS, "pkv_copy_blocks with integer pointers."},
    {"rms_norm", rms_norm, METH_VARARGS, "pkv_rms_norm with integer pointers."},
    {"silu_mul", silu_mul, METH_VARARGS, "pkv_silu_mul with integer pointers."},
    {"rope_append", rope_append, METH_VARARGS, "pkv_rope_append with integer pointers."},
    {"append", append, METH_VARARGS, "pkv_append with integer pointers."},
    {"stage", stage, METH_VARARGS, "Pack a call's metadata into pinned memory and copy it to the device."},
    {"forward", forward, METH_VARARGS, "One iteration's forward pass: rocBLAS products and the library's kernels."},
    {"event_create", event_create, METH_VARARGS, "A timing-free HIP event on a device, as an integer handle."},
    {"event_destroy", event_destroy, METH_VARARGS, "Destroy an event made by event_create."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_pkvhost", "Per-entry host work of a ModelRunner iteration.",
                       -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__pkvhost(void) {
  s_seq_id = PyUnicode_InternFromString("seq_id");
  s_token_ids = PyUnicode_InternFromString("token_ids");
  s_positions = PyUnicode_InternFromString("positions");
  s_block_table = PyUnicode_InternFromString("block_table");
  s_logits_index = PyUnicode_InternFromString("logits_index");
  kCopyQueueType.tp_basicsize = sizeof(CopyQueue);
  kCopyQueueType.tp_flags = Py_TPFLAGS_DEFAULT;
  kCopyQueueType.tp_doc = "CopyQueue(num_blocks): queued copy-on-write block copies, flushed as batched launches.";
  kCopyQueueType.tp_new = copy_queue_new;
  kCopyQueueType.tp_dealloc = reinterpret_cast<destructor>(copy_queue_dealloc);
  kCopyQueueType.tp_methods = kCopyQueueMethods;
  kCopyQueueType.tp_as_sequence = &kCopyQueueSequence;
  if (PyType_Ready(&kCopyQueueType) < 0) return nullptr;
  PyObject* module = PyModule_Create(&kModule);
  if (module == nullptr) return nullptr;
  Py_INCREF(&kCopyQueueType);
  if (PyModule_AddObject(module, "CopyQueue", reinterpret_cast<PyObject*>(&kCopyQueueType)) < 0) {
    Py_DECREF(&kCopyQueueType);
    Py_DECREF(module);
    return nullptr;
  }
  return module;
}
