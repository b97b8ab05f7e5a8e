// _pkvhost: the per-entry host work of one ModelRunner iteration, in C++ (a CPython extension).
//
// A batch is a tuple of BatchEntry objects (the reference's or this package's: anything with
// seq_id, token_ids, positions, block_table and logits_index). Walking them in Python costs about
// a microsecond per entry and attribute; here one pass reads each entry once. Three functions:
//
//   gather(entries, block_size, tokens, positions, slots, lengths, contexts, logits)
//       -> (total, problem, entry, position)
//       Flattens token ids and positions, computes every slot with the reference's rule
//       (runner.py:149-159: block_table[p // B] * B + p % B with Python's floor division and a
//       negative index counting from the table's end), and per entry its token count, context
//       length (positions[-1] + 1) and the flat row of its logits (-1 when it asks for none).
//       The first slot that cannot be formed is reported, not raised, so the caller can check
//       token ids and positions first, in the reference's order: problem 1 = a position past
//       the table (the reference's ValueError), 2 = a negative index before its start
//       (IndexError). Returns total = -(tokens needed), writing nothing, when the token buffers
//       are too small.
//   prefix_order(entries, lead, min_rows) -> list | None
//       The row order that puts decode entries sharing their first `lead` blocks next to each
//       other (runner.shared_prefix_order), or None when no such run would change.
//   arena_update(entries, row_of, key_of, held_len, held_obj, last_use, host, step, rows, index,
//                values) -> (changed entries, changed rows) | (-1, longest) | (-2, needed)
//       The block-table arena's step (tables.BlockTableArena.update): a row per entry (claiming the
//       least recently used row for a new sequence), and the flat indices and values of the
//       table entries that differ from what each row holds. Asks for a larger arena, before
//       changing anything, when the batch needs more rows or a wider table than it has.
//       held_obj keeps, per row, the tuple it was last filled from: a scheduler rebuilds each
//       table tuple from the same int objects every step, so an unchanged table compares equal
//       by identity, element by element, without converting a single id.
//
// Buffers are NumPy arrays passed through the buffer protocol (C-contiguous, writable, of the
// stated element type); nothing here allocates Python-visible memory besides the returned lists.
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

namespace {

// A writable C-contiguous buffer of T, released on scope exit.
template <typename T>
class Buf {
 public:
  Buf() { view_.obj = nullptr; }
  ~Buf() {
    if (view_.obj != nullptr) PyBuffer_Release(&view_);
  }
  bool get(PyObject* obj, const char* what) {
    if (PyObject_GetBuffer(obj, &view_, PyBUF_WRITABLE | PyBUF_C_CONTIGUOUS | PyBUF_FORMAT) != 0) return false;
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

// A sequence attribute as a fast sequence (a new reference), or null with an exception set.
PyObject* fast_attr(PyObject* obj, PyObject* name) {
  PyObject* value = PyObject_GetAttr(obj, name);
  if (value == nullptr) return nullptr;
  PyObject* fast = PySequence_Fast(value, "a batch entry field must be a sequence");
  Py_DECREF(value);
  return fast;
}

bool as_i64(PyObject* v, int64_t* out) {
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
  long long block_size;
  if (!PyArg_ParseTuple(args, "OLOOOOOO", &entries_obj, &block_size, &tokens_o, &positions_o, &slots_o,
                        &lengths_o, &contexts_o, &logits_o)) {
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
  Buf<int64_t> tokens, positions, slots, lengths, logits;
  Buf<int32_t> contexts;
  PyObject* result = nullptr;
  std::vector<PyObject*> toks(count, nullptr), poss(count, nullptr);
  int64_t total = 0;
  if (!tokens.get(tokens_o, "tokens") || !positions.get(positions_o, "positions") ||
      !slots.get(slots_o, "slots") || !lengths.get(lengths_o, "lengths") ||
      !contexts.get(contexts_o, "contexts") || !logits.get(logits_o, "logits")) {
    goto done;
  }
  if (lengths.size() < count || contexts.size() < count || logits.size() < count) {
    PyErr_SetString(PyExc_ValueError, "per-entry buffers are shorter than the batch");
    goto done;
  }
  for (Py_ssize_t e = 0; e < count; ++e) {
    toks[e] = fast_attr(items[e], s_token_ids);
    if (toks[e] == nullptr) goto done;
    poss[e] = fast_attr(items[e], s_positions);
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
    for (Py_ssize_t e = 0; e < count; ++e) {
      PyObject* entry = items[e];
      const Py_ssize_t n = PySequence_Fast_GET_SIZE(toks[e]);
      if (PySequence_Fast_GET_SIZE(poss[e]) != n) {
        PyErr_SetString(PyExc_ValueError, "token_ids and positions must have the same length");
        goto done;
      }
      PyObject** tok = PySequence_Fast_ITEMS(toks[e]);
      PyObject** pos = PySequence_Fast_ITEMS(poss[e]);
      PyObject* table = fast_attr(entry, s_block_table);
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
        int64_t index = floor_div(p, block_size);
        if (index < 0) index += width;
        if (index >= width || index < 0) {
          if (problem == 0) {
            problem = floor_div(p, block_size) >= width ? 1 : 2;
            bad_entry = e;
            bad_position = p;
          }
          slots.data()[at + i] = -1;
          continue;
        }
        int64_t block;
        if (!as_i64(blocks[index], &block)) {
          ok = false;
          break;
        }
        slots.data()[at + i] = block * block_size + (p - floor_div(p, block_size) * block_size);
      }
      Py_DECREF(table);
      if (!ok) goto done;
      lengths.data()[e] = n;
      int64_t last = 0;
      if (n > 0) last = positions.data()[at + n - 1];
      contexts.data()[e] = static_cast<int32_t>(last + 1);
      PyObject* index = PyObject_GetAttr(entry, s_logits_index);
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
    result = Py_BuildValue("(LiLL)", static_cast<long long>(total), problem, bad_entry, bad_position);
  }
done:
  for (PyObject* o : toks) Py_XDECREF(o);
  for (PyObject* o : poss) Py_XDECREF(o);
  Py_DECREF(entries);
  return result;
}

PyObject* prefix_order(PyObject*, PyObject* args) {
  PyObject* entries_obj;
  long long lead, min_rows;
  if (!PyArg_ParseTuple(args, "OLL", &entries_obj, &lead, &min_rows)) return nullptr;
  PyObject* entries = PySequence_Fast(entries_obj, "entries must be a sequence");
  if (entries == nullptr) return nullptr;
  const Py_ssize_t count = PySequence_Fast_GET_SIZE(entries);
  PyObject** items = PySequence_Fast_ITEMS(entries);
  std::vector<Py_ssize_t> decode;
  std::vector<int64_t> keys;  // lead ids per decode entry
  PyObject* prev_table = nullptr;  // the previous decode entry's table (owned)
  std::vector<char> is_decode(count, 0);
  PyObject* result = nullptr;
  for (Py_ssize_t e = 0; e < count; ++e) {
    PyObject* tok = PyObject_GetAttr(items[e], s_token_ids);
    if (tok == nullptr) goto done;
    const Py_ssize_t n = PyObject_Length(tok);
    Py_DECREF(tok);
    if (n < 0) goto done;
    if (n != 1) continue;
    PyObject* table = fast_attr(items[e], s_block_table);
    if (table == nullptr) goto done;
    if (PySequence_Fast_GET_SIZE(table) >= lead) {
      PyObject** blocks = PySequence_Fast_ITEMS(table);
      PyObject** prev_blocks = prev_table == nullptr ? nullptr : PySequence_Fast_ITEMS(prev_table);
      const size_t at = keys.size();
      keys.resize(at + lead);
      for (long long c = 0; c < lead; ++c) {
        // Sharers' tables usually hold the very same int objects: reuse the converted id (the
        // previous table is held, so its items are alive and their addresses unique).
        if (prev_blocks != nullptr && blocks[c] == prev_blocks[c]) {
          keys[at + c] = keys[at - lead + c];
          continue;
        }
        int64_t b;
        if (!as_i64(blocks[c], &b)) {
          Py_DECREF(table);
          goto done;
        }
        keys[at + c] = b;
      }
      Py_XDECREF(prev_table);
      prev_table = table;  // keeps the reference
      decode.push_back(e);
      is_decode[e] = 1;
    } else {
      Py_DECREF(table);
    }
  }
  {
    const Py_ssize_t nd = static_cast<Py_ssize_t>(decode.size());
    if (nd < min_rows || lead < 1) {
      result = Py_None;
      Py_INCREF(result);
      goto done;
    }
    auto key = [&](Py_ssize_t k) { return keys.data() + k * lead; };
    auto same = [&](Py_ssize_t a, Py_ssize_t b) { return std::memcmp(key(a), key(b), lead * sizeof(int64_t)) == 0; };
    {  // sharers have the same first block; all-distinct first blocks: nothing to group
      std::vector<int64_t> firsts(nd);
      for (Py_ssize_t k = 0; k < nd; ++k) firsts[k] = key(k)[0];
      std::sort(firsts.begin(), firsts.end());
      if (std::adjacent_find(firsts.begin(), firsts.end()) == firsts.end()) {
        result = Py_None;
        Py_INCREF(result);
        goto done;
      }
    }
    std::vector<Py_ssize_t> grouped(nd);  // positions in `decode`, stably sorted by key
    for (Py_ssize_t k = 0; k < nd; ++k) grouped[k] = k;
    std::stable_sort(grouped.begin(), grouped.end(), [&](Py_ssize_t a, Py_ssize_t b) {
      return std::lexicographical_compare(key(a), key(a) + lead, key(b), key(b) + lead);
    });
    Py_ssize_t shared = 0, adjacent = 0;
    for (Py_ssize_t k = 0; k + 1 < nd; ++k) {
      shared += same(grouped[k], grouped[k + 1]);
      if (decode[k + 1] == decode[k] + 1) adjacent += same(k, k + 1);
    }
    if (shared == 0 || shared == adjacent) {
      result = Py_None;
      Py_INCREF(result);
      goto done;
    }
    result = PyList_New(count);
    if (result == nullptr) goto done;
    Py_ssize_t at = 0;
    for (Py_ssize_t k = 0; k < nd; ++k) PyList_SET_ITEM(result, at++, PyLong_FromSsize_t(decode[grouped[k]]));
    for (Py_ssize_t e = 0; e < count; ++e) {
      if (!is_decode[e]) PyList_SET_ITEM(result, at++, PyLong_FromSsize_t(e));
    }
  }
done:
  Py_XDECREF(prev_table);
  Py_DECREF(entries);
  return result;
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
    tables[e] = fast_attr(items[e], s_block_table);
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
    PyObject* seen = PyDict_New();  // seq id -> occurrences so far in this batch
    if (seen == nullptr) goto done;
    bool ok = true;
    for (Py_ssize_t e = 0; e < count && ok; ++e) {
      PyObject* seq_id = PyObject_GetAttr(items[e], s_seq_id);
      if (seq_id == nullptr) {
        ok = false;
        break;
      }
      PyObject* key = seq_id;  // the same sequence twice in one batch gets a row per occurrence
      PyObject* prior = PyDict_GetItemWithError(seen, seq_id);
      long long repeat = 0;
      if (prior != nullptr) repeat = PyLong_AsLongLong(prior);
      else if (PyErr_Occurred()) ok = false;
      PyObject* next = ok ? PyLong_FromLongLong(repeat + 1) : nullptr;
      if (next == nullptr || PyDict_SetItem(seen, seq_id, next) != 0) ok = false;
      Py_XDECREF(next);
      if (ok && repeat > 0) {
        key = Py_BuildValue("(OL)", seq_id, repeat);
        if (key == nullptr) ok = false;
      } else {
        Py_INCREF(key);
      }
      Py_DECREF(seq_id);
      if (!ok) break;
      Py_ssize_t row = -1;
      PyObject* found = PyDict_GetItemWithError(row_of, key);
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
      PyObject* before = PyList_GET_ITEM(held_obj, row);
      if (is_tuple && before != Py_None && heldp[row] == n) {
        const int same = PyObject_RichCompareBool(tables[e], before, Py_EQ);
        if (same < 0) {
          ok = false;
          break;
        }
        if (same == 1) continue;  // the row already holds this table
      }
      int32_t* mirror = hostp + row * width;
      const Py_ssize_t old = heldp[row];
      Py_ssize_t start = 0;
      const Py_ssize_t common = std::min(old, n);
      for (; start < common; ++start) {
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
    Py_DECREF(seen);
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

PyMethodDef kMethods[] = {
    {"gather", gather, METH_VARARGS, "Flatten a batch: tokens, positions, slots, lengths, contexts, logits rows."},
    {"prefix_order", prefix_order, METH_VARARGS, "Row order grouping decode entries that share leading blocks."},
    {"arena_update", arena_update, METH_VARARGS, "One step of the block-table arena."},
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
  return PyModule_Create(&kModule);
}
