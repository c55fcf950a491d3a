// Host tick core of the CDB engine: the per-launch loops over depth work items,
// as a CPython extension (built with g++, no GPU code).
//
//   route_sync      routes one recurrent launch's rows on the synchronous exit
//                   horizon (cdb/continuous_api.py:1090-1183 with _record_exit
//                   :1205-1223): exits go to the coda list, the rest step on.
//   route_lists     route_sync from the device's routing lists (cdb_route_compact):
//                   the exiting rows, then the staying rows, each in launch order.
//   route_delayed   the same on the offset-one horizon, from each row's previous
//                   launch's decision (cdb/continuous_api.py:1124-1141).
//   fill_recurrent  writes one launch's packed metadata into the pinned staging
//                   arrays (cdb/model_runner.py:704-754 assembles the same facts).
//   BlockPool       the paged cache's block manager: FIFO free list, allocated
//                   map and peak (continuous_batching/cache_manager.py:72-90).
//   ItemQueue       the scheduler's depth and coda queues of work items, with
//                   enqueue_front / pop_batch / pop_front for the per-tick
//                   head re-insertion and bucket selection
//                   (continuous_depth_batching/scheduler.py:101-180, 322-346).
//   split_live      drops work items of finished requests before a launch.
//   select_eager    chooses a coda's eager successors (cdb/continuous_api.py:1304-1327).
//   coda_upload     a coda launch's slot upload and its successors' hidden slots.
//   consume_coda    a coda batch's sampled tokens: token append and finish checks
//                   (continuous_batching/requests.py:208-237) row by row.
//   schedule_next   the scheduler's per-tick bucket choice (coda > prefill > recurrent >
//                   undersized coda) with prompt admission and chunking
//                   (continuous_depth_batching/scheduler.py:101-140, 205-296;
//                   continuous_batching/scheduler_base.py:171-201, 416-545).
//
// The functions read and write the engine's own Python objects (DepthWorkItem,
// RequestState), so request state stays in one place; they replace the
// interpreter's per-row work, which is on the path between a launch's exit
// flags and the next launch.

#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <deque>
#include <vector>

namespace {

PyObject* s_recurrent_step;
PyObject* s_apply_exit_gate;
PyObject* s_state;
PyObject* s_current_token_exit_depth;
PyObject* s_exit_depths;
PyObject* s_hidden_slot;
PyObject* s_token_position;
PyObject* s_request_id;
PyObject* s_synthetic_exit_depth;
PyObject* s_status_field;
PyObject* s_position_offset;
PyObject* s_allocated_blocks;
PyObject* s_tokens_in_flight;
PyObject* s_generated_tokens;
PyObject* s_new_tokens_limit;
PyObject* s_replay_eos_finishes;
PyObject* s_next_synthetic_exit_depth;

// Metadata rows of the int32 block, as ModelRunner.META_* names them.
constexpr int kMetaPositions = 0, kMetaTableRows = 1, kMetaLayerOffset = 2, kMetaSteps = 3, kMetaSynthetic = 4;
constexpr int kMetaRows = 5;

bool get_long(PyObject* obj, PyObject* name, long* out) {
  PyObject* v = PyObject_GetAttr(obj, name);
  if (!v) return false;
  *out = PyLong_AsLong(v);
  Py_DECREF(v);
  return !(*out == -1 && PyErr_Occurred());
}

int get_truth(PyObject* obj, PyObject* name) {
  PyObject* v = PyObject_GetAttr(obj, name);
  if (!v) return -1;
  int t = PyObject_IsTrue(v);
  Py_DECREF(v);
  return t;
}

bool set_long(PyObject* obj, PyObject* name, long value) {
  PyObject* v = PyLong_FromLong(value);
  if (!v) return false;
  int rc = PyObject_SetAttr(obj, name, v);
  Py_DECREF(v);
  return rc == 0;
}

// hist[step] += 1 on a dict (a collections.Counter counts as one).
bool bump(PyObject* hist, long step) {
  PyObject* key = PyLong_FromLong(step);
  if (!key) return false;
  PyObject* cur = PyDict_GetItemWithError(hist, key);  // borrowed
  long n = 0;
  if (cur) {
    n = PyLong_AsLong(cur);
    if (n == -1 && PyErr_Occurred()) { Py_DECREF(key); return false; }
  } else if (PyErr_Occurred()) {
    Py_DECREF(key);
    return false;
  }
  PyObject* val = PyLong_FromLong(n + 1);
  int rc = val ? PyDict_SetItem(hist, key, val) : -1;
  Py_XDECREF(val);
  Py_DECREF(key);
  return rc == 0;
}

// Record an exit at `step` on the item's request (the _record_exit bookkeeping
// that the synchronous horizon needs; exit-KV copies are appended to backlog).
bool record_exit(PyObject* item, long step, int apply, PyObject* hist, PyObject* backlog, long max_steps) {
  if (apply) {
    PyObject* state = PyObject_GetAttr(item, s_state);
    if (!state) return false;
    bool ok = set_long(state, s_current_token_exit_depth, step);
    if (ok) {
      PyObject* depths = PyObject_GetAttr(state, s_exit_depths);
      ok = depths != nullptr;
      if (ok) {
        PyObject* v = PyLong_FromLong(step);
        ok = v && PyList_Check(depths) && PyList_Append(depths, v) == 0;
        if (!ok && !PyErr_Occurred()) PyErr_SetString(PyExc_TypeError, "state.exit_depths must be a list");
        Py_XDECREF(v);
        Py_DECREF(depths);
      }
    }
    Py_DECREF(state);
    if (!ok || !bump(hist, step)) return false;
  }
  if (backlog != Py_None && step < max_steps - 1) {
    PyObject* entry = Py_BuildValue("(Ol)", item, step);
    if (!entry) return false;
    int rc = PyList_Append(backlog, entry);
    Py_DECREF(entry);
    if (rc) return false;
  }
  return true;
}

PyObject* route_sync(PyObject*, PyObject* args) {
  PyObject *items, *flags_obj, *hist, *backlog;
  long max_steps;
  if (!PyArg_ParseTuple(args, "O!OlO!O", &PyList_Type, &items, &flags_obj, &max_steps, &PyDict_Type, &hist,
                        &backlog))
    return nullptr;
  if (backlog != Py_None && !PyList_Check(backlog)) {
    PyErr_SetString(PyExc_TypeError, "backlog must be a list or None");
    return nullptr;
  }
  Py_buffer flags;
  if (PyObject_GetBuffer(flags_obj, &flags, PyBUF_SIMPLE) != 0) return nullptr;
  const Py_ssize_t n = PyList_GET_SIZE(items);
  if (flags.len < n) {
    PyBuffer_Release(&flags);
    PyErr_SetString(PyExc_ValueError, "fewer exit flags than items");
    return nullptr;
  }
  const uint8_t* f = static_cast<const uint8_t*>(flags.buf);
  PyObject* coda = PyList_New(0);
  PyObject* refills = PyList_New(0);
  PyObject* exits = PyList_New(n);
  bool ok = coda && refills && exits;
  for (Py_ssize_t i = 0; ok && i < n; ++i) {
    PyObject* item = PyList_GET_ITEM(items, i);
    long step;
    int apply = get_truth(item, s_apply_exit_gate);
    ok = apply >= 0 && get_long(item, s_recurrent_step, &step);
    if (!ok) break;
    const bool leave = apply ? f[i] != 0 : step == max_steps - 1;
    PyObject* b = leave ? Py_True : Py_False;
    Py_INCREF(b);
    PyList_SET_ITEM(exits, i, b);
    if (leave) {
      ok = record_exit(item, step, apply, hist, backlog, max_steps) && PyList_Append(coda, item) == 0;
    } else {
      ok = set_long(item, s_recurrent_step, step + 1) && PyList_Append(refills, item) == 0;
    }
  }
  PyBuffer_Release(&flags);
  if (!ok) {
    Py_XDECREF(coda);
    Py_XDECREF(refills);
    Py_XDECREF(exits);
    return nullptr;
  }
  return Py_BuildValue("(NNN)", coda, refills, exits);
}

// route_lists(items, lists, max_steps, histogram, backlog) -> (coda_items, refills, exits)
// lists = [n_exit, n_stay, exiting rows..., staying rows...] as cdb_route_compact writes it. The
// lists must cover every row once, each in launch order; every row must apply the exit gate
// (the device lists carry the gate's decisions only).
PyObject* route_lists(PyObject*, PyObject* args) {
  PyObject *items, *lists_obj, *hist, *backlog;
  long max_steps;
  if (!PyArg_ParseTuple(args, "O!OlO!O", &PyList_Type, &items, &lists_obj, &max_steps, &PyDict_Type, &hist,
                        &backlog))
    return nullptr;
  if (backlog != Py_None && !PyList_Check(backlog)) {
    PyErr_SetString(PyExc_TypeError, "backlog must be a list or None");
    return nullptr;
  }
  Py_buffer buf;
  if (PyObject_GetBuffer(lists_obj, &buf, PyBUF_SIMPLE) != 0) return nullptr;
  const Py_ssize_t n = PyList_GET_SIZE(items);
  const int32_t* lists = static_cast<const int32_t*>(buf.buf);
  const Py_ssize_t have = buf.len / 4;
  const int32_t n_exit = have >= 2 ? lists[0] : -1, n_stay = have >= 2 ? lists[1] : -1;
  bool ok = n_exit >= 0 && n_stay >= 0 && n_exit + n_stay == n && have >= 2 + n;
  // Each list strictly increasing and together a partition of the rows.
  std::vector<uint8_t> seen(n, 0);
  for (int32_t k = 0; ok && k < n_exit + n_stay; ++k) {
    const int32_t r = lists[2 + k];
    const bool rising = k == 0 || k == n_exit || r > lists[1 + k];
    ok = r >= 0 && r < n && rising && !seen[r];
    if (ok) seen[r] = 1;
  }
  if (!ok) {
    PyBuffer_Release(&buf);
    PyErr_SetString(PyExc_ValueError, "routing lists do not partition the launch's rows in launch order");
    return nullptr;
  }
  PyObject* coda = PyList_New(0);
  PyObject* refills = PyList_New(0);
  PyObject* exits = PyList_New(n);
  ok = coda && refills && exits;
  for (Py_ssize_t i = 0; ok && i < n; ++i) {
    Py_INCREF(Py_False);
    PyList_SET_ITEM(exits, i, Py_False);
  }
  for (int32_t k = 0; ok && k < n_exit + n_stay; ++k) {
    const int32_t r = lists[2 + k];
    PyObject* item = PyList_GET_ITEM(items, r);
    long step;
    const int apply = get_truth(item, s_apply_exit_gate);
    ok = apply >= 0 && get_long(item, s_recurrent_step, &step);
    if (ok && !apply) {
      PyErr_SetString(PyExc_ValueError, "device routing needs every row to apply the exit gate");
      ok = false;
    }
    if (!ok) break;
    if (k < n_exit) {
      ok = record_exit(item, step, 1, hist, backlog, max_steps) && PyList_Append(coda, item) == 0;
      if (ok) {
        Py_INCREF(Py_True);
        PyList_SetItem(exits, r, Py_True);  // releases the False it replaces
      }
    } else {
      ok = set_long(item, s_recurrent_step, step + 1) && PyList_Append(refills, item) == 0;
    }
  }
  PyBuffer_Release(&buf);
  if (!ok) {
    Py_XDECREF(coda);
    Py_XDECREF(refills);
    Py_XDECREF(exits);
    return nullptr;
  }
  return Py_BuildValue("(NNN)", coda, refills, exits);
}

PyObject* fill_recurrent(PyObject*, PyObject* args) {
  PyObject *items, *i64_obj, *i32_obj, *row_of, *slot_of_step;
  long core_base, core_layers;
  if (!PyArg_ParseTuple(args, "O!OOO!llO!", &PyList_Type, &items, &i64_obj, &i32_obj, &PyDict_Type, &row_of,
                        &core_base, &core_layers, &PyTuple_Type, &slot_of_step))
    return nullptr;
  Py_buffer b64, b32;
  if (PyObject_GetBuffer(i64_obj, &b64, PyBUF_WRITABLE | PyBUF_C_CONTIGUOUS) != 0) return nullptr;
  if (PyObject_GetBuffer(i32_obj, &b32, PyBUF_WRITABLE | PyBUF_C_CONTIGUOUS) != 0) {
    PyBuffer_Release(&b64);
    return nullptr;
  }
  const Py_ssize_t n = PyList_GET_SIZE(items);
  const Py_ssize_t rows = b64.len / 8;
  const Py_ssize_t steps = PyTuple_GET_SIZE(slot_of_step);
  bool ok = true;
  if (b64.len % 8 || b32.len != (Py_ssize_t)(kMetaRows * rows * 4) || n > rows) {
    PyErr_SetString(PyExc_ValueError, "metadata buffers must be int64[rows] and int32[5, rows], rows >= items");
    ok = false;
  }
  int64_t* i64 = static_cast<int64_t*>(b64.buf);
  int32_t* i32 = static_cast<int32_t*>(b32.buf);
  for (Py_ssize_t r = 0; ok && r < n; ++r) {
    PyObject* item = PyList_GET_ITEM(items, r);
    long slot, pos, step;
    ok = get_long(item, s_hidden_slot, &slot) && get_long(item, s_token_position, &pos) &&
         get_long(item, s_recurrent_step, &step);
    if (!ok) break;
    if (step < 0 || step >= steps || pos < -1 || pos > INT32_MAX) {
      PyErr_Format(PyExc_ValueError, "row %zd: step %ld or position %ld out of range", r, step, pos);
      ok = false;
      break;
    }
    PyObject* state = PyObject_GetAttr(item, s_state);
    PyObject* rid = state ? PyObject_GetAttr(state, s_request_id) : nullptr;
    Py_XDECREF(state);
    PyObject* row = rid ? PyDict_GetItemWithError(row_of, rid) : nullptr;  // borrowed
    if (rid && !row && !PyErr_Occurred()) PyErr_SetObject(PyExc_KeyError, rid);
    Py_XDECREF(rid);
    if (!row) { ok = false; break; }
    const long table_row = PyLong_AsLong(row);
    const long slot_index = PyLong_AsLong(PyTuple_GET_ITEM(slot_of_step, step));
    if (PyErr_Occurred()) { ok = false; break; }
    long synth = -1;
    int apply = get_truth(item, s_apply_exit_gate);
    if (apply < 0) { ok = false; break; }
    PyObject* d = PyObject_GetAttr(item, s_synthetic_exit_depth);
    if (!d) { ok = false; break; }
    if (apply && d != Py_None) synth = PyLong_AsLong(d);
    Py_DECREF(d);
    if (synth == -1 && PyErr_Occurred()) { ok = false; break; }
    i64[r] = slot;
    i32[kMetaPositions * rows + r] = (int32_t)pos;
    i32[kMetaTableRows * rows + r] = (int32_t)table_row;
    i32[kMetaLayerOffset * rows + r] = (int32_t)(core_base + slot_index * core_layers);
    i32[kMetaSteps * rows + r] = (int32_t)step;
    i32[kMetaSynthetic * rows + r] = (int32_t)synth;
  }
  if (ok) {
    for (Py_ssize_t r = n; r < rows; ++r) {  // padding rows: no-ops in every kernel
      i64[r] = -1;
      i32[kMetaPositions * rows + r] = -1;
      i32[kMetaTableRows * rows + r] = 0;
      i32[kMetaLayerOffset * rows + r] = (int32_t)core_base;
      i32[kMetaSteps * rows + r] = 0;
      i32[kMetaSynthetic * rows + r] = -1;
    }
  }
  PyBuffer_Release(&b64);
  PyBuffer_Release(&b32);
  if (!ok) return nullptr;
  Py_RETURN_NONE;
}

// ---------------------------------------------------------------------------
// BlockPool: block ids handed out FIFO (popleft on allocate, append on free),
// with the allocated map guarding double frees and the peak count.
// ---------------------------------------------------------------------------
struct BlockPool {
  PyObject_HEAD
  std::deque<int32_t>* free_list;
  std::vector<uint8_t>* allocated;
  Py_ssize_t num_blocks, block_size, num_allocated, peak;
};

PyObject* BlockPool_new(PyTypeObject* type, PyObject* args, PyObject* kwds) {
  Py_ssize_t num_blocks = 0, block_size = 0;
  static const char* kw[] = {"num_blocks", "block_size", nullptr};
  if (!PyArg_ParseTupleAndKeywords(args, kwds, "n|n", const_cast<char**>(kw), &num_blocks, &block_size))
    return nullptr;
  if (num_blocks < 0 || num_blocks > INT32_MAX) {
    PyErr_SetString(PyExc_ValueError, "num_blocks must be in [0, 2^31)");
    return nullptr;
  }
  BlockPool* self = reinterpret_cast<BlockPool*>(type->tp_alloc(type, 0));
  if (!self) return nullptr;
  self->free_list = new std::deque<int32_t>();
  for (Py_ssize_t b = 0; b < num_blocks; ++b) self->free_list->push_back((int32_t)b);
  self->allocated = new std::vector<uint8_t>((size_t)num_blocks, 0);
  self->num_blocks = num_blocks;
  self->block_size = block_size;
  self->num_allocated = 0;
  self->peak = 0;
  return reinterpret_cast<PyObject*>(self);
}

void BlockPool_dealloc(PyObject* obj) {
  BlockPool* self = reinterpret_cast<BlockPool*>(obj);
  delete self->free_list;
  delete self->allocated;
  Py_TYPE(obj)->tp_free(obj);
}

PyObject* BlockPool_get_free_blocks(PyObject* obj, PyObject* arg) {
  BlockPool* self = reinterpret_cast<BlockPool*>(obj);
  const Py_ssize_t n = PyLong_AsSsize_t(arg);
  if (n == -1 && PyErr_Occurred()) return nullptr;
  if (n < 0) {
    PyErr_SetString(PyExc_ValueError, "cannot take a negative number of blocks");
    return nullptr;
  }
  if ((Py_ssize_t)self->free_list->size() < n) Py_RETURN_NONE;
  PyObject* out = PyList_New(n);
  if (!out) return nullptr;
  for (Py_ssize_t i = 0; i < n; ++i) {
    const int32_t b = self->free_list->front();
    PyObject* v = PyLong_FromLong(b);
    if (!v) {  // nothing was taken yet for this entry; return the ones already taken
      for (Py_ssize_t j = i - 1; j >= 0; --j) {
        const int32_t t = (int32_t)PyLong_AsLong(PyList_GET_ITEM(out, j));
        (*self->allocated)[t] = 0;
        self->free_list->push_front(t);
      }
      self->num_allocated -= i;
      Py_DECREF(out);
      return nullptr;
    }
    self->free_list->pop_front();
    (*self->allocated)[b] = 1;
    PyList_SET_ITEM(out, i, v);
  }
  self->num_allocated += n;
  self->peak = std::max(self->peak, self->num_allocated);
  return out;
}

PyObject* BlockPool_free_blocks(PyObject* obj, PyObject* arg) {
  BlockPool* self = reinterpret_cast<BlockPool*>(obj);
  PyObject* it = PyObject_GetIter(arg);
  if (!it) return nullptr;
  PyObject* v;
  while ((v = PyIter_Next(it))) {
    const long b = PyLong_AsLong(v);
    Py_DECREF(v);
    if (b == -1 && PyErr_Occurred()) break;
    if (b < 0 || b >= self->num_blocks || !(*self->allocated)[b]) {
      PyErr_Format(PyExc_ValueError, "Cannot free block %ld: block is not currently allocated", b);
      break;
    }
    (*self->allocated)[b] = 0;
    --self->num_allocated;
    self->free_list->push_back((int32_t)b);
  }
  Py_DECREF(it);
  if (PyErr_Occurred()) return nullptr;
  Py_RETURN_NONE;
}

PyObject* BlockPool_free_list(PyObject* obj, PyObject*) {
  BlockPool* self = reinterpret_cast<BlockPool*>(obj);
  PyObject* out = PyList_New((Py_ssize_t)self->free_list->size());
  if (!out) return nullptr;
  Py_ssize_t i = 0;
  for (int32_t b : *self->free_list) {
    PyObject* v = PyLong_FromLong(b);
    if (!v) { Py_DECREF(out); return nullptr; }
    PyList_SET_ITEM(out, i++, v);
  }
  return out;
}

PyObject* BlockPool_reset_peak_usage(PyObject* obj, PyObject*) {
  BlockPool* self = reinterpret_cast<BlockPool*>(obj);
  self->peak = self->num_allocated;
  Py_RETURN_NONE;
}

PyObject* BlockPool_num_free(PyObject* obj, void*) {
  return PyLong_FromSsize_t((Py_ssize_t)reinterpret_cast<BlockPool*>(obj)->free_list->size());
}
PyObject* BlockPool_num_allocated(PyObject* obj, void*) {
  return PyLong_FromSsize_t(reinterpret_cast<BlockPool*>(obj)->num_allocated);
}
PyObject* BlockPool_peak(PyObject* obj, void*) { return PyLong_FromSsize_t(reinterpret_cast<BlockPool*>(obj)->peak); }
PyObject* BlockPool_num_blocks(PyObject* obj, void*) {
  return PyLong_FromSsize_t(reinterpret_cast<BlockPool*>(obj)->num_blocks);
}
PyObject* BlockPool_block_size(PyObject* obj, void*) {
  return PyLong_FromSsize_t(reinterpret_cast<BlockPool*>(obj)->block_size);
}

PyMethodDef kBlockPoolMethods[] = {
    {"get_free_blocks", BlockPool_get_free_blocks, METH_O,
     "get_free_blocks(n) -> the next n free block ids (FIFO), or None when fewer are free"},
    {"free_blocks", BlockPool_free_blocks, METH_O, "free_blocks(blocks): return blocks to the end of the free list"},
    {"free_list", BlockPool_free_list, METH_NOARGS, "free_list() -> the free block ids in hand-out order"},
    {"reset_peak_usage", BlockPool_reset_peak_usage, METH_NOARGS, "reset_peak_usage(): peak = allocated now"},
    {nullptr, nullptr, 0, nullptr},
};

PyGetSetDef kBlockPoolGetSet[] = {
    {"num_free_blocks", BlockPool_num_free, nullptr, nullptr, nullptr},
    {"num_allocated_blocks", BlockPool_num_allocated, nullptr, nullptr, nullptr},
    {"peak_num_allocated_blocks", BlockPool_peak, nullptr, nullptr, nullptr},
    {"num_blocks", BlockPool_num_blocks, nullptr, nullptr, nullptr},
    {"block_size", BlockPool_block_size, nullptr, nullptr, nullptr},
    {nullptr, nullptr, nullptr, nullptr, nullptr},
};

PyTypeObject BlockPoolType = {PyVarObject_HEAD_INIT(nullptr, 0)};

// ---------------------------------------------------------------------------
// ItemQueue: a deque of work items (strong references) with the sequence
// protocol, so the scheduler's queues can be iterated, measured and cleared
// from Python while the per-tick batch operations below run in C++.
// ---------------------------------------------------------------------------
struct ItemQueue {
  PyObject_HEAD
  std::deque<PyObject*>* items;
};

bool is_queue(PyObject* obj);

PyObject* ItemQueue_new(PyTypeObject* type, PyObject* args, PyObject* kwds) {
  if (!PyArg_ParseTuple(args, ":ItemQueue") || (kwds && PyDict_Size(kwds))) {
    if (!PyErr_Occurred()) PyErr_SetString(PyExc_TypeError, "ItemQueue() takes no arguments");
    return nullptr;
  }
  ItemQueue* self = reinterpret_cast<ItemQueue*>(type->tp_alloc(type, 0));
  if (!self) return nullptr;
  self->items = new std::deque<PyObject*>();
  return reinterpret_cast<PyObject*>(self);
}

int ItemQueue_traverse(PyObject* obj, visitproc visit, void* arg) {
  ItemQueue* self = reinterpret_cast<ItemQueue*>(obj);
  if (self->items)
    for (PyObject* it : *self->items) Py_VISIT(it);
  return 0;
}

int ItemQueue_clear_refs(PyObject* obj) {
  ItemQueue* self = reinterpret_cast<ItemQueue*>(obj);
  if (self->items) {
    std::deque<PyObject*> old;
    old.swap(*self->items);
    for (PyObject* it : old) Py_DECREF(it);
  }
  return 0;
}

void ItemQueue_dealloc(PyObject* obj) {
  PyObject_GC_UnTrack(obj);
  ItemQueue_clear_refs(obj);
  delete reinterpret_cast<ItemQueue*>(obj)->items;
  Py_TYPE(obj)->tp_free(obj);
}

Py_ssize_t ItemQueue_len(PyObject* obj) { return (Py_ssize_t)reinterpret_cast<ItemQueue*>(obj)->items->size(); }

PyObject* ItemQueue_snapshot(ItemQueue* self) {
  PyObject* out = PyList_New((Py_ssize_t)self->items->size());
  if (!out) return nullptr;
  Py_ssize_t i = 0;
  for (PyObject* it : *self->items) {
    Py_INCREF(it);
    PyList_SET_ITEM(out, i++, it);
  }
  return out;
}

PyObject* ItemQueue_iter(PyObject* obj) {
  PyObject* snap = ItemQueue_snapshot(reinterpret_cast<ItemQueue*>(obj));
  if (!snap) return nullptr;
  PyObject* it = PyObject_GetIter(snap);
  Py_DECREF(snap);
  return it;
}

PyObject* ItemQueue_append(PyObject* obj, PyObject* item) {
  Py_INCREF(item);
  reinterpret_cast<ItemQueue*>(obj)->items->push_back(item);
  Py_RETURN_NONE;
}

PyObject* ItemQueue_appendleft(PyObject* obj, PyObject* item) {
  Py_INCREF(item);
  reinterpret_cast<ItemQueue*>(obj)->items->push_front(item);
  Py_RETURN_NONE;
}

PyObject* ItemQueue_popleft(PyObject* obj, PyObject*) {
  auto* q = reinterpret_cast<ItemQueue*>(obj)->items;
  if (q->empty()) {
    PyErr_SetString(PyExc_IndexError, "pop from an empty ItemQueue");
    return nullptr;
  }
  PyObject* it = q->front();
  q->pop_front();
  return it;  // the queue's reference passes to the caller
}

PyObject* ItemQueue_extend(PyObject* obj, PyObject* iterable) {
  PyObject* seq = PySequence_Fast(iterable, "ItemQueue.extend needs an iterable");
  if (!seq) return nullptr;
  auto* q = reinterpret_cast<ItemQueue*>(obj)->items;
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(seq);
  PyObject** items = PySequence_Fast_ITEMS(seq);
  for (Py_ssize_t i = 0; i < n; ++i) {
    Py_INCREF(items[i]);
    q->push_back(items[i]);
  }
  Py_DECREF(seq);
  Py_RETURN_NONE;
}

PyObject* ItemQueue_clear(PyObject* obj, PyObject*) {
  ItemQueue_clear_refs(obj);
  Py_RETURN_NONE;
}

PyMethodDef kItemQueueMethods[] = {
    {"append", ItemQueue_append, METH_O, "append(item)"},
    {"appendleft", ItemQueue_appendleft, METH_O, "appendleft(item)"},
    {"popleft", ItemQueue_popleft, METH_NOARGS, "popleft() -> item"},
    {"extend", ItemQueue_extend, METH_O, "extend(items)"},
    {"clear", ItemQueue_clear, METH_NOARGS, "clear()"},
    {nullptr, nullptr, 0, nullptr},
};

PySequenceMethods kItemQueueSeq = {};
PyTypeObject ItemQueueType = {PyVarObject_HEAD_INIT(nullptr, 0)};

bool is_queue(PyObject* obj) { return PyObject_TypeCheck(obj, &ItemQueueType); }

bool get_state_rid(PyObject* item, PyObject** rid) {
  PyObject* state = PyObject_GetAttr(item, s_state);
  if (!state) return false;
  *rid = PyObject_GetAttr(state, s_request_id);
  Py_DECREF(state);
  return *rid != nullptr;
}

// enqueue_front(queue, items, max_steps, in_flight) -> refill events added.
// The items return to the queue head in their order (continuous_depth_batching/
// scheduler.py:164-180): applied from the last item to the first, each request
// marked in flight, and a step-0 item landing on a non-empty queue counting as
// a refill. Peak counters are left to the caller (they only grow here).
PyObject* enqueue_front(PyObject*, PyObject* args) {
  PyObject *queue, *items, *in_flight;
  long max_steps;
  if (!PyArg_ParseTuple(args, "OO!lO!", &queue, &PyList_Type, &items, &max_steps, &PySet_Type, &in_flight))
    return nullptr;
  if (!is_queue(queue)) {
    PyErr_SetString(PyExc_TypeError, "queue must be an ItemQueue");
    return nullptr;
  }
  auto* q = reinterpret_cast<ItemQueue*>(queue)->items;
  long refills = 0;
  for (Py_ssize_t i = PyList_GET_SIZE(items) - 1; i >= 0; --i) {
    PyObject* item = PyList_GET_ITEM(items, i);
    long step;
    if (!get_long(item, s_recurrent_step, &step)) return nullptr;
    if (step < 0 || step >= max_steps) {
      PyErr_Format(PyExc_ValueError, "recurrent_step must be in [0, %ld), got %ld", max_steps, step);
      return nullptr;
    }
    PyObject* rid;
    if (!get_state_rid(item, &rid)) return nullptr;
    const int rc = PySet_Add(in_flight, rid);
    Py_DECREF(rid);
    if (rc) return nullptr;
    if (step == 0 && !q->empty()) ++refills;
    Py_INCREF(item);
    q->push_front(item);
  }
  return PyLong_FromLong(refills);
}

// pop_batch(queue, size, slot_of_step) -> the next recurrent batch (scheduler.py:322-346):
// the head item, then up to size - 1 more in queue order. With slot_of_step (a tuple,
// the KV slot each step writes) only items writing the head item's slot are taken;
// skipped items keep their order ahead of the untouched rest.
PyObject* pop_batch_from(std::deque<PyObject*>* q, Py_ssize_t size, PyObject* slot_of_step) {
  const bool filter = slot_of_step != Py_None;
  if (filter && !PyTuple_Check(slot_of_step)) {
    PyErr_SetString(PyExc_TypeError, "slot_of_step must be a tuple or None");
    return nullptr;
  }
  PyObject* batch = PyList_New(0);
  if (!batch || size <= 0 || q->empty()) return batch;
  auto slot_of = [&](PyObject* item, long* slot) -> bool {
    long step;
    if (!get_long(item, s_recurrent_step, &step)) return false;
    if (step < 0 || step >= PyTuple_GET_SIZE(slot_of_step)) {
      PyErr_Format(PyExc_ValueError, "recurrent_step %ld has no KV slot", step);
      return false;
    }
    *slot = PyLong_AsLong(PyTuple_GET_ITEM(slot_of_step, step));
    return !(*slot == -1 && PyErr_Occurred());
  };
  long target = 0;
  if (filter && !slot_of(q->front(), &target)) {
    Py_DECREF(batch);
    return nullptr;
  }
  std::vector<PyObject*> skipped;
  bool ok = true;
  while (ok && !q->empty() && PyList_GET_SIZE(batch) < size) {
    PyObject* item = q->front();
    long slot = target;
    if (filter && PyList_GET_SIZE(batch) > 0 && !slot_of(item, &slot)) { ok = false; break; }
    q->pop_front();
    if (slot == target) {
      ok = PyList_Append(batch, item) == 0;
      Py_DECREF(item);
    } else {
      skipped.push_back(item);  // keeps the queue's reference
    }
  }
  for (auto it = skipped.rbegin(); it != skipped.rend(); ++it) q->push_front(*it);
  if (!ok) {  // put the batch back at the head, in order, and report the error
    for (Py_ssize_t i = PyList_GET_SIZE(batch) - 1; i >= 0; --i) {
      PyObject* item = PyList_GET_ITEM(batch, i);
      Py_INCREF(item);
      q->push_front(item);
    }
    Py_DECREF(batch);
    return nullptr;
  }
  return batch;
}

PyObject* pop_batch(PyObject*, PyObject* args) {
  PyObject *queue, *slot_of_step;
  Py_ssize_t size;
  if (!PyArg_ParseTuple(args, "OnO", &queue, &size, &slot_of_step)) return nullptr;
  if (!is_queue(queue)) {
    PyErr_SetString(PyExc_TypeError, "queue must be an ItemQueue");
    return nullptr;
  }
  return pop_batch_from(reinterpret_cast<ItemQueue*>(queue)->items, size, slot_of_step);
}

// pop_front(queue, n) -> the first min(n, len) items.
PyObject* pop_front_from(std::deque<PyObject*>* q, Py_ssize_t n) {
  const Py_ssize_t k = std::max<Py_ssize_t>(0, std::min<Py_ssize_t>(n, (Py_ssize_t)q->size()));
  PyObject* out = PyList_New(k);
  if (!out) return nullptr;
  for (Py_ssize_t i = 0; i < k; ++i) {
    PyList_SET_ITEM(out, i, q->front());  // the queue's reference moves into the list
    q->pop_front();
  }
  return out;
}

PyObject* pop_front(PyObject*, PyObject* args) {
  PyObject* queue;
  Py_ssize_t n;
  if (!PyArg_ParseTuple(args, "On", &queue, &n)) return nullptr;
  if (!is_queue(queue)) {
    PyErr_SetString(PyExc_TypeError, "queue must be an ItemQueue");
    return nullptr;
  }
  return pop_front_from(reinterpret_cast<ItemQueue*>(queue)->items, n);
}

// split_live(items, finished) -> (live, dead): work items whose request status
// (RequestState._status) differs from `finished`, and the others, in order.
PyObject* split_live(PyObject*, PyObject* args) {
  PyObject* items;
  long finished;
  if (!PyArg_ParseTuple(args, "O!l", &PyList_Type, &items, &finished)) return nullptr;
  const Py_ssize_t n = PyList_GET_SIZE(items);
  PyObject* live = PyList_New(0);
  PyObject* dead = PyList_New(0);
  if (!live || !dead) { Py_XDECREF(live); Py_XDECREF(dead); return nullptr; }
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* item = PyList_GET_ITEM(items, i);
    PyObject* state = PyObject_GetAttr(item, s_state);
    if (!state) { Py_DECREF(live); Py_DECREF(dead); return nullptr; }
    long status;
    const bool got = get_long(state, s_status_field, &status);
    Py_DECREF(state);
    if (!got || PyList_Append(status == finished ? dead : live, item)) {
      Py_DECREF(live);
      Py_DECREF(dead);
      return nullptr;
    }
  }
  return Py_BuildValue("(NN)", live, dead);
}

// select_eager(coda_items, block_size, allocate, item_type, token) -> (items, rows, flags)
// The eager re-entries of a coda batch (cdb/continuous_api.py:1304-1327): every row whose
// request does not finish on its pending token (continuous_batching/requests.py:196-206:
// tokens in flight reach the length limit, unless EOS replay decides) advances its
// position by one and keeps a KV slot for it -- the request's last block when the new
// position still fits it, else allocate(state) (which takes blocks) -- and gets a successor
// item_type(state, token, position, 0, state.next_synthetic_exit_depth()) with its
// current exit depth cleared. A row that cannot get a slot keeps its position.
PyObject* select_eager(PyObject*, PyObject* args) {
  PyObject *coda, *allocate, *item_type, *token;
  long block_size;
  if (!PyArg_ParseTuple(args, "O!lOOO", &PyList_Type, &coda, &block_size, &allocate, &item_type, &token))
    return nullptr;
  const Py_ssize_t n = PyList_GET_SIZE(coda);
  PyObject* items = PyList_New(0);
  PyObject* rows = PyList_New(0);
  PyObject* flags = PyList_New(n);
  if (!items || !rows || !flags) {
    Py_XDECREF(items); Py_XDECREF(rows); Py_XDECREF(flags);
    return nullptr;
  }
  for (Py_ssize_t i = 0; i < n; ++i) {
    Py_INCREF(Py_False);
    PyList_SET_ITEM(flags, i, Py_False);
  }
  bool ok = true;
  for (Py_ssize_t idx = 0; ok && idx < n; ++idx) {
    PyObject* state = PyObject_GetAttr(PyList_GET_ITEM(coda, idx), s_state);
    if (!state) { ok = false; break; }
    // will_finish_on_pending_token()
    int replay = get_truth(state, s_replay_eos_finishes);
    long in_flight = 0, limit = 0, pos = 0, held = 0;
    bool finishes = false;
    ok = replay >= 0 && get_long(state, s_tokens_in_flight, &in_flight);
    if (ok && !replay && in_flight > 0) {
      PyObject* gen = PyObject_GetAttr(state, s_generated_tokens);
      ok = gen != nullptr && get_long(state, s_new_tokens_limit, &limit);
      if (ok) {
        const Py_ssize_t produced = PyObject_Length(gen);
        ok = produced >= 0;
        finishes = ok && produced + in_flight >= limit;
      }
      Py_XDECREF(gen);
    }
    if (ok && !finishes) {
      ok = get_long(state, s_position_offset, &pos) && get_long(state, s_allocated_blocks, &held);
      const long next = pos + 1;
      ok = ok && set_long(state, s_position_offset, next);
      bool slot = ok && held > 0 && held * block_size > next;
      if (ok && !slot) {
        PyObject* r = PyObject_CallOneArg(allocate, state);
        const int t = r ? PyObject_IsTrue(r) : -1;
        Py_XDECREF(r);
        ok = t >= 0;
        slot = t > 0;
        if (ok && !slot) ok = set_long(state, s_position_offset, pos);
      }
      if (ok && slot) {
        ok = PyObject_SetAttr(state, s_current_token_exit_depth, Py_None) == 0;
        PyObject* depth = ok ? PyObject_CallMethodNoArgs(state, s_next_synthetic_exit_depth) : nullptr;
        PyObject* position = depth ? PyLong_FromLong(next) : nullptr;
        PyObject* zero = position ? PyLong_FromLong(0) : nullptr;
        PyObject* succ = zero ? PyObject_CallFunctionObjArgs(item_type, state, token, position, zero, depth, nullptr)
                              : nullptr;
        PyObject* row = succ ? PyLong_FromSsize_t(idx) : nullptr;
        ok = row && PyList_Append(items, succ) == 0 && PyList_Append(rows, row) == 0;
        if (ok) {
          Py_INCREF(Py_True);
          PyList_SetItem(flags, idx, Py_True);  // steals; releases the False it replaces
        }
        Py_XDECREF(depth); Py_XDECREF(position); Py_XDECREF(zero); Py_XDECREF(succ); Py_XDECREF(row);
      }
    }
    Py_DECREF(state);
  }
  if (!ok) {
    Py_DECREF(items); Py_DECREF(rows); Py_DECREF(flags);
    return nullptr;
  }
  return Py_BuildValue("(NNN)", items, rows, flags);
}

// ---------------------------------------------------------------------------
// Scheduler tick: bucket selection in priority order and prompt admission
// with chunking (continuous_depth_batching/scheduler.py:101-140, 205-296,
// 322-349; continuous_batching/scheduler_base.py:171-201, 416-545), over the
// CDBScheduler object's own attributes and the RequestState objects it holds.
// ---------------------------------------------------------------------------

// An owned reference, released at scope exit.
class Ref {
 public:
  Ref() = default;
  explicit Ref(PyObject* p) : p_(p) {}
  Ref(const Ref&) = delete;
  Ref& operator=(const Ref&) = delete;
  ~Ref() { Py_XDECREF(p_); }
  PyObject* get() const { return p_; }
  PyObject* release() {
    PyObject* p = p_;
    p_ = nullptr;
    return p;
  }
  void reset(PyObject* p) {
    Py_XDECREF(p_);
    p_ = p;
  }
  explicit operator bool() const { return p_ != nullptr; }

 private:
  PyObject* p_ = nullptr;
};

constexpr long kPending = 0, kPrefilling = 1, kDecoding = 2, kFinishedStatus = 3;  // RequestStatus values
PyObject* g_status[4];     // the RequestStatus members PENDING, PREFILLING, DECODING, FINISHED
PyObject* g_finished;      // g_status[FINISHED]
PyObject* g_batch_type;    // ScheduledCDBBatch(kind, requests, depth_items, num_q_tokens, max_kv_read)
PyObject* g_future_type;   // FutureRequestState(state, has_new_token, query_length)

PyObject *s_active_requests, *s_waiting_requests, *s_waiting_order, *s_block_new_requests, *s_ready_queue,
    *s_coda_queue, *s_in_flight_ids, *s_max_num_seqs, *s_min_coda_batch_size, *s_min_free_slots, *s_safety_margin,
    *s_kv_pressure_mode, *s_max_model_len, *s_cache, *s_max_fast_path_len, *s_slot_of_step, *s_mixed_batches,
    *s_max_in_flight, *s_max_live, *s_max_resident, *s_resident_samples, *s_resident_sum, *s_steady_warmup,
    *s_advance_steady, *s_block_manager, *s_num_blocks, *s_block_size, *s_allocate_blocks, *s_get_num_free_blocks,
    *s_is_cpu_offloaded, *s_remaining_prefill, *s_tokens_to_process, *s_initial_tokens, *s_max_new_tokens,
    *s_status, *s_popleft, *s_reserve, *s_kind_coda, *s_kind_prefill, *s_kind_recurrent;

// ceil(a / b) for b > 0 and any sign of a, as Python's -(-a // b).
long ceil_div(long a, long b) {
  long q = a / b;
  if (a % b > 0) ++q;
  return q;
}

bool raise_peak(PyObject* obj, PyObject* name, long value) {
  long cur;
  if (!get_long(obj, name, &cur)) return false;
  return value <= cur || set_long(obj, name, value);
}

bool add_long(PyObject* obj, PyObject* name, long delta) {
  long cur;
  return get_long(obj, name, &cur) && set_long(obj, name, cur + delta);
}

// The scheduler's containers and constants, read once per call.
struct Sched {
  PyObject* self = nullptr;  // borrowed
  Ref active, waiting, in_flight, cache, pool;
  long max_num_seqs = 0, block_size = 0, num_blocks = 0;
  double safety_margin = 0.0;

  bool load(PyObject* s) {
    self = s;
    active.reset(PyObject_GetAttr(s, s_active_requests));
    waiting.reset(PyObject_GetAttr(s, s_waiting_requests));
    in_flight.reset(PyObject_GetAttr(s, s_in_flight_ids));
    cache.reset(PyObject_GetAttr(s, s_cache));
    if (!active || !waiting || !in_flight || !cache) return false;
    if (!PyDict_Check(active.get()) || !PyDict_Check(waiting.get()) || !PySet_Check(in_flight.get())) {
      PyErr_SetString(PyExc_TypeError, "scheduler: active/waiting requests must be dicts, in-flight ids a set");
      return false;
    }
    if (!get_long(s, s_max_num_seqs, &max_num_seqs) || !get_long(cache.get(), s_block_size, &block_size) ||
        !get_long(cache.get(), s_num_blocks, &num_blocks))
      return false;
    if (block_size <= 0) {
      PyErr_SetString(PyExc_ValueError, "scheduler: cache block_size must be positive");
      return false;
    }
    Ref margin(PyObject_GetAttr(s, s_safety_margin));
    if (!margin) return false;
    safety_margin = PyFloat_AsDouble(margin.get());
    if (safety_margin == -1.0 && PyErr_Occurred()) return false;
    // The block manager is read directly when it is the tick core's own BlockPool.
    Ref manager(PyObject_GetAttr(cache.get(), s_block_manager));
    if (manager && PyObject_TypeCheck(manager.get(), &BlockPoolType)) pool.reset(manager.release());
    else PyErr_Clear();
    return true;
  }

  bool free_blocks(long* out) {
    if (pool) {
      *out = (long)reinterpret_cast<BlockPool*>(pool.get())->free_list->size();
      return true;
    }
    Ref r(PyObject_CallMethodNoArgs(cache.get(), s_get_num_free_blocks));
    if (!r) return false;
    *out = PyLong_AsLong(r.get());
    return !(*out == -1 && PyErr_Occurred());
  }

  long residency_slots() const { return std::max<long>(0, max_num_seqs - (long)PyDict_GET_SIZE(active.get())); }
};

bool types_bound() {
  if (g_finished && g_batch_type && g_future_type) return true;
  PyErr_SetString(PyExc_RuntimeError, "the request and scheduler types are not bound to the tick core");
  return false;
}

// bind_request_types(RequestStatus, FutureRequestState), called where they are defined.
PyObject* bind_request_types(PyObject*, PyObject* args) {
  PyObject *status, *future;
  if (!PyArg_ParseTuple(args, "OO", &status, &future)) return nullptr;
  PyObject* members[4] = {nullptr, nullptr, nullptr, nullptr};
  for (long v = 0; v < 4; ++v) {
    members[v] = PyObject_CallFunction(status, "l", v);
    if (!members[v]) {
      for (long j = 0; j < v; ++j) Py_DECREF(members[j]);
      return nullptr;
    }
  }
  for (long v = 0; v < 4; ++v) {
    Py_XDECREF(g_status[v]);
    g_status[v] = members[v];
  }
  g_finished = g_status[kFinishedStatus];
  Py_INCREF(future);
  Py_XDECREF(g_future_type);
  g_future_type = future;
  Py_RETURN_NONE;
}

// bind_batch_type(ScheduledCDBBatch), called where it is defined.
PyObject* bind_batch_type(PyObject*, PyObject* batch) {
  Py_INCREF(batch);
  Py_XDECREF(g_batch_type);
  g_batch_type = batch;
  Py_RETURN_NONE;
}

bool load_sched(PyObject* self, Sched& S) { return types_bound() && S.load(self); }

// record_resident_sample (scheduler_base.py:315-398): the resident-set peak and mean, and
// the steady-state window when one is being tracked.
bool record_resident(Sched& S) {
  const long resident = (long)PyDict_GET_SIZE(S.active.get());
  if (!raise_peak(S.self, s_max_resident, resident) || !add_long(S.self, s_resident_samples, 1) ||
      !add_long(S.self, s_resident_sum, resident))
    return false;
  Ref warmup(PyObject_GetAttr(S.self, s_steady_warmup));
  if (!warmup) return false;
  if (warmup.get() == Py_None) return true;
  Ref arg(PyLong_FromLong(resident));
  Ref r(arg ? PyObject_CallMethodOneArg(S.self, s_advance_steady, arg.get()) : nullptr);
  return bool(r);
}

// Whether any active request is decoding (-1 on error).
int has_decode_work(Sched& S) {
  Py_ssize_t pos = 0;
  PyObject *key, *state;
  while (PyDict_Next(S.active.get(), &pos, &key, &state)) {
    long st;
    if (!get_long(state, s_status_field, &st)) return -1;
    if (st == kDecoding) return 1;
  }
  return 0;
}

// Prefill runs when nothing decodes or the free blocks exceed the safety margin
// (scheduler_base.py:171-201). Both tests are pure, so the cheap one goes first.
int admit_prefill(Sched& S) {
  long free;
  if (!S.free_blocks(&free)) return -1;
  if ((double)free > S.safety_margin * (double)S.num_blocks) return 1;
  const int decoding = has_decode_work(S);
  return decoding < 0 ? -1 : !decoding;
}

// Worst-case blocks of a request under reserve admission (utils.py:107-129).
bool reserved_peak(PyObject* state, long max_model_len, long block_size, long* out) {
  Ref initial(PyObject_GetAttr(state, s_initial_tokens));
  Ref budget(initial ? PyObject_GetAttr(state, s_max_new_tokens) : nullptr);
  if (!budget) return false;
  const Py_ssize_t prompt = PyObject_Length(initial.get());
  if (prompt < 0) return false;
  long total = max_model_len;
  if (budget.get() != Py_None) {
    const long mnt = PyLong_AsLong(budget.get());
    if (mnt == -1 && PyErr_Occurred()) return false;
    total = std::min<long>((long)prompt + mnt, max_model_len);
  }
  *out = ceil_div(total, block_size);
  return true;
}

// The prefill bucket (scheduler_base.py:416-460): active requests mid-prefill with no token
// in flight, then -- unless new requests are blocked -- waiting prompts that are not swapped
// out, in arrival order, up to the open residency slots; under reserve admission only those
// whose worst-case blocks still fit beside the active requests' commitments.
PyObject* prefill_bucket_of(Sched& S) {
  Ref out(PyList_New(0));
  if (!out) return nullptr;
  Py_ssize_t pos = 0;
  PyObject *key, *state;
  while (PyDict_Next(S.active.get(), &pos, &key, &state)) {
    long st;
    if (!get_long(state, s_status_field, &st)) return nullptr;
    if (st != kPrefilling) continue;
    Ref rid(PyObject_GetAttr(state, s_request_id));
    if (!rid) return nullptr;
    const int busy = PySet_Contains(S.in_flight.get(), rid.get());
    if (busy < 0 || (!busy && PyList_Append(out.get(), state))) return nullptr;
  }
  const int blocked = get_truth(S.self, s_block_new_requests);
  if (blocked < 0) return nullptr;
  if (blocked) return out.release();
  const long limit = S.residency_slots();
  Ref admissible(PyList_New(0));
  if (!admissible) return nullptr;
  if (limit > 0) {
    Ref order(PyObject_GetAttr(S.self, s_waiting_order));
    Ref it(order ? PyObject_GetIter(order.get()) : nullptr);
    if (!it) return nullptr;
    while (PyList_GET_SIZE(admissible.get()) < limit) {
      Ref rid(PyIter_Next(it.get()));
      if (!rid) {
        if (PyErr_Occurred()) return nullptr;
        break;
      }
      PyObject* waiting = PyDict_GetItemWithError(S.waiting.get(), rid.get());  // borrowed
      if (!waiting) {
        if (!PyErr_Occurred()) PyErr_SetObject(PyExc_KeyError, rid.get());
        return nullptr;
      }
      const int offloaded = get_truth(waiting, s_is_cpu_offloaded);
      if (offloaded < 0 || (!offloaded && PyList_Append(admissible.get(), waiting))) return nullptr;
    }
  }
  Ref mode(PyObject_GetAttr(S.self, s_kv_pressure_mode));
  if (!mode) return nullptr;
  const int reserve = PyObject_RichCompareBool(mode.get(), s_reserve, Py_EQ);
  if (reserve < 0) return nullptr;
  if (reserve) {
    long max_len, committed = 0, need;
    if (!get_long(S.self, s_max_model_len, &max_len)) return nullptr;
    pos = 0;
    while (PyDict_Next(S.active.get(), &pos, &key, &state)) {
      if (!reserved_peak(state, max_len, S.block_size, &need)) return nullptr;
      committed += need;
    }
    Py_ssize_t fit = 0;
    for (; fit < PyList_GET_SIZE(admissible.get()); ++fit) {
      if (!reserved_peak(PyList_GET_ITEM(admissible.get(), fit), max_len, S.block_size, &need)) return nullptr;
      if (committed + need > S.num_blocks) break;
      committed += need;
    }
    if (PyList_SetSlice(admissible.get(), fit, PyList_GET_SIZE(admissible.get()), nullptr)) return nullptr;
  }
  const Py_ssize_t n = PyList_GET_SIZE(out.get());
  if (PyList_SetSlice(out.get(), n, n, admissible.get())) return nullptr;
  return out.release();
}

// A bucket is admitted when it holds a request mid-prefill or enough residency slots are open.
int admit_bucket(Sched& S, PyObject* bucket) {
  const Py_ssize_t n = PyList_GET_SIZE(bucket);
  if (n == 0) return 0;
  for (Py_ssize_t i = 0; i < n; ++i) {
    long st;
    if (!get_long(PyList_GET_ITEM(bucket, i), s_status_field, &st)) return -1;
    if (st == kPrefilling) return 1;
  }
  long min_free;
  if (!get_long(S.self, s_min_free_slots, &min_free)) return -1;
  return S.residency_slots() >= min_free;
}

bool mark_in_flight(Sched& S, PyObject* rid) {
  if (PySet_Add(S.in_flight.get(), rid)) return false;
  const long live = (long)(PyDict_GET_SIZE(S.active.get()) + PyDict_GET_SIZE(S.waiting.get()));
  return raise_peak(S.self, s_max_in_flight, (long)PySet_GET_SIZE(S.in_flight.get())) &&
         raise_peak(S.self, s_max_live, live);
}

// Blocks for `n` more tokens past the request's length, taken from the cache when the held
// ones fall short (scheduler_base.py:520-531). 1 held or allocated, 0 not enough free, -1 error.
int allocate_for(Sched& S, PyObject* state, long n) {
  long current, held;
  if (!get_long(state, s_position_offset, &current) || !get_long(state, s_allocated_blocks, &held)) return -1;
  if (held * S.block_size - current >= n) return 1;
  const long needed = ceil_div(current + n, S.block_size) - held;
  Ref rid(PyObject_GetAttr(state, s_request_id));
  Ref count(rid ? PyLong_FromLong(needed) : nullptr);
  Ref offset(count ? PyLong_FromLong(held) : nullptr);
  Ref got(offset ? PyObject_CallMethodObjArgs(S.cache.get(), s_allocate_blocks, count.get(), rid.get(),
                                              offset.get(), nullptr)
                 : nullptr);
  if (!got) return -1;
  if (got.get() == Py_None) return 0;
  const long g = PyLong_AsLong(got.get());
  if (g == -1 && PyErr_Occurred()) return -1;
  return set_long(state, s_allocated_blocks, held + g) ? 1 : -1;
}

// Takes the first request_len prompt tokens of a candidate (scheduler_base.py:462-492): a
// pending request becomes active, and one whose prompt is used up moves to decoding with
// the rest of its prompt as the tokens to process.
bool take_prompt_chunk(Sched& S, PyObject* state, PyObject* tokens, long request_len, PyObject* taken) {
  const Py_ssize_t ntok = PyObject_Length(tokens);
  long st;
  Ref rid(PyObject_GetAttr(state, s_request_id));
  if (ntok < 0 || !rid || !get_long(state, s_status_field, &st)) return false;
  if (ntok <= request_len) {
    if (st == kPending && (PyDict_SetItem(S.active.get(), rid.get(), state) || PySet_Add(taken, rid.get())))
      return false;
    if (st <= kPrefilling) {
      Ref rest(PyObject_GetAttr(state, s_remaining_prefill));
      Ref none_left(rest ? PyList_New(0) : nullptr);
      if (!none_left || PyObject_SetAttr(state, s_tokens_to_process, rest.get()) ||
          PyObject_SetAttr(state, s_remaining_prefill, none_left.get()) ||
          PyObject_SetAttr(state, s_status, g_status[kDecoding]))
        return false;
    }
    return true;
  }
  if (st == kPending && (PyDict_SetItem(S.active.get(), rid.get(), state) ||
                         PyObject_SetAttr(state, s_status, g_status[kPrefilling]) || PySet_Add(taken, rid.get())))
    return false;
  Ref tail(PySequence_GetSlice(tokens, request_len, PY_SSIZE_T_MAX));
  Ref head(tail ? PySequence_GetSlice(tokens, 0, request_len) : nullptr);
  return head && PyObject_SetAttr(state, s_remaining_prefill, tail.get()) == 0 &&
         PyObject_SetAttr(state, s_tokens_to_process, head.get()) == 0;
}

// One prefill batch from the candidates in order, within the token and KV-read budgets
// (scheduler_base.py:494-545): a request whose whole remaining prompt does not fit the
// token budget is chunked, decode-only batches of single tokens ignore the read budget,
// and allocation failure skips a request (or ends the batch when the cache is empty and
// the request still waits). `taken` collects the ids leaving the waiting queue.
PyObject* fill_prefill(Sched& S, PyObject* candidates, long token_budget, long cache_budget, PyObject* taken,
                       long* num_q_tokens, long* max_kv_read) {
  Ref scheduled(PyList_New(0));
  long max_fast;
  if (!scheduled || !get_long(S.self, s_max_fast_path_len, &max_fast)) return nullptr;
  const double margin = S.safety_margin * (double)S.num_blocks;
  bool fast = true;
  long tokens_left = token_budget, reads_left = cache_budget;
  for (Py_ssize_t i = 0; i < PyList_GET_SIZE(candidates); ++i) {
    PyObject* state = PyList_GET_ITEM(candidates, i);
    long free;
    if (!S.free_blocks(&free)) return nullptr;
    if ((double)free < margin && PyList_GET_SIZE(scheduled.get()) > 0) break;
    Ref tokens(PyObject_GetAttr(state, s_remaining_prefill));
    if (!tokens) return nullptr;
    const Py_ssize_t ntok = PyObject_Length(tokens.get());
    if (ntok < 0) return nullptr;
    long request_len = std::min<long>((long)ntok, tokens_left);
    if (request_len == 0) continue;
    long position;
    if (!get_long(state, s_position_offset, &position)) return nullptr;
    const bool eligible = request_len == 1 && position < max_fast;
    const long read_needed = position;
    if (!(fast && eligible) && reads_left < read_needed) continue;
    const int got = allocate_for(S, state, request_len);
    if (got < 0) return nullptr;
    Ref rid(PyObject_GetAttr(state, s_request_id));
    if (!rid) return nullptr;
    if (!got) {
      if (free == 0) {
        const int waiting = PyDict_Contains(S.waiting.get(), rid.get());
        if (waiting < 0) return nullptr;
        if (waiting) break;
      }
      continue;
    }
    if (!take_prompt_chunk(S, state, tokens.get(), request_len, taken) || !mark_in_flight(S, rid.get()))
      return nullptr;
    Ref chunk(PyObject_GetAttr(state, s_tokens_to_process));
    const Py_ssize_t taken_len = chunk ? PyObject_Length(chunk.get()) : -1;
    if (taken_len < 0 || !get_long(state, s_position_offset, &position)) return nullptr;
    request_len = (long)taken_len;
    fast = fast && request_len == 1 && position < max_fast;
    tokens_left -= request_len;
    reads_left -= read_needed;
    Ref rest(PyObject_GetAttr(state, s_remaining_prefill));
    const int more = rest ? PyObject_IsTrue(rest.get()) : -1;
    if (more < 0) return nullptr;
    Ref future(PyObject_CallFunction(g_future_type, "OOl", state, more ? Py_False : Py_True, request_len));
    if (!future || PyList_Append(scheduled.get(), future.get())) return nullptr;
    PyObject* was_waiting = PyDict_GetItemWithError(S.waiting.get(), rid.get());  // borrowed
    if (was_waiting) {
      if (PyDict_DelItem(S.waiting.get(), rid.get()) || PySet_Add(taken, rid.get())) return nullptr;
    } else if (PyErr_Occurred()) {
      return nullptr;
    }
    if (tokens_left == 0 || (reads_left <= 0 && !fast)) break;
  }
  *num_q_tokens = token_budget - tokens_left;
  *max_kv_read = cache_budget - reads_left;
  return scheduled.release();
}

// Drops the taken ids from the waiting order: popped off the front while they lead it,
// else by rebuilding the order without them (scheduler_base.py:503-511).
bool drop_from_waiting_order(Sched& S, PyObject* taken) {
  if (PySet_GET_SIZE(taken) == 0) return true;
  Ref remaining(PySet_New(taken));
  Ref order(remaining ? PyObject_GetAttr(S.self, s_waiting_order) : nullptr);
  if (!order) return false;
  while (PySet_GET_SIZE(remaining.get()) > 0) {
    const Py_ssize_t n = PyObject_Length(order.get());
    if (n < 0) return false;
    if (n == 0) break;
    Ref head(PySequence_GetItem(order.get(), 0));
    const int lead = head ? PySet_Contains(remaining.get(), head.get()) : -1;
    if (lead < 0) return false;
    if (!lead) break;
    Ref popped(PyObject_CallMethodNoArgs(order.get(), s_popleft));
    if (!popped || PySet_Discard(remaining.get(), popped.get()) < 0) return false;
  }
  if (PySet_GET_SIZE(remaining.get()) == 0) return true;
  Ref kept(PyList_New(0));
  Ref it(kept ? PyObject_GetIter(order.get()) : nullptr);
  if (!it) return false;
  for (;;) {
    Ref rid(PyIter_Next(it.get()));
    if (!rid) {
      if (PyErr_Occurred()) return false;
      break;
    }
    const int gone = PySet_Contains(remaining.get(), rid.get());
    if (gone < 0 || (!gone && PyList_Append(kept.get(), rid.get()))) return false;
  }
  Ref fresh(PyObject_CallOneArg(reinterpret_cast<PyObject*>(Py_TYPE(order.get())), kept.get()));
  return fresh && PyObject_SetAttr(S.self, s_waiting_order, fresh.get()) == 0;
}

PyObject* make_batch(PyObject* kind, PyObject* requests, PyObject* items, long num_q_tokens, long max_kv_read) {
  return PyObject_CallFunction(g_batch_type, "OOOll", kind, requests, items, num_q_tokens, max_kv_read);
}

// The prefill batch of this tick, or None (scheduler.py:205-234).
PyObject* schedule_prefill_of(Sched& S, long token_budget, long cache_budget) {
  Ref bucket(prefill_bucket_of(S));
  if (!bucket) return nullptr;
  const int admitted = admit_bucket(S, bucket.get());
  if (admitted < 0) return nullptr;
  if (!admitted) Py_RETURN_NONE;
  Ref taken(PySet_New(nullptr));
  if (!taken) return nullptr;
  long num_q_tokens = 0, max_kv_read = 0;
  Ref scheduled(fill_prefill(S, bucket.get(), token_budget, cache_budget, taken.get(), &num_q_tokens, &max_kv_read));
  if (!scheduled || !drop_from_waiting_order(S, taken.get())) return nullptr;
  if (PyList_GET_SIZE(scheduled.get()) == 0) Py_RETURN_NONE;
  return make_batch(s_kind_prefill, scheduled.get(), Py_None, num_q_tokens, max_kv_read);
}

std::deque<PyObject*>* queue_attr(PyObject* self, PyObject* name, Ref& holder) {
  holder.reset(PyObject_GetAttr(self, name));
  if (!holder) return nullptr;
  if (!is_queue(holder.get())) {
    PyErr_SetString(PyExc_TypeError, "scheduler queues must be ItemQueues");
    return nullptr;
  }
  return reinterpret_cast<ItemQueue*>(holder.get())->items;
}

// schedule_next(scheduler, token_budget, cache_budget, allow_coda) -> ScheduledCDBBatch | None
// One homogeneous bucket per tick (scheduler.py:101-140): a coda batch once
// min_coda_batch_size tokens wait, else a prefill batch when admission allows, else the
// next recurrent batch (head item first, slot-homogeneous when required), else an
// undersized coda flush.
PyObject* schedule_next(PyObject*, PyObject* args) {
  PyObject* self;
  long token_budget, cache_budget;
  int allow_coda;
  if (!PyArg_ParseTuple(args, "Ollp", &self, &token_budget, &cache_budget, &allow_coda)) return nullptr;
  Sched S;
  if (!load_sched(self, S) || !record_resident(S)) return nullptr;
  Ref coda_holder, ready_holder;
  auto* coda = queue_attr(self, s_coda_queue, coda_holder);
  auto* ready = coda ? queue_attr(self, s_ready_queue, ready_holder) : nullptr;
  long min_coda;
  if (!ready || !get_long(self, s_min_coda_batch_size, &min_coda)) return nullptr;
  auto coda_batch = [&]() -> PyObject* {
    const Py_ssize_t n = std::min<Py_ssize_t>(S.max_num_seqs, (Py_ssize_t)coda->size());
    return pop_front_from(coda, n);
  };
  if (allow_coda && (long)coda->size() >= min_coda) {
    Ref batch(coda_batch());
    if (!batch) return nullptr;
    if (PyList_GET_SIZE(batch.get()) > 0) return make_batch(s_kind_coda, Py_None, batch.get(), 0, 0);
  }
  const int admit = admit_prefill(S);
  if (admit < 0) return nullptr;
  if (admit) {
    Ref prefill(schedule_prefill_of(S, token_budget, cache_budget));
    if (!prefill) return nullptr;
    if (prefill.get() != Py_None) return prefill.release();
  }
  const Py_ssize_t size = std::min<Py_ssize_t>(S.max_num_seqs, (Py_ssize_t)ready->size());
  if (size > 0) {
    Ref slot_of_step(PyObject_GetAttr(self, s_slot_of_step));
    Ref batch(slot_of_step ? pop_batch_from(ready, size, slot_of_step.get()) : nullptr);
    if (!batch || !add_long(self, s_mixed_batches, 1)) return nullptr;
    if (PyList_GET_SIZE(batch.get()) > 0) return make_batch(s_kind_recurrent, Py_None, batch.get(), 0, 0);
  }
  if (allow_coda) {
    Ref batch(coda_batch());
    if (!batch) return nullptr;
    if (PyList_GET_SIZE(batch.get()) > 0) return make_batch(s_kind_coda, Py_None, batch.get(), 0, 0);
  }
  Py_RETURN_NONE;
}

PyObject* schedule_prefill(PyObject*, PyObject* args) {
  PyObject* self;
  long token_budget, cache_budget;
  if (!PyArg_ParseTuple(args, "Oll", &self, &token_budget, &cache_budget)) return nullptr;
  Sched S;
  if (!load_sched(self, S)) return nullptr;
  return schedule_prefill_of(S, token_budget, cache_budget);
}

PyObject* prefill_bucket(PyObject*, PyObject* self) {
  Sched S;
  if (!load_sched(self, S)) return nullptr;
  return prefill_bucket_of(S);
}

PyObject* record_resident_sample(PyObject*, PyObject* self) {
  Sched S;
  if (!load_sched(self, S) || !record_resident(S)) return nullptr;
  Py_RETURN_NONE;
}

PyObject* prefill_admitted(PyObject*, PyObject* self) {
  Sched S;
  if (!load_sched(self, S)) return nullptr;
  const int admit = admit_prefill(S);
  if (admit < 0) return nullptr;
  return PyBool_FromLong(admit);
}

PyObject* allocate_if_needed(PyObject*, PyObject* args) {
  PyObject *self, *state;
  long n;
  if (!PyArg_ParseTuple(args, "OOl", &self, &state, &n)) return nullptr;
  Sched S;
  if (!load_sched(self, S)) return nullptr;
  const int got = allocate_for(S, state, n);
  if (got < 0) return nullptr;
  return PyBool_FromLong(got);
}

// ---------------------------------------------------------------------------
// Sampled-token bookkeeping (continuous_batching/requests.py:208-237) and the
// coda-result walk of the engine (cdb/continuous_api.py:1378-1420).
// ---------------------------------------------------------------------------
PyObject* g_perf_counter;  // time.perf_counter
PyObject *s_eos_ids, *s_stop_sequences, *s_first_token_time, *s_name, *s_get;

// Whether the generated tokens end with one of the request's stop sequences.
int matches_stop_sequence(PyObject* state, PyObject* generated) {
  Ref stops(PyObject_GetAttr(state, s_stop_sequences));
  Ref it(stops ? PyObject_GetIter(stops.get()) : nullptr);
  if (!it) return -1;
  const Py_ssize_t n = PyList_GET_SIZE(generated);
  for (;;) {
    Ref seq(PyIter_Next(it.get()));
    if (!seq) return PyErr_Occurred() ? -1 : 0;
    const int nonempty = PyObject_IsTrue(seq.get());
    if (nonempty < 0) return -1;
    if (!nonempty) continue;
    const Py_ssize_t len = PyObject_Length(seq.get());
    if (len < 0) return -1;
    if (n < len) continue;
    Ref tail(PyList_GetSlice(generated, n - len, n));
    const int eq = tail ? PyObject_RichCompareBool(tail.get(), seq.get(), Py_EQ) : -1;
    if (eq) return eq;
  }
}

// Record a sampled token on a decoding request: one fewer token in flight; the token is
// kept (and becomes the next token to process) when it is EOS or within the length limit;
// the request finishes on EOS, at the limit or on a stop sequence. 1 finished, 0 not, -1 error.
int update_completion_of(PyObject* state, PyObject* token) {
  long status, in_flight, limit;
  if (!get_long(state, s_status_field, &status)) return -1;
  if (status != kDecoding) {
    Ref rid(PyObject_GetAttr(state, s_request_id));
    Ref current(rid ? PyObject_GetAttr(state, s_status_field) : nullptr);
    Ref name(current ? PyObject_GetAttr(current.get(), s_name) : nullptr);
    if (name) PyErr_Format(PyExc_RuntimeError, "Cannot update request %S while status is %S", rid.get(), name.get());
    return -1;
  }
  if (!get_long(state, s_tokens_in_flight, &in_flight) ||
      !set_long(state, s_tokens_in_flight, std::max<long>(0, in_flight - 1)) ||
      !get_long(state, s_new_tokens_limit, &limit))
    return -1;
  Ref eos(PyObject_GetAttr(state, s_eos_ids));
  const int is_eos = eos ? PySequence_Contains(eos.get(), token) : -1;
  Ref generated(is_eos >= 0 ? PyObject_GetAttr(state, s_generated_tokens) : nullptr);
  if (!generated) return -1;
  if (!PyList_Check(generated.get())) {
    PyErr_SetString(PyExc_TypeError, "state.generated_tokens must be a list");
    return -1;
  }
  Py_ssize_t n = PyList_GET_SIZE(generated.get());
  if (is_eos || n < limit) {
    Ref first(PyObject_GetAttr(state, s_first_token_time));
    const double t = first ? PyFloat_AsDouble(first.get()) : -1.0;
    if (!first || (t == -1.0 && PyErr_Occurred())) return -1;
    if (t < 0) {
      Ref now(PyObject_CallNoArgs(g_perf_counter));
      if (!now || PyObject_SetAttr(state, s_first_token_time, now.get())) return -1;
    }
    Ref next(PyList_New(1));
    if (!next || PyList_Append(generated.get(), token)) return -1;
    Py_INCREF(token);
    PyList_SET_ITEM(next.get(), 0, token);
    if (PyObject_SetAttr(state, s_tokens_to_process, next.get())) return -1;
    ++n;
  }
  int done = is_eos || n >= limit;
  if (!done) done = matches_stop_sequence(state, generated.get());
  if (done < 0) return -1;
  if (done && PyObject_SetAttr(state, s_status, g_finished)) return -1;
  return done;
}

PyObject* update_completion(PyObject*, PyObject* args) {
  PyObject *state, *token;
  if (!PyArg_ParseTuple(args, "OO", &state, &token)) return nullptr;
  if (!g_finished) {
    PyErr_SetString(PyExc_RuntimeError, "RequestStatus is not bound to the tick core");
    return nullptr;
  }
  const int done = update_completion_of(state, token);
  if (done < 0) return nullptr;
  return PyBool_FromLong(done);
}

// consume_coda(items, tokens, eager) -> [(state, stage), ...]
// A coda batch's sampled tokens, row by row: rows of finished requests are skipped; an
// eagerly re-entered row only records its token; any other row first advances its
// request's position. Each request that finishes is returned with stage False (to retire),
// each unfinished non-eager one with stage True (its next decode token is to be staged),
// in row order.
PyObject* consume_coda(PyObject*, PyObject* args) {
  PyObject *items, *tokens, *eager;
  if (!PyArg_ParseTuple(args, "O!O!O", &PyList_Type, &items, &PyList_Type, &tokens, &eager)) return nullptr;
  if (!g_finished) {
    PyErr_SetString(PyExc_RuntimeError, "RequestStatus is not bound to the tick core");
    return nullptr;
  }
  const Py_ssize_t n = PyList_GET_SIZE(items);
  if (PyList_GET_SIZE(tokens) < n || (eager != Py_None && (!PyList_Check(eager) || PyList_GET_SIZE(eager) < n))) {
    PyErr_SetString(PyExc_ValueError, "consume_coda: tokens and eager flags must cover every item");
    return nullptr;
  }
  Ref actions(PyList_New(0));
  if (!actions) return nullptr;
  for (Py_ssize_t i = 0; i < n; ++i) {
    Ref state(PyObject_GetAttr(PyList_GET_ITEM(items, i), s_state));
    long status;
    if (!state || !get_long(state.get(), s_status_field, &status)) return nullptr;
    if (status == kFinishedStatus) continue;
    const int was_eager = eager == Py_None ? 0 : PyObject_IsTrue(PyList_GET_ITEM(eager, i));
    if (was_eager < 0) return nullptr;
    if (!was_eager) {
      long position;
      if (!get_long(state.get(), s_position_offset, &position) ||
          !set_long(state.get(), s_position_offset, position + 1))
        return nullptr;
    }
    const int done = update_completion_of(state.get(), PyList_GET_ITEM(tokens, i));
    if (done < 0) return nullptr;
    if (was_eager && !done) continue;
    Ref action(Py_BuildValue("(OO)", state.get(), done ? Py_False : Py_True));
    if (!action || PyList_Append(actions.get(), action.get())) return nullptr;
  }
  return actions.release();
}

// add_tokens_in_flight(items): one more sampled token in flight on each item's request.
PyObject* add_tokens_in_flight(PyObject*, PyObject* items) {
  if (!PyList_Check(items)) {
    PyErr_SetString(PyExc_TypeError, "items must be a list");
    return nullptr;
  }
  for (Py_ssize_t i = 0; i < PyList_GET_SIZE(items); ++i) {
    Ref state(PyObject_GetAttr(PyList_GET_ITEM(items, i), s_state));
    if (!state || !add_long(state.get(), s_tokens_in_flight, 1)) return nullptr;
  }
  Py_RETURN_NONE;
}

// coda_upload(items, successors, rows, upload_addr, upload_len, free_slots, next_slot, capacity) -> next_slot
// Fills a coda launch's int64 host upload (cdb/model_runner.py:1064-1125 stages the same
// facts): [the items' hidden slots | per item, its successor's slot or -1 | the successors'
// slots]. Each successor (one per listed coda row) gets a hidden slot: the most recently
// freed first (free_slots is a LIFO list), then fresh ones from next_slot below capacity
// (cdb/model_runner.py:1193-1203). Without successors only the items' slots are written.
PyObject* coda_upload(PyObject*, PyObject* args) {
  PyObject *items, *successors, *rows, *free_slots;
  unsigned long long addr;
  Py_ssize_t upload_len;
  long next_slot, capacity;
  if (!PyArg_ParseTuple(args, "O!O!O!KnO!ll", &PyList_Type, &items, &PyList_Type, &successors, &PyList_Type, &rows,
                        &addr, &upload_len, &PyList_Type, &free_slots, &next_slot, &capacity))
    return nullptr;
  const Py_ssize_t n = PyList_GET_SIZE(items), k = PyList_GET_SIZE(successors);
  if (PyList_GET_SIZE(rows) != k || n + (k ? n + k : 0) > upload_len || addr == 0) {
    PyErr_SetString(PyExc_ValueError, "coda_upload: rows must match the successors and the upload hold them all");
    return nullptr;
  }
  int64_t* upload = reinterpret_cast<int64_t*>(static_cast<uintptr_t>(addr));
  for (Py_ssize_t i = 0; i < n; ++i) {
    long slot;
    if (!get_long(PyList_GET_ITEM(items, i), s_hidden_slot, &slot)) return nullptr;
    upload[i] = slot;
  }
  if (k == 0) return PyLong_FromLong(next_slot);
  // Every successor row is checked before any hidden slot is taken, so a bad row leaves the
  // free list and the slot counter as they were.
  for (Py_ssize_t j = 0; j < k; ++j) {
    const long row = PyLong_AsLong(PyList_GET_ITEM(rows, j));
    if (row == -1 && PyErr_Occurred()) return nullptr;
    if (row < 0 || row >= n) {
      PyErr_Format(PyExc_ValueError, "coda_upload: successor row %ld outside the %zd coda rows", row, n);
      return nullptr;
    }
  }
  for (Py_ssize_t i = 0; i < n; ++i) upload[n + i] = -1;
  for (Py_ssize_t j = 0; j < k; ++j) {
    long slot;
    const Py_ssize_t nfree = PyList_GET_SIZE(free_slots);
    if (nfree > 0) {
      slot = PyLong_AsLong(PyList_GET_ITEM(free_slots, nfree - 1));
      if (slot == -1 && PyErr_Occurred()) return nullptr;
      if (PyList_SetSlice(free_slots, nfree - 1, nfree, nullptr)) return nullptr;
    } else {
      if (next_slot >= capacity) {
        PyErr_Format(PyExc_RuntimeError, "hidden-state bank exhausted (%ld slots)", capacity);
        return nullptr;
      }
      slot = next_slot++;
    }
    const long row = PyLong_AsLong(PyList_GET_ITEM(rows, j));
    upload[n + row] = slot;
    upload[2 * n + j] = slot;
    if (!set_long(PyList_GET_ITEM(successors, j), s_hidden_slot, slot)) return nullptr;
  }
  return PyLong_FromLong(next_slot);
}

// route_delayed(items, flags, max_steps, pending, histogram, backlog) -> (coda_items, refills, exits)
// Routes one recurrent launch's rows on the offset-one horizon (cdb/continuous_api.py:1124-1141,
// 1247-1280, 1699-1724): a row leaves at the last step, or when the decision its previous launch made for
// it says so; pending maps id(item) to that (PendingFlags, row) and is updated with this
// launch's (flags, row) for every row that steps on. Exits get the same bookkeeping as
// route_sync; survivors advance one step. The previous launch's flags are read through
// PendingFlags.get, which waits for them once and keeps them as a list.
PyObject* route_delayed(PyObject*, PyObject* args) {
  PyObject *items, *flags, *pending, *hist, *backlog;
  long max_steps;
  if (!PyArg_ParseTuple(args, "O!OlO!O!O", &PyList_Type, &items, &flags, &max_steps, &PyDict_Type, &pending,
                        &PyDict_Type, &hist, &backlog))
    return nullptr;
  if (backlog != Py_None && !PyList_Check(backlog)) {
    PyErr_SetString(PyExc_TypeError, "backlog must be a list or None");
    return nullptr;
  }
  const Py_ssize_t n = PyList_GET_SIZE(items);
  Ref coda(PyList_New(0)), refills(PyList_New(0)), exits(PyList_New(n));
  if (!coda || !refills || !exits) return nullptr;
  for (Py_ssize_t i = 0; i < n; ++i) {
    Py_INCREF(Py_False);
    PyList_SET_ITEM(exits.get(), i, Py_False);
  }
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* item = PyList_GET_ITEM(items, i);
    long step;
    const int apply = get_truth(item, s_apply_exit_gate);
    Ref key(PyLong_FromVoidPtr(item));
    if (apply < 0 || !key || !get_long(item, s_recurrent_step, &step)) return nullptr;
    // pending.pop(id(item), None)
    Ref previous(PyDict_GetItemWithError(pending, key.get()));
    if (previous) {
      Py_INCREF(previous.get());
      if (PyDict_DelItem(pending, key.get())) return nullptr;
    } else if (PyErr_Occurred()) {
      return nullptr;
    }
    int leave = step == max_steps - 1;
    if (!leave && apply && previous) {
      if (!PyTuple_Check(previous.get()) || PyTuple_GET_SIZE(previous.get()) != 2) {
        PyErr_SetString(PyExc_TypeError, "pending entries must be (flags, row) tuples");
        return nullptr;
      }
      Ref decided(PyObject_CallMethodOneArg(PyTuple_GET_ITEM(previous.get(), 0), s_get,
                                            PyTuple_GET_ITEM(previous.get(), 1)));
      leave = decided ? PyObject_IsTrue(decided.get()) : -1;
      if (leave < 0) return nullptr;
    }
    if (leave) {
      Py_INCREF(Py_True);
      if (PyList_SetItem(exits.get(), i, Py_True) || !record_exit(item, step, apply, hist, backlog, max_steps) ||
          PyList_Append(coda.get(), item))
        return nullptr;
      continue;
    }
    Ref row(PyLong_FromSsize_t(i));
    Ref entry(row ? PyTuple_Pack(2, flags, row.get()) : nullptr);
    if (!entry || PyDict_SetItem(pending, key.get(), entry.get()) || !set_long(item, s_recurrent_step, step + 1) ||
        PyList_Append(refills.get(), item))
      return nullptr;
  }
  return Py_BuildValue("(OOO)", coda.get(), refills.get(), exits.get());
}

PyMethodDef kMethods[] = {
    {"route_sync", route_sync, METH_VARARGS,
     "route_sync(items, flags, max_steps, histogram, backlog) -> (coda_items, refills, exits)"},
    {"route_lists", route_lists, METH_VARARGS,
     "route_lists(items, lists, max_steps, histogram, backlog) -> (coda_items, refills, exits)"},
    {"fill_recurrent", fill_recurrent, METH_VARARGS,
     "fill_recurrent(items, i64, i32, table_row_of, core_base, core_layers, slot_of_step)"},
    {"enqueue_front", enqueue_front, METH_VARARGS, "enqueue_front(queue, items, max_steps, in_flight) -> refills"},
    {"pop_batch", pop_batch, METH_VARARGS, "pop_batch(queue, size, slot_of_step) -> items"},
    {"pop_front", pop_front, METH_VARARGS, "pop_front(queue, n) -> items"},
    {"split_live", split_live, METH_VARARGS, "split_live(items, finished_status) -> (live, dead)"},
    {"select_eager", select_eager, METH_VARARGS,
     "select_eager(coda_items, block_size, allocate, item_type, token) -> (items, rows, flags)"},
    {"bind_request_types", bind_request_types, METH_VARARGS, "bind_request_types(RequestStatus, FutureRequestState)"},
    {"bind_batch_type", bind_batch_type, METH_O, "bind_batch_type(ScheduledCDBBatch)"},
    {"schedule_next", schedule_next, METH_VARARGS,
     "schedule_next(scheduler, token_budget, cache_budget, allow_coda) -> ScheduledCDBBatch | None"},
    {"schedule_prefill", schedule_prefill, METH_VARARGS,
     "schedule_prefill(scheduler, token_budget, cache_budget) -> ScheduledCDBBatch | None"},
    {"prefill_bucket", prefill_bucket, METH_O, "prefill_bucket(scheduler) -> prefill candidates"},
    {"record_resident_sample", record_resident_sample, METH_O, "record_resident_sample(scheduler)"},
    {"prefill_admitted", prefill_admitted, METH_O, "prefill_admitted(scheduler) -> bool"},
    {"allocate_if_needed", allocate_if_needed, METH_VARARGS,
     "allocate_if_needed(scheduler, state, tokens) -> whether the request holds blocks for them"},
    {"update_completion", update_completion, METH_VARARGS,
     "update_completion(state, token) -> whether the request finished on this sampled token"},
    {"consume_coda", consume_coda, METH_VARARGS, "consume_coda(items, tokens, eager) -> [(state, stage), ...]"},
    {"add_tokens_in_flight", add_tokens_in_flight, METH_O, "add_tokens_in_flight(items)"},
    {"route_delayed", route_delayed, METH_VARARGS,
     "route_delayed(items, flags, max_steps, pending, histogram, backlog) -> (coda_items, refills, exits)"},
    {"coda_upload", coda_upload, METH_VARARGS,
     "coda_upload(items, successors, rows, upload_addr, upload_len, free_slots, next_slot, capacity) -> next_slot"},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_tick", "CDB host tick core", -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__tick(void) {
  struct Name { PyObject** slot; const char* text; };
  const Name names[] = {
      {&s_recurrent_step, "recurrent_step"}, {&s_apply_exit_gate, "apply_exit_gate"}, {&s_state, "state"},
      {&s_current_token_exit_depth, "current_token_exit_depth"}, {&s_exit_depths, "exit_depths"},
      {&s_hidden_slot, "hidden_slot"}, {&s_token_position, "token_position"}, {&s_request_id, "request_id"},
      {&s_synthetic_exit_depth, "synthetic_exit_depth"}, {&s_status_field, "_status"},
      {&s_position_offset, "position_offset"}, {&s_allocated_blocks, "allocated_blocks"},
      {&s_tokens_in_flight, "tokens_in_flight"}, {&s_generated_tokens, "generated_tokens"},
      {&s_new_tokens_limit, "_new_tokens_limit"}, {&s_replay_eos_finishes, "replay_eos_finishes"},
      {&s_next_synthetic_exit_depth, "next_synthetic_exit_depth"},
      {&s_active_requests, "active_requests"}, {&s_waiting_requests, "waiting_requests"},
      {&s_waiting_order, "waiting_requests_order"}, {&s_block_new_requests, "block_new_requests"},
      {&s_ready_queue, "ready_queue"}, {&s_coda_queue, "coda_queue"}, {&s_in_flight_ids, "in_flight_request_ids"},
      {&s_max_num_seqs, "max_num_seqs"}, {&s_min_coda_batch_size, "min_coda_batch_size"},
      {&s_min_free_slots, "min_free_slots"}, {&s_safety_margin, "safety_margin"},
      {&s_kv_pressure_mode, "kv_pressure_mode"}, {&s_max_model_len, "max_model_len"}, {&s_cache, "cache"},
      {&s_max_fast_path_len, "max_decode_fast_path_length"}, {&s_slot_of_step, "_slot_of_step"},
      {&s_mixed_batches, "mixed_batches_scheduled"}, {&s_max_in_flight, "max_in_flight_requests"},
      {&s_max_live, "max_live_requests"}, {&s_max_resident, "max_resident_requests"},
      {&s_resident_samples, "resident_samples"}, {&s_resident_sum, "resident_sum"},
      {&s_steady_warmup, "steady_warmup_requests"}, {&s_advance_steady, "_advance_steady_window"},
      {&s_block_manager, "_block_manager"}, {&s_num_blocks, "num_blocks"}, {&s_block_size, "block_size"},
      {&s_allocate_blocks, "allocate_blocks"}, {&s_get_num_free_blocks, "get_num_free_blocks"},
      {&s_is_cpu_offloaded, "is_cpu_offloaded"}, {&s_remaining_prefill, "remaining_prefill_tokens"},
      {&s_tokens_to_process, "tokens_to_process"}, {&s_initial_tokens, "initial_tokens"},
      {&s_max_new_tokens, "max_new_tokens"}, {&s_status, "status"}, {&s_popleft, "popleft"},
      {&s_reserve, "reserve"}, {&s_kind_coda, "coda"}, {&s_kind_prefill, "prefill"},
      {&s_kind_recurrent, "recurrent"}, {&s_eos_ids, "_eos_token_ids"}, {&s_stop_sequences, "stop_sequences"},
      {&s_first_token_time, "first_token_time"}, {&s_name, "name"}, {&s_get, "get"},
  };
  for (const Name& nm : names) {
    *nm.slot = PyUnicode_InternFromString(nm.text);
    if (!*nm.slot) return nullptr;
  }
  {
    PyObject* time_module = PyImport_ImportModule("time");
    if (!time_module) return nullptr;
    g_perf_counter = PyObject_GetAttrString(time_module, "perf_counter");
    Py_DECREF(time_module);
    if (!g_perf_counter) return nullptr;
  }
  BlockPoolType.tp_name = "_tick.BlockPool";
  BlockPoolType.tp_basicsize = sizeof(BlockPool);
  BlockPoolType.tp_flags = Py_TPFLAGS_DEFAULT;
  BlockPoolType.tp_doc = "FIFO block manager: BlockPool(num_blocks, block_size=0)";
  BlockPoolType.tp_new = BlockPool_new;
  BlockPoolType.tp_dealloc = BlockPool_dealloc;
  BlockPoolType.tp_methods = kBlockPoolMethods;
  BlockPoolType.tp_getset = kBlockPoolGetSet;
  kItemQueueSeq.sq_length = ItemQueue_len;
  ItemQueueType.tp_name = "_tick.ItemQueue";
  ItemQueueType.tp_basicsize = sizeof(ItemQueue);
  ItemQueueType.tp_flags = Py_TPFLAGS_DEFAULT | Py_TPFLAGS_HAVE_GC;
  ItemQueueType.tp_doc = "Deque of work items: ItemQueue()";
  ItemQueueType.tp_new = ItemQueue_new;
  ItemQueueType.tp_dealloc = ItemQueue_dealloc;
  ItemQueueType.tp_traverse = ItemQueue_traverse;
  ItemQueueType.tp_clear = ItemQueue_clear_refs;
  ItemQueueType.tp_iter = ItemQueue_iter;
  ItemQueueType.tp_as_sequence = &kItemQueueSeq;
  ItemQueueType.tp_methods = kItemQueueMethods;
  if (PyType_Ready(&BlockPoolType) < 0 || PyType_Ready(&ItemQueueType) < 0) return nullptr;
  PyObject* module = PyModule_Create(&kModule);
  if (!module) return nullptr;
  Py_INCREF(&BlockPoolType);
  Py_INCREF(&ItemQueueType);
  if (PyModule_AddObject(module, "BlockPool", reinterpret_cast<PyObject*>(&BlockPoolType)) < 0 ||
      PyModule_AddObject(module, "ItemQueue", reinterpret_cast<PyObject*>(&ItemQueueType)) < 0) {
    Py_DECREF(module);
    return nullptr;
  }
  return module;
}
