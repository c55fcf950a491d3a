// Host tick core of the CDB engine: the per-launch loops over depth work items,
// as a CPython extension (built with g++, no GPU code).
//
//   route_sync      routes one recurrent launch's rows on the synchronous exit
//                   horizon (cdb/continuous_api.py:1090-1183 with _record_exit
//                   :1205-1223): exits go to the coda list, the rest step on.
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
PyObject* pop_batch(PyObject*, PyObject* args) {
  PyObject *queue, *slot_of_step;
  Py_ssize_t size;
  if (!PyArg_ParseTuple(args, "OnO", &queue, &size, &slot_of_step)) return nullptr;
  if (!is_queue(queue)) {
    PyErr_SetString(PyExc_TypeError, "queue must be an ItemQueue");
    return nullptr;
  }
  const bool filter = slot_of_step != Py_None;
  if (filter && !PyTuple_Check(slot_of_step)) {
    PyErr_SetString(PyExc_TypeError, "slot_of_step must be a tuple or None");
    return nullptr;
  }
  auto* q = reinterpret_cast<ItemQueue*>(queue)->items;
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

// pop_front(queue, n) -> the first min(n, len) items.
PyObject* pop_front(PyObject*, PyObject* args) {
  PyObject* queue;
  Py_ssize_t n;
  if (!PyArg_ParseTuple(args, "On", &queue, &n)) return nullptr;
  if (!is_queue(queue)) {
    PyErr_SetString(PyExc_TypeError, "queue must be an ItemQueue");
    return nullptr;
  }
  auto* q = reinterpret_cast<ItemQueue*>(queue)->items;
  const Py_ssize_t k = std::max<Py_ssize_t>(0, std::min<Py_ssize_t>(n, (Py_ssize_t)q->size()));
  PyObject* out = PyList_New(k);
  if (!out) return nullptr;
  for (Py_ssize_t i = 0; i < k; ++i) {
    PyList_SET_ITEM(out, i, q->front());  // the queue's reference moves into the list
    q->pop_front();
  }
  return out;
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

PyMethodDef kMethods[] = {
    {"route_sync", route_sync, METH_VARARGS,
     "route_sync(items, flags, max_steps, histogram, backlog) -> (coda_items, refills, exits)"},
    {"fill_recurrent", fill_recurrent, METH_VARARGS,
     "fill_recurrent(items, i64, i32, table_row_of, core_base, core_layers, slot_of_step)"},
    {"enqueue_front", enqueue_front, METH_VARARGS, "enqueue_front(queue, items, max_steps, in_flight) -> refills"},
    {"pop_batch", pop_batch, METH_VARARGS, "pop_batch(queue, size, slot_of_step) -> items"},
    {"pop_front", pop_front, METH_VARARGS, "pop_front(queue, n) -> items"},
    {"split_live", split_live, METH_VARARGS, "split_live(items, finished_status) -> (live, dead)"},
    {"select_eager", select_eager, METH_VARARGS,
     "select_eager(coda_items, block_size, allocate, item_type, token) -> (items, rows, flags)"},
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
  };
  for (const Name& nm : names) {
    *nm.slot = PyUnicode_InternFromString(nm.text);
    if (!*nm.slot) return nullptr;
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
