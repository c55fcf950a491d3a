// Host tick core of the CDB engine: the per-launch loops over depth work items,
// as a CPython extension (built with g++, no GPU code).
//
//   route_sync      routes one recurrent launch's rows on the synchronous exit
//                   horizon (cdb/continuous_api.py:1090-1183 with _record_exit
//                   :1205-1223): exits go to the coda list, the rest step on.
//   fill_recurrent  writes one launch's packed metadata into the pinned staging
//                   arrays (cdb/model_runner.py:704-754 assembles the same facts).
//
// Both read and write the engine's own Python objects (DepthWorkItem,
// RequestState), so the scheduler's state stays in one place; they replace the
// interpreter's per-row work, which is on the path between a launch's exit
// flags and the next launch.

#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <cstdint>
#include <cstring>

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

PyMethodDef kMethods[] = {
    {"route_sync", route_sync, METH_VARARGS,
     "route_sync(items, flags, max_steps, histogram, backlog) -> (coda_items, refills, exits)"},
    {"fill_recurrent", fill_recurrent, METH_VARARGS,
     "fill_recurrent(items, i64, i32, table_row_of, core_base, core_layers, slot_of_step)"},
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
      {&s_synthetic_exit_depth, "synthetic_exit_depth"},
  };
  for (const Name& nm : names) {
    *nm.slot = PyUnicode_InternFromString(nm.text);
    if (!*nm.slot) return nullptr;
  }
  return PyModule_Create(&kModule);
}
