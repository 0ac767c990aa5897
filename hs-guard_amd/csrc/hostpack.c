/*
 * Host side of one packed tick, native (CPython extension module hs_guard._hostpack).
 *
 * A serving tick spends its host time before the graph launch (turning the requests into the packed layout)
 * and after it (turning the packed outputs into the [R, n, lb, 3] array step_packed returns), with the GPU
 * idle in both. These three functions do that work in C over the request list itself, with the same results
 * as the numpy route in hs_guard/engine/slot_engine.py (pack_ticks, padded_rows), which stays the reference
 * for the tests:
 *
 *   scan(requests, max_slots, vocab[, strict]) -> (n, total, max_len), or None when a request would fail the
 *       tick's checks (a slot outside [0, max_slots), a slot twice, an empty request, a token id that is not an
 *       integer in [0, vocab)); the caller then runs its own checks, which raise the reference's errors
 *       (src/hs_guard/runtime.py:148-174; docs/ENGINE.md:9 requires in-vocabulary ids). strict: slots and ids
 *       must be Python ints (bool included), as the reference's isinstance(x, int) checks have it; otherwise
 *       numpy integers pass too.
 *   fill(requests, length, nb, tb, max_slots, vocab, out, lens, offsets, slots) -> None (ValueError for an id
 *       outside [0, vocab))
 *       out [2 tb + 4 nb] int64: ids | positions | offsets | lens | slots | starts of the packed tick with the
 *       rows longest first (stable), padding rows on the scratch slot max_slots (pack_ticks' layout);
 *       lens / offsets / slots [n] int64 in request order (offsets = where each request's tokens sit).
 *   scatter_padded(flat, R, T, lens, offsets, lb, out) -> None
 *       flat [R, T, 3] float32 (the tick's packed outputs), out [R, n, lb, 3] float32: request r's outputs at
 *       out[:, r, :lens[r]] and zeros after (padded_rows).
 *   gather_rows(flat, R, T, lens, offsets, out) -> None
 *       out [R, sum(lens), 3] float32: the requests' outputs one after another in request order
 *       (request_order).
 *
 * Token ids and slots are read with the integer protocol (Python ints, numpy integers); ids may be any
 * sequence. Arrays are passed as writable / readable C-contiguous buffers of the stated item size.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static int get_buffer(PyObject* obj, Py_buffer* view, Py_ssize_t itemsize, Py_ssize_t min_items, int writable,
                      const char* what) {
  if (PyObject_GetBuffer(obj, view, PyBUF_C_CONTIGUOUS | PyBUF_FORMAT | (writable ? PyBUF_WRITABLE : 0)) != 0)
    return -1;
  if (view->itemsize != itemsize || view->len / itemsize < min_items) {
    PyErr_Format(PyExc_ValueError, "%s: expected at least %zd items of %zd bytes", what, min_items, itemsize);
    PyBuffer_Release(view);
    return -1;
  }
  return 0;
}

/* slot and length of request i: requests[i] = (slot, ids) */
static int request_at(PyObject* seq, Py_ssize_t i, long long* slot, PyObject** ids_fast) {
  PyObject* item = PySequence_Fast_GET_ITEM(seq, i);
  if (!PyTuple_Check(item) && !PyList_Check(item)) {
    PyErr_SetString(PyExc_TypeError, "requests must be (slot, token_ids) pairs");
    return -1;
  }
  if (PySequence_Fast_GET_SIZE(item) != 2) {
    PyErr_SetString(PyExc_TypeError, "requests must be (slot, token_ids) pairs");
    return -1;
  }
  PyObject* s = PySequence_Fast_GET_ITEM(item, 0);
  *slot = PyLong_AsLongLong(s);
  if (*slot == -1 && PyErr_Occurred()) return -1;
  if (ids_fast) {
    *ids_fast = PySequence_Fast(PySequence_Fast_GET_ITEM(item, 1), "token ids must be a sequence");
    if (!*ids_fast) return -1;
  }
  return 0;
}

/* every id of a request an integer in [0, vocab) (numpy integers included unless strict); 0 otherwise, with no
   error set */
static int ids_in_vocab(PyObject* ids, long long vocab, int strict) {
  PyObject* fast = PySequence_Fast(ids, "token ids must be a sequence");
  if (!fast) {
    PyErr_Clear();
    return 0;
  }
  const Py_ssize_t len = PySequence_Fast_GET_SIZE(fast);
  PyObject** items = PySequence_Fast_ITEMS(fast);
  int ok = 1;
  for (Py_ssize_t t = 0; t < len && ok; ++t) {
    if (PyFloat_Check(items[t]) || (strict && !PyLong_Check(items[t]))) {
      /* integers only (bool is an int, as the reference's isinstance check has it) */
      ok = 0;
      break;
    }
    const long long v = PyLong_AsLongLong(items[t]);
    if (v == -1 && PyErr_Occurred()) {
      PyErr_Clear();
      ok = 0;
    } else if (v < 0 || v >= vocab) {
      ok = 0;
    }
  }
  Py_DECREF(fast);
  return ok;
}

static PyObject* scan(PyObject* self, PyObject* args) {
  PyObject *requests, *seq;
  long long max_slots, vocab;
  int strict = 0;
  if (!PyArg_ParseTuple(args, "OLL|i", &requests, &max_slots, &vocab, &strict)) return NULL;
  seq = PySequence_Fast(requests, "requests must be a sequence");
  if (!seq) return NULL;
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(seq);
  unsigned char* seen = (unsigned char*)calloc((size_t)(max_slots > 0 ? max_slots : 1), 1);
  if (!seen) {
    Py_DECREF(seq);
    return PyErr_NoMemory();
  }
  long long total = 0, max_len = 0;
  int ok = 1;
  for (Py_ssize_t i = 0; i < n && ok; ++i) {
    long long slot;
    PyObject* item = PySequence_Fast_GET_ITEM(seq, i);
    if ((!PyTuple_Check(item) && !PyList_Check(item)) || PySequence_Fast_GET_SIZE(item) != 2) {
      ok = 0;   /* let the caller's checks report it */
      break;
    }
    if ((strict && !PyLong_Check(PySequence_Fast_GET_ITEM(item, 0))) || request_at(seq, i, &slot, NULL) != 0) {
      PyErr_Clear();
      ok = 0;
      break;
    }
    const Py_ssize_t len = PyObject_Length(PySequence_Fast_GET_ITEM(item, 1));
    if (len < 0) {
      PyErr_Clear();
      ok = 0;
      break;
    }
    if (slot < 0 || slot >= max_slots || seen[slot] || len == 0 ||
        !ids_in_vocab(PySequence_Fast_GET_ITEM(item, 1), vocab, strict)) {
      ok = 0;
      break;
    }
    seen[slot] = 1;
    total += len;
    if (len > max_len) max_len = len;
  }
  free(seen);
  Py_DECREF(seq);
  if (!ok) Py_RETURN_NONE;
  return Py_BuildValue("(nLL)", n, total, max_len);
}

static PyObject* fill(PyObject* self, PyObject* args) {
  PyObject *requests, *length_o, *out_o, *lens_o, *offs_o, *slots_o;
  long long nb, tb, max_slots, vocab;
  if (!PyArg_ParseTuple(args, "OOLLLLOOOO", &requests, &length_o, &nb, &tb, &max_slots, &vocab, &out_o, &lens_o,
                        &offs_o, &slots_o))
    return NULL;
  PyObject* seq = PySequence_Fast(requests, "requests must be a sequence");
  if (!seq) return NULL;
  const Py_ssize_t n = PySequence_Fast_GET_SIZE(seq);
  Py_buffer length_b, out_b, lens_b, offs_b, slots_b;
  int have = 0;
  PyObject** ids = NULL;
  Py_ssize_t* order = NULL;
  PyObject* result = NULL;
  if (n > nb || tb < 0) {
    PyErr_SetString(PyExc_ValueError, "fill: more requests than rows, or a negative token bucket");
    goto done;
  }
  if (get_buffer(length_o, &length_b, 8, max_slots, 0, "length") != 0) goto done;
  have = 1;
  if (get_buffer(out_o, &out_b, 8, 2 * tb + 4 * nb, 1, "out") != 0) goto done;
  have = 2;
  if (get_buffer(lens_o, &lens_b, 8, n, 1, "lens") != 0) goto done;
  have = 3;
  if (get_buffer(offs_o, &offs_b, 8, n, 1, "offsets") != 0) goto done;
  have = 4;
  if (get_buffer(slots_o, &slots_b, 8, n, 1, "slots") != 0) goto done;
  have = 5;
  {
    const int64_t* length = (const int64_t*)length_b.buf;
    int64_t* out = (int64_t*)out_b.buf;
    int64_t* lens = (int64_t*)lens_b.buf;
    int64_t* offs_req = (int64_t*)offs_b.buf;
    int64_t* slots = (int64_t*)slots_b.buf;
    ids = (PyObject**)calloc((size_t)(n > 0 ? n : 1), sizeof(PyObject*));
    order = (Py_ssize_t*)malloc((size_t)(n > 0 ? n : 1) * sizeof(Py_ssize_t));
    if (!ids || !order) {
      PyErr_NoMemory();
      goto done;
    }
    long long max_len = 0, total = 0;
    for (Py_ssize_t i = 0; i < n; ++i) {
      long long slot;
      if (request_at(seq, i, &slot, &ids[i]) != 0) goto done;
      if (slot < 0 || slot >= max_slots) {
        PyErr_SetString(PyExc_ValueError, "Slot is outside the allocated range");
        goto done;
      }
      slots[i] = slot;
      lens[i] = PySequence_Fast_GET_SIZE(ids[i]);
      if (lens[i] > max_len) max_len = lens[i];
      total += lens[i];
    }
    if (total > tb) {
      PyErr_SetString(PyExc_ValueError, "fill: the tick's tokens exceed the token bucket");
      goto done;
    }
    /* rows longest first, ties in request order (a stable counting sort on the length) */
    {
      Py_ssize_t* start = (Py_ssize_t*)calloc((size_t)max_len + 2, sizeof(Py_ssize_t));
      if (!start) {
        PyErr_NoMemory();
        goto done;
      }
      for (Py_ssize_t i = 0; i < n; ++i) start[max_len - lens[i] + 1]++;
      for (long long k = 1; k <= max_len + 1; ++k) start[k] += start[k - 1];
      for (Py_ssize_t i = 0; i < n; ++i) order[start[max_len - lens[i]]++] = i;
      free(start);
    }
    int64_t* id_out = out;
    int64_t* pos = out + tb;
    int64_t* offs = out + 2 * tb;
    int64_t* lns = offs + nb;
    int64_t* sls = lns + nb;
    int64_t* sts = sls + nb;
    int64_t off = 0;
    for (Py_ssize_t k = 0; k < n; ++k) {
      const Py_ssize_t i = order[k];
      const int64_t st = length[slots[i]];
      PyObject** items = PySequence_Fast_ITEMS(ids[i]);
      for (int64_t t = 0; t < lens[i]; ++t) {
        const long long v = PyLong_AsLongLong(items[t]);
        if (v == -1 && PyErr_Occurred()) goto done;
        if (v < 0 || v >= vocab) {
          PyErr_SetString(PyExc_ValueError, "Each request requires nonempty in-vocabulary integer token IDs");
          goto done;
        }
        id_out[off + t] = v;
        pos[off + t] = st + t;
      }
      offs[k] = off;
      lns[k] = lens[i];
      sls[k] = slots[i];
      sts[k] = st;
      offs_req[i] = off;
      off += lens[i];
    }
    for (int64_t t = off; t < tb; ++t) id_out[t] = pos[t] = 0;
    for (int64_t k = n; k < nb; ++k) {
      offs[k] = off;
      lns[k] = 0;
      sls[k] = max_slots;
      sts[k] = 0;
    }
  }
  Py_INCREF(Py_None);
  result = Py_None;
done:
  if (ids) {
    for (Py_ssize_t i = 0; i < n; ++i) Py_XDECREF(ids[i]);
    free(ids);
  }
  free(order);
  if (have >= 5) PyBuffer_Release(&slots_b);
  if (have >= 4) PyBuffer_Release(&offs_b);
  if (have >= 3) PyBuffer_Release(&lens_b);
  if (have >= 2) PyBuffer_Release(&out_b);
  if (have >= 1) PyBuffer_Release(&length_b);
  Py_DECREF(seq);
  return result;
}

static PyObject* scatter_padded(PyObject* self, PyObject* args) {
  PyObject *flat_o, *lens_o, *offs_o, *out_o;
  Py_ssize_t R, T, lb;
  if (!PyArg_ParseTuple(args, "OnnOOnO", &flat_o, &R, &T, &lens_o, &offs_o, &lb, &out_o)) return NULL;
  Py_buffer flat_b, lens_b, offs_b, out_b;
  if (get_buffer(lens_o, &lens_b, 8, 0, 0, "lens") != 0) return NULL;
  const Py_ssize_t n = lens_b.len / 8;
  PyObject* result = NULL;
  int have = 1;
  if (get_buffer(offs_o, &offs_b, 8, n, 0, "offsets") != 0) goto done;
  have = 2;
  if (get_buffer(flat_o, &flat_b, 4, R * T * 3, 0, "flat") != 0) goto done;
  have = 3;
  if (get_buffer(out_o, &out_b, 4, R * n * lb * 3, 1, "out") != 0) goto done;
  have = 4;
  {
    const int64_t* lens = (const int64_t*)lens_b.buf;
    const int64_t* offs = (const int64_t*)offs_b.buf;
    const float* flat = (const float*)flat_b.buf;
    float* out = (float*)out_b.buf;
    for (Py_ssize_t i = 0; i < n; ++i)
      if (lens[i] < 0 || lens[i] > lb || offs[i] < 0 || offs[i] + lens[i] > T) {
        PyErr_SetString(PyExc_ValueError, "scatter_padded: a row lies outside the packed outputs or lb");
        goto done;
      }
    for (Py_ssize_t r = 0; r < R; ++r)
      for (Py_ssize_t i = 0; i < n; ++i) {
        float* dst = out + ((r * n + i) * lb) * 3;
        memcpy(dst, flat + (r * T + offs[i]) * 3, (size_t)lens[i] * 3 * sizeof(float));
        memset(dst + lens[i] * 3, 0, (size_t)(lb - lens[i]) * 3 * sizeof(float));
      }
  }
  Py_INCREF(Py_None);
  result = Py_None;
done:
  if (have >= 4) PyBuffer_Release(&out_b);
  if (have >= 3) PyBuffer_Release(&flat_b);
  if (have >= 2) PyBuffer_Release(&offs_b);
  PyBuffer_Release(&lens_b);
  return result;
}

static PyObject* gather_rows(PyObject* self, PyObject* args) {
  PyObject *flat_o, *lens_o, *offs_o, *out_o;
  Py_ssize_t R, T;
  if (!PyArg_ParseTuple(args, "OnnOOO", &flat_o, &R, &T, &lens_o, &offs_o, &out_o)) return NULL;
  Py_buffer flat_b, lens_b, offs_b, out_b;
  if (get_buffer(lens_o, &lens_b, 8, 0, 0, "lens") != 0) return NULL;
  const Py_ssize_t n = lens_b.len / 8;
  const int64_t* lens = (const int64_t*)lens_b.buf;
  PyObject* result = NULL;
  int have = 1;
  Py_ssize_t total = 0;
  for (Py_ssize_t i = 0; i < n; ++i) total += lens[i];
  if (get_buffer(offs_o, &offs_b, 8, n, 0, "offsets") != 0) goto done;
  have = 2;
  if (get_buffer(flat_o, &flat_b, 4, R * T * 3, 0, "flat") != 0) goto done;
  have = 3;
  if (get_buffer(out_o, &out_b, 4, R * total * 3, 1, "out") != 0) goto done;
  have = 4;
  {
    const int64_t* offs = (const int64_t*)offs_b.buf;
    const float* flat = (const float*)flat_b.buf;
    float* out = (float*)out_b.buf;
    for (Py_ssize_t i = 0; i < n; ++i)
      if (lens[i] < 0 || offs[i] < 0 || offs[i] + lens[i] > T) {
        PyErr_SetString(PyExc_ValueError, "gather_rows: a row lies outside the packed outputs");
        goto done;
      }
    for (Py_ssize_t r = 0; r < R; ++r) {
      float* dst = out + r * total * 3;
      for (Py_ssize_t i = 0; i < n; ++i) {
        memcpy(dst, flat + (r * T + offs[i]) * 3, (size_t)lens[i] * 3 * sizeof(float));
        dst += lens[i] * 3;
      }
    }
  }
  Py_INCREF(Py_None);
  result = Py_None;
done:
  if (have >= 4) PyBuffer_Release(&out_b);
  if (have >= 3) PyBuffer_Release(&flat_b);
  if (have >= 2) PyBuffer_Release(&offs_b);
  PyBuffer_Release(&lens_b);
  return result;
}

static PyMethodDef methods[] = {
    {"scan", scan, METH_VARARGS, "(n, total, max_len) of a tick's requests, or None if a check would fail"},
    {"fill", fill, METH_VARARGS, "pack a tick's requests into the packed layout (rows longest first)"},
    {"scatter_padded", scatter_padded, METH_VARARGS, "packed outputs [R, T, 3] -> padded [R, n, lb, 3]"},
    {"gather_rows", gather_rows, METH_VARARGS, "packed outputs [R, T, 3] -> request order [R, sum(lens), 3]"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_hostpack",
                                    "Native host packing of a streaming tick", -1, methods};

PyMODINIT_FUNC PyInit__hostpack(void) { return PyModule_Create(&module); }
