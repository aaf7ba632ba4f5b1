/*
 * Host bookkeeping of one batched verify step, as a CPython extension
 * (nanoengine_amd._host_step).  The per-slot work before and after the device step
 * -- which sequences need new KV blocks, where the blocks go in the tables, and
 * appending each sequence's emitted tokens -- is a loop over up to max_seqs slots
 * that costs ~1 us per slot through numpy and Python objects and ~0.1 us here.
 * nanoengine_amd/host_step.py holds the same three functions in Python; both
 * follow ne/engine/generation/speculative_generator.py:54-72 and
 * ne/engine/memory/paged_allocator.py:50-55.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>
#include <string.h>

typedef struct {
  Py_buffer view;
  int ok;
} Buf;

/* A C-contiguous buffer of `itemsize`-byte items with at least `min_items` items. */
static int get_buf(PyObject* obj, Buf* b, Py_ssize_t itemsize, Py_ssize_t min_items, int writable,
                   const char* name) {
  b->ok = 0;
  if (PyObject_GetBuffer(obj, &b->view, PyBUF_C_CONTIGUOUS | (writable ? PyBUF_WRITABLE : 0)) != 0) return -1;
  b->ok = 1;
  if (b->view.itemsize != itemsize || b->view.len / itemsize < min_items) {
    PyErr_Format(PyExc_ValueError, "%s: need >= %zd items of %zd bytes (got %zd of %zd)", name, min_items,
                 itemsize, b->view.len / (b->view.itemsize ? b->view.itemsize : 1), b->view.itemsize);
    return -1;
  }
  return 0;
}

static void release(Buf* bufs, int n) {
  for (int i = 0; i < n; ++i)
    if (bufs[i].ok) PyBuffer_Release(&bufs[i].view);
}

/* plan_growth(lengths i64[S], num_drafts i32[S], owned i64[S], active bool[S], block_size)
 *   -> (slots, counts, targets, total): each active slot whose length + guesses exceeds
 *   its blocks * block_size, in slot order, with the blocks it needs and the tokens. */
static PyObject* plan_growth(PyObject* self, PyObject* args) {
  PyObject *o_len, *o_nd, *o_owned, *o_act;
  long long bs;
  if (!PyArg_ParseTuple(args, "OOOOL", &o_len, &o_nd, &o_owned, &o_act, &bs)) return NULL;
  if (bs <= 0) return PyErr_Format(PyExc_ValueError, "block_size must be positive");
  Buf b[4];
  memset(b, 0, sizeof(b));
  PyObject *slots = NULL, *counts = NULL, *targets = NULL;
  if (get_buf(o_act, &b[3], 1, 0, 0, "active") != 0) goto fail;
  const Py_ssize_t S = b[3].view.len;
  if (get_buf(o_len, &b[0], 8, S, 0, "lengths") != 0 || get_buf(o_nd, &b[1], 4, S, 0, "num_drafts") != 0 ||
      get_buf(o_owned, &b[2], 8, S, 0, "owned") != 0)
    goto fail;
  const int64_t* len = (const int64_t*)b[0].view.buf;
  const int32_t* nd = (const int32_t*)b[1].view.buf;
  const int64_t* owned = (const int64_t*)b[2].view.buf;
  const uint8_t* act = (const uint8_t*)b[3].view.buf;
  slots = PyList_New(0);
  counts = PyList_New(0);
  targets = PyList_New(0);
  if (!slots || !counts || !targets) goto fail;
  long long total = 0;
  for (Py_ssize_t s = 0; s < S; ++s) {
    if (!act[s]) continue;
    const long long need = len[s] + nd[s];
    if (need <= owned[s] * bs) continue;
    const long long c = (need + bs - 1) / bs - owned[s];
    PyObject *ps = PyLong_FromSsize_t(s), *pc = PyLong_FromLongLong(c), *pt = PyLong_FromLongLong(need);
    int err = !ps || !pc || !pt || PyList_Append(slots, ps) || PyList_Append(counts, pc) ||
              PyList_Append(targets, pt);
    Py_XDECREF(ps);
    Py_XDECREF(pc);
    Py_XDECREF(pt);
    if (err) goto fail;
    total += c;
  }
  release(b, 4);
  return Py_BuildValue("(NNNL)", slots, counts, targets, total);
fail:
  release(b, 4);
  Py_XDECREF(slots);
  Py_XDECREF(counts);
  Py_XDECREF(targets);
  return NULL;
}

/* assign_blocks(tables i32[S, W], owned i64[S], slots, counts, blocks): slot slots[i]
 *   gets the next counts[i] entries of blocks at table positions owned .. owned + c - 1;
 *   owned grows by c. */
static PyObject* assign_blocks(PyObject* self, PyObject* args) {
  PyObject *o_tab, *o_owned, *o_slots, *o_counts, *o_blocks;
  if (!PyArg_ParseTuple(args, "OOO!O!O!", &o_tab, &o_owned, &PyList_Type, &o_slots, &PyList_Type, &o_counts,
                        &PyList_Type, &o_blocks))
    return NULL;
  Buf b[2];
  memset(b, 0, sizeof(b));
  if (PyObject_GetBuffer(o_tab, &b[0].view, PyBUF_C_CONTIGUOUS | PyBUF_WRITABLE | PyBUF_ND) != 0) return NULL;
  b[0].ok = 1;
  if (b[0].view.ndim != 2 || b[0].view.itemsize != 4) {
    PyErr_SetString(PyExc_ValueError, "tables must be a 2-D int32 array");
    goto fail;
  }
  const Py_ssize_t S = b[0].view.shape[0], W = b[0].view.shape[1];
  if (get_buf(o_owned, &b[1], 8, S, 1, "owned") != 0) goto fail;
  int32_t* tab = (int32_t*)b[0].view.buf;
  int64_t* owned = (int64_t*)b[1].view.buf;
  const Py_ssize_t n = PyList_GET_SIZE(o_slots), nb = PyList_GET_SIZE(o_blocks);
  if (PyList_GET_SIZE(o_counts) != n) {
    PyErr_SetString(PyExc_ValueError, "slots and counts differ in length");
    goto fail;
  }
  Py_ssize_t at = 0;
  for (Py_ssize_t i = 0; i < n; ++i) {
    const Py_ssize_t s = PyLong_AsSsize_t(PyList_GET_ITEM(o_slots, i));
    const Py_ssize_t c = PyLong_AsSsize_t(PyList_GET_ITEM(o_counts, i));
    if (PyErr_Occurred()) goto fail;
    if (s < 0 || s >= S || c < 0 || owned[s] + c > W || at + c > nb) {
      PyErr_Format(PyExc_ValueError, "block assignment out of range (slot %zd, %zd blocks)", s, c);
      goto fail;
    }
    for (Py_ssize_t j = 0; j < c; ++j) {
      const long blk = PyLong_AsLong(PyList_GET_ITEM(o_blocks, at + j));
      if (PyErr_Occurred()) goto fail;
      tab[s * W + owned[s] + j] = (int32_t)blk;
    }
    owned[s] += c;
    at += c;
  }
  release(b, 2);
  Py_RETURN_NONE;
fail:
  release(b, 2);
  return NULL;
}

/* finish_step(active, slots, out i32[S, R], num_out i32[S], num_drafts i32[S], act bool[S],
 *             lengths i64[S], generated i64[S], steps i64[S], max_new i64[S], honours bool[S],
 *             stop_ids tuple, result_type, on_cached or None) -> (results, finishing)
 *   Mirrors advance by the emitted counts for every active slot.  Then, per slot of
 *   `active` in order: the sequence's sampling step advances and its emitted tokens
 *   become a list; a slot that may finish (length limit reached, or a stop token
 *   emitted by a slot that honours stops) gets None in `results` and (slot, tokens) in
 *   `finishing` for the caller; any other appends the tokens, sets num_cached_tokens
 *   to len(token_ids) - 1, calls on_cached(seq) and gets
 *   result_type(tokens, None, num_drafts, emitted - 1). */
static PyObject *s_sampling_generator, *s_step, *s_token_ids, *s_num_cached_tokens, *s_one;

/* result_type(tokens, None, guesses, kept), stealing `tokens`.  A tuple subclass (a
 * NamedTuple) is filled in place, as tuple.__new__(result_type, items) does, without a
 * call into Python. */
static PyObject* make_result(PyObject* type, PyObject* tokens, long guesses, long kept) {
  if (PyType_Check(type) && PyType_IsSubtype((PyTypeObject*)type, &PyTuple_Type)) {
    PyObject* items = PyTuple_New(4);
    if (!items) {
      Py_DECREF(tokens);
      return NULL;
    }
    PyObject* g = PyLong_FromLong(guesses);
    PyObject* k = PyLong_FromLong(kept);
    Py_INCREF(Py_None);
    PyTuple_SET_ITEM(items, 0, tokens);
    PyTuple_SET_ITEM(items, 1, Py_None);
    PyTuple_SET_ITEM(items, 2, g ? g : (Py_INCREF(Py_None), Py_None));
    PyTuple_SET_ITEM(items, 3, k ? k : (Py_INCREF(Py_None), Py_None));
    if (!g || !k) {
      Py_DECREF(items);
      return NULL;
    }
    PyObject* targs = PyTuple_Pack(1, items);
    Py_DECREF(items);
    if (!targs) return NULL;
    PyObject* res = PyTuple_Type.tp_new((PyTypeObject*)type, targs, NULL);
    Py_DECREF(targs);
    return res;
  }
  return PyObject_CallFunction(type, "NOll", tokens, Py_None, guesses, kept);
}

/* One active slot of finish_step: advance its sampling step, then either queue it for the
   one-token-at-a-time finish (fin[s]) or append its tokens, set num_cached_tokens, call
   on_cached and record its result.  Returns nonzero with a Python error set. */
static int finish_slot(PyObject* seq, PyObject* key, Py_ssize_t s, Py_ssize_t R, const int32_t* out,
                       const int32_t* nout, const int32_t* nd, const unsigned char* fin, PyObject* o_type,
                       PyObject* o_cached, PyObject* results, PyObject* finishing) {
  const int32_t n = nout[s];
  /* seq.sampling_generator.step += 1 */
  PyObject* gobj = PyObject_GetAttr(seq, s_sampling_generator);
  if (!gobj) return 1;
  PyObject* st = PyObject_GetAttr(gobj, s_step);
  PyObject* st1 = st ? PyNumber_Add(st, s_one) : NULL;
  int err = !st1 || PyObject_SetAttr(gobj, s_step, st1);
  Py_XDECREF(st);
  Py_XDECREF(st1);
  Py_DECREF(gobj);
  if (err) return 1;
  PyObject* tokens = PyList_New(n);
  if (!tokens) return 1;
  for (int32_t j = 0; j < n; ++j) {
    PyObject* v = PyLong_FromLong(out[s * R + j]);
    if (!v) {
      Py_DECREF(tokens);
      return 1;
    }
    PyList_SET_ITEM(tokens, j, v);
  }
  if (fin[s]) {
    PyObject* pair = Py_BuildValue("(nN)", s, tokens);
    err = !pair || PyDict_SetItem(results, key, Py_None) || PyList_Append(finishing, pair);
    Py_XDECREF(pair);
    return err;
  }
  PyObject* ids = PyObject_GetAttr(seq, s_token_ids);
  if (!ids || !PyList_Check(ids)) {
    Py_XDECREF(ids);
    Py_DECREF(tokens);
    if (!PyErr_Occurred()) PyErr_SetString(PyExc_TypeError, "token_ids must be a list");
    return 1;
  }
  const Py_ssize_t old = PyList_GET_SIZE(ids);
  err = PyList_SetSlice(ids, old, old, tokens);
  PyObject* cached = err ? NULL : PyLong_FromSsize_t(PyList_GET_SIZE(ids) - 1);
  Py_DECREF(ids);
  err = err || !cached || PyObject_SetAttr(seq, s_num_cached_tokens, cached);
  Py_XDECREF(cached);
  if (!err && o_cached != Py_None) {
    PyObject* r = PyObject_CallOneArg(o_cached, seq);
    err = !r;
    Py_XDECREF(r);
  }
  if (err) {
    Py_DECREF(tokens);
    return 1;
  }
  PyObject* res = make_result(o_type, tokens, nd[s], n - 1);
  err = !res || PyDict_SetItem(results, key, res);
  Py_XDECREF(res);
  return err;
}

static PyObject* finish_step(PyObject* self, PyObject* args) {
  PyObject *o_active, *o_slots, *o_out, *o_nout, *o_nd, *o_act, *o_len, *o_gen, *o_steps, *o_max, *o_hon,
      *o_stops, *o_type, *o_cached;
  if (!PyArg_ParseTuple(args, "O!O!OOOOOOOOOO!OO", &PyList_Type, &o_active, &PyList_Type, &o_slots, &o_out,
                        &o_nout, &o_nd, &o_act, &o_len, &o_gen, &o_steps, &o_max, &o_hon, &PyTuple_Type, &o_stops,
                        &o_type, &o_cached))
    return NULL;
  Buf b[10];
  memset(b, 0, sizeof(b));
  PyObject *results = NULL, *finishing = NULL;
  unsigned char* fin = NULL;
  if (PyObject_GetBuffer(o_out, &b[0].view, PyBUF_C_CONTIGUOUS | PyBUF_ND) != 0) return NULL;
  b[0].ok = 1;
  if (b[0].view.ndim != 2 || b[0].view.itemsize != 4) {
    PyErr_SetString(PyExc_ValueError, "out must be a 2-D int32 array");
    goto fail;
  }
  const Py_ssize_t S = b[0].view.shape[0], R = b[0].view.shape[1];
  if (get_buf(o_nout, &b[1], 4, S, 0, "num_out") || get_buf(o_nd, &b[2], 4, S, 0, "num_drafts") ||
      get_buf(o_act, &b[3], 1, S, 0, "act") || get_buf(o_len, &b[4], 8, S, 1, "lengths") ||
      get_buf(o_gen, &b[5], 8, S, 1, "generated") || get_buf(o_steps, &b[6], 8, S, 1, "steps") ||
      get_buf(o_max, &b[7], 8, S, 0, "max_new") || get_buf(o_hon, &b[8], 1, S, 0, "honours"))
    goto fail;
  const int32_t* out = (const int32_t*)b[0].view.buf;
  const int32_t* nout = (const int32_t*)b[1].view.buf;
  const int32_t* nd = (const int32_t*)b[2].view.buf;
  const uint8_t* act = (const uint8_t*)b[3].view.buf;
  int64_t* len = (int64_t*)b[4].view.buf;
  int64_t* gen = (int64_t*)b[5].view.buf;
  int64_t* steps = (int64_t*)b[6].view.buf;
  const int64_t* max_new = (const int64_t*)b[7].view.buf;
  const uint8_t* hon = (const uint8_t*)b[8].view.buf;
  const Py_ssize_t nstops = PyTuple_GET_SIZE(o_stops);
  long long stops_small[64];
  if (nstops > 64) {
    PyErr_SetString(PyExc_ValueError, "at most 64 stop tokens");
    goto fail;
  }
  for (Py_ssize_t i = 0; i < nstops; ++i) {
    stops_small[i] = PyLong_AsLongLong(PyTuple_GET_ITEM(o_stops, i));
    if (PyErr_Occurred()) goto fail;
  }
  fin = (unsigned char*)PyMem_Calloc((size_t)S, 1);
  if (!fin) {
    PyErr_NoMemory();
    goto fail;
  }
  /* every input check comes before the first change to a mirror */
  for (Py_ssize_t s = 0; s < S; ++s) {
    if (act[s] && (nout[s] < 0 || nout[s] > R)) {
      PyErr_Format(PyExc_ValueError, "slot %zd emitted %d tokens (at most %zd)", s, nout[s], R);
      goto fail;
    }
  }
  const Py_ssize_t na = PyList_GET_SIZE(o_active), ns = PyList_GET_SIZE(o_slots);
  for (Py_ssize_t i = 0; i < na; ++i) {
    const Py_ssize_t s = PyLong_AsSsize_t(PyList_GET_ITEM(o_active, i));
    if (PyErr_Occurred()) goto fail;
    if (s < 0 || s >= S || s >= ns || !act[s] || PyList_GET_ITEM(o_slots, s) == Py_None) {
      PyErr_Format(PyExc_ValueError, "active slot %zd out of range, inactive or empty", s);
      goto fail;
    }
  }
  for (Py_ssize_t s = 0; s < S; ++s) {
    if (!act[s]) continue;
    const int32_t e = nout[s];
    len[s] += e;
    gen[s] += e;
    steps[s] += 1;
    int f = gen[s] >= max_new[s];
    if (!f && hon[s]) {
      for (int32_t j = 0; j < e && !f; ++j)
        for (Py_ssize_t t = 0; t < nstops; ++t)
          if ((long long)out[s * R + j] == stops_small[t]) {
            f = 1;
            break;
          }
    }
    fin[s] = (unsigned char)f;
  }
  results = PyDict_New();
  finishing = PyList_New(0);
  if (!results || !finishing) goto fail;
  for (Py_ssize_t i = 0; i < na; ++i) {
    PyObject* key = PyList_GET_ITEM(o_active, i);
    const Py_ssize_t s = PyLong_AsSsize_t(key);
    /* held across the calls back into Python below (a callback may change the slot list) */
    PyObject* seq = PyList_GET_ITEM(o_slots, s);
    Py_INCREF(seq);
    const int err_seq = finish_slot(seq, key, s, R, out, nout, nd, fin, o_type, o_cached, results, finishing);
    Py_DECREF(seq);
    if (err_seq) goto fail;
  }
  PyMem_Free(fin);
  release(b, 10);
  return Py_BuildValue("(NN)", results, finishing);
fail:
  PyMem_Free(fin);
  release(b, 10);
  Py_XDECREF(results);
  Py_XDECREF(finishing);
  return NULL;
}
static PyMethodDef methods[] = {
    {"plan_growth", plan_growth, METH_VARARGS, "slots that need KV blocks this step, their counts and targets"},
    {"assign_blocks", assign_blocks, METH_VARARGS, "write peeked blocks into the host block tables"},
    {"finish_step", finish_step, METH_VARARGS, "advance the mirrors and append each slot's emitted tokens"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_host_step", NULL, -1, methods};

PyMODINIT_FUNC PyInit__host_step(void) {
  s_sampling_generator = PyUnicode_InternFromString("sampling_generator");
  s_step = PyUnicode_InternFromString("step");
  s_token_ids = PyUnicode_InternFromString("token_ids");
  s_num_cached_tokens = PyUnicode_InternFromString("num_cached_tokens");
  s_one = PyLong_FromLong(1);
  if (!s_sampling_generator || !s_step || !s_token_ids || !s_num_cached_tokens || !s_one) return NULL;
  return PyModule_Create(&module);
}
