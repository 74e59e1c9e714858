/*
 * CPython fast-call bindings of the per-step C-ABI entries
 * (include/flashrwkv2_amd.h).  ctypes converts every argument through its
 * generic machinery, which costs several microseconds for a 20-argument call;
 * the decode path makes two such calls per step.  These METH_FASTCALL
 * functions take the same positional arguments (pointers as Python ints or
 * None, sizes as ints, scale as a float) and call the library directly.  They
 * add no logic: argument validation stays in the library and in the Python
 * layer.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>

#include "../../include/flashrwkv2_amd.h"

static int arg_ptr(PyObject* o, void** out) {
  if (o == Py_None) {
    *out = NULL;
    return 0;
  }
  *out = PyLong_AsVoidPtr(o);
  return (*out == NULL && PyErr_Occurred()) ? -1 : 0;
}

static int arg_i32(PyObject* o, int32_t* out) {
  const long long v = PyLong_AsLongLong(o);
  if (v == -1 && PyErr_Occurred()) return -1;
  if (v < INT32_MIN || v > INT32_MAX) {
    PyErr_SetString(PyExc_OverflowError, "argument does not fit in int32");
    return -1;
  }
  *out = (int32_t)v;
  return 0;
}

static int arg_i64(PyObject* o, int64_t* out) {
  const long long v = PyLong_AsLongLong(o);
  if (v == -1 && PyErr_Occurred()) return -1;
  *out = (int64_t)v;
  return 0;
}

static int arg_f32(PyObject* o, float* out) {
  const double v = PyFloat_AsDouble(o);
  if (v == -1.0 && PyErr_Occurred()) return -1;
  *out = (float)v;
  return 0;
}

static int want(Py_ssize_t nargs, Py_ssize_t n, const char* name) {
  if (nargs == n) return 0;
  PyErr_Format(PyExc_TypeError, "%s takes %zd arguments (%zd given)", name, n, nargs);
  return -1;
}

/* fr2_wkv7_prepare_metadata(qsl, slots, n, total_tokens, pool_size,
 * max_seqlen, live_tokens, live_seqs, status, seen, qsl_snap, slots_snap,
 * stream) */
static PyObject* prepare_metadata(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  void *qsl, *slots, *lt, *ls, *status, *seen, *qs, *ss, *stream;
  int32_t ns, total, pool, maxlen;
  if (want(n, 13, "prepare_metadata") || arg_ptr(a[0], &qsl) || arg_ptr(a[1], &slots) ||
      arg_i32(a[2], &ns) || arg_i32(a[3], &total) || arg_i32(a[4], &pool) ||
      arg_i32(a[5], &maxlen) || arg_ptr(a[6], &lt) || arg_ptr(a[7], &ls) ||
      arg_ptr(a[8], &status) || arg_ptr(a[9], &seen) || arg_ptr(a[10], &qs) ||
      arg_ptr(a[11], &ss) || arg_ptr(a[12], &stream))
    return NULL;
  return PyLong_FromLong(fr2_wkv7_prepare_metadata(qsl, slots, ns, total, pool, maxlen, lt, ls,
                                                   status, seen, qs, ss, stream));
}

/* The 19 arguments shared by the fp32-state entries, starting at a[0]:
 * qsl, slots, status, n, H, D, total_tokens, max_seqlen, dtype, state, r,
 * decay_logits, decay_bias, k, v, a, b, output, scale. */
struct Common {
  void *qsl, *slots, *status, *state, *r, *l, *bias, *k, *v, *a, *b, *out;
  int32_t n, h, d, maxlen, dtype;
  int64_t total;
  float scale;
};

static int arg_common(PyObject* const* a, struct Common* c) {
  return arg_ptr(a[0], &c->qsl) || arg_ptr(a[1], &c->slots) || arg_ptr(a[2], &c->status) ||
         arg_i32(a[3], &c->n) || arg_i32(a[4], &c->h) || arg_i32(a[5], &c->d) ||
         arg_i64(a[6], &c->total) || arg_i32(a[7], &c->maxlen) || arg_i32(a[8], &c->dtype) ||
         arg_ptr(a[9], &c->state) || arg_ptr(a[10], &c->r) || arg_ptr(a[11], &c->l) ||
         arg_ptr(a[12], &c->bias) || arg_ptr(a[13], &c->k) || arg_ptr(a[14], &c->v) ||
         arg_ptr(a[15], &c->a) || arg_ptr(a[16], &c->b) || arg_ptr(a[17], &c->out) ||
         arg_f32(a[18], &c->scale);
}

/* fr2_wkv7_recurrent_fp32_forward(<19 common>, stream) */
static PyObject* recurrent_fp32_forward(PyObject* self, PyObject* const* a, Py_ssize_t n) {
  (void)self;
  struct Common c;
  void* stream;
  if (want(n, 20, "recurrent_fp32_forward") || arg_common(a, &c) || arg_ptr(a[19], &stream))
    return NULL;
  return PyLong_FromLong(fr2_wkv7_recurrent_fp32_forward(
      c.qsl, c.slots, c.status, c.n, c.h, c.d, c.total, c.maxlen, c.dtype, c.state, c.r, c.l,
      c.bias, c.k, c.v, c.a, c.b, c.out, c.scale, stream));
}

/* fr2_wkv7_recurrent_fp32_forward_kernel(kernel, <19 common>, stream) */
static PyObject* recurrent_fp32_forward_kernel(PyObject* self, PyObject* const* a,
                                               Py_ssize_t n) {
  (void)self;
  struct Common c;
  int32_t kernel;
  void* stream;
  if (want(n, 21, "recurrent_fp32_forward_kernel") || arg_i32(a[0], &kernel) ||
      arg_common(a + 1, &c) || arg_ptr(a[20], &stream))
    return NULL;
  return PyLong_FromLong(fr2_wkv7_recurrent_fp32_forward_kernel(
      kernel, c.qsl, c.slots, c.status, c.n, c.h, c.d, c.total, c.maxlen, c.dtype, c.state, c.r,
      c.l, c.bias, c.k, c.v, c.a, c.b, c.out, c.scale, stream));
}

static PyMethodDef methods[] = {
    {"prepare_metadata", (PyCFunction)(void (*)(void))prepare_metadata, METH_FASTCALL,
     "fr2_wkv7_prepare_metadata"},
    {"recurrent_fp32_forward", (PyCFunction)(void (*)(void))recurrent_fp32_forward,
     METH_FASTCALL, "fr2_wkv7_recurrent_fp32_forward"},
    {"recurrent_fp32_forward_kernel", (PyCFunction)(void (*)(void))recurrent_fp32_forward_kernel,
     METH_FASTCALL, "fr2_wkv7_recurrent_fp32_forward_kernel"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_fastcall",
                                    "fast-call bindings of the per-step C-ABI entries", -1,
                                    methods, NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__fastcall(void) { return PyModule_Create(&module); }
