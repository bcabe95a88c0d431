/* CPython launch shims for the hot entry points of libmlpmk.so.
 *
 * ctypes converts each argument through its argtypes and builds a C array per
 * pointer list: ~2 us of host time per launch, a third of an eager small-batch
 * forward.  These functions take the same arguments as plain Python ints and
 * tuples (pointers as ints, None for NULL) and call the library through
 * function pointers handed over by `bind` -- the addresses of the library that
 * the ctypes binding loaded, so a build selected with MLPMK_LIBRARY is the one
 * called.  They return the library's status code; argument conversion errors
 * raise.  The library call itself runs with the GIL released, as ctypes does
 * it: a launch can block inside HIP (a full launch queue, the first load of a
 * code object, the device queries of a device's first call), and other Python
 * threads (data loaders) keep running meanwhile.  Built by the package
 * Makefile with gcc against the Python headers; the package uses ctypes when
 * this module is absent.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>

#include "../../include/mlpmk.h"

typedef __typeof__(mlpmk_fwd) fwd_t;
typedef __typeof__(mlpmk_bwd) bwd_t;
typedef __typeof__(mlpmk_bwd_ws) bwd_ws_t;
typedef __typeof__(mlpmk_wn_fwd) wn_fwd_t;
typedef __typeof__(mlpmk_wn_bwd) wn_bwd_t;

static fwd_t* g_fwd;
static bwd_t* g_bwd;
static bwd_ws_t* g_bwd_ws;
static wn_fwd_t* g_wn_fwd;
static wn_bwd_t* g_wn_bwd;

enum { kMaxDims = 16 };

static void* as_ptr(PyObject* o) {
  if (o == Py_None) return NULL;
  return PyLong_AsVoidPtr(o);
}

/* dims tuple -> C ints; returns the layer count or -1 with an exception set. */
static int as_dims(PyObject* o, int* dims) {
  if (!PyTuple_Check(o)) {
    PyErr_SetString(PyExc_TypeError, "dims must be a tuple of ints");
    return -1;
  }
  const Py_ssize_t n = PyTuple_GET_SIZE(o);
  if (n < 2 || n > kMaxDims) {
    PyErr_SetString(PyExc_ValueError, "dims must hold 2 .. 16 widths");
    return -1;
  }
  for (Py_ssize_t i = 0; i < n; ++i) {
    dims[i] = (int)PyLong_AsLong(PyTuple_GET_ITEM(o, i));
    if (dims[i] == -1 && PyErr_Occurred()) return -1;
  }
  return (int)n - 1;
}

/* Tuple or list of pointer ints (None for NULL) of exactly n entries. */
static int as_ptrs(PyObject* o, void** out, int n, const char* what) {
  PyObject* seq = PySequence_Fast(o, what);
  if (!seq) return -1;
  if (PySequence_Fast_GET_SIZE(seq) != n) {
    Py_DECREF(seq);
    PyErr_Format(PyExc_ValueError, "%s needs %d entries", what, n);
    return -1;
  }
  PyObject** items = PySequence_Fast_ITEMS(seq);
  for (int i = 0; i < n; ++i) {
    out[i] = as_ptr(items[i]);
    if (!out[i] && items[i] != Py_None && PyErr_Occurred()) {
      Py_DECREF(seq);
      return -1;
    }
  }
  Py_DECREF(seq);
  return 0;
}

static int check_nargs(Py_ssize_t nargs, Py_ssize_t want, const char* fn) {
  if (nargs == want) return 0;
  PyErr_Format(PyExc_TypeError, "%s takes %zd arguments (%zd given)", fn, want, nargs);
  return -1;
}

static int check_bound(void* fn) {
  if (fn) return 0;
  PyErr_SetString(PyExc_RuntimeError, "call bind() with the library's entry points first");
  return -1;
}

#define ERR_OUT() \
  if (PyErr_Occurred()) return NULL

/* bind(fwd, bwd, bwd_ws, wn_fwd, wn_bwd): entry-point addresses. */
static PyObject* py_bind(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (check_nargs(nargs, 5, "bind")) return NULL;
  void* a[5];
  for (int i = 0; i < 5; ++i) {
    a[i] = PyLong_AsVoidPtr(args[i]);
    ERR_OUT();
    if (!a[i]) {
      PyErr_SetString(PyExc_ValueError, "bind: NULL entry point");
      return NULL;
    }
  }
  g_fwd = (fwd_t*)a[0];
  g_bwd = (bwd_t*)a[1];
  g_bwd_ws = (bwd_ws_t*)a[2];
  g_wn_fwd = (wn_fwd_t*)a[3];
  g_wn_bwd = (wn_bwd_t*)a[4];
  Py_RETURN_NONE;
}

/* fwd(dims, dtype, x, w, out, stash_or_None, M, stream) -> status */
static PyObject* py_fwd(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (check_nargs(nargs, 8, "fwd") || check_bound((void*)g_fwd)) return NULL;
  int dims[kMaxDims];
  const int L = as_dims(args[0], dims);
  if (L < 0) return NULL;
  const int dtype = (int)PyLong_AsLong(args[1]);
  const void* x = as_ptr(args[2]);
  ERR_OUT();
  void* w[kMaxDims];
  if (as_ptrs(args[3], w, L, "w")) return NULL;
  void* out = as_ptr(args[4]);
  ERR_OUT();
  void* stash[kMaxDims];
  const int has_stash = args[5] != Py_None;
  if (has_stash && as_ptrs(args[5], stash, L - 1, "stash")) return NULL;
  const int64_t M = PyLong_AsLongLong(args[6]);
  void* stream = as_ptr(args[7]);
  ERR_OUT();
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = g_fwd(L, dims, dtype, x, (const void* const*)w, out, has_stash ? (float* const*)stash : NULL, M, stream);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(rc);
}

/* bwd(dims, dtype, x, w, stash, dout, dout_row_stride, dx_or_None, dw,
 *     workspace_or_None, workspace_bytes, M, stream) -> status
 * (mlpmk_bwd_ws with a workspace, mlpmk_bwd without) */
static PyObject* py_bwd(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (check_nargs(nargs, 13, "bwd") || check_bound((void*)g_bwd) || check_bound((void*)g_bwd_ws)) return NULL;
  int dims[kMaxDims];
  const int L = as_dims(args[0], dims);
  if (L < 0) return NULL;
  const int dtype = (int)PyLong_AsLong(args[1]);
  const void* x = as_ptr(args[2]);
  ERR_OUT();
  void* w[kMaxDims];
  void* stash[kMaxDims];
  void* dw[kMaxDims];
  if (as_ptrs(args[3], w, L, "w")) return NULL;
  if (as_ptrs(args[4], stash, L - 1, "stash")) return NULL;
  const void* dout = as_ptr(args[5]);
  const int64_t stride = PyLong_AsLongLong(args[6]);
  void* dx = as_ptr(args[7]);
  ERR_OUT();
  if (as_ptrs(args[8], dw, L, "dw")) return NULL;
  void* ws = as_ptr(args[9]);
  const int64_t ws_bytes = PyLong_AsLongLong(args[10]);
  const int64_t M = PyLong_AsLongLong(args[11]);
  void* stream = as_ptr(args[12]);
  ERR_OUT();
  int rc;
  Py_BEGIN_ALLOW_THREADS
  if (ws)
    rc = g_bwd_ws(L, dims, dtype, x, (const void* const*)w, (const float* const*)stash, dout, stride, dx,
                  (float* const*)dw, ws, ws_bytes, M, stream);
  else
    rc = g_bwd(L, dims, dtype, x, (const void* const*)w, (const float* const*)stash, dout, stride, dx,
               (float* const*)dw, M, stream);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(rc);
}

/* wn_fwd(dims, param_dtype, w_dtype, v, g, w, inv_norm, stream) -> status */
static PyObject* py_wn_fwd(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (check_nargs(nargs, 8, "wn_fwd") || check_bound((void*)g_wn_fwd)) return NULL;
  int dims[kMaxDims];
  const int L = as_dims(args[0], dims);
  if (L < 0) return NULL;
  const int pd = (int)PyLong_AsLong(args[1]);
  const int wd = (int)PyLong_AsLong(args[2]);
  const void* v = as_ptr(args[3]);
  const void* g = as_ptr(args[4]);
  void* w = as_ptr(args[5]);
  float* inv = (float*)as_ptr(args[6]);
  void* stream = as_ptr(args[7]);
  ERR_OUT();
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = g_wn_fwd(L, dims, pd, wd, v, g, w, inv, stream);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(rc);
}

/* wn_bwd(dims, param_dtype, dw, v, g, inv_norm, dv, dg, stream) -> status */
static PyObject* py_wn_bwd(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (check_nargs(nargs, 9, "wn_bwd") || check_bound((void*)g_wn_bwd)) return NULL;
  int dims[kMaxDims];
  const int L = as_dims(args[0], dims);
  if (L < 0) return NULL;
  const int pd = (int)PyLong_AsLong(args[1]);
  const float* dw = (const float*)as_ptr(args[2]);
  const void* v = as_ptr(args[3]);
  const void* g = as_ptr(args[4]);
  const float* inv = (const float*)as_ptr(args[5]);
  void* dv = as_ptr(args[6]);
  void* dg = as_ptr(args[7]);
  void* stream = as_ptr(args[8]);
  ERR_OUT();
  int rc;
  Py_BEGIN_ALLOW_THREADS
  rc = g_wn_bwd(L, dims, pd, dw, v, g, inv, dv, dg, stream);
  Py_END_ALLOW_THREADS
  return PyLong_FromLong(rc);
}

static PyMethodDef kMethods[] = {
    {"bind", (PyCFunction)(void (*)(void))py_bind, METH_FASTCALL, "bind(fwd, bwd, bwd_ws, wn_fwd, wn_bwd)"},
    {"fwd", (PyCFunction)(void (*)(void))py_fwd, METH_FASTCALL, "mlpmk_fwd"},
    {"bwd", (PyCFunction)(void (*)(void))py_bwd, METH_FASTCALL, "mlpmk_bwd / mlpmk_bwd_ws"},
    {"wn_fwd", (PyCFunction)(void (*)(void))py_wn_fwd, METH_FASTCALL, "mlpmk_wn_fwd"},
    {"wn_bwd", (PyCFunction)(void (*)(void))py_wn_bwd, METH_FASTCALL, "mlpmk_wn_bwd"},
    {NULL, NULL, 0, NULL}};

static struct PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_mlpmk_launch", NULL, -1, kMethods,
                                     NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__mlpmk_launch(void) { return PyModule_Create(&kModule); }
