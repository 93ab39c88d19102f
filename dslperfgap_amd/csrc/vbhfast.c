/* CPython binding of the launching entry points of libvbhip.so (include/vbhip.h).
 *
 * The same C ABI as the ctypes binding in _lib.py, called through
 * METH_FASTCALL functions that convert their arguments directly: about 0.1 us
 * per call where ctypes' argument conversion takes about 0.7 us, which is a
 * visible share of a small kernel's 2-3 us host path.  Each function takes
 * the entry point's arguments in the header's order (device pointers as
 * Python ints or None, sizes as ints, scalars as floats, the stream handle
 * last) and returns its status code; the GIL is released around the call, as
 * ctypes does.  No torch types are involved.
 *
 * The module does not link the library.  bind() receives the entry points'
 * addresses from the library instance the caller loaded (ctypes), so every
 * call -- launches, vbh_tune_override, vbh_last_error -- reaches that one
 * instance, whichever file it was loaded from.  Calls before bind() raise.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <limits.h>
#include <stdint.h>

#include "vbhip.h"

typedef union {
  void* p;
  long long q;
  double f;
} arg_t;

/* Parse `n` arguments by `fmt`: 'p' pointer (int or None), 'q' 64-bit
 * integer, 'i' integer in the range of a C int (anything else raises
 * OverflowError rather than wrapping), 'f' float.  Returns 0, or -1 with a
 * Python exception set. */
static int parse(PyObject* const* args, Py_ssize_t n, const char* fmt, arg_t* out) {
  Py_ssize_t want = (Py_ssize_t)strlen(fmt);
  if (n != want) {
    PyErr_Format(PyExc_TypeError, "expected %zd arguments, got %zd", want, n);
    return -1;
  }
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* o = args[i];
    switch (fmt[i]) {
      case 'p':
        if (o == Py_None) {
          out[i].p = NULL;
        } else {
          out[i].p = PyLong_AsVoidPtr(o);
          if (out[i].p == NULL && PyErr_Occurred()) return -1;
        }
        break;
      case 'q':
      case 'i':
        out[i].q = PyLong_AsLongLong(o);
        if (out[i].q == -1 && PyErr_Occurred()) return -1;
        if (fmt[i] == 'i' && (out[i].q < INT_MIN || out[i].q > INT_MAX)) {
          PyErr_Format(PyExc_OverflowError, "argument %zd: %lld does not fit a C int", i,
                       out[i].q);
          return -1;
        }
        break;
      case 'f':
        out[i].f = PyFloat_AsDouble(o);
        if (out[i].f == -1.0 && PyErr_Occurred()) return -1;
        break;
      default:
        PyErr_SetString(PyExc_SystemError, "bad argument format");
        return -1;
    }
  }
  return 0;
}

#define P(k) (a[k].p)
#define Q(k) ((int64_t)a[k].q)
#define I(k) ((int)a[k].q)
#define F(k) ((float)a[k].f)

/* Most arguments any entry point takes (parse() fills one arg_t per format
 * character, after checking that the call passed exactly that many). */
#define MAX_ARGS 24

/* `call` invokes the entry point through fn_<name>, set by bind(). */
#define ENTRY(name, fmt, call)                                                   \
  _Static_assert(sizeof(fmt) - 1 <= MAX_ARGS, #name ": too many arguments");     \
  static __typeof__(&name) fn_##name = NULL;                                     \
  static const char fmt_##name[] = fmt;                                          \
  static PyObject* py_##name(PyObject* self, PyObject* const* args, Py_ssize_t n) { \
    arg_t a[MAX_ARGS];                                                           \
    int rc;                                                                      \
    (void)self;                                                                  \
    if (fn_##name == NULL) {                                                     \
      PyErr_SetString(PyExc_RuntimeError, #name " is not bound: call bind() first"); \
      return NULL;                                                               \
    }                                                                            \
    if (parse(args, n, fmt_##name, a) < 0) return NULL;                          \
    Py_BEGIN_ALLOW_THREADS rc = call;                                            \
    Py_END_ALLOW_THREADS return PyLong_FromLong(rc);                             \
  }

ENTRY(vbh_layer_norm_fwd, "ppppqqfiip",
      fn_vbh_layer_norm_fwd(P(0), P(1), P(2), P(3), Q(4), Q(5), F(6), I(7), I(8), P(9)))
ENTRY(vbh_rms_norm_fwd, "pppqqfiip",
      fn_vbh_rms_norm_fwd(P(0), P(1), P(2), Q(3), Q(4), F(5), I(6), I(7), P(8)))
ENTRY(vbh_softmax_fwd, "ppqqiiip",
      fn_vbh_softmax_fwd(P(0), P(1), Q(2), Q(3), I(4), I(5), I(6), P(7)))
ENTRY(vbh_softmax_fwd_ws, "ppqqiiipqp",
      fn_vbh_softmax_fwd_ws(P(0), P(1), Q(2), Q(3), I(4), I(5), I(6), P(7), Q(8), P(9)))
ENTRY(vbh_softmax_dim_fwd, "ppqqqiiip",
      fn_vbh_softmax_dim_fwd(P(0), P(1), Q(2), Q(3), Q(4), I(5), I(6), I(7), P(8)))
ENTRY(vbh_logsumexp_fwd, "ppqqiip",
      fn_vbh_logsumexp_fwd(P(0), P(1), Q(2), Q(3), I(4), I(5), P(6)))
ENTRY(vbh_logsumexp_fwd_ws, "ppqqiipqp",
      fn_vbh_logsumexp_fwd_ws(P(0), P(1), Q(2), Q(3), I(4), I(5), P(6), Q(7), P(8)))
ENTRY(vbh_cross_entropy_fwd, "ppiipppqqqfffqqqqiip",
      fn_vbh_cross_entropy_fwd(P(0), P(1), I(2), I(3), P(4), P(5), P(6), Q(7), Q(8), Q(9), F(10),
                            F(11), F(12), Q(13), Q(14), Q(15), Q(16), I(17), I(18), P(19)))
ENTRY(vbh_cross_entropy_fwd_ws, "ppiipppqqqfffqqqqiipqp",
      fn_vbh_cross_entropy_fwd_ws(P(0), P(1), I(2), I(3), P(4), P(5), P(6), Q(7), Q(8), Q(9),
                                  F(10), F(11), F(12), Q(13), Q(14), Q(15), Q(16), I(17), I(18),
                                  P(19), Q(20), P(21)))
ENTRY(vbh_cross_entropy_fwd_noalloc, "ppiipppqqqfffqqqqiip",
      fn_vbh_cross_entropy_fwd_noalloc(P(0), P(1), I(2), I(3), P(4), P(5), P(6), Q(7), Q(8), Q(9),
                                       F(10), F(11), F(12), Q(13), Q(14), Q(15), Q(16), I(17),
                                       I(18), P(19)))
ENTRY(vbh_cross_entropy_bwd, "pppppiiqqqqqfffqqqip",
      fn_vbh_cross_entropy_bwd(P(0), P(1), P(2), P(3), P(4), I(5), I(6), Q(7), Q(8), Q(9), Q(10),
                            Q(11), F(12), F(13), F(14), Q(15), Q(16), Q(17), I(18), P(19)))
ENTRY(vbh_reduce_fwd, "pppqqqiiip",
      fn_vbh_reduce_fwd(P(0), P(1), P(2), Q(3), Q(4), Q(5), I(6), I(7), I(8), P(9)))
ENTRY(vbh_reduce_fwd_ws, "pppqqqiiipqp",
      fn_vbh_reduce_fwd_ws(P(0), P(1), P(2), Q(3), Q(4), Q(5), I(6), I(7), I(8), P(9), Q(10),
                           P(11)))
ENTRY(vbh_stream_copy, "ppqp", fn_vbh_stream_copy(P(0), P(1), Q(2), P(3)))
ENTRY(vbh_stream_read, "pqpqp", fn_vbh_stream_read(P(0), Q(1), P(2), Q(3), P(4)))

#define METHOD(name) {#name, (PyCFunction)(void (*)(void))py_##name, METH_FASTCALL, NULL}

/* Entry point name -> its slot, for bind() and FORMATS. */
#define SLOT(name) {#name, (void**)&fn_##name, fmt_##name}
static const struct {
  const char* name;
  void** fn;
  const char* fmt;
} slots[] = {
    SLOT(vbh_layer_norm_fwd),    SLOT(vbh_rms_norm_fwd),     SLOT(vbh_softmax_fwd),
    SLOT(vbh_softmax_dim_fwd),   SLOT(vbh_logsumexp_fwd),    SLOT(vbh_logsumexp_fwd_ws), SLOT(vbh_softmax_fwd_ws),
    SLOT(vbh_cross_entropy_fwd), SLOT(vbh_cross_entropy_fwd_ws), SLOT(vbh_cross_entropy_bwd),
    SLOT(vbh_cross_entropy_fwd_noalloc),
    SLOT(vbh_reduce_fwd),
    SLOT(vbh_reduce_fwd_ws),     SLOT(vbh_stream_copy),      SLOT(vbh_stream_read),
};
#define N_SLOTS (sizeof(slots) / sizeof(slots[0]))

/* bind({name: address}): set every entry point from the addresses of one
 * loaded library (all names must be present and nonzero). */
static PyObject* py_bind(PyObject* self, PyObject* addrs) {
  void* got[N_SLOTS];
  (void)self;
  if (!PyDict_Check(addrs)) {
    PyErr_SetString(PyExc_TypeError, "bind() takes a dict {entry point name: address}");
    return NULL;
  }
  for (size_t i = 0; i < N_SLOTS; ++i) {
    PyObject* v = PyDict_GetItemString(addrs, slots[i].name);
    if (v == NULL) {
      PyErr_Format(PyExc_KeyError, "bind(): no address for %s", slots[i].name);
      return NULL;
    }
    got[i] = PyLong_AsVoidPtr(v);
    if (got[i] == NULL) {
      if (!PyErr_Occurred())
        PyErr_Format(PyExc_ValueError, "bind(): null address for %s", slots[i].name);
      return NULL;
    }
  }
  for (size_t i = 0; i < N_SLOTS; ++i) *slots[i].fn = got[i];
  Py_RETURN_NONE;
}

static PyMethodDef methods[] = {
    {"bind", py_bind, METH_O, "bind({entry point name: address}) -- set the entry points"},
    METHOD(vbh_layer_norm_fwd),    METHOD(vbh_rms_norm_fwd),      METHOD(vbh_softmax_fwd),
    METHOD(vbh_softmax_dim_fwd),   METHOD(vbh_logsumexp_fwd),     METHOD(vbh_logsumexp_fwd_ws), METHOD(vbh_softmax_fwd_ws),
    METHOD(vbh_cross_entropy_fwd), METHOD(vbh_cross_entropy_fwd_ws),
    METHOD(vbh_cross_entropy_fwd_noalloc),
    METHOD(vbh_cross_entropy_bwd), METHOD(vbh_reduce_fwd),
    METHOD(vbh_reduce_fwd_ws),     METHOD(vbh_stream_copy),       METHOD(vbh_stream_read),
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {
    PyModuleDef_HEAD_INIT, "_vbhfast",
    "CPython binding of the launching entry points of libvbhip.so", -1, methods,
};

/* FORMATS: entry point name -> its argument format string, so that callers
 * can check the binding against their own declaration of the header. */
static int add_formats(PyObject* m) {
  PyObject* d = PyDict_New();
  if (d == NULL) return -1;
  for (size_t i = 0; i < N_SLOTS; ++i) {
    PyObject* v = PyUnicode_FromString(slots[i].fmt);
    if (v == NULL || PyDict_SetItemString(d, slots[i].name, v) < 0) {
      Py_XDECREF(v);
      Py_DECREF(d);
      return -1;
    }
    Py_DECREF(v);
  }
  if (PyModule_AddObject(m, "FORMATS", d) < 0) {
    Py_DECREF(d);
    return -1;
  }
  return 0;
}

PyMODINIT_FUNC PyInit__vbhfast(void) {
  PyObject* m = PyModule_Create(&module);
  if (m == NULL) return NULL;
  /* the header version this binding was compiled against */
  if (PyModule_AddIntConstant(m, "ABI_VERSION", VBH_ABI_VERSION) < 0 || add_formats(m) < 0) {
    Py_DECREF(m);
    return NULL;
  }
  return m;
}
