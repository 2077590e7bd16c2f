/*
 * CPython entry points for the per-call hot functions of libnia_attn.so.
 *
 * The same C ABI as the ctypes binding (nano-inference_amd/_lib.py), called through
 * function pointers taken from the library that ctypes loaded (bind()), so there is one
 * instance of the library and its device state.  Only the argument conversion differs:
 * ctypes spends ~2.5 us converting the 23 arguments of a decode call, a METH_FASTCALL
 * function well under one.  Each function takes the arguments of its C declaration in
 * include/nia_attn.h, in order, as Python ints (pointers: int or None) and floats, and
 * returns the int status; `kinds` maps each name to its argument kinds (p pointer,
 * l int64, i int32, f float, z size_t), which the tests check against the ctypes table.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>
#include <string.h>

#include "../../include/nia_attn.h"

typedef union {
  void* p;
  int64_t l;
  int32_t i;
  float f;
  size_t z;
} Arg;

static int convert(PyObject* const* args, Py_ssize_t n, const char* kinds, Arg* a) {
  const Py_ssize_t k = (Py_ssize_t)strlen(kinds);
  if (n != k) {
    PyErr_Format(PyExc_TypeError, "expected %zd arguments, got %zd", k, n);
    return -1;
  }
  for (Py_ssize_t j = 0; j < k; ++j) {
    PyObject* o = args[j];
    switch (kinds[j]) {
      case 'p':
        if (o == Py_None) {
          a[j].p = NULL;
        } else {
          a[j].p = PyLong_AsVoidPtr(o);
          if (a[j].p == NULL && PyErr_Occurred()) return -1;
        }
        break;
      case 'l': {
        const long long v = PyLong_AsLongLong(o);
        if (v == -1 && PyErr_Occurred()) return -1;
        a[j].l = (int64_t)v;
        break;
      }
      case 'i': {
        const long long v = PyLong_AsLongLong(o);
        if (v == -1 && PyErr_Occurred()) return -1;
        if (v < INT32_MIN || v > INT32_MAX) {
          PyErr_Format(PyExc_OverflowError, "argument %zd does not fit an int32", j);
          return -1;
        }
        a[j].i = (int32_t)v;
        break;
      }
      case 'f': {
        const double v = PyFloat_AsDouble(o);
        if (v == -1.0 && PyErr_Occurred()) return -1;
        a[j].f = (float)v;
        break;
      }
      case 'z': {
        const size_t v = PyLong_AsSize_t(o);
        if (v == (size_t)-1 && PyErr_Occurred()) return -1;
        a[j].z = v;
        break;
      }
      default:
        PyErr_SetString(PyExc_SystemError, "bad argument kind");
        return -1;
    }
  }
  return 0;
}

static PyObject* unbound(const char* name) {
  PyErr_Format(PyExc_RuntimeError, "%s: not bound to the library (call bind first)", name);
  return NULL;
}

/* One wrapper per function: its pointer (typed by the header's declaration), its kinds and
 * the call with each converted argument in declaration order. */
#define NIA_FAST(name, kinds, ...)                                                         \
  static __typeof__(&name) f_##name;                                                       \
  static const char k_##name[] = kinds;                                                    \
  static PyObject* w_##name(PyObject* self, PyObject* const* args, Py_ssize_t n) {         \
    (void)self;                                                                            \
    Arg a[sizeof(k_##name) - 1];                                                           \
    if (!f_##name) return unbound(#name);                                                  \
    if (convert(args, n, k_##name, a) < 0) return NULL;                                    \
    int32_t st;                                                                            \
    Py_BEGIN_ALLOW_THREADS st = f_##name(__VA_ARGS__);                                     \
    Py_END_ALLOW_THREADS return PyLong_FromLong(st);                                       \
  }

NIA_FAST(nia_kv_write, "pllpllpppiiiilip",
         a[0].p, a[1].l, a[2].l, a[3].p, a[4].l, a[5].l, a[6].p, a[7].p, a[8].p, a[9].i,
         a[10].i, a[11].i, a[12].i, a[13].l, a[14].i, a[15].p)
NIA_FAST(nia_kv_write_fp8, "pllpllpppppiiiilip",
         a[0].p, a[1].l, a[2].l, a[3].p, a[4].l, a[5].l, a[6].p, a[7].p, a[8].p, a[9].p,
         a[10].p, a[11].i, a[12].i, a[13].i, a[14].i, a[15].l, a[16].i, a[17].p)
NIA_FAST(nia_paged_decode, "pllpllpppiipiiiiilfpzip",
         a[0].p, a[1].l, a[2].l, a[3].p, a[4].l, a[5].l, a[6].p, a[7].p, a[8].p, a[9].i,
         a[10].i, a[11].p, a[12].i, a[13].i, a[14].i, a[15].i, a[16].i, a[17].l, a[18].f,
         a[19].p, a[20].z, a[21].i, a[22].p)
NIA_FAST(nia_paged_decode_fp8, "pllpllpppppiipiiiiilfpzp",
         a[0].p, a[1].l, a[2].l, a[3].p, a[4].l, a[5].l, a[6].p, a[7].p, a[8].p, a[9].p,
         a[10].p, a[11].i, a[12].i, a[13].p, a[14].i, a[15].i, a[16].i, a[17].i, a[18].i,
         a[19].l, a[20].f, a[21].p, a[22].z, a[23].p)
NIA_FAST(nia_prefill, "pllpllpllpllppppiiiiifiip",
         a[0].p, a[1].l, a[2].l, a[3].p, a[4].l, a[5].l, a[6].p, a[7].l, a[8].l, a[9].p,
         a[10].l, a[11].l, a[12].p, a[13].p, a[14].p, a[15].p, a[16].i, a[17].i, a[18].i,
         a[19].i, a[20].i, a[21].f, a[22].i, a[23].i, a[24].p)
NIA_FAST(nia_prefill_paged, "pllpllpppiipppiiiiiilfiip",
         a[0].p, a[1].l, a[2].l, a[3].p, a[4].l, a[5].l, a[6].p, a[7].p, a[8].p, a[9].i,
         a[10].i, a[11].p, a[12].p, a[13].p, a[14].i, a[15].i, a[16].i, a[17].i, a[18].i,
         a[19].i, a[20].l, a[21].f, a[22].i, a[23].i, a[24].p)
NIA_FAST(nia_qk_norm_rope_kv_write, "pllpllpllppfplipiipppiiiiilip",
         a[0].p, a[1].l, a[2].l, a[3].p, a[4].l, a[5].l, a[6].p, a[7].l, a[8].l, a[9].p,
         a[10].p, a[11].f, a[12].p, a[13].l, a[14].i, a[15].p, a[16].i, a[17].i, a[18].p,
         a[19].p, a[20].p, a[21].i, a[22].i, a[23].i, a[24].i, a[25].i, a[26].l, a[27].i,
         a[28].p)
NIA_FAST(nia_qk_norm_rope_kv_write_fp8, "pllpllpllppfplipiipppppiiiiilip",
         a[0].p, a[1].l, a[2].l, a[3].p, a[4].l, a[5].l, a[6].p, a[7].l, a[8].l, a[9].p,
         a[10].p, a[11].f, a[12].p, a[13].l, a[14].i, a[15].p, a[16].i, a[17].i, a[18].p,
         a[19].p, a[20].p, a[21].p, a[22].p, a[23].i, a[24].i, a[25].i, a[26].i, a[27].i,
         a[28].l, a[29].i, a[30].p)

#define NIA_ENTRY(name) {#name, (PyCFunction)(void (*)(void))w_##name, METH_FASTCALL, NULL}

/* bind(name, address): point `name` at the library's function (an int address). */
static PyObject* bind(PyObject* self, PyObject* const* args, Py_ssize_t n) {
  (void)self;
  if (n != 2) {
    PyErr_SetString(PyExc_TypeError, "bind(name, address)");
    return NULL;
  }
  const char* name = PyUnicode_AsUTF8(args[0]);
  if (!name) return NULL;
  void* addr = PyLong_AsVoidPtr(args[1]);
  if (!addr) {
    if (!PyErr_Occurred()) PyErr_SetString(PyExc_ValueError, "null function address");
    return NULL;
  }
#define NIA_BIND(fn)                          \
  if (strcmp(name, #fn) == 0) {               \
    f_##fn = (__typeof__(&fn))addr;           \
    Py_RETURN_NONE;                           \
  }
  NIA_BIND(nia_kv_write)
  NIA_BIND(nia_kv_write_fp8)
  NIA_BIND(nia_paged_decode)
  NIA_BIND(nia_paged_decode_fp8)
  NIA_BIND(nia_prefill)
  NIA_BIND(nia_prefill_paged)
  NIA_BIND(nia_qk_norm_rope_kv_write)
  NIA_BIND(nia_qk_norm_rope_kv_write_fp8)
#undef NIA_BIND
  PyErr_Format(PyExc_KeyError, "no fast entry point %s", name);
  return NULL;
}

static PyMethodDef methods[] = {
    {"bind", (PyCFunction)(void (*)(void))bind, METH_FASTCALL, "bind(name, address)"},
    NIA_ENTRY(nia_kv_write),
    NIA_ENTRY(nia_kv_write_fp8),
    NIA_ENTRY(nia_paged_decode),
    NIA_ENTRY(nia_paged_decode_fp8),
    NIA_ENTRY(nia_prefill),
    NIA_ENTRY(nia_prefill_paged),
    NIA_ENTRY(nia_qk_norm_rope_kv_write),
    NIA_ENTRY(nia_qk_norm_rope_kv_write_fp8),
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT,
                                    "_nia_fast",
                                    "CPython entry points for the hot calls of libnia_attn.so",
                                    -1,
                                    methods,
                                    NULL,
                                    NULL,
                                    NULL,
                                    NULL};

PyMODINIT_FUNC PyInit__nia_fast(void) {
  PyObject* m = PyModule_Create(&module);
  if (!m) return NULL;
  PyObject* kinds = PyDict_New();
  if (!kinds) return NULL;
#define NIA_KINDS(fn)                                               \
  {                                                                 \
    PyObject* k = PyUnicode_FromString(k_##fn);                     \
    if (!k || PyDict_SetItemString(kinds, #fn, k) < 0) return NULL; \
    Py_DECREF(k);                                                   \
  }
  NIA_KINDS(nia_kv_write)
  NIA_KINDS(nia_kv_write_fp8)
  NIA_KINDS(nia_paged_decode)
  NIA_KINDS(nia_paged_decode_fp8)
  NIA_KINDS(nia_prefill)
  NIA_KINDS(nia_prefill_paged)
  NIA_KINDS(nia_qk_norm_rope_kv_write)
  NIA_KINDS(nia_qk_norm_rope_kv_write_fp8)
#undef NIA_KINDS
  if (PyModule_AddObject(m, "kinds", kinds) < 0) return NULL;
  return m;
}
