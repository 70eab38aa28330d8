/* CPython entry point for the per-call hot path of a prepared decode call
 * (_pk.PreparedStrips): the six integers of pk_w4a16_strips_run go straight from Python
 * objects to the C ABI, without ctypes' per-argument conversion. Built by build.py against
 * the product library (linked by path, so the process shares the one copy that _pk loaded);
 * _pk falls back to ctypes when the module is missing or the library was loaded from
 * elsewhere. Same call, same kernel, same bits. */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>

#include "pico_kernels_amd.h"

/* strips_run(handle, a, c, ldc, M, stream) -> status (PK_OK or a PK_E* code) */
static PyObject* pkcall_strips_run(PyObject* self, PyObject* const* args, Py_ssize_t nargs) {
  (void)self;
  if (nargs != 6) {
    PyErr_SetString(PyExc_TypeError, "strips_run(handle, a, c, ldc, M, stream) takes 6 integers");
    return NULL;
  }
  void* h = PyLong_AsVoidPtr(args[0]);
  const void* a = PyLong_AsVoidPtr(args[1]);
  void* c = PyLong_AsVoidPtr(args[2]);
  const long long ldc = PyLong_AsLongLong(args[3]);
  const long m = PyLong_AsLong(args[4]);
  void* stream = PyLong_AsVoidPtr(args[5]);
  if (PyErr_Occurred()) return NULL;
  if (m < INT32_MIN || m > INT32_MAX) {
    PyErr_SetString(PyExc_OverflowError, "strips_run: M out of range");
    return NULL;
  }
  return PyLong_FromLong(pk_w4a16_strips_run(h, a, c, (int64_t)ldc, (int)m, stream));
}

static PyMethodDef pkcall_methods[] = {
    {"strips_run", (PyCFunction)(void (*)(void))pkcall_strips_run, METH_FASTCALL,
     "pk_w4a16_strips_run(handle, a, c, ldc, M, stream) -> status"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef pkcall_module = {PyModuleDef_HEAD_INIT, "_pkcall", NULL, -1,
                                           pkcall_methods, NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__pkcall(void) { return PyModule_Create(&pkcall_module); }
