/* A CPython binding of the decode GEMV entry points of libiqk_hip.so: the
 * launch path an eager decode call takes (a 1-token dispatch's kernel runs
 * for ~6 us, and a ctypes call with twelve converted arguments costs ~4 us of
 * host time).  Each function takes the C ABI's arguments as Python integers
 * (device pointers as addresses, the stream as its handle) and returns the
 * entry point's code; nothing else is done here.  It is built against the
 * library's own header and carries the digest of the sources it was built
 * with, which the loader compares with the library's. */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

#include <limits.h>
#include <stdint.h>

#include "iqk_hip.h"

#ifndef IQK_SOURCE_HASH
#define IQK_SOURCE_HASH "unset"
#endif

static int as_i64(PyObject *o, long long *v) {
    *v = PyLong_AsLongLong(o);
    return !(*v == -1 && PyErr_Occurred());
}

/* gemv(kind, member, n, out, num_experts, x, streams, n_streams, sel,
 *      pairs_per_row, mats, y, stream): kind 0 iqk_gemv, 1 iqk_gemv_floor,
 * 2 iqk_gemv_floor_grid; streams is the address of the stream pointer array. */
static PyObject *gemv(PyObject *self, PyObject *const *args, Py_ssize_t nargs) {
    (void)self;
    if (nargs != 13) {
        PyErr_SetString(PyExc_TypeError, "gemv takes 13 integer arguments");
        return NULL;
    }
    long long v[13];
    for (int i = 0; i < 13; ++i)
        if (!as_i64(args[i], &v[i])) return NULL;
    /* the narrow arguments: member and stream count (int), pairs per row and
     * pair count (uint32); a value out of range is refused, not truncated */
    if (v[1] < INT_MIN || v[1] > INT_MAX || v[7] < INT_MIN || v[7] > INT_MAX || v[9] < 0 || v[9] > UINT32_MAX ||
        v[10] < 0 || v[10] > UINT32_MAX) {
        PyErr_SetString(PyExc_OverflowError, "gemv: member, stream count, pairs per row or pair count out of range");
        return NULL;
    }
    int (*fn)(int, int64_t, int64_t, int64_t, const void *, const void *const *, int, const uint32_t *, uint32_t,
              uint32_t, void *, void *) = v[0] == 1 ? iqk_gemv_floor : v[0] == 2 ? iqk_gemv_floor_grid : iqk_gemv;
    const int rc = fn((int)v[1], (int64_t)v[2], (int64_t)v[3], (int64_t)v[4], (const void *)(uintptr_t)v[5],
                      (const void *const *)(uintptr_t)v[6], (int)v[7], (const uint32_t *)(uintptr_t)v[8],
                      (uint32_t)v[9], (uint32_t)v[10], (void *)(uintptr_t)v[11], (void *)(uintptr_t)v[12]);
    return PyLong_FromLong(rc);
}

static PyObject *source_hash(PyObject *self, PyObject *unused) {
    (void)self;
    (void)unused;
    return PyUnicode_FromString(IQK_SOURCE_HASH);
}

static PyMethodDef methods[] = {
    {"gemv", (PyCFunction)(void (*)(void))gemv, METH_FASTCALL, "iqk_gemv / _floor / _floor_grid"},
    {"source_hash", source_hash, METH_NOARGS, "digest of the kernel sources this binding was built with"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_iqk_launch", NULL, -1, methods,
                                    NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__iqk_launch(void) { return PyModule_Create(&module); }
