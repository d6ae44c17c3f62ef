/*
 * random_api.c -- CPython module ember_amd._core._em_random.
 *
 * Same names, arguments and draws as the reference's ember._core._em_random
 * (src/random/random_api.c:56-100, src/random/distributions_cpu.c:3-16):
 * values are drawn on the host with the C library's rand() (so a given
 * _seed() reproduces the reference's stream on the same libc) and copied to
 * the device once.  Unlike the reference (random_api.c:39-44, which lets
 * _Tensor(size) allocate and then allocates again, leaking the first
 * buffer), the tensor is allocated exactly once.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdlib.h>

#include "ember_amd.h"

/* _Tensor(size) from ember_amd._core._tensor, plus its device pointer. */
static PyObject *new_tensor(PyObject *shape, Py_ssize_t *size_out, float **dptr)
{
    Py_ssize_t size = 1;
    const Py_ssize_t nd = PyTuple_GET_SIZE(shape);
    for (Py_ssize_t i = 0; i < nd; i++) {
        const Py_ssize_t d = PyLong_AsSsize_t(PyTuple_GET_ITEM(shape, i));
        if (d == -1 && PyErr_Occurred()) return NULL;
        if (d < 0) {
            PyErr_SetString(PyExc_ValueError, "Dimensions cannot be negative");
            return NULL;
        }
        size *= d;
    }
    PyObject *mod = PyImport_ImportModule("ember_amd._core._tensor");
    if (!mod) return NULL;
    PyObject *type = PyObject_GetAttrString(mod, "_Tensor");
    Py_DECREF(mod);
    if (!type) return NULL;
    PyObject *t = PyObject_CallFunction(type, "n", size);
    Py_DECREF(type);
    if (!t) return NULL;
    PyObject *ptr = PyObject_GetAttrString(t, "data_ptr");
    if (!ptr) {
        Py_DECREF(t);
        return NULL;
    }
    *dptr = (float *)PyLong_AsVoidPtr(ptr);
    Py_DECREF(ptr);
    *size_out = size;
    return t;
}

/* Copies `n` host floats into the tensor `t`; drops `t` on failure. */
static PyObject *upload(PyObject *t, float *dptr, float *host, Py_ssize_t n)
{
    copy_to_device(dptr, host, (size_t)n * sizeof(float));
    PyMem_Free(host);
    const int st = ember_get_last_error();
    if (st) {
        Py_DECREF(t);
        PyErr_Format(PyExc_RuntimeError, "copy_to_device: %s", ember_error_string(st));
        return NULL;
    }
    return t;
}

static PyObject *py_uniform(PyObject *self, PyObject *args)
{
    float low, high;
    PyObject *shape;
    (void)self;
    if (!PyArg_ParseTuple(args, "ffO!", &low, &high, &PyTuple_Type, &shape)) return NULL;
    Py_ssize_t n;
    float *dptr;
    PyObject *t = new_tensor(shape, &n, &dptr);
    if (!t) return NULL;
    float *host = (float *)PyMem_Malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    if (!host) {
        Py_DECREF(t);
        return PyErr_NoMemory();
    }
    const float range = high - low;
    for (Py_ssize_t i = 0; i < n; i++) host[i] = low + ((float)rand() / (float)RAND_MAX) * range;
    return upload(t, dptr, host, n);
}

static PyObject *py_constant(PyObject *self, PyObject *args)
{
    float value;
    PyObject *shape;
    (void)self;
    if (!PyArg_ParseTuple(args, "fO!", &value, &PyTuple_Type, &shape)) return NULL;
    Py_ssize_t n;
    float *dptr;
    PyObject *t = new_tensor(shape, &n, &dptr);
    if (!t) return NULL;
    float *host = (float *)PyMem_Malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    if (!host) {
        Py_DECREF(t);
        return PyErr_NoMemory();
    }
    for (Py_ssize_t i = 0; i < n; i++) host[i] = value;
    return upload(t, dptr, host, n);
}

static PyObject *py_seed(PyObject *self, PyObject *args)
{
    int seed;
    (void)self;
    if (!PyArg_ParseTuple(args, "i", &seed)) return NULL;
    srand((unsigned)seed);
    Py_RETURN_NONE;
}

static PyMethodDef module_methods[] = {
    {"_uniform", (PyCFunction)py_uniform, METH_VARARGS, "Sample U(low, high) of a shape"},
    {"_constant", (PyCFunction)py_constant, METH_VARARGS, "Constant tensor of a shape"},
    {"_seed", (PyCFunction)py_seed, METH_VARARGS, "Seed the host generator (srand)"},
    {NULL, NULL, 0, NULL}};

static PyModuleDef random_module = {
    PyModuleDef_HEAD_INIT, .m_name = "ember_amd._core._em_random",
    .m_doc = "Random tensors (host draws, one upload)", .m_size = -1, .m_methods = module_methods,
};

PyMODINIT_FUNC PyInit__em_random(void)
{
    return PyModule_Create(&random_module);
}
