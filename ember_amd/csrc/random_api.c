/*
 * random_api.c -- CPython module ember_amd._core._em_random.
 *
 * Same names, arguments and draws as the reference's ember._core._em_random
 * (src/random/random_api.c:56-100, src/random/distributions_cpu.c:3-16):
 * values are drawn on the host, low + (r / RAND_MAX) * (high - low) with r
 * from the C library's rand() sequence for the given _seed(), and copied to
 * the device once.  Unlike the reference (random_api.c:39-44, which lets
 * _Tensor(size) allocate and then allocates again, leaking the first
 * buffer), the tensor is allocated exactly once.
 *
 * The sequence is produced by a private generator instead of calling rand():
 * rand() keeps one process-wide state, and the GPU runtime draws from it too
 * (some device allocations advance it), so the same _seed() gave different
 * weights depending on which allocations happened between the draws.  The
 * private generator is glibc's rand() algorithm (the additive feedback
 * generator r[i] = r[i-3] + r[i-31] over 31 words, seeded by the
 * Park-Miller multiplier 16807 mod 2^31-1, the first 310 outputs discarded,
 * each output r >> 1; seed 0 acts as 1), so a seed yields exactly the
 * values glibc's srand()/rand() yield in a process where nothing else calls
 * rand() -- checked against the C library in the CPU tests.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>
#include <stdlib.h>

#include "ember_amd.h"

/* ---- the rand() sequence (see the file comment) ---- */

#define EM_RNG_WORDS 31
#define EM_RNG_SEP 3
#define EM_RAND_MAX 2147483647

static int32_t g_rng[EM_RNG_WORDS];
static int g_front = EM_RNG_SEP, g_rear = 0;

static int32_t rng_next(void)
{
    const uint32_t v = (uint32_t)g_rng[g_front] + (uint32_t)g_rng[g_rear];
    g_rng[g_front] = (int32_t)v;
    if (++g_front == EM_RNG_WORDS) g_front = 0;
    if (++g_rear == EM_RNG_WORDS) g_rear = 0;
    return (int32_t)(v >> 1);
}

static void rng_seed(unsigned seed)
{
    /* The seed enters as a signed 32-bit word (seeds >= 2^31 are negative). */
    int32_t word = seed ? (int32_t)seed : 1;
    g_rng[0] = word;
    for (int i = 1; i < EM_RNG_WORDS; i++) {
        /* word = 16807 * word mod (2^31 - 1), without overflow (Schrage) */
        const int64_t hi = word / 127773, lo = word % 127773;
        int64_t next = 16807 * lo - 2836 * hi;
        if (next < 0) next += EM_RAND_MAX;
        word = (int32_t)next;
        g_rng[i] = word;
    }
    g_front = EM_RNG_SEP;
    g_rear = 0;
    for (int i = 0; i < 10 * EM_RNG_WORDS; i++) (void)rng_next();
}

static int g_rng_seeded = 0;

/* The generator starts as if seeded with 1, like rand() without srand(). */
static int32_t rng_rand(void)
{
    if (!g_rng_seeded) {
        rng_seed(1);
        g_rng_seeded = 1;
    }
    return rng_next();
}

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
    for (Py_ssize_t i = 0; i < n; i++)
        host[i] = low + ((float)rng_rand() / (float)EM_RAND_MAX) * range;
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
    rng_seed((unsigned)seed);
    g_rng_seeded = 1;
    Py_RETURN_NONE;
}

/* _host_rand(n) -> list of the next n raw values of the sequence (host only;
 * lets tests compare the generator with the C library's rand()). */
static PyObject *py_host_rand(PyObject *self, PyObject *args)
{
    Py_ssize_t n;
    (void)self;
    if (!PyArg_ParseTuple(args, "n", &n)) return NULL;
    if (n < 0) {
        PyErr_SetString(PyExc_ValueError, "n must be non-negative");
        return NULL;
    }
    PyObject *out = PyList_New(n);
    if (!out) return NULL;
    for (Py_ssize_t i = 0; i < n; i++) {
        PyObject *v = PyLong_FromLong(rng_rand());
        if (!v) {
            Py_DECREF(out);
            return NULL;
        }
        PyList_SET_ITEM(out, i, v);
    }
    return out;
}

static PyMethodDef module_methods[] = {
    {"_uniform", (PyCFunction)py_uniform, METH_VARARGS, "Sample U(low, high) of a shape"},
    {"_constant", (PyCFunction)py_constant, METH_VARARGS, "Constant tensor of a shape"},
    {"_seed", (PyCFunction)py_seed, METH_VARARGS, "Seed the host generator (srand)"},
    {"_host_rand", (PyCFunction)py_host_rand, METH_VARARGS, "Next n raw values of the sequence"},
    {NULL, NULL, 0, NULL}};

static PyModuleDef random_module = {
    PyModuleDef_HEAD_INIT, .m_name = "ember_amd._core._em_random",
    .m_doc = "Random tensors (host draws, one upload)", .m_size = -1, .m_methods = module_methods,
};

PyMODINIT_FUNC PyInit__em_random(void)
{
    return PyModule_Create(&random_module);
}
