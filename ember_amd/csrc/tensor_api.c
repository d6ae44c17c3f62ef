/*
 * tensor_api.c -- CPython module ember_amd._core._tensor: the binding the
 * Python front-end calls, over libember_amd.so.
 *
 * Mirrors the reference's ember._core._tensor (src/tensor/tensor_api.c):
 * the same _Tensor type (an owning handle of one float32 device buffer),
 * the same 44 function names with the same arguments and error behaviour
 * (TypeError / ValueError from argument checks, MemoryError when device
 * allocation fails), plus the two attention entry points the reference
 * lacks.  Differences:
 *   - sizes are Py_ssize_t, not int (the reference's `int size`,
 *     src/core/tensor_types.h:8, caps a tensor at 2^31-1 elements);
 *   - a device error becomes a RuntimeError instead of exit()
 *     (src/core/utils_gpu.cuh:13-19): every native call is followed by
 *     ember_get_last_error().
 * The device is the HIP null stream; results are synchronised when copied
 * back (_to_np / _to_list / _sum), as in the reference.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <limits.h>
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <structmember.h>

#include "ember_amd.h"

typedef struct {
    PyObject_HEAD
    float *d_ptr;
    Py_ssize_t size;
} TensorObject;

static PyTypeObject TensorType;

/* ---- errors ---- */

/* Raises for a status of libember_amd (the given one, else the sticky one). */
static int raise_status(int status, const char *what)
{
    int sticky = ember_get_last_error();
    int st = status ? status : sticky;
    if (!st) return 0;
    PyObject *exc = PyExc_RuntimeError;
    if (st == EMBER_ERR_INVALID_ARGUMENT || st == EMBER_ERR_UNSUPPORTED) exc = PyExc_ValueError;
    if (st == EMBER_ERR_OUT_OF_MEMORY) exc = PyExc_MemoryError;
    PyErr_Format(exc, "%s: %s", what, ember_error_string(st));
    return -1;
}

/* ---- allocation ---- */

static TensorObject *alloc_tensor(Py_ssize_t size)
{
    if (size < 0) {
        PyErr_SetString(PyExc_ValueError, "Tensor size cannot be negative");
        return NULL;
    }
    TensorObject *t = (TensorObject *)TensorType.tp_alloc(&TensorType, 0);
    if (!t) return NULL;
    t->size = size;
    t->d_ptr = (float *)alloc_memory((size_t)(size > 0 ? size : 1) * sizeof(float));
    if (!t->d_ptr) {
        (void)ember_get_last_error();
        Py_DECREF(t);
        PyErr_SetString(PyExc_MemoryError, "Failed to allocate device memory");
        return NULL;
    }
    return t;
}

/* Drops `t` and returns NULL if the last native call failed. */
static PyObject *finish(TensorObject *t, const char *what)
{
    if (raise_status(0, what)) {
        Py_DECREF(t);
        return NULL;
    }
    return (PyObject *)t;
}

static int fits_int(Py_ssize_t n, const char *what)
{
    if (n > INT_MAX) {
        PyErr_Format(PyExc_OverflowError, "%s: %zd elements exceed the operator's int size", what, n);
        return 0;
    }
    return 1;
}

/* ---- _Tensor type ---- */

static void Tensor_dealloc(TensorObject *self)
{
    if (self->d_ptr) free_memory(self->d_ptr);
    (void)ember_get_last_error();
    Py_TYPE(self)->tp_free((PyObject *)self);
}

static int Tensor_init(TensorObject *self, PyObject *args, PyObject *kwds)
{
    Py_ssize_t size = 0;
    (void)kwds;
    if (!PyArg_ParseTuple(args, "n", &size)) return -1;
    if (size < 0) {
        PyErr_SetString(PyExc_ValueError, "Tensor size cannot be negative");
        return -1;
    }
    if (self->d_ptr) free_memory(self->d_ptr);
    self->size = size;
    self->d_ptr = (float *)alloc_memory((size_t)(size > 0 ? size : 1) * sizeof(float));
    if (!self->d_ptr) {
        (void)ember_get_last_error();
        PyErr_SetString(PyExc_MemoryError, "Failed to allocate device memory");
        return -1;
    }
    return 0;
}

static PyObject *Tensor_copy_from_list(TensorObject *self, PyObject *args)
{
    PyObject *list;
    if (!PyArg_ParseTuple(args, "O!", &PyList_Type, &list)) return NULL;
    if (PyList_GET_SIZE(list) != self->size) {
        PyErr_Format(PyExc_ValueError, "List has %zd elements, Tensor has %zd",
                     PyList_GET_SIZE(list), self->size);
        return NULL;
    }
    float *host = (float *)PyMem_Malloc((size_t)(self->size > 0 ? self->size : 1) * sizeof(float));
    if (!host) return PyErr_NoMemory();
    for (Py_ssize_t i = 0; i < self->size; i++) {
        double x = PyFloat_AsDouble(PyList_GET_ITEM(list, i));
        if (x == -1.0 && PyErr_Occurred()) {
            PyMem_Free(host);
            return NULL;
        }
        host[i] = (float)x;
    }
    copy_to_device(self->d_ptr, host, (size_t)self->size * sizeof(float));
    PyMem_Free(host);
    if (raise_status(0, "_copy_from_list")) return NULL;
    Py_RETURN_NONE;
}

static PyObject *nested(const float *data, const Py_ssize_t *dims, int ndim, int d, Py_ssize_t *pos)
{
    PyObject *list = PyList_New(dims[d]);
    if (!list) return NULL;
    for (Py_ssize_t i = 0; i < dims[d]; i++) {
        PyObject *item = d == ndim - 1 ? PyFloat_FromDouble(data[(*pos)++])
                                       : nested(data, dims, ndim, d + 1, pos);
        if (!item) {
            Py_DECREF(list);
            return NULL;
        }
        PyList_SET_ITEM(list, i, item);
    }
    return list;
}

static PyObject *Tensor_to_list(TensorObject *self, PyObject *args)
{
    PyObject *shape;
    if (!PyArg_ParseTuple(args, "O!", &PyTuple_Type, &shape)) return NULL;
    const int ndim = (int)PyTuple_GET_SIZE(shape);
    Py_ssize_t dims[64];
    if (ndim > 64) {
        PyErr_SetString(PyExc_ValueError, "Too many dimensions");
        return NULL;
    }
    Py_ssize_t total = 1;
    for (int i = 0; i < ndim; i++) {
        dims[i] = PyLong_AsSsize_t(PyTuple_GET_ITEM(shape, i));
        if (dims[i] == -1 && PyErr_Occurred()) return NULL;
        if (dims[i] < 0) {
            PyErr_SetString(PyExc_ValueError, "Dimensions cannot be negative");
            return NULL;
        }
        total *= dims[i];
    }
    if (total != self->size) {
        PyErr_Format(PyExc_ValueError,
                     "Shape mismatch: Tensor has %zd elements, but requested shape requires %zd",
                     self->size, total);
        return NULL;
    }
    float *host = (float *)PyMem_Malloc((size_t)(total > 0 ? total : 1) * sizeof(float));
    if (!host) return PyErr_NoMemory();
    sync_device();
    copy_from_device(host, self->d_ptr, (size_t)total * sizeof(float));
    if (raise_status(0, "_to_list")) {
        PyMem_Free(host);
        return NULL;
    }
    PyObject *out;
    if (ndim == 0) {
        out = PyFloat_FromDouble(host[0]);
    } else {
        Py_ssize_t pos = 0;
        out = nested(host, dims, ndim, 0, &pos);
    }
    PyMem_Free(host);
    return out;
}

/* 1-D float32 numpy array of the tensor's contents (numpy imported lazily
 * through its Python API, so the module does not link the numpy C API). */
static PyObject *Tensor_to_np(TensorObject *self, PyObject *unused)
{
    (void)unused;
    PyObject *np = PyImport_ImportModule("numpy");
    if (!np) return NULL;
    PyObject *arr = PyObject_CallMethod(np, "empty", "(n)s", self->size, "float32");
    Py_DECREF(np);
    if (!arr) return NULL;
    Py_buffer view;
    if (PyObject_GetBuffer(arr, &view, PyBUF_C_CONTIGUOUS | PyBUF_WRITABLE) < 0) {
        Py_DECREF(arr);
        return NULL;
    }
    sync_device();
    copy_from_device(view.buf, self->d_ptr, (size_t)self->size * sizeof(float));
    PyBuffer_Release(&view);
    if (raise_status(0, "_to_np")) {
        Py_DECREF(arr);
        return NULL;
    }
    return arr;
}

static PyObject *Tensor_data_ptr(TensorObject *self, void *closure)
{
    (void)closure;
    return PyLong_FromVoidPtr(self->d_ptr);
}

static PyMethodDef Tensor_methods[] = {
    {"_copy_from_list", (PyCFunction)Tensor_copy_from_list, METH_VARARGS, "Load data from a flat list"},
    {"_to_list", (PyCFunction)Tensor_to_list, METH_VARARGS, "Export data as a nested list of the given shape"},
    {"_to_np", (PyCFunction)Tensor_to_np, METH_NOARGS, "Copy to a 1-D float32 numpy array"},
    {NULL, NULL, 0, NULL}};

static PyMemberDef Tensor_members[] = {
    {"size", T_PYSSIZET, offsetof(TensorObject, size), READONLY, "Number of float32 elements"},
    {NULL, 0, 0, 0, NULL}};

static PyGetSetDef Tensor_getset[] = {
    {"data_ptr", (getter)Tensor_data_ptr, NULL, "Device address of the buffer", NULL},
    {NULL, NULL, NULL, NULL, NULL}};

static PyTypeObject TensorType = {
    PyVarObject_HEAD_INIT(NULL, 0).tp_name = "ember_amd._core._tensor._Tensor",
    .tp_basicsize = sizeof(TensorObject),
    .tp_flags = Py_TPFLAGS_DEFAULT,
    .tp_doc = "Owning handle of one float32 device buffer",
    .tp_methods = Tensor_methods,
    .tp_members = Tensor_members,
    .tp_getset = Tensor_getset,
    .tp_new = PyType_GenericNew,
    .tp_init = (initproc)Tensor_init,
    .tp_dealloc = (destructor)Tensor_dealloc,
};

/* ---- host -> device ---- */

static PyObject *py_from_numpy(PyObject *module, PyObject *args)
{
    PyObject *obj;
    (void)module;
    if (!PyArg_ParseTuple(args, "O", &obj)) return NULL;
    Py_buffer view;
    if (PyObject_GetBuffer(obj, &view, PyBUF_C_CONTIGUOUS | PyBUF_FORMAT) < 0) {
        PyErr_Clear();
        PyErr_SetString(PyExc_TypeError,
                        "Object does not support the C-contiguous buffer protocol (is it a numpy array?)");
        return NULL;
    }
    if (view.format && strcmp(view.format, "f") != 0) {
        PyErr_Format(PyExc_TypeError,
                     "Expected float32 ('f'), got '%s'. Use array.astype('float32') in Python.",
                     view.format);
        PyBuffer_Release(&view);
        return NULL;
    }
    TensorObject *t = alloc_tensor(view.len / (Py_ssize_t)sizeof(float));
    if (!t) {
        PyBuffer_Release(&view);
        return NULL;
    }
    copy_to_device(t->d_ptr, view.buf, (size_t)t->size * sizeof(float));
    PyBuffer_Release(&view);
    return finish(t, "_from_numpy");
}

/* ---- element-wise operators (table in operators.def) ---- */

typedef void (*binary_fn)(const float *, const float *, float *, int);
typedef void (*scalar_fn)(const float *, float, float *, int);
typedef void (*unary_fn)(const float *, float *, int);
typedef void (*bcast_fn)(const float *, const float *, float *, const int *, const int *,
                         const int *, int);

static PyObject *do_binary(PyObject *args, binary_fn fn, const char *what)
{
    TensorObject *a, *b;
    if (!PyArg_ParseTuple(args, "O!O!", &TensorType, &a, &TensorType, &b)) return NULL;
    if (a->size != b->size) {
        PyErr_Format(PyExc_ValueError, "Size mismatch: %zd vs %zd", a->size, b->size);
        return NULL;
    }
    if (!fits_int(a->size, what)) return NULL;
    TensorObject *r = alloc_tensor(a->size);
    if (!r) return NULL;
    fn(a->d_ptr, b->d_ptr, r->d_ptr, (int)a->size);
    return finish(r, what);
}

static PyObject *do_scalar(PyObject *args, scalar_fn fn, const char *what)
{
    TensorObject *a;
    float y;
    if (!PyArg_ParseTuple(args, "O!f", &TensorType, &a, &y)) return NULL;
    if (!fits_int(a->size, what)) return NULL;
    TensorObject *r = alloc_tensor(a->size);
    if (!r) return NULL;
    fn(a->d_ptr, y, r->d_ptr, (int)a->size);
    return finish(r, what);
}

static PyObject *do_unary(PyObject *args, unary_fn fn, const char *what)
{
    TensorObject *a;
    if (!PyArg_ParseTuple(args, "O!", &TensorType, &a)) return NULL;
    if (!fits_int(a->size, what)) return NULL;
    TensorObject *r = alloc_tensor(a->size);
    if (!r) return NULL;
    fn(a->d_ptr, r->d_ptr, (int)a->size);
    return finish(r, what);
}

/* Reads a tuple of ints (at most 16). */
static int int_tuple(PyObject *tuple, int *out, int *n)
{
    *n = (int)PyTuple_GET_SIZE(tuple);
    if (*n > 16) {
        PyErr_SetString(PyExc_ValueError, "At most 16 dimensions are supported");
        return -1;
    }
    for (int i = 0; i < *n; i++) {
        long v = PyLong_AsLong(PyTuple_GET_ITEM(tuple, i));
        if (v == -1 && PyErr_Occurred()) return -1;
        if (v < 0 || v > INT_MAX) {
            PyErr_SetString(PyExc_ValueError, "Shape and stride entries must be non-negative ints");
            return -1;
        }
        out[i] = (int)v;
    }
    return 0;
}

static PyObject *do_bcast(PyObject *args, bcast_fn fn, const char *what)
{
    TensorObject *a, *b;
    PyObject *shape_t, *sa_t, *sb_t;
    if (!PyArg_ParseTuple(args, "O!O!O!O!O!", &TensorType, &a, &TensorType, &b, &PyTuple_Type,
                          &shape_t, &PyTuple_Type, &sa_t, &PyTuple_Type, &sb_t))
        return NULL;
    int shape[16], sa[16], sb[16], n, na, nb;
    if (int_tuple(shape_t, shape, &n) || int_tuple(sa_t, sa, &na) || int_tuple(sb_t, sb, &nb))
        return NULL;
    if (n != na || n != nb) {
        PyErr_SetString(PyExc_ValueError, "Dimension mismatch in broadcast arguments");
        return NULL;
    }
    Py_ssize_t total = 1, last_a = 0, last_b = 0;
    for (int i = 0; i < n; i++) {
        total *= shape[i];
        if (shape[i] > 0) {
            last_a += (Py_ssize_t)(shape[i] - 1) * sa[i];
            last_b += (Py_ssize_t)(shape[i] - 1) * sb[i];
        }
    }
    /* Every index the strides can reach must lie inside the operands. */
    if (total > 0 && (last_a >= a->size || last_b >= b->size)) {
        PyErr_SetString(PyExc_ValueError, "Broadcast strides reach past an operand");
        return NULL;
    }
    if (!fits_int(total, what)) return NULL;
    TensorObject *r = alloc_tensor(total);
    if (!r) return NULL;
    fn(a->d_ptr, b->d_ptr, r->d_ptr, shape, sa, sb, n);
    return finish(r, what);
}

#define EMBER_BINARY_OP(name, expr)                                            \
    static PyObject *py_##name##_tensor(PyObject *m, PyObject *args)           \
    {                                                                          \
        (void)m;                                                               \
        return do_binary(args, name##_tensor, "_" #name "_tensor");            \
    }
#define EMBER_SCALAR_OP(name, expr)                                            \
    static PyObject *py_##name##_scalar(PyObject *m, PyObject *args)           \
    {                                                                          \
        (void)m;                                                               \
        return do_scalar(args, name##_scalar, "_" #name "_scalar");            \
    }
#define EMBER_BROADCAST_OP(name, expr)                                         \
    static PyObject *py_##name##_broadcasted(PyObject *m, PyObject *args)      \
    {                                                                          \
        (void)m;                                                               \
        return do_bcast(args, name##_broadcasted, "_" #name "_broadcasted");   \
    }
#define EMBER_UNARY_OP(name, expr)                                             \
    static PyObject *py_##name(PyObject *m, PyObject *args)                    \
    {                                                                          \
        (void)m;                                                               \
        return do_unary(args, name##_tensor, "_" #name);                       \
    }
#include "operators.def"

/* ---- matmul, transpose, reductions: src/tensor/tensor_api.c:305-413 ---- */

static PyObject *py_matmul(PyObject *module, PyObject *args)
{
    TensorObject *a, *b;
    int n, m, k;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!O!iii", &TensorType, &a, &TensorType, &b, &n, &m, &k)) return NULL;
    if (n < 0 || m < 0 || k < 0) {
        PyErr_SetString(PyExc_ValueError, "matmul dimensions must be non-negative");
        return NULL;
    }
    if (a->size != (Py_ssize_t)n * k) {
        PyErr_Format(PyExc_ValueError, "Shape mismatch A: %zd != %d x %d", a->size, n, k);
        return NULL;
    }
    if (b->size != (Py_ssize_t)k * m) {
        PyErr_Format(PyExc_ValueError, "Shape mismatch B: %zd != %d x %d", b->size, k, m);
        return NULL;
    }
    TensorObject *r = alloc_tensor((Py_ssize_t)n * m);
    if (!r) return NULL;
    matmul(a->d_ptr, b->d_ptr, r->d_ptr, n, m, k);
    return finish(r, "_matmul");
}

static PyObject *py_matmul_batched(PyObject *module, PyObject *args)
{
    TensorObject *a, *b;
    int batch, n, m, k;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!O!iiii", &TensorType, &a, &TensorType, &b, &batch, &n, &m, &k))
        return NULL;
    if (batch < 0 || n < 0 || m < 0 || k < 0) {
        PyErr_SetString(PyExc_ValueError, "matmul dimensions must be non-negative");
        return NULL;
    }
    if (a->size != (Py_ssize_t)batch * n * k) {
        PyErr_Format(PyExc_ValueError, "Shape mismatch A: %zd != %d x %d x %d", a->size, batch, n, k);
        return NULL;
    }
    if (b->size != (Py_ssize_t)batch * k * m) {
        PyErr_Format(PyExc_ValueError, "Shape mismatch B: %zd != %d x %d x %d", b->size, batch, k, m);
        return NULL;
    }
    TensorObject *r = alloc_tensor((Py_ssize_t)batch * n * m);
    if (!r) return NULL;
    matmul_batched(a->d_ptr, b->d_ptr, r->d_ptr, batch, n, m, k);
    return finish(r, "_matmul_batched");
}

static PyObject *py_transpose(PyObject *module, PyObject *args)
{
    TensorObject *a;
    int n, m;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!ii", &TensorType, &a, &n, &m)) return NULL;
    if (n < 0 || m < 0 || a->size != (Py_ssize_t)n * m) {
        PyErr_Format(PyExc_ValueError, "Shape mismatch: %zd != %d x %d", a->size, n, m);
        return NULL;
    }
    TensorObject *r = alloc_tensor(a->size);
    if (!r) return NULL;
    transpose(a->d_ptr, r->d_ptr, n, m);
    return finish(r, "_transpose");
}

static PyObject *py_sum(PyObject *module, PyObject *args)
{
    TensorObject *a;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!", &TensorType, &a)) return NULL;
    if (!fits_int(a->size, "_sum")) return NULL;
    const float s = sum(a->d_ptr, (int)a->size);
    if (raise_status(0, "_sum")) return NULL;
    return PyFloat_FromDouble((double)s);
}

/* _mse_loss(pred, target, scale) -> (sum of squared differences, grad):
 * one pass for MSELoss (see mse_loss). */
static PyObject *py_mse_loss(PyObject *module, PyObject *args)
{
    TensorObject *p, *t;
    float scale;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!O!f", &TensorType, &p, &TensorType, &t, &scale)) return NULL;
    if (p->size != t->size) {
        PyErr_SetString(PyExc_ValueError, "_mse_loss: size mismatch");
        return NULL;
    }
    if (!fits_int(p->size, "_mse_loss")) return NULL;
    TensorObject *g = alloc_tensor(p->size);
    if (!g) return NULL;
    float loss = 0.0f;
    int st = mse_loss(p->d_ptr, t->d_ptr, g->d_ptr, (int)p->size, scale, &loss);
    if (raise_status(st, "_mse_loss")) {
        Py_DECREF(g);
        return NULL;
    }
    return Py_BuildValue("(dN)", (double)loss, (PyObject *)g);
}

typedef void (*axis_fn)(const float *, float *, int, int, int);

static PyObject *do_axis(PyObject *args, axis_fn fn, const char *what)
{
    TensorObject *a;
    PyObject *shape_t;
    int axis;
    if (!PyArg_ParseTuple(args, "O!O!i", &TensorType, &a, &PyTuple_Type, &shape_t, &axis)) return NULL;
    int shape[16], nd;
    if (int_tuple(shape_t, shape, &nd)) return NULL;
    if (axis < 0 || axis >= nd) {
        PyErr_Format(PyExc_ValueError, "Axis %d out of bound for %d dim Tensor", axis, nd);
        return NULL;
    }
    Py_ssize_t outer = 1, inner = 1;
    for (int i = 0; i < axis; i++) outer *= shape[i];
    for (int i = axis + 1; i < nd; i++) inner *= shape[i];
    if (outer * inner * shape[axis] != a->size) {
        PyErr_SetString(PyExc_ValueError, "Shape does not match the Tensor's size");
        return NULL;
    }
    if (!fits_int(a->size, what)) return NULL;
    TensorObject *r = alloc_tensor(outer * inner);
    if (!r) return NULL;
    fn(a->d_ptr, r->d_ptr, (int)outer, (int)inner, shape[axis]);
    return finish(r, what);
}

static PyObject *py_sum_axis(PyObject *m, PyObject *args)
{
    (void)m;
    return do_axis(args, sum_axis, "_sum_axis");
}

static PyObject *py_max_axis(PyObject *m, PyObject *args)
{
    (void)m;
    return do_axis(args, max_axis, "_max_axis");
}

/* _softmax(a, shape, axis) -> softmax along axis in one launch (same shape);
 * replaces the five-operator composition of ember/tensor/tensor.py:430-437. */
static PyObject *py_softmax(PyObject *module, PyObject *args)
{
    TensorObject *a;
    PyObject *shape_t;
    int axis;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!O!i", &TensorType, &a, &PyTuple_Type, &shape_t, &axis)) return NULL;
    int shape[16], nd;
    if (int_tuple(shape_t, shape, &nd)) return NULL;
    if (axis < 0 || axis >= nd) {
        PyErr_Format(PyExc_ValueError, "Axis %d out of bound for %d dim Tensor", axis, nd);
        return NULL;
    }
    Py_ssize_t outer = 1, inner = 1;
    for (int i = 0; i < axis; i++) outer *= shape[i];
    for (int i = axis + 1; i < nd; i++) inner *= shape[i];
    if (outer * inner * shape[axis] != a->size) {
        PyErr_SetString(PyExc_ValueError, "Shape does not match the Tensor's size");
        return NULL;
    }
    if (!fits_int(a->size, "_softmax")) return NULL;
    TensorObject *r = alloc_tensor(a->size);
    if (!r) return NULL;
    int st = softmax_axis(a->d_ptr, r->d_ptr, (int)outer, (int)inner, shape[axis]);
    if (raise_status(st, "_softmax")) {
        Py_DECREF(r);
        return NULL;
    }
    return (PyObject *)r;
}

/* ---- attention (new; no reference counterpart) ---- */

static int check_bhsd(TensorObject *t, long long B, long long H, long long S, long long D,
                      const char *name)
{
    if (t->size != (Py_ssize_t)(B * H * S * D)) {
        PyErr_Format(PyExc_ValueError, "%s holds %zd elements, expected B*H*S*D = %lld", name,
                     t->size, B * H * S * D);
        return -1;
    }
    return 0;
}

/* _attention_fwd(q, k, v, B, H, S, D, scale, causal) -> (o, lse), contiguous
 * (B, H, S, D) inputs; lse is (B, H, S) in natural log. */
static PyObject *py_attention_fwd(PyObject *module, PyObject *args)
{
    TensorObject *q, *k, *v;
    long long B, H, S, D;
    float scale;
    int causal;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!O!O!LLLLfp", &TensorType, &q, &TensorType, &k, &TensorType, &v,
                          &B, &H, &S, &D, &scale, &causal))
        return NULL;
    if (B < 0 || H < 0 || S < 0 || D <= 0) {
        PyErr_SetString(PyExc_ValueError, "attention extents must be non-negative (D positive)");
        return NULL;
    }
    if (check_bhsd(q, B, H, S, D, "q") || check_bhsd(k, B, H, S, D, "k") ||
        check_bhsd(v, B, H, S, D, "v"))
        return NULL;
    TensorObject *o = alloc_tensor(q->size);
    if (!o) return NULL;
    TensorObject *lse = alloc_tensor((Py_ssize_t)(B * H * S));
    if (!lse) {
        Py_DECREF(o);
        return NULL;
    }
    const int64_t sb = H * S * D, sh = S * D, ss = D;
    int st = attention_fwd(q->d_ptr, k->d_ptr, v->d_ptr, o->d_ptr, lse->d_ptr, B, H, S, D, scale,
                           causal, sb, sh, ss, sb, sh, ss);
    if (raise_status(st, "_attention_fwd")) {
        Py_DECREF(o);
        Py_DECREF(lse);
        return NULL;
    }
    return Py_BuildValue("(NN)", (PyObject *)o, (PyObject *)lse);
}

/* _attention_bwd(q, k, v, o, lse, d_o, B, H, S, D, scale, causal) -> (dq, dk, dv). */
static PyObject *py_attention_bwd(PyObject *module, PyObject *args)
{
    TensorObject *q, *k, *v, *o, *lse, *d_o;
    long long B, H, S, D;
    float scale;
    int causal;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!O!O!O!O!O!LLLLfp", &TensorType, &q, &TensorType, &k,
                          &TensorType, &v, &TensorType, &o, &TensorType, &lse, &TensorType, &d_o,
                          &B, &H, &S, &D, &scale, &causal))
        return NULL;
    if (B < 0 || H < 0 || S < 0 || D <= 0) {
        PyErr_SetString(PyExc_ValueError, "attention extents must be non-negative (D positive)");
        return NULL;
    }
    if (check_bhsd(q, B, H, S, D, "q") || check_bhsd(k, B, H, S, D, "k") ||
        check_bhsd(v, B, H, S, D, "v") || check_bhsd(o, B, H, S, D, "o") ||
        check_bhsd(d_o, B, H, S, D, "d_o") || check_bhsd(lse, B, H, S, 1, "lse"))
        return NULL;
    TensorObject *g[3] = {NULL, NULL, NULL};
    for (int i = 0; i < 3; i++) {
        g[i] = alloc_tensor(q->size);
        if (!g[i]) {
            for (int j = 0; j < i; j++) Py_DECREF(g[j]);
            return NULL;
        }
    }
    const int64_t sb = H * S * D, sh = S * D, ss = D;
    int st = attention_bwd(q->d_ptr, k->d_ptr, v->d_ptr, o->d_ptr, lse->d_ptr, d_o->d_ptr,
                           g[0]->d_ptr, g[1]->d_ptr, g[2]->d_ptr, B, H, S, D, scale, causal, sb,
                           sh, ss, sb, sh, ss);
    if (raise_status(st, "_attention_bwd")) {
        for (int i = 0; i < 3; i++) Py_DECREF(g[i]);
        return NULL;
    }
    return Py_BuildValue("(NNN)", (PyObject *)g[0], (PyObject *)g[1], (PyObject *)g[2]);
}

/* ---- transformer-block pieces (config 5) ---- */

static TensorObject *opt_tensor(PyObject *o, const char *name)
{
    if (o == Py_None) return NULL;
    if (!PyObject_TypeCheck(o, &TensorType)) {
        PyErr_Format(PyExc_TypeError, "%s must be a _Tensor or None", name);
        return (TensorObject *)-1;
    }
    return (TensorObject *)o;
}

/* _linear(x, w, bias|None, residual|None, n, m, k, act, want_pre) -> (y, pre|None):
 * y = act(x @ w + bias) + residual, one GEMM with a fused epilogue. */
static PyObject *py_linear(PyObject *module, PyObject *args)
{
    TensorObject *x, *w;
    PyObject *bo, *ro;
    int n, m, k, act, want_pre;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!O!OOiiiip", &TensorType, &x, &TensorType, &w, &bo, &ro, &n, &m,
                          &k, &act, &want_pre))
        return NULL;
    TensorObject *bias = opt_tensor(bo, "bias"), *res = opt_tensor(ro, "residual");
    if (bias == (TensorObject *)-1 || res == (TensorObject *)-1) return NULL;
    if (n < 0 || m < 0 || k < 0 || x->size != (Py_ssize_t)n * k || w->size != (Py_ssize_t)k * m ||
        (bias && bias->size != m) || (res && res->size != (Py_ssize_t)n * m)) {
        PyErr_SetString(PyExc_ValueError, "_linear: operand sizes do not match (n, m, k)");
        return NULL;
    }
    TensorObject *y = alloc_tensor((Py_ssize_t)n * m);
    if (!y) return NULL;
    TensorObject *pre = NULL;
    if (want_pre && !(pre = alloc_tensor((Py_ssize_t)n * m))) {
        Py_DECREF(y);
        return NULL;
    }
    int st = linear_fwd(x->d_ptr, w->d_ptr, bias ? bias->d_ptr : NULL, res ? res->d_ptr : NULL,
                        y->d_ptr, pre ? pre->d_ptr : NULL, n, m, k, act);
    if (raise_status(st, "_linear")) {
        Py_DECREF(y);
        Py_XDECREF(pre);
        return NULL;
    }
    if (!pre) return Py_BuildValue("(NO)", (PyObject *)y, Py_None);
    return Py_BuildValue("(NN)", (PyObject *)y, (PyObject *)pre);
}

/* _gemm(a, b, batch, n, m, k, trans_a, trans_b, bias|None, residual|None) -> out:
 * out = op(a) @ op(b) + bias + residual per batch, op(a) = a (n x k) or a^T
 * of a stored (k x n), op(b) = b (k x m) or b^T of b stored (m x k). */
static PyObject *py_gemm(PyObject *module, PyObject *args)
{
    TensorObject *a, *b;
    PyObject *bo, *ro;
    int batch, n, m, k, ta, tb;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!O!iiiippOO", &TensorType, &a, &TensorType, &b, &batch, &n, &m,
                          &k, &ta, &tb, &bo, &ro))
        return NULL;
    TensorObject *bias = opt_tensor(bo, "bias"), *res = opt_tensor(ro, "residual");
    if (bias == (TensorObject *)-1 || res == (TensorObject *)-1) return NULL;
    if (batch < 0 || n < 0 || m < 0 || k < 0 || a->size != (Py_ssize_t)batch * n * k ||
        b->size != (Py_ssize_t)batch * k * m || (bias && bias->size != m) ||
        (res && res->size != (Py_ssize_t)batch * n * m)) {
        PyErr_SetString(PyExc_ValueError, "_gemm: operand sizes do not match (batch, n, m, k)");
        return NULL;
    }
    TensorObject *out = alloc_tensor((Py_ssize_t)batch * n * m);
    if (!out) return NULL;
    int st = gemm_ex(a->d_ptr, b->d_ptr, out->d_ptr, batch, n, m, k, ta, tb,
                     bias ? bias->d_ptr : NULL, res ? res->d_ptr : NULL, NULL, 0);
    if (raise_status(st, "_gemm")) {
        Py_DECREF(out);
        return NULL;
    }
    return (PyObject *)out;
}

/* _gelu_bwd(dy, u, y=None): y None recomputes the GELU output from u. */
static PyObject *py_gelu_bwd(PyObject *module, PyObject *args)
{
    TensorObject *dy, *u;
    PyObject *yo = Py_None;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!O!|O", &TensorType, &dy, &TensorType, &u, &yo)) return NULL;
    TensorObject *y = NULL;
    if (yo != Py_None) {
        if (!PyObject_TypeCheck(yo, &TensorType)) {
            PyErr_SetString(PyExc_TypeError, "_gelu_bwd: y must be a _Tensor or None");
            return NULL;
        }
        y = (TensorObject *)yo;
    }
    if (dy->size != u->size || (y && y->size != u->size)) {
        PyErr_SetString(PyExc_ValueError, "_gelu_bwd: size mismatch");
        return NULL;
    }
    TensorObject *dx = alloc_tensor(u->size);
    if (!dx) return NULL;
    int st = gelu_bwd(dy->d_ptr, u->d_ptr, y ? y->d_ptr : NULL, dx->d_ptr, u->size);
    if (raise_status(st, "_gelu_bwd")) {
        Py_DECREF(dx);
        return NULL;
    }
    return (PyObject *)dx;
}

static PyObject *py_col_sum(PyObject *module, PyObject *args)
{
    TensorObject *x;
    long long rows, cols;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!LL", &TensorType, &x, &rows, &cols)) return NULL;
    if (rows < 0 || cols < 0 || x->size != (Py_ssize_t)(rows * cols)) {
        PyErr_SetString(PyExc_ValueError, "_col_sum: size mismatch");
        return NULL;
    }
    TensorObject *out = alloc_tensor((Py_ssize_t)cols);
    if (!out) return NULL;
    int st = col_sum(x->d_ptr, out->d_ptr, rows, cols);
    if (raise_status(st, "_col_sum")) {
        Py_DECREF(out);
        return NULL;
    }
    return (PyObject *)out;
}

/* _gelu_bwd_col_sum(dy, u, rows, cols) -> (dx, dbias): _gelu_bwd (output
 * recomputed) and _col_sum of its result in one pass, the same bits. */
static PyObject *py_gelu_bwd_col_sum(PyObject *module, PyObject *args)
{
    TensorObject *dy, *u;
    long long rows, cols;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!O!LL", &TensorType, &dy, &TensorType, &u, &rows, &cols)) return NULL;
    if (rows < 0 || cols < 0 || dy->size != u->size || u->size != (Py_ssize_t)(rows * cols)) {
        PyErr_SetString(PyExc_ValueError, "_gelu_bwd_col_sum: size mismatch");
        return NULL;
    }
    TensorObject *dx = alloc_tensor(u->size);
    if (!dx) return NULL;
    TensorObject *db = alloc_tensor((Py_ssize_t)cols);
    if (!db) {
        Py_DECREF(dx);
        return NULL;
    }
    int st = gelu_bwd_col_sum(dy->d_ptr, u->d_ptr, dx->d_ptr, db->d_ptr, rows, cols);
    if (raise_status(st, "_gelu_bwd_col_sum")) {
        Py_DECREF(dx);
        Py_DECREF(db);
        return NULL;
    }
    return Py_BuildValue("(NN)", dx, db);
}

static PyObject *py_layernorm_fwd(PyObject *module, PyObject *args)
{
    TensorObject *x, *g, *b;
    long long rows, d;
    float eps;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!O!O!LLf", &TensorType, &x, &TensorType, &g, &TensorType, &b, &rows,
                          &d, &eps))
        return NULL;
    if (rows < 0 || d <= 0 || x->size != (Py_ssize_t)(rows * d) || g->size != d || b->size != d) {
        PyErr_SetString(PyExc_ValueError, "_layernorm_fwd: size mismatch");
        return NULL;
    }
    TensorObject *y = alloc_tensor(x->size), *mean = NULL, *rstd = NULL;
    if (!y || !(mean = alloc_tensor((Py_ssize_t)rows)) || !(rstd = alloc_tensor((Py_ssize_t)rows))) {
        Py_XDECREF(y);
        Py_XDECREF(mean);
        return NULL;
    }
    int st = layernorm_fwd(x->d_ptr, g->d_ptr, b->d_ptr, y->d_ptr, mean->d_ptr, rstd->d_ptr, rows, d, eps);
    if (raise_status(st, "_layernorm_fwd")) {
        Py_DECREF(y);
        Py_DECREF(mean);
        Py_DECREF(rstd);
        return NULL;
    }
    return Py_BuildValue("(NNN)", (PyObject *)y, (PyObject *)mean, (PyObject *)rstd);
}

/* _layernorm_bwd(x, gamma, mean, rstd, dy, rows, d[, dres]) -> (dx, dgamma, dbeta);
 * dres (optional) is added to dx: the gradient reaching x through a residual. */
static PyObject *py_layernorm_bwd(PyObject *module, PyObject *args)
{
    TensorObject *x, *g, *mean, *rstd, *dy;
    PyObject *ro = Py_None;
    long long rows, d;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!O!O!O!O!LL|O", &TensorType, &x, &TensorType, &g, &TensorType,
                          &mean, &TensorType, &rstd, &TensorType, &dy, &rows, &d, &ro))
        return NULL;
    TensorObject *res = opt_tensor(ro, "dres");
    if (res == (TensorObject *)-1) return NULL;
    if (rows < 0 || d <= 0 || x->size != (Py_ssize_t)(rows * d) || dy->size != x->size ||
        g->size != d || mean->size != rows || rstd->size != rows || (res && res->size != x->size)) {
        PyErr_SetString(PyExc_ValueError, "_layernorm_bwd: size mismatch");
        return NULL;
    }
    TensorObject *dx = alloc_tensor(x->size), *dg = NULL, *db = NULL;
    if (!dx || !(dg = alloc_tensor((Py_ssize_t)d)) || !(db = alloc_tensor((Py_ssize_t)d))) {
        Py_XDECREF(dx);
        Py_XDECREF(dg);
        return NULL;
    }
    int st = layernorm_bwd(x->d_ptr, g->d_ptr, mean->d_ptr, rstd->d_ptr, dy->d_ptr,
                           res ? res->d_ptr : NULL, dx->d_ptr, dg->d_ptr, db->d_ptr, rows, d);
    if (raise_status(st, "_layernorm_bwd")) {
        Py_DECREF(dx);
        Py_DECREF(dg);
        Py_DECREF(db);
        return NULL;
    }
    return Py_BuildValue("(NNN)", (PyObject *)dx, (PyObject *)dg, (PyObject *)db);
}

/* Packed projections: qkv is (B, S, 3, H, D) (a QKV Linear's output), o is
 * (B, S, H, D); attention reads and writes them through strides, no copies. */
static PyObject *py_attention_fwd_packed(PyObject *module, PyObject *args)
{
    TensorObject *qkv;
    long long B, S, H, D;
    float scale;
    int causal;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!LLLLfp", &TensorType, &qkv, &B, &S, &H, &D, &scale, &causal))
        return NULL;
    if (B < 0 || S < 0 || H < 0 || D <= 0 || qkv->size != (Py_ssize_t)(B * S * 3 * H * D)) {
        PyErr_SetString(PyExc_ValueError, "_attention_fwd_packed: qkv must hold B*S*3*H*D elements");
        return NULL;
    }
    TensorObject *o = alloc_tensor((Py_ssize_t)(B * S * H * D)), *lse = NULL;
    if (!o || !(lse = alloc_tensor((Py_ssize_t)(B * H * S)))) {
        Py_XDECREF(o);
        return NULL;
    }
    const int64_t hd = H * D;
    int st = attention_fwd(qkv->d_ptr, qkv->d_ptr + hd, qkv->d_ptr + 2 * hd, o->d_ptr, lse->d_ptr, B,
                           H, S, D, scale, causal, S * 3 * hd, D, 3 * hd, S * hd, D, hd);
    if (raise_status(st, "_attention_fwd_packed")) {
        Py_DECREF(o);
        Py_DECREF(lse);
        return NULL;
    }
    return Py_BuildValue("(NN)", (PyObject *)o, (PyObject *)lse);
}

static PyObject *py_attention_bwd_packed(PyObject *module, PyObject *args)
{
    TensorObject *qkv, *o, *lse, *d_o;
    long long B, S, H, D;
    float scale;
    int causal;
    (void)module;
    if (!PyArg_ParseTuple(args, "O!O!O!O!LLLLfp", &TensorType, &qkv, &TensorType, &o, &TensorType, &lse,
                          &TensorType, &d_o, &B, &S, &H, &D, &scale, &causal))
        return NULL;
    if (B < 0 || S < 0 || H < 0 || D <= 0 || qkv->size != (Py_ssize_t)(B * S * 3 * H * D) ||
        o->size != (Py_ssize_t)(B * S * H * D) || d_o->size != o->size ||
        lse->size != (Py_ssize_t)(B * H * S)) {
        PyErr_SetString(PyExc_ValueError, "_attention_bwd_packed: size mismatch");
        return NULL;
    }
    TensorObject *g = alloc_tensor(qkv->size);
    if (!g) return NULL;
    const int64_t hd = H * D;
    int st = attention_bwd(qkv->d_ptr, qkv->d_ptr + hd, qkv->d_ptr + 2 * hd, o->d_ptr, lse->d_ptr,
                           d_o->d_ptr, g->d_ptr, g->d_ptr + hd, g->d_ptr + 2 * hd, B, H, S, D, scale,
                           causal, S * 3 * hd, D, 3 * hd, S * hd, D, hd);
    if (raise_status(st, "_attention_bwd_packed")) {
        Py_DECREF(g);
        return NULL;
    }
    return (PyObject *)g;
}

/* Fused optimiser steps over lists of _Tensor of matching sizes, updated in
 * place with one launch per 48 tensors:
 *   _adam_step(params, grads, means, variances, lr, beta1, beta2, eps, t)
 *     replaces Adam.apply (ember/optim/adam.py:24-45);
 *   _adamw_step(params, grads, means, variances, lr, beta1, beta2, eps,
 *               weight_decay, t)  replaces AdamW.apply (adamw.py:33-56);
 *   _sgd_step(params, grads, velocities, lr, momentum)  replaces SGD.apply
 *     (sgd.py:25-35). */
enum { OPT_ADAM, OPT_ADAMW, OPT_SGD };

static PyObject *opt_step(PyObject *args, int rule, const char *name)
{
    PyObject *lists[4] = {NULL, NULL, NULL, NULL};
    double lr = 0, b1 = 0, b2 = 0, eps = 0, wd = 0, momentum = 0;
    long long t = 1;
    int nl = 4;
    int ok;
    if (rule == OPT_ADAM)
        ok = PyArg_ParseTuple(args, "O!O!O!O!ddddL", &PyList_Type, &lists[0], &PyList_Type, &lists[1],
                              &PyList_Type, &lists[2], &PyList_Type, &lists[3], &lr, &b1, &b2, &eps, &t);
    else if (rule == OPT_ADAMW)
        ok = PyArg_ParseTuple(args, "O!O!O!O!dddddL", &PyList_Type, &lists[0], &PyList_Type, &lists[1],
                              &PyList_Type, &lists[2], &PyList_Type, &lists[3], &lr, &b1, &b2, &eps, &wd,
                              &t);
    else {
        nl = 3;
        ok = PyArg_ParseTuple(args, "O!O!O!dd", &PyList_Type, &lists[0], &PyList_Type, &lists[1],
                              &PyList_Type, &lists[2], &lr, &momentum);
    }
    if (!ok) return NULL;
    const Py_ssize_t n = PyList_GET_SIZE(lists[0]);
    for (int j = 1; j < nl; j++)
        if (PyList_GET_SIZE(lists[j]) != n) {
            PyErr_Format(PyExc_ValueError, "Optimizer expected %zd gradients / states, got %zd", n,
                         PyList_GET_SIZE(lists[j]));
            return NULL;
        }
    if (n > INT_MAX) return PyErr_NoMemory();
    float **tab = (float **)PyMem_Malloc((size_t)(nl * n + 1) * sizeof(float *));
    int64_t *sizes = (int64_t *)PyMem_Malloc((size_t)(n + 1) * sizeof(int64_t));
    if (!tab || !sizes) {
        PyMem_Free(tab);
        PyMem_Free(sizes);
        return PyErr_NoMemory();
    }
    for (Py_ssize_t i = 0; i < n; i++) {
        for (int j = 0; j < nl; j++) {
            PyObject *item = PyList_GET_ITEM(lists[j], i);
            if (!PyObject_TypeCheck(item, &TensorType)) {
                PyErr_Format(PyExc_TypeError, "%s expects lists of _Tensor", name);
                goto fail;
            }
            tab[j * n + i] = ((TensorObject *)item)->d_ptr;
            if (((TensorObject *)item)->size != ((TensorObject *)PyList_GET_ITEM(lists[0], i))->size) {
                PyErr_Format(PyExc_ValueError, "Size mismatch for parameter %zd", i);
                goto fail;
            }
        }
        sizes[i] = ((TensorObject *)PyList_GET_ITEM(lists[0], i))->size;
    }
    {
        const float *const *g = (const float *const *)(tab + n);
        int st;
        if (rule == OPT_ADAM)
            st = adam_step(tab, g, tab + 2 * n, tab + 3 * n, sizes, (int)n, lr, b1, b2, eps, (int64_t)t);
        else if (rule == OPT_ADAMW)
            st = adamw_step(tab, g, tab + 2 * n, tab + 3 * n, sizes, (int)n, lr, b1, b2, eps, wd,
                            (int64_t)t);
        else
            st = sgd_step(tab, g, tab + 2 * n, sizes, (int)n, lr, momentum);
        PyMem_Free(tab);
        PyMem_Free(sizes);
        if (raise_status(st, name)) return NULL;
        Py_RETURN_NONE;
    }
fail:
    PyMem_Free(tab);
    PyMem_Free(sizes);
    return NULL;
}

static PyObject *py_adam_step(PyObject *module, PyObject *args)
{
    (void)module;
    return opt_step(args, OPT_ADAM, "_adam_step");
}

static PyObject *py_adamw_step(PyObject *module, PyObject *args)
{
    (void)module;
    return opt_step(args, OPT_ADAMW, "_adamw_step");
}

static PyObject *py_sgd_step(PyObject *module, PyObject *args)
{
    (void)module;
    return opt_step(args, OPT_SGD, "_sgd_step");
}

static PyObject *py_synchronize(PyObject *module, PyObject *unused)
{
    (void)module;
    (void)unused;
    sync_device();
    if (raise_status(0, "_synchronize")) return NULL;
    Py_RETURN_NONE;
}

static PyObject *py_empty_cache(PyObject *module, PyObject *unused)
{
    (void)module;
    (void)unused;
    ember_empty_cache();
    if (raise_status(0, "_empty_cache")) return NULL;
    Py_RETURN_NONE;
}

static PyObject *py_memory_stats(PyObject *module, PyObject *unused)
{
    (void)module;
    (void)unused;
    size_t in_use = 0, cached = 0, peak = 0;
    ember_memory_stats(&in_use, &cached, &peak);
    if (raise_status(0, "_memory_stats")) return NULL;
    return Py_BuildValue("{s:K,s:K,s:K}", "in_use", (unsigned long long)in_use, "cached",
                         (unsigned long long)cached, "peak", (unsigned long long)peak);
}

/* ---- module ---- */

#define METHOD(pyname, fn, doc) {pyname, (PyCFunction)fn, METH_VARARGS, doc}

static PyMethodDef module_methods[] = {
#define EMBER_BINARY_OP(name, expr) METHOD("_" #name "_tensor", py_##name##_tensor, "Element-wise " #name),
#define EMBER_SCALAR_OP(name, expr) METHOD("_" #name "_scalar", py_##name##_scalar, "Element-wise " #name " with a scalar"),
#define EMBER_BROADCAST_OP(name, expr) METHOD("_" #name "_broadcasted", py_##name##_broadcasted, "Broadcast " #name),
#define EMBER_UNARY_OP(name, expr) METHOD("_" #name, py_##name, "Element-wise " #name),
#include "operators.def"
    METHOD("_matmul", py_matmul, "out(n x m) = a(n x k) @ b(k x m)"),
    METHOD("_matmul_batched", py_matmul_batched, "batched matmul, equal batch dims"),
    METHOD("_transpose", py_transpose, "2-D transpose"),
    METHOD("_from_numpy", py_from_numpy, "float32 C-contiguous buffer -> _Tensor"),
    METHOD("_sum", py_sum, "sum of all elements"),
    METHOD("_mse_loss", py_mse_loss, "MSE loss sum and gradient in one pass"),
    METHOD("_sum_axis", py_sum_axis, "sum over one axis"),
    METHOD("_max_axis", py_max_axis, "max over one axis"),
    METHOD("_softmax", py_softmax, "softmax along one axis, one launch"),
    METHOD("_attention_fwd", py_attention_fwd, "fused attention forward -> (o, lse)"),
    METHOD("_attention_bwd", py_attention_bwd, "fused attention backward -> (dq, dk, dv)"),
    METHOD("_adam_step", py_adam_step, "fused Adam step over lists of _Tensor, in place"),
    METHOD("_adamw_step", py_adamw_step, "fused AdamW step over lists of _Tensor, in place"),
    METHOD("_sgd_step", py_sgd_step, "fused SGD (momentum) step over lists of _Tensor, in place"),
    METHOD("_linear", py_linear, "act(x @ w + bias) + residual -> (y, pre)"),
    METHOD("_gemm", py_gemm, "op(a) @ op(b) + bias + residual with either operand transposed in place"),
    METHOD("_gelu_bwd", py_gelu_bwd, "backward of Ember's GELU"),
    METHOD("_col_sum", py_col_sum, "column sums (bias gradient)"),
    METHOD("_gelu_bwd_col_sum", py_gelu_bwd_col_sum, "GELU backward and its column sums in one pass"),
    METHOD("_layernorm_fwd", py_layernorm_fwd, "LayerNorm -> (y, mean, rstd)"),
    METHOD("_layernorm_bwd", py_layernorm_bwd, "LayerNorm backward -> (dx, dgamma, dbeta)"),
    METHOD("_attention_fwd_packed", py_attention_fwd_packed, "attention on packed (B,S,3,H,D) qkv"),
    METHOD("_attention_bwd_packed", py_attention_bwd_packed, "backward -> packed dqkv"),
    {"_synchronize", (PyCFunction)py_synchronize, METH_NOARGS, "wait for all queued device work"},
    {"_empty_cache", (PyCFunction)py_empty_cache, METH_NOARGS,
     "return the allocator's cached blocks on the current device to HIP"},
    {"_memory_stats", (PyCFunction)py_memory_stats, METH_NOARGS,
     "allocator bytes in use, cached and peak in use on the current device"},
    {NULL, NULL, 0, NULL}};

static PyModuleDef tensor_module = {
    PyModuleDef_HEAD_INIT, .m_name = "ember_amd._core._tensor",
    .m_doc = "Ember tensor backend on libember_amd (MI355X)", .m_size = -1,
    .m_methods = module_methods,
};

PyMODINIT_FUNC PyInit__tensor(void)
{
    if (PyType_Ready(&TensorType) < 0) return NULL;
    PyObject *m = PyModule_Create(&tensor_module);
    if (!m) return NULL;
    Py_INCREF(&TensorType);
    if (PyModule_AddObject(m, "_Tensor", (PyObject *)&TensorType) < 0) {
        Py_DECREF(&TensorType);
        Py_DECREF(m);
        return NULL;
    }
    return m;
}
