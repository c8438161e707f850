/*
 * _nova_call: a CPython fast-call binding of nova_forward_workspace for the
 * module's cached forward path. ctypes converts and checks eleven arguments
 * per call and needs a second foreign call to read the error code; this
 * METH_FASTCALL function does both in one call. The library's entry points
 * are handed over once (bind) as the addresses ctypes resolved, so this file
 * does not link against the library and there is one loaded copy of it.
 * The Python side falls back to ctypes when this module is not built.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>
#include <stdint.h>

typedef void (*forward_ws_fn)(void*, const void*, void*, void*, void*, int, int, int, int, int,
                              int);
typedef int (*last_error_fn)(void);
typedef const char* (*last_message_fn)(void);

static forward_ws_fn g_forward;
static last_error_fn g_error;
static last_message_fn g_message;

static PyObject* bind(PyObject* self, PyObject* args) {
    unsigned long long f, e, m;
    (void)self;
    if (!PyArg_ParseTuple(args, "KKK", &f, &e, &m)) return NULL;
    if (!f || !e || !m) {
        PyErr_SetString(PyExc_ValueError, "bind: null entry point");
        return NULL;
    }
    g_forward = (forward_ws_fn)(uintptr_t)f;
    g_error = (last_error_fn)(uintptr_t)e;
    g_message = (last_message_fn)(uintptr_t)m;
    Py_RETURN_NONE;
}

static void* as_ptr(PyObject* o) { return o == Py_None ? NULL : PyLong_AsVoidPtr(o); }

/* forward_ws(h, x, y, V, M, B, H, W, pad, nh, nw): pointers as ints (None =
 * NULL), raises RuntimeError with the library's message on failure. */
static PyObject* forward_ws(PyObject* self, PyObject* const* args, Py_ssize_t n) {
    void* p[5];
    int v[6];
    int i;
    (void)self;
    if (n != 11) {
        PyErr_SetString(PyExc_TypeError, "forward_ws takes 11 arguments");
        return NULL;
    }
    if (!g_forward) {
        PyErr_SetString(PyExc_RuntimeError, "forward_ws: library not bound");
        return NULL;
    }
    for (i = 0; i < 5; i++) p[i] = as_ptr(args[i]);
    for (i = 0; i < 6; i++) v[i] = (int)PyLong_AsLong(args[5 + i]);
    if (PyErr_Occurred()) return NULL;
    g_forward(p[0], p[1], p[2], p[3], p[4], v[0], v[1], v[2], v[3], v[4], v[5]);
    {
        const int code = g_error();
        if (code) {
            PyErr_Format(PyExc_RuntimeError, "nova_winograd forward: %s (code %d)", g_message(),
                         code);
            return NULL;
        }
    }
    Py_RETURN_NONE;
}

static PyMethodDef methods[] = {
    {"bind", bind, METH_VARARGS, "bind(forward_ws, get_last_error, get_last_error_message)"},
    {"forward_ws", (PyCFunction)(void (*)(void))forward_ws, METH_FASTCALL,
     "forward_ws(h, x, y, V, M, B, H, W, pad, nh, nw)"},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_nova_call", NULL, -1, methods,
                                    NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__nova_call(void) { return PyModule_Create(&module); }
