/* hoststep.c -- the optimizer step's per-tensor host bookkeeping in C.
 *
 * The reference's step() walks every parameter in Python: skip grad None,
 * ``state['step'] += 1`` (src/optim/adana.py:184-197;
 * src/optim/dana_star_mk4.py:243-262).  In the steady state of a run whose
 * gradient tensors persist between steps (the same ``p.grad`` objects, updated
 * in place), the optimizer's cached launch plan, scalar classes and device
 * tables all carry over, and what is left per tensor is that walk.  With
 * thousands of small tensors it dominates the step, so it is done here in one
 * C loop instead of several Python passes.
 */
#define PY_SSIZE_T_CLEAN
#include <Python.h>

/* advance_if_same(params, grads, states) -> bool
 *
 * True when params[i].grad is grads[i] for every i (identity); then every
 * dict in ``states`` has its "step" entry incremented by one.  False (and
 * nothing modified) as soon as one gradient differs. */
static PyObject *advance_if_same(PyObject *self, PyObject *args) {
    PyObject *params, *grads, *states;
    (void)self;
    if (!PyArg_ParseTuple(args, "O!O!O!", &PyList_Type, &params, &PyList_Type, &grads, &PyList_Type, &states))
        return NULL;
    const Py_ssize_t n = PyList_GET_SIZE(params);
    if (PyList_GET_SIZE(grads) != n) Py_RETURN_FALSE;
    static PyObject *grad_name = NULL, *step_name = NULL, *one = NULL;
    if (!grad_name && !(grad_name = PyUnicode_InternFromString("grad"))) return NULL;
    if (!step_name && !(step_name = PyUnicode_InternFromString("step"))) return NULL;
    if (!one && !(one = PyLong_FromLong(1))) return NULL;
    for (Py_ssize_t i = 0; i < n; ++i) {
        PyObject *g = PyObject_GetAttr(PyList_GET_ITEM(params, i), grad_name);
        if (!g) return NULL;
        const int same = g == PyList_GET_ITEM(grads, i);
        Py_DECREF(g);
        if (!same) Py_RETURN_FALSE;
    }
    const Py_ssize_t m = PyList_GET_SIZE(states);
    for (Py_ssize_t i = 0; i < m; ++i) {
        PyObject *st = PyList_GET_ITEM(states, i);
        if (!PyDict_Check(st)) {
            PyErr_SetString(PyExc_TypeError, "advance_if_same: state entries must be dicts");
            return NULL;
        }
        PyObject *v = PyDict_GetItemWithError(st, step_name);      /* borrowed */
        if (!v) {
            if (!PyErr_Occurred()) PyErr_SetString(PyExc_KeyError, "step");
            return NULL;
        }
        PyObject *w = PyNumber_Add(v, one);
        if (!w) return NULL;
        const int rc = PyDict_SetItem(st, step_name, w);
        Py_DECREF(w);
        if (rc) return NULL;
    }
    Py_RETURN_TRUE;
}

static PyMethodDef methods[] = {
    {"advance_if_same", advance_if_same, METH_VARARGS,
     "advance_if_same(params, grads, states) -> bool: if params[i].grad is grads[i] for all i, "
     "increment every states[j]['step'] and return True; otherwise change nothing and return False."},
    {NULL, NULL, 0, NULL},
};

static struct PyModuleDef module = {PyModuleDef_HEAD_INIT, "_hoststep", NULL, -1, methods, NULL, NULL, NULL, NULL};

PyMODINIT_FUNC PyInit__hoststep(void) { return PyModule_Create(&module); }
