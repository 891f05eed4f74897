/* hoststep.cpp -- the optimizer step's per-tensor host bookkeeping in C++.
 *
 * The reference's step() walks every parameter in Python: skip grad None,
 * ``state['step'] += 1`` (src/optim/adana.py:184-197;
 * src/optim/dana_star_mk4.py:243-262), and the in-place update bumps each
 * parameter's autograd version counter.  In the steady state of a run whose
 * gradient tensors persist between steps (the same ``p.grad`` tensors, updated
 * in place), the optimizer's cached launch plan, scalar classes and device
 * tables all carry over, and what is left per tensor is that walk.  With
 * thousands of small tensors it dominates the step.
 *
 * This module does the walk on torch's C++ tensors: a parameter's gradient is
 * read from its TensorImpl (no Python attribute lookup, no wrapper object) and
 * version counters are bumped directly.  Objects that are not exactly a
 * torch.Tensor or torch.nn.Parameter (subclasses may override attribute access)
 * take the generic Python path.
 */
#include <torch/csrc/autograd/python_variable.h>
#include <torch/csrc/autograd/variable.h>
#include <ATen/ops/from_blob.h>

#include <Python.h>

#include <cstdint>
#include <exception>

namespace {

PyObject *g_grad_name = nullptr;
PyObject *g_step_name = nullptr;
PyObject *g_params_name = nullptr;
PyObject *g_one = nullptr;

// True when params[i].grad is the gradient cached[i] (None: no gradient).
// Exact tensors compare TensorImpls, which is the identity of the Python
// objects: a live TensorImpl has at most one Python object, and the caller's
// list keeps the cached ones alive.
int same_grad(PyObject *p, PyObject *cached) {
    if (THPVariable_CheckExact(p)) {
        const at::Tensor &g = THPVariable_Unpack(p).unsafeGetTensorImpl()->grad();
        if (cached == Py_None) return !g.defined();
        if (!g.defined() || !THPVariable_Check(cached)) return 0;
        return g.unsafeGetTensorImpl() == THPVariable_Unpack(cached).unsafeGetTensorImpl();
    }
    PyObject *g = PyObject_GetAttr(p, g_grad_name);
    if (!g) return -1;
    const int same = g == cached;
    Py_DECREF(g);
    return same;
}

// The data pointer of tensor `t` (0 for None), or -1 with a Python error set.
int data_ptr_of(PyObject *t, uint64_t *out) {
    if (t == Py_None) {
        *out = 0;
        return 0;
    }
    if (THPVariable_CheckExact(t)) {
        *out = reinterpret_cast<uint64_t>(THPVariable_Unpack(t).data_ptr());
        return 0;
    }
    PyObject *r = PyObject_CallMethod(t, "data_ptr", nullptr);
    if (!r) return -1;
    *out = static_cast<uint64_t>(PyLong_AsUnsignedLongLong(r));
    Py_DECREF(r);
    return PyErr_Occurred() ? -1 : 0;
}

// states[i]["step"] += 1 for every dict; tensors stepped together hold equal
// counts, so the new int of the previous entry is reused (ints are immutable)
// when this entry's old int is equal.  0, or -1 with a Python error set.
int advance_states(PyObject *states) {
    const Py_ssize_t m = PyList_GET_SIZE(states);
    PyObject *prev_v = nullptr, *prev_w = nullptr;
    int rc = 0;
    for (Py_ssize_t i = 0; i < m && !rc; ++i) {
        PyObject *st = PyList_GET_ITEM(states, i);
        if (!PyDict_Check(st)) {
            PyErr_SetString(PyExc_TypeError, "step counters: state entries must be dicts");
            rc = -1;
            break;
        }
        PyObject *v = PyDict_GetItemWithError(st, g_step_name); /* borrowed */
        if (!v) {
            if (!PyErr_Occurred()) PyErr_SetString(PyExc_KeyError, "step");
            rc = -1;
            break;
        }
        const bool reuse = prev_v && (v == prev_v || (PyLong_CheckExact(v) && PyLong_CheckExact(prev_v) &&
                                                      PyObject_RichCompareBool(v, prev_v, Py_EQ) == 1));
        if (!reuse) {
            PyObject *w = PyNumber_Add(v, g_one);
            if (!w) {
                rc = -1;
                break;
            }
            Py_XDECREF(prev_v);
            Py_XDECREF(prev_w);
            Py_INCREF(v);
            prev_v = v;
            prev_w = w;
        }
        rc = PyDict_SetItem(st, g_step_name, prev_w);
    }
    Py_XDECREF(prev_v);
    Py_XDECREF(prev_w);
    return rc;
}

/* advance_if_same(params, grads, states[, param_ptrs[, grad_ptrs]]) -> bool
 *
 * True when params[i].grad is grads[i] for every i (None included); then every
 * dict in ``states`` has its "step" entry incremented by one.  False (and
 * nothing modified) as soon as one gradient differs. */
PyObject *advance_if_same(PyObject *, PyObject *args) {
    PyObject *params, *grads, *states, *pptrs = Py_None, *gptrs = Py_None;
    if (!PyArg_ParseTuple(args, "O!O!O!|OO", &PyList_Type, &params, &PyList_Type, &grads, &PyList_Type, &states,
                          &pptrs, &gptrs))
        return nullptr;
    const Py_ssize_t n = PyList_GET_SIZE(params);
    if (PyList_GET_SIZE(grads) != n) Py_RETURN_FALSE;
    const uint64_t *want_p = nullptr, *want_g = nullptr;
    if (pptrs != Py_None) {
        if (!PyBytes_Check(pptrs) || PyBytes_GET_SIZE(pptrs) != 8 * n) Py_RETURN_FALSE;
        want_p = reinterpret_cast<const uint64_t *>(PyBytes_AS_STRING(pptrs));
    }
    if (gptrs != Py_None) {
        if (!PyBytes_Check(gptrs) || PyBytes_GET_SIZE(gptrs) != 8 * n) Py_RETURN_FALSE;
        want_g = reinterpret_cast<const uint64_t *>(PyBytes_AS_STRING(gptrs));
    }
    try {
        for (Py_ssize_t i = 0; i < n; ++i) {
            PyObject *p = PyList_GET_ITEM(params, i), *g = PyList_GET_ITEM(grads, i);
            const int same = same_grad(p, g);
            if (same < 0) return nullptr;
            if (!same) Py_RETURN_FALSE;
            uint64_t ptr;
            if (want_p) {
                if (data_ptr_of(p, &ptr)) return nullptr;
                if (ptr != want_p[i]) Py_RETURN_FALSE;
            }
            if (want_g) {                          // the same gradient object may have new storage (set_)
                if (data_ptr_of(g, &ptr)) return nullptr;
                if (ptr != want_g[i]) Py_RETURN_FALSE;
            }
        }
    } catch (const std::exception &e) {
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
    if (advance_states(states)) return nullptr;
    Py_RETURN_TRUE;
}

/* advance_steps(states) -> None: every dict's "step" entry + 1. */
PyObject *advance_steps(PyObject *, PyObject *args) {
    PyObject *states;
    if (!PyArg_ParseTuple(args, "O!", &PyList_Type, &states)) return nullptr;
    if (advance_states(states)) return nullptr;
    Py_RETURN_NONE;
}

/* grads_of(params) -> (grads, absent)
 *
 * ``[p.grad for p in params]`` and a bytes object whose byte i is 1 where
 * params[i].grad is None. */
PyObject *grads_of(PyObject *, PyObject *args) {
    PyObject *params;
    if (!PyArg_ParseTuple(args, "O!", &PyList_Type, &params)) return nullptr;
    const Py_ssize_t n = PyList_GET_SIZE(params);
    PyObject *out = PyList_New(n);
    if (!out) return nullptr;
    PyObject *absent = PyBytes_FromStringAndSize(nullptr, n);
    if (!absent) {
        Py_DECREF(out);
        return nullptr;
    }
    char *ab = PyBytes_AS_STRING(absent);
    try {
        for (Py_ssize_t i = 0; i < n; ++i) {
            PyObject *p = PyList_GET_ITEM(params, i);
            PyObject *g;
            if (THPVariable_CheckExact(p)) {
                const at::Tensor &t = THPVariable_Unpack(p).unsafeGetTensorImpl()->grad();
                if (t.defined()) {
                    g = THPVariable_Wrap(t);
                } else {
                    Py_INCREF(Py_None);
                    g = Py_None;
                }
            } else {
                g = PyObject_GetAttr(p, g_grad_name);
            }
            if (!g) {
                Py_DECREF(out);
                Py_DECREF(absent);
                return nullptr;
            }
            ab[i] = g == Py_None ? 1 : 0;
            PyList_SET_ITEM(out, i, g);                      /* steals the reference */
        }
    } catch (const std::exception &e) {
        Py_DECREF(out);
        Py_DECREF(absent);
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
    return Py_BuildValue("NN", out, absent);
}

/* data_ptrs(tensors) -> bytes: each tensor's data_ptr() (0 for None) as
 * native uint64 values. */
PyObject *data_ptrs(PyObject *, PyObject *args) {
    PyObject *ts;
    if (!PyArg_ParseTuple(args, "O!", &PyList_Type, &ts)) return nullptr;
    const Py_ssize_t n = PyList_GET_SIZE(ts);
    PyObject *out = PyBytes_FromStringAndSize(nullptr, 8 * n);
    if (!out) return nullptr;
    uint64_t *w = reinterpret_cast<uint64_t *>(PyBytes_AS_STRING(out));
    try {
        for (Py_ssize_t i = 0; i < n; ++i) {
            if (data_ptr_of(PyList_GET_ITEM(ts, i), &w[i])) {
                Py_DECREF(out);
                return nullptr;
            }
        }
    } catch (const std::exception &e) {
        Py_DECREF(out);
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
    return out;
}

/* bump_versions(tensors) -> None
 *
 * The autograd version counter of every tensor in the list goes up by one,
 * as torch._C._increment_version(tensors) does (the in-place update of
 * each parameter). */
PyObject *bump_versions(PyObject *, PyObject *args) {
    PyObject *tensors;
    if (!PyArg_ParseTuple(args, "O!", &PyList_Type, &tensors)) return nullptr;
    const Py_ssize_t n = PyList_GET_SIZE(tensors);
    for (Py_ssize_t i = 0; i < n; ++i)
        if (!THPVariable_Check(PyList_GET_ITEM(tensors, i))) {
            PyErr_Format(PyExc_TypeError, "bump_versions: entry %zd is not a tensor", i);
            return nullptr;
        }
    try {
        for (Py_ssize_t i = 0; i < n; ++i)
            torch::autograd::impl::bump_version(THPVariable_Unpack(PyList_GET_ITEM(tensors, i)));
    } catch (const std::exception &e) {
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
    Py_RETURN_NONE;
}

/* same_params(param_groups, flat) -> bool
 *
 * True when the concatenation of every group's "params" is, object for
 * object, the list ``flat`` (the optimizer's cached parameter list). */
PyObject *same_params(PyObject *, PyObject *args) {
    PyObject *groups, *flat;
    if (!PyArg_ParseTuple(args, "OO!", &groups, &PyList_Type, &flat)) return nullptr;
    PyObject *gs = PySequence_Fast(groups, "same_params: param_groups must be a sequence");
    if (!gs) return nullptr;
    const Py_ssize_t ng = PySequence_Fast_GET_SIZE(gs), nf = PyList_GET_SIZE(flat);
    Py_ssize_t k = 0;
    bool same = true;
    for (Py_ssize_t g = 0; g < ng && same; ++g) {
        PyObject *grp = PySequence_Fast_GET_ITEM(gs, g);
        PyObject *ps = PyDict_Check(grp) ? PyDict_GetItemWithError(grp, g_params_name) : nullptr; /* borrowed */
        if (!ps) {
            if (!PyErr_Occurred()) PyErr_SetString(PyExc_KeyError, "params");
            Py_DECREF(gs);
            return nullptr;
        }
        PyObject *pf = PySequence_Fast(ps, "same_params: a group's params must be a sequence");
        if (!pf) {
            Py_DECREF(gs);
            return nullptr;
        }
        const Py_ssize_t np_ = PySequence_Fast_GET_SIZE(pf);
        if (k + np_ > nf) same = false;
        for (Py_ssize_t i = 0; i < np_ && same; ++i, ++k)
            same = PySequence_Fast_GET_ITEM(pf, i) == PyList_GET_ITEM(flat, k);
        Py_DECREF(pf);
    }
    Py_DECREF(gs);
    if (same && k == nf) Py_RETURN_TRUE;
    Py_RETURN_FALSE;
}

/* Same sizes, and the same strides on every dimension of size > 1 (any
 * strides for empty tensors). */
bool same_layout(const at::Tensor &a, const at::Tensor &b) {
    if (!a.sizes().equals(b.sizes())) return false;
    if (a.numel() == 0) return true;
    const auto n = a.sizes();
    const auto sa = a.strides(), sb = b.strides();
    for (size_t d = 0; d < n.size(); ++d)
        if (n[d] != 1 && sa[d] != sb[d]) return false;
    return true;
}

/* grads_match(params, grads, bf16) -> bool
 *
 * True when every grads[i] can stand in for the gradient the launch tables
 * were built with: a dense tensor on params[i]'s device with params[i]'s
 * shape and strides (the parameters' own layouts were checked when the
 * tables were built), float32 (bfloat16 when ``bf16``).  False for anything
 * else, including objects that are not exactly torch tensors: the caller
 * then checks them one by one (and raises the precise error). */
PyObject *grads_match(PyObject *, PyObject *args) {
    PyObject *params, *grads;
    int bf16 = 0;
    if (!PyArg_ParseTuple(args, "O!O!p", &PyList_Type, &params, &PyList_Type, &grads, &bf16)) return nullptr;
    const Py_ssize_t n = PyList_GET_SIZE(params);
    if (PyList_GET_SIZE(grads) != n) Py_RETURN_FALSE;
    const c10::ScalarType want = bf16 ? c10::ScalarType::BFloat16 : c10::ScalarType::Float;
    try {
        for (Py_ssize_t i = 0; i < n; ++i) {
            PyObject *p = PyList_GET_ITEM(params, i), *g = PyList_GET_ITEM(grads, i);
            if (!THPVariable_CheckExact(p) || !THPVariable_CheckExact(g)) Py_RETURN_FALSE;
            const at::Tensor &pt = THPVariable_Unpack(p), &gt = THPVariable_Unpack(g);
            if (!gt.defined() || gt.is_sparse() || gt.scalar_type() != want || gt.device() != pt.device() ||
                !same_layout(gt, pt))
                Py_RETURN_FALSE;
        }
    } catch (const std::exception &e) {
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
    Py_RETURN_TRUE;
}

/* grads_scan(params, bf16) -> (grads, absent, grad_ptrs, param_ptrs, match)
 *
 * One pass doing what grads_of(params), data_ptrs(grads), data_ptrs(params)
 * and grads_match(params, grads, bf16) do together: the gradients and their
 * None pattern, both pointer tables (0 for None), and True when every
 * parameter has a gradient that matches it as grads_match requires. */
PyObject *grads_scan(PyObject *, PyObject *args) {
    PyObject *params;
    int bf16 = 0;
    if (!PyArg_ParseTuple(args, "O!p", &PyList_Type, &params, &bf16)) return nullptr;
    const Py_ssize_t n = PyList_GET_SIZE(params);
    const c10::ScalarType want = bf16 ? c10::ScalarType::BFloat16 : c10::ScalarType::Float;
    PyObject *out = PyList_New(n);
    PyObject *absent = PyBytes_FromStringAndSize(nullptr, n);
    PyObject *gp = PyBytes_FromStringAndSize(nullptr, 8 * n);
    PyObject *pp = PyBytes_FromStringAndSize(nullptr, 8 * n);
    if (!out || !absent || !gp || !pp) {
        Py_XDECREF(out);
        Py_XDECREF(absent);
        Py_XDECREF(gp);
        Py_XDECREF(pp);
        return nullptr;
    }
    char *ab = PyBytes_AS_STRING(absent);
    uint64_t *gw = reinterpret_cast<uint64_t *>(PyBytes_AS_STRING(gp));
    uint64_t *pw = reinterpret_cast<uint64_t *>(PyBytes_AS_STRING(pp));
    bool match = true;
    try {
        for (Py_ssize_t i = 0; i < n; ++i) {
            PyObject *p = PyList_GET_ITEM(params, i);
            PyObject *g;
            if (THPVariable_CheckExact(p)) {
                const at::Tensor &pt = THPVariable_Unpack(p);
                const at::Tensor &t = pt.unsafeGetTensorImpl()->grad();
                pw[i] = reinterpret_cast<uint64_t>(pt.data_ptr());
                if (t.defined()) {
                    g = THPVariable_Wrap(t);
                    gw[i] = reinterpret_cast<uint64_t>(t.data_ptr());
                    match = match && !t.is_sparse() && t.scalar_type() == want && t.device() == pt.device() &&
                            same_layout(t, pt);
                } else {
                    Py_INCREF(Py_None);
                    g = Py_None;
                    gw[i] = 0;
                    match = false;
                }
            } else {
                g = PyObject_GetAttr(p, g_grad_name);
                match = false;
                if (g && (data_ptr_of(g, &gw[i]) || data_ptr_of(p, &pw[i]))) {
                    Py_DECREF(g);
                    g = nullptr;
                }
            }
            if (!g) {
                Py_DECREF(out);
                Py_DECREF(absent);
                Py_DECREF(gp);
                Py_DECREF(pp);
                return nullptr;
            }
            ab[i] = g == Py_None ? 1 : 0;
            PyList_SET_ITEM(out, i, g);                      /* steals the reference */
        }
    } catch (const std::exception &e) {
        Py_DECREF(out);
        Py_DECREF(absent);
        Py_DECREF(gp);
        Py_DECREF(pp);
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
    return Py_BuildValue("NNNNO", out, absent, gp, pp, match ? Py_True : Py_False);
}

/* bind_diag(buf, states, columns) -> None
 *
 * For every state dict states[j] and (col, key) in ``columns``: states[j][key]
 * = a new 0-d tensor over buf's element 5 * j + col, with a storage of its
 * own that keeps buf's storage alive.  A diagnostic kept from one step is
 * then not rewritten by the next (which writes a new buffer), and a deepcopy
 * of one parameter's state copies only its own elements. */
PyObject *bind_diag(PyObject *, PyObject *args) {
    PyObject *bufobj, *states, *columns;
    if (!PyArg_ParseTuple(args, "OO!O!", &bufobj, &PyList_Type, &states, &PyList_Type, &columns)) return nullptr;
    if (!THPVariable_Check(bufobj)) {
        PyErr_SetString(PyExc_TypeError, "bind_diag: buf must be a tensor");
        return nullptr;
    }
    const Py_ssize_t n = PyList_GET_SIZE(states), nc = PyList_GET_SIZE(columns);
    try {
        const at::Tensor &buf = THPVariable_Unpack(bufobj);
        if (!buf.is_contiguous() || buf.numel() < 5 * n) {
            PyErr_SetString(PyExc_ValueError, "bind_diag: buffer too small or not contiguous");
            return nullptr;
        }
        const c10::Storage keep = buf.storage();
        const auto es = buf.element_size();
        char *base = static_cast<char *>(buf.data_ptr());
        const auto opts = buf.options();
        for (Py_ssize_t j = 0; j < n; ++j) {
            PyObject *st = PyList_GET_ITEM(states, j);
            if (!PyDict_Check(st)) {
                PyErr_SetString(PyExc_TypeError, "bind_diag: state entries must be dicts");
                return nullptr;
            }
            for (Py_ssize_t c = 0; c < nc; ++c) {
                PyObject *ck = PyList_GET_ITEM(columns, c);
                long col;
                PyObject *key;
                if (!PyArg_ParseTuple(ck, "lO", &col, &key)) return nullptr;
                if (col < 0 || col >= 5) {
                    PyErr_SetString(PyExc_ValueError, "bind_diag: column out of range [0, 5)");
                    return nullptr;
                }
                at::Tensor t = at::from_blob(base + es * (5 * j + col), at::IntArrayRef{}, [keep](void *) {}, opts);
                PyObject *w = THPVariable_Wrap(std::move(t));
                if (!w) return nullptr;
                const int rc = PyDict_SetItem(st, key, w);
                Py_DECREF(w);
                if (rc) return nullptr;
            }
        }
    } catch (const std::exception &e) {
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
    Py_RETURN_NONE;
}

PyMethodDef methods[] = {
    {"bind_diag", bind_diag, METH_VARARGS,
     "bind_diag(buf, states, columns): states[j][key] = own-storage 0-d tensor over buf[5 * j + col] "
     "for (col, key) in columns"},
    {"grads_scan", grads_scan, METH_VARARGS,
     "grads_scan(params, bf16) -> (grads, absent, grad_ptrs, param_ptrs, match): grads_of, data_ptrs of the "
     "gradients and of the parameters, and grads_match, in one pass"},
    {"advance_if_same", advance_if_same, METH_VARARGS,
     "advance_if_same(params, grads, states[, param_ptrs[, grad_ptrs]]) -> bool: if params[i].grad is "
     "grads[i] for all i (and params[i] / grads[i] still have the data pointers given as native uint64 bytes), "
     "increment every states[j]['step'] and return True; otherwise change nothing and return False."},
    {"advance_steps", advance_steps, METH_VARARGS,
     "advance_steps(states) -> None: increment every states[j]['step']."},
    {"grads_of", grads_of, METH_VARARGS,
     "grads_of(params) -> (grads, absent): [p.grad for p in params] and a bytes of 1 where grad is None."},
    {"grads_match", grads_match, METH_VARARGS,
     "grads_match(params, grads, bf16) -> bool: every grad is a dense tensor of its param's "
     "device, shape and strides, float32 (bfloat16 when bf16)."},
    {"data_ptrs", data_ptrs, METH_VARARGS,
     "data_ptrs(tensors) -> bytes: each tensor's data_ptr() (0 for None) as native uint64."},
    {"bump_versions", bump_versions, METH_VARARGS,
     "bump_versions(tensors) -> None: increment each tensor's autograd version counter."},
    {"same_params", same_params, METH_VARARGS,
     "same_params(param_groups, flat) -> bool: the groups' params, concatenated, are the objects of flat."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef module = {PyModuleDef_HEAD_INIT, "_hoststep", nullptr, -1, methods, nullptr, nullptr, nullptr, nullptr};

}  // namespace

PyMODINIT_FUNC PyInit__hoststep(void) {
    if (!THPVariableClass) {
        PyErr_SetString(PyExc_ImportError, "adana_amd._hoststep: import torch first");
        return nullptr;
    }
    if (!(g_grad_name = PyUnicode_InternFromString("grad"))) return nullptr;
    if (!(g_step_name = PyUnicode_InternFromString("step"))) return nullptr;
    if (!(g_params_name = PyUnicode_InternFromString("params"))) return nullptr;
    if (!(g_one = PyLong_FromLong(1))) return nullptr;
    return PyModule_Create(&module);
}
