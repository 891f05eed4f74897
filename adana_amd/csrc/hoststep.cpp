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
 *
 * StepTable holds one laid-out plan's rows and does a step's host work in one
 * pass whether or not the gradients are new tensors: every gradient is checked
 * against its parameter and its pointer gathered, the step counters advance
 * and the parameters' version counters are bumped.  For plans of thousands of
 * rows, a few helper threads check and bump contiguous ranges of rows while
 * the calling thread advances the step counters, so the cache misses of a
 * cold walk (right after a backward pass) overlap.  A scan either does all of
 * this or changes nothing.  StepTable also keeps the diagnostics bound in the
 * state dicts, refreshed in place by each step, with any the caller still
 * refers to moved aside first.
 */
#include <torch/csrc/autograd/python_variable.h>
#include <torch/csrc/autograd/variable.h>
#include <ATen/ops/from_blob.h>

#include <Python.h>

#include <c10/core/InferenceMode.h>
#include <pthread.h>
#include <sched.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <exception>
#include <mutex>
#include <new>
#include <thread>
#include <utility>
#include <vector>

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

// Puts states[i]["step"] back to saved[i] for i < saved.size() and releases
// saved (a Python error already set is kept).
template <class State>
void restore_steps(State state, std::vector<PyObject *> &saved) {
    PyObject *et, *ev, *tb;
    PyErr_Fetch(&et, &ev, &tb);
    for (size_t i = 0; i < saved.size(); ++i) {
        if (PyDict_SetItem(state(i), g_step_name, saved[i])) PyErr_Clear();
        Py_DECREF(saved[i]);
    }
    saved.clear();
    PyErr_Restore(et, ev, tb);
}

// states[i]["step"] += 1 for every dict (i < n; state(i) returns it, borrowed);
// tensors stepped together hold equal counts, so the new int of the previous
// entry is reused (ints are immutable) when this entry's old int is equal.
// Returns 0 with the old values in ``saved`` (new references, for a later
// restore_steps); -1 with a Python error set and every dict as it was; or,
// with ints_only, 1 (every dict as it was, no error) as soon as a count is not
// an exact int -- adding to anything else may run Python code.
template <class State>
int advance_states_impl(size_t n, State state, std::vector<PyObject *> &saved, bool ints_only = false) {
    PyObject *prev_v = nullptr, *prev_w = nullptr;
    int rc = 0;
    saved.clear();
    saved.reserve(n);
    for (size_t i = 0; i < n && !rc; ++i) {
        if (i + 16 < n) __builtin_prefetch(state(i + 16), 0, 3);
        if (i + 8 < n && PyDict_Check(state(i + 8))) {
            const char *keys = reinterpret_cast<const char *>(reinterpret_cast<PyDictObject *>(state(i + 8))->ma_keys);
            __builtin_prefetch(keys, 1, 3);
            __builtin_prefetch(keys + 64, 1, 3);
        }
        PyObject *st = state(i);
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
        if (ints_only && !PyLong_CheckExact(v)) {
            rc = 1;
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
        Py_INCREF(v);
        if (PyDict_SetItem(st, g_step_name, prev_w)) {
            Py_DECREF(v);
            rc = -1;
            break;
        }
        saved.push_back(v);
    }
    Py_XDECREF(prev_v);
    Py_XDECREF(prev_w);
    if (rc) restore_steps(state, saved);
    return rc;
}
int advance_states(PyObject *states) {
    std::vector<PyObject *> saved;
    auto state = [states](size_t i) { return PyList_GET_ITEM(states, static_cast<Py_ssize_t>(i)); };
    const int rc = advance_states_impl(static_cast<size_t>(PyList_GET_SIZE(states)), state, saved);
    for (PyObject *o : saved) Py_DECREF(o);
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

/* Prefetch hints for a scan over thousands of tensors.  Each row's check
 * chases PyObject -> TensorImpl -> AutogradMeta -> gradient TensorImpl ->
 * StorageImpl, and its bookkeeping touches the state dict and the version
 * counter: a dozen cache lines per row, scattered over the heap and mostly
 * cold right after a backward pass.  Issued a few rows ahead, in the order
 * the chain resolves, they overlap those misses instead of taking them one
 * after another.  A prefetch never faults, so a stale address costs nothing
 * but the hint. */
inline void prefetch_lines(const void *p, int lines) {
    for (int k = 0; k < lines; ++k) __builtin_prefetch(static_cast<const char *>(p) + 64 * k, 0, 3);
}
static_assert(sizeof(c10::VariableVersion) == sizeof(void *),
              "c10::VariableVersion is expected to hold one pointer (its VersionCounter)");
// The VersionCounter object behind a tensor's version counter (for a hint only).
inline const void *version_counter_object(const at::TensorImpl *t) {
    return *reinterpret_cast<const void *const *>(&t->version_counter());
}
inline at::TensorImpl *impl_of(PyObject *exact_tensor) {
    return THPVariable_Unpack(exact_tensor).unsafeGetTensorImpl();
}
struct ScanPrefetch {
    PyObject *const *params;   // the rows [0, n) of one scan range
    size_t n;
    const at::TensorImpl *grad_ring[8] = {};
    // hints for the rows the scan reaches 16, 12, 8, 4 and 2 rows after row i
    void ahead(size_t i) {
        if (i + 16 < n) __builtin_prefetch(params[i + 16], 0, 3);
        if (i + 12 < n) prefetch_lines(impl_of(params[i + 12]), 3);
        if (i + 8 < n) {
            const at::TensorImpl *t = impl_of(params[i + 8]);
            if (t->autograd_meta()) prefetch_lines(t->autograd_meta(), 2);
            __builtin_prefetch(t->unsafe_storage().unsafeGetStorageImpl(), 0, 3);
            __builtin_prefetch(version_counter_object(t), 1, 3);
        }
        if (i + 4 < n) {
            const at::Tensor &g = impl_of(params[i + 4])->grad();
            const at::TensorImpl *gi = g.defined() ? g.unsafeGetTensorImpl() : nullptr;
            grad_ring[(i + 4) & 7] = gi;
            if (gi) prefetch_lines(gi, 3);
        }
        if (i + 2 < n && i >= 2) {
            const at::TensorImpl *gi = grad_ring[(i + 2) & 7];
            if (gi) __builtin_prefetch(gi->unsafe_storage().unsafeGetStorageImpl(), 0, 3);
        }
    }
};

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

/* ---------------------------------------------------------------------------
 * StepTable: one plan's rows (the stepped parameters, in launch order), their
 * state dicts, the parameters that had no gradient when the plan was built,
 * and the diagnostics bound into the state dicts.
 * ------------------------------------------------------------------------- */
struct TableData {
    std::vector<PyObject *> params, states, inactive;   // strong references
    std::vector<uint64_t> pptr;                          // parameter data pointers the plan holds
    std::vector<uint64_t> last;                          // gradient pointers of the last accepted scan
    std::vector<uint64_t> tmp;                           // this scan's pointers until it is accepted
    std::vector<PyObject *> saved;                       // a scan's old step counts until it is accepted
    bool busy = false;                                   // a scan of this table is running
    std::vector<PyObject *> diag;                        // bound diagnostics, ncols per row (strong)
    std::vector<c10::Storage> dstore;                    // their storages, one reference each (diag_rows)
    std::vector<std::pair<long, PyObject *>> cols;       // (kernel output column, state key), keys strong
    c10::ScalarType want = c10::ScalarType::Float;
};

struct StepTable {
    PyObject_HEAD
    TableData *d;
};

void release_all(std::vector<PyObject *> &v) {
    for (PyObject *o : v) Py_XDECREF(o);
    v.clear();
}

void table_dealloc(PyObject *self) {
    TableData *d = reinterpret_cast<StepTable *>(self)->d;
    if (d) {
        release_all(d->params);
        release_all(d->states);
        release_all(d->inactive);
        release_all(d->diag);
        for (auto &c : d->cols) Py_XDECREF(c.second);
        delete d;
    }
    Py_TYPE(self)->tp_free(self);
}

PyTypeObject StepTableType = {PyVarObject_HEAD_INIT(nullptr, 0)};

int copy_list(PyObject *lst, std::vector<PyObject *> &out) {
    if (!PyList_Check(lst)) {
        PyErr_SetString(PyExc_TypeError, "step_table: lists expected");
        return -1;
    }
    const Py_ssize_t n = PyList_GET_SIZE(lst);
    out.reserve(static_cast<size_t>(n));
    for (Py_ssize_t i = 0; i < n; ++i) {
        PyObject *o = PyList_GET_ITEM(lst, i);
        Py_INCREF(o);
        out.push_back(o);
    }
    return 0;
}

/* step_table(params, states, inactive, bf16) -> StepTable
 *
 * params: the plan's rows (exact torch.Tensor / nn.Parameter objects whose
 * gradients the plan expects at their own layout); states: their state dicts;
 * inactive: every other parameter of the optimizer (no gradient at plan
 * time); bf16: the gradients are bfloat16 (else float32). */
PyObject *step_table(PyObject *, PyObject *args) {
    PyObject *params, *states, *inactive;
    int bf16 = 0;
    if (!PyArg_ParseTuple(args, "O!O!O!p", &PyList_Type, &params, &PyList_Type, &states, &PyList_Type, &inactive,
                          &bf16))
        return nullptr;
    if (PyList_GET_SIZE(params) != PyList_GET_SIZE(states)) {
        PyErr_SetString(PyExc_ValueError, "step_table: one state dict per parameter");
        return nullptr;
    }
    StepTable *t = PyObject_New(StepTable, &StepTableType);
    if (!t) return nullptr;
    t->d = new (std::nothrow) TableData();
    if (!t->d) {
        Py_DECREF(t);
        return PyErr_NoMemory();
    }
    TableData &d = *t->d;
    d.want = bf16 ? c10::ScalarType::BFloat16 : c10::ScalarType::Float;
    if (copy_list(params, d.params) || copy_list(states, d.states) || copy_list(inactive, d.inactive)) {
        Py_DECREF(t);
        return nullptr;
    }
    try {
        d.pptr.resize(d.params.size());
        d.last.assign(d.params.size(), 0);
        d.tmp.assign(d.params.size(), 0);
        for (size_t i = 0; i < d.params.size(); ++i) {
            PyObject *p = d.params[i];
            if (!THPVariable_CheckExact(p) || !PyDict_Check(d.states[i])) {
                PyErr_SetString(PyExc_TypeError, "step_table: rows must be exact tensors with dict states");
                Py_DECREF(t);
                return nullptr;
            }
            d.pptr[i] = reinterpret_cast<uint64_t>(THPVariable_Unpack(p).const_data_ptr());
        }
        for (PyObject *p : d.inactive)
            if (!THPVariable_CheckExact(p)) {
                PyErr_SetString(PyExc_TypeError, "step_table: parameters must be exact tensors");
                Py_DECREF(t);
                return nullptr;
            }
    } catch (const std::exception &e) {
        Py_DECREF(t);
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
    return reinterpret_cast<PyObject *>(t);
}

/* One scan range's checks, rows [lo, hi) of the plan: every row has a dense
 * gradient of the plan's dtype on its parameter's device with its parameter's
 * shape and strides, the parameter keeps the storage the plan holds, and its
 * version counter can be bumped (inference tensors only in inference mode,
 * where the bump is a no-op).  The gradient pointers go to d.tmp; rows whose
 * pointer moved since the last accepted scan widen [*clo, *chi).  false as
 * soon as a row does not fit.  It reads tensors only (no Python API, no
 * reference counts), so helper threads run it while the caller holds the GIL. */
bool check_rows(TableData &d, size_t lo, size_t hi, bool inference, size_t *clo, size_t *chi) {
    ScanPrefetch ahead{d.params.data() + lo, hi - lo};
    for (size_t i = lo; i < hi; ++i) {
        ahead.ahead(i - lo);
        const at::Tensor &pt = THPVariable_Unpack(d.params[i]);
        if (reinterpret_cast<uint64_t>(pt.const_data_ptr()) != d.pptr[i]) return false;
        if (!inference && !pt.unsafeGetTensorImpl()->version_counter().enabled()) return false;
        const at::Tensor &g = pt.unsafeGetTensorImpl()->grad();
        if (!g.defined() || g.is_sparse() || g.scalar_type() != d.want || g.device() != pt.device() ||
            !same_layout(g, pt))
            return false;
        const uint64_t gp = reinterpret_cast<uint64_t>(g.const_data_ptr());
        d.tmp[i] = gp;
        if (gp != d.last[i]) {
            if (i < *clo) *clo = i;
            *chi = i + 1;
        }
    }
    return true;
}

// The bound diagnostics of rows [lo, hi) (flat indices j * ncols + c) that
// something besides the state dict and the table still refers to -- a Python
// reference, or another tensor over the same storage, as a view or detach()
// gives -- go to `held`; those whose state entry no longer is the bound tensor
// (replaced or deleted) to `lost`.  Reads reference counts only (no Python
// API), so helper threads run it while the caller holds the GIL: the caller
// meanwhile rebinds only the step counters of the same dicts, never these
// objects.
void diag_rows(const TableData &d, size_t lo, size_t hi, std::vector<size_t> &held, std::vector<size_t> &lost) {
    const size_t nc = d.cols.size();
    if (d.diag.empty() || nc == 0 || d.dstore.size() != d.diag.size()) return;
    const size_t k0 = lo * nc, k1 = hi * nc;
    // Two cold lines per entry, independent of each other: the object (its
    // reference count) and the storage the table cached at binding (its use
    // count: the bound tensor's reference and the table's, more when a view or
    // detach() shares it).  Hints 16 entries ahead.
    for (size_t k = k0; k < k1; ++k) {
        if (k + 16 < k1) {
            __builtin_prefetch(d.diag[k + 16], 0, 3);
            __builtin_prefetch(d.dstore[k + 16].unsafeGetStorageImpl(), 0, 3);
        }
        const Py_ssize_t rc = Py_REFCNT(d.diag[k]);
        if (rc > 2 || c10::raw::intrusive_ptr::use_count(d.dstore[k].unsafeGetStorageImpl()) > 2) held.push_back(k);
        else if (rc < 2) lost.push_back(k);
    }
}

// Bumps the version counters of rows [lo, hi), whose parameters the launch
// that follows updates in place (check_rows has passed them).
void bump_rows(TableData &d, size_t lo, size_t hi) {
    for (size_t i = lo; i < hi; ++i) {
        if (i + 8 < hi) __builtin_prefetch(version_counter_object(impl_of(d.params[i + 8])), 1, 3);
        at::TensorImpl *t = impl_of(d.params[i]);
        if (t->version_counter().enabled()) t->bump_version();
    }
}

/* Helper threads for the scans of long plans (thousands of rows).  Each
 * helper checks and then bumps one contiguous range of rows, so the cache
 * misses of the ranges overlap, while the calling thread, which holds the
 * GIL, advances the step counters.  Helpers never call into Python or touch
 * reference counts, and a scan waits for every helper it started before it
 * returns.  After fork() the child starts a pool of its own. */
constexpr int kMaxHelpers = 8;
constexpr size_t kParallelRows = 2048;   // shorter plans are scanned by the calling thread
constexpr size_t kMinRowsPerHelper = 1024;

struct ScanPool {
    std::mutex mu;
    std::condition_variable cv;
    uint64_t gen = 0;                     // moved (under mu) to start a job
    int started = 0;                      // helper threads running
    // the job, written before gen moves
    TableData *d = nullptr;
    int parts = 0;
    bool inference = false;
    struct Part {
        size_t lo, hi, clo, chi;
        bool ok;
    } part[kMaxHelpers];
    bool diag = false;                    // also classify the rows' bound diagnostics (diag_rows)
    bool diag_only = false;               // a diag_check job: no checks, no decision, no bumps
    std::vector<size_t> held[kMaxHelpers], lost[kMaxHelpers];
    std::atomic<int> checked{0}, finished{0};
    std::atomic<int> decision{0};         // 0 pending, 1 bump the versions, 2 stop
};
ScanPool *g_pool = nullptr;
bool g_pool_busy = false;   // a scan is using the helpers (the GIL guards this flag)
int g_helpers = 3;          // set at import by default_helpers()

// Helpers a scan uses by default: the CPUs this process may run on, less two
// (the calling thread and one to spare), at most kMaxHelpers.  More helpers
// overlap more of the cold rows' cache misses: on MI355X's host (16 CPUs),
// 10,000 rows after a backward pass, opt.step()'s host time was 0.69 ms with
// 3 helpers, 0.60 ms with 6 and 0.57 ms with 8 (medians of 3 x 20 steps).
int default_helpers() {
    cpu_set_t set;
    CPU_ZERO(&set);
    int cpus = 0;
    if (sched_getaffinity(0, sizeof set, &set) == 0) cpus = CPU_COUNT(&set);
    if (cpus <= 0) cpus = static_cast<int>(std::thread::hardware_concurrency());
    return std::clamp(cpus - 2, 0, kMaxHelpers);
}

inline void cpu_relax() { __builtin_ia32_pause(); }

void helper_main(ScanPool *P, int id) {
    uint64_t seen = 0;
    for (;;) {
        {
            std::unique_lock<std::mutex> lk(P->mu);
            P->cv.wait(lk, [&] { return P->gen != seen; });
            seen = P->gen;
            if (id >= P->parts) continue;
        }
        ScanPool::Part &r = P->part[id];
        if (P->diag_only) {
            try {
                diag_rows(*P->d, r.lo, r.hi, P->held[id], P->lost[id]);
                r.ok = true;
            } catch (...) {
                r.ok = false;
            }
            P->finished.fetch_add(1, std::memory_order_acq_rel);
            continue;
        }
        bool ok;
        try {
            ok = check_rows(*P->d, r.lo, r.hi, P->inference, &r.clo, &r.chi);
            // the diagnostics' check overlaps the caller's step counters
            if (ok && P->diag) diag_rows(*P->d, r.lo, r.hi, P->held[id], P->lost[id]);
        } catch (...) {
            ok = false;   // the caller's general path raises the precise error
        }
        r.ok = ok;
        P->checked.fetch_add(1, std::memory_order_acq_rel);
        int dec;
        while ((dec = P->decision.load(std::memory_order_acquire)) == 0) cpu_relax();
        if (dec == 1) bump_rows(*P->d, r.lo, r.hi);
        P->finished.fetch_add(1, std::memory_order_acq_rel);
    }
}

void pool_after_fork_child() { g_pool = nullptr; }

// The pool with at least `want` helpers running (fewer if threads cannot be started).
ScanPool *scan_pool(int want) {
    if (!g_pool) {
        static bool registered = false;
        if (!registered) {
            pthread_atfork(nullptr, nullptr, pool_after_fork_child);
            registered = true;
        }
        g_pool = new ScanPool();   // lives until the process ends, like its threads
    }
    ScanPool *P = g_pool;
    while (P->started < want) {
        try {
            std::thread(helper_main, P, P->started).detach();
        } catch (const std::exception &) {
            break;
        }
        ++P->started;
    }
    return P;
}

/* The scan's checks and version bumps on `parts` helpers while this thread
 * advances the step counters.  1: done; 0: a row does not fit (nothing
 * modified); -1: error, with a Python error set (nothing modified). */
int scan_parallel(TableData &d, ScanPool &P, int parts, size_t *lo, size_t *hi, bool diag, bool *python_ran,
                  std::vector<size_t> *held, std::vector<size_t> *lost) {
    const size_t n = d.params.size();
    P.d = &d;
    P.parts = parts;
    P.inference = c10::InferenceMode::is_enabled();
    P.diag = diag;
    P.diag_only = false;
    for (int k = 0; k < parts; ++k) {
        P.part[k] = {n * k / parts, n * (k + 1) / parts, n, 0, false};
        P.held[k].clear();
        P.lost[k].clear();
    }
    P.checked.store(0);
    P.finished.store(0);
    P.decision.store(0);
    {
        std::lock_guard<std::mutex> lk(P.mu);
        ++P.gen;
    }
    P.cv.notify_all();
    // From here on the helpers wait for a decision: however this function
    // leaves (an exception included), they get one and finish before it returns.
    struct Settle {
        ScanPool &P;
        int parts;
        bool done = false;
        ~Settle() {
            if (done) return;
            P.decision.store(2, std::memory_order_release);
            while (P.finished.load(std::memory_order_acquire) < parts) cpu_relax();
        }
    } settle{P, parts};
    // Exact-int counters advance now and are put back if a row does not fit;
    // any other kind of counter waits for the checks (adding to it may run
    // Python code, which must not run while the helpers read the tensors).
    auto state = [&d](size_t i) { return d.states[i]; };
    int arc = advance_states_impl(n, state, d.saved, true);
    while (P.checked.load(std::memory_order_acquire) < parts) cpu_relax();
    bool fits = true;
    for (int k = 0; k < parts; ++k) fits = fits && P.part[k].ok;
    if (fits && arc == 1) {
        arc = advance_states_impl(n, state, d.saved);
        *python_ran = true;
    }
    const bool go = fits && arc == 0;
    P.decision.store(go ? 1 : 2, std::memory_order_release);
    while (P.finished.load(std::memory_order_acquire) < parts) cpu_relax();
    settle.done = true;
    if (!go) {
        if (arc == 0) restore_steps(state, d.saved);
        return arc < 0 ? -1 : 0;
    }
    for (int k = 0; k < parts; ++k) {
        if (P.part[k].clo < *lo) *lo = P.part[k].clo;
        if (P.part[k].chi > *hi) *hi = P.part[k].chi;
    }
    if (held && lost) {
        for (int k = 0; k < parts; ++k) {
            held->insert(held->end(), P.held[k].begin(), P.held[k].end());
            lost->insert(lost->end(), P.lost[k].begin(), P.lost[k].end());
        }
    }
    return 1;
}

/* The bound diagnostics' check (diag_rows) of every row, on `parts` helpers:
 * their held and lost indices, in row order. */
void diag_parallel(TableData &d, ScanPool &P, int parts, std::vector<size_t> &held, std::vector<size_t> &lost) {
    const size_t n = d.params.size();
    P.d = &d;
    P.parts = parts;
    P.diag = true;
    P.diag_only = true;
    for (int k = 0; k < parts; ++k) {
        P.part[k] = {n * k / parts, n * (k + 1) / parts, n, 0, false};
        P.held[k].clear();
        P.lost[k].clear();
    }
    P.checked.store(0);
    P.finished.store(0);
    P.decision.store(0);
    {
        std::lock_guard<std::mutex> lk(P.mu);
        ++P.gen;
    }
    P.cv.notify_all();
    while (P.finished.load(std::memory_order_acquire) < parts) cpu_relax();
    bool ok = true;
    for (int k = 0; k < parts; ++k) ok = ok && P.part[k].ok;
    if (!ok) throw std::bad_alloc();
    for (int k = 0; k < parts; ++k) {
        held.insert(held.end(), P.held[k].begin(), P.held[k].end());
        lost.insert(lost.end(), P.lost[k].begin(), P.lost[k].end());
    }
}

// The helpers for a pass over the n rows of a plan (parts >= 2), or nullptr
// (a short plan, no helpers configured, or the helpers already serving a scan
// further up the stack).
ScanPool *pool_for(size_t n, int *parts) {
    *parts = 0;
    if (n >= kParallelRows && g_helpers > 0)
        *parts = static_cast<int>(std::min<size_t>(static_cast<size_t>(g_helpers), n / kMinRowsPerHelper));
    ScanPool *pool = (*parts >= 2 && !g_pool_busy) ? scan_pool(*parts) : nullptr;
    if (pool) *parts = std::min(*parts, pool->started);
    return (pool && *parts >= 2) ? pool : nullptr;
}

// Python list of the size_t values of v (new reference), or nullptr with an error set.
PyObject *index_list(const std::vector<size_t> &v) {
    PyObject *l = PyList_New(static_cast<Py_ssize_t>(v.size()));
    if (!l) return nullptr;
    for (size_t i = 0; i < v.size(); ++i) {
        PyObject *ix = PyLong_FromSize_t(v[i]);
        if (!ix) {
            Py_DECREF(l);
            return nullptr;
        }
        PyList_SET_ITEM(l, static_cast<Py_ssize_t>(i), ix);
    }
    return l;
}

/* StepTable.scan(out_address[, check_diag]) -> (lo, hi[, held, lost]) or None
 *
 * One step's host bookkeeping for the plan (src/optim/adana.py:184-197,
 * src/optim/dana_star_mk4.py:243-262) when the plan still fits: every row has
 * a gradient that is a dense tensor of its parameter's device, shape, strides
 * and the plan's dtype, every parameter keeps the storage the plan holds, and
 * no inactive parameter has gained a gradient.  Then the gradients' data
 * pointers are written to the uint64 array at out_address (one per row),
 * every state's "step" goes up by one, every parameter's version counter is
 * bumped (the launch that follows updates them in place), and the rows
 * [lo, hi) whose gradient pointer differs from the last accepted scan are
 * returned (lo == hi: none moved).  None, with nothing modified, when the
 * plan does not fit: the caller takes its general path (which also raises
 * the precise error for a bad gradient).  Plans of thousands of rows are
 * checked by helper threads (scan_threads).  With check_diag the same pass
 * also takes diag_check()'s lists: the helpers classify their rows' bound
 * diagnostics while the calling thread advances the step counters. */
PyObject *table_scan(PyObject *self, PyObject *args) {
    TableData &d = *reinterpret_cast<StepTable *>(self)->d;
    PyObject *addr_obj;
    int check_diag = 0;
    if (!PyArg_ParseTuple(args, "O|p", &addr_obj, &check_diag)) return nullptr;
    const unsigned long long addr = PyLong_AsUnsignedLongLong(addr_obj);
    if (PyErr_Occurred()) return nullptr;
    uint64_t *out = reinterpret_cast<uint64_t *>(static_cast<uintptr_t>(addr));
    const size_t n = d.params.size();
    if (n && !out) {
        PyErr_SetString(PyExc_ValueError, "StepTable.scan: null output array");
        return nullptr;
    }
    try {
        for (PyObject *p : d.inactive)
            if (THPVariable_Unpack(p).unsafeGetTensorImpl()->grad().defined()) Py_RETURN_NONE;
        size_t lo = n, hi = 0;
        // Python code run by a step counter that is not an int (its __add__) may
        // re-enter: a scan of this table then takes the general path, and a scan
        // of another table keeps off the helpers while they serve this one.
        if (d.busy) Py_RETURN_NONE;
        int parts = 0;
        ScanPool *pool = pool_for(n, &parts);
        struct Busy {          // set for the scan, cleared on every way out
            bool &table, *pool;
            ~Busy() {
                table = false;
                if (pool) *pool = false;
            }
        } busy{d.busy, pool ? &g_pool_busy : nullptr};
        d.busy = true;
        std::vector<size_t> held, lost;
        bool python_ran = false;
        if (busy.pool) {
            g_pool_busy = true;
            const int rc = scan_parallel(d, *pool, parts, &lo, &hi, check_diag, &python_ran, &held, &lost);
            if (rc < 0) return nullptr;
            if (rc == 0) Py_RETURN_NONE;
        } else {
            if (!check_rows(d, 0, n, c10::InferenceMode::is_enabled(), &lo, &hi)) Py_RETURN_NONE;
            if (check_diag) diag_rows(d, 0, n, held, lost);          // nothing modified yet
            auto state = [&d](size_t i) { return d.states[i]; };
            int arc = advance_states_impl(n, state, d.saved, true);
            if (arc == 1) {
                arc = advance_states_impl(n, state, d.saved);
                python_ran = true;
            }
            if (arc) return nullptr;
            bump_rows(d, 0, n);
        }
        bool diag_known = true;
        if (check_diag && python_ran) {
            // a counter's Python code ran after the check and may have touched
            // the states: check again (None on failure: the caller checks itself)
            try {
                held.clear();
                lost.clear();
                diag_rows(d, 0, n, held, lost);
            } catch (const std::exception &) {
                diag_known = false;
            }
        }

        for (PyObject *o : d.saved) Py_DECREF(o);
        d.saved.clear();
        for (size_t i = 0; i < n; ++i) out[i] = d.tmp[i];
        for (size_t i = lo; i < hi; ++i) d.last[i] = d.tmp[i];
        if (lo > hi) lo = hi = 0;
        if (!check_diag) return Py_BuildValue("nn", static_cast<Py_ssize_t>(lo), static_cast<Py_ssize_t>(hi));
        if (!diag_known)
            return Py_BuildValue("nnOO", static_cast<Py_ssize_t>(lo), static_cast<Py_ssize_t>(hi), Py_None, Py_None);
        PyObject *h = index_list(held);
        if (!h) return nullptr;
        PyObject *l = index_list(lost);
        if (!l) {
            Py_DECREF(h);
            return nullptr;
        }
        return Py_BuildValue("nnNN", static_cast<Py_ssize_t>(lo), static_cast<Py_ssize_t>(hi), h, l);
    } catch (const std::exception &e) {
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
}

/* scan_threads([k]) -> int: how many helper threads a scan of a plan of
 * thousands of rows uses (k given: set it, 0 to 8; 0 scans on the calling
 * thread alone).  Returns the value before the call. */
PyObject *scan_threads(PyObject *, PyObject *args) {
    int k = -1;
    if (!PyArg_ParseTuple(args, "|i", &k)) return nullptr;
    const int before = g_helpers;
    if (k >= 0) {
        if (k > kMaxHelpers) {
            PyErr_Format(PyExc_ValueError, "scan_threads: at most %d helper threads", kMaxHelpers);
            return nullptr;
        }
        g_helpers = k;
    } else if (PyTuple_GET_SIZE(args)) {
        PyErr_SetString(PyExc_ValueError, "scan_threads: k must be >= 0");
        return nullptr;
    }
    return PyLong_FromLong(before);
}

/* StepTable.forget() -> None: the next scan reports every row as moved (the
 * device copy of the gradient pointers must be written in full again). */
PyObject *table_forget(PyObject *self, PyObject *) {
    TableData &d = *reinterpret_cast<StepTable *>(self)->d;
    d.last.assign(d.last.size(), 0);
    Py_RETURN_NONE;
}

/* StepTable.grads_are(grads) -> bool: row i's current gradient is grads[i]
 * (the same tensor) for every row. */
PyObject *table_grads_are(PyObject *self, PyObject *arg) {
    TableData &d = *reinterpret_cast<StepTable *>(self)->d;
    if (!PyList_Check(arg) || static_cast<size_t>(PyList_GET_SIZE(arg)) != d.params.size()) Py_RETURN_FALSE;
    for (size_t i = 0; i < d.params.size(); ++i) {
        PyObject *g = PyList_GET_ITEM(arg, static_cast<Py_ssize_t>(i));
        if (!THPVariable_Check(g)) Py_RETURN_FALSE;
        const at::Tensor &cur = THPVariable_Unpack(d.params[i]).unsafeGetTensorImpl()->grad();
        if (!cur.defined() || cur.unsafeGetTensorImpl() != THPVariable_Unpack(g).unsafeGetTensorImpl())
            Py_RETURN_FALSE;
    }
    Py_RETURN_TRUE;
}

/* A new 0-d tensor over element k of buf with a storage of its own that keeps
 * buf's storage alive (a deepcopy of it copies only its own bytes). */
PyObject *diag_tensor(const at::Tensor &buf, int64_t k) {
    const c10::Storage keep = buf.storage();
    char *base = static_cast<char *>(buf.data_ptr());
    at::Tensor t = at::from_blob(base + buf.element_size() * k, at::IntArrayRef{}, [keep](void *) {}, buf.options());
    return THPVariable_Wrap(std::move(t));
}

/* StepTable.diag_bind(buf, columns) -> None
 *
 * Row j's state[key] = a new 0-d tensor over buf[len(columns)_all * j + col]
 * for every (col, key) in columns (buf holds 5 values per row, the kernel's
 * output), kept by the table for diag_check / diag_rehome. */
PyObject *table_diag_bind(PyObject *self, PyObject *args) {
    TableData &d = *reinterpret_cast<StepTable *>(self)->d;
    PyObject *bufobj, *columns;
    if (!PyArg_ParseTuple(args, "OO!", &bufobj, &PyList_Type, &columns)) return nullptr;
    if (!THPVariable_Check(bufobj)) {
        PyErr_SetString(PyExc_TypeError, "StepTable.diag_bind: buf must be a tensor");
        return nullptr;
    }
    try {
        const at::Tensor &buf = THPVariable_Unpack(bufobj);
        const size_t n = d.params.size();
        if (!buf.is_contiguous() || buf.numel() < static_cast<int64_t>(5 * n)) {
            PyErr_SetString(PyExc_ValueError, "StepTable.diag_bind: buffer too small or not contiguous");
            return nullptr;
        }
        for (auto &c : d.cols) Py_XDECREF(c.second);
        d.cols.clear();
        release_all(d.diag);
        d.dstore.clear();
        const Py_ssize_t nc = PyList_GET_SIZE(columns);
        for (Py_ssize_t c = 0; c < nc; ++c) {
            long col;
            PyObject *key;
            if (!PyArg_ParseTuple(PyList_GET_ITEM(columns, c), "lO", &col, &key)) return nullptr;
            if (col < 0 || col >= 5) {
                PyErr_SetString(PyExc_ValueError, "StepTable.diag_bind: column out of range [0, 5)");
                return nullptr;
            }
            Py_INCREF(key);
            d.cols.emplace_back(col, key);
        }
        d.diag.assign(n * d.cols.size(), nullptr);
        d.dstore.assign(n * d.cols.size(), c10::Storage());
        for (size_t j = 0; j < n; ++j)
            for (size_t c = 0; c < d.cols.size(); ++c) {
                PyObject *w = diag_tensor(buf, static_cast<int64_t>(5 * j) + d.cols[c].first);
                if (!w) return nullptr;
                if (PyDict_SetItem(d.states[j], d.cols[c].second, w)) {
                    Py_DECREF(w);
                    return nullptr;
                }
                d.diag[j * d.cols.size() + c] = w;                   // the table's reference
                d.dstore[j * d.cols.size() + c] = THPVariable_Unpack(w).storage();
            }
    } catch (const std::exception &e) {
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
    Py_RETURN_NONE;
}

/* StepTable.diag_check() -> (held, lost)
 *
 * Before a step rewrites the diagnostics buffer in place: the bound
 * diagnostics that something besides the state dict and the table still
 * refers to (a Python reference, or another tensor over its storage, as a
 * view or detach() gives) -- `held`, flat indices j * ncols + c -- and those
 * whose state entry no longer is the bound tensor (replaced or deleted) --
 * `lost`. */
PyObject *table_diag_check(PyObject *self, PyObject *) {
    TableData &d = *reinterpret_cast<StepTable *>(self)->d;
    try {
        std::vector<size_t> held, lost;
        int parts = 0;
        ScanPool *pool = d.busy ? nullptr : pool_for(d.params.size(), &parts);
        if (pool) {
            g_pool_busy = true;
            struct Release {
                ~Release() { g_pool_busy = false; }
            } release;
            diag_parallel(d, *pool, parts, held, lost);
        } else {
            diag_rows(d, 0, d.params.size(), held, lost);
        }
        PyObject *h = index_list(held);
        if (!h) return nullptr;
        PyObject *l = index_list(lost);
        if (!l) {
            Py_DECREF(h);
            return nullptr;
        }
        return Py_BuildValue("NN", h, l);
    } catch (const std::exception &e) {
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
}

void drop_storage(void *ctx) { delete static_cast<c10::Storage *>(ctx); }

/* StepTable.diag_rehome(held, copy, lost, buf) -> None
 *
 * held[i] (a flat index from diag_check) keeps its value: its storage (and so
 * every tensor sharing it) now reads element i of `copy`, which the caller
 * has filled with the current values on the launch's stream.  Then every
 * held and lost entry gets a new 0-d tensor over its element of `buf`, bound
 * in its state dict and kept by the table. */
PyObject *table_diag_rehome(PyObject *self, PyObject *args) {
    TableData &d = *reinterpret_cast<StepTable *>(self)->d;
    PyObject *held, *copyobj, *lost, *bufobj;
    if (!PyArg_ParseTuple(args, "O!OO!O", &PyList_Type, &held, &copyobj, &PyList_Type, &lost, &bufobj)) return nullptr;
    if (!THPVariable_Check(copyobj) || !THPVariable_Check(bufobj)) {
        PyErr_SetString(PyExc_TypeError, "StepTable.diag_rehome: tensors expected");
        return nullptr;
    }
    const size_t nc = d.cols.size();
    try {
        const at::Tensor &copy = THPVariable_Unpack(copyobj);
        const at::Tensor &buf = THPVariable_Unpack(bufobj);
        const Py_ssize_t nh = PyList_GET_SIZE(held);
        if (!copy.is_contiguous() || copy.numel() < nh || copy.scalar_type() != buf.scalar_type()) {
            PyErr_SetString(PyExc_ValueError, "StepTable.diag_rehome: copy does not match the held entries");
            return nullptr;
        }
        char *cbase = static_cast<char *>(copy.data_ptr());
        const int64_t es = copy.element_size();
        for (int pass = 0; pass < 2; ++pass) {
            PyObject *lst = pass == 0 ? held : lost;
            for (Py_ssize_t i = 0; i < PyList_GET_SIZE(lst); ++i) {
                const size_t k = PyLong_AsSize_t(PyList_GET_ITEM(lst, i));
                if (PyErr_Occurred()) return nullptr;
                if (k >= d.diag.size()) {
                    PyErr_SetString(PyExc_IndexError, "StepTable.diag_rehome: index out of range");
                    return nullptr;
                }
                if (pass == 0) {
                    c10::StorageImpl *si =
                        THPVariable_Unpack(d.diag[k]).unsafeGetTensorImpl()->unsafe_storage().unsafeGetStorageImpl();
                    si->set_data_ptr_noswap(c10::DataPtr(cbase + es * i, new c10::Storage(copy.storage()),
                                                         &drop_storage, copy.device()));
                }
                const size_t j = k / nc, c = k % nc;
                PyObject *w = diag_tensor(buf, static_cast<int64_t>(5 * j) + d.cols[c].first);
                if (!w) return nullptr;
                if (PyDict_SetItem(d.states[j], d.cols[c].second, w)) {
                    Py_DECREF(w);
                    return nullptr;
                }
                Py_DECREF(d.diag[k]);
                d.diag[k] = w;
                if (k < d.dstore.size()) d.dstore[k] = THPVariable_Unpack(w).storage();
            }
        }
    } catch (const std::exception &e) {
        PyErr_SetString(PyExc_RuntimeError, e.what());
        return nullptr;
    }
    Py_RETURN_NONE;
}

PyMethodDef table_methods[] = {
    {"scan", table_scan, METH_VARARGS,
     "scan(out_address[, check_diag]) -> (lo, hi) or None: check every row's gradient, write the gradient "
     "pointers, advance the step counters and bump the parameters' versions; the rows whose pointer moved, or "
     "None (nothing done).  With check_diag: (lo, hi, held, lost), diag_check()'s lists taken in the same pass "
     "(None, None if they could not be)"},
    {"forget", table_forget, METH_NOARGS, "forget() -> None: the next scan reports every row as moved"},
    {"grads_are", table_grads_are, METH_O, "grads_are(grads) -> bool: row i's gradient is grads[i] for every row"},
    {"diag_bind", table_diag_bind, METH_VARARGS,
     "diag_bind(buf, columns) -> None: bind a new 0-d tensor over buf[5 * j + col] as state[key] of every row"},
    {"diag_check", table_diag_check, METH_NOARGS,
     "diag_check() -> (held, lost): bound diagnostics still referred to elsewhere, and those no longer bound"},
    {"diag_rehome", table_diag_rehome, METH_VARARGS,
     "diag_rehome(held, copy, lost, buf) -> None: held entries read copy[i] from now on; held and lost entries "
     "are bound anew over buf"},
    {nullptr, nullptr, 0, nullptr},
};

PyMethodDef methods[] = {
    {"step_table", step_table, METH_VARARGS,
     "step_table(params, states, inactive, bf16) -> StepTable: the plan's rows, their state dicts, the other "
     "parameters (no gradient at plan time) and the gradients' dtype"},
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
    {"scan_threads", scan_threads, METH_VARARGS,
     "scan_threads([k]) -> int: helper threads for the scans of plans of thousands of rows (k given: set it, "
     "0 to 8; 0 = the calling thread alone); returns the previous value."},
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
    g_helpers = default_helpers();
    StepTableType.tp_name = "adana_amd._hoststep.StepTable";
    StepTableType.tp_basicsize = sizeof(StepTable);
    StepTableType.tp_dealloc = table_dealloc;
    StepTableType.tp_flags = Py_TPFLAGS_DEFAULT;
    StepTableType.tp_doc = "One laid-out plan's rows: the step's per-tensor host work in one pass";
    StepTableType.tp_methods = table_methods;
    if (PyType_Ready(&StepTableType) < 0) return nullptr;
    PyObject *m = PyModule_Create(&module);
    if (!m) return nullptr;
    Py_INCREF(&StepTableType);
    if (PyModule_AddObject(m, "StepTable", reinterpret_cast<PyObject *>(&StepTableType)) < 0) {
        Py_DECREF(&StepTableType);
        Py_DECREF(m);
        return nullptr;
    }
    return m;
}
