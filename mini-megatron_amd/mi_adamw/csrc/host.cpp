// host.cpp -- the steady-state host work of FusedAdamW.step(), in C++.
//
// mini-megatron's loop calls zero_grad() (which frees every gradient) and step() once
// per iteration (main.py:204,209).  After the first step the launch tables stay valid
// except for the gradient pointers, so each step only has to
//   1. read every parameter's gradient and check it (present, dense, contiguous),
//   2. check that nothing the tables encode changed: the parameter's storage, its state
//      dict entries (step view, exp_avg, exp_avg_sq, max_exp_avg_sq) and their storage,
//      and that every param group still has one step count,
//   3. write the moved gradient pointers into the device table (mi_adamw_set_grads) and
//      advance the step counts,
//   4. enqueue the norm pass and the update.
// Done in Python this is a few attribute reads and method calls per parameter
// (~1 us each, several times that with cold caches after a forward/backward).  Here it
// is one pass over the borrowed PyObjects and their at::Tensor handles.
//
// Nothing is changed before every check has passed: a failed check returns FALLBACK
// and FusedAdamW takes its general Python path for that step (first steps, parameters
// without gradients, replaced state, another stream, ...).
//
// Module _host (CPython extension, built against the installed torch):
//   bind(addresses)                     function pointers of libmi_adamw (ctypes)
//   plan(...) -> capsule                one launch's bookkeeping (see plan_new)
//   prepare(plan, stream) -> int        steps 1-3: READY, READY_MOVED, FALLBACK or ERROR
//   last_error(plan) -> int             the library's code behind the last ERROR
//   norm(plan, stream, d_norm) -> int   mi_adamw_grad_norm* (or sumsq + finalize)
//   update(plan, stream, hypers, n) -> int   mi_adamw_step*_prescaled, or with the
//                                       fused=True chain mi_adamw_step*_fused_chain
//   sync_versions(plan, dict)           dict[id(p)] = (p._version, p.data_ptr())

#include <Python.h>

#include <ATen/core/Tensor.h>
#include <torch/csrc/autograd/python_variable.h>

#include <cstdint>
#include <cstring>
#include <exception>
#include <vector>

#include "mi_adamw.h"

namespace {

// prepare()'s statuses.  A library error is reported as kError, with the library's own
// code (a negative MI_ADAMW_E_* or a positive hipError_t) kept in Plan::last_error, so
// that no error code can read as one of the other statuses.
constexpr int kReady = 0;
constexpr int kFallback = 1;
constexpr int kReadyMoved = 2;
constexpr int kError = 3;

// Entry points of libmi_adamw, bound once from the ctypes-loaded library so that both
// paths call the same instance.
struct Api {
    int (*set_grads)(mi_adamw_tensor*, int32_t, int32_t, const int32_t*, const uint64_t*,
                     const uint8_t*, void*) = nullptr;
    int (*grad_norm)(const mi_adamw_tensor*, const mi_adamw_chunk*, int64_t, int64_t, float,
                     double*, float*, float*, void*) = nullptr;
    int (*grad_norm_flat)(const float*, int64_t, int64_t, float, double*, float*, float*,
                          void*) = nullptr;
    int (*grad_sumsq)(const mi_adamw_tensor*, const mi_adamw_chunk*, int64_t, int64_t, float,
                      double*, double*, void*) = nullptr;
    int (*grad_sumsq_flat)(const float*, int64_t, int64_t, float, double*, double*,
                           void*) = nullptr;
    int (*norm_from_sumsq)(const double*, int32_t, float, float*, float*, void*) = nullptr;
    int (*step_prescaled)(const mi_adamw_tensor*, const mi_adamw_chunk*, int64_t, int64_t,
                          const mi_adamw_hyper*, int32_t, const float*, float, int32_t, int32_t,
                          int32_t, void*) = nullptr;
    int (*step_flat_prescaled)(const mi_adamw_tensor*, const mi_adamw_hyper*, const float*,
                               float, int64_t, int32_t, int32_t, int32_t, void*) = nullptr;
    int (*step_fused_chain)(const mi_adamw_tensor*, const mi_adamw_chunk*, int64_t, int64_t,
                            const mi_adamw_fused_hyper*, int32_t, const float*, const int32_t*,
                            const float*, float, int32_t, int32_t, int32_t, void*) = nullptr;
    int (*step_flat_fused_chain)(const mi_adamw_tensor*, const mi_adamw_fused_hyper*,
                                 const float*, float, int64_t, int32_t, int32_t, int32_t,
                                 void*) = nullptr;
};
Api g_api;
bool g_bound = false;

// Row of an entry whose gradient is not in any table row (an empty tensor) or whose
// gradient must stay where it is (a view of the flat gradient buffer).
constexpr int32_t kNoRow = -1;
constexpr int32_t kFixed = -2;

struct Entry {
    PyObject* p = nullptr;      // the parameter (owned reference)
    PyObject* st = nullptr;     // its state dict (owned)
    PyObject* obj[4] = {};      // state["step"], exp_avg, exp_avg_sq, max_exp_avg_sq (owned)
    uint64_t ptr[4] = {};       // data pointers of p, exp_avg, exp_avg_sq, max_exp_avg_sq
    uint64_t grad = 0;          // gradient pointer the device table holds
    int64_t numel = 0;          // the parameter's element count when the row was built
    int32_t row = kNoRow;       // table row to patch, or kNoRow / kFixed
    int32_t slot = 0;           // index into the step buffer
    int32_t hyper = 0;          // hyperparameter set (one per param group)
    uint8_t rest = 0;           // the row's other pointers are aligned for the vector path
};

struct Plan {
    std::vector<Entry> e;
    int n_state = 3;                 // state keys checked: step, exp_avg, exp_avg_sq (+ max)
    PyObject* keys[4] = {};          // interned key strings (owned)
    PyObject* keep = nullptr;        // tuple of objects whose memory the plan points into
    float* steps = nullptr;          // the CPU step buffer (fp32)
    int64_t n_steps = 0;
    double* hyper_steps = nullptr;   // out: the new step count of each hyperparameter set
    int32_t n_hyper = 0;
    // the launch
    bool tables = false;
    mi_adamw_tensor flat_row{};      // the single row of a table-free launch
    mi_adamw_tensor* d_rows = nullptr;
    const mi_adamw_chunk* d_chunks = nullptr;
    uint8_t* host_rows = nullptr;    // the host copy of the rows (64 B each), kept in step
    int64_t n_chunks = 0;
    int32_t n_rows = 0;
    int32_t flat_hyper = 0;
    int64_t chunk_elems = 0;
    int32_t max_blocks = 0, state_code = 0, flags = 0;
    bool clip = false;
    bool fused_chain = false;        // the hyperparameter sets are mi_adamw_fused_hyper
    float max_norm = 0.0f, prescale = 1.0f;
    double* partials = nullptr;
    float* coef = nullptr;
    double* sumsq = nullptr;
    uint64_t stream = 0;             // the stream the tables were last used on
    int last_error = 0;              // library code of prepare()'s last kError
    // scratch of prepare()
    std::vector<int32_t> prow;
    std::vector<uint64_t> pgrad;
    std::vector<uint8_t> pvec;
    std::vector<uint64_t> newgrad;
};

void plan_free(PyObject* capsule) {
    Plan* pl = static_cast<Plan*>(PyCapsule_GetPointer(capsule, "mi_adamw._host.Plan"));
    if (!pl) return;
    for (Entry& en : pl->e) {
        Py_XDECREF(en.p);
        Py_XDECREF(en.st);
        for (PyObject* o : en.obj) Py_XDECREF(o);
    }
    for (PyObject* k : pl->keys) Py_XDECREF(k);
    Py_XDECREF(pl->keep);
    delete pl;
}

Plan* get_plan(PyObject* capsule) {
    return static_cast<Plan*>(PyCapsule_GetPointer(capsule, "mi_adamw._host.Plan"));
}

uint64_t tensor_ptr(PyObject* obj) {
    return reinterpret_cast<uint64_t>(THPVariable_Unpack(obj).data_ptr());
}

bool is_tensor(PyObject* obj) { return obj && THPVariable_Check(obj); }

// ---------------------------------------------------------------------------

PyObject* py_bind(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
    constexpr int kN = 10;
    if (nargs != kN) {
        PyErr_SetString(PyExc_TypeError, "bind: 10 function addresses");
        return nullptr;
    }
    void* a[kN];
    for (int i = 0; i < kN; ++i) {
        a[i] = PyLong_AsVoidPtr(args[i]);
        if (!a[i]) {
            if (!PyErr_Occurred()) PyErr_SetString(PyExc_ValueError, "bind: null address");
            return nullptr;
        }
    }
    std::memcpy(&g_api.set_grads, &a[0], sizeof(void*));
    std::memcpy(&g_api.grad_norm, &a[1], sizeof(void*));
    std::memcpy(&g_api.grad_norm_flat, &a[2], sizeof(void*));
    std::memcpy(&g_api.grad_sumsq, &a[3], sizeof(void*));
    std::memcpy(&g_api.grad_sumsq_flat, &a[4], sizeof(void*));
    std::memcpy(&g_api.norm_from_sumsq, &a[5], sizeof(void*));
    std::memcpy(&g_api.step_prescaled, &a[6], sizeof(void*));
    std::memcpy(&g_api.step_flat_prescaled, &a[7], sizeof(void*));
    std::memcpy(&g_api.step_fused_chain, &a[8], sizeof(void*));
    std::memcpy(&g_api.step_flat_fused_chain, &a[9], sizeof(void*));
    g_bound = true;
    Py_RETURN_NONE;
}

// plan(params, states, slots, hypers, rows, rest, grads, amsgrad, steps, hyper_steps,
//      launch, options, keep) -> capsule
//   params, states:  lists (entry order) of parameters and their state dicts
//   slots, hypers, rows, rest, grads:  lists of ints per entry (step slot, hyperparameter
//                    set, table row or -1 / -2, row's other pointers aligned, gradient ptr)
//   amsgrad:         whether state["max_exp_avg_sq"] is part of the launch
//   steps:           address and length of the CPU step buffer: (ptr, n)
//   hyper_steps:     (address, n_hyper) of a float64 output array
//   launch:          (tables, d_rows, d_chunks, n_chunks, n_rows, host_rows, flat_row_addr,
//                     flat_hyper)
//   options:         (chunk_elems, max_blocks, state_code, flags, clip, max_norm, prescale,
//                     partials, coef, sumsq, stream, fused_chain)
//   keep:            objects to keep alive while the plan exists
PyObject* plan_new(PyObject* args);

PyObject* py_plan(PyObject*, PyObject* args) {
    try {
        return plan_new(args);
    } catch (const std::exception& ex) {
        PyErr_SetString(PyExc_ValueError, ex.what());
        return nullptr;
    }
}

PyObject* plan_new(PyObject* args) {
    PyObject *params, *states, *slots, *hypers, *rows, *rest, *grads, *steps_t, *hsteps_t,
        *launch_t, *opts_t, *keep;
    int amsgrad = 0;
    if (!PyArg_ParseTuple(args, "O!O!O!O!O!O!O!pO!O!O!O!O", &PyList_Type, &params, &PyList_Type,
                          &states, &PyList_Type, &slots, &PyList_Type, &hypers, &PyList_Type,
                          &rows, &PyList_Type, &rest, &PyList_Type, &grads, &amsgrad,
                          &PyTuple_Type, &steps_t, &PyTuple_Type, &hsteps_t, &PyTuple_Type,
                          &launch_t, &PyTuple_Type, &opts_t, &keep))
        return nullptr;
    const Py_ssize_t n = PyList_GET_SIZE(params);
    if (PyList_GET_SIZE(states) != n || PyList_GET_SIZE(slots) != n ||
        PyList_GET_SIZE(hypers) != n || PyList_GET_SIZE(rows) != n ||
        PyList_GET_SIZE(rest) != n || PyList_GET_SIZE(grads) != n) {
        PyErr_SetString(PyExc_ValueError, "plan: per-entry lists differ in length");
        return nullptr;
    }
    Plan* pl = new Plan();
    PyObject* capsule = PyCapsule_New(pl, "mi_adamw._host.Plan", plan_free);
    if (!capsule) {
        delete pl;
        return nullptr;
    }
    const char* names[4] = {"step", "exp_avg", "exp_avg_sq", "max_exp_avg_sq"};
    for (int k = 0; k < 4; ++k) {
        pl->keys[k] = PyUnicode_InternFromString(names[k]);
        if (!pl->keys[k]) goto fail;
    }
    pl->n_state = amsgrad ? 4 : 3;
    Py_INCREF(keep);
    pl->keep = keep;
    {
        unsigned long long sp = 0, hp = 0;
        long long ns = 0;
        int nh = 0;
        if (!PyArg_ParseTuple(steps_t, "KL", &sp, &ns) ||
            !PyArg_ParseTuple(hsteps_t, "Ki", &hp, &nh))
            goto fail;
        pl->steps = reinterpret_cast<float*>(sp);
        pl->n_steps = ns;
        pl->hyper_steps = reinterpret_cast<double*>(hp);
        pl->n_hyper = nh;
        int tables = 0;
        unsigned long long d_rows = 0, d_chunks = 0, host_rows = 0, flat_row = 0;
        long long n_chunks = 0;
        int n_rows = 0, flat_hyper = 0;
        if (!PyArg_ParseTuple(launch_t, "pKKLiKKi", &tables, &d_rows, &d_chunks, &n_chunks,
                              &n_rows, &host_rows, &flat_row, &flat_hyper))
            goto fail;
        pl->tables = tables;
        pl->d_rows = reinterpret_cast<mi_adamw_tensor*>(d_rows);
        pl->d_chunks = reinterpret_cast<const mi_adamw_chunk*>(d_chunks);
        pl->n_chunks = n_chunks;
        pl->n_rows = n_rows;
        pl->host_rows = reinterpret_cast<uint8_t*>(host_rows);
        if (!tables) {
            if (!flat_row) {
                PyErr_SetString(PyExc_ValueError, "plan: a table-free launch needs its row");
                goto fail;
            }
            std::memcpy(&pl->flat_row, reinterpret_cast<const void*>(flat_row),
                        sizeof(mi_adamw_tensor));
        }
        pl->flat_hyper = flat_hyper;
        long long chunk = 0;
        int max_blocks = 0, state_code = 0, flags = 0, clip = 0, fused_chain = 0;
        float max_norm = 0, prescale = 1;
        unsigned long long partials = 0, coef = 0, sumsq = 0, stream = 0;
        if (!PyArg_ParseTuple(opts_t, "LiiipffKKKKp", &chunk, &max_blocks, &state_code, &flags,
                              &clip, &max_norm, &prescale, &partials, &coef, &sumsq, &stream,
                              &fused_chain))
            goto fail;
        pl->fused_chain = fused_chain;
        pl->chunk_elems = chunk;
        pl->max_blocks = max_blocks;
        pl->state_code = state_code;
        pl->flags = flags;
        pl->clip = clip;
        pl->max_norm = max_norm;
        pl->prescale = prescale;
        pl->partials = reinterpret_cast<double*>(partials);
        pl->coef = reinterpret_cast<float*>(coef);
        pl->sumsq = reinterpret_cast<double*>(sumsq);
        pl->stream = stream;
    }
    pl->e.resize(n);
    for (Py_ssize_t i = 0; i < n; ++i) {
        Entry& en = pl->e[i];
        PyObject* p = PyList_GET_ITEM(params, i);
        PyObject* st = PyList_GET_ITEM(states, i);
        if (!is_tensor(p) || !PyDict_Check(st)) {
            PyErr_SetString(PyExc_TypeError, "plan: parameters must be tensors, states dicts");
            goto fail;
        }
        Py_INCREF(p);
        en.p = p;
        Py_INCREF(st);
        en.st = st;
        en.ptr[0] = tensor_ptr(p);
        en.numel = THPVariable_Unpack(p).numel();
        for (int k = 0; k < pl->n_state; ++k) {
            PyObject* o = PyDict_GetItemWithError(st, pl->keys[k]);
            if (!is_tensor(o)) {
                if (!PyErr_Occurred())
                    PyErr_Format(PyExc_ValueError, "plan: state[%s] is not a tensor", names[k]);
                goto fail;
            }
            Py_INCREF(o);
            en.obj[k] = o;
            if (k > 0) en.ptr[k] = tensor_ptr(o);
        }
        en.slot = static_cast<int32_t>(PyLong_AsLong(PyList_GET_ITEM(slots, i)));
        en.hyper = static_cast<int32_t>(PyLong_AsLong(PyList_GET_ITEM(hypers, i)));
        en.row = static_cast<int32_t>(PyLong_AsLong(PyList_GET_ITEM(rows, i)));
        en.rest = PyObject_IsTrue(PyList_GET_ITEM(rest, i)) ? 1 : 0;
        en.grad = PyLong_AsUnsignedLongLong(PyList_GET_ITEM(grads, i));
        if (PyErr_Occurred()) goto fail;
        if (en.slot < 0 || en.slot >= pl->n_steps || en.hyper < 0 || en.hyper >= pl->n_hyper ||
            en.row >= pl->n_rows || en.row < kFixed) {
            PyErr_SetString(PyExc_ValueError, "plan: slot, hyper or row out of range");
            goto fail;
        }
    }
    pl->prow.reserve(n);
    pl->pgrad.reserve(n);
    pl->pvec.reserve(n);
    pl->newgrad.resize(n);
    return capsule;
fail:
    Py_DECREF(capsule);
    return nullptr;
}

// The checks and the table update of one step.  Returns kReady / kReadyMoved after the
// step counts were advanced (and moved gradients written to the table), kFallback with
// nothing changed, or kError when mi_adamw_set_grads failed: then the step counts, the
// host rows and the entries' gradient pointers are unchanged, while the device table may
// hold part of the patch (its rows are patched 128 at a time), so the caller must drop
// the tables and the plan before the next step.
int prepare(Plan* pl, uint64_t stream) {
    if (stream != pl->stream) return kFallback;
    const size_t n = pl->e.size();
    pl->prow.clear();
    pl->pgrad.clear();
    pl->pvec.clear();
    for (size_t i = 0; i < n; ++i) {
        Entry& en = pl->e[i];
        const at::Tensor& p = THPVariable_Unpack(en.p);
        // the row covers en.numel elements of p, its gradient and its state, stepped by
        // memory position: a parameter narrowed or re-strided in place through .data keeps
        // its address but no longer matches the row
        if (reinterpret_cast<uint64_t>(p.data_ptr()) != en.ptr[0] || p.numel() != en.numel ||
            !p.is_contiguous())
            return kFallback;
        const at::Tensor& g = p.grad();
        if (!g.defined() || g.layout() != c10::kStrided || !g.is_contiguous() ||
            g.scalar_type() != p.scalar_type() || g.device() != p.device() ||
            g.numel() != en.numel)
            return kFallback;
        for (int k = 0; k < pl->n_state; ++k) {
            PyObject* o = PyDict_GetItem(en.st, pl->keys[k]);
            if (o != en.obj[k]) return kFallback;
            if (k > 0) {
                // a moment re-strided or narrowed in place through .data keeps its object
                // and address, but the row reads p's element count from it densely
                const at::Tensor& t = THPVariable_Unpack(o);
                if (reinterpret_cast<uint64_t>(t.data_ptr()) != en.ptr[k] ||
                    !t.is_contiguous() || t.numel() != en.numel)
                    return kFallback;
            }
        }
        const uint64_t gp = reinterpret_cast<uint64_t>(g.data_ptr());
        pl->newgrad[i] = gp;
        if (gp != en.grad) {
            if (en.row == kFixed) return kFallback;
            if (en.row >= 0) {
                pl->prow.push_back(en.row);
                pl->pgrad.push_back(gp);
                pl->pvec.push_back(en.rest && (gp % 16) == 0);
            }
        }
    }
    // every hyperparameter set (param group) steps from one count
    for (int32_t h = 0; h < pl->n_hyper; ++h) pl->hyper_steps[h] = -1.0;
    for (const Entry& en : pl->e) {
        const double s = pl->steps[en.slot];
        double& hs = pl->hyper_steps[en.hyper];
        if (hs < 0.0)
            hs = s;
        else if (hs != s)
            return kFallback;
    }
    const int moved = !pl->prow.empty();
    if (moved) {
        const int32_t m = static_cast<int32_t>(pl->prow.size());
        if (pl->tables) {
            const int rc = g_api.set_grads(pl->d_rows, pl->n_rows, m, pl->prow.data(),
                                           pl->pgrad.data(), pl->pvec.data(),
                                           reinterpret_cast<void*>(stream));
            if (rc != MI_ADAMW_OK) {
                pl->last_error = rc;
                return kError;
            }
        } else {
            // the single row of a table-free launch lives on the host
            pl->flat_row.grad = reinterpret_cast<float*>(pl->pgrad[0]);
            pl->flat_row.flags =
                (pl->flat_row.flags & ~MI_ADAMW_T_VEC) | (pl->pvec[0] ? MI_ADAMW_T_VEC : 0);
        }
        for (int32_t j = 0; j < m; ++j) {
            // keep the host copy of the rows equal to the device table
            uint8_t* r = pl->host_rows + 64 * static_cast<size_t>(pl->prow[j]);
            std::memcpy(r + 8, &pl->pgrad[j], 8);
            int32_t fl;
            std::memcpy(&fl, r + 60, 4);
            fl = (fl & ~MI_ADAMW_T_VEC) | (pl->pvec[j] ? MI_ADAMW_T_VEC : 0);
            std::memcpy(r + 60, &fl, 4);
        }
        for (size_t i = 0; i < n; ++i) pl->e[i].grad = pl->newgrad[i];
    }
    // step_t += 1 (adam.py:414) in the fp32 step buffer, for every parameter of the launch;
    // each hyperparameter set gets its parameters' new count
    for (const Entry& en : pl->e) {
        pl->steps[en.slot] += 1.0f;
        pl->hyper_steps[en.hyper] = pl->steps[en.slot];
    }
    return moved ? kReadyMoved : kReady;
}

PyObject* py_prepare(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
    if (nargs != 2) {
        PyErr_SetString(PyExc_TypeError, "prepare(plan, stream)");
        return nullptr;
    }
    Plan* pl = get_plan(args[0]);
    if (!pl) return nullptr;
    const uint64_t stream = PyLong_AsUnsignedLongLong(args[1]);
    if (PyErr_Occurred()) return nullptr;
    if (!g_bound) {
        PyErr_SetString(PyExc_RuntimeError, "mi_adamw._host: bind() was not called");
        return nullptr;
    }
    int rc;
    try {
        rc = prepare(pl, stream);
    } catch (const std::exception& ex) {
        // an at::Tensor accessor refused a tensor (no storage, ...): let the general path
        // take the step and report it
        (void)ex;
        rc = kFallback;
    }
    return PyLong_FromLong(rc);
}

PyObject* py_last_error(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
    if (nargs != 1) {
        PyErr_SetString(PyExc_TypeError, "last_error(plan)");
        return nullptr;
    }
    Plan* pl = get_plan(args[0]);
    if (!pl) return nullptr;
    return PyLong_FromLong(pl->last_error);
}

PyObject* py_norm(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
    if (nargs != 3) {
        PyErr_SetString(PyExc_TypeError, "norm(plan, stream, d_norm)");
        return nullptr;
    }
    Plan* pl = get_plan(args[0]);
    if (!pl) return nullptr;
    void* s = PyLong_AsVoidPtr(args[1]);
    float* norm = static_cast<float*>(PyLong_AsVoidPtr(args[2]));
    if (PyErr_Occurred()) return nullptr;
    int rc;
    if (pl->prescale != 1.0f) {
        rc = pl->tables ? g_api.grad_sumsq(pl->d_rows, pl->d_chunks, pl->n_chunks,
                                           pl->chunk_elems, pl->prescale, pl->partials,
                                           pl->sumsq, s)
                        : g_api.grad_sumsq_flat(pl->flat_row.grad, pl->flat_row.numel,
                                                pl->chunk_elems, pl->prescale, pl->partials,
                                                pl->sumsq, s);
        if (rc == MI_ADAMW_OK)
            rc = g_api.norm_from_sumsq(pl->sumsq, 1, pl->max_norm, norm, pl->coef, s);
    } else {
        rc = pl->tables ? g_api.grad_norm(pl->d_rows, pl->d_chunks, pl->n_chunks, pl->chunk_elems,
                                          pl->max_norm, pl->partials, norm, pl->coef, s)
                        : g_api.grad_norm_flat(pl->flat_row.grad, pl->flat_row.numel,
                                               pl->chunk_elems, pl->max_norm, pl->partials, norm,
                                               pl->coef, s);
    }
    return PyLong_FromLong(rc);
}

PyObject* py_update(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
    if (nargs != 4) {
        PyErr_SetString(PyExc_TypeError, "update(plan, stream, hypers, n_hyper)");
        return nullptr;
    }
    Plan* pl = get_plan(args[0]);
    if (!pl) return nullptr;
    void* s = PyLong_AsVoidPtr(args[1]);
    void* hv = PyLong_AsVoidPtr(args[2]);
    const long nh = PyLong_AsLong(args[3]);
    if (PyErr_Occurred()) return nullptr;
    const int32_t flags = pl->flags | (pl->clip ? MI_ADAMW_F_CLIP : 0);
    int rc;
    if (pl->fused_chain) {
        const mi_adamw_fused_hyper* fh = static_cast<const mi_adamw_fused_hyper*>(hv);
        if (pl->tables) {
            rc = g_api.step_fused_chain(pl->d_rows, pl->d_chunks, pl->n_chunks, pl->chunk_elems,
                                        fh, static_cast<int32_t>(nh), nullptr, nullptr,
                                        pl->coef, pl->prescale, pl->state_code, flags,
                                        pl->max_blocks, s);
        } else {
            if (pl->flat_hyper >= nh) return PyLong_FromLong(MI_ADAMW_E_INVALID);
            rc = g_api.step_flat_fused_chain(&pl->flat_row, fh + pl->flat_hyper, pl->coef,
                                             pl->prescale, pl->chunk_elems, pl->state_code,
                                             flags, pl->max_blocks, s);
        }
        return PyLong_FromLong(rc);
    }
    const mi_adamw_hyper* h = static_cast<const mi_adamw_hyper*>(hv);
    if (pl->tables) {
        rc = g_api.step_prescaled(pl->d_rows, pl->d_chunks, pl->n_chunks, pl->chunk_elems, h,
                                  static_cast<int32_t>(nh), pl->coef, pl->prescale,
                                  pl->state_code, flags, pl->max_blocks, s);
    } else {
        if (pl->flat_hyper >= nh) return PyLong_FromLong(MI_ADAMW_E_INVALID);
        rc = g_api.step_flat_prescaled(&pl->flat_row, h + pl->flat_hyper, pl->coef, pl->prescale,
                                       pl->chunk_elems, pl->state_code, flags, pl->max_blocks, s);
    }
    return PyLong_FromLong(rc);
}

PyObject* sync_versions(Plan* pl, PyObject* dict);

PyObject* py_sync_versions(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
    if (nargs != 2 || !PyDict_Check(args[1])) {
        PyErr_SetString(PyExc_TypeError, "sync_versions(plan, dict)");
        return nullptr;
    }
    Plan* pl = get_plan(args[0]);
    if (!pl) return nullptr;
    try {
        return sync_versions(pl, args[1]);
    } catch (const std::exception& ex) {
        PyErr_SetString(PyExc_RuntimeError, ex.what());
        return nullptr;
    }
}

PyObject* sync_versions(Plan* pl, PyObject* dict) {
    for (const Entry& en : pl->e) {
        const at::Tensor& p = THPVariable_Unpack(en.p);
        PyObject* key = PyLong_FromVoidPtr(en.p);
        PyObject* val = Py_BuildValue("(KK)", static_cast<unsigned long long>(p._version()),
                                      static_cast<unsigned long long>(
                                          reinterpret_cast<uint64_t>(p.data_ptr())));
        const int rc = (key && val) ? PyDict_SetItem(dict, key, val) : -1;
        Py_XDECREF(key);
        Py_XDECREF(val);
        if (rc < 0) return nullptr;
    }
    Py_RETURN_NONE;
}

PyMethodDef kMethods[] = {
    {"bind", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(py_bind)), METH_FASTCALL,
     "bind the library's entry points"},
    {"plan", py_plan, METH_VARARGS, "the bookkeeping of one launch"},
    {"prepare", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(py_prepare)),
     METH_FASTCALL, "checks, moved gradients, step counts"},
    {"last_error", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(py_last_error)),
     METH_FASTCALL, "the library code behind prepare()'s last ERROR"},
    {"norm", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(py_norm)), METH_FASTCALL,
     "enqueue the norm pass"},
    {"update", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(py_update)),
     METH_FASTCALL, "enqueue the update"},
    {"sync_versions",
     reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(py_sync_versions)), METH_FASTCALL,
     "record every parameter's version and address"},
    {nullptr, nullptr, 0, nullptr}};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_host",
                       "Native steady-state host path of mi_adamw.FusedAdamW.step()", -1,
                       kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__host(void) {
    PyObject* m = PyModule_Create(&kModule);
    if (!m) return nullptr;
    if (PyModule_AddIntConstant(m, "READY", kReady) < 0 ||
        PyModule_AddIntConstant(m, "READY_MOVED", kReadyMoved) < 0 ||
        PyModule_AddIntConstant(m, "FALLBACK", kFallback) < 0 ||
        PyModule_AddIntConstant(m, "ERROR", kError) < 0) {
        Py_DECREF(m);
        return nullptr;
    }
    return m;
}
