// Host side of the cached step plan (gefen_amd/gefen.py, _StepPlan.refresh):
// the per-tensor checks of a steady-state Gefen.step (gefen.py:1399-1420 and
// the parameter loop of _step_automatic, gefen.py:1208-1333) done in C++ on
// torch's own tensor objects instead of through ~7 Python attribute calls per
// tensor.
//
// PlanCore holds, for every parameter that had a gradient when the plan was
// built (in optimizer order): the parameter object, its data pointer, the
// gradient's element count and dtype, the parameter's state dict and its state
// tensor objects (the given state keys).  refresh() walks the optimizer's param groups and
// succeeds only if the parameters with a gradient are exactly those objects in
// that order, every gradient is a plain (no Python dispatch) strided contiguous
// tensor of the recorded dtype, size and device, every parameter keeps its data
// pointer and is contiguous, and every state dict still holds the same state
// tensors and an int "step".  Only then does it write each task row's gradient
// address, group hyperparameters and bias corrections and advance every
// state["step"]; on any mismatch it changes nothing and returns false (the
// caller rebuilds the plan).
//
// Built with the host compiler against torch's headers (no device code).

#include <Python.h>
#include <pybind11/pybind11.h>
#include <torch/csrc/autograd/python_variable.h>

#include <array>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

namespace py = pybind11;

namespace {

// CPython 3.6 - 3.11 give every dict a version tag that changes with each
// modification of that dict (PEP 509).  Where it exists, a param group or state
// dict whose tag equals the one recorded at the last refresh still holds the
// same value objects, so their lookups are skipped; elsewhere every value is
// looked up each time.
#if PY_VERSION_HEX >= 0x03060000 && PY_VERSION_HEX < 0x030C0000
constexpr bool kDictVersion = true;
inline uint64_t dict_version(PyObject* d) { return reinterpret_cast<PyDictObject*>(d)->ma_version_tag; }
#else
constexpr bool kDictVersion = false;
inline uint64_t dict_version(PyObject*) { return 0; }
#endif

// interned dict keys, created once at module import
PyObject* key_params_;
PyObject* key_step_;
PyObject* key_lr_;
PyObject* key_beta1_;
PyObject* key_beta2_;
PyObject* key_eps_;
PyObject* key_wd_;

PyObject* intern(const char* s) {
    PyObject* k = PyUnicode_InternFromString(s);
    if (!k) throw py::error_already_set();
    return k;
}

class PlanCore {
   public:
    // params: the parameters with a gradient, in optimizer order (their current
    // gradients give the recorded size, dtype and device); states: their state
    // dicts; state_keys: the state entries that must stay the same objects (their
    // current values are recorded).
    PlanCore(py::list params, py::list states, py::tuple state_keys) {
        const size_t n = params.size();
        if (states.size() != n) throw py::value_error("PlanCore: lists of different lengths");
        for (py::handle key : state_keys) {
            if (!PyUnicode_Check(key.ptr())) throw py::type_error("PlanCore: state keys are strings");
            skeys_.push_back(py::reinterpret_borrow<py::object>(key));
        }
        for (size_t k = 0; k < n; ++k) {
            py::handle p = params[k];
            if (!THPVariable_Check(p.ptr())) throw py::type_error("PlanCore: parameter is not a tensor");
            const at::Tensor& t = THPVariable_Unpack(p.ptr());
            const at::Tensor& g = t.grad();
            if (!g.defined()) throw py::value_error("PlanCore: parameter without a gradient");
            if (k == 0) {
                device_type_ = static_cast<int>(g.device().type());
                device_index_ = g.device().index();
            }
            params_.push_back(py::reinterpret_borrow<py::object>(p));
            pptr_.push_back(reinterpret_cast<uintptr_t>(t.data_ptr()));
            numel_.push_back(g.numel());
            dtype_.push_back(g.scalar_type());
            py::handle st = states[k];
            if (!PyDict_Check(st.ptr())) throw py::type_error("PlanCore: state is not a dict");
            states_.push_back(py::reinterpret_borrow<py::object>(st));
            std::vector<py::object> refs;
            for (const py::object& key : skeys_) {
                PyObject* v = PyDict_GetItem(st.ptr(), key.ptr());
                if (!v) throw py::key_error("PlanCore: state entry missing");
                refs.push_back(py::reinterpret_borrow<py::object>(v));
            }
            srefs_.push_back(std::move(refs));
        }
        gptr_.resize(n);
        step_.resize(n);
        hyper_.resize(n);
        sver_.assign(n, 0);
        committed_.assign(n, 0);
    }

    // table: address of the task table (rows of `stride` bytes); cols: byte offsets
    // within a row of grad, lr, beta1, beta2, eps, weight_decay, bias_correction_1,
    // bias_correction_2 (uint64 address, then doubles); steps_out: n int64 slots
    // receiving the advanced step counts.  Hyperparameters come from each
    // parameter's group (lr may be a 0-d tensor); the bias corrections are
    // 1 - beta ** step in double, as Python evaluates them (gefen.py:1278-1284).
    //
    // With cols = (grad,) only the gradient addresses and the step counts are
    // written (the caller handles the hyperparameters).
    bool refresh(py::handle param_groups, uintptr_t table, int64_t stride, py::tuple cols, uintptr_t steps_out) {
        if (!prepare(param_groups, table, stride, cols)) return false;
        commit(steps_out);
        return true;
    }

    // refresh(), then, when its checks passed, the step itself: run_fn is the
    // address of the C ABI's gefen_step_plan_run, called with (plan, table, number
    // of rows, stream) once the table rows are written, so a cached step costs one
    // call from Python.  The state dicts' "step" entries and steps_out are written
    // after the launches (they are not read before), which keeps those writes off
    // the GPU's wait for the first launch.  Returns -1 when the plan no longer
    // applies (nothing was changed or launched), else gefen_step_plan_run's status
    // (the step counts advance in either case).
    int step(py::handle param_groups, uintptr_t table, int64_t stride, py::tuple cols, uintptr_t steps_out,
             uintptr_t run_fn, uintptr_t plan, uintptr_t stream) {
        if (!run_fn || !plan) throw py::value_error("PlanCore.step: null run function or plan");
        if (!prepare(param_groups, table, stride, cols)) return -1;
        using RunFn = int (*)(void*, const void*, int, void*);
        const int rc = reinterpret_cast<RunFn>(run_fn)(reinterpret_cast<void*>(plan),
                                                       reinterpret_cast<const void*>(table),
                                                       static_cast<int>(params_.size()), reinterpret_cast<void*>(stream));
        commit(steps_out);
        return rc;
    }

    size_t size() const { return params_.size(); }

   private:
    // The checks of refresh() and the table rows: gradient addresses and, with
    // hyperparameter columns, the hyperparameters and bias corrections of step + 1.
    // A failed check (false) leaves the table and the state dicts as they were.
    bool prepare(py::handle param_groups, uintptr_t table, int64_t stride, py::tuple cols) {
        if (!PyList_Check(param_groups.ptr()) || (cols.size() != 8 && cols.size() != 1)) return false;
        const bool hyper = cols.size() == 8;
        size_t col[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (size_t i = 0; i < cols.size(); ++i) col[i] = cols[i].cast<size_t>();
        const size_t n = params_.size();
        size_t k = 0;
        const Py_ssize_t ngroups = PyList_GET_SIZE(param_groups.ptr());
        if ((size_t)ngroups > gcache_.size()) gcache_.resize((size_t)ngroups);
        for (Py_ssize_t gi = 0; gi < ngroups; ++gi) {
            PyObject* group = PyList_GET_ITEM(param_groups.ptr(), gi);
            if (!PyDict_Check(group)) return false;
            GroupCache& gc = gcache_[(size_t)gi];
            // the same group dict, unmodified since the last refresh: the same "params"
            // list object and the same hyperparameter objects
            const bool same_group = kDictVersion && gc.group.ptr() == group && gc.ver == dict_version(group);
            PyObject* plist = same_group ? gc.params.ptr() : PyDict_GetItem(group, key_params_);
            if (!plist || !PyList_Check(plist)) return false;
            if (!same_group) {
                gc.group = py::reinterpret_borrow<py::object>(group);
                gc.params = py::reinterpret_borrow<py::object>(plist);
                gc.ver = dict_version(group);
                gc.hyper_ok = false;
            }
            const Py_ssize_t np = PyList_GET_SIZE(plist);
            bool have_hyper = false;
            std::array<double, 5> h{};
            for (Py_ssize_t i = 0; i < np; ++i) {
                PyObject* p = PyList_GET_ITEM(plist, i);
                if (!THPVariable_Check(p)) return false;
                const at::Tensor& t = THPVariable_Unpack(p);
                const at::Tensor& g = t.grad();
                if (!g.defined()) continue;
                if (k == n || p != params_[k].ptr()) return false;
                if (g.key_set().has(c10::DispatchKey::Python) || g.layout() != at::kStrided ||
                    g.scalar_type() != dtype_[k] || g.numel() != numel_[k] || !g.is_contiguous() ||
                    static_cast<int>(g.device().type()) != device_type_ || g.device().index() != device_index_)
                    return false;
                if (reinterpret_cast<uintptr_t>(t.data_ptr()) != pptr_[k] || !t.is_contiguous()) return false;
                if (hyper && !have_hyper) {
                    if (gc.hyper_ok) {
                        h = gc.h;
                    } else {
                        bool immutable = false;
                        if (!group_hyper(group, h, &immutable)) return false;
                        // numbers are immutable: kept while the group dict is unmodified (a
                        // 0-d tensor lr can change in place and is read every time)
                        gc.h = h;
                        gc.hyper_ok = kDictVersion && immutable;
                    }
                    have_hyper = true;
                }
                gptr_[k] = reinterpret_cast<uint64_t>(g.data_ptr());
                hyper_[k] = h;
                ++k;
            }
        }
        if (k != n) return false;
        for (k = 0; k < n; ++k) {
            PyObject* st = states_[k].ptr();
            // unmodified since this refresh last wrote "step": same state tensors, and
            // "step" is the value written then
            if (kDictVersion && sver_[k] != 0 && sver_[k] == dict_version(st)) {
                step_[k] = committed_[k] + 1;
                continue;
            }
            for (size_t j = 0; j < skeys_.size(); ++j)
                if (PyDict_GetItem(st, skeys_[j].ptr()) != srefs_[k][j].ptr()) return false;
            PyObject* s = PyDict_GetItem(st, key_step_);
            if (!s || !PyLong_CheckExact(s)) return false;
            const long long v = PyLong_AsLongLong(s);
            if (v == -1 && PyErr_Occurred()) {
                PyErr_Clear();
                return false;
            }
            step_[k] = v + 1;
        }
        // every check passed: the table rows
        double last_b1 = 0.0, last_b2 = 0.0, bc1 = 0.0, bc2 = 0.0;
        long long last_step = -1;
        for (k = 0; k < n; ++k) {
            char* row = reinterpret_cast<char*>(table + k * stride);
            const uint64_t gp = gptr_[k];
            std::memcpy(row + col[0], &gp, 8);
            if (hyper) {
                const std::array<double, 5>& h = hyper_[k];
                if (step_[k] != last_step || h[1] != last_b1 || h[2] != last_b2) {
                    bc1 = 1.0 - std::pow(h[1], (double)step_[k]);
                    bc2 = 1.0 - std::pow(h[2], (double)step_[k]);
                    last_step = step_[k];
                    last_b1 = h[1];
                    last_b2 = h[2];
                }
                for (int c = 0; c < 5; ++c) std::memcpy(row + col[1 + c], &h[c], 8);
                std::memcpy(row + col[6], &bc1, 8);
                std::memcpy(row + col[7], &bc2, 8);
            }
        }
        return true;
    }

    // The advanced step counts of the last successful prepare(): each state's
    // "step" entry and steps_out (n int64 slots).
    void commit(uintptr_t steps_out) {
        int64_t* steps = reinterpret_cast<int64_t*>(steps_out);
        // one int object per distinct step count, shared by the state dicts that take it
        py::object step_obj;
        long long step_obj_val = -1;
        const size_t n = params_.size();
        for (size_t k = 0; k < n; ++k) {
            if (!step_obj || step_obj_val != step_[k]) {
                PyObject* v = PyLong_FromLongLong(step_[k]);
                if (!v) throw py::error_already_set();
                step_obj = py::reinterpret_steal<py::object>(v);
                step_obj_val = step_[k];
            }
            const int rc = PyDict_SetItem(states_[k].ptr(), key_step_, step_obj.ptr());
            sver_[k] = rc == 0 ? dict_version(states_[k].ptr()) : 0;
            committed_[k] = step_[k];
            if (rc != 0) throw py::error_already_set();
            steps[k] = step_[k];
        }
    }

    // lr (a number or a 0-d tensor), beta1, beta2, eps, weight_decay of a group,
    // the weight decay as the kernels take it.  For a float32 tensor lr with
    // weight decay, torch forms the decay factor in float32,
    // f = fl32(1 - fl32(lr * fl32(wd))) (gefen.py:1280-1281), while the kernels
    // form (float)(1 - lr * wd) in double: they get wd' = (1 - f) / lr instead,
    // for which that double expression lies within ~2^-51 (relative) of f and so
    // rounds to f exactly (gefen.py's _kernel_weight_decay does the same).  A
    // tensor lr of a 16-bit dtype with weight decay, lr <= 0 or f zero or not
    // finite is refused: the Python step applies torch's factor before the launch.
    // immutable: set when all five values are Python floats or ints.
    bool group_hyper(PyObject* group, std::array<double, 5>& h, bool* immutable = nullptr) {
        PyObject* keys[5] = {key_lr_, key_beta1_, key_beta2_, key_eps_, key_wd_};
        int lr_kind = 0;  // 0: number or float64 tensor, 1: float32 tensor, 2: other tensor
        bool numbers = true;
        for (int c = 0; c < 5; ++c) {
            PyObject* v = PyDict_GetItem(group, keys[c]);
            if (!v) return false;
            numbers = numbers && (PyFloat_CheckExact(v) || PyLong_CheckExact(v));
            if (c == 0 && THPVariable_Check(v)) {
                const at::ScalarType st = THPVariable_Unpack(v).scalar_type();
                lr_kind = st == at::kDouble ? 0 : (st == at::kFloat ? 1 : 2);
            }
            if (PyFloat_CheckExact(v)) {
                h[c] = PyFloat_AS_DOUBLE(v);
                continue;
            }
            PyObject* f = PyNumber_Float(v);  // ints, numpy scalars, 0-d tensors (.item())
            if (!f) {
                PyErr_Clear();
                return false;
            }
            h[c] = PyFloat_AS_DOUBLE(f);
            Py_DECREF(f);
        }
        if (immutable) *immutable = numbers;
        if (lr_kind == 0 || !(h[4] > 0.0)) return true;
        if (lr_kind != 1 || !(h[0] > 0.0)) return false;
        const volatile float prod = (float)h[0] * (float)h[4];  // volatile: each op rounded to float
        const volatile float f = 1.0f - prod;
        if (!std::isfinite(f) || f == 0.0f) return false;
        h[4] = (1.0 - (double)f) / h[0];
        return true;
    }

    int device_type_ = -1, device_index_ = -1;
    std::vector<py::object> params_;
    std::vector<uintptr_t> pptr_;
    std::vector<int64_t> numel_;
    std::vector<at::ScalarType> dtype_;
    std::vector<py::object> states_;
    std::vector<py::object> skeys_;
    std::vector<std::vector<py::object>> srefs_;
    std::vector<uint64_t> gptr_;
    std::vector<long long> step_;
    std::vector<std::array<double, 5>> hyper_;
    // per param group position: the group dict and its version at the last refresh,
    // its "params" list, and its hyperparameters when they are kept (numbers)
    struct GroupCache {
        py::object group, params;
        uint64_t ver = 0;
        bool hyper_ok = false;
        std::array<double, 5> h{};
    };
    std::vector<GroupCache> gcache_;
    std::vector<uint64_t> sver_;          // version of each state dict after its "step" was written (0: none)
    std::vector<long long> committed_;    // the "step" value written then
};

}  // namespace

PYBIND11_MODULE(_gefen_host, m) {
    m.doc() = "Host-side checks of the cached Gefen step plan";
    key_params_ = intern("params");
    key_step_ = intern("step");
    key_lr_ = intern("lr");
    key_beta1_ = intern("beta1");
    key_beta2_ = intern("beta2");
    key_eps_ = intern("eps");
    key_wd_ = intern("weight_decay");
    py::class_<PlanCore>(m, "PlanCore")
        .def(py::init<py::list, py::list, py::tuple>())
        .def("refresh", &PlanCore::refresh)
        .def("step", &PlanCore::step)
        .def("__len__", &PlanCore::size);
}
