// Host-side bookkeeping of the scalar plan's steady state, in C++.
//
// One optimizer step of a group of many small tensors (the C3 case: 840) is a
// single kernel sequence on the GPU, but the per-step Python work around it
// (checking that the group is unchanged, collecting the fresh grad pointers
// that autograd allocates, advancing every state["step"]) costs about 0.2 us
// per tensor and per item in CPython, which is as long as the GPU step itself.
// BatchGuard does the same checks and writes in one pass over the Python
// objects: gather() verifies each parameter (same object, same storage) and
// its grad (defined, contiguous, same dtype/device/numel as at plan time) and
// writes the grad pointers into a host array; bump() adds 1 to state["step"].
// Any mismatch makes gather() return false and the caller rebuilds the plan.
#include <torch/extension.h>

#include <cstdint>
#include <vector>

namespace {

struct BatchGuard {
    // Strong references: a parameter cannot be freed (and a new object created
    // at its address) while the guard lives, so the identity test is exact.
    std::vector<py::object> params;
    std::vector<const void*> pptr;   // param storage at plan time
    std::vector<int> gdtype;         // grad dtype at plan time (c10::ScalarType)
    std::vector<int64_t> numel;
    std::vector<int> device;

    explicit BatchGuard(const py::list& ps) {
        const size_t n = ps.size();
        params.reserve(n);
        for (size_t i = 0; i < n; ++i) {
            PyObject* o = ps[i].ptr();
            if (!THPVariable_Check(o)) throw std::invalid_argument("BatchGuard: parameters must be tensors");
            const at::Tensor& t = THPVariable_Unpack(o);
            const at::Tensor& g = t.grad();
            if (!g.defined()) throw std::invalid_argument("BatchGuard: every parameter needs a grad at plan time");
            params.push_back(py::reinterpret_borrow<py::object>(o));
            pptr.push_back(t.data_ptr());
            gdtype.push_back(static_cast<int>(g.scalar_type()));
            numel.push_back(t.numel());
            device.push_back(t.device().index());
        }
    }

    // Writes params[i].grad.data_ptr() to out[i]; false if anything differs
    // from plan time (then out is partially written and must not be used).
    bool gather(const py::list& ps, uintptr_t out_addr) const {
        const size_t n = params.size();
        if (ps.size() != n) return false;
        void** out = reinterpret_cast<void**>(out_addr);
        for (size_t i = 0; i < n; ++i) {
            PyObject* o = ps[i].ptr();
            if (o != params[i].ptr()) return false;
            const at::Tensor& t = THPVariable_Unpack(o);
            if (t.data_ptr() != pptr[i]) return false;
            const at::Tensor& g = t.grad();
            if (!g.defined() || static_cast<int>(g.scalar_type()) != gdtype[i] || g.numel() != numel[i] ||
                g.device().index() != device[i] || !g.device().is_cuda() || g.is_sparse() || !g.is_contiguous())
                return false;
            out[i] = g.data_ptr();
        }
        return true;
    }

    // state["step"] += 1 for each state dict (the library advanced its own copy).
    void bump(const py::list& states) const {
        static PyObject* key = PyUnicode_InternFromString("step");
        for (const py::handle& h : states) {
            PyObject* d = h.ptr();
            PyObject* v = PyDict_GetItemWithError(d, key);   // borrowed
            if (!v) {
                if (PyErr_Occurred()) throw py::error_already_set();
                throw std::invalid_argument("BatchGuard: a state has no 'step'");
            }
            const long long s = PyLong_AsLongLong(v);
            if (s == -1 && PyErr_Occurred()) throw py::error_already_set();
            PyObject* nv = PyLong_FromLongLong(s + 1);
            if (!nv) throw py::error_already_set();
            const int rc = PyDict_SetItem(d, key, nv);
            Py_DECREF(nv);
            if (rc != 0) throw py::error_already_set();
        }
    }
};

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "Per-step host bookkeeping of the CRESSO5 scalar plan";
    py::class_<BatchGuard>(m, "BatchGuard")
        .def(py::init<const py::list&>())
        .def("gather", &BatchGuard::gather)
        .def("bump", &BatchGuard::bump);
}
