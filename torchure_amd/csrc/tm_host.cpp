// tm_host.cpp -- host-side list primitives of the optimizer step (CPU only, no GPU work).
//
// The per-step host path walks every parameter: it gathers each grad, checks that the
// pointers cached in the tensor table are still the tensors' storage, compares autograd
// versions and bumps them after the raw-pointer writes. In Python each of those accesses
// costs 0.1-0.2 us per tensor, which for a list of 10,000 tensors adds up to tens of
// milliseconds per step. These functions do the same walks over Python lists in C++
// (about 15-20 ns per element), so the steady-state step stays far below the kernel time.
// They read tensor metadata only; nothing here allocates or touches device memory.

#include <torch/extension.h>
#include <pybind11/numpy.h>
#include <torch/csrc/autograd/python_variable.h>
#include <torch/csrc/autograd/variable.h>

#include <cstdint>
#include <stdexcept>
#include <utility>

namespace py = pybind11;

namespace {

// nullptr for None; throws for anything that is not a tensor.
inline const at::Tensor* tensor_or_null(PyObject* o) {
  if (o == Py_None) return nullptr;
  if (!THPVariable_Check(o)) throw py::type_error("torchure_amd._tm_host: expected a tensor or None");
  return &THPVariable_Unpack(o);
}

inline PyObject* list_item(const py::list& l, Py_ssize_t i) { return PyList_GET_ITEM(l.ptr(), i); }

// Effective grad of each master: p.grad if set, else works[i].grad (works[i] may be None).
// Returns (list of grad tensors or None, bytes of sources: 0 none, 1 p.grad, 2 works[i].grad).
py::tuple grads(const py::list& params, const py::list& works) {
  const Py_ssize_t n = PyList_GET_SIZE(params.ptr());
  if (PyList_GET_SIZE(works.ptr()) != n) throw py::value_error("params and works differ in length");
  py::list out(n);
  std::string src(static_cast<size_t>(n), '\0');
  for (Py_ssize_t i = 0; i < n; ++i) {
    const at::Tensor* p = tensor_or_null(list_item(params, i));
    PyObject* g = nullptr;
    if (p && p->grad().defined()) {
      g = THPVariable_Wrap(p->grad());
      src[i] = 1;
    } else if (const at::Tensor* w = tensor_or_null(list_item(works, i)); w && w->grad().defined()) {
      g = THPVariable_Wrap(w->grad());
      src[i] = 2;
    }
    if (!g) {
      Py_INCREF(Py_None);
      g = Py_None;
    }
    PyList_SET_ITEM(out.ptr(), i, g);  // steals the reference
  }
  return py::make_tuple(out, py::bytes(src));
}

// data_ptr of each tensor (0 for None).
py::array_t<uint64_t> ptrs(const py::list& ts) {
  const Py_ssize_t n = PyList_GET_SIZE(ts.ptr());
  py::array_t<uint64_t> out(n);
  uint64_t* o = out.mutable_data();
  for (Py_ssize_t i = 0; i < n; ++i) {
    const at::Tensor* t = tensor_or_null(list_item(ts, i));
    o[i] = (t && t->defined()) ? reinterpret_cast<uint64_t>(t->data_ptr()) : 0u;
  }
  return out;
}

// Autograd version counter of each tensor (-1 for None).
py::array_t<int64_t> versions(const py::list& ts) {
  const Py_ssize_t n = PyList_GET_SIZE(ts.ptr());
  py::array_t<int64_t> out(n);
  int64_t* o = out.mutable_data();
  for (Py_ssize_t i = 0; i < n; ++i) {
    const at::Tensor* t = tensor_or_null(list_item(ts, i));
    o[i] = t ? static_cast<int64_t>(t->_version()) : -1;
  }
  return out;
}

// Sum of the version counters (versions only grow, so an in-place change raises it).
int64_t version_sum(const py::list& ts) {
  const Py_ssize_t n = PyList_GET_SIZE(ts.ptr());
  int64_t s = 0;
  for (Py_ssize_t i = 0; i < n; ++i) {
    const at::Tensor* t = tensor_or_null(list_item(ts, i));
    if (t) s += static_cast<int64_t>(t->_version());
  }
  return s;
}

// True if every entry is a dense (strided), contiguous tensor.
bool dense_contiguous(const py::list& ts) {
  const Py_ssize_t n = PyList_GET_SIZE(ts.ptr());
  for (Py_ssize_t i = 0; i < n; ++i) {
    const at::Tensor* t = tensor_or_null(list_item(ts, i));
    if (!t || !t->defined() || t->layout() != at::kStrided || !t->is_contiguous()) return false;
  }
  return true;
}

// True if both lists hold the same Python objects in the same order.
bool same(const py::list& a, const py::list& b) {
  const Py_ssize_t n = PyList_GET_SIZE(a.ptr());
  if (PyList_GET_SIZE(b.ptr()) != n) return false;
  for (Py_ssize_t i = 0; i < n; ++i)
    if (list_item(a, i) != list_item(b, i)) return false;
  return true;
}

// Grad-table fields of each tensor: (data_ptr uint64, numel int64, code uint8) with code 0
// for a dense contiguous bfloat16 tensor on a GPU, 1 for float32 likewise, 255 otherwise
// (the caller then reports the exact reason from Python).
py::tuple grad_fields(const py::list& ts) {
  const Py_ssize_t n = PyList_GET_SIZE(ts.ptr());
  py::array_t<uint64_t> ptr(n);
  py::array_t<int64_t> numel(n);
  py::array_t<uint8_t> code(n);
  uint64_t* pp = ptr.mutable_data();
  int64_t* pn = numel.mutable_data();
  uint8_t* pc = code.mutable_data();
  for (Py_ssize_t i = 0; i < n; ++i) {
    const at::Tensor* t = tensor_or_null(list_item(ts, i));
    const bool strided = t && t->defined() && t->layout() == at::kStrided;  // sparse ones have no data_ptr
    uint8_t c = 255;
    if (strided && t->is_cuda() && t->is_contiguous()) {
      const auto st = t->scalar_type();
      c = st == at::kBFloat16 ? 0 : (st == at::kFloat ? 1 : 255);
    }
    pc[i] = c;
    pp[i] = strided ? reinterpret_cast<uint64_t>(t->data_ptr()) : 0u;
    pn[i] = strided ? t->numel() : 0;
  }
  return py::make_tuple(ptr, numel, code);
}

// True if, for every i, state_map[params[i]] is states[i] and that dict's "exp_avg",
// "exp_avg_sq" and "step" entries are ms[i], vs[i] and ss[i] (object identity). A missing
// entry is a mismatch: the lookup does not run a defaultdict's factory.
bool states_same(const py::dict& state_map, const py::list& params, const py::list& states,
                 const py::list& ms, const py::list& vs, const py::list& ss) {
  const Py_ssize_t n = PyList_GET_SIZE(params.ptr());
  for (const py::list* l : {&states, &ms, &vs, &ss})
    if (PyList_GET_SIZE(l->ptr()) != n) return false;
  static PyObject* k_m = PyUnicode_InternFromString("exp_avg");
  static PyObject* k_v = PyUnicode_InternFromString("exp_avg_sq");
  static PyObject* k_s = PyUnicode_InternFromString("step");
  auto item = [](PyObject* d, PyObject* k) -> PyObject* {  // borrowed, or nullptr if absent
    PyObject* r = PyDict_GetItemWithError(d, k);
    if (!r && PyErr_Occurred()) throw py::error_already_set();
    return r;
  };
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* st = item(state_map.ptr(), list_item(params, i));
    if (!st || st != list_item(states, i) || !PyDict_Check(st)) return false;
    if (item(st, k_m) != list_item(ms, i) || item(st, k_v) != list_item(vs, i) ||
        item(st, k_s) != list_item(ss, i))
      return false;
  }
  return true;
}

// True if getattr(objs[i], name, None) is expected[i] for every i.
bool attrs_same(const py::list& objs, const py::str& name, const py::list& expected) {
  const Py_ssize_t n = PyList_GET_SIZE(objs.ptr());
  if (PyList_GET_SIZE(expected.ptr()) != n) return false;
  for (Py_ssize_t i = 0; i < n; ++i) {
    PyObject* a = PyObject_GetAttr(list_item(objs, i), name.ptr());  // new reference
    if (!a) {
      if (!PyErr_ExceptionMatches(PyExc_AttributeError)) throw py::error_already_set();
      PyErr_Clear();
      Py_INCREF(Py_None);
      a = Py_None;
    }
    const bool same_obj = a == list_item(expected, i);
    Py_DECREF(a);
    if (!same_obj) return false;
  }
  return true;
}

// Bumps the autograd version counter of every tensor, as an in-place op would.
void bump(const py::list& ts) {
  const Py_ssize_t n = PyList_GET_SIZE(ts.ptr());
  for (Py_ssize_t i = 0; i < n; ++i)
    if (const at::Tensor* t = tensor_or_null(list_item(ts, i))) torch::autograd::impl::bump_version(*t);
}

// Working-copy bookkeeping: works[i]._tm_master_version = params[i]._version and
// works[i]._tm_copy_version = works[i]._version, the versions read now. Views of one buffer
// share one counter, so a step that bumps several such masters raises each one's version by
// more than one: the versions are read back after the bumps rather than counted.
void stamp(const py::list& params, const py::list& works) {
  const Py_ssize_t n = PyList_GET_SIZE(params.ptr());
  if (PyList_GET_SIZE(works.ptr()) != n) throw py::value_error("params and works differ in length");
  static PyObject* k_master = PyUnicode_InternFromString("_tm_master_version");
  static PyObject* k_copy = PyUnicode_InternFromString("_tm_copy_version");
  for (Py_ssize_t i = 0; i < n; ++i) {
    const at::Tensor* p = tensor_or_null(list_item(params, i));
    const at::Tensor* w = tensor_or_null(list_item(works, i));
    if (!p || !w) throw py::value_error("torchure_amd._tm_host.stamp: None in a pair");
    for (auto [key, t] : {std::pair{k_master, p}, std::pair{k_copy, w}}) {
      PyObject* v = PyLong_FromLongLong(static_cast<long long>(t->_version()));
      if (!v) throw py::error_already_set();
      const int rc = PyObject_SetAttr(list_item(works, i), key, v);
      Py_DECREF(v);
      if (rc != 0) throw py::error_already_set();
    }
  }
}

// True if works[i]._tm_master_version equals params[i]._version for every i (the master has
// not been modified in place since its working copy was last written).
bool stamped(const py::list& params, const py::list& works) {
  const Py_ssize_t n = PyList_GET_SIZE(params.ptr());
  if (PyList_GET_SIZE(works.ptr()) != n) return false;
  static PyObject* k_master = PyUnicode_InternFromString("_tm_master_version");
  for (Py_ssize_t i = 0; i < n; ++i) {
    const at::Tensor* p = tensor_or_null(list_item(params, i));
    if (!p) return false;
    PyObject* a = PyObject_GetAttr(list_item(works, i), k_master);  // new reference
    if (!a) {
      if (!PyErr_ExceptionMatches(PyExc_AttributeError)) throw py::error_already_set();
      PyErr_Clear();
      return false;
    }
    const long long v = PyLong_Check(a) ? PyLong_AsLongLong(a) : -1;
    Py_DECREF(a);
    if (v == -1 && PyErr_Occurred()) PyErr_Clear();
    if (v != static_cast<long long>(p->_version())) return false;
  }
  return true;
}

}  // namespace

PYBIND11_MODULE(_tm_host, m) {
  m.doc() = "torchure_amd host-side list primitives (CPU only)";
  m.def("grads", &grads, "effective grad per master (p.grad or its working copy's grad)");
  m.def("ptrs", &ptrs, "data_ptr of each tensor (0 for None)");
  m.def("versions", &versions, "autograd version of each tensor (-1 for None)");
  m.def("version_sum", &version_sum, "sum of autograd versions");
  m.def("dense_contiguous", &dense_contiguous, "all dense and contiguous");
  m.def("same", &same, "element-wise object identity of two lists");
  m.def("bump", &bump, "bump the autograd version of each tensor");
  m.def("stamp", &stamp, "record each master's and working copy's current version on the copy");
  m.def("stamped", &stamped, "every working copy's recorded master version is the master's current one");
  m.def("grad_fields", &grad_fields, "(data_ptr, numel, dtype code) of each grad");
  m.def("states_same", &states_same, "optimizer state dicts and their tensors are the given objects");
  m.def("attrs_same", &attrs_same, "getattr(obj, name, None) of each object is the given object");
}
