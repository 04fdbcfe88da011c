// Host-side scan of a step plan's tensors, once per optimizer step.
//
// A step plan keeps raw device pointers of every parameter and grad in its
// descriptor table.  Before each launch it must know whether the table is still
// right: a grad may be a new tensor (zero_grad(set_to_none=True) every step),
// and a parameter or grad may have had its storage swapped in place
// (`p.data = ...`, `module.to(dtype)`), which keeps the Python objects and
// changes address and dtype.  Checking that from Python costs about 100 ns per
// attribute read per tensor; this scan reads the tensors directly (about 10 ns
// each), which matters for groups of tens of thousands of tensors.
//
// Plain CPython module (no pybind11): every function takes Python lists of
// torch tensors and the addresses of caller-owned numpy buffers.

#include <Python.h>

#include <cstdint>

#include <torch/csrc/autograd/python_variable.h>

namespace {

// scan status (mirrored in apexw_amd/_plan.py)
constexpr long kSame = 0;        // every pointer and dtype as recorded
constexpr long kGradsMoved = 1;  // only grad pointers changed (written to the scratch buffer)
constexpr long kMissing = 2;     // a plan parameter lost its grad, or another parameter gained one
constexpr long kRebuilt = 3;     // a parameter's storage or dtype changed
constexpr long kSlowPath = 4;    // a grad is laid out unlike its parameter, or of another size
constexpr long kGradDtype = 5;   // a grad's dtype differs from the one the table was built for

bool unpack_list(PyObject* obj, const char* what) {
  if (!PyList_Check(obj)) {
    PyErr_Format(PyExc_TypeError, "%s must be a list of tensors", what);
    return false;
  }
  const Py_ssize_t n = PyList_GET_SIZE(obj);
  for (Py_ssize_t i = 0; i < n; ++i) {
    if (!THPVariable_Check(PyList_GET_ITEM(obj, i))) {
      PyErr_Format(PyExc_TypeError, "%s[%zd] is not a tensor", what, i);
      return false;
    }
  }
  return true;
}

bool as_addr(PyObject* obj, uintptr_t* out) {
  *out = static_cast<uintptr_t>(PyLong_AsUnsignedLongLong(obj));
  return !PyErr_Occurred();
}

// snapshot(params, p_ptrs_addr, dtypes_addr)
//   p_ptrs: uint64[n] <- data pointers; dtypes: int8[n] <- at::ScalarType codes
PyObject* snapshot(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != 3) {
    PyErr_SetString(PyExc_TypeError, "snapshot(params, p_ptrs_addr, dtypes_addr)");
    return nullptr;
  }
  uintptr_t pa, da;
  if (!unpack_list(args[0], "params") || !as_addr(args[1], &pa) || !as_addr(args[2], &da)) return nullptr;
  auto* p_ptrs = reinterpret_cast<uint64_t*>(pa);
  auto* dtypes = reinterpret_cast<int8_t*>(da);
  const Py_ssize_t n = PyList_GET_SIZE(args[0]);
  for (Py_ssize_t i = 0; i < n; ++i) {
    const at::Tensor& p = THPVariable_Unpack(PyList_GET_ITEM(args[0], i));
    p_ptrs[i] = reinterpret_cast<uint64_t>(p.data_ptr());
    dtypes[i] = static_cast<int8_t>(p.scalar_type());
  }
  Py_RETURN_NONE;
}

// scan(params, inactive, p_ptrs_addr, dtypes_addr, g_ptrs_addr, g_scratch_addr, g_dtypes_addr) -> status
//   params: the plan's parameters, in table order; inactive: the group's other
//   trainable parameters.  g_ptrs holds the grad pointers the table was built
//   from; on kGradsMoved the current ones are in g_scratch.  g_dtypes: the grad
//   dtypes the table was built for (a grad may differ from its parameter's dtype:
//   torch's Tensor.grad_dtype).
PyObject* scan(PyObject*, PyObject* const* args, Py_ssize_t nargs) {
  if (nargs != 7) {
    PyErr_SetString(PyExc_TypeError, "scan(params, inactive, p_ptrs, dtypes, g_ptrs, g_scratch, g_dtypes)");
    return nullptr;
  }
  uintptr_t pa, da, ga, sa, gda;
  if (!unpack_list(args[0], "params") || !unpack_list(args[1], "inactive") || !as_addr(args[2], &pa) ||
      !as_addr(args[3], &da) || !as_addr(args[4], &ga) || !as_addr(args[5], &sa) || !as_addr(args[6], &gda))
    return nullptr;
  const auto* p_ptrs = reinterpret_cast<const uint64_t*>(pa);
  const auto* dtypes = reinterpret_cast<const int8_t*>(da);
  const auto* g_ptrs = reinterpret_cast<const uint64_t*>(ga);
  auto* g_scratch = reinterpret_cast<uint64_t*>(sa);
  const auto* g_dtypes = reinterpret_cast<const int8_t*>(gda);

  const Py_ssize_t n_in = PyList_GET_SIZE(args[1]);
  for (Py_ssize_t i = 0; i < n_in; ++i) {
    const at::Tensor& p = THPVariable_Unpack(PyList_GET_ITEM(args[1], i));
    if (p.grad().defined()) return PyLong_FromLong(kMissing);
  }
  const Py_ssize_t n = PyList_GET_SIZE(args[0]);
  bool moved = false, slow = false, gdt = false;
  for (Py_ssize_t i = 0; i < n; ++i) {
    const at::Tensor& p = THPVariable_Unpack(PyList_GET_ITEM(args[0], i));
    if (reinterpret_cast<uint64_t>(p.data_ptr()) != p_ptrs[i] || static_cast<int8_t>(p.scalar_type()) != dtypes[i])
      return PyLong_FromLong(kRebuilt);
    const at::Tensor& g = p.grad();
    if (!g.defined()) return PyLong_FromLong(kMissing);
    if (static_cast<int8_t>(g.scalar_type()) != g_dtypes[i]) {
      gdt = true;
      continue;
    }
    // the step walks the grad in its parameter's memory layout
    if (g.strides() != p.strides() || g.numel() != p.numel()) {
      slow = true;
      continue;
    }
    const uint64_t gp = reinterpret_cast<uint64_t>(g.data_ptr());
    g_scratch[i] = gp;
    moved |= gp != g_ptrs[i];
  }
  if (gdt) return PyLong_FromLong(kGradDtype);
  if (slow) return PyLong_FromLong(kSlowPath);
  return PyLong_FromLong(moved ? kGradsMoved : kSame);
}

PyMethodDef kMethods[] = {
    {"snapshot", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(snapshot)), METH_FASTCALL,
     "Record data pointers and dtypes of a list of tensors."},
    {"scan", reinterpret_cast<PyCFunction>(reinterpret_cast<void (*)()>(scan)), METH_FASTCALL,
     "Check a step plan's tensors against the recorded pointers; returns a status code."},
    {nullptr, nullptr, 0, nullptr},
};

PyModuleDef kModule = {PyModuleDef_HEAD_INIT, "_host", "Per-step host scan of step-plan tensors.", -1, kMethods};

}  // namespace

PyMODINIT_FUNC PyInit__host() { return PyModule_Create(&kModule); }
