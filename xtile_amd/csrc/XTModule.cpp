// The compiled Python module `_xtile` over the C ABI of include/xtile_amd.h.
//
// Stands in for the reference's nanobind module of the same name
// (python/XTModule.cpp:210-231): the same function names, keyword names and
// exception types, with every call going through the C ABI instead of MLIR.
//
//   parse(asm) / _parse_module(asm)  a PyCapsule owning the module
//                                    (XTModule.cpp:112-126, capsule :82-110);
//                                    ValueError("failed to parse test module")
//   xt_serialize(module)             the same object back; RuntimeError with the
//                                    newline-joined diagnostics (runPass :128-151)
//   xt_to_nova(module)               the restated lowering, IR only (:154-159)
//   nova_optimize / nova_allocate / nova_threading / nova_barrier / nova_to_x1
//                                    NotImplementedError: the x1 NPU lowering has
//                                    no counterpart on the GPU (:169-207)
//   _module_asm(module)              the module's text (:228-230)
//
// `module` is the capsule itself or any object whose `_CAPIPtr` attribute is
// one (getCapsuleFromModuleObject, :37-51); anything else is a TypeError.
// What the GPU backend adds: canonicalize, func_names, signature, plan,
// launch and version.  The pybind11 form (nanobind is not installed here)
// differs from a nanobind one in the binding macros only.
//
// Load it after `import torch`: the library's HIP runtime must be the one
// torch already mapped (same SONAME), or the process holds two runtimes.

#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "xtile_amd.h"

namespace py = pybind11;

namespace {

constexpr const char* kCapsuleName = "xtile_amd.xt_module";

// Takes ownership of a string the library returned.
std::string take(char* s) {
  std::string r = s ? s : "";
  xt_free(s);
  return r;
}

[[noreturn]] void raise_status(int st, const std::string& msg, const std::string& fallback) {
  const std::string text = msg.empty() ? fallback : msg;
  switch (st) {
    case XT_ERR_PARSE:
      throw py::value_error("failed to parse test module" + (msg.empty() ? std::string() : "\n" + msg));
    case XT_ERR_TYPE:
      throw py::type_error(text);
    case XT_ERR_UNSUPPORTED:
      PyErr_SetString(PyExc_NotImplementedError, text.c_str());
      throw py::error_already_set();
    case XT_ERR_ARGUMENT:
      throw py::value_error(text);
    default:
      throw std::runtime_error(text);
  }
}

xt_module* unwrap(py::handle obj) {
  py::object cap;
  if (PyCapsule_CheckExact(obj.ptr()))
    cap = py::reinterpret_borrow<py::object>(obj);
  else if (py::hasattr(obj, "_CAPIPtr"))
    cap = obj.attr("_CAPIPtr");
  if (!cap || !PyCapsule_IsValid(cap.ptr(), kCapsuleName)) throw py::type_error("expected an xtile module object");
  return static_cast<xt_module*>(PyCapsule_GetPointer(cap.ptr(), kCapsuleName));
}

void free_capsule(PyObject* cap) {
  xt_module_free(static_cast<xt_module*>(PyCapsule_GetPointer(cap, kCapsuleName)));
}

py::object parse(py::object text) {
  if (!PyUnicode_Check(text.ptr())) throw py::type_error("asm must be a str");
  const std::string data = text.cast<std::string>();
  xt_module* m = nullptr;
  char* err = nullptr;
  const int st = xt_module_parse(data.data(), data.size(), &m, &err);
  const std::string msg = take(err);
  if (st != XT_OK) raise_status(st, msg, "failed to parse test module");
  PyObject* cap = PyCapsule_New(m, kCapsuleName, free_capsule);
  if (!cap) {
    xt_module_free(m);
    throw py::error_already_set();
  }
  return py::reinterpret_steal<py::object>(cap);
}

py::object run_pass(py::object module, const char* pass) {
  xt_module* m = unwrap(module);
  char* err = nullptr;
  const int st = xt_pass_run(m, pass, &err);
  const std::string msg = take(err);
  if (st != XT_OK) {
    std::string name = pass;
    for (char& c : name)
      if (c == '-') c = '_';
    raise_status(st, msg, "xtile." + name + " failed");
  }
  return module;
}

// A stage of the reference's x1 NPU lowering: the argument is checked as
// runPass checks it, then the stage is refused.
py::object x1_stage(py::object module, const char* name) {
  unwrap(module);
  const std::string text = std::string(name) +
                           " belongs to the reference's x1 NPU lowering, which the MI355X backend replaces "
                           "with HIP kernels; use xt.compile / xt.launch";
  PyErr_SetString(PyExc_NotImplementedError, text.c_str());
  throw py::error_already_set();
}

std::string module_asm(py::object module) {
  xt_module* m = unwrap(module);
  char* out = nullptr;
  char* err = nullptr;
  const int st = xt_module_print(m, &out, &err);
  const std::string msg = take(err);
  std::string text = take(out);
  if (st != XT_OK) raise_status(st, msg, "printing failed");
  return text;
}

std::vector<std::string> func_names(py::object module) {
  xt_module* m = unwrap(module);
  std::vector<std::string> names;
  const int n = xt_module_num_funcs(m);
  for (int k = 0; k < n; ++k) names.emplace_back(xt_module_func_name(m, k));
  return names;
}

std::string func_arg(const py::object& func) { return func.is_none() ? std::string() : func.cast<std::string>(); }

py::object signature(py::object module, py::object func) {
  xt_module* m = unwrap(module);
  const std::string f = func_arg(func);
  char* out = nullptr;
  char* err = nullptr;
  const int st = xt_func_signature(m, f.c_str(), &out, &err);
  const std::string msg = take(err);
  const std::string json = take(out);
  if (st != XT_OK) raise_status(st, msg, "signature failed");
  return py::module_::import("json").attr("loads")(json);
}

py::tuple plan(py::object module, py::object func) {
  xt_module* m = unwrap(module);
  const std::string f = func_arg(func);
  char* out = nullptr;
  char* err = nullptr;
  double nbytes = 0, nflops = 0;
  int st;
  {
    // planning a fused program compiles it (hiprtc): other threads may run
    py::gil_scoped_release nogil;
    st = xt_plan(m, f.c_str(), &out, &nbytes, &nflops, &err);
  }
  const std::string msg = take(err);
  const std::string desc = take(out);
  if (st != XT_OK) raise_status(st, msg, "planning failed");
  return py::make_tuple(desc, nbytes, nflops);
}

void launch(py::object module, py::object func, const std::vector<uintptr_t>& ptrs, const std::vector<size_t>& sizes,
            uintptr_t stream) {
  xt_module* m = unwrap(module);
  if (ptrs.size() != sizes.size()) throw py::value_error("ptrs and sizes differ in length");
  const std::string f = func_arg(func);
  std::vector<void*> bufs(ptrs.size());
  for (size_t i = 0; i < ptrs.size(); ++i) bufs[i] = reinterpret_cast<void*>(ptrs[i]);
  char* err = nullptr;
  int st;
  {
    py::gil_scoped_release nogil;
    st = xt_gpu_run(m, f.c_str(), bufs.data(), sizes.data(), (int)bufs.size(), reinterpret_cast<void*>(stream),
                    &err);
  }
  const std::string msg = take(err);
  if (st != XT_OK) raise_status(st, msg, "launch failed");
}

}  // namespace

PYBIND11_MODULE(_xtile, m) {
  m.doc() = "xtile module functions over the xtile_amd C ABI (MI355X backend)";
  m.def("parse", &parse, py::arg("asm"), "Parse xt text into a module capsule.");
  m.def("_parse_module", &parse, py::arg("asm"));
  m.def(
      "xt_to_nova", [](py::object mod) { return run_pass(mod, "xt-to-nova"); }, py::arg("module"),
      "Run the xt-to-nova lowering in place (IR only) and return the module.");
  m.def(
      "xt_serialize", [](py::object mod) { return run_pass(mod, "xt-serialize"); }, py::arg("module"),
      "Unroll the grid in place and return the module.");
  m.def(
      "canonicalize", [](py::object mod) { return run_pass(mod, "canonicalize"); }, py::arg("module"),
      "Fold x+0 / x-0 and drop dead pure ops in place; returns the module.");
  for (const char* name : {"nova_optimize", "nova_allocate", "nova_threading", "nova_barrier", "nova_to_x1"})
    m.def(
        name, [name](py::object mod) { return x1_stage(mod, name); }, py::arg("module"),
        "A stage of the x1 NPU lowering: raises NotImplementedError.");
  m.def("_module_asm", &module_asm, py::arg("module"));
  m.def("func_names", &func_names, py::arg("module"));
  m.def("signature", &signature, py::arg("module"), py::arg("func") = py::none());
  m.def("plan", &plan, py::arg("module"), py::arg("func") = py::none(),
        "(kernel description, algorithmic bytes, algorithmic FLOPs) of one launch.");
  m.def("launch", &launch, py::arg("module"), py::arg("func"), py::arg("ptrs"), py::arg("sizes"),
        py::arg("stream") = 0, "Enqueue func on stream (a hipStream_t as an integer) over device pointers.");
  m.def("version", []() { return std::string(xt_version()); });
}
