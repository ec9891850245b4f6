// Implementation of the C ABI declared in include/xtile_amd.h.
//
// A module owns its IR and a cache of launch plans (one per function); any
// pass invalidates the cache.  xt_gpu_run checks the caller's buffers against
// the function's memref types before anything is enqueued, so a kernel never
// sees a buffer smaller than the extent its grid addresses.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <string>

#include "../../include/xtile_amd.h"
#include "ir.h"
#include "kernels/launch.h"
#include "plan.h"

struct xt_module {
  std::unique_ptr<xt::Module> ir;
  std::mutex mu;
  std::map<std::string, xt::Plan> plans;
};

namespace {

char* dup_string(const std::string& s) {
  char* out = static_cast<char*>(std::malloc(s.size() + 1));
  if (out) std::memcpy(out, s.c_str(), s.size() + 1);
  return out;
}

int fail(char** err, int status, const std::string& msg) {
  if (err) *err = dup_string(msg);
  return status;
}

std::string func_key(const char* func) { return func ? std::string(func) : std::string(); }

// Caller holds m->mu.
int get_plan(xt_module* m, const std::string& func, xt::Plan& out, char** err) {
  auto it = m->plans.find(func);
  if (it != m->plans.end()) {
    out = it->second;
    return XT_OK;
  }
  xt::Plan p;
  std::string why;
  if (!xt::build_plan(*m->ir, func, p, why)) return fail(err, XT_ERR_UNSUPPORTED, why);
  if (p.kind == xt::PlanKind::Fused && !xtk::compile_fused(*p.fused, why))
    return fail(err, XT_ERR_UNSUPPORTED, "@" + p.func + ": " + why);
  m->plans.emplace(func, p);
  out = p;
  return XT_OK;
}

}  // namespace

extern "C" {

void xt_free(void* p) { std::free(p); }

const char* xt_version(void) { return "xtile_amd 0.1 (gfx950)"; }

int xt_module_parse(const char* text, size_t len, xt_module** out, char** err) {
  if (!out) return fail(err, XT_ERR_TYPE, "xt_module_parse: null output handle");
  *out = nullptr;
  if (!text && len) return fail(err, XT_ERR_TYPE, "xt_module_parse: null text");
  xt::Diag diag;
  auto ir = xt::parse_module(std::string(text ? text : "", len), diag);
  if (!ir) return fail(err, XT_ERR_PARSE, diag.joined());
  auto* m = new xt_module;
  m->ir = std::move(ir);
  *out = m;
  return XT_OK;
}

void xt_module_free(xt_module* m) { delete m; }

int xt_module_print(xt_module* m, char** out_text, char** err) {
  if (!m || !out_text) return fail(err, XT_ERR_TYPE, "expected an xtile module");
  std::lock_guard<std::mutex> lock(m->mu);
  *out_text = dup_string(xt::print_module(*m->ir));
  return XT_OK;
}

int xt_pass_run(xt_module* m, const char* pass, char** err) {
  if (!m) return fail(err, XT_ERR_TYPE, "expected an xtile module");
  std::string name = pass ? pass : "";
  std::lock_guard<std::mutex> lock(m->mu);
  m->plans.clear();
  xt::Diag diag;
  bool ok;
  if (name == "xt-serialize") ok = xt::pass_xt_serialize(*m->ir, diag);
  else if (name == "canonicalize") ok = xt::pass_canonicalize(*m->ir, diag);
  else if (name == "xt-to-nova") ok = xt::pass_xt_to_nova(*m->ir, diag);
  else return fail(err, XT_ERR_TYPE, "unknown pass '" + name + "'");
  if (ok) ok = xt::verify_module(*m->ir, diag);
  if (!ok) {
    std::string msg = diag.joined();
    if (msg.empty()) msg = "xtile." + name + " failed";
    return fail(err, XT_ERR_PASS, msg);
  }
  return XT_OK;
}

int xt_module_num_funcs(xt_module* m) {
  if (!m) return -1;
  std::lock_guard<std::mutex> lock(m->mu);
  return static_cast<int>(m->ir->funcs.size());
}

const char* xt_module_func_name(xt_module* m, int index) {
  if (!m) return nullptr;
  std::lock_guard<std::mutex> lock(m->mu);
  if (index < 0 || index >= static_cast<int>(m->ir->funcs.size())) return nullptr;
  return m->ir->funcs[index].name.c_str();
}

int xt_func_signature(xt_module* m, const char* func, char** out_json, char** err) {
  if (!m || !out_json) return fail(err, XT_ERR_TYPE, "expected an xtile module");
  std::lock_guard<std::mutex> lock(m->mu);
  const xt::Func* f = nullptr;
  std::string name = func_key(func);
  if (name.empty()) {
    if (m->ir->funcs.size() != 1)
      return fail(err, XT_ERR_ARGUMENT, "module has several functions; name one");
    f = &m->ir->funcs[0];
  } else {
    f = xt::find_func(*m->ir, name);
  }
  if (!f) return fail(err, XT_ERR_ARGUMENT, "no function named @" + name);
  std::ostringstream os;
  os << "{\"name\": \"" << f->name << "\", \"grid\": ";
  int32_t g[3];
  if (xt::get_grid(*f, g)) os << "[" << g[0] << ", " << g[1] << ", " << g[2] << "]";
  else os << "null";
  os << ", \"args\": [";
  for (size_t k = 0; k < f->args.size(); ++k) {
    const xt::Type& t = f->type_of(f->args[k]);
    os << (k ? ", " : "") << "{\"kind\": \""
       << (t.is_memref() ? "memref" : t.is_tensor() ? "tensor" : "scalar") << "\", \"dtype\": \""
       << xt::elem_name(t.elem) << "\", \"shape\": [";
    for (size_t d = 0; d < t.shape.size(); ++d) os << (d ? ", " : "") << t.shape[d];
    os << "]}";
  }
  os << "]}";
  *out_json = dup_string(os.str());
  return XT_OK;
}

int xt_plan(xt_module* m, const char* func, char** out_desc, double* algo_bytes,
            double* algo_flops, char** err) {
  if (!m) return fail(err, XT_ERR_TYPE, "expected an xtile module");
  xt::Plan p;
  {
    std::lock_guard<std::mutex> lock(m->mu);
    int st = get_plan(m, func_key(func), p, err);
    if (st != XT_OK) return st;
  }
  if (out_desc) *out_desc = dup_string(p.describe());
  if (algo_bytes) *algo_bytes = p.algo_bytes;
  if (algo_flops) *algo_flops = p.algo_flops;
  return XT_OK;
}

int xt_gpu_run(xt_module* m, const char* func, void* const* bufs, const size_t* buf_bytes,
               int nbufs, void* stream, char** err) {
  if (!m) return fail(err, XT_ERR_TYPE, "expected an xtile module");
  xt::Plan p;
  {
    std::lock_guard<std::mutex> lock(m->mu);
    int st = get_plan(m, func_key(func), p, err);
    if (st != XT_OK) return st;
  }
  if (nbufs != static_cast<int>(p.arg_types.size()))
    return fail(err, XT_ERR_ARGUMENT,
                "@" + p.func + " takes " + std::to_string(p.arg_types.size()) +
                    " buffers, got " + std::to_string(nbufs));
  if (!bufs || !buf_bytes) return fail(err, XT_ERR_ARGUMENT, "null buffer list");
  for (int k = 0; k < nbufs; ++k) {
    const xt::Type& t = p.arg_types[k];
    size_t need = static_cast<size_t>(t.numel()) * xt::elem_bytes(t.elem);
    if (!bufs[k]) return fail(err, XT_ERR_ARGUMENT, "buffer " + std::to_string(k) + " is null");
    if (buf_bytes[k] < need)
      return fail(err, XT_ERR_ARGUMENT,
                  "buffer " + std::to_string(k) + " holds " + std::to_string(buf_bytes[k]) +
                      " bytes; " + t.str() + " needs " + std::to_string(need));
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  std::string why;
  hipError_t e = hipSuccess;
  switch (p.kind) {
    case xt::PlanKind::EwBinary: e = xtk::launch_ew_binary(p, bufs, s, why); break;
    case xt::PlanKind::RowSoftmax: e = xtk::launch_row_softmax(p, bufs, s, why); break;
    case xt::PlanKind::Gemm: e = xtk::launch_gemm(p, bufs, s, why); break;
    case xt::PlanKind::Conv2d: e = xtk::launch_conv2d(p, bufs, s, why); break;
    case xt::PlanKind::TileVM: e = xtk::launch_tilevm(p, bufs, s, why); break;
    case xt::PlanKind::Fused: e = xtk::launch_fused(p, bufs, s, why); break;
  }
  if (!why.empty()) return fail(err, XT_ERR_ARGUMENT, why);
  if (e != hipSuccess)
    return fail(err, XT_ERR_DEVICE,
                std::string("HIP launch failed: ") + hipGetErrorString(e) + " (" + p.describe() +
                    ")");
  return XT_OK;
}

}  // extern "C"
