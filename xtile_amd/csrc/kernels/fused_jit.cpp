// Compiling and launching fused tile programs (fused.cpp writes their source).
//
// hiprtc compiles a program's kernel for gfx950 when its plan is built (no GPU
// is needed for that), with the flags of every other kernel of the library.
// Code objects are kept in memory by source, and on disk under `jit/` beside
// the library with their source (XTILE_AMD_JIT_CACHE names another directory,
// "off" turns the disk cache off), so a program is compiled once per machine.
// A launch loads the code object once per device (hipModuleLoadData) and
// enqueues `xt_fused` on the caller's stream.
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <map>
#include <mutex>
#include <sstream>

#include "launch.h"

namespace xtk {
namespace {

const char* kOptions[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
                          "-Xclang",               "-packed-fp32-ops"};

std::mutex g_mu;
std::map<std::string, std::string> g_code;                          // source -> code object
std::map<std::pair<uint64_t, int>, hipFunction_t> g_func;           // (source hash, device) -> kernel

uint64_t fnv1a(const std::string& s, uint64_t h = 1469598103934665603ull) {
  for (unsigned char c : s) h = (h ^ c) * 1099511628211ull;
  return h;
}

std::string cache_dir() {
  const char* env = std::getenv("XTILE_AMD_JIT_CACHE");
  if (env) return std::string(env) == "off" ? std::string() : std::string(env);
  Dl_info info;
  if (!dladdr(reinterpret_cast<void*>(&cache_dir), &info) || !info.dli_fname) return std::string();
  std::string lib(info.dli_fname);
  const size_t slash = lib.rfind('/');
  return (slash == std::string::npos ? std::string(".") : lib.substr(0, slash)) + "/jit";
}

std::string cache_key(const std::string& src) {
  std::string all = src;
  for (const char* o : kOptions) all += std::string("\n//") + o;
  char buf[40];
  std::snprintf(buf, sizeof(buf), "%016llx", static_cast<unsigned long long>(fnv1a(all)));
  return std::string(buf) + "_" + std::to_string(HIP_VERSION);
}

bool read_file(const std::string& path, std::string& out) {
  std::ifstream f(path, std::ios::binary);
  if (!f) return false;
  std::ostringstream ss;
  ss << f.rdbuf();
  out = ss.str();
  return !out.empty();
}

void write_file(const std::string& dir, const std::string& name, const std::string& data) {
  if (dir.empty()) return;
  mkdir(dir.c_str(), 0755);
  const std::string tmp = dir + "/" + name + ".tmp" + std::to_string(getpid());
  {
    std::ofstream f(tmp, std::ios::binary);
    if (!f) return;
    f.write(data.data(), static_cast<std::streamsize>(data.size()));
    if (!f) return;
  }
  std::rename(tmp.c_str(), (dir + "/" + name).c_str());
}

bool rtc(const std::string& src, std::string& code, std::string& err) {
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), "xt_fused.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS) {
    err = "hiprtc could not create the fused program";
    return false;
  }
  const hiprtcResult r = hiprtcCompileProgram(prog, static_cast<int>(sizeof(kOptions) / sizeof(kOptions[0])),
                                              kOptions);
  if (r != HIPRTC_SUCCESS) {
    size_t n = 0;
    hiprtcGetProgramLogSize(prog, &n);
    std::string log(n, '\0');
    if (n) hiprtcGetProgramLog(prog, &log[0]);
    err = std::string("hiprtc failed to compile the fused kernel: ") + hiprtcGetErrorString(r) + "\n" + log;
    hiprtcDestroyProgram(&prog);
    return false;
  }
  size_t n = 0;
  hiprtcGetCodeSize(prog, &n);
  code.assign(n, '\0');
  const bool ok = n > 0 && hiprtcGetCode(prog, &code[0]) == HIPRTC_SUCCESS;
  hiprtcDestroyProgram(&prog);
  if (!ok) err = "hiprtc returned no code object for the fused kernel";
  return ok;
}

}  // namespace

bool compile_fused(xt::FusedPlan& fp, std::string& err) {
  std::lock_guard<std::mutex> lock(g_mu);
  fp.id = fnv1a(fp.source);
  auto it = g_code.find(fp.source);
  if (it != g_code.end()) {
    fp.code = it->second;
    return true;
  }
  const std::string dir = cache_dir(), key = cache_key(fp.source);
  std::string code;
  if (dir.empty() || !read_file(dir + "/" + key + ".co", code)) {
    if (!rtc(fp.source, code, err)) return false;
    write_file(dir, key + ".co", code);
    write_file(dir, key + ".hip", fp.source);  // the source beside its code object, for reading
  }
  g_code.emplace(fp.source, code);
  fp.code = std::move(code);
  return true;
}

namespace {

// Index of the first access whose buffer is not aligned to vw elements, or -1.
int misaligned(const xt::VmPlan& vm, void* const* bufs, int vw, uintptr_t& align) {
  for (size_t k = 0; k < vm.access.size(); ++k) {
    const xt::VmAccess& a = vm.access[k];
    align = static_cast<uintptr_t>(vw) * xt::elem_bytes(a.elem);
    if (reinterpret_cast<uintptr_t>(bufs[a.arg]) % align) return static_cast<int>(a.arg);
  }
  return -1;
}

std::mutex g_scalar_mu;

// The plan's scalar-access variant, generated and compiled on first use
// (nullptr, with `err`, when the program does not fit the fused layout with
// vw = 1 or does not compile).
const xt::FusedPlan* scalar_variant(const xt::Plan& p, std::string& err) {
  xt::FusedPlan* fp = p.fused.get();
  std::lock_guard<std::mutex> lock(g_scalar_mu);
  if (!fp->scalar) {
    auto sp = std::make_shared<xt::FusedPlan>();
    const bool built = fp->staged ? xt::stage_vm(p.vm, p.grid, *sp, err, 1) : xt::fuse_vm(p.vm, p.grid, *sp, err, 1);
    if (!built || !compile_fused(*sp, err)) return nullptr;
    fp->scalar = std::move(sp);
  }
  return fp->scalar.get();
}

}  // namespace

hipError_t launch_fused(const xt::Plan& p, void* const* bufs, hipStream_t s, std::string& why) {
  const xt::FusedPlan* fp = p.fused.get();
  if (!fp || fp->code.empty()) {
    why = "fused plan has no compiled kernel";
    return hipErrorInvalidValue;
  }
  const xt::VmPlan& vm = p.vm;
  if (vm.access.size() > 8) {
    why = "fused kernels take at most 8 memref accesses";
    return hipErrorInvalidValue;
  }
  // Row accesses are vw-element vectors.  A buffer not aligned to one runs
  // the program's scalar-access variant (vw = 1), or the interpreter when
  // that variant does not fit the fused layout.
  uintptr_t align = 0;
  int bad = misaligned(vm, bufs, fp->vw, align);
  if (bad >= 0 && fp->vw > 1) {
    std::string err;
    const xt::FusedPlan* sp = scalar_variant(p, err);
    if (sp) {
      fp = sp;
      bad = misaligned(vm, bufs, 1, align);
    } else if (p.vm_fallback) {
      return launch_tilevm(p, bufs, s, why);
    } else {
      why = "buffer " + std::to_string(bad) + " is not aligned to " + std::to_string(align) +
            " bytes, which the fused kernel's row vectors need; its scalar variant: " + err +
            "; the tile interpreter: " + p.vm_fallback_why;
      return hipErrorInvalidValue;
    }
  }
  if (bad >= 0) {
    if (p.vm_fallback) return launch_tilevm(p, bufs, s, why);
    why = "buffer " + std::to_string(bad) + " is not aligned to its " + std::to_string(align) + "-byte elements";
    return hipErrorInvalidValue;
  }
  const long long blocks = static_cast<long long>(p.grid[0]) * p.grid[1] * p.grid[2];
  if (blocks < 1 || blocks > 0x7fffffffLL || blocks * fp->threads >= (1LL << 32)) {
    why = "fused kernel grid of " + std::to_string(blocks) + " blocks is out of range";
    return hipErrorInvalidValue;
  }
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  hipFunction_t fn = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_mu);
    auto key = std::make_pair(fp->id, dev);
    auto it = g_func.find(key);
    if (it == g_func.end()) {
      hipModule_t mod = nullptr;
      e = hipModuleLoadData(&mod, fp->code.data());
      if (e != hipSuccess) return e;
      e = hipModuleGetFunction(&fn, mod, "xt_fused");
      if (e != hipSuccess) return e;
      g_func.emplace(key, fn);  // the module stays loaded until the process ends
    } else {
      fn = it->second;
    }
  }
  struct {
    void* p[8];
  } args = {};
  for (size_t k = 0; k < vm.access.size(); ++k) args.p[k] = bufs[vm.access[k].arg];
  void* params[] = {&args};
  if (fp->workgroups < 1 || fp->workgroups > blocks) {
    why = "fused kernel launch size out of range";
    return hipErrorInvalidValue;
  }
  return hipModuleLaunchKernel(fn, static_cast<unsigned>(fp->workgroups), 1, 1, static_cast<unsigned>(fp->threads), 1, 1, 0,
                               s, params, nullptr);
}

}  // namespace xtk
