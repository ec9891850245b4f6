// Staged tile programs: the tile interpreter's lowering of a program (VmPlan)
// that the register-resident fused kernel declines - matmul / mma, transposes
// and permutes, values of several shapes - turned into the source of one HIP
// kernel.  The runtime compiles it with hiprtc (kernels/fused_jit.cpp) and
// launches it like a fused kernel.
//
// Execution.  One 256-thread workgroup (four waves) runs one Block.  Values
// live in LDS as f32, as the interpreter and the oracle hold them; every
// instruction is straight-line code with its shapes, strides and tile origins
// as compile-time constants, and a barrier separates an instruction from the
// next one that reads what it wrote or writes where it read.  A run of loads
// issues every global read before its first LDS write.
//   * matmul / mma: 32 x 32 output tiles dealt over the four waves, K in MFMA
//     steps: v_mfma_f32_32x32x16_f16 / _bf16 when both operands are f16 / bf16
//     tiles as loaded (or transposed / permuted: the values are then exact in
//     that type), v_mfma_i32_32x32x32_i8 with exact i32 sums for the
//     interpreter's exact i8 x i8 products, v_mfma_f32_32x32x2_f32 otherwise;
//     fragments are read from LDS and converted (exactly) in registers.  The
//     mma accumulator is added to the finished sum, as the interpreter does.
//   * reductions along a row: a power-of-two group of lanes per row with a
//     shuffle butterfly; along a column: one thread per column.
//   * permute / transpose: one thread per output element.
//
// LDS layout.  The generator allocates its own slots (liveness, first fit,
// 16-byte granules): a value of n elements is stored as rows of `krow`
// elements `pitch` apart in the value's row-major element order, so reshapes
// keep their meaning.  krow = pitch = the innermost dim, except for
//   * matmul operands: A[M, K] with krow = K, pitch = K rounded up to 4 mod 8
//     (f16 / bf16 / i8: the 16-byte fragment reads of sixteen rows fall in
//     sixteen distinct bank groups) or to 2 mod 4 (f32: 32 rows of single
//     floats in distinct banks); B[K, N] with krow = N, pitch 4 mod 8 for the
//     narrow types (the two half-waves' rows, 8 or 16 apart, in distinct banks);
//   * the source of a permute: an odd pitch (a column read is conflict-free).
// The first consumer in program order decides.
#include <algorithm>
#include <functional>
#include <map>
#include <sstream>
#include <vector>

#include "fused_common.h"
#include "plan.h"

namespace xt {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxLdsFloats = 160 * 1024 / 4;

enum MmMode { kMmF32 = 0, kMmF16 = 1, kMmBF16 = 2, kMmI8 = 3 };
// what a value is known to hold exactly: any f32, or values of a narrow type
enum VType { kVF32 = 0, kVF16 = 1, kVBF16 = 2, kVI8 = 3 };

struct Val {
  int def = -1, last = -1;  // producing instruction, last reader
  long long numel = 0;
  int d2 = 1;               // innermost dim at the definition
  int krow = 0, pitch = 0;  // layout (0: not chosen yet)
  int off = -1;             // LDS float offset
  int vt = kVF32;
  long long floats() const { return numel / krow * pitch; }
};

struct Reads {
  int a = -1, b = -1, c = -1, dst = -1;  // value ids
  int mode = kMmF32;                     // matmul
};

int pad_to(int k, int mod, int rem) { return k + ((rem - k % mod) % mod + mod) % mod; }

std::string S(long long v) { return std::to_string(v); }

class StagedGen {
 public:
  StagedGen(const VmPlan& vm, const int32_t grid[3], int max_vw) : vm_(vm), max_vw_(max_vw) {
    for (int d = 0; d < 3; ++d) grid_[d] = grid[d];
  }

  bool run(FusedPlan& out, std::string& why) {
    if (!analyze(why) || !layouts(why) || !allocate(why)) return false;
    std::ostringstream b;
    const size_t n = vm_.inst.size();
    size_t i = 0;
    bool any_mm[4] = {false, false, false, false};
    while (i < n) {
      const VmInst& in = vm_.inst[i];
      if (in.op == VmOp::Load) {
        // a run of loads: every global read, then every LDS write
        size_t j = i;
        int regs = 0;
        while (j < n && vm_.inst[j].op == VmOp::Load) {
          const int r = load_regs(static_cast<int>(j));
          if (j > i && regs + r > 128) break;
          regs += r;
          ++j;
        }
        for (size_t k = i; k < j; ++k) emit_load_read(b, static_cast<int>(k));
        for (size_t k = i; k < j; ++k) emit_load_write(b, static_cast<int>(k));
        i = j;
      } else {
        switch (in.op) {
          case VmOp::Store: emit_store(b, static_cast<int>(i)); break;
          case VmOp::Unary:
          case VmOp::Binary: emit_elementwise(b, static_cast<int>(i)); break;
          case VmOp::Reduce: emit_reduce(b, static_cast<int>(i)); break;
          case VmOp::Permute: emit_permute(b, static_cast<int>(i)); break;
          case VmOp::Matmul:
            emit_matmul(b, static_cast<int>(i));
            any_mm[rd_[i].mode] = true;
            break;
          default: why = "staged kernels take the interpreter's instructions"; return false;
        }
        ++i;
      }
      if (i < n) {
        // stores only read LDS and loads write distinct live slots: no
        // barrier between two of a kind
        const VmOp prev = vm_.inst[i - 1].op, next = vm_.inst[i].op;
        if (!((prev == VmOp::Store && next == VmOp::Store))) b << "  __syncthreads();\n";
      }
    }
    std::ostringstream k;
    k << "typedef float xf16v __attribute__((ext_vector_type(16)));\n"
      << "typedef int xi16v __attribute__((ext_vector_type(16)));\n"
      << "typedef int xi4v __attribute__((ext_vector_type(4)));\n"
      << "typedef _Float16 xh8 __attribute__((ext_vector_type(8)));\n"
      << "typedef short xs8 __attribute__((ext_vector_type(8)));\n"
      << "typedef __bf16 xb8 __attribute__((ext_vector_type(8)));\n";
    k << "extern \"C\" __global__ void __launch_bounds__(" << kThreads << ") xt_fused(FusedArgs a) {\n"
      << "#pragma clang fp contract(off)\n"
      << "  __shared__ __attribute__((aligned(16))) float S[" << std::max(4LL, high_) << "];\n"
      << "  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);\n"
      << "  (void)lane; (void)wave;\n"
      << "  const int bid = blockIdx.x;\n"
      << "  const int x = bid % " << grid_[0] << ", y = (bid / " << grid_[0] << ") % " << grid_[1]
      << ", z = bid / " << (long long)grid_[0] * grid_[1] << ";\n"
      << "  (void)x; (void)y; (void)z;\n";
    k << b.str() << "}\n";
    out.source = std::string(fused_preamble()) + k.str();
    out.threads = kThreads;
    out.vw = gvw_max_;
    out.staged = true;
    const long long blocks = (long long)grid_[0] * grid_[1] * grid_[2];
    out.workgroups = static_cast<int>(blocks);
    std::ostringstream lay;
    lay << "staged f32 threads=" << kThreads << " lds=" << high_ * 4 << "B";
    const char* names[4] = {"f32", "f16", "bf16", "i8"};
    std::string mm;
    for (int m = 0; m < 4; ++m)
      if (any_mm[m]) mm += (mm.empty() ? "" : ",") + std::string(names[m]);
    if (!mm.empty()) lay << " mfma=" << mm;
    out.layout = lay.str();
    return true;
  }

 private:
  const VmPlan& vm_;
  int max_vw_ = 4;
  int grid_[3];
  std::vector<Val> vals_;
  std::vector<Reads> rd_;
  long long high_ = 0;
  int gvw_max_ = 1;

  static bool fail(std::string& why, const std::string& msg) {
    why = msg;
    return false;
  }

  int new_val(int def, long long numel, int d2, int vt) {
    Val v;
    v.def = v.last = def;
    v.numel = numel;
    v.d2 = d2;
    v.vt = vt;
    vals_.push_back(v);
    return static_cast<int>(vals_.size()) - 1;
  }

  static long long prod(const int d[3]) { return (long long)d[0] * d[1] * d[2]; }

  bool analyze(std::string& why) {
    std::map<int, int> cur;  // LDS slot offset of the interpreter -> value id
    rd_.assign(vm_.inst.size(), Reads{});
    for (size_t i = 0; i < vm_.inst.size(); ++i) {
      const VmInst& in = vm_.inst[i];
      Reads& r = rd_[i];
      auto rd = [&](int slot, int& out) {
        auto it = cur.find(slot);
        if (it == cur.end()) return false;
        out = it->second;
        vals_[out].last = static_cast<int>(i);
        return true;
      };
      switch (in.op) {
        case VmOp::Load: {
          const Elem e = vm_.access[in.kind].elem;
          const int vt = e == Elem::F16 ? kVF16 : e == Elem::BF16 ? kVBF16 : e == Elem::I8 ? kVI8 : kVF32;
          r.dst = new_val(static_cast<int>(i), prod(in.dims), in.dims[2], vt);
          break;
        }
        case VmOp::Store:
          if (!rd(in.a, r.a)) return fail(why, "store of an unknown value");
          break;
        case VmOp::Unary:
          if (!rd(in.a, r.a)) return fail(why, "unary op of an unknown value");
          r.dst = new_val(static_cast<int>(i), prod(in.dims), in.dims[2],
                          in.kind == static_cast<int16_t>(VmUnary::Ftoi) ? kVI8 : kVF32);
          break;
        case VmOp::Binary:
          if (!rd(in.a, r.a) || !rd(in.b, r.b)) return fail(why, "binary op of an unknown value");
          r.dst = new_val(static_cast<int>(i), prod(in.dims), in.dims[2], kVF32);
          break;
        case VmOp::Reduce: {
          if (!rd(in.a, r.a)) return fail(why, "reduction of an unknown value");
          if (in.dims[0] != 1) return fail(why, "reductions take rank-2 tiles");
          const bool rows = in.aux[0] == 1;
          r.dst = new_val(static_cast<int>(i), rows ? in.dims[1] : in.dims[2], rows ? 1 : in.dims[2], kVF32);
          break;
        }
        case VmOp::Permute:
          if (!rd(in.a, r.a)) return fail(why, "permute of an unknown value");
          r.dst = new_val(static_cast<int>(i), prod(in.dims), in.dims[in.aux[2]], vals_[r.a].vt);
          break;
        case VmOp::Matmul: {
          if (!rd(in.a, r.a) || !rd(in.b, r.b) || (in.c >= 0 && !rd(in.c, r.c)))
            return fail(why, "matmul of an unknown value");
          const Val &A = vals_[r.a], &B = vals_[r.b];
          if (in.aux[1]) {
            if (A.vt != kVI8 || B.vt != kVI8) return fail(why, "an exact matmul of values that are not i8 tiles");
            r.mode = kMmI8;
          } else if (A.vt == kVF16 && B.vt == kVF16) {
            r.mode = kMmF16;
          } else if (A.vt == kVBF16 && B.vt == kVBF16) {
            r.mode = kMmBF16;
          } else {
            r.mode = kMmF32;
          }
          r.dst = new_val(static_cast<int>(i), (long long)in.dims[1] * in.dims[2], in.dims[2], kVF32);
          break;
        }
      }
      if (r.dst >= 0) cur[in.dst] = r.dst;
    }
    return true;
  }

  bool layouts(std::string& why) {
    for (size_t i = 0; i < vm_.inst.size(); ++i) {
      const VmInst& in = vm_.inst[i];
      const Reads& r = rd_[i];
      if (in.op == VmOp::Matmul) {
        const int K = in.aux[0], N = in.dims[2];
        Val &A = vals_[r.a], &B = vals_[r.b];
        if (!A.krow) {
          A.krow = K;
          A.pitch = r.mode == kMmF32 ? pad_to(K, 4, 2) : pad_to(K, 8, 4);
        }
        if (!B.krow) {
          B.krow = N;
          B.pitch = r.mode == kMmF32 ? N : pad_to(N, 8, 4);
        }
      } else if (in.op == VmOp::Permute) {
        Val& src = vals_[r.a];
        if (!src.krow) {
          src.krow = in.dims[2];
          src.pitch = in.dims[2] % 2 ? in.dims[2] : in.dims[2] + 1;
        }
      }
    }
    for (Val& v : vals_) {
      if (!v.krow) v.krow = v.pitch = std::max(1, v.d2);
      if (v.numel % v.krow) return fail(why, "staged layout rows do not divide a value");
    }
    return true;
  }

  bool allocate(std::string& why) {
    // a load whose value is never read keeps its slot until the run of loads
    // it belongs to has ended: the run's LDS writes are not ordered among
    // themselves
    const int n = static_cast<int>(vm_.inst.size());
    for (Val& v : vals_)
      if (v.last == v.def && vm_.inst[v.def].op == VmOp::Load) {
        int e = v.def;
        while (e + 1 < n && vm_.inst[e + 1].op == VmOp::Load) ++e;
        v.last = std::min(n - 1, e + 1);
      }
    std::vector<std::pair<long long, long long>> used;  // (offset, floats) of live values
    std::vector<int> at_def(vm_.inst.size(), -1);
    for (size_t v = 0; v < vals_.size(); ++v) at_def[vals_[v].def] = static_cast<int>(v);
    for (size_t i = 0; i < vm_.inst.size(); ++i) {
      const int v = at_def[i];
      if (v >= 0) {
        const long long fl = (vals_[v].floats() + 3) & ~3LL;
        long long at = 0;
        for (bool clash = true; clash;) {
          clash = false;
          for (auto& u : used)
            if (at < u.first + u.second && u.first < at + fl) {
              at = (u.first + u.second + 3) & ~3LL;
              clash = true;
            }
        }
        used.push_back({at, fl});
        vals_[v].off = static_cast<int>(at);
        high_ = std::max(high_, at + fl);
      }
      // values whose last use is this instruction (their slot is reused from the next one on)
      for (size_t w = 0; w < vals_.size(); ++w)
        if (vals_[w].last == static_cast<int>(i) && vals_[w].off >= 0)
          for (size_t k = 0; k < used.size(); ++k)
            if (used[k].first == vals_[w].off) {
              used.erase(used.begin() + k);
              break;
            }
    }
    if (high_ > kMaxLdsFloats)
      return fail(why, "staged kernel needs " + S((high_ * 4 + 1023) / 1024) + " KB of LDS (at most 160 KB)");
    return true;
  }

  // LDS float index of logical element `lin` of value v
  std::string phys(const Val& v, const std::string& lin) const {
    if (v.krow == v.pitch) return "(" + S(v.off) + " + (" + lin + "))";
    return "(" + S(v.off) + " + (" + lin + ") / " + S(v.krow) + " * " + S(v.pitch) + " + (" + lin + ") % " +
           S(v.krow) + ")";
  }

  // four consecutive elements from a multiple of 4 stay contiguous and aligned
  static bool vec4(const Val& v) { return v.krow % 4 == 0 && v.pitch % 4 == 0 && v.off % 4 == 0; }

  std::string origin(const TileAddr& o) const {
    std::ostringstream s;
    s << "(" << o.c0 << "LL";
    if (o.sx) s << " + (long long)x * " << o.sx << "LL";
    if (o.sy) s << " + (long long)y * " << o.sy << "LL";
    if (o.sz) s << " + (long long)z * " << o.sz << "LL";
    s << ")";
    return s.str();
  }

  // global vector width of a load / store: elements along a contiguous row
  int gvw(const VmInst& in) const {
    const VmAccess& acc = vm_.access[in.kind];
    const TileAddr& o = acc.addr;
    for (int w = std::min(4, max_vw_); w > 1; w /= 2) {
      if (in.dims[2] % w || acc.stride[2] != 1) continue;
      if (acc.stride[1] % w || acc.stride[0] % w || o.c0 % w || o.sx % w || o.sy % w || o.sz % w) continue;
      return w;
    }
    return 1;
  }

  // the element loop prologue: `e` the first of vw elements of this
  // thread's q-th group, i0 / i1 / i2 its coordinates in `d`
  void loop_open(std::ostringstream& b, long long n, int vw, const int d[3]) const {
    const long long groups = n / vw, iters = (groups + kThreads - 1) / kThreads;
    b << "#pragma unroll " << (iters <= 8 ? iters : 4) << "\n  for (int q = 0; q < " << iters << "; ++q) {\n"
      << "    const int e = (t + q * " << kThreads << ") * " << vw << ";\n";
    if (groups % kThreads) b << "    if (e < " << n << ") {\n";
    else b << "    {\n";
    b << "    const int i2 = e % " << d[2] << ", i1 = (e / " << d[2] << ") % " << d[1] << ", i0 = e / "
      << (long long)d[1] * d[2] << ";\n    (void)i0; (void)i1; (void)i2;\n";
  }
  static void loop_close(std::ostringstream& b) { b << "    }\n  }\n"; }

  // An element loop in two phases per chunk of CH groups of vw elements:
  // every LDS read of the chunk into registers indexed by j, then every
  // computation and LDS write.  (In one pass the compiler must keep each
  // read behind the previous group's write to the same shared array, and
  // with one wave per SIMD every group then waits out the LDS latency.)
  // `regs` floats a group; `read` / `write` emit a group's code given e,
  // i0, i1, i2 and j.
  void two_phase(std::ostringstream& b, long long n, int vw, const int d[3], int regs,
                 const std::function<void(std::ostringstream&)>& decl,
                 const std::function<void(std::ostringstream&)>& read,
                 const std::function<void(std::ostringstream&)>& write, int& CH) const {
    const long long groups = n / vw, iters = (groups + kThreads - 1) / kThreads;
    CH = static_cast<int>(std::max(1LL, std::min(iters, (long long)(64 / std::max(1, regs)))));
    decl(b);
    const long long chunks = (iters + CH - 1) / CH;
    auto guard = [&]() {
      std::string g;
      if (iters % CH) g = "q < " + S(iters);
      if (groups % kThreads) g += std::string(g.empty() ? "" : " && ") + "e < " + S(n);
      return g.empty() ? std::string("true") : g;
    };
    b << "#pragma unroll " << (chunks <= 4 ? chunks : 1) << "\n  for (int q0 = 0; q0 < " << iters << "; q0 += " << CH
      << ") {\n";
    for (int phase = 0; phase < 2; ++phase) {
      b << "#pragma unroll\n    for (int j = 0; j < " << CH << "; ++j) {\n      const int q = q0 + j;\n"
        << "      const int e = (t + q * " << kThreads << ") * " << vw << ";\n      if (" << guard() << ") {\n"
        << "      const int i2 = e % " << d[2] << ", i1 = (e / " << d[2] << ") % " << d[1] << ", i0 = e / "
        << (long long)d[1] * d[2] << ";\n      (void)i0; (void)i1; (void)i2;\n";
      (phase == 0 ? read : write)(b);
      b << "      }\n    }\n";
    }
    b << "  }\n";
  }

  int load_regs(int i) const {
    const VmInst& in = vm_.inst[i];
    const int w = gvw(in);
    return static_cast<int>((prod(in.dims) / w + kThreads - 1) / kThreads * w);
  }

  static const char* gtype(Elem e, int w) {
    switch (e) {
      case Elem::F32: return w == 4 ? "xf4" : w == 2 ? "xf2" : "float";
      case Elem::F16: return w == 4 ? "xh4" : w == 2 ? "xh2" : "_Float16";
      case Elem::BF16: return w == 4 ? "xu4" : w == 2 ? "xu2" : "unsigned short";
      default: return w == 4 ? "xc4" : w == 2 ? "xc2" : "signed char";
    }
  }
  static const char* gbase(Elem e) {
    return e == Elem::F32 ? "float" : e == Elem::F16 ? "_Float16" : e == Elem::BF16 ? "unsigned short" : "signed char";
  }
  static std::string to_f32(Elem e, const std::string& q) {
    return e == Elem::BF16 ? "xbf(" + q + ")" : e == Elem::F32 ? q : "(float)" + q;
  }
  bool streamed(int acc) const {
    const TileAddr& o = vm_.access[acc].addr;
    return o.sx != 0 || o.sy != 0 || o.sz != 0;
  }

  void emit_load_read(std::ostringstream& b, int i) {
    const VmInst& in = vm_.inst[i];
    const VmAccess& acc = vm_.access[in.kind];
    const int w = gvw(in);
    gvw_max_ = std::max(gvw_max_, w);
    const long long n = prod(in.dims);
    const long long iters = (n / w + kThreads - 1) / kThreads;
    const std::string R = "r" + S(i);
    b << "  // load " << i << ": [" << in.dims[0] << "," << in.dims[1] << "," << in.dims[2] << "] of a.p["
      << in.kind << "]\n";
    b << "  float " << R << "[" << iters * w << "];\n  {\n    const long long org = " << origin(acc.addr) << ";\n";
    loop_open(b, n, w, in.dims);
    b << "    const long long off = org + (long long)i0 * " << acc.stride[0] << "LL + (long long)i1 * "
      << acc.stride[1] << "LL + (long long)i2 * " << acc.stride[2] << "LL;\n";
    const char* ty = gtype(acc.elem, w);
    b << "    const " << ty << " qv = " << (streamed(in.kind) ? "__builtin_nontemporal_load(" : "*(")
      << "reinterpret_cast<const " << ty << "*>(static_cast<const " << gbase(acc.elem) << "*>(a.p[" << in.kind
      << "]) + off));\n";
    if (w == 1) b << "    " << R << "[q] = " << to_f32(acc.elem, "qv") << ";\n";
    else
      b << "#pragma unroll\n    for (int c = 0; c < " << w << "; ++c) " << R << "[q * " << w << " + c] = "
        << to_f32(acc.elem, "qv[c]") << ";\n";
    loop_close(b);
    b << "  }\n";
  }

  void emit_load_write(std::ostringstream& b, int i) {
    const VmInst& in = vm_.inst[i];
    const Val& v = vals_[rd_[i].dst];
    const int w = gvw(in);
    const long long n = prod(in.dims);
    const std::string R = "r" + S(i);
    b << "  {\n";
    loop_open(b, n, w, in.dims);
    if (w == 4 && vec4(v))
      b << "    *reinterpret_cast<xf4*>(&S[" << phys(v, "e") << "]) = xf4{" << R << "[q * 4], " << R
        << "[q * 4 + 1], " << R << "[q * 4 + 2], " << R << "[q * 4 + 3]};\n";
    else
      b << "#pragma unroll\n    for (int c = 0; c < " << w << "; ++c) S[" << phys(v, "e + c") << "] = " << R
        << "[q * " << w << " + c];\n";
    loop_close(b);
    b << "  }\n";
  }

  void emit_store(std::ostringstream& b, int i) {
    const VmInst& in = vm_.inst[i];
    const VmAccess& acc = vm_.access[in.kind];
    const Val& v = vals_[rd_[i].a];
    const int w = gvw(in);
    gvw_max_ = std::max(gvw_max_, w);
    const long long n = prod(in.dims);
    b << "  // store " << i << ": [" << in.dims[0] << "," << in.dims[1] << "," << in.dims[2] << "] to a.p["
      << in.kind << "]\n  {\n    const long long org = " << origin(acc.addr) << ";\n";
    loop_open(b, n, w, in.dims);
    b << "    const long long off = org + (long long)i0 * " << acc.stride[0] << "LL + (long long)i1 * "
      << acc.stride[1] << "LL + (long long)i2 * " << acc.stride[2] << "LL;\n";
    if (w == 4 && vec4(v)) b << "    const xf4 f = *reinterpret_cast<const xf4*>(&S[" << phys(v, "e") << "]);\n";
    else {
      b << "    float f[" << w << "];\n";
      b << "#pragma unroll\n    for (int c = 0; c < " << w << "; ++c) f[c] = S[" << phys(v, "e + c") << "];\n";
    }
    std::string conv;
    switch (acc.elem) {
      case Elem::F32: conv = "f[c]"; break;
      case Elem::F16: conv = "xto_f16(f[c])"; break;
      case Elem::BF16: conv = "xto_bf16(f[c])"; break;
      default: conv = "(signed char)xto_i8(f[c])"; break;
    }
    const char* base = acc.elem == Elem::F32 ? "float" : acc.elem == Elem::I8 ? "signed char" : "unsigned short";
    const char* ty = acc.elem == Elem::F32 ? gtype(Elem::F32, w) : acc.elem == Elem::I8 ? gtype(Elem::I8, w)
                                                                                          : gtype(Elem::BF16, w);
    if (w == 1) {
      b << "    { const int c = 0; *(static_cast<" << base << "*>(a.p[" << in.kind << "]) + off) = " << conv
        << "; }\n";
    } else {
      b << "    " << ty << " qv;\n#pragma unroll\n    for (int c = 0; c < " << w << "; ++c) qv[c] = " << conv
        << ";\n";
      b << "    " << (streamed(in.kind) ? "__builtin_nontemporal_store(qv, " : "*(") << "reinterpret_cast<" << ty
        << "*>(static_cast<" << base << "*>(a.p[" << in.kind << "]) + off)" << (streamed(in.kind) ? ");" : ") = qv;")
        << "\n";
    }
    loop_close(b);
    b << "  }\n";
  }

  // logical element index of an operand of dims `od` broadcast to the
  // result's (i0, i1, i2)
  static std::string bcast(const int od[3]) {
    std::string i0 = od[0] == 1 ? "0" : "i0", i1 = od[1] == 1 ? "0" : "i1", i2 = od[2] == 1 ? "0" : "i2";
    return "((" + i0 + " * " + S(od[1]) + " + " + i1 + ") * " + S(od[2]) + " + " + i2 + ")";
  }

  void emit_elementwise(std::ostringstream& b, int i) {
    const VmInst& in = vm_.inst[i];
    const Reads& r = rd_[i];
    const Val& D = vals_[r.dst];
    const long long n = prod(in.dims);
    const bool bin = in.op == VmOp::Binary;
    const Val& A = vals_[r.a];
    const Val* B = bin ? &vals_[r.b] : nullptr;
    int ad[3] = {in.dims[0], in.dims[1], in.dims[2]}, bd[3] = {1, 1, 1};
    if (bin)
      for (int d = 0; d < 3; ++d) {
        ad[d] = in.lhs[d];
        bd[d] = in.aux[d];
      }
    // four elements at a time when every operand that varies along the
    // innermost dim is contiguous there
    bool v4 = in.dims[2] % 4 == 0 && n % 4 == 0 && vec4(D) && (ad[2] == 1 || vec4(A)) &&
              (!bin || bd[2] == 1 || vec4(*B));
    const int w = v4 ? 4 : 1;
    const char* ty = w == 4 ? "xf4" : "float";
    b << "  // " << (bin ? "binary " : "unary ") << i << "\n  {\n";
    int CH = 1;
    auto operand = [&](std::ostringstream& o, const Val& v, const int od[3], const std::string& name) {
      const std::string lin = bcast(od);
      if (w == 4 && od[2] != 1)
        o << "      " << name << "[j] = *reinterpret_cast<const xf4*>(&S[" << phys(v, lin) << "]);\n";
      else if (w == 4)
        o << "      { const float s1 = S[" << phys(v, lin) << "]; " << name << "[j] = xf4{s1, s1, s1, s1}; }\n";
      else
        o << "      " << name << "[j] = S[" << phys(v, lin) << "];\n";
    };
    std::string expr;
    if (bin) {
      const char* op = in.kind == 0 ? " + " : in.kind == 1 ? " - " : " * ";
      expr = w == 4 ? "va[j][c]" + std::string(op) + "vb[j][c]" : "va[j]" + std::string(op) + "vb[j]";
    } else {
      expr = replace_x(unary_expr(in.kind), w == 4 ? "va[j][c]" : "va[j]");
    }
    const int regs = w * (bin ? 2 : 1);
    two_phase(
        b, n, w, in.dims, regs,
        [&](std::ostringstream& o) {
          const long long groups = n / w, iters = (groups + kThreads - 1) / kThreads;
          const long long ch = std::max(1LL, std::min(iters, (long long)(64 / std::max(1, regs))));
          o << "  " << ty << " va[" << ch << "];\n";
          if (bin) o << "  " << ty << " vb[" << ch << "];\n";
        },
        [&](std::ostringstream& o) {
          operand(o, A, ad, "va");
          if (bin) operand(o, *B, bd, "vb");
        },
        [&](std::ostringstream& o) {
          if (w == 4)
            o << "      xf4 ov;\n#pragma unroll\n      for (int c = 0; c < 4; ++c) ov[c] = " << expr
              << ";\n      *reinterpret_cast<xf4*>(&S[" << phys(D, "e") << "]) = ov;\n";
          else
            o << "      S[" << phys(D, "e") << "] = " << expr << ";\n";
        },
        CH);
    b << "  }\n";
  }

  void emit_reduce(std::ostringstream& b, int i) {
    const VmInst& in = vm_.inst[i];
    const Reads& r = rd_[i];
    const Val &A = vals_[r.a], &D = vals_[r.dst];
    const int R = in.dims[1], C = in.dims[2];
    const bool mx = in.kind == 1;
    const std::string init = mx ? "-__builtin_huge_valf()" : "0.0f";
    auto comb = [&](const std::string& p, const std::string& q) {
      return mx ? "fmaxf(" + p + ", " + q + ")" : p + " + " + q;
    };
    b << "  // reduce " << i << " over axis " << in.aux[0] << " of [" << R << "," << C << "]\n  {\n";
    if (in.aux[0] == 1) {
      // G lanes a row, G the smallest power of two that gives every thread
      // a row (at most 64, at most the row length): each lane combines its
      // share of the row in registers (float4 chunks g, g + G, ... when the
      // row allows), then log2(G) shuffle steps; rows beyond the 256
      // threads' first pass run in further passes, unrolled so that their
      // read and shuffle chains overlap.
      int G = 1;
      while (G < 64 && G * 2 <= C && (long long)R * G < kThreads) G *= 2;
      const int rows_per = kThreads / G;
      const long long passes = (R + rows_per - 1) / rows_per;
      const bool v4 = C % (4 * G) == 0 && vec4(A);
      const long long per = v4 ? C / (4 * G) : (C + G - 1) / G;
      b << "    const int g = t % " << G << ", r0 = t / " << G << ";\n";
      b << "#pragma unroll " << (passes <= 8 ? passes : 4) << "\n    for (int p = 0; p < " << passes << "; ++p) {\n"
        << "      const int r = r0 + p * " << rows_per << ";\n      float m = " << init << ";\n";
      if (R % rows_per) b << "      if (r < " << R << ") {\n";
      else b << "      {\n";
      b << "#pragma unroll " << (per <= 16 ? per : 8) << "\n        for (int j = 0; j < " << per << "; ++j) {\n";
      if (v4) {
        b << "          const xf4 q4 = *reinterpret_cast<const xf4*>(&S["
          << phys(A, "r * " + S(C) + " + 4 * (g + j * " + S(G) + ")") << "]);\n";
        b << "          m = " << comb(comb(comb(comb("m", "q4[0]"), "q4[1]"), "q4[2]"), "q4[3]") << ";\n";
      } else {
        b << "          const int c = g + j * " << G << ";\n";
        if (C % G) b << "          if (c < " << C << ") m = " << comb("m", "S[" + phys(A, "r * " + S(C) + " + c") + "]")
                     << ";\n";
        else b << "          m = " << comb("m", "S[" + phys(A, "r * " + S(C) + " + c") + "]") << ";\n";
      }
      b << "        }\n      }\n";
      for (int o = G / 2; o > 0; o /= 2)
        b << "      m = " << comb("m", "__shfl_xor(m, " + S(o) + ", " + S(G) + ")") << ";\n";
      b << "      if (g == 0" << (R % rows_per ? " && r < " + S(R) : "") << ") S[" << phys(D, "r") << "] = m;\n";
      b << "    }\n";
    } else {
      const long long iters = (C + kThreads - 1) / kThreads;
      b << "#pragma unroll\n    for (int q = 0; q < " << iters << "; ++q) {\n      const int c = t + q * " << kThreads
        << ";\n";
      if (C % kThreads) b << "      if (c < " << C << ") {\n";
      else b << "      {\n";
      b << "        float m = " << init << ";\n#pragma unroll 8\n        for (int rr = 0; rr < " << R
        << "; ++rr) m = " << comb("m", "S[" + phys(A, "rr * " + S(C) + " + c") + "]") << ";\n        S["
        << phys(D, "c") << "] = m;\n      }\n    }\n";
    }
    b << "  }\n";
  }

  void emit_permute(std::ostringstream& b, int i) {
    const VmInst& in = vm_.inst[i];
    const Reads& r = rd_[i];
    const Val &A = vals_[r.a], &D = vals_[r.dst];
    const int od[3] = {in.dims[in.aux[0]], in.dims[in.aux[1]], in.dims[in.aux[2]]};
    const long long n = prod(in.dims);
    b << "  // permute " << i << "\n  {\n";
    int CH = 1;
    // output (i0, i1, i2) = input index with dim perm[d] at i_d
    const std::string src = "(iv[0] * " + S(in.dims[1]) + " + iv[1]) * " + S(in.dims[2]) + " + iv[2]";
    two_phase(
        b, n, 1, od, 1,
        [&](std::ostringstream& o) {
          const long long iters = (n + kThreads - 1) / kThreads;
          o << "  float pv[" << std::max(1LL, std::min(iters, 64LL)) << "];\n";
        },
        [&](std::ostringstream& o) {
          o << "      int iv[3];\n      iv[" << in.aux[0] << "] = i0;\n      iv[" << in.aux[1] << "] = i1;\n      iv["
            << in.aux[2] << "] = i2;\n      pv[j] = S[" << phys(A, src) << "];\n";
        },
        [&](std::ostringstream& o) { o << "      S[" << phys(D, "e") << "] = pv[j];\n"; }, CH);
    b << "  }\n";
  }

  void emit_matmul(std::ostringstream& b, int i) {
    const VmInst& in = vm_.inst[i];
    const Reads& r = rd_[i];
    const Val &A = vals_[r.a], &B = vals_[r.b], &D = vals_[r.dst];
    const Val* C = r.c >= 0 ? &vals_[r.c] : nullptr;
    const int M = in.dims[1], N = in.dims[2], K = in.aux[0];
    const int mode = r.mode;
    // K elements per MFMA and per lane
    const int KB = mode == kMmF32 ? 2 : mode == kMmI8 ? 32 : 16, KL = KB / 2;
    const int MT = (M + 31) / 32, NT = (N + 31) / 32, steps = (K + KB - 1) / KB;
    const bool mg = M % 32 != 0, ng = N % 32 != 0, kg = K % KB != 0;
    b << "  // matmul " << i << ": [" << M << "," << K << "] x [" << K << "," << N << "]"
      << (C ? " + acc" : "") << ", " << (mode == kMmF32 ? "f32" : mode == kMmF16 ? "f16" : mode == kMmBF16 ? "bf16" : "i8")
      << " MFMA\n  {\n";
    b << "    const int l32 = lane & 31, h = lane >> 5;\n";
    b << "    for (int u = wave; u < " << MT * NT << "; u += 4) {\n"
      << "      const int row = (u / " << NT << ") * 32 + l32, col = (u % " << NT << ") * 32 + l32;\n";
    // two accumulators, even and odd K steps: consecutive MFMAs are then
    // independent and issue back to back (a dependent chain waits out each
    // MFMA's latency); their sum is the tile's (exact for i8)
    b << "      " << (mode == kMmI8 ? "xi16v" : "xf16v") << " acc0 = {}, acc1 = {};\n";
    // fragments of K step `st` into set `p` (fa<p>, fb<p>)
    const bool avec = KL >= 4 && A.krow == K && vec4(A) && !kg;
    auto read = [&](const std::string& st, int p) -> std::string {
      std::ostringstream o;
      const std::string FA = "fa" + S(p), FB = "fb" + S(p);
      o << "        {\n          const int k0 = (" << st << ") * " << KB << " + h * " << KL << ";\n";
      if (avec) {
        o << (mg ? "          if (row < " + S(M) + ") {\n" : "          {\n");
        o << "#pragma unroll\n            for (int j = 0; j < " << KL / 4 << "; ++j) {\n"
          << "              const xf4 q4 = *reinterpret_cast<const xf4*>(&S["
          << phys(A, "row * " + S(K) + " + k0 + 4 * j") << "]);\n              " << FA << "[4 * j] = q4[0]; " << FA
          << "[4 * j + 1] = q4[1]; " << FA << "[4 * j + 2] = q4[2]; " << FA << "[4 * j + 3] = q4[3];\n"
          << "            }\n          }\n";
        if (mg)
          o << "          else {\n#pragma unroll\n            for (int j = 0; j < " << KL << "; ++j) " << FA
            << "[j] = 0.0f;\n          }\n";
      } else {
        std::string cond;
        if (mg) cond = "row < " + S(M);
        if (kg) cond += (cond.empty() ? "" : " && ") + std::string("k < ") + S(K);
        o << "#pragma unroll\n          for (int j = 0; j < " << KL << "; ++j) {\n            const int k = k0 + j;\n"
          << "            " << FA << "[j] = ";
        if (!cond.empty()) o << "(" << cond << ") ? S[" << phys(A, "row * " + S(K) + " + k") << "] : 0.0f;\n";
        else o << "S[" << phys(A, "row * " + S(K) + " + k") << "];\n";
        o << "          }\n";
      }
      {
        std::string cond;
        if (ng) cond = "col < " + S(N);
        if (kg) cond += (cond.empty() ? "" : " && ") + std::string("k < ") + S(K);
        o << "#pragma unroll\n          for (int j = 0; j < " << KL << "; ++j) {\n            const int k = k0 + j;\n"
          << "            " << FB << "[j] = ";
        if (!cond.empty()) o << "(" << cond << ") ? S[" << phys(B, "k * " + S(N) + " + col") << "] : 0.0f;\n";
        else o << "S[" << phys(B, "k * " + S(N) + " + col") << "];\n";
        o << "          }\n";
      }
      o << "        }\n";
      return o.str();
    };
    auto mfma = [&](int p) -> std::string {
      std::ostringstream o;
      const std::string FA = "fa" + S(p), FB = "fb" + S(p);
      const std::string acc = "acc" + S(p % 2);
      switch (mode) {
        case kMmF32:
          o << "        " << acc << " = __builtin_amdgcn_mfma_f32_32x32x2f32(" << FA << "[0], " << FB << "[0], " << acc
            << ", 0, 0, 0);\n";
          break;
        case kMmF16:
          o << "        {\n          xh8 ha, hb;\n#pragma unroll\n          for (int j = 0; j < 8; ++j) { ha[j] = "
               "(_Float16)" << FA << "[j]; hb[j] = (_Float16)" << FB << "[j]; }\n"
            << "          " << acc << " = __builtin_amdgcn_mfma_f32_32x32x16_f16(ha, hb, " << acc << ", 0, 0, 0);\n        }\n";
          break;
        case kMmBF16:
          o << "        {\n          xs8 ha, hb;\n#pragma unroll\n          for (int j = 0; j < 8; ++j) { ha[j] = "
               "(short)(__float_as_uint(" << FA << "[j]) >> 16); hb[j] = (short)(__float_as_uint(" << FB
            << "[j]) >> 16); }\n"
            << "          " << acc << " = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(xb8, ha), "
               "__builtin_bit_cast(xb8, hb), " << acc << ", 0, 0, 0);\n        }\n";
          break;
        default:
          o << "        {\n          xi4v ia, ib;\n#pragma unroll\n          for (int j = 0; j < 4; ++j) {\n";
          for (const char* F : {"ia", "ib"}) {
            const std::string X = std::string(F) == "ia" ? FA : FB;
            o << "            " << F << "[j] = (int)((unsigned)((int)" << X << "[4 * j] & 255) | ((unsigned)((int)"
              << X << "[4 * j + 1] & 255) << 8) | ((unsigned)((int)" << X << "[4 * j + 2] & 255) << 16) | "
              << "((unsigned)((int)" << X << "[4 * j + 3] & 255) << 24));\n";
          }
          o << "          }\n          " << acc << " = __builtin_amdgcn_mfma_i32_32x32x32_i8(ia, ib, " << acc << ", 0, 0, 0);\n"
            << "        }\n";
          break;
      }
      return o.str();
    };
    // A ring of NS fragment sets: the reads of steps s + 1 .. s + NS - 1 are
    // in flight while step s's MFMA runs (an f32 step is one 64-cycle MFMA
    // on two floats a lane, so it reads furthest ahead).  The loop body has
    // no branch (the compiler waits for every LDS read at a block boundary):
    // look-ahead reads past the last step re-read the last step, and the
    // steps beyond the last whole group run after the loop from the sets the
    // loop's reads already filled.
    int NS = std::max(1, std::min(steps, mode == kMmF32 ? 8 : 4));
    if (NS > 1 && NS % 2) --NS;  // even: set j holds steps of parity j % 2
    const int full = steps / NS * NS, tail = steps - full;
    auto clamp = [&](const std::string& e) { return "min(" + e + ", " + S(steps - 1) + ")"; };
    b << "      float";
    for (int q = 0; q < NS; ++q) b << (q ? ", " : " ") << "fa" << q << "[" << KL << "], fb" << q << "[" << KL << "]";
    b << ";\n";
    for (int q = 0; q + 1 < NS; ++q) b << read(S(std::min(q, steps - 1)), q);
    b << "#pragma unroll 1\n      for (int s = 0; s < " << full << "; s += " << NS << ") {\n";
    // scheduling fences keep each step's look-ahead reads ahead of its MFMA
    // (left alone, the compiler sinks them next to their use)
    for (int j = 0; j < NS; ++j) {
      if (NS > 1) b << read(clamp("s + " + S(j + NS - 1)), (j + NS - 1) % NS);
      else b << read("s", 0);
      b << "        __builtin_amdgcn_sched_barrier(0);\n" << mfma(j) << "        __builtin_amdgcn_sched_barrier(0);\n";
    }
    b << "      }\n";
    for (int j = 0; j < tail; ++j) b << mfma(j);
    b << "      const auto acc = acc0 + acc1;\n";
    // D: lane l holds column col; register v holds row 8 (v / 4) + 4 h + v % 4 of the tile
    b << "#pragma unroll\n      for (int v = 0; v < 16; ++v) {\n"
      << "        const int rr = (u / " << NT << ") * 32 + 8 * (v >> 2) + 4 * h + (v & 3);\n";
    std::string cond;
    if (mg) cond = "rr < " + S(M);
    if (ng) cond += (cond.empty() ? "" : " && ") + std::string("col < ") + S(N);
    b << "        " << (cond.empty() ? "{" : "if (" + cond + ") {") << "\n";
    b << "          float o = " << (mode == kMmI8 ? "(float)acc[v]" : "acc[v]") << ";\n";
    if (C) b << "          o = o + S[" << phys(*C, "rr * " + S(N) + " + col") << "];\n";
    b << "          S[" << phys(D, "rr * " + S(N) + " + col") << "] = o;\n        }\n      }\n    }\n  }\n";
  }
};

}  // namespace

bool stage_vm(const VmPlan& vm, const int32_t grid[3], FusedPlan& out, std::string& why, int max_vw) {
  if (vm.access.size() > 8) {
    why = "staged kernels take at most 8 loads and stores";
    return false;
  }
  // a load must not read what the program stored (global writes are not
  // ordered before later reads of the workgroup)
  std::vector<int> stored;
  for (const VmInst& in : vm.inst) {
    if (in.op != VmOp::Load && in.op != VmOp::Store) continue;
    const int arg = vm.access[in.kind].arg;
    if (in.op == VmOp::Store) stored.push_back(arg);
    else if (std::find(stored.begin(), stored.end(), arg) != stored.end()) {
      why = "staged kernels do not load a memref the program has stored to";
      return false;
    }
  }
  const long long blocks = (long long)grid[0] * grid[1] * grid[2];
  if (blocks < 1 || blocks > 0x7fffffffLL) {
    why = "staged kernel grid out of range";
    return false;
  }
  StagedGen g(vm, grid, max_vw);
  return g.run(out, why);
}

}  // namespace xt
